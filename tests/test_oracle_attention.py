"""The oracle's attention prepare (RMSNorm + RoPE) and decode routes pinned
by identities and fp64 softmax (CPU). Reference arithmetic:
attention.metal:36-70, 262-313 (prepare), attention_decode.metal:51-431,
830-891 (decode routes), model.rs:327-347 (route choice at 1024).
"""
import numpy as np
import pytest

import oracle as O
from helpers import assert_bf16_close, bf16, f32, fp64_attention_gated, rng


def prepare_inputs(r):
    return dict(q=bf16(r.normal(0, 1, 4096)), k=bf16(r.normal(0, 1, 512)), v=bf16(r.normal(0, 1, 512)),
                qg=bf16(1 + 0.1 * r.normal(0, 1, 256)), kg=bf16(1 + 0.1 * r.normal(0, 1, 256)))


def normalised_fp64(x, gain):
    """bf16(bf16(x / rms(x)) * gain) with the rms in fp64."""
    xd = f32(x).astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(xd * xd) + 1e-6)
    return f32(bf16((f32(bf16(xd * inv)).astype(np.float64) * f32(gain)).astype(np.float32)))


def run_prepare(x, pos, cap=8):
    kc = np.zeros((2, cap, 256), np.uint16)
    vc = np.zeros((2, cap, 256), np.uint16)
    query = O.attn_prepare(x["q"], x["k"], x["v"], x["qg"], x["kg"], kc, vc, pos, cap)
    return query, kc, vc


def test_rope_position_zero_is_identity():
    x = prepare_inputs(rng(30))
    query, kc, vc = run_prepare(x, 0)
    for h in range(8):
        want = bf16(normalised_fp64(x["q"][h * 512:h * 512 + 256], x["qg"]))
        assert_bf16_close(query[h * 256:(h + 1) * 256], want, max_ulp=1, max_frac=0.02, what=f"q head {h}")
    for g in range(2):
        want = bf16(normalised_fp64(x["k"][g * 256:(g + 1) * 256], x["kg"]))
        assert_bf16_close(kc[g, 0], want, max_ulp=1, max_frac=0.02, what=f"k head {g}")
        assert np.array_equal(vc[g, 0], x["v"][g * 256:(g + 1) * 256]), "V row is copied"


@pytest.mark.parametrize("pos", [1, 17, 4095, 131071])
def test_rope_rotates_pairs(pos):
    """Dims (i, i+32), i < 32, rotate by pos * inv_freq[i]; dims >= 64 pass
    through; pair norms are preserved (fp64 rotation, bf16 tolerance)."""
    x = prepare_inputs(rng(31 + pos))
    q0, _, _ = run_prepare(x, 0, cap=pos + 1)
    qp, kc, _ = run_prepare(x, pos, cap=pos + 1)
    inv = np.array([O.lib().eo_rope_inv_freq(i) for i in range(32)], np.float32)
    ang = (np.float32(pos) * inv).astype(np.float64)
    for h in range(8):
        n = f32(q0[h * 256:(h + 1) * 256]).astype(np.float64)
        lo, hi = n[:32], n[32:64]
        want = np.concatenate([lo * np.cos(ang) - hi * np.sin(ang), lo * np.sin(ang) + hi * np.cos(ang), n[64:]])
        got = qp[h * 256:(h + 1) * 256]
        assert np.array_equal(got[64:], q0[h * 256 + 64:(h + 1) * 256])
        assert_bf16_close(got, bf16(want.astype(np.float32)), max_ulp=1, max_frac=0.1, atol_rel=2e-3,
                          what=f"head {h}")
        g = f32(got).astype(np.float64)
        assert np.allclose(np.hypot(g[:32], g[32:64]), np.hypot(lo, hi), rtol=1e-2, atol=1e-2)


def decode_inputs(r, length, cap=None):
    cap = cap or length + 4
    return dict(query=bf16(r.normal(0, 1, 2048)), kc=bf16(r.normal(0, 1, (2, cap, 256))),
                vc=bf16(r.normal(0, 1, (2, cap, 256))), q=bf16(r.normal(0, 1, 4096)), cap=cap)


def gate_of(o, q_proj):
    sig = np.array([O.lib().eo_sigmoid_bf(float(g)) for g in f32(q_proj).reshape(8, 512)[:, 256:].ravel()],
                   np.float32)
    return bf16(f32(o) * sig)


def test_single_position_returns_value_row():
    """N = 1: softmax weight 1, so the output is the V row exactly, gated."""
    x = decode_inputs(rng(40), 1)
    got = O.attn_decode_gated(x["query"], x["kc"], x["vc"], 1, x["cap"], x["q"])
    v = np.concatenate([x["vc"][h // 4, 0] for h in range(8)])
    assert np.array_equal(got, gate_of(v, x["q"]))


@pytest.mark.parametrize("length", [500, 3000])
def test_identical_keys_average_values(length):
    """Equal scores: the output is the mean of the V rows (both routes)."""
    x = decode_inputs(rng(41 + length), length)
    x["kc"][:, :length] = x["kc"][:, :1]
    got = O.attn_decode_gated(x["query"], x["kc"], x["vc"], length, x["cap"], x["q"])
    mean = np.concatenate([f32(x["vc"][h // 4, :length]).astype(np.float64).mean(0) for h in range(8)])
    # the long route rounds each chain's partial to bf16: near-zero means move
    # by many ulps but stay within 2e-2 of the output scale
    assert_bf16_close(got, gate_of(bf16(mean.astype(np.float32)), x["q"]), max_ulp=2,
                      max_frac=0.1 if length < 1024 else 0.5, atol_rel=2e-2, what="mean of V")


@pytest.mark.parametrize("length", [700, 2500])
def test_dominant_key_selects_its_row(length):
    """One key aligned with the query and far larger: its V row wins."""
    r = rng(42 + length)
    x = decode_inputs(r, length)
    x["kc"][:, :length] = bf16(0.01 * r.normal(0, 1, (2, length, 256)))
    star = length // 3
    for g in range(2):
        x["kc"][g, star] = bf16(20.0 * np.sign(f32(x["query"][g * 4 * 256:(g * 4 + 1) * 256])))
    x["query"] = np.concatenate([x["query"][(h // 4) * 4 * 256:((h // 4) * 4 + 1) * 256] for h in range(8)])
    got = O.attn_decode_gated(x["query"], x["kc"], x["vc"], length, x["cap"], x["q"])
    v = np.concatenate([x["vc"][h // 4, star] for h in range(8)])
    assert np.array_equal(got, gate_of(v, x["q"]))


@pytest.mark.parametrize("length", [1, 33, 1023, 1024, 1025, 4097])
def test_decode_matches_fp64_route(length):
    x = decode_inputs(rng(43 + length), length)
    got = O.attn_decode_gated(x["query"], x["kc"], x["vc"], length, x["cap"], x["q"])
    want = fp64_attention_gated(x["query"], x["kc"], x["vc"], length, x["q"])
    assert_bf16_close(got, want, max_ulp=2, max_frac=0.05, atol_rel=2e-3, what=f"N={length}")


def test_split_route_agrees_with_single_pass():
    """Above 1024 the two-pass route equals the one-pass softmax up to its
    bf16 partial rounding (the LSE merge is associative in exact arithmetic)."""
    length = 2048
    x = decode_inputs(rng(44), length)
    split = O.attn_decode_gated(x["query"], x["kc"], x["vc"], length, x["cap"], x["q"])
    single = O.attn_gate(O.attn_decode_single(x["query"], x["kc"], x["vc"], length, x["cap"]), x["q"])
    # 64 partials each rounded to bf16 (relative 2^-9) move the output by up to
    # ~1e-2 of its scale, many bf16 ulps for near-zero outputs
    assert_bf16_close(split, single, max_ulp=2, max_frac=0.5, atol_rel=1e-2, what="split vs single")


def test_chain_states():
    """Each chain's max is its largest score and its sum is >= 1 (the max term
    contributes exactly 1); chains take positions c, c+64, ..."""
    length = 1500
    x = decode_inputs(rng(45), length)
    parts, sums, maxs = O.attn_decode_split(x["query"], x["kc"], x["vc"], length, x["cap"])
    q = f32(x["query"]).reshape(8, 256).astype(np.float64) * 0.0625
    for h in range(8):
        s = f32(x["kc"][h // 4, :length]).astype(np.float64) @ q[h]
        for c in (0, 5, 63):
            assert abs(maxs[h, c] - s[c::64].max()) <= 1e-5 * (1 + abs(s).max())
            assert sums[h, c] >= 1.0
            assert abs(sums[h, c] - np.exp(s[c::64] - s[c::64].max()).sum()) <= 1e-5 * sums[h, c]

"""Audits of the decode operators at the edges of their inputs, in the manner
of the reference's own audits: every output buffer is surrounded by 0xa5
guard bytes that must survive the call (linear_input_norm_audit_005.rs:16-17,
gdn_input_audit_005.rs:18,31); inputs are swept over the scales 0, 0.001,
0.1, 1, 10 and 100 (linear_input_norm_audit_005.rs:29), carry injected
0, -0, +-1, +-1e-5 and +-88 (gdn_fusion_audit.rs:27) and exact +-0 at every
index i with i % 251 == 0 (linear_fusion_audit.rs:16). Every result is held
to the oracle bit for bit.

The attention cases also reach the kernel's edge paths: equal keys (every
running-max factor exactly 1, where the kernel skips its products by 1),
and score ranges of hundreds (exponentials below the series' cut-off of -86
are exactly 0).
"""
import numpy as np
import pytest

import esdecode as E
import oracle as O
from helpers import assert_bits_equal, bf16, f32, random_q4, rng

pytestmark = pytest.mark.gpu

GUARD = 256  # guard bytes on each side; keeps the payload 256-byte aligned
SCALES = [0.0, 0.001, 0.1, 1.0, 10.0, 100.0]
SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 1e-5, -1e-5, 88.0, -88.0], dtype=np.float32)


class Guarded:
    """A device buffer of `nbytes` between two 0xa5 guard regions."""

    def __init__(self, nbytes, init=None):
        self.nbytes = int(nbytes)
        self.buf = E.DeviceBuffer(self.nbytes + 2 * GUARD)
        self.buf.fill(0xA5)
        self.ptr = self.buf.ptr + GUARD
        if init is not None:
            self.buf.upload(np.ascontiguousarray(init), offset=GUARD)

    def numpy(self, dtype, count=None):
        return self.buf.numpy(dtype, count, offset=GUARD)

    def check_guards(self, what):
        raw = self.buf.numpy(np.uint8)
        head, tail = raw[:GUARD], raw[GUARD + self.nbytes:]
        assert (head == 0xA5).all(), f"{what}: {int((head != 0xA5).sum())} guard bytes before the output changed"
        assert (tail == 0xA5).all(), f"{what}: {int((tail != 0xA5).sum())} guard bytes after the output changed"


def audit_vector(r, n, scale, sigma=1.0):
    """bf16 N(0, sigma) * scale with the special values injected at random
    places and exact +-0 at i % 251 == 0."""
    x = r.normal(0, sigma, n).astype(np.float32) * np.float32(scale)
    idx = r.choice(n, size=min(n, 2 * SPECIALS.size), replace=False)
    x[idx] = np.resize(SPECIALS, idx.size)
    zeros = np.arange(0, n, 251)
    x[zeros] = np.where(np.arange(zeros.size) % 2 == 0, np.float32(0.0), np.float32(-0.0))
    return bf16(x)


@pytest.mark.parametrize("scale", SCALES)
@pytest.mark.parametrize("n,k", [(3584, 1024), (1024, 3584), (1000, 2048), (248320, 1024)])
def test_audit_q4_matvec(n, k, scale):
    print(f"case audit q4_matvec n={n} k={k} scale={scale}", flush=True)
    r = rng(7000 + n + k + int(scale * 1000))
    codes, scales, biases = random_q4(r, n, k)
    x = audit_vector(r, k, scale)
    W = E.DeviceQ4(codes, scales, biases)
    dx = Guarded(2 * k, x)
    dy, dyf = Guarded(2 * n), Guarded(4 * n)
    E.check(E.lib().es_q4_matvec(W.struct, dx.ptr, dy.ptr, dyf.ptr, None))
    E.synchronize()
    wy, wyf = O.q4_matvec(codes, scales, biases, x, want_f32=True)
    assert_bits_equal(dyf.numpy(np.float32, n), wyf, what="fp32 sums")
    assert_bits_equal(dy.numpy(np.uint16, n), wy, what="y")
    for b, w in ((dx, "x"), (dy, "y"), (dyf, "y_f32")):
        b.check_guards(w)
    assert np.array_equal(dx.numpy(np.uint16, k), x), "the input must be left as it was"


@pytest.mark.parametrize("scale", SCALES)
@pytest.mark.parametrize("k", [1024, 2048, 3584])
def test_audit_q4_matvec_add_aliasing(k, scale):
    """y = residual + W x written over the residual (the reference's
    in-place residual add)."""
    r = rng(7100 + k + int(scale * 1000))
    n = 1024
    codes, scales, biases = random_q4(r, n, k)
    x = audit_vector(r, k, scale)
    res = audit_vector(r, n, max(scale, 1.0))
    W = E.DeviceQ4(codes, scales, biases)
    dx, dh = Guarded(2 * k, x), Guarded(2 * n, res)
    E.check(E.lib().es_q4_matvec_add(W.struct, dx.ptr, dh.ptr, dh.ptr, None))
    E.synchronize()
    assert_bits_equal(dh.numpy(np.uint16, n), O.q4_matvec_add(codes, scales, biases, x, res), what="y")
    dh.check_guards("y")
    dx.check_guards("x")


@pytest.mark.parametrize("scale", SCALES)
def test_audit_rmsnorm_matvec_multi(scale):
    """Input RMSNorm feeding the GDN projections (q|k|v, z, a, b), including
    the all-zero input (norm of zeros) and +-88 entries."""
    r = rng(7200 + int(scale * 1000))
    x = audit_vector(r, 1024, scale, sigma=3.0)
    gain = audit_vector(r, 1024, 1.0, sigma=0.1) if scale else bf16(np.ones(1024))
    shapes = [6144, 2048, 16, 16]
    mats = [random_q4(r, n, 1024) for n in shapes]
    dev = [E.DeviceQ4(*m) for m in mats]
    arr = (E.Q4 * 4)(*[d.struct for d in dev])
    outs = [Guarded(2 * n) for n in shapes]
    ptrs = (E.c_void_p * 4)(*[o.ptr for o in outs])
    dx, dg, dn = Guarded(2048, x), Guarded(2048, gain), Guarded(2048)
    E.check(E.lib().es_q4_rmsnorm_matvec_multi(arr, 4, dx.ptr, dg.ptr, dn.ptr, ptrs, None))
    E.synchronize()
    u = O.rms_norm(x, gain)
    assert_bits_equal(dn.numpy(np.uint16, 1024), u, what="norm_out")
    for (c, s, b), o, n in zip(mats, outs, shapes):
        assert_bits_equal(o.numpy(np.uint16, n), O.q4_matvec(c, s, b, u), what=f"n={n}")
        o.check_guards(f"out n={n}")
    dn.check_guards("norm_out")


@pytest.mark.parametrize("scale", SCALES)
def test_audit_rmsnorm_gate_up_swiglu(scale):
    """Post RMSNorm + gate/up + SwiGLU: large activations reach the bf16
    sigmoid's saturated ends (+-88 and beyond)."""
    r = rng(7300 + int(scale * 1000))
    x = audit_vector(r, 1024, scale)
    gain = audit_vector(r, 1024, max(scale, 0.001), sigma=1.0)
    g = random_q4(r, 3584, 1024, scale_sigma=0.05)
    u = random_q4(r, 3584, 1024, scale_sigma=0.05)
    dG, dU = E.DeviceQ4(*g), E.DeviceQ4(*u)
    dx, dg = Guarded(2048, x), Guarded(2048, gain)
    dact, dn = Guarded(3584 * 2), Guarded(2048)
    E.check(E.lib().es_q4_rmsnorm_gate_up_swiglu(dG.struct, dU.struct, dx.ptr, dg.ptr, dn.ptr, dact.ptr, None))
    E.synchronize()
    un = O.rms_norm(x, gain)
    want = O.swiglu(O.q4_matvec(*g, un), O.q4_matvec(*u, un))
    assert_bits_equal(dn.numpy(np.uint16, 1024), un, what="norm_out")
    assert_bits_equal(dact.numpy(np.uint16, 3584), want, what="swiglu")
    dact.check_guards("act")
    dn.check_guards("norm_out")


@pytest.mark.parametrize("scale", SCALES)
def test_audit_gdn_recur_steps(scale):
    """Eight consecutive GDN decode steps (conv, q/k L2 norms, gates, delta
    rule) with scaled projections, gate inputs carrying +-88 (decay and beta
    saturated) and the state itself scaled: every readout, intermediate and
    the final state bit for bit, guards intact."""
    print(f"case audit gdn scale={scale}", flush=True)
    r = rng(7400 + int(scale * 1000))
    conv_w = bf16(r.normal(0, 0.5, (6144, 4)))
    a_log = (r.normal(0, 0.5, 16)).astype(np.float32)
    dt = bf16(r.normal(-1, 0.5, 16))
    state = (r.normal(0, 0.1, (16, 128, 128)) * max(scale, 0.001)).astype(np.float32)
    ostate = state.copy()
    hist = np.zeros((3, 6144), dtype=np.uint16)
    d_conv, d_alog, d_dt = Guarded(conv_w.nbytes, conv_w), Guarded(64, a_log), Guarded(32, dt)
    d_state = Guarded(state.nbytes, state)
    d_ring = Guarded(4 * 6144 * 2, np.zeros(4 * 6144, dtype=np.uint16))
    d_ab, d_y = Guarded(64), Guarded(4096)
    d_qkv, d_g, d_beta = Guarded(6144 * 2), Guarded(64), Guarded(32)
    for pos in range(8):
        raw = audit_vector(r, 6144, scale)
        ab = audit_vector(r, 32, max(scale, 1.0))
        d_ring.buf.upload(raw, offset=GUARD + (pos & 3) * 6144 * 2)
        d_ab.buf.upload(ab, offset=GUARD)
        E.check(E.lib().es_gdn_recur_step(d_ring.ptr, pos, d_conv.ptr, d_ab.ptr, d_alog.ptr, d_dt.ptr,
                                          d_state.ptr, d_y.ptr, d_qkv.ptr, d_g.ptr, d_beta.ptr, None))
        E.synchronize()
        conv, g, beta = O.gdn_conv_prepare(raw, hist, conv_w, ab[:16], ab[16:], a_log, dt)
        y = O.gdn_recur(conv, g, beta, ostate)
        assert_bits_equal(d_qkv.numpy(np.uint16, 6144), conv, what=f"qkv pos {pos}")
        assert_bits_equal(d_g.numpy(np.float32, 16), g, what=f"g pos {pos}")
        assert_bits_equal(d_beta.numpy(np.uint16, 16), beta, what=f"beta pos {pos}")
        assert_bits_equal(d_y.numpy(np.uint16, 2048), y, what=f"y pos {pos}")
    assert_bits_equal(d_state.numpy(np.float32, state.size), ostate.ravel(), what="state")
    for b, w in ((d_state, "state"), (d_ring, "ring"), (d_y, "y"), (d_qkv, "qkv"), (d_g, "g"), (d_beta, "beta"),
                 (d_ab, "ab"), (d_conv, "conv_w")):
        b.check_guards(w)


def attention_case(length, seed, mode, scale):
    """Inputs of one attention call. mode 'random': N(0,1) cache rows times
    scale; 'flat': every cached K row equal (all scores equal, so every
    running-max factor is exactly 1); 'wide': queries scaled so the scores
    span hundreds (most exponentials are exactly 0)."""
    r = rng(seed)
    cap = length + 8
    kc = audit_vector(r, 2 * cap * 256, scale).reshape(2, cap, 256)
    vc = audit_vector(r, 2 * cap * 256, max(scale, 0.001)).reshape(2, cap, 256)
    if mode == "flat":
        kc[:, :] = kc[:, :1]  # every cached K row of a KV head equal
    # q and k are RMS-normalised in the prologue: the query gain sets the
    # score range ('wide': gains of about 30, scores spanning hundreds)
    qg = bf16((30.0 if mode == "wide" else 1.0) * (1.0 + f32(audit_vector(r, 256, 1.0, sigma=0.1))))
    kg = bf16(1.0 + f32(audit_vector(r, 256, 1.0, sigma=0.1)))
    return dict(cap=cap, pos=length - 1, kc=kc, vc=vc, q=audit_vector(r, 4096, 1.0), k=audit_vector(r, 512, 1.0),
                v=audit_vector(r, 512, 1.0), qg=qg, kg=kg)


@pytest.mark.parametrize("mode,scale", [("random", 0.0), ("random", 0.001), ("random", 100.0), ("flat", 1.0),
                                        ("wide", 1.0)])
@pytest.mark.parametrize("length", [33, 1023, 1024, 5000])
def test_audit_attention(length, mode, scale):
    """Both routes (32 chains below 1024 attended positions, 64 chains from
    1024 on): gated output, query, the new K/V rows and the untouched cache
    rows bit for bit; guards intact around every output."""
    print(f"case audit attention length={length} mode={mode} scale={scale}", flush=True)
    x = attention_case(length, 7500 + length, mode, scale)
    cap, pos = x["cap"], x["pos"]
    d = {n: Guarded(x[n].nbytes, x[n]) for n in ("kc", "vc", "q", "k", "v", "qg", "kg")}
    f = Guarded(128, E.rope_inv_freq())
    sbytes = E.lib().es_attn_scratch_bytes(cap)
    scratch = Guarded(sbytes)
    gated, qout = Guarded(4096), Guarded(4096)
    E.check(E.lib().es_attn_decode(d["q"].ptr, d["k"].ptr, d["v"].ptr, d["qg"].ptr, d["kg"].ptr, d["kc"].ptr,
                                   d["vc"].ptr, cap, pos, f.ptr, E.splits_for(pos + 1), scratch.ptr, sbytes,
                                   gated.ptr, qout.ptr, None))
    E.synchronize()
    okc, ovc = x["kc"].copy(), x["vc"].copy()
    query = O.attn_prepare(x["q"], x["k"], x["v"], x["qg"], x["kg"], okc, ovc, pos, cap)
    want = O.attn_decode_gated(query, okc, ovc, pos + 1, cap, x["q"])
    kc = d["kc"].numpy(np.uint16, okc.size).reshape(okc.shape)
    vc = d["vc"].numpy(np.uint16, ovc.size).reshape(ovc.shape)
    assert_bits_equal(qout.numpy(np.uint16, 2048), query, what="query")
    assert np.array_equal(kc, okc), "K cache (new row bit for bit, other rows untouched)"
    assert np.array_equal(vc, ovc), "V cache (new row bit for bit, other rows untouched)"
    assert_bits_equal(gated.numpy(np.uint16, 2048), want, what="gated")
    for b, w in [(gated, "gated"), (qout, "query"), (scratch, "scratch")] + [(d[n], n) for n in d]:
        b.check_guards(w)


@pytest.mark.parametrize("scale", SCALES)
def test_audit_head_greedy(scale):
    """Final RMSNorm + tied head + LSE + greedy over the full vocabulary with
    the scaled hidden state (scale 0: the norm of zeros, logits from the
    biases alone): logits, LSE and token bit for bit; guards intact."""
    print(f"case audit head scale={scale}", flush=True)
    r = rng(7600 + int(scale * 1000))
    V = 248320
    table = random_q4(r, V, 1024)
    h = audit_vector(r, 1024, scale, sigma=2.0)
    gain = bf16(1.0 + f32(audit_vector(r, 1024, 1.0, sigma=0.1)))
    dT = E.DeviceQ4(*table)
    dh, dg = Guarded(2048, h), Guarded(2048, gain)
    logits, norm = Guarded(2 * V), Guarded(2048)
    sbytes = E.lib().es_head_scratch_bytes(V)
    scratch = Guarded(sbytes)
    tok, lse = Guarded(4), Guarded(4)
    E.check(E.lib().es_head_greedy(dT.struct, dh.ptr, dg.ptr, norm.ptr, logits.ptr, scratch.ptr, sbytes, tok.ptr,
                                   lse.ptr, None))
    E.synchronize()
    u = O.rms_norm(h, gain)
    lg = logits.numpy(np.uint16, V)
    assert_bits_equal(norm.numpy(np.uint16, 1024), u, what="final norm")
    assert_bits_equal(lg, O.q4_matvec(*table, u), what="logits")
    want_tok, want_lse = O.greedy(lg)
    assert float(lse.numpy(np.float32, 1)[0]) == want_lse
    assert int(tok.numpy(np.uint32, 1)[0]) == want_tok
    for b, w in ((logits, "logits"), (norm, "norm"), (scratch, "scratch"), (tok, "token"), (lse, "lse"),
                 (dh, "h"), (dg, "gain")):
        b.check_guards(w)


@pytest.mark.parametrize("gain_scale", [0.001, 10.0])
def test_audit_engine_steps_extreme_gains(gain_scale):
    """Decode steps of a 4-layer model on the XCD-cooperative kernels with
    every RMSNorm gain scaled (tiny or large activations through every
    fused kernel), prompt replayed token by token on the decode kernels:
    the greedy tokens and the teacher-forced logits of every step equal the
    oracle's decode steps bit for bit."""
    n_layers, vocab = 4, 4096
    blob = E.random_weights(n_layers, vocab, seed=77)
    views = E.tensor_views(blob, n_layers, vocab)
    for name, v in views.items():
        if name.endswith("layernorm.weight") or name.endswith("norm.weight"):
            v[...] = bf16(f32(v) * np.float32(gain_scale))
    eng = E.Engine(blob, n_layers, vocab, capacity=256)
    try:
        assert eng.xcd_kernels()
        eng.set_prefill(0)
        r = rng(7700)
        prompt = r.integers(0, vocab, 12).tolist()
        gen = eng.generate(prompt, 20, reset=True)
        forced = [gen[-1]] + r.integers(0, vocab, 5).tolist()
        am, lg = eng.forced_decode(forced, want_logits=True)
    finally:
        eng.close()
    orc = O.OracleModel(E.tensor_views(blob, n_layers, vocab), n_layers, vocab, capacity=256)
    want = orc.generate_stepwise(prompt, 20)
    assert gen == list(want)
    for i, t in enumerate(forced):
        tok, logits = orc.step(t, want_logits=True)
        assert_bits_equal(lg[i], logits, what=f"forced step {i} logits")
        assert int(am[i]) == tok

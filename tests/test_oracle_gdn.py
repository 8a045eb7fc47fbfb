"""The oracle's Gated DeltaNet decode step pinned by delta-rule invariants and
an fp64 recurrence (CPU). Reference arithmetic: gdn.metal:121-171 (conv +
prepare), gdn.metal:176-228 (recurrence, T=1), gdn.metal:230-255 (gated
RMSNorm).
"""
import numpy as np

import oracle as O
from helpers import assert_bf16_close, bf16, f32, rng

NH, DK = 16, 128


def conv_vec(q, k, v):
    """Recurrence input [6144] = q | k | v, each [16, 128] bf16."""
    return np.concatenate([q.ravel(), k.ravel(), v.ravel()]).astype(np.uint16)


def rand_qkv(r, scale=0.1):
    return (bf16(r.normal(0, scale, (NH, DK))), bf16(r.normal(0, scale, (NH, DK))),
            bf16(r.normal(0, 1, (NH, DK))))


def test_identity_gates_leave_state_and_read_it_out():
    """g = 1, beta = 0: the state is untouched bit for bit, y = bf16(S q)."""
    r = rng(20)
    q, k, v = rand_qkv(r)
    S = r.normal(0, 0.1, (NH, DK, DK)).astype(np.float32)
    S0 = S.copy()
    y = O.gdn_recur(conv_vec(q, k, v), np.ones(NH, np.float32), bf16(np.zeros(NH)), S)
    assert np.array_equal(S, S0)
    want = bf16(np.einsum("hvk,hk->hv", S0.astype(np.float64), f32(q).astype(np.float64)).astype(np.float32))
    assert_bf16_close(y, want.ravel(), max_ulp=1, max_frac=0.02, atol_rel=1e-4, what="readout")


def test_unit_key_writes_value_column():
    """beta = 1, g = 1, k = e_j: the delta rule replaces column j by v (up to
    the two fp32 roundings of S + (v - S)); other columns stay exact."""
    r = rng(21)
    q, _, v = rand_qkv(r)
    k = np.zeros((NH, DK), np.float32)
    j = 37
    k[:, j] = 1.0
    S = r.normal(0, 0.1, (NH, DK, DK)).astype(np.float32)
    S0 = S.copy()
    O.gdn_recur(conv_vec(q, bf16(k), v), np.ones(NH, np.float32), bf16(np.ones(NH)), S)
    others = np.ones(DK, bool)
    others[j] = False
    assert np.array_equal(S[:, :, others], S0[:, :, others])
    bound = 2.0**-23 * (np.abs(f32(v)) + np.abs(S0[:, :, j]))
    assert np.all(np.abs(S[:, :, j] - f32(v)) <= bound)


def test_pure_decay():
    """Zero q and k: S <- g S exactly (fp32 product), y = 0."""
    r = rng(22)
    z = bf16(np.zeros((NH, DK)))
    _, _, v = rand_qkv(r)
    g = r.uniform(0.5, 1.0, NH).astype(np.float32)
    S = r.normal(0, 0.1, (NH, DK, DK)).astype(np.float32)
    want = S * g[:, None, None]
    y = O.gdn_recur(conv_vec(z, z, v), g, bf16(np.full(NH, 0.5)), S)
    assert np.array_equal(S, want)
    assert np.all(f32(y) == 0)


def test_orthogonal_key_memory_is_zero():
    """State rows orthogonal to k: memory = 0, so S += k (v beta)."""
    r = rng(23)
    q, _, v = rand_qkv(r)
    k = np.zeros((NH, DK), np.float32)
    k[:, :64] = f32(bf16(r.normal(0, 0.1, (NH, 64))))
    S = np.zeros((NH, DK, DK), np.float32)
    S[:, :, 64:] = r.normal(0, 0.1, (NH, DK, 64))
    beta = bf16(np.full(NH, 0.75))
    S_new = S.copy()
    O.gdn_recur(conv_vec(q, bf16(k), v), np.ones(NH, np.float32), beta, S_new)
    want = S + k[:, None, :] * (f32(v)[:, :, None] * np.float32(0.75))
    assert np.allclose(S_new, want, rtol=2**-22, atol=2**-40)


def test_recurrence_fp64_over_steps():
    """Eight evolving steps against an fp64 delta rule fed the same inputs."""
    r = rng(24)
    S = r.normal(0, 0.1, (NH, DK, DK)).astype(np.float32)
    S64 = S.astype(np.float64)
    for _ in range(8):
        q, k, v = rand_qkv(r)
        g = r.uniform(0.8, 1.0, NH).astype(np.float32)
        beta = bf16(r.uniform(0, 1, NH))
        y = O.gdn_recur(conv_vec(q, k, v), g, beta, S)
        qd, kd, vd, bd = (f32(a).astype(np.float64) for a in (q, k, v, beta))
        S64 *= g[:, None, None].astype(np.float64)
        mem = np.einsum("hvk,hk->hv", S64, kd)
        delta = (vd - mem) * bd[:, None]
        S64 += delta[:, :, None] * kd[:, None, :]
        y64 = np.einsum("hvk,hk->hv", S64, qd)
        assert np.abs(S - S64).max() <= 1e-5 * np.abs(S64).max()
        assert_bf16_close(y, bf16(y64.astype(np.float32)).ravel(), max_ulp=1, max_frac=0.05, atol_rel=1e-3,
                          what="readout")


def test_conv_prepare_normalises_and_shifts_history():
    r = rng(25)
    raw = bf16(r.normal(0, 1, 6144))
    hist = bf16(r.normal(0, 1, (3, 6144)))
    hist0 = hist.copy()
    conv_w = bf16(r.normal(0, 0.2, (6144, 4)))
    a = bf16(r.normal(0, 1, NH))
    b = bf16(r.normal(0, 1, NH))
    a_log = r.uniform(-2, 2, NH).astype(np.float32)
    dt = bf16(r.normal(0, 1, NH))
    conv, g, beta = O.gdn_conv_prepare(raw, hist, conv_w, a, b, a_log, dt)
    # history shifts by one slot, newest last (gdn.metal:141-153)
    assert np.array_equal(hist[0], hist0[1]) and np.array_equal(hist[1], hist0[2])
    assert np.array_equal(hist[2], raw)
    # q rows have norm 128^-1/2, k rows norm 1 (bf16 rounding aside)
    qn = np.linalg.norm(f32(conv[:2048]).reshape(NH, DK), axis=1)
    kn = np.linalg.norm(f32(conv[2048:4096]).reshape(NH, DK), axis=1)
    assert np.allclose(qn, 128**-0.5, rtol=1e-2) and np.allclose(kn, 1.0, rtol=1e-2)
    # v: SiLU of the bf16 convolution, fp64 reference
    taps = np.stack([f32(hist0[0]), f32(hist0[1]), f32(hist0[2]), f32(raw)], axis=1).astype(np.float64)
    x = f32(bf16((taps * f32(conv_w)).sum(1).astype(np.float32))).astype(np.float64)
    silu = bf16((x / (1 + np.exp(-x))).astype(np.float32))
    assert_bf16_close(conv[4096:], silu[4096:], max_ulp=2, max_frac=0.6, atol_rel=1e-2, what="v conv")
    # gates: g = exp(-exp(A_log) softplus(a + dt)), beta = sigmoid_bf(b)
    ax = f32(bf16(f32(a) + f32(dt))).astype(np.float64)
    g64 = np.exp(-np.exp(a_log.astype(np.float64)) * np.log1p(np.exp(ax)))
    assert np.allclose(g, g64, rtol=2e-2)
    assert np.array_equal(f32(beta), np.array([O.lib().eo_sigmoid_bf(float(x)) for x in f32(b)], np.float32))


def test_norm_gate_fp64():
    r = rng(26)
    y = bf16(r.normal(0, 1, 2048))
    z = bf16(r.normal(0, 2, 2048))
    w = bf16(1 + 0.1 * r.normal(0, 1, 128))
    got = O.gdn_norm_gate(y, z, w)
    yd = f32(y).astype(np.float64).reshape(NH, DK)
    inv = 1.0 / np.sqrt((yd * yd).mean(1, keepdims=True) + 1e-6)
    nrm = f32(bf16((f32(bf16(yd * inv)).astype(np.float64) * f32(w)).astype(np.float32))).astype(np.float64)
    zd = f32(z).astype(np.float64).reshape(NH, DK)
    want = bf16((zd / (1 + np.exp(-zd)) * nrm).astype(np.float32)).ravel()
    assert_bf16_close(got, want, max_ulp=1, max_frac=0.05, atol_rel=1e-3, what="norm_gate")


def test_row_batched_gdn_equals_the_token_loop():
    """eo_gdn_conv_prepare_rows / eo_gdn_recur_rows / eo_gdn_norm_gate_rows
    (the oracle's batched forward) reorder the loops of the single-token
    functions without changing any operation: 37 tokens give the same bits as
    37 calls of each, history and state included."""
    r = rng(37)
    T = 37
    raw = bf16(r.normal(0, 1, (T, 6144)))
    hist = bf16(r.normal(0, 1, (3, 6144)))
    conv_w = bf16(r.normal(0, 0.5, (6144, 4)))
    a, b = bf16(r.normal(0, 1, (T, 16))), bf16(r.normal(0, 1, (T, 16)))
    a_log = r.uniform(-2, 2, 16).astype(np.float32)
    dt = bf16(r.normal(0.3, 0.5, 16))
    z = bf16(r.normal(0, 1, (T, 2048)))
    w = bf16(r.normal(1, 0.1, 128))
    state = r.normal(0, 0.1, (16, 128, 128)).astype(np.float32)
    h1, s1 = hist.copy(), state.copy()
    convs, gs, betas, ys, outs = [], [], [], [], []
    for t in range(T):
        c, g, be = O.gdn_conv_prepare(raw[t], h1, conv_w, a[t], b[t], a_log, dt)
        y = O.gdn_recur(c, g, be, s1)
        convs.append(c), gs.append(g), betas.append(be), ys.append(y)
        outs.append(O.gdn_norm_gate(y, z[t], w))
    h2, s2 = hist.copy(), state.copy()
    c2, g2, be2 = O.gdn_conv_prepare_rows(raw, h2, conv_w, a, b, a_log, dt)
    y2 = O.gdn_recur_rows(c2, g2, be2, s2)
    o2 = O.gdn_norm_gate_rows(y2, z, w)
    assert np.array_equal(c2, np.stack(convs)) and np.array_equal(be2, np.stack(betas))
    assert np.array_equal(g2.view(np.uint32), np.stack(gs).view(np.uint32))
    assert np.array_equal(y2, np.stack(ys)) and np.array_equal(o2, np.stack(outs))
    assert np.array_equal(h2, h1) and np.array_equal(s2.view(np.uint32), s1.view(np.uint32))

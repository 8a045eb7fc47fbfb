"""GPU parity of the prefill row operators (encode_forward with rows > 1,
model.rs:228-343) against the oracle's per-token operators.

Every row operator except attention evaluates its decode counterpart's fp32
operations in the same order for each row, so its outputs, the GDN state and
the KV cache rows must be bitwise equal to the oracle applied token by token.
The prefill attention takes its products on MFMA with the probabilities
rounded to bf16 (as the reference's attn_prefill does before its second
product), so it is compared with an fp64 softmax attention with the
tolerance stated in its test."""
import numpy as np
import pytest

import esdecode as E
import oracle as O
from helpers import assert_bits_equal, bf16, f32, random_q4, rng

pytestmark = pytest.mark.gpu


def test_embed_rows():
    r = rng(51)
    codes, scales, biases = random_q4(r, 600, 1024)
    toks = r.integers(0, 600, 37).astype(np.uint32)
    E_ = E.DeviceQ4(codes, scales, biases)
    dt = E.DeviceBuffer.from_numpy(toks)
    dh = E.DeviceBuffer(37 * 1024 * 2)
    E.check(E.lib().es_embed_rows(E_.struct, dt.ptr, 37, dh.ptr, None))
    E.synchronize()
    got = dh.numpy(np.uint16).reshape(37, 1024)
    for i, t in enumerate(toks):
        assert_bits_equal(got[i], O.embedding(codes, scales, biases, int(t)), what=f"row {i}")


@pytest.mark.parametrize("m", [1, 45])
def test_rmsnorm_rows(m):
    r = rng(52 + m)
    x = bf16(r.normal(0, 3, (m, 1024)))
    gain = bf16(r.normal(1, 0.2, 1024))
    dx, dg = E.DeviceBuffer.from_numpy(x), E.DeviceBuffer.from_numpy(gain)
    do = E.DeviceBuffer(m * 1024 * 2)
    E.check(E.lib().es_rmsnorm_rows(dx.ptr, dg.ptr, m, do.ptr, None))
    E.synchronize()
    got = do.numpy(np.uint16).reshape(m, 1024)
    for i in range(m):
        assert_bits_equal(got[i], O.rms_norm(x[i], gain), what=f"row {i}")


def test_swiglu_rows():
    r = rng(53)
    n = 7 * 3584 + 5
    g, u = bf16(r.normal(0, 3, n)), bf16(r.normal(0, 2, n))
    dg, du = E.DeviceBuffer.from_numpy(g), E.DeviceBuffer.from_numpy(u)
    do = E.DeviceBuffer(n * 2)
    E.check(E.lib().es_swiglu_rows(dg.ptr, du.ptr, n, do.ptr, None))
    E.synchronize()
    assert_bits_equal(do.numpy(np.uint16), O.swiglu(g, u), what="swiglu")


class GdnInputs:
    def __init__(self, r, pos0, m):
        self.pos0, self.m = pos0, m
        self.raw = bf16(r.normal(0, 1, (m, 6144)))
        self.a = bf16(r.normal(0, 1, (m, 16)))
        self.b = bf16(r.normal(0, 1, (m, 16)))
        self.conv_w = bf16(r.normal(0, 0.5, (6144, 4)))
        self.a_log = r.normal(0, 0.5, 16).astype(np.float32)
        self.dt = bf16(r.normal(0, 0.5, 16))
        # ring slots of positions pos0-4 .. pos0-1; positions before 0 are zero
        self.ring = np.zeros((4, 6144), dtype=np.uint16)
        for p in range(pos0 - 4, pos0):
            if p >= 0:
                self.ring[p & 3] = bf16(r.normal(0, 1, 6144))

    def history(self):
        h = np.zeros((3, 6144), dtype=np.uint16)
        for i, p in enumerate(range(self.pos0 - 3, self.pos0)):
            if p >= 0:
                h[i] = self.ring[p & 3]
        return h


@pytest.mark.parametrize("pos0,m", [(0, 1), (0, 3), (2, 5), (1001, 70), (7, 2)])
def test_gdn_prepare_rows(pos0, m):
    print(f"case gdn_prepare_rows pos0={pos0} m={m}", flush=True)
    x = GdnInputs(rng(60 + pos0 + m), pos0, m)
    d = {k: E.DeviceBuffer.from_numpy(getattr(x, k)) for k in ("raw", "a", "b", "conv_w", "a_log", "dt", "ring")}
    dq, dk, dv = (E.DeviceBuffer(m * 2048 * 2) for _ in range(3))
    dg, dbeta = E.DeviceBuffer(m * 64), E.DeviceBuffer(m * 64)
    E.check(E.lib().es_gdn_prepare_rows(d["raw"].ptr, d["ring"].ptr, d["conv_w"].ptr, d["a"].ptr, d["b"].ptr,
                                        d["a_log"].ptr, d["dt"].ptr, pos0, m, dq.ptr, dk.ptr, dv.ptr, dg.ptr,
                                        dbeta.ptr, None))
    E.synchronize()
    q, k, v = (b.numpy(np.uint16).reshape(m, 2048) for b in (dq, dk, dv))
    g, beta = dg.numpy(np.float32).reshape(m, 16), dbeta.numpy(np.float32).reshape(m, 16)
    hist = x.history()
    for t in range(m):
        conv, og, obeta = O.gdn_conv_prepare(x.raw[t], hist, x.conv_w, x.a[t], x.b[t], x.a_log, x.dt)
        assert_bits_equal(q[t], conv[:2048], what=f"q row {t}")
        assert_bits_equal(k[t], conv[2048:4096], what=f"k row {t}")
        assert_bits_equal(v[t], conv[4096:], what=f"v row {t}")
        assert_bits_equal(g[t], og, what=f"g row {t}")
        assert_bits_equal(beta[t], f32(obeta), what=f"beta row {t}")
    # the ring now holds the raw rows of the last four positions (gdn_history)
    ring = d["ring"].numpy(np.uint16).reshape(4, 6144)
    want = x.ring.copy()
    for t in range(max(0, m - 4), m):
        want[(pos0 + t) & 3] = x.raw[t]
    assert_bits_equal(ring, want, what="ring after the chunk")


@pytest.mark.parametrize("m", [1, 33, 100, 257])
def test_gdn_recur_rows(m):
    print(f"case gdn_recur_rows m={m}", flush=True)
    r = rng(70 + m)
    # q, k as the preparation leaves them (unit rows scaled), v, gates in range
    qk = r.normal(0, 1, (2, m, 16, 128))
    qk /= np.linalg.norm(qk, axis=-1, keepdims=True)
    q = bf16(qk[0] * 0.0078125).reshape(m, 2048)
    k = bf16(qk[1] * 128 ** -0.5).reshape(m, 2048)
    v = bf16(r.normal(0, 1, (m, 2048)))
    g = np.exp(-r.uniform(0.01, 1.5, (m, 16))).astype(np.float32)
    beta_bf = bf16(1 / (1 + np.exp(-r.normal(0, 1, (m, 16)))))
    state0 = r.normal(0, 0.1, (16, 128, 128)).astype(np.float32)
    d = [E.DeviceBuffer.from_numpy(a) for a in (q, k, v, g, f32(beta_bf), state0)]
    dy = E.DeviceBuffer(m * 2048 * 2)
    E.check(E.lib().es_gdn_recur_rows(d[0].ptr, d[1].ptr, d[2].ptr, d[3].ptr, d[4].ptr, m, d[5].ptr, dy.ptr, None))
    E.synchronize()
    y = dy.numpy(np.uint16).reshape(m, 2048)
    st = state0.copy()
    for t in range(m):
        conv = np.concatenate([q[t], k[t], v[t]])
        assert_bits_equal(y[t], O.gdn_recur(conv, g[t], beta_bf[t], st), what=f"y row {t}")
    assert_bits_equal(d[5].numpy(np.float32).reshape(16, 128, 128), st, what="state after the chunk")


def test_gdn_norm_gate_rows():
    r = rng(80)
    m = 19
    y, z = bf16(r.normal(0, 1, (m, 2048))), bf16(r.normal(0, 2, (m, 2048)))
    w = bf16(r.normal(1, 0.2, 128))
    d = [E.DeviceBuffer.from_numpy(a) for a in (y, z, w)]
    do = E.DeviceBuffer(m * 2048 * 2)
    E.check(E.lib().es_gdn_norm_gate_rows(d[0].ptr, d[1].ptr, d[2].ptr, m, do.ptr, None))
    E.synchronize()
    got = do.numpy(np.uint16).reshape(m, 2048)
    for t in range(m):
        assert_bits_equal(got[t], O.gdn_norm_gate(y[t], z[t], w), what=f"row {t}")


@pytest.mark.parametrize("pos0,m", [(0, 1), (0, 40), (517, 9)])
def test_attn_prepare_rows(pos0, m):
    r = rng(90 + pos0 + m)
    cap = 640
    qp = bf16(r.normal(0, 1, (m, 4096)))
    kp, vp = bf16(r.normal(0, 1, (m, 512))), bf16(r.normal(0, 1, (m, 512)))
    qg, kg = bf16(r.normal(1, 0.2, 256)), bf16(r.normal(1, 0.2, 256))
    kc0, vc0 = bf16(r.normal(0, 1, (2, cap, 256))), bf16(r.normal(0, 1, (2, cap, 256)))
    d = [E.DeviceBuffer.from_numpy(a) for a in (qp, kp, vp, qg, kg, E.rope_inv_freq(), kc0, vc0)]
    dquery = E.DeviceBuffer(m * 2048 * 2)
    E.check(E.lib().es_attn_prepare_rows(d[0].ptr, d[1].ptr, d[2].ptr, d[3].ptr, d[4].ptr, d[5].ptr, pos0, m,
                                         dquery.ptr, d[6].ptr, d[7].ptr, cap, None))
    E.synchronize()
    query = dquery.numpy(np.uint16).reshape(m, 2048)
    okc, ovc = kc0.copy(), vc0.copy()
    for t in range(m):
        want = O.attn_prepare(qp[t], kp[t], vp[t], qg, kg, okc, ovc, pos0 + t, cap)
        assert_bits_equal(query[t], want, what=f"query row {t}")
    assert_bits_equal(d[6].numpy(np.uint16).reshape(2, cap, 256), okc, what="K cache")
    assert_bits_equal(d[7].numpy(np.uint16).reshape(2, cap, 256), ovc, what="V cache")


def attention_f64(query, kc, vc, pos0, m):
    """Causal GQA softmax attention in fp64 over bf16 inputs: [m, 8, 256]."""
    qf = f32(query).astype(np.float64).reshape(m, 8, 256)
    K, V = f32(kc).astype(np.float64), f32(vc).astype(np.float64)
    out = np.empty((m, 8, 256))
    for t in range(m):
        n = pos0 + t + 1
        for h in range(8):
            s = K[h // 4, :n] @ qf[t, h] / 16.0
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ V[h // 4, :n]
    return out


@pytest.mark.parametrize("pos0,m", [(0, 1), (0, 37), (5, 64), (100, 130), (1000, 65), (31, 33)])
def test_attn_prefill(pos0, m):
    """Tolerance: the probabilities enter the second product as bf16 (relative
    error <= 2^-9 each) and the output is rounded to bf16, so an element may
    differ from the fp64 result by 2^-8 * max|V| over the attended rows plus
    one bf16 ulp of the result; the mean error must stay 8x below that."""
    print(f"case attn_prefill pos0={pos0} m={m}", flush=True)
    r = rng(100 + pos0 + m)
    cap = pos0 + m + 3
    # scores of a useful spread: q.k/16 with unit-ish rows of norm 16
    query = bf16(r.normal(0, 1, (m, 2048)))
    kc, vc = bf16(r.normal(0, 1, (2, cap, 256))), bf16(r.normal(0, 1, (2, cap, 256)))
    d = [E.DeviceBuffer.from_numpy(a) for a in (query, kc, vc)]
    do = E.DeviceBuffer(m * 2048 * 2)
    E.check(E.lib().es_attn_prefill(d[0].ptr, d[1].ptr, d[2].ptr, pos0, m, cap, do.ptr, None))
    E.synchronize()
    got = f32(do.numpy(np.uint16)).astype(np.float64).reshape(m, 8, 256)
    want = attention_f64(query, kc, vc, pos0, m)
    vmax = np.abs(f32(vc)).max()
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 1e-30))) - 7)
    err = np.abs(got - want)
    bound = 2.0 ** -8 * vmax + ulp
    assert np.all(err <= bound), f"max excess {np.max(err - bound)} at {np.unravel_index(np.argmax(err - bound), err.shape)}"
    assert err.mean() <= 2.0 ** -11 * vmax, f"mean error {err.mean()}"


def test_attn_prefill_first_row_is_the_first_value_row():
    """The first row of a chunk at position 0 attends to one key: its output is
    that key's V row exactly (softmax of one score is 1)."""
    r = rng(110)
    cap = 64
    query = bf16(r.normal(0, 1, (4, 2048)))
    kc, vc = bf16(r.normal(0, 1, (2, cap, 256))), bf16(r.normal(0, 1, (2, cap, 256)))
    d = [E.DeviceBuffer.from_numpy(a) for a in (query, kc, vc)]
    do = E.DeviceBuffer(4 * 2048 * 2)
    E.check(E.lib().es_attn_prefill(d[0].ptr, d[1].ptr, d[2].ptr, 0, 4, cap, do.ptr, None))
    E.synchronize()
    got = do.numpy(np.uint16).reshape(4, 8, 256)
    for h in range(8):
        assert_bits_equal(got[0, h], vc[h // 4, 0], what=f"head {h}")


def test_attn_gate_rows():
    r = rng(120)
    m = 21
    o, qp = bf16(r.normal(0, 1, (m, 2048))), bf16(r.normal(0, 2, (m, 4096)))
    d = [E.DeviceBuffer.from_numpy(a) for a in (o, qp)]
    dg = E.DeviceBuffer(m * 2048 * 2)
    E.check(E.lib().es_attn_gate_rows(d[0].ptr, d[1].ptr, m, dg.ptr, None))
    E.synchronize()
    got = dg.numpy(np.uint16).reshape(m, 2048)
    for t in range(m):
        assert_bits_equal(got[t], O.attn_gate(o[t], qp[t]), what=f"row {t}")


def test_row_ops_reject_bad_arguments():
    b = E.DeviceBuffer(1 << 16)
    L = E.lib()
    assert L.es_rmsnorm_rows(b.ptr, b.ptr, 0, b.ptr, None) != E.ES_OK
    assert L.es_attn_prefill(b.ptr, b.ptr, b.ptr, 10, 8, 16, b.ptr, None) != E.ES_OK
    assert L.es_attn_prefill(b.ptr, b.ptr, b.ptr, -1, 1, 16, b.ptr, None) != E.ES_OK
    # a KV head's rows are addressed by 32-bit byte offsets: capacity at most 2^22
    assert L.es_attn_prefill(b.ptr, b.ptr, b.ptr, 0, 1, (1 << 22) + 1, b.ptr, None) != E.ES_OK
    assert L.es_attn_prepare_rows(b.ptr, b.ptr, b.ptr, b.ptr, b.ptr, b.ptr, 9, 8, b.ptr, b.ptr, b.ptr, 16,
                                  None) != E.ES_OK
    assert L.es_gdn_recur_rows(b.ptr, b.ptr, b.ptr, b.ptr, b.ptr, 0, b.ptr, b.ptr, None) != E.ES_OK

"""GPU parity of the Q4 linear ops against the oracle (qmv_q4 family,
linear.metal:11-123, linear_input_norm.metal, linear_norm.metal).

The kernels and the oracle evaluate the same fp32 operations in the same
order, so outputs (bf16 and the fp32 pre-round sums) must be bitwise equal.
"""
import numpy as np
import pytest

import esdecode as E
import oracle as O
from helpers import assert_bits_equal, bf16, f32, random_q4, rng

pytestmark = pytest.mark.gpu

# isolated QMV shapes of the benchmark plus ragged tails
SHAPES = [(3584, 1024), (1024, 3584), (6144, 1024), (248320, 1024), (1024, 2048), (1000, 1024),
          (1000, 2048), (16, 1024), (5, 3584)]


@pytest.mark.parametrize("n,k", SHAPES)
def test_q4_matvec(n, k):
    print(f"case q4_matvec n={n} k={k}", flush=True)
    r = rng(1000 + n + k)
    codes, scales, biases = random_q4(r, n, k)
    x = bf16(r.normal(0, 1, k))
    W = E.DeviceQ4(codes, scales, biases)
    dx = E.DeviceBuffer.from_numpy(x)
    dy = E.DeviceBuffer(n * 2)
    dyf = E.DeviceBuffer(n * 4)
    E.check(E.lib().es_q4_matvec(W.struct, dx.ptr, dy.ptr, dyf.ptr, None))
    E.synchronize()
    y, yf = dy.numpy(np.uint16), dyf.numpy(np.float32)
    wy, wyf = O.q4_matvec(codes, scales, biases, x, want_f32=True)
    assert_bits_equal(yf, wyf, what=f"qmv fp32 {n}x{k}")
    assert_bits_equal(y, wy, what=f"qmv {n}x{k}")


@pytest.mark.parametrize("k", [1024, 2048, 3584])
def test_q4_matvec_add_inplace(k):
    r = rng(7 + k)
    n = 1024
    codes, scales, biases = random_q4(r, n, k)
    x = bf16(r.normal(0, 1, k))
    res = bf16(r.normal(0, 1, n))
    W = E.DeviceQ4(codes, scales, biases)
    dx = E.DeviceBuffer.from_numpy(x)
    dh = E.DeviceBuffer.from_numpy(res)
    E.check(E.lib().es_q4_matvec_add(W.struct, dx.ptr, dh.ptr, dh.ptr, None))  # y aliases residual
    E.synchronize()
    want = O.q4_matvec_add(codes, scales, biases, x, res)
    assert_bits_equal(dh.numpy(np.uint16), want, what=f"qmv_add k={k}")


def test_matvec_rejects_bad_shapes():
    r = rng(3)
    codes, scales, biases = random_q4(r, 8, 512)
    W = E.DeviceQ4(codes, scales, biases)
    dx = E.DeviceBuffer(1024)
    dy = E.DeviceBuffer(64)
    rc = E.lib().es_q4_matvec(W.struct, dx.ptr, dy.ptr, None, None)
    assert rc == E.ES_ERR_INVALID


def test_rmsnorm_multi_gdn_projections():
    """RMSNorm(x)*gain feeding qkv/z/a/b (gdn_input_g16 projections)."""
    r = rng(11)
    x = bf16(r.normal(0, 1, 1024) * 3.0)
    gain = bf16(1 + 0.1 * r.normal(0, 1, 1024))
    shapes = [6144, 2048, 16, 16]
    mats = [random_q4(r, n, 1024) for n in shapes]
    dev = [E.DeviceQ4(*m) for m in mats]
    arr = (E.Q4 * 4)(*[d.struct for d in dev])
    outs = [E.DeviceBuffer(n * 2) for n in shapes]
    ptrs = (E.c_void_p * 4)(*[o.ptr for o in outs])
    dx = E.DeviceBuffer.from_numpy(x)
    dg = E.DeviceBuffer.from_numpy(gain)
    dn = E.DeviceBuffer(2048)
    E.check(E.lib().es_q4_rmsnorm_matvec_multi(arr, 4, dx.ptr, dg.ptr, dn.ptr, ptrs, None))
    E.synchronize()
    u = O.rms_norm(x, gain)
    assert_bits_equal(dn.numpy(np.uint16), u, what="norm_out")
    for (c, s, b), o, n in zip(mats, outs, shapes):
        assert_bits_equal(o.numpy(np.uint16), O.q4_matvec(c, s, b, u), what=f"multi n={n}")


def test_rmsnorm_multi_rejects_row_count_not_multiple_of_8():
    """A wave's 8 rows must lie in one matrix, so every row count is a multiple of 8."""
    r = rng(13)
    mats = [random_q4(r, n, 1024) for n in (16, 12)]
    dev = [E.DeviceQ4(*m) for m in mats]
    arr = (E.Q4 * 2)(*[d.struct for d in dev])
    outs = [E.DeviceBuffer(n * 2) for n in (16, 12)]
    ptrs = (E.c_void_p * 2)(*[o.ptr for o in outs])
    dx = E.DeviceBuffer.from_numpy(bf16(r.normal(0, 1, 1024)))
    dg = E.DeviceBuffer.from_numpy(bf16(np.ones(1024)))
    rc = E.lib().es_q4_rmsnorm_matvec_multi(arr, 2, dx.ptr, dg.ptr, None, ptrs, None)
    assert rc == E.ES_ERR_INVALID


def test_gdn_in_proj_ring_slot():
    r = rng(12)
    x = bf16(r.normal(0, 1, 1024))
    gain = bf16(1 + 0.1 * r.normal(0, 1, 1024))
    mats = [random_q4(r, n, 1024) for n in (6144, 2048, 16, 16)]
    dev = [E.DeviceQ4(*m) for m in mats]
    ring = E.DeviceBuffer.zeros(4 * 6144 * 2)
    dz = E.DeviceBuffer(2048 * 2)
    dab = E.DeviceBuffer(32 * 2)
    dx = E.DeviceBuffer.from_numpy(x)
    dg = E.DeviceBuffer.from_numpy(gain)
    pos = 7
    E.check(E.lib().es_gdn_in_proj(dev[0].struct, dev[1].struct, dev[2].struct, dev[3].struct, dx.ptr, dg.ptr,
                                   None, ring.ptr, pos, dz.ptr, dab.ptr, None))
    E.synchronize()
    u = O.rms_norm(x, gain)
    rg = ring.numpy(np.uint16).reshape(4, 6144)
    assert_bits_equal(rg[pos & 3], O.q4_matvec(*mats[0], u), what="qkv slot")
    for s in range(4):
        if s != (pos & 3):
            assert not rg[s].any(), "only the position's slot may be written"
    assert_bits_equal(dz.numpy(np.uint16), O.q4_matvec(*mats[1], u), what="z")
    ab = dab.numpy(np.uint16)
    assert_bits_equal(ab[:16], O.q4_matvec(*mats[2], u), what="a")
    assert_bits_equal(ab[16:], O.q4_matvec(*mats[3], u), what="b")


def test_rmsnorm_gate_up_swiglu():
    r = rng(13)
    x = bf16(r.normal(0, 1, 1024))
    gain = bf16(1 + 0.1 * r.normal(0, 1, 1024))
    g = random_q4(r, 3584, 1024, scale_sigma=0.05)
    u = random_q4(r, 3584, 1024, scale_sigma=0.05)
    dG, dU = E.DeviceQ4(*g), E.DeviceQ4(*u)
    dx, dg = E.DeviceBuffer.from_numpy(x), E.DeviceBuffer.from_numpy(gain)
    dact = E.DeviceBuffer(3584 * 2)
    dn = E.DeviceBuffer(2048)
    E.check(E.lib().es_q4_rmsnorm_gate_up_swiglu(dG.struct, dU.struct, dx.ptr, dg.ptr, dn.ptr, dact.ptr, None))
    E.synchronize()
    un = O.rms_norm(x, gain)
    want = O.swiglu(O.q4_matvec(*g, un), O.q4_matvec(*u, un))
    assert_bits_equal(dn.numpy(np.uint16), un, what="norm_out")
    assert_bits_equal(dact.numpy(np.uint16), want, what="swiglu")


def test_embedding_bit_exact():
    r = rng(14)
    table = random_q4(r, 4096, 1024)
    dT = E.DeviceQ4(*table)
    for tok in (0, 1, 2047, 4095):
        dt = E.DeviceBuffer.from_numpy(np.array([tok], dtype=np.uint32))
        do = E.DeviceBuffer(2048)
        E.check(E.lib().es_embedding_q4(dT.struct, dt.ptr, do.ptr, None))
        E.synchronize()
        assert np.array_equal(do.numpy(np.uint16), O.embedding(*table, tok))

"""GPU parity of the batched prefill kernels (encode_forward with rows > 1,
model.rs:228-350) against the oracle's restatements. The prefill GEMM
accumulates in fp32 on MFMA in its own order, so its bf16 outputs agree with
the oracle's fp64 sums to within one bf16 ulp on the few elements whose fp32
value lies at a rounding boundary (tolerance stated per test)."""
import numpy as np
import pytest

import esdecode as E
import oracle as O
from helpers import assert_bf16_close, bf16, f32, random_q4, rng

pytestmark = pytest.mark.gpu

# N >= 2048 (K a multiple of 128) takes the 256 x 256 tiles, the rest the 128 x 128 tiles
GEMM_SHAPES = [(1, 16, 1024), (17, 1024, 1024), (128, 128, 64), (300, 6144, 1024), (257, 1024, 3584),
               (2048, 512, 1024), (64, 1000, 2048), (130, 16, 1024), (1, 2048, 1024), (513, 2304, 1024),
               (257, 2048, 3584), (600, 4096, 2048)]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_q4_gemm(m, n, k):
    print(f"case q4_gemm m={m} n={n} k={k}", flush=True)
    r = rng(2000 + m + n + k)
    codes, scales, biases = random_q4(r, n, k)
    x = bf16(r.normal(0, 1, (m, k)))
    W = E.DeviceQ4(codes, scales, biases)
    dx = E.DeviceBuffer.from_numpy(x)
    dy = E.DeviceBuffer(m * n * 2)
    E.check(E.lib().es_q4_gemm(W.struct, dx.ptr, m, None, dy.ptr, None))
    E.synchronize()
    got = dy.numpy(np.uint16).reshape(m, n)
    want = O.q4_gemm(codes, scales, biases, x)
    # tolerance: fp32 accumulation order only; <= 1 bf16 ulp on <= 1% of outputs
    assert_bf16_close(got, want, max_ulp=1, max_frac=0.01, what=f"gemm {m}x{n}x{k}")


@pytest.mark.parametrize("k", [1024, 3584])
def test_q4_gemm_residual_in_place(k):
    r = rng(3000 + k)
    m, n = 200, 1024
    codes, scales, biases = random_q4(r, n, k)
    x = bf16(r.normal(0, 1, (m, k)))
    res = bf16(r.normal(0, 1, (m, n)))
    W = E.DeviceQ4(codes, scales, biases)
    dx = E.DeviceBuffer.from_numpy(x)
    dh = E.DeviceBuffer.from_numpy(res)
    E.check(E.lib().es_q4_gemm(W.struct, dx.ptr, m, dh.ptr, dh.ptr, None))  # y aliases residual
    E.synchronize()
    want = O.q4_gemm(codes, scales, biases, x, residual=res)
    got = dh.numpy(np.uint16).reshape(m, n)
    # tolerance: one bf16 ulp of the GEMM term (the residual add after it can
    # cancel, so a 1-ulp difference there is many ulps of the sum) plus one
    # ulp of the sum; at most 1% of the outputs differ
    y = f32(O.q4_gemm(codes, scales, biases, x)).astype(np.float64)
    sum_ = f32(want).astype(np.float64)
    ulp = lambda v: 2.0 ** (np.floor(np.log2(np.maximum(np.abs(v), 1e-30))) - 7)
    d = np.abs(f32(got).astype(np.float64) - sum_)
    assert np.all(d <= ulp(y) + ulp(sum_)), f"gemm add k={k}: max excess {np.max(d - ulp(y) - ulp(sum_))}"
    assert np.mean(got != want) <= 0.01


@pytest.mark.parametrize("m,k", [(1, 1024), (300, 1024), (513, 3584)])
def test_wide_gemm_equals_narrow_tiles(m, k):
    """An N = 2048 GEMM (256 x 256 tiles) and its two 1024-row halves as
    separate GEMMs (128 x 128 tiles) give the same bits: every output element
    is the same chain of MFMAs over K in both."""
    print(f"case wide vs narrow m={m} k={k}", flush=True)
    r = rng(7000 + m + k)
    n = 2048
    codes, scales, biases = random_q4(r, n, k)
    x = bf16(r.normal(0, 1, (m, k)))
    W = E.DeviceQ4(codes, scales, biases)
    halves = [E.DeviceQ4(codes[h * 1024:(h + 1) * 1024], scales[h * 1024:(h + 1) * 1024],
                         biases[h * 1024:(h + 1) * 1024]) for h in range(2)]
    dx = E.DeviceBuffer.from_numpy(x)
    dy = E.DeviceBuffer(m * n * 2)
    dh = [E.DeviceBuffer(m * 1024 * 2) for _ in range(2)]
    E.check(E.lib().es_q4_gemm(W.struct, dx.ptr, m, None, dy.ptr, None))
    for h in range(2):
        E.check(E.lib().es_q4_gemm(halves[h].struct, dx.ptr, m, None, dh[h].ptr, None))
    E.synchronize()
    full = dy.numpy(np.uint16).reshape(m, n)
    for h in range(2):
        assert np.array_equal(full[:, h * 1024:(h + 1) * 1024], dh[h].numpy(np.uint16).reshape(m, 1024))


def test_q4_gemm_rejects_bad_arguments():
    r = rng(4)
    codes, scales, biases = random_q4(r, 8, 64)
    W = E.DeviceQ4(codes, scales, biases)
    dx = E.DeviceBuffer(4096)
    dy = E.DeviceBuffer(4096)
    assert E.lib().es_q4_gemm(W.struct, dx.ptr, 0, None, dy.ptr, None) != E.ES_OK
    assert E.lib().es_q4_gemm(W.struct, dx.ptr, 1, None, dx.ptr, None) != E.ES_OK


@pytest.mark.parametrize("m", [1, 130, 257])
def test_gemm_swiglu_equals_two_gemms_and_swiglu(m):
    """The fused gate/up GEMM with the SwiGLU epilogue gives, bit for bit,
    es_q4_gemm on gate and on up followed by es_swiglu_rows."""
    print(f"case gemm swiglu m={m}", flush=True)
    r = rng(6000 + m)
    n, k = 3584, 1024
    G = E.DeviceQ4(*random_q4(r, n, k))
    U = E.DeviceQ4(*random_q4(r, n, k))
    x = bf16(r.normal(0, 1, (m, k)))
    dx = E.DeviceBuffer.from_numpy(x)
    dg, du, da, df = (E.DeviceBuffer(m * n * 2) for _ in range(4))
    E.check(E.lib().es_q4_gemm(G.struct, dx.ptr, m, None, dg.ptr, None))
    E.check(E.lib().es_q4_gemm(U.struct, dx.ptr, m, None, du.ptr, None))
    E.check(E.lib().es_swiglu_rows(dg.ptr, du.ptr, m * n, da.ptr, None))
    E.check(E.lib().es_q4_gemm_swiglu(G.struct, U.struct, dx.ptr, m, df.ptr, None))
    E.synchronize()
    assert np.array_equal(da.numpy(np.uint16), df.numpy(np.uint16))

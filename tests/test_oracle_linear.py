"""The oracle's Q4 matvec, embedding, RMSNorm and SwiGLU pinned against
closed forms and fp64 brute force (CPU). Reference arithmetic:
linear.metal:11-123 (MLX affine Q4, group 64), linear.metal:300-331
(rms_norm_bf16), linear.metal:382-396 (swiglu_bf16).
"""
import numpy as np
import pytest

import oracle as O
from helpers import assert_bf16_close, bf16, dequant_f64, f32, random_q4, rng


@pytest.mark.parametrize("k", [1024, 2048, 3584])
def test_qmv_matches_fp64_dequant_then_dot(k):
    r = rng(10 + k)
    codes, scales, biases = random_q4(r, 96, k)
    x = bf16(r.normal(0, 1, k))
    y, yf = O.q4_matvec(codes, scales, biases, x, want_f32=True)
    want = dequant_f64(codes, scales, biases) @ f32(x).astype(np.float64)
    # fp32 accumulation of k terms: relative to the sum of magnitudes
    mag = np.abs(dequant_f64(codes, scales, biases)) @ np.abs(f32(x).astype(np.float64))
    assert np.all(np.abs(yf - want) <= 8 * k * 2.0**-24 * mag)
    assert np.array_equal(y, bf16(yf)), "output is the bf16 rounding of the fp32 sum"


def test_qmv_zero_codes_is_bias_times_group_sums():
    """All-zero codes: y = sum_g b_g * sum(x_g)."""
    r = rng(11)
    k = 1024
    codes = np.zeros((16, k // 8), dtype=np.uint32)
    scales = bf16(np.abs(r.normal(0, 0.02, (16, k // 64))))
    biases = bf16(r.normal(0, 0.01, (16, k // 64)))
    x = bf16(r.normal(0, 1, k))
    _, yf = O.q4_matvec(codes, scales, biases, x, want_f32=True)
    gs = f32(x).astype(np.float64).reshape(-1, 64).sum(1)
    want = f32(biases).astype(np.float64) @ gs
    mag = np.abs(f32(biases).astype(np.float64)) @ np.abs(f32(x).astype(np.float64)).reshape(-1, 64).sum(1)
    assert np.all(np.abs(yf - want) <= 4 * k * 2.0**-24 * mag)


def test_qmv_integer_dot_is_exact():
    """Unit scales, zero biases, small-integer x: every fp32 step is exact, so
    the result equals the integer dot product bit for bit."""
    r = rng(12)
    for k in (1024, 2048, 3584):
        codes = r.integers(0, 2**32, size=(32, k // 8), dtype=np.uint64).astype(np.uint32)
        scales = bf16(np.ones((32, k // 64)))
        biases = bf16(np.zeros((32, k // 64)))
        x = bf16(r.integers(-8, 9, k).astype(np.float32))
        y, yf = O.q4_matvec(codes, scales, biases, x, want_f32=True)
        shifts = np.arange(8, dtype=np.uint32) * 4
        q = ((codes[:, :, None] >> shifts) & 15).reshape(32, k).astype(np.int64)
        want = q @ f32(x).astype(np.int64)
        assert np.array_equal(yf.astype(np.int64), want)


def test_qmv_linearity_in_x():
    r = rng(13)
    codes, scales, biases = random_q4(r, 64, 2048)
    x1 = bf16(r.integers(-64, 64, 2048) / 64.0)
    x2 = bf16(r.integers(-64, 64, 2048) / 64.0)
    x12 = bf16(f32(x1) + f32(x2))
    assert np.array_equal(f32(x12), f32(x1) + f32(x2)), "sum stays exact in bf16"
    _, y1 = O.q4_matvec(codes, scales, biases, x1, want_f32=True)
    _, y2 = O.q4_matvec(codes, scales, biases, x2, want_f32=True)
    _, y12 = O.q4_matvec(codes, scales, biases, x12, want_f32=True)
    mag = np.abs(dequant_f64(codes, scales, biases)) @ (np.abs(f32(x1)) + np.abs(f32(x2))).astype(np.float64)
    assert np.all(np.abs(y12 - (y1.astype(np.float64) + y2)) <= 16 * 2048 * 2.0**-24 * mag)


def test_qmv_add_is_residual_plus_rounded_product():
    """qmv_add: y = bf16(residual + bf16(W x)) (linear.metal:77-123)."""
    r = rng(14)
    codes, scales, biases = random_q4(r, 1024, 3584)
    x = bf16(r.normal(0, 1, 3584))
    res = bf16(r.normal(0, 1, 1024))
    y = O.q4_matvec(codes, scales, biases, x)
    got = O.q4_matvec_add(codes, scales, biases, x, res)
    assert np.array_equal(got, bf16(f32(res) + f32(y)))


def test_embedding_is_exact_dequantised_row():
    """bf16(s*q + b): s*q is exact, one rounding to fp32, one to bf16."""
    r = rng(15)
    codes, scales, biases = random_q4(r, 50, 1024, scale_sigma=0.05, bias_sigma=0.05)
    for tok in (0, 7, 49):
        got = O.embedding(codes, scales, biases, tok)
        want = bf16(dequant_f64(codes[tok:tok + 1], scales[tok:tok + 1], biases[tok:tok + 1])[0].astype(np.float32))
        assert np.array_equal(got, want)


def test_rms_norm_constant_vector_closed_form():
    """x = c everywhere: every sum is exact, so the output is
    bf16(bf16(c * (1/sqrt(c^2 + eps))) * gain) computed in fp32."""
    r = rng(16)
    for c in (0.5, -3.0, 1.0 / 3.0, 1e-3, 7.25):
        cb = f32(bf16(np.float32(c))).item()
        x = bf16(np.full(1024, cb, dtype=np.float32))
        gain = bf16(1 + 0.1 * r.normal(0, 1, 1024))
        got = O.rms_norm(x, gain)
        c32 = np.float32(cb)
        ms = (c32 * c32 * np.float32(1024)) / np.float32(1024)
        inv = np.float32(1.0) / np.sqrt(ms + np.float32(1e-6), dtype=np.float32)
        nrm = f32(bf16(np.float32(c32 * inv))).item()
        want = bf16(np.float32(nrm) * f32(gain))
        assert np.array_equal(got, want), c


def test_rms_norm_fp64():
    r = rng(17)
    x = bf16(r.normal(0, 2, 1024))
    gain = bf16(1 + 0.1 * r.normal(0, 1, 1024))
    got = O.rms_norm(x, gain)
    xf = f32(x).astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(xf * xf) + 1e-6)
    want = bf16((f32(bf16(xf * inv)).astype(np.float64) * f32(gain)).astype(np.float32))
    assert_bf16_close(got, want, max_ulp=1, max_frac=0.02, what="rms_norm")


def test_swiglu_rounding_sequence():
    """silu = bf16(g * sigmoid_bf(g)), out = bf16(silu * up)."""
    r = rng(18)
    g = bf16(r.normal(0, 3, 3584))
    u = bf16(r.normal(0, 1, 3584))
    got = O.swiglu(g, u)
    sig = np.array([O.lib().eo_sigmoid_bf(float(v)) for v in f32(g)], dtype=np.float32)
    silu = f32(bf16(f32(g) * sig))
    assert np.array_equal(got, bf16(silu * f32(u)))
    # and within bf16 tolerance of the exact silu(g) * u
    gd = f32(g).astype(np.float64)
    exact = bf16((gd / (1 + np.exp(-gd)) * f32(u)).astype(np.float32))
    assert_bf16_close(got, exact, max_ulp=3, max_frac=0.6, atol_rel=1e-2, what="swiglu vs fp64")


# ---- row-batched linear (prefill) ----

def test_q4_gemm_constant_weights_closed_form():
    """All codes 0: every weight is exactly bf16(bias), so row r of the output
    is bf16(bias * sum(x[r])) per group; with one group and a power-of-two
    bias the products and sums are exact."""
    r = rng(501)
    n, k, m = 8, 64, 5
    codes = np.zeros((n, k // 8), dtype=np.uint32)
    scales = bf16(np.full((n, 1), 0.5))
    biases = bf16(np.full((n, 1), 0.25))
    x = bf16(np.round(r.normal(0, 4, (m, k))))  # small integers: exact sums
    y = O.q4_gemm(codes, scales, biases, x)
    want = bf16(0.25 * f32(x).astype(np.float64).sum(axis=1))
    assert np.array_equal(y, np.repeat(want[:, None], n, axis=1))


def test_q4_gemm_dequant_rounding_and_rows():
    """Within bf16 weight rounding of the unrounded fp64 dequantisation, row
    by row identical to a one-row call, residual added after the bf16 round."""
    r = rng(502)
    n, k, m = 96, 1024, 7
    codes, scales, biases = random_q4(r, n, k)
    x = bf16(r.normal(0, 1, (m, k)))
    y = O.q4_gemm(codes, scales, biases, x)
    exact = f32(x).astype(np.float64) @ dequant_f64(codes, scales, biases).T
    wq = O.q4_dequant_bf16(codes, scales, biases).astype(np.float64)
    unrounded = dequant_f64(codes, scales, biases)
    assert np.all(np.abs(wq - unrounded) <= np.abs(unrounded) * 2.0 ** -8 + 1e-30)
    err_bound = (np.abs(f32(x)).astype(np.float64) @ np.abs(unrounded).T) * 2.0 ** -8 + np.abs(exact) * 2.0 ** -7
    assert np.all(np.abs(f32(y) - exact) <= err_bound)
    for i in range(m):
        assert np.array_equal(O.q4_gemm(codes, scales, biases, x[i:i + 1])[0], y[i])
    res = bf16(r.normal(0, 1, (m, n)))
    ya = O.q4_gemm(codes, scales, biases, x, residual=res)
    assert np.array_equal(ya, bf16(f32(res) + f32(y)))


def test_q4_gemm_sees_weights_changed_in_place():
    """The oracle's cache of dequantised GEMM weights is keyed by content as
    well as address: rows planted into a weight after its first use (as the
    head tests plant rows) change the result."""
    r = rng(90)
    codes, scales, biases = random_q4(r, 64, 1024)
    x = bf16(r.normal(0, 1, (3, 1024)))
    before = O.q4_gemm(codes, scales, biases, x)
    codes[5] ^= np.uint32(0xFFFFFFFF)
    scales[7] = bf16(np.full(16, 0.5))
    after = O.q4_gemm(codes, scales, biases, x)
    fresh = O.q4_gemm(codes.copy(), scales.copy(), biases.copy(), x)
    assert np.array_equal(after, fresh)
    assert not np.array_equal(after[:, 5], before[:, 5])
    assert not np.array_equal(after[:, 7], before[:, 7])

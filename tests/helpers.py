"""Test data generators and comparison helpers (numpy only)."""
import numpy as np

import oracle as O


def rng(seed):
    return np.random.default_rng(seed)


def bf16(a):
    return O.f32_to_bf16(np.asarray(a, dtype=np.float32))


def f32(a):
    return O.bf16_to_f32(a)


def random_q4(r, n, k, scale_sigma=0.02, bias_sigma=0.01):
    """Uniform random codes, scales |N(0,s)|, biases N(0,b) (bf16)."""
    codes = r.integers(0, 2**32, size=(n, k // 8), dtype=np.uint64).astype(np.uint32)
    scales = bf16(np.abs(r.normal(0, scale_sigma, size=(n, k // 64))))
    biases = bf16(r.normal(0, bias_sigma, size=(n, k // 64)))
    return codes, scales, biases


def dequant_f64(codes, scales, biases):
    """Independent fp64 dequantisation: column c of row r uses nibble c%8 of word c//8."""
    n, k8 = codes.shape
    k = k8 * 8
    shifts = (np.arange(8, dtype=np.uint32) * 4)
    q = ((codes[:, :, None] >> shifts[None, None, :]) & 15).reshape(n, k).astype(np.float64)
    s = np.repeat(f32(scales).astype(np.float64), 64, axis=1)
    b = np.repeat(f32(biases).astype(np.float64), 64, axis=1)
    return s * q + b


def ulp_diff(a_bits, b_bits):
    """Distance in bf16 ulps between two bf16 arrays (sign-aware)."""
    def key(x):
        x = np.asarray(x, dtype=np.uint16).astype(np.int32)
        return np.where(x & 0x8000, -(x & 0x7FFF), x & 0x7FFF)
    return np.abs(key(a_bits) - key(b_bits))


def assert_bf16_close(got, want, max_ulp=1, max_frac=0.01, atol_rel=1e-5, what=""):
    """bf16 outputs of two fp32 computations that differ only in summation order.

    An element passes when it is within max_ulp bf16 ulps, or when its absolute
    difference is at most atol_rel * rms(want) (near-zero outputs, where fp32
    noise spans many bf16 ulps). At most max_frac of the elements may differ.
    """
    got = np.asarray(got).ravel()
    want = np.asarray(want).ravel()
    d = ulp_diff(got, want)
    gf, wf = f32(got), f32(want)
    atol = atol_rel * float(np.sqrt(np.mean(wf.astype(np.float64) ** 2)))
    bad = (d > max_ulp) & (np.abs(gf - wf) > atol)
    frac = float(np.mean(d > 0))
    i = int(np.argmax(bad)) if bad.any() else int(np.argmax(d))
    assert not bad.any() and frac <= max_frac, (
        f"{what}: {int(bad.sum())} elements beyond {max_ulp} ulp / atol {atol:.3g}, "
        f"differing fraction {frac:.4f}, max ulp {int(d.max())} "
        f"(e.g. [{i}] got {gf[i]}, want {wf[i]})")
    return d


def rel_err(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def assert_bits_equal(got, want, what=""):
    """Bitwise equality of two arrays (bf16 bit patterns or fp32)."""
    got = np.ascontiguousarray(got).ravel()
    want = np.ascontiguousarray(want).ravel()
    assert got.shape == want.shape, (what, got.shape, want.shape)
    gv = got.view(np.uint16 if got.dtype == np.uint16 else np.uint32)
    wv = want.view(np.uint16 if want.dtype == np.uint16 else np.uint32)
    bad = np.nonzero(gv != wv)[0]
    if bad.size:
        i = int(bad[0])
        g = f32(got[i:i + 1])[0] if got.dtype == np.uint16 else got[i]
        w = f32(want[i:i + 1])[0] if want.dtype == np.uint16 else want[i]
        raise AssertionError(f"{what}: {bad.size} of {gv.size} differ (first [{i}] got {g!r} want {w!r})")


def fp64_attention_gated(query, kc, vc, length, q_proj):
    """Decode attention of the reference's route in fp64 with its rounding
    points: below 1024 positions one softmax; from 1024 on 64 position chains
    (positions c, c+64, ...) whose unnormalised outputs are rounded to bf16
    before the merge (attention_decode.metal:423-430); then
    bf16(bf16(o) * sigmoid_bf(gate)) (attention_decode.metal:876-889)."""
    q = f32(query).reshape(8, 256).astype(np.float64) * 0.0625
    out = np.empty((8, 256))
    for h in range(8):
        K = f32(kc[h // 4, :length]).astype(np.float64)
        V = f32(vc[h // 4, :length]).astype(np.float64)
        s = K @ q[h]
        if length < 1024:
            p = np.exp(s - s.max())
            out[h] = (p @ V) / p.sum()
            continue
        m = np.array([s[c::64].max() for c in range(64)])
        sums = np.array([np.exp(s[c::64] - m[c]).sum() for c in range(64)])
        parts = np.stack([f32(bf16(np.exp(s[c::64] - m[c]) @ V[c::64])) for c in range(64)])
        f = np.exp(m - m.max())
        out[h] = (f @ parts.astype(np.float64)) / (f @ sums)
    gate = f32(q_proj).reshape(8, 512)[:, 256:].ravel()
    sig = np.array([O.lib().eo_sigmoid_bf(float(x)) for x in gate], dtype=np.float32)
    o = f32(bf16(out.ravel()))
    return bf16(o * sig)


def fp32_ulp(x):
    """Spacing of fp32 numbers at |x| (normal range)."""
    x = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(x, np.finfo(np.float32).tiny)))
    return np.exp2(e - 23)

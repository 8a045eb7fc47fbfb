"""The oracle's scalar numerics pinned against independent references (CPU).

bf16 rounding against torch's bfloat16 cast and the nearest-value definition;
exp, log and sin/cos against fp64 libm within stated ulp bounds plus their
exact special values; the bf16-stepped sigmoid and softplus
(linear.metal:389-395, gdn.metal:10-29) exhaustively over every bf16 input
against an fp64 evaluation of the same rounding sequence; the rotary
frequencies (attention.metal:62-63) against their closed form.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from helpers import bf16, f32, fp32_ulp, rng


def all_bf16():
    return np.arange(65536, dtype=np.uint16)


def test_bf16_widening_exhaustive():
    b = all_bf16()
    got = O.bf16_to_f32_c(b).view(np.uint32)
    assert np.array_equal(got, b.astype(np.uint32) << 16)


def test_bf16_rounding_matches_torch():
    r = rng(1)
    bits = r.integers(0, 2**32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    finite = np.isfinite(x)
    got = bf16(x)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[finite], want[finite])
    # NaN stays NaN (quiet), infinities stay infinities
    nan = np.isnan(x)
    assert np.all(np.isnan(f32(got[nan])))


def test_bf16_rounding_is_nearest_even():
    """Halfway cases go to the even neighbour; everything else to the nearer."""
    r = rng(2)
    hi = r.integers(0, 0x7F7F, 20000, dtype=np.uint32)
    lo = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], dtype=np.uint32)
    bits = (hi[:, None] << 16 | lo[None, :]).ravel()
    x = bits.view(np.float32).astype(np.float64)
    got = f32(bf16(bits.view(np.float32))).astype(np.float64)
    down = ((bits >> 16) << 16).view(np.float32).astype(np.float64)
    up = (((bits >> 16) + 1) << 16).astype(np.uint32).view(np.float32).astype(np.float64)
    tie = (bits & 0xFFFF) == 0x8000
    even_down = ((bits >> 16) & 1) == 0
    want = np.where(tie, np.where(even_down, down, up), np.where(np.abs(x - down) < np.abs(up - x), down, up))
    assert np.array_equal(got, want)


def ulps32(got, want):
    return np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64)) / fp32_ulp(want)


def test_exp_accuracy_and_specials():
    xs = np.concatenate([np.linspace(-85.99, 88.7, 200001), rng(3).uniform(-20, 20, 50000)]).astype(np.float32)
    got = np.array([O.exp(float(x)) for x in xs])
    want = np.exp(xs.astype(np.float64))
    assert ulps32(got, want).max() <= 2.0
    assert O.exp(0.0) == 1.0 and O.exp(-0.0) == 1.0
    assert O.exp(-86.0) == 0.0 and O.exp(-1e30) == 0.0 and O.exp(float("-inf")) == 0.0
    assert O.exp(88.8) == math.inf
    s = np.sort(xs)
    e = np.array([O.exp(float(x)) for x in s[::37]])
    assert np.all(np.diff(e) >= 0), "exp must be monotone"


def test_log_accuracy():
    r = rng(4)
    xs = np.concatenate([np.exp2(r.uniform(-120, 120, 100000)), r.uniform(0.5, 2.0, 100000)]).astype(np.float32)
    got = np.array([O.log(float(x)) for x in xs])
    want = np.log(xs.astype(np.float64))
    err = np.abs(got - want)
    assert np.all(err <= 2.0 * np.maximum(fp32_ulp(want), 2.0**-24))
    assert O.log(1.0) == 0.0


def test_sincos_accuracy_over_rotary_angles():
    r = rng(5)
    pos = r.integers(0, 262144, 30000)
    pair = r.integers(0, 32, 30000)
    inv = np.array([O.lib().eo_rope_inv_freq(int(p)) for p in range(32)], dtype=np.float32)
    ang = (pos.astype(np.float32) * inv[pair]).astype(np.float32)
    sc = np.array([O.sincos(float(a)) for a in ang])
    a64 = ang.astype(np.float64)
    assert np.abs(sc[:, 0] - np.sin(a64)).max() <= 2.5e-7
    assert np.abs(sc[:, 1] - np.cos(a64)).max() <= 2.5e-7
    assert O.sincos(0.0) == (0.0, 1.0)


def rb(v):
    """bf16 rounding of one fp32 value, as an fp32 scalar."""
    return np.float32(f32(bf16(np.float32(v))).item())


def sigmoid_bf_model(x):
    """fp64 exp, then the reference's bf16 steps (each fp32 op rounded)."""
    x = np.float32(x)
    with np.errstate(over="ignore"):
        e = rb(np.exp(np.float64(abs(x))))
    d = rb(np.float32(1.0) + e)
    p = rb(np.float32(1.0) / d)
    return rb(p if x < 0 else np.float32(1.0) - p)


def test_sigmoid_bf_exhaustive():
    xs = f32(all_bf16())
    xs = xs[np.isfinite(xs)]
    got = np.array([O.lib().eo_sigmoid_bf(float(x)) for x in xs], dtype=np.float32)
    want = np.array([sigmoid_bf_model(x) for x in xs], dtype=np.float32)
    diff = got != want
    # the series exp and fp64 exp can round to different bf16 neighbours only
    # when exp(|x|) sits on a bf16 rounding boundary
    assert diff.mean() < 2e-3
    assert np.all(np.abs(got[diff] - want[diff]) <= 2.0**-8 * np.maximum(np.abs(want[diff]), 2.0**-20) * 2)
    for x, w in [(0.0, 0.5), (-0.0, 0.5), (100.0, 1.0), (-100.0, 0.0)]:
        assert O.lib().eo_sigmoid_bf(x) == w
    assert O.lib().eo_sigmoid_bf(88.0) == 1.0
    assert O.lib().eo_sigmoid_bf(-88.0) < 1e-37


def softplus_bf_model(x):
    x = np.float32(x)
    e = rb(np.exp(-np.float64(abs(x))))
    l = rb(np.log1p(np.float64(e)))
    return rb(np.float32(max(x, np.float32(0))) + l)


def test_softplus_bf_exhaustive():
    xs = f32(all_bf16())
    xs = xs[np.isfinite(xs)]
    got = np.array([O.lib().eo_softplus_bf(float(x)) for x in xs], dtype=np.float32)
    want = np.array([softplus_bf_model(x) for x in xs], dtype=np.float32)
    diff = got != want
    assert diff.mean() < 2e-3
    assert np.all(np.abs(got[diff] - want[diff]) <= 2.0**-7 * np.maximum(np.abs(want[diff]), 2.0**-20))
    assert O.lib().eo_softplus_bf(0.0) == rb(math.log(2.0))
    assert O.lib().eo_softplus_bf(100.0) == 100.0


def test_rope_inverse_frequencies_closed_form():
    """inv_freq[i] = exp2(-(i/32) * log2(1e7)) with the exponent formed in
    fp32 as written (attention.metal:62-63): within 1 ulp of that, and within
    the exponent's two fp32 roundings (log2(1e7) and the product, together
    <= 1.5 |t| 2^-24) of the mathematical 1e7^(-i/32) (theta 1e7, 64 rotated
    dims): relative error <= (1.5 ln2 |t| + 1.5) 2^-24."""
    l2 = np.float32(math.log2(1e7))
    for i in range(32):
        got = O.lib().eo_rope_inv_freq(i)
        t = -(np.float32(i) / np.float32(32.0)) * l2
        assert abs(got - 2.0 ** float(t)) <= fp32_ulp(2.0 ** float(t)), i
        exact = 1e7 ** (-i / 32)
        bound = (1.5 * math.log(2) * abs(float(t)) + 1.5) * 2.0**-24
        assert abs(got / exact - 1) <= bound, i
    assert O.lib().eo_rope_inv_freq(0) == 1.0

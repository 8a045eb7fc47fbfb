"""The oracle's greedy head pinned by planted maxima, exact ties and an fp64
log-sum-exp (CPU). Reference: head_lse.metal:11-98 (block max/sum, log-sum-
exp tail), docs/protocol.md:44 (greedy = lowest id among maxima of
bf16(logit - lse)).
"""
import numpy as np
import pytest

import oracle as O
from helpers import bf16, f32, rng

V = 248320
BOUNDARIES = [0, 31, 32, 63, 64, 255, 256, 1023, 1024, 4095, 4096, 65535, 65536, V - 1]


def logits(seed, n=V, mu=4.0, sd=3.0):
    """N(4, 3) logits (the reference probe's distribution)."""
    return bf16(rng(seed).normal(mu, sd, n))


@pytest.mark.parametrize("where", BOUNDARIES)
def test_planted_maximum(where):
    x = logits(50)
    x[where] = bf16(np.float32(40.0))[0]
    tok, _ = O.greedy(x)
    assert tok == where


@pytest.mark.parametrize("i,j", [(0, 1), (31, 32), (255, 256), (1023, 1024), (4095, 4096), (100, V - 1),
                                 (65535, 65536)])
def test_exact_tie_picks_lowest_id(i, j):
    x = logits(51)
    x[i] = x[j] = bf16(np.float32(35.0))[0]
    tok, _ = O.greedy(x)
    assert tok == i


def test_near_tie_within_one_bf16_step_is_a_tie():
    """Logits that differ by less than the bf16 spacing of (logit - lse) tie
    after the reference's bf16(l - lse) and go to the lower id."""
    x = logits(52, mu=0.0, sd=0.1)
    x[7000] = bf16(np.float32(2.0))[0]
    x[9000] = bf16(np.float32(2.0078125))[0]  # next bf16 above 2.0
    tok, lse = O.greedy(x)
    d7 = f32(bf16(np.float32(f32(x[7000]) - lse))).item()
    d9 = f32(bf16(np.float32(f32(x[9000]) - lse))).item()
    assert tok == (7000 if d7 == d9 else 9000)


@pytest.mark.parametrize("n", [1, 100, 256, 257, 4096, 100003, V])
def test_lse_matches_fp64(n):
    x = logits(53 + n, n=n)
    tok, lse = O.greedy(x)
    xf = f32(x).astype(np.float64)
    m = xf.max()
    want = m + np.log(np.exp(xf - m).sum())
    assert abs(lse - want) <= 2.0**-7 * abs(want) + 1e-6, (lse, want)
    assert lse == f32(bf16(np.float32(lse))).item(), "lse is a bf16 value"
    assert tok == int(np.argmax(xf)) or f32(bf16(np.float32(xf[tok] - lse))).item() == f32(
        bf16(np.float32(m - lse))).item()


def test_flat_random_init_logits():
    """Logits of a random-init model are nearly flat: the chosen id is still a
    maximum of bf16(l - lse), the lowest such."""
    x = logits(54, mu=0.0, sd=0.05)
    tok, lse = O.greedy(x)
    d = f32(bf16((f32(x) - np.float32(lse)).astype(np.float32)))
    assert d[tok] == d.max() and tok == int(np.argmax(d == d.max()))

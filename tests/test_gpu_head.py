"""GPU parity of the vocab head: final RMSNorm + tied Q4 LM head + LSE +
greedy with lowest-id ties (head_lse.metal:11-98, linear.metal:300-331,
docs/protocol.md:44)."""
import numpy as np
import pytest

import esdecode as E
import oracle as O
from helpers import assert_bits_equal, bf16, f32, random_q4, rng

pytestmark = pytest.mark.gpu

V = 248320


def run_head(table, h, gain):
    dT = E.DeviceQ4(*table)
    dh, dg = E.DeviceBuffer.from_numpy(h), E.DeviceBuffer.from_numpy(gain)
    n = table[0].shape[0]
    logits = E.DeviceBuffer(n * 2)
    norm = E.DeviceBuffer(2048)
    scratch = E.DeviceBuffer.zeros(E.lib().es_head_scratch_bytes(n))
    tok = E.DeviceBuffer(4)
    lse = E.DeviceBuffer(4)
    for _ in range(2):  # a second call on the same scratch gives the same results
        E.check(E.lib().es_head_greedy(dT.struct, dh.ptr, dg.ptr, norm.ptr, logits.ptr, scratch.ptr, scratch.nbytes,
                                       tok.ptr, lse.ptr, None))
    E.synchronize()
    return (int(tok.numpy(np.uint32)[0]), float(lse.numpy(np.float32)[0]), logits.numpy(np.uint16),
            norm.numpy(np.uint16))


def test_head_random():
    r = rng(31)
    table = random_q4(r, V, 1024)
    h = bf16(r.normal(0, 2, 1024))
    gain = bf16(1 + 0.1 * r.normal(0, 1, 1024))
    tok, lse, logits, norm = run_head(table, h, gain)
    u = O.rms_norm(h, gain)
    assert_bits_equal(norm, u, what="final norm")
    assert_bits_equal(logits, O.q4_matvec(*table, u), what="logits")
    want_tok, want_lse = O.greedy(logits)
    assert lse == want_lse
    assert tok == want_tok


def test_head_planted_ties_pick_lowest_id():
    """Identical maximal rows at block/reduction boundaries -> lowest id."""
    r = rng(32)
    codes, scales, biases = random_q4(r, V, 1024, scale_sigma=0.002, bias_sigma=0.001)
    h = bf16(r.normal(0, 1, 1024))
    gain = bf16(np.ones(1024))
    u = f32(O.rms_norm(h, gain))
    # a row aligned with u: codes 15 where u > 0, 0 elsewhere, unit-ish scale
    q = np.where(u > 0, 15, 0).astype(np.uint32).reshape(128, 8)
    word = np.zeros(128, dtype=np.uint32)
    for j in range(8):
        word |= q[:, j] << (4 * j)
    planted = [255, 256, 1023, 1024, 4095, 4096, 100000, V - 1]
    for idx in planted:
        codes[idx] = word
        scales[idx] = bf16(np.full(16, 0.05))
        biases[idx] = bf16(np.zeros(16))
    tok, lse, logits, _ = run_head((codes, scales, biases), h, gain)
    assert len(set(logits[planted].tolist())) == 1, "planted rows must produce identical logits"
    assert tok == planted[0]
    assert O.greedy(logits)[0] == planted[0]


def test_head_small_vocab_ragged():
    r = rng(33)
    table = random_q4(r, 1000, 1024)
    h = bf16(r.normal(0, 1, 1024))
    gain = bf16(1 + 0.1 * r.normal(0, 1, 1024))
    tok, lse, logits, _ = run_head(table, h, gain)
    assert (tok, lse) == O.greedy(logits)

"""es_head_greedy_noalloc: the vocab head with its block partials in the
library's own device array (for callers that cannot allocate), against
es_head_greedy with caller scratch, bit for bit: logits, normalised input,
token and LSE, on two calls in a row (the second with a smaller vocabulary,
so stale partials of the first call would show), and the size limit."""
import numpy as np
import pytest

import esdecode as E
from helpers import bf16, random_q4, rng

pytestmark = pytest.mark.gpu


def run_head(fn_noalloc, table, h, g):
    n = table[0].shape[0]
    dT = E.DeviceQ4(*table)
    dh, dg = E.DeviceBuffer.from_numpy(h), E.DeviceBuffer.from_numpy(g)
    logits, norm = E.DeviceBuffer(n * 2), E.DeviceBuffer(2048)
    tok, lse = E.DeviceBuffer(4), E.DeviceBuffer(4)
    if fn_noalloc:
        E.check(E.lib().es_head_greedy_noalloc(dT.struct, dh.ptr, dg.ptr, norm.ptr, logits.ptr, tok.ptr, lse.ptr,
                                               None))
    else:
        scratch = E.DeviceBuffer(E.lib().es_head_scratch_bytes(n))
        E.check(E.lib().es_head_greedy(dT.struct, dh.ptr, dg.ptr, norm.ptr, logits.ptr, scratch.ptr, scratch.nbytes,
                                       tok.ptr, lse.ptr, None))
    E.synchronize()
    return (int(tok.numpy(np.uint32)[0]), lse.numpy(np.uint32)[0], logits.numpy(np.uint16), norm.numpy(np.uint16))


def test_noalloc_head_matches_the_scratch_head_on_consecutive_calls():
    r = rng(2026)
    for vocab in (248320, 1000):
        print(f"case noalloc head vocab={vocab}", flush=True)
        table = random_q4(r, vocab, 1024)
        h = bf16(r.normal(0, 1, 1024))
        g = bf16(r.normal(1, 0.1, 1024))
        got = run_head(True, table, h, g)
        want = run_head(False, table, h, g)
        assert got[0] == want[0], "token"
        assert got[1] == want[1], "lse bits"
        assert np.array_equal(got[2], want[2]), "logits"
        assert np.array_equal(got[3], want[3]), "normalised input"


def test_noalloc_head_rejects_a_vocabulary_past_its_scratch():
    r = rng(7)
    n = E.lib().es_head_scratch_bytes(1)  # keeps the library loaded before the limit check
    assert n > 0
    codes, scales, biases = random_q4(r, 8, 1024)
    q = E.Q4(0, 0, 0, 1048577, 1024)
    dT = E.DeviceQ4(codes, scales, biases)
    q.codes, q.scales, q.biases = dT.struct.codes, dT.struct.scales, dT.struct.biases
    buf = E.DeviceBuffer(4096)
    rc = E.lib().es_head_greedy_noalloc(q, buf.ptr, buf.ptr, None, buf.ptr, buf.ptr, None, None)
    assert rc == E.ES_ERR_INVALID
    assert "exceeds the in-library scratch limit of 1048576" in E.lib().es_last_error().decode()

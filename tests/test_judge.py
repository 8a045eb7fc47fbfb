"""The judge and its gates on the oracle alone (CPU): a stream equal to the
oracle's has no mismatch; a planted wrong token is found at its step with
its rank; the gates' thresholds (enginesmith.json) fire where they should."""
import numpy as np
import pytest

import esdecode as E
import oracle as O
from helpers import f32, rng
from judge import gates, judge, token_rank

SMALL = dict(n_layers=4, vocab=8192)


@pytest.fixture(scope="module")
def orc():
    blob = E.random_weights(SMALL["n_layers"], SMALL["vocab"], seed=5)
    views = E.tensor_views(blob, **SMALL)
    return O.OracleModel(views, SMALL["n_layers"], SMALL["vocab"], capacity=256)


def test_token_rank_follows_the_greedy_order():
    lf = np.array([1.0, 3.0, 2.0, 3.0, 0.5], dtype=np.float32)
    assert [token_rank(lf, t) for t in range(5)] == [3, 0, 2, 1, 4]


def test_oracle_stream_has_no_mismatch_and_planted_one_is_found(orc):
    prompt = rng(7).integers(0, SMALL["vocab"], 12).tolist()
    ref = orc.generate(prompt, 10)
    assert judge(orc, prompt, ref) == []
    bad = list(ref)
    # plant the oracle's second choice at step 4
    orc.reset()
    orc.consume_prompt(prompt[:-1])
    inp = prompt[-1]
    for i in range(5):
        tok, logits = orc.step(inp, want_logits=True)
        inp = bad[i]
    lf = f32(logits)
    second = int(np.argsort(-lf, kind="stable")[1])
    bad[4] = second
    m = judge(orc, prompt, bad)
    assert m[0][0] == 4 and m[0][2] == ref[4] and m[0][3] == token_rank(lf, second) == 1
    assert m[0][1] >= 0.0


def test_gate_thresholds():
    one = [(0, 0.1, 5, 1)]
    assert gates([(10, one * 2), (30, [])]) == []            # 20% of a case, 5% overall passes
    assert gates([(10, one * 3), (90, [])]) != []            # 30% fails the case gate
    assert gates([(10, one * 2), (10, one * 2)]) != []       # 20% overall fails the total gate
    assert gates([(100, [(0, 1.0, 5, 101)])]) != []          # rank past 100
    assert gates([(100, [(0, 1.0, 5, 100)])]) == []


def test_snapshot_restore_branches_like_a_fresh_run(orc):
    """A branch taken from a snapshot (steps that are then undone) leaves the
    oracle exactly where an uninterrupted run would be."""
    p = rng(9).integers(0, SMALL["vocab"], 20).tolist()
    want = orc.generate_stepwise(p, 4)
    orc.reset()
    for t in p[:10]:
        orc.step(t, want_head=False)
    snap = orc.snapshot()
    for t in (5, 6, 7):
        orc.step(t)
    orc.restore(snap)
    for t in p[10:-1]:
        orc.step(t, want_head=False)
    tok, got = p[-1], []
    for _ in range(4):
        tok = orc.step(tok)
        got.append(tok)
    assert got == want

"""Teacher-forced judging with the harness's gates (docs/protocol.md:59-70,
enginesmith.json "gates"): a candidate stream is replayed through the oracle
with the candidate's tokens forced; a step whose token is not the oracle's
greedy choice is a mismatch, reported as (step, margin, reference token,
rank). Gates: at most 20% mismatching steps per case, at most 10% over all
cases, and no mismatching token ranked past 100 in the oracle's logits."""
import numpy as np

from helpers import f32

CASE_MISMATCH_PERCENT = 20
TOTAL_MISMATCH_PERCENT = 10
MISMATCH_RANK = 100


def token_rank(logits_f32, token):
    """0-based rank of `token` under the greedy order (higher logit first,
    lower id first on ties)."""
    v = logits_f32[token]
    return int(np.count_nonzero(logits_f32 > v) + np.count_nonzero(logits_f32[:token] == v))


def judge(orc, prompt, tokens):
    """[(step, margin, reference token, rank)] for each mismatching step; the
    oracle consumes the prompt as Model::generate does (consume_prompt)."""
    orc.reset()
    orc.consume_prompt(list(prompt[:-1]))
    return judge_from(orc, prompt[-1], tokens)


def judge_from(orc, first, tokens):
    """judge() from the oracle's current state, whose next input is `first`
    (the prompt's last token)."""
    inp = first
    out = []
    for i, t in enumerate(tokens):
        ref, logits = orc.step(inp, want_logits=True)
        if ref != t:
            lf = f32(logits)
            out.append((i, float(lf[ref] - lf[t]), ref, token_rank(lf, t)))
        inp = t
    return out


def gates(cases):
    """cases: [(n_tokens, mismatches)]. Returns the list of gate violations."""
    bad = []
    total = sum(n for n, _ in cases)
    total_mism = sum(len(m) for _, m in cases)
    for i, (n, m) in enumerate(cases):
        if 100 * len(m) > CASE_MISMATCH_PERCENT * n:
            bad.append(f"case {i}: {len(m)}/{n} mismatches")
        for step, margin, ref, rank in m:
            if rank > MISMATCH_RANK:
                bad.append(f"case {i} step {step}: token ranked {rank} (reference {ref}, margin {margin:.4f})")
    if total and 100 * total_mism > TOTAL_MISMATCH_PERCENT * total:
        bad.append(f"total: {total_mism}/{total} mismatches")
    return bad

"""Pinning the oracle's batched prefill (encode_forward with rows > 1,
model.rs:228-343): its attention restatement against the decode attention
and closed forms, chunk invariance, and agreement with the token-by-token
decode replay of the same prompt. CPU only."""
import numpy as np
import pytest

import esdecode as E
import oracle as O
from helpers import bf16, f32, rng

SMALL = dict(n_layers=4, vocab=8192)


def test_attn_prefill_single_key_is_the_value_row():
    r = rng(1)
    cap = 8
    q = bf16(r.normal(0, 1, (3, 2048)))
    kc, vc = bf16(r.normal(0, 1, (2, cap, 256))), bf16(r.normal(0, 1, (2, cap, 256)))
    o = O.attn_prefill(q, kc, vc, 0, 3).reshape(3, 8, 256)
    for h in range(8):
        assert np.array_equal(o[0, h], vc[h // 4, 0])


def test_attn_prefill_equal_keys_average_the_values():
    """Identical keys give equal probabilities (exactly 1 after the max is
    subtracted): the output is the mean of the attended V rows."""
    r = rng(2)
    cap, rows = 16, 5
    q = bf16(r.normal(0, 1, (rows, 2048)))
    kc = np.repeat(bf16(r.normal(0, 1, (2, 1, 256))), cap, axis=1)
    vc = bf16(r.normal(0, 1, (2, cap, 256)))
    o = f32(O.attn_prefill(q, kc, vc, 3, rows)).reshape(rows, 8, 256)
    V = f32(vc).astype(np.float64)
    for t in range(rows):
        want = V[:, :3 + t + 1].mean(axis=1)
        for h in range(8):
            np.testing.assert_allclose(o[t, h], want[h // 4], rtol=2 ** -8, atol=1e-6)


@pytest.mark.parametrize("pos0,rows", [(0, 4), (30, 40), (1030, 3)])
def test_attn_prefill_agrees_with_the_decode_attention(pos0, rows):
    """Each row equals the decode attention (attn_decode / split route) of the
    same query at its position within the bf16 rounding of the probabilities:
    2^-8 * max|V| + one ulp."""
    r = rng(3 + pos0)
    cap = pos0 + rows
    q = bf16(r.normal(0, 1, (rows, 2048)))
    kc, vc = bf16(r.normal(0, 1, (2, cap, 256))), bf16(r.normal(0, 1, (2, cap, 256)))
    o = f32(O.attn_prefill(q, kc, vc, pos0, rows)).reshape(rows, 2048)
    vmax = np.abs(f32(vc)).max()
    for t in range(rows):
        n = pos0 + t + 1
        if n < 1024:
            d = f32(O.attn_decode_single(q[t], kc, vc, n, cap))
        else:
            parts, sums, maxs = O.attn_decode_split(q[t], kc, vc, n, cap)
            # the split route merges and gates in one kernel; a zero gate input
            # (sigmoid 0.5 in bf16) is undone below
            qp = np.zeros(4096, dtype=np.uint16)
            d = f32(O.attn_split_merge_gate(parts, sums, maxs, qp)) * 2.0
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(d), 1e-30))) - 7)
        assert np.all(np.abs(o[t] - d) <= 2.0 ** -8 * vmax + 2 * ulp), f"row {t}"


@pytest.fixture(scope="module")
def small_model():
    blob = E.random_weights(SMALL["n_layers"], SMALL["vocab"], seed=5)
    return blob, E.tensor_views(blob, **SMALL)


def _state(orc):
    return ({l: a.copy() for l, a in orc.state.items()}, {l: a.copy() for l, a in orc.history.items()},
            {l: a.copy() for l, a in orc.kcache.items()}, {l: a.copy() for l, a in orc.vcache.items()})


def test_prefill_chunks_compose(small_model):
    """Rows are independent in every batched operator except the recurrence
    and the cache, which carry across chunks: prefill(A + B) leaves the same
    state as prefill(A) then prefill(B), bit for bit."""
    _, views = small_model
    toks = rng(7).integers(0, SMALL["vocab"], 45).tolist()
    a = O.OracleModel(views, **SMALL, capacity=64)
    ha = a.prefill(toks)
    b = O.OracleModel(views, **SMALL, capacity=64)
    b.prefill(toks[:17])
    hb = b.prefill(toks[17:])
    assert a.position == b.position == 45
    assert np.array_equal(ha[17:], hb)
    for x, y in zip(_state(a), _state(b)):
        for l in x:
            assert np.array_equal(x[l].view(np.uint16) if x[l].dtype == np.uint16 else x[l].view(np.uint32),
                                  y[l].view(np.uint16) if y[l].dtype == np.uint16 else y[l].view(np.uint32)), l


def test_prefill_with_the_decode_operators_is_the_decode_replay(monkeypatch):
    """With the decode linears (qmv_q4 / qmv_add_q4 per row) in place of the
    batched GEMM and the decode attention per row in place of attn_prefill,
    the batched forward is the decode replay bit for bit: every other
    operator, the rounding points between them, the conv history, the
    recurrence order and the KV rows are the same. Eight layers, so the
    attention output of layer 3 feeds four later layers."""
    blob = E.random_weights(8, 4096, seed=9)
    views = E.tensor_views(blob, 8, 4096)

    def qmv_rows(codes, scales, biases, x, residual=None):
        x = np.ascontiguousarray(x)
        if residual is None:
            return np.stack([O.q4_matvec(codes, scales, biases, x[i]) for i in range(x.shape[0])])
        residual = np.ascontiguousarray(residual)
        return np.stack([O.q4_matvec_add(codes, scales, biases, x[i], residual[i]) for i in range(x.shape[0])])

    def decode_attention_rows(query, kcache, vcache, position, rows):
        return np.stack([O.attn_decode_single(np.ascontiguousarray(query[t]), kcache, vcache, position + t + 1,
                                              kcache.shape[1]) for t in range(rows)])

    toks = rng(10).integers(0, 4096, 41).tolist()
    monkeypatch.setattr(O, "q4_gemm", qmv_rows)
    monkeypatch.setattr(O, "attn_prefill", decode_attention_rows)
    a = O.OracleModel(views, 8, 4096, capacity=48)
    a.prefill(toks[:-1])
    ta, la = a.step(toks[-1], want_logits=True)
    b = O.OracleModel(views, 8, 4096, capacity=48)
    for t in toks[:-1]:
        b.step(t, want_head=False)
    tb, lb = b.step(toks[-1], want_logits=True)
    assert ta == tb and np.array_equal(la, lb)
    for x, y in zip(_state(a), _state(b)):
        for l in x:
            assert np.array_equal(x[l].view(np.uint16) if x[l].dtype == np.uint16 else x[l].view(np.uint32),
                                  y[l].view(np.uint16) if y[l].dtype == np.uint16 else y[l].view(np.uint32)), l


def test_prefill_agrees_with_the_decode_replay(small_model):
    """With its own arithmetic (weights dequantised to bf16 before the
    product, bf16 probabilities) the batched forward stays close to the
    decode steps: after a 60-token prompt the GDN states and KV rows agree to
    a relative error below 6% (random weights amplify the per-linear 0.2%
    from layer to layer: 0.5%, 2%, 3.5% measured) and the next-token logits
    to 5% of their range; a different greedy pick is a near tie."""
    _, views = small_model
    toks = rng(8).integers(0, SMALL["vocab"], 61).tolist()
    a = O.OracleModel(views, **SMALL, capacity=64)
    a.prefill(toks[:-1])
    ta, la = a.step(toks[-1], want_logits=True)
    b = O.OracleModel(views, **SMALL, capacity=64)
    for t in toks[:-1]:
        b.step(t, want_head=False)
    tb, lb = b.step(toks[-1], want_logits=True)
    for l in a.state:
        rel = np.linalg.norm(a.state[l] - b.state[l]) / np.linalg.norm(b.state[l])
        assert rel < 0.06, (l, rel)
    for ca, cb in ((a.kcache, b.kcache), (a.vcache, b.vcache)):
        for l in ca:
            x = f32(ca[l][:, :61]).astype(np.float64)
            y = f32(cb[l][:, :61]).astype(np.float64)
            assert np.linalg.norm(x - y) / np.linalg.norm(y) < 0.06, l
    fa, fb = f32(la), f32(lb)
    assert np.abs(fa - fb).max() <= 0.05 * (fb.max() - fb.min())
    if ta != tb:
        assert abs(fb[tb] - fb[ta]) <= 0.05


def test_prefill_wrong_residual_is_caught(small_model, monkeypatch):
    """Control for the test above: dropping the residual of the MLP's down
    projection in the oracle's prefill moves the state far outside those
    bounds."""
    _, views = small_model
    toks = rng(8).integers(0, SMALL["vocab"], 21).tolist()
    real = O.q4_gemm

    def no_down_residual(codes, scales, biases, x, residual=None):
        if residual is not None and codes.shape[1] * 8 == 3584:
            residual = None
        return real(codes, scales, biases, x, residual)

    monkeypatch.setattr(O, "q4_gemm", no_down_residual)
    a = O.OracleModel(views, **SMALL, capacity=32)
    a.prefill(toks[:-1])
    monkeypatch.setattr(O, "q4_gemm", real)
    b = O.OracleModel(views, **SMALL, capacity=32)
    for t in toks[:-1]:
        b.step(t, want_head=False)
    rel = max(np.linalg.norm(a.state[l] - b.state[l]) / np.linalg.norm(b.state[l]) for l in a.state)
    print(f"relative state error with the residual dropped: {rel:.3f}")
    assert rel > 0.3

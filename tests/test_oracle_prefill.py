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
    """On the route of a full forward (every linear a GEMM), rows are
    independent in every batched operator except the recurrence and the
    cache, which carry across chunks: prefill(A + B) leaves the same state as
    prefill(A) then prefill(B), bit for bit. This is what lets the engine
    group full-forward rows into chunks of any size."""
    _, views = small_model
    toks = rng(7).integers(0, SMALL["vocab"], 45).tolist()
    a = O.OracleModel(views, **SMALL, capacity=64)
    ha = a.prefill(toks, gemm_only=True)
    b = O.OracleModel(views, **SMALL, capacity=64)
    b.prefill(toks[:17], gemm_only=True)
    hb = b.prefill(toks[17:], gemm_only=True)
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
    toks = rng(8).integers(0, SMALL["vocab"], 41).tolist()  # 40 rows: every linear on the GEMM
    real = O.q4_gemm

    def no_down_residual(codes, scales, biases, x, residual=None):
        if residual is not None and codes.shape[1] * 8 == 3584:
            residual = None
        return real(codes, scales, biases, x, residual)

    monkeypatch.setattr(O, "q4_gemm", no_down_residual)
    a = O.OracleModel(views, **SMALL, capacity=48)
    a.prefill(toks[:-1])
    monkeypatch.setattr(O, "q4_gemm", real)
    b = O.OracleModel(views, **SMALL, capacity=48)
    for t in toks[:-1]:
        b.step(t, want_head=False)
    rel = max(np.linalg.norm(a.state[l] - b.state[l]) / np.linalg.norm(b.state[l]) for l in a.state)
    print(f"relative state error with the residual dropped: {rel:.3f}")
    assert rel > 0.3


# ---- the reference's prompt routing (model.rs:106-109, 189-198) ----
# Every linear shape of the model with the row limit model.rs:191-192 gives it.
MODEL_SHAPES = {(6144, 1024): 13, (2048, 1024): 33, (16, 1024): 33, (1024, 2048): 33, (4096, 1024): 25,
                (512, 1024): 33, (3584, 1024): 25, (1024, 3584): 25, (248320, 1024): 13}


def test_linear_row_limit_table():
    """The three limits of Model::linear: k <= 2048 and n <= 2048 -> 33;
    otherwise k <= 4096 and n <= 4096 -> 25; otherwise 13 (including the
    6144-row in_proj_qkv and the head). The engine's table (C ABI) agrees."""
    for (n, k), want in MODEL_SHAPES.items():
        assert O.linear_row_limit(n, k) == want, (n, k)
        assert E.lib().es_linear_row_limit(n, k) == want, (n, k)
    for n, k in ((2048, 2048), (2049, 2048), (2048, 2049), (4096, 4096), (4097, 4096), (4096, 4097), (1, 1)):
        assert E.lib().es_linear_row_limit(n, k) == O.linear_row_limit(n, k)
    assert E.lib().es_linear_row_limit(0, 1024) < 0


def _record_routes(monkeypatch):
    calls = []
    gemm, rows = O.q4_gemm, O.q4_matvec_rows

    def rec_gemm(codes, scales, biases, x, residual=None):
        calls.append(("gemm", codes.shape[0], codes.shape[1] * 8, x.shape[0]))
        return gemm(codes, scales, biases, x, residual)

    def rec_rows(codes, scales, biases, x, residual=None):
        calls.append(("qmv", codes.shape[0], codes.shape[1] * 8, x.shape[0]))
        return rows(codes, scales, biases, x, residual)

    monkeypatch.setattr(O, "q4_gemm", rec_gemm)
    monkeypatch.setattr(O, "q4_matvec_rows", rec_rows)
    return calls


@pytest.mark.parametrize("rows", [2, 12, 13, 24, 25, 32, 33])
def test_short_forward_routes_each_linear_by_its_limit(small_model, monkeypatch, rows):
    """A forward of r rows sends each linear to qmv_q4 rows when r is below
    its shape's limit and to the GEMM otherwise; every linear of every layer
    is called once."""
    _, views = small_model
    calls = _record_routes(monkeypatch)
    toks = rng(rows).integers(0, SMALL["vocab"], rows).tolist()
    O.OracleModel(views, **SMALL, capacity=40).prefill(toks)
    # GDN layers: qkv z a b out gate up down; the attention layer: q k v o gate up down
    assert len(calls) == 3 * 8 + 1 * 7
    for route, n, k, m in calls:
        assert m == rows
        want = "qmv" if rows < MODEL_SHAPES[(n, k)] else "gemm"
        assert route == want, (n, k, rows, route)


@pytest.mark.parametrize("n,forwards", [
    (1, [1]), (2, [2]), (33, [33]), (2047, [2047]), (2048, [2048]), (2049, [2048, 1]), (2050, [2048, 2]),
    (4096, [2048, 2048]), (4097, [2048, 2048, 1]), (4130, [2048, 2048, 34])])
def test_consume_prompt_forwards(small_model, monkeypatch, n, forwards):
    """Model::generate's prompt loop: forwards of 2048 rows from position 0,
    the last one shorter; a one-row forward is the decode step."""
    _, views = small_model
    seen = []
    orc = O.OracleModel(views, **SMALL, capacity=8)
    monkeypatch.setattr(orc, "prefill", lambda toks, gemm_only=False: seen.append(len(toks)))
    orc.consume_prompt(list(range(n)))
    assert seen == forwards


def test_routed_forward_with_decode_attention_is_the_decode_replay(monkeypatch):
    """A forward of 12 rows takes qmv_q4 rows for every linear (12 is below
    every limit). With the decode attention substituted for the flash
    attention, it is the decode replay of the same tokens bit for bit: the
    routed linears have the decode matvec's arithmetic, weights not rounded."""
    blob = E.random_weights(8, 4096, seed=9)
    views = E.tensor_views(blob, 8, 4096)

    def decode_attention_rows(query, kcache, vcache, position, rows):
        return np.stack([O.attn_decode_single(np.ascontiguousarray(query[t]), kcache, vcache, position + t + 1,
                                              kcache.shape[1]) for t in range(rows)])

    monkeypatch.setattr(O, "attn_prefill", decode_attention_rows)
    toks = rng(12).integers(0, 4096, 13).tolist()
    a = O.OracleModel(views, 8, 4096, capacity=16)
    a.prefill(toks[:-1])
    ta, la = a.step(toks[-1], want_logits=True)
    b = O.OracleModel(views, 8, 4096, capacity=16)
    for t in toks[:-1]:
        b.step(t, want_head=False)
    tb, lb = b.step(toks[-1], want_logits=True)
    assert ta == tb and np.array_equal(la, lb)
    for x, y in zip(_state(a), _state(b)):
        for l in x:
            assert np.array_equal(x[l].view(np.uint16) if x[l].dtype == np.uint16 else x[l].view(np.uint32),
                                  y[l].view(np.uint16) if y[l].dtype == np.uint16 else y[l].view(np.uint32)), l


def test_routed_forward_differs_from_the_gemm_route(small_model):
    """Control for the routing: the same 20-row forward with every linear on
    the GEMM (bf16-rounded weights) leaves different bits in the states, so
    the tests above would see a wrong route."""
    _, views = small_model
    toks = rng(20).integers(0, SMALL["vocab"], 20).tolist()
    a = O.OracleModel(views, **SMALL, capacity=24)
    a.prefill(toks)
    b = O.OracleModel(views, **SMALL, capacity=24)
    b.prefill(toks, gemm_only=True)
    assert not np.array_equal(a.state[0].view(np.uint32), b.state[0].view(np.uint32))

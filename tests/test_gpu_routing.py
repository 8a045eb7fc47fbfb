"""The reference's prompt routing (model.rs:106-109, 189-198) and the
LINEAR / GDN interface entries it needs, on the GPU through the C ABI:

- qmv_q4 with M rows (LINEAR_INTERFACE.md:19), add_bf16 (:23) and
  greedy_bf16 (:25) against the oracle, bit for bit;
- the GDN kernels over the reference's [3, 6144] history (GDN_INTERFACE.md:
  12-18) against the oracle's token-by-token restatement, bit for bit;
- the engine's prompt loop: 2048-row forwards from position 0, the last one
  routed per linear (qmv_q4 rows below the shape's row limit, the decode
  kernels for one row), judged against the oracle's consume_prompt.
"""
import numpy as np
import pytest

import esdecode as E
import oracle as O
from helpers import assert_bits_equal, bf16, f32, random_q4, rng
from judge import gates, judge_from

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=4, vocab=8192)
LINEAR_SHAPES = [(6144, 1024), (2048, 1024), (16, 1024), (1024, 2048), (4096, 1024), (512, 1024), (3584, 1024),
                 (1024, 3584)]


@pytest.mark.parametrize("n,k", LINEAR_SHAPES)
@pytest.mark.parametrize("rows", [2, 32])
def test_q4_matvec_rows(n, k, rows):
    """Each of the rows is the M = 1 matvec (oracle q4_matvec), with and
    without the residual (which may alias the output)."""
    print(f"case matvec rows n={n} k={k} rows={rows}", flush=True)
    r = rng(n + k + rows)
    codes, scales, biases = random_q4(r, n, k)
    x = bf16(r.normal(0, 1, (rows, k)))
    res = bf16(r.normal(0, 1, (rows, n)))
    W = E.DeviceQ4(codes, scales, biases)
    dx = E.DeviceBuffer.from_numpy(x)
    dy = E.DeviceBuffer(rows * n * 2)
    E.check(E.lib().es_q4_matvec_rows(W.struct, dx.ptr, rows, None, dy.ptr, None))
    dh = E.DeviceBuffer.from_numpy(res)
    E.check(E.lib().es_q4_matvec_rows(W.struct, dx.ptr, rows, dh.ptr, dh.ptr, None))
    E.synchronize()
    assert_bits_equal(dy.numpy(np.uint16), O.q4_matvec_rows(codes, scales, biases, x), what="rows")
    assert_bits_equal(dh.numpy(np.uint16), O.q4_matvec_rows(codes, scales, biases, x, res), what="rows + residual")


def test_q4_matvec_rows_rejects_bad_arguments():
    r = rng(4)
    codes, scales, biases = random_q4(r, 16, 1024)
    W = E.DeviceQ4(codes, scales, biases)
    dx = E.DeviceBuffer(4 * 1024 * 2)
    dy = E.DeviceBuffer(4 * 16 * 2)
    for rows in (0, 65536):
        assert E.lib().es_q4_matvec_rows(W.struct, dx.ptr, rows, None, dy.ptr, None) == E.ES_ERR_INVALID
    assert E.lib().es_q4_matvec_rows(W.struct, dx.ptr, 4, None, dx.ptr, None) == E.ES_ERR_INVALID


def test_add_bf16_with_aliasing():
    r = rng(5)
    n = 100003
    a, b = bf16(r.normal(0, 1, n)), bf16(r.normal(0, 3, n))
    want = O.f32_to_bf16(f32(a) + f32(b))  # one fp32 add is exact before the bf16 round
    da, db, do = E.DeviceBuffer.from_numpy(a), E.DeviceBuffer.from_numpy(b), E.DeviceBuffer(2 * n)
    E.check(E.lib().es_add_bf16(da.ptr, db.ptr, n, do.ptr, None))
    E.check(E.lib().es_add_bf16(da.ptr, db.ptr, n, da.ptr, None))  # out aliases a
    E.synchronize()
    assert_bits_equal(do.numpy(np.uint16), want, what="add")
    assert_bits_equal(da.numpy(np.uint16), want, what="add aliased")


@pytest.mark.parametrize("count", [1, 257, 4096, 248320])
def test_greedy_bf16(count):
    """greedy_bf16 over logits N(4, 3) with the maximum planted twice (at a
    block boundary and later): the lowest index wins and the LSE is the
    oracle's bit for bit."""
    print(f"case greedy count={count}", flush=True)
    r = rng(count)
    logits = bf16(r.normal(4, 3, count))
    top = bf16(np.array([30.0]))[0]
    first = min(count - 1, 256 * (count // 512))
    logits[first] = top
    logits[count - 1] = top
    want_tok, want_lse = O.greedy(logits)
    dl = E.DeviceBuffer.from_numpy(logits)
    scratch = E.DeviceBuffer(E.lib().es_head_scratch_bytes(count))
    tok, lse = E.DeviceBuffer(4), E.DeviceBuffer(4)
    E.check(E.lib().es_greedy_bf16(dl.ptr, count, scratch.ptr, scratch.nbytes, tok.ptr, lse.ptr, None))
    E.synchronize()
    assert int(tok.numpy(np.uint32)[0]) == want_tok == first
    assert np.float32(lse.numpy(np.float32)[0]).view(np.uint32) == np.float32(want_lse).view(np.uint32)
    if count > 256:
        short = E.DeviceBuffer(E.lib().es_head_scratch_bytes(count) - 8)
        assert E.lib().es_greedy_bf16(dl.ptr, count, short.ptr, short.nbytes, tok.ptr, lse.ptr, None) == \
            E.ES_ERR_INVALID


@pytest.mark.parametrize("rows", [1, 2, 19, 70])
def test_gdn_history_form(rows):
    """gdn_conv, gdn_history, gdn_prepare and gdn_recur over the reference's
    history (nonzero, so the short-history shifts of rows 1 and 2 show):
    normalised conv, g, beta, history, state and y equal the oracle's
    token-by-token gdn_conv_prepare + gdn_recur. 70 rows cross the
    recurrence's 64-token tile."""
    print(f"case gdn history form rows={rows}", flush=True)
    r = rng(29 + rows)
    raw = bf16(r.normal(0, 1, (rows, 6144)))
    hist0 = bf16(r.normal(0, 1, (3, 6144)))
    conv_w = bf16(r.normal(0, 0.5, (6144, 4)))
    a, b = bf16(r.normal(0, 1, (rows, 16))), bf16(r.normal(0, 1, (rows, 16)))
    a_log = r.uniform(-2, 2, 16).astype(np.float32)
    dt = bf16(r.normal(0.3, 0.5, 16))
    state0 = r.normal(0, 0.1, (16, 128, 128)).astype(np.float32)
    hist, state = hist0.copy(), state0.copy()
    w_conv, w_g, w_beta, w_y = [], [], [], []
    for t in range(rows):
        conv, g, beta = O.gdn_conv_prepare(raw[t], hist, conv_w, a[t], b[t], a_log, dt)
        w_y.append(O.gdn_recur(conv, g, beta, state))
        w_conv.append(conv)
        w_g.append(g)
        w_beta.append(beta)
    draw, dh, dw = E.DeviceBuffer.from_numpy(raw), E.DeviceBuffer.from_numpy(hist0), E.DeviceBuffer.from_numpy(conv_w)
    da, db = E.DeviceBuffer.from_numpy(a), E.DeviceBuffer.from_numpy(b)
    dal, ddt = E.DeviceBuffer.from_numpy(a_log), E.DeviceBuffer.from_numpy(dt)
    dconv = E.DeviceBuffer(rows * 6144 * 2)
    dg, dbeta = E.DeviceBuffer(rows * 16 * 4), E.DeviceBuffer(rows * 16 * 2)
    dstate = E.DeviceBuffer.from_numpy(state0)
    dy = E.DeviceBuffer(rows * 2048 * 2)
    L = E.lib()
    E.check(L.es_gdn_conv(draw.ptr, dh.ptr, dw.ptr, rows, dconv.ptr, None))
    E.check(L.es_gdn_history(draw.ptr, rows, dh.ptr, None))
    E.check(L.es_gdn_prepare(dconv.ptr, da.ptr, db.ptr, dal.ptr, ddt.ptr, rows, dg.ptr, dbeta.ptr, None))
    E.check(L.es_gdn_recur(dconv.ptr, dg.ptr, dbeta.ptr, rows, dstate.ptr, dy.ptr, None))
    E.synchronize()
    assert_bits_equal(dconv.numpy(np.uint16), np.stack(w_conv), what="normalised conv")
    assert_bits_equal(dg.numpy(np.float32), np.stack(w_g), what="g")
    assert_bits_equal(dbeta.numpy(np.uint16), np.stack(w_beta), what="beta")
    assert_bits_equal(dh.numpy(np.uint16), hist, what="history")
    assert_bits_equal(dy.numpy(np.uint16), np.stack(w_y), what="y")
    assert_bits_equal(dstate.numpy(np.float32), state, what="state")


# ---- the engine's prompt routing ----
@pytest.fixture(scope="module")
def small():
    blob = E.random_weights(SMALL["n_layers"], SMALL["vocab"], seed=5)
    eng = E.Engine(blob, SMALL["n_layers"], SMALL["vocab"], capacity=2200)
    orc = O.OracleModel(E.tensor_views(blob, **SMALL), **SMALL, capacity=2200)
    yield eng, orc
    eng.close()


def expected_split(consumed, chunk_rows):
    """(batched chunks, routed rows, decode rows) of the reference's
    decomposition of `consumed` prompt rows into 2048-row forwards, with the
    full-forward rows grouped into chunks of chunk_rows."""
    tail = consumed % 2048
    if tail >= 33:
        tail = 0
    body = consumed - tail
    return (-(-body // chunk_rows), tail if tail >= 2 else 0, 1 if tail == 1 else 0)


def engine_state(eng, n_kv):
    gdn = {l: eng.read_gdn(l) for l in range(SMALL["n_layers"]) if l % 4 != 3}
    kv = {l: (eng.read_kv(l, 0, 0, n_kv), eng.read_kv(l, 1, 0, n_kv)) for l in range(SMALL["n_layers"]) if l % 4 == 3}
    return gdn, kv


@pytest.mark.parametrize("n", [2, 3, 9])
def test_routed_short_prompt_is_bitwise(small, n):
    """Prompts of 2, 3 and 9 tokens: 1 row runs the decode kernels, 2 and 8
    rows run every linear as qmv_q4 rows (below every limit). The GDN layers
    and the K/V rows then carry the oracle's bits exactly, and since the
    flash attention's outputs of the prompt rows feed nothing after the last
    layer of this 4-layer model, every generated token is the oracle's."""
    eng, orc = small
    print(f"case routed short prompt {n}", flush=True)
    prompt = rng(300 + n).integers(0, SMALL["vocab"], n).tolist()
    toks = eng.generate(prompt, 12, reset=True)
    assert eng.prompt_split() == expected_split(n - 1, 2200)
    orc.reset()
    orc.consume_prompt(prompt[:-1])
    gdn, kv = engine_state(eng, n - 1 + 12)
    want = orc.decode(prompt[-1], 12)
    assert toks == want
    for l, (ring, state) in gdn.items():
        assert_bits_equal(state, orc.state[l], what=f"state {l}")
    for l, (k, v) in kv.items():
        assert_bits_equal(k, orc.kcache[l][:, :n - 1 + 12], what=f"K {l}")
        assert_bits_equal(v, orc.vcache[l][:, :n - 1 + 12], what=f"V {l}")


# prompt length: consumed rows = length - 1 = 2048 * full + tail
ROUTED_PROMPTS = [14, 26, 34, 2050, 2051, 2063, 2075, 2082]


def test_routed_prompts_pass_the_harness_gates(small):
    """Prompts whose last forward has 13 rows (in_proj_qkv on the GEMM, the
    rest on qmv_q4 rows), 25 rows (q, gate, up, down on the GEMM), 33 rows
    (all on the GEMM), and the same after a full 2048-row forward (2050: a
    one-row last forward on the decode kernels). 16 greedy tokens each,
    judged teacher-forced from the oracle's consume_prompt; the routing is
    also read back from the engine."""
    eng, orc = small
    base = rng(2082).integers(0, SMALL["vocab"], max(ROUTED_PROMPTS)).tolist()
    orc.reset()
    orc.prefill(base[:2048])
    snap2048 = orc.snapshot()
    cases = []
    for n in ROUTED_PROMPTS:
        print(f"case routed prompt {n}", flush=True)
        prompt = base[:n]
        toks = eng.generate(prompt, 16, reset=True)
        # the engine's chunk buffers hold min(4096, capacity 2200) rows
        assert eng.prompt_split() == expected_split(n - 1, 2200), (n, eng.prompt_split())
        if n - 1 >= 2048:
            orc.restore(snap2048)
            orc.consume_prompt(prompt[2048:n - 1])
        else:
            orc.reset()
            orc.consume_prompt(prompt[:n - 1])
        m = judge_from(orc, prompt[-1], toks)
        print(f"prompt {n}: {m}", flush=True)
        for step, margin, ref, rank in m:
            assert margin <= 0.1, (n, step, margin)
        cases.append((16, m))
    assert gates(cases) == []


def test_routed_tail_does_not_depend_on_the_chunk_size(small):
    """The full-forward rows before a routed tail run in chunks of any size
    with the same bits (2048 + 14 rows in one chunk, and in chunks of 1000)."""
    eng, _ = small
    prompt = rng(2063).integers(0, SMALL["vocab"], 2063).tolist()
    runs = []
    try:
        for rows in (4096, 1000):
            eng.set_prefill(rows)
            toks = eng.generate(prompt, 4, reset=True)
            runs.append((toks, eng.prompt_split(), engine_state(eng, 2066)))
    finally:
        eng.set_prefill(4096)
    (t0, s0, (g0, k0)), (t1, s1, (g1, k1)) = runs
    assert s0 == (1, 14, 0) and s1 == (3, 14, 0)
    assert t0 == t1
    for l in g0:
        assert np.array_equal(g0[l][0], g1[l][0])
        assert np.array_equal(g0[l][1].view(np.uint32), g1[l][1].view(np.uint32))
    for l in k0:
        assert np.array_equal(k0[l][0], k1[l][0]) and np.array_equal(k0[l][1], k1[l][1])

"""The HIP kernels reproduce the committed golden fixtures bit for bit
through the C ABI: Q4 matvec (K = 1024, 2048, 3584), one Gated DeltaNet
step, decode attention on both routes, and the small model's greedy tokens.
"""
import os
import sys

import numpy as np
import pytest

import esdecode as E
from conftest import ROOT
from helpers import assert_bits_equal

sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
import vectors as V  # noqa: E402

pytestmark = pytest.mark.gpu
GOLDEN = np.load(os.path.join(ROOT, "tests", "golden", "golden.npz"))


@pytest.mark.parametrize("name", ["qmv_k1024", "qmv_k2048", "qmv_k3584"])
def test_qmv_fixture(name):
    x = V.CASES[name]()
    W = E.DeviceQ4(x["codes"], x["scales"], x["biases"])
    dx = E.DeviceBuffer.from_numpy(x["x"])
    dy, dyf = E.DeviceBuffer(W.n * 2), E.DeviceBuffer(W.n * 4)
    E.check(E.lib().es_q4_matvec(W.struct, dx.ptr, dy.ptr, dyf.ptr, None))
    E.synchronize()
    assert_bits_equal(dy.numpy(np.uint16), GOLDEN[name + "/y"], what="y")
    assert_bits_equal(dyf.numpy(np.float32), GOLDEN[name + "/y_f32"], what="y_f32")


def test_gdn_step_fixture():
    """Ring slots 0..2 hold the reference's history rows, slot 3 the new
    projection, so position 3 reads taps (history, raw)."""
    x = V.CASES["gdn_step"]()
    ring = np.concatenate([x["history"].ravel(), x["raw"]]).astype(np.uint16)
    d = dict(ring=E.DeviceBuffer.from_numpy(ring), conv=E.DeviceBuffer.from_numpy(x["conv_w"]),
             ab=E.DeviceBuffer.from_numpy(np.concatenate([x["a"], x["b"]])),
             alog=E.DeviceBuffer.from_numpy(x["a_log"]), dt=E.DeviceBuffer.from_numpy(x["dt_bias"]),
             state=E.DeviceBuffer.from_numpy(x["state"]), y=E.DeviceBuffer(4096), qkv=E.DeviceBuffer(6144 * 2),
             g=E.DeviceBuffer(64), beta=E.DeviceBuffer(32))
    E.check(E.lib().es_gdn_recur_step(d["ring"].ptr, 3, d["conv"].ptr, d["ab"].ptr, d["alog"].ptr, d["dt"].ptr,
                                      d["state"].ptr, d["y"].ptr, d["qkv"].ptr, d["g"].ptr, d["beta"].ptr, None))
    E.synchronize()
    assert_bits_equal(d["qkv"].numpy(np.uint16), GOLDEN["gdn_step/conv"], what="conv")
    assert_bits_equal(d["g"].numpy(np.float32, 16), GOLDEN["gdn_step/g"], what="g")
    assert_bits_equal(d["beta"].numpy(np.uint16, 16), GOLDEN["gdn_step/beta"], what="beta")
    assert_bits_equal(d["y"].numpy(np.uint16, 2048), GOLDEN["gdn_step/y"], what="y")
    state = d["state"].numpy(np.float32).reshape(16, 128, 128)
    assert_bits_equal(state[0, 0], GOLDEN["gdn_step/state_head"], what="state row")
    import hashlib
    assert hashlib.sha256(state.tobytes()).hexdigest() == str(GOLDEN["gdn_step/state_sha256"])


@pytest.mark.parametrize("name", ["attn_n1", "attn_n100", "attn_n1023", "attn_n1024", "attn_n2500"])
def test_attention_fixture(name):
    x = V.CASES[name]()
    cap, pos = x["capacity"], x["position"]
    d = {n: E.DeviceBuffer.from_numpy(x[n]) for n in ("kc", "vc", "q_proj", "k", "v", "q_gain", "k_gain")}
    f = E.DeviceBuffer.from_numpy(E.rope_inv_freq())
    scratch = E.DeviceBuffer(E.lib().es_attn_scratch_bytes(cap))
    gated, qout = E.DeviceBuffer(4096), E.DeviceBuffer(4096)
    E.check(E.lib().es_attn_decode(d["q_proj"].ptr, d["k"].ptr, d["v"].ptr, d["q_gain"].ptr, d["k_gain"].ptr,
                                   d["kc"].ptr, d["vc"].ptr, cap, pos, f.ptr, E.splits_for(pos + 1), scratch.ptr,
                                   scratch.nbytes, gated.ptr, qout.ptr, None))
    E.synchronize()
    assert_bits_equal(qout.numpy(np.uint16), GOLDEN[name + "/query"], what="query")
    assert_bits_equal(gated.numpy(np.uint16), GOLDEN[name + "/gated"], what="gated")
    kc = d["kc"].numpy(np.uint16).reshape(2, cap, 256)
    assert_bits_equal(kc[:, pos], GOLDEN[name + "/k_row"], what="K row")


def test_model_tokens_fixture():
    m = V.MODEL
    blob = E.random_weights(m["n_layers"], m["vocab"], m["seed"], threads=4)
    eng = E.Engine(blob, m["n_layers"], m["vocab"], capacity=64)
    try:
        eng.set_prefill(0)  # the fixture is the token-by-token replay of the prompt
        got = eng.generate(m["prompt"], m["tokens"], reset=True)
    finally:
        eng.close()
    assert list(got) == [int(t) for t in GOLDEN["model/tokens"]]

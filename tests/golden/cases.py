"""Expected outputs of the golden cases, computed by the oracle.

Shared by gen_golden.py (which writes golden.npz) and the tests (which
recompute and compare). Large outputs are kept as a SHA-256 digest plus a
slice.
"""
import hashlib

import numpy as np

import oracle as O
import vectors as V


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def oracle_outputs(name: str, x: dict) -> dict:
    if name.startswith("qmv_"):
        y, yf = O.q4_matvec(x["codes"], x["scales"], x["biases"], x["x"], want_f32=True)
        return dict(y=y, y_f32=yf)
    if name == "rms_norm":
        return dict(out=O.rms_norm(x["x"], x["gain"]))
    if name == "swiglu":
        return dict(out=O.swiglu(x["gate"], x["up"]))
    if name == "gdn_step":
        hist = x["history"].copy()
        conv, g, beta = O.gdn_conv_prepare(x["raw"], hist, x["conv_w"], x["a"], x["b"], x["a_log"], x["dt_bias"])
        state = x["state"].copy()
        y = O.gdn_recur(conv, g, beta, state)
        gated = O.gdn_norm_gate(y, x["z"], x["norm_w"])
        return dict(conv=conv, g=g, beta=beta, y=y, gated=gated, state_head=state[0, 0].copy(),
                    state_sha256=np.array(digest(state)))
    if name.startswith("attn_"):
        kc, vc = x["kc"].copy(), x["vc"].copy()
        query = O.attn_prepare(x["q_proj"], x["k"], x["v"], x["q_gain"], x["k_gain"], kc, vc, x["position"],
                               x["capacity"])
        gated = O.attn_decode_gated(query, kc, vc, x["position"] + 1, x["capacity"], x["q_proj"])
        return dict(query=query, gated=gated, k_row=kc[:, x["position"]].copy())
    if name == "greedy":
        tok, lse = O.greedy(x["logits"])
        return dict(token=np.array(tok), lse=np.array(lse, dtype=np.float32))
    raise KeyError(name)


def oracle_model_tokens(E) -> np.ndarray:
    m = V.MODEL
    blob = E.random_weights(m["n_layers"], m["vocab"], m["seed"], threads=4)
    orc = O.OracleModel(E.tensor_views(blob, m["n_layers"], m["vocab"]), m["n_layers"], m["vocab"],
                        capacity=len(m["prompt"]) + m["tokens"] + 1)
    return np.array(orc.generate(m["prompt"], m["tokens"]), dtype=np.int64)

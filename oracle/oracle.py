"""ctypes binding of the CPU oracle (libesoracle.so).

TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the parity checker / timed CPU baseline.
The engine never imports this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_float, c_int, c_uint16, c_uint32, c_void_p

import numpy as np
import xxhash

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libesoracle.so")


def build() -> None:
    subprocess.run(["make", "-B", "-C", HERE], check=True, stdout=subprocess.DEVNULL)


class Linear(ctypes.Structure):
    _fields_ = [("w", c_void_p), ("s", c_void_p), ("b", c_void_p), ("n", c_int), ("k", c_int)]


class Layer(ctypes.Structure):
    _fields_ = [("is_attention", c_int), ("input_norm", c_void_p), ("post_norm", c_void_p),
                ("gate", Linear), ("up", Linear), ("down", Linear),
                ("qkv", Linear), ("z", Linear), ("a", Linear), ("b", Linear), ("out", Linear),
                ("conv_w", c_void_p), ("gdn_norm", c_void_p), ("dt_bias", c_void_p), ("a_log", c_void_p),
                ("q", Linear), ("k", Linear), ("v", Linear), ("o", Linear),
                ("q_norm", c_void_p), ("k_norm", c_void_p)]


class Model(ctypes.Structure):
    _fields_ = [("n_layers", c_int), ("vocab", c_int), ("embed", Linear), ("final_norm", c_void_p),
                ("layers", Layer * 64)]


class State(ctypes.Structure):
    _fields_ = [("capacity", c_int), ("history", c_void_p * 64), ("state", c_void_p * 64),
                ("kcache", c_void_p * 64), ("vcache", c_void_p * 64)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing: run make -C oracle")
        L = ctypes.CDLL(LIB_PATH)
        vp = c_void_p
        sig = {
            "eo_bf16_to_f32": (c_float, [c_uint16]),
            "eo_f32_to_bf16": (c_uint16, [c_float]),
            "eo_round_bf16": (c_float, [c_float]),
            "eo_f32_to_bf16_array": (None, [vp, vp, ctypes.c_size_t]),
            "eo_bf16_to_f32_array": (None, [vp, vp, ctypes.c_size_t]),
            "eo_exp": (c_float, [c_float]),
            "eo_log": (c_float, [c_float]),
            "eo_sincos": (None, [c_float, POINTER(c_float), POINTER(c_float)]),
            "eo_sigmoid_bf": (c_float, [c_float]),
            "eo_softplus_bf": (c_float, [c_float]),
            "eo_rope_inv_freq": (c_float, [c_int]),
            "eo_embedding": (None, [vp, vp, vp, c_int, c_uint32, vp]),
            "eo_q4_matvec": (None, [vp, vp, vp, c_int, c_int, vp, vp, vp]),
            "eo_q4_matvec_add": (None, [vp, vp, vp, c_int, c_int, vp, vp, vp]),
            "eo_rms_norm": (None, [vp, vp, c_int, c_float, vp]),
            "eo_swiglu": (None, [vp, vp, c_int, vp]),
            "eo_gdn_conv_prepare": (None, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
            "eo_gdn_recur": (None, [vp, vp, vp, vp, vp]),
            "eo_gdn_norm_gate": (None, [vp, vp, vp, vp]),
            "eo_gdn_conv_prepare_rows": (None, [vp, vp, vp, vp, vp, vp, vp, c_int, vp, vp, vp]),
            "eo_gdn_recur_rows": (None, [vp, vp, vp, c_int, vp, vp]),
            "eo_gdn_norm_gate_rows": (None, [vp, vp, vp, c_int, vp]),
            "eo_attn_prepare": (None, [vp, vp, vp, vp, vp, vp, vp, vp, c_int, c_int]),
            "eo_attn_decode_single": (None, [vp, vp, vp, c_int, c_int, vp]),
            "eo_attn_decode_split": (None, [vp, vp, vp, c_int, c_int, vp, vp, vp]),
            "eo_attn_split_merge_gate": (None, [vp, vp, vp, vp, vp]),
            "eo_attn_gate": (None, [vp, vp, vp]),
            "eo_attn_decode_gated": (None, [vp, vp, vp, c_int, c_int, vp, vp]),
            "eo_greedy": (c_uint32, [vp, c_int, POINTER(c_float)]),
            "eo_model_step": (c_uint32, [POINTER(Model), POINTER(State), c_uint32, c_int, c_int, vp, vp]),
            "eo_num_threads": (c_int, []),
            "eo_set_num_threads": (None, [c_int]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def P(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ---- numerics helpers (numpy, independent of the C code) ----
def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().eo_f32_to_bf16_array(P(a), P(out), a.size)
    return out


def exp(x: float) -> float:
    return float(lib().eo_exp(x))


def log(x: float) -> float:
    return float(lib().eo_log(x))


def sincos(x: float):
    s, c = c_float(), c_float()
    lib().eo_sincos(x, ctypes.byref(s), ctypes.byref(c))
    return float(s.value), float(c.value)


def bf16_to_f32_c(a: np.ndarray) -> np.ndarray:
    """The oracle's own bf16 -> fp32 widening (checked against bf16_to_f32)."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().eo_bf16_to_f32_array(P(a), P(out), a.size)
    return out


# ---- op wrappers ----
def q4_matvec(codes, scales, biases, x, want_f32=False):
    n, k8 = codes.shape
    y = np.empty(n, dtype=np.uint16)
    yf = np.empty(n, dtype=np.float32)
    lib().eo_q4_matvec(P(codes), P(scales), P(biases), n, k8 * 8, P(x), P(y), P(yf))
    return (y, yf) if want_f32 else y


# ---- row-batched linear (prefill) ----
REF_CHUNK = 2048  # rows per prompt forward (model.rs:7, :106-109)


def linear_row_limit(n: int, k: int) -> int:
    """Model::linear's route switch (model.rs:189-192; MLX 0.32.4
    get_qmv_batch_limit for the reference's GPU): a forward of fewer rows runs
    the [n, k] linear as qmv_q4 rows (the decode matvec arithmetic, weights
    not rounded), otherwise as qmm_q4_nax (bf16-dequantised weights)."""
    if k <= 2048 and n <= 2048:
        return 33
    if k <= 4096 and n <= 4096:
        return 25
    return 13


def q4_matvec_rows(codes, scales, biases, x, residual=None):
    """qmv_q4 with M rows (linear.metal:28-73): each row is q4_matvec (with
    a residual, q4_matvec_add). x [rows, k] bf16 bits."""
    x = np.asarray(x, dtype=np.uint16)
    if residual is None:
        return np.stack([q4_matvec(codes, scales, biases, x[i]) for i in range(x.shape[0])])
    residual = np.asarray(residual, dtype=np.uint16)
    return np.stack([q4_matvec_add(codes, scales, biases, x[i], residual[i]) for i in range(x.shape[0])])


_DEQUANT_CACHE: dict = {}
_DEQUANT_CACHE_BYTES = 1 << 30


def _fingerprint(a):
    """64-bit hash of an array's bytes (a weight changed in place gets a new key)."""
    return xxhash.xxh3_64_intdigest(memoryview(np.ascontiguousarray(a)).cast("B"))


def _dequant_cached(codes, scales, biases):
    """q4_dequant_bf16 of a weight as fp64, kept (the codes array with it, so
    its address stays unique) until the cache passes 1 GiB, oldest first. The
    key holds the arrays' addresses and a hash of their contents, so a weight
    modified in place after its first use is dequantised again."""
    key = (codes.__array_interface__["data"][0], codes.shape, scales.__array_interface__["data"][0],
           biases.__array_interface__["data"][0], _fingerprint(codes), _fingerprint(scales), _fingerprint(biases))
    hit = _DEQUANT_CACHE.get(key)
    if hit is not None:
        return hit[0]
    w = q4_dequant_bf16(codes, scales, biases).astype(np.float64)
    _DEQUANT_CACHE[key] = (w, codes, scales, biases)
    while sum(v[0].nbytes for v in _DEQUANT_CACHE.values()) > _DEQUANT_CACHE_BYTES and len(_DEQUANT_CACHE) > 1:
        del _DEQUANT_CACHE[next(iter(_DEQUANT_CACHE))]
    return w


def q4_dequant_bf16(codes, scales, biases):
    """qmm_q4_nax's staged weights (linear_nax.metal:1118-1123): each weight
    dequantised as bf16(fp32(scale) * q + fp32(bias)). scale * q is exact in
    fp32 (8-bit by 4-bit significands), so the sum is rounded once, as a fused
    multiply-add would round it. Returns fp32 values of the bf16 weights [n, k]."""
    n, k8 = codes.shape
    k = k8 * 8
    shifts = np.arange(8, dtype=np.uint32) * 4
    q = ((codes[:, :, None] >> shifts[None, None, :]) & 15).reshape(n, k).astype(np.float32)
    s = np.repeat(bf16_to_f32(scales), 64, axis=1)
    b = np.repeat(bf16_to_f32(biases), 64, axis=1)
    return bf16_to_f32(f32_to_bf16(s * q + b))


def q4_gemm(codes, scales, biases, x, residual=None):
    """Row-batched linear of the prefill path (qmm_q4_nax, linear_nax.metal:
    1096-1140; model.rs:189-199): y[r] = bf16(sum_k x[r,k] * w[n,k]) over the
    bf16-dequantised weights, the sum taken in fp64 and rounded to fp32 before
    the bf16 round (the kernel accumulates in fp32 in its own order, so
    results agree to within the fp32 rounding of the sum); with a residual,
    bf16(residual + bf16(sum)). x: [rows, k] bf16 bits."""
    w = _dequant_cached(codes, scales, biases)
    xf = bf16_to_f32(np.asarray(x, dtype=np.uint16)).astype(np.float64)
    acc = (xf @ w.T).astype(np.float32)
    y = f32_to_bf16(acc)
    if residual is not None:
        y = f32_to_bf16(bf16_to_f32(np.asarray(residual, dtype=np.uint16)) + bf16_to_f32(y))
    return y


def attn_prefill(query, kcache, vcache, position, rows):
    """Causal GQA attention of a chunk (attn_prefill, attention_prefill.metal:
    2256; model.rs:337-343): row r (position position+r) attends to cache rows
    0..position+r of KV head h//4 with scale 1/16; the softmax is taken in
    fp64 and its probabilities rounded to bf16 before the product with V (the
    kernel's second product takes bf16 operands), normalised by the sum of the
    unrounded probabilities; output rounded to bf16. query [rows, 2048] bf16
    bits, caches [2, capacity, 256]; returns [rows, 2048] bf16 bits. The
    kernel keeps a running maximum per block of keys, so its probabilities
    carry different rounding: results agree to a stated tolerance. Rows are
    taken 256 at a time to bound the score matrix."""
    qf = bf16_to_f32(np.asarray(query, dtype=np.uint16)).astype(np.float64).reshape(rows, 8, 256)
    out = np.empty((rows, 8, 256), dtype=np.float64)
    n_all = position + rows
    for kvh in range(2):
        K = bf16_to_f32(kcache[kvh, :n_all]).astype(np.float64)
        V = bf16_to_f32(vcache[kvh, :n_all]).astype(np.float64)
        for r0 in range(0, rows, 256):
            r1 = min(rows, r0 + 256)
            q = qf[r0:r1, 4 * kvh:4 * kvh + 4].reshape(-1, 256)           # [(r, h), d]
            s = (q @ K.T).reshape(r1 - r0, 4, n_all) / 16.0
            mask = np.arange(n_all)[None, :] > (position + np.arange(r0, r1))[:, None]
            s[np.broadcast_to(mask[:, None, :], s.shape)] = -np.inf
            p = np.exp(s - s.max(axis=-1, keepdims=True))
            pb = bf16_to_f32(f32_to_bf16(p.astype(np.float32))).astype(np.float64)
            o = (pb.reshape(-1, n_all) @ V).reshape(r1 - r0, 4, 256)
            out[r0:r1, 4 * kvh:4 * kvh + 4] = o / p.sum(axis=-1, keepdims=True)
    return f32_to_bf16(out.astype(np.float32).reshape(rows, 2048))


def q4_matvec_add(codes, scales, biases, x, residual):
    n, k8 = codes.shape
    y = np.empty(n, dtype=np.uint16)
    lib().eo_q4_matvec_add(P(codes), P(scales), P(biases), n, k8 * 8, P(x), P(residual), P(y))
    return y


def embedding(codes, scales, biases, token):
    out = np.empty(1024, dtype=np.uint16)
    lib().eo_embedding(P(codes), P(scales), P(biases), 1024, int(token), P(out))
    return out


def rms_norm(x, gain, eps=1e-6):
    out = np.empty(x.size, dtype=np.uint16)
    lib().eo_rms_norm(P(x), P(gain), x.size, eps, P(out))
    return out


def swiglu(gate, up):
    out = np.empty(gate.size, dtype=np.uint16)
    lib().eo_swiglu(P(gate), P(up), gate.size, P(out))
    return out


def gdn_conv_prepare(raw, history, conv_w, a, b, a_log, dt_bias):
    """history [3,6144] is updated in place; returns conv_out, g, beta."""
    conv = np.empty(6144, dtype=np.uint16)
    g = np.empty(16, dtype=np.float32)
    beta = np.empty(16, dtype=np.uint16)
    lib().eo_gdn_conv_prepare(P(raw), P(history), P(conv_w), P(a), P(b), P(a_log), P(dt_bias), P(conv), P(g),
                              P(beta))
    return conv, g, beta


def gdn_recur(conv, g, beta, state):
    """state [16,128,128] fp32 updated in place; returns y [2048]."""
    y = np.empty(2048, dtype=np.uint16)
    lib().eo_gdn_recur(P(conv), P(g), P(beta), P(state), P(y))
    return y


def gdn_conv_prepare_rows(raw, history, conv_w, a, b, a_log, dt_bias):
    """gdn_conv_prepare over T tokens in order (history updated in place);
    returns conv [T,6144], g [T,16], beta [T,16]."""
    raw = np.ascontiguousarray(raw, dtype=np.uint16)
    T = raw.shape[0]
    conv = np.empty((T, 6144), dtype=np.uint16)
    g = np.empty((T, 16), dtype=np.float32)
    beta = np.empty((T, 16), dtype=np.uint16)
    lib().eo_gdn_conv_prepare_rows(P(raw), P(history), P(conv_w), P(np.ascontiguousarray(a)),
                                   P(np.ascontiguousarray(b)), P(a_log), P(dt_bias), T, P(conv), P(g), P(beta))
    return conv, g, beta


def gdn_recur_rows(conv, g, beta, state):
    """gdn_recur over T tokens in order (state updated in place); y [T,2048]."""
    T = conv.shape[0]
    y = np.empty((T, 2048), dtype=np.uint16)
    lib().eo_gdn_recur_rows(P(conv), P(g), P(beta), T, P(state), P(y))
    return y


def gdn_norm_gate_rows(y, z, w):
    T = y.shape[0]
    out = np.empty((T, 2048), dtype=np.uint16)
    lib().eo_gdn_norm_gate_rows(P(np.ascontiguousarray(y)), P(np.ascontiguousarray(z)), P(w), T, P(out))
    return out


def gdn_norm_gate(y, z, w):
    out = np.empty(2048, dtype=np.uint16)
    lib().eo_gdn_norm_gate(P(y), P(z), P(w), P(out))
    return out


def attn_prepare(q_proj, k, v, q_gain, k_gain, kcache, vcache, position, capacity):
    query = np.empty(2048, dtype=np.uint16)
    lib().eo_attn_prepare(P(q_proj), P(k), P(v), P(q_gain), P(k_gain), P(query), P(kcache), P(vcache), position,
                          capacity)
    return query


def attn_decode_single(query, kcache, vcache, length, capacity):
    out = np.empty(2048, dtype=np.uint16)
    lib().eo_attn_decode_single(P(query), P(kcache), P(vcache), length, capacity, P(out))
    return out


def attn_decode_split(query, kcache, vcache, length, capacity):
    partials = np.empty((8, 64, 256), dtype=np.uint16)
    sums = np.empty((8, 64), dtype=np.float32)
    maxs = np.empty((8, 64), dtype=np.float32)
    lib().eo_attn_decode_split(P(query), P(kcache), P(vcache), length, capacity, P(partials), P(sums), P(maxs))
    return partials, sums, maxs


def attn_split_merge_gate(partials, sums, maxs, q_proj):
    out = np.empty(2048, dtype=np.uint16)
    lib().eo_attn_split_merge_gate(P(partials), P(sums), P(maxs), P(q_proj), P(out))
    return out


def attn_gate(o, q_proj):
    out = np.empty(2048, dtype=np.uint16)
    lib().eo_attn_gate(P(o), P(q_proj), P(out))
    return out


def attn_decode_gated(query, kcache, vcache, length, capacity, q_proj):
    out = np.empty(2048, dtype=np.uint16)
    lib().eo_attn_decode_gated(P(query), P(kcache), P(vcache), length, capacity, P(q_proj), P(out))
    return out


def greedy(logits):
    lse = c_float()
    tok = lib().eo_greedy(P(logits), logits.size, ctypes.byref(lse))
    return int(tok), float(lse.value)


# ---- full model ----
class OracleModel:
    """Oracle model over a weight blob (host views), plus its decode state."""

    def __init__(self, views: dict, n_layers: int, vocab: int, capacity: int):
        self.views = views  # keep arrays alive
        self.n_layers, self.vocab, self.capacity = n_layers, vocab, capacity
        m = Model()
        m.n_layers, m.vocab = n_layers, vocab

        def lin(name, n, k):
            return Linear(P(views[name + ".weight"]), P(views[name + ".scales"]), P(views[name + ".biases"]), n, k)

        m.embed = lin("embed_tokens", vocab, 1024)
        m.final_norm = P(views["norm.weight"])
        self.history, self.state, self.kcache, self.vcache = {}, {}, {}, {}
        st = State()
        st.capacity = capacity
        for l in range(n_layers):
            p = f"layers.{l}"
            L = m.layers[l]
            L.is_attention = 1 if l % 4 == 3 else 0
            L.input_norm = P(views[p + ".input_layernorm.weight"])
            L.post_norm = P(views[p + ".post_attention_layernorm.weight"])
            L.gate = lin(p + ".mlp.gate_proj", 3584, 1024)
            L.up = lin(p + ".mlp.up_proj", 3584, 1024)
            L.down = lin(p + ".mlp.down_proj", 1024, 3584)
            if L.is_attention:
                a = p + ".self_attn"
                L.q = lin(a + ".q_proj", 4096, 1024)
                L.k = lin(a + ".k_proj", 512, 1024)
                L.v = lin(a + ".v_proj", 512, 1024)
                L.o = lin(a + ".o_proj", 1024, 2048)
                L.q_norm = P(views[a + ".q_norm.weight"])
                L.k_norm = P(views[a + ".k_norm.weight"])
                self.kcache[l] = np.zeros((2, capacity, 256), dtype=np.uint16)
                self.vcache[l] = np.zeros((2, capacity, 256), dtype=np.uint16)
                st.kcache[l] = P(self.kcache[l])
                st.vcache[l] = P(self.vcache[l])
            else:
                g = p + ".linear_attn"
                L.qkv = lin(g + ".in_proj_qkv", 6144, 1024)
                L.z = lin(g + ".in_proj_z", 2048, 1024)
                L.a = lin(g + ".in_proj_a", 16, 1024)
                L.b = lin(g + ".in_proj_b", 16, 1024)
                L.out = lin(g + ".out_proj", 1024, 2048)
                L.conv_w = P(views[g + ".conv1d.weight"])
                L.gdn_norm = P(views[g + ".norm.weight"])
                L.dt_bias = P(views[g + ".dt_bias"])
                L.a_log = P(views[g + ".A_log"])
                self.history[l] = np.zeros((3, 6144), dtype=np.uint16)
                self.state[l] = np.zeros((16, 128, 128), dtype=np.float32)
                st.history[l] = P(self.history[l])
                st.state[l] = P(self.state[l])
        self.m, self.st = m, st
        self.position = 0

    def reset(self):
        for a in self.history.values():
            a[...] = 0
        for a in self.state.values():
            a[...] = 0
        self.position = 0

    def snapshot(self):
        """Copy of the state a later step reads back (GDN histories and states,
        position). KV rows need no copy: a step writes its own row before it
        attends, so rows past the restored position are rewritten before use."""
        return ({l: a.copy() for l, a in self.history.items()}, {l: a.copy() for l, a in self.state.items()},
                self.position)

    def restore(self, snap):
        hist, state, pos = snap
        for l, a in hist.items():
            self.history[l][...] = a
        for l, a in state.items():
            self.state[l][...] = a
        self.position = pos

    def step(self, token: int, want_head: bool = True, want_logits: bool = False):
        logits = np.empty(self.vocab, dtype=np.uint16) if want_logits else None
        tok = lib().eo_model_step(ctypes.byref(self.m), ctypes.byref(self.st), int(token), self.position,
                                  1 if want_head else 0, P(logits), None)
        self.position += 1
        return (int(tok), logits) if want_logits else int(tok)

    def generate(self, prompt, count: int):
        """Model::generate(reset=True) (model.rs:97-122): consume prompt[:-1]
        as the reference's prompt loop does, then emit count greedy ids."""
        self.reset()
        self.consume_prompt(list(prompt[:-1]))
        return self.decode(prompt[-1], count)

    def generate_stepwise(self, prompt, count: int):
        """As generate, but the prompt is replayed one decode step per token
        (the engine's es_engine_set_prefill(0) mode)."""
        self.reset()
        for t in prompt[:-1]:
            self.step(t, want_head=False)
        return self.decode(prompt[-1], count)

    def decode(self, token: int, count: int):
        out = []
        tok = token
        for _ in range(count):
            tok = self.step(tok)
            out.append(tok)
        return out

    def consume_prompt(self, tokens):
        """The prompt loop of Model::generate (model.rs:106-109): forwards of
        REF_CHUNK rows from the current position, the last one shorter; a
        one-row forward runs the decode step without the head."""
        pos = 0
        while pos < len(tokens):
            r = min(REF_CHUNK, len(tokens) - pos)
            self.prefill(tokens[pos:pos + r])
            pos += r

    def _q4(self, name, n, k):
        v = self.views
        return (v[name + ".weight"].reshape(n, k // 8), v[name + ".scales"].reshape(n, k // 64),
                v[name + ".biases"].reshape(n, k // 64))

    def _linear(self, name, n, k, x, residual=None, gemm_only=False):
        """Model::linear over x.shape[0] rows (model.rs:189-198): qmv_q4 rows
        below the shape's row limit, else qmm_q4_nax; with a residual, the
        add_bf16 that follows it."""
        w = self._q4(name, n, k)
        if not gemm_only and x.shape[0] < linear_row_limit(n, k):
            return q4_matvec_rows(*w, x, residual)
        return q4_gemm(*w, x, residual=residual)

    def prefill(self, tokens, gemm_only=False):
        """Reference forward over len(tokens) prompt tokens from the current
        position, no output (model.rs:181-188 and encode_forward, model.rs:
        228-343). One row runs the decode step without the head (rows == 1).
        Otherwise: embedding rows; per layer RMSNorm rows, the linears routed
        by Model::linear (see _linear; gemm_only forces qmm_q4_nax for every
        linear, the route of every row of a full REF_CHUNK forward), GDN
        conv/prepare/recurrence/gated norm token by token or attention
        prepare/attn_prefill/gate, the residual add bf16(h + bf16(out)) of
        add_bf16 after the output linear, post-norm, gate/up linears, SwiGLU,
        down linear with its residual. Updates histories, states, caches and
        position."""
        if len(tokens) == 1 and not gemm_only:
            self.step(int(tokens[0]), want_head=False)
            return None
        v = self.views
        m = len(tokens)
        pos0 = self.position
        lin = lambda name, n, k, x, residual=None: self._linear(name, n, k, x, residual, gemm_only)
        emb = self._q4("embed_tokens", self.vocab, 1024)
        h = np.stack([embedding(*emb, int(t)) for t in tokens])
        for l in range(self.n_layers):
            p = f"layers.{l}"
            gain = v[p + ".input_layernorm.weight"]
            u = np.stack([rms_norm(h[i], gain) for i in range(m)])
            if l % 4 != 3:
                g = p + ".linear_attn"
                raw = lin(g + ".in_proj_qkv", 6144, 1024, u)
                z = lin(g + ".in_proj_z", 2048, 1024, u)
                a = lin(g + ".in_proj_a", 16, 1024, u)
                b = lin(g + ".in_proj_b", 16, 1024, u)
                conv, gg, beta = gdn_conv_prepare_rows(raw, self.history[l], v[g + ".conv1d.weight"], a, b,
                                                       v[g + ".A_log"], v[g + ".dt_bias"])
                y = gdn_recur_rows(conv, gg, beta, self.state[l])
                gated = gdn_norm_gate_rows(y, z, v[g + ".norm.weight"])
                h = lin(g + ".out_proj", 1024, 2048, gated, residual=h)
            else:
                a = p + ".self_attn"
                qp = lin(a + ".q_proj", 4096, 1024, u)
                kp = lin(a + ".k_proj", 512, 1024, u)
                vp = lin(a + ".v_proj", 512, 1024, u)
                query = np.stack([attn_prepare(qp[t], kp[t], vp[t], v[a + ".q_norm.weight"], v[a + ".k_norm.weight"],
                                               self.kcache[l], self.vcache[l], pos0 + t, self.capacity)
                                  for t in range(m)])
                o = attn_prefill(query, self.kcache[l], self.vcache[l], pos0, m)
                gated = np.stack([attn_gate(o[t], qp[t]) for t in range(m)])
                h = lin(a + ".o_proj", 1024, 2048, gated, residual=h)
            gain = v[p + ".post_attention_layernorm.weight"]
            u = np.stack([rms_norm(h[i], gain) for i in range(m)])
            act = swiglu(lin(p + ".mlp.gate_proj", 3584, 1024, u),
                         lin(p + ".mlp.up_proj", 3584, 1024, u)).reshape(m, 3584)
            h = lin(p + ".mlp.down_proj", 1024, 3584, act, residual=h)
        self.position += m
        return h

    def load_ring(self, layer: int, ring: np.ndarray, position: int):
        """Engine ring [4,6144] -> reference history [3,6144] at `position`."""
        for i in range(3):
            self.history[layer][i] = ring[(position - 3 + i) & 3]


def set_threads(n: int) -> None:
    lib().eo_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().eo_num_threads())

"""Python binding of the decode engine's C ABI (include/es_decode.h).

Loads libesdecode.so from this directory with ctypes. There is no fallback:
if the library is missing or a call fails, an exception is raised. Device
memory is managed through the library's own plumbing (es_malloc & co), so no
GPU framework is needed to drive the engine.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_size_t, c_uint32, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libesdecode.so")
SERVER_PATH = os.path.join(HERE, "es_server")

ES_OK, ES_ERR_INVALID, ES_ERR_DEVICE, ES_ERR_CANCELLED = 0, 1, 2, 3

HIDDEN, FFN, VOCAB, CAPACITY = 1024, 3584, 248320, 262144


class EsError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class Q4(ctypes.Structure):
    _fields_ = [("codes", c_void_p), ("scales", c_void_p), ("biases", c_void_p), ("n", c_int32), ("k", c_int32)]


_lib = None

_SIGNATURES = {
    "es_last_error": (c_char_p, []),
    "es_device_count": (c_int, [POINTER(c_int)]),
    "es_device_name": (c_int, [c_int, c_char_p, c_int]),
    "es_set_device": (c_int, [c_int]),
    "es_malloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "es_free": (c_int, [c_void_p]),
    "es_memcpy_htod": (c_int, [c_void_p, c_void_p, c_size_t]),
    "es_memcpy_dtoh": (c_int, [c_void_p, c_void_p, c_size_t]),
    "es_memset": (c_int, [c_void_p, c_int, c_size_t]),
    "es_copy_d2d": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "es_time_copy_d2d": (c_int, [c_void_p, c_void_p, c_size_t, c_int, POINTER(c_double)]),
    "es_time_read": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t, c_int, POINTER(c_double)]),
    "es_synchronize": (c_int, []),
    "es_stream_create": (c_int, [POINTER(c_void_p)]),
    "es_stream_destroy": (c_int, [c_void_p]),
    "es_stream_synchronize": (c_int, [c_void_p]),
    "es_embedding_q4": (c_int, [POINTER(Q4), c_void_p, c_void_p, c_void_p]),
    "es_q4_matvec": (c_int, [POINTER(Q4), c_void_p, c_void_p, c_void_p, c_void_p]),
    "es_q4_matvec_add": (c_int, [POINTER(Q4), c_void_p, c_void_p, c_void_p, c_void_p]),
    "es_q4_rmsnorm_matvec_multi": (c_int, [POINTER(Q4), c_int, c_void_p, c_void_p, c_void_p, POINTER(c_void_p), c_void_p]),
    "es_q4_rmsnorm_gate_up_swiglu": (c_int, [POINTER(Q4), POINTER(Q4), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "es_gdn_in_proj": (c_int, [POINTER(Q4), POINTER(Q4), POINTER(Q4), POINTER(Q4), c_void_p, c_void_p, c_void_p,
                               c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "es_gdn_recur_step": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_void_p]),
    "es_gdn_gate_out_proj": (c_int, [POINTER(Q4), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "es_rope_inv_freq": (c_int, [POINTER(c_float)]),
    "es_attn_scratch_bytes": (c_size_t, [c_int]),
    "es_attn_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                               c_void_p, c_int, c_void_p, c_size_t, c_void_p, c_void_p, c_void_p]),
    "es_head_scratch_bytes": (c_size_t, [c_int]),
    "es_head_greedy": (c_int, [POINTER(Q4), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p,
                               c_void_p, c_void_p]),
    "es_head_greedy_noalloc": (c_int, [POINTER(Q4), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p]),
    "es_weights_total_bytes": (c_size_t, [c_int, c_int]),
    "es_weights_tensor_count": (c_int, [c_int]),
    "es_weights_tensor_info": (c_int, [c_int, c_int, c_int, c_char_p, c_int, POINTER(c_uint64), POINTER(c_uint64),
                                       POINTER(c_int)]),
    "es_weights_random": (c_int, [c_int, c_int, c_uint64, c_void_p, c_size_t, c_int]),
    "es_q4_matvec_rows": (c_int, [POINTER(Q4), c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "es_linear_row_limit": (c_int, [c_int, c_int]),
    "es_add_bf16": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "es_greedy_bf16": (c_int, [c_void_p, c_int, c_void_p, c_size_t, c_void_p, c_void_p, c_void_p]),
    "es_gdn_conv": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "es_gdn_history": (c_int, [c_void_p, c_int, c_void_p, c_void_p]),
    "es_gdn_prepare": (c_int, [c_void_p] * 5 + [c_int, c_void_p, c_void_p, c_void_p]),
    "es_gdn_recur": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "es_q4_gemm": (c_int, [POINTER(Q4), c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "es_q4_gemm_swiglu": (c_int, [POINTER(Q4), POINTER(Q4), c_void_p, c_int, c_void_p, c_void_p]),
    "es_embed_rows": (c_int, [POINTER(Q4), c_void_p, c_int, c_void_p, c_void_p]),
    "es_rmsnorm_rows": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "es_swiglu_rows": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "es_gdn_prepare_rows": (c_int, [c_void_p] * 7 + [c_int, c_int] + [c_void_p] * 6),
    "es_gdn_recur_rows": (c_int, [c_void_p] * 5 + [c_int, c_void_p, c_void_p, c_void_p]),
    "es_gdn_norm_gate_rows": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "es_attn_prepare_rows": (c_int, [c_void_p] * 6 + [c_int, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "es_attn_prefill": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
    "es_attn_gate_rows": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "es_weights_tensor_shape": (c_int, [c_int, c_int, c_int, POINTER(ctypes.c_int64), c_int]),
    "es_checkpoint_config": (c_int, [c_char_p, POINTER(c_int), POINTER(c_int)]),
    "es_checkpoint_load": (c_int, [c_char_p, c_int, c_int, c_void_p, c_size_t]),
    "es_engine_create": (c_void_p, [c_void_p, c_size_t, c_int, c_int, c_int]),
    "es_engine_destroy": (None, [c_void_p]),
    "es_engine_generate": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "es_engine_set_prefill": (c_int, [c_void_p, c_int]),
    "es_engine_prompt_split": (c_int, [c_void_p, POINTER(c_int), POINTER(c_int), POINTER(c_int)]),
    "es_engine_xcd_kernels": (c_int, [c_void_p]),
    "es_engine_set_xcd_kernels": (c_int, [c_void_p, c_int]),
    "es_engine_inject_exchange_fault": (c_int, [c_void_p, c_int]),
    "es_engine_cancel": (None, [c_void_p]),
    "es_engine_clear_cancel": (None, [c_void_p]),
    "es_engine_position": (c_int, [c_void_p]),
    "es_engine_forced_decode": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "es_engine_read_kv": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "es_engine_write_kv": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "es_engine_read_gdn": (c_int, [c_void_p, c_int, c_void_p, c_void_p]),
    "es_engine_write_gdn": (c_int, [c_void_p, c_int, c_void_p, c_void_p]),
    "es_engine_set_position": (c_int, [c_void_p, c_int, c_uint32]),
    "es_engine_fill_synthetic": (c_int, [c_void_p, c_int, c_uint64, c_uint32]),
    "es_engine_time_decode": (c_int, [c_void_p, c_int, c_int, POINTER(c_double)]),
    "es_engine_time_attention": (c_int, [c_void_p, c_int, c_int, c_int, POINTER(c_double)]),
    "es_engine_time_head": (c_int, [c_void_p, c_int, POINTER(c_double)]),
    "es_engine_splits_for": (c_int, [c_int]),
}


def lib():
    """The loaded libesdecode.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is missing: build it first (__graft_entry__.build())")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def exported_symbols():
    return sorted(_SIGNATURES)


def check(rc: int) -> None:
    if rc != ES_OK:
        raise EsError(rc, lib().es_last_error().decode())


def device_count() -> int:
    n = c_int(0)
    check(lib().es_device_count(ctypes.byref(n)))
    return n.value


def device_name(dev: int = 0) -> str:
    buf = ctypes.create_string_buffer(256)
    check(lib().es_device_name(dev, buf, 256))
    return buf.value.decode()


def synchronize() -> None:
    check(lib().es_synchronize())


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class DeviceBuffer:
    """A device allocation owned by Python (freed on close/GC)."""

    def __init__(self, nbytes: int):
        p = c_void_p()
        check(lib().es_malloc(ctypes.byref(p), max(1, int(nbytes))))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_numpy(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes)
        if arr.nbytes:
            check(lib().es_memcpy_htod(b.ptr, _ptr(arr), arr.nbytes))
        return b

    @classmethod
    def zeros(cls, nbytes: int) -> "DeviceBuffer":
        b = cls(nbytes)
        check(lib().es_memset(b.ptr, 0, b.nbytes))
        return b

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        check(lib().es_memcpy_htod(self.ptr + offset, _ptr(arr), arr.nbytes))

    def numpy(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        if out.nbytes:
            check(lib().es_memcpy_dtoh(_ptr(out), self.ptr + offset, out.nbytes))
        return out

    def fill(self, value: int = 0) -> None:
        check(lib().es_memset(self.ptr, value, self.nbytes))

    def close(self) -> None:
        if getattr(self, "ptr", None):
            lib().es_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceQ4:
    """A Q4 weight triple resident on the device."""

    def __init__(self, codes: np.ndarray, scales: np.ndarray, biases: np.ndarray):
        n, k8 = codes.shape
        self.n, self.k = int(n), int(k8 * 8)
        assert scales.shape == (n, self.k // 64) and biases.shape == (n, self.k // 64)
        self.codes = DeviceBuffer.from_numpy(codes.astype(np.uint32))
        self.scales = DeviceBuffer.from_numpy(scales.astype(np.uint16))
        self.biases = DeviceBuffer.from_numpy(biases.astype(np.uint16))
        self.struct = Q4(self.codes.ptr, self.scales.ptr, self.biases.ptr, self.n, self.k)


# ---------------------------------------------------------------- weights
def weights_total_bytes(n_layers: int, vocab: int) -> int:
    return int(lib().es_weights_total_bytes(n_layers, vocab))


def weights_layout(n_layers: int, vocab: int):
    """[(name, offset, bytes, dtype)] with dtype 0 u32, 1 bf16, 2 f32."""
    out = []
    name = ctypes.create_string_buffer(256)
    off, nb, dt = c_uint64(), c_uint64(), c_int()
    for i in range(lib().es_weights_tensor_count(n_layers)):
        check(lib().es_weights_tensor_info(n_layers, vocab, i, name, 256, ctypes.byref(off), ctypes.byref(nb),
                                           ctypes.byref(dt)))
        out.append((name.value.decode(), off.value, nb.value, dt.value))
    return out


def random_weights(n_layers: int, vocab: int, seed: int, threads: int = 0) -> np.ndarray:
    total = weights_total_bytes(n_layers, vocab)
    blob = np.empty(total, dtype=np.uint8)
    check(lib().es_weights_random(n_layers, vocab, seed, _ptr(blob), total, threads))
    return blob


def weights_shapes(n_layers: int, vocab: int) -> list:
    """Checkpoint shape of every tensor, in blob order."""
    dims = (ctypes.c_int64 * 8)()
    out = []
    for i in range(lib().es_weights_tensor_count(n_layers)):
        nd = lib().es_weights_tensor_shape(n_layers, vocab, i, dims, 8)
        if nd < 0:
            check(nd)
        out.append(tuple(int(dims[j]) for j in range(nd)))
    return out


def checkpoint_config(model_dir: str) -> tuple:
    """(n_layers, vocab) of a checkpoint directory's config.json (Weights::load checks)."""
    n, v = c_int(), c_int()
    check(lib().es_checkpoint_config(os.fsencode(model_dir), ctypes.byref(n), ctypes.byref(v)))
    return n.value, v.value


def load_checkpoint(model_dir: str, n_layers: int, vocab: int) -> np.ndarray:
    """Weight blob filled from the directory's *.safetensors files."""
    total = weights_total_bytes(n_layers, vocab)
    blob = np.empty(total, dtype=np.uint8)
    check(lib().es_checkpoint_load(os.fsencode(model_dir), n_layers, vocab, _ptr(blob), total))
    return blob


def tensor_views(blob: np.ndarray, n_layers: int, vocab: int) -> dict:
    """name -> numpy view into the blob."""
    dt = {0: np.uint32, 1: np.uint16, 2: np.float32}
    views = {}
    for name, off, nb, d in weights_layout(n_layers, vocab):
        views[name] = blob[off:off + nb].view(dt[d])
    return views


# ---------------------------------------------------------------- engine
class Engine:
    """Model::load / generate / cancelled over the C ABI."""

    def __init__(self, blob: np.ndarray, n_layers: int, vocab: int, capacity: int = CAPACITY):
        self.n_layers, self.vocab, self.capacity = n_layers, vocab, capacity
        blob = np.ascontiguousarray(blob)
        h = lib().es_engine_create(_ptr(blob), blob.nbytes, n_layers, vocab, capacity)
        if not h:
            raise EsError(ES_ERR_INVALID, lib().es_last_error().decode())
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().es_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def position(self) -> int:
        return int(lib().es_engine_position(self.h))

    def generate(self, prompt, max_tokens: int, reset: bool) -> list:
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.uint32))
        out = np.zeros(max(1, max_tokens), dtype=np.uint32)
        check(lib().es_engine_generate(self.h, _ptr(p) if p.size else None, int(p.size), int(max_tokens),
                                       1 if reset else 0, _ptr(out)))
        return out[:max_tokens].tolist()

    def set_prefill(self, chunk_rows: int) -> None:
        """Prompt consumption: batched chunks of at most chunk_rows rows (>= 2),
        or 0 for one decode step per prompt token."""
        check(lib().es_engine_set_prefill(self.h, int(chunk_rows)))

    def xcd_kernels(self) -> bool:
        """Whether decode steps use the XCD-cooperative kernels."""
        r = lib().es_engine_xcd_kernels(self.h)
        if r < 0:
            raise EsError(-r, lib().es_last_error().decode())
        return bool(r)

    def set_xcd_kernels(self, on: bool) -> None:
        """Decode steps on the XCD-cooperative kernels (True) or on one launch
        per dependency (False); both give the same bits."""
        check(lib().es_engine_set_xcd_kernels(self.h, 1 if on else 0))

    def inject_exchange_fault(self, mode: int) -> None:
        """Test hook: 1 sets the device error word of the XCD-cooperative
        kernels, 2 moves one block's exchange count so the waits on its words
        run out; the next request then fails and the engine recovers."""
        check(lib().es_engine_inject_exchange_fault(self.h, int(mode)))

    def prompt_split(self):
        """(batched chunks, routed rows, decode rows) of the last reset request."""
        c, r, d = c_int(), c_int(), c_int()
        check(lib().es_engine_prompt_split(self.h, ctypes.byref(c), ctypes.byref(r), ctypes.byref(d)))
        return c.value, r.value, d.value

    def cancel(self):
        lib().es_engine_cancel(self.h)

    def clear_cancel(self):
        lib().es_engine_clear_cancel(self.h)

    def forced_decode(self, tokens, want_logits: bool = False):
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        am = np.zeros(t.size, dtype=np.uint32)
        lg = np.zeros((t.size, self.vocab), dtype=np.uint16) if want_logits else None
        check(lib().es_engine_forced_decode(self.h, _ptr(t), int(t.size), _ptr(am),
                                            _ptr(lg) if lg is not None else None))
        return (am, lg) if want_logits else am

    def read_kv(self, layer: int, which: int, pos0: int, count: int) -> np.ndarray:
        out = np.empty((2, count, 256), dtype=np.uint16)
        check(lib().es_engine_read_kv(self.h, layer, which, pos0, count, _ptr(out)))
        return out

    def write_kv(self, layer: int, which: int, pos0: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data, dtype=np.uint16)
        check(lib().es_engine_write_kv(self.h, layer, which, pos0, data.shape[1], _ptr(data)))

    def read_gdn(self, layer: int):
        ring = np.empty((4, 6144), dtype=np.uint16)
        state = np.empty((16, 128, 128), dtype=np.float32)
        check(lib().es_engine_read_gdn(self.h, layer, _ptr(ring), _ptr(state)))
        return ring, state

    def write_gdn(self, layer: int, ring: np.ndarray, state: np.ndarray) -> None:
        ring = np.ascontiguousarray(ring, dtype=np.uint16)
        state = np.ascontiguousarray(state, dtype=np.float32)
        check(lib().es_engine_write_gdn(self.h, layer, _ptr(ring), _ptr(state)))

    def set_position(self, position: int, pending: int) -> None:
        check(lib().es_engine_set_position(self.h, position, pending))

    def fill_synthetic(self, length: int, seed: int, pending: int) -> None:
        check(lib().es_engine_fill_synthetic(self.h, length, seed, pending))

    def time_decode(self, steps: int, warmup: int) -> float:
        ms = c_double()
        check(lib().es_engine_time_decode(self.h, steps, warmup, ctypes.byref(ms)))
        return ms.value

    ATTN_PARTS = {"all": 0, "chains": 1, "merge": 2}

    def time_attention(self, layer: int, reps: int, part: str = "all") -> float:
        """Average ms of one attention layer's launches (or of one of them)."""
        ms = c_double()
        check(lib().es_engine_time_attention(self.h, layer, reps, self.ATTN_PARTS[part], ctypes.byref(ms)))
        return ms.value

    def time_head(self, reps: int) -> float:
        ms = c_double()
        check(lib().es_engine_time_head(self.h, reps, ctypes.byref(ms)))
        return ms.value


def splits_for(length: int) -> int:
    return int(lib().es_engine_splits_for(length))


def time_read(nbytes: int, reps: int = 10) -> float:
    """Average ms of the streaming-read kernel (256 blocks, contiguous chunks
    by global->LDS DMA) over nbytes, a multiple of 2 MiB."""
    src, out = DeviceBuffer(nbytes), DeviceBuffer(8 << 20)
    ms = c_double()
    try:
        check(lib().es_memset(src.ptr, 1, nbytes))
        check(lib().es_time_read(src.ptr, nbytes, out.ptr, out.nbytes, reps, ctypes.byref(ms)))
    finally:
        src.close()
        out.close()
    return ms.value


def time_copy(nbytes: int, reps: int = 10) -> float:
    """Average ms of a device-to-device copy of nbytes by the plain copy kernel."""
    src, dst = DeviceBuffer(nbytes), DeviceBuffer(nbytes)
    ms = c_double()
    try:
        check(lib().es_time_copy_d2d(dst.ptr, src.ptr, nbytes, reps, ctypes.byref(ms)))
    finally:
        src.close()
        dst.close()
    return ms.value


def rope_inv_freq() -> np.ndarray:
    out = np.zeros(32, dtype=np.float32)
    check(lib().es_rope_inv_freq(out.ctypes.data_as(POINTER(c_float))))
    return out

"""Host-side logic on the CPU: the C ABI library loads and exports every
declared entry point, the weight blob layout matches the checkpoint's tensor
inventory (weights.rs:50-52, model.rs:41-78), the seeded random-init
generator is deterministic and quantises as MLX affine Q4 (group 64), and
bench.py refuses multi-GPU runs. Nothing here launches a kernel.
"""
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import esdecode as E
from conftest import PKG, ROOT
from helpers import dequant_f64, f32

HEADER = os.path.join(ROOT, "include", "es_decode.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(es_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = E.lib()
    names = declared_symbols()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_the_header():
    """The Python binding types exactly the header's entry points."""
    assert set(E.exported_symbols()) == set(declared_symbols())


def test_protocol_server_built():
    path = os.path.join(PKG, "es_server")
    assert os.path.exists(path) and os.access(path, os.X_OK)


def test_layout_full_model():
    lay = E.weights_layout(24, 248320)
    assert len(lay) == 694
    names = [n for n, _, _, _ in lay]
    assert len(set(names)) == len(names)
    assert "embed_tokens.weight" in names and "norm.weight" in names
    assert "layers.3.self_attn.q_proj.weight" in names
    assert "layers.0.linear_attn.in_proj_qkv.weight" in names
    assert "layers.0.linear_attn.A_log" in names
    # offsets ascend, 256-byte aligned, no overlap
    offs = np.array([o for _, o, _, _ in lay])
    sizes = np.array([b for _, _, b, _ in lay])
    assert np.all(offs % 256 == 0)
    assert np.all(offs[1:] >= offs[:-1] + sizes[:-1])
    data = sum(b for _, _, b, _ in lay)
    assert data == 423_938_240
    # per decode token: every tensor once plus the gathered embedding row
    # (512 B of codes + 2 x 32 B of scales/biases)
    assert data + 512 + 64 == 423_938_816
    assert E.weights_total_bytes(24, 248320) >= offs[-1] + sizes[-1]


def test_layout_q4_shapes():
    """Q4 triples: codes [N, K/8] u32, scales and biases [N, K/64] bf16."""
    lay = {n: (o, b, d) for n, o, b, d in E.weights_layout(24, 248320)}
    for base, n, k in [("embed_tokens", 248320, 1024), ("layers.0.mlp.down_proj", 1024, 3584),
                       ("layers.3.self_attn.q_proj", 4096, 1024), ("layers.0.linear_attn.in_proj_qkv", 6144, 1024),
                       ("layers.1.linear_attn.out_proj", 1024, 2048)]:
        assert lay[base + ".weight"][1] == n * k // 2 and lay[base + ".weight"][2] == 0
        assert lay[base + ".scales"][1] == n * k // 64 * 2 and lay[base + ".scales"][2] == 1
        assert lay[base + ".biases"][1] == n * k // 64 * 2 and lay[base + ".biases"][2] == 1


@pytest.fixture(scope="module")
def small_blob():
    return E.random_weights(4, 4096, seed=123, threads=4)


def test_random_init_is_deterministic(small_blob):
    again = E.random_weights(4, 4096, seed=123, threads=2)
    assert np.array_equal(small_blob, again), "thread count must not change the weights"
    other = E.random_weights(4, 4096, seed=124, threads=4)
    assert not np.array_equal(small_blob, other)


def test_random_init_quantisation(small_blob):
    """Dequantised weights look like N(0, 0.02) rows quantised per group of
    64: every group's codes span 0..15, dequantised values stay inside the
    group's [min, min + 15 scale]."""
    v = E.tensor_views(small_blob, 4, 4096)
    codes = v["layers.0.mlp.gate_proj.weight"].reshape(3584, 128)
    scales = v["layers.0.mlp.gate_proj.scales"].reshape(3584, 16)
    biases = v["layers.0.mlp.gate_proj.biases"].reshape(3584, 16)
    w = dequant_f64(codes[:256], scales[:256], biases[:256])
    assert abs(w.mean()) < 2e-3 and 0.015 < w.std() < 0.025
    shifts = np.arange(8, dtype=np.uint32) * 4
    q = ((codes[:64, :, None] >> shifts) & 15).reshape(64, 16, 64)
    assert np.all(q.min(2) == 0) and np.all(q.max(2) >= 14)
    assert np.all(f32(scales) > 0)


def test_random_init_other_tensors(small_blob):
    v = E.tensor_views(small_blob, 4, 4096)
    gain = f32(v["layers.0.input_layernorm.weight"])
    assert abs(gain.mean() - 1) < 0.02 and 0.05 < gain.std() < 0.15
    a_log = v["layers.0.linear_attn.A_log"]
    assert np.all(a_log >= np.log(0.5) - 1e-6) and np.all(a_log <= np.log(2.0) + 1e-6)
    assert f32(v["layers.0.linear_attn.conv1d.weight"]).size == 6144 * 4


def test_rope_frequencies_match_oracle():
    import oracle as O
    got = E.rope_inv_freq()
    want = np.array([O.lib().eo_rope_inv_freq(i) for i in range(32)], dtype=np.float32)
    assert np.array_equal(got, want)


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stdout

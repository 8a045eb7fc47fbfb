"""Checkpoint loading (Weights::load / take / linear / done, weights.rs:11-53;
tensor order and shapes model.rs:38-79): config.json checks, safetensors
parsing and validation with the reference's error messages, and byte-exact
placement of every tensor in the weight blob. CPU only: the loader is host
code; the files are synthetic (no checkpoint is available offline)."""
import os
import struct
import subprocess

import numpy as np
import pytest
import torch
from safetensors import safe_open

import esdecode as E
from checkpoint_files import PREFIX, model_entries, write_checkpoint, write_config, write_safetensors

SMALL = dict(n_layers=4, vocab=8192)   # layers 0-2 GDN, layer 3 attention
TINY = dict(n_layers=1, vocab=256)     # one GDN layer: error cases


@pytest.fixture(scope="module")
def small_blob():
    return E.random_weights(SMALL["n_layers"], SMALL["vocab"], seed=11)


@pytest.fixture(scope="module")
def tiny_blob():
    return E.random_weights(TINY["n_layers"], TINY["vocab"], seed=12)


def assert_same_tensors(got, want, n_layers, vocab):
    for (name, off, nb, _dt) in E.weights_layout(n_layers, vocab):
        assert np.array_equal(got[off:off + nb], want[off:off + nb]), name


def test_tensor_count_and_shapes_match_the_reference_model():
    """694 text tensors for 24 layers (weights.rs:42); conv1d is [6144,4,1] and
    A_log the only F32 tensor (model.rs:69-72)."""
    assert E.lib().es_weights_tensor_count(24) == 694
    shapes = dict(zip([t[0] for t in E.weights_layout(24, 248320)], E.weights_shapes(24, 248320)))
    dts = {t[0]: t[3] for t in E.weights_layout(24, 248320)}
    assert shapes["embed_tokens.weight"] == (248320, 128)
    assert shapes["embed_tokens.scales"] == (248320, 16)
    assert shapes["layers.0.linear_attn.conv1d.weight"] == (6144, 4, 1)
    assert shapes["layers.3.self_attn.q_proj.weight"] == (4096, 128)
    assert shapes["layers.3.self_attn.o_proj.scales"] == (1024, 32)
    assert shapes["layers.23.mlp.down_proj.weight"] == (1024, 448)
    assert [n for n, d in dts.items() if d == 2] == [f"layers.{l}.linear_attn.A_log" for l in range(24) if l % 4 != 3]


def test_written_files_read_back_with_safetensors(tmp_path, small_blob):
    """The test writer produces files the safetensors library reads with the
    blob's bytes, names, dtypes and shapes (pins the writer independently)."""
    write_checkpoint(str(tmp_path), small_blob, **SMALL)
    files = sorted(p for p in os.listdir(tmp_path) if p.endswith(".safetensors"))
    seen = {}
    for fname in files:
        with safe_open(str(tmp_path / fname), framework="pt") as f:
            assert f.metadata() == {"format": "mlx"}
            for k in f.keys():
                seen[k] = f.get_tensor(k)
    want = {e[0]: e for e in model_entries(small_blob, **SMALL)}
    assert set(want) <= set(seen)
    assert set(seen) - set(want) == {"vision_tower.patch_embed.weight", "language_model.lm_head.bias"}
    tdt = {"U32": torch.uint32, "BF16": torch.bfloat16, "F32": torch.float32}
    for name, (_, dtype, shape, data) in want.items():
        t = seen[name]
        assert t.dtype == tdt[dtype] and tuple(t.shape) == tuple(shape), name
        raw = t.contiguous().view(torch.uint8).numpy().tobytes()
        assert raw == data, name


def test_roundtrip_places_every_tensor(tmp_path, small_blob):
    write_checkpoint(str(tmp_path), small_blob, **SMALL, files=3)
    got = E.load_checkpoint(str(tmp_path), **SMALL)
    assert_same_tensors(got, small_blob, **SMALL)
    # alignment gaps between tensors are zero
    covered = np.zeros(got.size, dtype=bool)
    for (_, off, nb, _) in E.weights_layout(**SMALL):
        covered[off:off + nb] = True
    assert not got[~covered].any()


def test_full_model_roundtrip_and_config(tmp_path):
    """All 694 tensors of the 24-layer model through two files, with the
    config.json of the reference checkpoint."""
    blob = E.random_weights(24, 248320, seed=13, threads=8)
    write_checkpoint(str(tmp_path), blob, 24, 248320, files=2)
    write_config(str(tmp_path))
    n, v = E.checkpoint_config(str(tmp_path))
    assert (n, v) == (24, 248320)
    got = E.load_checkpoint(str(tmp_path), n, v)
    assert_same_tensors(got, blob, 24, 248320)


@pytest.mark.parametrize("cfg", [dict(hidden=2048), dict(layers=28), dict(vocab=151936)])
def test_config_rejects_other_models(tmp_path, cfg):
    write_config(str(tmp_path), **cfg)
    with pytest.raises(E.EsError, match="unsupported model configuration"):
        E.checkpoint_config(str(tmp_path))


def test_config_missing_or_without_text_config(tmp_path):
    with pytest.raises(E.EsError, match="config.json"):
        E.checkpoint_config(str(tmp_path))
    (tmp_path / "config.json").write_text('{"hidden_size": 1024, "num_hidden_layers": 24, "vocab_size": 248320}')
    with pytest.raises(E.EsError, match="unsupported model configuration"):
        E.checkpoint_config(str(tmp_path))


def _load_err(path):
    with pytest.raises(E.EsError) as ei:
        E.load_checkpoint(str(path), **TINY)
    return str(ei.value)


def _with(entries, name, dtype=None, shape=None, data=None):
    out = []
    for n, d, s, b in entries:
        if n == PREFIX + name:
            d, s, b = dtype or d, shape if shape is not None else s, data if data is not None else b
        out.append((n, d, s, b))
    return out


def test_no_safetensors_files(tmp_path):
    (tmp_path / "model.bin").write_bytes(b"x" * 16)
    assert "no safetensors weights" in _load_err(tmp_path)


def test_short_file_and_bad_header_length(tmp_path):
    (tmp_path / "a.safetensors").write_bytes(b"\x01\x02")
    assert "short safetensors file" in _load_err(tmp_path)
    (tmp_path / "a.safetensors").write_bytes(struct.pack("<Q", 100) + b"{}")
    assert "invalid safetensors header" in _load_err(tmp_path)
    (tmp_path / "a.safetensors").write_bytes(struct.pack("<Q", 4) + b"{no}")
    assert "invalid header" in _load_err(tmp_path)


def test_unsupported_dtype_and_bounds(tmp_path, tiny_blob):
    ents = model_entries(tiny_blob, **TINY)
    write_safetensors(str(tmp_path / "m.safetensors"), _with(ents, "norm.weight", dtype="F16"))
    assert "unsupported dtype F16" in _load_err(tmp_path)
    # data size disagreeing with the shape
    write_safetensors(str(tmp_path / "m.safetensors"), _with(ents, "norm.weight", shape=[1023]))
    assert "tensor bounds: norm.weight" in _load_err(tmp_path)


def test_range_past_the_data_section(tmp_path, tiny_blob):
    ents = model_entries(tiny_blob, **TINY)
    path = tmp_path / "m.safetensors"
    write_safetensors(str(path), ents)
    raw = path.read_bytes()
    # drop the last 2 bytes of data: the last tensor's range now ends past the file
    path.write_bytes(raw[:-2])
    assert f"tensor bounds: {ents[-1][0][len(PREFIX):]}" in _load_err(tmp_path)


def test_duplicate_across_files(tmp_path, tiny_blob):
    ents = model_entries(tiny_blob, **TINY)
    write_safetensors(str(tmp_path / "a.safetensors"), ents)
    write_safetensors(str(tmp_path / "b.safetensors"), [e for e in ents if e[0] == PREFIX + "norm.weight"])
    assert "duplicate tensor norm.weight" in _load_err(tmp_path)


def test_count_missing_and_renamed(tmp_path, tiny_blob):
    ents = model_entries(tiny_blob, **TINY)
    n = len(ents)
    write_safetensors(str(tmp_path / "m.safetensors"), [e for e in ents if e[0] != PREFIX + "norm.weight"])
    assert f"expected {n} text tensors, got {n - 1}" in _load_err(tmp_path)
    renamed = [(PREFIX + "norm.gain", d, s, b) if nm == PREFIX + "norm.weight" else (nm, d, s, b)
               for nm, d, s, b in ents]
    write_safetensors(str(tmp_path / "m.safetensors"), renamed)
    assert "missing norm.weight" in _load_err(tmp_path)


def test_wrong_shape_or_dtype(tmp_path, tiny_blob):
    ents = model_entries(tiny_blob, **TINY)
    conv = "layers.0.linear_attn.conv1d.weight"
    write_safetensors(str(tmp_path / "m.safetensors"), _with(ents, conv, shape=[6144, 4]))
    assert f"wrong shape/dtype for {conv}" in _load_err(tmp_path)
    # dt_bias (BF16 [16], 32 bytes) declared as F32 [8]: bounds hold, dtype and shape do not
    dt = "layers.0.linear_attn.dt_bias"
    write_safetensors(str(tmp_path / "m.safetensors"), _with(ents, dt, dtype="F32", shape=[8]))
    assert f"wrong shape/dtype for {dt}" in _load_err(tmp_path)


def test_skips_tensors_outside_the_model_prefix(tmp_path, tiny_blob):
    ents = model_entries(tiny_blob, **TINY)
    extra = [("vision_tower.x", "I8", [3], bytes(3)), ("language_model.lm_head.weight", "U32", [1], bytes(4))]
    write_safetensors(str(tmp_path / "m.safetensors"), extra + ents)
    got = E.load_checkpoint(str(tmp_path), **TINY)
    assert_same_tensors(got, tiny_blob, **TINY)


def test_protocol_server_rejects_a_bad_checkpoint(tmp_path):
    """Load failures end the server before hello with the loader's message
    (Model::load errors end main.rs before serving); no GPU is touched."""
    write_config(str(tmp_path), layers=28)
    p = subprocess.run([E.SERVER_PATH, "--model", str(tmp_path)], input="", capture_output=True, text=True,
                       timeout=60)
    assert p.returncode != 0
    assert "unsupported model configuration" in p.stderr
    write_config(str(tmp_path))
    p = subprocess.run([E.SERVER_PATH, "--model", str(tmp_path)], input="", capture_output=True, text=True,
                       timeout=60)
    assert p.returncode != 0
    assert "no safetensors weights" in p.stderr

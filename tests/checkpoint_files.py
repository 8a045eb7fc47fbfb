"""Writing synthetic MLX-style checkpoint directories (config.json and
*.safetensors) from a weight blob, for the checkpoint loader tests.

safetensors format: u64 little-endian header length, a JSON header mapping
tensor names to {"dtype", "shape", "data_offsets": [start, end]} (offsets
into the data section that follows; "__metadata__" is free-form), padded
with spaces to a multiple of 8 bytes, then the raw little-endian data.
"""
import json
import os
import struct

import esdecode as E

PREFIX = "language_model.model."
DTYPES = {0: "U32", 1: "BF16", 2: "F32"}


def write_safetensors(path, entries, metadata=None):
    """entries: [(full_name, dtype, shape, bytes)] written in order."""
    header, off = {}, 0
    for name, dtype, shape, data in entries:
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        off += len(data)
    if metadata is not None:
        header["__metadata__"] = metadata
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for _, _, _, data in entries:
            f.write(data)


def model_entries(blob, n_layers, vocab):
    """[(full_name, dtype, shape, bytes)] of every text tensor in the blob."""
    out = []
    for (name, off, nb, dt), shape in zip(E.weights_layout(n_layers, vocab), E.weights_shapes(n_layers, vocab)):
        out.append((PREFIX + name, DTYPES[dt], shape, blob[off:off + nb].tobytes()))
    return out


def write_config(model_dir, hidden=1024, layers=24, vocab=248320):
    cfg = {"model_type": "qwen3_5", "text_config": {"hidden_size": hidden, "num_hidden_layers": layers,
                                                    "vocab_size": vocab}}
    with open(os.path.join(model_dir, "config.json"), "w") as f:
        json.dump(cfg, f)


def write_checkpoint(model_dir, blob, n_layers, vocab, files=2, extra=True):
    """The blob's tensors spread over `files` safetensors files, plus
    (extra=True) tensors the loader must skip: a vision tower tensor in an
    unsupported dtype and a language_model.* tensor outside the model prefix."""
    os.makedirs(model_dir, exist_ok=True)
    ents = model_entries(blob, n_layers, vocab)
    per = (len(ents) + files - 1) // files
    for i in range(files):
        part = ents[i * per:(i + 1) * per]
        if extra and i == 0:
            part = part + [("vision_tower.patch_embed.weight", "F16", [4, 4], bytes(32)),
                           ("language_model.lm_head.bias", "F32", [2], bytes(8))]
        write_safetensors(os.path.join(model_dir, f"model-{i + 1:05d}-of-{files:05d}.safetensors"), part,
                          metadata={"format": "mlx"})

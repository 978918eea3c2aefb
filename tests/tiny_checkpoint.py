"""A tiny deterministic Safetensors checkpoint for the .xksv container tests.

Shapes and contents exercise every block kind the archive compiler writes
(src/compile.cpp:441-468): 16-row BF16 slabs of several widths, a tail slab
of fewer rows, a 1-D BF16 vector (one 1 x n slab), an incompressible BF16
matrix (raw fallback), non-BF16 tensors (raw 1 MiB blocks) and an asset.
The same bytes are produced everywhere (numpy PCG64 generators).
"""
from __future__ import annotations

import json
import struct
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "xks-vectorforge_amd"))
import xksv_synth as syn  # noqa: E402

CONFIG = {"model_type": "llama", "hidden_size": 1024, "num_hidden_layers": 1}


def tensors():
    """(name, safetensors dtype, shape, little-endian bytes) in file order."""
    out = [
        ("model.embed_tokens.weight", "BF16", (20, 1024), syn.normal_bf16(9001, (20, 1024))),
        ("model.layers.0.self_attn.q_proj.weight", "BF16", (16, 512), syn.normal_bf16(9002, (16, 512))),
        ("model.layers.0.mlp.down_proj.weight", "BF16", (16, 1536), syn.normal_bf16(9003, (16, 1536))),
        ("model.layers.0.mlp.gate_proj.weight", "BF16", (17, 48), syn.normal_bf16(9004, (17, 48))),
        ("model.layers.0.input_layernorm.weight", "BF16", (1024,), syn.normal_bf16(9005, (1024,), 0.05, 1.0)),
        ("model.norm.weight", "F32", (64,), np.random.default_rng(9006).standard_normal(64).astype("<f4")),
        ("model.rotary.inv_freq", "I64", (3,), np.array([1, 2, 3], "<i8")),
        ("lm_head.weight", "BF16", (24, 256), syn.uniform16(9008, (24, 256))),
    ]
    return [(n, d, s, np.ascontiguousarray(a).view(np.uint8).tobytes()) for n, d, s, a in out]


def header_bytes() -> bytes:
    """The Safetensors JSON header, padded with spaces to a multiple of 8 bytes."""
    hdr, at = {}, 0
    for name, dtype, shape, data in tensors():
        hdr[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [at, at + len(data)]}
        at += len(data)
    text = json.dumps(hdr, separators=(",", ":")).encode()
    return text + b" " * (-len(text) % 8)


def write(directory: Path) -> Path:
    """Write model.safetensors and config.json into `directory`; returns the directory."""
    directory.mkdir(parents=True, exist_ok=True)
    hdr = header_bytes()
    with open(directory / "model.safetensors", "wb") as f:
        f.write(struct.pack("<Q", len(hdr)) + hdr)
        for _, _, _, data in tensors():
            f.write(data)
    (directory / "config.json").write_text(json.dumps(CONFIG, indent=2) + "\n")
    return directory

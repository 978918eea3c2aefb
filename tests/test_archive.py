"""The .xksv container on the host (CPU only).

Pinned by archives the reference's own compiler wrote (tests/golden/tiny_*.xksv,
from tests/golden/make_archives.py with oracle/_ref/xksv-native built from the
reference's sources):
* the reader parses them: header, index, every tensor's blocks, and the block
  table it derives covers each tensor exactly;
* the writer reproduces their bytes exactly from the same checkpoint, under
  both codecs and for any worker count [src/compile.cpp:312-511,
  tests/test_inspect.cpp:77-85];
* every compressed block decodes (oracle) to the checkpoint's bytes with the
  index's SHA-256, and every tensor to its recorded digest;
* a malformed header or index is refused.
"""
from __future__ import annotations

import hashlib
import json
import struct
from pathlib import Path

import numpy as np
import pytest

import tiny_checkpoint
import xksv_archive as xa
import xksv_hip
from conftest import GOLDEN

ARCHIVES = {"dfloat11": GOLDEN / "tiny_serial.xksv", "dfloat11-parallel": GOLDEN / "tiny_parallel.xksv"}


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    return tiny_checkpoint.write(tmp_path_factory.mktemp("ckpt") / "model")


def _source_bytes():
    return {name: data for name, _, _, data in tiny_checkpoint.tensors()}


@pytest.mark.parametrize("codec", sorted(ARCHIVES))
def test_reader_blocks_decode_to_the_checkpoint(oracle, codec):
    arc = xa.Archive(ARCHIVES[codec])
    assert arc.index["codec_preference"] == codec
    src = _source_bytes()
    assert list(arc.tensors) == [n for n, _, _, _ in tiny_checkpoint.tensors()]
    for name, t in arc.tensors.items():
        assert t["role"] == xa.tensor_role(name)
        got = b""
        for b in t["blocks"]:
            blob = bytes(arc.read(b["offset"], b["size"]))
            if b["codec"] == "raw":
                data = blob
            elif b["codec"] == "bf16-huffman-parallel32":
                rc, data = oracle.unpack_parallel(blob)
                assert rc == 0
            else:
                rc, data = oracle.unpack(blob, b["rows"], b["cols"])
                assert rc == 0
            assert hashlib.sha256(data).hexdigest() == b["sha256"]
            got += data
        assert got == src[name] and hashlib.sha256(got).hexdigest() == t["sha256"]
    table, lo, hi, bases, total = arc.block_table(list(arc.tensors))
    assert len(table) == sum(len(t["blocks"]) for t in arc.tensors.values())
    assert lo >= 16 and hi <= arc.limit
    assert set(int(c) for c in table["codec"]) <= {0, xksv_hip.CODEC_SERIAL, xksv_hip.CODEC_PARALLEL}


@pytest.mark.parametrize("codec", sorted(ARCHIVES))
@pytest.mark.parametrize("workers", [1, 3])
def test_writer_reproduces_reference_archive(hip, ckpt, tmp_path, codec, workers):
    out = tmp_path / "model.xksv"
    n = xa.compile_checkpoint(hip, ckpt, out, codec, workers=workers)
    assert n == ARCHIVES[codec].stat().st_size
    assert out.read_bytes() == ARCHIVES[codec].read_bytes()
    with pytest.raises(xa.ArchiveError):  # never replaces an existing file
        xa.compile_checkpoint(hip, ckpt, out, codec)


def test_tensor_roles():
    assert xa.tensor_role("model.embed_tokens.weight") == "token_embedding"
    assert xa.tensor_role("lm_head.weight") == "language_model_head"
    assert xa.tensor_role("model.layers.0.linear_attn.conv1d.weight") == "deltanet_convolution"
    assert xa.tensor_role("model.layers.0.linear_attn.A_log") == "deltanet_state_parameter"
    assert xa.tensor_role("model.layers.0.self_attn.q_norm.weight") == "attention_parameter"
    assert xa.tensor_role("model.layers.0.mlp.experts.0.up.weight") == "moe_expert"
    assert xa.tensor_role("model.layers.0.mlp.up_proj.weight") == "feed_forward_parameter"
    assert xa.tensor_role("model.norm.weight") == "normalization_parameter"
    assert xa.tensor_role("model.rotary.inv_freq") == "other"


def _rewrite(path: Path, tmp_path: Path, edit) -> Path:
    b = bytearray(path.read_bytes())
    edit(b)
    out = tmp_path / "edited.xksv"
    out.write_bytes(bytes(b))
    return out


def test_reader_rejects_malformed_archives(tmp_path):
    src = ARCHIVES["dfloat11-parallel"]
    (limit,) = struct.unpack_from("<Q", src.read_bytes(), 8)
    with pytest.raises(xa.ArchiveError):  # magic
        xa.Archive(_rewrite(src, tmp_path, lambda b: b.__setitem__(3, 0x57)))
    with pytest.raises(xa.ArchiveError):  # index offset past the end
        xa.Archive(_rewrite(src, tmp_path, lambda b: b.__setitem__(slice(8, 16), struct.pack("<Q", len(b) + 1))))
    with pytest.raises(xa.ArchiveError):  # index offset inside the header
        xa.Archive(_rewrite(src, tmp_path, lambda b: b.__setitem__(slice(8, 16), struct.pack("<Q", 8))))

    def dup(b):  # duplicate JSON key in the index
        text = bytes(b[limit:]).replace(b'"version":1', b'"version":1,"version":1')
        b[limit:] = text
    with pytest.raises(xa.ArchiveError):
        xa.Archive(_rewrite(src, tmp_path, dup))

    def version(b):
        b[limit:] = bytes(b[limit:]).replace(b'"version":1', b'"version":2')
    with pytest.raises(xa.ArchiveError):
        xa.Archive(_rewrite(src, tmp_path, version))

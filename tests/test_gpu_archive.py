"""The .xksv container through the GPU (GPU only).

* GPU-decode load [python/runtime.py:86-99] of archives the reference's
  compiler wrote: every tensor equals the checkpoint bit for bit;
* GPU verify [src/verify.cpp:121-307]: the golden archives verify, also
  against their source checkpoint; the reference's own corruption case
  (tests/test_inspect.cpp:60-73: a one-block raw archive whose first data byte
  is flipped) fails with a block checksum verdict; a flipped code byte the
  oracle rejects fails as a decode error; a flipped sign/mantissa byte decodes
  but fails the digest;
* ResidentLinear.from_archive: the layer's blocks (compressed and raw) from the
  archive, GEMV / GEMM against an fp64 product of the checkpoint's weight.
"""
from __future__ import annotations

import base64
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import tiny_checkpoint
import xksv_archive as xa
import xksv_hip
import xksv_synth as syn
import xksv_torch
from conftest import GOLDEN

pytestmark = pytest.mark.gpu
ARCHIVES = [GOLDEN / "tiny_serial.xksv", GOLDEN / "tiny_parallel.xksv"]


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    return tiny_checkpoint.write(tmp_path_factory.mktemp("ckpt") / "model")


@pytest.mark.parametrize("path", ARCHIVES, ids=lambda p: p.stem)
def test_gpu_load_is_bit_exact(hip, path):
    got = xa.load_tensors(hip, path)
    for name, dtype, shape, data in tiny_checkpoint.tensors():
        t = got[name]
        assert list(t.shape) == list(shape), name
        assert t.contiguous().view(torch.uint8).reshape(-1).cpu().numpy().tobytes() == data, name


@pytest.mark.parametrize("path", ARCHIVES, ids=lambda p: p.stem)
def test_gpu_verify_golden_archives(hip, ckpt, path):
    rep = xa.verify(hip, path)
    assert rep.ok, rep.failures
    assert rep.tensors == len(tiny_checkpoint.tensors())
    assert rep.bytes == sum(len(d) for *_, d in tiny_checkpoint.tensors())
    rep = xa.verify(hip, path, source=ckpt)
    assert rep.ok, rep.failures


def _inspect_test_archive(path: Path) -> Path:
    """The archive tests/test_inspect.cpp:60-67 writes: one BF16 tensor [2] stored as one
    raw block of 00 80 80 7f (SHA-256 3cace997...13bb)."""
    body = b"\x00\x80\x80\x7f"
    header = b'{"weight":{"dtype":"BF16","shape":[2],"data_offsets":[0,4]}}'
    digest = hashlib.sha256(body).hexdigest()
    assert digest.startswith("3cace997") and digest.endswith("13bb")
    index = {"version": 1, "format": "safetensors", "assets": [], "shards": [{
        "name": "model.safetensors", "header": base64.b64encode(header).decode(),
        "tensors": [{"name": "weight", "dtype": "BF16", "shape": [2], "start": 0, "size": 4, "sha256": digest,
                     "blocks": [{"offset": 16, "size": 4, "raw_size": 4, "codec": "raw", "sha256": digest}]}]}]}
    path.write_bytes(b"XKSV\x00\x01\r\n" + (20).to_bytes(8, "little") + body +
                     json.dumps(index, separators=(",", ":")).encode())
    return path


def test_gpu_verify_reference_corruption_case(hip, tmp_path):
    p = _inspect_test_archive(tmp_path / "model.xksv")
    assert xa.verify(hip, p).ok
    b = bytearray(p.read_bytes())
    b[16] ^= 1  # tests/test_inspect.cpp:72
    p.write_bytes(bytes(b))
    rep = xa.verify(hip, p)
    assert not rep.ok and rep.failures[0] == "block checksum failed: weight"
    assert rep.block_verdicts == {("weight", 0): xksv_hip.ERR_DIGEST}
    with pytest.raises(xa.ArchiveError):
        rep.raise_if_failed()


def _flip(src: Path, dst: Path, at: int) -> Path:
    b = bytearray(src.read_bytes())
    b[at] ^= 0xFF
    dst.write_bytes(bytes(b))
    return dst


def test_gpu_verify_corrupt_compressed_blocks(hip, oracle, tmp_path):
    """Per-block verdicts on the parallel archive's down_proj block: a code-bit flip
    the oracle rejects is a decode failure; a sign/mantissa flip decodes to wrong
    bytes and fails the digest; only that block is flagged."""
    src = GOLDEN / "tiny_parallel.xksv"
    arc = xa.Archive(src)
    name = "model.layers.0.mlp.down_proj.weight"
    b = arc.tensors[name]["blocks"][0]
    assert b["codec"] == "bf16-huffman-parallel32"
    blob = bytes(arc.read(b["offset"], b["size"]))
    back = next(k for k in range(2, 400)
                if oracle.unpack_parallel(blob[:-k] + bytes([blob[-k] ^ 0xFF]) + blob[len(blob) - k + 1:])[0])
    rep = xa.verify(hip, _flip(src, tmp_path / "code.xksv", b["offset"] + b["size"] - back))
    assert rep.failures == [f"block decoding failed: {name}"]
    assert list(rep.block_verdicts) == [(name, 0)] and rep.block_verdicts[(name, 0)] & xksv_hip.ERR_STREAM
    first_seg = 32 + 8 * int.from_bytes(blob[24:32], "little")
    rep = xa.verify(hip, _flip(src, tmp_path / "sm.xksv", b["offset"] + first_seg + 272 + 5))
    assert rep.failures == [f"block checksum failed: {name}"]
    assert rep.block_verdicts == {(name, 0): xksv_hip.ERR_DIGEST}


@pytest.mark.parametrize("path,name", [(GOLDEN / "tiny_parallel.xksv", "model.layers.0.mlp.down_proj.weight"),
                                       (GOLDEN / "tiny_serial.xksv", "model.embed_tokens.weight"),
                                       (GOLDEN / "tiny_parallel.xksv", "model.embed_tokens.weight")],
                         ids=["parallel-down", "serial-embed", "parallel-embed-raw-tail"])
@pytest.mark.parametrize("tokens", [1, 9])
@torch.no_grad()
def test_resident_linear_from_archive(hip, path, name, tokens):
    src = {n: (s, d) for n, _, s, d in tiny_checkpoint.tensors()}
    shape, data = src[name]
    w = np.frombuffer(data, np.uint16).reshape(shape)
    wt = torch.from_numpy(syn.bf16_to_f32(w).astype(np.float64)).to("cuda")
    rl = xksv_torch.ResidentLinear.from_archive(hip, path, name)
    x = torch.randn(tokens, shape[1], device="cuda", dtype=torch.float32)
    y = rl(x)
    want = x.double() @ wt.T
    assert (torch.linalg.norm(y.double() - want) / torch.linalg.norm(want)).item() <= 1e-5
    xb = x.to(torch.bfloat16)
    yb = rl(xb).float()  # bf16 in -> bf16 out: one final rounding, relative error <= 2^-8
    want = xb.double() @ wt.T
    assert (torch.linalg.norm(yb.double() - want) / torch.linalg.norm(want)).item() <= 2 ** -8
    assert torch.equal(rl.decode_weight().view(torch.int16).cpu(), torch.from_numpy(w.view(np.int16).copy()))
    rl.check_errors()

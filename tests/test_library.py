"""The product library on the host (CPU only, no GPU compute).

* libxksv_hip.so loads and exports every function include/xksv_hip.h declares,
  with the binding's signature table covering exactly that set;
* its host encoder (xksv_pack / xksv_pack_parallel, the archive compiler's
  per-slab step) is byte-identical to the reference on every golden case;
* xksv_encode_tensor applies the compiler's slab rule [src/compile.cpp:449-486]
  and reproduces the reference's per-slab encoded digests of a 4096x4096
  N(0, 0.02) matrix under both codecs;
* every kernel addresses LDS with DS instructions (no FLAT memory operations,
  which fault on LDS addresses that are not naturally aligned).
"""
from __future__ import annotations

import json
import re
import subprocess

import numpy as np
import pytest

import xksv_hip
import xksv_synth as syn
from conftest import GOLDEN, PKG, ROOT
from oracle_lib import gen, raw_bytes, sha

HEADER = ROOT / "include" / "xksv_hip.h"


def _declared_functions() -> set:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return set(re.findall(r"\b(xksv_[a-z0-9_]+)\s*\(", text))


def test_exports_every_declared_symbol(hip):
    declared = _declared_functions()
    assert len(declared) >= 24
    assert declared == set(xksv_hip.EXPORTS)
    for name in sorted(declared):
        assert getattr(hip.lib, name) is not None, name
    assert hip.lib.xksv_hip_version() >= 1


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(xksv_hip.XksvError):
        xksv_hip.Library(tmp_path / "libxksv_hip.so")


def test_host_encoder_matches_golden(hip, golden_cases):
    for case in golden_cases:
        raw = raw_bytes(gen(case["gen"]))
        rows, cols = case["rows"], case["cols"]
        for codec, op in (("serial", "xksv_pack"), ("parallel", "xksv_pack_parallel")):
            want = case[codec]
            rc, blob = hip.try_call(op, raw, rows, cols)
            assert (rc == 0) == (want["rc"] == 0), (codec, case["gen"])
            if rc == 0:
                assert len(blob) == want["size"] and sha(blob) == want["sha256"], (codec, case["gen"])


def test_encode_tensor_reproduces_reference_slabs(hip):
    slabs = json.loads((GOLDEN / "slabs_4096x4096_seed0.json").read_text())
    w = gen(slabs["gen"])
    for codec, key in ((xksv_hip.CODEC_SERIAL, "serial"), (xksv_hip.CODEC_PARALLEL, "parallel")):
        enc, table = hip.encode_tensor(w, codec)
        assert len(table) == 256
        assert (table["rows"] == 16).all() and (table["cols"] == 4096).all() and (table["codec"] == codec).all()
        assert (table["out_offset"] == np.arange(256) * 16 * 4096 * 2).all()
        for s, blk in enumerate(table):
            b = enc[blk["offset"]:blk["offset"] + blk["size"]].tobytes()
            assert [len(b), sha(b)] == slabs[key][s], (key, s)


@pytest.mark.parametrize("shape", [(40, 4096), (3, 14336), (4096,), (5, 7), (2, 600000)])
def test_encode_tensor_slabs_tile_the_tensor(hip, oracle, shape):
    """Blocks are contiguous, each <= 16 rows and <= 1 MiB, and decode (oracle) to their slice."""
    w = gen({"kind": "normal", "seed": 7, "shape": list(shape)})
    raw = raw_bytes(w)
    for codec in (xksv_hip.CODEC_SERIAL, xksv_hip.CODEC_PARALLEL):
        enc, table = hip.encode_tensor(w, codec)
        at = 0
        for blk in table:
            assert blk["out_offset"] == at
            piece = raw[at:at + blk["raw_size"]]
            b = enc[blk["offset"]:blk["offset"] + blk["size"]].tobytes()
            if blk["codec"] == xksv_hip.CODEC_RAW:
                assert b == piece and blk["rows"] == 0 and blk["cols"] == 0
            else:
                assert blk["rows"] <= 16 and blk["rows"] * blk["cols"] * 2 == blk["raw_size"] <= 1 << 20
                rc, out = (oracle.unpack_parallel(b) if blk["codec"] == xksv_hip.CODEC_PARALLEL
                           else oracle.unpack(b, int(blk["rows"]), int(blk["cols"])))
                assert rc == 0 and out == piece
            at += int(blk["raw_size"])
        assert at == len(raw)


def test_kernels_address_lds_without_flat_instructions(tmp_path):
    asm = tmp_path / "kernels.s"
    cmd = ["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-O3", "-std=c++17", "--cuda-device-only", "-S", "-o", str(asm),
           str(PKG / "csrc" / "xksv_kernels.hip")]
    subprocess.run(cmd, check=True, capture_output=True)
    text = asm.read_text()
    flat = [ln for ln in text.splitlines() if re.match(r"\s+flat_", ln)]
    assert not flat, flat[:5]
    assert "_ZN4xksv12_GLOBAL__N_117k_decode_parallel" in text
    # Private (scratch) memory: none in the per-wave decode kernels; the fused
    # GEMM item kernels and the workgroup serial decode, at their register
    # limit, may spill a few words outside the walk loops.
    kernels = re.findall(r"\.name:\s+(\S+)\n(?:.*\n)*?\s+\.private_segment_fixed_size:\s+(\d+)", text)
    assert kernels
    for name, size in kernels:
        assert int(size) == 0 or (("k_gemm_items" in name or "k_decode_serial_wg" in name) and int(size) <= 16), \
            (name, size)


@pytest.mark.parametrize("codec", [1, 2])
def test_encode_tensor_worker_count_determinism(hip, codec):
    """Encoded bytes and block table do not depend on the worker count
    (tests/test_inspect.cpp:77-85 pins the same for the compiler's Workers)."""
    w = syn.normal_bf16(31 + codec, (200, 4096))
    ref_enc, ref_table = hip.encode_tensor(w, codec, threads=1)
    for threads in (2, 3, 8):
        enc, table = hip.encode_tensor(w, codec, threads=threads)
        assert enc.tobytes() == ref_enc.tobytes() and table.tobytes() == ref_table.tobytes()


def test_encode_tensor_rejects_odd_bf16_byte_count(hip):
    """An odd byte count cannot be BF16 words: the encoder refuses it (a 1-byte tail
    would fit no slab) instead of looping."""
    import ctypes
    data = np.zeros(4097, np.uint8)
    out, size = ctypes.c_void_p(), ctypes.c_uint64()
    blocks, nblocks = ctypes.POINTER(xksv_hip.Block)(), ctypes.c_uint64()
    rc = hip.lib.xksv_encode_tensor(data.ctypes.data, data.nbytes, 1, 0, 2, 1, ctypes.byref(out),
                                    ctypes.byref(size), ctypes.byref(blocks), ctypes.byref(nblocks))
    assert rc == -1
    enc, table = hip.encode_tensor(data.view(np.uint8), 2, bf16=False)
    assert len(table) == 1 and table["codec"][0] == xksv_hip.CODEC_RAW and enc.tobytes() == data.tobytes()

"""Per-block SHA-256 of decoded bytes on the GPU (GPU only).

xksv_hip_plan_digests hashes every block's decoded bytes (the per-slab
digests of src/compile.cpp:255,443,489 that src/verify.cpp:262-273 checks).
Pinned against hashlib on: raw blocks of every length class of the padding
rule (r = n mod 64 below 56, exactly 55/56, 63/64/65, two-chunk padding) at
aligned and odd output offsets; whole tensors under both codecs; a damaged
block, whose digest must differ while the others stay exact; blocks of mixed
sizes, several to a hashing lane.
"""
from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

import xksv_hip
import xksv_synth as syn

pytestmark = pytest.mark.gpu

RAW = np.dtype(xksv_hip.BLOCK_DTYPE)


def _digests(plan, out, n):
    d = torch.zeros(n * 32, dtype=torch.uint8, device="cuda")
    plan.digests(out.data_ptr(), out.numel(), d.data_ptr(), d.numel())
    torch.cuda.synchronize()
    return [bytes(d[32 * i:32 * i + 32].cpu().numpy()) for i in range(n)]


@pytest.mark.parametrize("pad", [0, 3])
def test_raw_block_digests_match_hashlib(hip, pad):
    sizes = [1, 2, 55, 56, 57, 63, 64, 65, 119, 120, 127, 128, 1000, 4096, 131072, 131075]
    rng = np.random.default_rng(11 + pad)
    table = np.zeros(len(sizes), dtype=RAW)
    at, blobs = 0, []
    for i, n in enumerate(sizes):
        at += pad  # odd offsets exercise the unaligned loads
        blob = rng.integers(0, 256, n, dtype=np.uint8)
        table[i]["offset"] = at
        table[i]["size"] = n
        table[i]["raw_size"] = n
        table[i]["out_offset"] = at
        table[i]["codec"] = 0
        blobs.append((at, blob))
        at += n
    arc = np.zeros(at, dtype=np.uint8)
    for off, blob in blobs:
        arc[off:off + len(blob)] = blob
    d_arc = torch.from_numpy(arc).to("cuda")
    out = torch.zeros(at, dtype=torch.uint8, device="cuda")
    plan = xksv_hip.Plan(hip, table, at)
    plan.decode(d_arc.data_ptr(), out.data_ptr(), at)
    assert plan.errors()[0] == 0
    got = _digests(plan, out, len(sizes))
    for (off, blob), g in zip(blobs, got):
        assert g == hashlib.sha256(blob.tobytes()).digest(), len(blob)
    plan.close()


@pytest.mark.parametrize("codec", [1, 2])
@pytest.mark.parametrize("shape", [(64, 4096), (40, 14336), (3, 600000)])
def test_tensor_slab_digests(hip, codec, shape):
    w = syn.normal_bf16(sum(shape) + codec, shape)
    enc, table = hip.encode_tensor(w, codec)
    raw = w.tobytes()
    d_arc = torch.from_numpy(enc.copy()).to("cuda")
    out = torch.zeros(len(raw), dtype=torch.uint8, device="cuda")
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    plan.decode(d_arc.data_ptr(), out.data_ptr(), len(raw))
    assert plan.errors()[0] == 0
    got = _digests(plan, out, len(table))
    for t, g in zip(table, got):
        o, n = int(t["out_offset"]), int(t["raw_size"])
        assert g == hashlib.sha256(raw[o:o + n]).digest()
    plan.close()


def test_damaged_block_digest_differs(hip):
    w = syn.normal_bf16(9, (64, 4096))
    enc, table = hip.encode_tensor(w, 2)
    raw = w.tobytes()
    d_arc = torch.from_numpy(enc.copy()).to("cuda")
    out = torch.zeros(len(raw), dtype=torch.uint8, device="cuda")
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    plan.decode(d_arc.data_ptr(), out.data_ptr(), len(raw))
    out[int(table[2]["out_offset"]) + 7] ^= 1  # one bit of block 2's decoded bytes
    got = _digests(plan, out, len(table))
    for i, t in enumerate(table):
        o, n = int(t["out_offset"]), int(t["raw_size"])
        assert (got[i] == hashlib.sha256(raw[o:o + n]).digest()) == (i != 2)
    plan.close()


def test_packed_hashing_lanes(hip):
    """Blocks of mixed sizes in shuffled table order: the largest ones hashed alone, the smaller
    ones several to a lane (largest first, packed up to 0.6 of the largest); every digest lands
    in its own block's slot and equals hashlib's."""
    rng = np.random.default_rng(17)
    sizes = [458752] * 3 + [131072] * 40 + [65536] * 9 + [8192] * 7 + [1000, 57, 0, 3]
    rng.shuffle(sizes)
    table = np.zeros(len(sizes), dtype=RAW)
    at = 0
    for i, n in enumerate(sizes):
        table[i]["offset"] = table[i]["out_offset"] = at
        table[i]["size"] = table[i]["raw_size"] = n
        at += n + (-n % 16)  # keep most blocks 16-byte aligned
    data = rng.integers(0, 256, at, dtype=np.uint8)
    d_arc = torch.from_numpy(data).to("cuda")
    out = torch.zeros(at, dtype=torch.uint8, device="cuda")
    plan = xksv_hip.Plan(hip, table, at)
    plan.decode(d_arc.data_ptr(), out.data_ptr(), at)
    assert plan.errors()[0] == 0
    got = _digests(plan, out, len(sizes))
    for t, g in zip(table, got):
        o, n = int(t["out_offset"]), int(t["raw_size"])
        assert g == hashlib.sha256(data[o:o + n].tobytes()).digest(), n
    plan.close()

"""Llama-3-8B-shaped layer set under dfloat11-parallel through one plan (GPU only).

The whole-archive decode workload at the size of one decoder layer plus the
first 64 embedding slabs: q 4096x4096, k/v 1024x4096, o 4096x4096, gate/up
14336x4096, down 4096x14336 (16x14336 slabs), two RMSNorm vectors
1 + N(0, 0.05) (1x4096 slabs, which the slab rule leaves raw under
parallel32, src/compile.cpp:257-276,449-486) and 1024x4096 of the embedding.
Every block goes through one plan and one step, so the block queue sees 4096-
and 14336-wide XKSP2 blocks and raw blocks together.

Checked, as src/verify.cpp:239-273 checks an archive:
* the decoded bytes equal the inputs, byte for byte;
* every slab's SHA-256, computed on the GPU (xksv_hip_plan_digests), equals
  hashlib's digest of that slab of the input;
* the norm slabs are raw;
* a spread sample of blocks decoded by the oracle equals the GPU output.
"""
from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

import xksv_hip
import xksv_synth as syn

pytestmark = pytest.mark.gpu

LAYER = [(n, s) for n, s in syn.LLAMA3_8B_LAYER.items()]
EMBED_ROWS = 1024


def _tensors():
    out = [("embed_tokens", syn.normal_bf16(7000, (EMBED_ROWS, 4096)))]
    for i, (name, shape) in enumerate(LAYER):
        norm = name.endswith("norm")
        w = syn.normal_bf16(7001 + i, shape, 0.05, 1.0) if norm else syn.normal_bf16(7001 + i, shape)
        out.append((name, w))
    return out


@pytest.fixture(scope="module")
def layer_archive(hip):
    tensors = _tensors()
    encs, tables, arc_off, out_off, nblk = [], [], 0, 0, 0
    spans = {}
    for name, w in tensors:
        enc, table = hip.encode_tensor(w, xksv_hip.CODEC_PARALLEL)
        table = table.copy()
        table["offset"] += arc_off
        table["out_offset"] += out_off
        spans[name] = (nblk, len(table))
        nblk += len(table)
        encs.append(enc)
        tables.append(table)
        arc_off += enc.nbytes
        out_off += w.nbytes
    return tensors, np.concatenate(encs), np.concatenate(tables), out_off, spans


def test_llama3_layer_set_one_plan(hip, oracle, layer_archive):
    tensors, enc, table, total, spans = layer_archive
    widths = set(int(c) for c in table["cols"][table["codec"] == xksv_hip.CODEC_PARALLEL])
    assert widths == {4096, 14336}
    for name in ("input_layernorm", "post_attention_layernorm"):
        first, n = spans[name]
        assert n == 1 and table["codec"][first] == xksv_hip.CODEC_RAW, name
    print(f"[llama3 layer] {len(table)} blocks, {enc.nbytes} B encoded, {total} B decoded", flush=True)

    d_arc = torch.from_numpy(enc).to("cuda")
    d_out = torch.zeros(total, dtype=torch.uint8, device="cuda")
    d_dig = torch.zeros(32 * len(table), dtype=torch.uint8, device="cuda")
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    try:
        plan.decode(d_arc.data_ptr(), d_out.data_ptr(), total)
        plan.digests(d_out.data_ptr(), total, d_dig.data_ptr(), d_dig.numel())
        nbad, first, bits = plan.errors()
    finally:
        plan.close()
    assert nbad == 0, (first, bits)

    want = np.concatenate([w.reshape(-1) for _, w in tensors]).view(np.uint8)
    got = d_out.cpu().numpy()
    assert np.array_equal(got, want)

    digests = d_dig.cpu().numpy().reshape(-1, 32)
    for i, t in enumerate(table):
        o, r = int(t["out_offset"]), int(t["raw_size"])
        assert digests[i].tobytes() == hashlib.sha256(want[o:o + r].tobytes()).digest(), i

    par = np.flatnonzero(table["codec"] == xksv_hip.CODEC_PARALLEL)
    for i in par[np.linspace(0, len(par) - 1, 24).astype(int)]:
        t = table[i]
        blob = enc[int(t["offset"]):int(t["offset"] + t["size"])].tobytes()
        rc, ref = oracle.unpack_parallel(blob)
        o, r = int(t["out_offset"]), int(t["raw_size"])
        assert rc == 0 and ref == got[o:o + r].tobytes(), i

"""Fused decode-GEMM with bf16 activations (GPU only).

The layout is that of x @ W.T: X [batch, cols] bf16 row-major, Y [batch, rows]
fp32 row-major. The products use bf16 MFMA (v_mfma_f32_16x16x32_bf16) at every
batch when every substream covers whole 16x16 tiles; otherwise they use fp32
VALU FMAs. The check is the oracle's CPU decode followed by an fp64 GEMM
against the exact bf16 values of X. Tolerance: relative L2 error <= 2e-3 for
bf16 activations (the bf16-X bound of the path's parity contract), and every
run is also held to 1e-5. Both paths accumulate exactly-representable products
in fp32, so the real error is ~1e-7.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import xksv_hip
from oracle_lib import gen, raw_bytes

pytestmark = pytest.mark.gpu
TOL_BF16 = 2e-3
TOL_TIGHT = 1e-5


def _rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return np.linalg.norm(got - want) / (den if den else 1.0)


def _x_bf16(batch, cols, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randn(batch, cols, generator=g, device="cuda").to(torch.bfloat16).contiguous()


# 16x4096 and 16x8192: substreams of whole tiles (MFMA at every batch);
# 16x4112: unit-aligned but not tile-aligned (VALU at every batch);
# 7x19 and 5x4096: not 16-row slabs (decode to scratch + plain GEMM).
@pytest.mark.parametrize("rows,cols", [(16, 4096), (16, 8192), (16, 4112), (7, 19), (5, 4096)])
@pytest.mark.parametrize("batch", [1, 4, 8, 16, 24])
def test_parallel_gemm_bf16(hip, oracle, rows, cols, batch):
    w = gen({"kind": "normal", "seed": 500 + cols + batch, "shape": [rows, cols]})
    block = hip.call("xksv_pack_parallel", raw_bytes(w), rows, cols)
    x = _x_bf16(batch, cols, 7 + batch)
    y = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
    assert hip.gemm_parallel_bf16(block, batch, x.data_ptr(), y.data_ptr()) == 0
    want = oracle.gemm_f64(w, x.float().cpu().numpy().T.astype(np.float64)).T  # [batch, rows]
    err = _rel_l2(y.cpu().numpy(), want)
    assert err <= TOL_BF16 and err <= TOL_TIGHT, err
    y2 = torch.empty_like(y)
    assert hip.gemm_parallel_bf16(block, batch, x.data_ptr(), y2.data_ptr()) == 0
    assert torch.equal(y, y2)  # deterministic reduction order


def test_gemm_bf16_rejects_bad_input(hip):
    w = gen({"kind": "normal", "seed": 2, "shape": [16, 256]})
    block = hip.call("xksv_pack_parallel", raw_bytes(w), 16, 256)
    x = _x_bf16(8, 256, 1)
    y = torch.empty(8, 16, dtype=torch.float32, device="cuda")
    assert hip.lib.xksv_hip_gemm_parallel_bf16(block, len(block), 8, None, y.data_ptr()) == 1
    assert hip.gemm_parallel_bf16(block[:-1], 8, x.data_ptr(), y.data_ptr()) == 1
    assert hip.gemm_parallel_bf16(block, 0, x.data_ptr(), y.data_ptr()) == 1


@pytest.mark.parametrize("rows,cols,codec", [(512, 8192, 2), (64, 28672, 2), (256, 4096, 1), (40, 4096, 2)])
@pytest.mark.parametrize("batch", [1, 4, 8, 16])
def test_plan_gemm_bf16(hip, rows, cols, codec, batch):
    """Whole tensors at the Llama-3-70B slab widths (8192, 28672) through the plan.

    The 40-row tensor ends in an 8-row slab (decode to scratch); the serial
    tensor takes the MFMA consumer with one wave per slab."""
    g = torch.Generator(device="cuda")
    g.manual_seed(rows + cols + batch)
    wt = (torch.randn(rows, cols, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    words = wt.view(torch.int16).cpu().numpy().view(np.uint16)
    enc, table = hip.encode_tensor(words, codec)
    table["out_offset"] //= cols * 2  # GEMM plans index output rows
    arc = torch.from_numpy(enc).to("cuda")
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    x = _x_bf16(batch, cols, 3)
    y = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
    plan.gemm_bf16(arc.data_ptr(), x.data_ptr(), batch, y.data_ptr())
    assert plan.errors() == (0, -1, 0)
    want = (x.double() @ wt.double().T).cpu().numpy()
    err = _rel_l2(y.cpu().numpy(), want)
    assert err <= TOL_BF16 and err <= TOL_TIGHT, err
    plan.close()


@pytest.mark.parametrize("rows,cols", [(28672, 8192), (8192, 28672)])
def test_plan_gemm_bf16_70b_full_shapes(hip, rows, cols):
    """The Llama-3-70B MLP matrices at full size, N(0, 0.02) weights, batch 4 through the
    plan (MFMA consumer, codeword index), against fp64."""
    batch = 4
    g = torch.Generator(device="cuda")
    g.manual_seed(rows // 16 + cols)
    wt = (torch.randn(rows, cols, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    words = wt.view(torch.int16).cpu().numpy().view(np.uint16)
    enc, table = hip.encode_tensor(words, 2)
    table["out_offset"] //= cols * 2
    arc = torch.from_numpy(enc).to("cuda")
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    x = _x_bf16(batch, cols, 7)
    y = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
    plan.gemm_bf16(arc.data_ptr(), x.data_ptr(), batch, y.data_ptr())
    assert plan.errors() == (0, -1, 0)
    want = (x.double() @ wt.double().T).cpu().numpy()
    del wt
    err = _rel_l2(y.cpu().numpy(), want)
    assert err <= TOL_BF16 and err <= TOL_TIGHT, err
    plan.close()

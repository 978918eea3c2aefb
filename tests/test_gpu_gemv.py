"""Fused decode-GEMV/GEMM parity (GPU only).

Reference: cuda/decode.cu:28-45 (serial GEMV/GEMM), cuda/parallel.cu:27
(parallel GEMV); tests/test_cuda.py:24-43,66-74 shapes.  The check is the
oracle's CPU decode followed by an fp64 GEMM; tolerance: relative L2 error
<= 1e-5 for fp32 activations.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle_lib import gen, raw_bytes

pytestmark = pytest.mark.gpu
TOL_F32 = 1e-5


def _rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return np.linalg.norm(got - want) / (den if den else 1.0)


@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 19), (16, 32), (17, 33), (16, 4096), (32, 256)])
def test_serial_gemv(hip, oracle, rows, cols):
    w = gen({"kind": "normal", "seed": rows * 1000 + cols, "shape": [rows, cols]})
    block = hip.call("xksv_pack", raw_bytes(w), rows, cols)
    x = torch.randn(cols, dtype=torch.float32, device="cuda")
    y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    assert hip.gemv(block, rows, cols, x.data_ptr(), y.data_ptr()) == 0
    want = oracle.gemm_f64(w, x.cpu().numpy())
    assert _rel_l2(y.cpu().numpy(), want) <= TOL_F32
    # tests/test_cuda.py:31-33 tolerance, elementwise
    np.testing.assert_allclose(y.cpu().numpy(), want, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("rows,cols,batch", [(3, 7, 2), (17, 33, 4), (16, 512, 5), (16, 256, 16), (16, 256, 17), (16, 128, 37)])
def test_serial_gemm(hip, oracle, rows, cols, batch):
    """tests/test_cuda.py:35-43: X [cols, batch], Y [rows, batch] row-major fp32."""
    w = gen({"kind": "normal", "seed": 3 + batch, "shape": [rows, cols]})
    block = hip.call("xksv_pack", raw_bytes(w), rows, cols)
    x = torch.randn(cols, batch, dtype=torch.float32, device="cuda")
    y = torch.full((rows, batch), float("nan"), dtype=torch.float32, device="cuda")
    assert hip.gemm(block, rows, cols, batch, x.data_ptr(), y.data_ptr()) == 0
    want = oracle.gemm_f64(w, x.cpu().numpy())
    assert _rel_l2(y.cpu().numpy(), want) <= TOL_F32


@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 19), (16, 256), (16, 4096), (16, 4097), (16, 14336), (5, 4096)])
def test_parallel_gemv(hip, oracle, rows, cols):
    """tests/test_cuda.py:66-74 shapes plus the Llama MLP slab width."""
    w = gen({"kind": "normal", "seed": 11 + cols, "shape": [rows, cols]})
    block = hip.call("xksv_pack_parallel", raw_bytes(w), rows, cols)
    x = torch.randn(cols, dtype=torch.float32, device="cuda")
    y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    assert hip.gemv_parallel(block, x.data_ptr(), y.data_ptr()) == 0
    want = oracle.gemm_f64(w, x.cpu().numpy())
    assert _rel_l2(y.cpu().numpy(), want) <= TOL_F32
    # determinism: the cross-substream reduction order is fixed
    y2 = torch.empty_like(y)
    assert hip.gemv_parallel(block, x.data_ptr(), y2.data_ptr()) == 0
    assert torch.equal(y, y2)


@pytest.mark.parametrize("batch", [2, 4, 8, 16, 17, 20, 33])
def test_parallel_gemm(hip, oracle, batch):
    rows, cols = 16, 4096
    w = gen({"kind": "normal", "seed": 100 + batch, "shape": [rows, cols]})
    block = hip.call("xksv_pack_parallel", raw_bytes(w), rows, cols)
    x = torch.randn(cols, batch, dtype=torch.float32, device="cuda")
    y = torch.full((rows, batch), float("nan"), dtype=torch.float32, device="cuda")
    assert hip.gemm_parallel(block, batch, x.data_ptr(), y.data_ptr()) == 0
    assert _rel_l2(y.cpu().numpy(), oracle.gemm_f64(w, x.cpu().numpy())) <= TOL_F32


def test_gemv_rejects_null_x_and_corrupt_block(hip):
    """cuda/decode.cu:90 (x == NULL -> 1) and a truncated block -> 1."""
    w = gen({"kind": "normal", "seed": 1, "shape": [16, 64]})
    block = hip.call("xksv_pack_parallel", raw_bytes(w), 16, 64)
    y = torch.empty(16, dtype=torch.float32, device="cuda")
    x = torch.randn(64, dtype=torch.float32, device="cuda")
    assert hip.gemv_parallel(block, 0, y.data_ptr()) != 0
    assert hip.gemv_parallel(block[:-1], x.data_ptr(), y.data_ptr()) != 0
    sblock = hip.call("xksv_pack", raw_bytes(w), 16, 64)
    assert hip.gemv(sblock, 16, 64, 0, y.data_ptr()) != 0
    assert hip.gemv(sblock[:-1], 16, 64, x.data_ptr(), y.data_ptr()) != 0

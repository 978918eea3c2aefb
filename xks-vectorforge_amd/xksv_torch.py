"""GPU-resident compressed weights for torch.nn.Linear (fused decode-GEMM).

The reference installs a fused decode-GEMV on a model's bf16 linear layers
(python/runtime.py:248-287, `install_fused_gemv`): for a one-token input it
reads the layer's .xksv blocks from the archive file and calls
`xksv_cuda_gemv[_parallel]` per block with host-staged bytes; every other
input shape falls back to `F.linear` on decoded weights.  Its GPU-decode load
(python/runtime.py:86-99) decodes each block with `xksv_cuda_decode[_parallel]`
into the parameter's storage.

Here the blocks of a layer stay resident in HBM and one plan call runs the
fused decode-GEMM for the whole layer and any batch: the input is taken as
bf16 X [tokens, in_features] (the layout of x @ W.T) and the product is
accumulated in fp32 (bf16 MFMA from 8 tokens, fp32 FMAs below).  The weight
is never materialised.  `ResidentLinear.decode_weight` and
`decode_into` are the GPU-decode load.

Numerics: each output is the fp32 sum of exact products of bf16 weights and
bf16 activations, so the result differs from torch's bf16 `F.linear` only by
the final rounding to the activation dtype and by summation order (the
reference's own fused path is likewise allowed to differ: its test bounds the
logits by atol = rtol = 0.03, tests/test_stream.py:54-62).
"""
from __future__ import annotations

import numpy as np
import torch

import xksv_hip

CODEC_SERIAL = 1
CODEC_PARALLEL = 2


def _words(weight: torch.Tensor) -> np.ndarray:
    """A bf16 weight as uint16 words (host copy)."""
    return weight.detach().to(torch.bfloat16).contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


class ResidentLinear(torch.nn.Module):
    """y = x @ W.T (+ bias) with W held as .xksv blocks in device memory.

    `enc` / `table` are one tensor's encoded bytes and block table as written
    by `Library.encode_tensor` (the compiler's slab rule); `table` offsets are
    relative to `enc`, `out_offset` in bytes of the row-major weight.
    """

    def __init__(self, lib: xksv_hip.Library, enc: np.ndarray, table: np.ndarray, out_features: int,
                 in_features: int, bias: torch.Tensor | None = None, device: str | torch.device = "cuda",
                 check: bool = True):
        super().__init__()
        self.lib = lib
        self.in_features, self.out_features = int(in_features), int(out_features)
        self.check = check
        self.archive = torch.from_numpy(np.ascontiguousarray(enc).view(np.uint8).reshape(-1).copy()).to(device)
        self._decode_table = np.ascontiguousarray(table).copy()
        gemm_table = self._decode_table.copy()
        if np.any(gemm_table["out_offset"] % (2 * self.in_features)):
            raise ValueError("blocks must cover whole weight rows")
        gemm_table["out_offset"] //= 2 * self.in_features  # GEMM plans index output rows
        gemm_table["cols"][gemm_table["codec"] == 0] = self.in_features  # raw blocks: give the row width
        self.plan = xksv_hip.Plan(lib, gemm_table, self.archive.numel())
        self._decode_plan = None
        self.bias = None if bias is None else torch.nn.Parameter(bias.detach().clone(), requires_grad=False)

    @classmethod
    def from_linear(cls, lib: xksv_hip.Library, linear: torch.nn.Linear, codec: int = CODEC_PARALLEL,
                    check: bool = True) -> "ResidentLinear":
        """Encode `linear.weight` (bf16) with the slab rule and keep the blocks in HBM."""
        w = linear.weight
        if w.dim() != 2:
            raise ValueError("weight must be 2-D")
        enc, table = lib.encode_tensor(_words(w), codec)
        return cls(lib, enc, table, w.shape[0], w.shape[1], linear.bias, w.device if w.is_cuda else "cuda", check)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.in_features:
            raise ValueError(f"expected last dimension {self.in_features}, got {x.shape[-1]}")
        lead = x.shape[:-1]
        xb = x.reshape(-1, self.in_features).to(torch.bfloat16).contiguous()
        batch = xb.shape[0]
        y = torch.empty(batch, self.out_features, dtype=torch.float32, device=xb.device)
        if batch:
            stream = torch.cuda.current_stream(xb.device).cuda_stream
            self.plan.gemm_bf16(self.archive.data_ptr(), xb.data_ptr(), batch, y.data_ptr(), stream)
            if self.check:
                n, first, bits = self.plan.errors(stream)
                if n:
                    raise xksv_hip.XksvError(f"fused decode-GEMM failed on block {first} (error bits {bits:#x})")
        if self.bias is not None:
            y += self.bias.float()
        return y.to(x.dtype).reshape(*lead, self.out_features)

    def _decoder(self) -> xksv_hip.Plan:
        if self._decode_plan is None:
            self._decode_plan = xksv_hip.Plan(self.lib, self._decode_table, self.archive.numel())
        return self._decode_plan

    def decode_into(self, out: torch.Tensor) -> None:
        """GPU decode of the resident blocks into a bf16 [out_features, in_features] tensor."""
        if out.dtype != torch.bfloat16 or out.shape != (self.out_features, self.in_features) or not out.is_contiguous():
            raise ValueError("out must be a contiguous bf16 tensor of the weight's shape")
        stream = torch.cuda.current_stream(out.device).cuda_stream
        plan = self._decoder()
        plan.decode(self.archive.data_ptr(), out.data_ptr(), out.numel() * 2, stream)
        n, first, bits = plan.errors(stream)
        if n:
            raise xksv_hip.XksvError(f"GPU decode failed on block {first} (error bits {bits:#x})")

    def decode_weight(self) -> torch.Tensor:
        w = torch.empty(self.out_features, self.in_features, dtype=torch.bfloat16, device=self.archive.device)
        self.decode_into(w)
        return w

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}, "
                f"encoded_bytes={self.archive.numel()}")


def install_resident_linear(model: torch.nn.Module, lib: xksv_hip.Library | None = None,
                            codec: int = CODEC_PARALLEL, skip: tuple[str, ...] = ("lm_head",),
                            check: bool = True) -> int:
    """Replace the bf16 2-D `nn.Linear` layers of `model` (except names in
    `skip`) by ResidentLinear; returns how many were replaced.  Mirrors the
    layer selection of python/runtime.py:253-261 (bf16 weights, no lm_head);
    layers with a bias are kept resident too and add it after the GEMM."""
    lib = lib or xksv_hip.Library()
    targets = [(name, m) for name, m in model.named_modules()
               if isinstance(m, torch.nn.Linear) and name.split(".")[-1] not in skip and name not in skip
               and m.weight.dtype == torch.bfloat16 and m.weight.dim() == 2]
    for name, m in targets:
        parent_name, _, leaf = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, leaf, ResidentLinear.from_linear(lib, m, codec, check))
    return len(targets)

"""GPU-resident compressed weights for torch.nn.Linear (fused decode-GEMM).

The reference installs a fused decode-GEMV on a model's bf16 linear layers
(python/runtime.py:248-287, `install_fused_gemv`): for a one-token input it
reads the layer's .xksv blocks from the archive file and calls
`xksv_cuda_gemv[_parallel]` per block with host-staged bytes; every other
input shape falls back to `F.linear` on decoded weights.  Its GPU-decode load
(python/runtime.py:86-99) decodes each block with `xksv_cuda_decode[_parallel]`
into the parameter's storage.

Here the blocks of a layer stay resident in HBM and one plan call runs the
fused decode-GEMM for the whole layer and any batch.  The weight is never
materialised.  Activations pick the path:
  * fp32 (and fp16) inputs take the fp32-X path, the reference's own numerics
    (fp32 x, fp32 accumulation, python/runtime.py:267): each output is the
    fp32 sum of exact products, rel-L2 <= 1e-5 against fp64;
  * bf16 inputs take the bf16-X path in the layout of x @ W.T (bf16 MFMA
    from 2 tokens, fp32 dot products for one), fp32 accumulation.
`ResidentLinear.decode_weight` / `decode_into` are the GPU-decode load, and
`from_archive` builds the layer from an .xksv archive's blocks.

A forward pass never synchronises the host: block errors are ORed into a
sticky device word (`xksv_hip_plan_error_flags`) that `check_errors()` reads,
so a forward can run under HIP graph capture.  `check=True` restores a
synchronous check after every forward.

Numerics of the bf16 path differ from torch's bf16 `F.linear` only by the
final rounding to the activation dtype and by summation order (the
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
                 check: bool = False):
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
        self._errors = torch.zeros(1, dtype=torch.int32, device=self.archive.device)  # sticky XKSV_ERR_* bits
        # The first GEMM call prepares the plan's routing (one synchronisation):
        # do it here, so that forward never synchronises.
        x0 = torch.zeros(self.in_features, dtype=torch.float32, device=self.archive.device)
        y0 = torch.empty(self.out_features, dtype=torch.float32, device=self.archive.device)
        stream = torch.cuda.current_stream(self.archive.device).cuda_stream
        self.plan.gemm(self.archive.data_ptr(), x0.data_ptr(), 1, y0.data_ptr(), stream)
        self.plan.error_flags(self._errors.data_ptr(), stream)

    @classmethod
    def from_archive(cls, lib: xksv_hip.Library, archive, name: str, bias: torch.Tensor | None = None,
                     device: str | torch.device = "cuda", check: bool = False) -> "ResidentLinear":
        """A 2-D BF16 tensor of an .xksv archive (path or xksv_archive.Archive), its blocks
        -- compressed and raw, as the index lists them -- copied to HBM once."""
        import xksv_archive
        arc = archive if isinstance(archive, xksv_archive.Archive) else xksv_archive.Archive(archive)
        t = arc.tensors.get(name)
        if t is None or t["dtype"] != "BF16" or len(t["shape"]) != 2:
            raise ValueError(f"{name} is not a 2-D BF16 tensor of the archive")
        table, lo, hi, _, _ = arc.block_table([name])
        return cls(lib, np.array(arc.read(lo, hi - lo)), table, t["shape"][0], t["shape"][1], bias, device, check)

    @classmethod
    def from_linear(cls, lib: xksv_hip.Library, linear: torch.nn.Linear, codec: int = CODEC_PARALLEL,
                    check: bool = False) -> "ResidentLinear":
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
        x2 = x.reshape(-1, self.in_features)
        batch = x2.shape[0]
        if x.dtype == torch.bfloat16:
            xb = x2.contiguous()
            y = torch.empty(batch, self.out_features, dtype=torch.float32, device=x.device)
        else:  # fp32 X [in_features, batch], Y [out_features, batch] (cuda/decode.cu:94 layout)
            xb = x2.float().t().contiguous() if batch > 1 else x2.float().contiguous()
            y = torch.empty(self.out_features, batch, dtype=torch.float32, device=x.device)
        if batch:
            stream = torch.cuda.current_stream(x.device).cuda_stream
            if x.dtype == torch.bfloat16:
                self.plan.gemm_bf16(self.archive.data_ptr(), xb.data_ptr(), batch, y.data_ptr(), stream)
            else:
                self.plan.gemm(self.archive.data_ptr(), xb.data_ptr(), batch, y.data_ptr(), stream)
            self.plan.error_flags(self._errors.data_ptr(), stream)
            if self.check:
                self.check_errors()
        if x.dtype != torch.bfloat16:
            y = y.t()
        if self.bias is not None:
            y = y + self.bias.float()
        return y.to(x.dtype).reshape(*lead, self.out_features)

    def check_errors(self) -> None:
        """Raise XksvError if any forward so far met a block that failed to decode
        (synchronises the current stream); the record is then cleared."""
        bits = int(self._errors.item())
        if bits:
            self._errors.zero_()
            raise xksv_hip.XksvError(f"fused decode-GEMM met a corrupt block (error bits {bits:#x})")

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
                            check: bool = False, archive=None) -> int:
    """Replace the bf16 2-D `nn.Linear` layers of `model` (except names in
    `skip`) by ResidentLinear; returns how many were replaced.  Mirrors the
    layer selection of python/runtime.py:253-261 (bf16 weights, no lm_head);
    layers with a bias are kept resident too and add it after the GEMM.  With
    `archive` (path or Archive), each layer's blocks come from the archive's
    `<name>.weight` tensor instead of encoding the module's weight."""
    lib = lib or xksv_hip.Library()
    targets = [(name, m) for name, m in model.named_modules()
               if isinstance(m, torch.nn.Linear) and name.split(".")[-1] not in skip and name not in skip
               and m.weight.dtype == torch.bfloat16 and m.weight.dim() == 2]
    if archive is not None:
        import xksv_archive
        archive = archive if isinstance(archive, xksv_archive.Archive) else xksv_archive.Archive(archive)
    done = 0
    for name, m in targets:
        parent_name, _, leaf = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        if archive is not None:  # the layer's blocks from the archive, as python/runtime.py:253-261 selects them
            t = archive.tensors.get(name + ".weight")
            if t is None or t["dtype"] != "BF16" or list(t["shape"]) != list(m.weight.shape):
                continue
            layer = ResidentLinear.from_archive(lib, archive, name + ".weight", m.bias, m.weight.device, check)
        else:
            layer = ResidentLinear.from_linear(lib, m, codec, check)
        setattr(parent, leaf, layer)
        done += 1
    return done

"""Deterministic synthetic BF16 inputs for the XKSV compressed-weight path.

All generators are numpy-only (PCG64 via ``numpy.random.default_rng``) so the
same seed gives the same bytes in this container, on the GPU host and in the
golden-fixture script.  BF16 words are produced from float32 with
round-to-nearest-even, the rounding ``torch.Tensor.to(torch.bfloat16)`` uses.

Workloads mirror the shapes the reference's tests and benchmarks use
(tests/test_cuda.py:13-74, python/bench_parallel_decode.py:11-13) and the
Llama-3 layer shapes the compressed path is measured on.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "f32_to_bf16", "bf16_to_f32", "normal_bf16", "student_t_bf16", "uniform_bf16",
    "words_mod", "uniform16", "exponent_pattern", "LLAMA3_8B_LAYER", "LLAMA3_70B_MLP",
]


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round-to-nearest-even; NaNs stay quiet NaNs."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    out = ((u + (((u >> 16) & 1) + np.uint32(0x7FFF))) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def bf16_to_f32(w: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> float32 values (exact: bits << 16)."""
    return (np.asarray(w, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def normal_bf16(seed: int, shape, sigma: float = 0.02, mean: float = 0.0) -> np.ndarray:
    """BF16 = RNE(float32 N(mean, sigma)); float32 draw via standard_normal(dtype=float32)."""
    rng = np.random.default_rng(seed)
    n = int(np.prod(shape))
    x = rng.standard_normal(n, dtype=np.float32) * np.float32(sigma)
    if mean:
        x = x + np.float32(mean)
    return f32_to_bf16(x).reshape(shape)


def student_t_bf16(seed: int, shape, nu: float = 3.0, scale: float = 0.02) -> np.ndarray:
    """Heavy-tailed exponents: RNE(float32(t_nu * scale))."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_t(nu, int(np.prod(shape))) * scale).astype(np.float32)
    return f32_to_bf16(x).reshape(shape)


def uniform_bf16(seed: int, shape, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.uniform(lo, hi, int(np.prod(shape))).astype(np.float32)
    return f32_to_bf16(x).reshape(shape)


def words_mod(shape) -> np.ndarray:
    """Words i % 65536 (tests/test_cuda.py:45): every exponent and mantissa appears."""
    n = int(np.prod(shape))
    return (np.arange(n, dtype=np.uint64) % 65536).astype(np.uint16).reshape(shape)


def uniform16(seed: int, shape) -> np.ndarray:
    """Uniform random 16-bit words (tests/test_cuda.py:15, mode 1): near-incompressible."""
    rng = np.random.default_rng(seed)
    return rng.integers(0, 65536, int(np.prod(shape)), dtype=np.uint16).reshape(shape)


def exponent_pattern(seed: int, shape) -> np.ndarray:
    """((127 + i % 3) << 7) | random mantissa (tests/test_cuda.py:15, mode 0): three symbols."""
    rng = np.random.default_rng(seed)
    n = int(np.prod(shape))
    i = np.arange(n, dtype=np.uint32)
    return (((127 + i % 3) << 7) | rng.integers(0, 128, n, dtype=np.uint32)).astype(np.uint16).reshape(shape)


# Llama-3-8B decoder layer (hidden 4096, 8 KV heads of 128, MLP 14336) and
# the Llama-3-70B MLP shapes (hidden 8192, MLP 28672).
LLAMA3_8B_LAYER = {
    "q_proj": (4096, 4096), "k_proj": (1024, 4096), "v_proj": (1024, 4096),
    "o_proj": (4096, 4096), "gate_proj": (14336, 4096), "up_proj": (14336, 4096),
    "down_proj": (4096, 14336), "input_layernorm": (4096,), "post_attention_layernorm": (4096,),
}
LLAMA3_8B_LAYERS = 32
LLAMA3_8B_EMBED = (128256, 4096)
LLAMA3_70B_MLP = {"gate_up": (28672, 8192), "down": (8192, 28672)}

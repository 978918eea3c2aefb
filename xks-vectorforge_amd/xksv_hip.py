"""ctypes binding of libxksv_hip.so (the MI355X XKSV compressed-weight path).

Mirrors the reference's Python contract (python/xksv.py:138-162 ``Native``:
``call(op, data, rows, cols)``, ``unpack_parallel(data)``) and the ctypes
bindings of the GPU library (tests/test_cuda.py:9-74, python/runtime.py:40-44),
so code written against the reference binds this library unchanged.  Device
pointers are plain integers (e.g. ``torch.Tensor.data_ptr()``).

The library is built in-tree by ``make -C xks-vectorforge_amd`` (or
``__graft_entry__.build()``).  Loading fails loudly if it is missing: there is
no CPU fallback for any decode entry point.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("XKSV_HIP_LIBRARY", HERE / "libxksv_hip.so"))

CODEC_RAW, CODEC_SERIAL, CODEC_PARALLEL = 0, 1, 2
CODEC_NAMES = {"raw": CODEC_RAW, "bf16-huffman-tile16": CODEC_SERIAL, "bf16-huffman-parallel32": CODEC_PARALLEL}
ERR_HEADER, ERR_CODEBOOK, ERR_STREAM, ERR_SHAPE, ERR_DIGEST = 1, 2, 4, 8, 16


class Block(ctypes.Structure):
    """xksv_hip_block: one block of an archive index."""
    _fields_ = [("offset", ctypes.c_uint64), ("size", ctypes.c_uint64), ("raw_size", ctypes.c_uint64),
                ("out_offset", ctypes.c_uint64), ("rows", ctypes.c_uint64), ("cols", ctypes.c_uint64),
                ("codec", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


BLOCK_DTYPE = np.dtype([("offset", "<u8"), ("size", "<u8"), ("raw_size", "<u8"), ("out_offset", "<u8"),
                        ("rows", "<u8"), ("cols", "<u8"), ("codec", "<u4"), ("reserved", "<u4")])
assert BLOCK_DTYPE.itemsize == ctypes.sizeof(Block)

_vp, _sz, _u64, _u32, _int = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int
_pvp, _psz = ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t)

_SIGNATURES = {
    "xksv_free": (None, [_vp]),
    "xksv_pack": (_int, [_vp, _sz, _sz, _sz, _pvp, _psz]),
    "xksv_unpack": (_int, [_vp, _sz, _sz, _sz, _pvp, _psz]),
    "xksv_pack_parallel": (_int, [_vp, _sz, _sz, _sz, _pvp, _psz]),
    "xksv_unpack_parallel": (_int, [_vp, _sz, _pvp, _psz]),
    "xksv_hip_decode": (_int, [_vp, _sz, _sz, _sz, _vp]),
    "xksv_hip_gemv": (_int, [_vp, _sz, _sz, _sz, _vp, _vp]),
    "xksv_hip_gemm": (_int, [_vp, _sz, _sz, _sz, _sz, _vp, _vp]),
    "xksv_hip_decode_parallel": (_int, [_vp, _sz, _vp]),
    "xksv_hip_gemv_parallel": (_int, [_vp, _sz, _vp, _vp]),
    "xksv_hip_gemm_parallel": (_int, [_vp, _sz, _sz, _vp, _vp]),
    "xksv_hip_gemm_parallel_bf16": (_int, [_vp, _sz, _sz, _vp, _vp]),
    "xksv_hip_gemm_parallel_noalloc": (_int, [_vp, _sz, _sz, _vp, _vp]),
    "xksv_cuda_decode": (_int, [_vp, _sz, _sz, _sz, _vp]),
    "xksv_cuda_gemv": (_int, [_vp, _sz, _sz, _sz, _vp, _vp]),
    "xksv_cuda_gemm": (_int, [_vp, _sz, _sz, _sz, _sz, _vp, _vp]),
    "xksv_cuda_decode_parallel": (_int, [_vp, _sz, _vp]),
    "xksv_cuda_gemv_parallel": (_int, [_vp, _sz, _vp, _vp]),
    "xksv_hip_plan_create": (_int, [ctypes.POINTER(Block), _sz, _u64, _pvp]),
    "xksv_hip_plan_destroy": (_int, [_vp]),
    "xksv_hip_plan_decode": (_int, [_vp, _vp, _vp, _u64, _vp]),
    "xksv_hip_plan_index": (_int, [_vp, _vp, _vp]),
    "xksv_hip_plan_gemm": (_int, [_vp, _vp, _vp, _sz, _vp, _vp]),
    "xksv_hip_plan_gemm_bf16": (_int, [_vp, _vp, _vp, _sz, _vp, _vp]),
    "xksv_hip_plan_errors": (ctypes.c_int64, [_vp, _vp, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(_u32)]),
    "xksv_hip_plan_digests": (ctypes.c_int, [_vp, _vp, _u64, _vp, _u64, _vp]),
    "xksv_hip_plan_verify": (ctypes.c_int, [_vp, _vp, _u64, _vp, _u64, _vp, _vp]),
    "xksv_hip_plan_error_flags": (ctypes.c_int, [_vp, _vp, _vp]),
    "xksv_encode_tensor": (_int, [_vp, _u64, _int, _u64, _u32, _u32, _pvp, ctypes.POINTER(_u64),
                                  ctypes.POINTER(ctypes.POINTER(Block)), ctypes.POINTER(_u64)]),
    "xksv_hip_version": (_int, []),
    "xksv_hip_device_cus": (_int, []),
}
EXPORTS = tuple(_SIGNATURES)


class XksvError(RuntimeError):
    pass


class Library:
    """Handle on libxksv_hip.so with the reference's calling conventions."""

    def __init__(self, path: Path | str = LIB_PATH):
        path = Path(path)
        if not path.exists():
            raise XksvError(f"{path} is not built; run `make -C {HERE}` (no CPU fallback exists)")
        self.path = path
        self.lib = ctypes.CDLL(str(path))
        for name, (res, args) in _SIGNATURES.items():
            f = getattr(self.lib, name)
            f.restype = res
            f.argtypes = args

    # -- reference python/xksv.py:154-162 (Native.call / unpack_parallel) --
    def call(self, op: str, data: bytes, rows: int, cols: int) -> bytes:
        rc, out = self.try_call(op, data, rows, cols)
        if rc:
            raise XksvError(f"native {op} failed")
        return out

    def try_call(self, op: str, data: bytes, rows: int, cols: int):
        buf = ctypes.create_string_buffer(bytes(data), max(len(data), 1))
        out, size = ctypes.c_void_p(), ctypes.c_size_t()
        rc = getattr(self.lib, op)(buf, len(data), rows, cols, ctypes.byref(out), ctypes.byref(size))
        if rc:
            return rc, None
        try:
            return 0, ctypes.string_at(out, size.value)
        finally:
            self.lib.xksv_free(out)

    def unpack_parallel(self, data: bytes) -> bytes:
        rc, out = self.try_unpack_parallel(data)
        if rc:
            raise XksvError("parallel block decode failed")
        return out

    def try_unpack_parallel(self, data: bytes):
        buf = ctypes.create_string_buffer(bytes(data), max(len(data), 1))
        out, size = ctypes.c_void_p(), ctypes.c_size_t()
        rc = self.lib.xksv_unpack_parallel(buf, len(data), ctypes.byref(out), ctypes.byref(size))
        if rc:
            return rc, None
        try:
            return 0, ctypes.string_at(out, size.value)
        finally:
            self.lib.xksv_free(out)

    # -- GPU block entries (device pointers as ints) --
    def decode(self, block: bytes, rows: int, cols: int, out_ptr: int) -> int:
        return self.lib.xksv_hip_decode(ctypes.create_string_buffer(bytes(block), max(len(block), 1)), len(block),
                                        rows, cols, out_ptr)

    def decode_parallel(self, block: bytes, out_ptr: int) -> int:
        return self.lib.xksv_hip_decode_parallel(ctypes.create_string_buffer(bytes(block), max(len(block), 1)),
                                                 len(block), out_ptr)

    def gemv(self, block: bytes, rows: int, cols: int, x_ptr: int, y_ptr: int) -> int:
        return self.lib.xksv_hip_gemv(ctypes.create_string_buffer(bytes(block), max(len(block), 1)), len(block),
                                      rows, cols, x_ptr, y_ptr)

    def gemm(self, block: bytes, rows: int, cols: int, batch: int, x_ptr: int, y_ptr: int) -> int:
        return self.lib.xksv_hip_gemm(ctypes.create_string_buffer(bytes(block), max(len(block), 1)), len(block),
                                      rows, cols, batch, x_ptr, y_ptr)

    def gemv_parallel(self, block: bytes, x_ptr: int, y_ptr: int) -> int:
        return self.lib.xksv_hip_gemv_parallel(ctypes.create_string_buffer(bytes(block), max(len(block), 1)),
                                               len(block), x_ptr, y_ptr)

    def gemm_parallel(self, block: bytes, batch: int, x_ptr: int, y_ptr: int) -> int:
        return self.lib.xksv_hip_gemm_parallel(ctypes.create_string_buffer(bytes(block), max(len(block), 1)),
                                               len(block), batch, x_ptr, y_ptr)

    def gemm_parallel_noalloc(self, block: bytes, batch: int, x_ptr: int, y_ptr: int) -> int:
        """xksv_hip_gemm_parallel staged in the library's fixed device array (no allocation)."""
        return self.lib.xksv_hip_gemm_parallel_noalloc(ctypes.create_string_buffer(bytes(block), max(len(block), 1)),
                                                       len(block), batch, x_ptr, y_ptr)

    def gemm_parallel_bf16(self, block: bytes, batch: int, x_ptr: int, y_ptr: int) -> int:
        """bf16 X [batch, cols] -> fp32 Y [batch, rows] (layout of x @ W.T)."""
        return self.lib.xksv_hip_gemm_parallel_bf16(ctypes.create_string_buffer(bytes(block), max(len(block), 1)),
                                                    len(block), batch, x_ptr, y_ptr)

    # -- whole-tensor encoder (compile step) --
    def encode_tensor(self, words: np.ndarray, codec: int, shape_cols: int | None = None, bf16: bool = True,
                      threads: int = 0):
        """Encode a BF16 tensor (uint16 words, any shape) with the compiler's slab rule.

        Returns (encoded bytes as a uint8 array, block table as a BLOCK_DTYPE array)."""
        data = np.ascontiguousarray(words)
        if shape_cols is None:
            shape_cols = data.shape[1] if data.ndim == 2 else 0
        out, out_size = ctypes.c_void_p(), ctypes.c_uint64()
        blocks, nblocks = ctypes.POINTER(Block)(), ctypes.c_uint64()
        rc = self.lib.xksv_encode_tensor(data.ctypes.data, data.nbytes, int(bf16), shape_cols, codec, threads,
                                         ctypes.byref(out), ctypes.byref(out_size), ctypes.byref(blocks),
                                         ctypes.byref(nblocks))
        if rc:
            raise XksvError("xksv_encode_tensor failed")
        try:
            enc = np.ctypeslib.as_array(ctypes.cast(out, ctypes.POINTER(ctypes.c_uint8)),
                                        shape=(max(out_size.value, 1),))[:out_size.value].copy()
            raw = ctypes.string_at(blocks, nblocks.value * ctypes.sizeof(Block))
            table = np.frombuffer(raw, dtype=BLOCK_DTYPE).copy()
        finally:
            self.lib.xksv_free(out)
            self.lib.xksv_free(ctypes.cast(blocks, ctypes.c_void_p))
        return enc, table

    def device_cus(self) -> int:
        return self.lib.xksv_hip_device_cus()


class Plan:
    """Device-resident batched decode / fused GEMM over blocks of an archive in HBM."""

    def __init__(self, lib: Library, table: np.ndarray, archive_size: int):
        self.lib = lib
        table = np.ascontiguousarray(table, dtype=BLOCK_DTYPE)
        self._table = table
        handle = ctypes.c_void_p()
        ptr = table.ctypes.data_as(ctypes.POINTER(Block))
        if lib.lib.xksv_hip_plan_create(ptr, len(table), archive_size, ctypes.byref(handle)):
            raise XksvError("xksv_hip_plan_create failed")
        self.handle = handle

    def decode(self, archive_ptr: int, out_ptr: int, out_size: int, stream: int = 0) -> None:
        if self.lib.lib.xksv_hip_plan_decode(self.handle, archive_ptr, out_ptr, out_size, stream or None):
            raise XksvError("xksv_hip_plan_decode failed to launch")

    def index(self, archive_ptr: int, stream: int = 0) -> None:
        """Build the decode's codeword index of the plan's parallel32 blocks from the
        archive (once, for weights that stay resident); later decodes use it."""
        if self.lib.lib.xksv_hip_plan_index(self.handle, archive_ptr, stream or None):
            raise XksvError("xksv_hip_plan_index failed")

    def gemm(self, archive_ptr: int, x_ptr: int, batch: int, y_ptr: int, stream: int = 0) -> None:
        if self.lib.lib.xksv_hip_plan_gemm(self.handle, archive_ptr, x_ptr, batch, y_ptr, stream or None):
            raise XksvError("xksv_hip_plan_gemm failed to launch")

    def gemm_bf16(self, archive_ptr: int, x_ptr: int, batch: int, y_ptr: int, stream: int = 0) -> None:
        """bf16 X [batch, cols] -> fp32 Y [batch, M] (layout of x @ W.T)."""
        if self.lib.lib.xksv_hip_plan_gemm_bf16(self.handle, archive_ptr, x_ptr, batch, y_ptr, stream or None):
            raise XksvError("xksv_hip_plan_gemm_bf16 failed to launch")

    def digests(self, out_ptr: int, out_size: int, digests_ptr: int, digests_size: int, stream: int = 0) -> None:
        """SHA-256 of every block's decoded bytes in `out` (device) into
        `digests` (device, 32 bytes per block in table order)."""
        if self.lib.lib.xksv_hip_plan_digests(self.handle, out_ptr, out_size, digests_ptr, digests_size,
                                              stream or None):
            raise XksvError("xksv_hip_plan_digests failed to launch")

    def verify(self, out_ptr: int, out_size: int, expected_ptr: int, expected_size: int, verdicts_ptr: int,
               stream: int = 0) -> None:
        """Per-block verdicts (device uint32 per block) of the last decode into `out`:
        decode error bits, plus ERR_DIGEST where the block's SHA-256 differs from
        `expected` (device, 32 bytes per block in table order)."""
        if self.lib.lib.xksv_hip_plan_verify(self.handle, out_ptr, out_size, expected_ptr, expected_size,
                                             verdicts_ptr, stream or None):
            raise XksvError("xksv_hip_plan_verify failed to launch")

    def error_flags(self, flags_ptr: int, stream: int = 0) -> None:
        """Enqueue *flags (device uint32) |= OR of the last call's block error bits; no host sync."""
        if self.lib.lib.xksv_hip_plan_error_flags(self.handle, flags_ptr, stream or None):
            raise XksvError("xksv_hip_plan_error_flags failed to launch")

    def errors(self, stream: int = 0):
        """(number of failed blocks, first failing block or -1, OR of error bits)."""
        first, bits = ctypes.c_int64(), ctypes.c_uint32()
        n = self.lib.lib.xksv_hip_plan_errors(self.handle, stream or None, ctypes.byref(first), ctypes.byref(bits))
        if n < 0:
            raise XksvError("xksv_hip_plan_errors: HIP error")
        return n, first.value, bits.value

    def close(self) -> None:
        if self.handle:
            self.lib.lib.xksv_hip_plan_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

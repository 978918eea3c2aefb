"""ctypes handle on the CPU oracle (oracle/liboracle.so) plus shared test helpers.

Test infrastructure: the oracle is the checker for the HIP path, never part of it.
"""
from __future__ import annotations

import ctypes
import hashlib
import os
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "xks-vectorforge_amd"))
import xksv_synth as syn  # noqa: E402

ORACLE_SO = Path(os.environ.get("XKSV_ORACLE_LIBRARY", ROOT / "oracle" / "liboracle.so"))
REF_SO = ROOT / "oracle" / "_ref" / "libxksv_ref.so"


def sha(b: bytes) -> str:
    return hashlib.sha256(b).hexdigest()


class _Codec:
    """Common ctypes surface of liboracle.so (oracle_*) and oracle/_ref (xksv_*)."""

    def __init__(self, path: Path, prefix: str):
        self.lib = ctypes.CDLL(str(path))
        six = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
               ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t)]
        self._pack = getattr(self.lib, prefix + "pack")
        self._unpack = getattr(self.lib, prefix + "unpack")
        self._pack_parallel = getattr(self.lib, prefix + "pack_parallel")
        self._unpack_parallel = getattr(self.lib, prefix + "unpack_parallel")
        for f in (self._pack, self._unpack, self._pack_parallel):
            f.argtypes = six
            f.restype = ctypes.c_int
        self._unpack_parallel.argtypes = [ctypes.c_void_p, ctypes.c_size_t,
                                          ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t)]
        self._unpack_parallel.restype = ctypes.c_int
        self._free = getattr(self.lib, prefix + "free")
        self._free.argtypes = [ctypes.c_void_p]

    def _run(self, fn, data: bytes, *shape):
        buf = ctypes.create_string_buffer(bytes(data), max(len(data), 1))
        out, size = ctypes.c_void_p(), ctypes.c_size_t()
        rc = fn(buf, len(data), *shape, ctypes.byref(out), ctypes.byref(size))
        if rc:
            return rc, None
        try:
            return 0, ctypes.string_at(out, size.value)
        finally:
            self._free(out)

    def pack(self, raw: bytes, rows: int, cols: int):
        return self._run(self._pack, raw, rows, cols)

    def pack_parallel(self, raw: bytes, rows: int, cols: int):
        return self._run(self._pack_parallel, raw, rows, cols)

    def unpack(self, blob: bytes, rows: int, cols: int):
        return self._run(self._unpack, blob, rows, cols)

    def unpack_parallel(self, blob: bytes):
        return self._run(self._unpack_parallel, blob)


class Oracle(_Codec):
    def __init__(self, path: Path = ORACLE_SO):
        super().__init__(path, "oracle_")
        self.lib.oracle_tile.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                         ctypes.c_size_t, ctypes.c_void_p]
        self.lib.oracle_untile.argtypes = self.lib.oracle_tile.argtypes
        self.lib.oracle_gemm_f64.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_void_p,
                                             ctypes.c_size_t, ctypes.c_void_p]
        self.lib.oracle_gemm_f64.restype = None

    def tile(self, w: np.ndarray, rows: int, cols: int, tr: int = 16, tc: int = 16, inverse=False) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.uint16).reshape(-1)
        out = np.empty_like(w)
        fn = self.lib.oracle_untile if inverse else self.lib.oracle_tile
        assert fn(w.ctypes.data, rows, cols, tr, tc, out.ctypes.data) == 0
        return out

    def gemm_f64(self, w: np.ndarray, x: np.ndarray) -> np.ndarray:
        """Y = W (bf16 bits, [rows, cols]) @ X ([cols, batch]) accumulated in float64."""
        w = np.ascontiguousarray(w, dtype=np.uint16)
        rows, cols = w.shape
        x = np.ascontiguousarray(x, dtype=np.float64)
        batch = 1 if x.ndim == 1 else x.shape[1]
        y = np.empty((rows, batch), np.float64)
        self.lib.oracle_gemm_f64(w.ctypes.data, rows, cols, x.ctypes.data, batch, y.ctypes.data)
        return y if x.ndim == 2 else y[:, 0]


class Reference(_Codec):
    """The reference's own CPU codec, compiled from its sources by oracle/Makefile."""

    def __init__(self, path: Path = REF_SO):
        super().__init__(path, "xksv_")


def gen(spec: dict) -> np.ndarray:
    """Rebuild a golden case's input words from its generator spec."""
    kind, shape = spec["kind"], tuple(spec["shape"])
    if kind == "normal":
        return syn.normal_bf16(spec["seed"], shape, spec.get("sigma", 0.02), spec.get("mean", 0.0))
    if kind == "student_t":
        return syn.student_t_bf16(spec["seed"], shape, spec.get("nu", 3.0), spec.get("scale", 0.02))
    if kind == "uniform":
        return syn.uniform_bf16(spec["seed"], shape)
    if kind == "zeros":
        return np.zeros(shape, np.uint16)
    if kind == "const":
        return np.full(shape, spec["word"], np.uint16)
    if kind == "words_mod":
        return syn.words_mod(shape)
    if kind == "uniform16":
        return syn.uniform16(spec["seed"], shape)
    if kind == "exponent_pattern":
        return syn.exponent_pattern(spec["seed"], shape)
    if kind == "all_patterns":
        return np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(shape)
    raise ValueError(kind)


def apply_mutation(blob: bytes, m: dict) -> bytes:
    """Apply one corruption from tests/golden/corruptions.json to an encoded block."""
    b = bytearray(blob)
    op = m["op"]
    if op == "truncate":
        return bytes(b[:len(b) - m["n"]])
    if op == "append":
        return bytes(b) + bytes.fromhex(m["bytes"])
    if op == "set":
        v = bytes.fromhex(m["bytes"])
        b[m["at"]:m["at"] + len(v)] = v
        return bytes(b)
    if op in ("add64", "set64"):
        at = m["at"]
        cur = int.from_bytes(b[at:at + 8], "little")
        new = (cur + m["delta"]) % (1 << 64) if op == "add64" else m["value"]
        b[at:at + 8] = new.to_bytes(8, "little")
        return bytes(b)
    if op == "xor":
        b[m["at"]] ^= m["value"]
        return bytes(b)
    raise ValueError(op)


def raw_bytes(w: np.ndarray) -> bytes:
    return np.ascontiguousarray(w, dtype="<u2").tobytes()


def canonical_codes(lengths) -> dict:
    """RFC 1951 3.2.2 canonical codes {symbol: bit string} for a 256-entry lengths table."""
    maxlen = max(lengths)
    bl = [0] * (maxlen + 2)
    for l in lengths:
        if l:
            bl[l] += 1
    code, nxt = 0, [0] * (maxlen + 2)
    for bits in range(1, maxlen + 1):
        code = (code + bl[bits - 1]) << 1 if bits > 1 else 0
        nxt[bits] = code
    out = {}
    for s, l in enumerate(lengths):
        if l:
            out[s] = format(nxt[l], "0%db" % l)
            nxt[l] += 1
    return out


def craft_segment(lengths, symbols, sm) -> bytes:
    """A serial block/segment [count][bits][lengths][sm][codes] for explicit exponent symbols."""
    codes = canonical_codes(lengths)
    bits = "".join(codes[int(s)] for s in symbols)
    nbits = len(bits)
    padded = bits + "0" * (-nbits % 8)
    stream = bytes(int(padded[i:i + 8], 2) for i in range(0, len(padded), 8))
    return (len(symbols).to_bytes(8, "little") + nbits.to_bytes(8, "little") + bytes(lengths) +
            bytes(int(v) & 255 for v in sm) + stream)


def long_code_lengths(maxlen: int = 40) -> list:
    """Complete code with lengths 1, 2, ..., maxlen-1, maxlen-1 on symbols 100.. (codes > 32 bits)."""
    lens = [0] * 256
    for i in range(maxlen - 1):
        lens[100 + i] = i + 1
    lens[100 + maxlen - 1] = maxlen - 1
    return lens

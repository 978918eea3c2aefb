"""The .xksv container around the compressed blocks: reader, writer, GPU load and GPU verify.

Format [docs/format.md:3-13]: little-endian; the 8-byte magic ``XKSV 00 01 0d 0a``,
a u64 absolute offset of a UTF-8 JSON index at the end of the file, and the
asset and tensor blocks in between, which the index locates and which must
cover that region without holes or overlaps.  Each tensor's index entry lists
its blocks in order: ``offset``, ``size``, ``raw_size``, ``codec`` ("raw",
"bf16-huffman-tile16" or "bf16-huffman-parallel32"), ``rows``, ``cols`` (0 for
raw blocks) and the SHA-256 of the block's original bytes; the tensor entry
also records the SHA-256 of the whole tensor [src/compile.cpp:441-468,489-510].

* ``Archive`` reads the header and index (the checks of python/xksv.py:302-308,
  src/verify.cpp:124-133) and turns a tensor's index blocks into the block
  table of the plan API (``xksv_hip_block``), codec names mapped to ids.
* ``compile_checkpoint`` writes an archive from a Safetensors checkpoint with
  the compiler's slab rule, codec choice and raw fallback; its bytes are those
  of the reference's ``xksv-native compile`` [src/compile.cpp:292-511].
* ``load_tensors`` is the GPU-decode load of python/runtime.py:86-99: the
  selected tensors' encoded blocks go to HBM once and one plan decodes them all.
* ``verify`` is src/verify.cpp:121-307 with the decode and the per-block
  SHA-256 on the GPU (``xksv_hip_plan_verify``); tensor digests, asset digests
  and the structural checks run on the host.
"""
from __future__ import annotations

import base64
import hashlib
import json
import os
import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

import xksv_hip

MAGIC = b"XKSV\x00\x01\r\n"
HEADER = struct.Struct("<8sQ")
MAX_INDEX = 1_000_000_000      # largest JSON index a reader accepts [src/verify.cpp:129]
RAW_CHUNK = 1 << 20            # slab / raw block size cap [src/compile.cpp:39]
MAX_ASSET = 100_000_000        # [src/compile.cpp:395, src/verify.cpp:148]
CODECS = {"raw": xksv_hip.CODEC_RAW, "bf16-huffman-tile16": xksv_hip.CODEC_SERIAL,
          "bf16-huffman-parallel32": xksv_hip.CODEC_PARALLEL}
# codec preference of the compiler -> codec name of its compressed blocks [src/compile.cpp:266-268]
PREFERENCES = {"dfloat11": "bf16-huffman-tile16", "dfloat11-parallel": "bf16-huffman-parallel32"}
DTYPE_SIZES = {"BOOL": 1, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E5M2": 1, "I16": 2, "U16": 2, "F16": 2, "BF16": 2,
               "I32": 4, "U32": 4, "F32": 4, "I64": 8, "U64": 8, "F64": 8}
# Model assets the compiler stores, in this order, when the source is a directory [src/compile.cpp:292-311].
ASSET_NAMES = ("config.json", "generation_config.json", "tokenizer.json", "tokenizer_config.json", "vocab.json",
               "merges.txt", "special_tokens_map.json", "added_tokens.json", "chat_template.jinja", "tokenizer.model",
               "vocab.txt", "preprocessor_config.json", "processor_config.json", "video_preprocessor_config.json",
               "LICENSE", "NOTICE", "README.md", "adapter_config.json", "model.safetensors.index.json")
# Name -> role, first match wins [src/inspect.cpp:27-40, python/xksv.py:43-57].
_ROLES = ((("embed_tokens", "word_embeddings"), "token_embedding"),
          (("lm_head", "output_projection"), "language_model_head"),
          (("visual", "vision"), "vision_component"))
_DELTANET = ((("conv",), "deltanet_convolution"), (("in_proj",), "deltanet_input_projection"),
             (("out_proj",), "deltanet_output_projection"))
_ROLES_AFTER = ((("self_attn", ".attention."), "attention_parameter"), (("expert",), "moe_expert"),
                (("router",), "moe_router"), ((".mlp.", ".feed_forward."), "feed_forward_parameter"),
                (("norm",), "normalization_parameter"))


class ArchiveError(ValueError):
    """A malformed, inconsistent or corrupted archive or checkpoint."""


def tensor_role(name: str) -> str:
    """The tensor's role as the checkpoint inventory records it."""
    def first(table):
        for keys, role in table:
            if any(k in name for k in keys):
                return role
        return None
    role = first(_ROLES)
    if role:
        return role
    if "linear_attn" in name:
        return first(_DELTANET) or "deltanet_state_parameter"
    return first(_ROLES_AFTER) or "other"


def _parse_json(data: bytes | str):
    """JSON with duplicate keys rejected [src/verify.cpp:57-68]."""
    def pairs(items):
        out = {}
        for k, v in items:
            if k in out:
                raise ArchiveError(f"duplicate JSON key: {k}")
            out[k] = v
        return out
    try:
        return json.loads(data, object_pairs_hook=pairs)
    except json.JSONDecodeError as e:
        raise ArchiveError(f"invalid JSON: {e}") from None


def _dump_index(index: dict) -> bytes:
    """The index text as the compiler writes it: keys sorted, no whitespace, UTF-8."""
    return json.dumps(index, sort_keys=True, separators=(",", ":"), ensure_ascii=False).encode()


def _uint(v, what: str) -> int:
    if type(v) is not int or v < 0:
        raise ArchiveError(f"invalid {what} in archive")
    return v


def _strides(shape) -> list:
    out, stride = [], 1
    for dim in reversed(shape):
        out.append(stride)
        stride *= dim
    return list(reversed(out))


# ------------------------------------------------------------------ checkpoint inventory

@dataclass
class Shard:
    name: str
    path: Path
    header: bytes           # the JSON header exactly as stored in the file
    tensors: list           # descriptors sorted by data offset


def checkpoint_shards(source: Path) -> list:
    """The Safetensors shards of a checkpoint, as the compiler takes inventory of them
    [src/inspect.cpp:69-117]: a shard index's files, else every *.safetensors of a
    directory in name order, else the one file; tensors sorted by data offset."""
    source = Path(source)
    index = source / "model.safetensors.index.json"
    if source.is_dir() and index.is_file():
        wm = _parse_json(index.read_bytes()).get("weight_map")
        if not isinstance(wm, dict):
            raise ArchiveError("invalid shard index")
        names = set()
        for v in wm.values():
            if not isinstance(v, str) or Path(v).name != v or not v.endswith(".safetensors"):
                raise ArchiveError("invalid shard name")
            names.add(v)
        files = [source / n for n in sorted(names)]
    elif source.is_dir():
        files = sorted(p for p in source.iterdir() if p.suffix == ".safetensors")
    else:
        files = [source]
    if not files:
        raise ArchiveError("no Safetensors shards found")
    shards, seen = [], set()
    for path in files:
        size = path.stat().st_size
        with open(path, "rb") as f:
            (hlen,) = struct.unpack("<Q", f.read(8))
            if hlen > MAX_ASSET or hlen > size - 8:
                raise ArchiveError("invalid header length")
            header = f.read(hlen)
        root = _parse_json(header)
        if not isinstance(root, dict):
            raise ArchiveError("invalid Safetensors header")
        tensors, ranges = [], []
        for name in sorted(root):  # the inventory walks the header in key order
            if name == "__metadata__":
                continue
            if name in seen:
                raise ArchiveError(f"duplicate tensor: {name}")
            seen.add(name)
            d = root[name]
            dtype = d.get("dtype")
            if dtype not in DTYPE_SIZES:
                raise ArchiveError(f"unsupported dtype: {dtype}")
            shape = [_uint(x, "dimension") for x in d["shape"]]
            start, end = (_uint(x, "offset") for x in d["data_offsets"])
            count = int(np.prod(shape, dtype=object)) if shape else 1
            if end < start or end > size - 8 - hlen or end - start != count * DTYPE_SIZES[dtype]:
                raise ArchiveError(f"invalid tensor extent: {name}")
            tensors.append({"name": name, "dtype": dtype, "shape": shape, "strides": _strides(shape),
                            "role": tensor_role(name), "start": start, "size": end - start})
            if end > start:
                ranges.append((start, end))
        cursor = 0
        for a, b in sorted(ranges):
            if a != cursor:
                raise ArchiveError("overlapping or noncontiguous tensor data")
            cursor = b
        if cursor != size - 8 - hlen:
            raise ArchiveError("unreferenced tensor data")
        tensors.sort(key=lambda t: t["start"])
        shards.append(Shard(path.name, path, header, tensors))
    return shards


# ------------------------------------------------------------------ writer

def _file_sha(path: Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def compile_checkpoint(lib: "xksv_hip.Library", source, output, codec: str = "dfloat11", workers: int = 0) -> int:
    """Write the archive of a Safetensors checkpoint [src/compile.cpp:312-511].

    Every BF16 tensor is cut by the compiler's slab rule into slabs of <= 16 rows
    and <= 1 MiB (``xksv_encode_tensor``), each encoded with ``codec``
    ("dfloat11": serial blocks, "dfloat11-parallel": XKSP2 blocks) and kept raw
    when the encoding is not smaller; other dtypes go raw in 1 MiB blocks.  The
    index and file bytes equal the reference compiler's for the same checkpoint.
    The file is written beside ``output`` and published without replacing an
    existing file.  Returns the archive size in bytes."""
    if codec not in PREFERENCES:
        raise ArchiveError("compile requires a supported codec")
    source, output = Path(source), Path(output).absolute()
    if output.exists():
        raise ArchiveError("output already exists")
    shards = checkpoint_shards(source)
    if any(s.path.resolve() == output for s in shards):
        raise ArchiveError("output would overwrite source")
    index = {"version": 1, "format": "safetensors", "codec_preference": codec, "shards": [], "assets": []}
    partial = output.with_name(output.name + ".partial")
    codec_id = CODECS[PREFERENCES[codec]]
    with open(partial, "xb") as out:
        out.write(HEADER.pack(MAGIC, 0))
        if source.is_dir():
            for name in ASSET_NAMES:
                p = source / name
                if not p.is_file():
                    continue
                data = p.read_bytes()
                if len(data) > MAX_ASSET:
                    raise ArchiveError(f"asset too large: {name}")
                index["assets"].append({"name": name, "offset": out.tell(), "size": len(data),
                                        "sha256": hashlib.sha256(data).hexdigest()})
                out.write(data)
        for s in shards:
            entry = {"name": s.name, "header": base64.b64encode(s.header).decode(), "source_sha256": _file_sha(s.path),
                     "tensors": []}
            index["shards"].append(entry)
            data_start = 8 + len(s.header)
            with open(s.path, "rb") as src:
                for desc in s.tensors:
                    src.seek(data_start + desc["start"])
                    raw = np.frombuffer(src.read(desc["size"]), np.uint8)
                    if len(raw) != desc["size"]:
                        raise ArchiveError("unexpected end of source")
                    bf16 = desc["dtype"] == "BF16"
                    shape = desc["shape"]
                    cols = shape[1] if len(shape) == 2 and shape[1] else 0
                    t = dict(desc)
                    t["blocks"] = []
                    if len(raw):
                        enc, table = lib.encode_tensor(raw, codec_id, shape_cols=cols, bf16=bf16, threads=workers)
                    else:
                        enc, table = np.zeros(0, np.uint8), np.zeros(0, xksv_hip.BLOCK_DTYPE)
                    base = out.tell()
                    for b in table:
                        o, r = int(b["out_offset"]), int(b["raw_size"])
                        name = next(k for k, v in CODECS.items() if v == int(b["codec"]))
                        t["blocks"].append({"offset": base + int(b["offset"]), "size": int(b["size"]), "raw_size": r,
                                            "codec": name, "rows": int(b["rows"]), "cols": int(b["cols"]),
                                            "sha256": hashlib.sha256(raw[o:o + r]).hexdigest()})
                    out.write(enc.tobytes())
                    t["sha256"] = hashlib.sha256(raw).hexdigest()
                    entry["tensors"].append(t)
        limit = out.tell()
        out.write(_dump_index(index))
        out.seek(0)
        out.write(HEADER.pack(MAGIC, limit))
        out.flush()
        os.fsync(out.fileno())
    os.link(partial, output)
    partial.unlink()
    return output.stat().st_size


# ------------------------------------------------------------------ reader

class Archive:
    """An .xksv file: header, index and the blocks of every tensor."""

    def __init__(self, path):
        self.path = Path(path)
        self.size = self.path.stat().st_size
        with open(self.path, "rb") as f:
            head = f.read(HEADER.size)
            if len(head) < HEADER.size:
                raise ArchiveError("truncated archive")
            magic, limit = HEADER.unpack(head)
            if magic != MAGIC:
                raise ArchiveError("invalid archive magic")
            if limit < HEADER.size or limit > self.size or self.size - limit > MAX_INDEX:
                raise ArchiveError("invalid archive index offset")
            f.seek(limit)
            index = _parse_json(f.read(self.size - limit))
        if not isinstance(index, dict) or index.get("version") != 1 or index.get("format") != "safetensors":
            raise ArchiveError("unsupported archive")
        self.index, self.limit = index, limit
        self.tensors = {}
        for shard in index.get("shards", []):
            for t in shard.get("tensors", []):
                if t["name"] in self.tensors:
                    raise ArchiveError("duplicate archive tensor")
                self.tensors[t["name"]] = t

    def read(self, offset: int, size: int) -> np.ndarray:
        """Bytes [offset, offset + size) of the file (memory-mapped, read-only)."""
        if offset < 0 or size < 0 or offset + size > self.size:
            raise ArchiveError("file range outside the archive")
        if size == 0:
            return np.zeros(0, np.uint8)
        return np.memmap(self.path, np.uint8, "r", offset=offset, shape=(size,))

    def block_table(self, names, rows: bool = False, align: int = 256):
        """Block table of the plan API for tensors `names`, in that order.

        Returns (table, lo, hi, bases): block offsets are relative to archive byte
        `lo` (the region [lo, hi) holds every block); out_offset is the byte offset
        in one output buffer where each tensor starts at bases[name] (aligned to
        `align`), or with rows=True the first output row of the block (GEMM plans
        of one weight; raw blocks keep their rows from raw_size)."""
        recs, bases, at = [], {}, 0
        lo, hi = None, None
        for name in names:
            t = self.tensors.get(name)
            if t is None:
                raise ArchiveError(f"no tensor {name}")
            bases[name] = at
            pos, row = 0, 0
            shape = t["shape"]
            cols = shape[1] if rows and len(shape) == 2 else 0
            if rows and not cols:
                raise ArchiveError(f"{name} is not a matrix")
            for b in t["blocks"]:
                off, n, r = _uint(b["offset"], "offset"), _uint(b["size"], "size"), _uint(b["raw_size"], "size")
                codec = CODECS.get(b["codec"])
                if codec is None:
                    raise ArchiveError("unknown block codec")
                if off < HEADER.size or off > self.limit or n > self.limit - off or n > RAW_CHUNK or r > RAW_CHUNK:
                    raise ArchiveError("invalid block extent")
                br, bc = (0, 0) if codec == xksv_hip.CODEC_RAW else (_uint(b["rows"], "rows"), _uint(b["cols"], "cols"))
                if codec == xksv_hip.CODEC_RAW and n != r:
                    raise ArchiveError("invalid raw block")
                if codec != xksv_hip.CODEC_RAW and (not br or not bc or br * bc * 2 != r or t["dtype"] != "BF16"):
                    raise ArchiveError("invalid compressed block shape")
                if rows:
                    if r % (cols * 2):
                        raise ArchiveError(f"{name}: block is not whole rows")
                    out = row
                    row += r // (cols * 2)
                else:
                    out = at + pos
                recs.append((off, n, r, out, br, bc if codec else (cols if rows else 0), codec, 0))
                pos += r
                lo = off if lo is None else min(lo, off)
                hi = off + n if hi is None else max(hi, off + n)
            if pos != t["size"]:
                raise ArchiveError(f"tensor blocks do not cover the tensor: {name}")
            at = (at + pos + align - 1) // align * align
        table = np.array(recs, dtype=xksv_hip.BLOCK_DTYPE) if recs else np.zeros(0, xksv_hip.BLOCK_DTYPE)
        lo = lo or 0
        hi = hi or 0
        table["offset"] -= lo
        return table, lo, hi, bases, at


# ------------------------------------------------------------------ GPU load

TORCH_DTYPES = {"BF16": "bfloat16", "F16": "float16", "F32": "float32", "F64": "float64", "I8": "int8", "U8": "uint8",
                "I16": "int16", "I32": "int32", "I64": "int64", "BOOL": "bool"}


def load_tensors(lib: "xksv_hip.Library", archive, names=None, device: str = "cuda", stream: int = 0) -> dict:
    """GPU-decode load [python/runtime.py:86-99]: every selected tensor's blocks go
    to HBM in one copy, one plan decodes them (raw blocks copied), and each tensor
    is a view of the decoded buffer with its index dtype and shape.  Fails loudly
    (ArchiveError naming the tensor) when a block does not decode."""
    import torch
    arc = archive if isinstance(archive, Archive) else Archive(archive)
    names = list(arc.tensors) if names is None else list(names)
    table, lo, hi, bases, total = arc.block_table(names)
    d_arc = torch.from_numpy(np.array(arc.read(lo, hi - lo))).to(device)
    out = torch.empty(max(total, 1), dtype=torch.uint8, device=device)
    plan = xksv_hip.Plan(lib, table, hi - lo)
    try:
        plan.decode(d_arc.data_ptr(), out.data_ptr(), out.numel(), stream)
        nbad, first, bits = plan.errors(stream)
    finally:
        plan.close()
    if nbad:
        owner = _block_owner(arc, names, first)
        raise ArchiveError(f"GPU block decode failed: {owner} (error bits {bits})")
    result = {}
    for name in names:
        t = arc.tensors[name]
        dtype = TORCH_DTYPES.get(t["dtype"])
        view = out[bases[name]:bases[name] + t["size"]]
        result[name] = (view.view(getattr(torch, dtype)).reshape(t["shape"]) if dtype
                        else view.clone())
    return result


def _block_owner(arc: Archive, names, k: int) -> str:
    for name in names:
        n = len(arc.tensors[name]["blocks"])
        if k < n:
            return name
        k -= n
    return "?"


# ------------------------------------------------------------------ GPU verify

@dataclass
class VerifyReport:
    """Outcome of ``verify``: every failure found (the reference stops at the first)."""
    tensors: int = 0
    bytes: int = 0
    failures: list = field(default_factory=list)
    block_verdicts: dict = field(default_factory=dict)  # (tensor, block index) -> XKSV_ERR_* bits, failures only

    @property
    def ok(self) -> bool:
        return not self.failures

    def raise_if_failed(self) -> None:
        if self.failures:
            raise ArchiveError(self.failures[0])


def verify(lib: "xksv_hip.Library", path, source=None, allow_partial: bool = False, stream: int = 0) -> VerifyReport:
    """Archive verification [src/verify.cpp:121-307]: the index and block extents,
    asset digests, stored headers against tensor descriptors, every block decoded
    on the GPU and its SHA-256 (computed on the GPU) compared with the index, each
    tensor's SHA-256 and byte count, and data coverage of the file; with
    `source`, the checkpoint's headers and bytes too."""
    import torch
    rep = VerifyReport()
    fail = rep.failures.append
    try:
        arc = Archive(path)
    except ArchiveError as e:
        fail(str(e))
        return rep
    spans = []

    def span(off, n, cap):
        if type(off) is not int or type(n) is not int or off < HEADER.size or off > arc.limit or n < 0 or \
                n > arc.limit - off or n > cap:
            raise ArchiveError("invalid archive extent")
        spans.append((off, off + n))

    src_shards = {s.name: s for s in checkpoint_shards(source)} if source is not None else None
    try:
        names_seen = set()
        for asset in arc.index.get("assets", []):
            name = asset["name"]
            if not isinstance(name, str) or Path(name).name != name or name in (".", "..") or name in names_seen:
                raise ArchiveError("invalid stored filename" if name not in names_seen else "duplicate asset")
            names_seen.add(name)
            span(asset["offset"], asset["size"], MAX_ASSET)
            data = bytes(arc.read(asset["offset"], asset["size"]))
            if hashlib.sha256(data).hexdigest() != asset["sha256"]:
                fail(f"asset checksum failed: {name}")
            if source is not None:
                p = Path(source) / name
                if not p.is_file() or p.read_bytes() != data:
                    fail(f"source asset differs: {name}")
        order, shard_names = [], set()
        for shard in arc.index["shards"]:
            name = shard["name"]
            if not isinstance(name, str) or Path(name).name != name or name in shard_names:
                raise ArchiveError("invalid stored filename" if name not in shard_names else "duplicate shard")
            shard_names.add(name)
            try:
                header = base64.b64decode(shard["header"], validate=True)
            except ValueError:
                raise ArchiveError("invalid stored header encoding") from None
            stored = _parse_json(header)
            if not isinstance(stored, dict):
                raise ArchiveError("invalid shard header")
            if src_shards is not None:
                s = src_shards.get(name)
                if s is None:
                    raise ArchiveError(f"missing source shard: {name}")
                if s.header != header:
                    fail(f"source header differs: {name}")
            seen = set()
            for t in shard["tensors"]:
                tn = t["name"]
                if tn in seen or tn not in stored or tn == "__metadata__":
                    raise ArchiveError("invalid tensor name")
                seen.add(tn)
                dtype = t["dtype"]
                if dtype not in DTYPE_SIZES or not isinstance(t["shape"], list):
                    raise ArchiveError("invalid tensor type")
                count = 1
                for dim in t["shape"]:
                    count *= _uint(dim, "integer")
                start, length = _uint(t["start"], "integer"), _uint(t["size"], "integer")
                if length != count * DTYPE_SIZES[dtype]:
                    raise ArchiveError("invalid tensor size")
                d = stored[tn]
                if d.get("dtype") != dtype or d.get("shape") != t["shape"] or d.get("data_offsets") != [start, start + length]:
                    raise ArchiveError(f"tensor descriptor mismatch: {tn}")
                for b in t["blocks"]:
                    span(b["offset"], b["size"], RAW_CHUNK)
                    if b["codec"] == "bf16-huffman-parallel32":
                        head = bytes(arc.read(b["offset"], min(b["size"], 24)))
                        if len(head) < 24 or struct.unpack_from("<QQ", head, 8) != (b["rows"], b["cols"]):
                            raise ArchiveError("parallel block shape mismatch")
                order.append((tn, t))
            expected = len(stored) - (1 if "__metadata__" in stored else 0)
            if not allow_partial and len(seen) != expected:
                raise ArchiveError("stored tensor set mismatch")
        if src_shards is not None and set(src_shards) != shard_names:
            raise ArchiveError("source shard set differs")
        spans.sort()
        end = HEADER.size
        for a, b in spans:
            if a != end:
                raise ArchiveError("invalid archive data coverage")
            end = b
        if end != arc.limit:
            raise ArchiveError("unreferenced archive data")
    except (ArchiveError, KeyError, TypeError) as e:
        fail(str(e) if isinstance(e, ArchiveError) else f"invalid archive index: {e!r}")
        return rep

    # Decode every block on the GPU, then per-block SHA-256 verdicts on the GPU.
    names = [tn for tn, _ in order]
    try:
        table, lo, hi, bases, total = arc.block_table(names)
    except ArchiveError as e:
        fail(str(e))
        return rep
    digests = np.frombuffer(b"".join(bytes.fromhex(b["sha256"]) for _, t in order for b in t["blocks"]), np.uint8)
    if len(table):
        d_arc = torch.from_numpy(np.array(arc.read(lo, hi - lo))).to("cuda")
        out = torch.empty(max(total, 1), dtype=torch.uint8, device="cuda")
        d_exp = torch.from_numpy(digests.copy()).to("cuda")
        d_ver = torch.zeros(len(table), dtype=torch.int32, device="cuda")
        plan = xksv_hip.Plan(lib, table, hi - lo)
        try:
            plan.decode(d_arc.data_ptr(), out.data_ptr(), out.numel(), stream)
            plan.verify(out.data_ptr(), out.numel(), d_exp.data_ptr(), d_exp.numel(), d_ver.data_ptr(), stream)
            plan.errors(stream)
        finally:
            plan.close()
        verdicts = d_ver.cpu().numpy().view(np.uint32)
    else:
        out, verdicts = None, np.zeros(0, np.uint32)
    k = 0
    for tn, t in order:
        bad = False
        for i, _ in enumerate(t["blocks"]):
            v = int(verdicts[k])
            k += 1
            if v:
                rep.block_verdicts[(tn, i)] = v
                bad = True
        if bad:
            fail(f"block {'decoding' if any(rep.block_verdicts.get((tn, i), 0) & 15 for i in range(len(t['blocks']))) else 'checksum'} failed: {tn}")
            continue
        data = out[bases[tn]:bases[tn] + t["size"]].cpu().numpy().tobytes() if t["size"] else b""
        if hashlib.sha256(data).hexdigest() != t["sha256"]:
            fail(f"tensor checksum failed: {tn}")
            continue
        if src_shards is not None:
            s = next(s for s in src_shards.values() if any(d["name"] == tn for d in s.tensors))
            with open(s.path, "rb") as f:
                f.seek(8 + len(s.header) + t["start"])
                if f.read(t["size"]) != data:
                    fail(f"source bytes differ: {tn}")
                    continue
        rep.tensors += 1
        rep.bytes += t["size"]
    return rep

"""Device-resident batched path: whole tensors and archives resident in HBM (GPU only).

Pins decode of multi-block tensors (slab rule, raw fallback, both codecs) to
the input bytes and per-slab SHA-256 (src/verify.cpp:262-273 semantics), the
per-block error reporting, and the fused GEMV/GEMM over whole weight tensors
against an fp64 reference.
"""
from __future__ import annotations

import hashlib
import json

import numpy as np
import pytest
import torch

import xksv_hip
import xksv_synth as syn
from conftest import GOLDEN
from oracle_lib import gen, raw_bytes

pytestmark = pytest.mark.gpu


def _upload(arr: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(arr).view(np.uint8).reshape(-1).copy()).to("cuda")


def _decode_tensor(hip, words, codec, shape_cols=None):
    enc, table = hip.encode_tensor(words, codec, shape_cols)
    d_arc = _upload(enc)
    out = torch.zeros(words.nbytes, dtype=torch.uint8, device="cuda")
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    plan.decode(d_arc.data_ptr(), out.data_ptr(), out.numel())
    nbad, first, bits = plan.errors()
    plan.close()
    return enc, table, out, nbad


@pytest.mark.parametrize("codec", [1, 2])
def test_config1_4096x4096_per_slab_sha(hip, codec):
    """4096x4096 N(0, 0.02) seed 0, 256 slabs of 16x4096: every slab's SHA-256 and encoded digest."""
    slabs = json.loads((GOLDEN / "slabs_4096x4096_seed0.json").read_text())
    w = gen(slabs["gen"])
    enc, table, out, nbad = _decode_tensor(hip, w, codec)
    assert nbad == 0
    assert len(table) == 256 and set(table["codec"]) == {codec}
    key = "serial" if codec == 1 else "parallel"
    for s, t in enumerate(table):
        blob = enc[t["offset"]:t["offset"] + t["size"]].tobytes()
        assert [len(blob), hashlib.sha256(blob).hexdigest()] == slabs[key][s]
    host = out.cpu().numpy()
    for s in range(256):
        assert hashlib.sha256(host[s * 131072:(s + 1) * 131072].tobytes()).hexdigest() == slabs["raw"][s], s


@pytest.mark.parametrize("codec", [1, 2])
def test_config3_mixed_archive(hip, codec):
    """N(0,0.02), Student-t(3), U(-1,1) and zero 4096x4096 slabs, a uniform-bits slab (raw
    fallback) and an fp32 4096-vector stored raw; one plan over the whole archive."""
    parts = [syn.normal_bf16(31, (4096, 4096)), syn.student_t_bf16(32, (4096, 4096)),
             syn.uniform_bf16(33, (4096, 4096)), np.zeros((4096, 4096), np.uint16),
             syn.uniform16(34, (16, 4096))]
    fp32 = np.random.default_rng(35).standard_normal(4096).astype(np.float32)
    encs, tables, raws, base, obase = [], [], [], 0, 0
    for p in parts:
        e, t = hip.encode_tensor(p, codec)
        t = t.copy()
        t["offset"] += base
        t["out_offset"] += obase
        encs.append(e); tables.append(t); raws.append(raw_bytes(p))
        base += e.nbytes; obase += p.nbytes
    e, t = hip.encode_tensor(fp32.view(np.uint16), codec, bf16=False)
    assert set(t["codec"]) == {0}
    t = t.copy(); t["offset"] += base; t["out_offset"] += obase
    encs.append(e); tables.append(t); raws.append(fp32.tobytes())
    enc, table = np.concatenate(encs), np.concatenate(tables)
    d_arc = _upload(enc)
    total = sum(len(r) for r in raws)
    out = torch.zeros(total, dtype=torch.uint8, device="cuda")
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    plan.decode(d_arc.data_ptr(), out.data_ptr(), total)
    assert plan.errors()[0] == 0
    assert out.cpu().numpy().tobytes() == b"".join(raws)
    # the uniform-bits slab does not compress: stored raw
    uni = table[(table["out_offset"] >= 4 * 4096 * 4096 * 2) & (table["out_offset"] < 4 * 4096 * 4096 * 2 + 131072)]
    assert set(uni["codec"]) == {0}


def _corrupt_code_bits(oracle, enc, t) -> None:
    """Flip one byte of the last substream's code bits of block `t` in place, choosing
    (deterministically, nearest the end first) a byte whose flip the oracle rejects."""
    end = int(t["offset"] + t["size"])
    for back in range(2, 200):
        blob = bytearray(enc[int(t["offset"]):end].tobytes())
        blob[len(blob) - back] ^= 0xFF
        if oracle.unpack_parallel(bytes(blob))[0] != 0:
            enc[end - back] ^= 0xFF
            return
    raise AssertionError("no rejected flip found")


def test_plan_reports_corrupt_blocks(hip, oracle):
    """A block whose code bits the oracle rejects is the only one reported, with a
    stream error, and every other block decodes exactly."""
    w = syn.normal_bf16(41, (64, 4096))
    enc, table = hip.encode_tensor(w, 2)
    enc = enc.copy()
    _corrupt_code_bits(oracle, enc, table[2])
    d_arc = _upload(enc)
    out = torch.zeros(w.nbytes, dtype=torch.uint8, device="cuda")
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    plan.decode(d_arc.data_ptr(), out.data_ptr(), out.numel())
    n, first, bits = plan.errors()
    assert (n, first) == (1, 2) and bits == xksv_hip.ERR_STREAM
    host = out.cpu().numpy()
    for b in (0, 1, 3):
        assert host[b * 131072:(b + 1) * 131072].tobytes() == raw_bytes(w[16 * b:16 * b + 16])


@pytest.mark.parametrize("nblocks", [4, 300, 8192])
def test_plan_decode_both_schedules(hip, oracle, nblocks):
    """Parallel32 plans below and above twice the resident waves (6,144 on 256 CUs): the
    first two run one work item per substream, the last one wave per block.  Plan entry i
    decodes encoded 16x1024 slab i % 64 into its own output; the entries of the two corrupt
    slabs (code bits of slab 1, header magic of slab 2) are the only ones reported and every
    other entry decodes exactly."""
    w = syn.normal_bf16(43, (16 * 64, 1024))
    enc, base = hip.encode_tensor(w, 2, 1024)
    assert len(base) == 64 and set(base["codec"]) == {2}
    enc = enc.copy()
    _corrupt_code_bits(oracle, enc, base[1])
    enc[int(base[2]["offset"])] ^= 0x01  # magic
    assert oracle.unpack_parallel(enc[int(base[2]["offset"]):int(base[2]["offset"] + base[2]["size"])].tobytes())[0] != 0
    table = np.resize(base, nblocks).copy()
    table["out_offset"] = np.arange(nblocks, dtype=np.uint64) * 32768
    d_arc = _upload(enc)
    out = torch.zeros(nblocks * 32768, dtype=torch.uint8, device="cuda")
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    plan.decode(d_arc.data_ptr(), out.data_ptr(), out.numel())
    n, first, bits = plan.errors()
    plan.close()
    bad = np.isin(np.arange(nblocks) % 64, (1, 2))
    assert (n, first) == (int(bad.sum()), 1) and bits == xksv_hip.ERR_STREAM | xksv_hip.ERR_HEADER
    host = out.cpu().numpy().reshape(nblocks, -1)
    want = w.view(np.uint8).reshape(64, -1)[np.arange(nblocks) % 64]
    assert np.array_equal(host[~bad], want[~bad])


def test_plan_decode_mixed_sizes_report_table_slots(hip, oracle):
    """The plan decodes its parallel32 blocks largest first; errors still name table
    entries.  Table: 16x4096 and 16x14336 slabs interleaved (the 14336-wide ones run
    first), then a 5x4096 slab; entries 3 (4096-wide) and 4 (14336-wide) carry damaged
    code bits, entry 6 a damaged magic.  Errors are reported for exactly those entries,
    the first as 3, and every other entry decodes exactly, with and without the index."""
    parts, rows_out, want = [], [], []
    for i in range(8):
        rows, cols = (16, 14336) if i % 2 else (16, 4096)
        if i == 7:
            rows, cols = 5, 4096
        w = syn.normal_bf16(2000 + i, (rows, cols))
        parts.append(np.frombuffer(hip.call("xksv_pack_parallel", raw_bytes(w), rows, cols), np.uint8))
        rows_out.append((rows, cols))
        want.append(raw_bytes(w))
    table = np.zeros(len(parts), xksv_hip.BLOCK_DTYPE)
    off = out = 0
    for i, (p, (rows, cols)) in enumerate(zip(parts, rows_out)):
        table[i] = (off, p.nbytes, rows * cols * 2, out, rows, cols, xksv_hip.CODEC_PARALLEL, 0)
        off += p.nbytes
        out += rows * cols * 2
    enc = np.concatenate(parts).copy()
    _corrupt_code_bits(oracle, enc, table[3])
    _corrupt_code_bits(oracle, enc, table[4])
    enc[int(table[6]["offset"])] ^= 0x01
    d_arc = _upload(enc)
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    try:
        for indexed in (False, True):
            if indexed:
                plan.index(_upload(np.concatenate(parts)).data_ptr())  # from the clean archive
            o = torch.zeros(out, dtype=torch.uint8, device="cuda")
            plan.decode(d_arc.data_ptr(), o.data_ptr(), o.numel())
            n, first, bits = plan.errors()
            assert (n, first) == (3, 3) and bits == xksv_hip.ERR_STREAM | xksv_hip.ERR_HEADER, indexed
            host = o.cpu().numpy().tobytes()
            for i in range(len(parts)):
                if i not in (3, 4, 6):
                    a = int(table[i]["out_offset"])
                    assert host[a:a + len(want[i])] == want[i], (indexed, i)
    finally:
        plan.close()


@pytest.mark.parametrize("codec", [1, 2])
@pytest.mark.parametrize("shape", [(14336, 4096), (4096, 14336), (100, 4096), (1024, 4100)])
def test_plan_gemv_whole_tensor(hip, codec, shape):
    rows, cols = shape
    w = syn.normal_bf16(rows + cols + codec, shape)
    enc, table = hip.encode_tensor(w, codec)
    d_arc = _upload(enc)
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    # slab rule: out_offset is in bytes; plans for GEMM index rows
    table = table.copy()
    table["out_offset"] //= (cols * 2)
    plan.close()
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    x = torch.randn(cols, dtype=torch.float32, device="cuda")
    y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    plan.gemm(d_arc.data_ptr(), x.data_ptr(), 1, y.data_ptr())
    assert plan.errors()[0] == 0
    wt = torch.from_numpy(syn.bf16_to_f32(w).astype(np.float64)).to("cuda")
    want = (wt @ x.double()).cpu().numpy()
    got = y.cpu().numpy().astype(np.float64)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) <= 1e-5


@pytest.mark.parametrize("batch", [1, 8])
def test_plan_gemm_reports_corrupt_blocks(hip, oracle, batch):
    """Fused GEMM by substream: a block whose XKSP2 header is damaged (block 1)
    and one whose substream code bits are damaged (block 3) are reported, their
    Y rows are left untouched, and every other block's rows are exact."""
    rows, cols = 96, 4096
    w = syn.normal_bf16(77 + batch, (rows, cols))
    enc, table = hip.encode_tensor(w, 2)
    enc = enc.copy()
    table = table.copy()
    table["out_offset"] //= cols * 2
    t1, t3 = table[1], table[3]
    enc[t1["offset"]] ^= 0x01                       # magic
    _corrupt_code_bits(oracle, enc, t3)             # code bits of the last substream
    assert oracle.unpack_parallel(enc[t1["offset"]:t1["offset"] + t1["size"]].tobytes())[0] != 0
    d_arc = _upload(enc)
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    x = torch.randn(batch, cols, generator=g, device="cuda").to(torch.bfloat16).contiguous()
    y = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
    plan.gemm_bf16(d_arc.data_ptr(), x.data_ptr(), batch, y.data_ptr())
    n, first, bits = plan.errors()
    assert (n, first) == (2, 1) and bits == xksv_hip.ERR_HEADER | xksv_hip.ERR_STREAM
    got = y.cpu().numpy()
    wt = torch.from_numpy(syn.bf16_to_f32(w).astype(np.float64)).to("cuda")
    want = (x.double() @ wt.T).cpu().numpy()
    bad = {1, 3}
    for b in range(rows // 16):
        sl = got[:, 16 * b:16 * b + 16]
        if b in bad:
            assert np.isnan(sl).all()
        else:
            err = np.linalg.norm(sl - want[:, 16 * b:16 * b + 16]) / np.linalg.norm(want[:, 16 * b:16 * b + 16])
            assert err <= 1e-5, (b, err)
    plan.close()


def _resplit(hip, oracle, w, chunks) -> bytes:
    """An XKSP2 block of slab `w` (16 rows) with `chunks` substreams (src/c_api.cpp:44-65
    layout; any chunk count <= 32 is valid, src/c_api.cpp:66-72)."""
    rows, cols = w.shape
    tiled = oracle.tile(w, rows, cols)
    n = rows * cols
    segs = [hip.call("xksv_pack", raw_bytes(tiled[n * i // chunks:n * (i + 1) // chunks]), 1,
                     n * (i + 1) // chunks - n * i // chunks) for i in range(chunks)]
    blob = (b"XKSP2\0\0\0" + rows.to_bytes(8, "little") + cols.to_bytes(8, "little") + chunks.to_bytes(8, "little") +
            b"".join(len(s).to_bytes(8, "little") for s in segs) + b"".join(segs))
    assert oracle.unpack_parallel(blob) == (0, raw_bytes(w))
    return blob


@pytest.mark.parametrize("batch", [1, 3, 8])
def test_plan_gemm_nonstandard_chunk_counts(hip, oracle, batch):
    """Plan GEMMs over XKSP2 blocks re-split into 32, 5, 7, 1, 31 and 16 substreams: blocks
    whose substreams do not start on 8-element boundaries are routed to decode + plain GEMM,
    the others to the fused kernels; fp32 X and bf16 X (MFMA on whole-tile substreams) both match fp64."""
    cols = 1024
    counts = (32, 5, 7, 1, 31, 16)
    w = syn.normal_bf16(900 + batch, (16 * len(counts), cols))
    blobs = [_resplit(hip, oracle, w[16 * i:16 * i + 16], c) for i, c in enumerate(counts)]
    enc = np.frombuffer(b"".join(blobs), np.uint8)
    table = np.zeros(len(blobs), xksv_hip.BLOCK_DTYPE)
    off = 0
    for i, b in enumerate(blobs):
        table[i] = (off, len(b), 16 * cols * 2, 16 * i, 16, cols, xksv_hip.CODEC_PARALLEL, 0)
        off += len(b)
    d_arc = _upload(enc)
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    wt = torch.from_numpy(syn.bf16_to_f32(w).astype(np.float64)).to("cuda")
    try:
        x = torch.randn(cols, batch, dtype=torch.float32, device="cuda")
        y = torch.full((16 * len(counts), batch), float("nan"), dtype=torch.float32, device="cuda")
        plan.gemm(d_arc.data_ptr(), x.data_ptr(), batch, y.data_ptr())
        assert plan.errors()[0] == 0
        want = (wt @ x.double()).cpu().numpy()
        assert np.linalg.norm(y.cpu().numpy() - want) / np.linalg.norm(want) <= 1e-5
        xb = torch.randn(batch, cols, device="cuda").to(torch.bfloat16).contiguous()
        yb = torch.full((batch, 16 * len(counts)), float("nan"), dtype=torch.float32, device="cuda")
        plan.gemm_bf16(d_arc.data_ptr(), xb.data_ptr(), batch, yb.data_ptr())
        assert plan.errors()[0] == 0
        want = (xb.double() @ wt.T).cpu().numpy()
        assert np.linalg.norm(yb.cpu().numpy() - want) / np.linalg.norm(want) <= 2e-3
    finally:
        plan.close()


def test_plan_decode_tail_quarters_few_substreams(hip, oracle):
    """8,192 plan entries (one wave per block; the last grid's worth of blocks is claimed a
    quarter at a time) over 16x1024 slabs re-split into 1, 2, 3, 5 and 32 substreams, so
    some quarter claims hold no substream and others hold one or two; entry i decodes
    slab i % 5 into its own output, one slab's code bits are damaged: exactly its entries
    are reported and every other entry decodes exactly."""
    counts = (1, 2, 3, 5, 32)
    w = syn.normal_bf16(3100, (16 * len(counts), 1024))
    blobs = [_resplit(hip, oracle, w[16 * i:16 * i + 16], c) for i, c in enumerate(counts)]
    enc = np.frombuffer(b"".join(blobs), np.uint8).copy()
    base = np.zeros(len(blobs), xksv_hip.BLOCK_DTYPE)
    off = 0
    for i, b in enumerate(blobs):
        base[i] = (off, len(b), 32768, 0, 16, 1024, xksv_hip.CODEC_PARALLEL, 0)
        off += len(b)
    _corrupt_code_bits(oracle, enc, base[2])  # the 3-substream slab
    n = 8192
    table = np.resize(base, n).copy()
    table["out_offset"] = np.arange(n, dtype=np.uint64) * 32768
    d_arc = _upload(enc)
    out = torch.zeros(n * 32768, dtype=torch.uint8, device="cuda")
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    try:
        plan.decode(d_arc.data_ptr(), out.data_ptr(), out.numel())
        nbad, first, bits = plan.errors()
    finally:
        plan.close()
    bad = np.arange(n) % len(counts) == 2
    assert (nbad, first, bits) == (int(bad.sum()), 2, xksv_hip.ERR_STREAM)
    host = out.cpu().numpy().reshape(n, -1)
    want = w.view(np.uint8).reshape(len(counts), -1)[np.arange(n) % len(counts)]
    assert np.array_equal(host[~bad], want[~bad])


@pytest.mark.parametrize("cols", [4096, 4112])
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 8, 16])
def test_plan_gemm_staged_x(hip, batch, cols):
    """Indexed fused GEMMs copy each segment's x columns into LDS when x and its rows are
    16-byte aligned, and read x from global memory otherwise (x shifted by one element).
    4096 columns: substreams of whole tiles (bf16 MFMA, 8-tile segments);
    4112: substreams start mid-tile (VALU consumers, 9-tile segments).  Both layouts, both
    activation types, both placements match fp64; runs at one placement are bit-identical
    to each other."""
    rows = 64
    w = syn.normal_bf16(1300 + cols + batch, (rows, cols))
    enc, table = hip.encode_tensor(w, 2)
    table = table.copy()
    table["out_offset"] //= cols * 2
    d_arc = _upload(enc)
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    wt = torch.from_numpy(syn.bf16_to_f32(w).astype(np.float64)).to("cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(batch)
    try:
        for shift in (0, 1):
            xbuf = torch.randn(batch * cols + 8, generator=g, device="cuda")
            xb = xbuf.to(torch.bfloat16)[shift:shift + batch * cols].view(batch, cols)
            assert (xb.data_ptr() % 16 == 0) == (shift == 0)
            yb = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
            plan.gemm_bf16(d_arc.data_ptr(), xb.data_ptr(), batch, yb.data_ptr())
            assert plan.errors()[0] == 0
            want = (xb.double() @ wt.T).cpu().numpy()
            err = np.linalg.norm(yb.cpu().numpy() - want) / np.linalg.norm(want)
            assert err <= 2e-3 and err <= 1e-5, (shift, err)
            yb2 = torch.empty_like(yb)
            plan.gemm_bf16(d_arc.data_ptr(), xb.data_ptr(), batch, yb2.data_ptr())
            assert torch.equal(yb, yb2)
            xf = xbuf[shift:shift + batch * cols].view(cols, batch)
            yf = torch.full((rows, batch), float("nan"), dtype=torch.float32, device="cuda")
            plan.gemm(d_arc.data_ptr(), xf.data_ptr(), batch, yf.data_ptr())
            assert plan.errors()[0] == 0
            want = (wt @ xf.double()).cpu().numpy()
            err = np.linalg.norm(yf.cpu().numpy() - want) / np.linalg.norm(want)
            assert err <= 1e-5, (shift, err)
    finally:
        plan.close()


def _gemv(plan, d_arc, x, rows):
    y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    plan.gemm(d_arc.data_ptr(), x.data_ptr(), 1, y.data_ptr())
    return y, plan.errors()


def test_plan_gemv_index_across_archives(hip, oracle):
    """The fused GEMV's codeword index is built from the archive of the first GEMM call
    and checked on every use.  Same table, other archives:
    * sign-flipped weights (same code bits, so the index still holds): y is exact;
    * code bits changed after the index was built (a stale index): the changed
      segment does not chain and decodes speculatively, so a block the oracle
      rejects is reported and a block the oracle decodes differently gives the GEMV
      of the oracle's weights."""
    rows, cols = 64, 4096
    w = syn.normal_bf16(4242, (rows, cols))
    enc, table = hip.encode_tensor(w, 2)
    table = table.copy()
    table["out_offset"] //= cols * 2
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    x = torch.randn(cols, dtype=torch.float32, device="cuda")
    xd = x.cpu().numpy().astype(np.float64)
    try:
        y, errs = _gemv(plan, _upload(enc), x, rows)  # builds the index
        assert errs[0] == 0
        assert np.linalg.norm(y.cpu().numpy() - oracle.gemm_f64(w, xd)) <= 1e-5 * np.linalg.norm(oracle.gemm_f64(w, xd))
        wn = w ^ np.uint16(0x8000)
        enc_n, table_n = hip.encode_tensor(wn, 2)
        assert enc_n.nbytes == enc.nbytes and np.array_equal(table_n["size"], table["size"])
        yn, errs = _gemv(plan, _upload(enc_n), x, rows)
        assert errs[0] == 0 and torch.equal(yn, -y)

        # code bits of block 1, last substream: one flip the oracle rejects, one it accepts
        t = table[1]
        blob = enc[int(t["offset"]):int(t["offset"] + t["size"])].tobytes()
        rejected = accepted = None
        for back in range(2, 600):
            for bit in range(8):
                b = bytearray(blob)
                b[len(b) - back] ^= 1 << bit
                rc, dec = oracle.unpack_parallel(bytes(b))
                if rc and rejected is None:
                    rejected = (back, bit)
                if rc == 0 and dec != blob and accepted is None and dec != raw_bytes(w[16:32]):
                    accepted = (back, bit, dec)
            if rejected and accepted:
                break
        assert rejected is not None
        enc_r = enc.copy()
        enc_r[int(t["offset"] + t["size"]) - rejected[0]] ^= 1 << rejected[1]
        yr, errs = _gemv(plan, _upload(enc_r), x, rows)
        assert errs[:2] == (1, 1) and errs[2] == xksv_hip.ERR_STREAM
        keep = np.r_[0:16, 32:64]
        assert torch.equal(yr[keep], y[keep])
        y2, errs = _gemv(plan, _upload(enc), x, rows)  # status words are stored per call, not accumulated
        assert errs[0] == 0 and torch.equal(y2, y)
        if accepted is not None:
            back, bit, dec = accepted
            enc_a = enc.copy()
            enc_a[int(t["offset"] + t["size"]) - back] ^= 1 << bit
            ya, errs = _gemv(plan, _upload(enc_a), x, rows)
            assert errs[0] == 0
            wa = w.copy()
            wa[16:32] = np.frombuffer(dec, np.uint16).reshape(16, cols)
            want = oracle.gemm_f64(wa, xd)
            assert np.linalg.norm(ya.cpu().numpy() - want) <= 1e-5 * np.linalg.norm(want)
    finally:
        plan.close()


def test_plan_gemv_unindexed_items(hip, oracle):
    """Substreams whose segments are too long for the index (high-entropy exponents:
    about 6 bits per code) take the speculative path; y matches fp64."""
    rows, cols = 32, 4096
    rng = np.random.default_rng(77)
    w = ((rng.integers(64, 128, rows * cols, dtype=np.uint32) << 7) | rng.integers(0, 256, rows * cols, dtype=np.uint32))
    w = w.astype(np.uint16).reshape(rows, cols)
    enc, table = hip.encode_tensor(w, 2)
    assert set(table["codec"]) == {xksv_hip.CODEC_PARALLEL}
    table = table.copy()
    table["out_offset"] //= cols * 2
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    try:
        x = torch.randn(cols, dtype=torch.float32, device="cuda")
        y, errs = _gemv(plan, _upload(enc), x, rows)
        assert errs[0] == 0
        want = oracle.gemm_f64(w, x.cpu().numpy().astype(np.float64))
        assert np.linalg.norm(y.cpu().numpy() - want) <= 1e-5 * np.linalg.norm(want)
    finally:
        plan.close()

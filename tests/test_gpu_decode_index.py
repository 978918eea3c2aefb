"""Plan decode with a codeword index (xksv_hip_plan_index), GPU only.

The index is a load-time sidecar for weights that stay resident: per 2,048 symbols of
every parallel32 substream, the bit offset of every 32nd codeword.  Decodes after
xksv_hip_plan_index start each lane of a wave at a recorded codeword instead of
entering speculatively.  Every entry is checked as it is used, so the index may only
change speed: these tests hold the indexed decode to the same bytes and the same
per-block verdicts as the decode without an index and the oracle, for

* both decode schedules (one work item per substream below twice the resident waves,
  one wave per block above), with corrupt blocks reported exactly;
* an index built from another archive: same code bits (sign-flipped weights: exact),
  code bits changed after the index was built (one change the oracle rejects, one it
  decodes to other bytes);
* substreams the index cannot hold (blocks re-split into 1, 5, 7 and 31 substreams,
  high-entropy slabs whose segments are too long), 4,096- and 14,336-wide slabs,
  slabs of fewer than 16 rows, raw and serial blocks in the same plan;
* a rebuilt index, and an index over a plan with no parallel32 blocks.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import xksv_hip
import xksv_synth as syn
from oracle_lib import raw_bytes

pytestmark = pytest.mark.gpu


def _upload(arr: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(arr).view(np.uint8).reshape(-1).copy()).to("cuda")


def _decode(plan, d_arc, nbytes):
    out = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    plan.decode(d_arc.data_ptr(), out.data_ptr(), out.numel())
    return out.cpu().numpy(), plan.errors()


def _corrupt(oracle, enc, t, rejected: bool):
    """Flip one bit of block t's last substream's code bits (nearest the end first) that
    the oracle rejects (rejected=True) or decodes to other bytes; returns the oracle's
    bytes for an accepted flip, None for a rejected one."""
    off, end = int(t["offset"]), int(t["offset"] + t["size"])
    blob = enc[off:end].tobytes()
    clean = oracle.unpack_parallel(blob)[1]
    for back in range(2, 600):
        for bit in range(8):
            b = bytearray(blob)
            b[len(b) - back] ^= 1 << bit
            rc, dec = oracle.unpack_parallel(bytes(b))
            if rejected and rc:
                enc[end - back] ^= 1 << bit
                return None
            if not rejected and rc == 0 and dec != clean:
                enc[end - back] ^= 1 << bit
                return dec
    raise AssertionError("no such flip")


@pytest.mark.parametrize("nblocks", [4, 8192])
def test_indexed_decode_both_schedules(hip, oracle, nblocks):
    """Entry i decodes 16x1024 slab i % 64; slab 1's code bits and slab 2's magic are
    damaged after the index was built from the clean archive."""
    w = syn.normal_bf16(143, (16 * 64, 1024))
    enc, base = hip.encode_tensor(w, 2, 1024)
    table = np.resize(base, nblocks).copy()
    table["out_offset"] = np.arange(nblocks, dtype=np.uint64) * 32768
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    try:
        plan.index(_upload(enc).data_ptr())
        host, errs = _decode(plan, _upload(enc), nblocks * 32768)
        want = w.view(np.uint8).reshape(64, -1)[np.arange(nblocks) % 64]
        assert errs[0] == 0 and np.array_equal(host.reshape(nblocks, -1), want)
        bad_enc = enc.copy()
        _corrupt(oracle, bad_enc, base[1], rejected=True)
        bad_enc[int(base[2]["offset"])] ^= 0x01
        host, (n, first, bits) = _decode(plan, _upload(bad_enc), nblocks * 32768)
        bad = np.isin(np.arange(nblocks) % 64, (1, 2))
        assert (n, first) == (int(bad.sum()), 1) and bits == xksv_hip.ERR_STREAM | xksv_hip.ERR_HEADER
        assert np.array_equal(host.reshape(nblocks, -1)[~bad], want[~bad])
    finally:
        plan.close()


def test_indexed_decode_other_archives(hip, oracle):
    """Index built from archive A, decodes of A, of sign-flipped A (same code bits), of A
    with a rejected and with an accepted code-bit change, then of A again."""
    rows, cols = 64, 14336
    w = syn.normal_bf16(144, (rows, cols))
    enc, table = hip.encode_tensor(w, 2)
    assert set(table["cols"]) == {cols}
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    try:
        plan.index(_upload(enc).data_ptr())
        host, errs = _decode(plan, _upload(enc), w.nbytes)
        assert errs[0] == 0 and host.tobytes() == raw_bytes(w)
        wn = w ^ np.uint16(0x8000)
        enc_n, table_n = hip.encode_tensor(wn, 2)
        assert np.array_equal(table_n["size"], table["size"])
        host, errs = _decode(plan, _upload(enc_n), w.nbytes)
        assert errs[0] == 0 and host.tobytes() == raw_bytes(wn)
        enc_r = enc.copy()
        assert _corrupt(oracle, enc_r, table[1], rejected=True) is None
        host, errs = _decode(plan, _upload(enc_r), w.nbytes)
        assert errs == (1, 1, xksv_hip.ERR_STREAM)
        slab = cols * 32
        assert host[:slab].tobytes() == raw_bytes(w)[:slab] and host[2 * slab:].tobytes() == raw_bytes(w)[2 * slab:]
        enc_a = enc.copy()
        dec = _corrupt(oracle, enc_a, table[2], rejected=False)
        host, errs = _decode(plan, _upload(enc_a), w.nbytes)
        assert errs[0] == 0
        want = bytearray(raw_bytes(w))
        want[2 * slab:3 * slab] = dec
        assert host.tobytes() == bytes(want)
        host, errs = _decode(plan, _upload(enc), w.nbytes)
        assert errs[0] == 0 and host.tobytes() == raw_bytes(w)
    finally:
        plan.close()


def _resplit(hip, oracle, w, chunks) -> bytes:
    rows, cols = w.shape
    tiled = oracle.tile(w, rows, cols)
    n = rows * cols
    segs = [hip.call("xksv_pack", raw_bytes(tiled[n * i // chunks:n * (i + 1) // chunks]), 1,
                     n * (i + 1) // chunks - n * i // chunks) for i in range(chunks)]
    return (b"XKSP2\0\0\0" + rows.to_bytes(8, "little") + cols.to_bytes(8, "little") + chunks.to_bytes(8, "little") +
            b"".join(len(s).to_bytes(8, "little") for s in segs) + b"".join(segs))


def test_indexed_decode_mixed_plan(hip, oracle):
    """One plan: 4,096- and 14,336-wide parallel32 slabs, a 5-row slab, blocks re-split into
    1, 5, 7 and 31 substreams (the allotment holds 32), a high-entropy slab (segments too
    long to index), serial and raw blocks.  Bytes equal the inputs with and without the
    index; the index is then rebuilt and used again."""
    parts, table_rows = [], []
    off = out = 0

    def add(blob, rows, cols, codec, raw):
        nonlocal off, out
        parts.append(blob)
        table_rows.append((off, len(blob), len(raw), out, rows if codec else 0, cols if codec else 0, codec, 0))
        off += len(blob)
        out += len(raw)

    expect = []
    for i, (rows, cols) in enumerate([(16, 4096), (16, 14336), (5, 4096)]):
        w = syn.normal_bf16(150 + i, (rows, cols))
        add(hip.call("xksv_pack_parallel", raw_bytes(w), rows, cols), rows, cols, 2, raw_bytes(w))
        expect.append(raw_bytes(w))
    for i, chunks in enumerate((1, 5, 7, 31)):
        w = syn.normal_bf16(160 + i, (16, 4096))
        blob = _resplit(hip, oracle, w, chunks)
        assert oracle.unpack_parallel(blob) == (0, raw_bytes(w))
        add(blob, 16, 4096, 2, raw_bytes(w))
        expect.append(raw_bytes(w))
    rng = np.random.default_rng(170)
    w = ((rng.integers(64, 128, 16 * 4096, dtype=np.uint32) << 7) | rng.integers(0, 256, 16 * 4096, dtype=np.uint32))
    w = w.astype(np.uint16).reshape(16, 4096)
    add(hip.call("xksv_pack_parallel", raw_bytes(w), 16, 4096), 16, 4096, 2, raw_bytes(w))
    expect.append(raw_bytes(w))
    w = syn.normal_bf16(171, (16, 4096))
    add(hip.call("xksv_pack", raw_bytes(w), 16, 4096), 16, 4096, 1, raw_bytes(w))
    expect.append(raw_bytes(w))
    raw = syn.normal_bf16(172, (1, 4096)).tobytes()
    add(raw, 0, 0, 0, raw)
    expect.append(raw)
    enc = np.frombuffer(b"".join(parts), np.uint8)
    table = np.array(table_rows, dtype=xksv_hip.BLOCK_DTYPE)
    want = b"".join(expect)
    d_arc = _upload(enc)
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    try:
        host, errs = _decode(plan, d_arc, len(want))
        assert errs[0] == 0 and host.tobytes() == want
        for _ in range(2):
            plan.index(d_arc.data_ptr())
            host, errs = _decode(plan, d_arc, len(want))
            assert errs[0] == 0 and host.tobytes() == want
    finally:
        plan.close()


def test_index_without_parallel_blocks(hip):
    w = syn.normal_bf16(180, (16, 4096))
    enc, table = hip.encode_tensor(w, 1)
    assert set(table["codec"]) == {xksv_hip.CODEC_SERIAL}
    d_arc = _upload(enc)
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    try:
        plan.index(d_arc.data_ptr())
        host, errs = _decode(plan, d_arc, w.nbytes)
        assert errs[0] == 0 and host.tobytes() == raw_bytes(w)
    finally:
        plan.close()


def test_index_and_gemm_on_one_plan(hip, oracle):
    """A decode plan with the decode index and a GEMM plan over the same archive (whose fused
    GEMMs build their own index on the first call, and which then gets a decode index too):
    decodes and GEMVs interleaved stay exact."""
    rows, cols = 64, 4096
    w = syn.normal_bf16(190, (rows, cols))
    enc, table = hip.encode_tensor(w, 2)
    d_arc = _upload(enc)
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    gtable = table.copy()
    gtable["out_offset"] //= cols * 2
    gplan = xksv_hip.Plan(hip, gtable, enc.nbytes)
    try:
        plan.index(d_arc.data_ptr())
        x = torch.randn(cols, device="cuda")
        want_y = oracle.gemm_f64(w, x.cpu().numpy().astype(np.float64))
        for _ in range(2):
            host, errs = _decode(plan, d_arc, w.nbytes)
            assert errs[0] == 0 and host.tobytes() == raw_bytes(w)
            y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
            gplan.gemm(d_arc.data_ptr(), x.data_ptr(), 1, y.data_ptr())
            assert gplan.errors()[0] == 0
            got = y.cpu().numpy().astype(np.float64)
            assert np.linalg.norm(got - want_y) <= 1e-5 * np.linalg.norm(want_y)
            gplan.index(d_arc.data_ptr())  # a decode index on the GEMM plan too: GEMMs unaffected
    finally:
        plan.close()
        gplan.close()

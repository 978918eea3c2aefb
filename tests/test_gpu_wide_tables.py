"""Fused GEMV/GEMM at batch 1 over wide slabs (16,384 columns: substreams of 8,192 symbols), GPU only.

Long substreams run many segments of the decode walk per stream, and the batch-1 VALU
consumers (fp32 x) and the MFMA consumer (bf16 x) read them through both walks: the
indexed walk (plan, codeword index built on the first call) and the speculative one
(block API, no index; and wherever an index entry does not chain).  These tests pin both
walks to the oracle on edge cases of the two-symbol lookup table:

* crafted substreams, each from an explicit lengths table: 1-bit codes (two symbols per
  lookup, streams ending inside a pair), codes of exactly the window's 10 bits, codes of
  11-31 bits resolved inside the step, codes of up to 39 bits (the bit-serial path), flat
  3-bit codes (three fit the window, two are taken) and flat 5-bit codes (two filling the
  window);
* the plan (indexed walk) and the block API (speculative walk), fp32 and bf16 activations;
* code bits changed after the index was built (a stale index: the segment that no
  longer chains continues speculatively), one change the oracle rejects and one it
  decodes to other weights;
* high-entropy slabs whose segments are too long for the index.

Expected values: the oracle's CPU decode of the same bytes, then an fp64 GEMV (rel-L2
<= 1e-5 per 16-row slab for fp32 x; bf16 x is held to the same 1e-5, inside its 2e-3
bound), for a random x, for x restricted to each crafted substream's columns, and, exactly,
for one-hot x at the columns of each crafted substream's longest codes and of a few random
symbols (y is then that column of the weights).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import xksv_hip
import xksv_synth as syn
from oracle_lib import craft_segment, raw_bytes

pytestmark = pytest.mark.gpu
TOL = 1e-5
COLS = 16384  # 16-row slabs of 16,384 columns: substreams of 8,192 symbols (4 index segments)


def _rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return np.linalg.norm(got - want) / (den if den else 1.0)


def _upload(arr) -> torch.Tensor:
    a = np.frombuffer(bytes(arr), np.uint8) if isinstance(arr, (bytes, bytearray)) else arr
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).to("cuda")


def _chain(maxlen: int, top: int) -> list:
    """Complete code of lengths 1, 2, ..., maxlen - 1, maxlen - 1 on symbols top, top - 1, ...:
    the frequent short codes carry the largest exponents, so they dominate y."""
    lens = [0] * 256
    for i in range(maxlen - 1):
        lens[top - i] = i + 1
    lens[top - (maxlen - 1)] = maxlen - 1
    return lens


def _flat(bits: int, first: int) -> list:
    lens = [0] * 256
    for s in range(first, first + (1 << bits)):
        lens[s] = bits
    return lens


def _lengths(kind: str) -> list:
    """A complete lengths table; exponents stay between 2^-45 and 2^8 (finite BF16)."""
    lens = {
        "one_bit": _chain(3, 124),   # 1, 2, 2: pairs of short codes, lanes ending inside a pair
        "ten_bit": _chain(11, 124),  # up to 10 bits: codes that fill the window exactly
        "long31": _chain(32, 124),   # up to 31 bits: long codes resolved inside the step
        "long40": _chain(40, 124),   # up to 39 bits: the bit-serial path
        "flat3": _flat(3, 118),      # 3-bit codes: three fit the window, a lookup takes two
        "flat5": _flat(5, 104),      # two 5-bit codes fill the 10-bit window exactly
    }[kind]
    assert abs(sum(2.0 ** -l for l in lens if l) - 1.0) < 1e-12
    return lens


def _symbols(lens, n, rng) -> tuple[list, list]:
    """n symbols drawn 90 % by code length (2^-l) and 10 % uniformly, so long codes occur
    often; the three longest codes are placed first, in the middle and last.  Returns the
    symbols and those three positions."""
    syms = [s for s in range(256) if lens[s]]
    p = np.array([2.0 ** -lens[s] for s in syms])
    p = 0.9 * p / p.sum() + 0.1 / len(syms)
    pick = [syms[i] for i in rng.choice(len(syms), size=n, p=p)]
    longest = sorted(syms, key=lambda s: lens[s])[-3:]
    at = [0, n // 2, n - 1]
    for j, s in zip(at, longest):
        pick[j] = s
    return pick, at


def _split(blob: bytes):
    chunks = int.from_bytes(blob[24:32], "little")
    sizes = [int.from_bytes(blob[32 + 8 * i:40 + 8 * i], "little") for i in range(chunks)]
    segs, pos = [], 32 + 8 * chunks
    for n in sizes:
        segs.append(bytes(blob[pos:pos + n]))
        pos += n
    return bytes(blob[:32]), segs


def _join(head: bytes, segs) -> bytes:
    return head + b"".join(len(s).to_bytes(8, "little") for s in segs) + b"".join(segs)


def _crafted_block(hip, oracle, seed: int, kinds: dict):
    """A 16 x COLS XKSP2 block whose substreams listed in `kinds` (index -> lengths kind)
    are re-coded from explicit tables.  Returns the block, the oracle's weights and, per
    crafted substream, its column range and the columns holding its longest codes and a
    few random symbols."""
    w = syn.normal_bf16(seed, (16, COLS))
    head, segs = _split(hip.call("xksv_pack_parallel", raw_bytes(w), 16, COLS))
    rng = np.random.default_rng(seed)
    probes = {}
    per = 16 * COLS // len(segs)  # symbols per substream, whole 16x16 tiles
    for i, kind in kinds.items():
        n = int.from_bytes(segs[i][:8], "little")
        assert n == per
        lens = _lengths(kind)
        syms, at = _symbols(lens, n, rng)
        segs[i] = craft_segment(lens, syms, rng.integers(0, 256, n))
        # symbol j of substream i is tiled element per*i + j: tile (per*i + j) // 256,
        # column 16 * tile + (element % 16)
        cols = sorted({16 * ((per * i + j) // 256) + (per * i + j) % 16
                       for j in at + [int(v) for v in rng.integers(0, n, 5)]})
        probes[i] = ((16 * (per * i // 256), 16 * (per * (i + 1) // 256)), cols)
    blob = _join(head, segs)
    rc, dec = oracle.unpack_parallel(blob)
    assert rc == 0
    return blob, np.frombuffer(dec, np.uint16).reshape(16, COLS), probes


def _check_gemv(gemv, oracle, w, probes, seed):
    """gemv(x) -> y (numpy, fp32 x of COLS or bf16 x as float values) against the oracle's
    weights: random x (rel-L2 per 16-row block), x restricted to each crafted substream's
    columns (rel-L2 per block), and one-hot x at probe columns (exact: y is that column)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn(COLS, generator=g, device="cuda")
    tests = [(x, None)]
    for (c0, c1), _ in probes.values():
        xm = torch.zeros_like(x)
        xm[c0:c1] = x[c0:c1]
        tests.append((xm, None))
    for _, cols in probes.values():
        for c in cols:
            xo = torch.zeros_like(x)
            xo[c] = 1.0
            tests.append((xo, c))
    rows = w.shape[0]
    for xv, col in tests:
        y, xd = gemv(xv)
        if col is not None:
            assert np.array_equal(y, syn.bf16_to_f32(w[:, col])), col
            continue
        want = oracle.gemm_f64(w, xd)
        for b in range(0, rows, 16):
            assert _rel_l2(y[b:b + 16], want[b:b + 16]) <= TOL, b


# Per block: which substreams take which crafted table (first, middle and last substreams).
LAYOUTS = [
    {0: "one_bit", 15: "ten_bit", 31: "long31"},
    {0: "long40", 7: "flat3", 31: "one_bit"},
    {3: "long31", 16: "long40", 30: "flat5"},
    {},  # an ordinary slab
]


def _archive(hip, oracle, base_seed):
    """The LAYOUTS blocks as one archive (table rows index GEMM output rows)."""
    blobs, ws, probes = [], [], {}
    for i, kinds in enumerate(LAYOUTS):
        blob, w, pr = _crafted_block(hip, oracle, base_seed + i, kinds)
        blobs.append(blob)
        ws.append(w)
        for k, (rng_, cols) in pr.items():  # blocks share column ranges: merge the probes
            probes[k] = (rng_, sorted(set(probes.get(k, (rng_, []))[1]) | set(cols)))
    enc = np.frombuffer(b"".join(blobs), np.uint8)
    table = np.zeros(len(blobs), xksv_hip.BLOCK_DTYPE)
    off = 0
    for i, b in enumerate(blobs):
        table[i] = (off, len(b), 16 * COLS * 2, 16 * i, 16, COLS, xksv_hip.CODEC_PARALLEL, 0)
        off += len(b)
    return blobs, enc, table, np.concatenate(ws), probes


def test_plan_crafted_tables_both_activations(hip, oracle):
    """Indexed walk (plan; the index is built on the first call and reused after it) for
    fp32 x and bf16 x at batch 1, plus the plan decode (two-symbol tables) of the same
    archive, bit-exact."""
    _, enc, table, w, probes = _archive(hip, oracle, 610)
    rows = w.shape[0]
    d_arc = _upload(enc)
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    try:
        def f32(xv):
            y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
            plan.gemm(d_arc.data_ptr(), xv.data_ptr(), 1, y.data_ptr())
            assert plan.errors()[0] == 0
            return y.cpu().numpy(), xv.cpu().numpy().astype(np.float64)

        def bf16(xv):
            xb = xv.to(torch.bfloat16).reshape(1, COLS).contiguous()
            y = torch.full((1, rows), float("nan"), dtype=torch.float32, device="cuda")
            plan.gemm_bf16(d_arc.data_ptr(), xb.data_ptr(), 1, y.data_ptr())
            assert plan.errors()[0] == 0
            return y.cpu().numpy()[0], xb.double().cpu().numpy()[0]

        _check_gemv(f32, oracle, w, probes, 3)
        _check_gemv(bf16, oracle, w, probes, 4)
    finally:
        plan.close()
    out = torch.zeros(w.nbytes, dtype=torch.uint8, device="cuda")
    dt = table.copy()
    dt["out_offset"] = np.arange(len(table)) * 16 * COLS * 2
    dplan = xksv_hip.Plan(hip, dt, enc.nbytes)
    try:
        dplan.decode(d_arc.data_ptr(), out.data_ptr(), out.numel())
        assert dplan.errors()[0] == 0
    finally:
        dplan.close()
    assert np.array_equal(out.cpu().numpy().view(np.uint16).reshape(w.shape), w)


@pytest.mark.parametrize("layout", range(len(LAYOUTS)))
def test_block_api_crafted_tables(hip, oracle, layout):
    """Speculative walk (block API, no index), fp32 x and bf16 x at batch 1."""
    blob, w, probes = _crafted_block(hip, oracle, 700 + layout, LAYOUTS[layout])

    def f32(xv):
        y = torch.full((16,), float("nan"), dtype=torch.float32, device="cuda")
        assert hip.gemv_parallel(blob, xv.data_ptr(), y.data_ptr()) == 0
        return y.cpu().numpy(), xv.cpu().numpy().astype(np.float64)

    def bf16(xv):
        xb = xv.to(torch.bfloat16).reshape(1, COLS).contiguous()
        y = torch.full((1, 16), float("nan"), dtype=torch.float32, device="cuda")
        assert hip.gemm_parallel_bf16(blob, 1, xb.data_ptr(), y.data_ptr()) == 0
        return y.cpu().numpy()[0], xb.double().cpu().numpy()[0]

    _check_gemv(f32, oracle, w, probes, 10 + layout)
    _check_gemv(bf16, oracle, w, probes, 20 + layout)


def _flips(oracle, blob: bytes, seg_end: int, clean: bytes):
    """(rejected, accepted) byte flips in the code bits ending at seg_end: the first the
    oracle rejects, and the first it decodes to other weights (or None)."""
    rejected = accepted = None
    for back in range(1, 400):
        for bit in range(8):
            b = bytearray(blob)
            b[seg_end - back] ^= 1 << bit
            rc, dec = oracle.unpack_parallel(bytes(b))
            if rc and rejected is None:
                rejected = (seg_end - back, bit)
            if rc == 0 and dec != clean and accepted is None:
                accepted = (seg_end - back, bit, dec)
        if rejected and accepted:
            break
    return rejected, accepted


def test_plan_stale_index_wide(hip, oracle):
    """Code bits of a crafted wide substream changed after the plan indexed the archive:
    a change the oracle rejects is reported for that block only (other rows unchanged),
    one it accepts gives the GEMV of the oracle's weights; the clean archive afterwards
    gives the first result again."""
    blobs, enc, table, w, _ = _archive(hip, oracle, 820)
    rows = w.shape[0]
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    try:
        x = torch.randn(COLS, device="cuda")
        xd = x.cpu().numpy().astype(np.float64)
        y0 = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
        plan.gemm(_upload(enc).data_ptr(), x.data_ptr(), 1, y0.data_ptr())  # builds the index
        assert plan.errors()[0] == 0
        assert _rel_l2(y0.cpu().numpy(), oracle.gemm_f64(w, xd)) <= TOL
        # block 0, substream 15 (10-bit codes): flip inside its code bits
        blk = 0
        head, segs = _split(blobs[blk])
        seg_end = 32 + 8 * len(segs) + sum(len(s) for s in segs[:16])
        clean = raw_bytes(w[16 * blk:16 * blk + 16])
        rejected, accepted = _flips(oracle, blobs[blk], seg_end, clean)
        assert rejected is not None
        base = int(table[blk]["offset"])
        enc_r = enc.copy()
        enc_r[base + rejected[0]] ^= 1 << rejected[1]
        yr = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
        plan.gemm(_upload(enc_r).data_ptr(), x.data_ptr(), 1, yr.data_ptr())
        n, first, bits = plan.errors()
        assert (n, first, bits) == (1, blk, xksv_hip.ERR_STREAM)
        keep = np.r_[16 * (blk + 1):rows]
        assert torch.equal(yr[keep], y0[keep])
        if accepted is not None:
            pos, bit, dec = accepted
            enc_a = enc.copy()
            enc_a[base + pos] ^= 1 << bit
            ya = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
            plan.gemm(_upload(enc_a).data_ptr(), x.data_ptr(), 1, ya.data_ptr())
            assert plan.errors()[0] == 0
            wa = w.copy()
            wa[16 * blk:16 * blk + 16] = np.frombuffer(dec, np.uint16).reshape(16, COLS)
            assert _rel_l2(ya.cpu().numpy(), oracle.gemm_f64(wa, xd)) <= TOL
        y2 = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
        plan.gemm(_upload(enc).data_ptr(), x.data_ptr(), 1, y2.data_ptr())
        assert plan.errors()[0] == 0 and torch.equal(y2, y0)
    finally:
        plan.close()


def test_plan_unindexed_wide_items(hip, oracle):
    """High-entropy exponents (about 6 bits per code): segments too long for the index take
    the speculative walk; fp32 and bf16 x at batch 1."""
    rows = 32
    rng = np.random.default_rng(91)
    w = ((rng.integers(64, 128, rows * COLS, dtype=np.uint32) << 7) | rng.integers(0, 256, rows * COLS, dtype=np.uint32))
    w = w.astype(np.uint16).reshape(rows, COLS)
    enc, table = hip.encode_tensor(w, 2)
    assert set(table["codec"]) == {xksv_hip.CODEC_PARALLEL} and set(table["cols"]) == {COLS}
    table = table.copy()
    table["out_offset"] //= COLS * 2
    d_arc = _upload(enc)
    plan = xksv_hip.Plan(hip, table, enc.nbytes)
    try:
        x = torch.randn(COLS, device="cuda")
        y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
        plan.gemm(d_arc.data_ptr(), x.data_ptr(), 1, y.data_ptr())
        assert plan.errors()[0] == 0
        assert _rel_l2(y.cpu().numpy(), oracle.gemm_f64(w, x.cpu().numpy().astype(np.float64))) <= TOL
        xb = torch.randn(1, COLS, device="cuda").to(torch.bfloat16).contiguous()
        yb = torch.full((1, rows), float("nan"), dtype=torch.float32, device="cuda")
        plan.gemm_bf16(d_arc.data_ptr(), xb.data_ptr(), 1, yb.data_ptr())
        assert plan.errors()[0] == 0
        assert _rel_l2(yb.cpu().numpy()[0], oracle.gemm_f64(w, xb.double().cpu().numpy()[0])) <= TOL
    finally:
        plan.close()

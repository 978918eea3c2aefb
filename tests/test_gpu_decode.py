"""HIP decode parity: the GPU path through the C ABI against the oracle (GPU only).

Mirrors tests/test_cuda.py:13-65 of the reference (serial shapes x modes,
parallel shapes, truncated block) and extends it to every golden case, the
reference's verdicts on 587 corrupted blocks, blocks with codes longer than
32 bits (bit-serial path), and the GPU-backed CPU unpack entry points.
Bit-exact: every comparison is byte equality / SHA-256 equality.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle_lib import apply_mutation, craft_segment, gen, long_code_lengths, raw_bytes, sha

pytestmark = pytest.mark.gpu


def _dev_bytes(n):
    return torch.zeros(max(n, 1), dtype=torch.uint8, device="cuda")


def _host(t, n):
    return t[:n].cpu().numpy().tobytes()


@pytest.mark.parametrize("rows,cols", [(1, 1), (1, 256), (7, 19), (16, 32), (17, 33), (31, 103)])
@pytest.mark.parametrize("mode", [0, 1])
def test_serial_decode_reference_shapes(hip, oracle, rows, cols, mode):
    """tests/test_cuda.py:13-23: exponent-127..129 pattern and uniform 16-bit words."""
    spec = ({"kind": "uniform16", "seed": 51, "shape": [rows, cols]} if mode
            else {"kind": "exponent_pattern", "seed": 51, "shape": [rows, cols]})
    raw = raw_bytes(gen(spec))
    block = hip.call("xksv_pack", raw, rows, cols)
    assert block == oracle.pack(raw, rows, cols)[1]
    out = _dev_bytes(len(raw))
    assert hip.decode(block, rows, cols, out.data_ptr()) == 0
    assert _host(out, len(raw)) == raw


@pytest.mark.parametrize("rows,cols", [(1, 1), (1, 256), (7, 19), (16, 32), (16, 4096), (16, 4097)])
def test_parallel_decode_reference_shapes(hip, oracle, rows, cols):
    """tests/test_cuda.py:44-61: words i % 65536, checked against CPU unpack and the input."""
    raw = raw_bytes(gen({"kind": "words_mod", "shape": [rows, cols]}))
    block = hip.call("xksv_pack_parallel", raw, rows, cols)
    assert oracle.unpack_parallel(block) == (0, raw)
    out = _dev_bytes(len(raw))
    assert hip.decode_parallel(block, out.data_ptr()) == 0
    assert _host(out, len(raw)) == raw
    # tests/test_cuda.py:62-65: a truncated block must fail on CPU and GPU
    assert hip.decode_parallel(block[:-1], out.data_ptr()) != 0
    assert oracle.unpack_parallel(block[:-1])[0] != 0


def test_golden_cases_both_codecs(hip, golden_cases):
    for case in golden_cases:
        raw = raw_bytes(gen(case["gen"]))
        rows, cols = case["rows"], case["cols"]
        out = _dev_bytes(len(raw))
        if case["serial"]["rc"] == 0:
            block = hip.call("xksv_pack", raw, rows, cols)
            assert sha(block) == case["serial"]["sha256"]
            assert hip.decode(block, rows, cols, out.data_ptr()) == 0, case["gen"]
            assert sha(_host(out, len(raw))) == case["raw_sha256"], case["gen"]
        if case["parallel"]["rc"] == 0:
            block = hip.call("xksv_pack_parallel", raw, rows, cols)
            assert sha(block) == case["parallel"]["sha256"]
            out.zero_()
            assert hip.decode_parallel(block, out.data_ptr()) == 0, case["gen"]
            assert sha(_host(out, len(raw))) == case["raw_sha256"], case["gen"]


def test_corruption_verdicts_match_reference(hip, corruption_matrix):
    """A corrupted block fails on the GPU exactly when the reference's unpack fails,
    and decodes to the reference's output (SHA-256) when it succeeds."""
    checked = 0
    for base in corruption_matrix:
        rows, cols = base["gen"]["shape"]
        raw = raw_bytes(gen(base["gen"]))
        blob = hip.call("xksv_pack_parallel" if base["parallel"] else "xksv_pack", raw, rows, cols)
        assert sha(blob) == base["blob_sha256"]
        out = _dev_bytes(len(raw))
        for r in base["results"]:
            mb = apply_mutation(blob, r["mut"])
            if base["parallel"]:
                rc = hip.decode_parallel(mb, out.data_ptr())
                rc2, host = hip.try_unpack_parallel(mb)
            else:
                rc = hip.decode(mb, rows, cols, out.data_ptr())
                rc2, host = hip.try_call("xksv_unpack", mb, rows, cols)
            assert (rc == 0) == (r["rc"] == 0), (base["gen"], base["parallel"], r["mut"])
            assert (rc2 == 0) == (r["rc"] == 0), (base["gen"], base["parallel"], r["mut"])
            if r["rc"] == 0:
                assert sha(_host(out, len(raw))) == r["sha256"], r["mut"]
                assert sha(host) == r["sha256"], r["mut"]
            checked += 1
    assert checked == 587


def test_unpack_entry_points_decode_on_gpu(hip, golden_cases):
    for case in golden_cases[:20]:
        raw = raw_bytes(gen(case["gen"]))
        rows, cols = case["rows"], case["cols"]
        blob = hip.call("xksv_pack", raw, rows, cols)
        assert hip.call("xksv_unpack", blob, rows, cols) == raw
        if case["parallel"]["rc"] == 0:
            assert hip.unpack_parallel(hip.call("xksv_pack_parallel", raw, rows, cols)) == raw


@pytest.mark.parametrize("maxlen", [33, 40, 64])
def test_codes_longer_than_32_bits(hip, oracle, maxlen):
    """Lengths tables with codes of up to `maxlen` bits take the bit-serial path."""
    rng = np.random.default_rng(maxlen)
    lens = long_code_lengths(maxlen)
    syms = [s for s in range(256) if lens[s]]
    n = 16 * 40
    probs = np.array([2.0 ** -lens[s] for s in syms])
    pick = rng.choice(len(syms), size=n, p=probs / probs.sum())
    pick[:3] = [len(syms) - 1, len(syms) - 2, len(syms) - 3]  # force the longest codes in
    symbols = [syms[i] for i in pick]
    sm = rng.integers(0, 256, n)
    block = craft_segment(lens, symbols, sm)
    rc, want = oracle.unpack(block, 16, 40)
    assert rc == 0
    out = _dev_bytes(2 * n)
    assert hip.decode(block, 16, 40, out.data_ptr()) == 0
    assert _host(out, 2 * n) == want
    # invalid: flip the last code bit region so the stream runs out
    bad = block[:-1] + bytes([block[-1] ^ 0x01])
    assert (hip.decode(bad, 16, 40, out.data_ptr()) == 0) == (oracle.unpack(bad, 16, 40)[0] == 0)


def test_long_codes_in_one_parallel_substream(hip, oracle):
    """An XKSP2 block whose substream 3 uses 40-bit codes and the rest ordinary codes."""
    rows, cols = 16, 64
    w = gen({"kind": "normal", "seed": 99, "shape": [rows, cols]})
    blob = bytearray(hip.call("xksv_pack_parallel", raw_bytes(w), rows, cols))
    chunks = int.from_bytes(blob[24:32], "little")
    lens_hdr = [int.from_bytes(blob[32 + 8 * i:40 + 8 * i], "little") for i in range(chunks)]
    segs, pos = [], 32 + 8 * chunks
    for L in lens_hdr:
        segs.append(bytes(blob[pos:pos + L]))
        pos += L
    rng = np.random.default_rng(5)
    lens = long_code_lengths(40)
    syms = [s for s in range(256) if lens[s]]
    n3 = int.from_bytes(segs[3][:8], "little")
    symbols = [syms[-1]] + [syms[int(i)] for i in rng.integers(0, 6, n3 - 1)]
    segs[3] = craft_segment(lens, symbols, rng.integers(0, 256, n3))
    new = bytes(blob[:32]) + b"".join(len(s).to_bytes(8, "little") for s in segs) + b"".join(segs)
    rc, want = oracle.unpack_parallel(new)
    assert rc == 0
    out = _dev_bytes(len(want))
    assert hip.decode_parallel(new, out.data_ptr()) == 0
    assert _host(out, len(want)) == want


def test_nonstandard_chunk_counts(hip, oracle):
    """The reference accepts any chunk count <= 32 (src/c_api.cpp:70); re-split a block into 5 and 7."""
    from oracle_lib import Oracle  # noqa: F401
    rows, cols = 16, 96
    w = gen({"kind": "normal", "seed": 7, "shape": [rows, cols]})
    tiled = oracle.tile(w, rows, cols)
    for chunks in (1, 5, 7, 31):
        n = rows * cols
        segs = []
        for i in range(chunks):
            a, b = n * i // chunks, n * (i + 1) // chunks
            part = tiled[a:b]
            seg = hip.call("xksv_pack", raw_bytes(part), 1, b - a)
            segs.append(seg)
        blob = (b"XKSP2\0\0\0" + rows.to_bytes(8, "little") + cols.to_bytes(8, "little") +
                chunks.to_bytes(8, "little") + b"".join(len(s).to_bytes(8, "little") for s in segs) + b"".join(segs))
        rc, want = oracle.unpack_parallel(blob)
        assert rc == 0 and want == raw_bytes(w)
        out = _dev_bytes(len(want))
        assert hip.decode_parallel(blob, out.data_ptr()) == 0, chunks
        assert _host(out, len(want)) == want, chunks

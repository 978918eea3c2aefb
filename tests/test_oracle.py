"""Pin the CPU oracle before trusting it (CPU only).

The oracle (oracle/xksv_oracle.c) must reproduce the reference codec byte for
byte.  It is checked against:
  * golden vectors written by the compiled reference (tests/golden/*.json):
    encoded bytes/digests for 37 cases, per-slab digests of a 4096x4096
    N(0, 0.02) matrix under both codecs, and the reference's verdict on 587
    corrupted blocks;
  * closed forms the mathematics fixes: the exhaustive 65,536-pattern round
    trip (tests/test_core.cpp:12-13), Kraft equality of Huffman lengths, the
    RFC 1951 canonical assignment, and an independent numpy tiling;
  * the compiled reference itself (oracle/_ref) on fresh random inputs, when
    that library is present.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

from conftest import GOLDEN
from oracle_lib import REF_SO, Reference, apply_mutation, gen, raw_bytes, sha


def test_golden_cases_encode_byte_identical(oracle, golden_cases):
    for case in golden_cases:
        w = gen(case["gen"])
        raw = raw_bytes(w)
        assert sha(raw) == case["raw_sha256"], case["gen"]  # generator drift
        rows, cols = case["rows"], case["cols"]
        for codec, pack in (("serial", oracle.pack), ("parallel", oracle.pack_parallel)):
            want = case[codec]
            rc, blob = pack(raw, rows, cols)
            assert rc == want["rc"], (codec, case["gen"])
            if rc:
                continue
            assert len(blob) == want["size"] and sha(blob) == want["sha256"], (codec, case["gen"])
            if "hex" in want:
                assert blob.hex() == want["hex"]


def test_golden_cases_decode(oracle, golden_cases):
    for case in golden_cases:
        raw = raw_bytes(gen(case["gen"]))
        rows, cols = case["rows"], case["cols"]
        if case["serial"]["rc"] == 0:
            blob = bytes.fromhex(case["serial"]["hex"]) if "hex" in case["serial"] else oracle.pack(raw, rows, cols)[1]
            rc, out = oracle.unpack(blob, rows, cols)
            assert rc == 0 and out == raw
        if case["parallel"]["rc"] == 0:
            p = case["parallel"]
            blob = bytes.fromhex(p["hex"]) if "hex" in p else oracle.pack_parallel(raw, rows, cols)[1]
            rc, out = oracle.unpack_parallel(blob)
            assert rc == 0 and out == raw


def test_golden_lengths_tables(oracle, golden_cases):
    for case in golden_cases:
        s = case["serial"]
        if s["rc"]:
            continue
        raw = raw_bytes(gen(case["gen"]))
        _, blob = oracle.pack(raw, case["rows"], case["cols"])
        assert blob[16:272].hex() == s["lengths"][0]


def test_per_slab_digests_4096x4096(oracle):
    slabs = json.loads((GOLDEN / "slabs_4096x4096_seed0.json").read_text())
    w = gen(slabs["gen"])
    assert sha(raw_bytes(w)) == slabs["raw_sha256"]
    for s in range(256):
        raw = raw_bytes(w[16 * s:16 * s + 16])
        assert sha(raw) == slabs["raw"][s]
        rc, blob = oracle.pack(raw, 16, 4096)
        assert rc == 0 and [len(blob), sha(blob)] == slabs["serial"][s], s
        rc, pblob = oracle.pack_parallel(raw, 16, 4096)
        assert rc == 0 and [len(pblob), sha(pblob)] == slabs["parallel"][s], s
        if s % 64 == 0:
            assert oracle.unpack(blob, 16, 4096) == (0, raw)
            assert oracle.unpack_parallel(pblob) == (0, raw)


def test_corruption_verdicts_match_reference(oracle, corruption_matrix):
    """Success/failure and output digest on every corrupted block equal the reference's."""
    for base in corruption_matrix:
        rows, cols = base["gen"]["shape"]
        raw = raw_bytes(gen(base["gen"]))
        rc, blob = (oracle.pack_parallel if base["parallel"] else oracle.pack)(raw, rows, cols)
        assert rc == 0 and sha(blob) == base["blob_sha256"]
        for r in base["results"]:
            mb = apply_mutation(blob, r["mut"])
            rc, out = oracle.unpack_parallel(mb) if base["parallel"] else oracle.unpack(mb, rows, cols)
            assert rc == r["rc"], r["mut"]
            if rc == 0:
                assert sha(out) == r["sha256"], r["mut"]


def test_exhaustive_round_trip(oracle):
    """tests/test_core.cpp:12-15: all 65,536 BF16 patterns and shuffled prefixes round-trip."""
    allw = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    rng = np.random.default_rng(12345)
    perm = allw.copy()
    rng.shuffle(perm)
    for words in [allw] + [perm[:n] for n in (1, 2, 255, 4096, 65536)]:
        raw = raw_bytes(words)
        for pack, unpack in ((oracle.pack, lambda b: oracle.unpack(b, 1, len(words))),
                             (oracle.pack_parallel, oracle.unpack_parallel)):
            rc, blob = pack(raw, 1, len(words))
            assert rc == 0
            assert unpack(blob) == (0, raw)


def _kraft(lengths: bytes) -> float:
    return sum(2.0 ** -l for l in lengths if l)


def _canonical_rfc1951(lengths: bytes) -> dict:
    """RFC 1951 3.2.2: bl_count, next_code, then codes in symbol order."""
    maxlen = max(lengths)
    bl = [0] * (maxlen + 1)
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


def _decode_with(codes: dict, stream: bytes, nbits: int, n: int) -> list:
    inv = {v: k for k, v in codes.items()}
    bits = "".join(format(b, "08b") for b in stream)[:nbits]
    out, cur = [], ""
    for ch in bits:
        cur += ch
        if cur in inv:
            out.append(inv[cur])
            cur = ""
    assert cur == "" and len(out) == n
    return out


@pytest.mark.parametrize("gen_spec", [
    {"kind": "normal", "seed": 3, "shape": [16, 256]},
    {"kind": "student_t", "seed": 4, "shape": [16, 256]},
    {"kind": "uniform16", "seed": 5, "shape": [4, 64]},
    {"kind": "exponent_pattern", "seed": 6, "shape": [8, 32]},
])
def test_huffman_lengths_and_canonical_codes(oracle, gen_spec):
    """Kraft sum of a Huffman code over >=2 symbols is exactly 1; codes are RFC 1951 canonical,
    and the serial stream is exactly the concatenation of those codes in tiled order."""
    w = gen(gen_spec)
    rows, cols = gen_spec["shape"]
    rc, blob = oracle.pack(raw_bytes(w), rows, cols)
    assert rc == 0
    count, nbits = int.from_bytes(blob[:8], "little"), int.from_bytes(blob[8:16], "little")
    lengths = blob[16:272]
    assert count == rows * cols
    assert abs(_kraft(lengths) - 1.0) < 1e-12
    tiled = oracle.tile(w, rows, cols)
    exps = (tiled >> 7) & 255
    hist = np.bincount(exps, minlength=256)
    assert all((hist[s] > 0) == (lengths[s] > 0) for s in range(256))
    # Huffman optimality sanity: expected length within 1 bit of the entropy.
    p = hist[hist > 0] / hist.sum()
    avg = sum(hist[s] * lengths[s] for s in range(256)) / hist.sum()
    ent = -(p * np.log2(p)).sum()
    assert ent <= avg < ent + 1
    codes = _canonical_rfc1951(lengths)
    assert nbits == sum(len(codes[e]) for e in exps)
    assert _decode_with(codes, blob[272 + count:], nbits, count) == list(exps)
    sm = np.frombuffer(blob[272:272 + count], np.uint8)
    assert np.array_equal(sm, (((tiled >> 8) & 128) | (tiled & 127)).astype(np.uint8))


def test_single_symbol_block(oracle):
    """tests/test_core.cpp:16-17: one symbol gets a 1-bit code; dropping a bit must fail."""
    w = np.full(1000, 0x8000, np.uint16)
    rc, blob = oracle.pack(raw_bytes(w), 1, 1000)
    assert rc == 0
    assert blob[16 + 0] == 1 and sum(1 for b in blob[16:272] if b) == 1
    assert oracle.unpack(blob, 1, 1000) == (0, raw_bytes(w))
    bad = bytearray(blob)
    bad[8:16] = (int.from_bytes(blob[8:16], "little") - 1).to_bytes(8, "little")
    assert oracle.unpack(bytes(bad), 1, 1000)[0] != 0


def _np_tile(w, rows, cols, tr, tc):
    out = []
    for r in range(0, rows, tr):
        for c in range(0, cols, tc):
            out.append(w[r:r + tr, c:c + tc].reshape(-1))
    return np.concatenate(out) if out else np.zeros(0, np.uint16)


def test_tile_untile(oracle):
    """tests/test_core.cpp:18 shapes with 8x16 tiles, against an independent numpy tiling."""
    for rows in (0, 1, 7, 32, 33):
        for cols in (0, 1, 9, 32, 35):
            w = np.arange(rows * cols, dtype=np.uint16).reshape(rows, cols)
            t = oracle.tile(w, rows, cols, 8, 16) if rows * cols else np.zeros(0, np.uint16)
            assert np.array_equal(t, _np_tile(w, rows, cols, 8, 16))
            if rows * cols:
                assert np.array_equal(oracle.tile(t, rows, cols, 8, 16, inverse=True), w.reshape(-1))
    w = np.arange(17 * 33, dtype=np.uint16).reshape(17, 33)
    assert np.array_equal(oracle.tile(w, 17, 33), _np_tile(w, 17, 33, 16, 16))


def test_gemm_f64_against_numpy(oracle, rng):
    w = gen({"kind": "normal", "seed": 9, "shape": [17, 33]})
    x = rng.standard_normal((33, 4))
    from xksv_synth import bf16_to_f32
    want = bf16_to_f32(w).astype(np.float64) @ x
    np.testing.assert_allclose(oracle.gemm_f64(w, x), want, rtol=1e-12, atol=1e-12)


def test_parallel_validation_rules(oracle):
    """src/c_api.cpp:44-46,66-70: rows > 16 cannot be packed; chunk count bounds are enforced."""
    raw = raw_bytes(gen({"kind": "normal", "seed": 1, "shape": [17, 8]}))
    assert oracle.pack_parallel(raw, 17, 8)[0] != 0
    assert oracle.pack_parallel(raw, 0, 8)[0] != 0
    assert oracle.pack_parallel(raw[:-1], 17, 8)[0] != 0
    assert oracle.pack(raw, 17, 8)[0] == 0
    assert oracle.pack(raw, 16, 8)[0] != 0  # rows*cols != n/2


@pytest.mark.skipif(not REF_SO.exists(), reason="oracle/_ref not built (reference sources absent)")
def test_oracle_matches_compiled_reference_random(oracle):
    """Fresh random shapes and distributions: oracle bytes == reference bytes."""
    ref = Reference()
    rng = np.random.default_rng(77)
    for i in range(60):
        rows = int(rng.integers(1, 40))
        cols = int(rng.integers(1, 300))
        kind = ["normal", "student_t", "uniform16", "exponent_pattern", "uniform"][i % 5]
        spec = {"kind": kind, "seed": 500 + i, "shape": [rows, cols]}
        raw = raw_bytes(gen(spec))
        assert oracle.pack(raw, rows, cols) == ref.pack(raw, rows, cols), spec
        if rows <= 16:
            assert oracle.pack_parallel(raw, rows, cols) == ref.pack_parallel(raw, rows, cols), spec


@pytest.mark.parametrize("plant", [1, 2])
def test_golden_vectors_reject_planted_mistakes(tmp_path, golden_cases, plant):
    """Build the oracle with a deliberately wrong tie-break (1) or canonical order (2):
    the golden vectors must catch it."""
    import shutil
    import subprocess
    from conftest import ROOT
    from oracle_lib import Oracle
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    so = tmp_path / f"liboracle_plant{plant}.so"
    subprocess.run(["gcc", "-std=c11", "-O2", "-shared", "-fPIC", f"-DORACLE_PLANTED_MISTAKE={plant}",
                    "-o", str(so), str(ROOT / "oracle" / "xksv_oracle.c")], check=True)
    bad = Oracle(so)
    mismatches = 0
    for case in golden_cases:
        if case["serial"]["rc"]:
            continue
        rc, blob = bad.pack(raw_bytes(gen(case["gen"])), case["rows"], case["cols"])
        if rc or sha(blob) != case["serial"]["sha256"]:
            mismatches += 1
    assert mismatches > 0

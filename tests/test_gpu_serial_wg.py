"""Serial-codec blocks decoded by a workgroup each (GPU only).

Twelve waves share a block: each decodes its share of the code bits from a
speculative entry, the ranges' starts are proven in order, and the symbols are
placed at the prefix of the counts; short, bit-serial or overflowing streams
are decoded by one wave.  Every case is checked against the oracle's CPU
decode: same verdict, and the same bytes when the block decodes.

* shapes on both sides of the split threshold (768 code bits), unit-aligned
  16-row slabs and ragged ones (element-wise placement);
* a stream whose first bits hold far more codewords than a range's share of
  the scratch (the one-wave fallback);
* bit flips in the code bits of the first, a middle and the last range, and in
  the last byte;
* several blocks of both kinds through one plan.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import xksv_hip
import xksv_synth as syn
from oracle_lib import raw_bytes

pytestmark = pytest.mark.gpu


def _pack(hip, w):
    rows, cols = w.shape
    return hip.call("xksv_pack", raw_bytes(w), rows, cols)


def _skewed(rows, cols, seed):
    """First half of the tiled order one value (1-bit codes), the rest random words (long codes)."""
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 1 << 16, size=(rows, cols), dtype=np.uint16)
    w[:, : cols // 2] = 0x3F80
    return w


@pytest.mark.parametrize("shape", [(16, 4096), (64, 4096), (16, 64), (16, 48), (33, 129), (7, 19), (128, 96)])
def test_serial_blocks_match_oracle(hip, oracle, shape):
    w = syn.normal_bf16(4000 + shape[0] + shape[1], shape)
    blob = _pack(hip, w)
    rc, out = hip.try_call("xksv_unpack", blob, *shape)
    assert rc == 0 and out == raw_bytes(w) == oracle.unpack(blob, *shape)[1]


def test_overflowing_ranges_fall_back_to_one_wave(hip, oracle):
    w = _skewed(16, 4096, 7)
    blob = _pack(hip, w)
    rc, out = hip.try_call("xksv_unpack", blob, 16, 4096)
    assert rc == 0 and out == raw_bytes(w)


@pytest.mark.parametrize("where", [0.01, 0.3, 0.55, 0.97, 1.0])
def test_corrupt_code_bits_same_verdict(hip, oracle, where):
    rows, cols = 16, 4096
    w = syn.normal_bf16(4242, (rows, cols))
    blob = bytearray(_pack(hip, w))
    code0 = 272 + rows * cols
    for bit in range(8):
        bad = bytearray(blob)
        at = min(len(bad) - 1, code0 + int(where * (len(bad) - code0)))
        bad[at] ^= 1 << bit
        want_rc, want = oracle.unpack(bytes(bad), rows, cols)
        rc, out = hip.try_call("xksv_unpack", bytes(bad), rows, cols)
        assert (rc == 0) == (want_rc == 0), (where, bit)
        if rc == 0:
            assert out == want, (where, bit)


def test_serial_blocks_through_one_plan(hip, oracle):
    shapes = [(16, 4096)] * 6 + [(64, 4096), (16, 64), (33, 129)]
    mats = [syn.normal_bf16(5000 + i, s) for i, s in enumerate(shapes)] + [_skewed(16, 4096, 3)]
    shapes = shapes + [(16, 4096)]
    blobs = [_pack(hip, m) for m in mats]
    table = np.zeros(len(blobs), xksv_hip.BLOCK_DTYPE)
    off = out = 0
    for i, (b, (r, c)) in enumerate(zip(blobs, shapes)):
        table[i] = (off, len(b), r * c * 2, out, r, c, xksv_hip.CODEC_SERIAL, 0)
        off += len(b)
        out += r * c * 2
    arc = torch.from_numpy(np.frombuffer(b"".join(blobs), np.uint8).copy()).to("cuda")
    dst = torch.zeros(out, dtype=torch.uint8, device="cuda")
    plan = xksv_hip.Plan(hip, table, arc.numel())
    try:
        plan.decode(arc.data_ptr(), dst.data_ptr(), out)
        assert plan.errors()[0] == 0
        assert dst.cpu().numpy().tobytes() == b"".join(raw_bytes(m) for m in mats)
    finally:
        plan.close()

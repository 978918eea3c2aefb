"""Autotuner size rules (CPU): python/tune.py:21-23 -- raw when neither codec
is smaller than the raw bytes, the only smaller codec otherwise, serial when
parallel32 is more than 15 % larger; otherwise a measured choice per bucket."""
from __future__ import annotations

import xksv_tune as t


def test_size_rule_branches():
    raw = bytes(1000)
    assert t.size_rule(bytes(1000), bytes(1200), raw) == t.RAW
    assert t.size_rule(bytes(1001), bytes(900), raw) == t.PARALLEL
    assert t.size_rule(bytes(800), bytes(1000), raw) == t.SERIAL  # parallel not smaller than raw
    assert t.size_rule(bytes(800), bytes(921), raw) == t.SERIAL   # 921 > 1.15 * 800
    assert t.size_rule(bytes(800), bytes(920), raw) is None       # exactly 15 % larger: measured
    assert t.size_rule(bytes(800), bytes(700), raw) is None


def test_bucket_key():
    assert t.bucket(bytes(700), bytes(1000), 16, 4096) == "16:4096:11"
    assert t.bucket(bytes(1000), bytes(1000), 3, 5) == "3:5:16"

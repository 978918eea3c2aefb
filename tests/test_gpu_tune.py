"""GPU autotuner (GPU only), mirroring tests/test_autotune.py:13-17: a 16x4096
slab of three exponent values records a measured serial-vs-parallel32 choice,
and the chosen bytes decode back to the source exactly."""
from __future__ import annotations

import random
import struct

import pytest

import xksv_tune

pytestmark = pytest.mark.gpu


def test_tuner_records_measured_choice(hip):
    rng = random.Random(123)
    words = [((127 + i % 3) << 7) | rng.randrange(128) for i in range(16 * 4096)]
    raw = struct.pack("<%dH" % len(words), *words)
    serial = hip.call("xksv_pack", raw, 16, 4096)
    parallel = hip.call("xksv_pack_parallel", raw, 16, 4096)
    assert xksv_tune.size_rule(serial, parallel, raw) is None  # this slab is measured
    tuner = xksv_tune.GpuTuner(lib=hip)
    codec, data = tuner.select(serial, parallel, raw, 16, 4096)
    assert codec in (xksv_tune.SERIAL, xksv_tune.PARALLEL)
    key = xksv_tune.bucket(serial, raw, 16, 4096)
    choice = tuner.profile["choices"][key]
    assert choice["serial_seconds"] > 0 and choice["parallel_seconds"] > 0
    assert choice["prefer_parallel"] == (codec == xksv_tune.PARALLEL)
    back = hip.call("xksv_unpack", data, 16, 4096) if codec == xksv_tune.SERIAL else hip.unpack_parallel(data)
    assert back == raw
    # resuming with the profile reuses the measurement
    again = xksv_tune.GpuTuner(profile=tuner.profile, lib=hip)
    assert again.select(serial, parallel, raw, 16, 4096)[0] == codec
    assert again.profile["choices"][key] is choice
    with pytest.raises(ValueError):
        xksv_tune.GpuTuner(profile={"device": {"name": "other"}, "choices": {}}, lib=hip)

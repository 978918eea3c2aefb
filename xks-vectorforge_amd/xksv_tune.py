"""GPU block-decoder autotuning: serial vs parallel32 per slab bucket.

Mirrors the reference's conservative tuner (python/tune.py:20-42,
`GpuTuner.select`): raw when neither codec is smaller than the raw bytes;
otherwise the only smaller codec; otherwise serial when parallel32 is more
than 15 % larger (python/tune.py:23); otherwise the median of three timed GPU
decodes of each encoding, after a warmup, decides -- once per bucket
`rows:cols:16*serial/raw`, so similar slabs share one measurement.  The
profile dict has the reference's layout ({device, method, choices}) and can
be resumed on the same GPU.

Decodes run through this library's block entries (xksv_hip_decode /
xksv_hip_decode_parallel, host bytes in, device bytes out), the calls the
reference times through xksv_cuda_*.
"""
from __future__ import annotations

import statistics
import time

import xksv_hip

SERIAL = "bf16-huffman-tile16"
PARALLEL = "bf16-huffman-parallel32"
RAW = "raw"


def size_rule(serial: bytes, parallel: bytes, raw: bytes) -> str | None:
    """The size-only part of the choice (python/tune.py:21-23); None = measure."""
    if len(serial) >= len(raw) and len(parallel) >= len(raw):
        return RAW
    if len(serial) >= len(raw):
        return PARALLEL
    if len(parallel) >= len(raw) or len(parallel) * 100 > len(serial) * 115:
        return SERIAL
    return None


def bucket(serial: bytes, raw: bytes, rows: int, cols: int) -> str:
    return f"{rows}:{cols}:{len(serial) * 16 // len(raw)}"


class GpuTuner:
    def __init__(self, profile: dict | None = None, lib: xksv_hip.Library | None = None):
        import torch
        if not torch.cuda.is_available():
            raise ValueError("autotuning requires a GPU")
        self.torch = torch
        self.device = torch.cuda.current_device()
        props = torch.cuda.get_device_properties(self.device)
        identity = {"name": props.name, "gcn_arch": getattr(props, "gcnArchName", ""),
                    "compute_units": props.multi_processor_count}
        if profile is not None and profile.get("device") != identity:
            raise ValueError("resume GPU differs from the autotuning GPU")
        self.profile = profile if profile is not None else {
            "device": identity,
            "method": "median of three GPU block-decode wall times after warmup; parallel limited to 15% larger "
                      "than serial",
            "choices": {}}
        self.lib = lib or xksv_hip.Library()

    def _time(self, fn) -> float:
        fn()
        self.torch.cuda.synchronize(self.device)
        samples = []
        for _ in range(3):
            begin = time.perf_counter()
            fn()
            self.torch.cuda.synchronize(self.device)
            samples.append(time.perf_counter() - begin)
        return statistics.median(samples)

    def select(self, serial: bytes, parallel: bytes, raw: bytes, rows: int, cols: int):
        """(codec name, encoded bytes) for one slab."""
        rule = size_rule(serial, parallel, raw)
        if rule is not None:
            return rule, {RAW: raw, SERIAL: serial, PARALLEL: parallel}[rule]
        key = bucket(serial, raw, rows, cols)
        choice = self.profile["choices"].get(key)
        if choice is None:
            out = self.torch.empty(len(raw), device=f"cuda:{self.device}", dtype=self.torch.uint8)

            def run_serial():
                if self.lib.decode(serial, rows, cols, out.data_ptr()):
                    raise ValueError("GPU autotuning decode failed")

            def run_parallel():
                if self.lib.decode_parallel(parallel, out.data_ptr()):
                    raise ValueError("GPU autotuning decode failed")

            ts, tp = self._time(run_serial), self._time(run_parallel)
            choice = {"serial_seconds": ts, "parallel_seconds": tp, "prefer_parallel": tp < ts}
            self.profile["choices"][key] = choice
        return (PARALLEL, parallel) if choice["prefer_parallel"] else (SERIAL, serial)

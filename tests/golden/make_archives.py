"""Writes tests/golden/tiny_serial.xksv and tiny_parallel.xksv with the reference's own
archive compiler (oracle/_ref/xksv-native, built from the reference's sources by
`make -C oracle ref`) from the checkpoint of tests/tiny_checkpoint.py, and checks
them with the same binary's verifier.

    python tests/golden/make_archives.py
"""
from __future__ import annotations

import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(HERE.parent))
import tiny_checkpoint  # noqa: E402

EXE = ROOT / "oracle" / "_ref" / "xksv-native"


def main() -> int:
    if not EXE.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "ref"], check=True)
    with tempfile.TemporaryDirectory() as tmp:
        src = tiny_checkpoint.write(Path(tmp) / "ckpt")
        for codec, name in (("dfloat11", "tiny_serial.xksv"), ("dfloat11-parallel", "tiny_parallel.xksv")):
            out = Path(tmp) / name
            subprocess.run([str(EXE), "compile", str(src), "--output", str(out), "--codec", codec, "--workers", "2"],
                           check=True, capture_output=True)
            subprocess.run([str(EXE), "verify", str(out), "--source", str(src)], check=True, capture_output=True)
            (HERE / name).write_bytes(out.read_bytes())
            print(f"{name}: {out.stat().st_size} bytes")
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Builds libkanso_hip.so (gfx950) in-tree, and the CPU oracle used by the tests.

    python -m kanso_infer_amd.build            # HIP library + oracle
    python -m kanso_infer_amd.build --hip-only

The HIP sources are compiled with hipcc for gfx950 only. Flags that matter:
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed FP32 (v_pk_*_f32) code
  -fhip-fp32-correctly-rounded-divide-sqrt           IEEE division: the KV quantizers
                                                     must round like the Rust source
  -fno-gpu-flush-denormals-to-zero                   keep f32 denormals (quantizer parity)
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libkanso_hip.so"
ORACLE_DIR = ROOT / "oracle"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Wall",
    "-Wno-unused-function",
]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}")
    # hipcc's host pass warns about the device-only target feature; keep other output
    noise = "is not a recognized feature for this target"
    for line in (proc.stdout + proc.stderr).splitlines():
        if line.strip() and noise not in line and "(ignoring feature)" not in line:
            sys.stderr.write(line + "\n")


def build_hip(jobs: int = 8, incremental: bool = False) -> Path:
    """Compiles every HIP source (incremental: only those whose object is older than
    the source or any header) and links the library."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    headers = [*CSRC.glob("*.hpp"), *(ROOT / "include").glob("*.h")]
    newest_header = max((h.stat().st_mtime for h in headers), default=0.0)

    def compile_one(src: Path) -> Path:
        obj = BUILD / (src.stem + ".o")
        if incremental and obj.exists() and obj.stat().st_mtime > max(src.stat().st_mtime, newest_header):
            return obj
        _run([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
        return obj

    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, sources))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> Path:
    make = shutil.which("make")
    if make is None:
        raise RuntimeError("make not found")
    _run([make, "-C", str(ORACLE_DIR), "-s"])
    return ORACLE_DIR / "libkanso_oracle.so"


def main(argv: list[str] | None = None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--hip-only", action="store_true")
    ap.add_argument("--oracle-only", action="store_true")
    ap.add_argument("-j", type=int, default=8)
    ap.add_argument("--incremental", action="store_true",
                    help="recompile only sources older than their object (or a header)")
    args = ap.parse_args(argv)
    if not args.oracle_only:
        print(build_hip(args.j, args.incremental))
    if not args.hip_only:
        print(build_oracle())


if __name__ == "__main__":
    main()

"""Build the HIP libecpu for gfx950: pilm_amd/lib/libecpu.so.

    python -m pilm_amd.build            # compile (always) and link
    python -m pilm_amd.build --asm      # also write the gfx950 assembly to _build/

Every .hip file in pilm_amd/csrc is compiled with hipcc for gfx950 only.
Packed fp32 instructions are disabled for all device code.
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
CSRC = PKG / "csrc"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libecpu.so"
OBJ_DIR = PKG / "_build"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc" if Path("/opt/rocm/bin/hipcc").exists() else "hipcc")

DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
COMMON_FLAGS = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function", f"-I{PKG.parent / 'include'}"]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, asm: bool) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *DEVICE_FLAGS, "-c", str(src), "-o", str(obj)]
    subprocess.run(cmd, check=True)
    if asm:
        out = OBJ_DIR / (src.stem + f"-{ARCH}.s")
        subprocess.run([HIPCC, *COMMON_FLAGS, *DEVICE_FLAGS, "--offload-device-only", "-S", str(src),
                        "-o", str(out)], check=True)
    return obj


def build(asm: bool = False, jobs: int | None = None) -> Path:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found ({HIPCC}); the HIP library cannot be built")
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, asm), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    subprocess.run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)],
                   check=True)
    os.replace(tmp, LIB)
    return LIB


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--asm", action="store_true")
    args = ap.parse_args(argv)
    print(build(asm=args.asm))
    return 0


if __name__ == "__main__":
    sys.exit(main())

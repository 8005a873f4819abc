"""Build recipe for libllminfer_hip.so (the HIP backend behind include/llminfer_hip.h).

Compiles every source under llminfer_amd/csrc with hipcc for gfx950 and links
them into llminfer_amd/lib/libllminfer_hip.so, in-tree, so the library travels
with the repository snapshot. Objects go to _build/ (git-ignored).

    python -m llminfer_amd.build            # build (always recompiles)
    python -m llminfer_amd.build --jobs 4
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "llminfer_amd" / "csrc"
INCLUDE = ROOT / "include"
BUILD = ROOT / "_build" / "hip"
LIBDIR = ROOT / "llminfer_amd" / "lib"
LIBNAME = "libllminfer_hip.so"
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled for every device compile.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
          f"-I{INCLUDE}", f"-I{CSRC}", "-Wall", "-Wno-unused-function",
          "-fvisibility=hidden"]


# Per-file additions. norm_rope.hip, delta_front.hip, w8a8.hip and graph_ops.hip reproduce
# the reference's fp16 rounding points bit for bit, which needs every fp32 product rounded on its own: under
# the default -ffp-contract=fast the backend folds a product and the fp16
# conversion or add after it into one fused instruction.
FILE_FLAGS = {"norm_rope.hip": ["-ffp-contract=off"], "delta_front.hip": ["-ffp-contract=off"],
              "w8a8.hip": ["-ffp-contract=off"], "graph_ops.hip": ["-ffp-contract=off"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP backend cannot be built")


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *COMMON, *DEVICE_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src),
           "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{proc.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    LIBDIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, srcs))
    out = LIBDIR / LIBNAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", f"--offload-arch={ARCH}", "-o", str(tmp),
           *map(str, objs), "-Wl,--no-undefined", "-lpthread"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args(argv)
    build(args.jobs, verbose=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

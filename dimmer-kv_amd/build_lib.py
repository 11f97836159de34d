"""Build libdimmerkv_hip.so (gfx950) in-tree with hipcc.

    python dimmer-kv_amd/build_lib.py            # build
    python dimmer-kv_amd/build_lib.py --check    # print the exported symbols

Every HIP source is compiled with packed-FP32 code generation disabled
(``-Xclang -target-feature -Xclang -packed-fp32-ops``) and without fast-math,
so fp32 divisions stay correctly rounded and the dequantize kernel keeps the
reference's rounding order.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = ROOT / "include"
LIB = HERE / "libdimmerkv_hip.so"
SOURCES = ["dkv_pack.hip", "dkv_attend.hip"]
ARCH = os.environ.get("DKV_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


def flags() -> list[str]:
    return ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}", f"-I{CSRC}",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-result"]


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library (always rebuilds)."""
    build_dir = HERE / "_build"
    build_dir.mkdir(exist_ok=True)
    objects = []
    cc = hipcc()
    for src in SOURCES:
        obj = build_dir / (Path(src).stem + ".o")
        cmd = [cc, *flags(), "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr[-4000:]}")
        objects.append(str(obj))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", str(tmp), *objects]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB)
    return LIB


def exported_symbols(lib: Path = LIB) -> list[str]:
    res = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True)
    return sorted(line.split()[-1] for line in res.stdout.splitlines() if " T " in line and "dkv_" in line)


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("--check", action="store_true")
    parser.add_argument("-v", action="store_true")
    args = parser.parse_args()
    if args.check:
        print("\n".join(exported_symbols()))
        sys.exit(0)
    print(build(verbose=args.v))

"""Builds libqws.so (HIP, gfx950) in-tree: qwen-warp_amd/lib/libqws.so.

  python qwen-warp_amd/build.py

Flags: -ffp-contract=off (every floating-point operation one IEEE rounding, as the CPU definition),
no fast-math, packed fp32 instructions off (-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRC = [PKG / "csrc" / "qws_sample.hip", PKG / "csrc" / "qws_verify.hip", PKG / "csrc" / "qws_state.hip", PKG / "csrc" / "qws_pld.hip", PKG / "csrc" / "qws_head.hip",
       PKG / "csrc" / "qws_hooks.hip"]
OUT = PKG / "lib" / "libqws.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{ROOT / 'include'}"]


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, *map(str, SRC), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{errs}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

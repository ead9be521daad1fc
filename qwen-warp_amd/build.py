"""Builds libqws.so (HIP, gfx950) in-tree: qwen-warp_amd/lib/libqws.so.

  python qwen-warp_amd/build.py

Each source is compiled to an object in parallel (no device code crosses files: every kernel is launched from its own
file, the shared device helpers are inline), then the objects are linked.  Flags: -ffp-contract=off (every
floating-point operation one IEEE rounding, as the CPU definition), no fast-math, packed fp32 instructions off
(-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRC = [PKG / "csrc" / "qws_sample.hip", PKG / "csrc" / "qws_verify.hip", PKG / "csrc" / "qws_state.hip", PKG / "csrc" / "qws_pld.hip", PKG / "csrc" / "qws_head.hip",
       PKG / "csrc" / "qws_hooks.hip"]
OUT = PKG / "lib" / "libqws.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{ROOT / 'include'}"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}): {' '.join(map(str, cmd))}\n{errs}")


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="qws_build_") as td:
        objs = [Path(td) / (s.stem + ".o") for s in SRC]
        cmds = [[HIPCC, *FLAGS, "-c", str(s), "-o", str(o)] for s, o in zip(SRC, objs)]
        if verbose:
            for c in cmds:
                print(" ".join(c), flush=True)
        with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as ex:
            list(ex.map(_run, cmds))
        tmp = OUT.with_suffix(".so.tmp")
        _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
        os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

"""Build the MI355X library: hipcc for gfx950, in-tree.

Output: coding-basic-hw-2_amd/ggemm/libggemm_mi355x.so (objects in coding-basic-hw-2_amd/_build/).
Every source is compiled on each call (this is the "does it build" check).
Usage: python coding-basic-hw-2_amd/build_lib.py [-v]
"""
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
OUT = PKG / "ggemm" / "libggemm_mi355x.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
          f"-I{REPO / 'include'}", f"-I{CSRC}"]
# Device code: gfx950 only; no packed-FP32 instructions (v_pk_*_f32).
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wno-unused-command-line-argument"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(map(str, cmd)), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature: that warning is expected
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(map(str, cmd))}\n{err}")
    if err.strip() and verbose:
        print(err)


def build(verbose=False, jobs=None):
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    objs = []
    cmds = []
    for s in srcs:
        o = BUILD / (s.name + ".o")
        objs.append(o)
        lang = ["-x", "hip"] + DEVICE if s.suffix == ".hip" else ["-D__HIP_PLATFORM_AMD__"]
        cmds.append([HIPCC, *COMMON, *lang, "-c", str(s), "-o", str(o)])
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(cmds))) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    OUT.parent.mkdir(exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

"""Build ``libtree_attn.so`` (gfx950) and ``libtree_plan.so`` (host planner)
next to the ``tree_attention`` package.

    python tree-attention-scheduling_amd/csrc/build.py

Uses hipcc directly; no CMake, no JIT cache.  The library is placed in-tree so
it travels with the source snapshot to the GPU machine.  Each translation unit
has its own code-generation flags (see ``SOURCES``); the objects are linked
into one shared library.
"""
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent / "tree_attention"
INCLUDE = HERE.parent.parent / "include"
LIB = PKG / "libtree_attn.so"
PLAN_LIB = PKG / "libtree_plan.so"
# The planner's costs must round exactly like the Python planner's: no FMA
# contraction, no fast-math reassociation.
PLAN_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-Wall"]

COMMON = [
    "-O3", "-std=c++20", "--offload-arch=gfx950", "-fPIC",
    "-mcode-object-version=5",
    # packed-FP32 VALU forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
# (source, extra flags).  MFMA accumulators in VGPRs: every kernel fits in 256
# VGPRs, and with accumulators in AGPRs the allocator copied O between the two
# register files every step (the rescale multiplies O on the VALU).
# segment_tile.hip also builds with -fno-honor-nans: its row maxima then
# compile to v_max3_f32 chains without a canonicalising v_max per input; the
# kernel never produces NaN scores (masked tokens are selected to -inf).
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
SOURCES = [
    (HERE / "tree_attn.hip", VGPR_FORM),
    (HERE / "segment_tile.hip", VGPR_FORM + ["-fno-honor-nans"]),
    (HERE / "decode_append.hip", ["-ffp-contract=off"]),  # each RoPE product rounded, as the eager ops
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build the tree_attn library")
    return found


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{Path(cmd[0]).name} failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)


def build(verbose: bool = False, out: Path | None = None, defines=()) -> Path:
    """Compile every source and link ``out`` (default: the in-tree library)."""
    target = Path(out) if out is not None else LIB
    tmp = target.with_name(target.name + f".tmp{os.getpid()}")
    with tempfile.TemporaryDirectory() as work:
        objs = []
        for src, extra in SOURCES:
            obj = Path(work) / (src.stem + ".o")
            _run([hipcc(), *COMMON, *extra, *[f"-D{d}" for d in defines], f"-I{INCLUDE}", f"-I{HERE}",
                  "-c", str(src), "-o", str(obj)], verbose)
            objs.append(str(obj))
        _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", str(tmp)], verbose)
    os.replace(tmp, target)
    return target


def build_planner(verbose: bool = False, out: Path | None = None) -> Path:
    """Compile the host planner (planner.cpp) into ``out`` (default: in-tree) with g++."""
    target = Path(out) if out is not None else PLAN_LIB
    tmp = target.with_name(target.name + f".tmp{os.getpid()}")
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("g++ not found; it is required to build the planner library")
    _run([cxx, *PLAN_FLAGS, f"-I{INCLUDE}", str(HERE / "planner.cpp"), "-o", str(tmp)], verbose)
    os.replace(tmp, target)
    return target


if __name__ == "__main__":
    args = sys.argv[1:]
    out = None
    defines = []
    while args:
        a = args.pop(0)
        if a == "-o":
            out = Path(args.pop(0))
        elif a.startswith("-D"):
            defines.append(a[2:])
    print(build(verbose=True, out=out, defines=defines))
    if out is None:
        print(build_planner(verbose=True))

"""Build libezops_hip.so from csrc/ for gfx950 with hipcc (no JIT, no cmake).

Usage: python ez-ops_amd/build.py [-j N]
Objects go to ez-ops_amd/_build/, the library to ez-ops_amd/ezops/_lib/.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
BUILD = PKG_ROOT / "_build"
LIB = PKG_ROOT / "ezops" / "_lib" / "libezops_hip.so"
# The same sources with wave-level timeline recording compiled in (ezops.profiling).
PROF_LIB = PKG_ROOT / "ezops" / "_lib" / "libezops_hip_prof.so"
ARCH = "gfx950"

# Packed-fp32 VALU ops are disabled: hand-written or compiler-formed
# v_pk_*_f32 forms have been unreliable on the target machines.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src: Path, build_dir: Path = BUILD, extra: tuple = ()) -> Path:
    obj = build_dir / (src.name + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [hipcc(), "-O3", "-std=c++17", "-fPIC", "-Wall", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l).strip()
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{msg}")
    if msg:
        print(msg, file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = True, extra_flags: tuple = (), lib: Path = LIB,
          build_dir: Path = BUILD) -> Path:
    """Compile csrc/ into ``lib``; ``extra_flags`` (e.g. tile-size -D macros) go to every hipcc call."""
    build_dir.mkdir(parents=True, exist_ok=True)
    lib.parent.mkdir(parents=True, exist_ok=True)
    sources = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))
    jobs = jobs or min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, build_dir, tuple(extra_flags)), sources))
    tmp = lib.with_suffix(".so.tmp")
    rocm_lib = Path(hipcc()).resolve().parent.parent / "lib"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), f"-L{rocm_lib}",
           f"-Wl,-rpath,{rocm_lib}", "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, lib)  # atomic: a concurrent loader never sees a half-written file
    if verbose:
        print(f"built {lib} from {len(sources)} sources")
    return lib


KAT_SRC = PKG_ROOT.parent / "tests" / "kat_c_abi.cpp"
KAT_BIN = LIB.parent / "ezops_kat_c_abi"


def build_kat(verbose: bool = True) -> Path:
    """The C++ known-answer program of the C ABI (tests/kat_c_abi.cpp), linked
    against the in-tree library through an $ORIGIN rpath."""
    tmp = KAT_BIN.with_suffix(".tmp")
    cmd = [hipcc(), "-O2", "-std=c++17", str(KAT_SRC), f"-L{LIB.parent}", "-lezops_hip",
           "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"KAT build failed: {' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, KAT_BIN)
    if verbose:
        print(f"built {KAT_BIN}")
    return KAT_BIN


def build_all(jobs: int | None = None, verbose: bool = True) -> None:
    """The production library, its profiling variant and the C ABI KAT program."""
    build(jobs, verbose)
    build(jobs, verbose, extra_flags=("-DEZ_PROFILE=1",), lib=PROF_LIB, build_dir=BUILD / "prof")
    build_kat(verbose)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("-D", action="append", default=[], help="extra preprocessor definition (variant builds)")
    ap.add_argument("-o", type=Path, default=LIB, help="output library path")
    ap.add_argument("--all", action="store_true", help="also build the profiling variant (-DEZ_PROFILE=1)")
    args = ap.parse_args()
    if args.all:
        build_all(args.j)
        sys.exit(0)
    bdir = BUILD if args.o == LIB else args.o.parent / "_build"
    build(args.j, extra_flags=tuple(f"-D{d}" for d in args.D), lib=args.o, build_dir=bdir)

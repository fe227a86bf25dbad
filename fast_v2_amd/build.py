"""Build libfdllm_hip.so (gfx950 only) in-tree with hipcc.

    python -m fast_v2_amd.build              # compile if any source is newer
    python -m fast_v2_amd.build --force      # always compile
    python -m fast_v2_amd.build --timeline   # also the instrumented profiling build

The libraries land in fast_v2_amd/lib/ so they travel with the source tree:
libfdllm_hip.so (the operators), libfdllm_probes.so (the measurement probes bench.py
times the calls against) and, on request, libfdllm_hip_timeline.so.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libfdllm_hip.so"
# The same sources with FDLLM_TIMELINE: the split decode kernel also writes per-workgroup
# phase stamps (fast_v2_amd.timeline reads them). A profiling build, built on request and
# never loaded by default.
TIMELINE_LIB_PATH = LIB_DIR / "libfdllm_hip_timeline.so"
PROBES_LIB_PATH = LIB_DIR / "libfdllm_probes.so"
HEADER = REPO_DIR / "include" / "fdllm_hip.h"
PROBES_HEADER = REPO_DIR / "include" / "fdllm_probes.h"

SOURCES = [CSRC / "gather_rmsnorm.hip", CSRC / "block_attn.hip", CSRC / "rope_kv.hip", CSRC / "sampler.hip"]
DEPS = SOURCES + [CSRC / "fdllm_common.h", CSRC / "attn_plan.h", CSRC / "host_errors.h", HEADER]
PROBES_SOURCES = [CSRC / "probes.hip"]
PROBES_DEPS = PROBES_SOURCES + [PROBES_HEADER]

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-mcode-object-version=5",
    # Packed fp32 ops stay off: hipcc would otherwise form v_pk_{add,mul,fma}_f32.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Kernel-argument preloading: a kernel's leading scalar and pointer arguments (not
    # by-value structs) arrive in SGPRs at wave launch instead of by a load from the
    # argument segment, which takes one memory round trip off the front of the kernels
    # that lead with the pointers their first loads need (the gather went from 4.78 to
    # 4.40 us). Code objects keep the compatibility prologue that loads them the old way.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wno-unused-command-line-argument",
]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (looked at $HIPCC, PATH and /opt/rocm/bin/hipcc)")


def _stale(path: Path, deps) -> bool:
    if not path.exists():
        return True
    built = path.stat().st_mtime
    return any(p.stat().st_mtime > built for p in deps)


def needs_build(timeline: bool = False) -> bool:
    """True if the operator or probe library (and, with ``timeline``, the instrumented
    build) is missing or older than one of its sources."""
    return (_stale(LIB_PATH, DEPS) or _stale(PROBES_LIB_PATH, PROBES_DEPS)
            or (timeline and _stale(TIMELINE_LIB_PATH, DEPS)))


def build(force: bool = True, verbose: bool = False, timeline: bool = False) -> Path:
    """Compile every HIP source into the operator library and the probes library (and,
    with ``timeline``, the instrumented profiling build), concurrently; returns the path
    of the operator library."""
    if not force and not needs_build(timeline):
        return LIB_PATH
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    jobs = [(LIB_PATH, [], SOURCES), (PROBES_LIB_PATH, [], PROBES_SOURCES)]
    if timeline:
        jobs.append((TIMELINE_LIB_PATH, ["-DFDLLM_TIMELINE=1"], SOURCES))
    procs = []
    for path, extra, sources in jobs:
        tmp = path.with_suffix(f".so.tmp{os.getpid()}")
        cmd = [hipcc_path(), *HIPCC_FLAGS, *extra, "-I", str(REPO_DIR / "include"),
               *[str(s) for s in sources], "-o", str(tmp)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((path, tmp, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is expected.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    errors = []
    for path, tmp, proc in procs:
        _, err = proc.communicate()
        msgs = [l for l in (err or "").splitlines() if noise not in l]
        if proc.returncode != 0:
            tmp.unlink(missing_ok=True)
            errors.append(f"hipcc failed for {path.name}:\n" + "\n".join(msgs))
            continue
        if verbose and msgs:
            print("\n".join(msgs), file=sys.stderr)
        os.replace(tmp, path)
    if errors:
        raise RuntimeError("\n".join(errors))
    return LIB_PATH


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--force", action="store_true")
    ap.add_argument("--timeline", action="store_true", help="also build the instrumented profiling library")
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    path = build(force=args.force or needs_build(args.timeline), verbose=args.verbose, timeline=args.timeline)
    print(path)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

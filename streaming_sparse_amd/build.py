"""Build recipe for libssattn.so (gfx950) with hipcc; no JIT, built in-tree.

    python -m streaming_sparse_amd.build

Each source compiles to its own object (in parallel), then one link makes
the shared library.
"""
from __future__ import annotations

import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libssattn.so")
# measurement build: the same sources with the router's phase stamps and the
# attention kernel's step stamps compiled in
STAMPS_LIB = os.path.join(HERE, "libssattn_stamps.so")
SOURCES = ("attention.hip", "route.hip", "pset.hip", "summary.hip", "runtime.hip", "group.hip")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
         # packed fp32 VALU forms are excluded from code generation
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I", os.path.join(ROOT, "include")]
# Per-source flags.  The attention and router kernels test no value for NaN
# (their inputs are finite), so max/min of matrix-pipe results need no
# signalling-NaN quieting; pset.hip keeps IEEE NaN semantics (it tests scores
# for finiteness).
EXTRA = {"attention.hip": ["-fno-honor-nans"], "route.hip": ["-fno-honor-nans"]}
NOISE = "is not a recognized feature for this target"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


def _stderr(res) -> str:
    return "\n".join(line for line in res.stderr.splitlines() if NOISE not in line)


def build(verbose: bool = False, stamps: bool = False) -> str:
    """Compile and link the library; with stamps, the measurement build into
    libssattn_stamps.so instead: -DSSA_ROUTE_STAMPS (route_kernel records its
    phase boundaries, read by ssa_route_stamps and printed by
    streaming_sparse_amd.route_phases) and -DSSA_ATTN_STAMPS (attn_kernel
    records its steps, read by ssa_attn_stamps and printed by
    streaming_sparse_amd.attn_steps)."""
    cc = hipcc()
    target = STAMPS_LIB if stamps else LIB
    defs = ["-DSSA_ROUTE_STAMPS", "-DSSA_ATTN_STAMPS"] if stamps else []
    with tempfile.TemporaryDirectory(prefix="ssattn_build_") as tmpdir:
        objs, procs = [], []
        for src in SOURCES:
            obj = os.path.join(tmpdir, src.replace(".hip", ".o"))
            cmd = [cc, *FLAGS, *defs, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
            procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
            objs.append(obj)
        errs = []
        for cmd, proc in procs:
            out, err = proc.communicate()
            res = subprocess.CompletedProcess(cmd, proc.returncode, out, err)
            if res.returncode != 0:
                errs.append(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{_stderr(res)}")
            elif verbose and _stderr(res).strip():
                print(_stderr(res), file=sys.stderr)
        if errs:
            raise RuntimeError("\n".join(errs))
        tmp = target + ".tmp"
        cmd = [cc, "--offload-arch=gfx950", "-fPIC", "-shared", *objs, "-o", tmp]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed ({res.returncode}):\n{' '.join(cmd)}\n{_stderr(res)}")
    os.replace(tmp, target)
    return target


if __name__ == "__main__":
    print(build(verbose=True, stamps="--stamps" in sys.argv[1:]))

"""Build libqwfn_qsa.so (gfx950) in-tree with hipcc.

Run as ``python -m qwfnfer_amd.build``; ``__graft_entry__.build()`` calls
:func:`build`.  The library is written next to this file so it travels with the
source tree; nothing is installed.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libqwfn_qsa.so")
SOURCES = ["qsa_kernels.hip", "qsa_decode.hip", "qsa_decode_kv.hip", "qsa_idx.hip", "qsa_abi.hip"]
ARCH = "gfx950"

# -packed-fp32-ops off: v_pk_{add,mul,fma}_f32 are never emitted.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libqwfn_qsa.so)")


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)


def build(verbose: bool = False) -> str:
    """Compile the kernels and the C ABI into ``qwfnfer_amd/libqwfn_qsa.so``:
    one object per source, compiled in parallel, then one link."""
    from concurrent.futures import ThreadPoolExecutor

    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    objs = [os.path.join(CSRC, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    with ThreadPoolExecutor(len(srcs)) as ex:
        list(ex.map(lambda so: _run([hipcc(), *compile_flags, "-c", "-o", so[1], so[0]], verbose),
                    zip(srcs, objs)))
    tmp = LIB + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    for o in objs:
        os.remove(o)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))

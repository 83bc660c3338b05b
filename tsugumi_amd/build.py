"""Builds libtsugumi_hip.so in-tree with hipcc for gfx950.

Each source compiles to an object in tsugumi_amd/_build/ (in parallel), then
one link. `python -m tsugumi_amd.build` or tsugumi_amd.build.build().
libtsugumi_floors.so (csrc/floors.hip) holds the measurement kernels of
`bench.py --floors`; it is not part of the drop-in library.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libtsugumi_hip.so")
FLOORS_LIB = os.path.join(HERE, "libtsugumi_floors.so")
# the grouped GEMM's kernels build as one translation unit per (group size,
# scheme), in parallel with the rest
GEMM_SOURCES = ["gemm_g32_sym.hip", "gemm_g32_affine.hip", "gemm_g64_sym.hip",
                "gemm_g64_affine.hip"]
SOURCES = ["core.hip", "decode.hip", "qmv.hip", "shared.hip", "prefill.hip", "tail.hip",
           *GEMM_SOURCES,
           "host_routing.cpp",
           "moepack.cpp"]
FLOORS_SOURCES = ["floors.hip"]

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ROCM = os.environ.get("ROCM_PATH", os.path.dirname(os.path.dirname(os.path.realpath(HIPCC))))
# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32 (the
# host pass warns that it does not know the feature; that is harmless).
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Wall",
         "-Wno-unused-function", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-munsafe-fp-atomics"]


# HIP sources: the dispatch preloads the first 14 argument dwords of each
# kernel into SGPRs (the latency-bound kernels pass what their first loads
# need there, ahead of any by-value struct, which is never preloaded); where
# the firmware does not, each kernel's prologue loads them as usual.
HIP_FLAGS = ["-mllvm", "-amdgpu-kernarg-preload-count=14"]
# The grouped GEMM's atomics are all single-lane; the atomic optimizer would
# turn the fused GEMM's fetch of its next work item into a wave-wide form that
# waits for the result right after issue instead of where it is used.
SOURCE_FLAGS = {src: ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]
                for src in ["prefill.hip", *GEMM_SOURCES]}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(os.path.basename(src))[0] + ".o")
    cmd = [HIPCC, *FLAGS, *(HIP_FLAGS if src.endswith(".hip") else []), *SOURCE_FLAGS.get(src, [])]
    if src.endswith(".cpp"):  # host-only C++; may call the HIP runtime API
        cmd += ["-x", "c++", "-D__HIP_PLATFORM_AMD__", "-I" + os.path.join(ROCM, "include")]
    cmd += ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in r.stderr.splitlines() if noise not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def _link(objs, lib: str) -> None:
    tmp = lib + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = SOURCES + FLOORS_SOURCES
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = dict(zip(srcs, ex.map(_compile, srcs)))
    _link([objs[s] for s in SOURCES], LIB)
    _link([objs[s] for s in FLOORS_SOURCES], FLOORS_LIB)
    if verbose:
        print(f"built {LIB} and {FLOORS_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)

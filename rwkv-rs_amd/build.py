"""Build libwkv7_hip.so (the gfx950 kernels and their C ABI: include/wkv7.h
and include/rwkv_neighbors.h) in-tree.

    python rwkv-rs_amd/build.py          # or __graft_entry__.build()

hipcc cross-compiles for gfx950 without a GPU. Packed-FP32 instruction
generation is switched off (-packed-fp32-ops): the kernels are written for
scalar v_fmac_f32 with DPP operands, and packed FP32 forms are avoided on this
hardware pool.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libwkv7_hip.so")
SOURCES = ["wkv7_api.cpp", "wkv7_forward.hip", "wkv7_backward.hip", "wkv7_infer.hip",
           "wkv7_chunk_forward.hip", "wkv7_chunk_backward.hip", "wkv7_f32_chunk.hip",
           "wkv7_selftest.hip",
           "neighbors_api.cpp", "neighbors.hip", "lm_loss_api.cpp", "lm_loss.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the WKV7 kernels)")


def flags() -> list[str]:
    return [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def build(verbose: bool = False) -> str:
    """Compile every source and link the shared library. Always rebuilds."""
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *flags(), "-shared", "-o", tmp,
           *[os.path.join(CSRC, s) for s in SOURCES]]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l and "(ignoring feature)" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


def build_sanitized(out_dir: str, verbose: bool = False) -> str:
    """A CPU-checking build: the C ABI's host code (every *_api.cpp: argument
    validation, pointer-range arithmetic) compiled by g++ with AddressSanitizer
    and UndefinedBehaviorSanitizer, linked with the unchanged gfx950 kernels.
    Load it into a process that preloads gcc's libasan and libubsan. Returns
    the library path (out_dir/libwkv7_hip.so)."""
    os.makedirs(out_dir, exist_ok=True)
    objs = []
    rocm = os.path.dirname(os.path.dirname(os.path.realpath(hipcc())))
    for src in SOURCES:
        obj = os.path.join(out_dir, src + ".o")
        if src.endswith(".cpp"):
            cmd = ["g++", "-std=c++17", "-O1", "-g", "-fPIC", "-fno-omit-frame-pointer",
                   "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
                   "-D__HIP_PLATFORM_AMD__", f"-I{rocm}/include", "-c",
                   os.path.join(CSRC, src), "-o", obj]
        else:
            cmd = [hipcc(), *flags(), "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True, capture_output=not verbose)
        objs.append(obj)
    lib = os.path.join(out_dir, "libwkv7_hip.so")
    cmd = ["g++", "-shared", "-fsanitize=address,undefined", "-o", lib, *objs,
           f"-L{rocm}/lib", "-lamdhip64", f"-Wl,-rpath,{rocm}/lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return lib


if __name__ == "__main__":
    if len(sys.argv) > 2 and sys.argv[1] == "--sanitize":
        print(build_sanitized(sys.argv[2], verbose=True))
    else:
        print(build(verbose=True))

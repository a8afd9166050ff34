"""Builds libtqhip.so (HIP kernels + C ABI) in-tree for gfx950 with hipcc.

Usage: python tiny-llm_amd/build.py   (or tiny_llm_amd.build() from Python)

Also builds libtqceil.so from csrc/ceilings.hip: the machine-ceiling probes (stream
read, empty launch, dense MFMA) that bench.py reports beside the kernels.

Every HIP translation unit is compiled with packed-fp32 instructions disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops); hipcc's host pass warns
that it does not know the feature, which is harmless.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
REPO = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libtqhip.so")
CEIL_LIB = os.path.join(HERE, "libtqceil.so")  # machine-ceiling probes, loaded by bench.py only
BUILD_DIR = os.path.join(HERE, "_build")

SOURCES = ["i4_matvec.hip", "i4_set.hip", "vq2_matvec.hip", "i4_matmul.hip", "biip_rotate.hip", "i4_embed.hip", "decode_engine.hip", "decode_flow.hip", "host_copy.hip", "tqwen_model.cpp", "dispatch.cpp",
           "capi.cpp", "synth.cpp", "scratch.cpp", "device.cpp"]
ARCH = os.environ.get("TQHIP_ARCH", "gfx950")


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _flags() -> list[str]:
    return [
        "-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-command-line-argument",
        "-I", os.path.join(REPO, "include"), "-I", CSRC,
    ]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [_hipcc(), *_flags(), "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compiles every source and links libtqhip.so. Returns the library path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as pool:
        objs = list(pool.map(_compile, SOURCES))
    # Only the C ABI is exported: the library's copy of the tinyqwen registry
    # stays internal, so linking it into tiny-llm (which has its own) cannot
    # interpose one registry on the other.
    vers = os.path.join(BUILD_DIR, "exports.map")
    with open(vers, "w") as f:
        f.write("{ global: tqhip_*; tq_*; local: *; };\n")
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread",
           f"-Wl,--version-script={vers}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    # the machine-ceiling probes bench.py reports beside the kernels (not part of the product)
    tmp = CEIL_LIB + ".tmp"
    cmd = [_hipcc(), *_flags(), "-shared", os.path.join(CSRC, "ceilings.hip"), "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, CEIL_LIB)
    if verbose:
        print(f"built {LIB} and {CEIL_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

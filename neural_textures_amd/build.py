"""Builds libnt_hip.so (the gfx950 kernels behind include/nt/nt.h) in-tree with hipcc.

Usage: python -m neural_textures_amd.build   (or neural_textures_amd.build.build())

Every HIP source is compiled for gfx950 only, with:
  -ffp-contract=off           every fused multiply-add is an explicit fmaf() in the source
  -munsafe-fp-atomics         float atomics lower to global_atomic_add_f32 / ds_add_f32
  -target-feature -packed-fp32-ops   no packed fp32 VALU instructions
  -mllvm -amdgpu-mfma-vgpr-form      MFMA results in VGPRs where they fit: kernels that use
                                     more than 256 registers otherwise get their MFMA
                                     results in AGPRs and copy every one out before the VALU
                                     can use it (v_accvgpr_read)
nt_train16.hip is compiled a second time (UNITS["random"]) for its random-texel kernels
alone, with -amdgpu-sched-strategy=max-memory-clause.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIBRARY = os.path.join(HERE, "libnt_hip.so")
SOURCES = ["nt_api.cpp", "nt_train.hip", "nt_train16.hip", "nt_train16.hip:random", "nt_forward.hip", "nt_adam.hip",
           "nt_codec.hip", "nt_bc6.hip", "nt_sort.hip", "nt_model.cpp"]
# Objects built from a source a second time ("file:unit"): their defines and extra flags.
UNITS = {
    "random": ["-DNT_TRAIN16_RANDOM_UNIT", "-mllvm", "-amdgpu-sched-strategy=max-memory-clause"],
}
HOST_DIR = os.path.join(HERE, "host")
HOST_SOURCES = ["nt_host.cpp", "nt_train_main.cpp"]
HOST_PROGRAM = os.path.join(HOST_DIR, "nt_train")

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unknown-pragmas",
]


def _compile(entry: str) -> str:
    src, _, unit = entry.partition(":")
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + (f"_{unit}" if unit else "") + ".o")
    extra = UNITS[unit] if unit else []
    cmd = [HIPCC, *FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC, "-x", "hip", *FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compiles every source for gfx950 and links libnt_hip.so; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIBRARY + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIBRARY)
    build_host()
    if verbose:
        print(f"built {LIBRARY} and {HOST_PROGRAM}")
    return LIBRARY


def build_host() -> str:
    """Builds the C++ host program (host/nt_train) against libnt_hip.so."""
    objs = []
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD_DIR, "host_" + os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-Wall", "-c", os.path.join(HOST_DIR, src),
               "-o", obj]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for host/{src}:\n{res.stdout}\n{res.stderr}")
        objs.append(obj)
    tmp = HOST_PROGRAM + ".tmp"
    cmd = [HIPCC, "-o", tmp, *objs, "-L" + HERE, "-lnt_hip", "-Wl,-rpath,$ORIGIN/..",
           "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"host link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, HOST_PROGRAM)
    return HOST_PROGRAM


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

"""Builds libzinfer_hip.so in-tree with hipcc for gfx950.

Every HIP translation unit is compiled with -ffp-contract=off (the exact
sampling tail must round every product and sum separately, as the Zig
reference does) and without packed FP32 instructions.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libzinfer_hip.so")
PROBE_LIB = os.path.join(PKG, "libzi_probe.so")  # bench.py's plain-read reference, not the sampling ABI
# tests/test_gpu_capi.py's C caller of the ABI (gcc, header + shared library only)
CONSUMER_SRC = os.path.join(ROOT, "tests", "capi", "consumer.c")
CONSUMER = os.path.join(ROOT, "tests", "capi", "zi_consumer")
OBJ = os.path.join(ROOT, "_build", "obj")

SOURCES = ["zi_sample.hip", "zi_sample_cap.hip", "zi_exact.hip", "zi_whole.hip", "zi_argmax.hip", "zi_entropy.hip", "zi_grammar.hip", "zi_pruned.hip", "zi_dry.hip",
           "zi_api.cpp",
           "zi_host.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-I", os.path.join(ROOT, "include"),
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, src + ".o")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    probe_obj = _compile("zi_probe.hip")
    tmp = PROBE_LIB + ".tmp"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", probe_obj, "-o", tmp],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed (probe):\n{r.stderr}")
    os.replace(tmp, PROBE_LIB)
    r = subprocess.run(["gcc", "-O2", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), CONSUMER_SRC,
                        "-L", PKG, "-lzinfer_hip", "-Wl,-rpath,$ORIGIN/../../zinfer_amd", "-o", CONSUMER],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"gcc failed for the C consumer:\n{r.stderr}")
    if verbose:
        print(f"built {LIB}, {PROBE_LIB} and {CONSUMER}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

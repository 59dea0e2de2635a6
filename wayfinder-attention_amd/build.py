"""Build libwayfinder_hip.so for gfx950 with hipcc (run from anywhere).

Each source compiles to an object in parallel, then one link step produces
``lib/libwayfinder_hip.so`` next to this file. Compiles every time it is called.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libwayfinder_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
SOURCES = ["wf_abi.cpp", "wf_topk.hip", "wf_topk_bf16.hip", "wf_topk_f16.hip", "wf_topk_f32.hip",
           "wf_fused.hip", "wf_readout.hip", "wf_readout_bwd.hip", "wf_address.hip", "wf_layernorm.hip",
           "wf_probe.hip"]

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed-FP32 instructions stay off: they have misbehaved on this hardware pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


# Measurement build: the retrieval's translation units compiled with WF_TOPK_TIMING, linked
# with the product's other objects into lib/libwayfinder_hip_timing.so. Its retrieval records
# per-workgroup phase timestamps in place of the scores (read by bench.py --leg topk-phases);
# indices are unchanged. Not loaded by anything else.
TIMING_LIB = os.path.join(LIB_DIR, "libwayfinder_hip_timing.so")
TIMING_SOURCES = ["wf_topk.hip", "wf_topk_bf16.hip", "wf_topk_f16.hip", "wf_topk_f32.hip"]


def build_timing(verbose: bool = False) -> str:
    build(verbose)
    tdir = os.path.join(OBJ, "timing")
    os.makedirs(tdir, exist_ok=True)

    def comp(src: str) -> str:
        obj = os.path.join(tdir, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC, *COMMON, "-DWF_TOPK_TIMING", "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src} (timing):\n{r.stdout}\n{r.stderr}")
        return obj

    with cf.ThreadPoolExecutor(max_workers=len(TIMING_SOURCES)) as ex:
        tobjs = list(ex.map(comp, TIMING_SOURCES))
    rest = [os.path.join(OBJ, os.path.splitext(s)[0] + ".o") for s in SOURCES if s not in TIMING_SOURCES]
    tmp = TIMING_LIB + ".tmp"
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *tobjs, *rest, "-o", tmp],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc link failed (timing):\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, TIMING_LIB)
    if verbose:
        print(f"built {TIMING_LIB}")
    return TIMING_LIB


if __name__ == "__main__":
    if "--timing" in sys.argv[1:]:
        build_timing(verbose=True)
    else:
        build(verbose=True)
    sys.exit(0)

"""Build libtensorshrink_hip.so in-tree for gfx950 with hipcc.

    python -m tensorshrink_amd.build        (or tensorshrink_amd.build.build())

Each .hip file is compiled to an object in parallel, then linked into a shared
library next to this file. Device code is built with packed-FP32 instruction
selection disabled; bit-exact paths additionally pin their own FP contraction
with `#pragma clang fp contract(off)`.
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
LIB = os.path.join(HERE, "libtensorshrink_hip.so")
SOURCES = [
    "ts_api.hip",
    "ts_decode.hip",
    "ts_decode_b2_g64.hip",
    "ts_decode_b2_g128.hip",
    "ts_decode_b2_g256.hip",
    "ts_decode_b4_g32.hip",
    "ts_decode_b4_g64.hip",
    "ts_decode_b4_g128.hip",
    "ts_decode_b4_g256.hip",
    "ts_decode_b6_g64.hip",
    "ts_decode_b6_g128.hip",
    "ts_decode_b8_g32.hip",
    "ts_decode_b8_g64.hip",
    "ts_decode_b8_g128.hip",
    "ts_prefill.hip",
    "ts_gemm.hip",
    "ts_prefill_b2_g64.hip",
    "ts_prefill_b2_g128.hip",
    "ts_prefill_b2_g256.hip",
    "ts_prefill_b4_g32.hip",
    "ts_prefill_b4_g64.hip",
    "ts_prefill_b4_g128.hip",
    "ts_prefill_b4_g256.hip",
    "ts_prefill_b6_g64.hip",
    "ts_prefill_b6_g128.hip",
    "ts_prefill_b8_g32.hip",
    "ts_prefill_b8_g64.hip",
    "ts_prefill_b8_g128.hip",
    "ts_aux.hip",
    "ts_quantize.hip",
]
ARCH = os.environ.get("TS_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def flags() -> list:
    return [
        f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-result", "-Wno-unused-value",
        "-I", os.path.join(HERE, "..", "include"),
    ]


def _stale(src: str, obj: str) -> bool:
    """Object older than its source or any header (TS_BUILD_INCREMENTAL=1 only)."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [os.path.join(CSRC, src)] + [os.path.join(CSRC, h) for h in os.listdir(CSRC) if h.endswith(".h")]
    deps.append(os.path.join(HERE, "..", "include", "tensorshrink_hip.h"))
    return any(os.path.getmtime(d) > t for d in deps)


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    if os.environ.get("TS_BUILD_INCREMENTAL") == "1" and not _stale(src, obj):
        return obj
    cmd = [hipcc(), *flags(), "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr[-6000:]}")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    jobs = min(len(SOURCES), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    rocm_lib = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-L", rocm_lib, "-lhipblaslt", f"-Wl,-rpath,{rocm_lib}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()

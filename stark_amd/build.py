"""Compile the HIP sources under stark_amd/csrc into stark_amd/libstark_qmm.so (gfx950),
and the decode-step kernels of the end-to-end stand-in (stark_amd/csrc_decode) into
stark_amd/libstark_decode.so."""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libstark_qmm.so")
CSRC_DECODE = os.path.join(HERE, "csrc_decode")
DECODE_LIB = os.path.join(HERE, "libstark_decode.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # keep hipcc from forming packed-FP32 instructions (v_pk_fma_f32 and friends)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep atomics as written: the optimizer's wave-aggregated form reads the result at once
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall", "-Wno-unused-function",
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    # the drop-in library exports only the entry points its header marks STARK_QMM_API
    extra = ["-fvisibility=hidden", "-fvisibility-inlines-hidden"] if os.path.dirname(src) == CSRC else []
    cmd = [HIPCC, *FLAGS, *extra, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def _link(objs, lib, extra=()):
    tmp = lib + ".tmp"
    r = subprocess.run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, *extra, "-o", tmp],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)
    return lib


def build(jobs: int = 8) -> str:
    os.makedirs(OBJ, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    decode_sources = sorted(glob.glob(os.path.join(CSRC_DECODE, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(jobs, len(sources) + len(decode_sources))) as ex:
        objs = list(ex.map(_compile, sources + decode_sources))
    _link(objs[len(sources):], DECODE_LIB)
    return _link(objs[:len(sources)], LIB, [f"-Wl,--version-script={os.path.join(CSRC, 'exports.map')}"])


if __name__ == "__main__":
    print(build())
    sys.exit(0)

"""Build libmodgrad_q4k for gfx950 with hipcc (in-tree, no JIT cache).

Produces modgrad_amd/libmodgrad_q4k.so (loaded by modgrad_amd._lib) and
modgrad_amd/libmodgrad_q4k.a (for a Rust build.rs to link statically).
Run: python -m modgrad_amd.build
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
OBJ = os.path.join(HERE, "_obj")
SO = os.path.join(HERE, "libmodgrad_q4k.so")
AR = os.path.join(HERE, "libmodgrad_q4k.a")

SOURCES = ["q4k_abi.hip", "q4k_dequant.hip", "q4k_gemv.hip", "q4k_batched.hip", "q4k_q8.hip", "q4k_kquant.hip", "q4k_gemm.hip", "q4k_glue.hip", "q4k_q6k_mfma.hip", "q4k_noalloc.hip", "q4k_chain.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # no packed-FP32 instructions (v_pk_*_f32): some of their forms have given
    # silently wrong results on the target machines
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{os.path.join(ROOT, 'include')}",
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = SO + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, SO)
    if os.path.exists(AR):
        os.remove(AR)
    subprocess.run(["ar", "rcs", AR, *objs], check=True)
    if verbose:
        print(f"built {SO}")
    return SO


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

"""Build libtrnfft_amd.so (all HIP kernels + the C ABI) for gfx950 with hipcc, in-tree, and
libtfa_copy.so, the plain-copy kernels bench.py measures the achievable memory rate with.

Usage: python -m trnfft_amd.csrc.build   (or trnfft_amd.csrc.build.build()).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB = os.path.join(PKG, "libtrnfft_amd.so")
COPY_LIB = os.path.join(PKG, "libtfa_copy.so")
COPY_SOURCE = "bench_copy.hip"
SOURCES = [
    "plan.hip",
    "kernels_c2c.hip",
    "kernels_strided.hip",
    "kernels_bluestein.hip",
    "kernels_stft.hip",
    "kernels_stft_blue.hip",
    "kernels_gemm.hip",
    "kernels_fft2.hip",
    "kernels_real.hip",
    "kernels_istft.hip",
]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3",
    "--offload-arch=gfx950",
    "-std=c++17",
    "-fPIC",
    # no packed-fp32 (v_pk_*_f32) code generation on this pool
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


# per-source extra flags: the fused Bluestein kernels feed compile-time zeros (the zero-padded
# half of its forward input) into its first pass; ignoring the sign of zero lets the compiler drop
# the additions of those zeros (x + 0 -> x), which changes no result beyond the sign of a zero
EXTRA_FLAGS = {"kernels_bluestein.hip": ["-fno-signed-zeros"], "kernels_stft_blue.hip": ["-fno-signed-zeros"]}


def _compile(src: str, obj: str) -> None:
    cmd = [HIPCC, *FLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(HERE, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")


def _link(objs: list[str], out: str) -> None:
    tmp = out + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed for {os.path.basename(out)}:\n{res.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    """Compile every source and link the shared libraries; returns the main library's path."""
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found ({HIPCC})")
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    srcs = SOURCES + [COPY_SOURCE]
    objs = [os.path.join(objdir, s.rsplit(".", 1)[0] + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 1)) as ex:
        list(ex.map(lambda so: _compile(*so), zip(srcs, objs)))
    _link(objs[:-1], LIB)
    _link(objs[-1:], COPY_LIB)
    if verbose:
        print(f"built {LIB} and {COPY_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

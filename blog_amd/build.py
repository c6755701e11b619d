"""Builds blog_amd/libqlin.so for gfx950 with hipcc (in-tree, so it travels with the sources).

    python -m blog_amd.build          # or: python blog_amd/build.py
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libqlin.so")
ARCH = os.environ.get("QLIN_ARCH", "gfx950")

SOURCES = ["qlin_gemv.hip", "qlin_q4k_stream.hip", "qlin_mfma_gemv.hip", "qlin_q4k_gemm.hip", "qlin_f32_gemm.hip", "qlin_qblk_gemm.hip", "qlin_dequant.hip", "qlin_q8_1.hip", "qlin_moe.hip", "qlin_moe_grouped.hip", "qlin_embed_mla.hip", "qlin_dense.hip", "qlin_mla_latent.hip", "qlin_q8_1_moe.hip", "qlin_decoder.hip", "qlin_api.cpp", "qlin_gguf.cpp"]

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}",
    # packed-FP32 VALU forms have produced silent wrong results on this pool: never emit them
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep every IEEE operation as written (bit-exact dequant); explicit fmaf() calls still fuse
    "-ffp-contract=off",
    # leading scalar kernel arguments preloaded into SGPRs at wave launch (gfx950), so a wave's first
    # requests need no scalar load of the argument segment
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


def _compile(src: str, obj_dir: str = OBJ, defines: tuple = ()) -> str:
    obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
    cmd = ["hipcc", *FLAGS, *[f"-D{d}" for d in defines], "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False, out: str = LIB, obj_dir: str = OBJ, defines: tuple = ()) -> str:
    """Compiles every source and links `out`; `defines` are extra -D macros (tuning variants)."""
    os.makedirs(obj_dir, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda src: _compile(src, obj_dir, defines), SOURCES))
    tmp = out + ".tmp"
    cmd = ["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

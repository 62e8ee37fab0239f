"""Builds libeyebrowse_hip.so in-tree with hipcc for gfx950.

Every translation unit under ``eyebrowse_amd/csrc`` is compiled in parallel into
``eyebrowse_amd/_build`` and linked into ``eyebrowse_amd/libeyebrowse_hip.so``. Run as
``python -m eyebrowse_amd.build``; ``__graft_entry__.build()`` calls :func:`build`.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libeyebrowse_hip.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# Packed-FP32 VALU forms are disabled for every device pass; hipcc -O3 would otherwise
# emit them from ordinary float code.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(ROOT, 'include')}",
    f"-I{CSRC}",
]

SOURCES = [
    "eb_runtime.cpp",
    "eb_nn.cpp",
    "eb_elementwise.hip",
    "eb_rows.hip",
    "eb_decode.hip",
    "eb_prefill.hip",
    "eb_linear.hip",
    "eb_argmax.hip",
    "eb_noalloc.hip",
]


# Per-source flags: matrix-core results in VGPRs. The narrow-cache decode and the
# head_dim 256 prefill rescale their accumulators on the VALU; with AGPR results the
# compiler copied every accumulator across on every tile (the prefill: 128 copies at the
# top of each step, for a rescale most steps skip). Kernels without AGPRs are unchanged.
SOURCE_FLAGS = {
    "eb_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "eb_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: str) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, *COMMON_FLAGS, *SOURCE_FLAGS.get(src, []), *lang, "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    warn = "\n".join(line for line in r.stderr.splitlines()
                     if "packed-fp32-ops" not in line and line.strip())
    if warn.strip():
        print(f"[build] {src}:\n{warn}", file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    """Compile every HIP/C++ source for gfx950 and link the shared library."""
    os.makedirs(OBJ, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[build] {LIB}")
    return LIB


if __name__ == "__main__":
    build()

"""Build ``libmtplx_amd.so`` for gfx950 with hipcc (in-tree, no JIT cache).

Usage: ``python -m mtplx_amd.build`` (also called by ``__graft_entry__.build``).
Objects go to ``mtplx_amd/_build/``; the shared library to
``mtplx_amd/libmtplx_amd.so``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmtplx_amd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["qmv.hip", "qmv_xplain.hip", "qmv_xswiglu.hip", "qmv_xpre.hip", "qmv_xrmsnorm.hip", "qmv_rope.hip",
           "qmv_moe.hip", "qmv_generic.hip", "qmm_mfma.hip", "sampler.hip", "attention.hip", "model_ops.hip", "moe.hip"]

# Packed fp32 VALU instructions are disabled for every device pass: some
# of their forms have produced silently wrong results on MI355X boxes of this
# pool. hipcc's host pass warns that it does not know the feature; harmless.
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs: the group finish reads them directly
    # instead of copying each accumulator out of the AGPR file first.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-I", CSRC,
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")
    return obj


def build(verbose: bool = True) -> str:
    """Compile every HIP source and link the shared library; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    sources = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()

"""In-tree build of ``liblps.so`` for gfx950 with hipcc.

Flags: ``-ffp-contract=off`` and correctly rounded fp32 division keep the
penalty / temperature arithmetic bit-identical to IEEE fp32; packed-fp32 ops
are disabled (``-packed-fp32-ops``)."""

from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)                    # llm-pipeline_amd/
REPO = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
INCLUDE = os.path.join(REPO, "include")
OUT = os.path.join(HERE, "liblps.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-shared", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Wall", "-Werror=return-type", "-Werror=uninitialized",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # a private array moved to LDS is addressed by the flat work-item id, which
    # makes every wave read the dispatch packet (host memory) first
    "-mllvm", "-disable-promote-alloca-to-lds",
]


def build(verbose: bool = False) -> str:
    """Compile ``csrc/lps.hip`` into ``lps/liblps.so`` (always recompiles)."""
    src = os.path.join(CSRC, "lps.hip")
    tmp = OUT + ".tmp"
    cmd = [HIPCC, *FLAGS, "-I", INCLUDE, "-I", CSRC, "-o", tmp, src]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(" ".join(cmd))
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))

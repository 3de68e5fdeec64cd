"""Build libkvm_amd.so from kvm-paper_amd/csrc with hipcc for gfx950.

Usage: python kvm-paper_amd/kvm_amd/build.py   (or __graft_entry__.build())
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"
OUT = PKG / "libkvm_amd.so"
SOURCES = ["kvm_api.hip", "kvm_update.hip", "kvm_chain.hip", "kvm_decode.hip", "kvm_attn.hip", "kvm_attn_bwd.hip",
           "kvm_state_bwd.hip", "kvm_prefix.hip", "kvm_gemm.hip", "kvm_block.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # Keep the compiler from forming packed fp32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into one shared library (always rebuilds)."""
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, "-o", str(tmp), *[str(CSRC / s) for s in SOURCES]]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    log = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{log}")
    if verbose and log.strip():
        print(log)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

"""Build libkvm_amd.so from kvm-paper_amd/csrc with hipcc for gfx950, and the
torch operator library libkvm_amd_torch.so over it.

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


OPS_SOURCE = "kvm_torch_ops.cpp"
OPS_OUT = PKG / "libkvm_amd_torch.so"


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    log = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{log}")
    if verbose and log.strip():
        print(log)


def build_ops(verbose: bool = False) -> Path:
    """The torch operator library (kvm_amd::prefill, kvm_amd::decode_step)
    over libkvm_amd.so: host code only, against the installed ROCm torch."""
    import torch
    from torch.utils.cpp_extension import include_paths

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = OPS_OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-I{p}" for p in include_paths(device_type="cuda")], "-o", str(tmp), str(CSRC / OPS_SOURCE),
           f"-L{PKG}", "-lkvm_amd", f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]
    _run(cmd, verbose)
    os.replace(tmp, OPS_OUT)
    return OPS_OUT


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into one shared library, then the torch
    operator library over it (always rebuilds)."""
    tmp = OUT.with_suffix(".so.tmp")
    _run([HIPCC, *FLAGS, "-o", str(tmp), *[str(CSRC / s) for s in SOURCES]], verbose)
    os.replace(tmp, OUT)
    build_ops(verbose)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

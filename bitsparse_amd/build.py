"""In-tree build of libbitsparse_hip.so for gfx950 (hipcc, no cmake)."""
from __future__ import annotations

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "bitsparse_amd")
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
SOURCES = ["runtime.hip", "fp8.hip", "codec.hip", "dw_gemm.hip", "dw_gemm8.hip", "up_gemm.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed fp32 VALU ops stay disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def build_library(verbose: bool = False, out: str | None = None,
                  defines: tuple[str, ...] = ()) -> str:
    """Compile every HIP source into bitsparse_amd/libbitsparse_hip.so
    (or `out`, with extra -D `defines`, for tuning builds)."""
    out = out or os.path.join(PKG, "libbitsparse_hip.so")
    tmp = out + ".tmp"
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    cmd = ([hipcc()] + HIPCC_FLAGS + [f"-D{d}" for d in defines] +
           ["-I", INCLUDE, "-I", CSRC, "-o", tmp] + srcs)
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-8000:]}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build_library(verbose=True))

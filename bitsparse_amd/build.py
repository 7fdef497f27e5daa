"""In-tree build of libbitsparse_hip.so for gfx950 (hipcc, no cmake).

Each HIP source is compiled to its own object in a parallel process (the
sources share no device symbols), then the objects are linked into one
shared library."""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "bitsparse_amd")
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
SOURCES = ["runtime.hip", "fp8.hip", "codec.hip", "dw_gemm.hip", "dw_gemm8.hip", "up_gemm.hip", "probe.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 VALU ops stay disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n"
                           f"{res.stderr[-8000:]}")


def build_library(verbose: bool = False, out: str | None = None,
                  defines: tuple[str, ...] = ()) -> str:
    """Compile every HIP source into bitsparse_amd/libbitsparse_hip.so
    (or `out`, with extra -D `defines`, for tuning builds)."""
    out = out or os.path.join(PKG, "libbitsparse_hip.so")
    tmp = out + ".tmp"
    objdir = os.path.join(os.path.dirname(out), "_build",
                          os.path.basename(out).replace(".so", ""))
    os.makedirs(objdir, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    objs = [os.path.join(objdir, s.replace(".hip", ".o")) for s in srcs]
    common = [hipcc()] + HIPCC_FLAGS + [f"-D{d}" for d in defines] + ["-I", INCLUDE, "-I", CSRC]
    cmds = [common + ["-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(srcs, objs)]
    jobs = min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 8)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs, verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build_library(verbose=True))

"""Build recipe of libstratum_nf4.so (hipcc, gfx950, in-tree)."""

from __future__ import annotations

import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libstratum_nf4.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["nf4_abi.hip", "nf4_quant.hip", "nf4_gemm.hip", "swiglu.hip", "lora.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off and correctly rounded fp32 division keep the quantizer's
# scale/compare arithmetic identical to the reference rounding; denormals are
# kept; packed-fp32 instructions are disabled for device code.
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-shared",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]

# Per-source additions. The GEMM kernels are scheduled with LLVM's iterative
# ILP strategy: 1-3 % faster on most fused GEMM shapes (A/B-timed against the
# default scheduler, outputs bit-identical).
SOURCE_FLAGS = {
    "nf4_gemm.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
}


def _run(cmd: list, verbose: bool) -> subprocess.Popen:
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def _finish(proc: subprocess.Popen, what: str, verbose: bool) -> None:
    out, _ = proc.communicate()
    if proc.returncode != 0:
        sys.stderr.write(out)
        raise RuntimeError(f"hipcc failed building {what} (exit {proc.returncode})")
    # drop the host-compiler note about the device-only feature flag
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in out.splitlines() if ln.strip() and noise not in ln]
    if msgs and verbose:
        print("\n".join(msgs), flush=True)


def build(verbose: bool = False) -> str:
    """Compile every source to an object (in parallel), then link the library.
    Objects go to a private temporary directory; nothing but the library is
    left in the package."""
    import tempfile
    compile_flags = [f for f in FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="stm_build_") as tmpdir:
        objs, procs = [], []
        for src in SOURCES:
            obj = os.path.join(tmpdir, os.path.splitext(src)[0] + ".o")
            objs.append(obj)
            extra = SOURCE_FLAGS.get(src, [])
            procs.append((_run([HIPCC, *compile_flags, *extra, "-c", os.path.join(CSRC, src), "-o", obj], verbose),
                          src))
        for proc, src in procs:
            _finish(proc, src, verbose)
        tmp = LIB_PATH + ".tmp"
        _finish(_run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs], verbose), LIB_NAME,
                verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))

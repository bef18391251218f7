"""Builds libaether_hip.so (all HIP kernels + the C ABI) for gfx950 with hipcc.

Usage: python -m aether_amd.build   (or aether_amd.build.build())
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libaether_hip.so")
SOURCES = [
    "aeth_weights.hip",
    "aeth_dequant.hip",
    "aeth_gemv.hip",
    "aeth_gemm.hip",
    "aeth_decode_ops.hip",
    "aeth_prefill.hip",
    "aeth_host.cpp",
    "aeth_runner.cpp",
]
ARCH = os.environ.get("AETH_OFFLOAD_ARCH", "gfx950")


def hipcc():
    for c in (os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc"), "hipcc"):
        if os.path.sep not in c or os.path.exists(c):
            return c
    return "hipcc"


def command(out=LIB):
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    return [
        hipcc(),
        "-x", "hip",
        "--offload-arch=" + ARCH,
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-fvisibility=hidden",
        "-ffp-contract=fast-honor-pragmas",
        # packed-FP32 VALU forms are kept out of the device code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-result",
        "-Wno-unused-value",
        "-o", out,
    ] + srcs


def build(verbose=True):
    cmd = command(LIB + ".tmp")
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if out.strip() and verbose:
        print(out, flush=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed (rc=%d)" % r.returncode)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)

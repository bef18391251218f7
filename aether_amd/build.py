"""Builds libaether_hip.so (all HIP kernels + the C ABI) for gfx950 with hipcc.

Usage: python -m aether_amd.build   (or aether_amd.build.build())
"""
import concurrent.futures
import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libaether_hip.so")
SOURCES = [
    "aeth_weights.hip",
    "aeth_dequant.hip",
    "aeth_quantize.hip",
    "aeth_gemv.hip",
    "aeth_gemv_ext.hip",
    "aeth_gemm.hip",
    "aeth_gemm_kq.hip",
    "aeth_gemm_q6k.hip",
    "aeth_gemm_q80.hip",
    "aeth_decode_ops.hip",
    "aeth_prefill.hip",
    "aeth_backend.hip",
    "aeth_host.cpp",
    "aeth_blas.cpp",
    "aeth_runner.cpp",
    "aeth_gguf.cpp",
]
ARCH = os.environ.get("AETH_OFFLOAD_ARCH", "gfx950")


def hipcc():
    for c in (os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc"), "hipcc"):
        if os.path.sep not in c or os.path.exists(c):
            return c
    return "hipcc"


# per-source device flags: the GEMMs keep their MFMA accumulators in VGPRs, where
# the per-super-block epilogues operate on them without AGPR→VGPR copies
EXTRA = {
    "aeth_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "aeth_gemm_kq.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "aeth_gemm_q6k.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "aeth_gemm_q80.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}

COMMON = [
    "-x", "hip",
    "--offload-arch=" + ARCH,
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-ffp-contract=fast-honor-pragmas",
    # packed-FP32 VALU forms are kept out of the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
    "-Wno-unused-value",
]


def compile_command(src, obj, extra=()):
    """hipcc -c of one source (csrc-relative name or path) into obj."""
    path = src if os.path.isabs(src) else os.path.join(CSRC, src)
    return [hipcc()] + COMMON + ["-I", CSRC] + EXTRA.get(os.path.basename(path), []) + list(extra) + \
        ["-c", "-o", obj, path]


ROCM_LIB = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")


def link_command(objs, out):
    # rocBLAS serves the plain f32 GEMMs of the formats without a GEMM kernel of their own
    return [hipcc(), "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", out] + list(objs) + \
        ["-L" + ROCM_LIB, "-lrocblas", "-Wl,-rpath," + ROCM_LIB]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    return r.returncode, out


def build(verbose=True, out=LIB, sources=None, extra=()):
    """Compiles every source (in parallel) and links the shared library at out."""
    sources = list(sources or SOURCES)
    with tempfile.TemporaryDirectory(prefix="aeth_build_") as tmp:
        objs = [os.path.join(tmp, "%02d_%s.o" % (i, os.path.basename(s))) for i, s in enumerate(sources)]
        cmds = [compile_command(s, o, extra) for s, o in zip(sources, objs)]
        with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(cmds))) as ex:
            results = list(ex.map(_run, cmds))
        failed = False
        for cmd, (rc, text) in zip(cmds, results):
            if verbose:
                print(" ".join(cmd), flush=True)
            if text.strip() and (verbose or rc):
                print(text, flush=True)
            failed |= rc != 0
        if failed:
            raise RuntimeError("hipcc failed")
        cmd = link_command(objs, out + ".tmp")
        if verbose:
            print(" ".join(cmd), flush=True)
        rc, text = _run(cmd)
        if text.strip():
            print(text, flush=True)
        if rc != 0:
            raise RuntimeError("link failed (rc=%d)" % rc)
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    build()
    sys.exit(0)

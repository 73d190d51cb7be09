"""Build of the gfx950 HIP library libkv800_hip.so (in-tree, next to this file under _lib/).

    python -m lfm3_kv800_amd.build        (or lfm3_kv800_amd.build.build())

Each .hip source is compiled with hipcc for gfx950 only. kv800_quant.hip is compiled with -ffp-contract=off so that
every float32 multiply and add the quantizer performs is rounded exactly where the reference's torch ops round (its
fused multiply-adds are written explicitly). Packed FP32 instructions are disabled for all device code."""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
LIBDIR = os.path.join(HERE, "_lib")
LIB = os.path.join(LIBDIR, "libkv800_hip.so")
ARCH = "gfx950"
SOURCES = {"kv800_quant.hip": ["-ffp-contract=off"], "kv800_decode.hip": ["-fno-strict-aliasing", "-mllvm", "-amdgpu-mfma-vgpr-form"],
           "kv800_cache.hip": [], "kv800_prefill.hip": [], "lfm3_model.hip": [], "lfm3_gemm.hip": []}
COMMON = ["--offload-arch=" + ARCH, "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", INCLUDE, "-I", CSRC]


def hipcc():
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")
    return exe


def build(verbose=False):
    """Compile every source and link libkv800_hip.so; returns its path. Always recompiles."""
    os.makedirs(LIBDIR, exist_ok=True)
    objs = []
    cc = hipcc()
    for src, extra in SOURCES.items():
        obj = os.path.join(LIBDIR, src.replace(".hip", ".o"))
        cmd = [cc, *COMMON, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{msg}")
        if verbose and msg.strip():
            print(msg, flush=True)
        objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [cc, "--offload-arch=" + ARCH, "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    for o in objs:
        os.remove(o)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

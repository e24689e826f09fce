"""Builds libbq.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python bruce-engine_amd/build.py          # or __graft_entry__.build()

Objects go to bruce-engine_amd/_build/, the library to bruce-engine_amd/libbq.so.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libbq.so")
BENCH_LIB = os.path.join(HERE, "libbq_bench.so")
SOURCES = ["bq_quant.hip", "bq_gemv.hip", "bq_repack.hip", "bq_gemm.hip", "bq_q8s.hip", "bq_norm.hip", "bq_gguf.hip", "bq_decode.hip", "bq_api.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed fp32 (v_pk_*_f32) is disabled for the device code: float code is
# scalarised.  hipcc's host pass warns that it does not know the feature.
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs (not AGPRs): the epilogues read every accumulator
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wno-unused-command-line-argument",
]


def _compile(src):
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC] + CFLAGS + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    jobs = min(len(SOURCES), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    # timing driver for bench.py, linked against libbq.so
    bobj = _compile("bq_bench.hip")
    tmp = BENCH_LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, bobj, "-L" + HERE, "-lbq",
           "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, BENCH_LIB)
    if verbose:
        print("built", LIB, "and", BENCH_LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

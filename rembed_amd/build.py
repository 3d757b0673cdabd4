"""Build librembed_hip.so (gfx950) in-tree with hipcc.

Usage: python -m rembed_amd.build   (or rembed_amd.build.build() from Python)

Every source under rembed_amd/csrc is compiled for gfx950 only, with
-ffp-contract=off (the reference-parity epilogues and quantizers must not be
contracted into FMAs) and packed-fp32 instruction selection disabled.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librembed_hip.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-unused-function",
]


# Per-file code generation: the attention kernels keep their MFMA
# accumulators in VGPRs (no AGPR round trips for the online-softmax rescale,
# two waves per SIMD at head dim 128).
FILE_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith((".hip", ".cpp")))


def _compile(src):
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [HIPCC] + FLAGS + FILE_FLAGS.get(os.path.basename(src), []) + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    # ICU supplies the Unicode tables of the host-side tokenizer (tokenizer.cpp)
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC"] + objs + ["-licuuc", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_blaslt_ref()
    return LIB


BLASLT_SRC = os.path.join(HERE, "blaslt_ref.cpp")
BLASLT_BIN = os.path.join(HERE, "blaslt_ref")


def build_blaslt_ref():
    """The hipBLASLt comparison program of the int8 GEMM microbenchmark
    (`python -m rembed_amd.microbench --hipblaslt`); not linked into the
    library."""
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-O2", "-std=c++17", BLASLT_SRC, "-lhipblaslt",
           "-o", BLASLT_BIN]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {BLASLT_SRC}:\n{r.stderr}")
    return BLASLT_BIN


if __name__ == "__main__":
    build()
    sys.exit(0)

"""Builds libarclight_fattn.so in-tree with hipcc for gfx950.

    python -m arclight_amd.build            # compile every csrc/*.hip and link
    python -m arclight_amd.build --asm DIR  # also write each object's gfx950 assembly to DIR

All HIP code is built with the packed-FP32 target feature off
(-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
import argparse
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
OBJDIR = os.path.join(HERE, "_build")
LIB = os.path.join(LIBDIR, "libarclight_fattn.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-file code generation options. The prefill kernel keeps its MFMA
# accumulators in VGPRs, which its softmax reads directly (with AGPR
# accumulators the compiler moves every tile's scores and output blocks
# between the two register files).
EXTRA_FLAGS = {
    "fattn_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src, asm_dir=None):
    obj = os.path.join(OBJDIR, os.path.basename(src) + ".o")
    extra = EXTRA_FLAGS.get(os.path.basename(src), [])
    cmd = [HIPCC, *CFLAGS, *extra, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the device-only target feature; drop that note
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if asm_dir:
        os.makedirs(asm_dir, exist_ok=True)
        out = os.path.join(asm_dir, os.path.basename(src) + ".s")
        subprocess.run([HIPCC, *CFLAGS, *extra, "--cuda-device-only", "-S", src, "-o", out],
                       check=True, capture_output=True)
    return obj, err


def build(asm_dir=None, verbose=True):
    os.makedirs(OBJDIR, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = list(ex.map(lambda s: _compile(s, asm_dir), srcs))
    for obj, err in results:
        if err.strip() and verbose:
            print(err, file=sys.stderr)
    objs = [o for o, _ in results]
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--asm", default=None)
    a = ap.parse_args()
    build(asm_dir=a.asm)

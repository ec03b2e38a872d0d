"""Builds libkapel_hip.so in-tree for gfx950 with hipcc (no JIT, no cache).

python -m kapel_amd.build   (or __graft_entry__.build())
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libkapel_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed f32 instructions are kept out of the code objects; no contraction of
# separate multiplies and adds; IEEE division stays correctly rounded.
HIP_FLAGS = ["--offload-arch=" + ARCH, "-O3", "-fPIC", "-std=c++17",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-ffp-contract=off", "-Wno-unused-command-line-argument"]
# The many-row product's MFMA results go to VGPRs, where its VALU work reads
# them, rather than to AGPRs (a copy per element).
MM_FLAGS = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
HOST_FLAGS = ["-O3", "-fPIC", "-std=c++17", "-ffp-contract=off", "-fno-fast-math"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout)
        raise RuntimeError("build failed: " + " ".join(cmd))


def build(verbose=False):
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    units = (
        ("kh_kernels.hip", HIPCC, HIP_FLAGS),
        ("kh_gemv.hip", HIPCC, HIP_FLAGS),
        ("kh_gemv_k.hip", HIPCC, HIP_FLAGS),
        ("kh_gemv_b.hip", HIPCC, HIP_FLAGS),
        ("kh_gemv_i.hip", HIPCC, HIP_FLAGS),
        ("kh_gemv_q.hip", HIPCC, HIP_FLAGS),
        ("kh_mm.hip", HIPCC, HIP_FLAGS),
        ("kh_mm_k.hip", HIPCC, HIP_FLAGS + MM_FLAGS),
        ("kh_mm_b.hip", HIPCC, HIP_FLAGS + MM_FLAGS),
        ("kh_mm_i.hip", HIPCC, HIP_FLAGS + MM_FLAGS),
        ("kh_mm_q.hip", HIPCC, HIP_FLAGS + MM_FLAGS),
        ("kh_mmf.hip", HIPCC, HIP_FLAGS),
        ("kh_mmf_k.hip", HIPCC, HIP_FLAGS),
        ("kh_mmf_b.hip", HIPCC, HIP_FLAGS),
        ("kh_mmf_i.hip", HIPCC, HIP_FLAGS),
        ("kh_mmf_q.hip", HIPCC, HIP_FLAGS),
        ("kh_api.cpp", HIPCC, HIP_FLAGS),
        ("kh_quantize.cpp", "g++", HOST_FLAGS),
    )
    objs = [os.path.join(objdir, src + ".o") for src, _, _ in units]

    def compile_one(i):
        src, compiler, flags = units[i]
        _run([compiler, *flags, "-c", os.path.join(CSRC, src), "-o", objs[i]])
        if verbose:
            print("compiled", src)

    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(len(units)) as pool:
        list(pool.map(compile_one, range(len(units))))
    tmp = OUT + ".tmp"
    _run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))

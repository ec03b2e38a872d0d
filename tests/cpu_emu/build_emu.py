"""Builds libkapel_hip_emu.so: the library's unchanged sources compiled for
the host against the emulation headers in this directory, with
AddressSanitizer (test infrastructure only; never loaded by the product)."""
import hashlib
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(ROOT, "kapel_amd", "csrc")
OUT = os.path.join(HERE, "libkapel_hip_emu.so")
CLANG = os.environ.get("EMU_CXX", "/opt/rocm/lib/llvm/bin/clang++")
SOURCES = ["kh_kernels.hip", "kh_gemv.hip", "kh_gemv_k.hip", "kh_gemv_b.hip", "kh_gemv_i.hip",
           "kh_gemv_q.hip", "kh_mm_q.hip",
           "kh_mm.hip", "kh_mm_k.hip", "kh_mm_b.hip", "kh_mm_i.hip", "kh_mmf.hip", "kh_mmf_k.hip",
           "kh_mmf_b.hip", "kh_mmf_i.hip", "kh_mmf_q.hip", "kh_api.cpp", "kh_quantize.cpp"]
FLAGS = ["-std=c++20", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer", "-fPIC",
         "-ffp-contract=off", "-I", HERE, "-pthread", "-Wno-unused-command-line-argument"]


def asan_runtime():
    out = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"],
                         capture_output=True, text=True).stdout.strip()
    if os.path.exists(out):
        return out
    base = os.path.dirname(os.path.dirname(CLANG))
    for root, _, files in os.walk(os.path.join(base, "lib", "clang")):
        if "libclang_rt.asan-x86_64.so" in files:
            return os.path.join(root, "libclang_rt.asan-x86_64.so")
    raise RuntimeError("no ASan runtime")


def digest():
    h = hashlib.sha256()
    for name in sorted(os.listdir(CSRC)) + ["hip/hip_runtime.h", "hip/hip_fp16.h", "build_emu.py"]:
        path = os.path.join(CSRC, name) if not name.startswith(("hip/", "build")) else os.path.join(HERE, name)
        if os.path.isfile(path):
            h.update(open(path, "rb").read())
    return h.hexdigest()


def build():
    stamp = OUT + ".sha256"
    d = digest()
    if os.path.exists(OUT) and os.path.exists(stamp) and open(stamp).read() == d:
        return OUT
    objs = [os.path.join(HERE, src + ".emu.o") for src in SOURCES]
    from concurrent.futures import ThreadPoolExecutor

    def one(i):
        subprocess.run([CLANG, *FLAGS, "-x", "c++", "-c", os.path.join(CSRC, SOURCES[i]), "-o", objs[i]],
                       check=True)

    with ThreadPoolExecutor(8) as pool:
        list(pool.map(one, range(len(SOURCES))))
    subprocess.run([CLANG, "-shared", "-fsanitize=address", "-pthread", *objs, "-o", OUT], check=True)
    for obj in objs:
        os.remove(obj)
    open(stamp, "w").write(d)
    return OUT


if __name__ == "__main__":
    print(build())

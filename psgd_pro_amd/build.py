"""Builds psgd_pro_amd/libpsgdk.so (gfx950) from psgd_pro_amd/csrc with hipcc, in the source tree.

    python -m psgd_pro_amd.build [--jobs N]

Objects go to psgd_pro_amd/_build/; sources are compiled in parallel and the library is linked with hipcc.

    python -m psgd_pro_amd.build --asan

also builds psgd_pro_amd/_build/libpsgdk_asan.so: the same library with its host code (capi.cpp, the C ABI's
argument checks, workspace planning and launch set-up) built with AddressSanitizer, for the CPU tests that drive the
C ABI without a GPU (tests/test_asan_cpu.py loads it with the sanitizer runtime preloaded). Device code is built as
usual; the sanitizer applies to host code only.
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libpsgdk.so")
SOURCES = ["gemm.hip", "gemm_bf16.hip", "gemm_small.hip", "nlb.hip", "elem.hip", "capi.cpp", "noalloc.hip",
           "measure.hip"]
ARCH = os.environ.get("PSGDK_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: keep the compiler from forming packed fp32 arithmetic (v_pk_*_f32), which is avoided here.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-I", os.path.join(HERE, "..", "include"),
          "-Wall", "-Wno-unused-function"]


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON, *DEVICE_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (r.stderr or "").splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{err}")
    return obj, err


ASAN_LIB = os.path.join(BUILD, "libpsgdk_asan.so")
# host-only sanitizer flags (each -fsanitize= applies to the host pass through -Xarch_host)
ASAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]


def asan_runtime():
    """Path of the compiler's AddressSanitizer runtime (to preload into a Python that loads ASAN_LIB)."""
    r = subprocess.run([HIPCC, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = r.stdout.strip()
    if not os.path.isabs(path) or not os.path.exists(path):
        lib_dir = subprocess.run([HIPCC, "-print-runtime-dir"], capture_output=True, text=True).stdout.strip()
        path = os.path.join(lib_dir, "libclang_rt.asan-x86_64.so")
    return path


def build_asan(objects):
    """capi.cpp with the host sanitizer, linked with the other (regular) objects into ASAN_LIB."""
    obj = os.path.join(BUILD, "capi_asan.o")
    cmd = [HIPCC, "-O1", "-g", *[f for f in COMMON if f != "-O3"], *DEVICE_FLAGS, *ASAN_HOST, "-c",
           os.path.join(CSRC, "capi.cpp"), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stderr}")
    others = [o for o in objects if os.path.basename(o) != "capi.o"]
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-Xarch_host", "-fsanitize=address", "-shared-libasan",
           "-o", ASAN_LIB, obj, *others]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
    return ASAN_LIB


def build(jobs=None, verbose=False, asan=False):
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(_compile, SOURCES))
    for _, err in results:
        if err.strip() and verbose:
            print(err, file=sys.stderr)
    tmp = LIB + ".tmp"
    # --no-undefined: a symbol that no object defines fails the link, not the first dlopen
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-Wl,--no-undefined", "-o", tmp, *[o for o, _ in results]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, LIB)
    if asan:
        build_asan([o for o, _ in results])
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--asan", action="store_true", help="also build the host-sanitized library for the CPU tests")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose, a.asan))

"""Build the MI355X backend in-tree.

    lib/libvsl_hip.so     HIP kernels for gfx950 + the runtime half of the C ABI (include/vsl_hip.h)
    lib/libvsl_engine.so  host C++ engine (VulkanSymbioteEngine, GGUFLoader, ConfigManager, packs)
                          + its C ABI (include/vsl_engine.h); links libvsl_hip.so

Usage: python build.py [--jobs N]
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
INC = os.path.join(ROOT, "include")
HIP_DIR = os.path.join(HERE, "csrc", "hip")
HOST_DIR = os.path.join(HERE, "csrc", "host")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "lib")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", shutil.which("g++") or "g++")
# Packed FP32 instructions are disabled for all device code.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-Wall", "-Wno-unused-function", "-I", INC, "-I", HIP_DIR]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter", "-I", INC, "-I",
              os.path.join(HOST_DIR, "vk_symbiote")]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _stale(obj, src, headers):
    """True when obj is missing or older than its source or any header it may include."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(p) > t for p in [src, *headers])


def build(jobs=8, verbose=False, incremental=False):
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    hip_srcs = sorted(f for f in os.listdir(HIP_DIR) if f.endswith(".hip"))
    host_srcs = sorted(f for f in os.listdir(os.path.join(HOST_DIR, "src")) if f.endswith(".cpp"))
    inc_h = [os.path.join(INC, f) for f in os.listdir(INC) if f.endswith(".h")]
    hip_h = inc_h + [os.path.join(HIP_DIR, f) for f in os.listdir(HIP_DIR) if f.endswith(".h")]
    host_h = inc_h + [os.path.join(HOST_DIR, "vk_symbiote", f) for f in os.listdir(os.path.join(HOST_DIR, "vk_symbiote"))]
    jobs_list = []
    for f in hip_srcs:
        o, src = os.path.join(OBJ, f + ".o"), os.path.join(HIP_DIR, f)
        if not incremental or _stale(o, src, hip_h):
            jobs_list.append([HIPCC, *HIP_FLAGS, "-c", src, "-o", o])
    for f in host_srcs:
        o, src = os.path.join(OBJ, f + ".o"), os.path.join(HOST_DIR, "src", f)
        if not incremental or _stale(o, src, host_h):
            jobs_list.append([CXX, *HOST_FLAGS, "-c", src, "-o", o])
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for out in ex.map(_run, jobs_list):
            if verbose and out.strip():
                print(out)
    hip_lib = os.path.join(LIB, "libvsl_hip.so")
    eng_lib = os.path.join(LIB, "libvsl_engine.so")
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", hip_lib + ".tmp",
          *[os.path.join(OBJ, f + ".o") for f in hip_srcs]])
    os.replace(hip_lib + ".tmp", hip_lib)
    _run([CXX, "-shared", "-fPIC", "-o", eng_lib + ".tmp", *[os.path.join(OBJ, f + ".o") for f in host_srcs],
          f"-L{LIB}", "-lvsl_hip", "-Wl,-rpath,$ORIGIN", "-lpthread"])
    os.replace(eng_lib + ".tmp", eng_lib)
    return hip_lib, eng_lib


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--incremental", action="store_true", help="recompile only objects older than their sources")
    a = ap.parse_args()
    for p in build(a.jobs, a.verbose, a.incremental):
        print(p)
    sys.exit(0)

"""Build the engine library (HIP kernels + C ABI + host side) and the CLI.

Outputs, in-tree so they travel with the repository snapshot:
  furnace_amd/lib/libfurnace_hip.so   kernels for gfx950, C ABI, host side
  furnace_amd/lib/libfurnace_hip.a    the same objects as a static library
  furnace_amd/bin/furnace-hip         CLI (run / dump-tensor / synth)
  furnace_amd/bin/capi_static         tests/capi_static.c linked statically
                                      against libfurnace_hip.a
Objects go to furnace_amd/_build/.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "lib", "libfurnace_hip.so")
CLI = os.path.join(PKG, "bin", "furnace-hip")
STATIC = os.path.join(PKG, "lib", "libfurnace_hip.a")
CAPI_STATIC = os.path.join(PKG, "bin", "capi_static")
TESTS = os.path.join(os.path.dirname(PKG), "tests")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# packed-fp32 instructions are disabled for all device code: some of their
# forms have given wrong results on this hardware
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
             "-I/opt/rocm/include", "-D__HIP_PLATFORM_AMD__"]

HIP_SOURCES = ["kernels.hip", "prefill.hip", "sampler.hip", "resident.hip", "engine.hip"]
HOST_SOURCES = ["host/errors.cpp", "host/gguf.cpp", "host/model.cpp", "host/synth.cpp"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError("build step failed: %s\n%s" % (" ".join(cmd), out))
    return out


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    os.makedirs(os.path.dirname(CLI), exist_ok=True)
    jobs = []
    objs = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace("/", "_") + ".o")
        jobs.append([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, src.replace("/", "_") + ".o")
        jobs.append(["g++"] + CXX_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for out in ex.map(_run, jobs):
            if verbose and out.strip():
                print(out)
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "-o", tmp] + objs + ["-lpthread"])
    os.replace(tmp, LIB)
    tmp = STATIC + ".tmp"
    if os.path.exists(tmp):
        os.remove(tmp)
    _run(["ar", "rcs", tmp] + objs)
    os.replace(tmp, STATIC)
    _run(["g++"] + CXX_FLAGS + [os.path.join(CSRC, "host", "cli.cpp"), "-o", CLI,
          "-L" + os.path.dirname(LIB), "-lfurnace_hip", "-L/opt/rocm/lib", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN/../lib", "-Wl,-rpath,/opt/rocm/lib"])
    # a C caller linked against the archive (no libfurnace_hip.so at run time)
    cobj = os.path.join(BUILD, "capi_static.o")
    _run(["gcc", "-O2", "-std=c99", "-Wall", "-Wextra", "-c", os.path.join(TESTS, "capi_static.c"), "-o", cobj])
    _run([HIPCC, "-o", CAPI_STATIC, cobj, STATIC, "-lpthread", "-Wl,-rpath,/opt/rocm/lib"])
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", LIB, CLI)

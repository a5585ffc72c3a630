"""Build libeii.so (gfx950 HIP kernels + C ABI), the eii_check conformance checker and
libeii_hostcheck.so in place.

    python build.py            # everything, next to this file
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I" + CSRC, "-I" + INCLUDE]

LIB = os.path.join(HERE, "libeii.so")
CHECKER = os.path.join(HERE, "eii_check")
HOSTCHECK = os.path.join(HERE, "libeii_hostcheck.so")


def run(cmd):
    print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_lib():
    objs = []
    os.makedirs(os.path.join(HERE, "_build"), exist_ok=True)
    for src in ("kernels.hip", "engine.hip"):
        obj = os.path.join(HERE, "_build", src + ".o")
        run([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", LIB + ".tmp"] + objs)
    os.replace(LIB + ".tmp", LIB)


def build_checker():
    run([HIPCC, "-O2", "-std=c++17", "-Wall", "-I" + INCLUDE, os.path.join(CSRC, "eii_check.cpp"),
         "-L" + HERE, "-leii", "-Wl,-rpath,$ORIGIN", "-o", CHECKER + ".tmp"])
    os.replace(CHECKER + ".tmp", CHECKER)


def build_hostcheck():
    run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-I" + CSRC,
         os.path.join(CSRC, "hostcheck.cpp"), "-o", HOSTCHECK])


def build():
    build_lib()
    build_checker()
    build_hostcheck()


if __name__ == "__main__":
    build()
    sys.exit(0)

"""Build libeii.so (gfx950 HIP kernels + C ABI), the eii_check conformance checker and
libeii_hostcheck.so in place.

    python build.py                              # everything, next to this file
    python build.py --out DIR --opt="-O1 ..."    # libeii.so + eii_check into DIR, the HIP
                                                 # sources and eii_check compiled with these
                                                 # optimization flags instead of -O3 / -O2 (the
                                                 # build variants of python -m eii.conformance)

hipcc applies a plain -O level to the host and the device code alike; "-Xarch_host -O0" after it
lowers the host code only (the engine, the C ABI and eii_check) and leaves the device code at
the level before it.
"""
import argparse
import os
import shlex
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

OPT = ["-O3"]
HIP_FLAGS = ["--offload-arch=gfx950", "-std=c++17", "-fPIC", "-Wall",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I" + CSRC, "-I" + INCLUDE]

HOSTCHECK = os.path.join(HERE, "libeii_hostcheck.so")


def run(cmd):
    print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_lib(out=HERE, opt=OPT):
    objs = []
    os.makedirs(os.path.join(out, "_build"), exist_ok=True)
    lib = os.path.join(out, "libeii.so")
    for src in ("kernels.hip", "engine.hip"):
        obj = os.path.join(out, "_build", src + ".o")
        run([HIPCC] + opt + HIP_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", lib + ".tmp"] + objs)
    os.replace(lib + ".tmp", lib)


def build_checker(out=HERE, opt=("-O2",)):
    checker = os.path.join(out, "eii_check")
    run([HIPCC] + list(opt) + ["-std=c++17", "-Wall", "-I" + INCLUDE, os.path.join(CSRC, "eii_check.cpp"),
                               "-L" + out, "-leii", "-Wl,-rpath,$ORIGIN", "-o", checker + ".tmp"])
    os.replace(checker + ".tmp", checker)


def build_hostcheck():
    run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-I" + CSRC,
         os.path.join(CSRC, "hostcheck.cpp"), "-o", HOSTCHECK])


def build():
    build_lib()
    build_checker()
    build_hostcheck()


def main(argv=None):
    ap = argparse.ArgumentParser(description="build libeii.so, eii_check and libeii_hostcheck.so")
    ap.add_argument("--out", help="build libeii.so and eii_check into this directory instead")
    ap.add_argument("--opt", default=" ".join(OPT), help="optimization flags of the HIP sources")
    a = ap.parse_args(argv)
    if a.out is None and a.opt == " ".join(OPT):
        build()
    else:
        out = os.path.abspath(a.out or HERE)
        os.makedirs(out, exist_ok=True)
        build_lib(out, shlex.split(a.opt))
        build_checker(out, shlex.split(a.opt))
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Build libr3d_gfx950.so (gfx950 only) and the CPU oracle library in-tree.

    python -m libr3d_amd.build            # or: python libr3d_amd/build.py

hipcc compiles the HIP kernels for --offload-arch=gfx950 with packed-fp32 code
generation switched off and matrix-core results written to ordinary VGPRs
(-amdgpu-mfma-vgpr-form: the kernels scale and add every MFMA result with VALU
instructions, which read only VGPRs; with results in AGPRs each element first needs a
v_accvgpr_read, a third of the e4m3 prefill tile's VALU work) and kernel-argument
preloading (-amdgpu-kernarg-preload-count=16: the dispatch puts the leading 14 dwords of a
kernel's arguments in SGPRs, so a wave's first loads do not wait on an argument fetch;
firmware without the feature runs the compiler's fallback prologue that loads them).  The
host C++ (row table, plans) goes into the same shared object.  The oracle (oracle/Makefile) is test infrastructure and is built beside it.
"""
import hashlib
import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "libr3d_amd")
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libr3d_gfx950.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["r3d_gemm.hip", "r3d_logits.hip", "r3d_noalloc.hip", "r3d_plan.cpp", "r3d_rows.cpp",
           "r3d_dump.cpp", "r3d_head.cpp", "r3d_probe.hip"]
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-function",
    "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
]


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError("command failed (%d): %s" % (r.returncode, " ".join(cmd)))
    return out


def source_id():
    """SHA-256 (hex) of the compile flags, then of every file under libr3d_amd/csrc and
    include, in name order, each hashed as "<path relative to the repo root>\n<bytes>" --
    the identity the library reports through r3d_gfx950_build_id()."""
    h = hashlib.sha256()
    h.update((" ".join(f for f in FLAGS if not f.startswith("-I")) + "\n").encode())
    files = []
    for d in (CSRC, os.path.join(ROOT, "include")):
        for name in os.listdir(d):
            p = os.path.join(d, name)
            if os.path.isfile(p):
                files.append(os.path.relpath(p, ROOT).replace(os.sep, "/"))
    for rel in sorted(files):
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(rel.encode() + b"\n" + f.read())
    return h.hexdigest()


def build_library():
    tmp = LIB + ".tmp"
    cmd = ([HIPCC] + FLAGS + ['-DR3D_BUILD_ID="%s"' % source_id()] +
           [os.path.join(CSRC, s) for s in SOURCES] + ["-o", tmp])
    out = _run(cmd)
    if out.strip():
        sys.stderr.write(out + "\n")
    os.replace(tmp, LIB)
    return LIB


def build_oracle():
    make = shutil.which("make")
    if make is None:
        raise RuntimeError("make not found")
    _run([make, "-s", "-C", os.path.join(ROOT, "oracle")])
    return os.path.join(ROOT, "oracle", "libr3d_oracle.so")


def build_harness():
    """The C engine-side test harness (tests/c_abi): compiled against the public headers and
    linked against the library just built and the oracle."""
    make = shutil.which("make")
    if make is None:
        raise RuntimeError("make not found")
    _run([make, "-s", "-B", "-C", os.path.join(ROOT, "tests", "c_abi")])
    return os.path.join(ROOT, "tests", "c_abi", "abi_harness")


def build_all():
    build_oracle()
    lib = build_library()
    build_harness()
    return lib


if __name__ == "__main__":
    print(build_all())

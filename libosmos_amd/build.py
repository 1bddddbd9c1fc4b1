"""Builds libosmos_amd/libosmos_mi355x.so: every csrc/*.hip compiled by hipcc for gfx950 and every csrc/*.cpp (host
code: the GGUF reader) by the same compiler as plain C++ (each file in its own process, in parallel), linked into one
shared library whose exports are exactly include/**/*.h's declarations.

flags: -O3, -ffp-contract=off (every product and sum rounded on its own: the contracts' bits), packed-FP32 ops off
(-Xclang -target-feature -Xclang -packed-fp32-ops), MFMA results in VGPRs (-mllvm -amdgpu-mfma-vgpr-form=1), -fPIC. run: python -m libosmos_amd.build
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libosmos_mi355x.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-ffp-contract=off", "-Wall",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-mllvm", "-amdgpu-mfma-vgpr-form=1",  # MFMA results straight in VGPRs: the epilogues read them with no copy
         "-I" + os.path.join(os.path.dirname(HERE), "include")]


HOST_FLAGS = ["-x", "c++", "-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall",
              "-I" + os.path.join(os.path.dirname(HERE), "include")]


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def compile_one(src):
    obj = os.path.join(OUT, src.rsplit(".", 1)[0] + ".o")
    flags = FLAGS if src.endswith(".hip") else HOST_FLAGS
    cmd = [HIPCC] + flags + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if r.returncode:
        raise RuntimeError("hipcc failed on %s:\n%s" % (src, err))
    return obj


CALIB_SRC = os.path.join(HERE, "calib", "ceilings.hip")
CALIB_LIB = os.path.join(HERE, "libosmos_calib.so")


def build_calib():
    """the roofline calibration kernels (bench.py --ceilings), a library of their own: not part of the product"""
    tmp = CALIB_LIB + ".tmp"
    cmd = [HIPCC] + [f for f in FLAGS if not f.startswith("-I")] + ["-shared", CALIB_SRC, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError("hipcc failed on calib/ceilings.hip:\n" + r.stderr)
    os.replace(tmp, CALIB_LIB)
    return CALIB_LIB


def build(jobs=None):
    os.makedirs(OUT, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=jobs or min(len(srcs), os.cpu_count() or 4, 8)) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    build_calib()
    return LIB


if __name__ == "__main__":
    print(build())
    sys.exit(0)

"""Builds libtensorium_hip.so (gfx950) in-tree from tensorium_amd/csrc.

Every .hip source is compiled to an object with hipcc in parallel, then
linked into a shared library next to this file, where the loader in
nnhip.py finds it.  Flags:
  -ffp-contract=off   no implicit FMA contraction: element-wise kernels must
                      issue exactly the separate fp32 operations the reference
                      CPU path does (bit-exact parity); FMAs are explicit.
  -packed-fp32-ops    disabled: no v_pk_{add,mul,fma}_f32 generation.
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libtensorium_hip.so")
OBJ_DIR = os.path.join(HERE, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src):
    obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
    extra = os.environ.get("TNH_HIPCC_FLAGS", "").split()  # e.g. -D switches for kernel variants
    cmd = [HIPCC, *FLAGS, *extra, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    return src, obj, r.returncode, err


def build(verbose=False, jobs=None):
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    objs = []
    failed = []
    with cf.ThreadPoolExecutor(jobs) as ex:
        for src, obj, rc, err in ex.map(_compile, srcs):
            if err.strip() and (verbose or rc):
                print(err, file=sys.stderr)
            if rc:
                failed.append(src)
            objs.append(obj)
    if failed:
        raise RuntimeError("hipcc failed for: " + ", ".join(failed))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        print(r.stderr, file=sys.stderr)
        raise RuntimeError("link of libtensorium_hip.so failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

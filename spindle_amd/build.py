"""Builds the gfx950 HIP library spindle_amd/libspx.so with hipcc (in-tree, no JIT cache).

Every source under csrc/ is compiled as HIP for --offload-arch=gfx950 and linked into one
shared library whose C ABI is include/spx.h. Compile flags:
  -ffp-contract=off   the kernels place every fused multiply-add explicitly (fmaf), so the
                      compiler must not contract a*b+c on its own (rounding is part of parity)
  -packed-fp32-ops off  no packed fp32 instructions are generated
"""
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libspx.so")
BUILD = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-O3", "--offload-arch=gfx950", "-fPIC", "-std=c++17", "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-result", "-Wno-unused-function"]


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, "-x", "hip", "-c", src, "-o", obj] + FLAGS
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (r.stderr or "").splitlines() if "packed-fp32-ops" not in l)
    return obj, r.returncode, err


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = list(ex.map(_compile, srcs))
    bad = [(o, e) for o, rc, e in results if rc != 0]
    for o, rc, e in results:
        if e.strip() and (verbose or rc != 0):
            sys.stderr.write(e + "\n")
    if bad:
        raise RuntimeError("HIP compile failed: " + ", ".join(os.path.basename(o) for o, _ in bad))
    objs = [o for o, _, _ in results]
    tmp = OUT + ".tmp"
    r = subprocess.run([HIPCC, "-shared", "-o", tmp] + objs + ["--offload-arch=gfx950", "-lpthread"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))

"""Build libh3hip.so (HIP kernels for gfx950 + host C runtime) in-tree.

    python -m h3cli_amd.build          # or: from h3cli_amd.build import build; build()

Every .hip file under csrc/ is compiled by hipcc for gfx950 only, every .c file
under host/ by gcc, and the objects are linked into h3cli_amd/libh3hip.so. The
library is what travels to the GPU box; nothing is JIT-compiled at run time.
"""
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
OBJ = PKG / "_build"
LIB = PKG / "libh3hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # Packed-FP32 instructions are disabled for device code on this pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # No IEEE NaN quieting around min/max (it doubles the score-max work);
    # kernels test finiteness on bit patterns instead of with isfinite().
    "-mno-amdgpu-ieee", "-fno-honor-nans",
    "-Wno-unused-result", "-Wno-unused-value", "-Wno-unused-command-line-argument",
    f"-I{ROOT / 'include'}",
]
C_FLAGS = ["-O2", "-std=c11", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
           "-ffp-contract=off", f"-I{ROOT / 'include'}"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the device-only feature flag; drop that noise.
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(map(str, cmd))}\n{out}")
    return out


def build(verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    jobs = []
    for src in sorted(CSRC.glob("*.hip")):
        jobs.append([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(OBJ / (src.stem + ".hip.o"))])
    for src in sorted(HOST.glob("*.c")):
        jobs.append(["gcc", *C_FLAGS, "-c", str(src), "-o", str(OBJ / (src.stem + ".c.o"))])
    workers = min(len(jobs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with cf.ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        for out in ex.map(_run, jobs):
            if verbose and out.strip():
                print(out)
    objs = [str(OBJ / (s.stem + ".hip.o")) for s in sorted(CSRC.glob("*.hip"))]
    objs += [str(OBJ / (s.stem + ".c.o")) for s in sorted(HOST.glob("*.c"))]
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs, "-lpthread"])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

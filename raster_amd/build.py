"""Builds raster_amd/librq.so (gfx950 HIP kernels + the C ABI of include/rq.h).

    python -m raster_amd.build [--force]

Each .hip file in raster_amd/csrc is compiled to an object under
raster_amd/_build/ (in parallel), then the objects are linked into librq.so.
Without --force only objects older than their source or a shared header are
rebuilt. Packed-FP32 instruction selection is switched off
(-packed-fp32-ops) for every device compile; hipcc's host pass warns that it
does not know that feature, which is harmless. MFMA accumulators are kept in
VGPRs (-amdgpu-mfma-vgpr-form), except in the files of AGPR_SOURCES, whose
kernels run one wave per SIMD with accumulator tiles larger than the 256
architectural VGPRs.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librq.so")
HEADERS = [os.path.join(CSRC, "rq_internal.h"), os.path.join(os.path.dirname(HERE), "include", "rq.h")]
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: without it the register allocator copies
    # accumulator tiles between AGPRs around every MFMA
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function",
]
# one wave per SIMD, 192-224 accumulator registers per lane: those live in AGPRs
AGPR_SOURCES = {"gemm_wide.hip"}
# the dense f32 GEMM entries call rocBLAS (dense.hip)
LINK_LIBS = ["-L/opt/rocm/lib", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build librq)")


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _stale(src: str, obj: str) -> bool:
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(p) > t for p in [src, *HEADERS])


def flags_for(src: str) -> list[str]:
    if os.path.basename(src) not in AGPR_SOURCES:
        return list(FLAGS)
    out, skip = [], False
    for i, f in enumerate(FLAGS):
        if skip:
            skip = False
            continue
        if f == "-mllvm" and i + 1 < len(FLAGS) and FLAGS[i + 1] == "-amdgpu-mfma-vgpr-form":
            skip = True
            continue
        out.append(f)
    return out


def _compile(src: str, obj: str) -> tuple[str, int, list[str]]:
    tmp = obj + ".tmp"
    r = subprocess.run([hipcc(), *flags_for(src), "-c", "-o", tmp, src], capture_output=True, text=True)
    errs = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln]
    if r.returncode == 0:
        os.replace(tmp, obj)
    return src, r.returncode, errs


def build(verbose: bool = False, force: bool = False, jobs: int | None = None) -> str:
    os.makedirs(OBJ, exist_ok=True)
    pairs = [(s, os.path.join(OBJ, os.path.basename(s)[:-4] + ".o")) for s in sources()]
    todo = [(s, o) for s, o in pairs if force or _stale(s, o)]
    jobs = jobs or max(1, min(len(todo), os.cpu_count() or 1, 8))
    failed = []
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for src, rc, errs in ex.map(lambda so: _compile(*so), todo):
            if rc != 0:
                failed.append(f"{os.path.basename(src)}:\n" + "\n".join(errs))
            elif verbose and errs:
                print("\n".join(errs), file=sys.stderr)
    if failed:
        raise RuntimeError("librq build failed:\n" + "\n\n".join(failed))
    if todo or force or not os.path.exists(LIB):
        tmp = LIB + ".tmp"
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[o for _, o in pairs], *LINK_LIBS]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("librq link failed:\n" + r.stderr)
        os.replace(tmp, LIB)
    if verbose:
        print(f"compiled {len(todo)} of {len(pairs)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True, force="--force" in sys.argv))

"""Build recipe for libcinnamon_fp8.so (hand-written HIP for gfx950 only).

Compiles every ``csrc/*.hip`` with hipcc into objects under ``_build/`` and links
them into ``cinnamon_amd/libcinnamon_fp8.so`` in-tree, so the library travels
with the source tree to the GPU host.  The library links the HIP runtime by
soname (``libamdhip64.so.7``) and is loaded after ``import torch``, so it binds
to the runtime torch has already mapped.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
BUILD = os.path.join(os.path.dirname(HERE), "_build")
LIB = os.path.join(HERE, "libcinnamon_fp8.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    # packed fp32 VALU ops stay off (hand-written and compiler-made)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the GEMM epilogue FMAs read every MFMA result, and an
    # AGPR destination would add one v_accvgpr_read per element
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    f"-I{INCLUDE}",
    "-Wall",
    "-Wno-unused-function",
]


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str) -> tuple[str, str]:
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *COMMON, "-c", src, "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{p.stdout}\n{p.stderr}")
    return obj, p.stderr


def build(verbose: bool = False) -> str:
    """Compile all HIP sources and link the shared library; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = list(ex.map(_compile, srcs))
    objs = [o for o, _ in results]
    if verbose:
        for o, err in results:
            msgs = [l for l in err.splitlines() if "packed-fp32-ops" not in l and l.strip()]
            if msgs:
                print(f"[{os.path.basename(o)}]", "\n".join(msgs), file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{p.stdout}\n{p.stderr}")
    os.replace(tmp, LIB)
    return LIB


def build_bench_ceiling() -> str:
    """Compile bench.py's calibration kernel (bench_ceiling.hip at the repo root, not part of
    the library) into bench_ceiling.so beside it; returns its path."""
    root = os.path.dirname(HERE)
    src, out = os.path.join(root, "bench_ceiling.hip"), os.path.join(root, "bench_ceiling.so")
    cmd = [HIPCC, *COMMON, "-shared", src, "-o", out]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{p.stdout}\n{p.stderr}")
    return out


def build_test_checks() -> list[str]:
    """Compile the test suite's device checks (tests/gpu_checks/*.hip, test infrastructure
    that exercises the library's device helpers) into lib<name>.so beside each source."""
    root = os.path.dirname(HERE)
    d = os.path.join(root, "tests", "gpu_checks")
    outs = []
    for f in sorted(os.listdir(d)):
        if not f.endswith(".hip"):
            continue
        src, out = os.path.join(d, f), os.path.join(d, "lib" + f[:-4] + ".so")
        cmd = [HIPCC, *COMMON, "-shared", src, "-o", out]
        p = subprocess.run(cmd, capture_output=True, text=True)
        if p.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{p.stdout}\n{p.stderr}")
        outs.append(out)
    return outs


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_bench_ceiling())
    print(build_test_checks())

"""Build recipe for libzenith_hip.so (gfx950).

Replaces the reference's JIT build of the `zenith_cuda` torch extension
(zenith/build_cuda.py:50-141, torch.utils.cpp_extension.load with nvcc
-gencode flags). Here every ``csrc/*.hip`` file is compiled by hipcc for
gfx950 in parallel and linked into one plain shared library with a C ABI
(include/zk_api.h); no torch headers are involved, so the library loads with
ctypes from any Python.
"""

from __future__ import annotations

import concurrent.futures as _cf
import glob
import os
import shutil
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libzenith_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
OBJ_DIR = os.path.join(PKG_DIR, "_build")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-std=c++17",
    "-O3",
    "-fPIC",
    # gfx950: keep the compiler from emitting packed fp32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs (the unified register file allows
    # it): no accvgpr copies between the matrix products and the VALU work
    # on their results (softmax, epilogues)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm toolchain required to build libzenith_hip.so)")
    return path


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns about the gfx-only target feature; drop that line.
    out = "\n".join(
        ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln
    ).strip()
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out:
        print(out)


def build(verbose: bool = True, jobs: int | None = None) -> str:
    """Compile every csrc/*.hip for gfx950 and link libzenith_hip.so.

    Always recompiles (this is the "does it build" check). Returns the
    library path.
    """
    hipcc = _hipcc()
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    os.makedirs(OBJ_DIR, exist_ok=True)
    objs = []
    cmds = []
    for src in sources:
        obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, "-c", src, "-o", obj])
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 4)), 8)
    with _cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for fut in [ex.submit(_run, c) for c in cmds]:
            fut.result()
    tmp = LIB_PATH + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


SAN_DIR = os.path.join(OBJ_DIR, "host_sanitized")
SAN_LIB = os.path.join(SAN_DIR, "libzenith_hip_host_sanitized.so")
# AddressSanitizer and UndefinedBehaviorSanitizer on the host side of every
# source (argument checks, launch plans, dispatch); device code is built as
# in HIPCC_FLAGS. The library expects the ASan runtime to be loaded first
# (LD_PRELOAD of host_asan_runtime()), as for any sanitized shared library
# loaded into an uninstrumented program.
SAN_FLAGS = [
    "-Xarch_host", "-g",
    "-Xarch_host", "-fno-omit-frame-pointer",
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined",
]


def host_asan_runtime() -> str:
    """Path of the ASan runtime of the hipcc toolchain (to LD_PRELOAD)."""
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        raise RuntimeError("ASan runtime of the ROCm clang not found")
    return hits[-1]


def build_host_sanitized(jobs: int | None = None) -> str:
    """Build libzenith_hip.so with host-side ASan + UBSan into SAN_LIB.

    Rebuilt only when a source or header changed since the last build (the
    hash of their contents and the flags is kept beside the library).
    Returns the library path.
    """
    import hashlib

    hipcc = _hipcc()
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    inputs = sources + sorted(glob.glob(os.path.join(CSRC, "*.hpp")))
    inputs.append(os.path.join(os.path.dirname(PKG_DIR), "include", "zk_api.h"))
    h = hashlib.sha256(" ".join(HIPCC_FLAGS + SAN_FLAGS).encode())
    for p in inputs:
        with open(p, "rb") as f:
            h.update(f.read())
    stamp = os.path.join(SAN_DIR, "inputs.sha256")
    digest = h.hexdigest()
    if os.path.exists(SAN_LIB) and os.path.exists(stamp) and open(stamp).read() == digest:
        return SAN_LIB
    os.makedirs(SAN_DIR, exist_ok=True)
    objs, cmds = [], []
    for src in sources:
        obj = os.path.join(SAN_DIR, os.path.basename(src)[:-4] + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, *SAN_FLAGS, "-c", src, "-o", obj])
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 4)), 8)
    with _cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for fut in [ex.submit(_run, c) for c in cmds]:
            fut.result()
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address",
          "-Xarch_host", "-fsanitize=undefined", *objs, "-o", SAN_LIB])
    with open(stamp, "w") as f:
        f.write(digest)
    return SAN_LIB


if __name__ == "__main__":
    build()

"""ctypes / import access to the compiled CPU checkers. TEST INFRASTRUCTURE ONLY.

- libzk_oracle.so: own C restatement of the reference AVX2 GEMM (cpu_gemm.c).
- _ref/libzenith_ref_kernels.so: the reference's core/src/cpu_kernels.cpp,
  compiled unchanged (`make ref`); symbols are the C++ names of
  zenith::kernels::matmul_f32 / matmul_f32_naive / softmax_f32
  (core/include/zenith/kernels.hpp:65-72,169).
- _ref/zref_features*.so: the reference's python/src/features_bindings.hpp
  CPU fused ops (fused.add_layernorm, fused.bias_gelu).
"""

from __future__ import annotations

import ctypes
import glob
import importlib.util
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "libzk_oracle.so")
REF_DIR = os.path.join(HERE, "_ref")
REF_KERNELS = os.path.join(REF_DIR, "libzenith_ref_kernels.so")

_fp = ctypes.POINTER(ctypes.c_float)


def build(ref: bool | None = None) -> None:
    """make the own oracle library; also `make ref` when the reference
    sources are present (ref=None) or when asked (ref=True)."""
    subprocess.run(["make", "-s", "-C", HERE, "libzk_oracle.so"], check=True)
    want_ref = os.path.isdir("/root/reference/core/src") if ref is None else ref
    if want_ref:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_fp)


class _Gemm:
    def __init__(self, path: str, names: dict[str, str]):
        self.lib = ctypes.CDLL(path)
        self.fns = {}
        for key, sym in names.items():
            fn = getattr(self.lib, sym)
            fn.argtypes = [_fp, _fp, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
            fn.restype = None
            self.fns[key] = fn

    def matmul(self, a: np.ndarray, b: np.ndarray, kind: str = "avx2") -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        M, K = a.shape
        K2, N = b.shape
        assert K == K2
        c = np.empty((M, N), dtype=np.float32)
        self.fns[kind](_ptr(a), _ptr(b), _ptr(c), M, N, K)
        return c


_own = None
_ref = None


def own_gemm() -> _Gemm:
    """Own restatement (libzk_oracle.so), built on demand."""
    global _own
    if _own is None:
        if not os.path.exists(ORACLE_LIB):
            build(ref=False)
        _own = _Gemm(ORACLE_LIB, {"avx2": "zko_matmul_f32_avx2", "naive": "zko_matmul_f32_naive"})
    return _own


def ref_available() -> bool:
    return os.path.exists(REF_KERNELS)


def ref_gemm() -> _Gemm:
    """The reference's own cpu_kernels.cpp build (oracle/_ref)."""
    global _ref
    if _ref is None:
        _ref = _Gemm(REF_KERNELS, {
            "dispatch": "_ZN6zenith7kernels10matmul_f32EPKfS2_Pfiii",
            "avx2": "_ZN6zenith7kernels15matmul_f32_avx2EPKfS2_Pfiii",
            "naive": "_ZN6zenith7kernels16matmul_f32_naiveEPKfS2_Pfiii",
        })
        sm = getattr(_ref.lib, "_ZN6zenith7kernels11softmax_f32EPKfPfmm")
        sm.argtypes = [_fp, _fp, ctypes.c_size_t, ctypes.c_size_t]
        sm.restype = None
        _ref.fns["softmax"] = sm
    return _ref


def ref_softmax(x: np.ndarray) -> np.ndarray:
    """softmax over the last axis with the reference's softmax_f32."""
    g = ref_gemm()
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    g.fns["softmax"](_ptr(x), _ptr(y), x.size, x.shape[-1])
    return y


def ref_features():
    """The reference's CPU fused-op module (fused.add_layernorm / bias_gelu),
    or None when oracle/_ref was not built."""
    hits = glob.glob(os.path.join(REF_DIR, "zref_features*.so"))
    if not hits:
        return None
    spec = importlib.util.spec_from_file_location("zref_features", hits[0])
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod

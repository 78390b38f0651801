"""ctypes binding of libzenith_hip.so (the C ABI declared in include/zk_api.h).

The library is loaded on first use. There is deliberately no fallback: if the
shared library is missing or fails to load, every entry point raises
RuntimeError, so a GPU run can never silently take another code path.
"""

from __future__ import annotations

import ctypes
import os
import threading

from ._build import LIB_PATH

ZK_OK = 0
ZK_ERR_INVALID = -1
ZK_ERR_UNSUPPORTED = -2
ZK_ERR_HIP = -3

ZK_F32, ZK_F16, ZK_I8, ZK_I32 = 0, 1, 2, 3
ZK_GELU_TANH, ZK_GELU_ERF = 0, 1
(
    ZK_EPI_NONE,
    ZK_EPI_BIAS,
    ZK_EPI_BIAS_GELU_ERF,
    ZK_EPI_BIAS_GELU_TANH,
    ZK_EPI_BIAS_RESIDUAL,
    ZK_EPI_BIAS_RELU,
) = range(6)

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> argtypes (restype is int unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "zk_last_error": [],
    "zk_version": [],
    "zk_clock_probe": [_i32, _i32, _vp, _vp, _vp],
    "zk_relu": [_vp, _vp, _i64, _i32, _vp],
    "zk_sigmoid": [_vp, _vp, _i64, _i32, _vp],
    "zk_tanh": [_vp, _vp, _i64, _i32, _vp],
    "zk_gelu": [_vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp],
    "zk_layernorm": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _i32, _vp],
    "zk_layernorm_q8": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _f32, _vp],
    "zk_layernorm_q8_res_ln": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32,
                               _f32, _vp],
    "zk_layernorm_add": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _i32, _vp],
    "zk_transpose_f16": [_vp, _vp, _i64, _i64, _i64, _i64, _vp],
    "zk_gemm_f16": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32,
                    _vp, _vp, _i64, _i32, _vp],
    "zk_gemm_f32": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _vp],
    "zk_linear_f32": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _i32,
                      _vp, _i64, _vp],
    "zk_qkv_attn_f16": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _f32, _vp],
    "zk_qkv_attn_f16_ln": [_vp, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp,
                           _f32, _vp],
    "zk_qkv_attn_f16_frag": [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                             _i64, _vp, _f32, _vp],
    "zk_gemm_f16_res_stats": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64,
                              _vp, _vp, _vp, _vp, _vp],
    "zk_gemm_f16_ln": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _f32, _vp, _vp,
                       _vp, _i32, _vp],
    "zk_gemm_f16_ln_frag": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _f32, _vp, _vp,
                            _vp, _vp],
    "zk_gemm_f16_frag": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp],
    "zk_gemm_f16_res_stats_frag": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64,
                                   _vp, _vp, _vp, _vp, _vp],
    "zk_flash_attn_fwd": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                          ctypes.POINTER(_i64), _vp, _f32, _i32, _vp],
    "zk_flash_attn_fwd_masked": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                 ctypes.POINTER(_i64), _vp, _vp, ctypes.POINTER(_i64), _f32,
                                 _i32, _vp],
    "zk_quantize_i8": [_vp, _vp, _i64, _f32, _i32, _vp],
    "zk_gemm_i8": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _vp,
                   _vp, _vp, _i64, _i32, _i32, _vp],
    "zk_gemm_i8_requant": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _vp,
                           _vp, _i32, _f32, _vp],
    "zk_gemm_i8_res_stats": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _vp,
                             _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp],
    "zk_gemm_i8_requant_frag": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _vp, _vp,
                                _i32, _f32, _vp],
    "zk_gemm_i8_res_stats_frag": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _vp, _vp,
                                  _vp, _i64, _vp, _vp, _vp, _vp, _vp],
    "zk_gemm_workspace_size": [_i64, _i64, _i64, _i32],
    "zk_gemm_f16_ws": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32,
                       _vp, _vp, _i64, _i32, _vp, _i64, _vp],
    "zk_gemm_f16_add_ln": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                           _f32, _vp, _i64, _vp],
    "zk_gemm_f32_ws": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _vp, _i64, _vp],
    "zk_gemm_f16_noalloc": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32,
                            _vp, _vp, _i64, _i32, _vp],
    "zk_embedding": [_vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp],
    "zk_bert_embeddings": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                           _i64, _i64, _i64, _f32, _i32, _vp],
    "zk_add": [_vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp],
    "zk_softmax": [_vp, _vp, _i64, _i64, _i32, _vp],
    "zk_transpose_0213": [_vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp],
    "zk_convert": [_vp, _vp, _i64, _i32, _i32, _vp],
}
_RESTYPES = {"zk_last_error": ctypes.c_char_p, "zk_gemm_workspace_size": ctypes.c_int64}

_lock = threading.Lock()
_lib = None


def load(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and return the library; raise RuntimeError if unavailable."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        # ZENITH_HIP_LIB names another build of the library (e.g. the
        # host-sanitized one the CPU tests run the ABI checks against)
        p = path or os.environ.get("ZENITH_HIP_LIB") or LIB_PATH
        if not os.path.exists(p):
            raise RuntimeError(
                f"zenith_amd: HIP kernel library not found at {p}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` "
                "(or python -m zenith_amd._build)"
            )
        try:
            lib = ctypes.CDLL(p)
        except OSError as e:  # pragma: no cover - depends on the host
            raise RuntimeError(f"zenith_amd: cannot load {p}: {e}") from e
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        if path is None:
            _lib = lib
        return lib


def last_error() -> str:
    msg = load().zk_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> None:
    """Call a zk_* entry point and raise RuntimeError on a non-zero status."""
    rc = getattr(load(), name)(*args)
    if rc != ZK_OK:
        raise RuntimeError(f"{name} failed ({rc}): {last_error()}")


def strides_arg(vals) -> ctypes.Array:
    arr = (_i64 * len(vals))(*[int(v) for v in vals])
    return arr

"""C-ABI checks that need no GPU: libzenith_hip.so loads, exports every
function include/zk_api.h declares, and rejects bad arguments with the
documented status codes before touching the device."""

import ctypes
import os
import re

import pytest

from zenith_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "zk_api.h")).read()
    # function declarations: "<type> zk_name(" at the start of a line
    return sorted(set(re.findall(r"^(?:const\s+)?\w+\s*\*?\s*(zk_[a-z0-9_]+)\s*\(", src, re.M)))


def test_header_and_binding_agree():
    assert _declared() == sorted(L.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = L.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.zk_version() >= 100


@pytest.mark.parametrize("call,code", [
    (lambda lib: lib.zk_clock_probe(0, 10, None, None, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_relu(None, None, -1, L.ZK_F32, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_relu(None, None, 5, L.ZK_F32, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_relu(1, 1, 5, 7, None), L.ZK_ERR_UNSUPPORTED),
    (lambda lib: lib.zk_gelu(1, None, 1, 2, 2, 9, L.ZK_F32, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_layernorm(1, None, 1, 1, 1, 4, 0, 1e-5, L.ZK_F32, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_layernorm(1, None, 1, 1, 1, 4, 8, -1.0, L.ZK_F32, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_gemm_f16(16, 16, 16, 8, 8, 8, 8, 8, 8, 0, L.ZK_F16, None, None, 0, 0, None),
     L.ZK_ERR_UNSUPPORTED),
    (lambda lib: lib.zk_gemm_f16(16, 16, 16, 8, 8, 12, 12, 12, 8, 1, L.ZK_F16, None, None, 0, 0, None),
     L.ZK_ERR_UNSUPPORTED),  # K not a multiple of 8
    (lambda lib: lib.zk_gemm_f16(16, 16, 16, 8, 8, 8, 4, 8, 8, 1, L.ZK_F16, None, None, 0, 0, None),
     L.ZK_ERR_INVALID),  # lda < K
    (lambda lib: lib.zk_gemm_f16(16, 16, 16, 8, 8, 8, 8, 8, 8, 1, L.ZK_F16, None, None, 0, 1, None),
     L.ZK_ERR_INVALID),  # bias epilogue without bias
    (lambda lib: lib.zk_gemm_i8(16, 16, 16, 8, 8, 16, 16, 16, 8, 1.0, None, None, None, 0, 1,
                                L.ZK_I32, None), L.ZK_ERR_INVALID),  # int32 out + epilogue
    (lambda lib: lib.zk_gemm_i8(16, 16, 16, 8, 8, 16, 16, 16, 8, 1.0, None, None, None, 0, 0,
                                L.ZK_F16, None), L.ZK_ERR_INVALID),  # dequant without s_w
    (lambda lib: lib.zk_flash_attn_fwd(16, 16, 16, 16, 1, 1, 8, 8, 136, L.strides_arg([0] * 12),
                                       None, 0.125, L.ZK_F16, None), L.ZK_ERR_UNSUPPORTED),
    (lambda lib: lib.zk_flash_attn_fwd(16, 16, 16, 16, 1, 1, 8, 8, 129, L.strides_arg([0] * 12),
                                       None, 0.125, L.ZK_F32, None), L.ZK_ERR_UNSUPPORTED),
    (lambda lib: lib.zk_flash_attn_fwd(16, 16, 16, 16, 1, 1, 8, 8, 20, L.strides_arg([0] * 12),
                                       None, 0.125, L.ZK_F16, None),
     L.ZK_ERR_UNSUPPORTED),  # fp16 head_dim not a multiple of 8
    (lambda lib: lib.zk_gemm_f16(16, 16, 16, 8, 8, 8, 1 << 23, 8, 8, 1, L.ZK_F16, None, None, 0, 0,
                                 None), L.ZK_ERR_UNSUPPORTED),  # A tile span beyond 31 bits
    (lambda lib: lib.zk_gemm_f16(16, 16, 16, 8, 8, 8, 8, 1 << 23, 8, 1, L.ZK_F16, None, None, 0, 0,
                                 None), L.ZK_ERR_UNSUPPORTED),  # W tile span beyond 31 bits
    (lambda lib: lib.zk_gemm_i8(16, 16, 16, 8, 8, 131072, 131072, 131072, 8, 1.0, None, None, None,
                                0, 0, L.ZK_I32, None), L.ZK_ERR_UNSUPPORTED),  # 128^2 K = 2^31
    (lambda lib: lib.zk_gemm_i8(16, 16, 16, 8, 8, 16, 1 << 24, 16, 8, 1.0, None, None, None, 0, 0,
                                L.ZK_I32, None), L.ZK_ERR_UNSUPPORTED),  # int8 span
    (lambda lib: lib.zk_gemm_i8_requant(16, 16, 16, 8, 8, 16, 16, 1 << 24, 8, 1.0, 16, None, 0,
                                        1.0, None), L.ZK_ERR_UNSUPPORTED),  # int8 span (W)
    (lambda lib: lib.zk_qkv_attn_f16(16, 16, 16, 16, 2, 96, 768, 12, None, 0.125, None),
     L.ZK_ERR_UNSUPPORTED),  # fused QKV + attention: seq 64 or 128 only
    (lambda lib: lib.zk_qkv_attn_f16(16, 16, 16, 16, 2, 128, 768, 6, None, 0.125, None),
     L.ZK_ERR_UNSUPPORTED),  # head dim 128
    (lambda lib: lib.zk_qkv_attn_f16(16, None, 16, 16, 2, 128, 768, 12, None, 0.125, None),
     L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_qkv_attn_f16(16, 16, 16, 16, 2, 128, 768, 12, None, 0.0, None),
     L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_qkv_attn_f16(16, 16, 16, 16, -1, 128, 768, 12, None, 0.125, None),
     L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_qkv_attn_f16(16, 16, 16, 12, 2, 128, 768, 12, None, 0.125, None),
     L.ZK_ERR_UNSUPPORTED),  # ctx not 8-byte aligned
    (lambda lib: lib.zk_gemm_f16_res_stats(16, 16, 16, 8, 64, 64, 64, 64, 64, 16, 16, 64, None,
                                           None, None, 16, None),
     L.ZK_ERR_UNSUPPORTED),  # N not a multiple of the 96-column statistics segment
    (lambda lib: lib.zk_gemm_f16_res_stats(16, 16, 16, 8, 96, 64, 64, 64, 96, 16, 16, 96, 16,
                                           None, None, 16, None),
     L.ZK_ERR_INVALID),  # residual LayerNorm without gamma / beta
    (lambda lib: lib.zk_gemm_f16_res_stats(16, 16, 16, 8, 96, 64, 64, 64, 96, 16, 16, 96, None,
                                           None, None, None, None),
     L.ZK_ERR_INVALID),  # no statistics output
    (lambda lib: lib.zk_gemm_f16_ln(16, 16, 16, 8, 64, 96, 96, 96, 64, 16, 1e-12, 16, 16, None,
                                    L.ZK_EPI_BIAS_RELU, None), L.ZK_ERR_UNSUPPORTED),
    (lambda lib: lib.zk_gemm_f16_ln(16, 16, 16, 8, 64, 64, 64, 64, 64, 16, 1e-12, 16, 16, None,
                                    L.ZK_EPI_BIAS, None), L.ZK_ERR_UNSUPPORTED),  # K % 96
    (lambda lib: lib.zk_gemm_f16_ln(16, 16, 16, 8, 64, 1632, 1632, 1632, 64, 16, 1e-12, 16, 16,
                                    None, L.ZK_EPI_BIAS, None), L.ZK_ERR_UNSUPPORTED),  # K > 1536
    (lambda lib: lib.zk_gemm_f16_ln(16, 16, 16, 8, 64, 96, 96, 96, 64, None, 1e-12, 16, 16, None,
                                    L.ZK_EPI_BIAS, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_gemm_f16_ln(16, 16, 16, 8, 64, 96, 96, 96, 64, 16, -1.0, 16, 16, None,
                                    L.ZK_EPI_BIAS, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_qkv_attn_f16_ln(16, 16, None, 1e-12, 16, 16, None, 16, 2, 128, 768, 12,
                                        None, 0.125, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_qkv_attn_f16_ln(16, 16, 16, 1e-12, None, 16, None, 16, 2, 128, 768, 12,
                                        None, 0.125, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_gemm_i8_res_stats(16, 16, 16, 8, 64, 64, 64, 64, 64, 1.0, 16, 16, 16, 64,
                                          None, None, None, 16, None),
     L.ZK_ERR_UNSUPPORTED),  # N not a multiple of the 96-column statistics segment
    (lambda lib: lib.zk_gemm_i8_res_stats(16, 16, 16, 8, 96, 64, 64, 64, 96, 1.0, None, 16, 16,
                                          96, None, None, None, 16, None),
     L.ZK_ERR_INVALID),  # no weight scales
    (lambda lib: lib.zk_gemm_i8_res_stats(16, 16, 16, 8, 96, 72, 72, 72, 96, 1.0, 16, 16, 16, 96,
                                          None, None, None, 16, None),
     L.ZK_ERR_UNSUPPORTED),  # int8 K % 16
    (lambda lib: lib.zk_gemm_i8_res_stats(16, 16, 16, 8, 96, 64, 64, 64, 96, 1.0, 16, 16, None,
                                          96, None, None, None, 16, None),
     L.ZK_ERR_INVALID),  # no residual
    (lambda lib: lib.zk_gemm_f16_res_stats_frag(16, 16, 16, 8, 96, 96, 96, 96, 16, 16, 96, None,
                                                None, None, 16, None),
     L.ZK_ERR_UNSUPPORTED),  # fragment-ordered A: K a multiple of 64
    (lambda lib: lib.zk_gemm_f16_ln_frag(16, 16, 16, 8, 96, 96, 96, 96, 16, 1e-12, 16, 16, None,
                                         None), L.ZK_ERR_UNSUPPORTED),  # N a multiple of 64
    (lambda lib: lib.zk_gemm_i8_requant_frag(16, 16, 16, 8, 64, 64, 64, 64, 1.0, 16, 16, 2, 1.0,
                                             None), L.ZK_ERR_UNSUPPORTED),  # N % 128
    (lambda lib: lib.zk_gemm_f16_frag(16, 16, 16, 8, 96, 96, 96, 96, 16, None),
     L.ZK_ERR_UNSUPPORTED),  # fragment-ordered A: K a multiple of 64
    (lambda lib: lib.zk_gemm_f16_frag(16, 16, 16, 8, 96, 128, 128, 96, None, None),
     L.ZK_ERR_INVALID),  # no bias
    (lambda lib: lib.zk_qkv_attn_f16_frag(16, 16, 16, None, 1e-12, None, None, None, 8, 2, 128,
                                          768, 12, None, 0.125, None),
     L.ZK_ERR_UNSUPPORTED),  # fragment-ordered ctx must be 16-byte aligned
    (lambda lib: lib.zk_gemm_i8_res_stats_frag(16, 16, 16, 8, 96, 64, 64, 96, 1.0, 16, 16, 16, 96,
                                               None, None, None, 16, None),
     L.ZK_ERR_UNSUPPORTED),  # fragment-ordered int8 A: K % 128
    (lambda lib: lib.zk_layernorm_q8_res_ln(16, 16, None, 16, 16, 16, 16, 16, 16, 4, 8, 1e-12,
                                            0.1, None), L.ZK_ERR_INVALID),  # no residual stats
    (lambda lib: lib.zk_layernorm_q8_res_ln(16, 16, 16, 16, 16, 16, 16, 16, 16, 4, 8, 1e-12,
                                            0.0, None), L.ZK_ERR_INVALID),  # q_scale
    (lambda lib: lib.zk_layernorm_q8_res_ln(16, 16, 12, 16, 16, 16, 16, 16, 16, 4, 8, 1e-12,
                                            0.1, None), L.ZK_ERR_UNSUPPORTED),  # res_ln alignment
    (lambda lib: lib.zk_layernorm_add(16, None, 16, 16, 16, 4, 8, 1e-5, L.ZK_F32, None),
     L.ZK_ERR_INVALID),  # LayerNormAdd needs its residual
    (lambda lib: lib.zk_layernorm_add(16, 16, 16, 16, 16, 4, 8, 1e-5, L.ZK_I8, None),
     L.ZK_ERR_UNSUPPORTED),
    (lambda lib: lib.zk_flash_attn_fwd(16, 16, 16, 16, 1, 1, 8, 8, 64, L.strides_arg([0] * 12),
                                       None, -1.0, L.ZK_F16, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_quantize_i8(16, 16, 4, 0.0, L.ZK_F32, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_transpose_f16(16, 16, 4, 8, 4, 4, None), L.ZK_ERR_INVALID),
    (lambda lib: lib.zk_linear_f32(16, 16, 16, 8, 8, 8, 8, 8, 8, None, None, 0, 1, None, 0, None),
     L.ZK_ERR_INVALID),  # bias epilogue without bias
    (lambda lib: lib.zk_linear_f32(16, 16, 16, 8, 8, 8, 8, 8, 8, 16, None, 0, 4, None, 0, None),
     L.ZK_ERR_INVALID),  # residual epilogue without residual
    (lambda lib: lib.zk_linear_f32(16, 16, 16, 8, 8, 8, 8, 8, 8, 16, None, 0, 9, None, 0, None),
     L.ZK_ERR_INVALID),  # unknown epilogue
    (lambda lib: lib.zk_linear_f32(16, 16, 16, 8, 8, 8, 4, 8, 8, None, None, 0, 0, None, 0, None),
     L.ZK_ERR_INVALID),  # ldx < K
    (lambda lib: lib.zk_gemm_f16_add_ln(16, 16, 16, 16, 16, 16, None, 16, 8, 8, 8, 8, 8, 1e-12,
                                        None, 0, None), L.ZK_ERR_INVALID),  # no product buffer
    (lambda lib: lib.zk_gemm_f16_add_ln(16, 16, None, 16, 16, 16, 16, 16, 8, 8, 8, 8, 8, 1e-12,
                                        None, 0, None), L.ZK_ERR_INVALID),  # no bias
    (lambda lib: lib.zk_gemm_f16_add_ln(16, 16, 16, 16, 16, 16, 16, 16, 8, 8, 8, 8, 8, -1.0,
                                        None, 0, None), L.ZK_ERR_INVALID),  # eps
    (lambda lib: lib.zk_gemm_f16_add_ln(16, 16, 16, 16, 16, 16, 16, 16, 8, 8, 8, 4, 8, 1e-12,
                                        None, 0, None), L.ZK_ERR_INVALID),  # lda < K
    (lambda lib: lib.zk_gemm_f16_add_ln(16, 16, 16, 16, 16, 16, 16, 16, 8, 8, 12, 12, 12, 1e-12,
                                        None, 0, None), L.ZK_ERR_UNSUPPORTED),  # K % 8
    (lambda lib: lib.zk_gemm_f16_add_ln(16, 16, 16, 16, 16, 16, 16, 16, 8, 8, 8, 8, 8, 1e-12,
                                        None, -1, None), L.ZK_ERR_INVALID),  # workspace size
])
def test_argument_errors(call, code):
    lib = L.load()
    assert call(lib) == code
    assert L.last_error()


def test_zero_sized_calls_are_noops():
    lib = L.load()
    assert lib.zk_relu(None, None, 0, L.ZK_F32, None) == L.ZK_OK
    assert lib.zk_gemm_f16(None, None, None, 0, 8, 8, 8, 8, 8, 1, L.ZK_F16, None, None, 0, 0, None) == L.ZK_OK
    assert lib.zk_layernorm(None, None, None, None, None, 0, 768, 1e-5, L.ZK_F16, None) == L.ZK_OK


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not found"):
        L.load(str(tmp_path / "nope.so"))


def test_call_raises_with_message():
    with pytest.raises(RuntimeError, match="zk_relu"):
        L.call("zk_relu", None, None, -1, L.ZK_F32, None)


def test_c_types_are_plain():
    # no torch / C++ types in the ABI: every argument is a pointer or scalar
    for name, args in L.SIGNATURES.items():
        for a in args:
            assert a in (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float) or \
                a is ctypes.POINTER(ctypes.c_int64), (name, a)


def test_gemm_workspace_plan():
    """Split-K workspace sizes: small-M products are split (fp32 partials of
    M x N per split), large ones are not; pure host logic, no GPU."""
    from zenith_amd import _lib as L

    lib = L.load()
    ws = lib.zk_gemm_workspace_size(128, 768, 3072, L.ZK_F32)
    assert ws > 0 and ws % (128 * 768 * 4) == 0 and 2 <= ws // (128 * 768 * 4) <= 16
    assert lib.zk_gemm_workspace_size(4096, 768, 3072, L.ZK_F32) == 0
    assert lib.zk_gemm_workspace_size(4096, 3072, 768, L.ZK_F16) == 0
    assert lib.zk_gemm_workspace_size(64, 64, 64, L.ZK_F16) == 0  # too few K slices
    assert lib.zk_gemm_workspace_size(0, 768, 768, L.ZK_F32) == 0
    # fp16 FFN-down of one and of four 128-token sequences: 24 and 96 tiles of
    # 64 x 64; K = 3072 is 48 slices, deep enough for up to two workgroups per
    # CU at >= 12 slices each (4 splits at M = 512), shallow products keep at
    # most one per CU (the out-projection at M = 512: 2 splits)
    part = lambda M, N: M * N * 4  # noqa: E731
    assert lib.zk_gemm_workspace_size(128, 768, 3072, L.ZK_F16) == 10 * part(128, 768)
    assert lib.zk_gemm_workspace_size(512, 768, 3072, L.ZK_F16) == 4 * part(512, 768)
    assert lib.zk_gemm_workspace_size(512, 768, 768, L.ZK_F16) == 2 * part(512, 768)
    # the largest plan stays within the allocation-free entry point's 8 MiB
    worst = max(lib.zk_gemm_workspace_size(M, N, K, dt) for M in (64, 128, 320, 512, 960)
                for N in (64, 768, 1024, 3072) for K in (768, 3072, 16384)
                for dt in (L.ZK_F16, L.ZK_F32))
    assert 0 < worst <= 8 << 20

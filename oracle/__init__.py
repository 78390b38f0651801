"""CPU oracle for the zenith_amd BERT-encoder kernel set.

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import, call, link or execute anything in this package,
and only as the checker (or the timed CPU baseline) - never as a code path of
the product. zenith_amd never imports it.

Contents:
  ops.py        numpy restatement of the reference CPU path (GEMM, GELU,
                LayerNorm / Add+LayerNorm, masked attention, int8 quantise,
                int32 GEMM, MinMax calibration), each citing the reference.
  bert.py       the post-LN BERT layer / encoder composed from ops.py.
  cpu_gemm.c    C restatement of the reference's AVX2 fp32 GEMM
                (core/src/cpu_kernels.cpp:108-181) -> libzk_oracle.so.
  native.py     ctypes access to libzk_oracle.so and, when built, to
                oracle/_ref/ (the reference's own cpu_kernels.cpp and
                features_bindings.hpp compiled by `make ref`).

How each function is pinned (golden vectors, reference build, closed forms)
is in tests/test_oracle.py; a function with no such check is marked
"parity unpinned" there.
"""

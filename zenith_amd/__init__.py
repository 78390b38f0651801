"""zenith_amd: MI355X (gfx950) implementation of ZENITH's transformer-inference
kernel set (`zenith_cuda`) and the graph hooks that call it.

    from zenith_amd import zenith_cuda        # relu, gelu, layernorm, matmul,
                                              # flash_attention, wmma_matmul, ...
    from zenith_amd.encoder import BertEncoder

The kernels are hand-written HIP for gfx950 in zenith_amd/csrc, built into
libzenith_hip.so (C ABI: include/zk_api.h) and bound with ctypes.
"""

from ._build import LIB_PATH  # noqa: F401

__version__ = "0.1.0"


def load_library():
    """Load libzenith_hip.so (raises RuntimeError if it is not built)."""
    from . import _lib

    return _lib.load()

"""Import-name shim: `import zenith_cuda` resolves to the MI355X kernel module
(zenith_amd.zenith_cuda), so code written against the reference's torch
extension (core/bindings/cuda_bindings.cpp:134-145) runs unchanged when this
repository is on sys.path."""

from zenith_amd.zenith_cuda import *  # noqa: F401,F403
from zenith_amd.zenith_cuda import __all__  # noqa: F401

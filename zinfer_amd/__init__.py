"""zinfer_amd: MI355X (gfx950) sampling and constrained-decoding path for zinfer.

The product is the C ABI library libzinfer_hip.so (include/zinfer_hip.h):
hand-written HIP kernels plus a host mirror of zinfer's Zig Sampler API.
The Python modules only bind it for tests and the benchmark.
"""
from ._lib import LIB_PATH, ZiError, lib, params  # noqa: F401

__version__ = "0.1.0"

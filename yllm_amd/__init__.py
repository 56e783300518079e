"""yllm_amd -- MI355X (gfx950) attention hot path for the yllm engine.

The product is libyllm_hip.so (C ABI: include/yllm_hip.h), built in-tree by
yllm_amd.build.  This package is the Python host mirror used by the tests and
the benchmark.
"""
from ._lib import BF16, F16, F32, LIB_PATH, YhipError, lib  # noqa: F401

__all__ = ["lib", "LIB_PATH", "YhipError", "F16", "F32", "BF16"]

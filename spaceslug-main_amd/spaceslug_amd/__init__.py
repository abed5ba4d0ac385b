"""Host-side mirror of Spaceslug's native backend session for the MI355X int4 path.

The reference host (python/spaceslug/backend.py:44-67) binds its runtime
library with ctypes; BackendSession here does the same against
libspaceslug_runtime.so (HIP kernels for gfx950 + the C-ABI declared in
include/runtime_abi.h).
"""
from .backend import BackendError, BackendSession, ExecutionResult, Q4Chain, Q4Step, Q4Weight, library_path
from .parity import compare_float_arrays

__all__ = ["BackendError", "BackendSession", "ExecutionResult", "Q4Chain", "Q4Step", "Q4Weight",
           "compare_float_arrays", "library_path"]

"""MI355X-native backend for RustingStrata's quantized-matmul hot path (HIP for gfx950 behind a C ABI)."""
from . import ggml  # noqa: F401
from .backend import (ACT_ADD, ACT_STORE, ACT_SWIGLU, GEMM_BM, NUM_Q8_32, NUM_Q8K, SAME_X, SMALL_TILES, X_Q, Buf,  # noqa: F401
                      GpuTensor, HipBackend, StrataError, lib, quantize_rows)

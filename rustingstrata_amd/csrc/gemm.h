// Prefill GEMM over tile lists on int8 MFMA (Backend::gemm / gemm_dense, src/backend.rs:187-197).
#pragma once
#include "common.h"

namespace strata {

// The GEMM's X is quantized with quant_xq's layout under Q8_K numerics (one scale per 256 values: the super-block
// accumulates in int32, see gemm.hip).
inline uint64_t gemm_x_bytes(uint64_t cols, uint64_t n_x) { return n_x * (cols + cols / 8); }
hipError_t launch_gemm_quant_x(const float* x, uint64_t x_stride, int cols, int n_x, uint8_t* out, int mode, hipStream_t s);

struct GemmLaunch {
    int ty = 0;
    int rows = 0, cols = 0;
    const uint64_t* tiles = nullptr;  // [w, m0 | cnt << 32] per tile, or null for one dense matrix
    int n_tiles = 0;                  // tiles (or dense tiles of gemm_block_positions()); an upper bound with n_tiles_dev
    const int* n_tiles_dev = nullptr;
    const uint8_t* dense_w = nullptr;
    int dense_n = 0;
    const uint8_t* xq = nullptr;      // quantized X, n_x rows
    int n_x = 0;
    const int* xrow = nullptr;
    float* y = nullptr;
    int64_t y_stride = 0;
    int act = 0;
    // pair: a block's 128 weight rows are 64 rows of the tile's matrix and the same 64 rows of the matrix w2 bytes
    // further (gate and up), and it stores y = silu(first) * second for those 64 columns (rows % 64 == 0, y rows
    // 16-byte aligned)
    bool pair = false;
    int64_t w2 = 0;
    // tiles of a few dozen positions: the 64-position kernel with two steps of loads in flight (gemm_small.hip)
    bool small = false;
};
hipError_t launch_gemm(const GemmLaunch& g, hipStream_t s);
hipError_t launch_gemm_small(const GemmLaunch& g, hipStream_t s);
// Positions of one GEMM block (a tile list's chunks of this size give every block a full tile).
uint64_t gemm_block_positions();

}  // namespace strata

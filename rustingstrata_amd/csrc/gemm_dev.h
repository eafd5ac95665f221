// Device-side pieces shared by the int8 MFMA GEMM kernels (gemm.hip: 256-position blocks; gemm_small.hip:
// 64-position blocks for tile lists of a few dozen positions per tile).
#pragma once
#include <type_traits>

#include "dec16.h"
#include "gemm.h"
#include "kernels.h"

namespace strata {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int NXCD = 8;              // MI355X: 8 XCDs, each with its own L2
template <int T> struct GemmPlanes {
    static constexpr bool MIN = Dec<T>::MIN;
    static constexpr bool HI = T != Q2_K;                         // Q2_K's sc * q <= 45 fits the LO plane
    static constexpr int NP = (HI ? 2 : 1) + (MIN ? 1 : 0);        // planes
    static constexpr int NCH0 = (sb_bytes(T) + 15 + 15) / 16;     // 16-byte chunks covering a super-block at any offset
    static constexpr int NCH = NCH0 | 1;                           // odd: rows of the raw tile start in spread banks
    static constexpr int RAWP = 16 * NCH;                          // LDS pitch of a raw weight row
};

struct GemmArgs {
    const uint64_t* tiles;
    const int* n_tiles_dev;
    const uint8_t* dense_w;
    int dense_n;
    const int8_t* xq;     // n_x rows of cols int8
    const float* xd;      // then n_x rows of cols / 32 scales (8 equal ones per 256)
    const int* xrow;
    float* y;
    int64_t y_stride;
    int rows, cols, act;
    uint64_t rb;
    int max_tiles;        // tiles in the grid (an upper bound when the count is on the device)
    int yvec;             // y 16-byte aligned with a row stride of a multiple of 4 floats
    int gx;               // blocks per XCD
    int pair;             // gate/up pair mode (GemmLaunch::pair)
    int64_t w2;           // pair: byte offset of the second matrix
    int dense_p;          // dense: positions per tile (GM, or less to give every CU an item)
    int bal;              // tile lists: an item's fixed cost in 16-position tiles, 0..47 (< 0: split by count)
};

// silu(v) = v / (1 + e^-v) for the SwiGLU epilogues. e^-v = 2^t with t = -v log2(e) carried as th + tl (the
// product's rounding error and the tail of log2(e) in tl): 2^th by v_exp_f32 and 2^tl as 1 + tl ln 2. Within a few ulp
// of the correctly rounded value over the whole range (e^-v overflowing to inf gives -0, as silu's limit); the 4K
// MoE layer's outputs stay within 2e-6 of the CPU's with it (the requantized SwiGLU rows almost never change).
__device__ __forceinline__ float silu_dev(float v) {
    constexpr float L = 1.44269504088896341f, LLO = 1.9259630335e-08f, LN2 = 0.693147180559945f;
    const float x = -v, th = x * L, tl = __builtin_fmaf(x, L, -th) + x * LLO;
    const float e = __builtin_amdgcn_exp2f(th) * __builtin_fmaf(tl, LN2, 1.0f);
    return v * __builtin_amdgcn_rcpf(1.0f + e);
}


// f(std::integral_constant<int, I>) for I = B .. E - 1: the index is a constant expression in the body, so register
// arrays indexed by it stay in registers.
template <int B, int E, typename Fn>
__device__ __forceinline__ void static_for(Fn&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

}  // namespace strata

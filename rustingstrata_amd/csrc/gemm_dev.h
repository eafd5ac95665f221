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

// ---- the order of a tile list's items ----
// Items are (tile, row block) pairs, item = tile * nrb + row block. Item (tile t, row block r) costs c_t = bal + b_t,
// b_t = ceil(min(cnt_t, 256) / 16) the tile's MFMA position tiles (its bucket) and bal the weight decode in those
// units. A block of NWV waves plans its items at the start, one thread a tile (lists of up to 64 NWV tiles), in `sh`
// (PLAN_INTS ints of LDS that the block writes next only after a barrier).
//   1. Range x of nx takes the items whose cost midpoint falls in [x C / nx, (x + 1) C / nx), C = nrb sum c_t: a
//      contiguous range [ia, ib) (with one range per XCD, a tile's row blocks and an expert's tiles share its L2);
//      item r of tile t lies before range x iff nx (2 nrb P_t + 2 r c_t + c_t) < 2 x C, P_t the cost of the tiles
//      before t.
//   2. The range's items are ordered by bucket, larger first (a bucket's tiles and a tile's row blocks in index
//      order), and dealt to the range's gx blocks in a snake: block jb takes order positions q = k gx + jb for even k
//      and k gx + gx - 1 - jb for odd k, so the last items the blocks run are the cheapest.
// Every block of a range derives the same order from the tile list alone (no atomics, no timing), so the blocks'
// shares partition the range. Returns the block's item count with item k in lane k of `mine`, or -1 (the caller then
// deals [ia, ib) in index order) when a block would take more than 64 items. Every tile of the range has nrb items
// but the first and the last, which the range may cut. The block has 64 NWV threads and every one of them calls.
constexpr int NBK = 17;  // buckets 0 .. 16
constexpr int PLAN_INTS = 32 + 2 * 8 * NBK + 2 * NBK + 64;  // the plan's LDS ints (in `sh`)

// a / b for 0 <= a < 2^22, 0 < b < 2^10 through a float quotient and one correction step
__device__ __forceinline__ int div_small(int a, int b) {
    int q = (int)((float)a * __builtin_amdgcn_rcpf((float)b));
    if (q * b > a) q--;
    else if ((q + 1) * b <= a) q++;
    return q;
}

// The tile sizes go into `cnt` (thread t: tile t's count) before the list's length is known: `cap` slots are
// readable, the first ntiles of them tiles.
__device__ __forceinline__ int plan_load(const uint64_t* tiles, int cap) {
    const int tid = threadIdx.x;
    return tid < cap ? (int)((const uint32_t*)tiles)[4 * tid + 3] : 0;
}
template <int NWV>
__device__ __forceinline__ int plan_items(int cnt, int ntiles, int nrb, int bal, int nx, int x, int jb, int gx, int* sh,
                                          int& ia, int& ib, int& mine) {
    static_assert(NWV == 8, "the plan's per-wave LDS slots are sized for 8 waves");
    constexpr int NW = NWV;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const bool valid = tid < ntiles;
    const int bkt = valid ? (min(256, cnt) + 15) >> 4 : -1;
    const int ct = valid ? bal + bkt : 0;
    int* wsum = sh;          // [NW] the waves' cost sums
    int* full = sh + 8;      // [2][NW] the waves' tiles wholly before each boundary
    int* part = sh + 24;     // [2] the items of the tile a boundary cuts, before it
    int* tab = sh + 32;      // [NW][NBK] a wave's items of each bucket
    int* etab = tab + 8 * NBK;   // [NW][NBK] their sums over the earlier waves
    int* tot = etab + 8 * NBK;   // [NBK] the range's items of each bucket
    int* sbk = tot + NBK;        // [NBK] a bucket's first order position (the items of the larger buckets)
    int* list = sbk + NBK;       // [64] the block's items
    // 1. block prefix of the costs (c_t < 64: bit planes through ballots, the waves' sums through LDS), and the range
    int P = 0, wt = 0;
#pragma unroll
    for (int j = 0; j < 6; j++) {
        const uint64_t m = __ballot((ct >> j) & 1);
        P += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u)) << j;
        wt += (int)__popcll(m) << j;
    }
    if (lane == 0) wsum[w] = wt;
    if (tid < 2) part[tid] = 0;
    __syncthreads();
    int csum = 0;
#pragma unroll
    for (int v = 0; v < NW; v++) {
        const int s = wsum[v];
        csum += s;
        if (v < w) P += s;
    }
    const long long C = (long long)csum * nrb;
    const long long base = (long long)nx * (2LL * nrb * P + ct), u = 2LL * nx * ct;
    // the r in [0, nrb) with base + u r < R: none, all, or (the one tile the boundary cuts) a division
    auto before = [&](long long R) __attribute__((always_inline)) {
        if (!valid || R <= base) return 0;
        if (R > base + u * (nrb - 1)) return nrb;
        return (int)(((uint32_t)(R - base) + (uint32_t)u - 1u) / (uint32_t)u);
    };
    const int b0 = before(2LL * x * C), b1 = before(2LL * (x + 1) * C);  // (b1 = nrb throughout for the last range)
    const uint64_t f0 = __ballot(b0 == nrb), f1 = __ballot(b1 == nrb);
    if (lane == 0) {
        full[w] = (int)__popcll(f0);
        full[NW + w] = (int)__popcll(f1);
    }
    if (b0 > 0 && b0 < nrb) part[0] = b0;
    if (b1 > 0 && b1 < nrb) part[1] = b1;
    __syncthreads();
    int n0 = 0, n1 = 0;
#pragma unroll
    for (int v = 0; v < NW; v++) {
        n0 += full[v];
        n1 += full[NW + v];
    }
    ia = n0 * nrb + part[0];
    ib = n1 * nrb + part[1];
    const int n = ib - ia;
    if (n <= 0) return 0;
    if ((n + gx - 1) / gx > 64) return -1;
    // 2. each range tile's first order position: the buckets above its own, its bucket's items in earlier waves and
    // in earlier lanes of its wave
    const int ta = ia / nrb, tb = (ib - 1) / nrb;
    const int na = min(ib, (ta + 1) * nrb) - ia, nb = ib - max(ia, tb * nrb);
    const bool inr = valid && tid >= ta && tid <= tb;
    const int bt = inr ? bkt : -1;
    const int bta = __shfl(bt, ta & 63), btb = __shfl(bt, tb & 63);  // (meaningful in the waves of ta and tb)
    const bool wa = w == (ta >> 6), wb = w == (tb >> 6) && tb != ta;
    uint64_t mm = 0;
    int wcnt = 0;
#pragma unroll
    for (int b = 0; b < NBK; b++) {
        const uint64_t m = __ballot(bt == b);
        if (bt == b) mm = m;
        if (lane == b) wcnt = (int)__popcll(m) * nrb - (wa && bta == b ? nrb - na : 0) - (wb && btb == b ? nrb - nb : 0);
    }
    if (lane < NBK) tab[w * NBK + lane] = wcnt;
    const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mm, 0u));
    const int pre = below * nrb - (wa && bta == bt && ta < tid ? nrb - na : 0);
    __syncthreads();
    if (tid < NW * NBK) {
        const int v0 = tid / NBK, b = tid - v0 * NBK;
        int e = 0;
#pragma unroll
        for (int v = 0; v < NW - 1; v++) e += v < v0 ? tab[v * NBK + b] : 0;
        etab[tid] = e;
        if (v0 == NW - 1) tot[b] = e + tab[tid];
    }
    __syncthreads();
    if (tid < NBK) {
        int e = 0;
#pragma unroll
        for (int b = 1; b < NBK; b++) e += b > tid ? tot[b] : 0;
        sbk[tid] = e;
    }
    __syncthreads();
    if (inr) {
        const int R = sbk[bt] + etab[w * NBK + bt] + pre;
        const int nt = min(ib, (tid + 1) * nrb) - max(ia, tid * nrb), f = max(ia, tid * nrb);
        // the block's order positions in [R, R + nt): q_k increases with k, q_k in [k gx, k gx + gx)
        for (int k = max(div_small(R, gx) - 1, 0); k < 64 && k * gx < R + nt; k++) {
            const int q = k * gx + ((k & 1) ? gx - 1 - jb : jb);
            if (q >= R && q < R + nt) list[k] = f + (q - R);
        }
    }
    __syncthreads();
    const int q = lane * gx + ((lane & 1) ? gx - 1 - jb : jb);
    mine = q < n ? list[lane] : 0;
    return (int)__popcll(__ballot(q < n));
}

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

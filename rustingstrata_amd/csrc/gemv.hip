// Decode GEMV for the quantized types: y = W x for 1..4 inputs (gemv / gemvn / gemvq / gemvq2) and the MoE form
// (moe_gemv: one expert matrix and x row per slot).
//
// A block of 256 threads (4 wave64) computes R consecutive rows. It streams the rows' contiguous byte span from
// HBM with 16-byte coalesced loads (any block alignment: the span is read from its 16-byte-aligned cover) into
// LDS, together with the quantized x (int8 + per-32 scales, plus per-16 sums computed on the way in) and, for the
// IQ types, the codebook tables. A row is then shared by G lanes (G = the power of two at or above its number of
// 256-value super-blocks, at most 64): lane l takes super-blocks l, l + G, ... whole, accumulating each exactly in
// int32 and closing it with one float step (sbdot.h); the G partial sums meet by cross-lane reduction.
#include <algorithm>

#include "sbdot.h"
#include "kernels.h"
#include "xlane.h"
#include "route.h"
#include "../../include/strata_hip.h"

namespace strata {

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_CH = 6;                              // 16-byte chunks per thread per tile
constexpr int GEMV_TILE = GEMV_THREADS * 16 * GEMV_CH;               // 24 KB of weights per block
uint64_t gemv_max_row_bytes() { return GEMV_TILE - 32; }

struct GemvArgs {
    const uint8_t* w;
    int64_t w2;          // byte offset of the paired matrix (blockIdx.z == 1)
    float* y;
    int64_t y2;          // byte offset of the paired output
    const int8_t* xq;    // n_xrows rows of cols int8
    const float* xd;     // then their per-32 scales
    const int* ids;      // moe: expert of each slot (blockIdx.y), or null
    int64_t stride;      // moe: bytes between experts
    int xg;              // moe: slots per x row
    int rows, rows2, cols, R, nt, y_stride;
    uint64_t rb;
    int per32;           // x has per-32 scales (STRATA_NUM_Q8_32), else one per 256 (STRATA_NUM_Q8K)
    int G;               // lanes per row: the power of two at or above the row's super-blocks, at most 64
    int ntr, nslots, nz; // row tiles per matrix, slots (moe) and matrices (pair)
    const float* xf;     // single-input kernel: x as f32 (quantized in-lane) when xq is null
    const float* xu;     // with xf: x = silu(xf) * xu, rows x_stride floats apart (swiglu_q fused), or null
    uint64_t x_stride;   // floats between the f32 x rows
    uint32_t ntr_m, ns_m; // magic multipliers and shifts dividing by ntr and nslots (fdiv)
    int ntr_s, ns_s;
    int small;           // single-input kernel, one plain matrix: every tile spans at most GEMV1_CH_SMALL chunks a thread
    int quarter;         // single-input kernel: every tile fits one pass of a wave (at most 64 / G rows), and the four
                         // waves each take one quarter of every super-block (sb_quarter / sb_close)
    // single-input moe kernel that routes its one token first (MODE bit 3): every block ranks the rn logits at rp
    // (route_block4) and takes slot j's expert from its own result; block 0 also stores ids, wts, slots (= ids
    // above) and wh, as route_block_kernel does
    const float* rp;
    const int* rtable;
    int* rids;
    float* rwts;
    float* rwh;
    float rscale;
    int rn, rsig;
    // single-input plain kernel with the norm prologue (MODE bit 5): x (xf) is first h = rms_norm(x + nres + sum_j
    // nwh[j] nye[j]) * nw (rms_norm_q_kernel's one-round-trip arithmetic, combine slots in order), the GEMV then
    // runs on h; block 0 writes x + nres + the combine to nxw (when not null; never xf itself: other blocks read it)
    const float* nw;
    const float* nres;
    const float* nye;
    const float* nwh;
    float* nxw;
    float neps;
    int nck;
};

// LDS layout: [IqTables (IQ types)][x int8: nt * cols][x scales: nt * cols / 32 f32][x sums: nt * cols / 16
// int32][weight tile], each section rounded up to 16 bytes.
__host__ __device__ constexpr uint32_t up16(uint32_t v) { return (v + 15) & ~15u; }

// Sum over the g lanes of each aligned lane group (g a power of two <= 64).
// v of lane i + (CTRL's source offset) within the 16-lane row, 0 where the source leaves the row (DPP).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
// Sum over aligned groups of g lanes (g a power of two), complete in the group's first lane: in-row steps by DPP
// (xor 1, xor 2 by quad permutes, then + lane i + 4, + lane i + 8), wider ones by lane permutes. The additions pair
// the same values in the same order as an xor butterfly.
// The row's super-block terms (lane p of a group of g holds term p) added in super-block order, as the CPU dots'
// running sum does (src/cpu_moe.rs:319-377: sumf = 0, then sumf += each super-block's term); the sum is valid at the
// group's last lane. Within a row of 16 lanes: g - 1 steps s = f + (s of the lane below) (row_shr:1), so after them
// lane g - 1 holds f_{g-1} + (... + (f_1 + f_0)). Wider groups add the lanes' terms one by one through shuffles.
// Terms are first made +0 from -0, as the CPU's sum starts from +0.
template <int G>
__device__ __forceinline__ float ordered_sum_row(float f) {
    float s = f;
#pragma unroll
    for (int k = 1; k < G; k++) s = f + dpp_f<0x111>(s);  // row_shr:1
    return s;
}
// The same fold over the 64 lanes of a wave continued from a running sum: ((run + f_0) + f_1) + ... + f_63, in every
// lane (rows of more than 64 super-blocks: lane l holds super-block 64 p + l of pass p).
__device__ __forceinline__ float ordered_sum_from(float run, float v) {
    const float f = v + 0.0f;
    float s = run;
    for (int j = 0; j < 64; j++) s = s + __shfl(f, j);
    return s;
}
__device__ __forceinline__ float ordered_sum(float v, int g) {
    const float f = v + 0.0f;
    float s = f;
    if (g == 8) {  // 2048 columns, the common case: one straight chain
        s = ordered_sum_row<8>(f);
    } else if (g == 4) {
        s = ordered_sum_row<4>(f);
    } else if (g == 2) {
        s = ordered_sum_row<2>(f);
    } else if (g == 16) {
        s = ordered_sum_row<16>(f);
    } else if (g > 16) {
        const int base = (threadIdx.x & 63) & ~(g - 1);
        s = 0.0f;
        for (int j = 0; j < g; j++) s = s + __shfl(f, base + j);
    }
    return s;
}

template <int T, int NT, bool Q32>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_kernel(GemvArgs a) {
    constexpr bool IQ = T == IQ2_XXS || T == IQ3_S;
    constexpr int SBB = sb_bytes(T);
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, cols = a.cols;
    // LDS: [IqTables][x int8][x scales][x sums][weight tile]
    uint8_t* p = smem;
    IqTables* tab = (IqTables*)p;
    if constexpr (IQ) { load_iq_tables(tab); p += up16(sizeof(IqTables)); }
    int8_t* sx = (int8_t*)p;
    p += up16(NT * cols);
    float* sd = (float*)p;
    p += up16(NT * (cols / 32) * 4);
    int* ss = (int*)p;
    p += up16(NT * (cols / 16) * 4);
    uint8_t* tile = p;

    // Tiles: t -> (z, slot, row tile); block b takes tiles b, b + grid, ... and prefetches the next one into
    // registers while it computes the current one from LDS.
    const int total = a.ntr * a.nslots * a.nz;
    auto valid = [&](int t) {
        const int rt = t % a.ntr, rest = t / a.ntr, slot = rest % a.nslots, z = rest / a.nslots;
        if (rt * a.R >= (z ? a.rows2 : a.rows)) return false;
        return !a.ids || a.ids[slot] >= 0;  // a slot not routed here leaves its output untouched
    };
    auto next_valid = [&](int t) {
        while (t < total && !valid(t)) t += gridDim.x;
        return t;
    };
    struct Span { const uint8_t* W; float* Y; int r0, nr, xrow; uint64_t beg, g0; int nch; };
    auto span = [&](int t) {
        Span sp;
        const int rt = t % a.ntr, rest = t / a.ntr, slot = rest % a.nslots, z = rest / a.nslots;
        const int rows = z ? a.rows2 : a.rows;
        sp.r0 = rt * a.R;
        sp.nr = min(a.R, rows - sp.r0);
        sp.W = a.w + (z ? a.w2 : 0);
        sp.Y = (float*)((uint8_t*)a.y + (z ? a.y2 : 0));
        sp.xrow = 0;
        if (a.ids) {
            sp.W += (int64_t)a.ids[slot] * a.stride;
            sp.xrow = slot / a.xg;
            sp.Y += (int64_t)slot * rows;
        }
        sp.beg = (uint64_t)(sp.W + (uint64_t)sp.r0 * a.rb);
        sp.g0 = sp.beg & ~(uint64_t)15;
        sp.nch = (int)((((sp.beg + (uint64_t)sp.nr * a.rb) + 15) & ~(uint64_t)15) - sp.g0) >> 4;
        return sp;
    };
    v4u wv[GEMV_CH];
    auto issue = [&](const Span& sp) {
#pragma unroll
        for (int i = 0; i < GEMV_CH; i++) {
            const int c = tid + GEMV_THREADS * i;
            if (c < sp.nch) wv[i] = __builtin_nontemporal_load(gptr<v4u>(sp.g0 + 16 * (uint64_t)c));
        }
    };

    int t = next_valid(blockIdx.x);
    if (t >= total) return;
    Span sp = span(t);
    issue(sp);
    int cur_xrow = -1;
    const int G = a.G, wave = tid >> 6, lane = tid & 63, gl = lane & (G - 1);
    const int RPW = 64 / G, nsb = (cols + 255) >> 8;
    while (true) {
        __syncthreads();  // the previous tile's readers are done with the LDS tile (and x)
        if (sp.xrow != cur_xrow) {
            // x (int8 + scales, per-16 sums) of this tile's input row(s)
            for (int c = tid; c < NT * cols / 16; c += GEMV_THREADS) {
                const int u = c / (cols / 16), j = c % (cols / 16);
                const v4u q = *gptr<v4u>((uint64_t)(a.xq + (uint64_t)(sp.xrow + u) * cols + 16 * j));
                *(v4u*)(sx + 16 * c) = q;
                ss[c] = sdot4((int)q.x, 0x01010101, sdot4((int)q.y, 0x01010101, sdot4((int)q.z, 0x01010101, sdot4((int)q.w, 0x01010101, 0))));
            }
            for (int c = tid; c < NT * cols / 32; c += GEMV_THREADS) {
                const int u = c / (cols / 32), j = c % (cols / 32);
                sd[c] = *gptr<float>((uint64_t)(a.xd + (uint64_t)(sp.xrow + u) * (cols / 32) + j));
            }
            cur_xrow = sp.xrow;
        }
#pragma unroll
        for (int i = 0; i < GEMV_CH; i++) {
            const int c = tid + GEMV_THREADS * i;
            if (c < sp.nch) *(v4u*)(tile + 16 * c) = wv[i];
        }
        __syncthreads();
        const Span cs = sp;
        const int tn = next_valid(t + gridDim.x);
        if (tn < total) {
            sp = span(tn);
            issue(sp);  // in flight while this tile is computed
        }
        // Rows: G lanes each (64 / G rows per wave per pass), whole super-blocks per lane.
        for (int base = wave * RPW; base < cs.nr; base += 4 * RPW) {
            const int rr = base + lane / G;
            float acc[NT];
#pragma unroll
            for (int u = 0; u < NT; u++) acc[u] = 0.0f;
            // passes of G super-blocks, one a lane; a row of more than 64 (G = 64) takes several, the running sum
            // carried from pass to pass so the terms still meet in super-block order
            for (int p0 = 0; p0 < nsb; p0 += G) {
                const int sb = p0 + gl;
                float f[NT];
#pragma unroll
                for (int u = 0; u < NT; u++) f[u] = 0.0f;
                if (rr < cs.nr && sb < nsb) {
                    const uint8_t* rowp = tile + (cs.beg - cs.g0) + (uint64_t)rr * a.rb;
#pragma unroll
                    for (int u = 0; u < NT; u++) {
                        const XLds xv{sx + u * cols + 256 * sb, sd + u * (cols / 32) + 8 * sb, ss + u * (cols / 16) + 16 * sb};
                        const int nv = min(256, cols - 256 * sb);
                        f[u] = Q32 ? sb_dot_q32<T>(rowp + sb * SBB, xv, tab, nv) : sb_dot_q8k<T>(rowp + sb * SBB, xv, tab, nv);
                    }
                }
#pragma unroll
                for (int u = 0; u < NT; u++) acc[u] = p0 == 0 ? ordered_sum(f[u], G) : ordered_sum_from(acc[u], f[u]);
            }
            if (rr < cs.nr && gl == G - 1) {
#pragma unroll
                for (int u = 0; u < NT; u++) cs.Y[(int64_t)u * a.y_stride + cs.r0 + rr] = acc[u];
            }
        }
        if (tn >= total) break;
        t = tn;
    }
}

// The persistent grid: as many blocks as stay resident together (the kernel's occupancy at this LDS size), at most
// one per tile. Cached per (kernel, LDS size).
// ---- single-input GEMV with x in registers ----
// Every lane of a row group always takes the same super-block (lane l of a group of G: super-block l), so it keeps
// that 256-value slice of x in registers for the whole launch (reloaded only when a MoE tile switches x rows) and
// LDS carries nothing but the weight tiles. x arrives pre-quantized (xq) or as f32, quantized by each lane for its
// own slice with quant_xq's arithmetic (the same bits).
constexpr int GEMV1_CH = 12;
constexpr int GEMV1_WAVES = 4;          // waves of a single-input GEMV block
constexpr int GEMV1_THREADS = 64 * GEMV1_WAVES;
constexpr int GEMV1_TILE = GEMV1_THREADS * 16 * GEMV1_CH;
// 16-byte loads a thread of a full tile of one plain matrix, per type (the MoE and pair forms keep GEMV1_CH; lm-head
// rows 151936 x 2048 in the sweep, % of HBM peak with 10 /
// 12 / 14: Q4_K 72.8 / 70.1 / 67.3, Q5_K 74.3 / 69.4 / 68.9, Q6_K 67.2 / 68.5 / 71.4, Q8_0 75.9 / 77.7 / 78.6,
// Q3_K 43.8 / 42.6 / 40.8, Q2_K 48.4 / 49.6 / 47.5)
__host__ __device__ constexpr int gemv1_ch(int T) { return T == Q4_K || T == Q5_K || T == Q3_K ? 10 : T == Q6_K ? 14 : GEMV1_CH; }
constexpr int GEMV1_CH_SMALL = 5;  // (one plain matrix whose tiles span at most 20 KB: only the loads it needs)

// Quantize x row xr (n values) into LDS (n int8, then n / 32 scales) with quant_xq's arithmetic (quant.hip): the
// block's 256 threads take 8 values each, a group of 32 lanes one 256-value block.
// This thread's 8 values v (positions i.., zeros past n) of one 2048-value chunk, quantized into LDS.
// The staged x in LDS: value i at xpad(i) (16 bytes of padding after every 256, so the lanes of a wave reading
// different super-blocks' slices hit different banks), the per-32 scales, and the per-16 sums of the int8 values.
__device__ __forceinline__ int xpad(int i) { return i + 16 * (i >> 8); }
__host__ __device__ constexpr uint32_t xpad_bytes(uint32_t ncp) { return ncp + ncp / 16; }

template <bool Q32>
__device__ __forceinline__ void quant8_lds(const float (&v)[8], int i, bool live, int8_t* q, float* d, int* ss) {
    {
        float dd, mul;
        if constexpr (!Q32) {
            float bv = v[0];
            int bi = i;
#pragma unroll
            for (int j = 1; j < 8; j++) if (fabsf(v[j]) > fabsf(bv)) { bv = v[j]; bi = i + j; }
            // the first value of largest magnitude over the 32 lanes: the choice is unique, so the pairing of the
            // exchange steps does not matter
            auto step = [&](auto S) __attribute__((always_inline)) {
                constexpr int st = decltype(S)::value;
                const float ov = xl32f<st>(bv);
                const int oi = xl32<st>(bi);
                if (fabsf(ov) > fabsf(bv) || (fabsf(ov) == fabsf(bv) && oi < bi)) { bv = ov; bi = oi; }
            };
            step(std::integral_constant<int, 0>{});
            step(std::integral_constant<int, 1>{});
            step(std::integral_constant<int, 2>{});
            step(std::integral_constant<int, 3>{});
            step(std::integral_constant<int, 4>{});
            const float is = bv != 0.0f ? -127.0f / bv : 0.0f;
            dd = bv != 0.0f ? 1.0f / is : 0.0f;
            mul = is;
        } else {
            float mx = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) mx = fmaxf(mx, fabsf(v[j]));
            mx = fmaxf(mx, xl32f<0>(mx));
            mx = fmaxf(mx, xl32f<1>(mx));
            dd = mx / 127.0f;
            mul = mx > 0.0f ? 127.0f / mx : 0.0f;
        }
        uint32_t w[2] = {0, 0};
#pragma unroll
        for (int j = 0; j < 8; j++) w[j >> 2] |= (uint32_t)((int)fminf(__builtin_rintf(mul * v[j]), 127.0f) & 255) << (8 * (j & 3));
        // the 16-value group's sum: this lane's 8 and its neighbour's (lane ^ 1)
        int s8 = sdot4((int)w[0], 0x01010101, sdot4((int)w[1], 0x01010101, 0));
        s8 += xl32<0>(s8);
        if (live) {
            *(uint2*)(q + xpad(i)) = make_uint2(w[0], w[1]);
            if ((threadIdx.x & 3) == 0) d[i >> 5] = dd;
            if ((threadIdx.x & 1) == 0) ss[i >> 4] = s8;
        }
    }
}

typedef float v4f __attribute__((ext_vector_type(4)));
template <bool Q32, bool SW>
__device__ __forceinline__ void quant_row_lds(uint64_t xr, uint64_t ur, int n, int8_t* q, float* d, int* ss) {
    for (int c0 = 0; c0 < n; c0 += 8 * (int)blockDim.x) {
        const int i = c0 + threadIdx.x * 8;
        const bool live = i < n;
        float v[8];
        if (live) {
            const v4f p = *gptr<v4f>(xr + 4 * (uint64_t)i), r = *gptr<v4f>(xr + 4 * (uint64_t)i + 16);
            v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w; v[4] = r.x; v[5] = r.y; v[6] = r.z; v[7] = r.w;
            if constexpr (SW) {
                const v4f pu = *gptr<v4f>(ur + 4 * (uint64_t)i), ru = *gptr<v4f>(ur + 4 * (uint64_t)i + 16);
                const float u[8] = {pu.x, pu.y, pu.z, pu.w, ru.x, ru.y, ru.z, ru.w};
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = silu_f32(v[j]) * u[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = 0.0f;
        }
        quant8_lds<Q32>(v, i, live, q, d, ss);
    }
}

// x row xrow into the block's LDS copy (int8, then per-32 scales): copied from xq, or quantized from f32.
template <bool Q32, bool SW>
__device__ __forceinline__ void stage_x(const GemvArgs& a, int xrow, int8_t* xl, float* xld, int* xss) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    if (a.xq) {
        const uint64_t q = (uint64_t)(a.xq + (uint64_t)xrow * a.cols), d = (uint64_t)(a.xd + (uint64_t)xrow * (a.cols / 32));
        for (int c = threadIdx.x; c < a.cols / 16; c += blockDim.x) {
            const v4u t = *gptr<v4u>(q + 16 * c);
            *(v4u*)(xl + xpad(16 * c)) = t;
            xss[c] = sdot4((int)t.x, 0x01010101, sdot4((int)t.y, 0x01010101, sdot4((int)t.z, 0x01010101, sdot4((int)t.w, 0x01010101, 0))));
        }
        for (int c = threadIdx.x; c < a.cols / 32; c += blockDim.x) xld[c] = *gptr<float>(d + 4 * c);
    } else {
        quant_row_lds<Q32, SW>((uint64_t)(a.xf + (uint64_t)xrow * a.x_stride),
                               SW ? (uint64_t)(a.xu + (uint64_t)xrow * a.x_stride) : 0, a.cols, xl, xld, xss);
    }
    // zeros up to whole super-blocks (Q8_0 rows may end inside one)
    const int n = a.cols, nup = (n + 255) & ~255;
    for (int i = n + 4 * threadIdx.x; i < nup; i += 4 * blockDim.x) *(uint32_t*)(xl + xpad(i)) = 0;
    for (int j = n / 32 + threadIdx.x; j < nup / 32; j += blockDim.x) xld[j] = 0.0f;
    for (int j = n / 16 + threadIdx.x; j < nup / 16; j += blockDim.x) xss[j] = 0;
}

// The first tile's x row when it has at most 4096 values, requested before the tile's weights so that its arrival
// and quantization overlap the weights' flight: (f32 x) this thread's 8 values of each half (XH values); (xq) its
// 16-byte chunk and scale.
constexpr int XH = 8 * GEMV1_THREADS;  // values of one half of an early x row
constexpr int NORM_SLOTS = 8;  // combine slots the norm prologue takes
struct XEarly {
    v4f f0, f1, u0, u1, f2, f3;
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    v4u q;
    float d;
    // norm prologue: this thread's 8 values of res and nw, and of each combine slot, with the slots' weights
    v4f r0, r1, w0, w1, y0[NORM_SLOTS], y1[NORM_SLOTS];
    float ws[NORM_SLOTS];
};
template <bool SW, bool NORM = false>
__device__ __forceinline__ void x_fetch(const GemvArgs& a, int xrow, XEarly& e) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const int tid = threadIdx.x;
    if constexpr (NORM) {
        // one row of at most 2048 values: thread tid's values 8 tid .. 8 tid + 7, as rms_norm_q_kernel holds them
        if (8 * tid < a.cols) {
            const uint64_t o = 32 * (uint64_t)tid;
            e.f0 = *gptr<v4f>((uint64_t)a.xf + o);
            e.f1 = *gptr<v4f>((uint64_t)a.xf + o + 16);
            e.w0 = *gptr<v4f>((uint64_t)a.nw + o);
            e.w1 = *gptr<v4f>((uint64_t)a.nw + o + 16);
            if (a.nres) {
                e.r0 = *gptr<v4f>((uint64_t)a.nres + o);
                e.r1 = *gptr<v4f>((uint64_t)a.nres + o + 16);
            }
#pragma unroll
            for (int u = 0; u < NORM_SLOTS; u++) {
                e.ws[u] = u < a.nck ? a.nwh[u] : 0.0f;
                if (u < a.nck) {
                    const uint64_t yr = (uint64_t)(a.nye + (uint64_t)u * a.cols) + o;
                    e.y0[u] = *gptr<v4f>(yr);
                    e.y1[u] = *gptr<v4f>(yr + 16);
                }
            }
        }
        return;
    }
    if (a.xq) {
        if (tid < a.cols / 16) e.q = *gptr<v4u>((uint64_t)(a.xq + (uint64_t)xrow * a.cols) + 16 * tid);
        if (tid < a.cols / 32) e.d = *gptr<float>((uint64_t)(a.xd + (uint64_t)xrow * (a.cols / 32)) + 4 * tid);
    } else if (8 * tid < a.cols) {
        const uint64_t xr = (uint64_t)(a.xf + (uint64_t)xrow * a.x_stride) + 32 * (uint64_t)tid;
        e.f0 = *gptr<v4f>(xr);
        e.f1 = *gptr<v4f>(xr + 16);
        if constexpr (SW) {
            const uint64_t ur = (uint64_t)(a.xu + (uint64_t)xrow * a.x_stride) + 32 * (uint64_t)tid;
            e.u0 = *gptr<v4f>(ur);
            e.u1 = *gptr<v4f>(ur + 16);
        }
        // (the SwiGLU input takes the early path for its first half only: its second half's registers would be
        // live across the weight loads of a kernel already at 256 VGPRs)
        if constexpr (!SW)
            if (XH + 8 * tid < a.cols) {
                e.f2 = *gptr<v4f>(xr + 4 * XH);
                e.f3 = *gptr<v4f>(xr + 4 * XH + 16);
            }
    }
}
template <bool Q32, bool SW, bool NORM = false>
__device__ __forceinline__ void x_put(const GemvArgs& a, const XEarly& e, int8_t* xl, float* xld, int* xss,
                                      float* npart = nullptr) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const int tid = threadIdx.x, n = a.cols;
    if constexpr (NORM) {
        // rms_norm_q_kernel's one-round-trip path, operation for operation: x + res, then the combine's products
        // added in slot order (a slot of weight 0 adds nothing), the per-thread sum of squares, the DPP sum within
        // 32 lanes, the 8 half-waves in order; then h = v * scale * nw, quantized as quant_xq does
        const int i = 8 * tid;
        const bool live = i < n;
        float v[8], wn[8];
        if (live) {
            const float xv[8] = {e.f0.x, e.f0.y, e.f0.z, e.f0.w, e.f1.x, e.f1.y, e.f1.z, e.f1.w};
            const float wv[8] = {e.w0.x, e.w0.y, e.w0.z, e.w0.w, e.w1.x, e.w1.y, e.w1.z, e.w1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) { v[j] = xv[j]; wn[j] = wv[j]; }
            if (a.nres) {
                const float rv[8] = {e.r0.x, e.r0.y, e.r0.z, e.r0.w, e.r1.x, e.r1.y, e.r1.z, e.r1.w};
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = v[j] + rv[j];
            }
            if (a.nck) {
                float y[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int u = 0; u < NORM_SLOTS; u++) {
                    if (e.ws[u] != 0.0f) {
                        const float yv[8] = {e.y0[u].x, e.y0[u].y, e.y0[u].z, e.y0[u].w,
                                             e.y1[u].x, e.y1[u].y, e.y1[u].z, e.y1[u].w};
#pragma unroll
                        for (int q = 0; q < 8; q++) y[q] += e.ws[u] * yv[q];
                    }
                }
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = v[j] + y[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = wn[j] = 0.0f;
        }
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) s += v[j] * v[j];
        s += xl32f<0>(s);
        s += xl32f<1>(s);
        s += xl32f<2>(s);
        s += xl32f<3>(s);
        s += xl32f<4>(s);
        if ((tid & 31) == 0) npart[tid >> 5] = s;
        if (blockIdx.x == 0 && a.nxw && live) {
            *(float4*)(a.nxw + i) = make_float4(v[0], v[1], v[2], v[3]);
            *(float4*)(a.nxw + i + 4) = make_float4(v[4], v[5], v[6], v[7]);
        }
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int h = 0; h < 8; h++) tot += npart[h];
        const float sc = 1.0f / sqrtf(tot / (float)n + a.neps);
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = live ? v[j] * sc * wn[j] : 0.0f;
        quant8_lds<Q32>(v, i, live, xl, xld, xss);
        return;
    }
    if (a.xq) {
        if (tid < n / 16) {
            *(v4u*)(xl + xpad(16 * tid)) = e.q;
            xss[tid] = sdot4((int)e.q.x, 0x01010101, sdot4((int)e.q.y, 0x01010101, sdot4((int)e.q.z, 0x01010101, sdot4((int)e.q.w, 0x01010101, 0))));
        }
        if (tid < n / 32) xld[tid] = e.d;
    } else {
        // each half of XH values present: every thread takes 8 values of it
#pragma unroll
        for (int h = 0; h < (SW ? 1 : 2); h++) {
            if (XH * h < n) {
                const int i = XH * h + 8 * tid;
                const bool live = i < n;
                const v4f a0 = h ? e.f2 : e.f0, a1 = h ? e.f3 : e.f1;
                float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                if constexpr (SW) {
                    const v4f b0 = e.u0, b1 = e.u1;
                    const float u[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
                    for (int j = 0; j < 8; j++) v[j] = silu_f32(v[j]) * u[j];
                }
                if (!live) {
#pragma unroll
                    for (int j = 0; j < 8; j++) v[j] = 0.0f;
                }
                quant8_lds<Q32>(v, i, live, xl, xld, xss);
            }
        }
    }
    const int nup = (n + 255) & ~255;
    for (int i = n + 4 * tid; i < nup; i += 4 * blockDim.x) *(uint32_t*)(xl + xpad(i)) = 0;
    for (int j = n / 32 + tid; j < nup / 32; j += blockDim.x) xld[j] = 0.0f;
    for (int j = n / 16 + tid; j < nup / 16; j += blockDim.x) xss[j] = 0;
}

// This lane's 256-value slice (super-block sb) of the staged x into registers, with its per-16 sums.
__device__ __forceinline__ void load_x_slice(int sb, const int8_t* xl, const float* xld, const int* xss, XReg& x) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int c = 0; c < 16; c++) {
        const v4u t = *(const v4u*)(xl + 272 * sb + 16 * c);
        x.w[4 * c] = t.x; x.w[4 * c + 1] = t.y; x.w[4 * c + 2] = t.z; x.w[4 * c + 3] = t.w;
    }
#pragma unroll
    for (int j = 0; j < 8; j++) x.ds[j] = xld[8 * sb + j];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const v4u t = *(const v4u*)(xss + 16 * sb + 4 * c);
        x.sums[4 * c] = (int)t.x; x.sums[4 * c + 1] = (int)t.y; x.sums[4 * c + 2] = (int)t.z; x.sums[4 * c + 3] = (int)t.w;
    }
}


// SW: x rows are silu(xf) * xu (the fused SwiGLU input of the down projection); a separate instantiation, so the
// plain GEMV carries none of it.
// n / d for 0 <= n < 2^31 and d >= 1, from m and s of magic(d) (Granlund and Montgomery, "Division by invariant
// integers using multiplication", 1994: s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1).
__device__ __forceinline__ int fdiv(int n, uint32_t m, int s) { return (int)((__umulhi((uint32_t)n, m) + (uint32_t)n) >> s); }
static void magic(uint32_t d, uint32_t& m, int& s) {
    s = 0;
    while ((1ull << s) < d) s++;
    m = (uint32_t)((((1ull << s) - d) << 32) / d + 1);
}

// MODE: bit 0 SW (x rows are silu(xf) * xu), bit 1 the quarter split (GemvArgs::quarter), bit 2 one plain matrix
// (no expert ids, no pair: tile t is row tile t and every tile is valid, with none of the general indexing's
// divisions, tens of instructions each), bit 3 the routing prologue (GemvArgs::rp), bit 4 small tiles
// (GemvArgs::small: GEMV1_CH_SMALL loads a thread, a smaller LDS tile).
template <int T, bool Q32, int MODE>
__global__ __launch_bounds__(GEMV1_THREADS) void gemv1_kernel(GemvArgs a) {
    constexpr bool SW = MODE & 1, QU = MODE & 2, plain = MODE & 4, ROUTE = MODE & 8, NORM = MODE & 32;
    static_assert(!NORM || (plain && !SW && !ROUTE), "the norm prologue is for one plain matrix");
    constexpr int CH = (MODE & 16) ? GEMV1_CH_SMALL : plain ? gemv1_ch(T) : GEMV1_CH, TILE = GEMV1_THREADS * 16 * CH;
    constexpr bool IQ = T == IQ2_XXS || T == IQ3_S;
    constexpr int SBB = sb_bytes(T);
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, cols = a.cols;
    // LDS: [IqTables][x int8 (whole super-blocks, padded: xpad)][x scales][x per-16 sums][tile]
    const uint32_t ncp = (cols + 255) & ~255;
    const uint32_t o_x = IQ ? up16(sizeof(IqTables)) : 0u, o_xd = o_x + xpad_bytes(ncp), o_ss = o_xd + ncp / 8,
                   o_tile = o_ss + ncp / 4, o_part = o_tile + TILE + 16;
    int* xss = (int*)(smem + o_ss);
    IqTables* tab = (IqTables*)smem;
    static_assert(GEMV1_THREADS == 256, "load_iq_regs covers the tables with 256 threads");
    int8_t* xl = (int8_t*)(smem + o_x);
    float* xld = (float*)(smem + o_xd);
    uint8_t* tile = smem + o_tile;
    uint32_t* qpart = (uint32_t*)(smem + o_part);  // quarter split: waves 1-3's outputs, 2 words a lane

    const int total = a.ntr * a.nslots * a.nz;
    __shared__ RouteLds rl;  // (ROUTE) the routing's LDS; rl.tops[j]: slot j's expert
    auto expert = [&](int slot) {
        if constexpr (ROUTE) return rl.tops[slot];
        else return sload(a.ids + slot);
    };
    // one plain matrix (no slots, no pair, no expert ids): tile t is row tile t, and every tile is valid; the
    // divisions below (tens of instructions each) stay off that path
    auto valid = [&](int t) {
        if constexpr (plain) return true;
        const int rest = fdiv(t, a.ntr_m, a.ntr_s), rt = t - rest * a.ntr, z = fdiv(rest, a.ns_m, a.ns_s),
                  slot = rest - z * a.nslots;
        if (rt * a.R >= (z ? a.rows2 : a.rows)) return false;
        return !a.ids || expert(slot) >= 0;  // a slot not routed here leaves its output untouched
    };
    auto next_valid = [&](int t) {
        while (t < total && !valid(t)) t += gridDim.x;
        return t;
    };
    struct Span { float* Y; int r0, nr, xrow; uint64_t beg, g0; int nch; };
    auto span = [&](int t) {
        Span sp;
        if constexpr (plain) {
            sp.r0 = t * a.R;
            sp.nr = min(a.R, a.rows - sp.r0);
            sp.Y = a.y;
            sp.xrow = 0;
            sp.beg = (uint64_t)(a.w + (uint64_t)sp.r0 * a.rb);
        } else {
            const int rest = fdiv(t, a.ntr_m, a.ntr_s), rt = t - rest * a.ntr, z = fdiv(rest, a.ns_m, a.ns_s),
                      slot = rest - z * a.nslots;
            const int rows = z ? a.rows2 : a.rows;
            sp.r0 = rt * a.R;
            sp.nr = min(a.R, rows - sp.r0);
            const uint8_t* W = a.w + (z ? a.w2 : 0);
            sp.Y = (float*)((uint8_t*)a.y + (z ? a.y2 : 0));
            sp.xrow = 0;
            if (a.ids) {
                W += (int64_t)expert(slot) * a.stride;
                sp.xrow = slot / a.xg;
                sp.Y += (int64_t)slot * rows;
            }
            sp.beg = (uint64_t)(W + (uint64_t)sp.r0 * a.rb);
        }
        sp.g0 = sp.beg & ~(uint64_t)15;
        sp.nch = (int)((((sp.beg + (uint64_t)sp.nr * a.rb) + 15) & ~(uint64_t)15) - sp.g0) >> 4;
        return sp;
    };
    v4u wv[CH];
    // every lane loads every instruction (chunks past the span repeat its last chunk and land past the tile's bytes
    // in LDS), so no load or store sits under a branch and the LDS stores wait for their own loads only
    auto issue = [&](const Span& sp) {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int c = min(tid + GEMV1_THREADS * i, sp.nch - 1);
            wv[i] = __builtin_nontemporal_load(gptr<v4u>(sp.g0 + 16 * (uint64_t)c));
        }
    };

    const bool early = a.cols <= (SW ? 1 : 2) * XH;
    XEarly xe;
    if constexpr (ROUTE) {
        // the token's x (row 0) is requested before the routing, whose ranks then name the experts
        if (early) x_fetch<SW>(a, 0, xe);
        int id = 0, sl = -1;
        float w = 0.0f;
        route_block4(a.rp, a.rn, a.nslots, a.rscale, a.rtable, a.rsig, &rl, id, w, sl);
        // route_block4 leaves rank j's slot in rl.tops[j] (read after its closing barrier) and in thread j's sl
        if (blockIdx.x == 0 && tid < a.nslots) {
            a.rids[tid] = id;
            a.rwts[tid] = w;
            ((int*)a.ids)[tid] = sl;
            a.rwh[tid] = sl >= 0 ? w : 0.0f;
        }
    }
    int t = next_valid(blockIdx.x);
    if (t >= total) return;
    Span sp = span(t);
    if (!ROUTE && early) x_fetch<SW, NORM>(a, sp.xrow, xe);
    __shared__ float npart[NORM ? 8 : 1];  // the norm prologue's half-wave sums
    issue(sp);
    // the IQ codebooks into registers behind the first tile's loads (both round trips at once), into LDS before the
    // first tile is computed
    IqRegs iqr;
    if constexpr (IQ) iqr = load_iq_regs();
    // the tile after next is located while the next one is in flight
    int tn = next_valid(t + gridDim.x);
    Span spn = sp;
    if (tn < total) spn = span(tn);
    const int G = a.G, wave = tid >> 6, lane = tid & 63, gl = lane & (G - 1);
    const int RPW = 64 / G, nsb = (cols + 255) >> 8;
    const bool has_sb = gl < nsb;
    XReg x;
    int cur_xrow = -1;
    if constexpr (IQ) store_iq_regs(tab, iqr);  // visible after the barrier that ends the first tile's staging
    while (true) {
        __syncthreads();  // the previous tile's readers are done with the LDS tile
        if (sp.xrow != cur_xrow) {
            if (early && cur_xrow < 0) x_put<Q32, SW, NORM>(a, xe, xl, xld, xss, npart);
            else stage_x<Q32, SW>(a, sp.xrow, xl, xld, xss);
            __syncthreads();
            // every lane has its slice before the copy can change again: the next staging follows the loop's barrier
            if (has_sb && !QU) load_x_slice(gl, xl, xld, xss, x);
            cur_xrow = sp.xrow;
        }
#pragma unroll
        for (int i = 0; i < CH; i++)
            *(v4u*)(tile + 16 * (tid + GEMV1_THREADS * i)) = wv[i];
        __syncthreads();
        const Span cs = sp;
        const bool more = tn < total;
        if (more) {
            sp = spn;
            issue(sp);  // in flight while this tile is computed
            t = tn;
            tn = next_valid(t + gridDim.x);
            if (tn < total) spn = span(tn);
        }
        const int nv = min(256, cols - 256 * gl);
        if constexpr (QU) {
            // row lane / G of the tile, super-block gl, quarter `wave`; wave 0 closes the four quarters
            const int rr = lane / G;
            const bool live = rr < cs.nr && has_sb;
            uint32_t o0 = 0, o1 = 0;
            float D = 0.0f, M = 0.0f;
            if (live) {
                const uint8_t* b = tile + (cs.beg - cs.g0) + (uint64_t)rr * a.rb + gl * SBB;
                const XLds xv{xl + xpad(256 * gl), xld + 8 * gl, xss + 16 * gl};
                switch (wave) {
                case 0: sb_quarter<T, Q32, 0>(b, xv, tab, nv, o0, o1, D, M); break;
                case 1: sb_quarter<T, Q32, 1>(b, xv, tab, nv, o0, o1, D, M); break;
                case 2: sb_quarter<T, Q32, 2>(b, xv, tab, nv, o0, o1, D, M); break;
                default: sb_quarter<T, Q32, 3>(b, xv, tab, nv, o0, o1, D, M); break;
                }
            }
            if (wave) *(uint2*)(qpart + 128 * (wave - 1) + 2 * lane) = make_uint2(o0, o1);
            __syncthreads();
            if (wave == 0) {
                uint32_t o[8];
                o[0] = o0;
                o[1] = o1;
#pragma unroll
                for (int w = 1; w < 4; w++) {
                    const uint2 v = *(const uint2*)(qpart + 128 * (w - 1) + 2 * lane);
                    o[2 * w] = v.x;
                    o[2 * w + 1] = v.y;
                }
                float acc = live ? sb_close<T, Q32>(o, D, M, xld[8 * gl], nv) : 0.0f;
                acc = ordered_sum(acc, G);
                if (rr < cs.nr && gl == G - 1) cs.Y[cs.r0 + rr] = acc;
            }
            if (!more) break;
            continue;
        }
        for (int base = wave * RPW; base < cs.nr; base += GEMV1_WAVES * RPW) {
            const int rr = base + lane / G;
            float acc = 0.0f;
            if (rr < cs.nr && has_sb) {
                const uint8_t* b = tile + (cs.beg - cs.g0) + (uint64_t)rr * a.rb + gl * SBB;
                acc = Q32 ? sb_dot_q32<T>(b, x, tab, nv) : sb_dot_q8k<T>(b, x, tab, nv);
            }
            acc = ordered_sum(acc, G);
            if (rr < cs.nr && gl == G - 1) cs.Y[cs.r0 + rr] = acc;
        }
        if (!more) break;
    }
}


template <int T, bool Q32, int MODE>
static hipError_t gemv1_launch(const GemvArgs& a, long long tiles, size_t smem, hipStream_t s) {
    static int ncu = 0, per_cu = 0;
    static size_t cached_smem = 0;
    static size_t attr = 64 * 1024;  // dynamic LDS the kernel is set up for
    if (!ncu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
            ncu = 256;
    }
    // a wide row's x staging plus a full per-type tile can pass the default 64 KB of dynamic LDS (Q6_K at 16384
    // columns: ~82 KB); a CU has 160 KB
    if (smem > attr) {
        hipError_t e = hipFuncSetAttribute((const void*)gemv1_kernel<T, Q32, MODE>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
        attr = smem;
    }
    if (cached_smem != smem) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv1_kernel<T, Q32, MODE>, GEMV1_THREADS, smem) != hipSuccess || n < 1) n = 1;
        per_cu = n;
        cached_smem = smem;
    }
    long long blocks = (long long)per_cu * ncu;
    if (blocks > tiles) blocks = tiles;
    gemv1_kernel<T, Q32, MODE><<<dim3((unsigned)blocks), GEMV1_THREADS, smem, s>>>(a);
    return hipGetLastError();
}

template <int T>
static hipError_t gemv1_t(const GemvArgs& a, long long tiles, size_t smem, hipStream_t s) {
    const int mode = (a.xu ? 1 : 0) | (a.quarter ? 2 : 0) | (!a.xu && !a.ids && a.nz == 1 ? 4 : 0) | (a.rp ? 8 : 0) |
                     (a.small ? 16 : 0) | (a.nw ? 32 : 0);
    if (a.nw) {  // the norm prologue: one plain matrix, Q8_K numerics
        if (a.per32) return hipErrorNotSupported;
        switch (mode) {
        case 36: return gemv1_launch<T, false, 36>(a, tiles, smem, s);
        case 38: return gemv1_launch<T, false, 38>(a, tiles, smem, s);
        case 52: return gemv1_launch<T, false, 52>(a, tiles, smem, s);
        case 54: return gemv1_launch<T, false, 54>(a, tiles, smem, s);
        default: return hipErrorNotSupported;
        }
    }
    switch (mode) {
    case 20: return a.per32 ? gemv1_launch<T, true, 20>(a, tiles, smem, s) : gemv1_launch<T, false, 20>(a, tiles, smem, s);
    case 22: return a.per32 ? gemv1_launch<T, true, 22>(a, tiles, smem, s) : gemv1_launch<T, false, 22>(a, tiles, smem, s);
    case 8: return a.per32 ? gemv1_launch<T, true, 8>(a, tiles, smem, s) : gemv1_launch<T, false, 8>(a, tiles, smem, s);
    case 10: return a.per32 ? gemv1_launch<T, true, 10>(a, tiles, smem, s) : gemv1_launch<T, false, 10>(a, tiles, smem, s);
    case 0: return a.per32 ? gemv1_launch<T, true, 0>(a, tiles, smem, s) : gemv1_launch<T, false, 0>(a, tiles, smem, s);
    case 1: return a.per32 ? gemv1_launch<T, true, 1>(a, tiles, smem, s) : gemv1_launch<T, false, 1>(a, tiles, smem, s);
    case 2: return a.per32 ? gemv1_launch<T, true, 2>(a, tiles, smem, s) : gemv1_launch<T, false, 2>(a, tiles, smem, s);
    case 3: return a.per32 ? gemv1_launch<T, true, 3>(a, tiles, smem, s) : gemv1_launch<T, false, 3>(a, tiles, smem, s);
    case 4: return a.per32 ? gemv1_launch<T, true, 4>(a, tiles, smem, s) : gemv1_launch<T, false, 4>(a, tiles, smem, s);
    default: return a.per32 ? gemv1_launch<T, true, 6>(a, tiles, smem, s) : gemv1_launch<T, false, 6>(a, tiles, smem, s);
    }
}

template <int T, int NT, bool Q32>
static hipError_t gemv_nt(const GemvArgs& a, long long tiles, size_t smem, hipStream_t s) {
    static int ncu = 0;
    static size_t cached_smem = 0;
    static int per_cu = 0;
    if (!ncu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
            ncu = 256;
    }
    static size_t attr = 64 * 1024;  // dynamic LDS the kernel is set up for
    if (!attr) {  // wide rows (more than GEMV1_MAX_COLS values) stage more than 64 KB of x and tile
        if (hipFuncSetAttribute((const void*)gemv_kernel<T, NT, Q32>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
            return hipErrorInvalidValue;
        attr = true;
    }
    if (cached_smem != smem) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_kernel<T, NT, Q32>, GEMV_THREADS, smem) != hipSuccess || n < 1) n = 1;
        per_cu = n;
        cached_smem = smem;
    }
    long long blocks = (long long)per_cu * ncu;
    if (blocks > tiles) blocks = tiles;
    gemv_kernel<T, NT, Q32><<<dim3((unsigned)blocks), GEMV_THREADS, smem, s>>>(a);
    return hipGetLastError();
}

template <int T, bool Q32>
static hipError_t gemv_m(const GemvArgs& a, long long grid, size_t smem, hipStream_t s) {
    switch (a.nt) {
    case 1: return gemv_nt<T, 1, Q32>(a, grid, smem, s);
    case 2: return gemv_nt<T, 2, Q32>(a, grid, smem, s);
    case 3: return gemv_nt<T, 3, Q32>(a, grid, smem, s);
    case 4: return gemv_nt<T, 4, Q32>(a, grid, smem, s);
    }
    return hipErrorInvalidValue;
}

template <int T>
static hipError_t gemv_t(const GemvArgs& a, long long grid, size_t smem, hipStream_t s) {
    return a.per32 ? gemv_m<T, true>(a, grid, smem, s) : gemv_m<T, false>(a, grid, smem, s);
}

hipError_t launch_gemv(const GemvLaunch& g, hipStream_t s) {
    GemvArgs a{};
    a.w = g.w; a.w2 = g.pair ? g.w2 : 0; a.y = g.y; a.y2 = g.pair ? g.y2 : 0;
    a.xq = g.xq; a.xd = g.xq ? (const float*)(g.xq + (uint64_t)g.n_xrows * g.cols) : nullptr;
    a.xf = g.xf; a.xu = g.xu; a.x_stride = g.x_stride;
    a.ids = g.ids; a.stride = g.stride; a.xg = g.xg;
    a.rows = g.rows; a.rows2 = g.pair ? g.rows2 : 0; a.cols = g.cols; a.nt = g.nt; a.y_stride = g.y_stride;
    a.rb = row_bytes(g.ty, g.cols);
    a.per32 = g.numerics == STRATA_NUM_Q8_32;
    a.rp = g.rp; a.rtable = g.rtable; a.rids = g.rids; a.rwts = g.rwts; a.rwh = g.rwh; a.rscale = g.rscale;
    a.rn = g.rn; a.rsig = g.rsig;
    a.nw = g.nw; a.nres = g.nres; a.nye = g.nye; a.nwh = g.nwh; a.nxw = g.nxw; a.neps = g.neps; a.nck = g.nck;
    {
        int nsb = (g.cols + 255) / 256;
        a.G = 1;
        while (a.G < nsb && a.G < 64) a.G <<= 1;
    }
    static int ncu = 0;
    if (!ncu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
            ncu = 256;
    }
    const int maxrows = g.pair ? (g.rows > g.rows2 ? g.rows : g.rows2) : g.rows;
    const int nslots = g.ids ? g.k : 1, nz = g.pair ? 2 : 1;
    // Rows per tile: as many as fit the tile, but no fewer tiles than about 4 per CU.
    const bool single = g.nt == 1 && g.cols <= GEMV1_MAX_COLS;
    const bool plain1 = single && !g.xu && !g.ids && !g.pair;  // the kernel's one-plain-matrix instantiation
    const int rmax = (int)(((single ? GEMV1_THREADS * 16 * (plain1 ? gemv1_ch(g.ty) : GEMV1_CH) : GEMV_TILE) - 32) / a.rb);
    long long want = (long long)maxrows * nslots * nz / (4LL * ncu);
    a.R = (int)(want < 1 ? 1 : want > rmax ? rmax : want);
    if (a.R < 1) a.R = 1;
    const int rpb = (single ? GEMV1_WAVES : 4) * (64 / a.G);  // rows one pass of the block covers
    // A single-input tile covers at least one pass of the block (fewer, fuller blocks beat idle lanes: each block
    // also quantizes x itself), unless the matrix is so small that this would leave most CUs idle: then one tile per
    // CU (2048 rows of 2048 columns: 256 tiles of 8 rows, 0.3-0.6 us faster than 64 tiles of 32 rows).
    if (single && a.R < rpb) {
        const int fill = (int)std::max(1LL, (long long)maxrows * nslots * nz / ncu);
        a.R = 2 * fill <= rpb ? std::min(fill, rmax) : std::min(rpb, rmax);
    }
    if (single && a.R > rpb) a.R -= a.R % rpb;
    // x already quantized (no per-block quantization to amortize), or Q8_0 (whose per-32 float closes make a lane's
    // dot chain the longest), and one matrix: tiles of one wave pass (the quarter split) when they all fit one round of
    // blocks (Q6_K 5120 x 2048 from xq: 5.1 -> 4.7 us; 2048 x 4096: 4.9 -> 4.2 us; Q8_0 6144 x 2048: 6.9 -> 5.7 us)
    if (g.nw && !(single && plain1 && !g.xq && g.cols <= 2048 && g.cols % 8 == 0 && g.nck >= 0 &&
                  g.nck <= NORM_SLOTS && (g.nck == 0 || (g.nye && g.nwh)) && g.nxw != g.xf &&
                  (((uintptr_t)g.xf | (uintptr_t)g.nw | (uintptr_t)g.nres | (uintptr_t)g.nye | (uintptr_t)g.nxw) % 16) == 0))
        return hipErrorNotSupported;
    if (single && (g.xq || g.ty == Q8_0 || g.nw) && !g.ids && !g.pair && a.R > 64 / a.G &&
        (long long)(maxrows + 64 / a.G - 1) / (64 / a.G) <= 3LL * ncu)
        a.R = std::min(64 / a.G, rmax);
    a.ntr = (maxrows + a.R - 1) / a.R;
    a.nslots = nslots;
    a.nz = nz;
    magic((uint32_t)a.ntr, a.ntr_m, a.ntr_s);
    magic((uint32_t)a.nslots, a.ns_m, a.ns_s);
    const long long grid = (long long)a.ntr * nslots * nz;  // tiles
    if (g.rp && (!single || !g.ids || g.xu || g.k > 32 || g.k != g.xg || g.rn < g.k || g.rn > 128))
        return hipErrorNotSupported;
    bool iq = g.ty == IQ2_XXS || g.ty == IQ3_S;
    if (single) {
        const uint32_t ncp = (g.cols + 255) & ~255;
        a.quarter = a.R <= 64 / a.G;
        const uint64_t span_ch = ((uint64_t)a.R * a.rb + 15) / 16 + 1;  // 16-byte chunks a tile spans, at most
        a.small = !g.xu && !g.ids && !g.pair && span_ch <= (uint64_t)GEMV1_THREADS * GEMV1_CH_SMALL;
        const size_t smem1 = (iq ? up16(sizeof(IqTables)) : 0) + xpad_bytes(ncp) + ncp / 8 + ncp / 4 +
                             GEMV1_THREADS * 16 * (a.small ? GEMV1_CH_SMALL : plain1 ? gemv1_ch(g.ty) : GEMV1_CH) + 16 +
                             (a.quarter ? 3 * 64 * 8 : 0);
        switch (g.ty) {
        case Q8_0: return gemv1_t<Q8_0>(a, grid, smem1, s);
        case Q2_K: return gemv1_t<Q2_K>(a, grid, smem1, s);
        case Q3_K: return gemv1_t<Q3_K>(a, grid, smem1, s);
        case Q4_K: return gemv1_t<Q4_K>(a, grid, smem1, s);
        case Q5_K: return gemv1_t<Q5_K>(a, grid, smem1, s);
        case Q6_K: return gemv1_t<Q6_K>(a, grid, smem1, s);
        case IQ2_XXS: return gemv1_t<IQ2_XXS>(a, grid, smem1, s);
        case IQ3_S: return gemv1_t<IQ3_S>(a, grid, smem1, s);
        case IQ4_XS: return gemv1_t<IQ4_XS>(a, grid, smem1, s);
        }
        return hipErrorInvalidValue;
    }
    size_t smem = (iq ? up16(sizeof(IqTables)) : 0) + up16(g.nt * g.cols) + up16(g.nt * (g.cols / 32) * 4) +
                  up16(g.nt * (g.cols / 16) * 4) + GEMV_TILE + 16;
    switch (g.ty) {
    case Q8_0: return gemv_t<Q8_0>(a, grid, smem, s);
    case Q2_K: return gemv_t<Q2_K>(a, grid, smem, s);
    case Q3_K: return gemv_t<Q3_K>(a, grid, smem, s);
    case Q4_K: return gemv_t<Q4_K>(a, grid, smem, s);
    case Q5_K: return gemv_t<Q5_K>(a, grid, smem, s);
    case Q6_K: return gemv_t<Q6_K>(a, grid, smem, s);
    case IQ2_XXS: return gemv_t<IQ2_XXS>(a, grid, smem, s);
    case IQ3_S: return gemv_t<IQ3_S>(a, grid, smem, s);
    case IQ4_XS: return gemv_t<IQ4_XS>(a, grid, smem, s);
    }
    return hipErrorInvalidValue;
}

// ---- moe_down_combine in one launch ----
// Block (row block rb, token tk) of 1024 threads: rows r0 = rb R .. of all k slots of the token. Its 16 waves are 4
// groups of 4; group q takes pairs (slot, row) 16 q .. 16 q + 15 (64 / G pairs a wave pass, G lanes a pair, one
// super-block a lane) and its 4 waves one quarter each of every super-block (sb_quarter; the group's wave 0 closes
// them), so R = 4 (64 / G) / k rows. x of all k slots (quantized by quant_xq) is staged once per block as one
// flattened vector, every slot's rows padded like the single-input kernel's. Each
// (slot, row) dot lands in LDS and the first R threads then add the slots' weighted outputs to x in slot order,
// plus the shared expert, as combine_kernel does (src/cuda/kernels.cu:2742-2773).
constexpr int DC_THREADS = 1024;
struct DcArgs {
    const uint8_t* w;
    int64_t stride;       // bytes between experts
    const int* slots;     // t k expert slots (-1: not resident)
    const float* wh;      // t k combine weights
    const int8_t* xq;     // x pre-quantized (quant_xq layout of t k rows; row tk k + j for slot j of token tk)
    const float* xd;
    float* x;             // t rows of `rows` floats: x += combine
    const float* sh;      // shared expert output (t rows of `rows`) or null, gated by sigmoid(sg[tk]) when sg
    const float* sg;
    int rows, cols, k, R, G, nsb, nch;  // nch: 16-byte chunks a slot's span may take (its LDS pitch / 16)
    uint64_t rb;
    uint32_t nch_m;
    int nch_s;
};

__device__ __forceinline__ float dc_sigmoid(float v) { return 1.0f / (1.0f + (float)exp(-(double)v)); }

template <int T, bool Q32>
__global__ __launch_bounds__(DC_THREADS) void moe_down_combine_kernel(DcArgs a) {
    constexpr bool IQ = T == IQ2_XXS || T == IQ3_S;
    constexpr int SBB = sb_bytes(T);
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, tk = blockIdx.y;
    const int k = a.k, cols = a.cols, n = k * cols, R = a.R, G = a.G;
    const int r0 = blockIdx.x * R, nr = min(R, a.rows - r0);
    // LDS: [IqTables][x: n int8 (padded)][n / 32 scales][n / 16 sums][tile: k spans of 16 nch bytes][parts][ye]
    const uint32_t o_x = IQ ? up16(sizeof(IqTables)) : 0u, o_xd = o_x + xpad_bytes(n), o_ss = o_xd + n / 8,
                   o_tile = o_ss + n / 4, o_part = o_tile + 16 * a.nch * k, o_ye = o_part + 4 * 3 * 64 * 8,
                   o_sl = o_ye + 4 * k * R;
    IqTables* tab = (IqTables*)smem;
    if constexpr (IQ) load_iq_tables(tab);
    int8_t* xl = (int8_t*)(smem + o_x);
    float* xld = (float*)(smem + o_xd);
    int* xss = (int*)(smem + o_ss);
    uint8_t* tile = smem + o_tile;
    uint32_t* part = (uint32_t*)(smem + o_part);
    float* ye = (float*)(smem + o_ye);
    int* sslot = (int*)(smem + o_sl);
    float* swh = (float*)(sslot + k);

    // Requested first, none of them depending on anything of this launch: the token's slots and combine weights,
    // the combine's x and shared-expert values of this thread's row, and this thread's first chunk of x.
    if (tid < k) {
        sslot[tid] = a.slots[(uint64_t)tk * k + tid];
        swh[tid] = a.wh[(uint64_t)tk * k + tid];
    }
    const uint64_t orow = (uint64_t)tk * a.rows + r0 + tid;
    float xo = 0.0f, sho = 0.0f, sgv = 0.0f;
    if (tid < nr) {
        xo = a.x[orow];
        if (a.sh) sho = a.sh[orow];
        if (a.sg) sgv = a.sg[tk];
    }
    v4u xq0{};
    float xd0 = 0.0f;
    if (tid < n / 16) {
        const int i = 16 * tid, j = i / cols, cc = i - j * cols;
        xq0 = *gptr<v4u>((uint64_t)(a.xq + ((uint64_t)tk * k + j) * cols + cc));
    }
    if (tid < n / 32) {
        const int i = 32 * tid, j = i / cols, cc = i - j * cols;
        xd0 = *gptr<float>((uint64_t)(a.xd + ((uint64_t)tk * k + j) * (cols / 32) + cc / 32));
    }
    __syncthreads();  // the slots

    // the k spans' loads: chunk c of the flattened list is chunk c - j nch of slot j's span (rows r0 .. of its
    // expert, from the 16-byte-aligned cover); chunks past a span's end and spans of slots not resident are skipped
    constexpr int DC_CH = 8;  // loads a thread (k nch <= DC_CH DC_THREADS, checked on the host)
    v4u wv[DC_CH];
#pragma unroll
    for (int i = 0; i < DC_CH; i++) {
        const int c = tid + DC_THREADS * i;
        const int j = fdiv(c, a.nch_m, a.nch_s), cc = c - j * a.nch;
        if (j < k) {
            const int e = sslot[j];
            if (e >= 0) {
                const uint64_t beg = (uint64_t)(a.w + e * a.stride + (uint64_t)r0 * a.rb), g0 = beg & ~(uint64_t)15;
                const int nch = (int)((((beg + (uint64_t)nr * a.rb) + 15) & ~(uint64_t)15) - g0) >> 4;
                if (cc < nch) wv[i] = __builtin_nontemporal_load(gptr<v4u>(g0 + 16 * (uint64_t)cc));
            }
        }
    }
    // x of the k slots, flattened: value v of slot j at j cols + v
    {
        for (int c = tid; c < n / 16; c += DC_THREADS) {
            const int i = 16 * c, j = i / cols, cc = i - j * cols;
            const v4u q = c == tid ? xq0 : *gptr<v4u>((uint64_t)(a.xq + ((uint64_t)tk * k + j) * cols + cc));
            *(v4u*)(xl + xpad(i)) = q;
            xss[c] = sdot4((int)q.x, 0x01010101, sdot4((int)q.y, 0x01010101, sdot4((int)q.z, 0x01010101, sdot4((int)q.w, 0x01010101, 0))));
        }
        for (int c = tid; c < n / 32; c += DC_THREADS) {
            const int i = 32 * c, j = i / cols, cc = i - j * cols;
            xld[c] = c == tid ? xd0 : *gptr<float>((uint64_t)(a.xd + ((uint64_t)tk * k + j) * (cols / 32) + cc / 32));
        }
    }
#pragma unroll
    for (int i = 0; i < DC_CH; i++) {
        const int c = tid + DC_THREADS * i;
        const int j = fdiv(c, a.nch_m, a.nch_s);
        if (j < k) *(v4u*)(tile + 16 * c) = wv[i];
    }
    __syncthreads();

    // pair p = 16 q + lane / G of group q = wave / 4: slot p / R, row p % R; quarter wave % 4 of super-block lane % G
    const int grp = wave >> 2, qw = wave & 3, gl = lane & (G - 1);
    const int p = grp * (64 / G) + lane / G, j = p / R, rr = p - j * R;
    int e = -1;
    if (j < k) e = sslot[j];
    const bool live = j < k && e >= 0 && rr < nr && gl < a.nsb;
    const int nv = min(256, cols - 256 * gl);
    uint32_t o0 = 0, o1 = 0;
    float D = 0.0f, M = 0.0f;
    if (live) {
        const uint64_t beg = (uint64_t)(a.w + e * a.stride + (uint64_t)r0 * a.rb);
        const uint8_t* b = tile + 16 * a.nch * j + (beg & 15) + (uint64_t)rr * a.rb + gl * SBB;
        const int sb = j * a.nsb + gl;
        const XLds xv{xl + xpad(256 * sb), xld + 8 * sb, xss + 16 * sb};
        switch (qw) {
        case 0: sb_quarter<T, Q32, 0>(b, xv, tab, nv, o0, o1, D, M); break;
        case 1: sb_quarter<T, Q32, 1>(b, xv, tab, nv, o0, o1, D, M); break;
        case 2: sb_quarter<T, Q32, 2>(b, xv, tab, nv, o0, o1, D, M); break;
        default: sb_quarter<T, Q32, 3>(b, xv, tab, nv, o0, o1, D, M); break;
        }
    }
    if (qw) *(uint2*)(part + ((grp * 3 + qw - 1) * 64 + lane) * 2) = make_uint2(o0, o1);
    __syncthreads();
    if (qw == 0) {
        uint32_t o[8];
        o[0] = o0;
        o[1] = o1;
#pragma unroll
        for (int w = 1; w < 4; w++) {
            const uint2 v = *(const uint2*)(part + ((grp * 3 + w - 1) * 64 + lane) * 2);
            o[2 * w] = v.x;
            o[2 * w + 1] = v.y;
        }
        const int sb = j * a.nsb + gl;
        float acc = live ? sb_close<T, Q32>(o, D, M, live ? xld[8 * sb] : 0.0f, nv) : 0.0f;
        acc = ordered_sum(acc, G);
        if (j < k && rr < R && gl == G - 1) ye[j * R + rr] = acc;
    }
    __syncthreads();
    // the combine of each row: the slots' weighted outputs in slot order (a slot of weight 0 or not resident adds
    // nothing), then the shared expert
    if (tid < nr) {
        float y = 0.0f;
        for (int jj = 0; jj < k; jj++) {
            const float wj = swh[jj];
            if (wj != 0.0f && sslot[jj] >= 0) y += wj * ye[jj * R + tid];
        }
        if (a.sh) y += (a.sg ? dc_sigmoid(sgv) : 1.0f) * sho;
        a.x[orow] = xo + y;
    }
}

template <int T, bool Q32>
static hipError_t dc_launch(const DcArgs& a, int t, size_t smem, hipStream_t s) {
    static size_t attr = 64 * 1024;  // dynamic LDS the kernel is set up for
    if (!attr) {
        if (hipFuncSetAttribute((const void*)moe_down_combine_kernel<T, Q32>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
            return hipErrorInvalidValue;
        attr = true;
    }
    moe_down_combine_kernel<T, Q32><<<dim3((unsigned)((a.rows + a.R - 1) / a.R), (unsigned)t), DC_THREADS, smem, s>>>(a);
    return hipGetLastError();
}
template <int T>
static hipError_t dc_t(const DcArgs& a, bool q32, int t, size_t smem, hipStream_t s) {
    return q32 ? dc_launch<T, true>(a, t, smem, s) : dc_launch<T, false>(a, t, smem, s);
}

hipError_t launch_down_combine(const DownCombineLaunch& g, hipStream_t s) {
    DcArgs a{};
    a.w = g.w; a.stride = g.stride; a.slots = g.slots; a.wh = g.wh;
    a.xq = g.xq;
    a.xd = g.xq ? (const float*)(g.xq + (uint64_t)g.t * g.k * g.cols) : nullptr;
    a.x = g.x; a.sh = g.sh; a.sg = g.sg;
    a.rows = g.rows; a.cols = g.cols; a.k = g.k;
    a.rb = row_bytes(g.ty, g.cols);
    a.nsb = g.cols / 256;
    a.G = 1;
    while (a.G < a.nsb) a.G <<= 1;
    const int pairs = 4 * (64 / a.G);
    a.R = pairs / g.k;
    a.nch = (int)((a.R * a.rb + 15) / 16 + 1);
    magic((uint32_t)a.nch, a.nch_m, a.nch_s);
    const bool iq = g.ty == IQ2_XXS || g.ty == IQ3_S;
    const uint32_t n = (uint32_t)(g.k * g.cols);
    const size_t smem = (iq ? up16(sizeof(IqTables)) : 0) + xpad_bytes(n) + n / 8 + n / 4 + 16 * (size_t)a.nch * g.k +
                        4 * 3 * 64 * 8 + 4 * (size_t)g.k * a.R + 8 * (size_t)g.k;
    // shapes this layout does not take: the caller's two launches
    if (!g.xq || g.cols % 256 || a.G > 64 || a.R < 1 || g.k * a.nch > 8 * DC_THREADS || smem > 160 * 1024 ||
        g.t < 1 || g.t > 65535)
        return hipErrorNotSupported;
    const bool q32 = g.numerics == STRATA_NUM_Q8_32;
    switch (g.ty) {
    case Q8_0: return dc_t<Q8_0>(a, q32, g.t, smem, s);
    case Q2_K: return dc_t<Q2_K>(a, q32, g.t, smem, s);
    case Q3_K: return dc_t<Q3_K>(a, q32, g.t, smem, s);
    case Q4_K: return dc_t<Q4_K>(a, q32, g.t, smem, s);
    case Q5_K: return dc_t<Q5_K>(a, q32, g.t, smem, s);
    case Q6_K: return dc_t<Q6_K>(a, q32, g.t, smem, s);
    case IQ2_XXS: return dc_t<IQ2_XXS>(a, q32, g.t, smem, s);
    case IQ3_S: return dc_t<IQ3_S>(a, q32, g.t, smem, s);
    case IQ4_XS: return dc_t<IQ4_XS>(a, q32, g.t, smem, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace strata

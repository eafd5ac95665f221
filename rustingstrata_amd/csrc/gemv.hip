// Decode GEMV for the quantized types: y = W x for 1..4 inputs (gemv / gemvn / gemvq / gemvq2) and the MoE form
// (moe_gemv: one expert matrix and x row per slot).
//
// A block of 256 threads (4 wave64) computes R consecutive rows. It streams the rows' contiguous byte span from
// HBM with 16-byte coalesced loads (any block alignment: the span is read from its 16-byte-aligned cover) into
// LDS, together with the quantized x (int8 + per-32 scales, plus per-16 sums computed on the way in) and, for the
// IQ types, the codebook tables. Then each row is reduced by G lanes (G = 16, 32 or 64, by row length): lane l
// takes the row's 32-value tasks l, l + G, ... (a task is 32 weights decoded to int8 by task<T>), dots them with
// sdot4 against x and scales in f32; the G partial sums meet by cross-lane reduction.
#include "formats.h"
#include "kernels.h"

namespace strata {

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_CH = 6;                                          // 16-byte chunks per thread per tile
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
};

// LDS layout: [IqTables (IQ types)][x int8: nt * cols][x scales: nt * cols / 32 f32][x sums: nt * cols / 16
// int32][weight tile], each section rounded up to 16 bytes.
__host__ __device__ constexpr uint32_t up16(uint32_t v) { return (v + 15) & ~15u; }

template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, G);
    return v;
}

template <int T, int NT, int G>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_kernel(GemvArgs a) {
    constexpr bool IQ = T == IQ2_XXS || T == IQ3_S;
    constexpr int SBB = sb_bytes(T);
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x;
    const int z = blockIdx.z, slot = blockIdx.y;
    const int rows = z ? a.rows2 : a.rows;
    const int r0 = blockIdx.x * a.R;
    if (r0 >= rows) return;
    const int nr = min(a.R, rows - r0);
    const uint8_t* W = a.w + (z ? a.w2 : 0);
    float* Y = (float*)((uint8_t*)a.y + (z ? a.y2 : 0));
    int xrow = 0;
    if (a.ids) {
        int e = a.ids[slot];
        if (e < 0) return;  // slot not routed here: its output stays untouched
        W += (int64_t)e * a.stride;
        xrow = slot / a.xg;
        Y += (int64_t)slot * rows;
    }
    const int cols = a.cols;

    // 1. Issue the weight span loads into registers.
    const uint64_t beg = (uint64_t)(W + (uint64_t)r0 * a.rb), end = beg + (uint64_t)nr * a.rb;
    const uint64_t g0 = beg & ~(uint64_t)15;
    const int nch = (int)(((end + 15) & ~(uint64_t)15) - g0) >> 4;
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    v4u wv[GEMV_CH];
#pragma unroll
    for (int i = 0; i < GEMV_CH; i++) {
        int c = tid + GEMV_THREADS * i;
        if (c < nch) wv[i] = __builtin_nontemporal_load((const v4u*)(g0 + 16 * (uint64_t)c));
    }

    // 2. x (int8 + scales, per-16 sums) and the IQ tables into LDS.
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
    for (int c = tid; c < NT * cols / 16; c += GEMV_THREADS) {
        int t = c / (cols / 16), j = c % (cols / 16);
        uint4 q = *(const uint4*)(a.xq + (uint64_t)(xrow + t) * cols + 16 * j);
        *(uint4*)(sx + 16 * c) = q;
        ss[c] = sdot4((int)q.x, 0x01010101, sdot4((int)q.y, 0x01010101, sdot4((int)q.z, 0x01010101, sdot4((int)q.w, 0x01010101, 0))));
    }
    for (int c = tid; c < NT * cols / 32; c += GEMV_THREADS) {
        int t = c / (cols / 32), j = c % (cols / 32);
        sd[c] = a.xd[(uint64_t)(xrow + t) * (cols / 32) + j];
    }

    // 3. Weights into LDS.
#pragma unroll
    for (int i = 0; i < GEMV_CH; i++) {
        int c = tid + GEMV_THREADS * i;
        if (c < nch) *(v4u*)(tile + 16 * c) = wv[i];
    }
    __syncthreads();

    // 4. Rows: G lanes each, 64 / G rows per wave per pass.
    const int wave = tid >> 6, lane = tid & 63, gl = lane & (G - 1);
    constexpr int RPW = 64 / G;
    const int tpr = cols / 32;  // tasks per row
    for (int base = wave * RPW; base < nr; base += 4 * RPW) {
        const int rr = base + lane / G;
        float acc[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] = 0.0f;
        if (rr < nr) {
            const uint8_t* rowp = tile + (beg - g0) + (uint64_t)rr * a.rb;
            for (int i = gl; i < tpr; i += G) {
                const int sb = i >> 3;
                Task tk;
                task<T>(rowp + sb * SBB, i & 7, tab, tk);
                const int x0 = sb * 256 + tk.o0, x1 = sb * 256 + tk.o1;
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const int8_t* xs = sx + t * cols;
                    uint4 u0 = *(const uint4*)(xs + x0), u1 = *(const uint4*)(xs + x1);
                    int s0 = sdot4(tk.q[0], (int)u0.x, sdot4(tk.q[1], (int)u0.y, sdot4(tk.q[2], (int)u0.z, sdot4(tk.q[3], (int)u0.w, 0))));
                    int s1 = sdot4(tk.q[4], (int)u1.x, sdot4(tk.q[5], (int)u1.y, sdot4(tk.q[6], (int)u1.z, sdot4(tk.q[7], (int)u1.w, 0))));
                    const int* sst = ss + t * (cols / 16);
                    const int xs0 = sst[x0 >> 4], xs1 = sst[x1 >> 4];
                    if constexpr (Fmt<T>::BIAS != 0) { s0 -= Fmt<T>::BIAS * xs0; s1 -= Fmt<T>::BIAS * xs1; }
                    float f0 = tk.D * (float)(tk.sc0 * s0), f1 = tk.D * (float)(tk.sc1 * s1);
                    if constexpr (Fmt<T>::MIN) { f0 -= tk.M * (float)(tk.m0 * xs0); f1 -= tk.M * (float)(tk.m1 * xs1); }
                    const float* sdt = sd + t * (cols / 32);
                    acc[t] += sdt[x0 >> 5] * f0 + sdt[x1 >> 5] * f1;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] = group_sum<G>(acc[t]);
        if (rr < nr && gl == 0) {
#pragma unroll
            for (int t = 0; t < NT; t++) Y[(int64_t)t * a.y_stride + r0 + rr] = acc[t];
        }
    }
}

template <int T, int NT>
static hipError_t gemv_nt(const GemvArgs& a, dim3 grid, size_t smem, hipStream_t s) {
    int tpr = a.cols / 32;
    if (tpr >= 64) gemv_kernel<T, NT, 64><<<grid, GEMV_THREADS, smem, s>>>(a);
    else if (tpr >= 32) gemv_kernel<T, NT, 32><<<grid, GEMV_THREADS, smem, s>>>(a);
    else gemv_kernel<T, NT, 16><<<grid, GEMV_THREADS, smem, s>>>(a);
    return hipGetLastError();
}

template <int T>
static hipError_t gemv_t(const GemvArgs& a, dim3 grid, size_t smem, hipStream_t s) {
    switch (a.nt) {
    case 1: return gemv_nt<T, 1>(a, grid, smem, s);
    case 2: return gemv_nt<T, 2>(a, grid, smem, s);
    case 3: return gemv_nt<T, 3>(a, grid, smem, s);
    case 4: return gemv_nt<T, 4>(a, grid, smem, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemv(const GemvLaunch& g, hipStream_t s) {
    GemvArgs a{};
    a.w = g.w; a.w2 = g.pair ? g.w2 : 0; a.y = g.y; a.y2 = g.pair ? g.y2 : 0;
    a.xq = g.xq; a.xd = (const float*)(g.xq + (uint64_t)g.n_xrows * g.cols);
    a.ids = g.ids; a.stride = g.stride; a.xg = g.xg;
    a.rows = g.rows; a.rows2 = g.pair ? g.rows2 : 0; a.cols = g.cols; a.nt = g.nt; a.y_stride = g.y_stride;
    a.rb = row_bytes(g.ty, g.cols);
    a.R = (int)((GEMV_TILE - 32) / a.rb);
    int maxrows = g.pair ? (g.rows > g.rows2 ? g.rows : g.rows2) : g.rows;
    if (a.R > maxrows) a.R = maxrows;
    if (a.R < 1) a.R = 1;
    dim3 grid((unsigned)((maxrows + a.R - 1) / a.R), (unsigned)(g.ids ? g.k : 1), g.pair ? 2u : 1u);
    bool iq = g.ty == IQ2_XXS || g.ty == IQ3_S;
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

}  // namespace strata

// Prefill GEMM on int8 MFMA (v_mfma_i32_16x16x64_i8) over a tile list: for each tile [w, m0 | cnt << 32] the
// positions m0 .. m0 + cnt get y[m, 0..rows] (op) W x[xrow[m]] (Backend::gemm, src/backend.rs:187-191; reference
// kernel gemmi_q, src/cuda/kernels.cu:1355-1486).
//
// Exact integer super-blocks. X is int8 with one scale per 256 values (Q8_K). A weight of a super-block is
// D * (sc * (q - bias)) - M * m, with integer sc, q, m per 16/32-value group and float D, M per super-block. The
// integer v = sc * (q - bias) needs up to 13 bits, so it is split into two int8 digit planes, v = 64 HI + LO
// (LO in 0..63), and the group min m is a third plane (m repeated over its group). Each plane is an int8 matrix
// over the whole super-block, so one MFMA of K = 64 covers any mix of groups and the three int32 sums
//   HI.x, LO.x, M.x   (exact)
// close the super-block as  acc += dx * (D * (64 HI.x + LO.x) - M * M.x).  No per-group scaling in the K loop.
//
// Block: 256 threads, 64 positions x 64 weight rows; wave w owns 32 positions x 32 rows (2 x 2 MFMA tiles of 16).
// Per super-block: the 64 rows' raw blocks are staged in LDS with 16-byte loads, then for each half (128 k) the
// X rows (gathered through xrow) and the decoded planes go to LDS and the MFMAs run.
#include "formats.h"
#include "gemm.h"
#include "kernels.h"
#include "../../include/strata_hip.h"

namespace strata {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int GM = 64, GN = 64, GK = 128;      // positions, rows, k per stage
constexpr int GP = GK + 16;                    // LDS row pitch of the k chunks (bank-conflict-free b128 reads)

template <int T> struct GemmFmt {
    static constexpr bool MIN = Fmt<T>::MIN;
    static constexpr bool HI = T != Q2_K;                     // Q2_K's sc * q <= 45 fits one plane
    static constexpr int NP = (HI ? 2 : 1) + (MIN ? 1 : 0);    // planes
    static constexpr int RAWP = ((sb_bytes(T) + 15) & ~15) + 16;  // raw super-block slot per row in LDS
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
};

__device__ __forceinline__ float silu_dev(float v) { return v / (1.0f + (float)exp(-(double)v)); }

template <int T>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs a) {
    using F = GemmFmt<T>;
    constexpr int NP = F::NP, SBB = sb_bytes(T), RAWP = F::RAWP;
    constexpr int P_HI = 0, P_LO = F::HI ? 1 : 0, P_M = F::HI ? 2 : 1;
    constexpr bool IQ = T == IQ2_XXS || T == IQ3_S;
    extern __shared__ __align__(16) uint8_t smem[];
    int8_t* xs = (int8_t*)smem;                                 // [GM][GP]
    int8_t* pl = xs + GM * GP;                                  // [NP][GN][GP]
    uint8_t* raw = (uint8_t*)(pl + NP * GN * GP);               // [GN][RAWP]
    float* dx = (float*)(raw + GN * RAWP);                      // [GM]
    float* wD = dx + GM;                                        // [GN]
    float* wM = wD + GN;                                        // [GN]
    int* xr = (int*)(wM + GN);                                  // [GM] x row of each position
    IqTables* tab = (IqTables*)(xr + GM);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // Tile of this block.
    const int tile = blockIdx.y >> 1, half = blockIdx.y & 1;
    const uint8_t* W;
    int m0, cnt;
    if (a.tiles) {
        if (a.n_tiles_dev && tile >= *a.n_tiles_dev) return;
        uint64_t t0 = a.tiles[2 * tile], t1 = a.tiles[2 * tile + 1];
        W = (const uint8_t*)t0;
        m0 = (int)(uint32_t)t1;
        cnt = (int)(t1 >> 32);
    } else {
        W = a.dense_w;
        m0 = 128 * tile;
        cnt = min(128, a.dense_n - m0);
    }
    m0 += GM * half;
    cnt -= GM * half;
    if (cnt <= 0) return;
    if (cnt > GM) cnt = GM;
    const int n0 = blockIdx.x * GN;
    const int nrows = min(GN, a.rows - n0);
    const int cols = a.cols, nsb = cols / 256;

    if constexpr (IQ) load_iq_tables(tab);
    if (tid < GM) xr[tid] = tid < cnt ? (a.xrow ? a.xrow[m0 + tid] : m0 + tid) : -1;

    const int wm = 32 * (wave & 1), wn = 32 * (wave >> 1);
    float acc[2][2][4];
    v4i ia[NP][2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) acc[i][j][q] = 0.0f;

    for (int s = 0; s < nsb; s++) {
        __syncthreads();  // the previous super-block's readers are done with raw, dx, wD, wM
        // Raw super-block s of the 64 rows: row r's SBB bytes from its 16-byte-aligned cover.
        for (int c = tid; c < GN * (RAWP / 16); c += 256) {
            int r = c / (RAWP / 16), j = c % (RAWP / 16);
            if (r < nrows) {
                uint64_t beg = (uint64_t)(W + (uint64_t)(n0 + r) * a.rb + (uint64_t)s * SBB);
                uint64_t g0 = beg & ~(uint64_t)15;
                if (g0 + 16 * j < beg + SBB) *(uint4*)(raw + r * RAWP + 16 * j) = *(const uint4*)(g0 + 16 * j);
            }
        }
        if (tid < GM) {
            int x = xr[tid];
            dx[tid] = x >= 0 ? a.xd[(uint64_t)x * (cols / 32) + 8 * s] : 0.0f;
        }
#pragma unroll
        for (int p = 0; p < NP; p++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) ia[p][i][j] = (v4i){0, 0, 0, 0};
        __syncthreads();
        for (int hk = 0; hk < 2; hk++) {
            // X chunk: positions x k [128 s' .. + 128) as int8 (zero rows past cnt).
            for (int c = tid; c < GM * (GK / 16); c += 256) {
                int m = c / (GK / 16), j = c % (GK / 16);
                int x = xr[m];
                uint4 v = make_uint4(0, 0, 0, 0);
                if (x >= 0) v = *(const uint4*)(a.xq + (uint64_t)x * cols + 256 * s + GK * hk + 16 * j);
                *(uint4*)(xs + m * GP + 16 * j) = v;
            }
            // Planes: thread = (row, task) with tasks 4 hk .. 4 hk + 3 of the super-block.
            {
                int r = tid >> 2, k = 4 * hk + (tid & 3);
                int8_t* hi = pl + P_HI * GN * GP + r * GP;
                int8_t* lo = pl + P_LO * GN * GP + r * GP;
                int8_t* mm = pl + P_M * GN * GP + r * GP;
                if (r < nrows) {
                    uint64_t beg = (uint64_t)(W + (uint64_t)(n0 + r) * a.rb + (uint64_t)s * SBB);
                    const uint8_t* b = raw + r * RAWP + (beg & 15);
                    Task tk;
                    task<T>(b, k, tab, tk);
#pragma unroll
                    for (int g = 0; g < 2; g++) {
                        int o = (g ? tk.o1 : tk.o0) - GK * hk, sc = g ? tk.sc1 : tk.sc0;
                        uint32_t hw[4], lw[4];
#pragma unroll
                        for (int w = 0; w < 4; w++) {
                            uint32_t qv = (uint32_t)tk.q[4 * g + w], h = 0, l = 0;
#pragma unroll
                            for (int bb = 0; bb < 4; bb++) {
                                int v = sc * ((int)(int8_t)(qv >> (8 * bb)) - Fmt<T>::BIAS);
                                h |= (uint32_t)((v >> 6) & 255) << (8 * bb);
                                l |= (uint32_t)(v & 63) << (8 * bb);
                            }
                            hw[w] = h;
                            lw[w] = l;
                        }
                        if constexpr (F::HI) *(uint4*)(hi + o) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
                        *(uint4*)(lo + o) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
                        if constexpr (F::MIN) {
                            uint32_t mv = (uint32_t)(g ? tk.m1 : tk.m0) * 0x01010101u;
                            *(uint4*)(mm + o) = make_uint4(mv, mv, mv, mv);
                        }
                    }
                    if (hk == 0 && (tid & 3) == 0) { wD[r] = tk.D; wM[r] = tk.M; }
                } else {
#pragma unroll
                    for (int g = 0; g < 2; g++) {
                        int o = 32 * (tid & 3) + 16 * g;
                        if constexpr (F::HI) *(uint4*)(hi + o) = make_uint4(0, 0, 0, 0);
                        *(uint4*)(lo + o) = make_uint4(0, 0, 0, 0);
                        if constexpr (F::MIN) *(uint4*)(mm + o) = make_uint4(0, 0, 0, 0);
                    }
                    if (hk == 0 && (tid & 3) == 0) { wD[r] = 0.0f; wM[r] = 0.0f; }
                }
            }
            __syncthreads();
            // MFMA: k steps of 64; lane l holds A row (position) l % 16 and B column (weight row) l % 16, k bytes
            // 16 (l / 16) .. + 16 of the step.
#pragma unroll
            for (int kk = 0; kk < GK; kk += 64) {
                const int ko = kk + 16 * (lane >> 4);
                v4i av[2];
#pragma unroll
                for (int i = 0; i < 2; i++) av[i] = *(const v4i*)(xs + (wm + 16 * i + (lane & 15)) * GP + ko);
#pragma unroll
                for (int p = 0; p < NP; p++) {
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        v4i bv = *(const v4i*)(pl + p * GN * GP + (wn + 16 * j + (lane & 15)) * GP + ko);
#pragma unroll
                        for (int i = 0; i < 2; i++) ia[p][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i], bv, ia[p][i][j], 0, 0, 0);
                    }
                }
            }
            __syncthreads();
        }
        // Close the super-block: lane's weight row wn + 16 j + l % 16, positions wm + 16 i + 4 (l / 16) + q.
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int r = wn + 16 * j + (lane & 15);
            const float D = wD[r], M = wM[r];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float d = dx[wm + 16 * i + 4 * (lane >> 4) + q];
                    int iv = F::HI ? 64 * ia[P_HI][i][j][q] + ia[P_LO][i][j][q] : ia[P_LO][i][j][q];
                    float f = D * (float)iv;
                    if constexpr (F::MIN) f -= M * (float)ia[P_M][i][j][q];
                    acc[i][j][q] += d * f;
                }
        }
    }
    // Epilogue.
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int r = wn + 16 * j + (lane & 15);
        if (r >= nrows) continue;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int m = wm + 16 * i + 4 * (lane >> 4) + q;
                if (m >= cnt) continue;
                float* yp = a.y + (int64_t)(m0 + m) * a.y_stride + n0 + r;
                float v = acc[i][j][q];
                *yp = a.act == STRATA_ACT_STORE ? v : a.act == STRATA_ACT_SWIGLU ? silu_dev(*yp) * v : *yp + v;
            }
    }
}

template <int T>
static size_t gemm_smem() {
    using F = GemmFmt<T>;
    size_t b = GM * GP + F::NP * GN * GP + GN * F::RAWP + (GM + GN + GN) * 4 + GM * 4;
    if (T == IQ2_XXS || T == IQ3_S) b += sizeof(IqTables);
    return b;
}

template <int T>
static hipError_t gemm_t(const GemmLaunch& g, hipStream_t s) {
    GemmArgs a{};
    a.tiles = g.tiles; a.n_tiles_dev = g.n_tiles_dev; a.dense_w = g.dense_w; a.dense_n = g.dense_n;
    a.xq = (const int8_t*)g.xq; a.xd = (const float*)(g.xq + (uint64_t)g.n_x * g.cols);
    a.xrow = g.xrow; a.y = g.y; a.y_stride = g.y_stride; a.rows = g.rows; a.cols = g.cols; a.act = g.act;
    a.rb = row_bytes(T, g.cols);
    size_t smem = gemm_smem<T>();
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)gemm_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
        attr = true;
    }
    dim3 grid((unsigned)((g.rows + GN - 1) / GN), (unsigned)(2 * g.n_tiles));
    gemm_kernel<T><<<grid, 256, smem, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmLaunch& g, hipStream_t s) {
    switch (g.ty) {
    case Q2_K: return gemm_t<Q2_K>(g, s);
    case Q3_K: return gemm_t<Q3_K>(g, s);
    case Q4_K: return gemm_t<Q4_K>(g, s);
    case Q5_K: return gemm_t<Q5_K>(g, s);
    case Q6_K: return gemm_t<Q6_K>(g, s);
    case IQ2_XXS: return gemm_t<IQ2_XXS>(g, s);
    case IQ3_S: return gemm_t<IQ3_S>(g, s);
    case IQ4_XS: return gemm_t<IQ4_XS>(g, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemm_quant_x(const float* x, uint64_t x_stride, int cols, int n_x, uint8_t* out, int, hipStream_t s) {
    return launch_quant_xq(x, x_stride, cols, n_x, (int8_t*)out, STRATA_NUM_Q8K, s);
}

}  // namespace strata

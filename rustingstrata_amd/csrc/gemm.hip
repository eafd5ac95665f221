// Prefill GEMM on int8 MFMA (v_mfma_i32_16x16x64_i8) over a tile list: for each tile [w, m0 | cnt << 32] the
// positions m0 .. m0 + cnt get y[m, 0..rows] (op) W x[xrow[m]] (Backend::gemm, src/backend.rs:187-191; reference
// kernel gemmi_q, src/cuda/kernels.cu:1355-1486).
//
// Exact integer super-blocks. X is int8 with one scale per 256 values (Q8_K). A weight of a super-block is
// D * sc * (q - bias) - M * m with integer sc, q, m per 16/32-value group and float D, M per super-block; the integer
// v = sc * (q - bias) is split into two int8 digit planes v = 64 HI + LO, and the group min m is a third plane
// (dec16.h). Each plane is an int8 matrix over the whole super-block, so one MFMA of K = 64 covers any mix of groups
// and the int32 sums HI.x, LO.x, M.x (exact) close the super-block as
//     acc += dx * (D * (64 HI.x + LO.x) - M * M.x).
// No per-group scaling happens in the K loop.
//
// Block: 256 threads, one tile of up to 128 positions x 64 weight rows. Wave w owns weight rows 16 w .. 16 w + 15 and
// all positions (8 MFMA tiles of 16 positions), so every weight is decoded once per block, by the lane that feeds it
// to the MFMA: lane l decodes row l % 16, values 16 (l / 16) .. of each 64-deep K step, straight into its B operand.
// Per super-block the raw weight blocks of the 64 rows and the 128 gathered X rows are staged in LDS; the next
// super-block's are loaded into registers meanwhile.
#include "dec16.h"
#include "gemm.h"
#include "kernels.h"
#include "../../include/strata_hip.h"

namespace strata {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

constexpr int NXCD = 8;                        // MI355X: 8 XCDs, each with its own L2
constexpr int GM = 128, GN = 64;               // positions, weight rows per block
constexpr int XP = 256 + 16;                   // LDS pitch of an X row (one super-block of int8, bank-offset)
constexpr int XCH = GM * 16 / 256;             // 16-byte X chunks per thread per super-block

template <int T> struct GemmFmt {
    static constexpr bool MIN = Dec<T>::MIN;
    static constexpr bool HI = T != Q2_K;                        // Q2_K's sc * q <= 45 fits the LO plane
    static constexpr int NP = (HI ? 2 : 1) + (MIN ? 1 : 0);       // planes
    static constexpr int RAWP = ((sb_bytes(T) + 15) & ~15) + 16;  // raw super-block slot per row in LDS
    static constexpr int WCH = (GN * (RAWP / 16) + 255) / 256;    // 16-byte weight chunks per thread
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
};

__device__ __forceinline__ float silu_dev(float v) { return v / (1.0f + (float)exp(-(double)v)); }

template <int T>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs a) {
    using F = GemmFmt<T>;
    constexpr int NP = F::NP, SBB = sb_bytes(T), RAWP = F::RAWP, WCH = F::WCH;
    constexpr int P_HI = 0, P_LO = F::HI ? 1 : 0, P_M = F::HI ? 2 : 1;
    constexpr bool IQ = T == IQ2_XXS || T == IQ3_S;
    extern __shared__ __align__(16) uint8_t smem[];
    // LDS: [X: GM x XP][raw W: GN x RAWP][dx: GM][xr: GM][IqTables]
    int8_t* xs = (int8_t*)smem;
    uint8_t* raw = smem + GM * XP;
    float* dxs = (float*)(raw + GN * RAWP);
    int* xr = (int*)(dxs + GM);
    IqTables* tab = (IqTables*)(xr + GM);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // XCD-aware order: the hardware deals consecutive block ids to the 8 XCDs in turn, so logical block
    // (tile, row block) = consecutive ids within one XCD; a tile's row blocks and an expert's tiles then share that
    // XCD's L2 (its X rows and the expert's weights are read from L2 after the first block).
    const int ntiles = a.n_tiles_dev ? min(*a.n_tiles_dev, a.max_tiles) : a.max_tiles;
    const int nrb = (a.rows + GN - 1) / GN, total = nrb * ntiles;
    const int per_xcd = (total + NXCD - 1) / NXCD;
    const int lid = (blockIdx.x % NXCD) * per_xcd + blockIdx.x / NXCD;
    if (blockIdx.x / NXCD >= per_xcd || lid >= total) return;
    const int tile = lid / nrb, rb_idx = lid % nrb;
    const uint8_t* W;
    int m0, cnt;
    if (a.tiles) {
        const uint64_t t0 = a.tiles[2 * tile], t1 = a.tiles[2 * tile + 1];
        W = (const uint8_t*)t0;
        m0 = (int)(uint32_t)t1;
        cnt = min(GM, (int)(t1 >> 32));
    } else {
        W = a.dense_w;
        m0 = GM * tile;
        cnt = min(GM, a.dense_n - m0);
    }
    if (cnt <= 0) return;
    const int n0 = rb_idx * GN;
    const int nrows = min(GN, a.rows - n0);
    const int cols = a.cols, nsb = cols / 256;
    const int ntt = (cnt + 15) >> 4;  // 16-position MFMA tiles with work

    if constexpr (IQ) load_iq_tables(tab);
    if (tid < GM) xr[tid] = tid < cnt ? (a.xrow ? a.xrow[m0 + tid] : m0 + tid) : -1;
    __syncthreads();

    // Prefetch registers: X chunk c (position c / 16, 16 bytes at 16 (c % 16)), weight chunk c (row c / (RAWP / 16)).
    v4u xv[XCH], wv[WCH];
    float dxv = 0.0f;
    auto issue = [&](int s) {
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int c = tid + 256 * i, m = c >> 4, x = xr[m];
            xv[i] = (v4u){0, 0, 0, 0};
            if (x >= 0) xv[i] = *gptr<v4u>((uint64_t)(a.xq + (uint64_t)x * cols + 256 * s + 16 * (c & 15)));
        }
#pragma unroll
        for (int i = 0; i < WCH; i++) {
            const int c = tid + 256 * i, r = c / (RAWP / 16), j = c % (RAWP / 16);
            if (r < nrows) {
                const uint64_t beg = (uint64_t)(W + (uint64_t)(n0 + r) * a.rb + (uint64_t)s * SBB), g0 = beg & ~(uint64_t)15;
                if (g0 + 16 * j < beg + SBB) wv[i] = *gptr<v4u>(g0 + 16 * j);
            }
        }
        if (tid < GM) {
            const int x = xr[tid];
            dxv = x >= 0 ? *gptr<float>((uint64_t)(a.xd + (uint64_t)x * (cols / 32) + 8 * s)) : 0.0f;
        }
    };

    float acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) acc[i][q] = 0.0f;
    const int r = 16 * wave + (lane & 15);  // this lane's weight row in the block
    const uint64_t rbeg0 = (uint64_t)(W + (uint64_t)(n0 + r) * a.rb);

    issue(0);
    for (int s = 0; s < nsb; s++) {
        __syncthreads();  // the previous super-block's readers are done
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int c = tid + 256 * i;
            *(v4u*)(xs + (c >> 4) * XP + 16 * (c & 15)) = xv[i];
        }
#pragma unroll
        for (int i = 0; i < WCH; i++) {
            const int c = tid + 256 * i, rr = c / (RAWP / 16), j = c % (RAWP / 16);
            if (rr < GN) *(v4u*)(raw + rr * RAWP + 16 * j) = wv[i];
        }
        if (tid < GM) dxs[tid] = dxv;
        __syncthreads();
        if (s + 1 < nsb) issue(s + 1);

        const uint8_t* b = raw + r * RAWP + ((rbeg0 + (uint64_t)s * SBB) & 15);
        v4i ia[NP][8];
#pragma unroll
        for (int pl = 0; pl < NP; pl++)
#pragma unroll
            for (int i = 0; i < 8; i++) ia[pl][i] = (v4i){0, 0, 0, 0};
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            uint32_t hi[4], lo[4];
            int m;
#ifdef STRATA_GEMM_NODECODE
            hi[0] = hi[1] = hi[2] = hi[3] = lo[0] = lo[1] = lo[2] = lo[3] = (uint32_t)kk * 0x01010101u + b[0];
            m = 1;
#else
            Dec<T>::run(b, 4 * kk + (lane >> 4), tab, hi, lo, m);
#endif
            const v4i bh = {(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
            const v4i bl = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
            const int mw = (int)((uint32_t)m * 0x01010101u);
            const v4i bm = {mw, mw, mw, mw};
            const int ko = 64 * kk + 16 * (lane >> 4);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (i >= ntt) break;
                const v4i av = *(const v4i*)(xs + (16 * i + (lane & 15)) * XP + ko);
#ifdef STRATA_GEMM_NOMFMA
                ia[P_LO][i] += av + bh + bl + bm;
                continue;
#endif
                if constexpr (F::HI) ia[P_HI][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bh, ia[P_HI][i], 0, 0, 0);
                ia[P_LO][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bl, ia[P_LO][i], 0, 0, 0);
                if constexpr (F::MIN) ia[P_M][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bm, ia[P_M][i], 0, 0, 0);
            }
        }
        // Close the super-block: lane's outputs are weight row r, positions 16 i + 4 (l / 16) + q.
        float D, M;
        Dec<T>::scales(b, D, M);
#ifdef STRATA_GEMM_NOCLOSE
        acc[0][0] += (float)ia[P_LO][0][0] * D + (float)ia[0][ntt - 1][3];
        continue;
#endif
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (i >= ntt) break;
            const float4 d4 = *(const float4*)(dxs + 16 * i + 4 * (lane >> 4));
            const float dq[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int iv = F::HI ? 64 * ia[P_HI][i][q] + ia[P_LO][i][q] : ia[P_LO][i][q];
                float f = D * (float)iv;
                if constexpr (F::MIN) f -= M * (float)ia[P_M][i][q];
                acc[i][q] += dq[q] * f;
            }
        }
    }
    // Epilogue.
    if (r >= nrows) return;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        if (i >= ntt) break;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int m = 16 * i + 4 * (lane >> 4) + q;
            if (m >= cnt) continue;
            float* yp = a.y + (int64_t)(m0 + m) * a.y_stride + n0 + r;
            const float v = acc[i][q];
            *yp = a.act == STRATA_ACT_STORE ? v : a.act == STRATA_ACT_SWIGLU ? silu_dev(*yp) * v : *yp + v;
        }
    }
}

template <int T>
static size_t gemm_smem() {
    size_t b = GM * XP + GN * GemmFmt<T>::RAWP + GM * 4 + GM * 4;
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
    const size_t smem = gemm_smem<T>();
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)gemm_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
        attr = true;
    }
    a.max_tiles = g.n_tiles;
    const long long total = (long long)((g.rows + GN - 1) / GN) * g.n_tiles;
    const long long grid = (total + NXCD - 1) / NXCD * NXCD;
    gemm_kernel<T><<<dim3((unsigned)grid), 256, smem, s>>>(a);
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

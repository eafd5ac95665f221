// Prefill GEMM on int8 MFMA (v_mfma_i32_16x16x64_i8) over a tile list: for each tile [w, m0 | cnt << 32] the
// positions m0 .. m0 + cnt get y[m, 0..rows] (op) W x[xrow[m]] (Backend::gemm, src/backend.rs:187-191; reference
// kernel gemmi_q, src/cuda/kernels.cu:1355-1486).
//
// Exact integer super-blocks. X is int8 with one scale per 256 values (Q8_K). A weight of a super-block is
// D * sc * (q - bias) - M * m with integer sc, q, m per 16/32-value group and float D, M per super-block; the integer
// v = sc * (q - bias) is split into two int8 digit planes v = 256 H + L, and the group min m is a third plane
// (dec16.h). Each plane is an int8 matrix over the whole super-block, so one MFMA of K = 64 covers any mix of groups
// and the int32 sums H.x, L.x, M.x (exact) close the super-block as
//     acc += dx * (D * (256 H.x + L.x) - M * M.x).
// No per-group scaling happens in the K loop.
//
// Block: 512 threads (8 waves, two per SIMD), a tile of up to GM = 256 positions x GN = 128 weight rows. Wave w owns
// weight rows 16 w .. 16 w + 15 (one 16-row MFMA column) and every position (16 MFMA tiles of 16 positions), so each
// weight is decoded once per block, by the lane that feeds it to the MFMA, and serves 256 positions. Per super-block
// step every wave
//   1. decodes its rows' super-block into digit-plane B operands (registers), issuing the next step's X loads
//      between the decode units;
//   2. issues the next step's raw-weight loads for its own 16 rows into their LDS rows (only this wave reads
//      them, so no barrier: a wave that has decoded starts its tiles while the others still decode);
//   3. runs its 16 position tiles in pairs: the two tiles' MFMA chains interleaved, then their float close.
// The two waves of a SIMD overlap one's VALU work (decode, close) with the other's MFMAs.
// Loads go straight from global memory into LDS (global_load_lds_dwordx4: lane l of a wave's instruction writes the
// 16 bytes at its own address to LDS base + 16 l); X is double-buffered, so a step's X loads have the whole step to
// land.
// X sits in LDS as [position][256 bytes] with 16-byte chunk c of position p at chunk c ^ (p & 15): a 16-lane MFMA
// fragment read (16 positions, one chunk) then touches 16 distinct bank groups.
#include <algorithm>

#include "gemm_dev.h"
#include "../../include/strata_hip.h"

namespace strata {

constexpr int GM = 256, GN = 128;    // positions, weight rows per block
constexpr int NW = 8;                // waves per block
constexpr int NTT = GM / 16;         // MFMA position tiles per block
constexpr int XBUF = GM * 256;       // bytes of one X buffer

template <int T> struct GemmFmt : GemmPlanes<T> {
    static constexpr int WBUF = GN * GemmPlanes<T>::RAWP;         // bytes of one raw weight buffer
};

template <int T>
__global__ __launch_bounds__(64 * NW, 1) void gemm_kernel(GemmArgs a) {
    using F = GemmFmt<T>;
    constexpr int NP = F::NP, SBB = sb_bytes(T), NCH = F::NCH, RAWP = F::RAWP, WBUF = F::WBUF;
    constexpr int P_HI = 0, P_LO = F::HI ? 1 : 0, P_M = F::HI ? 2 : 1;
    constexpr bool IQ = T == IQ2_XXS || T == IQ3_S;
    extern __shared__ __align__(16) uint8_t smem[];
    // LDS: [X: 2 x GM x 256][raw W: GN x RAWP][dx: 2 x GM][IqTables]
    int8_t* xs = (int8_t*)smem;
    uint8_t* raw = smem + 2 * XBUF;
    float* dxs = (float*)(raw + WBUF);
    IqTables* tab = (IqTables*)(dxs + 2 * GM);

    // the wave index through a scalar register: LDS destinations and chunk numbers built from it stay scalar
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int cols = a.cols, nsb = cols / 256;

    // Items are (tile, row block) pairs, item = tile * nrb + row block. XCD x (the hardware deals consecutive block
    // ids to the 8 XCDs in turn) takes a contiguous run of items, so a tile's row blocks and an expert's tiles run on
    // one XCD and share its L2 (X rows, expert weights).
    // (tile lists: the tiles' sizes are requested with their count, for the items' plan below)
    const int cnt0 = a.tiles && a.bal >= 0 ? plan_load(a.tiles, a.max_tiles) : 0;
    const int ntiles = a.n_tiles_dev ? min(sload(a.n_tiles_dev), a.max_tiles) : a.max_tiles;
    // pair mode: an item covers 64 output columns (64 rows of each of the two matrices)
    const bool pair = a.pair != 0;
    const int GNO = pair ? GN / 2 : GN;
    const int nrb = (a.rows + GNO - 1) / GNO, total = nrb * ntiles;
    const int xcd = blockIdx.x % NXCD, jb = blockIdx.x / NXCD;
    // tile lists of up to 64 NW tiles: the block's items planned by cost (plan_items); otherwise XCD x takes an eighth
    // of the items and its a.gx blocks every a.gx-th item from their index jb
    int ibeg, iend, mine = 0, ns = -1;
    if (a.tiles && a.bal >= 0 && ntiles <= 64 * NW) {
        static_assert(PLAN_INTS * 4 <= XBUF, "the plan fits the second X buffer, first written after the first barrier");
        ns = plan_items<NW>(cnt0, ntiles, nrb, a.bal, NXCD, xcd, jb, a.gx, (int*)(xs + XBUF), ibeg, iend, mine);
        ibeg += jb;
    } else {
        const int per = (total + NXCD - 1) / NXCD;
        ibeg = xcd * per + jb;
        iend = min((xcd + 1) * per, total);
    }
    const bool mine_ok = ns >= 0;
    const int nitems = mine_ok ? ns : ibeg < iend ? (iend - ibeg + a.gx - 1) / a.gx : 0;
    if (nitems == 0) return;

    struct Item {
        uint64_t w;
        int m0, cnt, n0;
    };
    auto item_at = [&](int k) __attribute__((always_inline)) {
        Item it{0, 0, 0, 0};
        if (k >= nitems) return it;
        const int id = mine_ok ? __builtin_amdgcn_readlane(mine, k) : ibeg + k * a.gx, tile = id / nrb;
        it.n0 = (id - tile * nrb) * GNO;
        if (a.tiles) {
            const uint64_t t0 = sload(a.tiles + 2 * tile), t1 = sload(a.tiles + 2 * tile + 1);
            it.w = t0;
            it.m0 = (int)(uint32_t)t1;
            it.cnt = min(GM, (int)(t1 >> 32));
        } else {
            it.w = (uint64_t)a.dense_w;
            it.m0 = a.dense_p * tile;
            it.cnt = min(a.dense_p, a.dense_n - it.m0);
        }
        return it;
    };

    if constexpr (IQ) load_iq_tables(tab);

    // Per-lane load addresses of an item. X instruction j of wave w fills 1 KB of LDS: positions 4 (XI w + j) + l / 16,
    // LDS chunk l % 16, which holds X chunk (l % 16) ^ (p & 15). Weight instruction i of wave w fills chunks
    // c = 64 i + l of the wave's own 16 rows (block row 16 w + c / NCH, chunk c % NCH). An X instruction whose 4 positions are all
    // past cnt is skipped; positions past cnt in a partly live one load the item's first row (their results are never
    // stored); rows past `rows` read the last row. The scale of position tid (tid < GM) goes through a register.
    constexpr int XI = GM * 16 / 64 / NW;                     // X instructions per wave per step
    constexpr int WI = (16 * NCH + 63) / 64;                  // weight instructions per wave per step (its 16 rows)
    static_assert(NCH <= 15 && WI <= 8, "chunk numbers of a lane's weight instructions fit one word");
    static_assert(SBB < 225, "the no-chunk number 15 lands past every super-block");
    static_assert(XI % 4 == 0, "X instructions spread evenly over the 4 decode units");
    struct Addr {
        uint32_t xo[XI];   // X byte offset of each instruction's position row (+ chunk)
        uint32_t dxo;      // scale offset of position tid
        uint32_t rbeg;     // this lane's weight row: byte offset from W, plus W mod 16
        uint32_t wro[WI];  // byte offsets from W of the rows of this lane's weight chunks
        int cnt;           // the item's positions
    };
    const int rl = 16 * wave + (lane & 15);  // this lane's weight row in the block
    // Weight instruction i of this wave: chunk wchunk(i) of the wave's own 16 rows (the rows it decodes: block rows
    // 16 w .., in pair mode waves 0-3 the first matrix's 64 rows and 4-7 the second's), block row 16 w + wchunk / NCH,
    // LDS chunk 16 w NCH + wchunk. Each wave reloads its rows for the next step as soon as its own decode is done.
    const int wlim = 16 * NCH;
    auto wchunk = [&](int i) __attribute__((always_inline)) { return 64 * i + lane; };
    auto addr_of = [&](const Item& it) __attribute__((always_inline)) {
        Addr ad;
        ad.cnt = it.cnt;
        auto xrow_of = [&](int p) { p = p < it.cnt ? p : 0; return a.xrow ? a.xrow[it.m0 + p] : it.m0 + p; };
#pragma unroll
        for (int j = 0; j < XI; j++) {
            const int p = 4 * (XI * wave + j) + (lane >> 4);
            ad.xo[j] = (uint32_t)xrow_of(p) * (uint32_t)cols + 16 * ((lane & 15) ^ (p & 15));
        }
        ad.dxo = (uint32_t)xrow_of(tid & (GM - 1)) * (uint32_t)(cols / 32);
        ad.rbeg = (uint32_t)(it.w & 15) + (pair && wave >= 4 ? (uint32_t)(a.w2 & 15) : 0u) +
                  __umul24((uint32_t)min(it.n0 + (pair ? (rl & 63) : rl), a.rows - 1), (uint32_t)a.rb);
#pragma unroll
        for (int i = 0; i < WI; i++)
            ad.wro[i] = __umul24((uint32_t)min(it.n0 + ((16 * wave + min(wchunk(i) / NCH, 15)) & (GNO - 1)), a.rows - 1),
                                 (uint32_t)a.rb);
        return ad;
    };
    // X instruction j of super-block s of an item into the X buffer of step g (X and dx rotate by 2).
    auto load_x1 = [&](const Addr& ad, int s, int g, const int j) __attribute__((always_inline)) {
        if (4 * (XI * wave + j) < ad.cnt)
            load_lds16_so((uint64_t)(a.xq + 256 * s), ad.xo[j], xs + (g & 1) * XBUF + 1024 * (XI * wave + j));
    };
    // Chunk numbers c % NCH of this lane's weight instructions, 4 bits each (15: no chunk; NCH <= 15).
    uint32_t wcc = 0;
#pragma unroll
    for (int i = 0; i < WI; i++) wcc |= (uint32_t)(wchunk(i) < wlim ? wchunk(i) % NCH : 15) << (4 * i);
    // Raw weights of super-block s: the 16-byte covers of the rows' super-block, from the scalar base
    // (w + s * SBB) & ~15 and per-lane offsets ((w + s * SBB) & 15) + row offset, rounded down to 16, + 16 chunk
    // (a chunk past the super-block, or no chunk: offset 240 past the rounded start, is not loaded).
    auto load_w = [&](const Item& it, const Addr& ad, int s) __attribute__((always_inline)) {
        const uint64_t beg = it.w + (pair && wave >= 4 ? (uint64_t)a.w2 : 0) + (uint64_t)s * SBB, base = beg & ~(uint64_t)15;
        const uint32_t b15 = (uint32_t)(beg & 15);
#pragma unroll
        for (int i = 0; i < WI; i++) {
            const uint32_t t = b15 + ad.wro[i], o = (t & ~15u) + 16 * ((wcc >> (4 * i)) & 15);
            if (o < t + SBB) load_lds16_so(base, o, raw + 16 * (16 * NCH * wave + wchunk(i) - lane));
        }
    };
    float dxv = 0.0f;
    auto load_dx = [&](const Addr& ad, int s) __attribute__((always_inline)) {
        if (tid < GM) dxv = *gptr<float>((uint64_t)(a.xd + ad.dxo + 8 * s));
    };
    auto store_dx = [&](int g) __attribute__((always_inline)) {
        if (tid < GM) dxs[(g & 1) * GM + tid] = dxv;
    };

    float acc[NTT][4];
#pragma unroll
    for (int i = 0; i < NTT; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) acc[i][q] = 0.0f;
    const int kl = lane >> 4;                    // this lane's 16-value slot in each K step of 64
    const int aswz = lane & 15;                  // position & 15 of this lane's X fragment rows

    v4i B[4][NP];
    float D = 0.0f, M = 0.0f;
    // Decode super-block s of the item whose lane row offset is rbeg; hook(kk) runs after unit kk.
    auto decode = [&](uint32_t rbeg, int s, auto&& hook) __attribute__((always_inline)) {
        const uint8_t* b = raw + rl * RAWP + ((rbeg + (uint32_t)s * SBB) & 15);
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            uint32_t hi[4], lo[4];
            int m;
            Dec<T>::run(b, 4 * kk + kl, tab, hi, lo, m);
            if constexpr (F::HI) B[kk][P_HI] = (v4i){(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
            B[kk][P_LO] = (v4i){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
            if constexpr (F::MIN) {
                const int mw = (int)((uint32_t)m * 0x01010101u);
                B[kk][P_M] = (v4i){mw, mw, mw, mw};
            }
            hook(kk);
        }
        Dec<T>::scales(b, D, M);
    };
    // Tiles i and i + 1 together: their 2 NP accumulator chains interleave in the K loop, so an MFMA's result
    // feeds the next MFMA of its chain 2 NP issues later (the MFMA pipe stays full).
    auto mfma_pair = [&](const int i, int g, v4i (&c0)[NP], v4i (&c1)[NP]) __attribute__((always_inline)) {
        const int8_t* xb = xs + (g & 1) * XBUF;
        v4i a0[4], a1[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            a0[kk] = *(const v4i*)(xb + (16 * i + aswz) * 256 + 16 * ((4 * kk + kl) ^ aswz));
            a1[kk] = *(const v4i*)(xb + (16 * (i + 1) + aswz) * 256 + 16 * ((4 * kk + kl) ^ aswz));
        }
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int pl = 0; pl < NP; pl++) {
                c0[pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0[kk], B[kk][pl], kk ? c0[pl] : (v4i){0, 0, 0, 0}, 0, 0, 0);
                c1[pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[kk], B[kk][pl], kk ? c1[pl] : (v4i){0, 0, 0, 0}, 0, 0, 0);
            }
    };
    // Lane's outputs of tiles i and i + 1: weight row rl, positions 16 i + 4 kl + q (and 16 further), closed in one
    // loop so both accumulator chains end together (the compiler then keeps their MFMAs interleaved).
    auto close_pair = [&](const int i, int g, const v4i (&c0)[NP], const v4i (&c1)[NP]) __attribute__((always_inline)) {
        const float4 d0 = *(const float4*)(dxs + (g & 1) * GM + 16 * i + 4 * kl);
        const float4 d1 = *(const float4*)(dxs + (g & 1) * GM + 16 * (i + 1) + 4 * kl);
        const float dq0[4] = {d0.x, d0.y, d0.z, d0.w}, dq1[4] = {d1.x, d1.y, d1.z, d1.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int iv0 = F::HI ? (c0[P_HI][q] << 8) + c0[P_LO][q] : c0[P_LO][q];
            const int iv1 = F::HI ? (c1[P_HI][q] << 8) + c1[P_LO][q] : c1[P_LO][q];
            // the reference's float steps, rounded one by one (src/cpu_moe.rs:327-377):
            // sum += (D dx) s - (M dx) m, so the outputs carry the CPU dots' bits
            float f0 = (D * dq0[q]) * (float)iv0, f1 = (D * dq1[q]) * (float)iv1;
            if constexpr (F::MIN) {
                f0 = f0 - (M * dq0[q]) * (float)c0[P_M][q];
                f1 = f1 - (M * dq1[q]) * (float)c1[P_M][q];
            }
            acc[i][q] = acc[i][q] + f0;
            acc[i + 1][q] = acc[i + 1][q] + f1;
        }
    };
    // one tile (the last of an odd count: a tile pair would spend a whole tile's MFMAs and closes on no positions)
    auto mfma_one = [&](const int i, int g, v4i (&c0)[NP]) __attribute__((always_inline)) {
        const int8_t* xb = xs + (g & 1) * XBUF;
        v4i a0[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) a0[kk] = *(const v4i*)(xb + (16 * i + aswz) * 256 + 16 * ((4 * kk + kl) ^ aswz));
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int pl = 0; pl < NP; pl++)
                c0[pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0[kk], B[kk][pl], kk ? c0[pl] : (v4i){0, 0, 0, 0}, 0, 0, 0);
    };
    auto close_one = [&](const int i, int g, const v4i (&c0)[NP]) __attribute__((always_inline)) {
        const float4 d0 = *(const float4*)(dxs + (g & 1) * GM + 16 * i + 4 * kl);
        const float dq0[4] = {d0.x, d0.y, d0.z, d0.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int iv0 = F::HI ? (c0[P_HI][q] << 8) + c0[P_LO][q] : c0[P_LO][q];
            float f0 = (D * dq0[q]) * (float)iv0;
            if constexpr (F::MIN) f0 = f0 - (M * dq0[q]) * (float)c0[P_M][q];
            acc[i][q] = acc[i][q] + f0;
        }
    };
    auto tiles = [&](int g, int ntt) __attribute__((always_inline)) {
        static_for<0, NTT / 2>([&](auto I) {
            constexpr int i = 2 * decltype(I)::value;
            if (i + 1 < ntt) {
                v4i c0[NP], c1[NP];
                mfma_pair(i, g, c0, c1);
                close_pair(i, g, c0, c1);
            } else if (i < ntt) {
                v4i c0[NP];
                mfma_one(i, g, c0);
                close_one(i, g, c0);
            }
        });
    };
    // Results of an item: y[m0 + m, n0 + row] (op) acc; then the accumulators restart. With the whole row block
    // present and y rows 16-byte aligned, the block stages its outputs through the X buffer of step g (free once every
    // wave has run its tiles) as [128 positions][128 rows] floats, 128 positions a round, and writes whole 512-byte
    // rows with 16-byte accesses; the stage's row index is XOR-swizzled by (position / 4) & 3 so a wave's 4 position
    // groups write distinct banks. Otherwise each lane stores its own values.
    auto store = [&](const Item& it, int g) __attribute__((always_inline)) {
        const int ntt = (it.cnt + 15) >> 4;
        if (pair) {
            // y[m0 + m, n0 + c] = silu(first[c]) * second[c], c < 64: the stage holds the first matrix's outputs in
            // rows 0..63 and the second's in 64..127; each thread writes 4 float4 a round
            float* S = (float*)(xs + (g & 1) * XBUF);
            static_for<0, 2>([&](auto R) {
                constexpr int r = decltype(R)::value;
                if (128 * r < it.cnt) {
                    __syncthreads();  // the tiles (round 0) or the previous round's reads are done
                    static_for<0, 8>([&](auto I) {
                        constexpr int il = decltype(I)::value, i = 8 * r + il;
#pragma unroll
                        for (int q = 0; q < 4; q++) S[(16 * il + 4 * kl + q) * 128 + (rl ^ (kl << 4))] = acc[i][q];
                    });
                    __syncthreads();
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
                        const int idx = tid + 512 * jj, pr = idx >> 4, c4 = 4 * (idx & 15), m = 128 * r + pr;
                        if (m < it.cnt) {
                            const int swz = ((pr >> 2) & 3) << 4;
                            const float4 gv = *(const float4*)(S + pr * 128 + (c4 ^ swz));
                            const float4 uv = *(const float4*)(S + pr * 128 + ((64 + c4) ^ swz));
                            float4 o;
                            o.x = silu_dev(gv.x) * uv.x; o.y = silu_dev(gv.y) * uv.y;
                            o.z = silu_dev(gv.z) * uv.z; o.w = silu_dev(gv.w) * uv.w;
                            *(float4*)(a.y + (int64_t)(it.m0 + m) * a.y_stride + it.n0 + c4) = o;
                        }
                    }
                }
            });
        } else if (a.yvec && it.n0 + GN <= a.rows) {
            float* S = (float*)(xs + (g & 1) * XBUF);
            const int c4 = 4 * (lane & 31);
            auto put = [&](auto OP) __attribute__((always_inline)) {
                constexpr int op = decltype(OP)::value;
                static_for<0, 2>([&](auto R) {
                    constexpr int r = decltype(R)::value;
                    if (128 * r < it.cnt) {
                        __syncthreads();  // the tiles (round 0) or the previous round's reads are done
                        static_for<0, 8>([&](auto I) {
                            constexpr int il = decltype(I)::value, i = 8 * r + il;
#pragma unroll
                            for (int q = 0; q < 4; q++) S[(16 * il + 4 * kl + q) * 128 + (rl ^ (kl << 4))] = acc[i][q];
                        });
                        __syncthreads();
#pragma unroll
                        for (int jj = 0; jj < 8; jj++) {
                            const int pr = 16 * wave + 2 * jj + (lane >> 5), m = 128 * r + pr;
                            if (m < it.cnt) {
                                const float4 v = *(const float4*)(S + pr * 128 + (c4 ^ (((pr >> 2) & 3) << 4)));
                                float4* yp = (float4*)(a.y + (int64_t)(it.m0 + m) * a.y_stride + it.n0 + c4);
                                if constexpr (op == STRATA_ACT_STORE) {
                                    *yp = v;
                                } else {
                                    float4 o = *yp;
                                    if constexpr (op == STRATA_ACT_SWIGLU) {
                                        o.x = silu_dev(o.x) * v.x; o.y = silu_dev(o.y) * v.y;
                                        o.z = silu_dev(o.z) * v.z; o.w = silu_dev(o.w) * v.w;
                                    } else {
                                        o.x += v.x; o.y += v.y; o.z += v.z; o.w += v.w;
                                    }
                                    *yp = o;
                                }
                            }
                        }
                    }
                });
            };
            if (a.act == STRATA_ACT_STORE) put(std::integral_constant<int, STRATA_ACT_STORE>{});
            else if (a.act == STRATA_ACT_SWIGLU) put(std::integral_constant<int, STRATA_ACT_SWIGLU>{});
            else put(std::integral_constant<int, STRATA_ACT_ADD>{});
        } else if (it.n0 + rl < a.rows) {
            // row pointer of position 4 kl; position 16 i + 4 kl + q is (16 i + q) rows further
            float* yb = a.y + (int64_t)(it.m0 + 4 * kl) * a.y_stride + it.n0 + rl;
            const int left = it.cnt - 4 * kl;  // positions of this lane's column left from yb
            // the op is chosen once per item: one straight store loop per op
            auto put = [&](auto OP) __attribute__((always_inline)) {
                constexpr int op = decltype(OP)::value;
                static_for<0, NTT>([&](auto I) {
                    constexpr int i = decltype(I)::value;
                    if (i < ntt) {
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            if (16 * i + q < left) {
                                float* yp = yb + (int64_t)(16 * i + q) * a.y_stride;
                                const float v = acc[i][q];
                                if constexpr (op == STRATA_ACT_STORE) *yp = v;
                                else if constexpr (op == STRATA_ACT_SWIGLU) *yp = silu_dev(*yp) * v;
                                else *yp += v;
                            }
                        }
                    }
                });
            };
            if (a.act == STRATA_ACT_STORE) put(std::integral_constant<int, STRATA_ACT_STORE>{});
            else if (a.act == STRATA_ACT_SWIGLU) put(std::integral_constant<int, STRATA_ACT_SWIGLU>{});
            else put(std::integral_constant<int, STRATA_ACT_ADD>{});
        }
#pragma unroll
        for (int i = 0; i < NTT; i++)
#pragma unroll
            for (int q = 0; q < 4; q++) acc[i][q] = 0.0f;
    };

    // The super-block steps of this block's items run as one stream g = k * nsb + s (G steps): step g loads the X rows
    // and scales of step g + 1 and, once this wave has decoded its rows, their raw weights of step g + 1 into the
    // buffer just decoded. The load state (iL, aL, sL) describes step g + 1; cur and rbeg describe step g.
    const int G = nitems * nsb;
    int kL = 0, sL = 0;
    Item iL = item_at(0);
    Addr aL = addr_of(iL);
#pragma unroll
    for (int j = 0; j < XI; j++) load_x1(aL, 0, 0, j);
    load_w(iL, aL, 0);
    load_dx(aL, 0);
    store_dx(0);
    wait_loads();
    __syncthreads();
    Item cur = iL;
    uint32_t rbeg = aL.rbeg;
    auto advance = [&]() __attribute__((always_inline)) {
        if (++sL == nsb) {
            sL = 0;
            iL = item_at(++kL);
            aL = addr_of(iL);
        }
    };
    advance();
    int s = 0;
    for (int g = 0; g < G; g++) {
        const bool nx = g + 1 < G;
        if (nx) load_dx(aL, sL);
        decode(rbeg, s, [&](int kk) __attribute__((always_inline)) {
#pragma unroll
            for (int h = 0; h < XI / 4; h++)
                if (nx) load_x1(aL, sL, g + 1, (XI / 4) * kk + h);
        });
        // this wave's rows are decoded (and its reads of them done): their raw buffer takes the next step's weights
        wait_lds();
        if (nx) load_w(iL, aL, sL);
        tiles(g, (cur.cnt + 15) >> 4);
        if (s + 1 == nsb) store(cur, g);
        if (nx) store_dx(g + 1);
        cur = iL;
        rbeg = aL.rbeg;
        s = sL;
        advance();
        wait_loads();
        __syncthreads();
    }
}

template <int T>
static size_t gemm_smem() {
    size_t b = 2 * (size_t)XBUF + (size_t)GemmFmt<T>::WBUF + 2 * GM * 4;
    if (T == IQ2_XXS || T == IQ3_S) b += sizeof(IqTables);
    return b;
}

template <int T>
static hipError_t gemm_t(const GemmLaunch& g, hipStream_t s) {
    GemmArgs a{};
    a.tiles = g.tiles; a.n_tiles_dev = g.n_tiles_dev; a.dense_w = g.dense_w; a.dense_n = g.dense_n;
    a.xq = (const int8_t*)g.xq; a.xd = (const float*)(g.xq + (uint64_t)g.n_x * g.cols);
    a.xrow = g.xrow; a.y = g.y; a.y_stride = g.y_stride; a.rows = g.rows; a.cols = g.cols; a.act = g.act;
    a.yvec = ((uintptr_t)g.y % 16 == 0) && (g.y_stride % 4 == 0);
    a.pair = g.pair ? 1 : 0;
    a.w2 = g.w2;
    a.rb = row_bytes(T, g.cols);
    const size_t smem = gemm_smem<T>();
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)gemm_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
        attr = true;
    }
    // Persistent blocks, one per CU.
    static int ncu = 0;
    if (!ncu) {
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
    }
    const int gno = g.pair ? GN / 2 : GN;
    const long long nrb = (g.rows + gno - 1) / gno;
    a.max_tiles = g.n_tiles;
    a.dense_p = GM;
    if (!g.tiles) {
        // a dense matrix with few row blocks (the k and v projections) takes fewer positions per tile, down to 64,
        // until every CU has an item: the weights are then decoded more often, but no CU idles for the whole GEMM
        while (a.dense_p > 64 && (long long)((g.dense_n + a.dense_p - 1) / a.dense_p) * nrb < ncu) a.dense_p /= 2;
        a.max_tiles = (g.dense_n + a.dense_p - 1) / a.dense_p;
    }
    // tile lists split by cost over the XCDs; an item's decode costs about as much as 4 MFMA position tiles (3, 4 and
    // 5 measure the same on the 4096-token MoE layer; a split by count is 3% slower)
    a.bal = g.tiles ? 4 : -1;
    const long long total = nrb * a.max_tiles;
    const long long per = (total + NXCD - 1) / NXCD;
    const long long gx = std::min<long long>(per, std::max(ncu / NXCD, 1));
    a.gx = (int)std::max<long long>(gx, 1);
    const long long grid = (long long)a.gx * NXCD;
    gemm_kernel<T><<<dim3((unsigned)grid), 64 * NW, smem, s>>>(a);
    return hipGetLastError();
}


// ---- Q8_0 (src/cuda/kernels.cu:380-388): blocks of 32 int8 values, each with its own f16 scale ----
// The block scales are floats that differ within a super-block, so they cannot fold into integer planes; instead one
// K=64 MFMA step yields the two blocks' int32 sums separately (lanes 0-31 of the weight operand carry the first
// block's values and zeros for the second, lanes 32-63 the reverse: two MFMAs per step, no extra MFMA work), and each
// block closes in float at once: acc += dx (d0 s0 + d1 s1). A block of 4 waves takes a 64-row block of one tile and
// walks the tile's positions Q8_POS (128) at a time, the next step's X, scales and weights loaded into registers while the current one is computed; wave w owns rows 16 w .. 16 w + 15.
constexpr int Q8_ROWS = 64, Q8_POS = 128, Q8_SB = 272, Q8_RP = 280;  // rows, positions per pass, bytes per 256 values, LDS row pitch
constexpr int Q8_NT = Q8_POS / 16;  // MFMA position tiles per pass

__global__ __launch_bounds__(256) void gemm_q8_0_kernel(GemmArgs a) {
    __shared__ __align__(16) int8_t xs8[Q8_POS * 256];
    __shared__ __align__(16) uint8_t ws8[Q8_ROWS * Q8_RP];
    __shared__ float dx8[Q8_POS];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, kl = lane >> 4, aswz = lane & 15;
    const int ntiles = a.n_tiles_dev ? min(sload(a.n_tiles_dev), a.max_tiles) : a.max_tiles;
    const int tile = blockIdx.y, n0 = blockIdx.x * Q8_ROWS;
    if (tile >= ntiles) return;
    uint64_t w;
    int m0, cnt;
    if (a.tiles) {
        const uint64_t t0 = sload(a.tiles + 2 * tile), t1 = sload(a.tiles + 2 * tile + 1);
        w = t0;
        m0 = (int)(uint32_t)t1;
        cnt = min(GM, (int)(t1 >> 32));
    } else {
        w = (uint64_t)a.dense_w;
        m0 = GM * tile;
        cnt = min(GM, a.dense_n - m0);
    }
    const int cols = a.cols, nsb = cols / 256, rl = 16 * wave + (lane & 15);
    auto xrow_of = [&](int p) { p = p < cnt ? p : 0; return a.xrow ? a.xrow[m0 + p] : m0 + p; };
    // Per step (256 values): the X rows of the pass's positions (thread: 4 16-byte chunks), their scales and the
    // rows' 272 bytes of weights (thread: QW words of the rows' 4-byte-aligned covers) go through registers, the next
    // step's loads in flight while this one is computed from LDS.
    constexpr int QW = (Q8_ROWS * (Q8_RP / 4) + 255) / 256;
    v4i xv[Q8_POS * 16 / 256];
    uint32_t wv[QW];
    float dxv = 0.0f;
    for (int p0 = 0; p0 < cnt; p0 += Q8_POS) {
        uint32_t xoff[Q8_POS * 16 / 256];
#pragma unroll
        for (int u = 0; u < Q8_POS * 16 / 256; u++) {
            const int c = tid + 256 * u, p = c >> 4, ch = c & 15;
            xoff[u] = (uint32_t)xrow_of(p0 + p) * (uint32_t)cols + 16 * ch;
        }
        const uint32_t dxo = (uint32_t)xrow_of(p0 + (tid & (Q8_POS - 1))) * (uint32_t)(cols / 32);
        auto fetch = [&](int sb) {
#pragma unroll
            for (int u = 0; u < Q8_POS * 16 / 256; u++) xv[u] = *gptr<v4i>((uint64_t)(a.xq + xoff[u] + 256 * sb));
            if (tid < Q8_POS) dxv = *gptr<float>((uint64_t)(a.xd + dxo + 8 * sb));
#pragma unroll
            for (int u = 0; u < QW; u++) {
                const int c = tid + 256 * u, r = c / (Q8_RP / 4), j = c % (Q8_RP / 4);
                const uint64_t beg = w + (uint64_t)min(n0 + min(r, Q8_ROWS - 1), a.rows - 1) * a.rb + (uint64_t)sb * Q8_SB;
                const uint64_t a4 = beg & ~(uint64_t)3;
                wv[u] = 0;
                if (c < Q8_ROWS * (Q8_RP / 4) && a4 + 4 * (uint64_t)j < beg + Q8_SB) wv[u] = *gptr<uint32_t>(a4 + 4 * (uint64_t)j);
            }
        };
        float acc[Q8_NT][4];
#pragma unroll
        for (int i = 0; i < Q8_NT; i++)
#pragma unroll
            for (int q = 0; q < 4; q++) acc[i][q] = 0.0f;
        fetch(0);
        for (int sb = 0; sb < nsb; sb++) {
            __syncthreads();  // the previous step's readers are done
            // X: Q8_POS positions x 256 bytes, 16-byte chunk c of position p at chunk c ^ (p & 15)
#pragma unroll
            for (int u = 0; u < Q8_POS * 16 / 256; u++) {
                const int c = tid + 256 * u, p = c >> 4, ch = c & 15;
                *(v4i*)(xs8 + p * 256 + 16 * (ch ^ (p & 15))) = xv[u];
            }
            if (tid < Q8_POS) dx8[tid] = dxv;
#pragma unroll
            for (int u = 0; u < QW; u++) {
                const int c = tid + 256 * u;
                if (c < Q8_ROWS * (Q8_RP / 4)) *(uint32_t*)(ws8 + 4 * c) = wv[u];
            }
            __syncthreads();
            if (sb + 1 < nsb) fetch(sb + 1);
            const uint64_t rbeg = w + (uint64_t)min(n0 + rl, a.rows - 1) * a.rb + (uint64_t)sb * Q8_SB;
            const uint8_t* wr = ws8 + rl * Q8_RP + (uint32_t)(rbeg & 3);
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                // this lane's 16 values: block 2 kk + kl / 2, values 16 (kl & 1) ..
                uint32_t qv[4];
                words_a2<4>(wr + 34 * (2 * kk + (kl >> 1)) + 2 + 16 * (kl & 1), qv);
                const v4i qw = {(int)qv[0], (int)qv[1], (int)qv[2], (int)qv[3]}, z = {0, 0, 0, 0};
                const v4i b0 = kl < 2 ? qw : z, b1 = kl < 2 ? z : qw;
                const float d0 = h16(wr + 34 * (2 * kk)), d1 = h16(wr + 34 * (2 * kk + 1));
                // the 2 Q8_NT MFMAs first, then their closes (each result is used 2 Q8_NT issues after its MFMA)
                v4i c0[Q8_NT], c1[Q8_NT];
#pragma unroll
                for (int i = 0; i < Q8_NT; i++) {
                    const v4i av = *(const v4i*)(xs8 + (16 * i + aswz) * 256 + 16 * ((4 * kk + kl) ^ aswz));
                    c0[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b0, z, 0, 0, 0);
                    c1[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b1, z, 0, 0, 0);
                }
#pragma unroll
                for (int i = 0; i < Q8_NT; i++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {  // sum += (d dx) s per 32-block, in order (src/cpu_moe.rs:319-325)
                        const float dxq = dx8[16 * i + 4 * kl + q];
                        acc[i][q] = acc[i][q] + (d0 * dxq) * (float)c0[i][q];
                        acc[i][q] = acc[i][q] + (d1 * dxq) * (float)c1[i][q];
                    }
            }
        }
        // outputs: weight row n0 + rl, positions p0 + 16 i + 4 kl + q
        if (n0 + rl < a.rows) {
#pragma unroll
            for (int i = 0; i < Q8_NT; i++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int m = p0 + 16 * i + 4 * kl + q;
                    if (m < cnt) {
                        float* yp = a.y + (int64_t)(m0 + m) * a.y_stride + n0 + rl;
                        if (a.act == STRATA_ACT_STORE) *yp = acc[i][q];
                        else if (a.act == STRATA_ACT_SWIGLU) *yp = silu_dev(*yp) * acc[i][q];
                        else *yp += acc[i][q];
                    }
                }
        }
    }
}

static hipError_t gemm_q8_0(const GemmLaunch& g, hipStream_t s) {
    GemmArgs a{};
    a.tiles = g.tiles; a.n_tiles_dev = g.n_tiles_dev; a.dense_w = g.dense_w; a.dense_n = g.dense_n;
    a.xq = (const int8_t*)g.xq; a.xd = (const float*)(g.xq + (uint64_t)g.n_x * g.cols);
    a.xrow = g.xrow; a.y = g.y; a.y_stride = g.y_stride; a.rows = g.rows; a.cols = g.cols; a.act = g.act;
    a.rb = row_bytes(Q8_0, g.cols);
    a.max_tiles = g.n_tiles;
    if (g.n_tiles > 65535) return hipErrorInvalidValue;
    gemm_q8_0_kernel<<<dim3((unsigned)((g.rows + Q8_ROWS - 1) / Q8_ROWS), (unsigned)g.n_tiles), 256, 0, s>>>(a);
    return hipGetLastError();
}

uint64_t gemm_block_positions() { return GM; }

hipError_t launch_gemm(const GemmLaunch& g, hipStream_t s) {
    if (g.small && g.tiles && g.ty != Q8_0) return launch_gemm_small(g, s);
    switch (g.ty) {
    case Q8_0: return gemm_q8_0(g, s);
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

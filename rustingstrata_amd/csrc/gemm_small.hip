// Grouped GEMM on int8 MFMA for tile lists whose tiles hold a few dozen positions (a 512-token MoE layer over 128
// experts routes ~32 rows to an expert): the same products and the same bits as gemm_kernel (gemm.hip; reference
// kernels gemmi_q / gemms_*, src/cuda/kernels.cu:1355-1497, chosen by tile size in src/cuda/mod.rs:587-620).
//
// With few positions a block's super-block step is short (the 16 rows a wave decodes, then one or two MFMA tile
// pairs), so a weight load issued one step ahead does not land in time. This kernel keeps two steps in flight:
//   * a block takes 64 positions x 128 weight rows (8 waves, 16 rows each, as gemm_kernel; pair mode 64 gate + 64 up);
//   * X rows and their scales sit in a ring of three LDS buffers, raw weights in two per wave, and step g issues the
//     loads of step g + 2 (X and scales between its decode units, its own weight rows right after its decode);
//   * every wave issues the same number of loads each step (positions past a tile's count load its first row, weight
//     chunks a row does not need reload its first chunk into the wave's padded region), so the end of step g waits
//     with vmcnt for step g + 1's loads alone, and the block barrier does not drain step g + 2's;
//   * a tile of more than 64 positions runs as consecutive 64-position chunks (any tile list is computed whole; the
//     fast case is a tile list built with chunks of 64, strata_moe_sort's chunk = 64).
// Each wave keeps its own copy of a step's 64 X scales (one 4-byte load-to-LDS per lane), so scales need no barrier.
#include <algorithm>

#include "gemm_dev.h"
#include "../../include/strata_hip.h"

namespace strata {

namespace {
constexpr int SM = 64;                  // positions per block
constexpr int SN = 128;                 // weight rows per block (pair: 64 + 64)
constexpr int SW = 8;                   // waves per block
constexpr int STT = SM / 16;            // MFMA position tiles per block
constexpr int SXB = SM * 256;           // bytes of one X buffer
constexpr int SXI = SM * 16 / 64 / SW;  // X load instructions per wave and step
constexpr int NXB = 3;                  // X (and scale) buffers: steps g, g + 1, g + 2
constexpr int SDX = SW * SM;            // floats of one scale buffer (a copy per wave)
}  // namespace

template <int T> struct SmallFmt : GemmPlanes<T> {
    static constexpr int WI = (16 * GemmPlanes<T>::NCH + 63) / 64;  // weight load instructions per wave and step
    static constexpr int WREG = 64 * WI * 16;                        // LDS bytes of a wave's raw rows (whole instructions)
    static constexpr int WBUF = SW * WREG;                           // bytes of one raw weight buffer
    static constexpr int NLOAD = SXI + WI + 1;                       // loads per wave and step
};

// Scale-after decode for the formats whose scales are per 32-value group (Q4_K, Q5_K, IQ3_S, IQ4_XS): the
// weights enter the MFMA as their raw int8 codes q (|q| <= 127), one K=32 MFMA (v_mfma_i32_16x16x32_i8) per group
// gives each group's exact sum d_g = q . x, and the close forms s = sum_g sc_g d_g in int32: the same integer as the
// digit planes' 256 H.x + L.x, so the same bits, with a fraction of the decode work (no per-value scale product and
// byte split). Group g's values 8 kl .. 8 kl + 7 (lane group kl) of the row at b go to q[0..1]; sc the group's integer
// scale, m its min (formats with mins). Layouts: src/quant/mod.rs (Q4_K 209-221, Q5_K 223-237, IQ2_XXS 287-297,
// IQ3_S 345-361, IQ4_XS 363-376). Measured on the 512-token GEMMs: Q5_K gate/up 172-177 -> 164 us, IQ3_S 0.112-0.116
// -> 0.092 ms, IQ4_XS 0.089-0.097 -> 0.083 ms.
template <int T> struct Dsa {
    static constexpr bool ON = false;
};
template <bool Q5> struct DsaQ45 {
    static constexpr bool ON = true, MIN = true;
    struct Row { uint32_t sc_lo, sc_hi, m_lo, m_hi; uint2 qh; };
    __device__ static Row row(const uint8_t* b, int kl) {
        const uint4 h = *(const uint4*)b;  // d, dmin, 12 bytes of packed 6-bit scales / mins (scale_min_k4)
        Row r;
        r.sc_lo = h.y & 0x3F3F3F3Fu;
        r.m_lo = h.z & 0x3F3F3F3Fu;
        r.sc_hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
        r.m_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
        if constexpr (Q5) r.qh = *(const uint2*)(b + 16 + 8 * kl);
        return r;
    }
    __device__ static void run(const uint8_t* b, const Row& r, int g, int kl, const IqTables*, uint32_t* q, int& sc, int& m) {
        const uint2 w = *(const uint2*)(b + (Q5 ? 48 : 16) + 32 * (g >> 1) + 8 * kl);
        const uint32_t ws[2] = {w.x, w.y}, hs[2] = {r.qh.x, r.qh.y};
#pragma unroll
        for (int i = 0; i < 2; i++) {
            q[i] = (ws[i] >> (4 * (g & 1))) & 0x0F0F0F0Fu;
            // bit g of each qh byte to bit 4: a rotate right by g - 4 (mod 32), masked
            if constexpr (Q5) q[i] |= __builtin_amdgcn_alignbit(hs[i], hs[i], (uint32_t)(g + 28) & 31) & 0x10101010u;
        }
        sc = (int)(((g < 4 ? r.sc_lo : r.sc_hi) >> (8 * (g & 3))) & 0xFF);
        m = (int)(((g < 4 ? r.m_lo : r.m_hi) >> (8 * (g & 3))) & 0xFF);
    }
};
template <> struct Dsa<Q4_K> : DsaQ45<false> {};
template <> struct Dsa<Q5_K> : DsaQ45<true> {};
// (IQ2_XXS keeps the digit planes: its per-group header reads made this form slower, 0.105 -> 0.126 ms for the
// configs[3] 512-token GEMM)
template <> struct Dsa<IQ2_XXS> {
    static constexpr bool ON = false, MIN = false;
    struct Row {};
    __device__ static Row row(const uint8_t*, int) { return Row{}; }
    // group g: grid entry kl of the 4 (8 values with its 7-bit sign index); sc = 2 ls + 1
    __device__ static void run(const uint8_t* b, const Row&, int g, int kl, const IqTables* tab, uint32_t* q, int& sc, int& m) {
        const uint32_t gi = rd32<2>(b + 2 + 8 * g), aux = rd32<2>(b + 6 + 8 * g);
        const uint64_t grid = tab->iq2xxs[(gi >> (8 * kl)) & 255];
        const uint32_t sg = tab->ksigns[(aux >> (7 * kl)) & 127];
        q[0] = (uint32_t)neg_bytes((uint32_t)grid, sg);
        q[1] = (uint32_t)neg_bytes((uint32_t)(grid >> 32), sg >> 4);
        sc = (int)(2 * (aux >> 28) + 1);
        m = 0;
    }
};
template <> struct Dsa<IQ3_S> {
    static constexpr bool ON = true, MIN = false;
    struct Row {};
    __device__ static Row row(const uint8_t*, int) { return Row{}; }
    // group g: grid pair kl (two 4-value entries, 9-bit indices with a qh bit), sign byte kl; sc = 1 + 2 nibble
    __device__ static void run(const uint8_t* b, const Row&, int g, int kl, const IqTables* tab, uint32_t* q, int& sc, int& m) {
        const uint32_t q2 = rd16(b + 2 + 8 * g + 2 * kl), hb = b[66 + g], sg = b[74 + 4 * g + kl];
        const uint32_t g1 = tab->iq3s[(q2 & 255) | ((hb << (8 - 2 * kl)) & 256)];
        const uint32_t g2 = tab->iq3s[((q2 >> 8) & 255) | ((hb << (7 - 2 * kl)) & 256)];
        q[0] = (uint32_t)neg_bytes(g1, sg);
        q[1] = (uint32_t)neg_bytes(g2, sg >> 4);
        sc = (int)(1 + 2 * ((b[106 + (g >> 1)] >> (4 * (g & 1))) & 0xF));
        m = 0;
    }
};
template <> struct Dsa<IQ4_XS> {
    static constexpr bool ON = true, MIN = false;
    struct Row { uint32_t sh; };
    __device__ static Row row(const uint8_t* b, int) { return Row{rd16(b + 2)}; }
    // group g: values 0..15 are the low nibbles of its 16 bytes, 16..31 the high ones; sc = ls - 32
    __device__ static void run(const uint8_t* b, const Row& r, int g, int kl, const IqTables*, uint32_t* q, int& sc, int& m) {
        const uint2 w = *(const uint2*)(b + 8 + 16 * g + 8 * (kl & 1));
        q[0] = (uint32_t)iq4nl_lut((w.x >> (4 * (kl >> 1))) & 0x0F0F0F0Fu);
        q[1] = (uint32_t)iq4nl_lut((w.y >> (4 * (kl >> 1))) & 0x0F0F0F0Fu);
        sc = (int)(((b[4 + (g >> 1)] >> (4 * (g & 1))) & 0xF) | (((r.sh >> (2 * g)) & 3) << 4)) - 32;
        m = 0;
    }
};

template <int T>
__global__ __launch_bounds__(64 * SW, 1) void gemm_small_kernel(GemmArgs a) {
    using F = SmallFmt<T>;
    constexpr int NP = F::NP, SBB = sb_bytes(T), NCH = F::NCH, RAWP = F::RAWP, WI = F::WI, WREG = F::WREG,
                  WBUF = F::WBUF, NLOAD = F::NLOAD;
    constexpr int P_HI = 0, P_LO = F::HI ? 1 : 0, P_M = F::HI ? 2 : 1;
    constexpr bool IQ = T == IQ2_XXS || T == IQ3_S;
    static_assert(NCH <= 15 && WI <= 8, "chunk numbers of a lane's weight instructions fit one word");
    static_assert(SBB < 225, "the no-chunk number 15 lands past every super-block");
    static_assert(SXI == 2, "the decode hook issues two X instructions and the scales");
    extern __shared__ __align__(16) uint8_t smem[];
    // LDS: [X: NXB x SXB][scales: NXB x SDX floats][raw W: 2 x WBUF][IqTables]
    int8_t* xs = (int8_t*)smem;
    float* dxs = (float*)(smem + NXB * SXB);
    uint8_t* raw = (uint8_t*)(dxs + NXB * SDX);
    IqTables* tab = (IqTables*)(raw + 2 * WBUF);

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int cols = a.cols, nsb = cols / 256;

    // Items (tile, row block), item = tile * nrb + row block, dealt round the whole grid: with tiles this small the
    // items' costs vary with their expert's load, and one range for the grid balances the blocks better than giving
    // each XCD a contiguous range (measured 0.285 -> 0.268 ms for a 512-token layer's grouped GEMMs). Tile lists of
    // up to 512 tiles are planned (plan_items: larger tiles first, in a snake over the blocks; the slowest block of the
    // 512-token gate/up GEMM ended at 1.26x the mean block's end time with the items in index order); longer ones
    // deal block b the items b, b + grid, ... A tile of more than 64 positions runs as consecutive 64-position chunks
    // of its item.
    const int cnt0 = a.bal >= 0 ? plan_load(a.tiles, a.max_tiles) : 0;  // requested with the count
    const int ntiles = a.n_tiles_dev ? min(sload(a.n_tiles_dev), a.max_tiles) : a.max_tiles;
    const bool pair = a.pair != 0;
    const int GNO = pair ? SN / 2 : SN;
    const int nrb = (a.rows + GNO - 1) / GNO, total = nrb * ntiles;
    const int ibeg = blockIdx.x, gstep = gridDim.x;
    int mine = 0, ns = -1;
    if (a.bal >= 0 && ntiles <= 64 * SW) {
        int ia, ib;
        static_assert(PLAN_INTS * 4 <= SXB, "the plan fits X slot 2, first written after the first barrier");
        ns = plan_items<SW>(cnt0, ntiles, nrb, a.bal, 1, 0, ibeg, gstep, (int*)(xs + 2 * SXB), ia, ib, mine);
    }
    const bool mine_ok = ns >= 0;
    const int nitems = mine_ok ? ns : ibeg < total ? (total - ibeg + gstep - 1) / gstep : 0;

    struct Item {
        uint64_t w;
        int m0, cnt, n0;  // cnt 0: no item
        int rest;         // positions of the tile after this chunk
    };
    // chunk pc of item k (k < nitems)
    auto item_at = [&](int k, int pc) __attribute__((always_inline)) {
        Item it;
        const int id = mine_ok ? __builtin_amdgcn_readlane(mine, k) : ibeg + k * gstep, tile = id / nrb;
        it.n0 = (id - tile * nrb) * GNO;
        const uint64_t t0 = sload(a.tiles + 2 * tile), t1 = sload(a.tiles + 2 * tile + 1);
        const int cnt = min(256, (int)(t1 >> 32)) - SM * pc;
        it.w = t0;
        it.m0 = (int)(uint32_t)t1 + SM * pc;
        it.cnt = max(0, min(SM, cnt));
        it.rest = cnt - it.cnt;
        return it;
    };
    // the next chunk with positions: chunk pc + 1 of item k while the tile has positions left, else the first chunk
    // of the next item with positions (cnt 0 past the last item)
    auto next_item = [&](int& k, int& pc, const Item& prev) __attribute__((always_inline)) {
        if (prev.rest > 0) {
            ++pc;
            return item_at(k, pc);
        }
        Item it{0, 0, 0, 0, 0};
        pc = 0;
        for (++k; k < nitems; k++) {
            it = item_at(k, 0);
            if (it.cnt > 0) break;
        }
        return it;
    };

    if constexpr (IQ) load_iq_tables(tab);

    struct Addr {
        uint32_t xo[SXI];  // X byte offsets of this lane's two position rows (+ chunk)
        uint32_t dxo;      // byte offset of the scales of position `lane`
        uint32_t rbeg;     // this lane's decode row: byte offset from W, plus W mod 16
        uint32_t wro[WI];  // byte offsets from W of the rows of this lane's weight chunks
    };
    const int rl = 16 * wave + (lane & 15);
    const int wlim = 16 * NCH;
    auto wchunk = [&](int i) __attribute__((always_inline)) { return 64 * i + lane; };
    auto addr_of = [&](const Item& it) __attribute__((always_inline)) {
        Addr ad;
        auto xrow_of = [&](int p) { p = p < it.cnt ? p : 0; return a.xrow ? a.xrow[it.m0 + p] : it.m0 + p; };
#pragma unroll
        for (int j = 0; j < SXI; j++) {
            const int p = 4 * (SXI * wave + j) + (lane >> 4);
            ad.xo[j] = (uint32_t)xrow_of(p) * (uint32_t)cols + 16 * ((lane & 15) ^ (p & 15));
        }
        ad.dxo = 4u * (uint32_t)xrow_of(lane) * (uint32_t)(cols / 32);
        ad.rbeg = (uint32_t)(it.w & 15) + (pair && wave >= 4 ? (uint32_t)(a.w2 & 15) : 0u) +
                  __umul24((uint32_t)min(it.n0 + (pair ? (rl & 63) : rl), a.rows - 1), (uint32_t)a.rb);
#pragma unroll
        for (int i = 0; i < WI; i++)
            ad.wro[i] = __umul24((uint32_t)min(it.n0 + ((16 * wave + min(wchunk(i) / NCH, 15)) & (GNO - 1)), a.rows - 1),
                                 (uint32_t)a.rb);
        return ad;
    };
    uint32_t wcc = 0;  // chunk number within its row of each weight instruction's chunk (15: none)
#pragma unroll
    for (int i = 0; i < WI; i++) wcc |= (uint32_t)(wchunk(i) < wlim ? wchunk(i) % NCH : 15) << (4 * i);

    // The loads of one step; every call issues exactly SXI, 1 and WI instructions.
    auto load_x = [&](const Addr& ad, int s, int xb, const int j) __attribute__((always_inline)) {
        load_lds16_so((uint64_t)(a.xq + 256 * s), ad.xo[j], xs + xb * SXB + 1024 * (SXI * wave + j));
    };
    auto load_dx = [&](const Addr& ad, int s, int xb) __attribute__((always_inline)) {
        load_lds4_so((uint64_t)(a.xd + 8 * s), ad.dxo, dxs + xb * SDX + SM * wave);
    };
    auto load_w = [&](const Item& it, const Addr& ad, int s, int wb) __attribute__((always_inline)) {
        const uint64_t beg = it.w + (pair && wave >= 4 ? (uint64_t)a.w2 : 0) + (uint64_t)s * SBB, base = beg & ~(uint64_t)15;
        const uint32_t b15 = (uint32_t)(beg & 15);
        uint8_t* dst = raw + wb * WBUF + wave * WREG;
#pragma unroll
        for (int i = 0; i < WI; i++) {
            const uint32_t t = b15 + ad.wro[i];
            uint32_t o = (t & ~15u) + 16 * ((wcc >> (4 * i)) & 15);
            if (o >= t + SBB) o = t & ~15u;  // a chunk the row does not need: its first chunk again
            load_lds16_so(base, o, dst + 16 * 64 * i);
        }
    };

    float acc[STT][4];
#pragma unroll
    for (int i = 0; i < STT; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) acc[i][q] = 0.0f;
    const int kl = lane >> 4, aswz = lane & 15;
    constexpr bool SA = Dsa<T>::ON;
    v4i B[4][NP];
    // scale-after form: the 8 groups' codes (8 bytes a lane each), integer scales and min words
    uint32_t Bq[8][2], Bm[8];
    int scg[8];
    float D = 0.0f, M = 0.0f;
    auto decode = [&](uint32_t rbeg, int s, int wb, auto&& hook) __attribute__((always_inline)) {
        const uint8_t* b = raw + wb * WBUF + wave * WREG + (lane & 15) * RAWP + ((rbeg + (uint32_t)s * SBB) & 15);
        if constexpr (SA) {
            using DS = Dsa<T>;
            const auto r = DS::row(b, kl);
#pragma unroll
            for (int g = 0; g < 8; g++) {
                int m;
                DS::run(b, r, g, kl, tab, Bq[g], scg[g], m);
                if constexpr (DS::MIN) Bm[g] = (uint32_t)m * 0x01010101u;
                if (g & 1) hook(g >> 1);
            }
            Dec<T>::scales(b, D, M);
            return;
        }
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
    auto mfma_pair = [&](const int i, int xb, v4i (&c0)[NP], v4i (&c1)[NP]) __attribute__((always_inline)) {
        const int8_t* xp = xs + xb * SXB;
        v4i a0[4], a1[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            a0[kk] = *(const v4i*)(xp + (16 * i + aswz) * 256 + 16 * ((4 * kk + kl) ^ aswz));
            a1[kk] = *(const v4i*)(xp + (16 * (i + 1) + aswz) * 256 + 16 * ((4 * kk + kl) ^ aswz));
        }
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int pl = 0; pl < NP; pl++) {
                c0[pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0[kk], B[kk][pl], kk ? c0[pl] : (v4i){0, 0, 0, 0}, 0, 0, 0);
                c1[pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[kk], B[kk][pl], kk ? c1[pl] : (v4i){0, 0, 0, 0}, 0, 0, 0);
            }
    };
    // the reference's float steps, rounded one by one (src/cpu_moe.rs:327-377): sum += (D dx) s - (M dx) m
    auto close_pair = [&](const int i, int xb, const v4i (&c0)[NP], const v4i (&c1)[NP]) __attribute__((always_inline)) {
        const float* dw = dxs + xb * SDX + SM * wave;
        const float4 d0 = *(const float4*)(dw + 16 * i + 4 * kl);
        const float4 d1 = *(const float4*)(dw + 16 * (i + 1) + 4 * kl);
        const float dq0[4] = {d0.x, d0.y, d0.z, d0.w}, dq1[4] = {d1.x, d1.y, d1.z, d1.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int iv0 = F::HI ? (c0[P_HI][q] << 8) + c0[P_LO][q] : c0[P_LO][q];
            const int iv1 = F::HI ? (c1[P_HI][q] << 8) + c1[P_LO][q] : c1[P_LO][q];
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
    auto mfma_one = [&](const int i, int xb, v4i (&c0)[NP]) __attribute__((always_inline)) {
        const int8_t* xp = xs + xb * SXB;
        v4i a0[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) a0[kk] = *(const v4i*)(xp + (16 * i + aswz) * 256 + 16 * ((4 * kk + kl) ^ aswz));
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int pl = 0; pl < NP; pl++)
                c0[pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0[kk], B[kk][pl], kk ? c0[pl] : (v4i){0, 0, 0, 0}, 0, 0, 0);
    };
    auto close_one = [&](const int i, int xb, const v4i (&c0)[NP]) __attribute__((always_inline)) {
        const float4 d0 = *(const float4*)(dxs + xb * SDX + SM * wave + 16 * i + 4 * kl);
        const float dq0[4] = {d0.x, d0.y, d0.z, d0.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int iv0 = F::HI ? (c0[P_HI][q] << 8) + c0[P_LO][q] : c0[P_LO][q];
            float f0 = (D * dq0[q]) * (float)iv0;
            if constexpr (F::MIN) f0 = f0 - (M * dq0[q]) * (float)c0[P_M][q];
            acc[i][q] = acc[i][q] + f0;
        }
    };
    // scale-after tile i: group g's K=32 MFMA on the A fragment X[p][32 g + 8 kl .. + 7] (8 bytes), the min chain
    // over the groups with B = the group's min (formats with mins), then s = sum_g sc_g d_g and the float close
    auto tile_sa = [&](const int i, int xb) __attribute__((always_inline)) {
        const int8_t* xp = xs + xb * SXB + (16 * i + aswz) * 256 + 8 * (kl & 1);
        long af[8];
#pragma unroll
        for (int g = 0; g < 8; g++) af[g] = *(const long*)(xp + 16 * ((2 * g + (kl >> 1)) ^ aswz));
        v4i d[8], mn = (v4i){0, 0, 0, 0};
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const long bq = (long)(((uint64_t)Bq[g][1] << 32) | Bq[g][0]);
            d[g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[g], bq, (v4i){0, 0, 0, 0}, 0, 0, 0);
            if constexpr (F::MIN) {
                const long bm = (long)(((uint64_t)Bm[g] << 32) | Bm[g]);
                mn = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[g], bm, mn, 0, 0, 0);
            }
        }
        const float4 d0 = *(const float4*)(dxs + xb * SDX + SM * wave + 16 * i + 4 * kl);
        const float dq0[4] = {d0.x, d0.y, d0.z, d0.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            int sv = __mul24(scg[0], d[0][q]);
#pragma unroll
            for (int g = 1; g < 8; g++) sv += __mul24(scg[g], d[g][q]);
            // the reference's float steps, rounded one by one (src/cpu_moe.rs:327-377): sum += (D dx) s - (M dx) m
            float f0 = (D * dq0[q]) * (float)sv;
            if constexpr (F::MIN) f0 = f0 - (M * dq0[q]) * (float)mn[q];
            acc[i][q] = acc[i][q] + f0;
        }
    };
    auto tiles = [&](int xb, int ntt) __attribute__((always_inline)) {
        if constexpr (SA) {
            static_for<0, STT>([&](auto I) {
                constexpr int i = decltype(I)::value;
                if (i < ntt) tile_sa(i, xb);
            });
            return;
        }
        static_for<0, STT / 2>([&](auto I) {
            constexpr int i = 2 * decltype(I)::value;
            if (i + 1 < ntt) {
                v4i c0[NP], c1[NP];
                mfma_pair(i, xb, c0, c1);
                close_pair(i, xb, c0, c1);
            } else if (i < ntt) {
                v4i c0[NP];
                mfma_one(i, xb, c0);
                close_one(i, xb, c0);
            }
        });
    };
    // Results of an item. Pair mode: the up waves (4-7) stage their outputs in the X buffer of this step, the gate
    // waves (0-3) store silu(gate) x up for their (row, position) outputs. Otherwise each lane stores its own values.
    auto store = [&](const Item& it, int xb) __attribute__((always_inline)) {
        const int ntt = (it.cnt + 15) >> 4;
        const int col = pair ? (rl & 63) : rl;
        float* yb = a.y + (int64_t)(it.m0 + 4 * kl) * a.y_stride + it.n0 + col;
        const int left = it.cnt - 4 * kl;
        if (pair) {
            float* S = (float*)(xs + xb * SXB);  // [64 positions][64 columns], column XOR-swizzled by 16 kl
            lds_barrier();                        // every wave's tiles are done with this X buffer
            if (wave >= 4) {
                static_for<0, STT>([&](auto I) {
                    constexpr int i = decltype(I)::value;
#pragma unroll
                    for (int q = 0; q < 4; q++) S[(16 * i + 4 * kl + q) * 64 + (col ^ (kl << 4))] = acc[i][q];
                });
            }
            lds_barrier();
            if (wave < 4) {
                static_for<0, STT>([&](auto I) {
                    constexpr int i = decltype(I)::value;
                    if (i < ntt) {
#pragma unroll
                        for (int q = 0; q < 4; q++)
                            if (16 * i + q < left)
                                yb[(int64_t)(16 * i + q) * a.y_stride] =
                                    silu_dev(acc[i][q]) * S[(16 * i + 4 * kl + q) * 64 + (col ^ (kl << 4))];
                    }
                });
            }
        } else if (it.n0 + rl < a.rows) {
            auto put = [&](auto OP) __attribute__((always_inline)) {
                constexpr int op = decltype(OP)::value;
                static_for<0, STT>([&](auto I) {
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
        for (int i = 0; i < STT; i++)
#pragma unroll
            for (int q = 0; q < 4; q++) acc[i][q] = 0.0f;
    };

    // The step stream: cur (step g), q1 (step g + 1) and the load state L (step g + 2: item index kL, super-block sL).
    struct Step {
        Item it;
        uint32_t rbeg;
        int s;
    };
    int kL = -1, pcL = 0, sL = 0;
    Item iL = next_item(kL, pcL, Item{0, 0, 0, 0, 0});
    if (iL.cnt == 0) return;  // no work: no load was issued
    Addr aL = addr_of(iL);
    auto advance = [&]() __attribute__((always_inline)) {
        if (++sL == nsb) {
            sL = 0;
            iL = next_item(kL, pcL, iL);
            if (iL.cnt) aL = addr_of(iL);
        }
    };
    auto issue_all = [&](int xb, int wb) __attribute__((always_inline)) {
        load_x(aL, sL, xb, 0);
        load_x(aL, sL, xb, 1);
        load_dx(aL, sL, xb);
        load_w(iL, aL, sL, wb);
    };
    // prologue: steps 0 and 1
    Step cur{iL, aL.rbeg, sL};
    issue_all(0, 0);
    advance();
    Step q1{iL, aL.rbeg, sL};
    if (iL.cnt) {
        issue_all(1, 1);
        advance();
        wait_vm<NLOAD>();
    } else {
        wait_vm<0>();
    }
    __syncthreads();  // the IQ tables and step 0's X

    int xb = 0, wb = 0;  // buffers of step g
    while (true) {
        const bool l2 = iL.cnt != 0;  // step g + 2 exists
        const int xb2 = xb == 0 ? 2 : xb - 1;
        decode(cur.rbeg, cur.s, wb, [&](int kk) __attribute__((always_inline)) {
            if (l2) {
                if (kk < SXI) load_x(aL, sL, xb2, kk);
                else if (kk == SXI) load_dx(aL, sL, xb2);
            }
        });
        wait_lds();  // this wave's reads of its raw rows are done: step g + 2's rows take the buffer
        if (l2) load_w(iL, aL, sL, wb);
        tiles(xb, (cur.it.cnt + 15) >> 4);
        const bool last = cur.s + 1 == nsb;
        if (last) store(cur.it, xb);
        if (q1.it.cnt == 0) break;  // step g was the block's last
        cur = q1;
        if (l2) {
            q1 = Step{iL, aL.rbeg, sL};
            advance();
        } else {
            q1.it.cnt = 0;
        }
        // step g + 1's loads have landed (step g + 2's may still fly, unless an item's stores were issued after them)
        if (last || !l2) wait_vm<0>();
        else wait_vm<NLOAD>();
        lds_barrier();
        xb = xb == 2 ? 0 : xb + 1;
        wb ^= 1;
    }
}

template <int T>
static size_t gemm_small_smem() {
    size_t b = (size_t)NXB * SXB + (size_t)NXB * SDX * 4 + 2 * (size_t)SmallFmt<T>::WBUF;
    if (T == IQ2_XXS || T == IQ3_S) b += sizeof(IqTables);
    return b;
}

template <int T>
static hipError_t gemm_small_t(const GemmLaunch& g, hipStream_t s) {
    GemmArgs a{};
    a.tiles = g.tiles; a.n_tiles_dev = g.n_tiles_dev;
    a.xq = (const int8_t*)g.xq; a.xd = (const float*)(g.xq + (uint64_t)g.n_x * g.cols);
    a.xrow = g.xrow; a.y = g.y; a.y_stride = g.y_stride; a.rows = g.rows; a.cols = g.cols; a.act = g.act;
    a.pair = g.pair ? 1 : 0;
    a.w2 = g.w2;
    a.rb = row_bytes(T, g.cols);
    a.max_tiles = g.n_tiles;
    a.bal = 4;  // the items' plan orders them by position tiles only (one range for the grid: no cost split)
    const size_t smem = gemm_small_smem<T>();
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)gemm_small_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
        attr = true;
    }
    static int ncu = 0;
    if (!ncu) {
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
    }
    const int gno = g.pair ? SN / 2 : SN;
    const long long total = (long long)((g.rows + gno - 1) / gno) * g.n_tiles;
    if (total >= (1ll << 31)) return hipErrorInvalidValue;
    const long long grid = std::max<long long>(std::min<long long>(total, ncu), 1);  // persistent: one block per CU
    gemm_small_kernel<T><<<dim3((unsigned)grid), 64 * SW, smem, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_gemm_small(const GemmLaunch& g, hipStream_t s) {
    switch (g.ty) {
    case Q2_K: return gemm_small_t<Q2_K>(g, s);
    case Q3_K: return gemm_small_t<Q3_K>(g, s);
    case Q4_K: return gemm_small_t<Q4_K>(g, s);
    case Q5_K: return gemm_small_t<Q5_K>(g, s);
    case Q6_K: return gemm_small_t<Q6_K>(g, s);
    case IQ2_XXS: return gemm_small_t<IQ2_XXS>(g, s);
    case IQ3_S: return gemm_small_t<IQ3_S>(g, s);
    case IQ4_XS: return gemm_small_t<IQ4_XS>(g, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace strata

// Device decoders of the GGUF block formats, in two forms:
//  * dequant32<T>: 32 values of a 256-value super-block as f32, with the reference's float operations in the
//    reference's order (src/quant/mod.rs), so that under -ffp-contract=off the bits are dequant_row's;
//  * task<T>: the integer form the GEMV and GEMM kernels consume. A task is 32 weights of a super-block as int8
//    (8 packed words), split into two groups of 16 whose x positions inside the super-block are o0 and o1; each
//    group has an integer scale sc, an integer min m and a value bias, and the super-block float scales D and M,
//    so that the 16 weights of group g dequantize to D * sc_g * (q - bias) - M * m_g.
//
// Super-block = 256 values: one block of the K and IQ types, 8 consecutive blocks of Q8_0.
#pragma once
#include "common.h"
#define STRATA_TABLE_QUAL static __constant__ const
#include "../../include/strata_iq_tables.h"
#undef STRATA_TABLE_QUAL

namespace strata {

// ---------------------------------------------------------------------------------------------------------
// Byte access. Global memory reads in dequant32 are byte loads; task<T> reads LDS copies whose alignment mod 16
// equals the global one. A is the alignment task<T> may assume for the super-block start.
template <int A>
__device__ __forceinline__ uint32_t rd32(const uint8_t* p) {
    if constexpr (A >= 4) return *(const uint32_t*)p;
    else return (uint32_t)((const uint16_t*)p)[0] | (uint32_t)((const uint16_t*)p)[1] << 16;
}
__device__ __forceinline__ uint32_t rd16(const uint8_t* p) { return *(const uint16_t*)p; }
__device__ __forceinline__ float h16(const uint8_t* p) { return f16_to_f32((uint32_t)p[0] | (uint32_t)p[1] << 8); }

// scale_min_k4 (src/quant/mod.rs:59-62) over the 12 scale bytes at q.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int& s, int& m) {
    if (j < 4) { s = q[j] & 63; m = q[j + 4] & 63; }
    else { s = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4); m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4); }
}
// The same on the three little-endian words of the 12 bytes.
__device__ __forceinline__ void scale_min_k4w(int j, uint32_t w0, uint32_t w1, uint32_t w2, int& s, int& m) {
    uint32_t sh = 8 * (j & 3), a = (w0 >> sh) & 255, c = (w1 >> sh) & 255, e = (w2 >> sh) & 255;
    if (j < 4) { s = a & 63; m = c & 63; }
    else { s = (e & 0xF) | ((a >> 6) << 4); m = (e >> 4) | ((c >> 6) << 4); }
}
// Scale `is` (0..15, bias 32 kept) of a Q3_K block from its 12 scale bytes (q3k_scales, src/quant/mod.rs:173-186).
__device__ __forceinline__ int q3k_scale(const uint8_t* sc, int is) {
    int low = (sc[is & 7] >> (4 * (is >> 3))) & 0xF;
    int hs = (sc[8 + (is & 3)] >> (2 * (is >> 2))) & 3;
    return low | (hs << 4);
}

// The IQ tables, in LDS while a kernel runs (each lane looks up random entries).
struct IqTables {
    uint64_t iq2xxs[256];
    uint32_t iq3s[512];
    uint8_t ksigns[128];
};
// Copy the tables into LDS (all threads of the block take part; the caller synchronises).
__device__ __forceinline__ void load_iq_tables(IqTables* t) {
    for (int i = threadIdx.x; i < 512; i += blockDim.x) {
        t->iq3s[i] = STRATA_IQ3S_GRID[i];
        if (i < 256) t->iq2xxs[i] = STRATA_IQ2XXS_GRID[i];
        if (i < 128) t->ksigns[i] = STRATA_KSIGNS_IQ2XS[i];
    }
}
// The same in two halves for a block of 256 threads: the thread's entries into registers (the loads may then fly with
// the kernel's first weight loads), and later into LDS (the caller synchronises after the store).
struct IqRegs {
    uint32_t g3[2];
    uint64_t g2;
    uint8_t ks;
};
__device__ __forceinline__ IqRegs load_iq_regs() {
    const int i = threadIdx.x;
    IqRegs r;
    r.g3[0] = STRATA_IQ3S_GRID[i];
    r.g3[1] = STRATA_IQ3S_GRID[i + 256];
    r.g2 = STRATA_IQ2XXS_GRID[i];
    r.ks = STRATA_KSIGNS_IQ2XS[i & 127];
    return r;
}
__device__ __forceinline__ void store_iq_regs(IqTables* t, const IqRegs& r) {
    const int i = threadIdx.x;
    t->iq3s[i] = r.g3[0];
    t->iq3s[i + 256] = r.g3[1];
    t->iq2xxs[i] = r.g2;
    if (i < 128) t->ksigns[i] = r.ks;
}

// ---------------------------------------------------------------------------------------------------------
// Exact dequantization of values 32 k .. 32 k + 32 of the super-block at b (global memory).

template <int T> __device__ void dequant32(const uint8_t* b, int k, float* y);

template <> __device__ __forceinline__ void dequant32<Q8_0>(const uint8_t* b, int k, float* y) {  // mod.rs:86
    const uint8_t* p = b + 34 * k;
    float d = h16(p);
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)p[2 + j] * d;
}
template <> __device__ __forceinline__ void dequant32<Q2_K>(const uint8_t* b, int k, float* y) {  // mod.rs:156-170
    float d = h16(b + 80), mn = h16(b + 82);
    int n = k >> 2, shift = 2 * (k & 3);
    for (int half = 0; half < 2; half++) {
        uint8_t s = b[2 * k + half];
        float dl = d * (float)(s & 0xF), ml = mn * (float)(s >> 4);
        for (int l = 0; l < 16; l++) y[16 * half + l] = dl * (float)((b[16 + 32 * n + l + 16 * half] >> shift) & 3) - ml;
    }
}
template <> __device__ __forceinline__ void dequant32<Q3_K>(const uint8_t* b, int k, float* y) {  // mod.rs:188-207
    float d_all = h16(b + 108);
    int n = k >> 2, shift = 2 * (k & 3);
    uint8_t m = (uint8_t)(1u << (4 * n + (k & 3)));
    for (int half = 0; half < 2; half++) {
        float dl = d_all * (float)(q3k_scale(b + 96, 2 * k + half) - 32);
        for (int l = 0; l < 16; l++) {
            int i = l + 16 * half;
            int v = ((b[32 + 32 * n + i] >> shift) & 3) - ((b[i] & m) ? 0 : 4);
            y[i] = dl * (float)v;
        }
    }
}
template <> __device__ __forceinline__ void dequant32<Q4_K>(const uint8_t* b, int k, float* y) {  // mod.rs:209-221
    float d = h16(b), mn = h16(b + 2);
    int s, m;
    scale_min_k4(k, b + 4, s, m);
    float d1 = d * (float)s, m1 = mn * (float)m;
    const uint8_t* q = b + 16 + 32 * (k >> 1);
    int sh = 4 * (k & 1);
    for (int l = 0; l < 32; l++) y[l] = d1 * (float)((q[l] >> sh) & 0xF) - m1;
}
template <> __device__ __forceinline__ void dequant32<Q5_K>(const uint8_t* b, int k, float* y) {  // mod.rs:223-237
    float d = h16(b), mn = h16(b + 2);
    int s, m;
    scale_min_k4(k, b + 4, s, m);
    float d1 = d * (float)s, m1 = mn * (float)m;
    const uint8_t *q = b + 48 + 32 * (k >> 1), *qh = b + 16;
    int sh = 4 * (k & 1);
    uint8_t u = (uint8_t)(1u << k);
    for (int l = 0; l < 32; l++) y[l] = d1 * ((float)((q[l] >> sh) & 0xF) + ((qh[l] & u) ? 16.0f : 0.0f)) - m1;
}
template <> __device__ __forceinline__ void dequant32<Q6_K>(const uint8_t* b, int k, float* y) {  // mod.rs:239-256
    float d = h16(b + 208);
    int n = k >> 2, qd = k & 3;  // values 32 qd + l of half n
    const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n, *sc = b + 192 + 8 * n;
    for (int l = 0; l < 32; l++) {
        int lo = qd & 1 ? ql[l + 32] : ql[l];
        int nib = qd & 2 ? lo >> 4 : lo & 0xF;
        int q = (nib | (((qh[l] >> (2 * qd)) & 3) << 4)) - 32;
        y[l] = d * (float)(int8_t)sc[l / 16 + 2 * qd] * (float)q;
    }
}
template <> __device__ __forceinline__ void dequant32<IQ2_XXS>(const uint8_t* b, int k, float* y) {  // mod.rs:287-297
    float d = h16(b);
    const uint8_t* qs = b + 2 + 8 * k;
    uint32_t aux = (uint32_t)qs[4] | (uint32_t)qs[5] << 8 | (uint32_t)qs[6] << 16 | (uint32_t)qs[7] << 24;
    float db = d * (0.5f + (float)(aux >> 28)) * 0.25f;
    for (int l = 0; l < 4; l++) {
        uint64_t grid = STRATA_IQ2XXS_GRID[qs[l]];
        uint8_t signs = STRATA_KSIGNS_IQ2XS[(aux >> (7 * l)) & 127];
        for (int j = 0; j < 8; j++) y[8 * l + j] = db * (float)(uint8_t)(grid >> (8 * j)) * ((signs >> j) & 1 ? -1.0f : 1.0f);
    }
}
template <> __device__ __forceinline__ void dequant32<IQ3_S>(const uint8_t* b, int k, float* y) {  // mod.rs:345-361
    float d = h16(b);
    float db = d * (float)(1 + 2 * ((b[106 + k / 2] >> (4 * (k % 2))) & 0xF));
    unsigned hb = b[66 + k];
    for (int l = 0; l < 4; l++) {
        uint32_t g1 = STRATA_IQ3S_GRID[b[2 + 8 * k + 2 * l] | ((hb << (8 - 2 * l)) & 256)];
        uint32_t g2 = STRATA_IQ3S_GRID[b[2 + 8 * k + 2 * l + 1] | ((hb << (7 - 2 * l)) & 256)];
        uint8_t sg = b[74 + 4 * k + l];
        for (int j = 0; j < 4; j++) {
            y[8 * l + j] = db * (float)(uint8_t)(g1 >> (8 * j)) * ((sg >> j) & 1 ? -1.0f : 1.0f);
            y[8 * l + j + 4] = db * (float)(uint8_t)(g2 >> (8 * j)) * ((sg >> (j + 4)) & 1 ? -1.0f : 1.0f);
        }
    }
}
template <> __device__ __forceinline__ void dequant32<IQ4_XS>(const uint8_t* b, int k, float* y) {  // mod.rs:363-376
    float d = h16(b);
    unsigned sh = b[2] | b[3] << 8;
    int ls = ((b[4 + k / 2] >> (4 * (k % 2))) & 0xF) | (((sh >> (2 * k)) & 3) << 4);
    float dl = d * (float)(ls - 32);
    for (int j = 0; j < 16; j++) {
        uint8_t q = b[8 + 16 * k + j];
        y[j] = dl * (float)STRATA_KVALUES_IQ4NL[q & 0xF];
        y[j + 16] = dl * (float)STRATA_KVALUES_IQ4NL[q >> 4];
    }
}

// ---------------------------------------------------------------------------------------------------------
// Integer tasks.

struct Task {
    int q[8];        // q[0..3]: group 0 (16 values at o0), q[4..7]: group 1 (16 values at o1); int8 each
    int o0, o1;      // x positions inside the super-block (multiples of 16)
    int sc0, sc1;    // integer scales
    int m0, m1;      // integer mins (0 where the format has none)
    float D, M;      // super-block float scales (M = 0 where the format has no min)
};

// Alignment each format's task<T> needs at the super-block start (gcd of 16 and the super-block bytes).
template <int T> struct Fmt;
template <> struct Fmt<Q8_0> { static constexpr int ALIGN = 2, BIAS = 0; static constexpr bool MIN = false; };
template <> struct Fmt<Q2_K> { static constexpr int ALIGN = 4, BIAS = 0; static constexpr bool MIN = true; };
template <> struct Fmt<Q3_K> { static constexpr int ALIGN = 2, BIAS = 4; static constexpr bool MIN = false; };
template <> struct Fmt<Q4_K> { static constexpr int ALIGN = 16, BIAS = 0; static constexpr bool MIN = true; };
template <> struct Fmt<Q5_K> { static constexpr int ALIGN = 16, BIAS = 0; static constexpr bool MIN = true; };
template <> struct Fmt<Q6_K> { static constexpr int ALIGN = 2, BIAS = 32; static constexpr bool MIN = false; };
template <> struct Fmt<IQ2_XXS> { static constexpr int ALIGN = 2, BIAS = 0; static constexpr bool MIN = false; };
template <> struct Fmt<IQ3_S> { static constexpr int ALIGN = 2, BIAS = 0; static constexpr bool MIN = false; };
template <> struct Fmt<IQ4_XS> { static constexpr int ALIGN = 8, BIAS = 0; static constexpr bool MIN = false; };

template <int T> __device__ void task(const uint8_t* b, int k, const IqTables* tab, Task& t);

template <> __device__ __forceinline__ void task<Q8_0>(const uint8_t* b, int k, const IqTables*, Task& t) {
    const uint8_t* p = b + 34 * k;
#pragma unroll
    for (int j = 0; j < 8; j++) t.q[j] = (int)rd32<2>(p + 2 + 4 * j);
    t.o0 = 32 * k; t.o1 = 32 * k + 16;
    t.sc0 = t.sc1 = 1; t.m0 = t.m1 = 0;
    t.D = f16_to_f32(rd16(p)); t.M = 0.0f;
}
template <> __device__ __forceinline__ void task<Q2_K>(const uint8_t* b, int k, const IqTables*, Task& t) {
    int n = k >> 2, sh = 2 * (k & 3);
    const uint8_t* q = b + 16 + 32 * n;
#pragma unroll
    for (int j = 0; j < 8; j++) t.q[j] = (int)((rd32<4>(q + 4 * j) >> sh) & 0x03030303u);
    uint32_t s2 = rd16(b + 2 * k);  // scale bytes 2k, 2k + 1: low nibble scale, high nibble min
    t.o0 = 32 * k; t.o1 = 32 * k + 16;
    t.sc0 = s2 & 0xF; t.m0 = (s2 >> 4) & 0xF; t.sc1 = (s2 >> 8) & 0xF; t.m1 = (s2 >> 12) & 0xF;
    uint32_t dm = rd32<4>(b + 80);
    t.D = f16_to_f32(dm & 0xFFFF); t.M = f16_to_f32(dm >> 16);
}
// Scales 4 w .. 4 w + 3 of a Q3_K block (q3k_scales, src/quant/mod.rs:173-186) as 4 bytes, each 6-bit scale with
// its bit 5 flipped: as a signed 6-bit field that byte is the scale minus 32.
__device__ __forceinline__ uint32_t q3k_scale_word(const uint8_t* sc, int w) {
    const uint32_t lo = rd32<2>(sc + 4 * (w & 1)), hi = rd32<2>(sc + 8);
    const uint32_t nib = (w & 2 ? lo >> 4 : lo) & 0x0F0F0F0Fu;
    // the 2 high bits of scale 4 w + i are bits 2 w, 2 w + 1 of byte i of hi
    const int s = 4 - 2 * w;
    return (nib | ((s >= 0 ? hi << s : hi >> -s) & 0x30303030u)) ^ 0x20202020u;
}
template <> __device__ __forceinline__ void task<Q3_K>(const uint8_t* b, int k, const IqTables*, Task& t) {
    int n = k >> 2, sh = 2 * (k & 3), hb = 4 * n + (k & 3);
    const uint8_t* q = b + 32 + 32 * n;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        // bit hb of each hmask byte to bit 2 (one shift of the word, then the mask): value + 4
        const uint32_t h = rd32<2>(b + 4 * j), hs = hb <= 2 ? h << (2 - hb) : h >> (hb - 2);
        t.q[j] = (int)(((rd32<2>(q + 4 * j) >> sh) & 0x03030303u) | (hs & 0x04040404u));
    }
    t.o0 = 32 * k; t.o1 = 32 * k + 16;
    const uint32_t scw = q3k_scale_word(b + 96, k >> 1);  // scales 2 k, 2 k + 1: bytes 2 (k & 1), + 1
    t.sc0 = __builtin_amdgcn_sbfe((int)scw, 16 * (k & 1), 6);
    t.sc1 = __builtin_amdgcn_sbfe((int)scw, 16 * (k & 1) + 8, 6);
    t.m0 = t.m1 = 0;
    t.D = f16_to_f32(rd16(b + 108)); t.M = 0.0f;
}
template <> __device__ __forceinline__ void task<Q4_K>(const uint8_t* b, int k, const IqTables*, Task& t) {
    uint4 h = *(const uint4*)b;
    int i = k >> 1, hh = k & 1;
    uint4 w = *(const uint4*)(b + 16 + 32 * i + 16 * hh);
    uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; j++) { t.q[j] = (int)(ws[j] & 0x0F0F0F0Fu); t.q[4 + j] = (int)((ws[j] >> 4) & 0x0F0F0F0Fu); }
    t.o0 = 64 * i + 16 * hh; t.o1 = t.o0 + 32;
    scale_min_k4w(2 * i, h.y, h.z, h.w, t.sc0, t.m0);
    scale_min_k4w(2 * i + 1, h.y, h.z, h.w, t.sc1, t.m1);
    t.D = f16_to_f32(h.x & 0xFFFF); t.M = f16_to_f32(h.x >> 16);
}
template <> __device__ __forceinline__ void task<Q5_K>(const uint8_t* b, int k, const IqTables*, Task& t) {
    uint4 h = *(const uint4*)b;
    int i = k >> 1, hh = k & 1;
    uint4 w = *(const uint4*)(b + 48 + 32 * i + 16 * hh);
    uint4 qh = *(const uint4*)(b + 16 + 16 * hh);
    uint32_t ws[4] = {w.x, w.y, w.z, w.w}, hs[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        t.q[j] = (int)((ws[j] & 0x0F0F0F0Fu) | (((hs[j] >> (2 * i)) & 0x01010101u) << 4));
        t.q[4 + j] = (int)(((ws[j] >> 4) & 0x0F0F0F0Fu) | (((hs[j] >> (2 * i + 1)) & 0x01010101u) << 4));
    }
    t.o0 = 64 * i + 16 * hh; t.o1 = t.o0 + 32;
    scale_min_k4w(2 * i, h.y, h.z, h.w, t.sc0, t.m0);
    scale_min_k4w(2 * i + 1, h.y, h.z, h.w, t.sc1, t.m1);
    t.D = f16_to_f32(h.x & 0xFFFF); t.M = f16_to_f32(h.x >> 16);
}
template <> __device__ __forceinline__ void task<Q6_K>(const uint8_t* b, int k, const IqTables*, Task& t) {
    int n = k >> 2, a = k & 1, hi = (k >> 1) & 1;
    const uint8_t *ql = b + 64 * n + 32 * hi + 16 * a, *qh = b + 128 + 32 * n + 16 * a;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t l = rd32<2>(ql + 4 * j), h = rd32<2>(qh + 4 * j);
        t.q[j] = (int)((l & 0x0F0F0F0Fu) | (((h >> (2 * hi)) & 0x03030303u) << 4));           // value + 32
        t.q[4 + j] = (int)(((l >> 4) & 0x0F0F0F0Fu) | (((h >> (4 + 2 * hi)) & 0x03030303u) << 4));
    }
    t.o0 = 128 * n + 32 * hi + 16 * a; t.o1 = t.o0 + 64;
    const uint8_t* sc = b + 192 + 8 * n;
    t.sc0 = (int8_t)sc[a + 2 * hi]; t.sc1 = (int8_t)sc[a + 4 + 2 * hi];
    t.m0 = t.m1 = 0;
    t.D = f16_to_f32(rd16(b + 208)); t.M = 0.0f;
}
template <> __device__ __forceinline__ void task<IQ2_XXS>(const uint8_t* b, int k, const IqTables* tab, Task& t) {
    uint32_t g = rd32<2>(b + 2 + 8 * k), aux = rd32<2>(b + 6 + 8 * k);
#pragma unroll
    for (int l = 0; l < 4; l++) {
        uint64_t grid = tab->iq2xxs[(g >> (8 * l)) & 255];
        uint32_t s = tab->ksigns[(aux >> (7 * l)) & 127];
        t.q[2 * l] = neg_bytes((uint32_t)grid, s);
        t.q[2 * l + 1] = neg_bytes((uint32_t)(grid >> 32), s >> 4);
    }
    t.o0 = 32 * k; t.o1 = 32 * k + 16;
    t.sc0 = t.sc1 = 2 * (int)(aux >> 28) + 1;
    t.m0 = t.m1 = 0;
    t.D = 0.125f * f16_to_f32(rd16(b)); t.M = 0.0f;
}
template <> __device__ __forceinline__ void task<IQ3_S>(const uint8_t* b, int k, const IqTables* tab, Task& t) {
    uint32_t q0 = rd32<2>(b + 2 + 8 * k), q1 = rd32<2>(b + 6 + 8 * k), sg = rd32<2>(b + 74 + 4 * k);
    uint32_t hb = b[66 + k];
#pragma unroll
    for (int l = 0; l < 4; l++) {
        uint32_t qq = l < 2 ? q0 >> (16 * l) : q1 >> (16 * (l - 2));
        uint32_t g1 = tab->iq3s[(qq & 255) | ((hb << (8 - 2 * l)) & 256)];
        uint32_t g2 = tab->iq3s[((qq >> 8) & 255) | ((hb << (7 - 2 * l)) & 256)];
        uint32_t s = sg >> (8 * l);
        t.q[2 * l] = neg_bytes(g1, s);
        t.q[2 * l + 1] = neg_bytes(g2, s >> 4);
    }
    t.o0 = 32 * k; t.o1 = 32 * k + 16;
    t.sc0 = t.sc1 = 1 + 2 * ((b[106 + k / 2] >> (4 * (k & 1))) & 0xF);
    t.m0 = t.m1 = 0;
    t.D = f16_to_f32(rd16(b)); t.M = 0.0f;
}
// KVALUES_IQ4NL of the 4 nibbles in the low 4 bits of each byte of n (v_perm_b32 on the table in 4 words).
__device__ __forceinline__ int iq4nl_lut(uint32_t n) {
    constexpr uint32_t t0 = (uint8_t)-127 | (uint8_t)-104 << 8 | (uint8_t)-83 << 16 | (uint32_t)(uint8_t)-65 << 24;
    constexpr uint32_t t1 = (uint8_t)-49 | (uint8_t)-35 << 8 | (uint8_t)-22 << 16 | (uint32_t)(uint8_t)-10 << 24;
    constexpr uint32_t t2 = 1u | 13u << 8 | 25u << 16 | 38u << 24;
    constexpr uint32_t t3 = 53u | 69u << 8 | 89u << 16 | 113u << 24;
    uint32_t sel = n & 0x07070707u, hi_mask = ((n >> 3) & 0x01010101u) * 0xFFu;
    uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel), hi = __builtin_amdgcn_perm(t3, t2, sel);
    return (int)((lo & ~hi_mask) | (hi & hi_mask));
}
template <> __device__ __forceinline__ void task<IQ4_XS>(const uint8_t* b, int k, const IqTables*, Task& t) {
    uint2 w0 = *(const uint2*)(b + 8 + 16 * k), w1 = *(const uint2*)(b + 16 + 16 * k);
    uint32_t ws[4] = {w0.x, w0.y, w1.x, w1.y};
#pragma unroll
    for (int j = 0; j < 4; j++) { t.q[j] = iq4nl_lut(ws[j] & 0x0F0F0F0Fu); t.q[4 + j] = iq4nl_lut((ws[j] >> 4) & 0x0F0F0F0Fu); }
    uint32_t sh = rd16(b + 2);
    int ls = ((b[4 + k / 2] >> (4 * (k & 1))) & 0xF) | (((sh >> (2 * k)) & 3) << 4);
    t.o0 = 32 * k; t.o1 = 32 * k + 16;
    t.sc0 = t.sc1 = ls - 32;
    t.m0 = t.m1 = 0;
    t.D = f16_to_f32(rd16(b)); t.M = 0.0f;
}

}  // namespace strata

// 16 consecutive weights of a super-block (values 16 p .. 16 p + 15) as int8 digit planes for the int8 MFMA GEMM.
//
// A weight of a super-block is D * sc * (q - bias) - M * m with integer sc, q, m constant over its 16 (Q6_K, Q2_K,
// Q3_K) or 32 (the others) values. The integer v = sc * (q - bias) (|v| <= 4096) is split as v = 64 HI + LO with
// LO in 0..63 and HI in -64..63, each an int8 plane; m is a third plane where the format has mins. The split is
// exact, so HI.x, LO.x and M.x sum exactly in int32.
//
// dec16<T>(b, p, hi, lo, m) reads the super-block at b (LDS, the alignment of the global copy mod 16) and writes the
// four words of HI and LO and the min m (0 without mins). Layouts: src/quant/mod.rs (Q2_K 156-170, Q3_K 173-207,
// Q4_K 209-221, Q5_K 223-237, Q6_K 239-256, IQ2_XXS 287-297, IQ3_S 345-361, IQ4_XS 363-376).
#pragma once
#include "sbdot.h"

namespace strata {

__device__ __forceinline__ uint32_t pk_mul16(uint32_t a, uint32_t b) {  // low 16 bits of each 16-bit product
    typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
    v2u16 x = __builtin_bit_cast(v2u16, a), y = __builtin_bit_cast(v2u16, b);
    return __builtin_bit_cast(uint32_t, (v2u16)(x * y));
}
__device__ __forceinline__ uint32_t pk_ashr6(uint32_t a) {  // arithmetic >> 6 of each signed 16-bit half
    typedef short v2i16 __attribute__((ext_vector_type(2)));
    v2i16 x = __builtin_bit_cast(v2i16, a);
    return __builtin_bit_cast(uint32_t, (v2i16)(x >> (v2i16){6, 6}));
}
// bytes 0 and 2 of lo16 and hi16 interleaved: byte0 = lo16.b0, byte1 = hi16.b0, byte2 = lo16.b2, byte3 = hi16.b2
__device__ __forceinline__ uint32_t pack_even_bytes(uint32_t hi16, uint32_t lo16) {
    return __builtin_amdgcn_perm(hi16, lo16, 0x06020400u);
}

// The planes of one word of 4 values: bytes 0, 2 and 1, 3 go to 16-bit lanes, v = sc * (q - bias) in each lane
// (|v| <= 4096), HI = v >> 6 and LO = v & 63 packed back to bytes. UNSIGNED: q and sc are non-negative and bias is
// 0 (the K-quants with mins); otherwise q is signed (SGN, the IQ codebook values) or biased by `bias`.
template <bool UNSIGNED>
__device__ __forceinline__ void planes4(uint32_t q, uint32_t sc16, uint32_t bias16, bool sgn, uint32_t& hi, uint32_t& lo) {
    typedef short v2i16 __attribute__((ext_vector_type(2)));
    uint32_t a = q & 0x00FF00FFu, b = (q >> 8) & 0x00FF00FFu;
    if constexpr (!UNSIGNED) {
        v2i16 va16 = __builtin_bit_cast(v2i16, a), vb16 = __builtin_bit_cast(v2i16, b);
        if (sgn) {  // sign-extend each byte to 16 bits
            va16 = (va16 ^ (v2i16){0x80, 0x80}) - (v2i16){0x80, 0x80};
            vb16 = (vb16 ^ (v2i16){0x80, 0x80}) - (v2i16){0x80, 0x80};
        } else {
            const v2i16 bb = __builtin_bit_cast(v2i16, bias16);
            va16 -= bb;
            vb16 -= bb;
        }
        a = __builtin_bit_cast(uint32_t, va16);
        b = __builtin_bit_cast(uint32_t, vb16);
    }
    const uint32_t va = pk_mul16(a, sc16), vb = pk_mul16(b, sc16);
    const uint32_t ha = UNSIGNED ? (va >> 6) & 0x03FF03FFu : pk_ashr6(va), hb = UNSIGNED ? (vb >> 6) & 0x03FF03FFu : pk_ashr6(vb);
    hi = pack_even_bytes(hb, ha);
    lo = pack_even_bytes(vb & 0x003F003Fu, va & 0x003F003Fu);
}

template <int T> struct Dec;

// Q4_K / Q5_K: sub-block j = p / 2 (32 values), l0 = 16 (p & 1); q = nibble (j & 1) of qs[32 (j / 2) + l] (+16 from
// bit j of qh[l] for Q5_K); sc, m = scale_min_k4(j); D = d, M = dmin.
template <bool Q5>
__device__ __forceinline__ void dec16_q45(const uint8_t* b, int p, uint32_t* hi, uint32_t* lo, int& m) {
    const int j = p >> 1, l0 = 16 * (p & 1);
    const uint4 h = *(const uint4*)b;
    int sc;
    scale_min_k4w(j, h.y, h.z, h.w, sc, m);
    const uint4 w = *(const uint4*)(b + (Q5 ? 48 : 16) + 32 * (j >> 1) + l0);
    uint32_t ws[4] = {w.x, w.y, w.z, w.w}, hs[4] = {0, 0, 0, 0};
    if constexpr (Q5) {
        const uint4 qh = *(const uint4*)(b + 16 + l0);
        hs[0] = qh.x; hs[1] = qh.y; hs[2] = qh.z; hs[3] = qh.w;
    }
    const uint32_t sc16 = (uint32_t)sc * 0x00010001u;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t q = (ws[i] >> (4 * (j & 1))) & 0x0F0F0F0Fu;
        if constexpr (Q5) q |= ((hs[i] >> j) << 4) & 0x10101010u;
        planes4<true>(q, sc16, 0, false, hi[i], lo[i]);
    }
}
template <> struct Dec<Q4_K> {
    static constexpr bool MIN = true;
    __device__ static void run(const uint8_t* b, int p, const IqTables*, uint32_t* hi, uint32_t* lo, int& m) { dec16_q45<false>(b, p, hi, lo, m); }
    __device__ static void scales(const uint8_t* b, float& D, float& M) { uint32_t dm = *(const uint32_t*)b; D = f16_to_f32(dm & 0xFFFF); M = f16_to_f32(dm >> 16); }
};
template <> struct Dec<Q5_K> {
    static constexpr bool MIN = true;
    __device__ static void run(const uint8_t* b, int p, const IqTables*, uint32_t* hi, uint32_t* lo, int& m) { dec16_q45<true>(b, p, hi, lo, m); }
    __device__ static void scales(const uint8_t* b, float& D, float& M) { uint32_t dm = *(const uint32_t*)b; D = f16_to_f32(dm & 0xFFFF); M = f16_to_f32(dm >> 16); }
};

// Q6_K: half n = p / 8, quadrant qd = (p / 2) & 3 (values 32 qd + l of the half), l0 = 16 (p & 1); q = nibble
// (qd >> 1) of ql[64 n + 32 (qd & 1) + l] | bits 2 qd.. of qh[32 n + l] << 4; sc = int8 scale 8 n + l0 / 16 + 2 qd;
// bias 32.
template <> struct Dec<Q6_K> {
    static constexpr bool MIN = false;
    __device__ static void run(const uint8_t* b, int p, const IqTables*, uint32_t* hi, uint32_t* lo, int& m) {
        const int n = p >> 3, qd = (p >> 1) & 3, l0 = 16 * (p & 1);
        uint32_t ql[4], qh[4];
        words_a2<4>(b + 64 * n + 32 * (qd & 1) + l0, ql);
        words_a2<4>(b + 128 + 32 * n + l0, qh);
        const int sc = (int8_t)b[192 + 8 * n + (l0 >> 4) + 2 * qd];
        const uint32_t sc16 = (uint32_t)(sc & 0xFFFF) * 0x00010001u;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = ((ql[i] >> (4 * (qd >> 1))) & 0x0F0F0F0Fu) | (((qh[i] >> (2 * qd)) << 4) & 0x30303030u);
            planes4<false>(q, sc16, 0x00200020u, false, hi[i], lo[i]);
        }
        m = 0;
    }
    __device__ static void scales(const uint8_t* b, float& D, float& M) { D = f16_to_f32(rd16(b + 208)); M = 0.0f; }
};

// Q2_K: n = p / 8, shift j = (p / 2) & 3, l0 = 16 (p & 1): q = (qs[32 n + l] >> 2 j) & 3, scale byte p: sc low nibble,
// m high nibble; D = d, M = dmin. sc * q <= 45: the HI plane is zero.
template <> struct Dec<Q2_K> {
    static constexpr bool MIN = true;
    __device__ static void run(const uint8_t* b, int p, const IqTables*, uint32_t* hi, uint32_t* lo, int& m) {
        const int n = p >> 3, j = (p >> 1) & 3, l0 = 16 * (p & 1);
        uint32_t ws[4];
#pragma unroll
        for (int i = 0; i < 4; i++) ws[i] = rd32<4>(b + 16 + 32 * n + l0 + 4 * i);  // Q2_K blocks are 4-aligned
        const uint32_t s = b[p];
        const uint32_t sc16 = (s & 0xF) * 0x00010001u;
        m = (int)(s >> 4);
#pragma unroll
        for (int i = 0; i < 4; i++) planes4<true>((ws[i] >> (2 * j)) & 0x03030303u, sc16, 0, false, hi[i], lo[i]);
    }
    __device__ static void scales(const uint8_t* b, float& D, float& M) { D = f16_to_f32(rd16(b + 80)); M = f16_to_f32(rd16(b + 82)); }
};

// Q3_K: n = p / 8, j = (p / 2) & 3, l0 = 16 (p & 1): q = ((qs[32 + 32 n + l] >> 2 j) & 3) | bit (4 n + j) of hm[l]
// << 2, bias 4; sc = q3k scale p - 32.
template <> struct Dec<Q3_K> {
    static constexpr bool MIN = false;
    __device__ static void run(const uint8_t* b, int p, const IqTables*, uint32_t* hi, uint32_t* lo, int& m) {
        const int n = p >> 3, j = (p >> 1) & 3, l0 = 16 * (p & 1), hb = 4 * n + j;
        uint32_t qs[4], hm[4];
        words_a2<4>(b + 32 + 32 * n + l0, qs);
        words_a2<4>(b + l0, hm);
        const int sc = q3k_scale(b + 96, p) - 32;
        const uint32_t sc16 = (uint32_t)(sc & 0xFFFF) * 0x00010001u;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = ((qs[i] >> (2 * j)) & 0x03030303u) | (((hm[i] >> hb) & 0x01010101u) << 2);
            planes4<false>(q, sc16, 0x00040004u, false, hi[i], lo[i]);
        }
        m = 0;
    }
    __device__ static void scales(const uint8_t* b, float& D, float& M) { D = f16_to_f32(rd16(b + 108)); M = 0.0f; }
};

// IQ4_XS: sub-block ib = p / 2; values KVALUES[nibble (p & 1) of qs[16 ib + l]], l < 16; sc = ls - 32.
template <> struct Dec<IQ4_XS> {
    static constexpr bool MIN = false;
    __device__ static void run(const uint8_t* b, int p, const IqTables*, uint32_t* hi, uint32_t* lo, int& m) {
        const int ib = p >> 1, nib = p & 1;
        const uint2 w0 = *(const uint2*)(b + 8 + 16 * ib), w1 = *(const uint2*)(b + 16 + 16 * ib);
        const uint32_t ws[4] = {w0.x, w0.y, w1.x, w1.y};
        const uint32_t sh = rd16(b + 2);
        const int ls = ((b[4 + ib / 2] >> (4 * (ib & 1))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4);
        const uint32_t sc16 = (uint32_t)((ls - 32) & 0xFFFF) * 0x00010001u;
#pragma unroll
        for (int i = 0; i < 4; i++) planes4<false>((uint32_t)iq4nl_lut((ws[i] >> (4 * nib)) & 0x0F0F0F0Fu), sc16, 0, true, hi[i], lo[i]);
        m = 0;
    }
    __device__ static void scales(const uint8_t* b, float& D, float& M) { D = f16_to_f32(rd16(b)); M = 0.0f; }
};

// IQ2_XXS: sub-block ib = p / 2, grid entries l = 2 (p & 1), + 1: 8 values each = grid bytes with signs; sc = 2 ls + 1,
// D = d / 8.
template <> struct Dec<IQ2_XXS> {
    static constexpr bool MIN = false;
    __device__ static void run(const uint8_t* b, int p, const IqTables* tab, uint32_t* hi, uint32_t* lo, int& m) {
        const int ib = p >> 1, h = p & 1;
        const uint32_t g = rd32<2>(b + 2 + 8 * ib), aux = rd32<2>(b + 6 + 8 * ib);
        const uint32_t sc16 = (2 * (aux >> 28) + 1) * 0x00010001u;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int l = 2 * h + e;
            const uint64_t grid = tab->iq2xxs[(g >> (8 * l)) & 255];
            const uint32_t s = tab->ksigns[(aux >> (7 * l)) & 127];
            planes4<false>((uint32_t)neg_bytes((uint32_t)grid, s), sc16, 0, true, hi[2 * e], lo[2 * e]);
            planes4<false>((uint32_t)neg_bytes((uint32_t)(grid >> 32), s >> 4), sc16, 0, true, hi[2 * e + 1], lo[2 * e + 1]);
        }
        m = 0;
    }
    __device__ static void scales(const uint8_t* b, float& D, float& M) { D = 0.125f * f16_to_f32(rd16(b)); M = 0.0f; }
};

// IQ3_S: sub-block ib = p / 2, grid pairs l = 2 (p & 1), + 1 (two 4-value entries each, 9-bit index with a qh bit),
// sign byte l; sc = 1 + 2 nibble.
template <> struct Dec<IQ3_S> {
    static constexpr bool MIN = false;
    __device__ static void run(const uint8_t* b, int p, const IqTables* tab, uint32_t* hi, uint32_t* lo, int& m) {
        const int ib = p >> 1, h = p & 1;
        const uint32_t qq = rd32<2>(b + 2 + 8 * ib + 4 * h), sg = rd16(b + 74 + 4 * ib + 2 * h), hb = b[66 + ib];
        const uint32_t sc16 = (uint32_t)(1 + 2 * ((b[106 + ib / 2] >> (4 * (ib & 1))) & 0xF)) * 0x00010001u;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int l = 2 * h + e;
            const uint32_t q2 = qq >> (16 * e);
            const uint32_t g1 = tab->iq3s[(q2 & 255) | ((hb << (8 - 2 * l)) & 256)];
            const uint32_t g2 = tab->iq3s[((q2 >> 8) & 255) | ((hb << (7 - 2 * l)) & 256)];
            const uint32_t s = sg >> (8 * e);
            planes4<false>((uint32_t)neg_bytes(g1, s), sc16, 0, true, hi[2 * e], lo[2 * e]);
            planes4<false>((uint32_t)neg_bytes(g2, s >> 4), sc16, 0, true, hi[2 * e + 1], lo[2 * e + 1]);
        }
        m = 0;
    }
    __device__ static void scales(const uint8_t* b, float& D, float& M) { D = f16_to_f32(rd16(b)); M = 0.0f; }
};

}  // namespace strata

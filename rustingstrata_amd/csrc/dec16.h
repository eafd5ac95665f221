// 16 consecutive weights of a super-block (values 16 p .. 16 p + 15) as int8 digit planes for the int8 MFMA GEMM.
//
// A weight of a super-block is D * sc * (q - bias) - M * m with integer sc, q, m constant over its 16 (Q6_K, Q2_K,
// Q3_K) or 32 (the others) values. The integer v = sc * (q - bias) (|v| <= 4096) is split as v = 256 H + L with
// L in -128..127 and H in -16..16, each an int8 plane; m is a third plane where the format has mins. The split is
// exact, so H.x, L.x and M.x sum exactly in int32.
//
// The split costs one packed 16-bit multiply-add per two values: u = sc * q + (128 - bias * sc) = v + 128 in each
// 16-bit lane, whose high byte is H = floor(u / 256) and whose low byte minus 128 (its top bit flipped) is L.
//
// Dec<T>::run(b, p, tab, H, L, m) reads the super-block at b (LDS, the alignment of the global copy mod 16) and
// writes the four words of H and L and the min m (0 without mins). Layouts: src/quant/mod.rs (Q2_K 156-170, Q3_K
// 173-207, Q4_K 209-221, Q5_K 223-237, Q6_K 239-256, IQ2_XXS 287-297, IQ3_S 345-361, IQ4_XS 363-376).
#pragma once
#include "sbdot.h"

namespace strata {

typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

// Split of u = sc * q + add per 16-bit lane (mod 2^16) for the bytes of q given as qa (bytes 0 and 2 in the low
// byte of each 16-bit lane) and qb (bytes 1 and 3): H = high bytes, L = low bytes ^ 0x80, in value order.
__device__ __forceinline__ void split16(uint32_t qa, uint32_t qb, uint32_t sc16, uint32_t add16, uint32_t& H, uint32_t& L) {
    const v2u16 sc = __builtin_bit_cast(v2u16, sc16), ad = __builtin_bit_cast(v2u16, add16);
    const uint32_t ua = __builtin_bit_cast(uint32_t, (v2u16)(__builtin_bit_cast(v2u16, qa) * sc + ad));
    const uint32_t ub = __builtin_bit_cast(uint32_t, (v2u16)(__builtin_bit_cast(v2u16, qb) * sc + ad));
    H = __builtin_amdgcn_perm(ub, ua, 0x07030501u);
    L = __builtin_amdgcn_perm(ub, ua, 0x06020400u) ^ 0x80808080u;
}
// The planes of 4 unsigned bytes q: v = sc * q - bias * sc; add16 = (128 - bias * sc) in both halves.
__device__ __forceinline__ void planes_u(uint32_t q, uint32_t sc16, uint32_t add16, uint32_t& H, uint32_t& L) {
    split16(q & 0x00FF00FFu, __builtin_amdgcn_perm(q, q, 0x0c030c01u), sc16, add16, H, L);
}
// The planes of 4 signed bytes q (sign-extended to 16 bits by the byte permute): v = sc * q; add16 = 128.
__device__ __forceinline__ void planes_s(uint32_t q, uint32_t sc16, uint32_t& H, uint32_t& L) {
    split16(__builtin_amdgcn_perm(0u, q << 8, 0x09030801u), __builtin_amdgcn_perm(0u, q, 0x09030801u), sc16,
            0x00800080u, H, L);
}
__device__ __forceinline__ uint32_t rep16(int v) { return ((uint32_t)v & 0xFFFFu) * 0x00010001u; }

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
    const uint32_t sc16 = rep16(sc);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t q = (ws[i] >> (4 * (j & 1))) & 0x0F0F0F0Fu;
        // bit j of each qh byte to bit 4: a rotate right by j - 4 (mod 32); bits that wrap are masked off
        if constexpr (Q5) q |= __builtin_amdgcn_alignbit(hs[i], hs[i], (uint32_t)(j + 28) & 31) & 0x10101010u;
        planes_u(q, sc16, 0x00800080u, hi[i], lo[i]);
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
        const uint32_t sc16 = rep16(sc), add16 = rep16(128 - 32 * sc);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // bits 2 qd, 2 qd + 1 of each qh byte to bits 4, 5: a rotate right by 2 qd - 4 (mod 32), masked
            const uint32_t q = ((ql[i] >> (4 * (qd >> 1))) & 0x0F0F0F0Fu) |
                               (__builtin_amdgcn_alignbit(qh[i], qh[i], (uint32_t)(2 * qd + 28) & 31) & 0x30303030u);
            planes_u(q, sc16, add16, hi[i], lo[i]);
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
        // sc * q <= 45: each byte's product stays in its byte, so one packed 16-bit multiply scales all four
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo[i] = __builtin_bit_cast(uint32_t, (v2u16)(__builtin_bit_cast(v2u16, (ws[i] >> (2 * j)) & 0x03030303u) *
                                                         __builtin_bit_cast(v2u16, sc16)));
            hi[i] = 0;
        }
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
        const uint32_t sc16 = rep16(sc), add16 = rep16(128 - 4 * sc);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = ((qs[i] >> (2 * j)) & 0x03030303u) | (((hm[i] >> hb) & 0x01010101u) << 2);
            planes_u(q, sc16, add16, hi[i], lo[i]);
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
        const uint32_t sc16 = rep16(ls - 32);
#pragma unroll
        for (int i = 0; i < 4; i++) planes_s((uint32_t)iq4nl_lut((ws[i] >> (4 * nib)) & 0x0F0F0F0Fu), sc16, hi[i], lo[i]);
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
            planes_s((uint32_t)neg_bytes((uint32_t)grid, s), sc16, hi[2 * e], lo[2 * e]);
            planes_s((uint32_t)neg_bytes((uint32_t)(grid >> 32), s >> 4), sc16, hi[2 * e + 1], lo[2 * e + 1]);
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
            planes_s((uint32_t)neg_bytes(g1, s), sc16, hi[2 * e], lo[2 * e]);
            planes_s((uint32_t)neg_bytes(g2, s >> 4), sc16, hi[2 * e + 1], lo[2 * e + 1]);
        }
        m = 0;
    }
    __device__ static void scales(const uint8_t* b, float& D, float& M) { D = f16_to_f32(rd16(b)); M = 0.0f; }
};

}  // namespace strata

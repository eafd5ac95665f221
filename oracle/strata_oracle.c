/* CPU oracle for the quantized-matmul hot path (test infrastructure only; see strata_oracle.h).
 *
 * Built with -ffp-contract=off: the reference (Rust) never fuses a multiply and an add, and the dequantized
 * values and dot products here must carry the reference's bits. Every float expression keeps the reference's
 * evaluation order (left to right, as Rust evaluates it). */
#include "strata_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "../include/strata_iq_tables.h"

enum { Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, IQ2_XXS = 16, IQ3_S = 21, IQ4_XS = 23 };

/* GgmlType::block_elems / block_bytes, src/quant/mod.rs:37-43. */
int or_block_elems(int ty) { return ty == Q8_0 ? 32 : 256; }
int or_block_bytes(int ty) {
    switch (ty) {
    case Q8_0: return 34;
    case Q2_K: return 84;
    case Q3_K: return 110;
    case Q4_K: return 144;
    case Q5_K: return 176;
    case Q6_K: return 210;
    case IQ2_XXS: return 66;
    case IQ3_S: return 110;
    case IQ4_XS: return 136;
    default: return 0;
    }
}

/* IEEE binary16 -> binary32, exact (the `half` crate's to_f32; src/quant/mod.rs:57). */
float or_f16(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 31, man = h & 1023, bits;
    if (exp == 31) bits = sign | 0x7f800000u | (man << 13);
    else if (exp) bits = sign | ((exp + 112) << 23) | (man << 13);
    else if (!man) bits = sign;
    else { /* subnormal: renormalise */
        int e = 113;
        while (!(man & 1024)) { man <<= 1; e--; }
        bits = sign | ((uint32_t)e << 23) | ((man & 1023) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
static float h16(const uint8_t* b) { return or_f16((uint16_t)(b[0] | b[1] << 8)); }
static uint32_t u32le(const uint8_t* b) { return (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24; }

/* scale_min_k4, src/quant/mod.rs:59-62. */
static void scale_min_k4(int j, const uint8_t* q, int* s, int* m) {
    if (j < 4) { *s = q[j] & 63; *m = q[j + 4] & 63; }
    else { *s = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4); *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4); }
}

/* ---- dequantization: src/quant/mod.rs ---- */

static void dq_q8_0(const uint8_t* b, float* y) { /* mod.rs:86 */
    float d = h16(b);
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)b[2 + j] * d;
}

static void dq_q2k(const uint8_t* b, float* y) { /* mod.rs:156-170 */
    const uint8_t* sc = b;
    float d = h16(b + 80), mn = h16(b + 82);
    int q = 16, is = 0, o = 0;
    for (int n = 0; n < 2; n++) {
        for (int shift = 0; shift < 8; shift += 2)
            for (int half = 0; half < 2; half++) {
                uint8_t s = sc[is++];
                float dl = d * (float)(s & 0xF), ml = mn * (float)(s >> 4);
                for (int l = 0; l < 16; l++) y[o++] = dl * (float)((b[q + l + 16 * half] >> shift) & 3) - ml;
            }
        q += 32;
    }
}

/* q3k_scales, mod.rs:173-186: 16 6-bit scales, bias 32 kept. */
static void q3k_scales(const uint8_t* b, int8_t* scales) {
    uint32_t aux[4];
    for (int i = 0; i < 3; i++) aux[i] = u32le(b + 96 + 4 * i);
    uint32_t k1 = 0x03030303u, k2 = 0x0f0f0f0fu, tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & k2) | (((tmp >> 4) & k1) << 4);
    aux[3] = ((aux[1] >> 4) & k2) | (((tmp >> 6) & k1) << 4);
    aux[0] = (aux[0] & k2) | ((tmp & k1) << 4);
    aux[1] = (aux[1] & k2) | (((tmp >> 2) & k1) << 4);
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) scales[4 * i + j] = (int8_t)(aux[i] >> (8 * j));
}

static void dq_q3k(const uint8_t* b, float* y) { /* mod.rs:188-207 */
    const uint8_t* hm = b;
    float d_all = h16(b + 108);
    int8_t scales[16];
    q3k_scales(b, scales);
    int q = 32, is = 0, o = 0;
    uint8_t m = 1;
    for (int n = 0; n < 2; n++) {
        for (int shift = 0; shift < 8; shift += 2) {
            for (int half = 0; half < 2; half++) {
                float dl = d_all * (float)((int)scales[is++] - 32);
                for (int l = 0; l < 16; l++) {
                    int i = l + 16 * half;
                    int v = ((b[q + i] >> shift) & 3) - ((hm[i] & m) ? 0 : 4);
                    y[o++] = dl * (float)v;
                }
            }
            m <<= 1;
        }
        q += 32;
    }
}

static void dq_q4k(const uint8_t* b, float* y) { /* mod.rs:209-221 */
    float d = h16(b), mn = h16(b + 2);
    const uint8_t* sc = b + 4;
    int q = 16, o = 0;
    for (int j = 0; j < 4; j++) {
        int s1, m1, s2, m2;
        scale_min_k4(2 * j, sc, &s1, &m1);
        scale_min_k4(2 * j + 1, sc, &s2, &m2);
        float d1 = d * (float)s1, mm1 = mn * (float)m1, d2 = d * (float)s2, mm2 = mn * (float)m2;
        for (int l = 0; l < 32; l++) y[o + l] = d1 * (float)(b[q + l] & 0xF) - mm1;
        for (int l = 0; l < 32; l++) y[o + 32 + l] = d2 * (float)(b[q + l] >> 4) - mm2;
        q += 32;
        o += 64;
    }
}

static void dq_q5k(const uint8_t* b, float* y) { /* mod.rs:223-237 */
    float d = h16(b), mn = h16(b + 2);
    const uint8_t *sc = b + 4, *qh = b + 16;
    int q = 48, o = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0; j < 4; j++) {
        int s1, m1, s2, m2;
        scale_min_k4(2 * j, sc, &s1, &m1);
        scale_min_k4(2 * j + 1, sc, &s2, &m2);
        float d1 = d * (float)s1, mm1 = mn * (float)m1, d2 = d * (float)s2, mm2 = mn * (float)m2;
        for (int l = 0; l < 32; l++) y[o + l] = d1 * ((float)(b[q + l] & 0xF) + ((qh[l] & u1) ? 16.0f : 0.0f)) - mm1;
        for (int l = 0; l < 32; l++) y[o + 32 + l] = d2 * ((float)(b[q + l] >> 4) + ((qh[l] & u2) ? 16.0f : 0.0f)) - mm2;
        q += 32;
        o += 64;
        u1 <<= 2;
        u2 <<= 2;
    }
}

static void dq_q6k(const uint8_t* b, float* y) { /* mod.rs:239-256 */
    float d = h16(b + 208);
    for (int n = 0; n < 2; n++) {
        const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n, *sc = b + 192 + 8 * n;
        float* yo = y + 128 * n;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = ((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
            int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            yo[l] = d * (float)(int8_t)sc[is] * (float)q1;
            yo[l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
            yo[l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
            yo[l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
        }
    }
}

/* sign, mod.rs:258: -1 where bit j of the sign byte is set. */
static float sgn(uint8_t signs, int j) { return (signs & STRATA_KMASK_IQ2XS[j]) ? -1.0f : 1.0f; }

static void dq_iq2xxs(const uint8_t* b, float* y) { /* mod.rs:287-297 */
    float d = h16(b);
    for (int ib = 0; ib < 8; ib++) {
        const uint8_t* qs = b + 2 + 8 * ib;
        uint32_t aux = u32le(b + 6 + 8 * ib);
        float db = d * (0.5f + (float)(aux >> 28)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            uint64_t grid = STRATA_IQ2XXS_GRID[qs[l]];
            uint8_t signs = STRATA_KSIGNS_IQ2XS[(aux >> (7 * l)) & 127];
            for (int j = 0; j < 8; j++) y[32 * ib + 8 * l + j] = db * (float)(uint8_t)(grid >> (8 * j)) * sgn(signs, j);
        }
    }
}

static void dq_iq3s(const uint8_t* b, float* y) { /* mod.rs:345-361 */
    float d = h16(b);
    const uint8_t *qs = b + 2, *qh = b + 66, *signs = b + 74, *sc = b + 106;
    for (int ib = 0; ib < 8; ib++) {
        float db = d * (float)(1 + 2 * ((sc[ib / 2] >> (4 * (ib % 2))) & 0xF));
        for (int l = 0; l < 4; l++) {
            unsigned hb = qh[ib];
            uint32_t g1 = STRATA_IQ3S_GRID[qs[8 * ib + 2 * l] | ((hb << (8 - 2 * l)) & 256)];
            uint32_t g2 = STRATA_IQ3S_GRID[qs[8 * ib + 2 * l + 1] | ((hb << (7 - 2 * l)) & 256)];
            uint8_t sg = signs[4 * ib + l];
            int o = 32 * ib + 8 * l;
            for (int j = 0; j < 4; j++) {
                y[o + j] = db * (float)(uint8_t)(g1 >> (8 * j)) * sgn(sg, j);
                y[o + j + 4] = db * (float)(uint8_t)(g2 >> (8 * j)) * sgn(sg, j + 4);
            }
        }
    }
}

static void dq_iq4xs(const uint8_t* b, float* y) { /* mod.rs:363-376 */
    float d = h16(b);
    unsigned sh = b[2] | b[3] << 8;
    const uint8_t *sl = b + 4, *qs = b + 8;
    for (int ib = 0; ib < 8; ib++) {
        int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4);
        float dl = d * (float)(ls - 32);
        for (int j = 0; j < 16; j++) {
            uint8_t q = qs[16 * ib + j];
            y[32 * ib + j] = dl * (float)STRATA_KVALUES_IQ4NL[q & 0xF];
            y[32 * ib + j + 16] = dl * (float)STRATA_KVALUES_IQ4NL[q >> 4];
        }
    }
}

int or_dequant_row(int ty, const uint8_t* src, size_t n, float* dst) {
    int be = or_block_elems(ty), bb = or_block_bytes(ty);
    if (!bb || n % (size_t)be) return -1;
    for (size_t i = 0; i < n / (size_t)be; i++) {
        const uint8_t* b = src + i * bb;
        float* y = dst + i * be;
        switch (ty) {
        case Q8_0: dq_q8_0(b, y); break;
        case Q2_K: dq_q2k(b, y); break;
        case Q3_K: dq_q3k(b, y); break;
        case Q4_K: dq_q4k(b, y); break;
        case Q5_K: dq_q5k(b, y); break;
        case Q6_K: dq_q6k(b, y); break;
        case IQ2_XXS: dq_iq2xxs(b, y); break;
        case IQ3_S: dq_iq3s(b, y); break;
        case IQ4_XS: dq_iq4xs(b, y); break;
        }
    }
    return 0;
}

/* ---- Q8_K activations: src/cpu_moe.rs:28-46 ---- */

void or_quantize_q8k(const float* x, size_t n, or_q8k* out) {
    for (size_t blk = 0; blk * 256 < n; blk++) {
        float b[256] = {0};
        size_t len = n - blk * 256 < 256 ? n - blk * 256 : 256;
        memcpy(b, x + blk * 256, len * sizeof(float));
        or_q8k* o = out + blk;
        float amax = 0.0f;
        for (int i = 0; i < 256; i++) amax = fmaxf(amax, fabsf(b[i]));
        if (amax == 0.0f) { memset(o, 0, sizeof *o); continue; }
        float max = 0.0f;
        for (int i = 0; i < 256; i++) if (fabsf(b[i]) == amax) { max = b[i]; break; } /* the first of largest |v| */
        float is = -127.0f / max;
        for (int i = 0; i < 256; i++) {
            int q = (int)nearbyintf(is * b[i]); /* round_ties_even under the default rounding mode */
            o->qs[i] = (int8_t)(q < 127 ? q : 127);
        }
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int i = 0; i < 16; i++) s += o->qs[16 * g + i];
            o->bs[g] = (int16_t)s;
        }
        o->d = 1.0f / is;
    }
}

/* ---- integer dots against Q8_K: src/cpu_moe.rs (scalar kernels) ---- */

/* grouped, cpu_moe.rs:214-217: sum over 16 groups of 16 of sc(j) * (a . q). Integer, so order-free. */
static int32_t grouped(const int8_t* a, const int8_t* q, const int* sc) {
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
        int32_t g = 0;
        for (int i = 16 * j; i < 16 * j + 16; i++) g += (int32_t)a[i] * q[i];
        s += sc[j] * g;
    }
    return s;
}

static float dot_q8_0(const uint8_t* row, size_t cols, const or_q8k* xq) { /* cpu_moe.rs:319-325 */
    float sum = 0.0f;
    for (size_t i = 0; i < cols / 32; i++) {
        const uint8_t* b = row + 34 * i;
        const or_q8k* y = xq + i / 8;
        int o = (int)(i % 8) * 32;
        int32_t s = 0;
        for (int j = 0; j < 32; j++) s += (int32_t)(int8_t)b[2 + j] * y->qs[o + j];
        sum += h16(b) * y->d * (float)s;
    }
    return sum;
}

static float dot_q2k(const uint8_t* row, size_t cols, const or_q8k* xq) { /* cpu_moe.rs:232-243 */
    float sumf = 0.0f;
    for (size_t bi = 0; bi < cols / 256; bi++) {
        const uint8_t* b = row + 84 * bi;
        const or_q8k* y = xq + bi;
        int8_t a[256];
        int sc[16];
        for (int i = 0; i < 256; i++) a[i] = (int8_t)((b[16 + 32 * (i / 128) + i % 32] >> (2 * (i / 32 % 4))) & 3);
        for (int j = 0; j < 16; j++) sc[j] = b[j] & 0xF;
        int32_t s = grouped(a, y->qs, sc), m = 0;
        for (int j = 0; j < 16; j++) m += (b[j] >> 4) * (int32_t)y->bs[j];
        sumf += y->d * h16(b + 80) * (float)s - y->d * h16(b + 82) * (float)m;
    }
    return sumf;
}

static float dot_q3k(const uint8_t* row, size_t cols, const or_q8k* xq) { /* cpu_moe.rs:245-257 */
    float sumf = 0.0f;
    for (size_t bi = 0; bi < cols / 256; bi++) {
        const uint8_t* b = row + 110 * bi;
        const or_q8k* y = xq + bi;
        int8_t scl[16], a[256];
        int sc[16];
        q3k_scales(b, scl);
        for (int j = 0; j < 16; j++) sc[j] = (int)scl[j] - 32;
        for (int i = 0; i < 256; i++) {
            int k = i / 32 % 4 + 4 * (i / 128);
            a[i] = (int8_t)(((b[32 + 32 * (i / 128) + i % 32] >> (2 * (k % 4))) & 3) - (((b[i % 32] >> k) & 1) ? 0 : 4));
        }
        sumf += h16(b + 108) * y->d * (float)grouped(a, y->qs, sc);
    }
    return sumf;
}

static float dot_q4k(const uint8_t* row, size_t cols, const or_q8k* xq) { /* cpu_moe.rs:327-338 */
    float sumf = 0.0f;
    for (size_t bi = 0; bi < cols / 256; bi++) {
        const uint8_t* b = row + 144 * bi;
        const or_q8k* y = xq + bi;
        int s8[8], m8[8], sc[16];
        for (int j = 0; j < 8; j++) scale_min_k4(j, b + 4, &s8[j], &m8[j]);
        int8_t a[256];
        for (int i = 0; i < 256; i++) a[i] = (int8_t)((b[16 + 32 * (i / 64) + i % 32] >> (4 * (i / 32 % 2))) & 0xF);
        for (int j = 0; j < 16; j++) sc[j] = s8[j / 2];
        int32_t s = grouped(a, y->qs, sc), m = 0;
        for (int j = 0; j < 8; j++) m += m8[j] * ((int32_t)y->bs[2 * j] + y->bs[2 * j + 1]);
        sumf += h16(b) * y->d * (float)s - h16(b + 2) * y->d * (float)m;
    }
    return sumf;
}

static float dot_q5k(const uint8_t* row, size_t cols, const or_q8k* xq) { /* cpu_moe.rs:341-358 */
    float sumf = 0.0f;
    for (size_t bi = 0; bi < cols / 256; bi++) {
        const uint8_t* b = row + 176 * bi;
        const or_q8k* y = xq + bi;
        int s8[8], m8[8], sc[16];
        for (int j = 0; j < 8; j++) scale_min_k4(j, b + 4, &s8[j], &m8[j]);
        int8_t a[256];
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++) {
                uint8_t q = b[48 + 32 * j + l], h = (uint8_t)(b[16 + l] >> (2 * j));
                a[64 * j + l] = (int8_t)((q & 0xF) | ((h & 1) << 4));
                a[64 * j + 32 + l] = (int8_t)((q >> 4) | ((h & 2) << 3));
            }
        for (int j = 0; j < 16; j++) sc[j] = s8[j / 2];
        int32_t s = grouped(a, y->qs, sc), m = 0;
        for (int j = 0; j < 8; j++) m += m8[j] * ((int32_t)y->bs[2 * j] + y->bs[2 * j + 1]);
        sumf += h16(b) * y->d * (float)s - h16(b + 2) * y->d * (float)m;
    }
    return sumf;
}

static float dot_q6k(const uint8_t* row, size_t cols, const or_q8k* xq) { /* cpu_moe.rs:360-377 */
    float sumf = 0.0f;
    for (size_t bi = 0; bi < cols / 256; bi++) {
        const uint8_t* b = row + 210 * bi;
        const or_q8k* y = xq + bi;
        int8_t a[256];
        for (int n = 0; n < 2; n++) {
            const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n;
            int8_t* an = a + 128 * n;
            for (int l = 0; l < 32; l++) {
                an[l] = (int8_t)(((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
                an[l + 32] = (int8_t)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                an[l + 64] = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                an[l + 96] = (int8_t)(((ql[l + 32] >> 4) | ((qh[l] >> 6) << 4)) - 32);
            }
        }
        int sc[16];
        for (int j = 0; j < 16; j++) sc[j] = (int8_t)b[192 + j];
        sumf += h16(b + 208) * y->d * (float)grouped(a, y->qs, sc);
    }
    return sumf;
}

/* dot8, cpu_moe.rs:51-53: grid bytes times +-1 signs times q8. */
static int32_t dot8(uint64_t g, uint8_t signs, const int8_t* q) {
    int32_t s = 0;
    for (int j = 0; j < 8; j++) s += (int32_t)(uint8_t)(g >> (8 * j)) * ((signs >> j) & 1 ? -1 : 1) * q[j];
    return s;
}

static float dot_iq2xxs(const uint8_t* row, size_t cols, const or_q8k* xq) { /* cpu_moe.rs:74-86 */
    float sumf = 0.0f;
    for (size_t bi = 0; bi < cols / 256; bi++) {
        const uint8_t* b = row + 66 * bi;
        const or_q8k* y = xq + bi;
        int32_t bsum = 0;
        for (int ib = 0; ib < 8; ib++) {
            uint32_t aux = u32le(b + 6 + 8 * ib);
            int32_t s = 0;
            for (int l = 0; l < 4; l++)
                s += dot8(STRATA_IQ2XXS_GRID[b[2 + 8 * ib + l]], STRATA_KSIGNS_IQ2XS[(aux >> (7 * l)) & 127], y->qs + 32 * ib + 8 * l);
            bsum += s * (int32_t)(2 * (aux >> 28) + 1);
        }
        sumf += h16(b) * y->d * (float)bsum;
    }
    return 0.125f * sumf;
}

static float dot_iq3s(const uint8_t* row, size_t cols, const or_q8k* xq) { /* cpu_moe.rs:174-193 */
    float sumf = 0.0f;
    for (size_t bi = 0; bi < cols / 256; bi++) {
        const uint8_t* b = row + 110 * bi;
        const or_q8k* y = xq + bi;
        const uint8_t *qs = b + 2, *qh = b + 66, *signs = b + 74, *sc = b + 106;
        int32_t bsum = 0;
        for (int ib = 0; ib < 8; ib++) {
            int32_t s = 0;
            for (int l = 0; l < 4; l++) {
                uint32_t g1 = STRATA_IQ3S_GRID[qs[8 * ib + 2 * l] | (((unsigned)qh[ib] << (8 - 2 * l)) & 256)];
                uint32_t g2 = STRATA_IQ3S_GRID[qs[8 * ib + 2 * l + 1] | (((unsigned)qh[ib] << (7 - 2 * l)) & 256)];
                s += dot8((uint64_t)g1 | (uint64_t)g2 << 32, signs[4 * ib + l], y->qs + 32 * ib + 8 * l);
            }
            bsum += s * (2 * ((sc[ib / 2] >> (4 * (ib % 2))) & 0xF) + 1);
        }
        sumf += h16(b) * y->d * (float)bsum;
    }
    return sumf;
}

static float dot_iq4xs(const uint8_t* row, size_t cols, const or_q8k* xq) { /* cpu_moe.rs:195-212 */
    float sumf = 0.0f;
    for (size_t bi = 0; bi < cols / 256; bi++) {
        const uint8_t* b = row + 136 * bi;
        const or_q8k* y = xq + bi;
        float dd = h16(b) * y->d;
        unsigned sh = b[2] | b[3] << 8;
        const uint8_t *sl = b + 4, *qs = b + 8;
        for (int ib = 0; ib < 8; ib++) {
            int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4);
            const int8_t* q8 = y->qs + 32 * ib;
            int32_t s = 0;
            for (int j = 0; j < 16; j++) {
                uint8_t q = qs[16 * ib + j];
                s += (int32_t)q8[j] * STRATA_KVALUES_IQ4NL[q & 0xF] + (int32_t)q8[j + 16] * STRATA_KVALUES_IQ4NL[q >> 4];
            }
            sumf += dd * (float)(ls - 32) * (float)s;
        }
    }
    return sumf;
}

static int g_avx2 = 0;
void or_set_avx2(int on) { g_avx2 = on; }

float or_int_dot(int ty, const uint8_t* row, size_t cols, const or_q8k* xq) {
    if (g_avx2) {
        or_dot_fn f = or_avx2_dot(ty);
        if (f) return f(row, cols, xq);
    }
    switch (ty) {
    case Q8_0: return dot_q8_0(row, cols, xq);
    case Q2_K: return dot_q2k(row, cols, xq);
    case Q3_K: return dot_q3k(row, cols, xq);
    case Q4_K: return dot_q4k(row, cols, xq);
    case Q5_K: return dot_q5k(row, cols, xq);
    case Q6_K: return dot_q6k(row, cols, xq);
    case IQ2_XXS: return dot_iq2xxs(row, cols, xq);
    case IQ3_S: return dot_iq3s(row, cols, xq);
    case IQ4_XS: return dot_iq4xs(row, cols, xq);
    default: return NAN;
    }
}

static size_t row_bytes(int ty, size_t cols) { return cols / (size_t)or_block_elems(ty) * (size_t)or_block_bytes(ty); }

void or_matvec(int ty, const uint8_t* w, size_t rows, size_t cols, const float* x, float* y, int threads) {
    size_t nb = (cols + 255) / 256, rb = row_bytes(ty, cols);
    or_q8k* xq = (or_q8k*)malloc(nb * sizeof(or_q8k));
    or_quantize_q8k(x, cols, xq);
    long chunks = (long)((rows + 31) / 32);
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
    for (long c = 0; c < chunks; c++) {
        size_t r1 = (size_t)c * 32 + 32 < rows ? (size_t)c * 32 + 32 : rows;
        for (size_t r = (size_t)c * 32; r < r1; r++) y[r] = or_int_dot(ty, w + r * rb, cols, xq);
    }
    (void)threads;
    free(xq);
}

/* quant8 / quant_x without LLAMA_Q8, src/cuda/kernels.cu:640-678: per 32 values d = max|v| / 127,
 * q = round-half-even(v * (127 / max|v|)). */
void or_quant_xq32(const float* x, size_t x_stride, size_t n, size_t nt, uint8_t* out) {
    float* scales = (float*)(out + nt * n);
    for (size_t t = 0; t < nt; t++) {
        const float* xr = x + t * x_stride;
        for (size_t g = 0; g < n / 32; g++) {
            float mx = 0.0f;
            for (int i = 0; i < 32; i++) mx = fmaxf(mx, fabsf(xr[32 * g + i]));
            float d = mx / 127.0f, id = mx > 0.0f ? 127.0f / mx : 0.0f;
            for (int i = 0; i < 32; i++) out[t * n + 32 * g + i] = (uint8_t)(int8_t)(int)nearbyintf(xr[32 * g + i] * id);
            scales[t * (n / 32) + g] = d;
        }
    }
}

/* ---- routing, sort, combine ---- */

float or_silu(float x) { return x / (1.0f + expf(-x)); }

/* ops::rms_norm (src/ops.rs:3-7): ms = the sum of x^2 in index order / n, s = 1 / sqrt(ms + eps), out = x * s * w. */
void or_rms_norm(const float* x, const float* w, float eps, int n, float* out) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    const float ms = ss / (float)n;
    const float s = 1.0f / sqrtf(ms + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * s * w[i];
}

void or_route(const float* logits, int n, int k, int sigmoid, float extra_scale, int32_t* ids, float* wts) {
    float* p = (float*)malloc((size_t)n * sizeof(float));
    memcpy(p, logits, (size_t)n * sizeof(float));
    if (sigmoid) {
        for (int i = 0; i < n; i++) p[i] = 1.0f / (1.0f + expf(-p[i])); /* ops::sigmoid, ops.rs:15 */
    } else { /* ops::softmax, ops.rs:18-24 */
        float m = -INFINITY, s = 0.0f;
        for (int i = 0; i < n; i++) m = fmaxf(m, p[i]);
        for (int i = 0; i < n; i++) { p[i] = expf(p[i] - m); s += p[i]; }
        for (int i = 0; i < n; i++) p[i] /= s;
    }
    /* ops::top_k, ops.rs:102-107: descending, ties to the lower index (a selection, same order as the sort). */
    char* taken = (char*)calloc((size_t)n, 1);
    float sum = 0.0f;
    for (int j = 0; j < k; j++) {
        int best = -1;
        for (int i = 0; i < n; i++)
            if (!taken[i] && (best < 0 || p[i] > p[best])) best = i;
        taken[best] = 1;
        ids[j] = best;
        sum += p[best];
    }
    float scale = 1.0f / fmaxf(sum, 6.103515625e-5f);
    if (extra_scale != 0.0f) scale *= extra_scale;
    for (int j = 0; j < k; j++) wts[j] = p[ids[j]] * scale;
    free(taken);
    free(p);
}

void or_sort_by_expert(const int32_t* ids, int t, int k, int n_expert, int32_t* off, int32_t* xrow, int32_t* inv) {
    memset(off, 0, (size_t)(n_expert + 1) * sizeof(int32_t));
    for (int i = 0; i < t * k; i++) off[ids[i] + 1]++;
    for (int e = 0; e < n_expert; e++) off[e + 1] += off[e];
    int32_t* fill = (int32_t*)malloc((size_t)n_expert * sizeof(int32_t));
    memcpy(fill, off, (size_t)n_expert * sizeof(int32_t));
    for (int i = 0; i < t * k; i++) {
        int s = fill[ids[i]]++;
        xrow[s] = i / k;
        inv[i] = s;
    }
    free(fill);
}

void or_combine_seq(float* x, const float* ye, const float* wts, const int32_t* inv, int k, int n, int t) {
    for (int tt = 0; tt < t; tt++)
        for (int d = 0; d < n; d++) {
            float y = 0.0f;
            for (int j = 0; j < k; j++) y += wts[tt * k + j] * ye[(size_t)inv[tt * k + j] * n + d];
            x[(size_t)tt * n + d] += y;
        }
}

/* experts_multi: gate and up of every (token, expert) pair, silu(g) * u, down, then ys[t] += w * o in token and
 * router order (cpu_moe.rs:1483-1514; batch_rows 1424-1444 computes each row as int_dot of the pair's x). */
void or_experts_multi(int ty_gu, int ty_down, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                      int n_embd, int n_ff, const float* hs, int t, const int32_t* ids, const float* wts, int k,
                      float* ys, int threads) {
    size_t np = (size_t)t * k;
    size_t rb_gu = row_bytes(ty_gu, (size_t)n_embd), rb_d = row_bytes(ty_down, (size_t)n_ff);
    size_t mat_gu = rb_gu * (size_t)n_ff, mat_d = rb_d * (size_t)n_embd;
    size_t nbe = ((size_t)n_embd + 255) / 256, nbf = ((size_t)n_ff + 255) / 256;
    or_q8k* xh = (or_q8k*)malloc((size_t)t * nbe * sizeof(or_q8k));
    for (int tt = 0; tt < t; tt++) or_quantize_q8k(hs + (size_t)tt * n_embd, (size_t)n_embd, xh + (size_t)tt * nbe);
    float* a = (float*)malloc(np * 2 * (size_t)n_ff * sizeof(float));
    long jobs = (long)(np * 2 * (size_t)n_ff);
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads)
#endif
    for (long i = 0; i < jobs; i++) {
        size_t p = (size_t)i / (2 * (size_t)n_ff), m = (size_t)i / (size_t)n_ff % 2, r = (size_t)i % (size_t)n_ff;
        const uint8_t* wmat = (m ? up : gate) + (size_t)ids[p] * mat_gu;
        a[i] = or_int_dot(ty_gu, wmat + r * rb_gu, (size_t)n_embd, xh + (p / (size_t)k) * nbe);
    }
    float* acts = (float*)malloc(np * (size_t)n_ff * sizeof(float));
    for (size_t p = 0; p < np; p++)
        for (int i = 0; i < n_ff; i++) acts[p * n_ff + i] = or_silu(a[p * 2 * n_ff + i]) * a[p * 2 * n_ff + n_ff + i];
    or_q8k* xa = (or_q8k*)malloc(np * nbf * sizeof(or_q8k));
    for (size_t p = 0; p < np; p++) or_quantize_q8k(acts + p * n_ff, (size_t)n_ff, xa + p * nbf);
    float* o = (float*)malloc(np * (size_t)n_embd * sizeof(float));
    long jobs2 = (long)(np * (size_t)n_embd);
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads)
#endif
    for (long i = 0; i < jobs2; i++) {
        size_t p = (size_t)i / (size_t)n_embd, r = (size_t)i % (size_t)n_embd;
        o[i] = or_int_dot(ty_down, down + (size_t)ids[p] * mat_d + r * rb_d, (size_t)n_ff, xa + p * nbf);
    }
    memset(ys, 0, (size_t)t * n_embd * sizeof(float));
    for (size_t p = 0; p < np; p++) {
        float w = wts[p];
        float* y = ys + (p / (size_t)k) * n_embd;
        for (int d = 0; d < n_embd; d++) y[d] += w * o[p * n_embd + d];
    }
    (void)threads;
    free(xh); free(a); free(acts); free(xa); free(o);
}

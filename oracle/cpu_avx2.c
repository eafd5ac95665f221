/* CPU oracle, the timed AVX2 variant of the integer dots (TEST INFRASTRUCTURE ONLY: see strata_oracle.h).
 *
 * The reference CPU path dispatches these types to AVX2 kernels when built for x86-64-v3 (src/cpu_moe.rs:1364-1391,
 * kernels 380-982): the same integer super-block sums as the scalar dots, with the float closes in eight f32 lanes
 * and one horizontal sum per row, so their f32 results differ from the scalar ones in the last bits. bench.py times
 * this variant as the CPU baseline; the scalar dots stay the parity checker. Each function names the reference
 * kernel it restates. Types: Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0. */
#include <immintrin.h>
#include <stdint.h>
#include <string.h>

#include "strata_oracle.h"

static inline float f16v(const uint8_t* b) { return or_f16((uint16_t)(b[0] | b[1] << 8)); }

static inline float hsum8(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    return _mm_cvtss_f32(_mm_add_ss(s, _mm_movehdup_ps(s)));
}
static inline __m256i ld32(const void* p) { return _mm256_loadu_si256((const __m256i*)p); }
/* u8 weights (0..127) times s8 activations, pairs summed to i16, then times lo (first 16 values) and hi (last 16),
 * summed to 8 i32. */
static inline __m256i udot32(__m256i w, __m256i q, int lo, int hi) {
    __m256i p = _mm256_maddubs_epi16(w, q);
    return _mm256_madd_epi16(p, _mm256_set_m128i(_mm_set1_epi16((short)hi), _mm_set1_epi16((short)lo)));
}
/* bits 2k, 2k + 1 of every byte */
static inline __m256i crumb(__m256i v, int k) {
    return _mm256_and_si256(_mm256_srl_epi16(v, _mm_cvtsi32_si128(2 * k)), _mm256_set1_epi8(3));
}
static void scale_min(int j, const uint8_t* q, int* sc, int* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* avx2::dot_q4k, src/cpu_moe.rs:869-890 */
static float dot_q4k_avx2(const uint8_t* row, size_t cols, const or_q8k* xq) {
    const __m256i m4 = _mm256_set1_epi8(0xF);
    __m256 acc = _mm256_setzero_ps();
    float sumf = 0.0f;
    for (size_t i = 0; i < cols / 256; i++) {
        const uint8_t* b = row + 144 * i;
        const or_q8k* y = xq + i;
        int sc[8], mn[8];
        for (int j = 0; j < 8; j++) scale_min(j, b + 4, &sc[j], &mn[j]);
        __m256i sumi = _mm256_setzero_si256();
        for (int j = 0; j < 4; j++) {
            __m256i bits = ld32(b + 16 + 32 * j);
            sumi = _mm256_add_epi32(sumi, udot32(_mm256_and_si256(bits, m4), ld32(y->qs + 64 * j), sc[2 * j], sc[2 * j]));
            sumi = _mm256_add_epi32(sumi, udot32(_mm256_and_si256(_mm256_srli_epi16(bits, 4), m4), ld32(y->qs + 64 * j + 32),
                                                 sc[2 * j + 1], sc[2 * j + 1]));
        }
        int m = 0;
        for (int j = 0; j < 8; j++) m += mn[j] * (y->bs[2 * j] + y->bs[2 * j + 1]);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(y->d * f16v(b)), _mm256_cvtepi32_ps(sumi), acc);
        sumf -= y->d * f16v(b + 2) * (float)m;
    }
    return hsum8(acc) + sumf;
}

/* avx2::dot_q5k, src/cpu_moe.rs:922-949 */
static float dot_q5k_avx2(const uint8_t* row, size_t cols, const or_q8k* xq) {
    const __m256i m4 = _mm256_set1_epi8(0xF), one = _mm256_set1_epi8(1);
    __m256 acc = _mm256_setzero_ps();
    float sumf = 0.0f;
    for (size_t i = 0; i < cols / 256; i++) {
        const uint8_t* b = row + 176 * i;
        const or_q8k* y = xq + i;
        int sc[8], mn[8];
        for (int j = 0; j < 8; j++) scale_min(j, b + 4, &sc[j], &mn[j]);
        const __m256i qh = ld32(b + 16);
        __m256i sumi = _mm256_setzero_si256();
        for (int j = 0; j < 4; j++) {
            __m256i bits = ld32(b + 48 + 32 * j);
            __m256i h0 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srl_epi16(qh, _mm_cvtsi32_si128(2 * j)), one), 4);
            __m256i h1 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srl_epi16(qh, _mm_cvtsi32_si128(2 * j + 1)), one), 4);
            __m256i w0 = _mm256_or_si256(_mm256_and_si256(bits, m4), h0);
            __m256i w1 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(bits, 4), m4), h1);
            sumi = _mm256_add_epi32(sumi, udot32(w0, ld32(y->qs + 64 * j), sc[2 * j], sc[2 * j]));
            sumi = _mm256_add_epi32(sumi, udot32(w1, ld32(y->qs + 64 * j + 32), sc[2 * j + 1], sc[2 * j + 1]));
        }
        int m = 0;
        for (int j = 0; j < 8; j++) m += mn[j] * (y->bs[2 * j] + y->bs[2 * j + 1]);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(y->d * f16v(b)), _mm256_cvtepi32_ps(sumi), acc);
        sumf -= y->d * f16v(b + 2) * (float)m;
    }
    return hsum8(acc) + sumf;
}

/* avx2::dot_q6k, src/cpu_moe.rs:951-981: unsigned 6-bit codes, the -32 offset through the group sums */
static float dot_q6k_avx2(const uint8_t* row, size_t cols, const or_q8k* xq) {
    const __m256i m4 = _mm256_set1_epi8(0xF);
    __m256 acc = _mm256_setzero_ps();
    float sumf = 0.0f;
    for (size_t i = 0; i < cols / 256; i++) {
        const uint8_t* b = row + 210 * i;
        const or_q8k* y = xq + i;
        const int8_t* sc = (const int8_t*)(b + 192);
        __m256i sumi = _mm256_setzero_si256();
        for (int n = 0; n < 2; n++) {
            __m256i la = ld32(b + 64 * n), lb = ld32(b + 64 * n + 32), qh = ld32(b + 128 + 32 * n);
            __m256i w[4];
            w[0] = _mm256_or_si256(_mm256_and_si256(la, m4), _mm256_slli_epi16(crumb(qh, 0), 4));
            w[1] = _mm256_or_si256(_mm256_and_si256(lb, m4), _mm256_slli_epi16(crumb(qh, 1), 4));
            w[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(la, 4), m4), _mm256_slli_epi16(crumb(qh, 2), 4));
            w[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(lb, 4), m4), _mm256_slli_epi16(crumb(qh, 3), 4));
            for (int k = 0; k < 4; k++) {
                int g = 8 * n + 2 * k;
                sumi = _mm256_add_epi32(sumi, udot32(w[k], ld32(y->qs + 128 * n + 32 * k), sc[g], sc[g + 1]));
            }
        }
        int m = 0;
        for (int g = 0; g < 16; g++) m += sc[g] * y->bs[g];
        const float d = y->d * f16v(b + 208);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
        sumf -= 32.0f * d * (float)m;
    }
    return hsum8(acc) + sumf;
}

/* avx2::dot_q8_0, src/cpu_moe.rs:892-905: |w| times q8 with w's sign */
static float dot_q8_0_avx2(const uint8_t* row, size_t cols, const or_q8k* xq) {
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc = _mm256_setzero_ps();
    for (size_t i = 0; i < cols / 32; i++) {
        const uint8_t* b = row + 34 * i;
        const or_q8k* y = xq + i / 8;
        __m256i w = ld32(b + 2);
        __m256i p = _mm256_maddubs_epi16(_mm256_sign_epi8(w, w), _mm256_sign_epi8(ld32(y->qs + i % 8 * 32), w));
        __m256 ds = _mm256_set1_ps(f16v(b) * y->d);
        acc = _mm256_fmadd_ps(ds, _mm256_cvtepi32_ps(_mm256_madd_epi16(p, ones)), acc);
    }
    return hsum8(acc);
}

/* avx2::dot_q2k, src/cpu_moe.rs:757-777 */
static float dot_q2k_avx2(const uint8_t* row, size_t cols, const or_q8k* xq) {
    __m256 acc = _mm256_setzero_ps();
    for (size_t i = 0; i < cols / 256; i++) {
        const uint8_t* b = row + 84 * i;
        const or_q8k* y = xq + i;
        const uint8_t* sc = b;
        __m256i sumi = _mm256_setzero_si256();
        for (int n = 0; n < 2; n++) {
            __m256i bits = ld32(b + 16 + 32 * n);
            for (int k = 0; k < 4; k++) {
                int g = 8 * n + 2 * k;
                sumi = _mm256_add_epi32(sumi, udot32(crumb(bits, k), ld32(y->qs + 32 * (4 * n + k)), sc[g] & 0xF,
                                                     sc[g + 1] & 0xF));
            }
        }
        __m256i mins = _mm256_cvtepu8_epi16(
            _mm_and_si128(_mm_srli_epi16(_mm_loadu_si128((const __m128i*)sc), 4), _mm_set1_epi8(0xF)));
        __m256i m = _mm256_madd_epi16(mins, _mm256_loadu_si256((const __m256i*)y->bs));
        acc = _mm256_fmadd_ps(_mm256_set1_ps(y->d * f16v(b + 80)), _mm256_cvtepi32_ps(sumi), acc);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(-y->d * f16v(b + 82)), _mm256_cvtepi32_ps(m), acc);
    }
    return hsum8(acc);
}

/* Q3_K's 16 6-bit scales (quant::q3k_scales, src/quant/mod.rs:173-186). */
static void q3k_scales(const uint8_t* b, int* out) {
    const uint8_t* s = b + 96;
    for (int j = 0; j < 16; j++) {
        int lo = j < 8 ? s[j] & 0xF : s[j - 8] >> 4;
        int hi = (s[8 + j % 4] >> (2 * (j / 4))) & 3;
        out[j] = lo | hi << 4;
    }
}

/* avx2::dot_q3k, src/cpu_moe.rs:779-803: weight = crumb - 4 where the high bit is clear, signs moved onto q8 */
static float dot_q3k_avx2(const uint8_t* row, size_t cols, const or_q8k* xq) {
    __m256 acc = _mm256_setzero_ps();
    for (size_t i = 0; i < cols / 256; i++) {
        const uint8_t* b = row + 110 * i;
        const or_q8k* y = xq + i;
        int sc[16];
        q3k_scales(b, sc);
        const __m256i hm = ld32(b);
        __m256i sumi = _mm256_setzero_si256();
        for (int n = 0; n < 2; n++) {
            __m256i bits = ld32(b + 32 + 32 * n);
            for (int k = 0; k < 4; k++) {
                int kk = 4 * n + k;
                __m256i mask = _mm256_set1_epi8((char)(1 << kk));
                __m256i low = _mm256_cmpeq_epi8(_mm256_and_si256(hm, mask), _mm256_setzero_si256());
                __m256i w = _mm256_sub_epi8(crumb(bits, k), _mm256_and_si256(low, _mm256_set1_epi8(4)));
                __m256i p = _mm256_maddubs_epi16(_mm256_sign_epi8(w, w), _mm256_sign_epi8(ld32(y->qs + 32 * kk), w));
                __m256i s = _mm256_set_m128i(_mm_set1_epi16((short)(sc[2 * kk + 1] - 32)), _mm_set1_epi16((short)(sc[2 * kk] - 32)));
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(p, s));
            }
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(y->d * f16v(b + 108)), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum8(acc);
}

/* The AVX2 kernel of type ty, or null where the oracle has none (the scalar dot is used then). */
or_dot_fn or_avx2_dot(int ty) {
    switch (ty) {
    case 8: return dot_q8_0_avx2;
    case 10: return dot_q2k_avx2;
    case 11: return dot_q3k_avx2;
    case 12: return dot_q4k_avx2;
    case 13: return dot_q5k_avx2;
    case 14: return dot_q6k_avx2;
    }
    return 0;
}

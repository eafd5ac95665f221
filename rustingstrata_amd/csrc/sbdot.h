// Super-block dot products for the GEMV: one lane takes a whole 256-value super-block of a weight row (read from
// LDS) against the same 256 values of x (int8 in LDS, Q8_K numerics: one x scale per super-block), accumulating
// exactly in int32, and closes it with one float step
//     acc += dx * (D * sum_g sc_g * (q_g . x_g - bias * sum x_g) - M * sum_g m_g * sum x_g).
// Integer products of a group scale (|sc| < 2^8) and a group sum (|s| < 2^18) use 24-bit multiplies.
// This is the structure of the reference CPU dots (src/cpu_moe.rs:319-377: exact integer group sums, then
// d_w * d_x * s - dmin * d_x * m in f32).
#pragma once
#include "formats.h"

namespace strata {

// x of one input for one super-block, through one of two accessors with the same interface:
//   q16(o): the 16 int8 values at offset o (a multiple of 16), s(g): the sum of the 16 values of group g,
//   d(j): the scale of 32-group j (under Q8_K all 8 are the super-block's one scale).
// XLds reads LDS; XReg holds the slice in registers (indices must fold to constants: callers unroll fully).
struct XLds {
    const int8_t* qp;
    const float* dp;
    const int* sp;
    __device__ __forceinline__ uint4 q16(int o) const { return *(const uint4*)(qp + o); }
    __device__ __forceinline__ int s(int g) const { return sp[g]; }
    __device__ __forceinline__ float d(int j) const { return dp[j]; }
};
struct XReg {
    uint32_t w[64];
    int sums[16];
    float ds[8];
    __device__ __forceinline__ uint4 q16(int o) const { return make_uint4(w[o / 4], w[o / 4 + 1], w[o / 4 + 2], w[o / 4 + 3]); }
    __device__ __forceinline__ int s(int g) const { return sums[g]; }
    __device__ __forceinline__ float d(int j) const { return ds[j]; }
};

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return __builtin_amdgcn_ubfe(w, 8 * i, 8); }
__device__ __forceinline__ int sbyte_of(uint32_t w, int i) { return __builtin_amdgcn_sbfe((int)w, 8 * i, 8); }
__device__ __forceinline__ int dot16(const uint32_t* w, const uint4& x0, const uint4& x1, int acc = 0) {
    acc = sdot4((int)w[0], (int)x0.x, acc);
    acc = sdot4((int)w[1], (int)x0.y, acc);
    acc = sdot4((int)w[2], (int)x0.z, acc);
    acc = sdot4((int)w[3], (int)x0.w, acc);
    acc = sdot4((int)w[4], (int)x1.x, acc);
    acc = sdot4((int)w[5], (int)x1.y, acc);
    acc = sdot4((int)w[6], (int)x1.z, acc);
    return sdot4((int)w[7], (int)x1.w, acc);
}
__device__ __forceinline__ int dot4w(uint32_t a, uint32_t b, uint32_t c, uint32_t d, const uint4& x, int acc = 0) {
    acc = sdot4((int)a, (int)x.x, acc);
    acc = sdot4((int)b, (int)x.y, acc);
    acc = sdot4((int)c, (int)x.z, acc);
    return sdot4((int)d, (int)x.w, acc);
}
// v << n for n >= 0, v >> -n otherwise: one shift once n is a constant (the callers' loops unroll fully).
__device__ __forceinline__ uint32_t shl_by(uint32_t v, int n) { return n >= 0 ? v << n : v >> -n; }
// n words from a 2-byte-aligned LDS address: aligned reads, shifted into place (v_alignbyte_b32). (gfx950 also
// reads unaligned LDS addresses in hardware, but measured slower here: the Q6_K GEMV and GEMM lost 7-12%.)
template <int N>
__device__ __forceinline__ void words_a2(const uint8_t* p, uint32_t* out) {
    // stay a derivation of p (pointer arithmetic, not an integer round trip), so the reads keep p's address space
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    const uint32_t* a = (const uint32_t*)(p - sh);
    uint32_t prev = a[0];
#pragma unroll
    for (int i = 0; i < N; i++) {
        uint32_t nx = a[i + 1];
        out[i] = align_bytes(nx, prev, sh);
        prev = nx;
    }
}

// ---- Q4_K / Q5_K: 8 sub-blocks of 32, 6-bit scales and mins (src/cpu_moe.rs:327-358) ----
// Quarters [P0, P1) of the super-block (quarter p: values 64p .. 64p + 63, sub-blocks 2p and 2p + 1); all four for
// the whole dot.
template <bool Q5, int P0, int P1, class X>
__device__ __forceinline__ void sb_q45(const uint8_t* b, const X& x, int& isum, int& msum, float& D, float& M) {
    const uint4 h = *(const uint4*)b;
    D = f16_to_f32(h.x & 0xFFFF);
    M = f16_to_f32(h.x >> 16);
    // packed 6-bit scales / mins of sub-blocks 0..3 and 4..7 (scale_min_k4, src/quant/mod.rs:59-62)
    const uint32_t sc_lo = h.y & 0x3F3F3F3Fu, m_lo = h.z & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t m_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    uint4 qh0, qh1;
    if constexpr (Q5) { qh0 = *(const uint4*)(b + 16); qh1 = *(const uint4*)(b + 32); }
    const uint8_t* qs = b + (Q5 ? 48 : 16);
    int is = 0;
#pragma unroll
    for (int p = P0; p < P1; p++) {
        const uint4 w0 = *(const uint4*)(qs + 32 * p), w1 = *(const uint4*)(qs + 32 * p + 16);
        uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            lo[i] = w[i] & 0x0F0F0F0Fu;
            hi[i] = (w[i] >> 4) & 0x0F0F0F0Fu;
        }
        if constexpr (Q5) {
            uint32_t qh[8] = {qh0.x, qh0.y, qh0.z, qh0.w, qh1.x, qh1.y, qh1.z, qh1.w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                // bit 2p (2p + 1) of each qh byte to bit 4: one shift by a constant, then the mask
                lo[i] |= shl_by(qh[i], 4 - 2 * p) & 0x10101010u;
                hi[i] |= shl_by(qh[i], 3 - 2 * p) & 0x10101010u;
            }
        }
        const int s_lo = dot16(lo, x.q16(64 * p), x.q16(64 * p + 16));
        const int s_hi = dot16(hi, x.q16(64 * p + 32), x.q16(64 * p + 48));
        const uint32_t scw = p < 2 ? sc_lo : sc_hi;
        is += __mul24((int)byte_of(scw, (2 * p) & 3), s_lo) + __mul24((int)byte_of(scw, (2 * p + 1) & 3), s_hi);
    }
    isum = is;
    // min term: sum_j m_j * (sum of x over sub-block j)
    int ms = 0;
#pragma unroll
    for (int j = 2 * P0; j < 2 * P1; j++) ms += __mul24((int)byte_of(j < 4 ? m_lo : m_hi, j & 3), x.s(2 * j) + x.s(2 * j + 1));
    msum = ms;
}

// ---- Q6_K: 16 groups of 16, int8 scales, values q - 32 (src/cpu_moe.rs:360-377) ----
// Quarters [P0, P1): quarter 2n + (qd >> 1) is half n's passes qd (values 128n + 32qd .. + 31) for its two qd.
template <int P0, int P1, class X>
__device__ __forceinline__ void sb_q6(const uint8_t* b, const X& x, int& isum, float& D) {
    uint32_t sc[4];
    words_a2<4>(b + 192, sc);
    D = f16_to_f32(rd16(b + 208));
    int is = 0;
#pragma unroll
    for (int n = 0; n < 2; n++) {
        if (2 * n + 1 < P0 || 2 * n >= P1) continue;
        // half n: 64 bytes of low nibbles (ql[l] = words 0..7, ql[l + 32] = words 8..15), 32 bytes of high bits
        uint32_t ql[16], qh[8];
        words_a2<16>(b + 64 * n, ql);
        words_a2<8>(b + 128 + 32 * n, qh);
#pragma unroll
        for (int qd = 0; qd < 4; qd++)
#pragma unroll
            for (int a = 0; a < 2; a++) {
                if (2 * n + (qd >> 1) < P0 || 2 * n + (qd >> 1) >= P1) continue;
                uint32_t v[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int wi = 4 * a + i;
                    const uint32_t q = ql[(qd & 1 ? 8 : 0) + wi], hb = qh[wi];
                    const uint32_t nib = qd & 2 ? (q >> 4) & 0x0F0F0F0Fu : q & 0x0F0F0F0Fu;
                    v[i] = nib | (shl_by(hb, 4 - 2 * qd) & 0x30303030u);  // q + 32, in 0..63
                }
                const int xo = 128 * n + 32 * qd + 16 * a;
                const int s = dot4w(v[0], v[1], v[2], v[3], x.q16(xo)) - 32 * x.s(xo >> 4);
                const int g = 8 * n + a + 2 * qd;  // scale index: l / 16 + 2 qd within the half
                is += __mul24(sbyte_of(sc[g >> 2], g & 3), s);
            }
    }
    isum = is;
}

// ---- Q8_0: 8 blocks of 32 with an f16 scale each (src/cpu_moe.rs:319-325): returns sum_b (d_b dx) s_b ----
// The (d_b dx) s_b of block k (one term of the sum).
template <class X>
__device__ __forceinline__ float q8_0_term(const uint8_t* b, const X& x, int k, float dx) {
    uint32_t q[8];
    words_a2<8>(b + 34 * k + 2, q);  // the 32 int8 after the block's f16 scale
    const int s = dot16(q, x.q16(32 * k), x.q16(32 * k + 16));
    return (f16_to_f32(rd16(b + 34 * k)) * dx) * (float)s;
}
template <class X>
__device__ __forceinline__ float sb_q8_0(const uint8_t* b, const X& x, int nb, float dx) {
    float f = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        if (k >= nb) break;  // a partial last super-block (Q8_0 rows are multiples of 32 values)
        f = f + q8_0_term(b, x, k, dx);
    }
    return f;
}

// ---- generic: any type through task<T> (8 tasks of 32 values) ----
// Tasks [K0, K1).
template <int T, int K0, int K1, class X>
__device__ __forceinline__ void sb_generic(const uint8_t* b, const X& x, const IqTables* tab, int& isum, int& msum,
                                           float& D, float& M) {
    int is = 0, ms = 0;
#pragma unroll
    for (int k = K0; k < K1; k++) {
        Task t;
        task<T>(b, k, tab, t);
        int s0 = dot4w(t.q[0], t.q[1], t.q[2], t.q[3], x.q16(t.o0)), s1 = dot4w(t.q[4], t.q[5], t.q[6], t.q[7], x.q16(t.o1));
        const int a0 = x.s(t.o0 >> 4), a1 = x.s(t.o1 >> 4);
        if constexpr (Fmt<T>::BIAS != 0) { s0 -= Fmt<T>::BIAS * a0; s1 -= Fmt<T>::BIAS * a1; }
        is += __mul24(t.sc0, s0) + __mul24(t.sc1, s1);
        if constexpr (Fmt<T>::MIN) ms += __mul24(t.m0, a0) + __mul24(t.m1, a1);
        if (k == 0) { D = t.D; M = t.M; }
    }
    isum = is;
    msum = ms;
}

// The super-block's contribution, Q8_K numerics (one x scale for the whole super-block), in the CPU dots' float
// steps (src/cpu_moe.rs:319-377): (D dx) s - (M dx) m, each product rounded; Q8_0 adds its 32-blocks' (d dx) s in
// order. Summed over a row's super-blocks in order (ordered_sum), the K-quant, IQ2_XXS and IQ3_S rows carry the CPU
// dots' bits; Q8_0 (whose CPU sum runs over 32-blocks across super-blocks) and IQ4_XS (a float step per 32-value
// sub-block, src/cpu_moe.rs:195-212) stay within rounding of them.
template <int T, class X>
__device__ __forceinline__ float sb_dot_q8k(const uint8_t* b, const X& x, const IqTables* tab, int nvals) {
    const float dx = x.d(0);
    if constexpr (T == Q4_K || T == Q5_K) {
        int is, ms;
        float D, M;
        sb_q45<T == Q5_K, 0, 4>(b, x, is, ms, D, M);
        return (D * dx) * (float)is - (M * dx) * (float)ms;
    } else if constexpr (T == Q6_K) {
        int is;
        float D;
        sb_q6<0, 4>(b, x, is, D);
        return (D * dx) * (float)is;
    } else if constexpr (T == Q8_0) {
        return sb_q8_0(b, x, nvals >> 5, dx);
    } else {
        int is, ms = 0;
        float D, M = 0.0f;
        sb_generic<T, 0, 8>(b, x, tab, is, ms, D, M);
        float f = (D * dx) * (float)is;
        if constexpr (Fmt<T>::MIN) f = f - (M * dx) * (float)ms;
        return f;
    }
}

// The same under per-32 x scales (the reference GPU's default numerics): every 32-group has its own dx, so each task
// closes in float.
// Task k's term of that sum.
template <int T, class X>
__device__ __forceinline__ float q32_term(const uint8_t* b, const X& x, const IqTables* tab, int k) {
    Task t;
    task<T>(b, k, tab, t);
    int s0 = dot4w(t.q[0], t.q[1], t.q[2], t.q[3], x.q16(t.o0)), s1 = dot4w(t.q[4], t.q[5], t.q[6], t.q[7], x.q16(t.o1));
    const int a0 = x.s(t.o0 >> 4), a1 = x.s(t.o1 >> 4);
    if constexpr (Fmt<T>::BIAS != 0) { s0 -= Fmt<T>::BIAS * a0; s1 -= Fmt<T>::BIAS * a1; }
    float f0 = t.D * (float)__mul24(t.sc0, s0), f1 = t.D * (float)__mul24(t.sc1, s1);
    if constexpr (Fmt<T>::MIN) { f0 -= t.M * (float)__mul24(t.m0, a0); f1 -= t.M * (float)__mul24(t.m1, a1); }
    return x.d(t.o0 >> 5) * f0 + x.d(t.o1 >> 5) * f1;
}
template <int T, class X>
__device__ __forceinline__ float sb_dot_q32(const uint8_t* b, const X& x, const IqTables* tab, int nvals) {
    float f = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        if (32 * k >= nvals) break;  // a partial last super-block (Q8_0 only)
        f += q32_term<T>(b, x, tab, k);
    }
    return f;
}

// ---- quarter split: four waves take one quarter (values 64W .. 64W + 63) each of the same super-blocks, and wave 0
// closes them with the super-block's float steps (sb_close) in the order sb_dot_q8k / sb_dot_q32 take them, so the
// result carries the same bits. Integer numerics (Q8_K, all types but Q8_0): o0, o1 = the quarter's exact integer
// sums (scale-weighted products, min-weighted x sums); float steps (per-32 scales, or Q8_0): o0, o1 = the float
// terms of its two 32-value tasks 2W and 2W + 1, added in task order by the close. D and M: the super-block scales
// (set by quarter 0).
template <int T, bool Q32>
constexpr bool quarter_ints() { return !Q32 && T != Q8_0; }

template <int T, bool Q32, int W, class X>
__device__ __forceinline__ void sb_quarter(const uint8_t* b, const X& x, const IqTables* tab, int nvals, uint32_t& o0,
                                           uint32_t& o1, float& D, float& M) {
    if constexpr (!quarter_ints<T, Q32>()) {
        float t0 = 0.0f, t1 = 0.0f;
        if constexpr (Q32) {
            if (64 * W < nvals) t0 = q32_term<T>(b, x, tab, 2 * W);
            if (64 * W + 32 < nvals) t1 = q32_term<T>(b, x, tab, 2 * W + 1);
        } else {
            const float dx = x.d(0);
            if (64 * W < nvals) t0 = q8_0_term(b, x, 2 * W, dx);
            if (64 * W + 32 < nvals) t1 = q8_0_term(b, x, 2 * W + 1, dx);
        }
        o0 = __float_as_uint(t0);
        o1 = __float_as_uint(t1);
    } else {
        int is = 0, ms = 0;
        if constexpr (T == Q4_K || T == Q5_K) {
            sb_q45<T == Q5_K, W, W + 1>(b, x, is, ms, D, M);
        } else if constexpr (T == Q6_K) {
            sb_q6<W, W + 1>(b, x, is, D);
        } else {
            sb_generic<T, 2 * W, 2 * W + 2>(b, x, tab, is, ms, D, M);
        }
        o0 = (uint32_t)is;
        o1 = (uint32_t)ms;
    }
}

// o[2W], o[2W + 1]: quarter W's outputs; D, M from quarter 0; dx: x's scale (Q8_K numerics).
template <int T, bool Q32>
__device__ __forceinline__ float sb_close(const uint32_t (&o)[8], float D, float M, float dx, int nvals) {
    if constexpr (!quarter_ints<T, Q32>()) {
        float f = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (32 * k >= nvals) break;
            f += __uint_as_float(o[k]);
        }
        return f;
    } else {
        const int is = (int)(o[0] + o[2] + o[4] + o[6]), ms = (int)(o[1] + o[3] + o[5] + o[7]);
        float f = (D * dx) * (float)is;
        if constexpr (Fmt<T>::MIN) f = f - (M * dx) * (float)ms;
        return f;
    }
}

}  // namespace strata

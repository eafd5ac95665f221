// Attention over the f16 KV cache (Backend::attn_prefill_m and Backend::attn_decode_gq, src/backend.rs:337-343,
// 383-410; reference kernels src/cuda/kernels.cu:2123-2626 decode and 2787-3216 prefill). Cache rows: position p,
// KV head g at (p nkv + g) hd halves. Query head h reads KV head h / (nh / nkv). Output head h of token t:
// softmax(q . k scale) V over its positions, with an optional per-head sink logit (one more logit that takes mass and
// adds nothing) and an optional gate (times sigmoid(qg[t, h 2 hd + hd + d])), as Model::attention
// (src/model.rs:771-793) computes it.
//
// Prefill runs on f16 MFMA (v_mfma_f32_16x16x32_f16) without giving up f32 accuracy: q is split into f16 hi + lo
// parts (q = hi + lo to 2^-22 relative) and so are the softmax weights, each product pair summed in f32, while K and V
// are exact in f16 (the cache format). Both are scaled by powers of two first so that no part is a subnormal f16. Scores are computed transposed (S^T = K Q^T: keys on the MFMA rows), so the
// softmax weights leave the score MFMA in exactly the register layout the P V MFMA takes as its B operand, and V sits
// in LDS transposed ([dim][key]) for the A operand. Decode splits a token's positions over blocks (each serving all
// query heads of one KV head) and merges the partial softmax sums in a second launch.
#include <climits>

#include "decoder.h"
#include "quant8.h"
#include "xlane.h"

namespace strata {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t b) {
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

// Maximum and sum over the 64 lanes of a wave, returned to every lane: DPP and swizzle steps within each half, then
// the two halves' results through scalar lane reads (no LDS round trip per step).
__device__ __forceinline__ float wave_max64(float v) {
    v = fmaxf(v, xl32f<0>(v));
    v = fmaxf(v, xl32f<1>(v));
    v = fmaxf(v, xl32f<2>(v));
    v = fmaxf(v, xl32f<3>(v));
    v = fmaxf(v, xl32f<4>(v));
    return fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
                 __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)));
}
__device__ __forceinline__ float wave_sum64(float v) {
    v += xl32f<0>(v);
    v += xl32f<1>(v);
    v += xl32f<2>(v);
    v += xl32f<3>(v);
    v += xl32f<4>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
}

// 2^x by the hardware's v_exp_f32 (within 1 ulp; 2^-inf = 0). The softmaxes work in log2 units: scores times log2(e)
// (one rounding, relative 2^-24 of the exponent, so about |s| 2^-24 ln 2 of each weight: ~1e-7 for the scores that
// carry the weight), then exp2 of the difference from the running maximum.
constexpr float LOG2E = 1.44269504088896341f;
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Word i (0..3, a constant) of v.
__device__ __forceinline__ uint32_t u4c(const uint4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// Positions of token t: base .. end (inclusive); a sliding window keeps the last `win`.
__device__ __forceinline__ void att_range(const int* step, int t, int win, int& base, int& n_pos) {
    const int end = step[2 * t];
    base = win > 0 ? max(end + 1 - win, 0) : 0;
    n_pos = end + 1 - base;
}

// Eight softmax weights p (in [0, 1]) times 2^14 as f16 hi and lo parts for the P V MFMA: hi rounded toward zero two
// at a time (v_cvt_pkrtz_f16_f32), lo the remainder (also toward zero), so hi + lo carries each weight to ~2^-21 of
// its value and the lo parts stay normal f16 numbers down to p ~ 2^-17.
__device__ __forceinline__ void split_p8(const float (&p)[8], h8& hi, h8& lo) {
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float a = p[2 * e] * 16384.0f, b = p[2 * e + 1] * 16384.0f;
        const auto hh = __builtin_amdgcn_cvt_pkrtz(a, b);
        const auto ll = __builtin_amdgcn_cvt_pkrtz(a - (float)hh[0], b - (float)hh[1]);
        hw[e] = __builtin_bit_cast(uint32_t, hh);
        lw[e] = __builtin_bit_cast(uint32_t, ll);
    }
    hi = __builtin_bit_cast(h8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
    lo = __builtin_bit_cast(h8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
}

// ---------------- decode ----------------
// Positions a split of a token with n_pos positions: at least one chunk of 64, so short contexts use few waves.
__device__ __forceinline__ int split_len(int n_pos, int ns) { return max((n_pos + ns - 1) / ns, 64); }

// Layout of the K tile ([key][dim]) and the V tile transposed ([dim][key]) in LDS, 64 keys.
template <int HD> struct PfLayout {
    static constexpr int KP = HD + 8;          // halves per K row in LDS (16-byte pad: rows start in spread banks)
    static constexpr int VP = 64 + 4;          // halves per V^T row (8-byte pad)
};

// grid (ATT_SPLITS, nkv, nt), 4 waves a block. Block (s, g, t) serves the G = nh / nkv query heads of KV head g over
// the s-th share of token t's positions, 64 keys a chunk, and wave w takes keys 16 w .. 16 w + 15 of each chunk with
// its own online softmax (running max m, sum l, accumulator o per head), on f16 MFMA with f32 accuracy:
//   S^T (16 keys x 16 heads) = K (A: key row, 8 dims a lane; v_mfma_f32_16x16x32_f16) Q^T (B: head column; q split
//   into f16 hi and lo after scaling it by a power of two that puts its largest value in [2^13, 2^14));
//   the softmax of a head runs over the lane's 4 values and its 4 lane groups;
//   O^T (16 dims x 16 heads, DT dim tiles) += V^T (A: dim row, 4 keys; v_mfma_f32_16x16x16f16) P^T (B: the lane's
//   own 4 weights, times 2^14, split hi and lo: the score tile's layout is the K = 16 operand's).
// Each wave loads its 16 keys' K and V rows (lane l: keys 4 (l % 4) .. + 3, dims 8 (l / 4) .. + 7), K into its own
// LDS rows as is and V transposed. After the last chunk the four waves' (m, l, o) meet in LDS and the block leaves
// [acc (hd) | max | sum] per head in part (max in log2 units); attn_merge_kernel combines the splits.
// NR (one decode token): the query heads arrive raw and the block applies rms_norm_rope_qk itself (norm_rope_kernel's
// arithmetic: the same bits), and the block whose split holds the token's own position also norms and ropes its key
// head, stores the new key and value into the f16 caches and uses them for that position (no block reads it from the
// cache): one launch in place of rms_norm_rope_qk + kv store + attention.
constexpr int DEC_WAVES = 4;
template <int HD>
struct DecLayout {
    static constexpr int KP = HD + 8;    // halves per K row (16-byte pad: rows start in spread banks)
    static constexpr int VP = 16 + 4;    // halves per V^T row of a wave's 16 keys (8-byte pad)
    static constexpr int WAVE = 16 * KP * 2 + HD * VP * 2;  // bytes of one wave's K and V^T tiles
    static constexpr int MERGE = DEC_WAVES * (HD * 16 + 32) * 4;  // the waves' o, m and l for the block merge
    static constexpr int BYTES = DEC_WAVES * WAVE > MERGE ? DEC_WAVES * WAVE : MERGE;
};
template <int HD, int G, bool NR>
__global__ __launch_bounds__(64 * DEC_WAVES) void attn_decode_kernel(const float* __restrict__ q,
                                                                     const uint16_t* __restrict__ kc,
                                                                     const uint16_t* __restrict__ vc,
                                                                     float* __restrict__ part, const int* step, int nh,
                                                                     int nkv, float scale, int win, NormRope nr) {
    using L = DecLayout<HD>;
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    constexpr int KS = HD / 32, DT = HD / 16, NDG = HD / 8;  // K-steps of the scores; dim tiles; 8-dim groups
    __shared__ __align__(16) uint8_t lds[L::BYTES];
    const int split = blockIdx.x, g = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    uint16_t* ks = (uint16_t*)(lds + wave * L::WAVE);
    uint16_t* vs = ks + 16 * L::KP;
    const int h0 = g * G, ns = gridDim.x;
    const uint64_t kvd = (uint64_t)nkv * HD;
    // the query first (it does not depend on the position), then the first chunk's K and V rows as soon as the
    // position is known, so the round trips overlap
    f4 qv[2 * KS];  // dims 32 k + 8 lg .. + 3 and + 4 .. + 7
    if constexpr (!NR) {
        const float* qr = q + (uint64_t)t * nh * HD + (uint64_t)(h0 + l16) * HD;
#pragma unroll
        for (int k = 0; k < KS; k++) {
            qv[2 * k] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
            qv[2 * k + 1] = qv[2 * k];
            if (l16 < G) {
                qv[2 * k] = *(const f4*)(qr + 32 * k + 8 * lg);
                qv[2 * k + 1] = *(const f4*)(qr + 32 * k + 8 * lg + 4);
            }
        }
    }
    int base, n_pos;
    att_range(step, t, win, base, n_pos);
    const int per_s = split_len(n_pos, ns);
    const int p0 = split * per_s, p1 = min(n_pos, p0 + per_s);
    if (p0 >= n_pos) return;  // (the whole block) past the token's positions: the merge reads only the splits that have some
    // NR: the new position's key and value (f16), in LDS for the split that holds the position
    __shared__ __align__(16) uint16_t knew[NR ? HD : 8], vnew[NR ? HD : 8];
    const int pos_new = step[0];
    const bool last = NR && p1 == n_pos;
    const int kq = lane & 3, dg = lane >> 2;  // this lane's load keys 4 kq .., dims 8 dg ..
    const bool loader = dg < NDG;
    // NR: the chunk's K and V rows (this wave's 16 keys; keys past nc repeat key nc - 1: finite, and their weights are
    // 0) go into these function-scope registers, the first chunk's requested before the norms and rope, which run
    // while they are in flight (without NR they are requested in the loop, behind the query's loads)
    uint4 kbn[NR ? 4 : 1], vbn[NR ? 4 : 1];
    auto load_n = [&](int c0) __attribute__((always_inline)) {
        const int nc = min(64, p1 - c0);
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const int kp = base + c0 + min(16 * wave + 4 * kq + kk, nc - 1);
            const uint64_t off = (uint64_t)kp * kvd + g * HD + 8 * min(dg, NDG - 1);
            kbn[kk & (NR ? 3 : 0)] = *(const uint4*)(kc + off);
            vbn[kk & (NR ? 3 : 0)] = *(const uint4*)(vc + off);
        }
    };
    if constexpr (NR) load_n(p0);
    if constexpr (NR) {
        // raw heads into LDS: the G query heads, then (last split) the key and value heads of KV head g
        __shared__ __align__(16) float raw[(G + 2) * HD];
        __shared__ float ssq[G + 1];
        const int nhd = G + (last ? 2 : 0);
        for (int c = tid; c < nhd * HD / 4; c += 64 * DEC_WAVES) {
            const int j = c / (HD / 4), i = 4 * (c % (HD / 4));
            const float* src = j < G ? nr.qx + (uint64_t)(h0 + j) * nr.q_stride
                                     : j == G ? nr.x + (uint64_t)g * nr.x_stride : nr.v + (uint64_t)g * HD;
            *(float4*)&raw[j * HD + i] = *(const float4*)(src + i);
        }
        __syncthreads();
        // the heads' sums of squares in index order, a lane per head (the reference's iterator sum), by wave 1 while
        // wave 0 computes the rope angles
        __shared__ float rsn[HD / 2], rcs[HD / 2];
        if (wave == 1 && lane < G + (last ? 1 : 0)) {
            const float* xr = raw + lane * HD;
            ssq[lane] = nr_sumsq(HD, [&](int i0, float4 (&r)[8]) {
#pragma unroll
                for (int c = 0; c < 8; c++) r[c] = *(const float4*)&xr[i0 + 4 * c];
            });
        }
        // the rope angles of pair i (lane i of wave 0; n_rot / 2 <= 64), f64 as ops::rope_neox
        const int half = nr.n_rot / 2;
        constexpr int NPJ = (HD / 2 + 63) / 64;
        if (wave == 0 && lane < half) {
            const double f = lane < nr.nfreq ? nr.freq[lane] : pow((double)nr.base, -2.0 * (double)lane / (double)nr.n_rot);
            double sd, cd;
            sincos((double)pos_new * f, &sd, &cd);
            rsn[lane] = (float)sd;
            rcs[lane] = (float)cd;
        }
        __syncthreads();
        float sn[NPJ], cs[NPJ];
#pragma unroll
        for (int j = 0; j < NPJ; j++) {
            const int i = lane + 64 * j;
            sn[j] = i < half ? rsn[i] : 0.0f;
            cs[j] = i < half ? rcs[i] : 0.0f;
        }
        // head j by wave j % 4: x * (1 / sqrt(ss / n + eps)) * w, then the rope, in place
        for (int j = wave; j < G + (last ? 1 : 0); j += DEC_WAVES) {
            float* hr = raw + j * HD;
            const float* wr = j < G ? nr.qw : nr.w;
            const float sc = 1.0f / sqrtf(ssq[j] / (float)HD + nr.eps);
#pragma unroll
            for (int u = 0; u < HD / 64; u++) hr[lane + 64 * u] = hr[lane + 64 * u] * sc * wr[lane + 64 * u];
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int u = 0; u < NPJ; u++) {
                const int i = lane + 64 * u;
                if (i < half) {
                    const float pa = hr[i], pb = hr[i + half];
                    hr[i] = pa * cs[u] - pb * sn[u];
                    hr[i + half] = pa * sn[u] + pb * cs[u];
                }
            }
            __builtin_amdgcn_wave_barrier();
            if (j == G) {
                // the new key and value: into the caches (row pos_new nkv + g) and into LDS for this split
                const uint64_t e = ((uint64_t)pos_new * nkv + g) * HD;
#pragma unroll
                for (int u = 0; u < HD / 64; u++) {
                    const int i = lane + 64 * u;
                    const _Float16 kh = (_Float16)hr[i], vh = (_Float16)raw[(G + 1) * HD + i];
                    const uint16_t kb16 = __builtin_bit_cast(uint16_t, kh), vb16 = __builtin_bit_cast(uint16_t, vh);
                    knew[i] = kb16;
                    vnew[i] = vb16;
                    ((uint16_t*)nr.kc)[e + i] = kb16;
                    ((uint16_t*)nr.vc)[e + i] = vb16;
                }
            }
        }
        __syncthreads();
        // the query fragments from the normed, roped heads
#pragma unroll
        for (int k = 0; k < KS; k++) {
            qv[2 * k] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
            qv[2 * k + 1] = qv[2 * k];
            if (l16 < G) {
                qv[2 * k] = *(const f4*)&raw[l16 * HD + 32 * k + 8 * lg];
                qv[2 * k + 1] = *(const f4*)&raw[l16 * HD + 32 * k + 8 * lg + 4];
            }
        }
    }
    // Q^T fragments: head h0 + l16 (zero past G), dims 32 k + 8 lg .. + 7; usc undoes the scaling (times `scale`)
    h8 qh[KS], ql[KS];
    float usc = 0.0f;
    f4 o[DT];
#pragma unroll
    for (int d = 0; d < DT; d++) o[d] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    for (int c0 = p0; c0 < p1; c0 += 64) {
        const int nc = min(64, p1 - c0);
        // stage(kb, vb): the query's fragments (first chunk), then the chunk's K rows and V^T into the wave's LDS tiles
        auto stage = [&](uint4 (&kb)[4], uint4 (&vb)[4]) __attribute__((always_inline)) {
            if (c0 == p0) {
                // the query's fragments while the first chunk's rows are in flight: scaled by the power of two
                // that puts its largest value in [2^13, 2^14), so the lo parts stay normal f16 numbers
                float mx = 0.0f;
#pragma unroll
                for (int k = 0; k < 2 * KS; k++)
#pragma unroll
                    for (int e = 0; e < 4; e++) mx = fmaxf(mx, fabsf(qv[k][e]));
                mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                int ex = 0;
                if (mx > 0.0f) (void)frexpf(mx, &ex);  // mx < 2^ex
                const float up = ldexpf(1.0f, 14 - ex);
                usc = ldexpf(scale * LOG2E, ex - 14);  // scores in log2 units: the softmax's exps are exp2s
#pragma unroll
                for (int k = 0; k < KS; k++)
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float x = qv[2 * k + (e >> 2)][e & 3] * up;
                        const _Float16 hi = (_Float16)x;
                        qh[k][e] = hi;
                        ql[k][e] = (_Float16)(x - (float)hi);
                    }
            }
            if (loader) {
#pragma unroll
                for (int kk = 0; kk < 4; kk++) *(uint4*)&ks[(4 * kq + kk) * L::KP + 8 * dg] = kb[kk];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int sh = 16 * (e & 1);
                    const uint32_t a0 = (u4c(vb[0], e >> 1) >> sh) & 0xFFFFu, a1 = (u4c(vb[1], e >> 1) >> sh) & 0xFFFFu;
                    const uint32_t a2 = (u4c(vb[2], e >> 1) >> sh) & 0xFFFFu, a3 = (u4c(vb[3], e >> 1) >> sh) & 0xFFFFu;
                    *(uint2*)&vs[(8 * dg + e) * L::VP + 4 * kq] = make_uint2(a0 | (a1 << 16), a2 | (a3 << 16));
                }
            }
        };
        if constexpr (NR) {
            if (c0 != p0) load_n(c0);
            if (last) {
                // the new position (its cache row may not have landed yet): this block's own key and value
#pragma unroll
                for (int kk = 0; kk < 4; kk++)
                    if (base + c0 + min(16 * wave + 4 * kq + kk, nc - 1) == pos_new) {
                        kbn[kk & (NR ? 3 : 0)] = *(const uint4*)&knew[8 * min(dg, NDG - 1)];
                        vbn[kk & (NR ? 3 : 0)] = *(const uint4*)&vnew[8 * min(dg, NDG - 1)];
                    }
            }
            stage(*(uint4(*)[4])kbn, *(uint4(*)[4])vbn);
        } else {
            uint4 kb[4], vb[4];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int kp = base + c0 + min(16 * wave + 4 * kq + kk, nc - 1);
                const uint64_t off = (uint64_t)kp * kvd + g * HD + 8 * min(dg, NDG - 1);
                kb[kk] = *(const uint4*)(kc + off);
                vb[kk] = *(const uint4*)(vc + off);
            }
            stage(kb, vb);
        }
        __builtin_amdgcn_wave_barrier();
        // S^T: lane holds keys 16 wave + 4 lg + i of head l16
        f4 sv = (f4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < KS; k++) {
            const h8 kf = *(const h8*)&ks[l16 * L::KP + 32 * k + 8 * lg];
            sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[k], sv, 0, 0, 0);
            sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[k], sv, 0, 0, 0);
        }
        // online softmax of head l16 over the wave's keys of the chunk
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v = sv[i];  // the raw score: usc (> 0) is applied in the exponent's fma
            if (16 * wave + 4 * lg + i >= nc) v = -INFINITY;
            sv[i] = v;
            mx = fmaxf(mx, v);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(m, mx * usc);  // max(v) usc = max(v usc): a positive factor keeps the order
        const float alpha = m == -INFINITY ? 0.0f : exp2_hw(m - mnew);
        const float mref = mnew == -INFINITY ? 0.0f : mnew;  // a wave with no key yet: every p is 0
        float sum = 0.0f, p[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            p[i] = exp2_hw(__builtin_fmaf(sv[i], usc, -mref));  // exp2(-inf) = 0
            sum += p[i];
        }
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        l = l * alpha + sum;
        m = mnew;
#pragma unroll
        for (int d = 0; d < DT; d++) o[d] *= alpha;
        // O^T += V^T P^T over the wave's 16 keys: the weights times 2^14 as f16 hi and lo parts (rounded toward
        // zero, the lo parts normal down to p ~ 2^-17)
        h4 ph, pl;
        {
            const float a0 = p[0] * 16384.0f, a1 = p[1] * 16384.0f, a2 = p[2] * 16384.0f, a3 = p[3] * 16384.0f;
            const auto h01 = __builtin_amdgcn_cvt_pkrtz(a0, a1), h23 = __builtin_amdgcn_cvt_pkrtz(a2, a3);
            const auto l01 = __builtin_amdgcn_cvt_pkrtz(a0 - (float)h01[0], a1 - (float)h01[1]);
            const auto l23 = __builtin_amdgcn_cvt_pkrtz(a2 - (float)h23[0], a3 - (float)h23[1]);
            ph = __builtin_bit_cast(h4, make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23)));
            pl = __builtin_bit_cast(h4, make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)));
        }
#pragma unroll
        for (int d = 0; d < DT; d++) {
            const h4 vf = __builtin_bit_cast(h4, *(const uint2*)&vs[(16 * d + l16) * L::VP + 4 * lg]);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x16f16(vf, ph, o[d], 0, 0, 0);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x16f16(vf, pl, o[d], 0, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();  // ks and vs are rewritten by the next chunk
    }
    // the four waves' partials meet in LDS: ow[w][dim][head], mw[w][head], lw[w][head]
    __syncthreads();  // every wave is done with its K and V tiles
    float* ow = (float*)lds;
    float* mw = ow + DEC_WAVES * HD * 16;
    float* lw = mw + DEC_WAVES * 16;
#pragma unroll
    for (int d = 0; d < DT; d++)
#pragma unroll
        for (int i = 0; i < 4; i++) ow[(wave * HD + 16 * d + 4 * lg + i) * 16 + l16] = o[d][i];
    if (lg == 0) {
        mw[wave * 16 + l16] = m;
        lw[wave * 16 + l16] = l;
    }
    __syncthreads();
    // thread: head tid / 16, dims (tid % 16) HD / 16 ..; the waves added in wave order
    constexpr int DPT = HD / 16;
    const int hh = tid >> 4, dd0 = (tid & 15) * DPT;
    if (hh < G) {
        float mws[DEC_WAVES], M = -INFINITY;
#pragma unroll
        for (int w = 0; w < DEC_WAVES; w++) {
            mws[w] = mw[w * 16 + hh];
            M = fmaxf(M, mws[w]);
        }
        float ew[DEC_WAVES], Lsum = 0.0f;
#pragma unroll
        for (int w = 0; w < DEC_WAVES; w++) {
            ew[w] = mws[w] == -INFINITY ? 0.0f : exp2_hw(mws[w] - M);
            Lsum += lw[w * 16 + hh] * ew[w];
        }
        float* pp = part + ((uint64_t)(t * nh + h0 + hh) * ns + split) * (HD + 2);
#pragma unroll
        for (int e = 0; e < DPT; e++) {
            float acc = 0.0f;
#pragma unroll
            for (int w = 0; w < DEC_WAVES; w++) acc += ow[(w * HD + dd0 + e) * 16 + hh] * ew[w];
            pp[dd0 + e] = acc * (1.0f / 16384.0f);  // the weights' 2^14 taken out
        }
        if ((tid & 15) == 0) {
            pp[HD] = M;
            pp[HD + 1] = Lsum;
        }
    }
}

// grid (nh / HPB, nt), HPB groups of 4 waves, group j serving head HPB blockIdx.x + j: out = sum_s acc_s 2^(m_s - M) /
// (sum_s l_s 2^(m_s - M) + 2^(sink log2(e) - M)) (sigmoid gate), the maxima in log2 units.
// Wave w of a group takes splits w, w + 4, ..: their weights (a lane each), then the weighted sum of their partial rows
// (lane = dims), all of its loads in flight together; the 4 wave sums are added in wave order through LDS.
// With xq (HPB = 256 / HD: a block's heads are one 256-value group of the row) the block also quantizes its outputs
// as quant_xq does into xq ([nt rows of nh HD int8][nt rows of nh HD / 32 scales]), for a GEMV that takes x
// pre-quantized.
template <int HD, int HPB>
__global__ __launch_bounds__(256 * HPB) void attn_merge_kernel(const float* __restrict__ part, const float* __restrict__ qg,
                                                               float* __restrict__ out, int nh, int ns,
                                                               const float* __restrict__ sink, const int* step, int win,
                                                               int8_t* xq, int mode) {
    constexpr int DL = HD / 64, SW = ATT_SPLITS / 4;  // dims a lane; splits a wave
    __shared__ float sm[HPB][4], sd[HPB][4], so[HPB][4][HD];
    __shared__ __align__(16) float ob[HPB * HD];
    const int grp = threadIdx.x >> 8, h = blockIdx.x * HPB + grp, t = blockIdx.y;
    const int wave = (threadIdx.x >> 6) & 3, lane = threadIdx.x & 63;
    const float* pp = part + (uint64_t)(t * nh + h) * ns * (HD + 2);
    {
        // the splits that hold positions (the decode leaves the others unwritten)
        int base, n_pos;
        att_range(step, t, win, base, n_pos);
        const int per_s = split_len(n_pos, ns);
        ns = min(ns, (n_pos + per_s - 1) / per_s);
    }
    const float sk = sink ? sink[h] * LOG2E : -INFINITY;  // the splits' maxima are in log2 units
    // this wave's splits: s = wave + 4 i, i < SW (lane i < SW holds split i's max and sum)
    const int sl = wave + 4 * lane;
    const float ms = lane < SW && sl < ns ? pp[sl * (HD + 2) + HD] : -INFINITY;
    const float ls = lane < SW && sl < ns ? pp[sl * (HD + 2) + HD + 1] : 0.0f;
    // (8-byte loads where a lane's dims pair up; splits past ns are not loaded: a wave-uniform bound)
    float a[SW][DL];
#pragma unroll
    for (int i = 0; i < SW; i++) {
        if (wave + 4 * i < ns) {
            const float* src = pp + (wave + 4 * i) * (HD + 2) + DL * lane;
            if constexpr (DL == 2) {
                const float2 v = *(const float2*)src;
                a[i][0] = v.x;
                a[i][1] = v.y;
            } else {
#pragma unroll
                for (int d = 0; d < DL; d++) a[i][d] = src[d];
            }
        } else {
#pragma unroll
            for (int d = 0; d < DL; d++) a[i][d] = 0.0f;
        }
    }
    float M = wave_max64(ms);
    if (lane == 0) sm[grp][wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(fmaxf(sm[grp][0], sm[grp][1]), fmaxf(sm[grp][2], sm[grp][3])), sk);
    const float e = ms == -INFINITY ? 0.0f : exp2_hw(ms - M);
    const float den = wave_sum64(ls * e);
    float o[DL];
#pragma unroll
    for (int d = 0; d < DL; d++) o[d] = 0.0f;
#pragma unroll
    for (int i = 0; i < SW; i++) {
        const float es = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), i));
#pragma unroll
        for (int d = 0; d < DL; d++) o[d] += a[i][d] * es;
    }
    if (lane == 0) sd[grp][wave] = den;
#pragma unroll
    for (int d = 0; d < DL; d++) so[grp][wave][DL * lane + d] = o[d];
    __syncthreads();
    if (wave == 0) {
        float dt = sd[grp][0] + sd[grp][1] + sd[grp][2] + sd[grp][3];
        if (sk != -INFINITY) dt += exp2_hw(sk - M);
#pragma unroll
        for (int d = 0; d < DL; d++) {
            const int dd = DL * lane + d;
            const float ov = so[grp][0][dd] + so[grp][1][dd] + so[grp][2][dd] + so[grp][3][dd];
            float r = dt > 0.0f ? ov / dt : 0.0f;
            if (qg) r *= sigmoid_f(qg[(uint64_t)t * nh * 2 * HD + h * 2 * HD + HD + dd]);
            out[(uint64_t)t * nh * HD + h * HD + dd] = r;
            ob[grp * HD + dd] = r;
        }
    }
    if constexpr (HPB * HD == 256) {
        if (xq) {
            __syncthreads();
            if (threadIdx.x < 32) {
                const int i = 8 * threadIdx.x, n = nh * HD, nt = gridDim.y;
                const float4 v0 = *(const float4*)&ob[i], v1 = *(const float4*)&ob[i + 4];
                const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
                const uint64_t c0 = (uint64_t)blockIdx.x * 256;
                quant8_group(v, i, true, mode, xq + (uint64_t)t * n + c0,
                             (float*)(xq + (uint64_t)nt * n) + ((uint64_t)t * n + c0) / 32);
            }
        }
    }
}

template <int HD, int G>
static void decode_t(const float* q, const uint16_t* kc, const uint16_t* vc, float* part, const int* step, int nh,
                     int nkv, float scale, int nt, int win, const NormRope* nr, hipStream_t s) {
    const dim3 grid(ATT_SPLITS, (unsigned)nkv, (unsigned)nt), block(64 * DEC_WAVES);
    if (nr)
        attn_decode_kernel<HD, G, true><<<grid, block, 0, s>>>(q, kc, vc, part, step, nh, nkv, scale, win, *nr);
    else
        attn_decode_kernel<HD, G, false><<<grid, block, 0, s>>>(q, kc, vc, part, step, nh, nkv, scale, win, NormRope{});
}

hipError_t launch_attn_decode(const float* q, const uint16_t* kc, const uint16_t* vc, const float* qg, float* out,
                              float* part, const int* step, int nh, int nkv, int hd, float scale, int nt,
                              const float* sink, int win, hipStream_t s, const NormRope* nr0, int8_t* xq, int mode) {
    if (nt <= 0) return hipSuccess;
    if (xq && (nh * hd) % 256) return hipErrorNotSupported;
    const int G = nh / nkv;
    NormRope nrf;
    const NormRope* nr = nullptr;
    if (nr0) {
        // one token, heads of hd (rows of the f16 caches), the rope frequencies from the host's pow as in
        // launch_norm_rope
        if (nt != 1 || nr0->n != hd || nr0->n_rot > hd || nr0->n_rot % 2 || !nr0->kc || !nr0->vc ||
            ((uintptr_t)nr0->qx | (uintptr_t)nr0->x | (uintptr_t)nr0->v) % 16 || nr0->q_stride % 4 || nr0->x_stride % 4)
            return hipErrorNotSupported;
        nrf = *nr0;
        nrf.nfreq = nrf.n_rot / 2 <= NormRope::NFREQ ? nrf.n_rot / 2 : 0;
        for (int i = 0; i < nrf.nfreq; i++) nrf.freq[i] = std::pow((double)nrf.base, -2.0 * (double)i / (double)nrf.n_rot);
        nr = &nrf;
    }
#define DEC(HD_, G_) if (hd == HD_ && G == G_) decode_t<HD_, G_>(q, kc, vc, part, step, nh, nkv, scale, nt, win, nr, s); else
    DEC(128, 1) DEC(128, 2) DEC(128, 4) DEC(128, 8) DEC(64, 1) DEC(64, 2) DEC(64, 4) DEC(64, 8)
    return hipErrorInvalidValue;
#undef DEC
    if (xq && hd == 128)
        attn_merge_kernel<128, 2><<<dim3((unsigned)(nh / 2), (unsigned)nt), dim3(512), 0, s>>>(part, qg, out, nh, ATT_SPLITS, sink, step, win, xq, mode);
    else if (xq)
        attn_merge_kernel<64, 4><<<dim3((unsigned)(nh / 4), (unsigned)nt), dim3(1024), 0, s>>>(part, qg, out, nh, ATT_SPLITS, sink, step, win, xq, mode);
    else if (hd == 128)
        attn_merge_kernel<128, 1><<<dim3((unsigned)nh, (unsigned)nt), dim3(256), 0, s>>>(part, qg, out, nh, ATT_SPLITS, sink, step, win, nullptr, mode);
    else
        attn_merge_kernel<64, 1><<<dim3((unsigned)nh, (unsigned)nt), dim3(256), 0, s>>>(part, qg, out, nh, ATT_SPLITS, sink, step, win, nullptr, mode);
    return hipGetLastError();
}

// ---------------- prefill ----------------
// grid (ceil(ceil(t / 16) / 2), nkv), G waves: wave w is query head g G + w over the block's two 16-query MFMA columns
// j, the 16-row tiles qb and ceil(t / 16) - 1 - qb (from the two ends of the chunk, so that the blocks' causal work
// is even), and every K/V tile in LDS serves the whole GQA group. Query row i sits at position step[0] + i and sees
// keys base(i) .. step[0] + i (base 0, or the sliding window's start); a column takes part in a key tile only while
// the tile holds keys its rows see. Per tile of 64 keys:
//   S^T (16 keys x 16 queries, 4 key sub-tiles kt) = sum over dims of K (A: key row, 8 dims a lane) with Q^T hi and lo
//   (B: query column, the same 8 dims); lane holds keys 16 kt + 4 (l / 16) + i of query 16 j + l % 16.
//   Online softmax per query column (the lane's 16 values, then across the 4 lane groups).
//   O^T (16 dims x 16 queries, 8 dim tiles dt) += V^T (A: dim row, 8 keys) P^T hi and lo (B: the lane's own p values:
//   keys 4 (l / 16) + i of sub-tiles 2 c and 2 c + 1 make the 8 K-elements of k-step c, and V^T's A fragment reads
//   the same keys).
constexpr int PF_BK = 64;  // keys a tile (PfLayout's 64)

template <int HD, int G>
__global__ __launch_bounds__(64 * G) void attn_prefill_kernel(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                              const uint16_t* __restrict__ vc, const float* __restrict__ qg,
                                                              float* __restrict__ out, const int* step, int T, int nh,
                                                              int nkv, float scale, const float* __restrict__ sink,
                                                              int win) {
    using L = PfLayout<HD>;
    constexpr int KS = HD / 32, DT = HD / 16, NTH = 64 * G;
    __shared__ __align__(16) uint16_t ks[PF_BK * L::KP];
    __shared__ __align__(16) uint16_t vs[HD * L::VP];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    const int g = blockIdx.y, h = g * G + wave, pos0 = step[0];
    const uint64_t kvd = (uint64_t)nkv * HD;
    // the block's two query columns are 16-row tiles from opposite ends of the T rows (tiles qb and nht - 1 - qb),
    // so every block has about the same causal work; each column's MFMAs and softmax stop at its own last key
    const int nht = (T + 15) / 16, qb = blockIdx.x;
    const int r0[2] = {16 * qb, 16 * (nht - 1 - qb)};
    const bool two = nht - 1 - qb != qb;
    int lastj[2], firstj[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        lastj[j] = pos0 + min(r0[j] + 15, T - 1);  // the last key the column's rows see
        firstj[j] = win > 0 ? max(pos0 + r0[j] + 1 - win, 0) : 0;
    }
    if (!two) {
        lastj[1] = -1;
        firstj[1] = INT_MAX;
    }
    const int last = max(lastj[0], lastj[1]), first = min(firstj[0], firstj[1]);
    // Q^T fragments (B operand): query r0[j] + l16, dims 32 ks + 8 lg .. + 7, split into f16 hi and lo after scaling
    // the query by a power of two that puts its largest value in [2^13, 2^14): the lo parts then stay normal f16
    // numbers (no subnormal precision loss) and the hi parts cannot overflow. usc[j] undoes it (times `scale`).
    h8 qh[2][KS], ql[2][KS];
    float usc[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int row = r0[j] + l16;
        const float* qr = q + (uint64_t)row * nh * HD + h * HD;
        float v[KS][8];
        float mx = 0.0f;
#pragma unroll
        for (int k = 0; k < KS; k++) {
            if (row < T && (j == 0 || two)) {
                const float4 a = *(const float4*)(qr + 32 * k + 8 * lg), b = *(const float4*)(qr + 32 * k + 8 * lg + 4);
                v[k][0] = a.x; v[k][1] = a.y; v[k][2] = a.z; v[k][3] = a.w;
                v[k][4] = b.x; v[k][5] = b.y; v[k][6] = b.z; v[k][7] = b.w;
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) v[k][e] = 0.0f;
            }
#pragma unroll
            for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(v[k][e]));
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        int ex = 0;
        if (mx > 0.0f) (void)frexpf(mx, &ex);  // mx < 2^ex
        const float up = ldexpf(1.0f, 14 - ex);
        usc[j] = ldexpf(scale * LOG2E, ex - 14);  // scores in log2 units: the softmax's exps are exp2s
#pragma unroll
        for (int k = 0; k < KS; k++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float x = v[k][e] * up;
                const _Float16 hi = (_Float16)x;
                qh[j][k][e] = hi;
                ql[j][k][e] = (_Float16)(x - (float)hi);
            }
    }
    f4 o[2][DT];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int d = 0; d < DT; d++) o[j][d] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
    const int qpos[2] = {pos0 + r0[0] + l16, pos0 + r0[1] + l16};  // the lane's query position per column j
    // K tile [key][dim] and V tile transposed [dim][key], chunk i = tid + NTH u of a tile: key i % 64, dims
    // 8 (i / 64) ..; the next tile's chunks are loaded into registers while this one is computed. Keys past `last`
    // are zeros (finite: p = 0 times them).
    constexpr int NPT = PF_BK * HD / 8 / NTH;  // 16-byte chunks a thread of each of K and V
    uint4 kr[NPT], vr4[NPT];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int u = 0; u < NPT; u++) {
            const int i = tid + NTH * u, key = i % PF_BK, c = (i / PF_BK) * 8, kp = k0 + key;
            kr[u] = make_uint4(0, 0, 0, 0);
            vr4[u] = kr[u];
            if (kp <= last) {
                kr[u] = *(const uint4*)(kc + (uint64_t)kp * kvd + g * HD + c);
                vr4[u] = *(const uint4*)(vc + (uint64_t)kp * kvd + g * HD + c);
            }
        }
    };
    const int kbeg = first / PF_BK * PF_BK;
    fetch(kbeg);
    for (int k0 = kbeg; k0 <= last; k0 += PF_BK) {
        __syncthreads();  // the previous tile's readers are done
#pragma unroll
        for (int u = 0; u < NPT; u++) {
            const int i = tid + NTH * u, key = i % PF_BK, c = (i / PF_BK) * 8;
            *(uint4*)&ks[key * L::KP + c] = kr[u];
            const uint32_t w4[4] = {vr4[u].x, vr4[u].y, vr4[u].z, vr4[u].w};
#pragma unroll
            for (int e = 0; e < 8; e++) vs[(c + e) * L::VP + key] = (uint16_t)(w4[e >> 1] >> (16 * (e & 1)));
        }
        __syncthreads();
        if (k0 + PF_BK <= last) fetch(k0 + PF_BK);
        bool live[2];
#pragma unroll
        for (int j = 0; j < 2; j++) live[j] = k0 <= lastj[j] && k0 + PF_BK - 1 >= firstj[j];
        // S^T
        f4 s[2][4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            h8 kf[KS];
#pragma unroll
            for (int k = 0; k < KS; k++) kf[k] = *(const h8*)&ks[(16 * kt + l16) * L::KP + 32 * k + 8 * lg];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                f4 c = (f4){0.0f, 0.0f, 0.0f, 0.0f};
                if (live[j])
#pragma unroll
                for (int k = 0; k < KS; k++) {
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[k], qh[j][k], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[k], ql[j][k], c, 0, 0, 0);
                }
                s[j][kt] = c;
            }
        }
        // online softmax per query column; keys outside first .. qpos masked, on the tiles that have such keys
#pragma unroll
        for (int j = 0; j < 2; j++) {
            if (!live[j]) continue;
            const bool edge = k0 + PF_BK - 1 > pos0 + r0[j] || (win > 0 && k0 < lastj[j] + 1 - win);
            const int qp = qpos[j], lo = win > 0 ? qp + 1 - win : INT_MIN;
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int kp = k0 + 16 * kt + 4 * lg + i;
                    float v = s[j][kt][i];  // the raw score: usc (> 0) is applied in the exponent's fma
                    if (edge && (kp > qp || kp < lo)) v = -INFINITY;
                    s[j][kt][i] = v;
                    mx = fmaxf(mx, v);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mnew = fmaxf(m[j], mx * usc[j]);  // max(v) usc = max(v usc): a positive factor keeps the order
            const float alpha = m[j] == -INFINITY ? 0.0f : exp2_hw(m[j] - mnew);
            const float mref = mnew == -INFINITY ? 0.0f : mnew;  // a column with no key yet: every p is 0
            float sum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float p = exp2_hw(__builtin_fmaf(s[j][kt][i], usc[j], -mref));  // exp2(-inf) = 0
                    s[j][kt][i] = p;
                    sum += p;
                }
            sum += __shfl_xor(sum, 16, 64);
            sum += __shfl_xor(sum, 32, 64);
            l[j] = l[j] * alpha + sum;
            m[j] = mnew;
            if (__ballot(alpha != 1.0f))  // the running maximum moved for some column of the wave
#pragma unroll
                for (int d = 0; d < DT; d++) o[j][d] *= alpha;
        }
        // O^T += V^T P^T
#pragma unroll
        for (int c = 0; c < 2; c++) {
            h8 ph[2], pl[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                if (!live[j]) continue;
                float p[8];
#pragma unroll
                for (int e = 0; e < 8; e++) p[e] = s[j][2 * c + (e >> 2)][e & 3];
                split_p8(p, ph[j], pl[j]);
            }
#pragma unroll
            for (int d = 0; d < DT; d++) {
                const uint16_t* vr = &vs[(16 * d + l16) * L::VP + 32 * c + 4 * lg];
                const uint2 a0 = *(const uint2*)vr, a1 = *(const uint2*)(vr + 16);
                const h8 vf = __builtin_bit_cast(h8, make_uint4(a0.x, a0.y, a1.x, a1.y));
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    if (!live[j]) continue;
                    o[j][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, ph[j], o[j][d], 0, 0, 0);
                    o[j][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl[j], o[j][d], 0, 0, 0);
                }
            }
        }
    }
    // out[row, h HD + 16 dt + 4 lg + i] for query row r0[j] + l16
    const float sk = sink ? sink[h] * LOG2E : -INFINITY;  // in the scores' log2 units
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int row = r0[j] + l16;
        if (row >= T || (j == 1 && !two)) continue;
        const float M = fmaxf(m[j], sk);
        const float sc = m[j] == -INFINITY ? 0.0f : exp2_hw(m[j] - M);
        const float den = l[j] * sc + (sk == -INFINITY ? 0.0f : exp2_hw(sk - M));
        const float inv = den > 0.0f ? sc / den * (1.0f / 16384.0f) : 0.0f;  // O carries the weights' 2^14
        float* orow = out + (uint64_t)row * nh * HD + h * HD;
        const float* gate = qg ? qg + (uint64_t)row * nh * 2 * HD + h * 2 * HD + HD : nullptr;
#pragma unroll
        for (int d = 0; d < DT; d++) {
            const int col = 16 * d + 4 * lg;
            float4 r = make_float4(o[j][d][0] * inv, o[j][d][1] * inv, o[j][d][2] * inv, o[j][d][3] * inv);
            if (gate) {
                r.x *= sigmoid_f(gate[col]); r.y *= sigmoid_f(gate[col + 1]);
                r.z *= sigmoid_f(gate[col + 2]); r.w *= sigmoid_f(gate[col + 3]);
            }
            *(float4*)(orow + col) = r;
        }
    }
}

hipError_t launch_attn_prefill(const float* q, const uint16_t* kc, const uint16_t* vc, const float* qg, float* out,
                               const int* step, int t, int nh, int nkv, int hd, float scale, const float* sink, int win,
                               hipStream_t s) {
    if (t <= 0) return hipSuccess;
    const int G = nh / nkv;
    const dim3 grid((unsigned)(((t + 15) / 16 + 1) / 2), (unsigned)nkv);  // a pair of 16-row query tiles a block
#define PF(HD_, G_)                                                                                               \
    if (hd == HD_ && G == G_)                                                                                     \
        attn_prefill_kernel<HD_, G_><<<grid, dim3(64 * G_), 0, s>>>(q, kc, vc, qg, out, step, t, nh, nkv, scale,  \
                                                                     sink, win);                                  \
    else
    PF(128, 1) PF(128, 2) PF(128, 4) PF(128, 8) PF(64, 1) PF(64, 2) PF(64, 4) PF(64, 8)
    return hipErrorInvalidValue;
#undef PF
    return hipGetLastError();
}

}  // namespace strata

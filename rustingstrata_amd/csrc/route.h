// Routing of a token (shared by the route kernels and the GEMV's routing prologue).
#pragma once
#include <hip/hip_runtime.h>

#include "xlane.h"

namespace strata {

// exp for the router and SwiGLU: exp in double, rounded once to f32. This is the correctly rounded f32 exp except
// in vanishingly rare cases, and so agrees with the host libm expf the reference calls (src/ops.rs:14-24) wherever
// that one is correctly rounded.
__device__ __forceinline__ float exp_f32(float x) { return (float)exp((double)x); }

// Routing of one token by one wave64 (Model::route src/model.rs:837-851; topk_warp src/cuda/kernels.cu:2633-2686):
// the n logits at pr (n <= 64 ROUTE_R, ROUTE_R a lane) through softmax (or sigmoid) and top-k. Lane j < k gets rank
// j's expert `id`, its weight `w` (p / the top-k sum, times extra_scale when not 0) and `slot` = table[id] (-1
// without a table). se: 64 ROUTE_R floats of LDS for this wave.
template <int ROUTE_R>
__device__ __forceinline__ void route_wave(const float* __restrict__ pr, int n, int k, float extra_scale,
                                           const int* __restrict__ table, int sigmoid, float* se, int& id_out,
                                           float& w_out, int& slot_out) {
    const int lane = threadIdx.x & 63;
    float v[ROUTE_R];
#pragma unroll
    for (int r = 0; r < ROUTE_R; r++) { int i = lane + 64 * r; v[r] = i < n ? pr[i] : -INFINITY; }
    // the slot table's entries, fetched with the logits (the chosen ones are read from these registers at the end)
    int tv[ROUTE_R];
#pragma unroll
    for (int r = 0; r < ROUTE_R; r++) { int i = lane + 64 * r; tv[r] = table && i < n ? table[i] : -1; }
    if (sigmoid) {
#pragma unroll
        for (int r = 0; r < ROUTE_R; r++) v[r] = 1.0f / (1.0f + exp_f32(-v[r]));  // ops::sigmoid
    } else {
        // ops::softmax: m = max, v = exp(v - m), s = the sum in index order, v /= s.
        float m = -INFINITY;
#pragma unroll
        for (int r = 0; r < ROUTE_R; r++) m = fmaxf(m, v[r]);
        m = fmaxf(m, xl32f<0>(m));
        m = fmaxf(m, xl32f<1>(m));
        m = fmaxf(m, xl32f<2>(m));
        m = fmaxf(m, xl32f<3>(m));
        m = fmaxf(m, xl32f<4>(m));
        m = fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0)),
                  __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32)));
#pragma unroll
        for (int r = 0; r < ROUTE_R; r++) {
            int i = lane + 64 * r;
            if (i < n) v[r] = exp_f32(v[r] - m);
            se[i] = i < n ? v[r] : 0.0f;  // entries past n add +0: the sum keeps its bits
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        // one lane adds in index order (the reference's sum): 64 values a chunk read ahead into registers, 4 per LDS
        // access, then added one by one
        float s = 0.0f;
        if (lane == 0) {
#pragma unroll
            for (int c = 0; c < 64 * ROUTE_R; c += 64) {
                float4 q[16];
#pragma unroll
                for (int u = 0; u < 16; u++) q[u] = *(const float4*)&se[c + 4 * u];
#pragma unroll
                for (int u = 0; u < 16; u++) {
                    s += q[u].x;
                    s += q[u].y;
                    s += q[u].z;
                    s += q[u].w;
                }
            }
        }
        s = __shfl(s, 0);
#pragma unroll
        for (int r = 0; r < ROUTE_R; r++) v[r] = v[r] / s;
    }
    // ops::top_k: k rounds of the wave's largest value, ties to the lower index. v >= 0, so its bits order as it;
    // key = bits + 1, 0 for taken or absent entries. A round takes the largest key by 32-bit max steps, then the
    // lowest index holding it from ballots in index order (entry r of lane l is index 64 r + l).
    uint32_t key[ROUTE_R];
#pragma unroll
    for (int r = 0; r < ROUTE_R; r++) key[r] = lane + 64 * r < n ? __float_as_uint(v[r]) + 1u : 0u;
    int my_id = 0;
    float my_p = 0.0f;
    for (int j = 0; j < k; j++) {
        uint32_t best = key[0];
#pragma unroll
        for (int r = 1; r < ROUTE_R; r++) best = max(best, key[r]);
        best = max(best, (uint32_t)xl32<0>((int)best));
        best = max(best, (uint32_t)xl32<1>((int)best));
        best = max(best, (uint32_t)xl32<2>((int)best));
        best = max(best, (uint32_t)xl32<3>((int)best));
        best = max(best, (uint32_t)xl32<4>((int)best));
        best = max((uint32_t)__builtin_amdgcn_readlane((int)best, 0), (uint32_t)__builtin_amdgcn_readlane((int)best, 32));
        int bi = 0;
#pragma unroll
        for (int r = 0; r < ROUTE_R; r++) {
            const uint64_t m = __ballot(key[r] == best);
            if (m) {
                bi = 64 * r + (int)__builtin_ctzll(m);
                break;
            }
        }
#pragma unroll
        for (int r = 0; r < ROUTE_R; r++)
            if (bi == 64 * r + lane) key[r] = 0u;
        if (lane == j) { my_id = bi; my_p = __uint_as_float(best - 1u); }
    }
    // Weights: p / max(sum of the top k in rank order, 2^-14) (times extra_scale when not 0).
    float sum = 0.0f;
    for (int j = 0; j < k; j++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_p), j));
    float scale = 1.0f / fmaxf(sum, 6.103515625e-5f);
    if (extra_scale != 0.0f) scale *= extra_scale;
    int slot = -1;  // table[my_id]: entry my_id >> 6 of lane my_id & 63
#pragma unroll
    for (int r = 0; r < ROUTE_R; r++) {
        const int c = __shfl(tv[r], my_id & 63);
        if ((my_id >> 6) == r) slot = c;
    }
    id_out = my_id;
    w_out = my_p * scale;
    slot_out = slot;
}


// The same routing of one token (n <= 128) by the four waves of a 256-thread block, all of which call it. The ranking
// value of an expert is e = exp(v - max) (softmax) or p = sigmoid(v), ordered with ties to the lower index as 64-bit
// keys (bits(e) + 1) << 32 | ~index. Wave 0 adds the softmax sum s in index order while waves 1-3 count, for each
// expert, the keys above its own (44, 44 and 40 of the experts); the k + 1 highest then give p = e / s in rank order.
// Dividing by s keeps the order, except that two different e may round to one p, whose tie the reference breaks by
// index: where that happens among them (or at the k-th place) wave 0 routes the token again with route_wave. Thread
// j < k gets rank j's id, w and slot. L: RouteLds in LDS.
struct RouteLds {
    uint64_t key[128];
    float e[128];
    int rank[3][128];
    float topv[33];
    int topi[33];
    int tops[33];
    float s;
};
__device__ __forceinline__ void route_block4(const float* __restrict__ pr, int n, int k, float extra_scale,
                                             const int* __restrict__ table, int sigmoid, RouteLds* L, int& id_out,
                                             float& w_out, int& slot_out) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    float v[2];
    int tv[2];  // the slot table's entries, fetched with the logits
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int i = lane + 64 * r;
        v[r] = i < n ? pr[i] : -INFINITY;
        tv[r] = table && i < n ? table[i] : -1;
    }
    if (sigmoid) {
#pragma unroll
        for (int r = 0; r < 2; r++) v[r] = 1.0f / (1.0f + exp_f32(-v[r]));  // ops::sigmoid
    } else {
        float m = fmaxf(v[0], v[1]);
        m = fmaxf(m, xl32f<0>(m));
        m = fmaxf(m, xl32f<1>(m));
        m = fmaxf(m, xl32f<2>(m));
        m = fmaxf(m, xl32f<3>(m));
        m = fmaxf(m, xl32f<4>(m));
        m = fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0)),
                  __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32)));
#pragma unroll
        for (int r = 0; r < 2; r++) if (lane + 64 * r < n) v[r] = exp_f32(v[r] - m);
    }
    uint64_t key[2];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int i = lane + 64 * r;
        key[r] = i < n ? ((uint64_t)(__float_as_uint(v[r]) + 1u) << 32) | (uint32_t)~(uint32_t)i : 0ull;
        if (wave == 0) {
            L->key[i] = key[r];
            L->e[i] = i < n ? v[r] : 0.0f;  // entries past n add +0: the sum keeps its bits
        }
    }
    __syncthreads();
    if (wave == 0) {
        if (!sigmoid && lane == 0) {
            // ops::softmax's sum in index order, 4 values a read
            float s = 0.0f;
#pragma unroll
            for (int c = 0; c < 128; c += 64) {
                float4 q[16];
#pragma unroll
                for (int u = 0; u < 16; u++) q[u] = *(const float4*)&L->e[c + 4 * u];
#pragma unroll
                for (int u = 0; u < 16; u++) {
                    s += q[u].x;
                    s += q[u].y;
                    s += q[u].z;
                    s += q[u].w;
                }
            }
            L->s = s;
        }
    } else {
        // keys above each of this lane's two, among experts [44 (wave - 1), 44 wave) (to 128), 4 read at a time
        // ahead of their comparisons (absent entries past n hold key 0: above nothing)
        const uint64_t* kp = L->key + 44 * (wave - 1);
        const int cnt = wave == 3 ? 40 : 44;
        int c0 = 0, c1 = 0;
#pragma unroll
        for (int j = 0; j < 44; j += 4) {
            if (j < cnt) {
                const uint64_t k0 = kp[j], k1 = kp[j + 1], k2 = kp[j + 2], k3 = kp[j + 3];
                c0 += (k0 > key[0]) + (k1 > key[0]) + (k2 > key[0]) + (k3 > key[0]);
                c1 += (k0 > key[1]) + (k1 > key[1]) + (k2 > key[1]) + (k3 > key[1]);
            }
        }
        L->rank[wave - 1][lane] = c0;
        L->rank[wave - 1][lane + 64] = c1;
    }
    __syncthreads();
    if (wave == 0) {
        // the k + 1 highest keys into rank order
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int i = lane + 64 * r;
            const int rk = L->rank[0][i] + L->rank[1][i] + L->rank[2][i];
            if (i < n && rk <= k) {
                L->topv[rk] = v[r];
                L->topi[rk] = i;
                L->tops[rk] = tv[r];
            }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        const float s = L->s;
        float p = 0.0f, pn = 0.0f, e = 0.0f, en = 0.0f;
        int id = 0, sl = -1;
        if (lane < k) {
            e = L->topv[lane];
            id = L->topi[lane];
            sl = L->tops[lane];
            p = sigmoid ? e : e / s;
            if (lane + 1 < n) {
                en = L->topv[lane + 1];
                pn = sigmoid ? en : en / s;
            }
        }
        // a tie made by the division between ranks lane and lane + 1 (the k-th included)
        const bool bad = lane < k && lane + 1 < n && !sigmoid && p == pn && e != en;
        if (!__ballot(bad)) {
            // weights: p / max(sum of the top k in rank order, 2^-14) (times extra_scale when not 0)
            float sum = 0.0f;
            for (int j = 0; j < k; j++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), j));
            float scale = 1.0f / fmaxf(sum, 6.103515625e-5f);
            if (extra_scale != 0.0f) scale *= extra_scale;
            if (lane < k) {
                L->topv[lane] = p * scale;
                L->topi[lane] = id;
                L->tops[lane] = sl;
            }
        } else {
            int fid, fslot;
            float fw;
            route_wave<2>(pr, n, k, extra_scale, table, sigmoid, L->e, fid, fw, fslot);
            if (lane < k) {
                L->topv[lane] = fw;
                L->topi[lane] = fid;
                L->tops[lane] = fslot;
            }
        }
    }
    __syncthreads();
    if (tid < k) {
        id_out = L->topi[tid];
        w_out = L->topv[tid];
        slot_out = L->tops[tid];
    }
}

}  // namespace strata

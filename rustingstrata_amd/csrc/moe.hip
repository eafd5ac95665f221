// MoE routing, the stable sort of (token, expert) pairs with its tile lists, and the combines.
#include "moe.h"
#include "route.h"
#include "xlane.h"

namespace strata {

// ---- routing (Model::route src/model.rs:837-851; topk_warp src/cuda/kernels.cu:2633-2686) ----
// One wave64 per token, ROUTE_R logits per lane (n <= 64 ROUTE_R): an instantiation per 1, 2, 4, 8.
template <int ROUTE_R>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ p, int n, int k, float extra_scale,
                                                    const int* __restrict__ table, int* ids, float* wts, int* slots,
                                                    float* wh, int T, int sigmoid) {
    __shared__ float se[4][64 * ROUTE_R];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + wave;
    if (t >= T) return;  // whole waves only
    int id, slot;
    float w;
    route_wave<ROUTE_R>(p + (uint64_t)t * n, n, k, extra_scale, table, sigmoid, se[wave], id, w, slot);
    if (lane < k) {
        const int o = t * k + lane;
        ids[o] = id;
        wts[o] = w;
        if (table) {
            slots[o] = slot;
            wh[o] = slot >= 0 ? w : 0.0f;
        }
    }
}

// A 256-thread block per token (n <= 128: few tokens, where the route's latency is the cost).
__global__ __launch_bounds__(256) void route_block_kernel(const float* __restrict__ p, int n, int k, float extra_scale,
                                                          const int* __restrict__ table, int* ids, float* wts,
                                                          int* slots, float* wh, int sigmoid) {
    __shared__ RouteLds L;
    const int t = blockIdx.x;
    int id, slot;
    float w;
    route_block4(p + (uint64_t)t * n, n, k, extra_scale, table, sigmoid, &L, id, w, slot);
    if (threadIdx.x < k) {
        const int o = t * k + threadIdx.x;
        ids[o] = id;
        wts[o] = w;
        if (table) {
            slots[o] = slot;
            wh[o] = slot >= 0 ? w : 0.0f;
        }
    }
}

constexpr int ROUTE_BLOCK_MAX_T = 16;  // tokens up to which each gets a block of its own
hipError_t launch_route(const float* p, int n, int k, float extra_scale, const int* table, int* ids, float* wts,
                        int* slots, float* wh, int t, int sigmoid, hipStream_t s) {
    const dim3 grid((unsigned)((t + 3) / 4)), block(256);
    if (n <= 128 && k <= 32 && t <= ROUTE_BLOCK_MAX_T) {
        route_block_kernel<<<dim3((unsigned)t), block, 0, s>>>(p, n, k, extra_scale, table, ids, wts, slots, wh, sigmoid);
        return hipGetLastError();
    }
    if (n <= 64) route_kernel<1><<<grid, block, 0, s>>>(p, n, k, extra_scale, table, ids, wts, slots, wh, t, sigmoid);
    else if (n <= 128) route_kernel<2><<<grid, block, 0, s>>>(p, n, k, extra_scale, table, ids, wts, slots, wh, t, sigmoid);
    else if (n <= 256) route_kernel<4><<<grid, block, 0, s>>>(p, n, k, extra_scale, table, ids, wts, slots, wh, t, sigmoid);
    else route_kernel<8><<<grid, block, 0, s>>>(p, n, k, extra_scale, table, ids, wts, slots, wh, t, sigmoid);
    return hipGetLastError();
}

// ---- combines ----

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + exp_f32(-x)); }

// moe_combine (mb = 0; src/cuda/kernels.cu:2742-2773): grid (ceil(n / 256), t).
__global__ __launch_bounds__(256) void combine_kernel(float* x, const float* ye, const float* w, int k, const float* sh,
                                                      const float* sg, int n) {
    int tk = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    x += (uint64_t)tk * n; ye += (uint64_t)tk * k * n; w += (uint64_t)tk * k;
    // 8 slots' loads at a time, then their products in slot order (a slot with weight 0 may hold anything; its
    // product is not added)
    float y = 0.0f;
    for (int j0 = 0; j0 < k; j0 += 8) {
        float wv[8], yv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u < k ? j0 + u : k - 1;
            wv[u] = j0 + u < k ? w[j] : 0.0f;
            yv[u] = ye[(uint64_t)j * n + i];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) if (wv[u] != 0.0f) y += wv[u] * yv[u];
    }
    if (sh) y += (sg ? sigmoid_f32(sg[tk]) : 1.0f) * sh[(uint64_t)tk * n + i];
    x[i] += y;
}

hipError_t launch_combine(float* x, const float* ye, const float* w, int k, const float* sh, const float* sg, int n,
                          int t, hipStream_t s) {
    combine_kernel<<<dim3((unsigned)((n + 255) / 256), (unsigned)t), dim3(256), 0, s>>>(x, ye, w, k, sh, sg, n);
    return hipGetLastError();
}

// moe_combine_seq (src/cuda/kernels.cu:2776-2785): x[t] += sum_j wts[t, j] ye[inv[t, j]] (j in order), + the shared
// expert. A pair the sort rejected (inv < 0) adds nothing.
__global__ __launch_bounds__(256) void combine_seq_kernel(float* x, const float* ye, const float* wts, const int* inv,
                                                          int k, const float* sh, const float* sg, int n) {
    int t = blockIdx.y, d = blockIdx.x * 256 + threadIdx.x;
    if (d >= n) return;
    // 8 pairs' loads at a time (their slots, then their ye rows), then the products in pair order
    float y = 0.0f;
    for (int j0 = 0; j0 < k; j0 += 8) {
        int sv[8];
        float wv[8], yv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u < k ? j0 + u : k - 1;
            sv[u] = j0 + u < k ? inv[t * k + j] : -1;
            wv[u] = wts[t * k + j];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) yv[u] = ye[(uint64_t)(sv[u] >= 0 ? sv[u] : 0) * n + d];
#pragma unroll
        for (int u = 0; u < 8; u++) if (sv[u] >= 0) y += wv[u] * yv[u];
    }
    uint64_t i = (uint64_t)t * n + d;
    if (sh) y += (sg ? sigmoid_f32(sg[t]) : 1.0f) * sh[i];
    x[i] += y;
}

// The same, 4 consecutive outputs a thread (n % 4 == 0, x, ye and sh 16-byte aligned): the token's slots and weights
// come through scalar loads, each output's sum keeps the pair order above.
__global__ __launch_bounds__(256) void combine_seq4_kernel(float* x, const float* ye, const float* wts, const int* inv,
                                                           int k, const float* sh, const float* sg, int n) {
    const int t = blockIdx.y, d = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (d >= n) return;
    float4 y = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j0 = 0; j0 < k; j0 += 8) {
        int sv[8];
        float wv[8];
        float4 yv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u < k ? j0 + u : k - 1;
            sv[u] = j0 + u < k ? sload(inv + t * k + j) : -1;
            wv[u] = sload(wts + t * k + j);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) yv[u] = *(const float4*)(ye + (uint64_t)(sv[u] >= 0 ? sv[u] : 0) * n + d);
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (sv[u] >= 0) {
                y.x += wv[u] * yv[u].x; y.y += wv[u] * yv[u].y;
                y.z += wv[u] * yv[u].z; y.w += wv[u] * yv[u].w;
            }
        }
    }
    const uint64_t i = (uint64_t)t * n + d;
    if (sh) {
        const float gs = sg ? sigmoid_f32(sg[t]) : 1.0f;
        const float4 s4 = *(const float4*)(sh + i);
        y.x += gs * s4.x; y.y += gs * s4.y; y.z += gs * s4.z; y.w += gs * s4.w;
    }
    float4 o = *(const float4*)(x + i);
    o.x += y.x; o.y += y.y; o.z += y.z; o.w += y.w;
    *(float4*)(x + i) = o;
}

hipError_t launch_combine_seq(float* x, const float* ye, const float* wts, const int* inv, int k, const float* sh,
                              const float* sg, int n, int t, hipStream_t s) {
    const bool v4 = n % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)ye % 16 == 0 && (uintptr_t)sh % 16 == 0;
    if (v4)
        combine_seq4_kernel<<<dim3((unsigned)((n / 4 + 255) / 256), (unsigned)t), dim3(256), 0, s>>>(x, ye, wts, inv, k, sh, sg, n);
    else
        combine_seq_kernel<<<dim3((unsigned)((n + 255) / 256), (unsigned)t), dim3(256), 0, s>>>(x, ye, wts, inv, k, sh, sg, n);
    return hipGetLastError();
}

// ---- stable sort of the (token, j) pairs by expert, and the tile lists ----
// The host counting sort of src/gpu_model/prefill.rs:563-573, exactly, in three launches over W waves, wave gw owning
// the contiguous pair segment [gw S, (gw + 1) S):
//   count:   each wave counts its segment's experts into cnt[e * W + gw] (expert-major) and its bad ids into bad[gw];
//   scan:    one block turns each expert's row of cnt into exclusive prefixes over the waves (a wave of the block
//            per expert, coalesced) and the experts' totals into off (experts ascending); writes the tile lists, the
//            tile count and the bad-id count;
//   scatter: each wave starts expert e at off[e] + its prefix (waves in order within an expert) and walks its
//            segment in order, 64 pairs at a time, assigning slots with the rank among equal experts inside the 64
//            (ballot match on the key bits).
constexpr int SORT_WAVES = 16, SORT_MAX_E = 512, SORT_U = 4, SORT_SEG = 64 * SORT_U;

static int sort_waves(int n_pairs) { return n_pairs > 0 ? (n_pairs + SORT_SEG - 1) / SORT_SEG : 1; }
size_t sort_scratch_bytes(int n_expert, int n_pairs) {
    const int W = sort_waves(n_pairs);
    return ((size_t)n_expert * W + W) * sizeof(int);
}

// The ids of a wave's segment, SORT_U rounds of 64 (their loads in flight together); -1 past the segment.
__device__ __forceinline__ void sort_ids(const int* ids, int s0, int s1, int lane, int (&eu)[SORT_U]) {
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
        const int i = s0 + 64 * u + lane;
        eu[u] = i < s1 ? ids[i] : -1;
    }
}

__global__ __launch_bounds__(1024) void sort_count_kernel(SortLaunch a, int W) {
    __shared__ int hist[SORT_WAVES][SORT_MAX_E];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, E = a.n_expert;
    const int gw = blockIdx.x * SORT_WAVES + wave, N = a.t * a.k;
    for (int e = lane; e < E; e += 64) hist[wave][e] = 0;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    if (gw >= W) return;
    const int s0 = min(N, gw * SORT_SEG), s1 = min(N, s0 + SORT_SEG);
    int eu[SORT_U];
    sort_ids(a.ids, s0, s1, lane, eu);
    int bad = 0;
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
        if (s0 + 64 * u + lane < s1) {
            const int e = eu[u];
            if (e >= 0 && e < E) atomicAdd(&hist[wave][e], 1);
            else bad++;
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    for (int e = lane; e < E; e += 64) a.scratch[(uint64_t)e * W + gw] = hist[wave][e];
    bad += __shfl_xor(bad, 1);
    bad += __shfl_xor(bad, 2);
    bad += __shfl_xor(bad, 4);
    bad += __shfl_xor(bad, 8);
    bad += __shfl_xor(bad, 16);
    bad += __shfl_xor(bad, 32);
    if (lane == 0) a.scratch[(uint64_t)E * W + gw] = bad;
}

__global__ __launch_bounds__(1024) void sort_scan_kernel(SortLaunch a, int W) {
    __shared__ int part[16];
    __shared__ int offs[SORT_MAX_E + 1], tbase[SORT_MAX_E + 1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, E = a.n_expert;
    int* cnt = a.scratch;
    const uint64_t L = (uint64_t)E * W;
    // expert e's row of wave counts (coalesced, 64 waves at a time) into exclusive prefixes within the expert; the
    // expert's total into offs[e]. This wave's (expert, 64-count chunk) pairs p = ei nch + ch (expert wave + 16 ei)
    // go 8 at a time: the 8 loads together, then their scans in order (one round trip per 8 chunks, not per chunk).
    {
        const int nch = (W + 63) / 64, nE = wave < E ? (E - wave + 15) / 16 : 0, P = nE * nch;
        int carry = 0;
        for (int p0 = 0; p0 < P; p0 += 8) {
            int c[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int p = p0 + u, ei = p / nch, ch = p - ei * nch, w = 64 * ch + lane;
                c[u] = p < P && w < W ? cnt[(uint64_t)(wave + 16 * ei) * W + w] : 0;
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int p = p0 + u;
                if (p < P) {
                    const int ei = p / nch, ch = p - ei * nch, e = wave + 16 * ei, w = 64 * ch + lane;
                    if (ch == 0) carry = 0;
                    const int inc = wave_incl_scan(c[u]);
                    if (w < W) cnt[(uint64_t)e * W + w] = carry + inc - c[u];
                    carry += __builtin_amdgcn_readlane(inc, 63);
                    if (ch == nch - 1 && lane == 0) offs[e] = carry;
                }
            }
        }
    }
    // the bad-id count: each thread sums waves tid, tid + 1024, ..., then the block in order
    int bad = 0;
    if (a.err)
        for (int w = tid; w < W; w += 1024) bad += cnt[L + w];
    __syncthreads();
    if (wave == 0) {  // exclusive scan of the expert totals, in expert order
        int run = 0;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + lane;
            const int c = e < E ? offs[e] : 0;
            const int ic = wave_incl_scan(c);
            if (e < E) offs[e] = run + ic - c;
            run += __builtin_amdgcn_readlane(ic, 63);
        }
        if (lane == 0) offs[E] = run;
    }
    __syncthreads();
    if (tid < E) tbase[tid] = (offs[tid + 1] - offs[tid] + a.chunk - 1) / a.chunk;
    __syncthreads();
    if (wave == 0) {  // exclusive scan of the tile counts over experts, in order
        int trun = 0;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + lane;
            const int tc = e < E ? tbase[e] : 0;
            const int itc = wave_incl_scan(tc);
            if (e < E) tbase[e] = trun + itc - tc;
            trun += __builtin_amdgcn_readlane(itc, 63);
        }
        if (lane == 0) tbase[E] = trun;
    }
    __syncthreads();
    if (tid <= E) a.off[tid] = offs[tid];
    // Tiles: expert e's slots off[e] .. off[e + 1] in chunks of a.chunk positions.
    if (tid < E) {
        const int c = offs[tid + 1] - offs[tid], tb = tbase[tid];
        for (int j = 0; j * a.chunk < c; j++) {
            const uint64_t m0 = (uint64_t)(offs[tid] + j * a.chunk), cn = (uint64_t)min(a.chunk, c - j * a.chunk);
            for (int m = 0; m < a.n_mats; m++) {
                uint64_t* tl = a.tiles + 2 * ((uint64_t)m * a.max_tiles + tb + j);
                tl[0] = a.bases[m] + (uint64_t)tid * a.strides[m];
                tl[1] = m0 | cn << 32;
            }
        }
    }
    if (a.err) {
        bad = __builtin_amdgcn_readlane(wave_incl_scan(bad), 63);
        if (lane == 0) part[wave] = bad;
    }
    __syncthreads();
    if (tid == 0) {
        *a.n_tiles = tbase[E];
        if (a.err) {
            int b = 0;
            for (int w = 0; w < 16; w++) b += part[w];
            *a.err = b;
        }
    }
}

__global__ __launch_bounds__(1024) void sort_scatter_kernel(SortLaunch a, int W) {
    __shared__ int hist[SORT_WAVES][SORT_MAX_E];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, E = a.n_expert;
    const int gw = blockIdx.x * SORT_WAVES + wave, N = a.t * a.k;
    if (gw >= W) return;
    const int s0 = min(N, gw * SORT_SEG), s1 = min(N, s0 + SORT_SEG);
    int eu[SORT_U];
    sort_ids(a.ids, s0, s1, lane, eu);
    for (int e = lane; e < E; e += 64) hist[wave][e] = a.off[e] + a.scratch[(uint64_t)e * W + gw];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
        const int c0 = s0 + 64 * u;
        if (c0 >= s1) break;
        const int i = c0 + lane;
        const bool live = i < s1;
        const int e = eu[u];
        const bool ok = live && e >= 0 && e < E;
        const int key = ok ? e : (live ? 2046 : 2047);
        uint64_t peers = ~0ull;
#pragma unroll
        for (int b = 0; b < 11; b++) {
            const uint64_t m = __ballot((key >> b) & 1);
            peers &= ((key >> b) & 1) ? m : ~m;
        }
        const int rank = __popcll(peers & ((1ull << lane) - 1));
        const int slot = ok ? hist[wave][e] + rank : -1;
        __builtin_amdgcn_wave_barrier();
        if (ok && rank == 0) hist[wave][e] += __popcll(peers);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        if (live) {
            a.inv[i] = slot;
            if (ok) a.xrow[slot] = i / a.k;
        }
    }
}

hipError_t launch_sort(const SortLaunch& a, hipStream_t s) {
    const int W = sort_waves(a.t * a.k), blocks = (W + SORT_WAVES - 1) / SORT_WAVES;
    sort_count_kernel<<<blocks, 1024, 0, s>>>(a, W);
    sort_scan_kernel<<<1, 1024, 0, s>>>(a, W);
    sort_scatter_kernel<<<blocks, 1024, 0, s>>>(a, W);
    return hipGetLastError();
}

}  // namespace strata

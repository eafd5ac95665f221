// MoE glue kernels: routing, stable sort by expert with tile lists, SwiGLU + quantization, combines.
#pragma once
#include "common.h"

namespace strata {

// router_topk (table == null) or moe_route (slots = table[ids], wh = hit weights).
hipError_t launch_route(const float* p, int n, int k, float extra_scale, const int* table, int* ids, float* wts,
                        int* slots, float* wh, int t, int sigmoid, hipStream_t s);
hipError_t launch_swiglu_q(const float* g, const float* u, int n, int rows, int8_t* xq, int mode, hipStream_t s);
hipError_t launch_combine(float* x, const float* ye, const float* w, int k, const float* sh, const float* sg, int n,
                          int t, hipStream_t s);
hipError_t launch_combine_seq(float* x, const float* ye, const float* wts, const int* inv, int k, const float* sh,
                              const float* sg, int n, int t, hipStream_t s);

struct SortLaunch {
    const int* ids = nullptr;
    int t = 0, k = 0, n_expert = 0;
    int* off = nullptr;     // n_expert + 1
    int* xrow = nullptr;    // t * k
    int* inv = nullptr;     // t * k
    int n_mats = 0;
    uint64_t bases[3] = {0, 0, 0}, strides[3] = {0, 0, 0};
    uint64_t* tiles = nullptr;  // n_mats lists of max_tiles 16-byte tiles
    int max_tiles = 0;
    int chunk = 128;            // positions per tile
    int* n_tiles = nullptr;
    int* err = nullptr;
    int* scratch = nullptr;     // sort_scratch_bytes(n_expert, t * k) bytes
};
size_t sort_scratch_bytes(int n_expert, int n_pairs);
hipError_t launch_sort(const SortLaunch& a, hipStream_t s);

}  // namespace strata

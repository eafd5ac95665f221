// Dequantization (the Backend::dequant test op) and activation quantization (Backend::quant_xq).
#include "formats.h"
#include "kernels.h"
#include "xlane.h"
#include "moe.h"
#include "../../include/strata_hip.h"

namespace strata {

// One thread per 32 values: thread i of the grid writes values 32 i .. of row i / (cols / 32).
template <int T>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w, uint64_t rb, int cols,
                                                      uint64_t groups, float* __restrict__ out) {
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= groups) return;
    int gpr = cols / 32;
    uint64_t r = i / gpr;
    int g = (int)(i % gpr);
    const uint8_t* sb = w + r * rb + (uint64_t)(g / 8) * sb_bytes(T);
    float v[32];
    dequant32<T>(sb, g % 8, v);
    float4* o = (float4*)(out + r * cols + 32 * g);
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
}

template <int T>
static hipError_t dequant_t(const uint8_t* w, uint64_t rows, uint64_t cols, float* out, hipStream_t s) {
    uint64_t groups = rows * (cols / 32);
    if (!groups) return hipSuccess;
    dequant_kernel<T><<<dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, s>>>(w, row_bytes(T, cols), (int)cols, groups, out);
    return hipGetLastError();
}

hipError_t launch_dequant(int ty, const uint8_t* w, uint64_t rows, uint64_t cols, float* out, hipStream_t s) {
    switch (ty) {
    case Q8_0: return dequant_t<Q8_0>(w, rows, cols, out, s);
    case Q2_K: return dequant_t<Q2_K>(w, rows, cols, out, s);
    case Q3_K: return dequant_t<Q3_K>(w, rows, cols, out, s);
    case Q4_K: return dequant_t<Q4_K>(w, rows, cols, out, s);
    case Q5_K: return dequant_t<Q5_K>(w, rows, cols, out, s);
    case Q6_K: return dequant_t<Q6_K>(w, rows, cols, out, s);
    case IQ2_XXS: return dequant_t<IQ2_XXS>(w, rows, cols, out, s);
    case IQ3_S: return dequant_t<IQ3_S>(w, rows, cols, out, s);
    case IQ4_XS: return dequant_t<IQ4_XS>(w, rows, cols, out, s);
    }
    return hipErrorInvalidValue;
}

// quant_xq. A group of 32 lanes covers 256 values, 8 per lane (the Q8_K block); a block of 256 threads covers 2048
// values of one row (grid = (ceil(n / 2048), nt)). Lanes past n hold zeros, which is quantize_q8k's zero padding.
//  Q8K: the block's scale is -127 / (the signed value of largest magnitude, the first such), q = min(127,
//       round-half-even(is * v)), d = 1 / is for each of its 32-groups (src/cpu_moe.rs:28-46).
//  Q8_32: per 32 values (4 lanes) d = max|v| / 127, q = round-half-even(v * 127 / max|v|) (src/cuda/kernels.cu:640-660).
// SWIGLU: the values are silu(g) * u (swiglu_q, src/cuda/kernels.cu:1826-1839), with g at x and u at u.
__device__ __forceinline__ float silu_f32(float v) { return v / (1.0f + (float)exp(-(double)v)); }

template <bool SWIGLU>
__global__ __launch_bounds__(256) void quant_xq_kernel(const float* __restrict__ x, const float* __restrict__ u,
                                                       uint64_t x_stride, int n, int nt, int8_t* __restrict__ out, int mode) {
    int t = blockIdx.y;
    int i = blockIdx.x * 2048 + threadIdx.x * 8;
    const float* xr = x + (uint64_t)t * x_stride;
    float v[8];
    bool live = i < n;
    if (live) {
        float4 a = *(const float4*)(xr + i), b = *(const float4*)(xr + i + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        if constexpr (SWIGLU) {
            const float* ur = u + (uint64_t)t * x_stride;
            float4 c = *(const float4*)(ur + i), e = *(const float4*)(ur + i + 4);
            float uu[8] = {c.x, c.y, c.z, c.w, e.x, e.y, e.z, e.w};
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = silu_f32(v[j]) * uu[j];
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = 0.0f;
    }
    float d, mul;
    if (mode == STRATA_NUM_Q8K) {
        // Candidate: the first value of largest magnitude among this lane's 8, then across the 32 lanes (lowest index).
        float bv = v[0];
        int bi = i;
#pragma unroll
        for (int j = 1; j < 8; j++) if (fabsf(v[j]) > fabsf(bv)) { bv = v[j]; bi = i + j; }
            // the first value of largest magnitude over the 32 lanes: the choice is unique, so the pairing of the
            // exchange steps does not matter
            auto step = [&](auto S) __attribute__((always_inline)) {
                constexpr int st = decltype(S)::value;
                const float ov = xl32f<st>(bv);
                const int oi = xl32<st>(bi);
                if (fabsf(ov) > fabsf(bv) || (fabsf(ov) == fabsf(bv) && oi < bi)) { bv = ov; bi = oi; }
            };
            step(std::integral_constant<int, 0>{});
            step(std::integral_constant<int, 1>{});
            step(std::integral_constant<int, 2>{});
            step(std::integral_constant<int, 3>{});
            step(std::integral_constant<int, 4>{});
        float is = bv != 0.0f ? -127.0f / bv : 0.0f;
        d = bv != 0.0f ? 1.0f / is : 0.0f;
        mul = is;
    } else {
        float mx = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) mx = fmaxf(mx, fabsf(v[j]));
        mx = fmaxf(mx, xl32f<0>(mx));
        mx = fmaxf(mx, xl32f<1>(mx));
        d = mx / 127.0f;
        mul = mx > 0.0f ? 127.0f / mx : 0.0f;
    }
    if (!live) return;
    uint32_t w[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float r = __builtin_rintf(mul * v[j]);
        int q = (int)fminf(r, 127.0f);
        w[j >> 2] |= (uint32_t)(q & 255) << (8 * (j & 3));
    }
    *(uint2*)(out + (uint64_t)t * n + i) = make_uint2(w[0], w[1]);
    if ((threadIdx.x & 3) == 0) ((float*)(out + (uint64_t)nt * n))[(uint64_t)t * (n / 32) + i / 32] = d;
}

hipError_t launch_quant_xq(const float* x, uint64_t x_stride, int n, int nt, int8_t* out, int mode, hipStream_t s) {
    if (!n || !nt) return hipSuccess;
    quant_xq_kernel<false><<<dim3((unsigned)((n + 2047) / 2048), (unsigned)nt), dim3(256), 0, s>>>(x, nullptr, x_stride, n, nt, out, mode);
    return hipGetLastError();
}

hipError_t launch_swiglu_q(const float* g, const float* u, int n, int rows, int8_t* xq, int mode, hipStream_t s) {
    if (!n || !rows) return hipSuccess;
    quant_xq_kernel<true><<<dim3((unsigned)((n + 2047) / 2048), (unsigned)rows), dim3(256), 0, s>>>(g, u, n, n, rows, xq, mode);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) dst[i] = src[i];
}

hipError_t launch_copy(const void* src, void* dst, uint64_t bytes, hipStream_t s) {
    uint64_t n = bytes / 16;
    if (!n) return hipSuccess;
    uint64_t blocks = (n + 255) / 256;
    copy_kernel<<<dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256), 0, s>>>((const uint4*)src, (uint4*)dst, n);
    return hipGetLastError();
}

}  // namespace strata

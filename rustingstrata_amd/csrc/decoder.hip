// The decoder stack around the quantized matmuls: per-head RMS norm with NEOX rope and the f16 KV-cache store
// (Backend::rms_norm_rope_kv / rms_norm_rope_qk / rope_pairs / kv_store, src/backend.rs:250-277,380), argmax over
// logit rows (Backend::argmax_rows, :246), x += y and SwiGLU (:282-284), float-weight matmuls (the router's F32
// weights through gemv / gemm_dense), embedding rows (Model::embed, src/model.rs:334-339, on the device) and seeded
// synthetic GGUF blocks.
#include <cmath>

#include "decoder.h"
#include "formats.h"
#include "xlane.h"

namespace strata {

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    _Float16 h = (_Float16)v;  // round to nearest even, as __float2half_rn
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}


// ---- rms_norm + rope (+ KV store) ----
// One wave per head, n <= 512, the head staged in LDS. The sum of squares runs in index order on one lane (n adds per
// head, a small part of the launch), and out = x * (1 / sqrt(ss / n + eps)) * w in the reference's operation order,
// so the normed head has the CPU's bits (src/ops.rs:3-7; kernel
// src/cuda/kernels.cu:2196-2227). The rope turns pair (i, i + n_rot / 2) by theta = pos * base^(-2 i / n_rot), theta
// in f64 and its sine and cosine rounded to f32 as ops::rope_neox does (src/ops.rs:36-45).
constexpr int NR_WAVES = 4;

// Head gb (query heads first, then key heads) of a launch: its source row, norm weights, output row and whether it
// stores to the KV cache.
struct NrHead {
    const float* xr;
    const float* w;
    float* o;
    const float* vr;  // value row (key heads of a storing launch), else null
    int b, per;
};
__device__ __forceinline__ NrHead nr_head(const NormRope& a, int gb) {
    NrHead h;
    if (gb < a.qrows) {
        h.b = gb; h.per = a.qper;
        h.xr = a.qx + (uint64_t)(gb / a.qper) * a.q_tstride + (uint64_t)(gb % a.qper) * a.q_stride;
        h.w = a.qw; h.o = a.qo + (uint64_t)gb * a.n; h.vr = nullptr;
    } else {
        const int b = gb - a.qrows, tk = b / a.per, hh = b - tk * a.per;
        h.b = b; h.per = a.per;
        h.xr = a.x + (uint64_t)tk * a.x_tstride + (uint64_t)hh * a.x_stride; h.w = a.w; h.o = a.out + (uint64_t)b * a.n;
        h.vr = a.kc ? a.v + (uint64_t)tk * a.v_tstride + (uint64_t)hh * a.n : nullptr;
    }
    return h;
}

// One head by one wave: out = x * (1 / sqrt(ss / n + eps)) * w, rope, and (key heads of a storing launch) the f16
// KV store. s: the wave's 512-float LDS stage. HAVE_SS: ss is given (else lane 0 sums the head from the stage).
template <bool HAVE_SS>
__device__ __forceinline__ void nr_run(const NormRope& a, const NrHead& h, float* s, int lane, float ss) {
    const int n = a.n, half = a.n_rot / 2;
    const bool store = h.vr != nullptr;
    // every load of the wave first (the head, its norm weights, the value row), then the rope angles while they land
    constexpr int NV = 512 / 64;
    float xv[NV], wv[NV], vv[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = lane + 64 * j;
        if (i < n) {
            xv[j] = h.xr[i];
            wv[j] = h.w[i];
            if (store) vv[j] = h.vr[i];
        }
    }
    const int pos = a.step[0] + h.b / h.per;
    float sn[NV / 2], cs[NV / 2];
#pragma unroll
    for (int j = 0; j < NV / 2; j++) {
        const int i = lane + 64 * j;
        if (i < half) {
            const double f = i < a.nfreq ? a.freq[i] : pow((double)a.base, -2.0 * (double)i / (double)a.n_rot);
            double sd, cd;
            sincos((double)pos * f, &sd, &cd);
            sn[j] = (float)sd;
            cs[j] = (float)cd;
        }
    }
    if constexpr (!HAVE_SS) {
#pragma unroll
        for (int j = 0; j < NV; j++)
            if (lane + 64 * j < n) s[lane + 64 * j] = xv[j];
        __builtin_amdgcn_wave_barrier();
        if (lane == 0)
            ss = nr_sumsq(n, [&](int i0, float4 (&r)[8]) {
#pragma unroll
                for (int c = 0; c < 8; c++) r[c] = *(const float4*)&s[i0 + 4 * c];
            });
        ss = __shfl(ss, 0, 64);
        __builtin_amdgcn_wave_barrier();  // lane 0's reads are done before the normed values overwrite the stage
    }
    const float sc = 1.0f / sqrtf(ss / (float)n + a.eps);
#pragma unroll
    for (int j = 0; j < NV; j++)
        if (lane + 64 * j < n) s[lane + 64 * j] = xv[j] * sc * wv[j];
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < NV / 2; j++) {
        const int i = lane + 64 * j;
        if (i < half) {
            const float p = s[i], q = s[i + half];
            s[i] = p * cs[j] - q * sn[j];
            s[i + half] = p * sn[j] + q * cs[j];
        }
    }
    __builtin_amdgcn_wave_barrier();
    const uint64_t e = ((uint64_t)pos * h.per + h.b % h.per) * n;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = lane + 64 * j;
        if (i < n) {
            const float r = s[i];
            h.o[i] = r;
            if (store) {
                a.kc[e + i] = f32_to_f16_bits(r);
                a.vc[e + i] = f32_to_f16_bits(vv[j]);
            }
        }
    }
    __builtin_amdgcn_wave_barrier();  // the stage is reused by the wave's next head
}

// A wave per head (decode: few heads, each wave's latency is the launch's).
__global__ __launch_bounds__(64 * NR_WAVES) void norm_rope_kernel(NormRope a) {
    __shared__ __align__(16) float sh[NR_WAVES][512];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int gb = (int)blockIdx.x * NR_WAVES + wave;
    if (gb >= a.qrows + a.rows) return;
    nr_run<false>(a, nr_head(a, gb), sh[wave], lane, 0.0f);
}

// Many heads of 128 values, all rotated (a prefill chunk): a block takes NR_MANY heads. Its threads stage the heads
// (and the value rows of stored key heads) in LDS with every load issued at once; wave 0 then sums the squares a lane
// per head (the heads' sequential chains run side by side); each wave then takes 16 consecutive heads, a lane per
// rope pair (i, i + 64), recomputing the pair's angle only when the position changes. The arithmetic is
// norm_rope_kernel's, so both kernels give the same bits.
constexpr int NR_MANY = 64, NR_P = 129;  // heads a block; LDS pitch of a staged head (bank spread for the sums)
__global__ __launch_bounds__(64 * NR_WAVES) void norm_rope_many_kernel(NormRope a) {
    __shared__ float xs[NR_MANY][NR_P], vs[NR_MANY][NR_P];
    __shared__ float ssq[NR_MANY];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int total = a.qrows + a.rows, g0 = (int)blockIdx.x * NR_MANY;
    const float qw0 = a.qrows ? a.qw[lane] : 0.0f, qw1 = a.qrows ? a.qw[lane + 64] : 0.0f;
    const float kw0 = a.rows ? a.w[lane] : 0.0f, kw1 = a.rows ? a.w[lane + 64] : 0.0f;
    // 16-byte chunk c = tid + 256 u of the block: head c / 32, values 4 (c % 32) ..
    float4 xv[8], vv[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int c = tid + 256 * u, j = c >> 5, g = g0 + j;
        if (g < total) {
            const NrHead h = nr_head(a, g);
            xv[u] = *(const float4*)(h.xr + 4 * (c & 31));
            if (h.vr) vv[u] = *(const float4*)(h.vr + 4 * (c & 31));
        }
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int c = tid + 256 * u, j = c >> 5, g = g0 + j, i = 4 * (c & 31);
        if (g < total) {
            xs[j][i] = xv[u].x; xs[j][i + 1] = xv[u].y; xs[j][i + 2] = xv[u].z; xs[j][i + 3] = xv[u].w;
            if (g >= a.qrows && a.kc) {
                vs[j][i] = vv[u].x; vs[j][i + 1] = vv[u].y; vs[j][i + 2] = vv[u].z; vs[j][i + 3] = vv[u].w;
            }
        }
    }
    __syncthreads();
    if (wave == 0) {
        float ss = 0.0f;
        if (g0 + lane < total) {
            const float* xr = xs[lane];
            ss = nr_sumsq(128, [&](int i0, float4 (&r)[8]) {
#pragma unroll
                for (int c = 0; c < 8; c++) r[c] = make_float4(xr[i0 + 4 * c], xr[i0 + 4 * c + 1], xr[i0 + 4 * c + 2], xr[i0 + 4 * c + 3]);
            });
        }
        ssq[lane] = ss;
    }
    __syncthreads();
    int cur = -1;  // position of the pair angle held
    float sn = 0.0f, cs = 1.0f;
    for (int jj = 0; jj < NR_MANY / NR_WAVES; jj++) {
        const int j = (NR_MANY / NR_WAVES) * wave + jj, g = g0 + j;
        if (g >= total) break;
        const NrHead h = nr_head(a, g);
        const int pos = a.step[0] + h.b / h.per;
        if (pos != cur) {
            cur = pos;
            const double f = lane < a.nfreq ? a.freq[lane] : pow((double)a.base, -2.0 * (double)lane / 128.0);
            double sd, cd;
            sincos((double)pos * f, &sd, &cd);
            sn = (float)sd;
            cs = (float)cd;
        }
        const bool q = g < a.qrows;
        const float sc = 1.0f / sqrtf(ssq[j] / 128.0f + a.eps);
        const float p = xs[j][lane] * sc * (q ? qw0 : kw0), r = xs[j][lane + 64] * sc * (q ? qw1 : kw1);
        const float o0 = p * cs - r * sn, o1 = p * sn + r * cs;
        h.o[lane] = o0;
        h.o[lane + 64] = o1;
        if (h.vr) {
            const uint64_t e = ((uint64_t)pos * h.per + h.b % h.per) * 128;
            a.kc[e + lane] = f32_to_f16_bits(o0);
            a.kc[e + lane + 64] = f32_to_f16_bits(o1);
            a.vc[e + lane] = f32_to_f16_bits(vs[j][lane]);
            a.vc[e + lane + 64] = f32_to_f16_bits(vs[j][lane + 64]);
        }
    }
}

// rope_neox of pairs lo .. hi - 1 only (Backend::rope_pairs, src/backend.rs:254; kernel src/cuda/kernels.cu:1596-1610),
// in place on `heads` rows `stride` floats apart, head b of token b / per at position step[0] + b / per.
__global__ __launch_bounds__(64 * NR_WAVES) void rope_pairs_kernel(float* x, uint64_t stride, int heads, int per,
                                                                   int n_rot, const int* step, float base, int lo, int hi) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = (int)blockIdx.x * NR_WAVES + wave;
    if (b >= heads) return;
    const int pos = step[0] + b / per, half = n_rot / 2;
    float* h = x + (uint64_t)b * stride;
    for (int i = lane; i < half; i += 64) {
        if (i < lo || i >= hi) continue;
        const double theta = (double)pos * pow((double)base, -2.0 * (double)i / (double)n_rot);
        const float sn = (float)sin(theta), c = (float)cos(theta);
        const float p = h[i], q = h[i + half];
        h[i] = p * c - q * sn;
        h[i + half] = p * sn + q * c;
    }
}

hipError_t launch_norm_rope(const NormRope& a0, hipStream_t s) {
    const int total = a0.qrows + a0.rows;
    if (total <= 0) return hipSuccess;
    // the rope frequencies depend only on the pair index: the host's pow (the one the CPU reference calls) fills
    // them once per launch, so the kernel's f64 work is the sine and cosine
    NormRope a = a0;
    if (!a.q_tstride) a.q_tstride = (uint64_t)a.qper * a.q_stride;
    if (!a.x_tstride) a.x_tstride = (uint64_t)a.per * a.x_stride;
    if (!a.v_tstride) a.v_tstride = (uint64_t)a.per * a.n;
    a.nfreq = a.n_rot / 2 <= NormRope::NFREQ ? a.n_rot / 2 : 0;
    for (int i = 0; i < a.nfreq; i++) a.freq[i] = std::pow((double)a.base, -2.0 * (double)i / (double)a.n_rot);
    const bool vec = ((uintptr_t)a.qx | (uintptr_t)a.x | (uintptr_t)a.v) % 16 == 0 && a.q_stride % 4 == 0 &&
                     a.x_stride % 4 == 0 && a.q_tstride % 4 == 0 && a.x_tstride % 4 == 0 && a.v_tstride % 4 == 0;
    if (total >= 4 * NR_MANY && vec && a.n == 128 && a.n_rot == 128)  // the many-heads form: 16-byte chunks, heads of 128
        norm_rope_many_kernel<<<dim3((unsigned)((total + NR_MANY - 1) / NR_MANY)), dim3(64 * NR_WAVES), 0, s>>>(a);
    else
        norm_rope_kernel<<<dim3((unsigned)((total + NR_WAVES - 1) / NR_WAVES)), dim3(64 * NR_WAVES), 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_rope_pairs(float* x, uint64_t stride, int heads, int per, int n_rot, const int* step, float base,
                             int lo, int hi, hipStream_t s) {
    if (heads <= 0 || hi <= lo) return hipSuccess;
    rope_pairs_kernel<<<dim3((unsigned)((heads + NR_WAVES - 1) / NR_WAVES)), dim3(64 * NR_WAVES), 0, s>>>(
        x, stride, heads, per, n_rot, step, base, lo, hi);
    return hipGetLastError();
}

// kv_store (src/cuda/kernels.cu:2181-2186): value i of the t tokens' rows of n goes to cache element step[0] n + i.
__global__ __launch_bounds__(256) void kv_store_kernel(const float* k, const float* v, uint16_t* kc, uint16_t* vc,
                                                       uint64_t n, uint64_t total, const int* step) {
    const uint64_t base = (uint64_t)step[0] * n;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256) {
        kc[base + i] = f32_to_f16_bits(k[i]);
        vc[base + i] = f32_to_f16_bits(v[i]);
    }
}

hipError_t launch_kv_store(const float* k, const float* v, uint16_t* kc, uint16_t* vc, int n, int t, const int* step,
                           hipStream_t s) {
    const uint64_t total = (uint64_t)n * t;
    if (!total) return hipSuccess;
    const uint64_t blocks = std::min<uint64_t>((total + 255) / 256, 4096);
    kv_store_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(k, v, kc, vc, (uint64_t)n, total, step);
    return hipGetLastError();
}

// ---- argmax ----
// ops::argmax's order (src/ops.rs:110-112): the largest value under f32::total_cmp, the first index on ties. A value
// and its index pack into one 64-bit key whose unsigned maximum is that choice: the total-order image of the bits
// above, ~index below.
constexpr int AMAX_PARTS = 64;

__device__ __forceinline__ uint64_t amax_key(float v, int i) {
    const int32_t b = __float_as_int(v);
    const uint32_t u = (uint32_t)(b ^ (int32_t)((uint32_t)(b >> 31) >> 1)) ^ 0x80000000u;
    return ((uint64_t)u << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)k, o, 64), hi = __shfl_xor((uint32_t)(k >> 32), o, 64);
        const uint64_t other = ((uint64_t)hi << 32) | lo;
        k = other > k ? other : k;
    }
    return k;
}

__global__ __launch_bounds__(256) void argmax_part_kernel(const float* x, int n, uint64_t* part) {
    __shared__ uint64_t sk[4];
    const float* xr = x + (uint64_t)blockIdx.y * n;
    uint64_t best = 0;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += AMAX_PARTS * 256) {
        const uint64_t k = amax_key(xr[i], i);
        best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) sk[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = sk[0];
        for (int w = 1; w < 4; w++) b = sk[w] > b ? sk[w] : b;
        part[(uint64_t)blockIdx.y * AMAX_PARTS + blockIdx.x] = b;
    }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const uint64_t* part, int* out) {
    const uint64_t k = wave_max_u64(part[(uint64_t)blockIdx.x * AMAX_PARTS + threadIdx.x]);
    if (threadIdx.x == 0) out[blockIdx.x] = (int)(0xFFFFFFFFu - (uint32_t)k);
}

uint64_t argmax_part_bytes(int rows) { return (uint64_t)rows * AMAX_PARTS * 8; }

hipError_t launch_argmax_rows(const float* x, int n, int rows, uint64_t* part, int* out, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    argmax_part_kernel<<<dim3(AMAX_PARTS, (unsigned)rows), dim3(256), 0, s>>>(x, n, part);
    argmax_final_kernel<<<dim3((unsigned)rows), dim3(64), 0, s>>>(part, out);
    return hipGetLastError();
}

// ---- elementwise ----
__global__ __launch_bounds__(256) void add_kernel(float* x, const float* y, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) x[i] = x[i] + y[i];
}
__global__ __launch_bounds__(256) void swiglu_kernel(float* g, const float* u, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256)
        g[i] = silu_f32(g[i]) * u[i];
}
static unsigned ew_blocks(uint64_t n) { return (unsigned)std::min<uint64_t>((n + 255) / 256, 8192); }

hipError_t launch_add(float* x, const float* y, uint64_t n, hipStream_t s) {
    if (!n) return hipSuccess;
    add_kernel<<<dim3(ew_blocks(n)), dim3(256), 0, s>>>(x, y, n);
    return hipGetLastError();
}
hipError_t launch_swiglu(float* g, const float* u, uint64_t n, hipStream_t s) {
    if (!n) return hipSuccess;
    swiglu_kernel<<<dim3(ew_blocks(n)), dim3(256), 0, s>>>(g, u, n);
    return hipGetLastError();
}

// ---- embedding rows: out[i] = dequant(row min(ids[i], rows - 1)) (Model::embed, src/model.rs:334-339) ----
template <int T>
__global__ __launch_bounds__(256) void get_rows_kernel(const uint8_t* __restrict__ w, uint64_t rb, uint64_t rows,
                                                       int cols, const int* ids, uint64_t groups, float* __restrict__ out) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= groups) return;
    const int gpr = cols / 32;
    const uint64_t r = i / gpr;
    const int g = (int)(i % gpr);
    const int id = ids[r];
    const uint64_t src = id < 0 ? 0 : (uint64_t)id >= rows ? rows - 1 : (uint64_t)id;
    const uint8_t* sb = w + src * rb + (uint64_t)(g / 8) * sb_bytes(T);
    float v[32];
    dequant32<T>(sb, g % 8, v);
    float4* o = (float4*)(out + r * cols + 32 * g);
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
}

template <int T>
static hipError_t get_rows_t(const uint8_t* w, uint64_t rows, uint64_t cols, const int* ids, int n, float* out,
                             hipStream_t s) {
    const uint64_t groups = (uint64_t)n * (cols / 32);
    if (!groups) return hipSuccess;
    get_rows_kernel<T><<<dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, s>>>(w, row_bytes(T, cols), rows,
                                                                                   (int)cols, ids, groups, out);
    return hipGetLastError();
}

hipError_t launch_get_rows(int ty, const uint8_t* w, uint64_t rows, uint64_t cols, const int* ids, int n, float* out,
                           hipStream_t s) {
    switch (ty) {
    case Q8_0: return get_rows_t<Q8_0>(w, rows, cols, ids, n, out, s);
    case Q2_K: return get_rows_t<Q2_K>(w, rows, cols, ids, n, out, s);
    case Q3_K: return get_rows_t<Q3_K>(w, rows, cols, ids, n, out, s);
    case Q4_K: return get_rows_t<Q4_K>(w, rows, cols, ids, n, out, s);
    case Q5_K: return get_rows_t<Q5_K>(w, rows, cols, ids, n, out, s);
    case Q6_K: return get_rows_t<Q6_K>(w, rows, cols, ids, n, out, s);
    case IQ2_XXS: return get_rows_t<IQ2_XXS>(w, rows, cols, ids, n, out, s);
    case IQ3_S: return get_rows_t<IQ3_S>(w, rows, cols, ids, n, out, s);
    case IQ4_XS: return get_rows_t<IQ4_XS>(w, rows, cols, ids, n, out, s);
    }
    return hipErrorInvalidValue;
}

// ---- f32-weight GEMV: one wave per weight row, every input of the launch on that row ----
constexpr int GF_NT = 4;
__global__ __launch_bounds__(256) void gemv_f32_kernel(const float* __restrict__ w, int rows, int cols,
                                                       const float* __restrict__ x, uint64_t x_stride, float* y,
                                                       uint64_t y_stride, int nt, int act) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float4* wr = (const float4*)(w + (uint64_t)r * cols);
    float acc[GF_NT] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c = lane; c < cols / 4; c += 64) {
        const float4 wv = wr[c];
#pragma unroll
        for (int t = 0; t < GF_NT; t++) {
            if (t < nt) {
                const float4 xv = ((const float4*)(x + t * x_stride))[c];
                acc[t] += wv.x * xv.x + wv.y * xv.y + wv.z * xv.z + wv.w * xv.w;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < GF_NT; t++) {
        if (t < nt) {
            const float v = wave_sum_xor(acc[t]);
            if (lane == 0) {
                float* yo = y + t * y_stride + r;
                *yo = act == 2 ? *yo + v : v;
            }
        }
    }
}

// One input (a decode step): a wave per row, a block per wave; each pass loads GF1_U 16-byte chunks of the row and of
// x per lane before using any, so a 2048-value row takes one memory round trip. A lane sums the same chunks in the
// same order as gemv_f32_kernel, so both kernels give the same bits.
constexpr int GF1_U = 8;
__global__ __launch_bounds__(64) void gemv_f32_1_kernel(const float* __restrict__ w, int rows, int cols,
                                                        const float* __restrict__ x, float* y, int act) {
    const int r = blockIdx.x, lane = threadIdx.x, n4 = cols / 4;
    const float4* wr = (const float4*)(w + (uint64_t)r * cols);
    const float4* xr = (const float4*)x;
    float acc = 0.0f;
    for (int c0 = 0; c0 < n4; c0 += 64 * GF1_U) {
        float4 wv[GF1_U], xv[GF1_U];
#pragma unroll
        for (int u = 0; u < GF1_U; u++) {
            const int c = c0 + lane + 64 * u;
            wv[u] = c < n4 ? wr[c] : make_float4(0.f, 0.f, 0.f, 0.f);
            xv[u] = c < n4 ? xr[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < GF1_U; u++)
            if (c0 + lane + 64 * u < n4) acc += wv[u].x * xv[u].x + wv[u].y * xv[u].y + wv[u].z * xv[u].z + wv[u].w * xv[u].w;
    }
    const float v = wave_sum_xor(acc);
    if (lane == 0) y[r] = act == 2 ? y[r] + v : v;
}

hipError_t launch_gemv_f32(const float* w, int rows, int cols, const float* x, uint64_t x_stride, float* y,
                           uint64_t y_stride, int nt, int act, hipStream_t s) {
    if (!rows || !nt) return hipSuccess;
    if (nt == 1) {
        gemv_f32_1_kernel<<<dim3((unsigned)rows), dim3(64), 0, s>>>(w, rows, cols, x, y, act);
        return hipGetLastError();
    }
    for (int t0 = 0; t0 < nt; t0 += GF_NT) {
        const int n = std::min(GF_NT, nt - t0);
        gemv_f32_kernel<<<dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s>>>(w, rows, cols, x + t0 * x_stride, x_stride,
                                                                                y + t0 * y_stride, y_stride, n, act);
    }
    return hipGetLastError();
}

// ---- f32-weight GEMM (gemm_dense of a float matrix): each output's dot runs over k in index order with a multiply
// then an add, as Tensor::matvec's f32 iterator sum (src/weights.rs:29-37): the CPU's bits. That makes every output
// one dependent chain of 2 cols instructions, so the kernel is built for VALU throughput with two waves a SIMD: a
// block of 4 waves takes 64 positions (a lane each) x 8 weight rows (2 a wave, 2 chains a lane); per step of 64 k the
// block stages x transposed ([k][position]: a lane's reads hit distinct banks) and the 8 rows' weights in LDS, and a
// lane reads its x value once per k and the weights as wave-wide broadcasts (one 16-byte read for 4 k of a row). ----
constexpr int GF_M = 64, GF_RW = 4, GF_R = 4 * GF_RW, GF_K = 64;  // GF_RW rows (chains) a wave (4: 102 -> 87 us at 4096 x 128 x 2048)
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ w, int rows, int cols,
                                                       const float* __restrict__ x, uint64_t x_stride, float* y,
                                                       uint64_t y_stride, int n, int act) {
    __shared__ __align__(16) float xs[GF_K][GF_M + 1];  // (+1: the staging writes spread over banks)
    __shared__ __align__(16) float ws[GF_R][GF_K];
    const int m0 = blockIdx.x * GF_M, r0 = blockIdx.y * GF_R, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // staging: x rows m0 + tid / KQ + SP i (i < NP), k k0 + 4 (tid % KQ) .. + 3; w row r0 + tid / KQ (< GF_R)
    constexpr int KQ = GF_K / 4, SP = 256 / KQ, NP = GF_M / SP;
    static_assert(GF_R <= SP, "one pass stages the weight rows");
    const int sm = tid / KQ, sk = 4 * (tid % KQ);
    float acc[GF_RW] = {};
    float4 xv[NP], wv;
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int m = m0 + sm + SP * i;
            xv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < n && k0 + sk < cols) xv[i] = *(const float4*)(x + (uint64_t)m * x_stride + k0 + sk);
        }
        wv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (sm < GF_R && r0 + sm < rows && k0 + sk < cols) wv = *(const float4*)(w + (uint64_t)(r0 + sm) * cols + k0 + sk);
    };
    load(0);
    for (int k0 = 0; k0 < cols; k0 += GF_K) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int m = sm + SP * i;
            xs[sk][m] = xv[i].x; xs[sk + 1][m] = xv[i].y; xs[sk + 2][m] = xv[i].z; xs[sk + 3][m] = xv[i].w;
        }
        if (sm < GF_R) *(float4*)&ws[sm][sk] = wv;
        __syncthreads();
        if (k0 + GF_K < cols) load(k0 + GF_K);
        const int kn = min(GF_K, cols - k0);
        const float* wr = &ws[GF_RW * wave][0];
        // the whole step unrolled (cols % 4 == 0; a shorter last step ends early), so its LDS reads run ahead
#pragma unroll
        for (int k = 0; k < GF_K; k += 4) {
            if (k >= kn) break;
            const float a[4] = {xs[k][lane], xs[k + 1][lane], xs[k + 2][lane], xs[k + 3][lane]};
            float4 wj[GF_RW];
#pragma unroll
            for (int j = 0; j < GF_RW; j++) wj[j] = *(const float4*)(wr + j * GF_K + k);
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int j = 0; j < GF_RW; j++) acc[j] += a[e] * (e == 0 ? wj[j].x : e == 1 ? wj[j].y : e == 2 ? wj[j].z : wj[j].w);
        }
    }
    const int m = m0 + lane;
    if (m < n) {
#pragma unroll
        for (int j = 0; j < GF_RW; j++) {
            const int r = r0 + GF_RW * wave + j;
            if (r >= rows) continue;
            float* yo = y + (uint64_t)m * y_stride + r;
            const float v = acc[j];
            *yo = act == 0 ? v : act == 1 ? silu_f32(*yo) * v : *yo + v;
        }
    }
}

hipError_t launch_gemm_f32(const float* w, int rows, int cols, const float* x, uint64_t x_stride, float* y,
                           uint64_t y_stride, int n, int act, hipStream_t s) {
    if (!rows || !n) return hipSuccess;
    gemm_f32_kernel<<<dim3((unsigned)((n + GF_M - 1) / GF_M), (unsigned)((rows + GF_R - 1) / GF_R)), dim3(256), 0, s>>>(
        w, rows, cols, x, x_stride, y, y_stride, n, act);
    return hipGetLastError();
}

// ---- synthetic weights: random block bytes with every f16 scale field in [lo, hi) (the reference's random_tensor
// design, tests/kernels.rs:1473-1550), from a counter-based hash of (seed, position) ----
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void fill_bytes_kernel(uint8_t* w, uint64_t bytes, uint64_t seed) {
    const uint64_t words = bytes / 4;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < (bytes + 3) / 4; i += (uint64_t)gridDim.x * 256) {
        const uint32_t r = (uint32_t)mix64(seed * 0x9E3779B97F4A7C15ull + i);
        if (i < words) {
            ((uint32_t*)w)[i] = r;
        } else {
            for (uint64_t b = 4 * i; b < bytes; b++) w[b] = (uint8_t)(r >> (8 * (b - 4 * i)));
        }
    }
}

__global__ __launch_bounds__(256) void fill_scales_kernel(uint8_t* w, uint64_t n_blocks, int bb, int f0, int f1,
                                                          uint64_t seed, float lo, float hi) {
    for (uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x; b < n_blocks; b += (uint64_t)gridDim.x * 256) {
        const uint64_t r = mix64(~seed * 0xD1B54A32D192ED03ull + b);
        const float u0 = (float)(uint32_t)r * 2.3283064365386963e-10f, u1 = (float)(uint32_t)(r >> 32) * 2.3283064365386963e-10f;
        *(uint16_t*)(w + b * bb + f0) = f32_to_f16_bits(lo + (hi - lo) * u0);
        if (f1 >= 0) *(uint16_t*)(w + b * bb + f1) = f32_to_f16_bits(lo + (hi - lo) * u1);
    }
}

hipError_t launch_fill_blocks(int ty, uint8_t* w, uint64_t n_blocks, uint64_t seed, float lo, float hi, hipStream_t s) {
    if (!n_blocks) return hipSuccess;
    const int bb = block_bytes(ty);
    int f0 = 0, f1 = -1;  // offsets of the f16 scale fields in a block (d, and dmin where the type has one)
    switch (ty) {
    case Q2_K: f0 = 80; f1 = 82; break;
    case Q3_K: f0 = 108; break;
    case Q4_K: case Q5_K: f0 = 0; f1 = 2; break;
    case Q6_K: f0 = 208; break;
    default: f0 = 0; break;
    }
    const uint64_t bytes = n_blocks * (uint64_t)bb;
    fill_bytes_kernel<<<dim3(ew_blocks((bytes + 3) / 4)), dim3(256), 0, s>>>(w, bytes, seed);
    fill_scales_kernel<<<dim3(ew_blocks(n_blocks)), dim3(256), 0, s>>>(w, n_blocks, bb, f0, f1, seed, lo, hi);
    return hipGetLastError();
}

}  // namespace strata

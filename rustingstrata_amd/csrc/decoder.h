// Launchers of the decoder-stack kernels around the quantized matmuls (decoder.hip, attn.hip): norms with rope and
// the KV cache store, argmax, float-weight matmuls, embedding rows, attention. Arguments are checked in api.hip.
#pragma once
#include "common.h"

namespace strata {

// rms_norm_rope over `rows` heads of n: head b (token b / per, position step[0] + b / per) from x + b x_stride into
// out + b n, normed with w then NEOX-roped on its first n_rot values; with
// kc, also stored with its v row (v + b n) into the f16 caches at row (position per + b % per). q rows first: the
// first qrows heads come from qx (q_stride, qw, qo, qper) and are never stored. With token strides (below) head b
// is read at token b / per times the token stride plus head b % per times the head stride (a fused q/k/v output).
struct NormRope {
    const float* x = nullptr; uint64_t x_stride = 0; const float* w = nullptr; float* out = nullptr;
    int n = 0, rows = 0, per = 1;
    const float* v = nullptr; uint16_t* kc = nullptr; uint16_t* vc = nullptr;
    int qrows = 0; const float* qx = nullptr; uint64_t q_stride = 0; const float* qw = nullptr; float* qo = nullptr;
    int qper = 1;
    float eps = 0, base = 0; int n_rot = 0; const int* step = nullptr;
    // floats between consecutive tokens' first heads of q, x (keys) and v; 0: the heads of all tokens back to back
    // (qper q_stride, per x_stride, per n)
    uint64_t q_tstride = 0, x_tstride = 0, v_tstride = 0;
    // base^(-2 i / n_rot) for the first nfreq pairs (filled by launch_norm_rope on the host)
    static constexpr int NFREQ = 128;
    int nfreq = 0; double freq[NFREQ] = {};
};
hipError_t launch_norm_rope(const NormRope& a, hipStream_t s);

// The sum of squares of x[0 .. n) in index order, as ops::rms_norm's iterator sum (a multiply, then an add): the
// CPU's bits. sq(i0, r) loads values i0 .. i0 + 31 as 8 float4; the next 32 are loaded while the current 32 are added
// (n % 32 == 0).
template <typename Load>
__device__ __forceinline__ float nr_sumsq(int n, Load&& ld) {
    float ss = 0.0f;
    float4 r[8], nx[8];
    ld(0, r);
    for (int i0 = 0; i0 < n; i0 += 32) {
        if (i0 + 32 < n) ld(i0 + 32, nx);
#pragma unroll
        for (int c = 0; c < 8; c++) {
            ss += r[c].x * r[c].x; ss += r[c].y * r[c].y; ss += r[c].z * r[c].z; ss += r[c].w * r[c].w;
        }
#pragma unroll
        for (int c = 0; c < 8; c++) r[c] = nx[c];
    }
    return ss;
}

hipError_t launch_rope_pairs(float* x, uint64_t stride, int heads, int per, int n_rot, const int* step, float base,
                             int lo, int hi, hipStream_t s);
hipError_t launch_kv_store(const float* k, const float* v, uint16_t* kc, uint16_t* vc, int n, int t, const int* step,
                           hipStream_t s);
// part: at least argmax_part_bytes(rows) bytes of scratch.
uint64_t argmax_part_bytes(int rows);
hipError_t launch_argmax_rows(const float* x, int n, int rows, uint64_t* part, int* out, hipStream_t s);
hipError_t launch_add(float* x, const float* y, uint64_t n, hipStream_t s);
hipError_t launch_swiglu(float* g, const float* u, uint64_t n, hipStream_t s);
hipError_t launch_get_rows(int ty, const uint8_t* w, uint64_t rows, uint64_t cols, const int* ids, int n, float* out,
                           hipStream_t s);
// y[t * y_stride + r] = W[r] . x[t * x_stride] for an f32 matrix W (rows x cols), t < nt; act 2 adds to y.
hipError_t launch_gemv_f32(const float* w, int rows, int cols, const float* x, uint64_t x_stride, float* y,
                           uint64_t y_stride, int nt, int act, hipStream_t s);
// gemm_dense with f32 weights: y[m * y_stride + r] (op) W[r] . x[m * x_stride], m < n; act 0 store, 1 SwiGLU, 2 add.
hipError_t launch_gemm_f32(const float* w, int rows, int cols, const float* x, uint64_t x_stride, float* y,
                           uint64_t y_stride, int n, int act, hipStream_t s);
hipError_t launch_fill_blocks(int ty, uint8_t* w, uint64_t n_blocks, uint64_t seed, float lo, float hi, hipStream_t s);

// Attention (attn.hip). Caches: f16 rows of nkv * hd values per position.
constexpr int ATT_SPLITS = 128;  // position splits of a decode token (part rows per head)
// With nr (one token): the query heads are nr's raw q rows (q unused) and rms_norm_rope_qk with the KV store of nr
// runs inside the launch (the same bits as launch_norm_rope first). With xq: out also quantized as quant_xq does
// under numerics `mode` (nh hd a multiple of 256). hipErrorNotSupported for shapes it does not take.
hipError_t launch_attn_decode(const float* q, const uint16_t* kc, const uint16_t* vc, const float* qg, float* out,
                              float* part, const int* step, int nh, int nkv, int hd, float scale, int nt,
                              const float* sink, int win, hipStream_t s, const NormRope* nr = nullptr,
                              int8_t* xq = nullptr, int mode = 0);
hipError_t launch_attn_prefill(const float* q, const uint16_t* kc, const uint16_t* vc, const float* qg, float* out,
                               const int* step, int t, int nh, int nkv, int hd, float scale, const float* sink, int win,
                               hipStream_t s);

}  // namespace strata

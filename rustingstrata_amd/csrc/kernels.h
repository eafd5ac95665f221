// Launchers the C-ABI layer (api.hip) calls; each validates nothing and launches on `s`. Arguments are checked in
// api.hip, where the errors of the reference's Backend methods are reproduced.
#pragma once
#include "common.h"

namespace strata {

// Bytes of the quant_xq layout for nt rows of n values: nt * n int8 then nt * n / 32 f32 scales.
inline uint64_t xq_bytes(uint64_t n, uint64_t nt) { return nt * (n + n / 8); }

hipError_t launch_dequant(int ty, const uint8_t* w, uint64_t rows, uint64_t cols, float* out, hipStream_t s);
// quant_xq under numerics `mode` (STRATA_NUM_*): rows t < nt of x (t * x_stride floats apart) into out.
// h = rms_norm(x + res) * nw (+ its quantization into xq when not null), y = W h for an F32 rows x n matrix, one
// launch; x is not written. hipErrorNotSupported: n > 2048, n % 8, or rows not 16-byte aligned.
hipError_t launch_rms_norm_gemv_f32(const float* x, const float* res, const float* nw, float* h, int8_t* xq, int n,
                                   float eps, int mode, const float* W, int rows, float* y, hipStream_t s);
hipError_t launch_quant_xq(const float* x, uint64_t x_stride, int n, int nt, int8_t* out, int mode, hipStream_t s);
// With ye: x += sum_j wh[j] ye[j] over each row's ck slots (moe_combine's arithmetic) in place of res; rows of at most
// 2048 values (a multiple of 8, 16-byte aligned) only, else hipErrorNotSupported.
hipError_t launch_rms_norm_q(float* x, uint64_t x_stride, const float* w, float* out, uint64_t out_stride, int n, int rows,
                             float eps, int8_t* xq, const float* res, int mode, hipStream_t s, const float* ye = nullptr,
                             const float* wh = nullptr, int ck = 0);

struct GemvLaunch {
    int ty = 0;
    const uint8_t* w = nullptr;   // matrix (dense) or expert base (moe)
    int rows = 0, cols = 0;
    int nt = 1;                   // inputs per weight read (1..4)
    int numerics = 0;             // STRATA_NUM_*: how xq was quantized
    const int8_t* xq = nullptr;   // quant_xq layout of n_xrows rows of cols; null: quantize xf in the kernel (nt == 1)
    const float* xf = nullptr;    // x as f32, rows x_stride floats apart
    const float* xu = nullptr;    // with xf (nt == 1): x = silu(xf) * xu, same row layout
    uint64_t x_stride = 0;
    int n_xrows = 1;
    float* y = nullptr;
    int y_stride = 0;             // floats between the outputs of consecutive inputs (dense)
    // moe_gemv: slot j uses expert ids[j] (skipped when < 0) at w + ids[j] * stride, x row j / xg, output y + j rows
    const int* ids = nullptr;
    int k = 1, xg = 1;
    int64_t stride = 0;
    // second matrix (gemvq2 / paired moe_gemv): at byte offset w2, output at byte offset y2, rows2 rows
    bool pair = false;
    int64_t w2 = 0, y2 = 0;
    int rows2 = 0;
    // moe_gemv of one token that routes it first (single input, no SwiGLU input): the launch ranks the rn <= 128
    // logits at rp as moe_route does (top k, k <= 32) and writes ids, wts, wh and the slots (to `ids` above, which the
    // GEMV's slots then are). hipErrorNotSupported: a shape this does not take.
    const float* rp = nullptr;
    const int* rtable = nullptr;
    int* rids = nullptr;
    float* rwts = nullptr;
    float* rwh = nullptr;
    float rscale = 0.0f;
    int rn = 0, rsig = 0;
    // one plain matrix, single f32 input xf of at most 2048 values: the GEMV runs on h = rms_norm(xf + nres + sum_j
    // nwh[j] nye[j] (j < nck <= 8, rows of cols floats)) * nw with rms_norm_q's arithmetic; block 0 writes xf + nres +
    // the combine to nxw (may be null; not xf). hipErrorNotSupported: any other shape.
    const float* nw = nullptr;
    const float* nres = nullptr;
    const float* nye = nullptr;
    const float* nwh = nullptr;
    float* nxw = nullptr;
    float neps = 0.0f;
    int nck = 0;
};
hipError_t launch_gemv(const GemvLaunch& g, hipStream_t s);
// moe_down_combine as one launch: x[tk] += sum_j wh[tk k + j] W_{slots[j]} x_j (slots in order) + the shared expert,
// x_j row tk k + j of xq. hipErrorNotSupported: a shape the fused layout does not take (cols not a multiple of 256,
// too many slots for its rows), for the caller's two launches.
struct DownCombineLaunch {
    int ty = 0, numerics = 0;
    const uint8_t* w = nullptr;
    int64_t stride = 0;
    int rows = 0, cols = 0, k = 1, t = 1;
    const int* slots = nullptr;
    const float* wh = nullptr;
    const int8_t* xq = nullptr;
    float* x = nullptr;
    const float* sh = nullptr;
    const float* sg = nullptr;
};
hipError_t launch_down_combine(const DownCombineLaunch& g, hipStream_t s);
// Streaming copy of `bytes` (multiple of 16), the reference kernel for HBM byte counters.
hipError_t launch_copy(const void* src, void* dst, uint64_t bytes, hipStream_t s);
// Streaming read of `bytes` (multiple of 16; 0: an empty launch), the floor a GEMV of the same bytes is measured against.
hipError_t launch_read(const void* src, uint64_t bytes, uint32_t* sink, hipStream_t s);
// Largest row size (bytes) launch_gemv accepts.
uint64_t gemv_max_row_bytes();
// Columns the single-input kernel takes (a lane keeps one super-block's x in registers, at most 64 lanes a row);
// launch_gemv runs wider single-input rows on the multi-input kernel, which needs x pre-quantized (GemvLaunch::xq).
constexpr int GEMV1_MAX_COLS = 16384;

}  // namespace strata

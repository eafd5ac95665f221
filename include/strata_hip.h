/* strata_hip: MI355X (gfx950) backend for RustingStrata's quantized-matmul hot path, as a C ABI.
 *
 * Each entry point is one method of the reference's `Backend` trait (src/backend.rs:98-443) on the hot path, with
 * the trait's argument meaning: device addresses as uint64_t, strides in floats unless named otherwise, ops queued
 * in order on the context's one stream, host copies synchronous. Every function returns 0 on success and -1 on
 * error; the message is then in strata_last_error() (per thread). As in the reference, an op that rejects its
 * arguments (unsupported type or shape) returns the error without launching anything.
 *
 * Weight type ids are the GGUF ids of `GgmlType::from_u32` (src/quant/mod.rs:15-19): Q8_0 8, Q2_K 10, Q3_K 11,
 * Q4_K 12, Q5_K 13, Q6_K 14, IQ2_XXS 16, IQ3_S 21, IQ4_XS 23. Weights are the raw GGUF block bytes, rows of
 * `cols` values, row r at ptr + r * row_bytes (src/weights.rs:11-37), no repacking at upload. F32 (0) matrices, the
 * form Backend::upload gives F32/F16 GGUF tensors (src/backend.rs:156-166), are accepted by gemv and gemm_dense. */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct strata_ctx strata_ctx;

/* GpuTensor (src/backend.rs:32-45): `rows` x `cols` of type `ty` from device address `ptr`. */
typedef struct {
    int32_t ty;
    int32_t reserved;
    uint64_t rows;
    uint64_t cols;
    uint64_t ptr;
} strata_tensor;

/* Activation numerics. STRATA_NUM_Q8K quantizes x as the reference CPU path does (quantize_q8k,
 * src/cpu_moe.rs:28-46: one scale per 256 values, -127 / the signed value of largest magnitude, ties to even), so
 * results match cpu_moe::matvec to accumulation order; it is what the reference GPU does under
 * STRATA_LLAMA_NUMERICS (src/cuda/kernels.cu:619-651). STRATA_NUM_Q8_32 is the reference GPU default (one scale
 * per 32 values, max / 127; src/cuda/kernels.cu:640-660). Both write the quant_xq layout. */
enum { STRATA_NUM_Q8K = 0, STRATA_NUM_Q8_32 = 1 };

/* `gemm` act flags (src/backend.rs:187-191, SAME_X at src/backend.rs:91). */
/* GGUF type id of float32 tensors. */
enum { STRATA_F32 = 0 };

enum { STRATA_ACT_STORE = 0, STRATA_ACT_SWIGLU = 1, STRATA_ACT_ADD = 2, STRATA_SAME_X = 4, STRATA_X_Q = 8,
       STRATA_SMALL_TILES = 16 };
/* STRATA_X_Q (quantized-matrix GEMMs, no counterpart in the reference): x is X already quantized in strata_quant_xq's
 * layout under STRATA_NUM_Q8K (n_x rows of cols int8, then their scales; x_stride = cols), e.g. the xq that
 * strata_rms_norm_q wrote beside its output, so the GEMM skips its own quantization of X (the same bits). */

/* ---- context, memory and queue: backend::open and the memory methods of Backend ---- */

/* backend::open (src/backend.rs:60-75) -> cuda::Gpu::new (src/cuda/mod.rs:464-526): bind GPU `device`, create the
 * context's stream and scratch. */
int strata_open(int device, strata_ctx** out);
void strata_close(strata_ctx* ctx);
/* Message of the last failed call on this thread ("" if none). */
const char* strata_last_error(void);
/* Backend::device (src/backend.rs:102). */
int strata_device_name(strata_ctx* ctx, char* buf, size_t len);
/* Activation numerics for every later op (default STRATA_NUM_Q8K). */
int strata_set_numerics(strata_ctx* ctx, int mode);
int strata_get_numerics(strata_ctx* ctx);
/* Backend::alloc (src/backend.rs:108): zeroed, at least 1 byte, 256-byte aligned. */
int strata_alloc(strata_ctx* ctx, size_t bytes, uint64_t* addr);
/* Dropping the last Buf clone (src/backend.rs:18-30). */
int strata_free(strata_ctx* ctx, uint64_t addr);
/* Backend::htod / dtoh / dtod (src/backend.rs:109-111): synchronous; the device range must lie inside one
 * allocation of this context (the reference bounds-checks against the Buf, src/cuda/mod.rs:789,816,825). */
int strata_htod(strata_ctx* ctx, const void* src, uint64_t dst, size_t bytes);
int strata_dtoh(strata_ctx* ctx, uint64_t src, void* dst, size_t bytes);
int strata_dtod(strata_ctx* ctx, uint64_t src, uint64_t dst, size_t bytes);
/* Backend::memset (src/backend.rs:113): zero `bytes` from dst, queued. */
int strata_memset(strata_ctx* ctx, uint64_t dst, size_t bytes);
/* Backend::mem_info (src/backend.rs:115). */
int strata_mem_info(strata_ctx* ctx, size_t* free_bytes, size_t* total_bytes);
/* Backend::sync (src/backend.rs:117). */
int strata_sync(strata_ctx* ctx);
/* The context's HIP stream (a hipStream_t), for callers that order their own work against it. */
void* strata_stream(strata_ctx* ctx);

/* ---- recorded graphs: Backend::graph (src/backend.rs:118-120; CUDA graphs in src/cuda/mod.rs:868-888) ----
 * strata_graph_begin starts recording the ops queued on the context's stream; strata_graph_end stops and returns an
 * executable graph; strata_graph_launch replays it on the stream. As in the trait, the recorded ops must read their
 * per-call values from device memory. Ops whose scratch would have to grow cannot be recorded (run them once
 * before recording): they return an error while recording. Scratch that a later, larger eager call replaces stays
 * allocated while any graph of the context exists (the graphs keep its address), and is freed when the last one is
 * destroyed. A STRATA_SAME_X gemm inside a recording reuses only a quantization recorded in the same recording
 * (strata_graph_begin forgets the cached X). */
int strata_graph_begin(strata_ctx* ctx);
int strata_graph_end(strata_ctx* ctx, void** graph);
int strata_graph_launch(strata_ctx* ctx, void* graph);
int strata_graph_destroy(strata_ctx* ctx, void* graph);

/* ---- dequant and activation quantization ---- */

/* Backend::dequant (src/backend.rs:227-228): out = the first `rows` rows of w as f32, bit-identical to
 * quant::dequant_row (src/quant/mod.rs:65-91). */
int strata_dequant(strata_ctx* ctx, const strata_tensor* w, uint64_t rows, uint64_t out);
/* Backend::quant_xq (src/backend.rs:229-231): nt rows of n floats (row t at x + 4 t x_stride bytes) into nt * n
 * int8 then nt * n / 32 f32 scales (one per 32 values), nt * (n + n / 8) bytes, under the context's numerics.
 * n must be a multiple of 32. */
int strata_quant_xq(strata_ctx* ctx, uint64_t x, uint64_t x_stride, uint64_t n, uint64_t nt, uint64_t out);

/* ---- decode GEMV ---- */

/* Backend::gemv (src/backend.rs:199): y = W x over all rows. cols must be a multiple of 256 (of 32 for Q8_0),
 * as Gpu::gemv_cols requires (src/cuda/mod.rs:567-571), and a row at most 24512 bytes (one weight tile; e.g. 43520
 * Q4_K or 23040 Q8_0 columns). gemv, gemvn and gemvq take any such row; the MoE, paired and no-alloc GEMVs take up
 * to 16384 columns. */
int strata_gemv(strata_ctx* ctx, const strata_tensor* w, uint64_t x, uint64_t y);
/* Backend::gemvn (src/backend.rs:202): y[t] = W x[t] for t < nt (1..4), each weight block read once; bit-equal
 * to strata_gemv per input. */
int strata_gemvn(strata_ctx* ctx, const strata_tensor* w, uint64_t x, uint64_t x_stride, uint64_t y,
                 uint64_t y_stride, uint64_t nt);
/* No counterpart in the reference: strata_gemvn for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The same bits as strata_gemvn; the quantized
 * x of the nt inputs goes to a fixed device array of 73728 bytes per GPU (4 inputs of 16384 values) instead of the
 * context's growable scratch, so the call makes no allocation. Larger requests are rejected with an error. Every
 * call on one GPU shares that array: calls that overlap on one GPU (other streams or contexts) race. */
int strata_gemvn_noalloc(strata_ctx* ctx, const strata_tensor* w, uint64_t x, uint64_t x_stride, uint64_t y,
                         uint64_t y_stride, uint64_t nt);
/* Backend::gemvq (src/backend.rs:204): strata_gemvn reading x pre-quantized by strata_quant_xq at xq (0 =
 * quantize x itself). */
int strata_gemvq(strata_ctx* ctx, const strata_tensor* w, uint64_t x, uint64_t x_stride, uint64_t xq, uint64_t y,
                 uint64_t y_stride, uint64_t nt);
/* Backend::gemvq2 (src/backend.rs:206-209): gemvq of a into ya and of b into yb on the same x, one launch when the
 * types and column counts agree (src/cuda/mod.rs:936-944). */
int strata_gemvq2(strata_ctx* ctx, const strata_tensor* a, const strata_tensor* b, uint64_t x, uint64_t x_stride,
                  uint64_t xq, uint64_t ya, uint64_t yb, uint64_t nt);
/* Backend::moe_gemv (src/backend.rs:223-226): for j < k with ids[j] >= 0, y[j] (rows floats at y + 4 j rows bytes)
 * = W_j x[j / xg], W_j the rows x cols matrix of type ty at w + ids[j] * stride bytes; slots with ids[j] < 0 are
 * left untouched. has_pair: also the matrices at byte offset w2 into outputs at byte offset y2 (the paired gate/up
 * launch). xq != 0: x pre-quantized by strata_quant_xq (k / xg rows), read in place of x. */
int strata_moe_gemv(strata_ctx* ctx, int ty, uint64_t rows, uint64_t cols, uint64_t w, uint64_t stride,
                    uint64_t ids, uint64_t k, uint64_t x, uint64_t x_stride, uint64_t xg, uint64_t y,
                    int has_pair, int64_t w2, int64_t y2, uint64_t xq);

/* ---- MoE routing and combine ---- */

/* Backend::router_topk (src/backend.rs:411-412; kernel src/cuda/kernels.cu:2633-2686): for each of t tokens, softmax
 * (or sigmoid) over n logits, the k largest (ties to the lower index, ops::top_k src/ops.rs:102-107), weights
 * renormalised by 1 / max(sum, 6.1035e-5) times extra_scale (when not 0). ids / wts: rows of k. n <= 512,
 * k <= 32, else an error (src/cuda/mod.rs:1214-1218). */
int strata_router_topk(strata_ctx* ctx, uint64_t p, uint64_t n, uint64_t k, float extra_scale, uint64_t ids,
                       uint64_t wts, uint64_t t, int sigmoid);
/* Backend::moe_route with mb = 0 (src/backend.rs:413-417, moe_mailbox_optional 424; kernel
 * src/cuda/kernels.cu:2693-2723): router_topk, then slots[j] = table[ids[j]] (-1: not resident) and wh[j] =
 * wts[j] on a hit, else 0. */
int strata_moe_route(strata_ctx* ctx, uint64_t p, uint64_t n, uint64_t k, float extra_scale, uint64_t table,
                     uint64_t ids, uint64_t wts, uint64_t slots, uint64_t wh, uint64_t t, int sigmoid);
/* Backend::moe_route with mb = 0 for one token followed by Backend::moe_gemv of its k slots on the token's x (the
 * decode sequence src/gpu_model.rs:3383-3390; src/backend.rs:413-417, 223-226) as one launch: every block of the
 * GEMV ranks the n logits itself (n <= 128; more: two launches) and takes slot j's expert from that ranking, and the
 * launch stores ids, wts, slots and wh as strata_moe_route does. The GEMV is strata_moe_gemv with ids = slots,
 * xg = k (one x row of cols floats, or xq pre-quantized) and the optional pair; rows = 0 routes only. Outputs
 * equal strata_moe_route then strata_moe_gemv bit for bit. */
int strata_moe_route_gemv(strata_ctx* ctx, uint64_t p, uint64_t n, uint64_t k, float extra_scale, uint64_t table,
                          uint64_t ids, uint64_t wts, uint64_t slots, uint64_t wh, int sigmoid, int ty, uint64_t rows,
                          uint64_t cols, uint64_t w, uint64_t stride, uint64_t x, uint64_t y, int has_pair, int64_t w2,
                          int64_t y2, uint64_t xq);
/* Backend::rms_norm (src/backend.rs:232; ops::rms_norm src/ops.rs:3-7; kernel src/cuda/kernels.cu:1504-1550): `rows`
 * rows (x_stride, out_stride in floats), out[r] = x[r] * (1 / sqrt(mean(x[r]^2) + eps)) * w; out may be x. */
int strata_rms_norm(strata_ctx* ctx, uint64_t x, uint64_t x_stride, uint64_t w, uint64_t out, uint64_t out_stride,
                    uint64_t n, uint64_t rows, float eps);
/* Backend::rms_norm_q (src/backend.rs:233-235): strata_rms_norm that first adds res (rows x_stride apart, when not 0)
 * into x in place, and also writes out quantized as strata_quant_xq does into xq (when not 0; n a multiple of 32):
 * [rows x n int8][rows x n / 32 f32 scales]. */
int strata_rms_norm_q(strata_ctx* ctx, uint64_t x, uint64_t x_stride, uint64_t w, uint64_t out, uint64_t out_stride,
                      uint64_t n, uint64_t rows, float eps, uint64_t xq, uint64_t res);
/* Backend::moe_combine with mb = 0 and no shared expert (src/backend.rs:418-419) followed by Backend::rms_norm_q
 * (src/backend.rs:233-235) of the same rows, as a layer's end meets the next layer's attention norm in the decode
 * (src/gpu_model.rs:3383-3412, then 1950-2016): per token row r, x[r] += sum_{j<k, wh[r k + j] != 0} wh[r k + j]
 * ye[r k + j] (in slot order), then out = rms_norm(x) * w and xq as strata_rms_norm_q writes them. With res (not 0,
 * rows n floats apart) x += res comes first, as strata_rms_norm_q's res. x rows are n floats apart (moe_combine's
 * layout); rows of up to 2048 values (a multiple of 8, 16-byte aligned) run as one launch, others as separate calls.
 * The same bits as strata_add(x, res), strata_moe_combine, then strata_rms_norm_q. */
int strata_combine_rms_norm_q(strata_ctx* ctx, uint64_t x, uint64_t x_stride, uint64_t ye, uint64_t wh, uint64_t k,
                              uint64_t w, uint64_t out, uint64_t out_stride, uint64_t n, uint64_t rows, float eps,
                              uint64_t xq, uint64_t res);
/* No single counterpart in the reference (a decode fusion of src/gpu_model.rs:3383-3412 and 1950-2016): the MoE
 * combine of one token with the next norm and the GEMV that reads it, in one launch. x_out = x + res + sum_j wh[j]
 * ye[j] (slots j < k in order, rows of n = w->cols floats; res may be 0, k may be 0), then y = W h with h =
 * rms_norm(x_out) * nw quantized as Q8_K: the bits of strata_combine_rms_norm_q (strata_rms_norm_q with res when
 * k = 0) followed by strata_gemvq on its quantized output. x is only read (every block of the GEMV normalizes the row
 * itself), x_out (when not 0) is written, and must not overlap x, res or ye. One row of at most 2048 values (a multiple of 8),
 * k <= 8, 16-byte aligned rows, STRATA_NUM_Q8K; otherwise an error, and the caller makes the two calls. */
int strata_combine_rms_norm_gemv(strata_ctx* ctx, uint64_t x, uint64_t res, uint64_t ye, uint64_t wh, uint64_t k,
                                 uint64_t nw, float eps, const strata_tensor* w, uint64_t x_out, uint64_t y);
/* Backend::rms_norm_q of one row (src/backend.rs:233-235) followed by Backend::gemv of an F32 matrix on its output
 * (the decode's FFN norm and router logits, src/gpu_model.rs:3370-3383) in one launch: h = rms_norm(x + res) * nw
 * (strata_rms_norm_q's bits), xq its quantization (when not 0), y = w h (strata_gemv's bits for an F32 matrix of n
 * columns). x is NOT written: the caller adds res into x later (strata_combine_rms_norm_q takes it as its res).
 * n <= 2048, a multiple of 8, 16-byte aligned rows; otherwise an error. */
int strata_rms_norm_q_gemv_f32(strata_ctx* ctx, uint64_t x, uint64_t res, uint64_t nw, uint64_t h, uint64_t xq,
                               uint64_t n, float eps, const strata_tensor* w, uint64_t y);
/* Backend::swiglu_q (src/backend.rs:313-318; kernel src/cuda/kernels.cu:1826-1839): silu(g) * u over `rows` rows
 * of n floats, quantized into xq as strata_quant_xq does; g is left as is. *ret = xq (the address the following
 * GEMV reads). */
int strata_swiglu_q(strata_ctx* ctx, uint64_t g, uint64_t u, uint64_t n, uint64_t rows, uint64_t xq, uint64_t* ret);
/* Backend::moe_combine with mb = 0 (src/backend.rs:418-419; kernel src/cuda/kernels.cu:2742-2773): per token,
 * x += sum_{j<k, w[j] != 0} w[j] ye[j] (+ sigmoid(sg) sh, or + sh when sg is 0; sh 0 = no shared expert). */
int strata_moe_combine(strata_ctx* ctx, uint64_t x, uint64_t ye, uint64_t w, uint64_t k, uint64_t sh, uint64_t sg,
                       uint64_t n, uint64_t t);
/* Backend::moe_down_combine with mb = 0 (src/backend.rs:436-442): moe_gemv of the down experts (k slots per token,
 * x = h rows of cols, pre-quantized at xq when not 0) into ye, then moe_combine of ye into x with weights wh. With
 * xq and cols a multiple of 256 both run as one launch whose blocks each hold all k slots of some output rows (ye
 * is then not written); otherwise ye is the experts' outputs. Either way x gets the same bits. */
int strata_moe_down_combine(strata_ctx* ctx, int ty, uint64_t rows, uint64_t cols, uint64_t w, uint64_t stride,
                            uint64_t slots, uint64_t k, uint64_t h, uint64_t ye, uint64_t xq, uint64_t x, uint64_t wh,
                            uint64_t sh, uint64_t sg, uint64_t t);
/* Backend::swiglu_q followed by Backend::moe_down_combine with mb = 0 (src/backend.rs:313-318, 436-442; the decode
 * sequence src/gpu_model.rs:3383-3412) in one GEMV launch: the x row of slot j is silu(g[j]) * u[j] (t * k rows of
 * cols floats each, g and u with the same layout), quantized inside the down GEMV with swiglu_q's arithmetic (the same
 * int8 values and scales), then moe_combine of ye into x with weights wh. x = 0: the down GEMV into ye only (its
 * combine left to strata_combine_rms_norm_q). */
int strata_moe_down_swiglu_combine(strata_ctx* ctx, int ty, uint64_t rows, uint64_t cols, uint64_t w, uint64_t stride,
                                   uint64_t slots, uint64_t k, uint64_t g, uint64_t u, uint64_t ye, uint64_t x,
                                   uint64_t wh, uint64_t sh, uint64_t sg, uint64_t t);
/* Backend::moe_combine_seq (src/backend.rs:356; kernel src/cuda/kernels.cu:2776-2785): x[t] += sum_{j<k}
 * wts[t, j] ye[inv[t, j]] (+ sigmoid(sg[t]) sh[t], or + sh[t] when sg is 0; sh 0 = none), j in order. */
int strata_moe_combine_seq(strata_ctx* ctx, uint64_t x, uint64_t ye, uint64_t wts, uint64_t inv, uint64_t k,
                           uint64_t sh, uint64_t sg, uint64_t n, uint64_t t);

/* ---- prefill grouped GEMM ---- */

/* The host half of GpuModel's prefill MoE block moved onto the device (src/gpu_model/prefill.rs:554-575 and the
 * tile builder 618-642): sorts the (token, j) pairs by expert stably, writes off[n_expert + 1] (exclusive prefix counts),
 * xrow[t * k] (token of each sorted slot), inv[t * k] (slot of pair t * k + j), and for each of the n_mats
 * matrices m a tile list of 16-byte tiles [w_m(e), m0 | cnt << 32] (chunks of at most `chunk` slots per expert,
 * experts ascending, w_m(e) = bases[m] + e * strides[m]) at tiles + m * max_tiles * 16. chunk: 128 (0) is the
 * reference's GEMM_BM (src/backend.rs:16); strata_gemm_block_positions() (256) fills this backend's GEMM blocks.
 * The tile count is written to *n_tiles_dev (device int32). max_tiles must be at least t * k / chunk + n_expert.
 * No host synchronisation:
 * pass the same max_tiles and n_tiles_dev to strata_gemm_grouped. An id outside 0..n_expert is replaced by no
 * tile, counted in err_dev (device int32, may be 0), and the caller checks it after a sync (the reference fails the
 * prefill there, src/gpu_model/prefill.rs:557-560). */
int strata_moe_sort(strata_ctx* ctx, uint64_t ids, uint64_t t, uint64_t k, uint64_t n_expert, uint64_t off,
                    uint64_t xrow, uint64_t inv, uint64_t n_mats, const uint64_t* bases, const uint64_t* strides,
                    uint64_t tiles, uint64_t max_tiles, uint64_t n_tiles_dev, uint64_t err_dev, uint64_t chunk);
/* Backend::gemm (src/backend.rs:187-191): for each tile [w, m0 | cnt << 32] of the device tile list, positions
 * m0 .. m0 + cnt get y[m, 0..rows] (op) W x[xrow[m]] (x row m when xrow is 0), W the rows x cols matrix of type ty
 * at w. act: STRATA_ACT_STORE, STRATA_ACT_SWIGLU (y = silu(y) * result), STRATA_ACT_ADD, | STRATA_SAME_X (x is
 * unchanged since the previous gemm that read it: its int8 copy is reused) | STRATA_SMALL_TILES (the 64-position
 * GEMM form, for tiles of a few dozen positions; the same bits). n_x: rows of x the tiles read. A tile holds at most
 * strata_gemm_block_positions() (256) positions (the reference's host tiles hold at most GEMM_BM = 128,
 * src/backend.rs:16, src/gpu_model/prefill.rs:618-642); positions past 256 of a tile are not computed. cols must be a multiple of 256 (the reference needs 64,
 * src/cuda/mod.rs:584; every hot-path shape is a multiple of 256). */
int strata_gemm(strata_ctx* ctx, int ty, uint64_t rows, uint64_t cols, uint64_t tiles, uint64_t n_tiles, uint64_t x,
                uint64_t x_stride, uint64_t n_x, uint64_t xrow, uint64_t y, uint64_t y_stride, int act);
/* strata_gemm with the tile count read on the device from n_tiles_dev (at most max_tiles), as strata_moe_sort
 * leaves it: no host round trip between routing and the expert GEMMs. All max_tiles slots of the tile buffer must be
 * readable (the GEMM reads the tiles' sizes with the count to plan its blocks' work); slots past the count are
 * ignored. */
int strata_gemm_grouped(strata_ctx* ctx, int ty, uint64_t rows, uint64_t cols, uint64_t tiles, uint64_t max_tiles,
                        uint64_t n_tiles_dev, uint64_t x, uint64_t x_stride, uint64_t n_x, uint64_t xrow, uint64_t y,
                        uint64_t y_stride, int act);
/* The gate and up projections of the prefill MoE block in one grouped GEMM (src/gpu_model/prefill.rs: gemm of the
 * gate experts with act store, then of the up experts with act SwiGLU over the same tiles and X): for each tile the
 * up matrix is the gate matrix's address + up_offset bytes, and y[m, 0..rows) = silu(W_gate x) * (W_up x), the same
 * bits as the two calls. rows must be a multiple of 64, y rows 16-byte aligned; not for Q8_0. flags: STRATA_SAME_X,
 * STRATA_SMALL_TILES or 0, as in strata_gemm; max_tiles as in strata_gemm_grouped. */
int strata_gemm_grouped_gate_up(strata_ctx* ctx, int ty, uint64_t rows, uint64_t cols, uint64_t tiles,
                                uint64_t max_tiles, uint64_t n_tiles_dev, uint64_t x, uint64_t x_stride, uint64_t n_x,
                                uint64_t xrow, uint64_t y, uint64_t y_stride, int64_t up_offset, int flags);
/* Backend::gemm_dense (src/backend.rs:196): y[m] (op) W x[m] for m < n, one matrix (tiles of 128 positions,
 * src/cuda/mod.rs:908-910). */
int strata_gemm_dense(strata_ctx* ctx, const strata_tensor* w, uint64_t n, uint64_t x, uint64_t x_stride, uint64_t y,
                      uint64_t y_stride, int act);
/* Positions per block of this backend's GEMM (no counterpart in the reference): tile lists with chunks of this
 * size (strata_moe_sort's chunk) give every block a full tile. */
uint64_t strata_gemm_block_positions(void);
/* Backend::int8_gemm (src/backend.rs:192-194): 1 if gemm of type ty runs on int8 matrix cores (every supported
 * type does here), 0 for an unsupported type. */
int strata_int8_gemm(strata_ctx* ctx, int ty);
/* Backend::prequant_gemm_x (src/backend.rs:197): quantize x (n rows) ahead, for a later gemm with STRATA_SAME_X. */
int strata_prequant_gemm_x(strata_ctx* ctx, const strata_tensor* w, uint64_t n, uint64_t x, uint64_t x_stride);

/* ---- the decoder stack around the matmuls (src/backend.rs:232-410; the layer sequences of
 *      src/gpu_model/prefill.rs:315-712 and src/gpu_model.rs:1950-2016) ----
 * `step` arguments are device int32 arrays read at run time (so recorded graphs replay): prefill ops put token t of a
 * call at position step[0] + t; decode attention reads token t's position from step[2 t]. KV caches are f16 rows of
 * n_kv_head * head_dim values per position (Backend::kv_words: n words for n values). */

/* Backend::kv_words (src/backend.rs:186): u16 words of an f16 cache for n values. */
uint64_t strata_kv_words(uint64_t n);
/* Backend::argmax_rows (src/backend.rs:246; kernels src/cuda/kernels.cu:1574-1592): out[r] = index of the largest
 * value of row r (rows of n floats), the first on ties, under f32::total_cmp as ops::argmax (src/ops.rs:110-112). */
int strata_argmax_rows(strata_ctx* ctx, uint64_t x, uint64_t n, uint64_t rows, uint64_t out);
/* Backend::rope_pairs / rope_neox (src/backend.rs:250-254; ops::rope_neox src/ops.rs:36-45): in place on `heads`
 * rows `stride` floats apart, `per` heads a token, token t at position step[0] + t; pairs (i, i + n_rot / 2) for
 * lo <= i < hi turn by pos * base^(-2 i / n_rot) (f64 angle, f32 sine and cosine). */
int strata_rope_pairs(strata_ctx* ctx, uint64_t x, uint64_t stride, uint64_t heads, uint64_t per, uint64_t n_rot,
                      uint64_t step, float base, uint64_t lo, uint64_t hi);
int strata_rope_neox(strata_ctx* ctx, uint64_t x, uint64_t stride, uint64_t heads, uint64_t per, uint64_t n_rot,
                     uint64_t step, float base);
/* Backend::rms_norm_rope (src/backend.rs:267): rms_norm of `rows` heads of n (x rows x_stride apart, out rows of n)
 * with w, then rope_neox. n a multiple of 32 up to 512, n_rot <= n. */
int strata_rms_norm_rope(strata_ctx* ctx, uint64_t x, uint64_t x_stride, uint64_t w, uint64_t out, uint64_t n,
                         uint64_t rows, float eps, uint64_t per, uint64_t n_rot, uint64_t step, float base);
/* Backend::rms_norm_rope_kv (src/backend.rs:272; kernel src/cuda/kernels.cu:2196-2227): rms_norm_rope of the k heads,
 * then the normed, roped k head and its v row (v rows of n like out) stored as f16 into kc / vc at cache row
 * (position * per + head); kc = 0 stores nothing. */
int strata_rms_norm_rope_kv(strata_ctx* ctx, uint64_t x, uint64_t x_stride, uint64_t w, uint64_t out, uint64_t n,
                            uint64_t rows, float eps, uint64_t per, uint64_t n_rot, uint64_t step, float base,
                            uint64_t v, uint64_t kc, uint64_t vc);
/* Backend::rms_norm_rope_qk (src/backend.rs:274-277): rms_norm_rope of the q heads (qrows rows of q, q_stride apart,
 * into qo) and rms_norm_rope_kv of the k heads (rows of n), in one launch. */
int strata_rms_norm_rope_qk(strata_ctx* ctx, uint64_t q, uint64_t q_stride, uint64_t qw, uint64_t qo, uint64_t qrows,
                            uint64_t qper, uint64_t k, uint64_t kw, uint64_t ko, uint64_t krows, uint64_t kper, uint64_t n,
                            float eps, uint64_t n_rot, uint64_t step, float base, uint64_t v, uint64_t kc, uint64_t vc);
/* strata_rms_norm_rope_qk reading the heads from a fused q/k/v output (the prefill's one GEMM over a layer's q, k and
 * v rows): token t's query head h at q + t q_tstride + h q_stride, key head g at k + t k_tstride + g n, value row at
 * v + t v_tstride + g n (floats). Outputs (qo, ko) and the KV store as strata_rms_norm_rope_qk, the same bits. */
int strata_rms_norm_rope_qk_t(strata_ctx* ctx, uint64_t q, uint64_t q_tstride, uint64_t q_stride, uint64_t qw,
                              uint64_t qo, uint64_t qrows, uint64_t qper, uint64_t k, uint64_t k_tstride, uint64_t kw,
                              uint64_t ko, uint64_t krows, uint64_t kper, uint64_t n, float eps, uint64_t n_rot,
                              uint64_t step, float base, uint64_t v, uint64_t v_tstride, uint64_t kc, uint64_t vc);
/* Backend::kv_store (src/backend.rs:380; kernel src/cuda/kernels.cu:2181-2186): t tokens of n values (k and v
 * rows) into the f16 caches at positions step[0] ... */
int strata_kv_store(strata_ctx* ctx, uint64_t k, uint64_t v, uint64_t kc, uint64_t vc, uint64_t n, uint64_t t,
                    uint64_t step, uint64_t hd);
/* Backend::attn_prefill / attn_prefill_m with qm = 0 (src/backend.rs:337-343; kernel src/cuda/kernels.cu:2787-3216):
 * query row i of t (q rows of nh * hd floats, after norm and rope) at position step[0] + i attends to cached keys
 * 0 .. step[0] + i (the last `win` only when win > 0); out rows of nh * hd = softmax(q k scale) V, times
 * sigmoid(gate) when qg is not 0 (qg rows of nh * 2 hd, the gate at + hd per head), with a per-head sink logit when
 * sink is not 0. head_dim 64 or 128, nh / nkv in 1, 2, 4, 8. A QSA mask (qm != 0) is an error here. */
int strata_attn_prefill(strata_ctx* ctx, uint64_t q, uint64_t kc, uint64_t vc, uint64_t qg, uint64_t out, uint64_t step,
                        uint64_t t, uint64_t nh, uint64_t nkv, uint64_t hd, float scale);
int strata_attn_prefill_m(strata_ctx* ctx, uint64_t q, uint64_t kc, uint64_t vc, uint64_t qg, uint64_t out, uint64_t step,
                          uint64_t t, uint64_t nh, uint64_t nkv, uint64_t hd, float scale, uint64_t qm, uint64_t mw,
                          uint64_t sink, uint64_t win);
/* Floats of the `part` buffer attn_decode needs per token. */
uint64_t strata_attn_part_floats(uint64_t nh, uint64_t hd);
/* Backend::rms_norm_rope_kv of one decode token's heads (src/backend.rs:250-277: q heads normed with qw and roped,
 * the key head normed with kw, roped and stored with its value row into the f16 caches at row step[0] nkv + g)
 * followed by Backend::attn_decode_gq over the caches (src/backend.rs:383-410), as one launch: every block norms and
 * ropes the query heads it serves itself, and the block whose position split holds step[0] also builds that
 * position's key and value, stores them and uses them directly. q: nh raw heads q_stride floats apart; k, v: nkv raw
 * heads of hd floats; out and part as strata_attn_decode_gq (one token). The same bits as strata_rms_norm_rope_qk
 * with the KV store followed by strata_attn_decode_gq; q, k, v 16-byte aligned with strides of a multiple of 4.
 * xq (not 0; nh hd a multiple of 256): out also quantized as strata_quant_xq does, for the o projection's
 * strata_gemvq. */
int strata_rms_norm_rope_attn_decode(strata_ctx* ctx, uint64_t q, uint64_t q_stride, uint64_t qw, uint64_t k,
                                     uint64_t kw, uint64_t v, float eps, uint64_t n_rot, float base, uint64_t kc,
                                     uint64_t vc, uint64_t qg, uint64_t out, uint64_t part, uint64_t step, uint64_t nh,
                                     uint64_t nkv, uint64_t hd, float scale, uint64_t sink, uint64_t win, uint64_t xq);
/* Backend::attn_decode / attn_decode_gq (src/backend.rs:383-410; kernels src/cuda/kernels.cu:2123-2626): nt query
 * tokens (rows of q, qg and out per token), token t over positions 0 ..= step[2 t] (the last `win` when win > 0),
 * otherwise as strata_attn_prefill. part: nt * strata_attn_part_floats(nh, hd) floats of scratch. K / V loads are
 * always shared across the GQA group here (gq_min is accepted and ignored). */
int strata_attn_decode(strata_ctx* ctx, uint64_t q, uint64_t kc, uint64_t vc, uint64_t qg, uint64_t out, uint64_t part,
                       uint64_t step, uint64_t nh, uint64_t nkv, uint64_t hd, float scale, uint64_t nt);
int strata_attn_decode_gq(strata_ctx* ctx, uint64_t q, uint64_t kc, uint64_t vc, uint64_t qg, uint64_t out, uint64_t part,
                          uint64_t step, uint64_t nh, uint64_t nkv, uint64_t hd, float scale, int gq_min, uint64_t nt,
                          uint64_t sink, uint64_t win);
/* Backend::add (src/backend.rs:282): x += y over n floats. */
int strata_add(strata_ctx* ctx, uint64_t x, uint64_t y, uint64_t n);
/* Backend::swiglu (src/backend.rs:284): g = silu(g) * u over n floats. */
int strata_swiglu(strata_ctx* ctx, uint64_t g, uint64_t u, uint64_t n);
/* Model::embed on the device (src/model.rs:334-339; the reference dequantizes token rows on the host): out[i] = row
 * min(ids[i], rows - 1) of w as f32, for the n device int32 ids. No trait counterpart. */
int strata_get_rows(strata_ctx* ctx, const strata_tensor* w, uint64_t ids, uint64_t n, uint64_t out);
/* Synthetic weights on the device (no counterpart in the reference, whose tests build random tensors on the host,
 * tests/kernels.rs:1473-1550): fill the tensor's blocks with seeded random bytes, every f16 scale field (d, and dmin
 * where the type has one) set to a value in [lo, hi). The same seed gives the same bytes. */
int strata_fill_blocks(strata_ctx* ctx, const strata_tensor* w, uint64_t seed, float lo, float hi);

/* ---- weight quantizers (host) ----
 * The reference has none for these types (src/quant/mod.rs:1-2 only dequantizes). These make GGUF-valid blocks
 * from f32 rows, for synthetic weights: rows of `cols` values (a multiple of 256; 32 for Q8_0) into rows *
 * row_bytes bytes. Any valid packing serves: parity is checked on the bytes, whatever produced them. Supports
 * Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K and IQ4_XS. Threads over rows. */
int strata_quantize_rows(int ty, const float* src, uint64_t rows, uint64_t cols, uint8_t* dst);
/* Bytes of one row of `cols` values of type ty (GgmlType::row_bytes, src/quant/mod.rs:47); 0 if unsupported. */
uint64_t strata_row_bytes(int ty, uint64_t cols);

/* ---- measurement (no counterpart in the reference: its harness times with CUDA events, tests/kernels.rs:270-331) */

/* A HIP event recorded on the context's stream; elapsed milliseconds between two recorded events. */
int strata_event_create(strata_ctx* ctx, void** ev);
int strata_event_record(strata_ctx* ctx, void* ev);
int strata_event_elapsed(void* start, void* end, float* ms);
int strata_event_destroy(void* ev);
/* A plain streaming copy kernel (16-byte loads and stores) of `bytes` (a multiple of 16) from src to dst: the known-size
 * reference against which rocprofv3's FETCH_SIZE / WRITE_SIZE counters are scaled. */
int strata_copy_kernel(strata_ctx* ctx, uint64_t src, uint64_t dst, uint64_t bytes);
/* A plain streaming read of `bytes` (a multiple of 16) from src, 16-byte loads (sink: 256 bytes the kernel may write,
 * so the loads are not dropped); bytes = 0 is an empty launch. The floor a GEMV of the same bytes is compared with. */
int strata_read_kernel(strata_ctx* ctx, uint64_t src, uint64_t bytes, uint64_t sink);

#ifdef __cplusplus
}
#endif

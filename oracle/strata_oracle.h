/* CPU oracle for the quantized-matmul hot path: a C restatement of the reference's CPU algorithms.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library, the Python backend) links, loads or calls
 * this code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker or as
 * the timed CPU baseline. Each function names the reference file:line it restates.
 *
 * Type ids are GGUF/ggml ids (src/quant/mod.rs:15-19): Q8_0 8, Q2_K 10, Q3_K 11, Q4_K 12, Q5_K 13, Q6_K 14,
 * IQ2_XXS 16, IQ3_S 21, IQ4_XS 23. */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Q8_K activation block: src/cpu_moe.rs:13. */
typedef struct { float d; int8_t qs[256]; int16_t bs[16]; } or_q8k;

int or_block_elems(int ty);
int or_block_bytes(int ty);
float or_f16(uint16_t h);

/* dequant_row, src/quant/mod.rs:65-91. Returns 0, or -1 for a type the oracle does not cover. */
int or_dequant_row(int ty, const uint8_t* src, size_t n, float* dst);
/* quantize_q8k, src/cpu_moe.rs:28-46: ceil(n / 256) blocks, a short tail zero-padded. */
void or_quantize_q8k(const float* x, size_t n, or_q8k* out);
/* int_dot's scalar kernels, src/cpu_moe.rs:74-377 (dispatch 1364-1391, scalar branch 1390); with or_set_avx2(1) the
 * AVX2 kernels of oracle/cpu_avx2.c (branch 1389) for the types that have one. */
float or_int_dot(int ty, const uint8_t* row, size_t cols, const or_q8k* xq);
typedef float (*or_dot_fn)(const uint8_t* row, size_t cols, const or_q8k* xq);
/* The AVX2 dot of a type (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0), or null. */
or_dot_fn or_avx2_dot(int ty);
/* Select the dots or_int_dot (and so or_matvec and or_experts_multi) runs: 0 scalar (the default, the parity
 * checker), 1 AVX2 where available (the reference's timed path on x86-64-v3). Process-wide. */
void or_set_avx2(int on);
/* cpu_moe::matvec, src/cpu_moe.rs:1405-1420: threads over chunks of 32 rows (rayon par_chunks_mut(32)).
 * threads <= 0: all available. */
void or_matvec(int ty, const uint8_t* w, size_t rows, size_t cols, const float* x, float* y, int threads);
/* The reference GPU activation quantizer (quant8 without LLAMA_Q8, src/cuda/kernels.cu:640-685): nt rows of n
 * floats (row t at x + t * x_stride) into nt * n int8 followed by nt * n / 32 f32 scales. */
void or_quant_xq32(const float* x, size_t x_stride, size_t n, size_t nt, uint8_t* out);

/* Model::route, src/model.rs:837-851 (+ ops::softmax 18-24, ops::top_k 102-107, ops::sigmoid 15). */
void or_route(const float* logits, int n, int k, int sigmoid, float extra_scale, int32_t* ids, float* wts);
/* The prefill counting sort, src/gpu_model/prefill.rs:563-573: off[n_expert + 1], xrow[t * k], inv[t * k]. */
void or_sort_by_expert(const int32_t* ids, int t, int k, int n_expert, int32_t* off, int32_t* xrow, int32_t* inv);
/* moe_combine_seq, src/cuda/kernels.cu:2776-2785: x[t, d] += sum_j wts[t, j] ye[inv[t, j], d] (no shared expert). */
void or_combine_seq(float* x, const float* ye, const float* wts, const int32_t* inv, int k, int n, int t);
/* experts_multi, src/cpu_moe.rs:1483-1514, with every token's experts given by (ids, wts) rows of k and the three
 * expert-stacked matrices at gate / up / down (expert e at e * rows * row_bytes). ys[t] (n_embd floats) is
 * overwritten. Threads as in or_matvec. */
void or_experts_multi(int ty_gu, int ty_down, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                      int n_embd, int n_ff, const float* hs, int t, const int32_t* ids, const float* wts, int k,
                      float* ys, int threads);
/* ops::silu, src/ops.rs:14. */
float or_silu(float x);
void or_rms_norm(const float* x, const float* w, float eps, int n, float* out);

/* ---- the decoder stack around the hot path (oracle/attention.c) ---- */
/* ops::rope_neox, src/ops.rs:36-45, in place on one head. */
void or_rope_neox(float* x, int n_rot, long pos, float base);
/* ops::argmax, src/ops.rs:110-112. */
int or_argmax(const float* x, int n);
/* The attention of one token, Model::attention src/model.rs:771-793, over cells p0 .. p1 - 1. */
void or_attention(const float* q, const float* kc, const float* vc, int p0, int p1, int nh, int nkv, int hd,
                  float scale, const float* sinks, const float* gate, int gate_stride, float* out, float* sc);

#ifdef __cplusplus
}
#endif

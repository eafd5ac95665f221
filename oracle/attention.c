/* CPU oracle, attention-side functions of the decoder stack (TEST INFRASTRUCTURE ONLY: see strata_oracle.h).
 * Restates the reference's scalar f32 CPU math: ops::rope_neox (src/ops.rs:36-45), ops::argmax (src/ops.rs:110-112),
 * ops::softmax_sink (src/ops.rs:27-34), ops::sigmoid (src/ops.rs:15) and the per-token attention of
 * Model::attention (src/model.rs:747-795). Compiled with -ffp-contract=off: one rounding per C operation, as Rust. */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "strata_oracle.h"

/* ops::rope_neox, src/ops.rs:36-45: pairs (i, i + n_rot / 2); theta in f64, sin and cos rounded to f32. */
void or_rope_neox(float* x, int n_rot, long pos, float base) {
    int half = n_rot / 2;
    for (int i = 0; i < half; i++) {
        double theta = (double)pos * pow((double)base, -2.0 * (double)i / (double)n_rot);
        float s = (float)sin(theta), c = (float)cos(theta);
        float a = x[i], b = x[i + half];
        x[i] = a * c - b * s;
        x[i + half] = a * s + b * c;
    }
}

/* f32::total_cmp order (IEEE totalOrder) as a signed integer key. */
static int32_t total_key(float v) {
    int32_t b;
    memcpy(&b, &v, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

/* ops::argmax, src/ops.rs:110-112: the first index of the largest value under total_cmp. */
int or_argmax(const float* x, int n) {
    int b = 0;
    for (int i = 1; i < n; i++)
        if (total_key(x[i]) > total_key(x[b])) b = i;
    return b;
}

static float or_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* ops::softmax_sink, src/ops.rs:18-34 (has_sink 0: ops::softmax). */
static void softmax_sink(float* x, int n, int has_sink, float sink) {
    float m = has_sink ? sink : -INFINITY;
    for (int i = 0; i < n; i++) m = fmaxf(m, x[i]);
    float s = has_sink ? expf(sink - m) : 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - m);
        s += x[i];
    }
    for (int i = 0; i < n; i++) x[i] /= s;
}

/* The attention of one token in Model::attention, src/model.rs:771-793, after the q/k norms, rope and the cache
 * append: for each head i (kv head g = i / (nh / nkv)), scores over the cells p0 .. p1 - 1 (q . k summed in
 * dimension order, times scale), softmax (with the head's sink logit when sinks is not null), out = sum of p v in
 * cell order, times sigmoid(gate) when gate is not null (gate row of head i at gate + i * gate_stride).
 * kc / vc: rows of nkv * hd floats per position. sc: p1 - p0 floats of scratch. */
void or_attention(const float* q, const float* kc, const float* vc, int p0, int p1, int nh, int nkv, int hd,
                  float scale, const float* sinks, const float* gate, int gate_stride, float* out, float* sc) {
    int n = p1 - p0;
    for (int i = 0; i < nh; i++) {
        int g = i / (nh / nkv);
        const float* qh = q + (size_t)i * hd;
        for (int c = 0; c < n; c++) {
            const float* kt = kc + ((size_t)(p0 + c) * nkv + g) * hd;
            float s = 0.0f;
            for (int d = 0; d < hd; d++) s += qh[d] * kt[d];
            sc[c] = s * scale;
        }
        softmax_sink(sc, n, sinks != NULL, sinks ? sinks[i] : 0.0f);
        float* oh = out + (size_t)i * hd;
        for (int d = 0; d < hd; d++) oh[d] = 0.0f;
        for (int c = 0; c < n; c++) {
            const float* vt = vc + ((size_t)(p0 + c) * nkv + g) * hd;
            for (int d = 0; d < hd; d++) oh[d] += sc[c] * vt[d];
        }
        if (gate)
            for (int d = 0; d < hd; d++) oh[d] *= or_sigmoid(gate[(size_t)i * gate_stride + d]);
    }
}

"""The Qwen3-MoE decoder stack on this backend: the layer sequences of the reference's GpuModel for an attention +
routed-MoE model (chunked prefill, src/gpu_model/prefill.rs:315-712; one decode token, src/gpu_model.rs:1950-2016,
3100-3419), driven through the C ABI with every expert resident in HBM (no CPU offload, no mailbox).

Config 5 of the build is the Qwen3-30B-A3B shape (48 layers, hidden 2048, 32 query heads and 4 KV heads of 128,
128 experts, top-8, expert intermediate 768, vocabulary 151936) with a UD-Q2_K_XL-like type mix: Q2_K gate/up and
Q3_K down experts, Q6_K attention, Q8_0 token embeddings and output head, F32 norms and router. `Weights.random`
builds such a model from a seed on the device (random blocks with realistic scale fields); `Weights.from_host`
takes host arrays (tests build small models with them and check the device stack against the CPU oracle).

Per prefill chunk of t tokens at position pos (step[0] = pos):
    x = embed(tokens)
    per layer: h = rms_norm(x) ; q, k, v = gemm_dense(qkv, h) (one GEMM over the layer's q/k/v rows) ;
    rms_norm_rope_qk (q/k norms, NEOX rope, f16 KV store, reading the heads in place) ; attn_prefill (causal) ;
    x += gemm_dense(o, attn) ; h = rms_norm(x) ;
    logits = gemm_dense(router F32, h) ; router_topk ; moe_sort (on the device; 64-position tiles and the small-tile
    GEMM form when the chunk routes few rows to an expert) ; gate/up grouped GEMM with the SwiGLU epilogue ; down
    grouped GEMM ; x += moe_combine_seq.
Per decode token (recorded once as a graph and replayed; the step buffer carries the position):
    x = embed(token) ; per layer: x += mix + the previous layer's combine, h = rms_norm(x), q, k, v = W h as one
    launch (combine_rms_norm_gemv; x alternates between two rows) ; rms_norm_rope_qk with the
    KV store and attn_decode as one launch ; mix = gemvq(o) ; h, hq = rms_norm_q(x + mix) and logits = gemv(router, h) as one launch ;
    moe_route and the paired gate/up moe_gemv as one launch (moe_route_gemv) ; the down GEMV (moe_down_swiglu_combine, SwiGLU inside) ; its
    x += mix and the combine x += sum w y run with the next layer's attention norm and q/k/v GEMV ; then the
    output norm and output gemv (with the last of them, one launch), argmax_rows. Rows wider than 2048 values take
    the separate launches (combine_rms_norm_q, gemvq; rms_norm_q, gemv).
"""
import numpy as np

from . import ggml
from .backend import ACT_ADD, ACT_STORE, NUM_Q8K, X_Q, Buf, GpuTensor, StrataError


class Config:
    def __init__(self, n_layer=48, n_embd=2048, n_head=32, n_head_kv=4, head_dim=128, n_expert=128, n_expert_used=8,
                 n_ff_exp=768, n_vocab=151936, rope_base=1e6, eps=1e-6, ty_attn=ggml.Q6_K, ty_gate_up=ggml.Q2_K,
                 ty_down=ggml.Q3_K, ty_embd=ggml.Q8_0, ty_out=ggml.Q8_0):
        self.n_layer, self.n_embd, self.n_head, self.n_head_kv, self.head_dim = n_layer, n_embd, n_head, n_head_kv, head_dim
        self.n_expert, self.n_expert_used, self.n_ff_exp, self.n_vocab = n_expert, n_expert_used, n_ff_exp, n_vocab
        self.rope_base, self.eps = rope_base, eps
        self.ty_attn, self.ty_gate_up, self.ty_down, self.ty_embd, self.ty_out = ty_attn, ty_gate_up, ty_down, ty_embd, ty_out

    @classmethod
    def qwen3_30b_a3b(cls, n_layer=48):
        return cls(n_layer=n_layer)


# f16 scale ranges for random blocks whose values have a standard deviation near 0.02 (N(0, 0.02)-like weights):
# Q8_0 d q (q uniform int8, sd ~74 d); Q6_K d sc (q - 32) (sd ~1370 d); Q2_K d sc q - dmin m (sd ~12 d);
# Q3_K d (sc - 32) q3 (sd ~42 d).
SCALE = {ggml.Q8_0: (2.2e-4, 3.2e-4), ggml.Q6_K: (1.2e-5, 1.8e-5), ggml.Q2_K: (1.4e-3, 2.0e-3),
         ggml.Q3_K: (4.0e-4, 5.5e-4), ggml.Q4_K: (1.0e-3, 1.6e-3), ggml.Q5_K: (5e-4, 8e-4)}


class Layer:
    __slots__ = ("attn_norm", "qkv", "q", "k", "v", "q_norm", "k_norm", "o", "ffn_norm", "router", "gate_up", "down",
                 "e_gu", "e_down", "up_off")


class Weights:
    """Device tensors of the model. A layer's routed experts are the GGUF expert-stacked tensors (expert e of a matrix
    at e * rows * row_bytes): gate then up in one buffer (so the up matrix of every expert sits a fixed offset after
    its gate matrix, the pairing the fused gate/up kernels take), down in another."""

    def __init__(self, hip, cfg):
        self.hip, self.cfg = hip, cfg
        self.layers = []

    def strides(self):
        c = self.cfg
        return (ggml.row_bytes(c.ty_gate_up, c.n_embd) * c.n_ff_exp, ggml.row_bytes(c.ty_down, c.n_ff_exp) * c.n_embd)

    def _quant(self, ty, rows, cols, seed, buf=None, offset=0):
        t = GpuTensor(ty, rows, cols, buf if buf is not None else self.hip.alloc(rows * ggml.row_bytes(ty, cols)), offset)
        lo, hi = SCALE[ty]
        self.hip.fill_blocks(t, seed, lo, hi)
        return t

    @classmethod
    def random(cls, hip, cfg, seed=0):
        """A random-init model of cfg's shapes, built on the device from `seed` (the same seed, the same bytes)."""
        w = cls(hip, cfg)
        c = cfg
        rng = np.random.default_rng(seed)
        s = seed * 1000003
        w.embd = w._quant(c.ty_embd, c.n_vocab, c.n_embd, s + 1)
        w.output = w._quant(c.ty_out, c.n_vocab, c.n_embd, s + 2)
        w.output_norm = hip.upload((1.0 + 0.1 * rng.standard_normal(c.n_embd)).astype(np.float32))
        e_gu, e_down = w.strides()
        for il in range(c.n_layer):
            ly = Layer()
            b = s + 100 * (il + 1)
            ly.attn_norm = hip.upload((1.0 + 0.1 * rng.standard_normal(c.n_embd)).astype(np.float32))
            ly.ffn_norm = hip.upload((1.0 + 0.1 * rng.standard_normal(c.n_embd)).astype(np.float32))
            ly.q_norm = hip.upload((1.0 + 0.1 * rng.standard_normal(c.head_dim)).astype(np.float32))
            ly.k_norm = hip.upload((1.0 + 0.1 * rng.standard_normal(c.head_dim)).astype(np.float32))
            # q, k and v rows in one buffer (one GEMV serves all three in decode), each filled from its own seed
            nq, nkv = c.n_head * c.head_dim, c.n_head_kv * c.head_dim
            rb = ggml.row_bytes(c.ty_attn, c.n_embd)
            qkv = hip.alloc((nq + 2 * nkv) * rb)
            ly.q = w._quant(c.ty_attn, nq, c.n_embd, b + 1, qkv, 0)
            ly.k = w._quant(c.ty_attn, nkv, c.n_embd, b + 2, qkv, nq * rb)
            ly.v = w._quant(c.ty_attn, nkv, c.n_embd, b + 3, qkv, (nq + nkv) * rb)
            ly.qkv = GpuTensor(c.ty_attn, nq + 2 * nkv, c.n_embd, qkv)
            ly.o = w._quant(c.ty_attn, c.n_embd, c.n_head * c.head_dim, b + 4)
            ly.router = hip.upload_f32((0.02 * rng.standard_normal((c.n_expert, c.n_embd))).astype(np.float32))
            # gate and up stacks: 2 * n_expert matrices of n_ff_exp rows, one fill
            ly.gate_up = w._quant(c.ty_gate_up, 2 * c.n_expert * c.n_ff_exp, c.n_embd, b + 5).buf
            ly.down = w._quant(c.ty_down, c.n_expert * c.n_embd, c.n_ff_exp, b + 6).buf
            ly.e_gu, ly.e_down, ly.up_off = e_gu, e_down, c.n_expert * e_gu
            w.layers.append(ly)
        return w

    @classmethod
    def from_host(cls, hip, cfg, embd, output, output_norm, layers):
        """Upload host weights: layers = [dict(attn_norm, q, k, v, q_norm, k_norm, o, ffn_norm, router (f32
        [n_expert, n_embd]), gate, up, down (expert-stacked block bytes, expert e at e * rows * row_bytes))]."""
        w = cls(hip, cfg)
        c = cfg
        w.embd = hip.upload_tensor(c.ty_embd, embd)
        w.output = hip.upload_tensor(c.ty_out, output)
        w.output_norm = hip.upload(np.asarray(output_norm, np.float32))
        e_gu, e_down = w.strides()
        for L in layers:
            ly = Layer()
            ly.attn_norm = hip.upload(np.asarray(L["attn_norm"], np.float32))
            ly.ffn_norm = hip.upload(np.asarray(L["ffn_norm"], np.float32))
            ly.q_norm = hip.upload(np.asarray(L["q_norm"], np.float32))
            ly.k_norm = hip.upload(np.asarray(L["k_norm"], np.float32))
            ly.o = hip.upload_tensor(c.ty_attn, L["o"])
            qkv = [np.ascontiguousarray(L[n]) for n in ("q", "k", "v")]
            ly.qkv = hip.upload_tensor(c.ty_attn, np.concatenate(qkv))
            rb = qkv[0].shape[1]
            ly.q = GpuTensor(c.ty_attn, qkv[0].shape[0], c.n_embd, ly.qkv.buf, 0)
            ly.k = GpuTensor(c.ty_attn, qkv[1].shape[0], c.n_embd, ly.qkv.buf, qkv[0].shape[0] * rb)
            ly.v = GpuTensor(c.ty_attn, qkv[2].shape[0], c.n_embd, ly.qkv.buf, (qkv[0].shape[0] + qkv[1].shape[0]) * rb)
            ly.router = hip.upload_f32(L["router"])
            ly.gate_up = hip.upload(np.concatenate([np.ascontiguousarray(L["gate"]).reshape(-1),
                                                    np.ascontiguousarray(L["up"]).reshape(-1)]))
            ly.down = hip.upload(np.ascontiguousarray(L["down"]).reshape(-1))
            ly.e_gu, ly.e_down, ly.up_off = e_gu, e_down, c.n_expert * e_gu
            w.layers.append(ly)
        return w


class Model:
    """GpuModel for the Qwen3-MoE stack: KV caches for `ctx` positions, prefill chunks of up to `chunk` tokens (4096 by
    default, the reference's prefill chunk when it is not calibrated: src/main.rs:30,407)."""

    def __init__(self, hip, weights, ctx=4096 + 256, chunk=4096):
        self.hip, self.w, self.c = hip, weights, weights.cfg
        c = self.c
        self.ctx, self.chunk = ctx, chunk
        self.pos = 0
        kv = c.n_head_kv * c.head_dim
        # this model's f16 KV caches, one pair per layer (several models may share one Weights)
        self.kc = [hip.alloc(ctx * hip.kv_words(kv) * 2) for _ in weights.layers]
        self.vc = [hip.alloc(ctx * hip.kv_words(kv) * 2) for _ in weights.layers]
        self.step = hip.alloc(8)
        H, nh, hd, E, k, F = c.n_embd, c.n_head, c.head_dim, c.n_expert, c.n_expert_used, c.n_ff_exp
        n = chunk
        A = hip.alloc
        # prefill buffers (rows of the chunk)
        self.x = A(n * H * 4)
        self.x2 = A(H * 4)  # the decode's second hidden-state row
        self.h = A(n * H * 4)
        self.qkvp = A(n * (nh * hd + 2 * kv) * 4)  # the chunk's q, k and v rows from one GEMM
        self.hqp = A(n * (H + H // 8))  # h quantized by the norms (quant_xq layout), the GEMMs' X
        self.qb = A(n * nh * hd * 4)
        self.kk = A(n * kv * 4)
        self.att = A(n * nh * hd * 4)
        self.rl = A(n * E * 4)
        self.ids, self.wts = A(n * k * 4), A(n * k * 4)
        self.off, self.xrow, self.inv = A((E + 1) * 4), A(n * k * 4), A(n * k * 4)
        self.max_tiles = n * k // 64 + E  # room for the tile lists of either GEMM form (64 or 256 positions a tile)
        self.tiles, self.ntd, self.err = A(2 * self.max_tiles * 16), A(4), A(4)
        self.ge, self.ye = A(n * k * F * 4), A(n * k * H * 4)
        self.tok_in = A(n * 4)
        # decode buffers
        self.hq = A(H + H // 8)
        self.mix = A(H * 4)
        # the decode's q, k and v outputs of the one q/k/v GEMV, back to back
        self.dqkv = A((nh * hd + 2 * kv) * 4)
        self.dq, self.dk, self.dv = int(self.dqkv), int(self.dqkv) + 4 * nh * hd, int(self.dqkv) + 4 * (nh * hd + kv)
        self.dqo, self.dko = A(nh * hd * 4), A(kv * 4)
        self.aq = A(nh * hd + nh * hd // 8)  # the attention output quantized (quant_xq layout) for the o GEMV
        self.datt = A(nh * hd * 4)
        self.part = A(hip.attn_part_floats(nh, hd) * 4)
        self.dl = A(E * 4)
        self.dids, self.dwts, self.dslots, self.dwh = A(k * 4), A(k * 4), A(k * 4), A(k * 4)
        self.table = hip.upload(np.arange(E, dtype=np.int32))
        self.g2 = A(2 * k * F * 4)
        self.ye1 = A(k * H * 4)
        self.logits = A(c.n_vocab * 4)
        self.tok = A(4)
        self._graph = None  # the recorded decode token (this model's own: it holds this model's addresses)

    def reset(self):
        self.pos = 0

    def _set_step(self, pos):
        self.hip.htod(np.array([pos, 0], dtype=np.int32), self.step)

    # ---- prefill (src/gpu_model/prefill.rs:315-712) ----
    def prefill_chunk(self, tokens, layer_hook=None):
        """One chunk; layer_hook(il, x) (if given) runs after each layer with the chunk's hidden rows (a debugging and
        test probe, like the reference's STRATA_NAN_TRACE; it may read x, which syncs)."""
        hip, c, w = self.hip, self.c, self.w
        t = len(tokens)
        if t > self.chunk or t == 0:
            raise StrataError(f"prefill chunk of {t} tokens (1 to {self.chunk})")
        if self.pos + t > self.ctx:
            raise StrataError(f"context full ({self.ctx} tokens)")
        H, nh, nkv, hd, E, k, F = c.n_embd, c.n_head, c.n_head_kv, c.head_dim, c.n_expert, c.n_expert_used, c.n_ff_exp
        kv = nkv * hd
        hip.htod(np.asarray(tokens, dtype=np.int32), self.tok_in)
        self._set_step(self.pos)
        hip.get_rows(w.embd, self.tok_in, t, self.x)
        scale = 1.0 / np.sqrt(hd)
        if layer_hook:
            layer_hook(-1, self.x)
        for il, ly in enumerate(w.layers):
            # h quantized by the norm itself (X_Q: the GEMM takes it as is; the GEMM's X is always Q8_K numerics)
            xq_ok = hip.numerics() == NUM_Q8K
            hip.rms_norm_q(self.x, H, ly.attn_norm, self.h, H, H, t, c.eps, xq=self.hqp if xq_ok else 0)
            # q, k and v as one GEMM over the layer's q/k/v rows; the norms, rope and KV store read its heads in place
            qkv_n = nh * hd + 2 * kv
            if xq_ok:
                hip.gemm_dense(ly.qkv, t, self.hqp, H, self.qkvp, qkv_n, ACT_STORE | X_Q)
            else:
                hip.gemm_dense(ly.qkv, t, self.h, H, self.qkvp, qkv_n, ACT_STORE)
            hip.rms_norm_rope_qk_t(self.qkvp, qkv_n, hd, ly.q_norm, self.qb, t * nh, nh, int(self.qkvp) + 4 * nh * hd,
                                   qkv_n, ly.k_norm, self.kk, t * nkv, nkv, hd, c.eps, hd, self.step, c.rope_base,
                                   int(self.qkvp) + 4 * (nh * hd + kv), qkv_n, self.kc[il], self.vc[il])
            hip.attn_prefill(self.qb, self.kc[il], self.vc[il], 0, self.att, self.step, t, nh, nkv, hd, scale)
            hip.gemm_dense(ly.o, t, self.att, nh * hd, self.x, H, ACT_ADD)
            hip.rms_norm_q(self.x, H, ly.ffn_norm, self.h, H, H, t, c.eps, xq=self.hqp if xq_ok else 0)
            hip.gemm_dense(ly.router, t, self.h, H, self.rl, E, ACT_STORE)
            hip.router_topk(self.rl, E, k, 0.0, self.ids, self.wts, t)
            # few routed rows an expert (short chunks): 64-position tiles and the GEMM form for them
            tchunk, small = hip.moe_tile_plan(t, k, E)
            hip.moe_sort(self.ids, t, k, E, self.off, self.xrow, self.inv,
                         [(int(ly.gate_up), ly.e_gu), (int(ly.down), ly.e_down)], self.tiles, self.max_tiles,
                         self.ntd, err_dev=self.err, chunk=tchunk)
            hip.gemm_grouped_gate_up(c.ty_gate_up, F, H, self.tiles, self.max_tiles, self.ntd,
                                     self.hqp if xq_ok else self.h, H, t, self.xrow, self.ge, F, ly.up_off,
                                     flags=(X_Q if xq_ok else 0) | small)
            hip.gemm_grouped(c.ty_down, H, F, int(self.tiles) + self.max_tiles * 16, self.max_tiles, self.ntd, self.ge,
                             F, t * k, 0, self.ye, H, ACT_STORE | small)
            hip.moe_combine_seq(self.x, self.ye, self.wts, self.inv, k, 0, 0, H, t)
            if layer_hook:
                layer_hook(il, self.x)
        self.pos += t
        self.last_row = t - 1

    def prefill(self, tokens, layer_hook=None):
        """Chunked prefill (prefill_with, src/gpu_model/prefill.rs:135-163): the logits of the last token, and its
        greedy choice, on the device (logits, tok)."""
        for i in range(0, len(tokens), self.chunk):
            self.prefill_chunk(tokens[i:i + self.chunk], layer_hook)
        hip, c = self.hip, self.c
        H = c.n_embd
        last = int(self.x) + 4 * self.last_row * H
        hip.rms_norm(last, H, self.w.output_norm, self.h, H, H, 1, c.eps)
        hip.gemv(self.w.output, self.h, self.logits)
        hip.argmax_rows(self.logits, c.n_vocab, 1, self.tok)
        # the decode's hidden state starts from the last token's row (x row 0 of the decode buffers)
        return self.logits, self.tok

    # ---- decode (src/gpu_model.rs:1950-2016, 3100-3419) ----
    def _decode_ops(self):
        hip, c, w = self.hip, self.c, self.w
        H, nh, nkv, hd, E, k, F = c.n_embd, c.n_head, c.n_head_kv, c.head_dim, c.n_expert, c.n_expert_used, c.n_ff_exp
        kv = nkv * hd
        # the FFN norm and the router logits as one launch, and a layer's combine with the next norm and the GEMV
        # reading it as one launch, take rows of up to 2048 values (and at most 8 slots, Q8_K numerics)
        fused_router = H <= self.hip.RMS_NORM_GEMV_MAX
        fused_qkv = fused_router and k <= 8 and hip.numerics() == NUM_Q8K
        # the hidden state: in the fused form every q/k/v GEMV block reads x while block 0 writes x + mix + the
        # combine, so the layers alternate between two rows
        xs = [self.x, self.x2]
        cur = 0
        x = xs[cur]
        hip.get_rows(w.embd, self.tok, 1, x)
        for li, ly in enumerate(w.layers):
            if fused_qkv:
                # x (+ the previous layer's mix and combine, into the other row), this layer's attention norm and the
                # q/k/v GEMV in one launch (the bits of combine_rms_norm_q, or rms_norm_q, then gemvq)
                if li == 0:
                    hip.combine_rms_norm_gemv(x, 0, 0, 0, 0, ly.attn_norm, c.eps, ly.qkv, 0, self.dqkv)
                else:
                    hip.combine_rms_norm_gemv(x, self.mix, self.ye1, self.dwh, k, ly.attn_norm, c.eps, ly.qkv,
                                              xs[1 - cur], self.dqkv)
                    cur = 1 - cur
                    x = xs[cur]
            else:
                if li == 0:
                    hip.rms_norm_q(x, H, ly.attn_norm, self.h, H, H, 1, c.eps, xq=self.hq)
                else:  # the previous layer's x += mix, its combine (x += sum w y) and this layer's attention norm
                    hip.combine_rms_norm_q(x, self.ye1, self.dwh, k, ly.attn_norm, self.h, H, 1, c.eps, xq=self.hq,
                                           res=self.mix if fused_router else 0)
                hip.gemvq(ly.qkv, self.h, H, self.hq, self.dqkv, nh * hd + 2 * kv, 1)  # q, k and v in one launch
            # q/k norms, rope and the KV store inside the attention launch (the same bits as rms_norm_rope_qk with
            # the KV store, then attn_decode)
            hip.rms_norm_rope_attn_decode(self.dq, hd, ly.q_norm, self.dk, ly.k_norm, self.dv, c.eps, hd, c.rope_base,
                                          self.kc[li], self.vc[li], 0, self.datt, self.part, self.step, nh, nkv, hd,
                                          float(1.0 / np.sqrt(hd)), xq=self.aq)
            hip.gemvq(ly.o, self.datt, nh * hd, self.aq, self.mix, H, 1)  # x quantized by the attention's merge
            # h, hq = rms_norm_q(x + mix) and the router logits in one launch (x += mix is left to the next
            # combine_rms_norm_q, which adds mix before the combine: the same bits)
            if fused_router:
                hip.rms_norm_q_gemv_f32(x, self.mix, ly.ffn_norm, self.h, self.hq, H, c.eps, ly.router, self.dl)
            else:  # rows too wide for the fused launch: x += mix here, the norm, then the router GEMV (the same bits)
                hip.rms_norm_q(x, H, ly.ffn_norm, self.h, H, H, 1, c.eps, xq=self.hq, res=self.mix)
                hip.gemv(ly.router, self.h, self.dl)
            # the route inside the gate/up GEMV launch (moe_route then moe_gemv, the same bits)
            hip.moe_route_gemv(self.dl, E, k, 0.0, self.table, self.dids, self.dwts, self.dslots, self.dwh,
                               c.ty_gate_up, F, H, ly.gate_up, ly.e_gu, self.h, self.g2, pair=(ly.up_off, k * F * 4),
                               xq=self.hq)
            # the down GEMV (SwiGLU quantized inside) into ye1; its combine runs with the next norm
            hip.moe_down_swiglu_combine(c.ty_down, H, F, ly.down, ly.e_down, self.dslots, k, self.g2,
                                        int(self.g2) + k * F * 4, self.ye1, 0, self.dwh, 0, 0, 1)
        if fused_qkv:
            hip.combine_rms_norm_gemv(x, self.mix, self.ye1, self.dwh, k, w.output_norm, c.eps, w.output, 0,
                                      self.logits)
        else:
            hip.combine_rms_norm_q(x, self.ye1, self.dwh, k, w.output_norm, self.h, H, 1, c.eps,
                                   res=self.mix if fused_router else 0)
            hip.gemv(w.output, self.h, self.logits)
        hip.argmax_rows(self.logits, c.n_vocab, 1, self.tok)

    def decode_step(self, graph=True):
        """One greedy token from the token in self.tok at position self.pos: the decode ops (recorded once as a graph
        and replayed) leave the next token in self.tok and its logits in self.logits."""
        if self.pos >= self.ctx:
            raise StrataError(f"context full ({self.ctx} tokens)")
        self._set_step(self.pos)
        if graph:
            if self._graph is None:
                # the graph keeps every buffer it addresses alive (the weights with their KV caches, this model's
                # scratch) until it is destroyed
                keep = [self.w] + self.kc + self.vc + [v for v in vars(self).values() if isinstance(v, Buf)]
                self._graph = self.hip.record_graph(self._decode_ops, keep)
            self._graph.launch()
        else:
            self._decode_ops()
        self.pos += 1

    def close(self):
        """Destroy the recorded decode graph (it is also destroyed when the model is collected)."""
        if self._graph is not None:
            self._graph.close()
            self._graph = None

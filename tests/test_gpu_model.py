"""The Qwen3-MoE decoder stack (rustingstrata_amd/qwen3moe.py: chunked prefill and graph-replayed greedy decode)
against the reference's per-token CPU forward restated from the oracle's pieces: Model::attention
(src/model.rs:747-795) with q/k norms and NEOX rope, the expert FFN of cpu_moe::experts_multi
(src/cpu_moe.rs:1483-1514) with Model::route, and cpu_moe::matvec for every quantized matrix (the Q8_K activations
the device path uses too). The KV cache holds f16 values as on the device.

A small model (2 layers, hidden 512, 4 query heads over 2 KV heads of 64, 8 experts top-2) keeps the CPU side fast;
the prefill runs in three chunks, so chunk boundaries and cache positions are exercised.

Two kinds of check. Layer by layer, teacher-forced: the oracle layer runs on the device's own input rows; nine rows
in ten must agree to rel-L2 1e-5 (they land near 1e-7) and every row to 2e-2. Each op alone is bit-exact or within
1e-6 in the op tests, but inside a layer the activations are requantized to int8 four times, and a last-bit
difference of an f32 norm or sum (the device sums a norm's squares as a tree, the CPU in index order) moves an int8
value by one step now and then, which moves that row's outputs by up to about 1e-2 of their scale. End to end over
the prompt and the decode tokens, where those steps compound through the layers and the attention over all earlier
tokens: logits within rel-L2 5e-2, and the same greedy token wherever the oracle's top two logits are clearly apart.
A wiring mistake (a wrong head, position, cache row, expert or residual) misses these by orders of magnitude.
"""
import numpy as np
import pytest

from oracle import oracle as O
from rustingstrata_amd import ggml
from rustingstrata_amd.qwen3moe import Config, Model, Weights
from tests.helpers import random_blocks, rel_l2

pytestmark = pytest.mark.gpu


def small_cfg():
    return Config(n_layer=2, n_embd=512, n_head=4, n_head_kv=2, head_dim=64, n_expert=8, n_expert_used=2,
                  n_ff_exp=256, n_vocab=300)


def host_weights(c, seed):
    rng = np.random.default_rng(seed)
    sc = {ggml.Q8_0: (2.2e-4, 3.2e-4), ggml.Q6_K: (1.2e-5, 1.8e-5), ggml.Q2_K: (1.4e-3, 2.0e-3),
          ggml.Q3_K: (4.0e-4, 5.5e-4)}
    rb = lambda ty, rows, cols, s: random_blocks(ty, rows, cols, seed=s, scale=sc[ty])
    norm = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    layers = []
    for il in range(c.n_layer):
        b = seed + 100 * (il + 1)
        layers.append(dict(attn_norm=norm(c.n_embd), ffn_norm=norm(c.n_embd), q_norm=norm(c.head_dim),
                           k_norm=norm(c.head_dim),
                           q=rb(c.ty_attn, c.n_head * c.head_dim, c.n_embd, b + 1),
                           k=rb(c.ty_attn, c.n_head_kv * c.head_dim, c.n_embd, b + 2),
                           v=rb(c.ty_attn, c.n_head_kv * c.head_dim, c.n_embd, b + 3),
                           o=rb(c.ty_attn, c.n_embd, c.n_head * c.head_dim, b + 4),
                           router=(0.05 * rng.standard_normal((c.n_expert, c.n_embd))).astype(np.float32),
                           gate=rb(c.ty_gate_up, c.n_expert * c.n_ff_exp, c.n_embd, b + 5),
                           up=rb(c.ty_gate_up, c.n_expert * c.n_ff_exp, c.n_embd, b + 6),
                           down=rb(c.ty_down, c.n_expert * c.n_embd, c.n_ff_exp, b + 7)))
    return dict(embd=rb(c.ty_embd, c.n_vocab, c.n_embd, seed + 1), output=rb(c.ty_out, c.n_vocab, c.n_embd, seed + 2),
                output_norm=norm(c.n_embd), layers=layers)


class RefModel:
    """The per-token CPU forward (Model::step_embed_h's attention + MoE layers) from the oracle's functions."""

    def __init__(self, c, W):
        self.c, self.W = c, W
        self.kcl = [[] for _ in range(c.n_layer)]
        self.vcl = [[] for _ in range(c.n_layer)]
        self.pos = 0

    def layer(self, il, x, pos, kc, vc):
        """Layer il for one token at position pos; kc / vc: the layer's cache rows so far (appended to)."""
        c, L = self.c, self.W["layers"][il]
        H, nh, nkv, hd = c.n_embd, c.n_head, c.n_head_kv, c.head_dim
        h = O.rms_norm(x, L["attn_norm"], c.eps)[0]
        q = O.matvec(c.ty_attn, L["q"], nh * hd, H, h)
        k = O.matvec(c.ty_attn, L["k"], nkv * hd, H, h)
        v = O.matvec(c.ty_attn, L["v"], nkv * hd, H, h)
        qn = np.concatenate([O.rope_neox(O.rms_norm(q[i * hd:(i + 1) * hd], L["q_norm"], c.eps)[0], hd, pos,
                                         c.rope_base)[0] for i in range(nh)])
        kn = np.concatenate([O.rope_neox(O.rms_norm(k[i * hd:(i + 1) * hd], L["k_norm"], c.eps)[0], hd, pos,
                                         c.rope_base)[0] for i in range(nkv)])
        kc.append(kn.astype(np.float16).astype(np.float32))  # the device cache is f16
        vc.append(v.astype(np.float16).astype(np.float32))
        att = O.attention(qn, np.stack(kc), np.stack(vc), 0, pos + 1, nh, nkv, hd, float(1 / np.sqrt(hd)))
        x = x + O.matvec(c.ty_attn, L["o"], H, nh * hd, att)
        h = O.rms_norm(x, L["ffn_norm"], c.eps)[0]
        logits = np.cumsum(L["router"] * h[None, :], axis=1, dtype=np.float32)[:, -1]
        ids, wts = O.route(logits[None, :], c.n_expert_used)
        return x + O.experts_multi(c.ty_gate_up, c.ty_down, L["gate"], L["up"], L["down"], H, c.n_ff_exp, h[None, :],
                                   ids, wts)[0]

    def step(self, tok):
        c, W = self.c, self.W
        H, nh, nkv, hd = c.n_embd, c.n_head, c.n_head_kv, c.head_dim
        x = O.dequant(c.ty_embd, W["embd"][min(tok, c.n_vocab - 1)], H)
        for il in range(c.n_layer):
            x = self.layer(il, x, self.pos, self.kcl[il], self.vcl[il])
        self.pos += 1
        h = O.rms_norm(x, W["output_norm"], c.eps)[0]
        return O.matvec(c.ty_out, W["output"], c.n_vocab, H, h)


def check_logits(got, want, tol=5e-2):
    assert rel_l2(got, want) <= tol, rel_l2(got, want)
    top = np.sort(want)[::-1]
    if top[0] - top[1] > 2 * tol * np.abs(want).max():
        assert int(np.argmax(got)) == O.argmax(want)


def stage_check(c, L, x, p, mid, xout, kc, vc, tol=1e-5):
    """One layer at position p, teacher-forced stage by stage on the device's own intermediate rows (mid: q after its
    norm and rope, the attention output, the FFN norm's h, the routed ids and weights; kc / vc: the layer's f16 KV
    cache rows as f32), each stage against the oracle within rel-L2 tol (ids exactly, weights within 1e-6): the
    q projection with the q norm and rope (Model::attention's q), the attention over the device's cache
    (src/model.rs:771-793), the o projection and the FFN norm, the route (Model::route on the F32 router's sequential
    sums), and the expert FFN (cpu_moe::experts_multi) added to the layer's residual."""
    H, nh, nkv, hd, k = c.n_embd, c.n_head, c.n_head_kv, c.head_dim, c.n_expert_used
    h = O.rms_norm(x, L["attn_norm"], c.eps)[0]
    q = O.matvec(c.ty_attn, L["q"], nh * hd, H, h)
    qn = np.concatenate([O.rope_neox(O.rms_norm(q[i * hd:(i + 1) * hd], L["q_norm"], c.eps)[0], hd, p,
                                     c.rope_base)[0] for i in range(nh)])
    assert rel_l2(mid["q"], qn) <= tol, ("q", p, rel_l2(mid["q"], qn))
    att = O.attention(mid["q"], kc[:p + 1], vc[:p + 1], 0, p + 1, nh, nkv, hd, float(1 / np.sqrt(hd)))
    assert rel_l2(mid["att"], att) <= tol, ("attention", p, rel_l2(mid["att"], att))
    x2 = x + O.matvec(c.ty_attn, L["o"], H, nh * hd, mid["att"])
    h2 = O.rms_norm(x2, L["ffn_norm"], c.eps)[0]
    assert rel_l2(mid["h"], h2) <= tol, ("ffn norm", p, rel_l2(mid["h"], h2))
    lg = np.cumsum(L["router"] * mid["h"][None, :], axis=1, dtype=np.float32)[:, -1]
    rid, rw = O.route(lg[None, :], k)
    assert np.array_equal(mid["ids"], rid[0]), ("route", p)
    assert np.abs(mid["wts"] - rw[0]).max() <= 1e-6, ("route weights", p)
    y = O.experts_multi(c.ty_gate_up, c.ty_down, L["gate"], L["up"], L["down"], H, c.n_ff_exp, mid["h"][None, :],
                        mid["ids"][None, :], mid["wts"][None, :])[0]
    assert rel_l2(xout, x2 + y) <= tol, ("experts", p, rel_l2(xout, x2 + y))


def mid_rows(hip, m, c, n):
    """The prefill's intermediate rows of the layer just run (n chunk rows): q, attention, FFN-norm h, ids, weights."""
    nh, hd, k, H = c.n_head, c.head_dim, c.n_expert_used, c.n_embd
    return dict(q=hip.get(m.qb, np.float32, n * nh * hd).reshape(n, nh * hd),
                att=hip.get(m.att, np.float32, n * nh * hd).reshape(n, nh * hd),
                h=hip.get(m.h, np.float32, n * H).reshape(n, H),
                ids=hip.get(m.ids, np.int32, n * k).reshape(n, k), wts=hip.get(m.wts, np.float32, n * k).reshape(n, k))


CFGS = {
    "small": small_cfg,
    # the configs[4] head shape: head_dim 128, 8 query heads over each KV head
    "hd128_gqa8": lambda: Config(n_layer=2, n_embd=1024, n_head=16, n_head_kv=2, head_dim=128, n_expert=16,
                                 n_expert_used=4, n_ff_exp=256, n_vocab=300),
    # a hidden size past the fused FFN-norm + router launch (its unfused form)
    "wide4096": lambda: Config(n_layer=1, n_embd=4096, n_head=4, n_head_kv=2, head_dim=64, n_expert=8,
                               n_expert_used=2, n_ff_exp=256, n_vocab=300),
}


@pytest.mark.parametrize("name", list(CFGS))
def test_prefill_chunks_and_decode_match_cpu_forward(hip, name):
    c = CFGS[name]()
    W = host_weights(c, seed=7)
    weights = Weights.from_host(hip, c, W["embd"], W["output"], W["output_norm"], W["layers"])
    m = Model(hip, weights, ctx=128, chunk=32)
    prompt = np.random.default_rng(3).integers(0, c.n_vocab, 70).tolist()
    ref = RefModel(c, W)
    for tok in prompt:
        want = ref.step(tok)
    logits, tok = m.prefill(prompt)
    got = hip.get(logits, np.float32, c.n_vocab)
    check_logits(got, want)
    next_tok = int(hip.get(tok, np.int32, 1)[0])
    assert next_tok == int(np.argmax(got))
    for i in range(5):
        want = ref.step(next_tok)
        m.decode_step(graph=i > 0)  # the first token eagerly, then graph replays
        got = hip.get(m.logits, np.float32, c.n_vocab)
        check_logits(got, want)
        next_tok = int(hip.get(m.tok, np.int32, 1)[0])
        assert next_tok == int(np.argmax(got))
    m.close()


def test_layers_teacher_forced(hip):
    """Each layer of the device prefill (two chunks) against the oracle layer run on the device's own input rows."""
    c = small_cfg()
    W = host_weights(c, seed=11)
    weights = Weights.from_host(hip, c, W["embd"], W["output"], W["output_norm"], W["layers"])
    m = Model(hip, weights, ctx=128, chunk=24)
    prompt = np.random.default_rng(4).integers(0, c.n_vocab, 40).tolist()
    rows, mids = {}, {}
    chunk_no = [0]

    def hook(il, x):
        n = min(24, 40 - 24 * chunk_no[0])
        rows[(chunk_no[0], il)] = hip.get(x, np.float32, n * c.n_embd).reshape(n, c.n_embd)
        if il >= 0:
            mids[(chunk_no[0], il)] = mid_rows(hip, m, c, n)
        if il == c.n_layer - 1:
            chunk_no[0] += 1

    m.prefill(prompt, layer_hook=hook)
    ref = RefModel(c, W)
    kv = c.n_head_kv * c.head_dim
    for il in range(c.n_layer):
        kc, vc, errs = [], [], []
        kcd = hip.get(m.kc[il], np.float16, 40 * kv).astype(np.float32).reshape(40, kv)
        vcd = hip.get(m.vc[il], np.float16, 40 * kv).astype(np.float32).reshape(40, kv)
        for ch in range(2):
            xin, xout = rows[(ch, il - 1)], rows[(ch, il)]
            for r in range(xin.shape[0]):
                # every stage of every row from the device's own intermediate rows: within 1e-5
                stage_check(c, W["layers"][il], xin[r], 24 * ch + r, {key: v[r] for key, v in mids[(ch, il)].items()},
                            xout[r], kcd, vcd)
                want = ref.layer(il, xin[r].copy(), 24 * ch + r, kc, vc)
                errs.append(rel_l2(xout[r], want))
        errs = np.array(errs)
        # the whole layer from the same input row: a requantized int8 value (of the attention output, of h, of a
        # SwiGLU row) that lands one step over moves a row by up to ~1e-2 of its scale, now and then
        assert np.mean(errs <= 1e-5) >= 0.9 and errs.max() <= 2e-2, (il, errs)


def test_random_model_full_shape_runs(hip):
    """The config-5 shapes (two of the 48 layers, full vocabulary): a 300-token prefill and 3 decode tokens run and
    give finite logits, and the graph replay of a token equals its eager run."""
    c = Config.qwen3_30b_a3b(n_layer=2)
    w = Weights.random(hip, c, seed=1)
    m = Model(hip, w, ctx=512, chunk=256)
    logits, tok = m.prefill(np.random.default_rng(0).integers(0, c.n_vocab, 300).tolist())
    assert np.isfinite(hip.get(logits, np.float32, c.n_vocab)).all()
    start_pos, start_tok = m.pos, hip.get(tok, np.int32, 1)
    m.decode_step(graph=False)
    eager = hip.get(m.logits, np.float32, c.n_vocab)
    assert np.isfinite(eager).all()
    # replay the same token at the same position through the recorded graph: the same bits
    m.pos = start_pos
    hip.htod(start_tok, m.tok)
    m.decode_step(graph=True)
    assert np.array_equal(hip.get(m.logits, np.float32, c.n_vocab), eager)
    m.close()


def test_models_in_sequence_keep_their_own_graphs(hip):
    """Each model records its own decode graph and destroys it with itself: models built one after another on one
    backend (no drop_graphs between them, so a later model may reuse an earlier one's addresses) decode the same tokens
    as an eager run."""
    import gc
    c = small_cfg()
    W = host_weights(c, seed=7)
    weights = Weights.from_host(hip, c, W["embd"], W["output"], W["output_norm"], W["layers"])
    prompt = np.random.default_rng(5).integers(0, c.n_vocab, 20).tolist()

    def run(graph):
        m = Model(hip, weights, ctx=64, chunk=32)
        m.prefill(prompt)
        toks = []
        for _ in range(4):
            m.decode_step(graph=graph)
            toks.append(int(hip.get(m.tok, np.int32, 1)[0]))
        return toks, hip.get(m.logits, np.float32, c.n_vocab)

    want_toks, want_logits = run(False)
    for _ in range(3):
        toks, logits = run(True)
        gc.collect()
        assert toks == want_toks and np.array_equal(logits, want_logits)


def test_config4_full_workload(hip):
    """configs[4] at its workload: the 48-layer Qwen3-30B-A3B-shaped random model, a 4096-token uniform-random prompt
    prefilled, then 128 greedy decode tokens.

    * The prompt in one chunk of 4096 and in two of 2048 gives the same logits and KV caches, bit for bit (per-token
      results do not depend on the chunking: every grouped-GEMM output keeps the CPU's per-super-block order, and the
      attention rows sum their keys in one fixed order).
    * 128 decode tokens replayed from the recorded graph equal 128 eager tokens (tokens and last logits, bit for bit),
      and every logit is finite.
    * Layers 0 and 47 at sampled prompt positions, teacher-forced stage by stage on the device's own intermediate rows
      (the oracle's Model::attention, cpu_moe::matvec, Model::route and cpu_moe::experts_multi): q after its norm and
      rope, the attention output, the FFN norm's h, the routed ids and weights, the layer output. At full shape the
      attention output (f32 from f16 MFMA, ~1e-6 off the CPU's) is requantized to int8 for the o projection, and over
      4096 values about one of them lands on the other side of a rounding step per row; the layer output amplifies
      such a step (the expert FFN's own requantizations), so the whole layer from the same input row is held to
      rel-L2 5e-2 while every stage from the device's own rows is held to 1e-5."""
    from rustingstrata_amd.qwen3moe import Config
    c = Config.qwen3_30b_a3b()
    w = Weights.random(hip, c, seed=5)
    prompt = np.random.default_rng(6).integers(0, c.n_vocab, 4096).tolist()
    H, nh, nkv, hd, E, k = c.n_embd, c.n_head, c.n_head_kv, c.head_dim, c.n_expert, c.n_expert_used
    kv = nkv * hd
    pos = (1, 63, 1000, 2047, 2048, 3001, 4095)
    xin, xout, mid = {}, {}, {}

    def rows_of(buf, width, dtype=np.float32):
        return np.stack([hip.get(buf, dtype, width, at=p * width) for p in pos])

    def hook(il, x):
        if il in (-1, 46):
            xin[il + 1] = rows_of(x, H)
        if il in (0, 47):
            xout[il] = rows_of(x, H)
            mid[il] = dict(q=rows_of(a.qb, nh * hd), att=rows_of(a.att, nh * hd), h=rows_of(a.h, H),
                           ids=rows_of(a.ids, k, np.int32), wts=rows_of(a.wts, k))

    a = Model(hip, w, ctx=4096 + 160, chunk=4096)
    la, ta = a.prefill(prompt, layer_hook=hook)
    logits_a = hip.get(la, np.float32, c.n_vocab)
    assert np.isfinite(logits_a).all()
    b = Model(hip, w, ctx=4096 + 160, chunk=2048)
    lb, tb = b.prefill(prompt)
    assert np.array_equal(hip.get(lb, np.float32, c.n_vocab), logits_a)
    for il in (0, 47):
        assert np.array_equal(hip.get(a.kc[il], np.uint16, 4096 * kv), hip.get(b.kc[il], np.uint16, 4096 * kv)), il
        assert np.array_equal(hip.get(a.vc[il], np.uint16, 4096 * kv), hip.get(b.vc[il], np.uint16, 4096 * kv)), il

    # 128 greedy tokens: a from its graph, b eagerly
    toks_a, toks_b = [], []
    for i in range(128):
        a.decode_step(graph=True)
        b.decode_step(graph=False)
        toks_a.append(int(hip.get(a.tok, np.int32, 1)[0]))
        toks_b.append(int(hip.get(b.tok, np.int32, 1)[0]))
    la_last = hip.get(a.logits, np.float32, c.n_vocab)
    assert toks_a == toks_b
    assert np.isfinite(la_last).all() and np.array_equal(la_last, hip.get(b.logits, np.float32, c.n_vocab))

    def host(t):
        return hip.get(t.buf, np.uint8, t.bytes(), at=t.ptr - int(t.buf)).reshape(t.rows, -1)

    e_gu, e_down = w.strides()
    for il in (0, 47):
        ly = w.layers[il]
        f32 = lambda buf, n: hip.get(buf, np.float32, n)
        gu = hip.get(ly.gate_up, np.uint8, 2 * E * e_gu)
        L = dict(attn_norm=f32(ly.attn_norm, H), ffn_norm=f32(ly.ffn_norm, H), q_norm=f32(ly.q_norm, hd),
                 k_norm=f32(ly.k_norm, hd), q=host(ly.q), k=host(ly.k), v=host(ly.v), o=host(ly.o),
                 router=hip.get(ly.router.buf, np.float32, E * H).reshape(E, H),
                 gate=gu[:E * e_gu], up=gu[E * e_gu:], down=hip.get(ly.down, np.uint8, E * e_down))
        layers = [None] * c.n_layer
        layers[il] = L
        ref = RefModel(c, dict(layers=layers))
        kc = hip.get(a.kc[il], np.float16, 4096 * kv).astype(np.float32).reshape(4096, kv)
        vc = hip.get(a.vc[il], np.float16, 4096 * kv).astype(np.float32).reshape(4096, kv)
        M = mid[il]
        for j, p in enumerate(pos):
            x = xin[il][j]
            stage_check(c, L, x, p, {key: v[j] for key, v in M.items()}, xout[il][j], kc, vc)
            # the whole layer from the same input row (and its own key and value rows against the cache)
            kl, vl = list(kc[:p]), list(vc[:p])
            want = ref.layer(il, x.copy(), p, kl, vl)
            assert np.abs(kl[p] - kc[p]).max() <= 1e-3 * np.abs(kc[p]).max(), (il, p)
            assert np.abs(vl[p] - vc[p]).max() <= 1e-3 * np.abs(vc[p]).max(), (il, p)
            assert rel_l2(xout[il][j], want) <= 5e-2, (il, p, rel_l2(xout[il][j], want))
    a.close()
    b.close()

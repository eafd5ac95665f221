"""GPU parity of the decoder-stack ops around the matmuls (config 5's layer: norms with rope and the KV store,
attention, argmax, the F32 router matmuls, embedding rows) through the C ABI, against the CPU oracle's restatement
of the reference's CPU math (ops::rope_neox, ops::rms_norm, ops::argmax, Model::attention).

The KV cache is f16 on the device (the reference GPU's cache format), so the attention oracle reads the same
f16-rounded K and V; outputs then agree within the 1e-3 max relative error bar (they land near 1e-6).
"""
import numpy as np
import pytest

import rustingstrata_amd as S
from oracle import oracle as O
from rustingstrata_amd import ggml
from tests.helpers import max_rel_err, normal, random_blocks, rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-3


def up(hip, a):
    return hip.upload(np.ascontiguousarray(a))


def i32(hip, v):
    return up(hip, np.asarray(v, dtype=np.int32))


def test_argmax_rows_total_order(hip):
    rows, n = 4, 151936
    x = normal((rows, n), seed=1)
    x[1, 77] = x[1, 99] = 9.0                  # tie: the first wins
    x[2, :] = -0.0
    x[2, 500] = 0.0                            # +0 above -0
    x[3, 1234] = np.inf
    x[3, 2000] = np.nan                        # a positive NaN above everything (total_cmp)
    out = hip.alloc(rows * 4)
    hip.argmax_rows(up(hip, x), n, rows, out)
    got = hip.get(out, np.int32, rows)
    want = [O.argmax(x[r]) for r in range(rows)]
    assert got.tolist() == want == [want[0], 77, 500, 2000]


def test_rope_neox_and_pairs(hip):
    nh, hd, T, pos0 = 32, 128, 5, 3000
    x = normal((T * nh, hd), seed=2)
    xb = up(hip, x)
    step = i32(hip, [pos0, 0])
    hip.rope_neox(xb, hd, T * nh, nh, hd, step, 1e6)
    got = hip.get(xb, np.float32, T * nh * hd).reshape(T * nh, hd)
    want = np.concatenate([O.rope_neox(x[r], hd, pos0 + r // nh, 1e6) for r in range(T * nh)])
    assert max_rel_err(got, want) <= 1e-6
    assert np.mean(got == want) > 0.999
    # pairs 10..40 only, the rest untouched
    xb = up(hip, x)
    hip.rope_pairs(xb, hd, T * nh, nh, hd, step, 1e6, 10, 40)
    got = hip.get(xb, np.float32, T * nh * hd).reshape(T * nh, hd)
    untouched = np.r_[0:10, 40:64, 64:74, 104:128]
    assert np.array_equal(got[:, untouched], x[:, untouched])
    assert max_rel_err(got[:, 10:40], want[:, 10:40]) <= 1e-6


@pytest.mark.parametrize("T", [3, 12])
def test_rms_norm_rope_qk_and_kv_store(hip, T):
    """rms_norm_rope_qk (src/backend.rs:274-277): q heads normed and roped; k heads normed, roped and stored with
    their v rows as f16 at cache row position * nkv + head. T = 3 runs the wave-per-head kernel, T = 12 (432 heads,
    a partial last block) the lane-per-head sums of the many-heads kernel; both also reading the heads in place from
    fused q/k/v rows (rms_norm_rope_qk_t)."""
    nh, nkv, hd, pos0, eps = 32, 4, 128, 17, 1e-6
    q = normal((T, nh * hd), seed=3)
    k = normal((T, nkv * hd), seed=4)
    v = normal((T, nkv * hd), seed=5)
    qw, kw = normal(hd, seed=6) * 0.5 + 1, normal(hd, seed=7) * 0.5 + 1
    P = 40
    kc, vc = hip.alloc(P * nkv * hd * 2), hip.alloc(P * nkv * hd * 2)
    qo, ko = hip.alloc(T * nh * hd * 4), hip.alloc(T * nkv * hd * 4)
    hip.rms_norm_rope_qk(up(hip, q), hd, up(hip, qw), qo, T * nh, nh, up(hip, k), up(hip, kw), ko, T * nkv, nkv, hd,
                         eps, hd, i32(hip, [pos0, 0]), 1e6, up(hip, v), kc, vc)
    want_q = np.stack([O.rope_neox(O.rms_norm(q.reshape(-1, hd)[r], qw, eps)[0], hd, pos0 + r // nh, 1e6)[0]
                       for r in range(T * nh)])
    want_k = np.stack([O.rope_neox(O.rms_norm(k.reshape(-1, hd)[r], kw, eps)[0], hd, pos0 + r // nkv, 1e6)[0]
                       for r in range(T * nkv)])
    got_q = hip.get(qo, np.float32, T * nh * hd).reshape(-1, hd)
    got_k = hip.get(ko, np.float32, T * nkv * hd).reshape(-1, hd)
    # the norm sums in the CPU's order: the same bits but for the rare rope angle whose f64 sine or cosine rounds
    # to another f32
    assert max_rel_err(got_q, want_q) <= 1e-6 and max_rel_err(got_k, want_k) <= 1e-6
    assert np.mean(got_q == want_q) > 0.999 and np.mean(got_k == want_k) > 0.999
    kcache = hip.get(kc, np.uint16, P * nkv * hd).reshape(P, nkv * hd)
    vcache = hip.get(vc, np.uint16, P * nkv * hd).reshape(P, nkv * hd)
    assert np.array_equal(kcache[pos0:pos0 + T].reshape(-1), got_k.astype(np.float16).view(np.uint16).reshape(-1))
    assert np.array_equal(vcache[pos0:pos0 + T], v.astype(np.float16).view(np.uint16))
    assert not kcache[:pos0].any() and not kcache[pos0 + T:].any()
    # the same heads read in place from one fused q/k/v row per token (rms_norm_rope_qk_t): the same bits
    W = nh * hd + 2 * nkv * hd
    qkv = up(hip, np.concatenate([q, k, v], axis=1))
    kc3, vc3 = hip.alloc(P * nkv * hd * 2), hip.alloc(P * nkv * hd * 2)
    qo3, ko3 = hip.alloc(T * nh * hd * 4), hip.alloc(T * nkv * hd * 4)
    hip.rms_norm_rope_qk_t(qkv, W, hd, up(hip, qw), qo3, T * nh, nh, int(qkv) + 4 * nh * hd, W, up(hip, kw), ko3,
                           T * nkv, nkv, hd, eps, hd, i32(hip, [pos0, 0]), 1e6, int(qkv) + 4 * (nh + nkv) * hd, W,
                           kc3, vc3)
    assert np.array_equal(hip.get(qo3, np.uint32, T * nh * hd), got_q.reshape(-1).view(np.uint32))
    assert np.array_equal(hip.get(ko3, np.uint32, T * nkv * hd), got_k.reshape(-1).view(np.uint32))
    assert np.array_equal(hip.get(kc3, np.uint16, P * nkv * hd), kcache.reshape(-1))
    assert np.array_equal(hip.get(vc3, np.uint16, P * nkv * hd), vcache.reshape(-1))
    with pytest.raises(S.StrataError, match="token stride"):
        hip.rms_norm_rope_qk_t(qkv, 8, hd, up(hip, qw), qo3, T * nh, nh, int(qkv), W, up(hip, kw), ko3, T * nkv, nkv,
                               hd, eps, hd, i32(hip, [pos0, 0]), 1e6, int(qkv), W, kc3, vc3)
    # kv_store of the same rows at another position: the same f16 bits
    kc2, vc2 = hip.alloc(P * nkv * hd * 2), hip.alloc(P * nkv * hd * 2)
    hip.kv_store(ko, up(hip, v), kc2, vc2, nkv * hd, T, i32(hip, [5, 0]), hd)
    k2 = hip.get(kc2, np.uint16, P * nkv * hd).reshape(P, nkv * hd)
    assert np.array_equal(k2[5:5 + T], kcache[pos0:pos0 + T])


def attention_f64(q, kf, vf, p0, p1, nh, nkv, hd, scale):
    """The same attention in f64 (no sink, no gate): the accuracy yardstick for long position ranges, where the CPU
    oracle's own f32 sums drift."""
    out = np.empty(nh * hd)
    for i in range(nh):
        g = i // (nh // nkv)
        s = kf[p0:p1, g * hd:(g + 1) * hd].astype(np.float64) @ q[i * hd:(i + 1) * hd].astype(np.float64) * scale
        p = np.exp(s - s.max())
        out[i * hd:(i + 1) * hd] = p @ vf[p0:p1, g * hd:(g + 1) * hd].astype(np.float64) / p.sum()
    return out


def f16_cache(rng, P, width, scale=1.0):
    return (rng.standard_normal((P, width)) * scale).astype(np.float16)


@pytest.mark.parametrize("nh,nkv,hd", [(32, 4, 128), (8, 8, 64), (16, 4, 64)])
@pytest.mark.parametrize("positions", [1, 37, 300, 4096])
def test_attn_decode_matches_cpu_attention(hip, nh, nkv, hd, positions):
    rng = np.random.default_rng(positions + nh)
    P, nt = positions + 3, 2
    kc16, vc16 = f16_cache(rng, P, nkv * hd, 1.5), f16_cache(rng, P, nkv * hd)
    q = normal((nt, nh * hd), seed=positions)
    steps = [positions - 1, 0, max(positions - 2, 0), 0]   # token t over 0 ..= step[2 t]
    out = hip.alloc(nt * nh * hd * 4)
    part = hip.alloc(nt * hip.attn_part_floats(nh, hd) * 4)
    scale = 1.0 / np.sqrt(hd)
    hip.attn_decode(up(hip, q), up(hip, kc16), up(hip, vc16), 0, out, part, i32(hip, steps), nh, nkv, hd, scale, nt)
    got = hip.get(out, np.float32, nt * nh * hd).reshape(nt, nh * hd)
    kf, vf = kc16.astype(np.float32), vc16.astype(np.float32)
    for t in range(nt):
        want = O.attention(q[t], kf, vf, 0, steps[2 * t] + 1, nh, nkv, hd, scale)
        assert max_rel_err(got[t], want) <= TOL, (t, max_rel_err(got[t], want))
        # at least as close to the f64 attention as the f32 CPU path is
        exact = attention_f64(q[t], kf, vf, 0, steps[2 * t] + 1, nh, nkv, hd, scale)
        assert rel_l2(got[t], exact) <= max(1e-6, 2 * rel_l2(want, exact)), (t, rel_l2(got[t], exact), rel_l2(want, exact))


def test_attn_decode_sink_gate_window(hip):
    nh, nkv, hd, P = 32, 4, 128, 500
    rng = np.random.default_rng(9)
    kc16, vc16 = f16_cache(rng, P, nkv * hd), f16_cache(rng, P, nkv * hd)
    q = normal((1, nh * hd), seed=10)
    qg = normal((1, nh * 2 * hd), seed=11)
    sink = normal(nh, seed=12) + 2
    out = hip.alloc(nh * hd * 4)
    part = hip.alloc(hip.attn_part_floats(nh, hd) * 4)
    win, pos = 128, 450
    hip.attn_decode(up(hip, q), up(hip, kc16), up(hip, vc16), up(hip, qg), out, part, i32(hip, [pos, 0]), nh, nkv, hd,
                    0.1, 1, sink=up(hip, sink), win=win)
    got = hip.get(out, np.float32, nh * hd)
    kf, vf = kc16.astype(np.float32), vc16.astype(np.float32)
    want = O.attention(q[0], kf, vf, pos + 1 - win, pos + 1, nh, nkv, hd, 0.1, sinks=sink, gate=qg[0, hd:],
                       gate_stride=2 * hd)
    assert max_rel_err(got, want) <= TOL and rel_l2(got, want) <= 1e-6


@pytest.mark.parametrize("nh,nkv,hd,pos,n_rot,win,extras", [(32, 4, 128, 4099, 128, 0, False), (32, 4, 128, 63, 128, 0, True),
                                                         (8, 8, 64, 0, 64, 0, False), (16, 4, 64, 300, 32, 0, False),
                                                         (32, 4, 128, 450, 128, 128, True), (16, 8, 128, 64, 128, 0, False)])
def test_rms_norm_rope_attn_decode_equals_unfused(hip, nh, nkv, hd, pos, n_rot, win, extras):
    """rms_norm_rope_attn_decode (the q/k norms, rope and KV store inside the attention launch) gives the attention
    output and the caches bit-equal to rms_norm_rope_qk with the KV store followed by attn_decode
    (src/backend.rs:250-277, 383-410): positions at a split edge (63, 64), the first (0), a partial rope (n_rot 32),
    a window with sink and gate, GQA groups 1, 2, 4 and 8; and the output against the CPU attention over the caches."""
    rng = np.random.default_rng(pos + nh + hd)
    P = pos + 5
    kc16, vc16 = f16_cache(rng, P, nkv * hd, 1.5), f16_cache(rng, P, nkv * hd)
    qkv = normal(nh * hd + 2 * nkv * hd, seed=pos + 1)
    qw = np.random.default_rng(pos + 2).uniform(0.5, 1.5, hd).astype(np.float32)
    kw = np.random.default_rng(pos + 3).uniform(0.5, 1.5, hd).astype(np.float32)
    xb, qwb, kwb = up(hip, qkv), up(hip, qw), up(hip, kw)
    q, k, v = int(xb), int(xb) + 4 * nh * hd, int(xb) + 4 * (nh + nkv) * hd
    step = i32(hip, [pos, 0])
    qg = up(hip, normal(nh * 2 * hd, seed=pos + 4)) if extras else 0
    sink = up(hip, normal(nh, seed=pos + 5) + 2) if extras else 0
    kc1, vc1, kc2, vc2 = up(hip, kc16), up(hip, vc16), up(hip, kc16), up(hip, vc16)
    qo, ko = hip.alloc(nh * hd * 4), hip.alloc(nkv * hd * 4)
    o1, o2 = hip.alloc(nh * hd * 4), hip.alloc(nh * hd * 4)
    part = hip.alloc(hip.attn_part_floats(nh, hd) * 4)
    scale, eps, base = 1.0 / np.sqrt(hd), 1e-6, 1e6
    hip.rms_norm_rope_qk(q, hd, qwb, qo, nh, nh, k, kwb, ko, nkv, nkv, hd, eps, n_rot, step, base, v, kc1, vc1)
    hip.attn_decode(qo, kc1, vc1, qg, o1, part, step, nh, nkv, hd, scale, 1, sink=sink, win=win)
    aq = hip.alloc(nh * hd + nh * hd // 8)
    hip.rms_norm_rope_attn_decode(q, hd, qwb, k, kwb, v, eps, n_rot, base, kc2, vc2, qg, o2, part, step, nh, nkv, hd,
                                  scale, sink=sink, win=win, xq=aq)
    # the output quantized by the merge: quant_xq's bits
    aq2 = hip.alloc(nh * hd + nh * hd // 8)
    hip.quant_xq(o2, nh * hd, nh * hd, 1, aq2)
    assert np.array_equal(hip.get(aq, np.uint8, nh * hd + nh * hd // 8), hip.get(aq2, np.uint8, nh * hd + nh * hd // 8))
    m = P * nkv * hd
    assert np.array_equal(hip.get(kc1, np.uint16, m), hip.get(kc2, np.uint16, m))
    assert np.array_equal(hip.get(vc1, np.uint16, m), hip.get(vc2, np.uint16, m))
    g1, g2 = hip.get(o1, np.float32, nh * hd), hip.get(o2, np.float32, nh * hd)
    assert np.array_equal(g1.view(np.uint32), g2.view(np.uint32)), int((g1 != g2).sum())
    if not extras:
        kf = hip.get(kc2, np.uint16, m).view(np.float16).astype(np.float32).reshape(P, nkv * hd)
        vf = hip.get(vc2, np.uint16, m).view(np.float16).astype(np.float32).reshape(P, nkv * hd)
        want = O.attention(hip.get(qo, np.float32, nh * hd), kf, vf, 0, pos + 1, nh, nkv, hd, scale)
        assert max_rel_err(g2, want) <= TOL


def prefill_case(hip, nh, nkv, hd, T, pos0, seed, rows=None, sink=None, gate=False, win=0):
    """Runs the prefill and checks the given rows: within 1e-3 max relative error of the CPU attention (or of the
    CPU's own distance from the f64 attention, whichever is larger: long, diffuse rows average V down to small
    outputs where f32 rounding of either side shows), and at least as close to the f64 attention as the CPU is."""
    rng = np.random.default_rng(seed)
    P = pos0 + T
    kc16, vc16 = f16_cache(rng, P, nkv * hd, 1.5), f16_cache(rng, P, nkv * hd)
    q = normal((T, nh * hd), seed=seed + 1)
    qg = normal((T, nh * 2 * hd), seed=seed + 2) if gate else None
    out = hip.alloc(T * nh * hd * 4)
    scale = 1.0 / np.sqrt(hd)
    hip.attn_prefill(up(hip, q), up(hip, kc16), up(hip, vc16), 0 if qg is None else up(hip, qg), out,
                     i32(hip, [pos0, 0]), T, nh, nkv, hd, scale, sink=0 if sink is None else up(hip, sink), win=win)
    got = hip.get(out, np.float32, T * nh * hd).reshape(T, nh * hd)
    kf, vf = kc16.astype(np.float32), vc16.astype(np.float32)
    worst = 0.0
    for i in (range(T) if rows is None else rows):
        p1 = pos0 + i + 1
        p0 = max(p1 - win, 0) if win else 0
        want = O.attention(q[i], kf, vf, p0, p1, nh, nkv, hd, scale, sinks=sink,
                           gate=None if qg is None else qg[i, hd:], gate_stride=2 * hd)
        err = max_rel_err(got[i], want)
        worst = max(worst, err)
        if sink is None and qg is None:
            exact = attention_f64(q[i], kf, vf, p0, p1, nh, nkv, hd, scale)
            assert err <= max(TOL, 2 * max_rel_err(want, exact)), (i, err, max_rel_err(want, exact))
            assert rel_l2(got[i], exact) <= max(1e-6, 2 * rel_l2(want, exact)), (i, rel_l2(got[i], exact))
        else:
            assert err <= TOL, (i, err)
    return worst


@pytest.mark.parametrize("nh,nkv,hd,T,pos0", [(32, 4, 128, 333, 0), (32, 4, 128, 100, 77), (8, 8, 64, 65, 3),
                                              (16, 4, 64, 1, 10), (4, 2, 128, 130, 0)])
def test_attn_prefill_matches_cpu_attention(hip, nh, nkv, hd, T, pos0):
    """Causal prefill over the f16 cache: query i at position pos0 + i sees keys 0 .. pos0 + i; f16 MFMA with split,
    power-of-two-scaled operands keeps the outputs at the f32 CPU attention's own rounding level."""
    prefill_case(hip, nh, nkv, hd, T, pos0, seed=T + pos0)


def test_attn_prefill_sink_gate_window(hip):
    sink = normal(32, seed=20) + 1
    prefill_case(hip, 32, 4, 128, 150, 40, seed=21, sink=sink, gate=True, win=64)


def test_attn_prefill_full_size(hip):
    """configs[4]'s layer shape at its full prompt: 4096 tokens, 32 query heads over 4 KV heads of 128; rows sampled
    over the whole triangle (every 64th, plus the last)."""
    rows = list(range(0, 4096, 64)) + [4095]
    prefill_case(hip, 32, 4, 128, 4096, 0, seed=30, rows=rows)


def test_f32_gemv_and_gemm_dense(hip):
    """The router's F32 weights (ffn_gate_inp, 128 x 2048): gemv (1 and 3 inputs) and gemm_dense (act store / add)
    against the f64 products (f32 sums of 2048 products: within 1e-4)."""
    E, H, T = 128, 2048, 300
    w = normal((E, H), seed=40, std=0.02)
    x = normal((T, H), seed=41)
    t = hip.upload_f32(w)
    xb = up(hip, x)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    y = hip.alloc(3 * E * 4)
    hip.gemv(t, xb, y)
    assert max_rel_err(hip.get(y, np.float32, E), want[0]) <= 1e-4
    hip.gemvn(t, xb, H, y, E, 3)
    assert max_rel_err(hip.get(y, np.float32, 3 * E).reshape(3, E), want[:3]) <= 1e-4
    yy = hip.alloc(T * E * 4)
    hip.gemm_dense(t, T, xb, H, yy, E, S.ACT_STORE)
    got = hip.get(yy, np.float32, T * E).reshape(T, E)
    # gemm_dense sums each dot in index order as Tensor::matvec's f32 iterator sum (src/weights.rs:29-37): the CPU's
    # bits (np.cumsum over float32 products is that sequential sum)
    seq = np.stack([np.cumsum(w * x[m][None, :], axis=1, dtype=np.float32)[:, -1] for m in range(T)])
    assert np.array_equal(got.view(np.uint32), seq.view(np.uint32)), int((got != seq).sum())
    assert max_rel_err(got, want) <= 1e-3
    hip.gemm_dense(t, T, xb, H, yy, E, S.ACT_ADD)
    assert np.array_equal(hip.get(yy, np.float32, T * E).reshape(T, E), seq + seq)


@pytest.mark.parametrize("ty", [ggml.Q8_0, ggml.Q6_K, ggml.Q2_K])
def test_get_rows_is_dequant_of_the_rows(hip, ty):
    rows, cols = 1000, 2048
    w = random_blocks(ty, rows, cols, seed=50 + ty)
    t = hip.upload_tensor(ty, w)
    ids = np.array([0, 999, 5, 5, 123456, 42], dtype=np.int32)   # past the end: the last row (Model::embed's min)
    out = hip.alloc(len(ids) * cols * 4)
    hip.get_rows(t, i32(hip, ids), len(ids), out)
    got = hip.get(out, np.float32, len(ids) * cols).reshape(len(ids), cols)
    for i, r in enumerate(np.minimum(ids, rows - 1)):
        assert np.array_equal(got[i].view(np.uint32), O.dequant(ty, w[r], cols).view(np.uint32)), i


def test_fill_blocks_seeded(hip):
    ty, rows, cols = ggml.Q4_K, 64, 2048
    rb = ggml.row_bytes(ty, cols)
    a, b = hip.alloc(rows * rb), hip.alloc(rows * rb)
    ta, tb = S.GpuTensor(ty, rows, cols, a), S.GpuTensor(ty, rows, cols, b)
    hip.fill_blocks(ta, 7, 0.01, 0.02)
    hip.fill_blocks(tb, 7, 0.01, 0.02)
    x, y = hip.get(a, np.uint8, rows * rb), hip.get(b, np.uint8, rows * rb)
    assert np.array_equal(x, y)
    blk = x.reshape(-1, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)
    assert d.min() >= 0.0099 and d.max() <= 0.0201
    hip.fill_blocks(tb, 8, 0.01, 0.02)
    assert not np.array_equal(hip.get(b, np.uint8, rows * rb), x)
    # the bytes between the scale fields are spread over all values
    assert len(np.unique(blk[:, 16:])) == 256


def test_add_and_swiglu(hip):
    g, u = normal(1000, seed=60), normal(1000, seed=61)
    gb, ub = up(hip, g), up(hip, u)
    hip.swiglu(gb, ub, 1000)
    want = np.array([O.silu(v) for v in g], dtype=np.float32) * u
    assert max_rel_err(hip.get(gb, np.float32, 1000), want) <= 1e-6
    hip.add(gb, ub, 1000)
    assert max_rel_err(hip.get(gb, np.float32, 1000), want + u) <= 1e-6


def test_decoder_ops_reject_shapes(hip):
    b = hip.alloc(1 << 16)
    with pytest.raises(S.StrataError, match="head_dim 96"):
        hip.attn_decode(b, b, b, 0, b, b, b, 32, 4, 96, 0.1, 1)
    with pytest.raises(S.StrataError, match="GQA group of 16"):
        hip.attn_prefill(b, b, b, 0, b, b, 4, 32, 2, 128, 0.1)
    with pytest.raises(S.StrataError, match="n_rot 200"):
        hip.rms_norm_rope(b, 128, b, b, 128, 4, 1e-6, 4, 200, b, 1e6)

"""The CPU oracle pinned against the reference's own golden vectors and against what the mathematics fixes.

Reference-held vectors: tests/golden/reference/ holds copies of the reference's dequant fixtures
(tests/fixtures/{Q2_K,Q3_K,Q4_K,Q5_K,Q6_K,Q8_0,IQ4_XS}.{raw,f32}, written by gguf-py; and
tools/deepseek_ref/dequant/{q5_k,q8_0,iq2_xxs}.{blk,f32}, written by ggml's to_float). IQ3_S has no reference-held
vector: it is pinned here by a hand-built known-answer block and by the dot/dequant cross-check below.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O
from rustingstrata_amd import ggml
from tests.helpers import random_blocks

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference")


def xs(n):
    """tests/kernels.rs:7-9: ((i * 0.7548777).fract() - 0.5) * 2 in f32."""
    v = np.arange(n, dtype=np.float32) * np.float32(0.7548777)
    return ((v - np.trunc(v)) - np.float32(0.5)) * np.float32(2.0)


@pytest.mark.parametrize("name,ty", [("Q2_K", ggml.Q2_K), ("Q3_K", ggml.Q3_K), ("Q4_K", ggml.Q4_K), ("Q5_K", ggml.Q5_K),
                                     ("Q6_K", ggml.Q6_K), ("Q8_0", ggml.Q8_0), ("IQ4_XS", ggml.IQ4_XS)])
def test_dequant_matches_gguf_py_fixtures(name, ty):
    raw = np.fromfile(os.path.join(GOLD, f"{name}.raw"), dtype=np.uint8)
    want = np.fromfile(os.path.join(GOLD, f"{name}.f32"), dtype=np.float32)
    assert raw.size == ggml.row_bytes(ty, want.size)
    got = O.dequant(ty, raw, want.size)
    # tests/quant.rs:12-14 accepts 1e-6 * max(|w|, 1); the oracle reproduces the vectors bit for bit.
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), np.abs(got - want).max()


@pytest.mark.parametrize("name,ty", [("q5_k", ggml.Q5_K), ("q8_0", ggml.Q8_0), ("iq2_xxs", ggml.IQ2_XXS)])
def test_dequant_matches_ggml_fixtures(name, ty):
    blk = np.fromfile(os.path.join(GOLD, f"ggml_{name}.blk"), dtype=np.uint8)
    want = np.fromfile(os.path.join(GOLD, f"ggml_{name}.f32"), dtype=np.float32)
    got = O.dequant(ty, blk, want.size)
    # tests/quant_ggml.rs:11-12: exact.
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_iq3s_oracle_vectors_stable():
    """tests/golden/oracle/IQ3_S.{raw,f32} (written by tests/golden/make_oracle_vectors.py; oracle-derived, not
    reference-held): the oracle still reproduces them bit for bit, and every value is db * grid * sign with
    db = d (1 + 2 sc) over the odd grid bytes 1..15 (src/quant/mod.rs:345-361)."""
    d = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle")
    raw = np.fromfile(os.path.join(d, "IQ3_S.raw"), dtype=np.uint8)
    want = np.fromfile(os.path.join(d, "IQ3_S.f32"), dtype=np.float32)
    got = O.dequant(ggml.IQ3_S, raw, want.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    blk = raw.reshape(-1, 110)
    dd = blk[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    for b in range(blk.shape[0]):
        for ib in range(8):
            sc = (blk[b, 106 + ib // 2] >> (4 * (ib & 1))) & 15
            db = np.float32(dd[b] * np.float32(1 + 2 * int(sc)))
            q = np.abs(want[256 * b + 32 * ib:256 * b + 32 * ib + 32]) / db
            assert np.all(np.isin(np.round(q), np.arange(1, 16, 2))), (b, ib)


def test_iq3s_known_answer():
    """A hand-built IQ3_S block (layout src/quant/mod.rs:345-361): d = 0.5, sub-block 0 scale nibble 3 -> db = 3.5;
    qs[0] = 0 -> IQ3S_GRID[0] = 0x01010101 (four 1s); qs[1] = 5 with qh bit 1 set -> index 256 + 5; sign byte 0 of
    sub-block 0 = 0b0000_0101 (elements 0 and 2 negated); sub-block 1 scale nibble 0 -> db = 0.5."""
    from tests.iq_tables import IQ3S_GRID
    b = np.zeros(110, dtype=np.uint8)
    b[0:2] = np.array([0.5], dtype=np.float16).view(np.uint8)
    b[2] = 0          # ib 0, l 0: grid index low byte for g1
    b[3] = 5          # ib 0, l 0: g2 low byte
    b[66] = 0b10      # qh of ib 0: bit 1 -> 9th bit of g2 (shift 7 - 2 l = 7 for l = 0)
    b[74] = 0b0000_0101
    b[106] = 0x03     # scales: ib 0 low nibble 3, ib 1 high nibble 0
    y = O.dequant(ggml.IQ3_S, b, 256)
    g2 = IQ3S_GRID[256 + 5]
    want0 = [3.5 * 1 * s for s in (-1, 1, -1, 1)] + [3.5 * ((g2 >> (8 * j)) & 255) for j in range(4)]
    assert list(y[:8]) == want0
    # every other entry of sub-block 0 uses grid index 0 (value 1), plus, times db = 3.5
    assert np.all(y[8:32] == 3.5)
    # sub-block 1: qs 0, qh 0, signs 0, scale 1 + 2 * 0 = 1 -> db = 0.5 times grid value 1
    assert np.all(y[32:64] == 0.5)


def test_iq_tables_invariants():
    """KSIGNS_IQ2XS: 7 stored bits plus an even-parity bit 7 (src/quant/tables.rs:5); IQ3_S grid bytes are odd
    1..15; IQ2_XXS grid bytes are 0x08, 0x19 or 0x2b."""
    from tests.iq_tables import IQ2XXS_GRID, IQ3S_GRID, KSIGNS
    for i, s in enumerate(KSIGNS):
        assert s & 127 == i
        assert bin(s).count("1") % 2 == 0
    for g in IQ3S_GRID:
        for j in range(4):
            v = (g >> (8 * j)) & 255
            assert v % 2 == 1 and 1 <= v <= 15
    for g in IQ2XXS_GRID:
        for j in range(8):
            assert (g >> (8 * j)) & 255 in (0x08, 0x19, 0x2B)


def test_quantize_q8k_properties():
    """quantize_q8k (src/cpu_moe.rs:28-46): scale -127 / (first value of largest magnitude), q = min(127, rne(is v))."""
    x = xs(1024) * 3.0
    x[5] = -7.0
    x[300] = 7.0      # tie in magnitude after a larger block start: first one decides in its own block
    x[256] = 6.0
    x[257] = -6.0     # block 1: the first of equal magnitude (+6 at 256) decides the sign
    d, qs, bs = O.quantize_q8k(x)
    assert d.shape == (4,)
    # block 0: max |v| is 7 at index 5 (negative): is = -127 / -7 > 0, so x[5] -> q = -127.
    assert qs[0, 5] == -127 and d[0] > 0
    # block 1: max |v| is 7 at 300 (positive): is < 0, so x[300] -> -127, and d < 0.
    assert qs[1, 300 - 256] == -127 and d[1] < 0
    is_ = np.float32(-127.0) / np.float32(7.0)
    assert d[1] == np.float32(1.0) / is_
    # reconstruction within half a step, group sums exact
    rec = (qs.astype(np.float32) * d[:, None]).reshape(-1)
    assert np.all(np.abs(rec - x) <= np.abs(np.repeat(d, 256)) * 0.5 + 1e-7)
    assert np.array_equal(bs, qs.reshape(4, 16, 16).astype(np.int32).sum(-1))
    # zero block and a short (zero-padded) tail
    z = np.zeros(256 + 64, dtype=np.float32)
    z[256:] = 1.0
    d, qs, _ = O.quantize_q8k(z)
    assert d[0] == 0 and not qs[0].any()
    assert qs[1, :64].tolist() == [-127] * 64 and not qs[1, 64:].any()


@pytest.mark.parametrize("ty", ggml.TYPES)
def test_int_dots_match_dequant(ty):
    """src/cpu_moe.rs:1593-1618: every integer dot equals the f64 dot of dequant(w) with dequant(Q8_K(x)) to 1e-5."""
    n = 1024
    x = xs(n)
    row = random_blocks(ty, 1, n, seed=ty)[0]
    w = O.dequant(ty, row, n).astype(np.float64)
    d, qs, _ = O.quantize_q8k(x)
    seen = (d[:, None] * qs.astype(np.float32)).astype(np.float32).reshape(-1)
    want = float(np.dot(w, seen.astype(np.float64)))
    got = O.int_dot(ty, row, x)
    assert abs(got - want) / max(abs(want), 1e-3) < 1e-5, (got, want)


def test_route_ties_and_weights():
    """tests/kernels.rs:1244-1282: token 1 ties experts 7 and 200 (lower index first); token 2 ties at the k-th place."""
    n, k, t = 256, 8, 3
    x = xs(n * t) * 4.0
    x[n + 7] = 9.0
    x[n + 200] = 9.0
    x[2 * n + 30] = 5.0
    x[2 * n + 31] = 5.0
    x[2 * n + 255] = 5.0
    ids, w = O.route(x.reshape(t, n), k, extra_scale=2.5)
    assert ids[1, :2].tolist() == [7, 200]
    for r in range(t):
        lg = x[r * n:(r + 1) * n].astype(np.float64)
        p = np.exp(lg - lg.max())
        p /= p.sum()
        order = sorted(range(n), key=lambda i: (-p[i], i))[:k]
        assert ids[r].tolist() == order
        s = sum(p[i] for i in order)
        assert np.allclose(w[r], [p[i] / s * 2.5 for i in order], rtol=1e-5, atol=0)
    assert ids[2].tolist().count(30) == 1 and ids[2].tolist().count(31) == 1


def test_route_sigmoid():
    """tests/kernels.rs:2056-2083: sigmoid scores, top-k renormalised and scaled."""
    n, k, t = 17, 4, 3
    lg = xs(t * n).reshape(t, n)
    ids, w = O.route(lg, k, sigmoid=True, extra_scale=1.5)
    for r in range(t):
        p = 1.0 / (1.0 + np.exp(-lg[r].astype(np.float64)))
        order = sorted(range(n), key=lambda i: (-p[i], i))[:k]
        assert sorted(ids[r].tolist()) == sorted(order)
        s = sum(p[i] for i in order)
        for j, i in enumerate(ids[r]):
            assert abs(w[r, j] - p[i] / s * 1.5) <= 1e-5


def test_sort_is_the_stable_counting_sort():
    """src/gpu_model/prefill.rs:563-573 against a brute-force stable sort of the pair indices by expert."""
    rng = np.random.default_rng(3)
    t, k, E = 200, 8, 64
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(t)]).astype(np.int32)
    off, xrow, inv = O.sort_by_expert(ids, E)
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")
    assert np.array_equal(xrow, (order // k).astype(np.int32))
    assert np.array_equal(inv[order], np.arange(t * k, dtype=np.int32))
    assert np.array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]).astype(np.int32))


def test_combine_seq_closed_form():
    """tests/kernels.rs:923-948: x[t] += sum_j wts[t, j] ye[inv[t, j]]."""
    n, k, t, ne = 300, 3, 5, 20
    x0 = xs(t * n).reshape(t, n)
    ye = xs(ne * n + 1)[1:].reshape(ne, n)
    wts = xs(t * k + 2)[2:].reshape(t, k)
    inv = np.array([(i * 7) % ne for i in range(t * k)], dtype=np.int32).reshape(t, k)
    got = O.combine_seq(x0, ye, wts, inv)
    want = x0.astype(np.float64) + np.einsum("tj,tjd->td", wts.astype(np.float64), ye[inv].astype(np.float64))
    assert np.abs(got - want).max() < 1e-5


def test_matvec_equals_row_dots():
    """cpu_moe::matvec's parallel chunks give each row's int_dot exactly."""
    rows, cols = 70, 512
    for ty in (ggml.Q4_K, ggml.Q6_K, ggml.Q8_0):
        w = random_blocks(ty, rows, cols, seed=11)
        x = xs(cols)
        y = O.matvec(ty, w, rows, cols, x, threads=4)
        for r in range(rows):
            assert y[r] == np.float32(O.int_dot(ty, w[r], x))


def test_experts_multi_matches_f64():
    """experts_multi against an f64 restatement on dequantized weights with the same Q8_K activations."""
    E, H, F, t, k = 4, 256, 256, 3, 2
    gate = random_blocks(ggml.Q5_K, E * F, H, seed=1)
    up = random_blocks(ggml.Q5_K, E * F, H, seed=2)
    down = random_blocks(ggml.Q6_K, E * H, F, seed=3)
    hs = xs(t * H).reshape(t, H)
    ids = np.array([[0, 2], [3, 1], [2, 0]], dtype=np.int32)
    wts = np.array([[0.6, 0.4], [0.5, 0.5], [0.9, 0.1]], dtype=np.float32)
    ys = O.experts_multi(ggml.Q5_K, ggml.Q6_K, gate, up, down, H, F, hs, ids, wts)
    G = O.dequant(ggml.Q5_K, gate, E * F * H).reshape(E, F, H).astype(np.float64)
    U = O.dequant(ggml.Q5_K, up, E * F * H).reshape(E, F, H).astype(np.float64)
    D = O.dequant(ggml.Q6_K, down, E * H * F).reshape(E, H, F).astype(np.float64)

    def seen(v):
        d, qs, _ = O.quantize_q8k(v)
        return (d[:, None] * qs.astype(np.float32)).reshape(-1)[: v.size].astype(np.float64)

    for tt in range(t):
        want = np.zeros(H)
        for j in range(k):
            e = ids[tt, j]
            xh = seen(hs[tt])
            g, u = G[e] @ xh, U[e] @ xh
            a = (g / (1 + np.exp(-g)) * u).astype(np.float32)
            want += wts[tt, j] * (D[e] @ seen(a))
        err = np.abs(ys[tt] - want).max() / np.abs(want).max()
        assert err < 2e-3, err  # the f32 SwiGLU may round an activation to the other int8 step


def test_rms_norm_pinned():
    """ops::rms_norm (src/ops.rs:3-7) pinned by what the mathematics fixes: a constant row normalizes to exactly 1
    (0.5 * 256 squares sum exactly); the result is invariant under power-of-two scaling of x (every step scales
    exactly) and linear in w; mean(out^2 / w^2) = 1 with eps = 0; and the float64 formula to 1e-6."""
    n = 256
    out = O.rms_norm(np.full(n, 0.5, np.float32), np.ones(n, np.float32), 0.0)
    assert np.array_equal(out, np.ones((1, n), np.float32))
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 768)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 768).astype(np.float32)
    a = O.rms_norm(x, w, 0.0)
    assert np.array_equal(O.rms_norm(x * np.float32(8.0), w, 0.0), a)
    assert np.array_equal(O.rms_norm(x, w * np.float32(2.0), 0.0), a * np.float32(2.0))
    assert np.abs((O.rms_norm(x, np.ones(768, np.float32), 0.0).astype(np.float64) ** 2).mean(axis=1) - 1).max() < 1e-5
    eps = 1e-6
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + eps) * w
    assert np.abs(O.rms_norm(x, w, eps) - want).max() / np.abs(want).max() < 1e-6


def test_quant_xq32_known_answers():
    """The reference GPU's per-32 quantization (src/cuda/kernels.cu:640-660): d = max|v| / 127, q = rn(v * (127 /
    max|v|)) with ties to even (__float2int_rn), an all-zero group giving d = 0, q = 0. Hand-computed groups fail
    the plausible slips: d = max / 128, id = 1 / d, ties away from zero, a missed extreme."""
    x = np.zeros((2, 128), dtype=np.float32)
    # group 0: max 127 -> d = 1, id = 1 exactly; exact .5 ties round to even
    x[0, :8] = [127.0, -127.0, 2.5, 3.5, -2.5, 0.5, 1.5, -126.5]
    # group 1: all zero
    # group 2: max 0.3 (at the last element): 127 / 0.3 = 423.3333 in f32, while 1 / (0.3 / 127) = 423.33334; the
    # value below lands on 1.49999.. with the first and on 1.5000.. with the second
    x[0, 64] = np.float32(0.0035433070734143257)
    x[0, 95] = np.float32(0.3)
    # group 3: negative extreme -> -127, and a value of exactly half the maximum
    x[0, 96], x[0, 97] = -8.0, 4.0
    x[1, :32] = np.float32(0.25)          # row 1, group 0: all at the maximum -> 127 each, d = 0.25 / 127
    q, d = O.quant_xq32(x)
    assert q[0, :8].tolist() == [127, -127, 2, 4, -2, 0, 2, -126]
    assert d[0, 0] == np.float32(1.0)
    assert d[0, 1] == 0 and not q[0, 32:64].any()
    assert q[0, 64] == 1 and q[0, 95] == 127
    assert d[0, 2] == np.float32(np.float32(0.3) / np.float32(127.0))
    assert q[0, 96] == -127 and q[0, 97] == 64 and d[0, 3] == np.float32(np.float32(8.0) / np.float32(127.0))
    assert q[1, :32].tolist() == [127] * 32 and d[1, 0] == np.float32(np.float32(0.25) / np.float32(127.0))
    assert not q[1, 32:].any() and not d[1, 1:].any()


def test_quantize_q8k_ties_to_even():
    """quantize_q8k rounds is * v with round_ties_even (src/cpu_moe.rs:39): a block whose first largest magnitude is
    -127 has is = 1 exactly, so .5 values are exact ties; d = 1 / is = 1."""
    x = np.zeros(256, dtype=np.float32)
    x[:8] = [-127.0, 2.5, 3.5, -2.5, -3.5, 0.5, 126.5, 127.0]
    d, qs, bs = O.quantize_q8k(x)
    assert d[0] == np.float32(1.0)
    assert qs[0, :8].tolist() == [-127, 2, 4, -2, -4, 0, 126, 127]
    assert bs[0, 0] == sum([-127, 2, 4, -2, -4, 0, 126, 127])


def test_iq3s_known_answer_all_qh_bits_and_sign_bytes():
    """IQ3_S (src/quant/mod.rs:345-361), stated as the format defines it: the j-th of a sub-block's 8 grid indices
    (j = 0..7, 4 values each) is qs[8 ib + j] plus 256 times bit j of qh[ib]; value e of the sub-block takes the sign
    of bit e % 8 of signs[4 ib + e / 8]; db = d (1 + 2 sc[ib])."""
    from tests.iq_tables import IQ3S_GRID
    rng = np.random.default_rng(7)
    b = np.zeros(110, dtype=np.uint8)
    b[0:2] = np.array([0.25], dtype=np.float16).view(np.uint8)
    b[2:66] = rng.integers(0, 256, 64, dtype=np.uint8)
    b[66:74] = [0b1010_0110, 0b0101_1001, 0xFF, 0x00, 0b1000_0001, 0b0111_1110, 0b0011_1100, 0b1100_0011]
    b[74:106] = rng.integers(0, 256, 32, dtype=np.uint8)
    b[106:110] = [0x21, 0x43, 0x65, 0xF7]
    y = O.dequant(ggml.IQ3_S, b, 256)
    want = np.empty(256, dtype=np.float32)
    d = np.float32(0.25)
    for ib in range(8):
        sc = (b[106 + ib // 2] >> (4 * (ib % 2))) & 15
        db = np.float32(d * np.float32(1 + 2 * int(sc)))
        for j in range(8):
            idx = int(b[2 + 8 * ib + j]) + 256 * ((int(b[66 + ib]) >> j) & 1)
            g = IQ3S_GRID[idx]
            for c in range(4):
                e = 4 * j + c
                neg = (int(b[74 + 4 * ib + e // 8]) >> (e % 8)) & 1
                want[32 * ib + e] = db * np.float32((g >> (8 * c)) & 255) * np.float32(-1.0 if neg else 1.0)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


# ---- the decoder stack's CPU functions (oracle/attention.c) ----

def test_rope_neox_closed_forms():
    """ops::rope_neox (src/ops.rs:36-45): position 0 is the identity; pair (i, i + n_rot / 2) turns by
    theta_i = pos * base^(-2 i / n_rot) (i = 0: theta = pos exactly; i = 1 checked against f64 numpy); each pair keeps
    its length; dims past n_rot are untouched; turning by p1 then p2 is turning by p1 + p2 (to rounding)."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 128)).astype(np.float32)
    assert np.array_equal(O.rope_neox(x, 128, 0, 1e6), x)
    y = O.rope_neox(x, 128, 37, 1e6)
    c, s = np.float32(np.cos(37.0)), np.float32(np.sin(37.0))
    assert np.array_equal(y[:, 0], (x[:, 0] * c - x[:, 64] * s).astype(np.float32))
    th1 = 37.0 * 1e6 ** (-2.0 / 128)
    assert np.allclose(y[:, 1], x[:, 1] * np.cos(th1) - x[:, 65] * np.sin(th1), rtol=0, atol=1e-5)
    assert np.allclose(y[:, 65], x[:, 1] * np.sin(th1) + x[:, 65] * np.cos(th1), rtol=0, atol=1e-5)
    for i in range(64):
        assert np.allclose(np.hypot(y[:, i], y[:, i + 64]), np.hypot(x[:, i], x[:, i + 64]), rtol=1e-5)
    # partial rotation: n_rot 64 leaves dims 64.. alone and pairs (i, i + 32)
    z = O.rope_neox(x, 64, 5, 1e4)
    assert np.array_equal(z[:, 64:], x[:, 64:])
    assert np.allclose(np.hypot(z[:, 3], z[:, 35]), np.hypot(x[:, 3], x[:, 35]), rtol=1e-5)
    assert np.allclose(O.rope_neox(O.rope_neox(x, 128, 300, 1e6), 128, 1000, 1e6), O.rope_neox(x, 128, 1300, 1e6),
                       atol=5e-5)


def test_argmax_total_order():
    """ops::argmax (src/ops.rs:110-112): first index on ties; under total_cmp +0 is above -0 and a positive NaN above
    everything."""
    assert O.argmax(np.array([1, 5, 5, 2], np.float32)) == 1
    assert O.argmax(np.array([-0.0, 0.0, -0.0], np.float32)) == 1
    assert O.argmax(np.array([np.inf, np.nan, 3], np.float32)) == 1
    assert O.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    x = np.random.default_rng(1).standard_normal(151936).astype(np.float32)
    assert O.argmax(x) == int(np.argmax(x))


def test_attention_known_answers():
    """Model::attention (src/model.rs:771-793): one cell gives its V row exactly; the GQA map sends query head i to
    KV head i / (nh / nkv) (distinct constant V rows per KV head); a large sink logit takes all the mass; the gate
    multiplies by sigmoid; in general the output is the f64 softmax-weighted mean of V."""
    rng = np.random.default_rng(4)
    nh, nkv, hd, P = 8, 2, 16, 9
    q = rng.standard_normal(nh * hd).astype(np.float32)
    kc = rng.standard_normal((P, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((P, nkv * hd)).astype(np.float32)
    one = O.attention(q, kc, vc, 4, 5, nh, nkv, hd, 0.25)
    for i in range(nh):
        g = i // (nh // nkv)
        assert np.array_equal(one[i * hd:(i + 1) * hd], vc[4, g * hd:(g + 1) * hd])
    vconst = np.concatenate([np.full((P, hd), -3.0), np.full((P, hd), 7.0)], axis=1).astype(np.float32)
    o = O.attention(q, kc, vconst, 0, P, nh, nkv, hd, 0.25).reshape(nh, hd)
    assert np.allclose(o[:4], -3.0, atol=1e-5) and np.allclose(o[4:], 7.0, atol=1e-5)
    o = O.attention(q, kc, vc, 0, P, nh, nkv, hd, 0.25, sinks=np.full(nh, 80.0, np.float32))
    assert np.abs(o).max() < 1e-20
    gate = rng.standard_normal(nh * 2 * hd).astype(np.float32)
    plain = O.attention(q, kc, vc, 2, P, nh, nkv, hd, 0.25)
    gated = O.attention(q, kc, vc, 2, P, nh, nkv, hd, 0.25, gate=gate[hd:], gate_stride=2 * hd)
    sig = 1 / (1 + np.exp(-gate.reshape(nh, 2 * hd)[:, hd:].astype(np.float64)))
    assert np.allclose(gated, plain * sig.reshape(-1), rtol=1e-6, atol=1e-7)
    # f64 brute force
    want = np.empty((nh, hd))
    for i in range(nh):
        g = i // (nh // nkv)
        s = kc[2:, g * hd:(g + 1) * hd].astype(np.float64) @ q[i * hd:(i + 1) * hd].astype(np.float64) * 0.25
        p = np.exp(s - s.max())
        want[i] = p @ vc[2:, g * hd:(g + 1) * hd].astype(np.float64) / p.sum()
    assert np.allclose(plain.reshape(nh, hd), want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("ty", [ggml.Q2_K, ggml.Q3_K, ggml.Q4_K, ggml.Q5_K, ggml.Q6_K, ggml.Q8_0])
def test_avx2_dots_match_scalar(ty):
    """The AVX2 dots (the timed CPU baseline, src/cpu_moe.rs:757-981) compute the same integer super-block sums as the
    scalar dots and close them in 8 f32 lanes: within f32 rounding of the scalar results (1e-5 relative), and equal
    to the f64 dot of dequant(w) with dequant(Q8_K(x))."""
    n, rows = 2048, 64
    w = random_blocks(ty, rows, n, seed=90 + ty)
    x = xs(n) * 3
    try:
        O.set_avx2(False)
        scalar = O.matvec(ty, w, rows, n, x, threads=1)
        O.set_avx2(True)
        fast = O.matvec(ty, w, rows, n, x, threads=1)
    finally:
        O.set_avx2(False)
    assert np.allclose(fast, scalar, rtol=1e-5, atol=1e-6 * np.abs(scalar).max()), np.abs(fast - scalar).max()
    d, qs, _ = O.quantize_q8k(x)
    seen = (d[:, None] * qs.astype(np.float32)).reshape(-1).astype(np.float64)
    wf = O.dequant(ty, w, rows * n).reshape(rows, n).astype(np.float64)
    assert np.allclose(fast, wf @ seen, rtol=1e-5, atol=1e-5 * np.abs(wf @ seen).max())

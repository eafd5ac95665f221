"""GPU parity of the HIP path (through the C ABI) against the CPU oracle on identical seeded inputs.

Bars: dequant, quantized activations, routing ids, sort/gather indices bit-exact; fp32 outputs within max relative
error 1e-3 (floor 1e-3 max|r|), the accumulation-order tolerance of the task.
"""
import os

import numpy as np
import pytest

import rustingstrata_amd as S
from oracle import oracle as O
from rustingstrata_amd import ggml
from tests.helpers import max_rel_err, normal, random_blocks, rel_l2, zipf_logits

pytestmark = pytest.mark.gpu
TOL = 1e-3


def up(hip, a):
    return hip.upload(np.ascontiguousarray(a))


def down(hip, buf, dtype, n):
    return hip.get(buf, dtype, n)


def seen_q8k(x):
    d, qs, _ = O.quantize_q8k(x)
    return (d[:, None] * qs.astype(np.float32)).reshape(-1)[: x.size].astype(np.float64)


@pytest.mark.parametrize("ty", ggml.TYPES)
def test_dequant_bit_exact(hip, ty):
    rows, cols = 37, 768 if ty != ggml.Q8_0 else 96
    w = random_blocks(ty, rows, cols, seed=100 + ty)
    t = hip.upload_tensor(ty, w)
    out = hip.alloc(rows * cols * 4)
    hip.dequant(t, rows, out)
    got = down(hip, out, np.float32, rows * cols)
    want = O.dequant(ty, w, rows * cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name,ty", [("Q2_K", ggml.Q2_K), ("Q3_K", ggml.Q3_K), ("Q4_K", ggml.Q4_K), ("Q5_K", ggml.Q5_K),
                                     ("Q6_K", ggml.Q6_K), ("Q8_0", ggml.Q8_0), ("IQ4_XS", ggml.IQ4_XS),
                                     ("ggml_q5_k", ggml.Q5_K), ("ggml_q8_0", ggml.Q8_0), ("ggml_iq2_xxs", ggml.IQ2_XXS),
                                     ("IQ3_S", ggml.IQ3_S)])
def test_dequant_reference_fixtures(hip, name, ty):
    import os
    d = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference")
    if name == "IQ3_S":  # oracle-derived (the reference holds no IQ3_S vector): tests/golden/make_oracle_vectors.py
        d = os.path.join(os.path.dirname(d), "oracle")
    raw = np.fromfile(os.path.join(d, name + (".blk" if name.startswith("ggml") else ".raw")), dtype=np.uint8)
    want = np.fromfile(os.path.join(d, name + ".f32"), dtype=np.float32)
    cols = ggml.block_elems(ty) * (raw.size // ggml.block_bytes(ty))
    t = S.GpuTensor(ty, 1, cols, up(hip, raw))
    out = hip.alloc(cols * 4)
    hip.dequant(t, 1, out)
    got = down(hip, out, np.float32, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n,nt", [(2048, 1), (768, 3), (320, 2)])
def test_quant_xq_q8k_bit_exact(hip, n, nt):
    x = normal((nt, n), seed=n + nt)
    x[0, 17] = -x[0].__abs__().max() * 1.5  # a negative extreme
    xb = up(hip, x)
    out = hip.alloc(nt * (n + n // 8))
    hip.quant_xq(xb, n, n, nt, out)
    raw = down(hip, out, np.uint8, nt * (n + n // 8))
    q = raw[: nt * n].view(np.int8).reshape(nt, n)
    sc = raw[nt * n:].view(np.float32).reshape(nt, n // 32)
    for t in range(nt):
        d, qs, _ = O.quantize_q8k(x[t])
        assert np.array_equal(q[t], qs.reshape(-1)[:n])
        assert np.array_equal(sc[t].view(np.uint32), np.repeat(d, 8)[: n // 32].view(np.uint32))


def test_quant_xq_many_rows(hip):
    """More rows than one grid dimension addresses (66000 rows of 256): sampled rows bit-exact."""
    n, nt = 256, 66000
    x = normal((nt, n), seed=77)
    xb = up(hip, x)
    out = hip.alloc(nt * (n + n // 8))
    hip.quant_xq(xb, n, n, nt, out)
    raw = down(hip, out, np.uint8, nt * (n + n // 8))
    q = raw[: nt * n].view(np.int8).reshape(nt, n)
    sc = raw[nt * n:].view(np.float32).reshape(nt, n // 32)
    for t in [0, 1, 65534, 65535, 65536, nt - 1] + list(np.random.default_rng(1).integers(0, nt, 10)):
        d, qs, _ = O.quantize_q8k(x[t])
        assert np.array_equal(q[t], qs.reshape(-1))
        assert np.array_equal(sc[t].view(np.uint32), np.repeat(d, 8).view(np.uint32))


def test_quant_xq_q8k_magnitude_tie(hip):
    """Equal largest magnitudes of opposite sign in one 256-block, in different 16-lane rows: the first one sets the
    scale's sign (src/cpu_moe.rs:28-46), whatever order the lanes compare in."""
    n = 512
    x = normal((1, n), seed=9) * 0.1
    x[0, 200] = 7.0
    x[0, 60] = -7.0
    x[0, 300] = 3.0
    x[0, 511] = -3.0
    xb = up(hip, x)
    out = hip.alloc(n + n // 8)
    hip.quant_xq(xb, n, n, 1, out)
    raw = down(hip, out, np.uint8, n + n // 8)
    d, qs, _ = O.quantize_q8k(x[0])
    assert np.array_equal(raw[:n].view(np.int8), qs.reshape(-1)[:n])
    assert np.array_equal(raw[n:].view(np.float32).view(np.uint32), np.repeat(d, 8)[: n // 32].view(np.uint32))
    assert raw[n:].view(np.float32)[0] > 0  # -127 / (-7): the negative value came first


@pytest.mark.parametrize("n,rows,res,inplace", [(2048, 3, False, False), (768, 5, True, False), (4096, 2, True, True),
                                               (320, 4, False, True)])
def test_rms_norm_q(hip, n, rows, res, inplace):
    """Backend::rms_norm_q (src/backend.rs:233-235): x += res (bit-exact), out against ops::rms_norm (src/ops.rs:3-7)
    to 1e-6 (the GPU sums the squares in a tree, the CPU in index order), xq bit-exact against quant_xq of the same
    out; out may be x."""
    x = normal((rows, n), seed=n + rows)
    r = normal((rows, n), seed=n + rows + 1) if res else None
    w = np.random.default_rng(n).uniform(0.5, 1.5, n).astype(np.float32)
    xb, wb = up(hip, x), up(hip, w)
    rb = up(hip, r) if res else 0
    ob = xb if inplace else hip.alloc(rows * n * 4)
    xq = hip.alloc(rows * (n + n // 8))
    hip.rms_norm_q(xb, n, wb, ob, n, n, rows, 1e-6, xq=xq, res=rb)
    xs = x + r if res else x
    if res and not inplace:
        assert np.array_equal(down(hip, xb, np.float32, rows * n).reshape(rows, n), xs)
    got = down(hip, ob, np.float32, rows * n).reshape(rows, n)
    want = O.rms_norm(xs, w, 1e-6)
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-6
    q2 = hip.alloc(rows * (n + n // 8))
    hip.quant_xq(ob, n, n, rows, q2)
    assert np.array_equal(down(hip, xq, np.uint8, rows * (n + n // 8)), down(hip, q2, np.uint8, rows * (n + n // 8)))
    # without xq and res: rms_norm
    o2 = hip.alloc(rows * n * 4)
    hip.rms_norm(ob, n, wb, o2, n, n, rows, 1e-6)
    assert np.abs(down(hip, o2, np.float32, rows * n).reshape(rows, n) - O.rms_norm(got, w, 1e-6)).max() < 1e-5


@pytest.mark.parametrize("numerics", [S.NUM_Q8K, S.NUM_Q8_32])
@pytest.mark.parametrize("n,rows,k,quant,res", [(2048, 1, 8, True, True), (768, 3, 6, True, False),
                                               (2048, 2, 12, False, True), (512, 4, 1, True, False),
                                               (4096, 2, 8, True, True)])
def test_combine_rms_norm_q_equals_two_calls(hip, numerics, n, rows, k, quant, res):
    """combine_rms_norm_q (x += res, a layer's moe_combine and the next attention norm in one launch) leaves x, out and
    xq bit-equal to add, moe_combine then rms_norm_q (src/backend.rs:418-419, 233-235), with slots of weight 0, more
    slots than one round of 8 (k = 12), and n = 4096 (separate launches); out against ops::rms_norm of the new x."""
    rng = np.random.default_rng(n + rows + k)
    x0 = normal((rows, n), seed=n + k)
    ye = normal((rows * k, n), seed=n + k + 1)
    wh = rng.uniform(0.1, 0.5, rows * k).astype(np.float32)
    wh[::5] = 0.0
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    yb, whb, wb = up(hip, ye), up(hip, wh), up(hip, w)
    old = hip.numerics()
    hip.set_numerics(numerics)
    try:
        xa, xb = up(hip, x0), up(hip, x0)
        oa, ob = hip.alloc(rows * n * 4), hip.alloc(rows * n * 4)
        qa, qb = (hip.alloc(rows * (n + n // 8)), hip.alloc(rows * (n + n // 8))) if quant else (0, 0)
        rb = up(hip, normal((rows, n), seed=n + k + 2)) if res else 0
        if res:
            hip.add(xa, rb, rows * n)
        hip.moe_combine(xa, yb, whb, k, 0, 0, n, rows)
        hip.rms_norm_q(xa, n, wb, oa, n, n, rows, 1e-6, xq=qa)
        hip.combine_rms_norm_q(xb, yb, whb, k, wb, ob, n, rows, 1e-6, xq=qb, res=rb)
    finally:
        hip.set_numerics(old)
    for a, b, m in ((xa, xb, rows * n), (oa, ob, rows * n)):
        assert np.array_equal(down(hip, a, np.uint32, m), down(hip, b, np.uint32, m))
    if quant:
        assert np.array_equal(down(hip, qa, np.uint8, rows * (n + n // 8)), down(hip, qb, np.uint8, rows * (n + n // 8)))
    xc = down(hip, xb, np.float32, rows * n).reshape(rows, n)
    want = O.rms_norm(xc, w, 1e-6)
    got = down(hip, ob, np.float32, rows * n).reshape(rows, n)
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-6
    # x itself against the combine in f64 (slot order aside)
    if res:
        x0 = x0 + normal((rows, n), seed=n + k + 2)
    wx = x0.astype(np.float64) + np.einsum("rk,rkn->rn", wh.reshape(rows, k).astype(np.float64), ye.reshape(rows, k, n))
    assert np.abs(xc - wx).max() < 1e-5


@pytest.mark.parametrize("ty,rows,n", [(ggml.Q6_K, 5120, 2048), (ggml.Q8_0, 3001, 2048), (ggml.Q4_K, 700, 1024),
                                        (ggml.Q2_K, 4096, 2048), (ggml.Q5_K, 64, 512)])
@pytest.mark.parametrize("k,res", [(8, True), (5, True), (0, True), (0, False)])
def test_combine_rms_norm_gemv_equals_two_calls(hip, ty, rows, n, k, res):
    """combine_rms_norm_gemv (the previous layer's x += res and MoE combine, this layer's norm and the GEMV reading it,
    in one launch) against combine_rms_norm_q (rms_norm_q when k = 0) then gemvq on its quantized output: x_out and y
    bit-equal, x untouched; slots of weight 0; the matrix types and shapes of the decode (q/k/v, the output head)."""
    rng = np.random.default_rng(rows + n + k)
    x0 = normal(n, seed=n + k + rows)
    ye = normal((max(k, 1), n), seed=n + k + 1)
    wh = rng.uniform(0.1, 0.5, max(k, 1)).astype(np.float32)
    wh[::3] = 0.0
    nw = rng.uniform(0.5, 1.5, n).astype(np.float32)
    r0 = normal(n, seed=n + 7)
    w = random_blocks(ty, rows, n, seed=rows + ty)
    t = hip.upload_tensor(ty, w)
    yb, whb, nwb, rb = up(hip, ye), up(hip, wh), up(hip, nw), (up(hip, r0) if res else 0)
    xa, xb, xo = up(hip, x0), up(hip, x0), hip.alloc(n * 4)
    h, hq = hip.alloc(n * 4), hip.alloc(n + n // 8)
    ya, yf = hip.alloc(rows * 4), hip.alloc(rows * 4)
    if k:
        hip.combine_rms_norm_q(xa, yb, whb, k, nwb, h, n, 1, 1e-6, xq=hq, res=rb)
    else:
        hip.rms_norm_q(xa, n, nwb, h, n, n, 1, 1e-6, xq=hq, res=rb)
    hip.gemvq(t, h, n, hq, ya, rows, 1)
    hip.combine_rms_norm_gemv(xb, rb, yb if k else 0, whb if k else 0, k, nwb, 1e-6, t, xo, yf)
    assert np.array_equal(down(hip, xb, np.float32, n), x0)  # x is only read
    assert np.array_equal(down(hip, xo, np.uint32, n), down(hip, xa, np.uint32, n))
    assert np.array_equal(down(hip, yf, np.uint32, rows), down(hip, ya, np.uint32, rows))
    with pytest.raises(S.StrataError, match="x_out overlaps"):
        hip.combine_rms_norm_gemv(xb, rb, 0, 0, 0, nwb, 1e-6, t, xb, yf)
    if k:
        with pytest.raises(S.StrataError, match="x_out overlaps"):
            hip.combine_rms_norm_gemv(xb, rb, yb, whb, k, nwb, 1e-6, t, int(yb) + 4 * n, yf)


@pytest.mark.parametrize("numerics", [S.NUM_Q8K, S.NUM_Q8_32])
@pytest.mark.parametrize("n,rows", [(2048, 128), (512, 61), (1024, 3)])
def test_rms_norm_q_gemv_f32_equals_two_calls(hip, numerics, n, rows):
    """rms_norm_q_gemv_f32 (the decode's FFN norm and router logits in one launch): h and hq bit-equal to
    rms_norm_q(x + res), y bit-equal to gemv of the F32 matrix on that h (src/backend.rs:233-235, src/gpu_model.rs
    router), x left as it was; a row count that is not a multiple of 4 (61)."""
    x0, r0 = normal(n, seed=n + 1), normal(n, seed=n + 2)
    w = np.random.default_rng(n).uniform(0.5, 1.5, n).astype(np.float32)
    W = (0.05 * normal((rows, n), seed=n + 3)).astype(np.float32)
    wb, Wt = up(hip, w), hip.upload_f32(W)
    old = hip.numerics()
    hip.set_numerics(numerics)
    try:
        xa, xb, rb = up(hip, x0), up(hip, x0), up(hip, r0)
        ha, hb = hip.alloc(n * 4), hip.alloc(n * 4)
        qa, qb = hip.alloc(n + n // 8), hip.alloc(n + n // 8)
        ya, yb = hip.alloc(rows * 4), hip.alloc(rows * 4)
        hip.rms_norm_q(xa, n, wb, ha, n, n, 1, 1e-6, xq=qa, res=rb)
        hip.gemv(Wt, ha, ya)
        hip.rms_norm_q_gemv_f32(xb, rb, wb, hb, qb, n, 1e-6, Wt, yb)
    finally:
        hip.set_numerics(old)
    assert np.array_equal(down(hip, xb, np.float32, n), x0)
    assert np.array_equal(down(hip, ha, np.uint32, n), down(hip, hb, np.uint32, n))
    assert np.array_equal(down(hip, qa, np.uint8, n + n // 8), down(hip, qb, np.uint8, n + n // 8))
    assert np.array_equal(down(hip, ya, np.uint32, rows), down(hip, yb, np.uint32, rows))
    h = down(hip, hb, np.float32, n)
    assert np.abs(h - O.rms_norm((x0 + r0)[None, :], w, 1e-6)[0]).max() / np.abs(h).max() < 1e-6
    yw = W.astype(np.float64) @ h.astype(np.float64)
    assert np.abs(down(hip, yb, np.float32, rows) - yw).max() / np.abs(yw).max() < 1e-5
    with pytest.raises(S.StrataError, match="rms_norm_q_gemv_f32"):
        hip.rms_norm_q_gemv_f32(xb, rb, wb, hb, qb, n + 8, 1e-6, Wt, yb)


def test_quant_xq_per32_bit_exact(hip):
    n, nt = 1024, 2
    x = normal((nt, n), seed=5)
    hip.set_numerics(S.NUM_Q8_32)
    try:
        xb = up(hip, x)
        out = hip.alloc(nt * (n + n // 8))
        hip.quant_xq(xb, n, n, nt, out)
        raw = down(hip, out, np.uint8, nt * (n + n // 8))
    finally:
        hip.set_numerics(S.NUM_Q8K)
    q, sc = O.quant_xq32(x)
    assert np.array_equal(raw[: nt * n].view(np.int8).reshape(nt, n), q)
    assert np.array_equal(raw[nt * n:].view(np.float32).reshape(nt, n // 32).view(np.uint32), sc.view(np.uint32))


def gemv_case(hip, ty, rows, cols, seed):
    w = random_blocks(ty, rows, cols, seed=seed)
    x = normal(cols, seed=seed + 1)
    t = hip.upload_tensor(ty, w)
    y = hip.alloc(rows * 4)
    hip.gemv(t, up(hip, x), y)
    return w, x, t, down(hip, y, np.float32, rows)


@pytest.mark.parametrize("ty", ggml.TYPES)
@pytest.mark.parametrize("rows,cols", [(257, 2048), (64, 768), (33, 4096), (40, 3072)])
def test_gemv_matches_cpu_matvec(hip, ty, rows, cols):
    if ty == ggml.Q8_0 and cols == 768:
        cols = 736  # Q8_0 rows need only a multiple of 32
    w, x, _, got = gemv_case(hip, ty, rows, cols, seed=7 * ty + cols)
    want = O.matvec(ty, w, rows, cols, x)
    assert max_rel_err(got, want) <= TOL, max_rel_err(got, want)
    if ty not in (ggml.Q8_0, ggml.IQ4_XS):
        # the CPU dot's float steps and its super-block order: the same bits
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int((got != want).sum())
    # and against the f64 dot of the dequantized weights with the same Q8_K activations
    wf = O.dequant(ty, w, rows * cols).reshape(rows, cols).astype(np.float64)
    assert rel_l2(got, wf @ seen_q8k(x)) < 1e-5


@pytest.mark.parametrize("ty", [ggml.Q4_K, ggml.Q5_K, ggml.Q6_K, ggml.Q8_0])
@pytest.mark.parametrize("rows", [6144, 151936])
def test_gemv_sweep_shapes(hip, ty, rows):
    """configs[1] at full size (the fused-QKV-like and lm-head-like shapes, 2048 columns): every row against the
    oracle's cpu_moe::matvec (tiles of many rows: a row past a tile's loaded bytes would show here)."""
    cols = 2048
    w = random_blocks(ty, rows, cols, seed=rows + ty)
    x = normal(cols, seed=rows + ty + 1)
    t = hip.upload_tensor(ty, w)
    y = hip.alloc(rows * 4)
    hip.gemv(t, up(hip, x), y)
    got = down(hip, y, np.float32, rows)
    want = O.matvec(ty, w, rows, cols, x, threads=min(16, os.cpu_count() or 1))
    assert max_rel_err(got, want) <= TOL, max_rel_err(got, want)


@pytest.mark.parametrize("ty", [ggml.Q3_K, ggml.Q4_K, ggml.Q6_K])
@pytest.mark.parametrize("cols", [14336, 16384])
def test_gemv_wide_rows_full_tiles(hip, ty, cols):
    """One plain matrix of wide rows (up to the single-input kernel's 16384 columns) and thousands of rows, so every
    block takes the type's full tile with x's staging beside it (past 64 KB of LDS for Q6_K): the CPU dot's bits on
    every row."""
    rows = 3000
    w = random_blocks(ty, rows, cols, seed=cols + ty)
    x = normal(cols, seed=cols + ty + 1)
    t = hip.upload_tensor(ty, w)
    y = hip.alloc(rows * 4)
    hip.gemv(t, up(hip, x), y)
    got = down(hip, y, np.float32, rows)
    want = O.matvec(ty, w, rows, cols, x, threads=min(16, os.cpu_count() or 1))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int((got != want).sum())


@pytest.mark.parametrize("ty", [ggml.Q2_K, ggml.Q3_K, ggml.Q4_K, ggml.Q5_K, ggml.Q6_K, ggml.IQ2_XXS, ggml.IQ3_S])
def test_gemv_bits_over_random_shapes(hip, ty):
    """The CPU dot's bits over seeded random shapes (1-300 rows, 256-8192 columns) and weight scales spanning
    2^-14..2^4 (down to f16 subnormal-adjacent d): the per-super-block float steps and their order hold everywhere."""
    rng = np.random.default_rng(500 + ty)
    for case in range(6):
        rows, cols = int(rng.integers(1, 301)), 256 * int(rng.integers(1, 33))
        lo = float(2.0 ** rng.integers(-14, 4))
        w = random_blocks(ty, rows, cols, seed=int(rng.integers(1 << 30)), scale=(lo, 2 * lo))
        x = normal(cols, seed=int(rng.integers(1 << 30)), std=float(2.0 ** rng.integers(-6, 6)))
        t = hip.upload_tensor(ty, w)
        y = hip.alloc(rows * 4)
        hip.gemv(t, up(hip, x), y)
        got = down(hip, y, np.float32, rows)
        want = O.matvec(ty, w, rows, cols, x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (case, rows, cols, lo, int((got != want).sum()))


@pytest.mark.parametrize("ty", ggml.TYPES)
def test_gemv_wide_rows(hip, ty):
    """Rows of more than 16384 values (dense FFN down projections: 18944, 24576 columns) run on the multi-input
    kernel, several super-blocks a lane with the running sum carried in super-block order: the CPU dot's bits
    (within rounding for Q8_0 and IQ4_XS, as for narrow rows); gemvn of two inputs gives each input's gemv bits."""
    for cols in (18944, 24576):
        if ggml.row_bytes(ty, cols) > 24512:
            continue  # a row must fit one weight tile (24 KB)
        rows = 37
        w, x, t, got = gemv_case(hip, ty, rows, cols, seed=cols + ty)
        want = O.matvec(ty, w, rows, cols, x)
        assert max_rel_err(got, want) <= TOL, (cols, max_rel_err(got, want))
        if ty not in (ggml.Q8_0, ggml.IQ4_XS):
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (cols, int((got != want).sum()))
        xs = np.stack([x, normal(cols, seed=cols + ty + 5)])
        y2 = hip.alloc(2 * rows * 4)
        hip.gemvn(t, up(hip, xs), cols, y2, rows, 2)
        got2 = down(hip, y2, np.float32, 2 * rows).reshape(2, rows)
        assert np.array_equal(got2[0].view(np.uint32), got.view(np.uint32))
        want2 = O.matvec(ty, w, rows, cols, xs[1])
        assert max_rel_err(got2[1], want2) <= TOL


def test_gemv_wide_rows_limits(hip):
    """Rows past the 24 KB weight tile are refused; the MoE GEMV keeps the single-input kernel's 16384 columns."""
    w = random_blocks(ggml.Q8_0, 1, 32768, seed=1)
    t = hip.upload_tensor(ggml.Q8_0, w)
    with pytest.raises(S.StrataError, match="exceeds the GEMV tile"):
        hip.gemv(t, up(hip, normal(32768, seed=2)), hip.alloc(4))
    with pytest.raises(S.StrataError, match="at most 16384"):
        hip.moe_gemv(ggml.Q4_K, 4, 18944, t.ptr, 0, up(hip, np.zeros(1, np.int32)), 1, up(hip, normal(18944, seed=3)),
                     18944, 1, hip.alloc(16))


@pytest.mark.parametrize("cols", [2048, 3072, 4096])
def test_gemv_per32_numerics(hip, cols):
    """Reference GPU numerics (per-32 x scales): against f64 dequant times as_seen(x) (tests/kernels.rs:11-19,61)."""
    ty, rows = ggml.Q5_K, 100
    hip.set_numerics(S.NUM_Q8_32)
    try:
        w, x, _, got = gemv_case(hip, ty, rows, cols, seed=9)
    finally:
        hip.set_numerics(S.NUM_Q8K)
    q, sc = O.quant_xq32(x[None, :])
    seen = (q[0].astype(np.float32) * np.repeat(sc[0], 32)).astype(np.float64)
    wf = O.dequant(ty, w, rows * cols).reshape(rows, cols).astype(np.float64)
    assert rel_l2(got, wf @ seen) < 1e-5


@pytest.mark.parametrize("ty", [ggml.Q4_K, ggml.Q6_K, ggml.IQ3_S, ggml.Q8_0])
def test_gemvn_bit_equals_gemv(hip, ty):
    """tests/kernels.rs:151-212: gemvn over nt = 1..4 inputs gives gemv's bits per input; gemvq with a
    pre-quantized x too."""
    rows, cols = 130, 1024
    w = random_blocks(ty, rows, cols, seed=3)
    t = hip.upload_tensor(ty, w)
    xs = normal((4, cols), seed=4)
    xb = up(hip, xs)
    singles = []
    for i in range(4):
        y = hip.alloc(rows * 4)
        hip.gemv(t, int(xb) + 4 * cols * i, y)
        singles.append(down(hip, y, np.float32, rows))
    for nt in range(1, 5):
        y = hip.alloc(nt * rows * 4)
        hip.gemvn(t, xb, cols, y, rows, nt)
        got = down(hip, y, np.float32, nt * rows).reshape(nt, rows)
        for i in range(nt):
            assert np.array_equal(got[i].view(np.uint32), singles[i].view(np.uint32)), (nt, i)
    xq = hip.alloc(4 * (cols + cols // 8))
    hip.quant_xq(xb, cols, cols, 4, xq)
    y = hip.alloc(4 * rows * 4)
    hip.gemvq(t, 0, 0, xq, y, rows, 4)
    got = down(hip, y, np.float32, 4 * rows).reshape(4, rows)
    for i in range(4):
        assert np.array_equal(got[i].view(np.uint32), singles[i].view(np.uint32))


def test_gemvq2_pair(hip):
    ty, cols = ggml.Q5_K, 2048
    wa, wb = random_blocks(ty, 96, cols, seed=1), random_blocks(ty, 40, cols, seed=2)
    ta, tb = hip.upload_tensor(ty, wa), hip.upload_tensor(ty, wb)
    x = normal(cols, seed=3)
    xb = up(hip, x)
    ya, yb = hip.alloc(96 * 4), hip.alloc(40 * 4)
    hip.gemvq2(ta, tb, xb, cols, 0, ya, yb, 1)
    ga, gb = down(hip, ya, np.float32, 96), down(hip, yb, np.float32, 40)
    y1, y2 = hip.alloc(96 * 4), hip.alloc(40 * 4)
    hip.gemv(ta, xb, y1)
    hip.gemv(tb, xb, y2)
    assert np.array_equal(ga, down(hip, y1, np.float32, 96)) and np.array_equal(gb, down(hip, y2, np.float32, 40))


def test_moe_gemv_selects_experts(hip):
    """tests/kernels.rs:97-147,1572-1654: slot j uses expert ids[j] and x row j / xg; ids < 0 stays untouched; the
    paired launch equals two launches."""
    ty, E, rows, cols = ggml.Q5_K, 5, 96, 2048
    rb = ggml.row_bytes(ty, cols)
    w = random_blocks(ty, E * rows, cols, seed=21)
    w2 = random_blocks(ty, E * rows, cols, seed=22)
    wb = up(hip, np.concatenate([w, w2]))
    ids = np.array([3, -1, 1, 4], dtype=np.int32)
    k = ids.size
    xs = normal((2, cols), seed=23)
    xb = up(hip, xs)
    sentinel = np.full(2 * k * rows, 7.25, dtype=np.float32)
    y = up(hip, sentinel)
    hip.moe_gemv(ty, rows, cols, wb, rows * rb, up(hip, ids), k, xb, cols, 2, y,
                 pair=(E * rows * rb, k * rows * 4))
    got = down(hip, y, np.float32, 2 * k * rows).reshape(2, k, rows)
    for j, e in enumerate(ids):
        if e < 0:
            assert np.all(got[:, j] == 7.25)
            continue
        for p, wm in enumerate((w, w2)):
            want = O.matvec(ty, wm[e * rows:(e + 1) * rows], rows, cols, xs[j // 2])
            assert max_rel_err(got[p, j], want) <= TOL


def test_router_topk_matches_route(hip):
    """tests/kernels.rs:1244-1282 cases, plus Zipf-skewed batches at the edges of 1, 2, 4 and 8 logits a lane: ids
    bit-exact, weights to 1e-6."""
    n, k, t = 256, 8, 3
    v = np.arange(n * t, dtype=np.float32) * np.float32(0.7548777)
    x = ((v - np.trunc(v)) - np.float32(0.5)) * np.float32(2.0) * 4.0
    x[n + 7] = 9.0
    x[n + 200] = 9.0
    x[2 * n + 30] = x[2 * n + 31] = x[2 * n + 255] = 5.0
    # the widest case (512 experts, top 32) with equal maxima in both 32-lane halves and past lane 64 (index 5 wins)
    wide = zipf_logits(6, 512, seed=3)
    wide[0, 5] = wide[0, 40] = wide[0, 300] = 20.0
    wide[1, 63] = wide[1, 64] = 20.0
    for logits, kk, scale, sig in [(x.reshape(t, n), k, 2.5, False), (zipf_logits(512, 128, seed=1), 8, 0.0, False),
                                   (zipf_logits(64, 17, seed=2), 4, 1.5, True), (wide, 32, 0.0, False),
                                   (wide, 32, 0.0, True), (zipf_logits(9, 64, seed=4), 8, 0.0, False),
                                   (zipf_logits(9, 65, seed=5), 8, 0.0, False), (zipf_logits(9, 129, seed=6), 8, 0.0, False),
                                   (zipf_logits(9, 257, seed=7), 8, 0.0, False)]:
        tt, nn = logits.shape
        ids, wts = hip.alloc(tt * kk * 4), hip.alloc(tt * kk * 4)
        hip.router_topk(up(hip, logits), nn, kk, scale, ids, wts, tt, sig)
        gi = down(hip, ids, np.int32, tt * kk).reshape(tt, kk)
        gw = down(hip, wts, np.float32, tt * kk).reshape(tt, kk)
        wi, ww = O.route(logits, kk, sigmoid=sig, extra_scale=scale)
        assert np.array_equal(gi, wi)
        assert np.abs(gw - ww).max() <= 1e-6
    assert gi is not None


def test_moe_route_table(hip):
    n, k, t = 128, 8, 16
    logits = zipf_logits(t, n, seed=5)
    table = np.arange(n, dtype=np.int32)
    table[::3] = -1
    bufs = [hip.alloc(t * k * 4) for _ in range(4)]
    hip.moe_route(up(hip, logits), n, k, 0.0, up(hip, table), *bufs, t)
    ids, wts, slots, wh = [down(hip, b, dt, t * k) for b, dt in zip(bufs, (np.int32, np.float32, np.int32, np.float32))]
    wi, ww = O.route(logits, k)
    assert np.array_equal(ids, wi.reshape(-1))
    assert np.array_equal(slots, table[ids])
    assert np.array_equal(wh, np.where(slots >= 0, wts, 0.0).astype(np.float32))


def test_rejects_oversized_grids(hip):
    """Token and row counts past what one launch addresses are errors before anything runs."""
    b = hip.alloc(64)
    with pytest.raises(S.StrataError, match="moe_combine_seq: too large"):
        hip.moe_combine_seq(b, b, b, b, 8, 0, 0, 2048, 70000)
    with pytest.raises(S.StrataError, match="moe_combine: too large"):
        hip.moe_combine(b, b, b, 8, 0, 0, 2048, 70000)
    with pytest.raises(S.StrataError, match="swiglu_q: too large"):
        hip.swiglu_q(b, b, 768, 1 << 31, b)
    with pytest.raises(S.StrataError, match="quant_xq: too large"):
        hip.quant_xq(b, 768, 768, 1 << 31, b)


def test_router_rejects_shapes(hip):
    b = hip.alloc(64)
    with pytest.raises(S.StrataError, match="router_topk: 600 experts, top 8"):
        hip.router_topk(b, 600, 8, 0.0, b, b, 1)


@pytest.mark.parametrize("t,k,E,chunk", [(1, 8, 128, 128), (333, 8, 128, 128), (4096, 8, 128, 128), (50, 4, 7, 128),
                                         (4096, 8, 128, 256), (333, 8, 128, 256), (9001, 8, 128, 256)])
def test_sort_bit_exact(hip, t, k, E, chunk):
    """chunk 128 is the reference's tile size (GEMM_BM, src/backend.rs:16); 256 fills this backend's GEMM blocks."""
    logits = zipf_logits(t, E, seed=t)
    ids, _ = O.route(logits, k)
    off_w, xrow_w, inv_w = O.sort_by_expert(ids, E)
    max_tiles = t * k // chunk + E
    off, xrow, inv = hip.alloc((E + 1) * 4), hip.alloc(t * k * 4), hip.alloc(t * k * 4)
    tiles, ntd, err = hip.alloc(3 * max_tiles * 16), hip.alloc(4), hip.alloc(4)
    mats = [(1 << 40, 1000), (2 << 40, 2000), (3 << 40, 3000)]
    hip.moe_sort(up(hip, ids), t, k, E, off, xrow, inv, mats, tiles, max_tiles, ntd, err, chunk=0 if chunk == 128 else chunk)
    assert np.array_equal(down(hip, off, np.int32, E + 1), off_w)
    assert np.array_equal(down(hip, xrow, np.int32, t * k), xrow_w)
    assert np.array_equal(down(hip, inv, np.int32, t * k), inv_w)
    assert down(hip, err, np.int32, 1)[0] == 0
    # tiles: the host tile builder of src/gpu_model/prefill.rs:618-642, per matrix
    want = []
    for e in range(E):
        for m0 in range(off_w[e], off_w[e + 1], chunk):
            want.append((e, int(m0), int(min(chunk, off_w[e + 1] - m0))))
    nt = int(down(hip, ntd, np.int32, 1)[0])
    assert nt == len(want)
    tl = down(hip, tiles, np.uint64, 3 * max_tiles * 2).reshape(3, max_tiles, 2)
    for m, (base, stride) in enumerate(mats):
        for i, (e, m0, c) in enumerate(want):
            assert int(tl[m, i, 0]) == base + e * stride
            assert int(tl[m, i, 1]) == m0 | (c << 32)


def test_empty_inputs_are_no_ops(hip):
    """Zero rows, tokens, slots or tiles: every entry point returns cleanly and writes nothing (a sentinel stays), and
    a sort of no pairs yields zero offsets and zero tiles, which a grouped GEMM then reads as no work."""
    E, k, H, F = 8, 2, 512, 256
    sentinel = np.full(64, 7.25, dtype=np.float32)
    y = up(hip, sentinel)
    b = hip.alloc(4096)
    ty = ggml.Q4_K
    w = up(hip, random_blocks(ty, 4, H, seed=5))
    hip.dequant(S.GpuTensor(ty, 4, H, w), 0, y)
    hip.quant_xq(b, H, H, 0, y)
    hip.swiglu_q(b, b, H, 0, y)
    hip.gemv(S.GpuTensor(ty, 0, H, w), b, y)
    hip.moe_gemv(ty, F, H, w, 0, b, 0, b, H, 1, y)
    hip.router_topk(b, E, k, 0.0, y, y, 0)
    hip.moe_route(b, E, k, 0.0, b, y, y, y, y, 0)
    hip.moe_combine_seq(y, b, b, b, k, 0, 0, H, 0)
    hip.moe_combine(y, b, b, k, 0, 0, H, 0)
    hip.gemm(ty, F, H, b, 0, b, H, 0, 0, y, F, S.ACT_STORE)
    assert np.array_equal(down(hip, y, np.float32, 64), sentinel)
    # a sort of no pairs, then the grouped GEMM over its (empty) tile list
    off, xrow, inv = up(hip, np.full(E + 1, -1, np.int32)), hip.alloc(16), hip.alloc(16)
    max_tiles = E
    tiles, ntd, err = hip.alloc(max_tiles * 16), up(hip, np.array([-1], np.int32)), hip.alloc(4)
    hip.moe_sort(b, 0, k, E, off, xrow, inv, [(int(w), 0)], tiles, max_tiles, ntd, err)
    assert np.array_equal(down(hip, off, np.int32, E + 1), np.zeros(E + 1, np.int32))
    assert down(hip, ntd, np.int32, 1)[0] == 0 and down(hip, err, np.int32, 1)[0] == 0
    hip.gemm_grouped(ty, 64, H, tiles, max_tiles, ntd, b, H, 0, xrow, y, 64, S.ACT_STORE)
    hip.gemm_grouped(ty, 64, H, tiles, max_tiles, ntd, b, H, 0, xrow, y, 64, S.ACT_STORE | S.SMALL_TILES)
    for fl in (0, S.SMALL_TILES):
        hip.gemm_grouped_gate_up(ty, 64, H, tiles, max_tiles, ntd, b, H, 0, xrow, y, 64, 0, flags=fl)
    assert np.array_equal(down(hip, y, np.float32, 64), sentinel)


def test_sort_counts_bad_ids(hip):
    ids = np.array([[0, 5], [9, 1]], dtype=np.int32)  # 9 is out of range for 6 experts
    E, t, k = 6, 2, 2
    off, xrow, inv = hip.alloc((E + 1) * 4), hip.alloc(t * k * 4), hip.alloc(t * k * 4)
    tiles, ntd, err = hip.alloc(16 * 16), hip.alloc(4), hip.alloc(4)
    hip.moe_sort(up(hip, ids), t, k, E, off, xrow, inv, [(0, 0)], tiles, 16, ntd, err)
    assert down(hip, err, np.int32, 1)[0] == 1
    assert down(hip, inv, np.int32, 4)[2] == -1


def test_combine_seq_and_combine(hip):
    n, k, t, ne = 300, 3, 5, 20
    rng = np.random.default_rng(0)
    x0 = normal((t, n), seed=1)
    ye = normal((ne, n), seed=2)
    wts = rng.uniform(0, 1, (t, k)).astype(np.float32)
    inv = np.array([(i * 7) % ne for i in range(t * k)], dtype=np.int32).reshape(t, k)
    xb = up(hip, x0)
    hip.moe_combine_seq(xb, up(hip, ye), up(hip, wts), up(hip, inv), k, 0, 0, n, t)
    got = down(hip, xb, np.float32, t * n).reshape(t, n)
    want = O.combine_seq(x0, ye, wts, inv)
    assert np.array_equal(got, want)  # same sum order
    # decode combine with a gated shared expert
    yek = normal((t, k, n), seed=3)
    sh, sg = normal((t, n), seed=4), normal(t, seed=5)
    wts[0, 1] = 0.0
    xb = up(hip, x0)
    hip.moe_combine(xb, up(hip, yek), up(hip, wts), k, up(hip, sh), up(hip, sg), n, t)
    got = down(hip, xb, np.float32, t * n).reshape(t, n)
    want = x0 + np.einsum("tj,tjd->td", wts, yek) + (1 / (1 + np.exp(-sg.astype(np.float64))))[:, None] * sh
    assert rel_l2(got, want) < 1e-6


@pytest.mark.parametrize("n,k", [(300, 3), (302, 3), (2048, 9), (302, 9)])
def test_combine_seq_paths(hip, n, k):
    """moe_combine_seq in both of its kernels (4 outputs a thread when n % 4 == 0, else 1), more than 8 pairs a
    token, rejected pairs (inv < 0) and a gated shared expert: bit-exact against the same float32 sums in pair order."""
    t, ne = 6, 40
    rng = np.random.default_rng(n + k)
    x0, ye = normal((t, n), seed=7), normal((ne, n), seed=8)
    wts = rng.uniform(0, 1, (t, k)).astype(np.float32)
    inv = rng.integers(0, ne, (t, k)).astype(np.int32)
    inv[1, 0] = inv[4, k - 1] = -1
    sh, sg = normal((t, n), seed=9), normal(t, seed=10)
    xb = up(hip, x0)
    hip.moe_combine_seq(xb, up(hip, ye), up(hip, wts), up(hip, inv), k, up(hip, sh), up(hip, sg), n, t)
    got = down(hip, xb, np.float32, t * n).reshape(t, n)
    want = x0.copy()
    for i in range(t):
        y = np.zeros(n, dtype=np.float32)
        for j in range(k):
            if inv[i, j] >= 0:
                y = y + wts[i, j] * ye[inv[i, j]]
        gs = np.float32(1.0) / (np.float32(1.0) + np.float32(np.exp(-np.float64(sg[i]))))
        y = y + gs * sh[i]
        want[i] = want[i] + y
    assert np.array_equal(got, want)


def test_swiglu_q(hip):
    n, rows = 768, 8
    g, u = normal((rows, n), seed=1), normal((rows, n), seed=2)
    xq = hip.alloc(rows * (n + n // 8))
    r = hip.swiglu_q(up(hip, g), up(hip, u), n, rows, xq)
    assert r == int(xq)
    raw = down(hip, xq, np.uint8, rows * (n + n // 8))
    q = raw[: rows * n].view(np.int8).reshape(rows, n)
    a = np.array([[O.silu(v) for v in row] for row in g], dtype=np.float32) * u
    mism = 0
    for t in range(rows):
        _, qs, _ = O.quantize_q8k(a[t])
        mism += int((q[t] != qs.reshape(-1)[:n]).sum())
    assert mism <= 2  # the GPU exp may differ from libm's in the last bit, moving a value across a rounding step


def tile_list(hip, base, stride, spans):
    """[w, m0 | cnt << 32] tiles (src/gpu_model/prefill.rs:618-642)."""
    t = np.array([[base + e * stride, m0 | (c << 32)] for e, m0, c in spans], dtype=np.uint64)
    return up(hip, t), len(spans)


@pytest.mark.parametrize("ty", [ggml.Q4_K, ggml.Q5_K, ggml.Q6_K, ggml.IQ2_XXS, ggml.IQ3_S, ggml.IQ4_XS, ggml.Q2_K, ggml.Q3_K,
                                ggml.Q8_0])
@pytest.mark.parametrize("fl", [0, S.SMALL_TILES], ids=["blocks256", "small64"])
def test_gemm_tiles_match_cpu(hip, ty, fl):
    """tests/kernels.rs:355-447: tiles (0, 128), (128, 16), (144, 26) with X gathered through xrow; act store, then
    SwiGLU into the stored gate, then add. Tiles (170, 256) and (426, 200) fill this backend's 256-position blocks;
    200 rows give one whole 128-row block (outputs staged through LDS) and a partial one (stored lane by lane).
    SMALL_TILES: the 64-position kernel (tiles past 64 positions taken as several items), the same bits."""
    rows, cols, E, n_x = 200, 512, 3, 100
    rb = ggml.row_bytes(ty, cols)
    w = random_blocks(ty, E * rows, cols, seed=ty)
    wb = up(hip, w)
    x = normal((n_x, cols), seed=2)
    npos = 626
    xrow = np.random.default_rng(3).integers(0, n_x, npos).astype(np.int32)
    spans = [(0, 0, 128), (2, 128, 16), (1, 144, 26), (2, 170, 256), (0, 426, 200)]
    tiles, nt = tile_list(hip, int(wb), rows * rb, spans)
    y = hip.alloc(npos * rows * 4)
    xb, xr = up(hip, x), up(hip, xrow)
    hip.gemm(ty, rows, cols, tiles, nt, xb, cols, n_x, xr, y, rows, S.ACT_STORE | fl)
    got = down(hip, y, np.float32, npos * rows).reshape(npos, rows)
    want = np.zeros((npos, rows), dtype=np.float32)
    for e, m0, c in spans:
        we = w[e * rows:(e + 1) * rows]
        for m in range(m0, m0 + c):
            want[m] = O.matvec(ty, we, rows, cols, x[xrow[m]])
    assert max_rel_err(got, want) <= TOL, max_rel_err(got, want)
    if ty != ggml.IQ4_XS:
        # the CPU dots' float steps per super-block (per 32-block for Q8_0), in order: the same bits. IQ4_XS closes
        # each 32-value sub-block in float on the CPU (src/cpu_moe.rs:195-212), here once per super-block.
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int((got != want).sum())
    # act 1: y = silu(y) * (W x) with the same x (SAME_X), then act 2: y += W x
    hip.gemm(ty, rows, cols, tiles, nt, xb, cols, n_x, xr, y, rows, S.ACT_SWIGLU | S.SAME_X | fl)
    got2 = down(hip, y, np.float32, npos * rows).reshape(npos, rows)
    want2 = want / (1 + np.exp(-want.astype(np.float64))) * want
    assert max_rel_err(got2, want2) <= TOL
    hip.gemm(ty, rows, cols, tiles, nt, xb, cols, n_x, xr, y, rows, S.ACT_ADD | S.SAME_X | fl)
    got3 = down(hip, y, np.float32, npos * rows).reshape(npos, rows)
    assert max_rel_err(got3, want2 + want) <= TOL


@pytest.mark.parametrize("ty", [ggml.Q4_K, ggml.Q5_K, ggml.Q6_K, ggml.IQ2_XXS, ggml.IQ3_S, ggml.IQ4_XS, ggml.Q2_K, ggml.Q3_K])
def test_gemm_small_tiles_same_bits_random_lists(hip, ty):
    """The 64-position GEMM form against the 256-position one over seeded random tile lists (counts 1-256, so tiles
    of more than 64 positions run as several chunks; experts in random order, gathered X rows, partial row blocks):
    the same bits for every type (IQ4_XS included: both forms close its super-blocks from the same integer sum)."""
    rng = np.random.default_rng(900 + ty)
    rows, cols, E, n_x = 136, 768, 5, 60
    rb = ggml.row_bytes(ty, cols)
    w = random_blocks(ty, E * rows, cols, seed=901 + ty)
    wb = up(hip, w)
    x = normal((n_x, cols), seed=902 + ty)
    spans, m0 = [], 0
    for _ in range(9):
        c = int(rng.integers(1, 257))
        spans.append((int(rng.integers(0, E)), m0, c))
        m0 += c
    npos = m0
    xrow = rng.integers(0, n_x, npos).astype(np.int32)
    tiles, nt = tile_list(hip, int(wb), rows * rb, spans)
    xb, xr = up(hip, x), up(hip, xrow)
    ya, yb = hip.alloc(npos * rows * 4), hip.alloc(npos * rows * 4)
    hip.gemm(ty, rows, cols, tiles, nt, xb, cols, n_x, xr, ya, rows, S.ACT_STORE)
    hip.gemm(ty, rows, cols, tiles, nt, xb, cols, n_x, xr, yb, rows, S.ACT_STORE | S.SAME_X | S.SMALL_TILES)
    a, b = down(hip, ya, np.uint32, npos * rows), down(hip, yb, np.uint32, npos * rows)
    assert np.array_equal(a, b), int((a != b).sum())


@pytest.mark.parametrize("seed", range(6))
def test_gemm_plans_over_random_lists(hip, seed):
    """Both GEMM forms over seeded random tile lists of 1-500 tiles (1-256 positions each, experts in random order,
    gathered X rows) and 64-2048 rows: the 256-position form (its items planned over the XCDs) and the 64-position form
    (planned over the grid) give the same bits, and sampled positions carry the CPU dots' bits."""
    rng = np.random.default_rng(1400 + seed)
    ty = [ggml.Q4_K, ggml.Q5_K, ggml.Q6_K, ggml.Q2_K, ggml.Q3_K, ggml.IQ3_S][seed]
    rows = int(rng.choice([64, 128, 200, 384, 1024, 2048]))
    cols, E, n_x = 512, 7, 96
    n_tiles = int(rng.integers(1, 501))
    cmax = int(rng.choice([8, 64, 256]))
    rb = ggml.row_bytes(ty, cols)
    w = random_blocks(ty, E * rows, cols, seed=1401 + seed)
    wb = up(hip, w)
    x = normal((n_x, cols), seed=1402 + seed)
    spans, m0 = [], 0
    for _ in range(n_tiles):
        c = int(rng.integers(1, cmax + 1))
        spans.append((int(rng.integers(0, E)), m0, c))
        m0 += c
    npos = m0
    xrow = rng.integers(0, n_x, npos).astype(np.int32)
    tiles, nt = tile_list(hip, int(wb), rows * rb, spans)
    xb, xr = up(hip, x), up(hip, xrow)
    ya, yb = hip.alloc(npos * rows * 4), hip.alloc(npos * rows * 4)
    hip.gemm(ty, rows, cols, tiles, nt, xb, cols, n_x, xr, ya, rows, S.ACT_STORE)
    hip.gemm(ty, rows, cols, tiles, nt, xb, cols, n_x, xr, yb, rows, S.ACT_STORE | S.SAME_X | S.SMALL_TILES)
    a, b = down(hip, ya, np.uint32, npos * rows), down(hip, yb, np.uint32, npos * rows)
    assert np.array_equal(a, b), int((a != b).sum())
    got = a.view(np.float32).reshape(npos, rows)
    starts = np.array([m for _, m, _ in spans])
    for m in rng.choice(npos, min(npos, 24), replace=False):
        e = spans[int(np.searchsorted(starts, m, side="right")) - 1][0]
        want = O.matvec(ty, w[e * rows:(e + 1) * rows], rows, cols, x[xrow[m]])
        assert np.array_equal(got[m].view(np.uint32), want.view(np.uint32)), (int(m), e)


@pytest.mark.parametrize("ty", [ggml.Q4_K, ggml.Q6_K])
@pytest.mark.parametrize("case", ["plan_300", "count_600", "index_order"])
def test_gemm_item_plans_cover_every_tile(hip, ty, case):
    """The GEMMs' ways of dealing a tile list's items to their blocks, each against the CPU dots (the same bits), with
    the 64-position form bit-equal to the 256-position one: plan_300, 300 tiles of 1-256 positions (the cost split over
    the XCDs and the larger-tiles-first order); count_600, 600 tiles of 1-20 positions (past the 512 tiles a block
    plans: an eighth of the items an XCD, and index order over the grid); index_order, 80 tiles over 32768 rows (256
    row blocks a tile: past 64 items a block, the plan's range dealt in index order)."""
    rng = np.random.default_rng(1300 + ty + len(case))
    if case == "index_order":
        rows, cols, E, n_tiles, cmax = 32768, 256, 2, 80, 3
    else:
        rows, cols, E = 200, 512, 6
        n_tiles, cmax = (300, 256) if case == "plan_300" else (600, 20)
    rb = ggml.row_bytes(ty, cols)
    w = random_blocks(ty, E * rows, cols, seed=1301 + ty)
    wb = up(hip, w)
    n_x = 64
    x = normal((n_x, cols), seed=1302 + ty)
    spans, m0 = [], 0
    for _ in range(n_tiles):
        c = int(rng.integers(1, cmax + 1))
        spans.append((int(rng.integers(0, E)), m0, c))
        m0 += c
    npos = m0
    xrow = rng.integers(0, n_x, npos).astype(np.int32)
    tiles, nt = tile_list(hip, int(wb), rows * rb, spans)
    y, y64 = hip.alloc(npos * rows * 4), hip.alloc(npos * rows * 4)
    xb, xr = up(hip, x), up(hip, xrow)
    hip.gemm(ty, rows, cols, tiles, nt, xb, cols, n_x, xr, y, rows, S.ACT_STORE)
    # the 64-position form over the same list (index_order: past 64 items a block of its grid too)
    hip.gemm(ty, rows, cols, tiles, nt, xb, cols, n_x, xr, y64, rows, S.ACT_STORE | S.SAME_X | S.SMALL_TILES)
    got = down(hip, y, np.float32, npos * rows).reshape(npos, rows)
    got64 = down(hip, y64, np.float32, npos * rows).reshape(npos, rows)
    assert np.array_equal(got.view(np.uint32), got64.view(np.uint32)), int((got != got64).sum())
    # one CPU dot per (expert, X row) pair, shared by the positions that gather it
    cache = {}
    want = np.empty((npos, rows), dtype=np.float32)
    for e, m0, c in spans:
        for m in range(m0, m0 + c):
            key = (e, int(xrow[m]))
            if key not in cache:
                cache[key] = O.matvec(ty, w[e * rows:(e + 1) * rows], rows, cols, x[xrow[m]])
            want[m] = cache[key]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int((got != want).sum())


@pytest.mark.parametrize("ty", [ggml.Q4_K, ggml.Q5_K, ggml.Q6_K, ggml.IQ2_XXS, ggml.IQ3_S, ggml.IQ4_XS, ggml.Q2_K, ggml.Q3_K])
@pytest.mark.parametrize("fl", [0, S.SMALL_TILES], ids=["blocks256", "small64"])
def test_gemm_gate_up_fused_matches_two_calls(hip, ty, fl):
    """gemm_grouped_gate_up gives the bits of gemm (gate, act store) followed by gemm (up, act SwiGLU, same X) over the
    same tiles (src/gpu_model/prefill.rs), with partial and full 256-position tiles and 3 column blocks of 64."""
    rows, cols, E, n_x = 192, 512, 3, 100
    rb = ggml.row_bytes(ty, cols)
    w = random_blocks(ty, 2 * E * rows, cols, seed=100 + ty)  # gate experts, then up experts
    wb = up(hip, w)
    up_off = E * rows * rb
    x = normal((n_x, cols), seed=5)
    npos = 626
    xrow = np.random.default_rng(6).integers(0, n_x, npos).astype(np.int32)
    spans = [(0, 0, 128), (2, 128, 16), (1, 144, 26), (2, 170, 256), (0, 426, 200)]
    tg, nt = tile_list(hip, int(wb), rows * rb, spans)
    tu, _ = tile_list(hip, int(wb) + up_off, rows * rb, spans)
    ntd = up(hip, np.array([nt], dtype=np.int32))
    xb, xr = up(hip, x), up(hip, xrow)
    y1, y2 = hip.alloc(npos * rows * 4), hip.alloc(npos * rows * 4)
    hip.gemm(ty, rows, cols, tg, nt, xb, cols, n_x, xr, y1, rows, S.ACT_STORE)
    hip.gemm(ty, rows, cols, tu, nt, xb, cols, n_x, xr, y1, rows, S.ACT_SWIGLU | S.SAME_X)
    hip.gemm_grouped_gate_up(ty, rows, cols, tg, nt, ntd, xb, cols, n_x, xr, y2, rows, up_off, flags=fl)
    a, b = down(hip, y1, np.float32, npos * rows), down(hip, y2, np.float32, npos * rows)
    assert np.array_equal(a, b), np.abs(a - b).max()
    # against the oracle through the gate and up results
    want_g = np.zeros((npos, rows), dtype=np.float32)
    want_u = np.zeros((npos, rows), dtype=np.float32)
    for e, m0, c in spans:
        for m in range(m0, m0 + c):
            want_g[m] = O.matvec(ty, w[e * rows:(e + 1) * rows], rows, cols, x[xrow[m]])
            want_u[m] = O.matvec(ty, w[(E + e) * rows:(E + e + 1) * rows], rows, cols, x[xrow[m]])
    with np.errstate(over="ignore"):
        want = want_g / (1 + np.exp(-want_g.astype(np.float64))) * want_u
    assert max_rel_err(b.reshape(npos, rows), want) <= TOL
    with pytest.raises(S.StrataError, match="a multiple of 64"):
        hip.gemm_grouped_gate_up(ty, 200, cols, tg, nt, ntd, xb, cols, n_x, xr, y2, 200, up_off)
    with pytest.raises(S.StrataError, match="Q8_0 has no fused"):
        hip.gemm_grouped_gate_up(ggml.Q8_0, rows, cols, tg, nt, ntd, xb, cols, n_x, xr, y2, rows, up_off)


@pytest.mark.parametrize("ty", [ggml.Q5_K, ggml.Q8_0])
def test_gemm_dense(hip, ty):
    rows, cols, n = 200, 1024, 300
    w = random_blocks(ty, rows, cols, seed=8)
    t = hip.upload_tensor(ty, w)
    x = normal((n, cols), seed=9)
    y = hip.alloc(n * rows * 4)
    hip.gemm_dense(t, n, up(hip, x), cols, y, rows, S.ACT_STORE)
    got = down(hip, y, np.float32, n * rows).reshape(n, rows)
    want = np.stack([O.matvec(ty, w, rows, cols, x[i]) for i in range(n)])
    assert max_rel_err(got, want) <= TOL


@pytest.mark.parametrize("ty", [ggml.Q2_K, ggml.Q4_K, ggml.Q5_K, ggml.Q6_K, ggml.IQ3_S, ggml.Q8_0])
def test_gemm_dense_bits_over_random_shapes(hip, ty):
    """gemm_dense against the CPU dot's bits over seeded random shapes: rows 1-400 (partial 128-row blocks), 256-4096
    columns, 1-600 positions (partial 256-position blocks), weight scales 2^-12..2^2."""
    rng = np.random.default_rng(700 + ty)
    for case in range(3):
        rows, cols, n = int(rng.integers(1, 401)), 256 * int(rng.integers(1, 17)), int(rng.integers(1, 601))
        lo = float(2.0 ** rng.integers(-12, 2))
        w = random_blocks(ty, rows, cols, seed=int(rng.integers(1 << 30)), scale=(lo, 2 * lo))
        x = normal((n, cols), seed=int(rng.integers(1 << 30)))
        t = hip.upload_tensor(ty, w)
        y = hip.alloc(n * rows * 4)
        hip.gemm_dense(t, n, up(hip, x), cols, y, rows, S.ACT_STORE)
        got = down(hip, y, np.float32, n * rows).reshape(n, rows)
        want = np.stack([O.matvec(ty, w, rows, cols, x[i]) for i in range(n)])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (case, rows, cols, n, int((got != want).sum()))


def moe_weights(E, H, F, seed):
    gate = random_blocks(ggml.Q5_K, E * F, H, seed=seed)
    upw = random_blocks(ggml.Q5_K, E * F, H, seed=seed + 1)
    dn = random_blocks(ggml.Q6_K, E * H, F, seed=seed + 2)
    return gate, upw, dn


def test_moe_prefill_layer_matches_experts_multi(hip):
    """route -> device sort -> grouped gate / up (SwiGLU) / down -> combine_seq, against cpu_moe::experts_multi."""
    E, H, F, T, k = 16, 512, 256, 96, 4
    gate, upw, dn = moe_weights(E, H, F, seed=40)
    hs = normal((T, H), seed=41)
    logits = zipf_logits(T, E, seed=42)
    ids_w, wts_w = O.route(logits, k)
    want = O.experts_multi(ggml.Q5_K, ggml.Q6_K, gate, upw, dn, H, F, hs, ids_w, wts_w)
    got = run_prefill(hip, E, H, F, T, k, gate, upw, dn, hs, logits)
    assert max_rel_err(got, want) <= TOL, max_rel_err(got, want)
    # gate and up as one grouped GEMM, and the 64-position kernel over 64-position tiles: the same bits
    assert np.array_equal(run_prefill(hip, E, H, F, T, k, gate, upw, dn, hs, logits, fused=True), got)
    assert np.array_equal(run_prefill(hip, E, H, F, T, k, gate, upw, dn, hs, logits, fused=True, small=True), got)


def test_moe_prefill_layer_full_size(hip):
    """configs[2] at its full size (128 experts, hidden 2048, intermediate 768, top-8, 4096 tokens, Zipf-skewed
    routing): the device layer against cpu_moe::experts_multi on every token, and the fused gate/up launch equal to
    the two-call sequence bit for bit."""
    E, H, F, T, k = 128, 2048, 768, 4096, 8
    gate, upw, dn = moe_weights(E, H, F, seed=140)
    hs = normal((T, H), seed=141)
    logits = zipf_logits(T, E, seed=142)
    ids_w, wts_w = O.route(logits, k)
    want = O.experts_multi(ggml.Q5_K, ggml.Q6_K, gate, upw, dn, H, F, hs, ids_w, wts_w,
                           threads=min(16, os.cpu_count() or 1))
    got = run_prefill(hip, E, H, F, T, k, gate, upw, dn, hs, logits, fused=True)
    assert max_rel_err(got, want) <= TOL, max_rel_err(got, want)
    assert np.array_equal(run_prefill(hip, E, H, F, T, k, gate, upw, dn, hs, logits), got)


def test_moe_prefill_layer_512_tokens(hip):
    """configs[2] at its 512-token size (128 experts, Zipf-skewed: most experts get a few dozen routed rows, so the
    grouped GEMMs run their small-tile form): the device layer against cpu_moe::experts_multi on every token, fused
    and unfused gate/up bit for bit."""
    E, H, F, T, k = 128, 2048, 768, 512, 8
    gate, upw, dn = moe_weights(E, H, F, seed=240)
    hs = normal((T, H), seed=241)
    logits = zipf_logits(T, E, seed=242)
    ids_w, wts_w = O.route(logits, k)
    want = O.experts_multi(ggml.Q5_K, ggml.Q6_K, gate, upw, dn, H, F, hs, ids_w, wts_w,
                           threads=min(16, os.cpu_count() or 1))
    got = run_prefill(hip, E, H, F, T, k, gate, upw, dn, hs, logits, fused=True, small=True)
    assert max_rel_err(got, want) <= TOL, max_rel_err(got, want)
    assert np.array_equal(run_prefill(hip, E, H, F, T, k, gate, upw, dn, hs, logits, small=True), got)
    assert np.array_equal(run_prefill(hip, E, H, F, T, k, gate, upw, dn, hs, logits, fused=True), got)


def run_prefill(hip, E, H, F, T, k, gate, upw, dn, hs, logits, fused=False, small=False):
    """The prefill MoE block; small: tiles of at most 64 positions and the 64-position GEMM kernel."""
    rb_gu, rb_d = ggml.row_bytes(ggml.Q5_K, H), ggml.row_bytes(ggml.Q6_K, F)
    g_b, u_b, d_b = up(hip, gate), up(hip, upw), up(hip, dn)
    hb, lb = up(hip, hs), up(hip, logits)
    ids, wts = hip.alloc(T * k * 4), hip.alloc(T * k * 4)
    hip.router_topk(lb, E, k, 0.0, ids, wts, T)
    chunk = 64 if small else hip.gemm_block_positions()
    fl = S.SMALL_TILES if small else 0
    max_tiles = T * k // chunk + E
    off, xrow, inv = hip.alloc((E + 1) * 4), hip.alloc(T * k * 4), hip.alloc(T * k * 4)
    tiles, ntd = hip.alloc(3 * max_tiles * 16), hip.alloc(4)
    hip.moe_sort(ids, T, k, E, off, xrow, inv, [(int(g_b), F * rb_gu), (int(u_b), F * rb_gu), (int(d_b), H * rb_d)],
                 tiles, max_tiles, ntd, chunk=chunk)
    ge, ye = hip.alloc(T * k * F * 4), hip.alloc(T * k * H * 4)
    if fused:
        hip.gemm_grouped_gate_up(ggml.Q5_K, F, H, tiles, max_tiles, ntd, hb, H, T, xrow, ge, F, int(u_b) - int(g_b),
                                 flags=fl)
    else:
        hip.gemm_grouped(ggml.Q5_K, F, H, tiles, max_tiles, ntd, hb, H, T, xrow, ge, F, S.ACT_STORE | fl)
        hip.gemm_grouped(ggml.Q5_K, F, H, int(tiles) + max_tiles * 16, max_tiles, ntd, hb, H, T, xrow, ge, F,
                         S.ACT_SWIGLU | S.SAME_X | fl)
    hip.gemm_grouped(ggml.Q6_K, H, F, int(tiles) + 2 * max_tiles * 16, max_tiles, ntd, ge, F, T * k, 0, ye, H,
                     S.ACT_STORE | fl)
    x = hip.alloc(T * H * 4)
    hip.moe_combine_seq(x, ye, wts, inv, k, 0, 0, H, T)
    return down(hip, x, np.float32, T * H).reshape(T, H)


def test_moe_decode_layer_matches_experts(hip):
    """The decode sequence of src/gpu_model.rs:3383-3412: moe_route -> paired gate/up moe_gemv -> swiglu_q ->
    moe_down_combine, against cpu_moe::experts, at configs[2]'s shape (128 experts)."""
    E, H, F, k = 128, 2048, 768, 8
    gate, upw, dn = moe_weights(E, H, F, seed=50)
    h = normal(H, seed=51)
    logits = zipf_logits(1, E, seed=52)
    ids_w, wts_w = O.route(logits, k)
    want = O.experts_multi(ggml.Q5_K, ggml.Q6_K, gate, upw, dn, H, F, h[None, :], ids_w, wts_w)[0]
    rb_gu, rb_d = ggml.row_bytes(ggml.Q5_K, H), ggml.row_bytes(ggml.Q6_K, F)
    gu = up(hip, np.concatenate([gate, upw]))
    d_b = up(hip, dn)
    table = up(hip, np.arange(E, dtype=np.int32))
    ids, wts, slots, wh = [hip.alloc(k * 4) for _ in range(4)]
    hip.moe_route(up(hip, logits), E, k, 0.0, table, ids, wts, slots, wh, 1)
    hb = up(hip, h)
    xq = hip.alloc(H + H // 8)
    hip.quant_xq(hb, H, H, 1, xq)
    g = hip.alloc(2 * k * F * 4)
    hip.moe_gemv(ggml.Q5_K, F, H, gu, F * rb_gu, slots, k, hb, H, k, g, pair=(E * F * rb_gu, k * F * 4), xq=xq)
    aq = hip.alloc(k * (F + F // 8))
    aqr = hip.swiglu_q(g, int(g) + k * F * 4, F, k, aq)
    x = hip.alloc(H * 4)
    ye = hip.alloc(k * H * 4)
    hip.moe_down_combine(ggml.Q6_K, H, F, d_b, H * rb_d, slots, k, 0, ye, aqr, x, wh, 0, 0, 1)
    got = down(hip, x, np.float32, H)
    assert max_rel_err(got, want) <= TOL, max_rel_err(got, want)
    # h quantized inside the gate/up GEMV and the fused tail (swiglu inside the down GEMV): the same bits
    g2, x2 = hip.alloc(2 * k * F * 4), hip.alloc(H * 4)
    hip.moe_gemv(ggml.Q5_K, F, H, gu, F * rb_gu, slots, k, hb, H, k, g2, pair=(E * F * rb_gu, k * F * 4))
    assert np.array_equal(down(hip, g2, np.float32, 2 * k * F), down(hip, g, np.float32, 2 * k * F))
    hip.moe_down_swiglu_combine(ggml.Q6_K, H, F, d_b, H * rb_d, slots, k, g2, int(g2) + k * F * 4, ye, x2, wh, 0, 0, 1)
    assert np.array_equal(down(hip, x2, np.float32, H), got)
    # the whole token (route, gate/up, fused tail) recorded as a graph (the way the reference's decode replays CUDA
    # graphs, src/cuda/mod.rs:868-888): each replay, with other logits and eager work in between, equals the eager
    # token bit for bit
    lb = up(hip, logits)

    def token(xo):
        hip.moe_route(lb, E, k, 0.0, table, ids, wts, slots, wh, 1)
        hip.moe_gemv(ggml.Q5_K, F, H, gu, F * rb_gu, slots, k, hb, H, k, g2, pair=(E * F * rb_gu, k * F * 4))
        hip.moe_down_swiglu_combine(ggml.Q6_K, H, F, d_b, H * rb_d, slots, k, g2, int(g2) + k * F * 4, ye, xo, wh,
                                    0, 0, 1)

    x3 = hip.alloc(H * 4)
    hip.graph("decode", lambda: token(x3))
    for i in range(3):
        hip.htod(zipf_logits(1, E, seed=90 + i), lb)
        hip.htod(np.zeros(H, dtype=np.float32), x3)
        hip.graph("decode", None)
        got_g = down(hip, x3, np.float32, H)
        x4 = hip.alloc(H * 4)
        token(x4)
        assert np.array_equal(got_g, down(hip, x4, np.float32, H)), i
        iw, ww = O.route(zipf_logits(1, E, seed=90 + i), k)
        want_i = O.experts_multi(ggml.Q5_K, ggml.Q6_K, gate, upw, dn, H, F, h[None, :], iw, ww)[0]
        assert max_rel_err(got_g, want_i) <= TOL, (i, max_rel_err(got_g, want_i))
    hip.drop_graphs()


@pytest.mark.parametrize("numerics", [S.NUM_Q8K, S.NUM_Q8_32])
@pytest.mark.parametrize("F", [768, 3072])
def test_moe_down_swiglu_combine_matches_unfused(hip, numerics, F):
    """The fused decode tail gives the same x bits as swiglu_q, the down moe_gemv and moe_combine as three launches
    (src/gpu_model.rs:3383-3412), with x quantized inside (moe_down_swiglu_combine) or from xq (moe_down_combine);
    3 tokens, a shared expert, a slot not resident and a slot of weight 0. F = 3072: 16 lanes a row, 2 rows a block."""
    E, H, k, t = 16, 512, 8, 3
    _, _, dn = moe_weights(E, H, F, seed=60)
    rb_d = ggml.row_bytes(ggml.Q6_K, F)
    d_b = up(hip, dn)
    rng = np.random.default_rng(61)
    sl = rng.integers(0, E, t * k).astype(np.int32)
    sl[4] = -1
    w = rng.random(t * k).astype(np.float32)
    w[4] = 0.0
    w[13] = 0.0
    slots, wh = up(hip, sl), up(hip, w)
    gu = rng.standard_normal((2, t * k, F)).astype(np.float32) * 3
    g = up(hip, gu)
    u = int(g) + t * k * F * 4
    sh, sg = up(hip, normal((t, H), seed=62)), up(hip, normal(t, seed=63))
    x0 = normal((t, H), seed=64)
    old = hip.numerics()
    hip.set_numerics(numerics)
    try:
        xa, xb, xc = up(hip, x0), up(hip, x0), up(hip, x0)
        ya, yb = hip.alloc(t * k * H * 4), hip.alloc(t * k * H * 4)
        aq = hip.alloc(t * k * (F + F // 8))
        aqr = hip.swiglu_q(g, u, F, t * k, aq)
        hip.moe_gemv(ggml.Q6_K, H, F, d_b, H * rb_d, slots, t * k, 0, F, 1, ya, xq=aqr)
        hip.moe_combine(xa, ya, wh, k, sh, sg, H, t)
        hip.moe_down_combine(ggml.Q6_K, H, F, d_b, H * rb_d, slots, k, 0, yb, aqr, xb, wh, sh, sg, t)
        hip.moe_down_swiglu_combine(ggml.Q6_K, H, F, d_b, H * rb_d, slots, k, g, u, yb, xc, wh, sh, sg, t)
    finally:
        hip.set_numerics(old)
    ga = down(hip, xa, np.float32, t * H)
    assert np.array_equal(ga, down(hip, xb, np.float32, t * H))
    assert np.array_equal(ga, down(hip, xc, np.float32, t * H))
    with pytest.raises(S.StrataError, match="null g or u"):
        hip.moe_down_swiglu_combine(ggml.Q6_K, H, F, d_b, H * rb_d, slots, k, g, 0, yb, xb, wh, 0, 0, t)


@pytest.mark.parametrize("ty", ggml.TYPES)
@pytest.mark.parametrize("k,F,t", [(8, 768, 1), (4, 512, 2), (6, 1024, 1), (16, 256, 2)])
def test_down_combine_one_launch_all_types(hip, ty, k, F, t):
    """moe_down_combine as one launch (every slot of a block's rows in the block) against moe_gemv + moe_combine
    bit for bit, for every type, slot counts that do and do not divide the block's pairs (k = 6: 10 rows a block),
    a partial last row block (H = 1000), a slot not resident; and against the oracle."""
    E, H = 5, 1000
    rb = ggml.row_bytes(ty, F)
    dn = random_blocks(ty, E * H, F, seed=300 + ty)
    d_b = up(hip, dn)
    rng = np.random.default_rng(301)
    sl = rng.integers(0, E, t * k).astype(np.int32)
    sl[1] = -1
    w = rng.uniform(0.1, 0.5, t * k).astype(np.float32)
    w[1] = 0.0
    slots, wh = up(hip, sl), up(hip, w)
    h = normal((t * k, F), seed=302)
    hb = up(hip, h)
    xq = hip.alloc(t * k * (F + F // 8))
    hip.quant_xq(hb, F, F, t * k, xq)
    x0 = normal((t, H), seed=303)
    xa, xb = up(hip, x0), up(hip, x0)
    ya, yb = hip.alloc(t * k * H * 4), hip.alloc(t * k * H * 4)
    hip.moe_gemv(ty, H, F, d_b, H * rb, slots, t * k, hb, F, 1, ya, xq=xq)
    hip.moe_combine(xa, ya, wh, k, 0, 0, H, t)
    hip.moe_down_combine(ty, H, F, d_b, H * rb, slots, k, hb, yb, xq, xb, wh, 0, 0, t)
    ga, gb = down(hip, xa, np.float32, t * H), down(hip, xb, np.float32, t * H)
    assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), int((ga != gb).sum())
    want = x0.astype(np.float64).copy()
    for tt in range(t):
        for j in range(k):
            e = sl[tt * k + j]
            if e >= 0 and w[tt * k + j] != 0:
                want[tt] += w[tt * k + j] * O.matvec(ty, dn[e * H:(e + 1) * H], H, F, h[tt * k + j])
    assert max_rel_err(gb.reshape(t, H), want) <= TOL


@pytest.mark.parametrize("ty", ggml.TYPES)
@pytest.mark.parametrize("n,k,F,H,pair,sig", [(128, 8, 768, 2048, True, False), (64, 4, 512, 1024, False, True),
                                              (96, 6, 300, 512, True, False), (256, 8, 256, 512, False, False)])
def test_moe_route_gemv_equals_two_launches(hip, ty, n, k, F, H, pair, sig):
    """moe_route_gemv (the route of one token computed by every block of its gate/up GEMV) gives ids, wts, slots, wh
    and the experts' outputs bit for bit equal to moe_route then moe_gemv (src/gpu_model.rs:3383-3390): softmax and
    sigmoid routing, an extra scale, experts not resident (table -1), the paired launch, x as f32 or pre-quantized,
    n = 256 (routed by its own launch), three tokens in a row (no state kept between launches)."""
    cols = F if F % 256 == 0 else 256
    rb = ggml.row_bytes(ty, cols)
    wm = random_blocks(ty, (2 if pair else 1) * n * F, cols, seed=500 + ty)
    wb = up(hip, wm)
    tab = np.arange(n, dtype=np.int32)
    tab[::5] = -1
    table = up(hip, tab)
    x = normal(cols, seed=501)
    xb = up(hip, x)
    xq = hip.alloc(cols + cols // 8)
    hip.quant_xq(xb, cols, cols, 1, xq)
    pr = (n * F * rb, k * F * 4) if pair else None
    outs = [[hip.alloc(k * 4) for _ in range(4)] + [hip.alloc(2 * k * F * 4)] for _ in range(2)]
    for tok in range(3):
        lb = up(hip, zipf_logits(1, n, seed=510 + tok)[0])
        for q in (0, xq):
            ids, wts, slots, wh, y = outs[0]
            hip.moe_route(lb, n, k, 0.5, table, ids, wts, slots, wh, 1, sigmoid=sig)
            hip.moe_gemv(ty, F, cols, wb, F * rb, slots, k, xb, cols, k, y, pair=pr, xq=q)
            ids2, wts2, slots2, wh2, y2 = outs[1]
            hip.moe_route_gemv(lb, n, k, 0.5, table, ids2, wts2, slots2, wh2, ty, F, cols, wb, F * rb, xb, y2,
                               pair=pr, xq=q, sigmoid=sig)
            for a, b, dt in ((ids, ids2, np.int32), (wts, wts2, np.float32), (slots, slots2, np.int32),
                             (wh, wh2, np.float32)):
                assert np.array_equal(down(hip, a, dt, k).view(np.uint32), down(hip, b, dt, k).view(np.uint32)), tok
            ya, yb = down(hip, y, np.float32, 2 * k * F), down(hip, y2, np.float32, 2 * k * F)
            assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), (tok, int((ya != yb).sum()))


def test_moe_route_gemv_division_ties(hip):
    """moe_route_gemv on tokens whose softmax division ties two experts (the ranking of the unnormalised values names
    them in the other order, so blocks that requested their first tile from the ranking request it again): ids equal
    ops::top_k's, and every output equals moe_route then moe_gemv bit for bit."""
    logits, flips = _division_tie_logits(12, seed=7)
    assert flips >= 3
    n, k, F, cols = 128, 8, 256, 512
    ty = ggml.Q4_K
    rb = ggml.row_bytes(ty, cols)
    wb = up(hip, random_blocks(ty, 2 * n * F, cols, seed=77))
    table = up(hip, np.arange(n, dtype=np.int32))
    xb = up(hip, normal(cols, seed=78))
    pr = (n * F * rb, k * F * 4)
    for row in logits:
        lb = up(hip, row)
        a = [hip.alloc(k * 4) for _ in range(4)] + [hip.alloc(2 * k * F * 4)]
        b = [hip.alloc(k * 4) for _ in range(4)] + [hip.alloc(2 * k * F * 4)]
        hip.moe_route(lb, n, k, 0.0, table, a[0], a[1], a[2], a[3], 1)
        hip.moe_gemv(ty, F, cols, wb, F * rb, a[2], k, xb, cols, k, a[4], pair=pr)
        hip.moe_route_gemv(lb, n, k, 0.0, table, b[0], b[1], b[2], b[3], ty, F, cols, wb, F * rb, xb, b[4], pair=pr)
        wi, _ = O.route(row[None, :], k)
        assert np.array_equal(down(hip, b[0], np.int32, k), wi.reshape(-1))
        for x, y, m in zip(a, b, (k, k, k, k, 2 * k * F)):
            assert np.array_equal(down(hip, x, np.uint32, m), down(hip, y, np.uint32, m))


@pytest.mark.parametrize("ty", [ggml.Q6_K, ggml.Q4_K, ggml.Q8_0])
def test_gemm_from_rms_norm_q_xq(hip, ty):
    """STRATA_X_Q: a GEMM over the X that rms_norm_q quantized beside its output (the prefill's norms feeding the
    q/k/v and gate/up GEMMs) equals the GEMM quantizing the f32 output itself, bit for bit (gemm_dense and the fused
    gate/up grouped GEMM); a quantized X with another row stride is an error."""
    T, H, R = 300, 512, 192
    x = normal((T, H), seed=90)
    w = np.random.default_rng(91).uniform(0.5, 1.5, H).astype(np.float32)
    xb, wb = up(hip, x), up(hip, w)
    h = hip.alloc(T * H * 4)
    xq = hip.alloc(T * (H + H // 8))
    hip.rms_norm_q(xb, H, wb, h, H, H, T, 1e-6, xq=xq)
    W = hip.upload_tensor(ty, random_blocks(ty, R, H, seed=92 + ty))
    ya, yb = hip.alloc(T * R * 4), hip.alloc(T * R * 4)
    hip.gemm_dense(W, T, h, H, ya, R, S.ACT_STORE)
    hip.gemm_dense(W, T, xq, H, yb, R, S.ACT_STORE | S.X_Q)
    assert np.array_equal(down(hip, ya, np.uint32, T * R), down(hip, yb, np.uint32, T * R))
    with pytest.raises(S.StrataError, match="quantized X"):
        hip.gemm_dense(W, T, xq, 2 * H, yb, R, S.ACT_STORE | S.X_Q)
    if ty == ggml.Q8_0:
        return
    # the fused gate/up grouped GEMM over 2 experts' tiles (rows 0..149 on expert 0, 150..299 on expert 1)
    E, F = 2, 128
    rb = ggml.row_bytes(ty, H)
    gu = up(hip, random_blocks(ty, 2 * E * F, H, seed=93 + ty))
    tiles = np.zeros(2 * 2, dtype=np.uint64)
    for e, (m0, cnt) in enumerate(((0, 150), (150, 150))):
        tiles[2 * e] = int(gu) + e * F * rb
        tiles[2 * e + 1] = m0 | (cnt << 32)
    tb, ntd, xrow = up(hip, tiles), up(hip, np.array([2], dtype=np.int32)), up(hip, np.arange(T, dtype=np.int32))
    ga, gb = hip.alloc(T * F * 4), hip.alloc(T * F * 4)
    hip.gemm_grouped_gate_up(ty, F, H, tb, 2, ntd, h, H, T, xrow, ga, F, E * F * rb)
    hip.gemm_grouped_gate_up(ty, F, H, tb, 2, ntd, xq, H, T, xrow, gb, F, E * F * rb, flags=S.X_Q)
    assert np.array_equal(down(hip, ga, np.uint32, T * F), down(hip, gb, np.uint32, T * F))


def test_errors_do_not_launch(hip):
    t = S.GpuTensor(ggml.Q4_K, 4, 300, hip.alloc(4 * 2048))
    with pytest.raises(S.StrataError, match="GEMV needs a multiple of 256"):
        hip.gemv(t, 0, 0)
    t = S.GpuTensor(ggml.Q4_K, 4, 512, hip.alloc(4 * 2048))
    with pytest.raises(S.StrataError, match="gemvn: 5 inputs"):
        hip.gemvn(t, 0, 0, 0, 0, 5)
    with pytest.raises(S.StrataError, match="unsupported quant type"):
        hip.gemv(S.GpuTensor(99, 1, 256, hip.alloc(64)), 0, 0)
    b = hip.alloc(16)
    with pytest.raises(S.StrataError, match="outside"):
        hip.htod(np.zeros(32, dtype=np.uint8), b)


def test_graph_replays_read_device_memory(hip):
    """Backend::graph (src/backend.rs:118-120): a recorded GEMV sequence replays with the values device memory holds
    at replay time; replays interleave with eager work and each one matches the eager result."""
    ty, rows, cols = ggml.Q4_K, 300, 2048
    w = random_blocks(ty, rows, cols, seed=61)
    t = hip.upload_tensor(ty, w)
    xb, y = hip.alloc(cols * 4), hip.alloc(rows * 4)
    hip.htod(normal(cols, seed=62), xb)
    hip.gemv(t, xb, y)  # warm: any scratch is sized before recording
    hip.graph("g1", lambda: hip.gemv(t, xb, y))
    for i in range(3):
        x = normal(cols, seed=70 + i)
        hip.htod(x, xb)
        hip.graph("g1", None)
        got = down(hip, y, np.float32, rows)
        y2 = hip.alloc(rows * 4)
        hip.gemv(t, xb, y2)  # eager work between replays
        assert np.array_equal(got, down(hip, y2, np.float32, rows)), i
        assert max_rel_err(got, O.matvec(ty, w, rows, cols, x)) <= TOL
    hip.drop_graphs()


def test_moe_gemv_from_gguf_slots(hip, tmp_path):
    """A MoE layer read from a GGUF into expert slots (gate | up | down per slot, src/expert_cache.rs:66-90): the
    paired gate/up moe_gemv and the down moe_gemv address each expert at base + off + e * slot_bytes."""
    from rustingstrata_amd import gguf
    from tests.test_gguf import moe_layer_file
    E, H, F = 4, 512, 256
    p = str(tmp_path / "moe.gguf")
    gate, upw, dn = moe_layer_file(p, E, H, F)
    g = gguf.Gguf(p)
    buf, mats, slot = gguf.upload_experts(hip, g, 0)
    ids = np.array([2, 0, 3], dtype=np.int32)
    k = len(ids)
    x = normal(H, seed=77)
    idb = up(hip, ids)
    y = hip.alloc(2 * k * F * 4)
    hip.moe_gemv(ggml.Q5_K, F, H, int(buf) + mats[0].off, slot, idb, k, up(hip, x), H, k, y,
                 pair=(mats[1].off - mats[0].off, k * F * 4))
    got = down(hip, y, np.float32, 2 * k * F).reshape(2, k, F)
    for j, e in enumerate(ids):
        assert max_rel_err(got[0, j], O.matvec(ggml.Q5_K, gate[e * F:(e + 1) * F], F, H, x)) <= TOL
        assert max_rel_err(got[1, j], O.matvec(ggml.Q5_K, upw[e * F:(e + 1) * F], F, H, x)) <= TOL
    act = normal((k, F), seed=78)
    yd = hip.alloc(k * H * 4)
    hip.moe_gemv(ggml.Q6_K, H, F, int(buf) + mats[2].off, slot, idb, k, up(hip, act), F, 1, yd)
    gd = down(hip, yd, np.float32, k * H).reshape(k, H)
    for j, e in enumerate(ids):
        assert max_rel_err(gd[j], O.matvec(ggml.Q6_K, dn[e * H:(e + 1) * H], H, F, act[j])) <= TOL



def test_moe_prefill_from_gguf_slots(hip, tmp_path):
    """The prefill MoE block over experts uploaded in slots from a GGUF: moe_sort builds the tile lists with the slot
    stride (gate at off[gate], down at off[down]), the fused gate/up GEMM finds up at off[up] - off[gate] from each
    gate, then the down GEMM and the ordered combine; against cpu_moe::experts_multi."""
    from rustingstrata_amd import gguf
    from tests.test_gguf import moe_layer_file
    E, H, F, T, k = 4, 512, 256, 40, 2
    p = str(tmp_path / "moe.gguf")
    gate, upw, dn = moe_layer_file(p, E, H, F)
    g = gguf.Gguf(p)
    buf, mats, slot = gguf.upload_experts(hip, g, 0)
    hs = normal((T, H), seed=90)
    logits = zipf_logits(T, E, seed=91)
    ids_w, wts_w = O.route(logits, k)
    want = O.experts_multi(ggml.Q5_K, ggml.Q6_K, gate, upw, dn, H, F, hs, ids_w, wts_w)
    ids, wts = hip.alloc(T * k * 4), hip.alloc(T * k * 4)
    hip.router_topk(up(hip, logits), E, k, 0.0, ids, wts, T)
    chunk = hip.gemm_block_positions()
    max_tiles = T * k // chunk + E
    off, xrow, inv = hip.alloc((E + 1) * 4), hip.alloc(T * k * 4), hip.alloc(T * k * 4)
    tiles, ntd = hip.alloc(2 * max_tiles * 16), hip.alloc(4)
    hip.moe_sort(ids, T, k, E, off, xrow, inv, [(int(buf) + mats[0].off, slot), (int(buf) + mats[2].off, slot)],
                 tiles, max_tiles, ntd, chunk=chunk)
    ge, ye, x = hip.alloc(T * k * F * 4), hip.alloc(T * k * H * 4), hip.alloc(T * H * 4)
    hb = up(hip, hs)
    hip.gemm_grouped_gate_up(ggml.Q5_K, F, H, tiles, max_tiles, ntd, hb, H, T, xrow, ge, F, mats[1].off - mats[0].off)
    hip.gemm_grouped(ggml.Q6_K, H, F, int(tiles) + max_tiles * 16, max_tiles, ntd, ge, F, T * k, 0, ye, H, S.ACT_STORE)
    hip.moe_combine_seq(x, ye, wts, inv, k, 0, 0, H, T)
    got = down(hip, x, np.float32, T * H).reshape(T, H)
    assert max_rel_err(got, want) <= TOL, max_rel_err(got, want)


@pytest.mark.parametrize("t", [1, 3])
def test_down_combine_equals_two_launches(hip, t):
    """moe_down_combine (src/backend.rs:436-442): the same x bits as moe_gemv followed by moe_combine, with a slot not
    resident (id -1, weight 0) and a slot of weight 0, over repeated calls; and against the oracle."""
    E, H, F, k = 16, 2048, 768, 8
    dn = random_blocks(ggml.Q6_K, E * H, F, seed=71)
    rb = ggml.row_bytes(ggml.Q6_K, F)
    db = up(hip, dn)
    rng = np.random.default_rng(72)
    slots = np.stack([rng.choice(E, k, replace=False) for _ in range(t)]).astype(np.int32)
    slots[0, 3] = -1
    wh = rng.uniform(0.05, 0.3, (t, k)).astype(np.float32)
    wh[0, 3] = 0.0
    wh[-1, 5] = 0.0
    h = normal((t * k, F), seed=73)
    x0 = normal((t, H), seed=74)
    sb, whb, hb = up(hip, slots), up(hip, wh), up(hip, h)
    ye1, ye2 = hip.alloc(t * k * H * 4), hip.alloc(t * k * H * 4)
    xa, xb = up(hip, x0), up(hip, x0)
    for rep in range(3):
        hip.moe_down_combine(ggml.Q6_K, H, F, db, H * rb, sb, k, hb, ye1, 0, xa, whb, 0, 0, t)
        hip.moe_gemv(ggml.Q6_K, H, F, db, H * rb, sb, t * k, hb, F, 1, ye2)
        hip.moe_combine(xb, ye2, whb, k, 0, 0, H, t)
        ga, gb = hip.get(xa, np.float32, t * H), hip.get(xb, np.float32, t * H)
        assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), (rep, int((ga != gb).sum()))
    # and against the oracle: x0 + 3 * sum_j w_j W_j h_j (three calls)
    want = x0.astype(np.float64).copy()
    for tt in range(t):
        for j in range(k):
            if slots[tt, j] >= 0 and wh[tt, j] != 0:
                y = O.matvec(ggml.Q6_K, dn[slots[tt, j] * H:(slots[tt, j] + 1) * H], H, F, h[tt * k + j])
                want[tt] += 3 * wh[tt, j] * y
    assert max_rel_err(ga.reshape(t, H), want) <= TOL



def test_moe_gemv_one_slot_not_resident(hip):
    """A single MoE slot whose id is -1 leaves its output untouched (the one-slot launch is not a plain matrix);
    with a resident id it is that expert's matvec."""
    ty, rows, cols, E = ggml.Q4_K, 64, 512, 3
    rb = ggml.row_bytes(ty, cols)
    wblk = random_blocks(ty, E * rows, cols, seed=91)
    wb = up(hip, wblk)
    x = normal(cols, seed=92)
    xb = up(hip, x)
    for e in (-1, 2):
        y = up(hip, np.full(rows, 3.5, np.float32))
        hip.moe_gemv(ty, rows, cols, wb, rows * rb, up(hip, np.array([e], np.int32)), 1, xb, cols, 1, y)
        got = down(hip, y, np.float32, rows)
        if e < 0:
            assert np.all(got == np.float32(3.5))
        else:
            assert max_rel_err(got, O.matvec(ty, wblk[e * rows:(e + 1) * rows], rows, cols, x)) <= TOL


def _division_tie_logits(count, seed):
    """Router logit rows (128 experts) in which two experts among the top 8 have different exp(v - max) that the
    softmax's division by the sum rounds to one p: the tie the reference breaks by index (ops::top_k), which the
    ranking of the unnormalised values would order the other way when the larger one has the higher index."""
    rng = np.random.default_rng(seed)
    rows, flips = [], 0
    while len(rows) < count:
        v = (rng.standard_normal(128) * 0.3).astype(np.float32)
        order = np.argsort(-v)
        a, b = order[rng.integers(1, 7)], order[rng.integers(9, 40)]
        m = v.max()
        ea = np.float32(np.exp(np.float64(np.float32(v[a] - m))))
        x, target = v[a], np.nextafter(ea, np.float32(0))
        for _ in range(50):
            x = np.nextafter(x, np.float32(-np.inf))
            eb = np.float32(np.exp(np.float64(np.float32(x - m))))
            if eb <= target:
                break
        if eb != target:
            continue
        v[b] = x
        e = np.exp((v - m).astype(np.float32).astype(np.float64)).astype(np.float32)
        p = (e / np.cumsum(e, dtype=np.float32)[-1]).astype(np.float32)
        if e[a] != e[b] and p[a] == p[b]:
            rows.append(v)
            flips += int(b < a)
    return np.stack(rows), flips


def test_route_division_ties(hip):
    """The per-token route (a block per token for up to 16 tokens) on rows with a tie made by the softmax's division
    (some with the larger e at the higher index, which the ranking of e alone would get wrong), and sigmoid rows:
    ids bit-exact with ops::top_k's, weights to 1e-6, slots and wh from the table."""
    logits, flips = _division_tie_logits(12, seed=7)
    assert flips >= 3  # cases where the tie reverses the order of the unnormalised values
    n, k, t = 128, 8, logits.shape[0]
    for lg, sig in [(logits, False), (zipf_logits(5, 100, seed=8), True), (zipf_logits(16, 128, seed=9), False)]:
        tt = lg.shape[0]
        table = np.arange(lg.shape[1], dtype=np.int32)
        table[::5] = -1
        bufs = [hip.alloc(tt * k * 4) for _ in range(4)]
        hip.moe_route(up(hip, lg), lg.shape[1], k, 0.0, up(hip, table), *bufs, tt, sig)
        ids, wts, slots, wh = [down(hip, b, dt, tt * k) for b, dt in
                               zip(bufs, (np.int32, np.float32, np.int32, np.float32))]
        wi, ww = O.route(lg, k, sigmoid=sig)
        assert np.array_equal(ids, wi.reshape(-1))
        assert np.abs(wts - ww.reshape(-1)).max() <= 1e-6
        assert np.array_equal(slots, table[ids])
        assert np.array_equal(wh, np.where(slots >= 0, wts, 0.0).astype(np.float32))
    assert t == 12

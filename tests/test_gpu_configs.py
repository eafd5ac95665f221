"""BASELINE configs at their stated workloads on the GPU, through the C ABI, against the CPU oracle.

one Q4_K 4096 x 4096 dequant-GEMV, weights from the repo quantizer over seeded N(0, 0.02).
IQ2_XXS / IQ3_S / IQ4_XS experts (128 of them, 2048 x 768 each, random grid indices, signs and scales),
T = 1 through moe_gemv over the 8 routed slots and T = 512 through route -> moe_sort -> gemm_grouped.
Bars as in test_gpu_parity: fp32 within max relative error 1e-3; the CPU dot's bits where the close is exact.
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
THREADS = min(16, os.cpu_count() or 1)
EXACT = (ggml.IQ2_XXS, ggml.IQ3_S)  # IQ4_XS closes each 32-value sub-block in float on the CPU


def test_config0_q4k_4096x4096(hip):
    rows = cols = 4096
    wf = normal((rows, cols), seed=2024, std=0.02)
    w = S.quantize_rows(ggml.Q4_K, wf)
    x = normal(cols, seed=2025)
    t = hip.upload_tensor(ggml.Q4_K, w)
    y = hip.alloc(rows * 4)
    hip.gemv(t, hip.upload(x), y)
    got = hip.get(y, np.float32, rows)
    want = O.matvec(ggml.Q4_K, w, rows, cols, x, threads=THREADS)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int((got != want).sum())
    # and the output is that of the f32 weights up to 4-bit quantization noise (~8% rel-L2 for N(0, 0.02) rows;
    # an output unrelated to the weights would be ~140%)
    ref = wf.astype(np.float64) @ x.astype(np.float64)
    assert rel_l2(got, ref) < 0.15


def expert_bank(ty, E, rows, cols, seed):
    return random_blocks(ty, E * rows, cols, seed=seed)


def per_pair_check(ty, w, rows, cols, pairs, xs, got, sample):
    """got[s] = W_{e_s} x_{t_s}: all pairs against the f64 dot of the dequantized expert with the Q8_K activations,
    and `sample` of them against cpu_moe::matvec (bits for the exact types)."""
    seen = {}
    for t in sorted({t for _, t in pairs}):
        d, qs, _ = O.quantize_q8k(xs[t])
        seen[t] = (d[:, None] * qs.astype(np.float32)).reshape(-1)[:cols].astype(np.float64)
    by_e = {}
    for s, (e, t) in enumerate(pairs):
        by_e.setdefault(e, []).append((s, t))
    for e, lst in by_e.items():
        we = O.dequant(ty, w[e * rows:(e + 1) * rows], rows * cols).reshape(rows, cols).astype(np.float64)
        for s, t in lst:
            assert rel_l2(got[s], we @ seen[t]) < 1e-5, (s, e, t)
    for s in sample:
        e, t = pairs[s]
        want = O.matvec(ty, w[e * rows:(e + 1) * rows], rows, cols, xs[t], threads=THREADS)
        assert max_rel_err(got[s], want) <= TOL, (s, max_rel_err(got[s], want))
        if ty in EXACT:
            assert np.array_equal(got[s].view(np.uint32), want.view(np.uint32)), (s, int((got[s] != want).sum()))


@pytest.mark.parametrize("ty", [ggml.IQ2_XXS, ggml.IQ3_S, ggml.IQ4_XS])
@pytest.mark.parametrize("rows,cols", [(2048, 768), (768, 2048)])
def test_config3_moe_gemv_t1(hip, ty, rows, cols):
    """T = 1: the 8 routed experts of 128 (Zipf-skewed logits) through moe_gemv."""
    E, k = 128, 8
    w = expert_bank(ty, E, rows, cols, seed=300 + ty + rows)
    wb = hip.upload(w)
    rb = ggml.row_bytes(ty, cols)
    logits = zipf_logits(1, E, seed=301 + ty)
    ids_w, _ = O.route(logits, k)
    x = normal(cols, seed=302 + ty)
    y = hip.alloc(k * rows * 4)
    hip.moe_gemv(ty, rows, cols, wb, rows * rb, hip.upload(ids_w[0]), k, hip.upload(x), cols, k, y)
    got = hip.get(y, np.float32, k * rows).reshape(k, rows)
    pairs = [(int(e), 0) for e in ids_w[0]]
    per_pair_check(ty, w, rows, cols, pairs, x[None, :], got, sample=range(k))


@pytest.mark.parametrize("ty", [ggml.IQ2_XXS, ggml.IQ3_S, ggml.IQ4_XS])
@pytest.mark.parametrize("small", [False, True], ids=["tiles256", "tiles64"])
def test_config3_grouped_gemm_t512(hip, ty, small):
    """T = 512: route -> device sort -> gemm_grouped over 128 experts of 2048 x 768, with 256-position tiles and with
    the 64-position tiles and GEMM form the backend picks at this size (SMALL_TILES); every routed (token, expert)
    pair checked against the dequantized f64 dot, 256 of them against cpu_moe::matvec."""
    E, k, T, rows, cols = 128, 8, 512, 2048, 768
    w = expert_bank(ty, E, rows, cols, seed=400 + ty)
    wb = hip.upload(w)
    rb = ggml.row_bytes(ty, cols)
    xs = normal((T, cols), seed=401 + ty)
    logits = zipf_logits(T, E, seed=402 + ty)
    ids_w, _ = O.route(logits, k)
    ids = hip.alloc(T * k * 4)
    hip.router_topk(hip.upload(logits), E, k, 0.0, ids, hip.alloc(T * k * 4), T)
    assert np.array_equal(hip.get(ids, np.int32, T * k).reshape(T, k), ids_w)
    chunk, fl = hip.moe_tile_plan(T, k, E, small)
    assert (fl != 0) == small and hip.moe_tile_plan(T, k, E) == (64, S.SMALL_TILES)
    max_tiles = T * k // chunk + E
    off, xrow, inv = hip.alloc((E + 1) * 4), hip.alloc(T * k * 4), hip.alloc(T * k * 4)
    tiles, ntd = hip.alloc(max_tiles * 16), hip.alloc(4)
    hip.moe_sort(ids, T, k, E, off, xrow, inv, [(int(wb), rows * rb)], tiles, max_tiles, ntd, chunk=chunk)
    y = hip.alloc(T * k * rows * 4)
    hip.gemm_grouped(ty, rows, cols, tiles, max_tiles, ntd, hip.upload(xs), cols, T, xrow, y, rows, S.ACT_STORE | fl)
    got = hip.get(y, np.float32, T * k * rows).reshape(T * k, rows)
    off_w, xrow_w, _ = O.sort_by_expert(ids_w, E)
    assert np.array_equal(hip.get(xrow, np.int32, T * k), xrow_w)
    pairs = []
    for e in range(E):
        for s in range(off_w[e], off_w[e + 1]):
            pairs.append((e, int(xrow_w[s])))
    sample = np.random.default_rng(5).choice(T * k, 256, replace=False)
    per_pair_check(ty, w, rows, cols, pairs, xs, got, sample=sorted(sample.tolist()))

"""Seeded synthetic inputs shared by the tests (numpy only; no GPU)."""
import numpy as np

from rustingstrata_amd import ggml


def f16_bytes(v):
    return np.array([v], dtype=np.float16).view(np.uint8)


def random_blocks(ty, rows, cols, seed, scale=(0.01, 0.02)):
    """Random block bytes with every f16 super-block scale set to a value in [scale) (the design of the reference's
    random_tensor, tests/kernels.rs:1473-1550: random bytes, scale fields overwritten)."""
    rng = np.random.default_rng(seed)
    rb = ggml.row_bytes(ty, cols)
    b = rng.integers(0, 256, size=(rows, rb), dtype=np.uint8)
    bb = ggml.block_bytes(ty)
    nb = rb // bb
    v = b.reshape(rows, nb, bb)
    for off in ggml.F16_FIELDS[ty]:
        s = rng.uniform(scale[0], scale[1], size=(rows, nb)).astype(np.float16)
        v[:, :, off:off + 2] = s.view(np.uint8).reshape(rows, nb, 2)
    return b


def normal(shape, seed, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def max_rel_err(got, want):
    """max_i |g_i - r_i| / max(|r_i|, 1e-3 max_j |r_j|): the parity metric for fp32 outputs."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    floor = 1e-3 * max(np.abs(want).max(), 1e-30)
    return float((np.abs(got - want) / np.maximum(np.abs(want), floor)).max())


def rel_l2(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def zipf_logits(t, n_expert, seed, s=1.1, scale=2.0):
    """Router logits N(0, 1) plus a per-expert Zipf(s) bias over a seeded permutation of the experts."""
    rng = np.random.default_rng(seed)
    rank = rng.permutation(n_expert) + 1
    bias = scale * rank.astype(np.float64) ** -s / 1.0
    return (rng.standard_normal((t, n_expert)) + bias[None, :] * 4.0).astype(np.float32)

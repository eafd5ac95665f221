"""Host-side checks that need no GPU: the C-ABI library loads and exports every symbol include/strata_hip.h
declares, and the host quantizers make blocks the oracle decodes back to their inputs."""
import os
import re

import numpy as np
import pytest

import rustingstrata_amd as S
from oracle import oracle as O
from rustingstrata_amd import ggml

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "strata_hip.h")).read()
    return sorted(set(re.findall(r"\b(strata_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = S.lib()
    names = declared()
    assert len(names) >= 38
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(S.backend.SIGNATURES), set(names) ^ set(S.backend.SIGNATURES)


def test_row_bytes():
    lib = S.lib()
    for ty in ggml.TYPES:
        assert lib.strata_row_bytes(ty, 2048) == ggml.row_bytes(ty, 2048)
    assert lib.strata_row_bytes(12, 100) == 0 and lib.strata_row_bytes(99, 256) == 0


@pytest.mark.parametrize("ty,tol", [(ggml.Q8_0, 0.01), (ggml.Q4_K, 0.15), (ggml.Q5_K, 0.08), (ggml.Q6_K, 0.05),
                                    (ggml.Q2_K, 0.5), (ggml.Q3_K, 0.3), (ggml.IQ4_XS, 0.12)])
def test_quantizer_round_trip(ty, tol):
    rng = np.random.default_rng(ty)
    w = (rng.standard_normal((16, 512)) * 0.02).astype(np.float32)
    b = S.quantize_rows(ty, w)
    assert b.shape == (16, ggml.row_bytes(ty, 512))
    back = O.dequant(ty, b, w.size).reshape(w.shape)
    err = np.linalg.norm(back - w) / np.linalg.norm(w)
    assert err < tol, err


def test_unsupported_quantizer_raises():
    with pytest.raises(S.StrataError):
        S.quantize_rows(ggml.IQ3_S, np.zeros((1, 256), dtype=np.float32))


def test_no_gpu_open_fails_cleanly():
    """Without a GPU, opening the backend raises (no silent CPU path)."""
    import ctypes
    ctx = ctypes.c_void_p()
    rc = S.lib().strata_open(0, ctypes.byref(ctx))
    if rc == 0:  # a GPU is present here
        S.lib().strata_close(ctx)
        pytest.skip("a GPU is present")
    assert S.lib().strata_last_error()


def test_size_helpers():
    """The host-side size queries the bindings use: an f16 cache takes one u16 word a value (Backend::kv_words,
    src/backend.rs:186), a GEMM block holds 256 positions, and the decode attention's partials take hd + 2 floats per
    head and position split (128 splits)."""
    from rustingstrata_amd import backend as B
    lib = B.lib()
    assert all(lib.strata_kv_words(n) == n for n in (0, 1, 128, 512, 4096))
    assert lib.strata_gemm_block_positions() == 256
    assert lib.strata_attn_part_floats(32, 128) == 32 * 128 * 130
    assert lib.strata_attn_part_floats(8, 64) == 8 * 128 * 66


def test_config4_shape():
    """the Qwen3-30B-A3B-shaped stack (48 layers, hidden 2048, 32 query heads over 4 KV heads of 128,
    128 experts top-8 of intermediate 768, vocabulary 151936) with the UD-Q2_K_XL-like mix (Q2_K/Q3_K experts, Q6_K
    attention, Q8_0 embeddings and output)."""
    from rustingstrata_amd.qwen3moe import Config
    c = Config.qwen3_30b_a3b()
    assert (c.n_layer, c.n_embd, c.n_head, c.n_head_kv, c.head_dim) == (48, 2048, 32, 4, 128)
    assert (c.n_expert, c.n_expert_used, c.n_ff_exp, c.n_vocab) == (128, 8, 768, 151936)
    assert (c.ty_gate_up, c.ty_down, c.ty_attn, c.ty_embd, c.ty_out) == (ggml.Q2_K, ggml.Q3_K, ggml.Q6_K, ggml.Q8_0,
                                                                          ggml.Q8_0)

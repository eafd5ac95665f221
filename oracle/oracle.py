"""ctypes face of the CPU oracle (oracle/liboracle.so, built by oracle/Makefile).

TEST INFRASTRUCTURE ONLY: the checker for tests/, __graft_entry__.smoke() and the timed CPU baseline of bench.py.
The product (rustingstrata_amd) never imports this module. Each function names the reference file:line it restates
(see strata_oracle.h).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
_lib = None


class Q8K(ctypes.Structure):  # src/cpu_moe.rs:13
    _fields_ = [("d", ctypes.c_float), ("qs", ctypes.c_int8 * 256), ("bs", ctypes.c_int16 * 16)]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        l = ctypes.CDLL(LIB)
        P, U, I, F = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float
        sig = {
            "or_dequant_row": ([I, P, U, P], I),
            "or_quantize_q8k": ([P, U, P], None),
            "or_int_dot": ([I, P, U, P], F),
            "or_matvec": ([I, P, U, U, P, P, I], None),
            "or_quant_xq32": ([P, U, U, U, P], None),
            "or_route": ([P, I, I, I, F, P, P], None),
            "or_sort_by_expert": ([P, I, I, I, P, P, P], None),
            "or_combine_seq": ([P, P, P, P, I, I, I], None),
            "or_experts_multi": ([I, I, P, P, P, I, I, P, I, P, P, I, P, I], None),
            "or_silu": ([F], F),
            "or_rms_norm": ([P, P, F, I, P], None),
            "or_f16": ([ctypes.c_uint16], F),
            "or_rope_neox": ([P, I, ctypes.c_long, F], None),
            "or_set_avx2": ([I], None),
            "or_argmax": ([P, I], I),
            "or_attention": ([P, P, P, I, I, I, I, I, F, P, P, I, P, P], None),
        }
        for n, (a, r) in sig.items():
            f = getattr(l, n)
            f.argtypes, f.restype = a, r
        _lib = l
    return _lib


def _p(a):
    return a.ctypes.data


def set_avx2(on):
    """Select the AVX2 dots (the reference's timed x86-64-v3 path) for int_dot / matvec / experts_multi, or the
    scalar ones (the default, the parity checker)."""
    lib().or_set_avx2(1 if on else 0)


def dequant(ty, blocks, n):
    """quant::dequant_row over the whole byte array (n values)."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    if lib().or_dequant_row(ty, _p(blocks), n, _p(out)) != 0:
        raise ValueError(f"oracle cannot dequantize type {ty} x {n}")
    return out


def quantize_q8k(x):
    """cpu_moe::quantize_q8k: (d [nb], qs [nb, 256] int8, bs [nb, 16] int16)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nb = (x.size + 255) // 256
    arr = (Q8K * nb)()
    lib().or_quantize_q8k(_p(x), x.size, ctypes.addressof(arr))
    d = np.array([b.d for b in arr], dtype=np.float32)
    qs = np.array([list(b.qs) for b in arr], dtype=np.int8)
    bs = np.array([list(b.bs) for b in arr], dtype=np.int16)
    return d, qs, bs


def q8k_blocks(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    nb = (x.size + 255) // 256
    arr = (Q8K * nb)()
    lib().or_quantize_q8k(_p(x), x.size, ctypes.addressof(arr))
    return arr


def int_dot(ty, row, x):
    """int_dot(ty)(row, quantize_q8k(x)): one row's Q8_K integer dot (scalar kernels, src/cpu_moe.rs)."""
    row = np.ascontiguousarray(row, dtype=np.uint8)
    arr = q8k_blocks(x)
    return lib().or_int_dot(ty, _p(row), np.asarray(x).size, ctypes.addressof(arr))


def matvec(ty, w, rows, cols, x, threads=0):
    """cpu_moe::matvec: y = W x with Q8_K activations."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    lib().or_matvec(ty, _p(w), rows, cols, _p(x), _p(y), threads)
    return y


def quant_xq32(x):
    """The reference GPU's per-32 quantization: (int8 [nt, n], f32 scales [nt, n / 32])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nt, n = x.shape
    out = np.empty(nt * n + nt * n // 8, dtype=np.uint8)
    lib().or_quant_xq32(_p(x), n, n, nt, _p(out))
    return out[: nt * n].view(np.int8).reshape(nt, n), out[nt * n:].view(np.float32).reshape(nt, n // 32)


def route(logits, k, sigmoid=False, extra_scale=0.0):
    """Model::route per token: (ids [t, k] int32, wts [t, k] f32)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    t, n = logits.shape
    ids = np.empty((t, k), dtype=np.int32)
    wts = np.empty((t, k), dtype=np.float32)
    for i in range(t):
        lib().or_route(_p(logits[i]), n, k, int(sigmoid), extra_scale, _p(ids[i]), _p(wts[i]))
    return ids, wts


def sort_by_expert(ids, n_expert):
    """The prefill counting sort: (off [E + 1], xrow [t k], inv [t k])."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    t, k = ids.shape
    off = np.empty(n_expert + 1, dtype=np.int32)
    xrow = np.empty(t * k, dtype=np.int32)
    inv = np.empty(t * k, dtype=np.int32)
    lib().or_sort_by_expert(_p(ids), t, k, n_expert, _p(off), _p(xrow), _p(inv))
    return off, xrow, inv


def combine_seq(x, ye, wts, inv):
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    t, n = x.shape
    k = wts.shape[1]
    lib().or_combine_seq(_p(x), _p(np.ascontiguousarray(ye, dtype=np.float32)), _p(np.ascontiguousarray(wts, dtype=np.float32)),
                         _p(np.ascontiguousarray(inv, dtype=np.int32)), k, n, t)
    return x


def experts_multi(ty_gu, ty_down, gate, up, down, n_embd, n_ff, hs, ids, wts, threads=0):
    """cpu_moe::experts_multi for all tokens: ys [t, n_embd]."""
    hs = np.ascontiguousarray(hs, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    wts = np.ascontiguousarray(wts, dtype=np.float32)
    t, k = ids.shape
    ys = np.empty((t, n_embd), dtype=np.float32)
    lib().or_experts_multi(ty_gu, ty_down, _p(gate), _p(up), _p(down), n_embd, n_ff, _p(hs), t, _p(ids), _p(wts), k,
                           _p(ys), threads)
    return ys


def rms_norm(x, w, eps):
    """ops::rms_norm (src/ops.rs:3-7) per row of x."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(x)
    for r in range(x.shape[0]):
        lib().or_rms_norm(_p(x[r]), _p(w), ctypes.c_float(eps), x.shape[1], _p(out[r]))
    return out


def silu(x):
    return lib().or_silu(float(x))


def rope_neox(x, n_rot, pos, base):
    """ops::rope_neox (src/ops.rs:36-45) on each row (one head) of x, at position pos; returns a copy."""
    x = np.array(np.atleast_2d(x), dtype=np.float32, copy=True, order="C")
    for r in range(x.shape[0]):
        lib().or_rope_neox(_p(x[r]), n_rot, pos, base)
    return x


def argmax(x):
    """ops::argmax (src/ops.rs:110-112): first index of the largest value under total_cmp."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().or_argmax(_p(x), x.size))


def attention(q, kc, vc, p0, p1, nh, nkv, hd, scale, sinks=None, gate=None, gate_stride=0):
    """Model::attention's per-token attention (src/model.rs:771-793) over cells p0 .. p1 - 1: q [nh * hd], kc / vc
    [positions, nkv * hd]; returns out [nh * hd]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(kc, dtype=np.float32)
    vc = np.ascontiguousarray(vc, dtype=np.float32)
    out = np.empty(nh * hd, dtype=np.float32)
    sc = np.empty(max(p1 - p0, 1), dtype=np.float32)
    sk = None if sinks is None else np.ascontiguousarray(sinks, dtype=np.float32)
    g = None if gate is None else np.ascontiguousarray(gate, dtype=np.float32)
    lib().or_attention(_p(q), _p(kc), _p(vc), p0, p1, nh, nkv, hd, ctypes.c_float(scale),
                       None if sk is None else _p(sk), None if g is None else _p(g), gate_stride, _p(out), _p(sc))
    return out

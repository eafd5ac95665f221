"""Host side of the MI355X backend: the reference's `Backend` trait (src/backend.rs:98-443) for the quantized-matmul
hot path, over the C ABI of libstrata_hip.so (include/strata_hip.h).

Method names, argument meaning and error behaviour follow the trait: device addresses are ints, strides are in
floats, ops queue in order on one stream, host copies are synchronous, and an op that rejects its arguments raises
StrataError (the trait's `Err`) without launching anything. `Buf` and `GpuTensor` mirror src/backend.rs:18-45.

The library must be built (rustingstrata_amd/build.py); nothing here falls back to another implementation.
"""
import ctypes
import os
import weakref

import numpy as np

from . import ggml

LIB_PATH = os.environ.get("STRATA_HIP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libstrata_hip.so")
NUM_Q8K, NUM_Q8_32 = 0, 1
ACT_STORE, ACT_SWIGLU, ACT_ADD, SAME_X, X_Q, SMALL_TILES = 0, 1, 2, 4, 8, 16
GEMM_BM = 128  # positions per tile (src/backend.rs:16)
F32_TYPE = 0   # GGUF type id of float32 matrices (gemv / gemm_dense accept them)


class StrataError(RuntimeError):
    """An op refused its arguments or a HIP call failed (the trait's anyhow::Error)."""


class _Tensor(ctypes.Structure):
    _fields_ = [("ty", ctypes.c_int32), ("reserved", ctypes.c_int32), ("rows", ctypes.c_uint64),
                ("cols", ctypes.c_uint64), ("ptr", ctypes.c_uint64)]


U64, I64, I32, F32, P = ctypes.c_uint64, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_void_p
TP = ctypes.POINTER(_Tensor)
CTX = ctypes.c_void_p

# name -> argument types (every function returns int status unless listed in _RESTYPES)
SIGNATURES = {
    "strata_open": [I32, ctypes.POINTER(CTX)],
    "strata_close": [CTX],
    "strata_last_error": [],
    "strata_device_name": [CTX, ctypes.c_char_p, ctypes.c_size_t],
    "strata_set_numerics": [CTX, I32],
    "strata_get_numerics": [CTX],
    "strata_alloc": [CTX, ctypes.c_size_t, ctypes.POINTER(U64)],
    "strata_free": [CTX, U64],
    "strata_htod": [CTX, P, U64, ctypes.c_size_t],
    "strata_dtoh": [CTX, U64, P, ctypes.c_size_t],
    "strata_dtod": [CTX, U64, U64, ctypes.c_size_t],
    "strata_memset": [CTX, U64, ctypes.c_size_t],
    "strata_mem_info": [CTX, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)],
    "strata_sync": [CTX],
    "strata_stream": [CTX],
    "strata_graph_begin": [CTX],
    "strata_graph_end": [CTX, ctypes.POINTER(P)],
    "strata_graph_launch": [CTX, P],
    "strata_graph_destroy": [CTX, P],
    "strata_dequant": [CTX, TP, U64, U64],
    "strata_quant_xq": [CTX, U64, U64, U64, U64, U64],
    "strata_rms_norm": [CTX, U64, U64, U64, U64, U64, U64, U64, ctypes.c_float],
    "strata_rms_norm_q": [CTX, U64, U64, U64, U64, U64, U64, U64, ctypes.c_float, U64, U64],
    "strata_rms_norm_rope_attn_decode": [CTX, U64, U64, U64, U64, U64, U64, ctypes.c_float, U64, ctypes.c_float, U64,
                                         U64, U64, U64, U64, U64, U64, U64, U64, ctypes.c_float, U64, U64, U64],
    "strata_rms_norm_rope_qk_t": [CTX, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64,
                                  ctypes.c_float, U64, U64, ctypes.c_float, U64, U64, U64, U64],
    "strata_combine_rms_norm_q": [CTX, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, ctypes.c_float, U64, U64],
    "strata_rms_norm_q_gemv_f32": [CTX, U64, U64, U64, U64, U64, U64, ctypes.c_float, TP, U64],
    "strata_combine_rms_norm_gemv": [CTX, U64, U64, U64, U64, U64, U64, ctypes.c_float, TP, U64, U64],
    "strata_gemv": [CTX, TP, U64, U64],
    "strata_gemvn": [CTX, TP, U64, U64, U64, U64, U64],
    "strata_gemvn_noalloc": [CTX, TP, U64, U64, U64, U64, U64],
    "strata_gemvq": [CTX, TP, U64, U64, U64, U64, U64, U64],
    "strata_gemvq2": [CTX, TP, TP, U64, U64, U64, U64, U64, U64],
    "strata_moe_gemv": [CTX, I32, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, I32, I64, I64, U64],
    "strata_router_topk": [CTX, U64, U64, U64, F32, U64, U64, U64, I32],
    "strata_moe_route": [CTX, U64, U64, U64, F32, U64, U64, U64, U64, U64, U64, I32],
    "strata_moe_route_gemv": [CTX, U64, U64, U64, F32, U64, U64, U64, U64, U64, I32, I32, U64, U64, U64, U64, U64,
                              U64, I32, I64, I64, U64],
    "strata_swiglu_q": [CTX, U64, U64, U64, U64, U64, ctypes.POINTER(U64)],
    "strata_moe_combine": [CTX, U64, U64, U64, U64, U64, U64, U64, U64],
    "strata_moe_down_combine": [CTX, I32, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64],
    "strata_moe_down_swiglu_combine": [CTX, I32, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64],
    "strata_moe_combine_seq": [CTX, U64, U64, U64, U64, U64, U64, U64, U64, U64],
    "strata_moe_sort": [CTX, U64, U64, U64, U64, U64, U64, U64, U64, ctypes.POINTER(U64), ctypes.POINTER(U64),
                        U64, U64, U64, U64, U64],
    "strata_gemm": [CTX, I32, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, I32],
    "strata_gemm_grouped": [CTX, I32, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, I32],
    "strata_gemm_grouped_gate_up": [CTX, I32, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, ctypes.c_int64, I32],
    "strata_gemm_dense": [CTX, TP, U64, U64, U64, U64, U64, I32],
    "strata_gemm_block_positions": [],
    "strata_int8_gemm": [CTX, I32],
    "strata_prequant_gemm_x": [CTX, TP, U64, U64, U64],
    "strata_quantize_rows": [I32, P, U64, U64, P],
    "strata_row_bytes": [I32, U64],
    "strata_event_create": [CTX, ctypes.POINTER(P)],
    "strata_event_record": [CTX, P],
    "strata_event_elapsed": [P, P, ctypes.POINTER(F32)],
    "strata_event_destroy": [P],
    "strata_copy_kernel": [CTX, U64, U64, U64],
    "strata_read_kernel": [CTX, U64, U64, U64],
    "strata_kv_words": [U64],
    "strata_argmax_rows": [CTX, U64, U64, U64, U64],
    "strata_rope_pairs": [CTX, U64, U64, U64, U64, U64, U64, F32, U64, U64],
    "strata_rope_neox": [CTX, U64, U64, U64, U64, U64, U64, F32],
    "strata_rms_norm_rope": [CTX, U64, U64, U64, U64, U64, U64, F32, U64, U64, U64, F32],
    "strata_rms_norm_rope_kv": [CTX, U64, U64, U64, U64, U64, U64, F32, U64, U64, U64, F32, U64, U64, U64],
    "strata_rms_norm_rope_qk": [CTX, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, F32, U64, U64, F32,
                                U64, U64, U64],
    "strata_kv_store": [CTX, U64, U64, U64, U64, U64, U64, U64, U64],
    "strata_attn_prefill": [CTX, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, F32],
    "strata_attn_prefill_m": [CTX, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, F32, U64, U64, U64, U64],
    "strata_attn_part_floats": [U64, U64],
    "strata_attn_decode": [CTX, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, F32, U64],
    "strata_attn_decode_gq": [CTX, U64, U64, U64, U64, U64, U64, U64, U64, U64, U64, F32, I32, U64, U64, U64],
    "strata_add": [CTX, U64, U64, U64],
    "strata_swiglu": [CTX, U64, U64, U64],
    "strata_get_rows": [CTX, TP, U64, U64, U64],
    "strata_fill_blocks": [CTX, TP, U64, F32, F32],
}
_RESTYPES = {"strata_close": None, "strata_last_error": ctypes.c_char_p, "strata_stream": P, "strata_row_bytes": U64,
             "strata_gemm_block_positions": U64, "strata_kv_words": U64, "strata_attn_part_floats": U64}

_lib = None


def lib():
    """The loaded library. Raises if it is not built: there is no fallback path."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise StrataError(f"{LIB_PATH} is not built: run rustingstrata_amd/build.py (or __graft_entry__.build())")
        l = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            f = getattr(l, name)
            f.argtypes = args
            f.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = l
    return _lib


def _check(rc):
    if rc != 0:
        raise StrataError(lib().strata_last_error().decode())


def quantize_rows(ty, w):
    """f32 rows -> GGUF blocks of type ty (uint8 [rows, row_bytes]) with the library's host quantizer."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    out = np.empty((rows, ggml.row_bytes(ty, cols)), dtype=np.uint8)
    if lib().strata_quantize_rows(ty, w.ctypes.data, rows, cols, out.ctypes.data) != 0:
        raise StrataError(f"no host quantizer for {ggml.name(ty)} with {cols} columns")
    return out


class Buf:
    """`len` bytes of device memory at `addr`, freed when the last reference drops (src/backend.rs:18-30)."""

    def __init__(self, backend, addr, length):
        self.addr, self.len = addr, length
        self._fin = weakref.finalize(self, HipBackend._free_addr, backend._ctx_ref, addr)

    def __int__(self):
        return self.addr


class GpuTensor:
    """`rows` x `cols` of type `ty` from device address `ptr` (src/backend.rs:32-45); keeps its Buf alive."""

    def __init__(self, ty, rows, cols, buf, offset=0):
        self.ty, self.rows, self.cols, self.buf = ty, rows, cols, buf
        self.ptr = int(buf) + offset

    def bytes(self):
        return ggml.row_bytes(self.ty, self.cols) * self.rows

    def _c(self):
        return ctypes.byref(_Tensor(self.ty, 0, self.rows, self.cols, self.ptr))


class Graph:
    """An executable graph recorded from the ops a function queues; destroyed by close() or when collected, before
    the buffers it keeps alive can be freed."""

    def __init__(self, backend, f, keep=()):
        self.backend = backend
        _check(lib().strata_graph_begin(backend._ctx))
        try:
            f()
        finally:
            out = P()
            rc = lib().strata_graph_end(backend._ctx, ctypes.byref(out))
        _check(rc)
        self.handle = out
        self._fin = weakref.finalize(self, Graph._destroy, backend._ctx_ref, out, tuple(keep))

    @staticmethod
    def _destroy(ref, handle, keep):
        # keep (the buffers the graph addresses) is released only after this returns
        if ref.ctx is not None:
            lib().strata_graph_destroy(ref.ctx, handle)

    def launch(self):
        if not self._fin.alive:
            raise StrataError("launch of a destroyed graph")
        _check(lib().strata_graph_launch(self.backend._ctx, self.handle))

    def close(self):
        self._fin()


class _CtxRef:
    def __init__(self, ctx):
        self.ctx = ctx


class HipBackend:
    """The MI355X backend (the counterpart of cuda::Gpu, src/cuda/mod.rs)."""

    name = "hip"

    def __init__(self, device=0, numerics=NUM_Q8K):
        l = lib()
        ctx = CTX()
        _check(l.strata_open(device, ctypes.byref(ctx)))
        self._ctx = ctx
        self._ctx_ref = _CtxRef(ctx)
        self._fin = weakref.finalize(self, HipBackend._close, self._ctx_ref)
        self.set_numerics(numerics)

    @staticmethod
    def _close(ref):
        if ref.ctx is not None:
            lib().strata_close(ref.ctx)
            ref.ctx = None

    @staticmethod
    def _free_addr(ref, addr):
        if ref.ctx is not None:
            lib().strata_free(ref.ctx, addr)

    def close(self):
        self._fin()

    # ---- context ----
    def device(self):
        buf = ctypes.create_string_buffer(256)
        _check(lib().strata_device_name(self._ctx, buf, 256))
        return buf.value.decode()

    def set_numerics(self, mode):
        _check(lib().strata_set_numerics(self._ctx, mode))

    def numerics(self):
        return lib().strata_get_numerics(self._ctx)

    # ---- memory (src/backend.rs:108-117) ----
    def alloc(self, nbytes):
        a = U64()
        _check(lib().strata_alloc(self._ctx, nbytes, ctypes.byref(a)))
        return Buf(self, a.value, max(nbytes, 1))

    def htod(self, src, dst, off=0):
        src = np.ascontiguousarray(src)
        _check(lib().strata_htod(self._ctx, src.ctypes.data, int(dst) + off, src.nbytes))

    def dtoh(self, src, off, dst):
        assert dst.flags["C_CONTIGUOUS"]
        _check(lib().strata_dtoh(self._ctx, int(src) + off, dst.ctypes.data, dst.nbytes))

    def dtod(self, src, src_off, dst, dst_off, nbytes):
        _check(lib().strata_dtod(self._ctx, int(src) + src_off, int(dst) + dst_off, nbytes))

    def memset(self, dst, nbytes=None):
        _check(lib().strata_memset(self._ctx, int(dst), dst.len if nbytes is None else nbytes))

    def mem_info(self):
        f, t = ctypes.c_size_t(), ctypes.c_size_t()
        _check(lib().strata_mem_info(self._ctx, ctypes.byref(f), ctypes.byref(t)))
        return f.value, t.value

    def sync(self):
        _check(lib().strata_sync(self._ctx))

    # typed helpers (`put` / `get`, src/backend.rs:447-462)
    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        b = self.alloc(arr.nbytes)
        self.htod(arr, b)
        return b

    def get(self, buf, dtype, n, at=0):
        out = np.empty(n, dtype=dtype)
        self.dtoh(buf, at * np.dtype(dtype).itemsize, out)
        return out

    def upload_tensor(self, ty, blocks):
        """Backend::upload_raw (src/backend.rs:179-183): raw block bytes [rows, row_bytes] as a GpuTensor."""
        rows = blocks.shape[0]
        cols = blocks.shape[1] // ggml.block_bytes(ty) * ggml.block_elems(ty)
        return GpuTensor(ty, rows, cols, self.upload(blocks))

    # ---- recorded graphs (Backend::graph, src/backend.rs:118-120) ----
    def record_graph(self, f, keep=()):
        """Record the ops `f` queues as a Graph (replayed by Graph.launch). The graph holds the raw addresses of the
        buffers those ops use: pass them (or the objects owning them) as `keep`, and the graph keeps them alive until
        it is destroyed, so no replay can touch freed memory."""
        return Graph(self, f, keep)

    def graph(self, key, f):
        """Run the ops `f` queues as the graph recorded under `key`, recording it on first use; `f` runs only when
        recording, so its ops must read per-call values from device memory. The caller keeps the buffers the ops use
        alive until drop_graphs()."""
        if not hasattr(self, "_graphs"):
            self._graphs = {}
        g = self._graphs.get(key)
        if g is None:
            g = self._graphs[key] = Graph(self, f)
        g.launch()

    def drop_graphs(self):
        for g in getattr(self, "_graphs", {}).values():
            g.close()
        self._graphs = {}

    # ---- ops ----
    def dequant(self, w, rows, out):
        _check(lib().strata_dequant(self._ctx, w._c(), rows, int(out)))

    def quant_xq(self, x, x_stride, n, nt, out):
        _check(lib().strata_quant_xq(self._ctx, int(x), x_stride, n, nt, int(out)))

    def rms_norm(self, x, x_stride, w, out, out_stride, n, rows, eps):
        _check(lib().strata_rms_norm(self._ctx, int(x), x_stride, int(w), int(out), out_stride, n, rows, eps))

    def combine_rms_norm_q(self, x, ye, wh, k, w, out, n, rows, eps, xq=0, res=0):
        """x += res (when given), moe_combine (no shared expert) of ye into x, then rms_norm_q of x, in one launch
        where the rows allow."""
        _check(lib().strata_combine_rms_norm_q(self._ctx, int(x), n, int(ye), int(wh), k, int(w), int(out), n, n, rows,
                                               eps, int(xq), int(res)))

    RMS_NORM_GEMV_MAX = 2048  # values of a row the fused norm + GEMV launches take

    def combine_rms_norm_gemv(self, x, res, ye, wh, k, nw, eps, w, x_out, y):
        """x_out = x + res + sum_j wh[j] ye[j] (j < k), y = W rms_norm(x_out) nw, one launch (the bits of
        combine_rms_norm_q then gemvq); res, ye / wh (k = 0) and x_out may be 0."""
        _check(lib().strata_combine_rms_norm_gemv(self._ctx, int(x), int(res), int(ye), int(wh), k, int(nw), eps,
                                                   w._c(), int(x_out), int(y)))


    def rms_norm_q_gemv_f32(self, x, res, nw, h, xq, n, eps, w, y):
        """h = rms_norm(x + res) * nw (and xq), y = w h for an F32 matrix, one launch; x is not written."""
        _check(lib().strata_rms_norm_q_gemv_f32(self._ctx, int(x), int(res), int(nw), int(h), int(xq), n, eps,
                                                w._c(), int(y)))

    def rms_norm_q(self, x, x_stride, w, out, out_stride, n, rows, eps, xq=0, res=0):
        _check(lib().strata_rms_norm_q(self._ctx, int(x), x_stride, int(w), int(out), out_stride, n, rows, eps, int(xq),
                                       int(res)))

    def gemv(self, w, x, y):
        _check(lib().strata_gemv(self._ctx, w._c(), int(x), int(y)))

    def gemvn(self, w, x, x_stride, y, y_stride, nt):
        _check(lib().strata_gemvn(self._ctx, w._c(), int(x), x_stride, int(y), y_stride, nt))

    def gemvn_noalloc(self, w, x, x_stride, y, y_stride, nt):
        _check(lib().strata_gemvn_noalloc(self._ctx, w._c(), int(x), x_stride, int(y), y_stride, nt))

    def gemvq(self, w, x, x_stride, xq, y, y_stride, nt):
        _check(lib().strata_gemvq(self._ctx, w._c(), int(x), x_stride, int(xq), int(y), y_stride, nt))

    def gemvq2(self, a, b, x, x_stride, xq, ya, yb, nt):
        _check(lib().strata_gemvq2(self._ctx, a._c(), b._c(), int(x), x_stride, int(xq), int(ya), int(yb), nt))

    def moe_gemv(self, ty, rows, cols, w, stride, ids, k, x, x_stride, xg, y, pair=None, xq=0):
        has, w2, y2 = (1, pair[0], pair[1]) if pair is not None else (0, 0, 0)
        _check(lib().strata_moe_gemv(self._ctx, ty, rows, cols, int(w), stride, int(ids), k, int(x), x_stride, xg,
                                     int(y), has, w2, y2, int(xq)))

    def router_topk(self, p, n, k, extra_scale, ids, wts, t, sigmoid=False):
        _check(lib().strata_router_topk(self._ctx, int(p), n, k, extra_scale, int(ids), int(wts), t, int(sigmoid)))

    def moe_route(self, p, n, k, extra_scale, table, ids, wts, slots, wh, t, sigmoid=False):
        _check(lib().strata_moe_route(self._ctx, int(p), n, k, extra_scale, int(table), int(ids), int(wts),
                                      int(slots), int(wh), t, int(sigmoid)))

    def moe_route_gemv(self, p, n, k, extra_scale, table, ids, wts, slots, wh, ty, rows, cols, w, stride, x, y,
                       pair=None, xq=0, sigmoid=False):
        """moe_route of one token, then moe_gemv of its k slots (ids = slots, xg = k) as one launch."""
        has, w2, y2 = (1, pair[0], pair[1]) if pair is not None else (0, 0, 0)
        _check(lib().strata_moe_route_gemv(self._ctx, int(p), n, k, extra_scale, int(table), int(ids), int(wts),
                                           int(slots), int(wh), int(sigmoid), ty, rows, cols, int(w), stride, int(x),
                                           int(y), has, w2, y2, int(xq)))

    def swiglu_q(self, g, u, n, rows, xq):
        r = U64()
        _check(lib().strata_swiglu_q(self._ctx, int(g), int(u), n, rows, int(xq), ctypes.byref(r)))
        return r.value

    def moe_combine(self, x, ye, w, k, sh, sg, n, t):
        _check(lib().strata_moe_combine(self._ctx, int(x), int(ye), int(w), k, int(sh), int(sg), n, t))

    def moe_down_combine(self, ty, rows, cols, w, stride, slots, k, h, ye, xq, x, wh, sh, sg, t):
        _check(lib().strata_moe_down_combine(self._ctx, ty, rows, cols, int(w), stride, int(slots), k, int(h),
                                             int(ye), int(xq), int(x), int(wh), int(sh), int(sg), t))

    def moe_down_swiglu_combine(self, ty, rows, cols, w, stride, slots, k, g, u, ye, x, wh, sh, sg, t):
        """swiglu_q(g, u) then moe_down_combine in one GEMV launch (the x rows quantized inside it)."""
        _check(lib().strata_moe_down_swiglu_combine(self._ctx, ty, rows, cols, int(w), stride, int(slots), k, int(g),
                                                    int(u), int(ye), int(x), int(wh), int(sh), int(sg), t))

    def moe_combine_seq(self, x, ye, wts, inv, k, sh, sg, n, t):
        _check(lib().strata_moe_combine_seq(self._ctx, int(x), int(ye), int(wts), int(inv), k, int(sh), int(sg), n, t))

    def moe_sort(self, ids, t, k, n_expert, off, xrow, inv, mats, tiles, max_tiles, n_tiles_dev, err_dev=0, chunk=0):
        """Device counting sort of the (token, j) pairs by expert + tile lists; mats = [(base, stride), ...];
        chunk = positions per tile (0: the reference's 128)."""
        n = len(mats)
        bases = (U64 * max(n, 1))(*[m[0] for m in mats])
        strides = (U64 * max(n, 1))(*[m[1] for m in mats])
        _check(lib().strata_moe_sort(self._ctx, int(ids), t, k, n_expert, int(off), int(xrow), int(inv), n, bases,
                                     strides, int(tiles), max_tiles, int(n_tiles_dev), int(err_dev), chunk))

    # Routed rows per expert (T k / E) up to which a prefill MoE block takes 64-position tiles and the
    # 64-position GEMM kernel (SMALL_TILES); above it, tiles of gemm_block_positions() (configs[2] layer: 512 tokens,
    # 32 rows an expert: 0.277 against 0.300 ms; 1024 tokens, 64 rows: 0.358 against 0.373 ms; 2048 tokens, 128
    # rows: 0.592 against 0.540 ms).
    SMALL_TILE_ROWS = 64

    def moe_tile_plan(self, t, k, n_expert, small=None):
        """(tile chunk for moe_sort, GEMM flag) for a prefill MoE block of t tokens routed top-k over n_expert."""
        if small is None:
            small = t * k <= self.SMALL_TILE_ROWS * n_expert
        return (64, SMALL_TILES) if small else (self.gemm_block_positions(), 0)

    def gemm_block_positions(self):
        return int(lib().strata_gemm_block_positions())

    def gemm(self, ty, rows, cols, tiles, n_tiles, x, x_stride, n_x, xrow, y, y_stride, act):
        _check(lib().strata_gemm(self._ctx, ty, rows, cols, int(tiles), n_tiles, int(x), x_stride, n_x, int(xrow),
                                 int(y), y_stride, act))

    def gemm_grouped_gate_up(self, ty, rows, cols, tiles, max_tiles, n_tiles_dev, x, x_stride, n_x, xrow, y,
                             y_stride, up_offset, flags=0):
        """y = silu(W_gate x) * (W_up x) over a gate tile list; the up matrix sits up_offset bytes after each gate."""
        _check(lib().strata_gemm_grouped_gate_up(self._ctx, ty, rows, cols, int(tiles), max_tiles, int(n_tiles_dev),
                                                 int(x), x_stride, n_x, int(xrow), int(y), y_stride, up_offset, flags))

    def gemm_grouped(self, ty, rows, cols, tiles, max_tiles, n_tiles_dev, x, x_stride, n_x, xrow, y, y_stride, act):
        _check(lib().strata_gemm_grouped(self._ctx, ty, rows, cols, int(tiles), max_tiles, int(n_tiles_dev), int(x),
                                         x_stride, n_x, int(xrow), int(y), y_stride, act))

    def gemm_dense(self, w, n, x, x_stride, y, y_stride, act):
        _check(lib().strata_gemm_dense(self._ctx, w._c(), n, int(x), x_stride, int(y), y_stride, act))

    def int8_gemm(self, ty):
        return bool(lib().strata_int8_gemm(self._ctx, ty))

    def prequant_gemm_x(self, w, n, x, x_stride):
        _check(lib().strata_prequant_gemm_x(self._ctx, w._c(), n, int(x), x_stride))

    # ---- the decoder stack (src/backend.rs:232-410) ----
    def upload_f32(self, w):
        """An F32 matrix (Backend::upload of an F32/F16 GGUF tensor, src/backend.rs:156-166) as a GpuTensor."""
        w = np.ascontiguousarray(np.atleast_2d(w), dtype=np.float32)
        return GpuTensor(F32_TYPE, w.shape[0], w.shape[1], self.upload(w))

    @staticmethod
    def kv_words(n):
        return int(lib().strata_kv_words(n))

    def argmax_rows(self, x, n, rows, out):
        _check(lib().strata_argmax_rows(self._ctx, int(x), n, rows, int(out)))

    def rope_pairs(self, x, stride, heads, per, n_rot, step, base, lo, hi):
        _check(lib().strata_rope_pairs(self._ctx, int(x), stride, heads, per, n_rot, int(step), base, lo, hi))

    def rope_neox(self, x, stride, heads, per, n_rot, step, base):
        _check(lib().strata_rope_neox(self._ctx, int(x), stride, heads, per, n_rot, int(step), base))

    def rms_norm_rope(self, x, x_stride, w, out, n, rows, eps, per, n_rot, step, base):
        _check(lib().strata_rms_norm_rope(self._ctx, int(x), x_stride, int(w), int(out), n, rows, eps, per, n_rot,
                                          int(step), base))

    def rms_norm_rope_kv(self, x, x_stride, w, out, n, rows, eps, per, n_rot, step, base, v, kc, vc):
        _check(lib().strata_rms_norm_rope_kv(self._ctx, int(x), x_stride, int(w), int(out), n, rows, eps, per, n_rot,
                                             int(step), base, int(v), int(kc), int(vc)))

    def rms_norm_rope_qk(self, q, q_stride, qw, qo, qrows, qper, k, kw, ko, krows, kper, n, eps, n_rot, step, base, v,
                         kc, vc):
        _check(lib().strata_rms_norm_rope_qk(self._ctx, int(q), q_stride, int(qw), int(qo), qrows, qper, int(k), int(kw),
                                             int(ko), krows, kper, n, eps, n_rot, int(step), base, int(v), int(kc),
                                             int(vc)))

    def rms_norm_rope_attn_decode(self, q, q_stride, qw, k, kw, v, eps, n_rot, base, kc, vc, qg, out, part, step, nh,
                                  nkv, hd, scale, sink=0, win=0, xq=0):
        """rms_norm_rope_qk of one token's raw q / k heads with the KV store, then attn_decode, as one launch (out
        also quantized into xq when given)."""
        _check(lib().strata_rms_norm_rope_attn_decode(self._ctx, int(q), q_stride, int(qw), int(k), int(kw), int(v), eps,
                                                      n_rot, base, int(kc), int(vc), int(qg), int(out), int(part),
                                                      int(step), nh, nkv, hd, scale, int(sink), win, int(xq)))

    def rms_norm_rope_qk_t(self, q, q_tstride, q_stride, qw, qo, qrows, qper, k, k_tstride, kw, ko, krows, kper, n,
                           eps, n_rot, step, base, v, v_tstride, kc, vc):
        """rms_norm_rope_qk over heads read at token strides (a fused q/k/v output)."""
        _check(lib().strata_rms_norm_rope_qk_t(self._ctx, int(q), q_tstride, q_stride, int(qw), int(qo), qrows, qper,
                                               int(k), k_tstride, int(kw), int(ko), krows, kper, n, eps, n_rot,
                                               int(step), base, int(v), v_tstride, int(kc), int(vc)))

    def kv_store(self, k, v, kc, vc, n, t, step, hd):
        _check(lib().strata_kv_store(self._ctx, int(k), int(v), int(kc), int(vc), n, t, int(step), hd))

    def attn_prefill(self, q, kc, vc, qg, out, step, t, nh, nkv, hd, scale, sink=0, win=0):
        _check(lib().strata_attn_prefill_m(self._ctx, int(q), int(kc), int(vc), int(qg), int(out), int(step), t, nh,
                                           nkv, hd, scale, 0, 0, int(sink), win))

    @staticmethod
    def attn_part_floats(nh, hd):
        return int(lib().strata_attn_part_floats(nh, hd))

    def attn_decode(self, q, kc, vc, qg, out, part, step, nh, nkv, hd, scale, nt, sink=0, win=0):
        _check(lib().strata_attn_decode_gq(self._ctx, int(q), int(kc), int(vc), int(qg), int(out), int(part), int(step),
                                           nh, nkv, hd, scale, 0, nt, int(sink), win))

    def add(self, x, y, n):
        _check(lib().strata_add(self._ctx, int(x), int(y), n))

    def swiglu(self, g, u, n):
        _check(lib().strata_swiglu(self._ctx, int(g), int(u), n))

    def get_rows(self, w, ids, n, out):
        _check(lib().strata_get_rows(self._ctx, w._c(), int(ids), n, int(out)))

    def fill_blocks(self, w, seed, lo, hi):
        _check(lib().strata_fill_blocks(self._ctx, w._c(), seed, lo, hi))

    # ---- timing on the backend's stream ----
    def event(self):
        e = P()
        _check(lib().strata_event_create(self._ctx, ctypes.byref(e)))
        return e

    def record(self, e):
        _check(lib().strata_event_record(self._ctx, e))

    def copy_kernel(self, src, dst, nbytes):
        _check(lib().strata_copy_kernel(self._ctx, int(src), int(dst), nbytes))

    def read_kernel(self, src, nbytes, sink):
        _check(lib().strata_read_kernel(self._ctx, int(src), nbytes, int(sink)))

    @staticmethod
    def elapsed_ms(e0, e1):
        ms = F32()
        _check(lib().strata_event_elapsed(e0, e1, ctypes.byref(ms)))
        return ms.value

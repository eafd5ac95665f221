"""GGUF files for the hot path: a v2/v3 reader over a read-only memory map (Gguf::open, src/gguf.rs:95-172), a writer
for synthetic files, and the expert-slot layout of routed experts (ExpertCache::new, src/expert_cache.rs:14-24,66-90):
a slot holds one expert's gate, up and down matrices back to back, each starting on a 16-byte boundary, so the
device buffer of a layer's experts is `n_expert` slots of `slot_bytes` and moe_gemv addresses expert e of matrix m at
base + off[m] + e * slot_bytes.

The byte format (little-endian): "GGUF", u32 version, u64 tensor count, u64 key count; keys as (string, u32 type,
value); tensor infos as (string name, u32 n_dims, u64 dims..., u32 ggml type, u64 offset); then, at the next multiple
of `general.alignment` (32 when absent), the tensor data. Strings are u64 length + bytes; arrays are u32 element type,
u64 count, elements. dims[0] is the number of elements per row.
"""
import mmap
import os
import struct

import numpy as np

from . import ggml

# Value types (src/gguf.rs:66-87)
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", U64: "<Q", I64: "<q", F64: "<d"}
# Plain-float tensor types besides the block formats: (elements, bytes) per block
_FLOAT_TYPES = {0: (1, 4), 1: (1, 2), 30: (1, 2)}  # F32, F16, BF16


class GgufError(ValueError):
    pass


def row_bytes(ty, cols):
    """Bytes of one row of `cols` values of ggml type `ty` (None for a type outside this library)."""
    if ty in _FLOAT_TYPES:
        e, b = _FLOAT_TYPES[ty]
        return cols // e * b
    if ty in ggml.BLOCK_BYTES:
        return ggml.row_bytes(ty, cols)
    return None


class TensorInfo:
    __slots__ = ("name", "dims", "ty", "offset", "file")

    def __init__(self, name, dims, ty, offset, file):
        self.name, self.dims, self.ty, self.offset, self.file = name, dims, ty, offset, file

    @property
    def nbytes(self):
        rb = row_bytes(self.ty, self.dims[0] if self.dims else 0)
        if rb is None:
            return None
        n = rb
        for d in self.dims[1:]:
            n *= d
        return n

    def __repr__(self):
        return f"TensorInfo({self.name!r}, dims={self.dims}, ty={self.ty}, offset={self.offset})"


class _Cur:
    def __init__(self, b):
        self.b, self.p = b, 0

    def take(self, n):
        if n < 0 or self.p + n > len(self.b):
            raise GgufError("GGUF truncated")
        s = self.b[self.p:self.p + n]
        self.p += n
        return s

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def str(self):
        return bytes(self.take(self.u64())).decode("utf-8", errors="replace")

    def val(self, t):
        if t in _SCALAR:
            fmt = _SCALAR[t]
            return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]
        if t == BOOL:
            return self.take(1)[0] != 0
        if t == STR:
            return self.str()
        if t == ARR:
            et, n = self.u32(), self.u64()
            if n > len(self.b) - self.p:
                raise GgufError("GGUF array length exceeds remaining data")
            return [self.val(et) for _ in range(n)]
        raise GgufError(f"unknown GGUF value type {t}")


class Gguf:
    """An open GGUF (all shards of a split model): `meta` (key -> value), `tensors` (name -> TensorInfo), `bytes(t)`
    (the tensor's raw bytes, a read-only view of the map)."""

    def __init__(self, path):
        self.meta, self.tensors, self._maps = {}, {}, []
        self._open_one(path, 0)
        n = self.meta.get("split.count", 1)
        if isinstance(n, int) and n > 1:
            name = os.path.basename(path)
            tag = f"-00001-of-{n:05d}.gguf"
            if not name.endswith(tag):
                raise GgufError(f"{path}: split model; open its first shard (*{tag})")
            stem = name[:-len(tag)]
            for i in range(1, n):
                shard = os.path.join(os.path.dirname(path), f"{stem}-{i + 1:05d}-of-{n:05d}.gguf")
                before = set(self.tensors)
                other = self._open_one(shard, i)
                for k in other:
                    if k in before:
                        raise GgufError(f"tensor {k} in two shards")

    def _open_one(self, path, file):
        with open(path, "rb") as f:
            size = os.fstat(f.fileno()).st_size
            mm = mmap.mmap(f.fileno(), size, access=mmap.ACCESS_READ) if size else b""
        b = memoryview(mm)
        c = _Cur(b)
        if bytes(c.take(4)) != b"GGUF":
            raise GgufError(f"{path}: not a GGUF file")
        ver = c.u32()
        if not 2 <= ver <= 3:
            raise GgufError(f"unsupported GGUF version {ver}")
        nt, nkv = c.u64(), c.u64()
        meta = {}
        for _ in range(nkv):
            k = c.str()
            t = c.u32()
            meta[k] = c.val(t)
        tensors = {}
        for _ in range(nt):
            name = c.str()
            nd = c.u32()
            dims = [c.u64() for _ in range(nd)]
            ty, off = c.u32(), c.u64()
            tensors[name] = TensorInfo(name, dims, ty, off, file)
        align = meta.get("general.alignment", 32)
        if not isinstance(align, int) or align <= 0:
            raise GgufError("invalid GGUF alignment")
        data = -(-c.p // align) * align
        for t in tensors.values():
            n = t.nbytes
            if n is None:
                continue  # a type outside this library: reported when used
            if t.offset + n > max(len(b) - data, 0):
                raise GgufError(f"{path}: GGUF truncated (tensor {t.name} lies past the end of the file; re-download it)")
        if file == 0:
            self.meta = meta
        assert len(self._maps) == file, "shards are opened in order"
        names = list(tensors)
        self.tensors.update(tensors)
        self._maps.append((mm, b, data))
        return names

    def get(self, key):
        if key not in self.meta:
            raise GgufError(f"missing GGUF key {key}")
        return self.meta[key]

    def bytes(self, t):
        if isinstance(t, str):
            t = self.tensors[t]
        n = t.nbytes
        if n is None:
            raise GgufError(f"tensor {t.name}: ggml type {t.ty} is not supported here")
        _, b, data = self._maps[t.file]
        return np.frombuffer(b, dtype=np.uint8, count=n, offset=data + t.offset)

    def close(self):
        """Unmap the files; a map that arrays from `bytes` still view stays open until they are gone."""
        for mm, b, _ in self._maps:
            try:
                b.release()
                if isinstance(mm, mmap.mmap):
                    mm.close()
            except BufferError:
                pass
        self._maps = []


def _w_str(out, s):
    s = s.encode()
    out += struct.pack("<Q", len(s)) + s


def _w_val(out, t, v):
    if t in _SCALAR:
        out += struct.pack(_SCALAR[t], v)
    elif t == BOOL:
        out += bytes([1 if v else 0])
    elif t == STR:
        _w_str(out, v)
    elif t == ARR:
        et, items = v
        out += struct.pack("<IQ", et, len(items))
        for x in items:
            _w_val(out, et, x)
    else:
        raise GgufError(f"unknown GGUF value type {t}")


def write_gguf(path, meta, tensors, alignment=32, version=3):
    """Write a GGUF: meta = [(key, type, value)] (arrays: (element type, [values])); tensors = [(name, dims, ggml
    type, raw bytes)], each placed at the next multiple of `alignment` of the data section."""
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", version, len(tensors), len(meta))
    for k, t, v in meta:
        _w_str(out, k)
        out += struct.pack("<I", t)
        _w_val(out, t, v)
    off, offs = 0, []
    for name, dims, ty, raw in tensors:
        _w_str(out, name)
        out += struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", ty, off)
        offs.append(off)
        off += -(-len(raw) // alignment) * alignment
    out += bytes(-len(out) % alignment)
    base = len(out)
    out += bytes(off)
    for (_, _, _, raw), o in zip(tensors, offs):
        out[base + o:base + o + len(raw)] = bytes(raw)
    with open(path, "wb") as f:
        f.write(out)


# ---- expert slots (src/expert_cache.rs:14-24,66-90) ----

MATS = ("ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight")


class Mat:
    """One expert's matrix in a slot: type, rows (out), cols (in), byte offset in the slot, bytes."""
    __slots__ = ("ty", "rows", "cols", "off", "bytes")

    def __init__(self, ty, rows, cols, off, nbytes):
        self.ty, self.rows, self.cols, self.off, self.bytes = ty, rows, cols, off, nbytes

    def __repr__(self):
        return f"Mat(ty={self.ty}, rows={self.rows}, cols={self.cols}, off={self.off}, bytes={self.bytes})"


def slot_layout(g, layer):
    """(mats, slot_bytes, n_expert) of layer `layer`'s routed experts: each matrix of an expert starts on a 16-byte
    boundary of the slot (the GEMV kernels read 16-byte words)."""
    mats, off, n_exp = [], 0, None
    for name in MATS:
        t = g.tensors.get(f"blk.{layer}.{name}")
        if t is None:
            raise GgufError(f"missing tensor blk.{layer}.{name}")
        if len(t.dims) != 3:
            raise GgufError(f"blk.{layer}.{name}: {len(t.dims)} dims (expected cols, rows, experts)")
        cols, rows, ne = t.dims
        if n_exp is not None and ne != n_exp:
            raise GgufError(f"blk.{layer}.{name}: {ne} experts, {n_exp} in the others")
        n_exp = ne
        rb = row_bytes(t.ty, cols)
        if rb is None or t.ty not in ggml.BLOCK_BYTES:
            raise GgufError(f"blk.{layer}.{name}: ggml type {t.ty} is not a block format of this library")
        mats.append(Mat(t.ty, rows, cols, off, rb * rows))
        off = -(-(off + rb * rows) // 16) * 16
    return mats, off, n_exp


def upload_experts(hip, g, layer):
    """A device buffer of the layer's experts in slots (slot e = expert e): returns (buffer, mats, slot_bytes)."""
    mats, slot, ne = slot_layout(g, layer)
    host = np.zeros((ne, slot), dtype=np.uint8)
    for m, name in zip(mats, MATS):
        raw = g.bytes(f"blk.{layer}.{name}").reshape(ne, m.bytes)
        host[:, m.off:m.off + m.bytes] = raw
    return hip.upload(host), mats, slot

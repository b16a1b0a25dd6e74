"""TEST INFRASTRUCTURE ONLY: a restatement of the GGUF container format (v3),
as ggml's published specification lays it out, for writing test packages and
for checking what libsynth_hip's reader reports.

Only tests/, __graft_entry__.smoke() and bench.py may import this module. The
product's reader (synthesize.cpp_amd/csrc/shp_gguf.cpp) never does.

Layout, all little-endian:
    u32 magic (the bytes "GGUF"), u32 version, u64 n_tensors, u64 n_kv
    n_kv    x  string key, u32 value type, value
    n_tensors x string name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64 offset
    zero padding to general.alignment (u32, default 32), then the data section;
    tensor t's bytes start at data_start + offset_t, offset_t a multiple of the
    alignment, in ggml's memory layout (ne[0] fastest).
A string is u64 byte length + bytes; an array is u32 element type + u64 count +
elements. The reference reads packages through ggml's gguf.h
(src/arch/qwen3-tts/weights.cpp:1-80) and resolves tensors by name, type and
shape (src/arch/qwen3-tts/catalog.cpp:77-104).
"""
import struct

import numpy as np

MAGIC = b"GGUF"
VERSION = 3
DEFAULT_ALIGNMENT = 32

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
           I64: "<q", F64: "<d"}

# ggml tensor types: (id, elements per block, bytes per block)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q5_K, GGML_I32, GGML_BF16 = 0, 1, 8, 13, 26, 30
BLOCKS = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 10: (256, 84),
          11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 24: (1, 1), 25: (1, 2), 26: (1, 4),
          27: (1, 8), 28: (1, 8), 30: (1, 2)}


def tensor_nbytes(gtype, ne):
    be, bb = BLOCKS[gtype]
    assert ne[0] % be == 0
    rows = int(np.prod(ne[1:])) if len(ne) > 1 else 1
    return ne[0] // be * bb * rows


def _string(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype == STRING:
        return _string(v)
    if vtype == ARRAY:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, x) for x in items)
    return struct.pack(_SCALAR[vtype], v)


def write(path, kv, tensors, alignment=None, version=VERSION):
    """kv: list of (key, value type, value) -- arrays as (element type, items);
    tensors: list of (name, ggml type, ne list, raw bytes). general.alignment is
    written first when `alignment` is given. Offsets are assigned in order,
    each padded to the alignment. Returns the data section's start."""
    align = alignment or DEFAULT_ALIGNMENT
    items = ([("general.alignment", U32, align)] if alignment else []) + list(kv)
    head = MAGIC + struct.pack("<IQQ", version, len(tensors), len(items))
    for key, vtype, v in items:
        head += _string(key) + struct.pack("<I", vtype) + _value(vtype, v)
    offsets, off = [], 0
    for name, gtype, ne, raw in tensors:
        assert len(raw) == tensor_nbytes(gtype, ne)
        offsets.append(off)
        off += -(-len(raw) // align) * align
    for (name, gtype, ne, raw), o in zip(tensors, offsets):
        head += _string(name) + struct.pack("<I", len(ne)) + struct.pack("<%dQ" % len(ne), *ne)
        head += struct.pack("<IQ", gtype, o)
    data_start = -(-len(head) // align) * align
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data_start - len(head)))
        for (name, gtype, ne, raw), o in zip(tensors, offsets):
            f.seek(data_start + o)
            f.write(raw)
        end = data_start + off
        f.truncate(end)
    return data_start


class _Cursor:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, fmt):
        v = struct.unpack_from(fmt, self.buf, self.pos)
        self.pos += struct.calcsize(fmt)
        return v[0] if len(v) == 1 else v

    def string(self):
        n = self.take("<Q")
        s = bytes(self.buf[self.pos:self.pos + n])
        assert len(s) == n
        self.pos += n
        return s.decode()

    def value(self, vtype):
        if vtype == STRING:
            return self.string()
        if vtype == ARRAY:
            etype, n = self.take("<IQ")
            return (etype, [self.value(etype) for _ in range(n)])
        return self.take(_SCALAR[vtype])


def read(path):
    """Returns (version, kv dict key -> (type, value), tensors dict name ->
    (ggml type, ne list, absolute file offset, nbytes), data_start)."""
    buf = open(path, "rb").read()
    c = _Cursor(buf)
    assert buf[:4] == MAGIC
    c.pos = 4
    version, n_t, n_kv = c.take("<IQQ")
    kv = {}
    for _ in range(n_kv):
        key = c.string()
        vtype = c.take("<I")
        kv[key] = (vtype, c.value(vtype))
    align = kv.get("general.alignment", (U32, DEFAULT_ALIGNMENT))[1]
    infos = []
    for _ in range(n_t):
        name = c.string()
        nd = c.take("<I")
        ne = list(c.take("<%dQ" % nd)) if nd > 1 else [c.take("<Q")]
        gtype, off = c.take("<IQ")
        infos.append((name, gtype, ne, off))
    data_start = -(-c.pos // align) * align
    tensors = {name: (gtype, ne, data_start + off, tensor_nbytes(gtype, ne)) for name, gtype, ne, off in infos}
    return version, kv, tensors, data_start

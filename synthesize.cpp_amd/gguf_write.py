"""Writes GGUF v3 packages of tensors, the container libsynth_hip's reader
(include/synth_gguf.h) loads: for tools that cut table packages and for the
benchmark's load measurement. The reference cuts its packages with its own
converter and quantizer (tools/synthesize-quantize); this writer emits the
same container layout for the tensor types the gathers read.

Layout (little-endian): "GGUF", u32 version 3, u64 n_tensors, u64 n_kv;
key/values (u64-length strings, u32 value type, value); tensor infos (name,
u32 n_dims, u64 ne[n_dims], u32 ggml type, u64 offset); zero padding to
general.alignment; then each tensor's bytes at its offset, padded to the
alignment.
"""
import struct

GGUF_U32, GGUF_STRING = 4, 8
_TYPE_BLOCKS = {0: (1, 4), 1: (1, 2), 8: (32, 34), 26: (1, 4), 30: (1, 2)}  # F32 F16 Q8_0 I32 BF16


def _gguf_string(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, tensors, strings=(), alignment=32):
    """tensors: (name, ggml type, ne list, bytes-like) in file order; strings:
    (key, value) string metadata. Returns the file offset of the data section."""
    kv = [("general.alignment", GGUF_U32, alignment)] + [(k, GGUF_STRING, v) for k, v in strings]
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    for key, vtype, v in kv:
        head += _gguf_string(key) + struct.pack("<I", vtype)
        head += struct.pack("<I", v) if vtype == GGUF_U32 else _gguf_string(v)
    offsets, off = [], 0
    for name, gtype, ne, raw in tensors:
        be, bb = _TYPE_BLOCKS[gtype]
        rows = 1
        for e in ne[1:]:
            rows *= e
        if ne[0] % be or len(raw) != ne[0] // be * bb * rows:
            raise ValueError("tensor %s: %d bytes do not match its shape" % (name, len(raw)))
        offsets.append(off)
        off += -(-len(raw) // alignment) * alignment
    for (name, gtype, ne, _), o in zip(tensors, offsets):
        head += _gguf_string(name) + struct.pack("<I", len(ne)) + struct.pack("<%dQ" % len(ne), *ne)
        head += struct.pack("<IQ", gtype, o)
    data_start = -(-len(head) // alignment) * alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data_start - len(head)))
        for (_, _, _, raw), o in zip(tensors, offsets):
            f.seek(data_start + o)
            f.write(raw)
        f.truncate(data_start + off)
    return data_start

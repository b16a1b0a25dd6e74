"""Host-side encoders/decoders of the ggml tensor formats the gathers read.

BF16 and F16 rows are stored as raw 16-bit patterns; Q8_0 rows as 34-byte
blocks {f16 d; int8 qs[32]} (ggml's block_q8_0, the embedding-table type of
the Q8_MIXED profile, src/arch/qwen3-tts/catalog.cpp:186-193).
"""
import numpy as np

Q8_0_BLOCK_ELEMS = 32
Q8_0_BLOCK_BYTES = 34


def f32_to_bf16_bits(x):
    """ggml_compute_fp32_to_bf16: round half to even, NaN forced quiet."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u.astype(np.uint64) + (0x7FFF + ((u >> 16) & 1))) >> 16).astype(np.uint16)
    quiet = ((u >> 16) | 64).astype(np.uint16)
    return np.where(nan, quiet, rounded).astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_f16_bits(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_bits_to_f32(b):
    return np.asarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def q8_0_pack(d_bits, qs):
    """d_bits: uint16 (rows, nblocks) f16 scales; qs: int8 (rows, nblocks, 32).
    Returns uint8 (rows, nblocks*34) raw blocks."""
    d_bits = np.ascontiguousarray(d_bits, dtype=np.uint16)
    qs = np.ascontiguousarray(qs, dtype=np.int8)
    rows, nb = d_bits.shape
    out = np.empty((rows, nb, Q8_0_BLOCK_BYTES), dtype=np.uint8)
    out[:, :, 0:2] = d_bits.view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = qs.view(np.uint8)
    return out.reshape(rows, nb * Q8_0_BLOCK_BYTES)


def q8_0_unpack(raw, ne0):
    """Inverse of q8_0_pack: returns (d_bits (rows, nb), qs (rows, nb, 32))."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    rows = raw.shape[0]
    nb = ne0 // Q8_0_BLOCK_ELEMS
    blk = raw.reshape(rows, nb, Q8_0_BLOCK_BYTES)
    d_bits = np.ascontiguousarray(blk[:, :, 0:2]).view(np.uint16).reshape(rows, nb)
    qs = np.ascontiguousarray(blk[:, :, 2:]).view(np.int8)
    return d_bits, qs


def q8_0_dequant(raw, ne0):
    """Closed form of dequantize_row_q8_0: qs * f16(d), one (exact) f32 product."""
    d_bits, qs = q8_0_unpack(raw, ne0)
    d = f16_bits_to_f32(d_bits)
    return (qs.astype(np.float32) * d[:, :, None]).reshape(raw.shape[0], ne0)


def q8_0_quantize(x):
    """ggml's reference quantizer (quantize_row_q8_0_ref): per block d = amax/127,
    qs = round(x/d) to nearest, ties away from zero; d stored as f16."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, ne0 = x.shape
    blk = x.reshape(rows, ne0 // 32, 32)
    amax = np.abs(blk).max(axis=-1)
    d = amax / np.float32(127.0)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), np.float32(0.0)).astype(np.float32)
    v = blk * inv[:, :, None]
    qs = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int8)
    return q8_0_pack(f32_to_f16_bits(d), qs)


def q8_0_synthetic(rng, rows, ne0, d_lo=1e-3, d_hi=1e-2):
    """Synthetic Q8_0 table: qs ~ U{-127..127}, d ~ U[d_lo, d_hi] rounded to f16."""
    nb = ne0 // Q8_0_BLOCK_ELEMS
    qs = rng.integers(-127, 128, size=(rows, nb, 32), dtype=np.int8)
    d = rng.uniform(d_lo, d_hi, size=(rows, nb)).astype(np.float32)
    return q8_0_pack(f32_to_f16_bits(d), qs)

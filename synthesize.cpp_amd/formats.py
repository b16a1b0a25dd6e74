"""Host-side encoders/decoders of the ggml tensor formats the gathers read.

BF16 and F16 rows are stored as raw 16-bit patterns; Q8_0 rows as 34-byte
blocks {f16 d; int8 qs[32]} (ggml's block_q8_0, the embedding-table type of
the Q8_MIXED profile, src/arch/qwen3-tts/catalog.cpp:186-193); Q5_K rows as
176-byte super-blocks of 256 elements (ggml's block_q5_K, the Q5_K_MIXED
profile's).
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


# ---------------------------------------------------------------------------
# Q5_K: ggml's block_q5_K, the Matrix-role tables of Q5_K_MIXED packages
# (src/arch/qwen3-tts/catalog.cpp:165-192): 256-element super-blocks of 176
# bytes -- f16 d, f16 dmin, scales[12], qh[32], qs[128]. Sub-block s (0..7)
# of 32 elements carries a 6-bit scale sc[s] and min m[s]; element i of it is
# the 5-bit q whose low nibble sits in qs[32*(s//2) + i] (low half for even s,
# high half for odd s) and whose bit 4 is bit s of qh[i]. Its value is
# (d*sc)*q - dmin*m.
# ---------------------------------------------------------------------------

Q5_K_BLOCK_ELEMS = 256
Q5_K_BLOCK_BYTES = 176


def q5_k_pack(d_bits, dmin_bits, sc, m, q):
    """d_bits, dmin_bits: uint16 (rows, nb) f16 super-block scales; sc, m:
    (rows, nb, 8) 6-bit sub-block scales and mins; q: (rows, nb, 256) 5-bit
    quants, element order. Returns uint8 (rows, nb*176) raw super-blocks.

    The 6-bit pairs are stored as ggml packs them: scales[s] and scales[s+4]
    hold sc[s] and m[s] for s < 4 in their low six bits; for s >= 4 the low
    and high nibbles of scales[s+4] hold sc[s] and m[s]'s low four bits, and
    their top two bits ride in the high two bits of scales[s-4] (sc) and
    scales[s] (m)."""
    d_bits = np.ascontiguousarray(d_bits, dtype=np.uint16)
    sc = np.asarray(sc, dtype=np.uint8)
    m = np.asarray(m, dtype=np.uint8)
    q = np.asarray(q, dtype=np.uint8)
    rows, nb = d_bits.shape
    assert sc.shape == m.shape == (rows, nb, 8) and q.shape == (rows, nb, 256)
    assert (sc < 64).all() and (m < 64).all() and (q < 32).all()
    out = np.zeros((rows, nb, Q5_K_BLOCK_BYTES), dtype=np.uint8)
    out[:, :, 0:2] = d_bits.view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:4] = np.ascontiguousarray(dmin_bits, dtype=np.uint16).view(np.uint8).reshape(rows, nb, 2)
    scales = np.zeros((rows, nb, 12), dtype=np.uint8)
    for s in range(4):
        scales[:, :, s] = sc[:, :, s] | ((sc[:, :, s + 4] >> 4) << 6)
        scales[:, :, s + 4] = m[:, :, s] | ((m[:, :, s + 4] >> 4) << 6)
        scales[:, :, s + 8] = (sc[:, :, s + 4] & 15) | ((m[:, :, s + 4] & 15) << 4)
    out[:, :, 4:16] = scales
    sub = q.reshape(rows, nb, 8, 32)  # [sub-block s, element i]
    qh = np.zeros((rows, nb, 32), dtype=np.uint8)
    for s in range(8):
        qh |= ((sub[:, :, s, :] >> 4) & 1) << s
    out[:, :, 16:48] = qh
    qs = np.zeros((rows, nb, 4, 32), dtype=np.uint8)
    for j in range(4):
        qs[:, :, j, :] = (sub[:, :, 2 * j, :] & 15) | ((sub[:, :, 2 * j + 1, :] & 15) << 4)
    out[:, :, 48:] = qs.reshape(rows, nb, 128)
    return out.reshape(rows, nb * Q5_K_BLOCK_BYTES)


def q5_k_fields(rng, rows, ne0, d_lo=1e-4, d_hi=1e-3):
    """Random fields of a Q5_K table: q ~ U{0..31}, sc, m ~ U{0..63}, d and
    dmin ~ U[d_lo, d_hi] rounded to f16 (bit patterns)."""
    nb = ne0 // Q5_K_BLOCK_ELEMS
    q = rng.integers(0, 32, size=(rows, nb, 256), dtype=np.uint8)
    sc = rng.integers(0, 64, size=(rows, nb, 8), dtype=np.uint8)
    m = rng.integers(0, 64, size=(rows, nb, 8), dtype=np.uint8)
    d = f32_to_f16_bits(rng.uniform(d_lo, d_hi, size=(rows, nb)))
    dmin = f32_to_f16_bits(rng.uniform(d_lo, d_hi, size=(rows, nb)))
    return d, dmin, sc, m, q


def q5_k_synthetic(rng, rows, ne0, d_lo=1e-4, d_hi=1e-3):
    """Synthetic Q5_K table (raw super-blocks) from q5_k_fields."""
    return q5_k_pack(*q5_k_fields(rng, rows, ne0, d_lo, d_hi))


def q5_k_values(d_bits, dmin_bits, sc, m, q):
    """The values a Q5_K table built by q5_k_pack holds: (d*sc)*q - dmin*m,
    element order, rounded once to f32. Evaluated in double, where both
    products and their difference are exact for scales of comparable
    magnitude (exponents of d and dmin within 2^30 of each other)."""
    d = f16_bits_to_f32(d_bits).astype(np.float64)
    dmin = f16_bits_to_f32(dmin_bits).astype(np.float64)
    rows, nb = d.shape
    scale = (d[:, :, None] * sc.astype(np.float64))[:, :, :, None]
    mins = (dmin[:, :, None] * m.astype(np.float64))[:, :, :, None]
    v = scale * q.reshape(rows, nb, 8, 32).astype(np.float64) - mins
    return v.astype(np.float32).reshape(rows, nb * 256)

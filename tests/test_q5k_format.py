"""The Q5_K table format (ggml's block_q5_K, the Matrix-role tables of the
reference's Q5_K_MIXED packages, src/arch/qwen3-tts/catalog.cpp:165-192) and
the oracle's restatement of dequantize_row_q5_K, without a GPU.

Pins, none of them a retyping of the decoder:
  - two super-blocks assembled by hand, byte by byte, from chosen scales,
    mins and quants, whose values are worked out by hand (the second has
    non-zero quants in every sub-block, uses every qh bit and both nibbles
    of every scales[8..11] byte): the package encoder (formats.q5_k_pack)
    must produce exactly those bytes, and the oracle must decode them to
    exactly those values;
  - random tables: the oracle's values equal (d*sc)*q - dmin*m evaluated
    exactly and rounded once (formats.q5_k_values), element for element;
  - planted layout mistakes (halves of the quant byte swapped, the fifth bit
    taken from the wrong qh bit, the scale/min packing of sub-blocks 4..7
    read from the wrong bytes) each change some value of a random table.
The GPU kernels are held to the oracle bit for bit in tests/test_gpu_q5k.py.
"""
import numpy as np
import pytest

import formats as F
import ggml_ref as R

SC = [1, 2, 3, 4, 33, 34, 35, 63]
M = [5, 6, 7, 8, 17, 18, 40, 62]
Q_SET = {0: 17, 33: 30, 200: 16, 255: 31}  # element -> quant; every other quant is 0


def hand_block():
    """The 176 bytes of the super-block with d = 1.0, dmin = 0.5, scales SC,
    mins M and quants Q_SET, spelled out field by field."""
    b = bytearray(176)
    b[0:2] = bytes([0x00, 0x3C])        # d = 1.0 (f16 0x3c00)
    b[2:4] = bytes([0x00, 0x38])        # dmin = 0.5 (f16 0x3800)
    # scales[0..3]: sc[0..3] in the low six bits, sc[4..7] >> 4 in the top two
    #   1 | 2<<6, 2 | 2<<6, 3 | 2<<6, 4 | 3<<6   (33, 34, 35 >> 4 = 2; 63 >> 4 = 3)
    # scales[4..7]: m[0..3] in the low six bits, m[4..7] >> 4 in the top two
    #   5 | 1<<6, 6 | 1<<6, 7 | 2<<6, 8 | 3<<6   (17, 18 >> 4 = 1; 40 >> 4 = 2; 62 >> 4 = 3)
    # scales[8..11]: sc[4..7] & 15 in the low nibble, m[4..7] & 15 in the high one
    #   1 | 1<<4, 2 | 2<<4, 3 | 8<<4, 15 | 14<<4
    b[4:16] = bytes([129, 130, 131, 196, 69, 70, 135, 200, 17, 34, 131, 239])
    # qh[i] bit s = bit 4 of the quant of element 32s + i
    b[16 + 0] = 0x01   # element 0 (s 0, i 0): 17 = 16 + 1
    b[16 + 1] = 0x02   # element 33 (s 1, i 1): 30 = 16 + 14
    b[16 + 8] = 0x40   # element 200 (s 6, i 8): 16 = 16 + 0
    b[16 + 31] = 0x80  # element 255 (s 7, i 31): 31 = 16 + 15
    # qs[32j + i]: low nibble element 64j + i, high nibble element 64j + 32 + i
    b[48 + 0] = 0x01   # element 0's low four bits
    b[48 + 1] = 0xE0   # element 33 (j 0, high half, i 1): 14
    b[48 + 104] = 0x00  # element 200 (j 3, low half, i 8): 0
    b[48 + 127] = 0xF0  # element 255 (j 3, high half, i 31): 15
    return bytes(b)


def hand_values():
    """(d*sc)*q - dmin*m for the hand block, worked out: q = 0 elements give
    -0.5*m of their sub-block."""
    v = np.repeat(np.float32(-0.5) * np.array(M, np.float32), 32)
    v[0] = 1 * 17 - 0.5 * 5     # 14.5
    v[33] = 2 * 30 - 0.5 * 6    # 57
    v[200] = 35 * 16 - 0.5 * 40  # 540
    v[255] = 63 * 31 - 0.5 * 62  # 1922
    return v.astype(np.float32)


# A second block: non-zero quants in every sub-block (one with the fifth bit,
# so all eight qh bits are used, and one without), both nibbles of every
# scales[8..11] byte non-zero, top bits of scales[0..7] of every value 0..3,
# a sub-block with m = 0 (its zero quants give +0.0).
D2, DMIN2 = 0x3400, 0x4000  # 0.25, 2.0
SC2 = [63, 1, 17, 32, 47, 50, 5, 60]
M2 = [0, 63, 9, 21, 48, 31, 12, 3]
Q_SET2 = {32 * s + (5 * s + 3) % 32: 16 + s for s in range(8)}
Q_SET2.update({32 * s + (7 * s + 11) % 32: 15 - s for s in range(8)})


def hand_block2():
    b = bytearray(176)
    b[0:2] = bytes([0x00, 0x34])        # d = 0.25 (f16 0x3400)
    b[2:4] = bytes([0x00, 0x40])        # dmin = 2.0 (f16 0x4000)
    # scales[j], j < 4: sc[j] | (sc[j+4] >> 4) << 6
    #   63 | 2<<6 = 191, 1 | 3<<6 = 193, 17 | 0 = 17, 32 | 3<<6 = 224   (47, 50, 5, 60 >> 4 = 2, 3, 0, 3)
    # scales[j+4]: m[j] | (m[j+4] >> 4) << 6
    #   0 | 3<<6 = 192, 63 | 1<<6 = 127, 9 | 0 = 9, 21 | 0 = 21         (48, 31, 12, 3 >> 4 = 3, 1, 0, 0)
    # scales[8+j]: (sc[j+4] & 15) | (m[j+4] & 15) << 4
    #   15 | 0<<4 = 15, 2 | 15<<4 = 242, 5 | 12<<4 = 197, 12 | 3<<4 = 60
    b[4:16] = bytes([191, 193, 17, 224, 192, 127, 9, 21, 15, 242, 197, 60])
    # sub-block s: element 32s + (5s+3)%32 holds 16 + s (fifth bit set), so
    # qh[(5s+3)%32] carries bit s: qh[3]=0x01, qh[8]=0x02, qh[13]=0x04,
    # qh[18]=0x08, qh[23]=0x10, qh[28]=0x20, qh[1]=0x40, qh[6]=0x80
    for i, v in ((3, 0x01), (8, 0x02), (13, 0x04), (18, 0x08), (23, 0x10), (28, 0x20), (1, 0x40), (6, 0x80)):
        b[16 + i] = v
    # qs[32j + i]: sub-block 2j in the low nibble, 2j+1 in the high one.
    # The fifth-bit quants' low nibbles s: qs[3] lo 0, qs[8] hi 1, qs[45] lo 2,
    # qs[50] hi 3, qs[87] lo 4, qs[92] hi 5, qs[97] lo 6, qs[102] hi 7;
    # element 32s + (7s+11)%32 holds 15 - s: qs[11] lo 15, qs[18] hi 14,
    # qs[57] lo 13, qs[32] hi 12, qs[71] lo 11, qs[78] hi 10, qs[117] lo 9, qs[124] hi 8
    for i, v in ((3, 0x00), (8, 0x10), (45, 0x02), (50, 0x30), (87, 0x04), (92, 0x50), (97, 0x06), (102, 0x70),
                 (11, 0x0F), (18, 0xE0), (57, 0x0D), (32, 0xC0), (71, 0x0B), (78, 0xA0), (117, 0x09), (124, 0x80)):
        b[48 + i] = v
    return bytes(b)


def hand_values2():
    """Worked out: d*sc = 15.75, 0.25, 4.25, 8, 11.75, 12.5, 1.25, 15 and
    dmin*m = 0, 126, 18, 42, 96, 62, 24, 6; a zero quant gives 0 - dmin*m
    (+0.0 in sub-block 0)."""
    base = [0.0, -126.0, -18.0, -42.0, -96.0, -62.0, -24.0, -6.0]
    v = np.repeat(np.array(base, np.float32), 32)
    fifth = [252.0, -121.75, 58.5, 110.0, 139.0, 200.5, 3.5, 339.0]    # (d*sc)*(16+s) - dmin*m
    plain = [236.25, -122.5, 37.25, 54.0, 33.25, 63.0, -12.75, 114.0]  # (d*sc)*(15-s) - dmin*m
    for s in range(8):
        v[32 * s + (5 * s + 3) % 32] = fifth[s]
        v[32 * s + (7 * s + 11) % 32] = plain[s]
    return v


def hand_fields2():
    q = np.zeros((1, 1, 256), np.uint8)
    for e, v in Q_SET2.items():
        q[0, 0, e] = v
    return (np.array([[D2]], np.uint16), np.array([[DMIN2]], np.uint16),
            np.array([[SC2]], np.uint8), np.array([[M2]], np.uint8), q)


def hand_fields():
    q = np.zeros((1, 1, 256), np.uint8)
    for e, v in Q_SET.items():
        q[0, 0, e] = v
    return (np.array([[0x3C00]], np.uint16), np.array([[0x3800]], np.uint16),
            np.array([[SC]], np.uint8), np.array([[M]], np.uint8), q)


def oracle_rows(raw, ne0, ids):
    return R.run(lambda g: g.get_rows(raw, R.Q5_K, ne0, np.asarray(ids, np.int32)))


def test_encoder_reproduces_the_hand_assembled_block():
    assert F.q5_k_pack(*hand_fields()).tobytes() == hand_block()
    assert F.q5_k_values(*hand_fields())[0].tolist() == hand_values().tolist()


def test_oracle_decodes_the_hand_block_to_the_hand_values():
    raw = np.frombuffer(hand_block(), np.uint8).reshape(1, 176)
    got = oracle_rows(raw, 256, [0])[0]
    assert got.tolist() == hand_values().tolist()


def test_second_hand_block():
    """Every sub-block's scale and min, every qh bit, both nibbles of every
    scales[8..11] byte: the encoder writes the bytes spelled out above, and
    the oracle decodes them to the worked-out values bit for bit (including
    the +0.0 of sub-block 0's zero quants)."""
    assert F.q5_k_pack(*hand_fields2()).tobytes() == hand_block2()
    raw = np.frombuffer(hand_block2(), np.uint8).reshape(1, 176)
    got = oracle_rows(raw, 256, [0])[0]
    assert np.array_equal(got.view(np.uint32), hand_values2().view(np.uint32))
    assert F.q5_k_values(*hand_fields2())[0].view(np.uint32).tolist() == hand_values2().view(np.uint32).tolist()


@pytest.mark.parametrize("ne0", [256, 1024, 2048])
def test_oracle_equals_the_exact_formula(ne0):
    rng = np.random.default_rng(20260728 + ne0)
    f = F.q5_k_fields(rng, 40, ne0)
    raw = F.q5_k_pack(*f)
    want = F.q5_k_values(*f)
    ids = rng.integers(0, 40, 64)
    got = oracle_rows(raw, ne0, ids)
    assert np.array_equal(got.view(np.uint32), want[ids].view(np.uint32))


def test_the_value_is_one_rounding():
    """(d*sc)*q and dmin*m are exact in f32 (at most 22 and 17 significant
    bits), so fused and unfused evaluations agree: checked on the whole f16
    range of d and dmin that keeps the products finite."""
    rng = np.random.default_rng(5)
    d = F.f16_bits_to_f32(rng.integers(0, 0x7800, 4096).astype(np.uint16)).astype(np.float32)
    dmin = F.f16_bits_to_f32(rng.integers(0, 0x7800, 4096).astype(np.uint16)).astype(np.float32)
    sc, m, q = rng.integers(0, 64, 4096), rng.integers(0, 64, 4096), rng.integers(0, 32, 4096)
    d1 = (d * sc.astype(np.float32)).astype(np.float32)
    m1 = (dmin * m.astype(np.float32)).astype(np.float32)
    assert np.array_equal(d1.astype(np.float64), d.astype(np.float64) * sc)  # exact
    assert np.array_equal(m1.astype(np.float64), dmin.astype(np.float64) * m)
    p = (d1 * q.astype(np.float32)).astype(np.float32)
    assert np.array_equal(p.astype(np.float64), d1.astype(np.float64) * q)


def _decode(raw, ne0, mistake=None):
    """A numpy decoder of the layout, with an optional planted mistake."""
    rows = raw.shape[0]
    blk = raw.reshape(rows, ne0 // 256, 176)
    d = F.f16_bits_to_f32(np.ascontiguousarray(blk[:, :, 0:2]).view(np.uint16)[..., 0])
    dmin = F.f16_bits_to_f32(np.ascontiguousarray(blk[:, :, 2:4]).view(np.uint16)[..., 0])
    sc_b = blk[:, :, 4:16].astype(np.int32)
    qh, qs = blk[:, :, 16:48].astype(np.int32), blk[:, :, 48:].astype(np.int32)
    out = np.empty((rows, ne0 // 256, 256), np.float32)
    for s in range(8):
        if s < 4:
            sc, m = sc_b[..., s] & 63, sc_b[..., s + 4] & 63
        elif mistake == "packing":
            sc = (sc_b[..., s + 4] & 15) | ((sc_b[..., s] >> 6) << 4)
            m = (sc_b[..., s + 4] >> 4) | ((sc_b[..., s - 4] >> 6) << 4)
        else:
            sc = (sc_b[..., s + 4] & 15) | ((sc_b[..., s - 4] >> 6) << 4)
            m = (sc_b[..., s + 4] >> 4) | ((sc_b[..., s] >> 6) << 4)
        half = 1 - (s & 1) if mistake == "halves" else s & 1
        bit = s // 2 if mistake == "qh_bit" else s
        nib = (qs[..., 32 * (s // 2):32 * (s // 2) + 32] >> (4 * half)) & 15
        q = nib | (((qh >> bit) & 1) << 4)
        d1 = (d * sc.astype(np.float32)).astype(np.float32)
        m1 = (dmin * m.astype(np.float32)).astype(np.float32)
        out[:, :, 32 * s:32 * s + 32] = d1[..., None] * q.astype(np.float32) - m1[..., None]
    return out.reshape(rows, ne0)


@pytest.mark.parametrize("mistake", [None, "halves", "qh_bit", "packing"])
def test_planted_layout_mistakes_are_caught(mistake):
    rng = np.random.default_rng(11)
    f = F.q5_k_fields(rng, 16, 1024)
    got = _decode(F.q5_k_pack(*f), 1024, mistake)
    same = np.array_equal(got.view(np.uint32), F.q5_k_values(*f).view(np.uint32))
    assert same == (mistake is None)
    hand = _decode(np.frombuffer(hand_block(), np.uint8).reshape(1, 176), 256, mistake)[0]
    assert np.array_equal(hand, hand_values()) == (mistake is None)
    hand2 = _decode(np.frombuffer(hand_block2(), np.uint8).reshape(1, 176), 256, mistake)[0]
    assert np.array_equal(hand2.view(np.uint32), hand_values2().view(np.uint32)) == (mistake is None)

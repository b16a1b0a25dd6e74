// Geometry and integer decoding of the Q5_K reads of the gather->sum windows,
// shared by the kernels and the host check (tests/host/q5k_window_check.cpp),
// so both use one formula.
//
// A Q5_K super-block (ggml's block_q5_K) holds 256 elements in 176 bytes:
// f16 d at byte 0, f16 dmin at 2, scales[12] at 4, qh[32] at 16, qs[128] at
// 48. Element e = 64j + 32h + i (j < 4, h < 2, i < 32) has the 4-bit quant
// (qs[32j + i] >> 4h) & 15, the fifth bit (qh[i] >> s) & 1 and the 6-bit
// scale and min of its sub-block s = 2j + h: for s < 4, scales[s] & 63 and
// scales[s + 4] & 63; for s >= 4, (scales[s + 4] & 15) | (scales[s - 4] >> 6) << 4
// and (scales[s + 4] >> 4) | (scales[s] >> 6) << 4 (ggml's get_scale_min_k4).
//
// A 1024-element slab is four super-blocks, 704 bytes. Lane l of a wave owns
// elements 16k..16k+15 (k = l % 16) of super-block b = l / 16 of the slab,
// which all lie in sub-block s = k / 2 (j = k / 4, h = s & 1) at
// i = 16(k & 1)..16(k & 1) + 15. It reads three aligned pieces, all inside
// its super-block [176b, 176b + 176):
//   - the header, d | dmin << 16 and scales[0..11]: [176b, 176b + 16)
//   - qh[i .. i + 15]:        [176b + 16 + i, +16)
//   - qs[32j + i .. + 15]:    [176b + 48 + 32j + i, +16)
// Quant byte t of the lane (element 16k + t) is then nibble h of qs byte t
// plus bit s of qh byte t, moved to bit 4.
#pragma once

#include <cstdint>

#ifndef SHP_HD
#    if defined(__HIPCC__)
#        define SHP_HD __host__ __device__
#    else
#        define SHP_HD
#    endif
#endif

namespace shp {

constexpr uint32_t kQ5KSuperBytes = 176;
constexpr uint32_t kQ5KSuperElems = 256;
constexpr uint32_t kQ5KSlabElems  = 1024;
constexpr uint32_t kQ5KSlabBytes  = kQ5KSlabElems / kQ5KSuperElems * kQ5KSuperBytes;  // 704
constexpr uint32_t kQ5KMaxSlabs   = 4;  // widest row of the window kernel: 4096 elements

// Four slabs of super-blocks whose every element decodes to -0.0f: d = -0.0
// (f16 0x8000), dmin = +0.0, zero scales, mins and quants, so each value is
// fma(-0 * 0, q, -(+0 * 0)) = -0.0f, and acc + -0.0f == acc for every f32 acc
// (including -0.0 and NaN). A gather->sum slot past the last group reads it
// and adds nothing.
struct Q5KNegZeroRow {
    uint32_t w[kQ5KMaxSlabs * kQ5KSlabBytes / 4];
};

SHP_HD constexpr Q5KNegZeroRow q5k_neg_zero_row() {
    Q5KNegZeroRow r{};
    for (uint32_t i = 0; i < kQ5KMaxSlabs * kQ5KSlabBytes / 4; ++i) {
        r.w[i] = i % (kQ5KSuperBytes / 4) == 0u ? 0x00008000u : 0u;
    }
    return r;
}

struct Q5KWinPos {
    uint32_t hdr;  // byte offset of the lane's super-block (its header) in the slab
    uint32_t qh;   // byte offset of its four qh dwords
    uint32_t qs;   // byte offset of its four qs dwords
    uint32_t s;    // its sub-block
};

SHP_HD inline Q5KWinPos q5k_win_pos(int l) {
    const uint32_t b   = static_cast<uint32_t>(l) / 16u;
    const uint32_t k   = static_cast<uint32_t>(l) % 16u;
    const uint32_t i   = 16u * (k & 1u);
    const uint32_t blk = kQ5KSuperBytes * b;
    return Q5KWinPos{ blk, blk + 16u + i, blk + 48u + 32u * (k / 4u) + i, k / 2u };
}

// x rotated right by r (0..31): one v_alignbit_b32 on the device.
SHP_HD inline uint32_t rotr32(uint32_t x, uint32_t r) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_alignbit(x, x, r);
#else
    return (x >> r) | (x << ((32u - r) & 31u));
#endif
}

// The four 5-bit quants of sub-block s held by qs and qh dwords covering the
// same four elements, one per byte. Rotating qh right by s - 4 (mod 32) moves
// bit s of every byte to bit 4 of the same byte.
SHP_HD inline uint32_t q5k_quads(uint32_t qs, uint32_t qh, uint32_t s) {
    return ((qs >> (4u * (s & 1u))) & 0x0F0F0F0Fu) | (rotr32(qh, (s + 28u) & 31u) & 0x10101010u);
}

// Bits off..off+width-1 of x (width < 32): one v_bfe_u32 on the device.
SHP_HD inline uint32_t ubits(uint32_t x, uint32_t off, uint32_t width) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_ubfe(x, off, width);
#else
    return (x >> off) & ((1u << width) - 1u);
#endif
}

// The 6-bit scale and min of sub-block s from the scale dwords w1..w3
// (scales[0..11], little-endian). Every byte sub-block s needs sits at the
// same shift sh = 8(s & 3) of one of them: b1 = scales[s & 3] in w1,
// b2 = scales[4 + (s & 3)] in w2, b3 = scales[8 + (s & 3)] in w3. Both
// cases are one form, low four bits | two high bits << 4, with the sources
// picked by selects rather than branches:
//   s < 4:  sc = (b1 & 15) | (b1 >> 4 & 3) << 4,  m = (b2 & 15) | (b2 >> 4 & 3) << 4
//   s >= 4: sc = (b3 & 15) | (b1 >> 6) << 4,      m = (b3 >> 4) | (b2 >> 6) << 4
SHP_HD inline void q5k_scale_min(uint32_t w1, uint32_t w2, uint32_t w3, uint32_t s, uint32_t & sc, uint32_t & m) {
    const uint32_t sh  = 8u * (s & 3u);
    const bool     hi  = s >= 4u;
    const uint32_t top = sh + (hi ? 6u : 4u);  // offset of the two high bits in w1 and w2
    sc                 = ubits(hi ? w3 : w1, sh, 4u) | (ubits(w1, top, 2u) << 4);
    m                  = ubits(hi ? w3 : w2, sh + (hi ? 4u : 0u), 4u) | (ubits(w2, top, 2u) << 4);
}

}  // namespace shp

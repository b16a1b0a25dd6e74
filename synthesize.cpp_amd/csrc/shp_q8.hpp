// Geometry of the Q8_0 half-block reads, shared by the gather kernels and the
// host bounds check (tests/host/q8_bounds_check.cpp), so both use one formula.
//
// A Q8_0 row of ne0 elements is ne0/32 blocks of {f16 d; int8 qs[32]}, 34
// bytes each, starting on a 4-byte boundary. Lane l owns elements
// 16l..16l+15: half h = l & 1 of block b = l >> 1. Its quants occupy bytes
// [34b + 2 + 16h, 34b + 18 + 16h) of the row: 4-byte aligned when b is odd,
// 2 bytes off when b is even. The lane reads three aligned pieces:
//   - the dword holding d:        [dbase, dbase + 4)
//   - a dwordx4 at the quants:    [qbase, qbase + 16)
//   - one more dword:             [tail, tail + 4)
// When the quants are 2 bytes off (qsh), tail = qbase + 16 and the five
// dwords qbase..qbase+20 are shifted by 2 bytes (v_alignbyte) to give the
// 16 quants. When they are aligned, the dwordx4 holds them all and the extra
// dword is not used, so it is read from qbase + 12 (inside the row) instead
// of qbase + 16, which for the row's last half-block is past its end.
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

constexpr uint32_t kQ8BlockBytes = 34;
constexpr uint32_t kQ8BlockElems = 32;

struct Q8HalfPos {
    uint32_t qbase;  // byte offset of the dwordx4 (4-aligned)
    uint32_t tail;   // byte offset of the fifth dword (4-aligned)
    uint32_t dbase;  // byte offset of the dword holding d (4-aligned)
    bool     qsh;    // quants start 2 bytes into the dwordx4
    bool     dhi;    // d is the high half of its dword
};

SHP_HD inline Q8HalfPos q8_half_pos(int l) {
    const uint32_t b    = static_cast<uint32_t>(l) >> 1;
    const uint32_t qoff = kQ8BlockBytes * b + 2u + 16u * (static_cast<uint32_t>(l) & 1u);
    const uint32_t doff = kQ8BlockBytes * b;
    const uint32_t qb   = qoff & ~3u;
    const bool     qsh  = (qoff & 2u) != 0;
    return Q8HalfPos{ qb, qsh ? qb + 16u : qb + 12u, doff & ~3u, qsh, (doff & 2u) != 0 };
}

// Bytes sh..sh+3 of the 8-byte little-endian value hi:lo (sh in 0..3): one
// v_alignbyte_b32 on the device. The byte shift is an operand, so shifted and
// aligned lanes run the same instruction on the same registers. (Writing it
// as `qsh ? align(w[i+1], w[i]) : w[i]` lets the compiler select between two
// array addresses, which is a dynamic index: the lane's words then live in
// LDS instead of registers.)
SHP_HD inline uint32_t bytes_at(uint32_t hi, uint32_t lo, uint32_t sh) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_alignbyte(hi, lo, sh);
#else
    return static_cast<uint32_t>(((static_cast<uint64_t>(hi) << 32) | lo) >> (8u * sh));
#endif
}

// The f16 bits of d and the four quant dwords (little-endian bytes) of a lane,
// from the six dwords it loaded: w[0] at dbase, w[1..4] at qbase, w[5] at tail.
SHP_HD inline uint32_t q8_half_dbits(const uint32_t (&w)[6], const Q8HalfPos & p) {
    return (w[0] >> (p.dhi ? 16u : 0u)) & 0xffffu;
}

SHP_HD inline uint32_t q8_half_quads(const uint32_t (&w)[6], const Q8HalfPos & p, int i) {
    return bytes_at(w[2 + i], w[1 + i], p.qsh ? 2u : 0u);
}

// ---------------------------------------------------------------------------
// Five-dword windows (the gather->sum over 1024-element slabs).
//
// Lane l again owns half h = l & 1 of block b = l >> 1 of a 1088-byte slab,
// with quants at qs = 34b + 2 + 16h, but reads one window of five aligned
// dwords [base, base + 20), base = (qs - 2) & ~3: the quants are bytes
// shift..shift+15 of it, shift = qs - base, which is 2 (qs = 2 mod 4) or 4
// (qs = 0 mod 4). Quant dword i is bytes shift..shift+3 of w[i+1]:w[i], one
// v_perm_b32 with a per-lane selector. For the even lane (h = 0) the window
// starts at d or two bytes before it, so w[0] holds d -- in its high half
// exactly when shift is 4; the odd lane of the pair has the same b, the same
// shift, and takes w[0] from its even neighbour. Every window lies inside
// [34b - 2, 34b + 34), so inside the slab: lane 0 starts at byte 0 and lane 63
// ends at byte 1088.
// ---------------------------------------------------------------------------

constexpr uint32_t kQ8SlabElems = 1024;
constexpr uint32_t kQ8SlabBytes = kQ8SlabElems / kQ8BlockElems * kQ8BlockBytes;  // 1088

struct Q8WinPos {
    uint32_t base;  // byte offset of the window in the slab (4-aligned)
    uint32_t sel;   // v_perm_b32 selector: bytes 2..5 or 4..7 of hi:lo
    uint32_t dsh;   // bit shift of d within the (even lane's) w[0]: 0 or 16
};

SHP_HD inline Q8WinPos q8_win_pos(int l) {
    const uint32_t b     = static_cast<uint32_t>(l) >> 1;
    const uint32_t qs    = kQ8BlockBytes * b + 2u + 16u * (static_cast<uint32_t>(l) & 1u);
    const uint32_t base  = (qs - 2u) & ~3u;
    const bool     four  = qs - base == 4u;
    return Q8WinPos{ base, four ? 0x07060504u : 0x05040302u, four ? 16u : 0u };
}

// Four slabs of a Q8_0 row whose every block is d = -0.0 (f16 0x8000) and 32
// zero quants: a window of it decodes to 0 * -0.0 = -0.0, and acc + -0.0 ==
// acc for every f32 acc (including -0.0 and NaN), so a gather->sum slot that
// reads it adds nothing. Two blocks are 68 bytes = 17 dwords: d of the first
// is the low half of dword 0, d of the second the high half of dword 8.
struct Q8NegZeroRow {
    uint32_t w[4 * kQ8SlabBytes / 4];
};

SHP_HD constexpr Q8NegZeroRow q8_neg_zero_row() {
    Q8NegZeroRow r{};
    for (uint32_t i = 0; i < 4 * kQ8SlabBytes / 4; ++i) {
        r.w[i] = i % 17u == 0u ? 0x00008000u : (i % 17u == 8u ? 0x80000000u : 0u);
    }
    return r;
}

// Bytes of hi:lo (lo = bytes 0..3) picked by the four selector bytes (each
// 0..7): one v_perm_b32 on the device.
SHP_HD inline uint32_t perm_bytes(uint32_t hi, uint32_t lo, uint32_t sel) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_perm(hi, lo, sel);
#else
    const uint64_t v = (static_cast<uint64_t>(hi) << 32) | lo;
    uint32_t       r = 0;
    for (int i = 0; i < 4; ++i) {
        r |= static_cast<uint32_t>((v >> (8u * ((sel >> (8 * i)) & 7u))) & 0xffu) << (8 * i);
    }
    return r;
#endif
}

// ---------------------------------------------------------------------------
// LDS-staged rows (ne0 = 1024, 2048, 4096; rows 16-byte aligned).
//
// A wave copies one row (68 dwords per 256 elements) into a private LDS
// buffer with aligned loads: NQ/4 rounds of one dwordx4 per lane (dwords
// 4l..4l+3 of each 256-dword round), then one dword per lane for the 4*NQ
// dwords left (lanes l < 4*NQ). NQ = ne0/256.
//
// Lane l then decodes output quad k (elements 256k + 4l .. 256k + 4l + 3), so
// that the wave's k-th float4 store covers 1 KB of contiguous output. The four
// quants sit in block blk = 8k + (l >> 3), at byte 34*blk + 2 + 4*(l & 7):
// 4-byte aligned for odd blk, 2 bytes off for even blk. The lane reads the
// dword at that offset rounded down (adw), the next one (adw + 1) and the
// dword holding d (ddw); bytes_at(lds[adw + 1], lds[adw], sh) are the quants.
// For the last block (odd, so sh = 0) dword adw + 1 can lie one dword past
// the row: the buffer carries kQ8StagePadDwords of padding for it.
// ---------------------------------------------------------------------------

constexpr uint32_t kQ8StagePadDwords = 4;

SHP_HD constexpr uint32_t q8_row_dwords(uint32_t nq) {
    return 68u * nq;
}

struct Q8QuadPos {
    uint32_t adw;  // dword index holding the first quant (rounded down)
    uint32_t ddw;  // dword index holding d
    uint32_t sh;   // byte shift of the quants within adw:adw+1 (0 or 2)
    uint32_t dsh;  // bit shift of d within its dword (0 or 16)
};

SHP_HD inline Q8QuadPos q8_quad_pos(int k, int l) {
    const uint32_t blk  = 8u * static_cast<uint32_t>(k) + (static_cast<uint32_t>(l) >> 3);
    const uint32_t qoff = kQ8BlockBytes * blk + 2u + 4u * (static_cast<uint32_t>(l) & 7u);
    const uint32_t doff = kQ8BlockBytes * blk;
    return Q8QuadPos{ qoff >> 2, doff >> 2, qoff & 3u, (doff & 2u) ? 16u : 0u };
}

}  // namespace shp

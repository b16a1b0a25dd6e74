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

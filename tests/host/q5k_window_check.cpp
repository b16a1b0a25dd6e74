// Host check of the Q5_K window geometry and integer decoding of the
// gather->sum kernel (shp_q5k.hpp).
//
// For random 1024-element slabs (four super-blocks, 704 bytes, placed at the
// very end of a buffer) and every lane of the wave:
//   1. the lane's three 16-byte pieces (the header, qh bytes, qs bytes) lie
//      inside its own super-block, 4-byte aligned;
//   2. the 64 lanes' elements 16l..16l+15 tile the slab exactly once;
//   3. the scale, min and 16 quants the kernel decodes from those pieces
//      equal ggml's byte-level definition (get_scale_min_k4 and the qs/qh bit
//      layout of dequantize_row_q5_K), written out here from the bytes with
//      no shared code.
// Scale bytes are drawn from all 256 values, so every bit of the packed
// scales is exercised. Also checks the -0.0 row that slots past the last
// group read (every lane decodes d = -0, dmin = +0, scale, min and quants 0)
// and that such a slot's fma(-0, q, -0) = -0 adds nothing to any sum, and
// rotr32 against a plain rotate.
// Prints "<lanes checked> <failures>" and exits non-zero on any failure.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "shp_q5k.hpp"

static long checked = 0, failures = 0;

static void fail(const char * what, int l) {
    if (++failures <= 10) {
        std::printf("FAIL %s lane=%d\n", what, l);
    }
}

// ggml's get_scale_min_k4 over the 12 scale bytes, for sub-block j.
static void ref_scale_min(const uint8_t * q, int j, uint32_t & sc, uint32_t & m) {
    if (j < 4) {
        sc = q[j] & 63u;
        m  = q[j + 4] & 63u;
    } else {
        sc = (q[j + 4] & 0xFu) | ((q[j - 4] >> 6) << 4);
        m  = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// The 5-bit quant of element e of a super-block, from its bytes.
static uint32_t ref_quant(const uint8_t * blk, int e) {
    const int j = e / 64, h = (e / 32) % 2, i = e % 32;
    const uint8_t ql = blk[48 + 32 * j + i];
    const uint8_t qh = blk[16 + i];
    return ((ql >> (4 * h)) & 0xFu) + (((qh >> (2 * j + h)) & 1u) ? 16u : 0u);
}

static uint32_t dword_at(const std::vector<uint8_t> & buf, size_t base, uint32_t off) {
    uint32_t v;
    std::memcpy(&v, buf.data() + base + off, 4);
    return v;
}

static void check_slab(std::mt19937 & rng) {
    const size_t         guard = 64;
    std::vector<uint8_t> buf(guard + shp::kQ5KSlabBytes);
    for (auto & b : buf) {
        b = static_cast<uint8_t>(rng());
    }
    const size_t base = guard;  // the slab ends exactly at the end of the buffer
    std::vector<int> hits(shp::kQ5KSlabElems, 0);
    for (int l = 0; l < 64; ++l) {
        ++checked;
        const shp::Q5KWinPos p   = shp::q5k_win_pos(l);
        const uint32_t       b   = static_cast<uint32_t>(l) / 16u;
        const uint32_t       lo  = shp::kQ5KSuperBytes * b;
        const uint32_t       hi  = lo + shp::kQ5KSuperBytes;
        const bool in_block = p.hdr % 4 == 0 && p.qh % 4 == 0 && p.qs % 4 == 0 && p.hdr >= lo && p.hdr + 16 <= hi &&
                              p.qh >= lo && p.qh + 16 <= hi && p.qs >= lo && p.qs + 16 <= hi;
        if (!in_block || p.hdr != lo) {
            fail("piece outside the lane's super-block", l);
            continue;
        }
        uint32_t w[4];
        for (int t = 0; t < 4; ++t) {
            w[t] = dword_at(buf, base, p.hdr + 4u * static_cast<uint32_t>(t));
        }
        const uint8_t * blk = buf.data() + base + lo;
        uint32_t        sc, m, rsc, rm;
        shp::q5k_scale_min(w[1], w[2], w[3], p.s, sc, m);
        const int e0 = 16 * (l % 16);  // the lane's first element in the super-block
        ref_scale_min(blk + 4, (e0 / 64) * 2 + (e0 / 32) % 2, rsc, rm);
        if (sc != rsc || m != rm) {
            fail("scale/min", l);
        }
        if ((w[0] & 0xffffu) != (blk[0] | (blk[1] << 8)) || (w[0] >> 16) != (blk[2] | (blk[3] << 8))) {
            fail("d/dmin bits", l);
        }
        for (int t = 0; t < 4; ++t) {
            const uint32_t q4 = shp::q5k_quads(dword_at(buf, base, p.qs + 4u * t), dword_at(buf, base, p.qh + 4u * t), p.s);
            for (int k = 0; k < 4; ++k) {
                const int e = e0 + 4 * t + k;
                if (((q4 >> (8 * k)) & 0xffu) != ref_quant(blk, e)) {
                    fail("quant", l);
                }
                ++hits[256 * b + static_cast<uint32_t>(e)];
            }
        }
    }
    for (uint32_t e = 0; e < shp::kQ5KSlabElems; ++e) {
        if (hits[e] != 1) {
            fail("lanes do not tile the slab", static_cast<int>(e));
        }
    }
}

static void check_neg_zero_row() {
    const shp::Q5KNegZeroRow z = shp::q5k_neg_zero_row();
    for (uint32_t slab = 0; slab < shp::kQ5KMaxSlabs; ++slab) {
        for (int l = 0; l < 64; ++l) {
            const shp::Q5KWinPos p    = shp::q5k_win_pos(l);
            const uint32_t       off  = slab * shp::kQ5KSlabBytes;
            const uint32_t *     w    = z.w + (off + p.hdr) / 4;
            uint32_t             sc, m;
            shp::q5k_scale_min(w[1], w[2], w[3], p.s, sc, m);
            if (w[0] != 0x00008000u || sc != 0 || m != 0) {
                fail("-0.0 row header", l);
            }
            for (int t = 0; t < 4; ++t) {
                if (shp::q5k_quads(z.w[(off + p.qs) / 4 + t], z.w[(off + p.qh) / 4 + t], p.s) != 0) {
                    fail("-0.0 row quants", l);
                }
            }
        }
    }
}

static void check_dead_slot_and_rotate(std::mt19937 & rng) {
    const float accs[] = { -0.0f, 0.0f, 1.0f, -3.5f, 1e-45f, -1e-45f, 3.4e38f, INFINITY, -INFINITY, NAN };
    for (float acc : accs) {
        for (int q = 0; q < 32; ++q) {
            const float v   = std::fma(-0.0f, static_cast<float>(q), -0.0f);
            const float sum = acc + v;
            uint32_t    a, s;
            std::memcpy(&a, &acc, 4);
            std::memcpy(&s, &sum, 4);
            if (a != s) {
                fail("dead slot changes the sum", q);
            }
        }
    }
    for (int rep = 0; rep < 100000; ++rep) {
        const uint32_t x = static_cast<uint32_t>(rng());
        const uint32_t r = static_cast<uint32_t>(rng()) % 32u;
        const uint64_t xx = (static_cast<uint64_t>(x) << 32) | x;
        if (shp::rotr32(x, r) != static_cast<uint32_t>(xx >> r)) {
            fail("rotr32", static_cast<int>(r));
        }
    }
}

int main() {
    std::mt19937 rng(20260728);
    for (int rep = 0; rep < 2000; ++rep) {
        check_slab(rng);
    }
    check_neg_zero_row();
    check_dead_slot_and_rotate(rng);
    std::printf("%ld %ld\n", checked, failures);
    return failures == 0 ? 0 : 1;
}

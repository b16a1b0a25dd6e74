// Host check of the Q8_0 read geometry the gather kernels use (shp_q8.hpp).
//
// For every row width the half-block kernels take (256..4096) and every lane:
//   1. each byte the lane reads (the d dword, the dwordx4, the tail dword) lies
//      inside the row, [0, ne0/32*34);
//   2. decoding the six dwords exactly as the kernel does gives the lane's
//      block scale bits and its 16 quants, compared with the block's bytes
//      read directly.
// The row is filled with random bytes and placed at the very end of a buffer
// followed by guard bytes that no read may touch. Also checks the block-pair
// reads (68 bytes at 68*bp) of the other widths that are multiples of 64, the
// LDS-staged quads, and the gather->sum's five-dword windows per 1024-element
// slab.
// Prints "<lanes checked> <failures>" and exits non-zero on any failure.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "shp_q8.hpp"

static long checked = 0, failures = 0;

static void fail(const char * what, int ne0, int l) {
    if (++failures <= 10) {
        std::printf("FAIL %s ne0=%d lane=%d\n", what, ne0, l);
    }
}

static uint32_t load_dword(const std::vector<uint8_t> & buf, size_t row0, uint32_t off, uint32_t rowbytes, int ne0,
                           int l, bool & ok) {
    if (off % 4 != 0 || off + 4 > rowbytes) {
        fail("read outside the row", ne0, l);
        ok = false;
        return 0;
    }
    uint32_t v;
    std::memcpy(&v, buf.data() + row0 + off, 4);
    return v;
}

static void check_half(int ne0, std::mt19937 & rng) {
    const uint32_t rowbytes = static_cast<uint32_t>(ne0 / 32) * shp::kQ8BlockBytes;
    const size_t   guard    = 64;
    std::vector<uint8_t> buf(rowbytes + guard);
    for (auto & b : buf) {
        b = static_cast<uint8_t>(rng());
    }
    const size_t row0 = 0;
    for (int l = 0; l < ne0 / 16; ++l) {
        ++checked;
        const shp::Q8HalfPos p = shp::q8_half_pos(l);
        bool                 ok = true;
        uint32_t             w[6];
        w[0] = load_dword(buf, row0, p.dbase, rowbytes, ne0, l, ok);
        for (int i = 0; i < 4; ++i) {
            w[1 + i] = load_dword(buf, row0, p.qbase + 4u * i, rowbytes, ne0, l, ok);
        }
        w[5] = load_dword(buf, row0, p.tail, rowbytes, ne0, l, ok);
        if (!ok) {
            continue;
        }
        const int      b     = l >> 1;
        const int      h     = l & 1;
        const uint8_t * blk  = buf.data() + row0 + static_cast<size_t>(b) * shp::kQ8BlockBytes;
        const uint32_t dbits = static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8);
        if (shp::q8_half_dbits(w, p) != dbits) {
            fail("scale bits", ne0, l);
        }
        for (int i = 0; i < 4; ++i) {
            const uint32_t q = shp::q8_half_quads(w, p, i);
            for (int k = 0; k < 4; ++k) {
                const uint8_t want = blk[2 + 16 * h + 4 * i + k];
                if (static_cast<uint8_t>(q >> (8 * k)) != want) {
                    fail("quant byte", ne0, l);
                }
            }
        }
    }
}

// LDS-staged rows: the staging reads tile [0, rowbytes) exactly, and every
// quad's three LDS reads lie inside the row plus its padding and decode to
// the quad's scale and quants.
static void check_quads(int ne0, std::mt19937 & rng) {
    const uint32_t nq       = static_cast<uint32_t>(ne0) / 256u;
    const uint32_t rowdw    = shp::q8_row_dwords(nq);
    const uint32_t rowbytes = rowdw * 4u;
    if (rowbytes != static_cast<uint32_t>(ne0 / 32) * shp::kQ8BlockBytes) {
        fail("row size", ne0, -1);
        return;
    }
    std::vector<int> hits(rowdw, 0);
    for (int l = 0; l < 64; ++l) {
        for (uint32_t r = 0; r < nq / 4; ++r) {
            for (int i = 0; i < 4; ++i) {
                const uint32_t dw = 256u * r + 4u * static_cast<uint32_t>(l) + static_cast<uint32_t>(i);
                if (dw < rowdw) {
                    ++hits[dw];
                } else {
                    fail("staging read past the row", ne0, l);
                }
            }
        }
        if (static_cast<uint32_t>(l) < 4u * nq) {
            const uint32_t dw = 256u * (nq / 4) + static_cast<uint32_t>(l);
            if (dw < rowdw) {
                ++hits[dw];
            } else {
                fail("staging tail read past the row", ne0, l);
            }
        }
    }
    for (uint32_t dw = 0; dw < rowdw; ++dw) {
        if (hits[dw] != 1) {
            fail("staging does not tile the row", ne0, static_cast<int>(dw));
        }
    }
    std::vector<uint32_t> lds(rowdw + shp::kQ8StagePadDwords);
    for (auto & w : lds) {
        w = static_cast<uint32_t>(rng());
    }
    const uint8_t * row = reinterpret_cast<const uint8_t *>(lds.data());
    for (int l = 0; l < 64; ++l) {
        for (int k = 0; k < static_cast<int>(nq); ++k) {
            ++checked;
            const shp::Q8QuadPos p = shp::q8_quad_pos(k, l);
            if (p.adw + 1 >= rowdw + shp::kQ8StagePadDwords || p.ddw >= rowdw || (p.sh != 0 && p.adw + 1 >= rowdw)) {
                fail("quad read outside the buffer", ne0, l);
                continue;
            }
            const uint32_t q     = shp::bytes_at(lds[p.adw + 1], lds[p.adw], p.sh);
            const uint32_t dbits = (lds[p.ddw] >> p.dsh) & 0xffffu;
            const int      e     = 256 * k + 4 * l;
            const int      blk   = e / 32;
            const uint8_t * b    = row + static_cast<size_t>(blk) * shp::kQ8BlockBytes;
            if (dbits != (static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8))) {
                fail("quad scale bits", ne0, l);
            }
            for (int i = 0; i < 4; ++i) {
                if (static_cast<uint8_t>(q >> (8 * i)) != b[2 + e % 32 + i]) {
                    fail("quad quant byte", ne0, l);
                }
            }
        }
    }
}

// Five-dword windows of the gather->sum: every lane of every 1088-byte slab
// of the row reads [base, base + 20) inside its slab (hence the row); the
// even lane of each pair finds d at dsh in its own w[0], which the odd lane
// borrows; perm_bytes(w[i+1], w[i], sel) are the lane's 16 quants.
static void check_windows(int ne0, std::mt19937 & rng) {
    const uint32_t rowbytes = static_cast<uint32_t>(ne0 / 32) * shp::kQ8BlockBytes;
    std::vector<uint8_t> buf(rowbytes);
    for (auto & b : buf) {
        b = static_cast<uint8_t>(rng());
    }
    for (int s = 0; s < ne0 / static_cast<int>(shp::kQ8SlabElems); ++s) {
        const uint32_t slab0 = static_cast<uint32_t>(s) * shp::kQ8SlabBytes;
        uint32_t       w0_even = 0;
        for (int l = 0; l < 64; ++l) {
            ++checked;
            const shp::Q8WinPos p = shp::q8_win_pos(l);
            bool                ok = p.base + 20u <= shp::kQ8SlabBytes;
            uint32_t            w[5];
            for (int i = 0; i < 5 && ok; ++i) {
                w[i] = load_dword(buf, 0, slab0 + p.base + 4u * i, rowbytes, ne0, l, ok);
            }
            if (!ok) {
                fail("window outside the slab", ne0, l);
                continue;
            }
            if ((l & 1) == 0) {
                w0_even = w[0];
            }
            const int       b     = s * 32 + (l >> 1);
            const int       h     = l & 1;
            const uint8_t * blk   = buf.data() + static_cast<size_t>(b) * shp::kQ8BlockBytes;
            const uint32_t  dbits = static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8);
            if (((w0_even >> p.dsh) & 0xffffu) != dbits) {
                fail("window scale bits", ne0, l);
            }
            for (int i = 0; i < 4; ++i) {
                const uint32_t q = shp::perm_bytes(w[i + 1], w[i], p.sel);
                for (int k = 0; k < 4; ++k) {
                    if (static_cast<uint8_t>(q >> (8 * k)) != blk[2 + 16 * h + 4 * i + k]) {
                        fail("window quant byte", ne0, l);
                    }
                }
            }
        }
    }
}

// The row read for gather->sum slots past the last group: every block of its
// four slabs is d = -0.0 (f16 0x8000) and 32 zero quants.
static void check_neg_zero_row() {
    constexpr shp::Q8NegZeroRow r = shp::q8_neg_zero_row();
    const uint8_t *             b = reinterpret_cast<const uint8_t *>(r.w);
    for (uint32_t blk = 0; blk < 4 * shp::kQ8SlabElems / shp::kQ8BlockElems; ++blk) {
        ++checked;
        const uint8_t * p = b + blk * shp::kQ8BlockBytes;
        bool            ok = p[0] == 0x00 && p[1] == 0x80;
        for (int i = 2; i < 34; ++i) {
            ok = ok && p[i] == 0;
        }
        if (!ok) {
            fail("negative-zero row block", 4096, static_cast<int>(blk));
        }
    }
    if (sizeof(r.w) != 4 * shp::kQ8SlabBytes) {
        fail("negative-zero row size", 4096, -1);
    }
}

static void check_pairs(int ne0) {
    const uint32_t rowbytes = static_cast<uint32_t>(ne0 / 32) * shp::kQ8BlockBytes;
    for (int bp = 0; bp < ne0 / 64; ++bp) {
        ++checked;
        const uint32_t first = 68u * static_cast<uint32_t>(bp);
        if (first % 4 != 0 || first + 68 > rowbytes) {
            fail("pair read outside the row", ne0, bp);
        }
    }
}

int main() {
    std::mt19937 rng(20260728);
    for (int ne0 : { 256, 512, 1024, 2048, 4096 }) {
        for (int rep = 0; rep < 4; ++rep) {
            check_half(ne0, rng);
        }
    }
    for (int ne0 : { 1024, 2048, 4096 }) {
        for (int rep = 0; rep < 4; ++rep) {
            check_quads(ne0, rng);
            check_windows(ne0, rng);
        }
    }
    check_neg_zero_row();
    for (int ne0 : { 64, 128, 192, 320, 3072, 6144 }) {
        check_pairs(ne0);
    }
    std::printf("%ld %ld\n", checked, failures);
    return failures == 0 ? 0 : 1;
}

// Row gather with dequant (F32 / F16 / BF16 / Q8_0 -> F32) and the
// multi-codebook gather->sum, for gfx950.
//
// Every conversion is exact, so results are bit-identical to ggml-CPU:
// F16 -> F32 uses the hardware conversion, BF16 is a 16-bit shift, and a Q8_0
// element is the single product qs*fp16(d), which needs at most 19 significant
// bits and therefore never rounds. The gather->sum adds group rows in group
// order in f32, exactly as the unfused ggml_add chain does.
//
// Q8_0 layout: 32-element blocks of {f16 d; int8 qs[32]} = 34 bytes, so
// blocks are only 2-byte aligned. get_rows of 1024/2048/4096-wide rows in
// 16-byte aligned tables stages each row through LDS with aligned loads; other
// rows of 256..4096 elements are read by half-blocks (16 quants per lane, from
// a 4-byte aligned 5-dword window plus the scale's dword, shifted into place
// with v_alignbyte); other widths that are a multiple of 64 by block pairs (68
// bytes = 17 aligned dwords per lane). The gather->sum of 1024/2048/4096-wide
// rows reads one five-dword window per lane and group and decodes it in
// registers. (Geometry of every read: shp_q8.hpp.)

#include <atomic>

#include "shp_internal.hpp"
#include "shp_q5k.hpp"
#include "shp_q8.hpp"

namespace shp {
namespace {

// A 16-byte vector that only promises 4-byte alignment, so Q8_0 block pairs
// can be fetched with dwordx4 loads.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

struct GatherArgs {
    const char *    src;
    int64_t         snb1;
    int64_t         snb2;
    int64_t         snb3;
    int64_t         srows;
    const int32_t * ids;
    int64_t         inb0;
    int64_t         inb1;
    int64_t         inb2;
    float *         dst;
    int64_t         dnb1;
    int64_t         dnb2;
    int64_t         dnb3;
    int64_t         n;
    int64_t         ne11;
    int64_t         total;   // < 2^32
    int32_t         ne0;
    int32_t         staged;  // Q8_0 / Q5_K through LDS: ne0 in {1024, 2048, 4096}, rows 16-byte aligned
    // Output row R = r + n*(i11 + ne11*i12) by multiply-shift divisions, with
    // no branch on the batch form: an unbatched gather is n = total, ne11 = 1.
    FastDiv         fn;
    FastDiv         fne11;
};

constexpr int kMaxGroups = 64;

struct GatherSumArgs {
    const char *    tab[kMaxGroups];
    int64_t         tnb1[kMaxGroups];
    int64_t         trows[kMaxGroups];
    const int32_t * ids;
    int64_t         ids_gstride;  // bytes between consecutive groups' id runs
    float *         dst;
    int64_t         dnb1;
    int64_t         frames;
    int32_t         ngroups;
    int32_t         ne0;
    // A slot g past the last group (the kernels read whole chunks of slots)
    // reads row 0 of a -0.0 row (tab[g] = kQ8NegZeroRow, kQ5KNegZeroRow,
    // kNegZeroF32 or kNegZero16; tnb1[g] = rstride[g] = 0), which adds nothing to the sum,
    // and carries group 0's row count (group 0's id is read for it, so its
    // bounds check repeats group 0's).
    // Q8_0 and Q5_K window kernels only: every table has fewer than 2^31
    // bytes, so a row offset is 32-bit: row id * rstride[g].
    uint32_t        rows32[kMaxGroups];
    uint32_t        rstride[kMaxGroups];
};

__device__ __forceinline__ float sbyte(uint32_t w, int k) {
    return static_cast<float>(static_cast<int32_t>(w << (24 - 8 * k)) >> 24);
}

// Loads the 17 dwords of block pair `bp` of a Q8_0 row (row 4-byte aligned).
__device__ __forceinline__ void q8_load_pair(const char * row, int bp, uint32_t (&D)[17]) {
    const char * p = row + static_cast<int64_t>(bp) * 68;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const u32x4_a4 v = *reinterpret_cast<const u32x4_a4 *>(p + 16 * k);
        D[4 * k + 0]     = v.x;
        D[4 * k + 1]     = v.y;
        D[4 * k + 2]     = v.z;
        D[4 * k + 3]     = v.w;
    }
    D[16] = *reinterpret_cast<const uint32_t *>(p + 64);
}

// Decodes a loaded block pair into 64 floats, element j of output o[j].
__device__ __forceinline__ void q8_decode_pair(const uint32_t (&D)[17], float (&o)[64]) {
    const float d0 = f16_bits_to_f32(D[0] & 0xffffu);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const uint32_t w = __builtin_amdgcn_alignbyte(D[m + 1], D[m], 2);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o[4 * m + k] = sbyte(w, k) * d0;
        }
    }
    const float d1 = f16_bits_to_f32(D[8] >> 16);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const uint32_t w = D[9 + m];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o[32 + 4 * m + k] = sbyte(w, k) * d1;
        }
    }
}

__device__ __forceinline__ float q8_elem(const char * row, int e) {
    const char *   blk = row + static_cast<int64_t>(e / 32) * 34;
    const uint32_t dh  = static_cast<uint32_t>(reinterpret_cast<const uint8_t *>(blk)[0]) |
                        (static_cast<uint32_t>(reinterpret_cast<const uint8_t *>(blk)[1]) << 8);
    const int8_t q = reinterpret_cast<const int8_t *>(blk + 2)[e % 32];
    return static_cast<float>(q) * f16_bits_to_f32(dh);
}

// Q5_K, ggml's block_q5_K (layout and the scale/min packing in shp_q5k.hpp).
// The value is (d*sc)*q - dmin*m. d*sc and dmin*m have at most 17
// significant bits and (d*sc)*q at most 22, so every product is exact in f32
// and the subtraction is the one rounding -- as in ggml-CPU's
// dequantize_row_q5_K, whether or not its build fuses the multiply-add.
//
// In 32-bit words: w0 = d | dmin << 16, w1..w3 = scales[0..11].
struct Q5KCoef {
    float d1;  // d * sc
    float m1;  // dmin * m
};

__device__ __forceinline__ Q5KCoef q5k_coef(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, int s) {
    uint32_t sc, m;
    q5k_scale_min(w1, w2, w3, static_cast<uint32_t>(s), sc, m);
    return Q5KCoef{ f16_bits_to_f32(w0 & 0xffffu) * static_cast<float>(sc),
                    f16_bits_to_f32(w0 >> 16) * static_cast<float>(m) };
}

// The 5-bit quant of byte k of a lane's qs and qh words, sub-block s (h = s & 1).
__device__ __forceinline__ float q5k_quant(uint32_t qs, uint32_t qh, int k, int s) {
    const uint32_t nib = (qs >> (8 * k + 4 * (s & 1))) & 15u;
    const uint32_t hb  = (qh >> (8 * k + s)) & 1u;
    return static_cast<float>(nib | (hb << 4));
}

__device__ __forceinline__ float q5k_value(const Q5KCoef & c, float q) {
    return c.d1 * q - c.m1;
}

__device__ __forceinline__ uint32_t ld_u32(const char * p) {
    return static_cast<uint32_t>(reinterpret_cast<const uint8_t *>(p)[0]) |
           (static_cast<uint32_t>(reinterpret_cast<const uint8_t *>(p)[1]) << 8) |
           (static_cast<uint32_t>(reinterpret_cast<const uint8_t *>(p)[2]) << 16) |
           (static_cast<uint32_t>(reinterpret_cast<const uint8_t *>(p)[3]) << 24);
}

// One element of a Q5_K row at any alignment (the generic kernels).
__device__ __forceinline__ float q5k_elem(const char * row, int e) {
    const char * blk = row + static_cast<int64_t>(e / 256) * 176;
    const int    r   = e % 256;
    const int    j   = r / 64;
    const int    h   = (r / 32) & 1;
    const int    i   = r % 32;
    const int    s   = 2 * j + h;
    const Q5KCoef c  = q5k_coef(ld_u32(blk), ld_u32(blk + 4), ld_u32(blk + 8), ld_u32(blk + 12), s);
    const uint32_t qs = reinterpret_cast<const uint8_t *>(blk + 48)[32 * j + i];
    const uint32_t qh = reinterpret_cast<const uint8_t *>(blk + 16)[i];
    return q5k_value(c, q5k_quant(qs, qh, 0, s));
}

template <int TYPE> __device__ __forceinline__ float elem(const char * row, int e) {
    if constexpr (TYPE == SHP_TYPE_F32) {
        return reinterpret_cast<const float *>(row)[e];
    } else if constexpr (TYPE == SHP_TYPE_BF16) {
        return bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(row)[e]);
    } else if constexpr (TYPE == SHP_TYPE_F16) {
        return f16_bits_to_f32(reinterpret_cast<const uint16_t *>(row)[e]);
    } else if constexpr (TYPE == SHP_TYPE_Q5_K) {
        return q5k_elem(row, e);
    } else {
        return q8_elem(row, e);
    }
}

// The kernel arguments a gather wave needs before its first load. FLAT: the
// ids are one vector (ne11 = ne12 = 1), so output row R is lookup R and the
// batch coordinates, their divisions and strides are not needed.
template <bool FLAT = false> __device__ __forceinline__ void gather_args_in_sgprs(const GatherArgs & a) {
    if constexpr (FLAT) {
        args_in_sgprs(a.total, a.ids, a.inb0, a.src, a.snb1, a.srows, a.ne0, a.dst, a.dnb1);
    } else {
        args_in_sgprs(a.total, a.ids, a.inb0, a.inb1, a.inb2, a.fn.d, a.fn.m, a.fn.l, a.fne11.d, a.fne11.m, a.fne11.l,
                      a.src, a.snb1, a.snb2, a.snb3, a.srows, a.ne0);
    }
}

template <bool FLAT = false>
__device__ __forceinline__ void gather_coords(const GatherArgs & a, int64_t R, int32_t & id, const char *& srow,
                                              float *& drow) {
    if constexpr (FLAT) {
        id   = ld_const(reinterpret_cast<const int32_t *>(reinterpret_cast<const char *>(a.ids) + R * a.inb0));
        srow = a.src + static_cast<int64_t>(id) * a.snb1;
        drow = reinterpret_cast<float *>(reinterpret_cast<char *>(a.dst) + R * a.dnb1);
        return;
    }
    const uint32_t q   = fastdiv(static_cast<uint32_t>(R), a.fn);
    const uint32_t i12 = fastdiv(q, a.fne11);
    const int64_t  r   = R - static_cast<int64_t>(q) * a.fn.d;
    const int64_t  i11 = q - i12 * a.fne11.d;
    id   = ld_const(reinterpret_cast<const int32_t *>(reinterpret_cast<const char *>(a.ids) + r * a.inb0 + i11 * a.inb1 +
                                                  static_cast<int64_t>(i12) * a.inb2));
    srow = a.src + static_cast<int64_t>(id) * a.snb1 + i11 * a.snb2 + i12 * a.snb3;
    drow = reinterpret_cast<float *>(reinterpret_cast<char *>(a.dst) + r * a.dnb1 + i11 * a.dnb2 + i12 * a.dnb3);
}

constexpr uint32_t kQNaN = 0x7fc00000u;

// The row the Q8_0 gather->sum kernels read for slots past the last group
// (shp_q8.hpp: every block d = -0.0, zero quants). Only read; the host passes
// its address (hipGetSymbolAddress) in the slot's table pointer.
__device__ Q8NegZeroRow kQ8NegZeroRow = q8_neg_zero_row();

// The same for the Q5_K windows (shp_q5k.hpp: every super-block d = -0.0,
// dmin = +0.0, zero scales and quants).
__device__ __align__(16) Q5KNegZeroRow kQ5KNegZeroRow = q5k_neg_zero_row();

// The same for the F32 / F16 / BF16 gather->sum: rows of up to kSumVecMaxNe0
// elements that are all -0.0 (f32 0x80000000; f16 and bf16 0x8000 in each
// half of a dword).
constexpr int kSumVecMaxNe0 = 2048;

template <uint32_t W> struct NegZeroDwords {
    uint32_t w[kSumVecMaxNe0];
    constexpr NegZeroDwords() : w{} {
        for (int i = 0; i < kSumVecMaxNe0; ++i) {
            w[i] = W;
        }
    }
};

__device__ __align__(16) NegZeroDwords<0x80000000u> kNegZeroF32;
__device__ __align__(16) NegZeroDwords<0x80008000u> kNegZero16;

// A 4-element chunk of an F32 (16 bytes) or F16/BF16 (8 bytes) row, and its
// exact conversion to f32.
template <int TYPE> struct SumChunk {
    typedef uint2 type;  // four 16-bit values
};

template <> struct SumChunk<SHP_TYPE_F32> {
    typedef uint4 type;
};

template <int TYPE> __device__ __forceinline__ f32x4 cvt_sum_chunk(const typename SumChunk<TYPE>::type & v) {
    if constexpr (TYPE == SHP_TYPE_F32) {
        return f32x4{ __uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w) };
    } else if constexpr (TYPE == SHP_TYPE_BF16) {
        return f32x4{ bf16_bits_to_f32(v.x & 0xffffu), bf16_bits_to_f32(v.x >> 16), bf16_bits_to_f32(v.y & 0xffffu),
                      bf16_bits_to_f32(v.y >> 16) };
    } else {
        return f32x4{ f16_bits_to_f32(v.x & 0xffffu), f16_bits_to_f32(v.x >> 16), f16_bits_to_f32(v.y & 0xffffu),
                      f16_bits_to_f32(v.y >> 16) };
    }
}

// F32/F16/BF16 get_rows, LPR lanes per row (up to 256: a 2048-wide BF16 row
// is one block). Lane l owns the 4-element chunks l + LPR*j (j < CPL): one
// 16-byte (F32) or 8-byte (F16/BF16) load each and one float4 store each, so
// each load and store instruction of a wave covers one contiguous run. For
// LPR >= 64 the row is uniform over the wave, so the id is a scalar load and
// the row base scalar. The row loads are unconditional (a lane past the row
// re-reads chunk 0). Table rows use ordinary loads so that rows gathered again
// (repeated tokens, a table that fits the Infinity Cache) can hit; the f32
// output is streamed out with nontemporal stores.
template <int TYPE, int LPR, int CPL, bool FLAT>
__global__ __launch_bounds__(256) void k_get_rows_vec(const GatherArgs a) {
    gather_args_in_sgprs<FLAT>(a);
    typedef typename SumChunk<TYPE>::type Chunk;
    const int     l = threadIdx.x % LPR;
    const int64_t R = static_cast<int64_t>(blockIdx.x) * (256 / LPR) + row_in_block<LPR>();
    if (R >= a.total) {
        return;
    }
    int32_t      id;
    const char * srow;
    float *      drow;
    gather_coords<FLAT>(a, R, id, srow, drow);
    const bool    ok  = id >= 0 && id < a.srows;
    const int     n4  = a.ne0 / 4;
    const Chunk * row = reinterpret_cast<const Chunk *>(ok ? srow : a.src);
    Chunk         v[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = l + LPR * j;
        v[j]        = row[c < n4 ? c : 0];
    }
    f32x4 * out = reinterpret_cast<f32x4 *>(drow);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = l + LPR * j;
        if (c < n4) {
            st_stream(out + c, ok ? cvt_sum_chunk<TYPE>(v[j]) : splat4(__uint_as_float(kQNaN)));
        }
    }
}

// Q8_0, one block pair per lane, LPR lanes per row.
template <int LPR> __global__ __launch_bounds__(256) void k_get_rows_q8(const GatherArgs a) {
    gather_args_in_sgprs(a);
    const int     l = threadIdx.x % LPR;
    const int64_t R = static_cast<int64_t>(blockIdx.x) * (256 / LPR) + threadIdx.x / LPR;
    if (R >= a.total) {
        return;
    }
    int32_t      id;
    const char * srow;
    float *      drow;
    gather_coords(a, R, id, srow, drow);
    const int npairs = a.ne0 / 64;
    const bool bad   = id < 0 || id >= a.srows;
    for (int bp = l; bp < npairs; bp += LPR) {
        float o[64];
        if (bad) {
#pragma unroll
            for (int j = 0; j < 64; ++j) {
                o[j] = __uint_as_float(kQNaN);
            }
        } else {
            uint32_t D[17];
            q8_load_pair(srow, bp, D);
            q8_decode_pair(D, o);
        }
        float4 * out = reinterpret_cast<float4 *>(drow + bp * 64);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            out[k] = make_float4(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
        }
    }
}

__device__ __forceinline__ int32_t group_id(const GatherSumArgs & a, int g, int64_t f) {
    return *reinterpret_cast<const int32_t *>(reinterpret_cast<const char *>(a.ids) + g * a.ids_gstride + f * 4);
}

// ---------------------------------------------------------------------------
// Q8_0 by half-blocks: lane l of a row owns elements 16l..16l+15 (geometry in
// shp_q8.hpp). A 1024-wide row is one wave: its 64 lanes' reads tile the
// row's 1088 bytes.
// ---------------------------------------------------------------------------

struct Q8Half {
    uint32_t w[6];  // [0] the dword holding d, [1..4] the dwordx4, [5] the tail dword
};

// The lane's three reads; shp_q8.hpp states why each stays inside the row.
__device__ __forceinline__ Q8Half q8_half_load(const char * row, const Q8HalfPos & p) {
    Q8Half         h;
    const u32x4_a4 v = *reinterpret_cast<const u32x4_a4 *>(row + p.qbase);
    h.w[0]           = *reinterpret_cast<const uint32_t *>(row + p.dbase);
    h.w[1]           = v.x;
    h.w[2]           = v.y;
    h.w[3]           = v.z;
    h.w[4]           = v.w;
    h.w[5]           = *reinterpret_cast<const uint32_t *>(row + p.tail);
    return h;
}

// The 16 dequantised values q * fp16(d), each one exact product.
__device__ __forceinline__ void q8_half_decode(const Q8Half & h, const Q8HalfPos & p, float (&o)[16]) {
    const float d = f16_bits_to_f32(q8_half_dbits(h.w, p));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t q = q8_half_quads(h.w, p, i);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o[4 * i + k] = sbyte(q, k) * d;
        }
    }
}

__device__ __forceinline__ void store16(float * dst, const float (&o)[16]) {
    f32x4 * out = reinterpret_cast<f32x4 *>(dst);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        st_stream(out + k, f32x4{ o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3] });
    }
}

// Q8_0 get_rows: LPR = ne0/16 lanes per row.
template <int LPR> __global__ __launch_bounds__(256) void k_get_rows_q8h(const GatherArgs a) {
    gather_args_in_sgprs(a);
    const int64_t R = static_cast<int64_t>(blockIdx.x) * (256 / LPR) + row_in_block<LPR>();
    if (R >= a.total) {
        return;
    }
    const int l = static_cast<int>(threadIdx.x) % LPR;
    int32_t      id;
    const char * srow;
    float *      drow;
    gather_coords(a, R, id, srow, drow);
    float o[16];
    if (id < 0 || id >= a.srows) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            o[j] = __uint_as_float(kQNaN);
        }
    } else {
        const Q8HalfPos p = q8_half_pos(l);
        q8_half_decode(q8_half_load(srow, p), p, o);
    }
    store16(drow + 16 * l, o);
}

// Q8_0 gather->sum: LPR = ne0/16 lanes per frame. Groups are taken in chunks
// of 16 in three phases -- every id, then every row offset, then every row
// load (6 dwords per group per lane) -- so a chunk costs one id round trip and
// one row round trip, not one per group. The ids are vector loads (in-order
// vmcnt lets all 16 overlap). Per group the kernel keeps only the table base
// and a 32-bit row count in scalar registers; row offsets are 32-bit. Slots
// past the last group read kQ8NegZeroRow and add nothing. The sum is taken in
// group order from -0.0f, the identity of f32 addition (-0 + v == v bit for
// bit), so group 0 needs no special case.
constexpr int kSumChunk = 16;

template <bool FIRST>
__device__ __forceinline__ void q8_sum_chunk(const GatherSumArgs & a, int g0, int64_t f, const Q8HalfPos & p,
                                             float (&acc)[16], uint32_t & bad) {
    uint32_t id[kSumChunk];
#pragma unroll
    for (int j = 0; j < kSumChunk; ++j) {
        const int g = FIRST ? j : g0 + j;
        id[j]       = static_cast<uint32_t>(group_id(a, g < a.ngroups ? g : 0, f));
    }
    uint32_t off[kSumChunk];
#pragma unroll
    for (int j = 0; j < kSumChunk; ++j) {
        const int      g  = FIRST ? j : g0 + j;
        const uint32_t ok = id[j] < a.rows32[g] ? 1u : 0u;  // unsigned: a negative id is out of range too
        bad |= ok ^ 1u;
        off[j] = (ok ? id[j] : 0u) * a.rstride[g];
    }
    Q8Half h[kSumChunk];
#pragma unroll
    for (int j = 0; j < kSumChunk; ++j) {
        h[j] = q8_half_load(a.tab[FIRST ? j : g0 + j] + off[j], p);
    }
#pragma unroll
    for (int j = 0; j < kSumChunk; ++j) {
        float o[16];
        q8_half_decode(h[j], p, o);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            acc[k] = acc[k] + o[k];
        }
    }
}

template <int LPR> __global__ __launch_bounds__(256) void k_get_rows_sum_q8h(const GatherSumArgs a) {
    const int64_t f = static_cast<int64_t>(blockIdx.x) * (256 / LPR) + static_cast<int>(threadIdx.x) / LPR;
    if (f >= a.frames) {
        return;
    }
    const int       l = static_cast<int>(threadIdx.x) % LPR;
    const Q8HalfPos p = q8_half_pos(l);
    float           acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        acc[j] = -0.0f;
    }
    uint32_t bad = 0;
    q8_sum_chunk<true>(a, 0, f, p, acc, bad);
    for (int g0 = kSumChunk; g0 < a.ngroups; g0 += kSumChunk) {
        q8_sum_chunk<false>(a, g0, f, p, acc, bad);
    }
    if (bad != 0) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            acc[k] = __uint_as_float(kQNaN);
        }
    }
    store16(reinterpret_cast<float *>(reinterpret_cast<char *>(a.dst) + f * a.dnb1) + 16 * l, acc);
}

// Q8_0 gather->sum by five-dword windows (ne0 = 1024*NS, rows 4-byte aligned;
// geometry and its bounds in shp_q8.hpp). One wave per 1024-element slab of a
// frame; lane l owns elements 16l..16l+15 of the slab. A chunk of G groups
// costs two round trips: one vector load brings the G ids (lane j reads group
// j's) and readlane makes them scalar; then every group's window (a dword and
// a dwordx4 at a scalar row base plus the lane's offset) is requested before
// the first is decoded, and each is decoded in group order as it arrives. No
// LDS and no branches: a slot past the last group reads kQ8NegZeroRow, which
// adds exactly nothing. Each value enters the sum as fma(q, d, acc): q*d has
// at most 19 significant bits, so it is exact in f32 and the fused form rounds
// once, exactly as acc + q*d does -- one instruction less per element, and
// the decode is what bounds this kernel. The sum starts at -0.0f, the
// identity of f32 addition. FIRST: the chunk of groups 0..G-1, whose kernel
// argument slots are compile-time offsets. The kernel is built for at most 4
// waves per SIMD (128 VGPRs): a 4096-frame sum at ne0 = 1024 is 16 waves per
// CU, all resident at once, so the registers buy every window of a chunk in
// flight rather than occupancy the launch cannot use.
template <int G, bool FIRST>
__device__ __forceinline__ void q8w_chunk(const GatherSumArgs & a, int g0, int64_t f, uint32_t off, const Q8WinPos & p,
                                          float (&acc)[16], uint32_t & bad) {
    const int      l   = static_cast<int>(threadIdx.x) % kWave;
    const int      gl  = (FIRST ? 0 : g0) + l % G;
    const uint32_t ids = static_cast<uint32_t>(group_id(a, gl < a.ngroups ? gl : 0, f));
    uint32_t w[G][5];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const int      g    = (FIRST ? 0 : g0) + j;
        const uint32_t id   = __builtin_amdgcn_readlane(ids, j);
        const uint32_t ok   = id < a.rows32[g] ? 1u : 0u;  // unsigned: a negative id is out of range too
        bad |= ok ^ 1u;
        const char *   src  = a.tab[g] + (ok ? id : 0u) * a.rstride[g] + off;
        const u32x4_a4 v   = *reinterpret_cast<const u32x4_a4 *>(src + 4);
        w[j][0]            = *reinterpret_cast<const uint32_t *>(src);
        w[j][1]            = v.x;
        w[j][2]            = v.y;
        w[j][3]            = v.z;
        w[j][4]            = v.w;
    }
#pragma unroll
    for (int j = 0; j < G; ++j) {
        // quad_perm(0,0,2,2): both lanes of a pair take the even lane's w[0].
        const uint32_t dw =
            static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(w[j][0]), 0xA0, 0xF, 0xF, false));
        const float d = f16_bits_to_f32(dw >> p.dsh);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t q = perm_bytes(w[j][i + 1], w[j][i], p.sel);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                acc[4 * i + k] = __builtin_fmaf(sbyte(q, k), d, acc[4 * i + k]);
            }
        }
    }
}

template <int NS, int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_get_rows_sum_q8w(
    const GatherSumArgs a) {
    args_in_sgprs(a.frames, a.ids, a.ids_gstride, a.ngroups);
    __shared__ f32x4 s_out[4][kQ8SlabElems / 4];  // one slab per wave, for the store transpose
    const int     wi = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int64_t wv = static_cast<int64_t>(blockIdx.x) * 4 + wi;
    const int64_t f    = wv / NS;
    const int     slab = static_cast<int>(wv % NS);
    if (f >= a.frames) {
        return;
    }
    const int      l   = static_cast<int>(threadIdx.x) % kWave;
    const Q8WinPos p   = q8_win_pos(l);
    const uint32_t off = static_cast<uint32_t>(slab) * kQ8SlabBytes + p.base;
    float          acc[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        acc[k] = -0.0f;
    }
    uint32_t bad = 0;
    q8w_chunk<G, true>(a, 0, f, off, p, acc, bad);
    for (int g0 = G; g0 < a.ngroups; g0 += G) {
        q8w_chunk<G, false>(a, g0, f, off, p, acc, bad);
    }
    if (bad != 0) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            acc[k] = __uint_as_float(kQNaN);
        }
    }
    // The lane's 16 sums are contiguous; stored straight, each store
    // instruction would put 16 bytes into each of 64 different 64-byte
    // segments (four times the write requests of a contiguous store, ~15 %
    // of this kernel's time). A wave-private LDS transpose makes store k the
    // contiguous kilobyte 256k..256k+255 of the slab.
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        s_out[wi][4 * l + k] = f32x4{ acc[4 * k], acc[4 * k + 1], acc[4 * k + 2], acc[4 * k + 3] };
    }
    __syncwarp();
    f32x4 * out = reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(reinterpret_cast<char *>(a.dst) + f * a.dnb1) +
                                            kQ8SlabElems * slab);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        st_stream(out + 64 * k + l, s_out[wi][64 * k + l]);
    }
}

// ---------------------------------------------------------------------------
// Q8_0 through LDS (ne0 = 256*NQ with NQ = 4, 8, 16; rows 16-byte aligned;
// geometry and its bounds in shp_q8.hpp). One wave per output row: the row's
// bytes arrive with aligned dwordx4 loads, go through a wave-private LDS
// buffer, and each lane decodes the elements of its coalesced float4 stores
// (elements 256k + 4l..+3), so every load and every store of the wave is a
// contiguous, aligned run.
// ---------------------------------------------------------------------------

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int NQ> struct Q8Row {
    u32x4    v[NQ / 4];  // dwords 256r + 4l .. 256r + 4l + 3
    uint32_t x;          // dword 256*(NQ/4) + l, for lanes l < 4*NQ
};

template <int NQ> __device__ __forceinline__ Q8Row<NQ> q8_row_load(const char * row, int l) {
    Q8Row<NQ>     r;
    const u32x4 * v = reinterpret_cast<const u32x4 *>(row);
#pragma unroll
    for (int q = 0; q < NQ / 4; ++q) {
        r.v[q] = v[64 * q + l];
    }
    r.x = l < 4 * NQ ? reinterpret_cast<const uint32_t *>(row)[256 * (NQ / 4) + l] : 0u;
    return r;
}

template <int NQ> __device__ __forceinline__ void q8_row_stage(uint32_t * lds, const Q8Row<NQ> & r, int l) {
#pragma unroll
    for (int q = 0; q < NQ / 4; ++q) {
        reinterpret_cast<u32x4 *>(lds)[64 * q + l] = r.v[q];
    }
    if (l < 4 * NQ) {
        lds[256 * (NQ / 4) + l] = r.x;
    }
}

// Quad k of lane l: the four values q * fp16(d), each one exact product,
// stored as soon as it is decoded (a NaN quad when the id is out of range).
template <int NQ>
__device__ __forceinline__ void q8_row_decode_store(const uint32_t * lds, int l, bool ok, float * drow) {
    f32x4 * out = reinterpret_cast<f32x4 *>(drow);
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const Q8QuadPos p = q8_quad_pos(k, l);
        const uint32_t  q = bytes_at(lds[p.adw + 1], lds[p.adw], p.sh);
        const float     d = f16_bits_to_f32((lds[p.ddw] >> p.dsh) & 0xffffu);
        f32x4           o{ sbyte(q, 0) * d, sbyte(q, 1) * d, sbyte(q, 2) * d, sbyte(q, 3) * d };
        if (!ok) {
            o = splat4(__uint_as_float(kQNaN));
        }
        st_stream(out + 64 * k + l, o);
    }
}

// Rows (waves) per block of the LDS-staged get_rows: 4 measured 1-2 % faster
// than one-wave blocks at [1024,2048] x4096 (Q8_0 and Q5_K).
constexpr int kStagedWpb = 4;

// One wave per row. An id out of range reads row 0 of the table and stores
// NaN, with no branch between the id and the row loads; each quad is stored
// as soon as it is decoded. Measured on MI355X at [1024,2048] x4096 against
// the branch on the id with all 16 values stored at the end: 4.54 against
// 4.68 us.
template <int NQ, int WPB, bool FLAT>
__global__ __launch_bounds__(WPB * kWave) void k_get_rows_q8s(const GatherArgs a) {
    gather_args_in_sgprs<FLAT>(a);
    __shared__ uint32_t s_row[WPB][q8_row_dwords(NQ) + kQ8StagePadDwords];
    // The row is uniform over the wave: readfirstlane lets the id be one scalar
    // load and the table row base a scalar.
    const int           w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int           l = static_cast<int>(threadIdx.x) % kWave;
    const int64_t       R = static_cast<int64_t>(blockIdx.x) * WPB + w;
    if (R >= a.total) {
        return;  // no block barrier below: only this wave uses s_row[w]
    }
    int32_t      id;
    const char * srow;
    float *      drow;
    gather_coords<FLAT>(a, R, id, srow, drow);
    const bool      ok = (id >= 0) & (id < a.srows);
    const Q8Row<NQ> r  = q8_row_load<NQ>(ok ? srow : a.src, l);
    q8_row_stage<NQ>(s_row[w], r, l);
    __syncwarp();
    q8_row_decode_store<NQ>(s_row[w], l, ok, drow);
}

// ---------------------------------------------------------------------------
// Q5_K rows (ne0 = 256 * super-blocks, rows 4-byte aligned): lane l owns
// elements 4l..4l+3 of every super-block, so each float4 store instruction of
// the wave writes one super-block's contiguous kilobyte. Those four elements
// lie in sub-block s = l/8 (j = l/16, h = (l/8) & 1, i = 4(l%8)): their quant
// bytes are the aligned dword qs[32j + i ..] and their fifth bits the aligned
// dword qh[i ..], read with the super-block's first four dwords (d, dmin and
// the packed scales; the same for every lane).
// ---------------------------------------------------------------------------

constexpr int kQ5KChunk = 4;  // super-blocks whose loads go out before the first decode

struct Q5KLane {
    int qh_dw;  // dword of qh within the super-block
    int qs_dw;  // dword of qs within the super-block
    int s;      // sub-block
};

__device__ __forceinline__ Q5KLane q5k_lane(int l) {
    return Q5KLane{ 4 + (l % 8), 12 + 8 * (l / 16) + (l % 8), l / 8 };
}

struct Q5KWords {
    uint32_t w[4];  // d | dmin, scales
    uint32_t qh;
    uint32_t qs;
};

__device__ __forceinline__ Q5KWords q5k_load(const uint32_t * blk, const Q5KLane & p) {
    return Q5KWords{ { blk[0], blk[1], blk[2], blk[3] }, blk[p.qh_dw], blk[p.qs_dw] };
}

__device__ __forceinline__ f32x4 q5k_decode(const Q5KWords & v, const Q5KLane & p) {
    const Q5KCoef c = q5k_coef(v.w[0], v.w[1], v.w[2], v.w[3], p.s);
    return f32x4{ q5k_value(c, q5k_quant(v.qs, v.qh, 0, p.s)), q5k_value(c, q5k_quant(v.qs, v.qh, 1, p.s)),
                  q5k_value(c, q5k_quant(v.qs, v.qh, 2, p.s)), q5k_value(c, q5k_quant(v.qs, v.qh, 3, p.s)) };
}

// get_rows: one wave per output row.
__global__ __launch_bounds__(256) void k_get_rows_q5k(const GatherArgs a) {
    gather_args_in_sgprs(a);
    const int     l = static_cast<int>(threadIdx.x) % kWave;
    const int64_t R = static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    if (R >= a.total) {
        return;
    }
    int32_t      id;
    const char * srow;
    float *      drow;
    gather_coords(a, R, id, srow, drow);
    const bool     ok  = id >= 0 && id < a.srows;
    const int      nsb = a.ne0 / 256;
    const Q5KLane  p   = q5k_lane(l);
    f32x4 *        out = reinterpret_cast<f32x4 *>(drow);
    for (int b0 = 0; b0 < nsb; b0 += kQ5KChunk) {
        Q5KWords v[kQ5KChunk];
#pragma unroll
        for (int k = 0; k < kQ5KChunk; ++k) {
            const int b = b0 + k < nsb ? b0 + k : b0;  // past the row: re-read one inside it
            v[k]        = q5k_load(reinterpret_cast<const uint32_t *>((ok ? srow : a.src) + static_cast<int64_t>(b) * 176), p);
        }
#pragma unroll
        for (int k = 0; k < kQ5KChunk; ++k) {
            if (b0 + k < nsb) {
                st_stream(out + 64 * (b0 + k) + l, ok ? q5k_decode(v[k], p) : splat4(__uint_as_float(kQNaN)));
            }
        }
    }
}

// get_rows of 16-byte aligned rows of NSB = ne0/256 super-blocks (ne0 1024,
// 2048, 4096): the wave copies its row (11 aligned 16-byte words per
// super-block) into a wave-private LDS buffer with one dwordx4 per lane and
// round, then decodes each super-block's 4 elements per lane from LDS as
// above -- a few wide loads in front of the decode instead of six dword loads
// per super-block and lane. An id out of range reads row 0 and stores NaN.
template <int NSB, int WPB, bool FLAT>
__global__ __launch_bounds__(WPB * kWave) void k_get_rows_q5ks(const GatherArgs a) {
    gather_args_in_sgprs<FLAT>(a);
    constexpr int kWords  = 11 * NSB;  // 16-byte words per row
    constexpr int kRounds = (kWords + kWave - 1) / kWave;
    __shared__ u32x4 s_row[WPB][kWords];
    const int        w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int        l = static_cast<int>(threadIdx.x) % kWave;
    const int64_t    R = static_cast<int64_t>(blockIdx.x) * WPB + w;
    if (R >= a.total) {
        return;  // no block barrier below: only this wave uses s_row[w]
    }
    int32_t      id;
    const char * srow;
    float *      drow;
    gather_coords<FLAT>(a, R, id, srow, drow);
    const bool    ok  = (id >= 0) & (id < a.srows);
    const u32x4 * src = reinterpret_cast<const u32x4 *>(ok ? srow : a.src);
    u32x4         v[kRounds];
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
        const int i = kWave * r + l;
        if (i < kWords) {
            v[r] = src[i];
        }
    }
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
        const int i = kWave * r + l;
        if (i < kWords) {
            s_row[w][i] = v[r];
        }
    }
    __syncwarp();
    const uint32_t * lds = reinterpret_cast<const uint32_t *>(s_row[w]);
    const Q5KLane    p   = q5k_lane(l);
    f32x4 *          out = reinterpret_cast<f32x4 *>(drow);
#pragma unroll
    for (int b = 0; b < NSB; ++b) {
        f32x4 o = q5k_decode(q5k_load(lds + 44 * b, p), p);
        if (!ok) {
            o = splat4(__uint_as_float(kQNaN));
        }
        st_stream(out + 64 * b + l, o);
    }
}

// Any type / alignment: one wave per row, element by element.
template <int TYPE> __global__ __launch_bounds__(256) void k_get_rows_generic(const GatherArgs a) {
    const int     lane = threadIdx.x % kWave;
    const int64_t R    = static_cast<int64_t>(blockIdx.x) * (256 / kWave) + threadIdx.x / kWave;
    if (R >= a.total) {
        return;
    }
    int32_t      id;
    const char * srow;
    float *      drow;
    gather_coords(a, R, id, srow, drow);
    const bool bad = id < 0 || id >= a.srows;
    for (int e = lane; e < a.ne0; e += kWave) {
        drow[e] = bad ? __uint_as_float(kQNaN) : elem<TYPE>(srow, e);
    }
}

// ---------------------------------------------------------------------------
// gather -> ordered sum over groups
// ---------------------------------------------------------------------------

// F32/F16/BF16 gather->sum, one wave per frame. Lane l owns the 4-element
// chunks l + 64j (j < CPL) of the row: one 16-byte (F32) or 8-byte (F16/BF16)
// load each and one float4 store each, so every load and store instruction
// of the wave covers one contiguous run. A chunk of G groups costs two round
// trips: one vector load brings the G ids (lane j reads group j's; readlane
// makes them scalar), then every group's chunks are requested before the
// first is added. Group 0 is copied (ggml's acc = rows_0) and the others are
// added in group order. A slot past the last group reads a row of -0.0
// (kNegZeroF32 / kNegZero16, the host's pointer and a row stride of 0), and
// acc + -0.0 == acc for every f32 acc, so the slots cost no branch. (G = 1
// when there is one group, so its copy is never followed by such an add.)
template <int TYPE, int CPL, int G, bool FIRST>
__device__ __forceinline__ void vsum_chunk(const GatherSumArgs & a, int g0, int64_t f, int n4, f32x4 (&acc)[CPL],
                                           uint32_t & bad) {
    typedef typename SumChunk<TYPE>::type Chunk;
    const int     l   = static_cast<int>(threadIdx.x) % kWave;
    const int     gl  = (FIRST ? 0 : g0) + l % G;
    const int32_t ids = group_id(a, gl < a.ngroups ? gl : 0, f);
    Chunk         v[G][CPL];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const int     g  = (FIRST ? 0 : g0) + j;
        const int32_t id = __builtin_amdgcn_readlane(ids, j);
        const bool    ok = id >= 0 && id < a.trows[g];
        bad |= ok ? 0u : 1u;
        const Chunk * row = reinterpret_cast<const Chunk *>(a.tab[g] + static_cast<int64_t>(ok ? id : 0) * a.tnb1[g]);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int i = c * kWave + l;
            v[j][c]     = row[i < n4 ? i : 0];
        }
    }
#pragma unroll
    for (int j = 0; j < G; ++j) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const f32x4 o = cvt_sum_chunk<TYPE>(v[j][c]);
            if (FIRST && j == 0) {
                acc[c] = o;
            } else {
                acc[c] = f32x4{ acc[c].x + o.x, acc[c].y + o.y, acc[c].z + o.z, acc[c].w + o.w };
            }
        }
    }
}

template <int TYPE, int CPL, int G> __global__ __launch_bounds__(256) void k_get_rows_sum_vec(const GatherSumArgs a) {
    args_in_sgprs(a.frames, a.ids, a.ids_gstride, a.ngroups, a.ne0);
    const int64_t f =
        static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    if (f >= a.frames) {
        return;
    }
    const int l  = static_cast<int>(threadIdx.x) % kWave;
    const int n4 = a.ne0 / 4;
    f32x4     acc[CPL];
    uint32_t  bad = 0;
    vsum_chunk<TYPE, CPL, G, true>(a, 0, f, n4, acc, bad);
    for (int g0 = G; g0 < a.ngroups; g0 += G) {
        vsum_chunk<TYPE, CPL, G, false>(a, g0, f, n4, acc, bad);
    }
    f32x4 * drow = reinterpret_cast<f32x4 *>(reinterpret_cast<char *>(a.dst) + f * a.dnb1);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int i = c * kWave + l;
        if (i < n4) {
            drow[i] = bad != 0 ? splat4(__uint_as_float(kQNaN)) : acc[c];
        }
    }
}

// Group slots per chunk of the F32/F16/BF16 sum: about 64 VGPRs of loads in
// flight (CPL chunks of 4 or 2 dwords per group), at most 16.
template <int TYPE> constexpr int vsum_slots(int cpl) {
    const int words = cpl * (TYPE == SHP_TYPE_F32 ? 4 : 2);
    return 64 / words > 16 ? 16 : (64 / words < 1 ? 1 : 64 / words);
}

template <int TYPE, int CPL> void launch_vsum(const GatherSumArgs & a, hipStream_t stream) {
    constexpr int G = vsum_slots<TYPE>(CPL);
    const dim3    grid(static_cast<unsigned>((a.frames + 3) / 4));
    if (a.ngroups == 1) {
        hipLaunchKernelGGL((k_get_rows_sum_vec<TYPE, CPL, 1>), grid, dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL((k_get_rows_sum_vec<TYPE, CPL, G>), grid, dim3(256), 0, stream, a);
    }
}

// Any type / shape: one wave per frame, element by element, groups in order.
template <int TYPE> __global__ __launch_bounds__(256) void k_get_rows_sum_generic(const GatherSumArgs a) {
    const int     lane = threadIdx.x % kWave;
    const int64_t f    = static_cast<int64_t>(blockIdx.x) * (256 / kWave) + threadIdx.x / kWave;
    if (f >= a.frames) {
        return;
    }
    bool bad = false;
    for (int g = 0; g < a.ngroups; ++g) {
        const int32_t id = group_id(a, g, f);
        bad              = bad || id < 0 || id >= a.trows[g];
    }
    float * drow = reinterpret_cast<float *>(reinterpret_cast<char *>(a.dst) + f * a.dnb1);
    for (int e = lane; e < a.ne0; e += kWave) {
        float acc = 0.0f;
        for (int g = 0; g < a.ngroups && !bad; ++g) {
            const int32_t id = group_id(a, g, f);
            const float   v  = elem<TYPE>(a.tab[g] + static_cast<int64_t>(id) * a.tnb1[g], e);
            acc              = g == 0 ? v : acc + v;
        }
        drow[e] = bad ? __uint_as_float(kQNaN) : acc;
    }
}

int lanes_for(int64_t units) {
    return units >= 64 ? 64 : (units >= 32 ? 32 : 16);
}

template <int TYPE, bool FLAT> shp_status_t launch_get_rows_vec(const GatherArgs & a, hipStream_t stream);

// One vector of ids (a.total == a.n): the staged and vector kernels take the
// flat coordinates (measured on MI355X, Q8_0 [1024,2048] x4096: 4.65 -> 4.56
// us, the same bits).
template <int TYPE> shp_status_t launch_get_rows(const GatherArgs & a, bool vec, hipStream_t stream) {
    if (dry_run()) {
        return SHP_OK;
    }
    if (vec) {
        return a.total == a.n ? launch_get_rows_vec<TYPE, true>(a, stream) : launch_get_rows_vec<TYPE, false>(a, stream);
    }
    const int64_t blocks = (a.total + 3) / 4;
    hipLaunchKernelGGL(k_get_rows_generic<TYPE>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
    return launch_status();
}

template <int TYPE, bool FLAT> shp_status_t launch_get_rows_vec(const GatherArgs & a, hipStream_t stream) {
    if constexpr (TYPE == SHP_TYPE_Q5_K) {
        const dim3 grid(static_cast<unsigned>((a.total + kStagedWpb - 1) / kStagedWpb));
        const dim3 block(kStagedWpb * kWave);
        if (a.staged && a.ne0 == 1024) {
            hipLaunchKernelGGL((k_get_rows_q5ks<4, kStagedWpb, FLAT>), grid, block, 0, stream, a);
        } else if (a.staged && a.ne0 == 2048) {
            hipLaunchKernelGGL((k_get_rows_q5ks<8, kStagedWpb, FLAT>), grid, block, 0, stream, a);
        } else if (a.staged && a.ne0 == 4096) {
            hipLaunchKernelGGL((k_get_rows_q5ks<16, kStagedWpb, FLAT>), grid, block, 0, stream, a);
        } else {
            hipLaunchKernelGGL(k_get_rows_q5k, dim3(static_cast<unsigned>((a.total + 3) / 4)), dim3(256), 0, stream,
                               a);
        }
        return launch_status();
    } else if constexpr (TYPE == SHP_TYPE_Q8_0) {
        if (a.staged) {
            const dim3 grid(static_cast<unsigned>((a.total + kStagedWpb - 1) / kStagedWpb));
            const dim3 block(kStagedWpb * kWave);
            switch (a.ne0) {
                case 1024:
                    hipLaunchKernelGGL((k_get_rows_q8s<4, kStagedWpb, FLAT>), grid, block, 0, stream, a);
                    break;
                case 2048:
                    hipLaunchKernelGGL((k_get_rows_q8s<8, kStagedWpb, FLAT>), grid, block, 0, stream, a);
                    break;
                default:
                    hipLaunchKernelGGL((k_get_rows_q8s<16, kStagedWpb, FLAT>), grid, block, 0, stream, a);
                    break;
            }
            return launch_status();
        }
        const int nhalf = a.ne0 / 16;
        if (nhalf >= 16 && nhalf <= 256 && (nhalf & (nhalf - 1)) == 0) {
            const int64_t blocks = (a.total * nhalf + 255) / 256;
            switch (nhalf) {
                case 16:
                    hipLaunchKernelGGL(k_get_rows_q8h<16>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
                    break;
                case 32:
                    hipLaunchKernelGGL(k_get_rows_q8h<32>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
                    break;
                case 64:
                    hipLaunchKernelGGL(k_get_rows_q8h<64>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
                    break;
                case 128:
                    hipLaunchKernelGGL(k_get_rows_q8h<128>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
                    break;
                default:
                    hipLaunchKernelGGL(k_get_rows_q8h<256>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
                    break;
            }
            return launch_status();
        }
        const int lpr = lanes_for(a.ne0 / 64);
        const int64_t blocks = (a.total * lpr + 255) / 256;
        if (lpr == 64) {
            hipLaunchKernelGGL(k_get_rows_q8<64>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
        } else if (lpr == 32) {
            hipLaunchKernelGGL(k_get_rows_q8<32>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
        } else {
            hipLaunchKernelGGL(k_get_rows_q8<16>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
        }
    } else {
        // 4-element chunks: up to 256 lanes per row, 1..8 chunks per lane.
        const int64_t n4     = a.ne0 / 4;
        const int     lpr    = n4 >= 256 ? 256 : (n4 >= 128 ? 128 : lanes_for(n4));
        const dim3    grid(static_cast<unsigned>((a.total * lpr + 255) / 256));
        if (lpr == 256) {
            if (n4 <= 256) {
                hipLaunchKernelGGL((k_get_rows_vec<TYPE, 256, 1, FLAT>), grid, dim3(256), 0, stream, a);
            } else if (n4 <= 512) {
                hipLaunchKernelGGL((k_get_rows_vec<TYPE, 256, 2, FLAT>), grid, dim3(256), 0, stream, a);
            } else if (n4 <= 1024) {
                hipLaunchKernelGGL((k_get_rows_vec<TYPE, 256, 4, FLAT>), grid, dim3(256), 0, stream, a);
            } else {
                hipLaunchKernelGGL((k_get_rows_vec<TYPE, 256, 8, FLAT>), grid, dim3(256), 0, stream, a);
            }
        } else if (lpr == 128) {
            hipLaunchKernelGGL((k_get_rows_vec<TYPE, 128, 2, FLAT>), grid, dim3(256), 0, stream, a);
        } else if (lpr == 64) {
            hipLaunchKernelGGL((k_get_rows_vec<TYPE, 64, 2, FLAT>), grid, dim3(256), 0, stream, a);
        } else if (lpr == 32) {
            hipLaunchKernelGGL((k_get_rows_vec<TYPE, 32, 2, FLAT>), grid, dim3(256), 0, stream, a);
        } else {
            hipLaunchKernelGGL((k_get_rows_vec<TYPE, 16, 2, FLAT>), grid, dim3(256), 0, stream, a);
        }
    }
    return launch_status();
}

// Q8_0 widths the LDS-staged get_rows takes (one wave per row, NQ = ne0/256;
// the same widths for Q5_K) and the windowed gather->sum takes (ne0/1024
// waves per frame).
bool q8_staged_width(int64_t ne0) {
    return ne0 == 1024 || ne0 == 2048 || ne0 == 4096;
}

// The windowed Q8_0 gather->sum: NS waves per frame, G = 8 group slots when
// 8 groups or fewer are summed, else 16.
template <int NS> void launch_q8w(const GatherSumArgs & a, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((a.frames * NS + 3) / 4));
    if (a.ngroups <= 8) {
        hipLaunchKernelGGL((k_get_rows_sum_q8w<NS, 8>), grid, dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL((k_get_rows_sum_q8w<NS, 16>), grid, dim3(256), 0, stream, a);
    }
}

// Q5_K gather->sum, narrow rows (ne0 = 256 or 512): one wave per frame, lane
// l owning elements 4l..4l+3 of each of the row's super-blocks (as
// k_get_rows_q5k). Groups go in chunks: the chunk's ids, then every group's
// words for every super-block, are requested before the first decode; each
// decoded row is added to the sum in group order, from -0.0f (the identity of
// f32 addition), so the result is the node run's ((row_0 + row_1) + row_2) +
// ... bit for bit.
constexpr int kQ5KSumGroups = 4;

template <int NSB> __global__ __launch_bounds__(256) void k_get_rows_sum_q5k(const GatherSumArgs a) {
    args_in_sgprs(a.frames, a.ids, a.ids_gstride, a.ngroups);
    const int     l = static_cast<int>(threadIdx.x) % kWave;
    const int64_t f = static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    if (f >= a.frames) {
        return;
    }
    const Q5KLane p = q5k_lane(l);
    f32x4         acc[NSB];
#pragma unroll
    for (int b = 0; b < NSB; ++b) {
        acc[b] = splat4(-0.0f);
    }
    uint32_t bad = 0;
    for (int g0 = 0; g0 < a.ngroups; g0 += kQ5KSumGroups) {
        Q5KWords v[kQ5KSumGroups][NSB];
#pragma unroll
        for (int j = 0; j < kQ5KSumGroups; ++j) {
            const int      g  = g0 + j < a.ngroups ? g0 + j : g0;  // past the last group: re-read one inside
            const int32_t  id = *reinterpret_cast<const int32_t *>(reinterpret_cast<const char *>(a.ids) +
                                                                   g * a.ids_gstride + f * 4);
            const uint32_t ok = static_cast<uint32_t>(id) < static_cast<uint64_t>(a.trows[g]) ? 1u : 0u;
            bad |= (ok ^ 1u) & (g0 + j < a.ngroups ? 1u : 0u);
            const char * row = a.tab[g] + (ok ? static_cast<int64_t>(id) : 0) * a.tnb1[g];
#pragma unroll
            for (int b = 0; b < NSB; ++b) {
                v[j][b] = q5k_load(reinterpret_cast<const uint32_t *>(row + b * 176), p);
            }
        }
#pragma unroll
        for (int j = 0; j < kQ5KSumGroups; ++j) {
            if (g0 + j < a.ngroups) {
#pragma unroll
                for (int b = 0; b < NSB; ++b) {
                    const f32x4 y = q5k_decode(v[j][b], p);
                    acc[b]        = f32x4{ acc[b].x + y.x, acc[b].y + y.y, acc[b].z + y.z, acc[b].w + y.w };
                }
            }
        }
    }
    f32x4 * out = reinterpret_cast<f32x4 *>(reinterpret_cast<char *>(a.dst) + f * a.dnb1);
#pragma unroll
    for (int b = 0; b < NSB; ++b) {
        st_stream(out + 64 * b + l, bad != 0 ? splat4(__uint_as_float(kQNaN)) : acc[b]);
    }
}

// Q5_K gather->sum by 1024-element slabs (ne0 = 1024*NS, rows 4-byte aligned,
// every table under 2^31 bytes so a row offset is 32-bit; geometry and its
// bounds in shp_q5k.hpp). One wave per slab of a frame; lane l owns elements
// 16l..16l+15 of the slab, all in one sub-block. One vector load brings every
// group's id (lane g reads group g's; at most 64 groups), checked and clamped
// there for all groups at once, and readlane makes each scalar. The pieces
// are raw buffer loads: the table is a scalar resource, the row offset a
// scalar offset and the lane's place in the row a constant vector offset, so
// no address is computed per lane.
//
// Groups go in chunks of kQ5KWinGroups through two register buffers: chunk
// c + 1's loads are issued before chunk c is decoded, so every wave keeps a
// chunk in flight while it decodes. (All of a launch's waves start together;
// loading a chunk, then decoding it, keeps them in step -- the vector unit
// idle while they all wait, the memory idle while they all decode: 13 %
// slower at configs[2]'s shape.) The decode is about five vector
// instructions per element and group -- the quant assembly of shp_q5k.hpp, a
// byte conversion, the fma and the add, which the reference's two roundings
// keep apart. It is not what bounds the kernel: on MI355X at configs[2]'s
// shape, taking the decode out saves 15 % and taking two of the three loads
// per group out 5 %, and neither persistent waves that carry the pipeline
// across frames nor a sliding window of 4-8 groups in flight is faster: the
// rest is the rate at which scattered 704-byte rows are served.
// Slots past the last group read kQ5KNegZeroRow, which adds exactly nothing;
// the prefetch past the end of the loop reads it too (or group 63's rows,
// undecoded, when there are 64 groups).
//
// Each value is fma(d*sc, q, -(dmin*m)): the product is exact (at most 22
// significant bits), so the fused form rounds once, as the reference's
// y = d1*q - m1 does. The sum starts at -0.0f, the identity of f32 addition,
// and takes the groups in order, so it is the node run's
// ((row_0 + row_1) + row_2) + ... bit for bit. At most 4 waves per SIMD (128
// VGPRs), as for the Q8_0 windows: a 4096-frame sum at ne0 = 1024 is 16
// waves per CU, all resident at once.
constexpr int kQ5KWinGroups = 4;

// A raw buffer resource over a table: no stride, every offset below 2^31 in
// range (the window kernel's tables are under 2^31 bytes), dword data format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t table_rsrc(const char * base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(base), 0, 0x7fffffff, 0x00020000);
}

// One chunk's pieces per lane: the 16-byte header (d | dmin << 16, scales),
// four qh dwords, four qs dwords per group.
struct Q5KChunk {
    u32x4 hd[kQ5KWinGroups];
    u32x4 qh[kQ5KWinGroups];
    u32x4 qs[kQ5KWinGroups];
};

__device__ __forceinline__ void q5kw_load(const GatherSumArgs & a, int g0, uint32_t ids, uint32_t base,
                                          const Q5KWinPos & p, Q5KChunk & c) {
#pragma unroll
    for (int j = 0; j < kQ5KWinGroups; ++j) {
        const int                    g   = g0 + j < kMaxGroups ? g0 + j : kMaxGroups - 1;
        const __amdgpu_buffer_rsrc_t tab = table_rsrc(a.tab[g]);
        const int ro = static_cast<int>(__builtin_amdgcn_readlane(ids, g) * a.rstride[g] + base);
        c.hd[j] = __builtin_amdgcn_raw_buffer_load_b128(tab, static_cast<int>(p.hdr), ro, 0);
        c.qh[j] = __builtin_amdgcn_raw_buffer_load_b128(tab, static_cast<int>(p.qh), ro, 0);
        c.qs[j] = __builtin_amdgcn_raw_buffer_load_b128(tab, static_cast<int>(p.qs), ro, 0);
    }
}

__device__ __forceinline__ void q5kw_decode(const Q5KChunk & c, const Q5KWinPos & p, float (&acc)[16]) {
#pragma unroll
    for (int j = 0; j < kQ5KWinGroups; ++j) {
        const Q5KCoef k5 = q5k_coef(c.hd[j].x, c.hd[j].y, c.hd[j].z, c.hd[j].w, static_cast<int>(p.s));
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t q4 = q5k_quads(c.qs[j][t], c.qh[j][t], p.s);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float q  = static_cast<float>((q4 >> (8 * k)) & 0xffu);
                acc[4 * t + k] = acc[4 * t + k] + __builtin_fmaf(k5.d1, q, -k5.m1);
            }
        }
    }
}

template <int NS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_get_rows_sum_q5kw(
    const GatherSumArgs a) {
    args_in_sgprs(a.frames, a.ids, a.ids_gstride, a.ngroups);
    __shared__ f32x4 s_out[4][kQ5KSlabElems / 4];  // one slab per wave, for the store transpose
    const int     wi   = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int64_t wv   = static_cast<int64_t>(blockIdx.x) * 4 + wi;
    const int64_t f    = wv / NS;
    const int     slab = static_cast<int>(wv % NS);
    if (f >= a.frames) {
        return;
    }
    const int       l    = static_cast<int>(threadIdx.x) % kWave;
    const Q5KWinPos p    = q5k_win_pos(l);
    const uint32_t  base = static_cast<uint32_t>(slab) * kQ5KSlabBytes;
    // Group l's id, checked against group l's row count once for every group
    // (unsigned: a negative id is out of range too) and clamped to row 0 when
    // out of range. Lanes past the last group take group 0's id and row count,
    // as their slots do.
    const uint32_t  idv  = static_cast<uint32_t>(group_id(a, l < a.ngroups ? l : 0, f));
    const bool      okv  = idv < (&a.rows32[0])[l];
    const uint64_t  bad  = __builtin_amdgcn_ballot_w64(!okv);
    const uint32_t  ids  = okv ? idv : 0u;
    float           acc[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        acc[k] = -0.0f;
    }
    Q5KChunk ca, cb;
    q5kw_load(a, 0, ids, base, p, ca);
    for (int g0 = 0; g0 < a.ngroups; g0 += 2 * kQ5KWinGroups) {
        q5kw_load(a, g0 + kQ5KWinGroups, ids, base, p, cb);
        q5kw_decode(ca, p, acc);
        q5kw_load(a, g0 + 2 * kQ5KWinGroups, ids, base, p, ca);
        q5kw_decode(cb, p, acc);
    }
    if (bad != 0) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            acc[k] = __uint_as_float(kQNaN);
        }
    }
    // The wave-private LDS transpose of the Q8_0 windows: store k writes the
    // contiguous kilobyte 256k..256k+255 of the slab.
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        s_out[wi][4 * l + k] = f32x4{ acc[4 * k], acc[4 * k + 1], acc[4 * k + 2], acc[4 * k + 3] };
    }
    __syncwarp();
    f32x4 * out = reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(reinterpret_cast<char *>(a.dst) + f * a.dnb1) +
                                            kQ5KSlabElems * slab);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        st_stream(out + 64 * k + l, s_out[wi][64 * k + l]);
    }
}

template <int NS> void launch_q5kw(const GatherSumArgs & a, hipStream_t stream) {
    hipLaunchKernelGGL(k_get_rows_sum_q5kw<NS>, dim3(static_cast<unsigned>((a.frames * NS + 3) / 4)), dim3(256), 0,
                       stream, a);
}

template <int TYPE> shp_status_t launch_get_rows_sum(const GatherSumArgs & a, bool vec, hipStream_t stream) {
    if (vec) {
        if constexpr (TYPE == SHP_TYPE_Q5_K) {
            switch (a.ne0) {
                case 256:
                    hipLaunchKernelGGL(k_get_rows_sum_q5k<1>, dim3(static_cast<unsigned>((a.frames + 3) / 4)),
                                       dim3(256), 0, stream, a);
                    break;
                case 512:
                    hipLaunchKernelGGL(k_get_rows_sum_q5k<2>, dim3(static_cast<unsigned>((a.frames + 3) / 4)),
                                       dim3(256), 0, stream, a);
                    break;
                case 1024:
                    launch_q5kw<1>(a, stream);
                    break;
                case 2048:
                    launch_q5kw<2>(a, stream);
                    break;
                default:
                    launch_q5kw<4>(a, stream);
                    break;
            }
            return launch_status();
        } else if constexpr (TYPE == SHP_TYPE_Q8_0) {
            if (q8_staged_width(a.ne0)) {
                const int ns = a.ne0 / static_cast<int>(kQ8SlabElems);
                if (ns == 1) {
                    launch_q8w<1>(a, stream);
                } else if (ns == 2) {
                    launch_q8w<2>(a, stream);
                } else {
                    launch_q8w<4>(a, stream);
                }
                return launch_status();
            }
            const int nhalf = a.ne0 / 16;
            if (nhalf >= 16 && nhalf <= 256 && (nhalf & (nhalf - 1)) == 0) {
                const int64_t blocks = (a.frames * nhalf + 255) / 256;
                switch (nhalf) {
                    case 16:
                        hipLaunchKernelGGL(k_get_rows_sum_q8h<16>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
                        break;
                    case 32:
                        hipLaunchKernelGGL(k_get_rows_sum_q8h<32>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
                        break;
                    case 64:
                        hipLaunchKernelGGL(k_get_rows_sum_q8h<64>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
                        break;
                    case 128:
                        hipLaunchKernelGGL(k_get_rows_sum_q8h<128>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
                        break;
                    default:
                        hipLaunchKernelGGL(k_get_rows_sum_q8h<256>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
                        break;
                }
                return launch_status();
            }
            const int64_t blocks = (a.frames + 3) / 4;
            hipLaunchKernelGGL(k_get_rows_sum_generic<TYPE>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                               a);
        } else {
            const int cpl = (a.ne0 / 4 + kWave - 1) / kWave;
            if (cpl <= 1) {
                launch_vsum<TYPE, 1>(a, stream);
            } else if (cpl <= 2) {
                launch_vsum<TYPE, 2>(a, stream);
            } else if (cpl <= 4) {
                launch_vsum<TYPE, 4>(a, stream);
            } else {
                launch_vsum<TYPE, 8>(a, stream);
            }
        }
        return launch_status();
    }
    const int64_t blocks = (a.frames + 3) / 4;
    hipLaunchKernelGGL(k_get_rows_sum_generic<TYPE>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
    return launch_status();
}


bool gather_type_ok(int32_t t) {
    return t == SHP_TYPE_F32 || t == SHP_TYPE_F16 || t == SHP_TYPE_BF16 || t == SHP_TYPE_Q8_0 || t == SHP_TYPE_Q5_K;
}

// Q5_K widths of the vector gather->sum: super-blocks held per lane (256,
// 512), or 1024-element slabs over tables with 32-bit row offsets.
bool q5k_sum_width(int64_t ne0, bool dense32) {
    return ne0 == 256 || ne0 == 512 || (dense32 && (ne0 == 1024 || ne0 == 2048 || ne0 == 4096));
}

}  // namespace
}  // namespace shp

using namespace shp;

extern "C" shp_status_t shp_get_rows(const shp_tensor * src,
                                     const shp_tensor * ids,
                                     shp_tensor *       dst,
                                     shp_stream_t       stream) {
    if (!well_formed(src) || !well_formed(ids) || !well_formed(dst)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (!gather_type_ok(src->type) || dst->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    // ggml_get_rows: a [ne0, rows, ne2, ne3], b I32 [n, ne2, ne3] -> [ne0, n, ne2, ne3].
    if (ids->type != SHP_TYPE_I32 || ids->ne[3] != 1 || ids->ne[1] != src->ne[2] || ids->ne[2] != src->ne[3] ||
        dst->ne[0] != src->ne[0] || dst->ne[1] != ids->ne[0] || dst->ne[2] != ids->ne[1] ||
        dst->ne[3] != ids->ne[2] || src->ne[0] > INT32_MAX) {
        return SHP_ERR_INVALID_ARG;
    }
    if (!i32_aligned(*ids)) {
        return SHP_ERR_UNSUPPORTED;
    }
    GatherArgs a{};
    a.src   = static_cast<const char *>(src->data);
    a.snb1  = static_cast<int64_t>(src->nb[1]);
    a.snb2  = static_cast<int64_t>(src->nb[2]);
    a.snb3  = static_cast<int64_t>(src->nb[3]);
    a.srows = src->ne[1];
    a.ids   = static_cast<const int32_t *>(ids->data);
    a.inb0  = static_cast<int64_t>(ids->nb[0]);
    a.inb1  = static_cast<int64_t>(ids->nb[1]);
    a.inb2  = static_cast<int64_t>(ids->nb[2]);
    a.dst   = static_cast<float *>(dst->data);
    a.dnb1  = static_cast<int64_t>(dst->nb[1]);
    a.dnb2  = static_cast<int64_t>(dst->nb[2]);
    a.dnb3  = static_cast<int64_t>(dst->nb[3]);
    a.n     = ids->ne[0];
    a.ne11  = ids->ne[1];
    a.total = ids->ne[0] * ids->ne[1] * ids->ne[2];
    // Q8_0 and Q5_K rows through LDS: 1024/2048/4096 wide, 16-byte aligned
    a.staged  = (src->type == SHP_TYPE_Q8_0 || src->type == SHP_TYPE_Q5_K) && q8_staged_width(src->ne[0]) &&
               rows_aligned(*src, 16) && rows_aligned(*dst, 16);
    a.ne0   = static_cast<int32_t>(src->ne[0]);
    if (a.total > int64_t{ UINT32_MAX } / 256) {  // output rows (and their lanes) by 32-bit divisions
        return SHP_ERR_UNSUPPORTED;
    }
    a.fn    = make_fastdiv(static_cast<uint32_t>(a.n));
    a.fne11 = make_fastdiv(static_cast<uint32_t>(a.ne11));
    const bool dst16 = rows_aligned(*dst, 16);
    const hipStream_t st = as_stream(stream);
    switch (src->type) {
        case SHP_TYPE_F32:
            return launch_get_rows<SHP_TYPE_F32>(a, dst16 && rows_aligned(*src, 16) && src->ne[0] % 4 == 0 &&
                                                        src->ne[0] <= 8192, st);
        case SHP_TYPE_F16:
            return launch_get_rows<SHP_TYPE_F16>(a, dst16 && rows_aligned(*src, 16) && src->ne[0] % 4 == 0 &&
                                                        src->ne[0] <= 8192, st);
        case SHP_TYPE_BF16:
            return launch_get_rows<SHP_TYPE_BF16>(a, dst16 && rows_aligned(*src, 16) && src->ne[0] % 4 == 0 &&
                                                         src->ne[0] <= 8192, st);
        case SHP_TYPE_Q5_K:
            return launch_get_rows<SHP_TYPE_Q5_K>(a, dst16 && rows_aligned(*src, 4), st);
        default:
            return launch_get_rows<SHP_TYPE_Q8_0>(a, dst16 && rows_aligned(*src, 4) && src->ne[0] % 64 == 0, st);
    }
}

// The address of a -0.0 row (kQ8NegZeroRow, kQ5KNegZeroRow, kNegZeroF32 or
// kNegZero16, by table type) on the device that `stream` runs on (the current device for the
// null stream), where each device holds its own copy; looked up once per
// device and type, with that device made current for the lookup and the
// caller's device restored after it; null if HIP reports an error.
const char * neg_zero_row_address(int32_t type, hipStream_t stream) {
    constexpr int                    kMaxDevices = 64;
    static std::atomic<const char *> cache[kMaxDevices][4];
    const int k = type == SHP_TYPE_Q8_0 ? 0 : (type == SHP_TYPE_F32 ? 1 : (type == SHP_TYPE_Q5_K ? 3 : 2));
    int                              cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) {
        return nullptr;
    }
    hipDevice_t dev = cur;
    if (stream != nullptr && hipStreamGetDevice(stream, &dev) != hipSuccess) {
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        return nullptr;
    }
    const char * p = cache[dev][k].load(std::memory_order_acquire);
    if (p == nullptr) {
        if (dev != cur && hipSetDevice(dev) != hipSuccess) {
            return nullptr;
        }
        void *     q  = nullptr;
        hipError_t rc = k == 0   ? hipGetSymbolAddress(&q, HIP_SYMBOL(kQ8NegZeroRow))
                        : k == 1 ? hipGetSymbolAddress(&q, HIP_SYMBOL(kNegZeroF32))
                        : k == 2 ? hipGetSymbolAddress(&q, HIP_SYMBOL(kNegZero16))
                                 : hipGetSymbolAddress(&q, HIP_SYMBOL(kQ5KNegZeroRow));
        if (dev != cur && hipSetDevice(cur) != hipSuccess) {
            return nullptr;
        }
        if (rc != hipSuccess || q == nullptr) {
            return nullptr;
        }
        p = static_cast<const char *>(q);
        cache[dev][k].store(p, std::memory_order_release);
    }
    return p;
}

extern "C" shp_status_t shp_get_rows_sum(const shp_tensor * tables,
                                         int32_t            n_tables,
                                         const shp_tensor * ids,
                                         shp_tensor *       dst,
                                         shp_stream_t       stream) {
    if (tables == nullptr || n_tables < 1 || n_tables > kMaxGroups || !well_formed(ids) || !well_formed(dst)) {
        return SHP_ERR_INVALID_ARG;
    }
    const int32_t type = tables[0].type;
    if (!gather_type_ok(type) || dst->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    const int64_t ne0    = tables[0].ne[0];
    const int64_t frames = ids->ne[0];
    // codes [frames, groups], frames fastest and contiguous (code-predictor.cpp:86-92).
    if (ids->type != SHP_TYPE_I32 || ids->ne[1] != n_tables || ids->ne[2] != 1 || ids->ne[3] != 1 ||
        !contiguous(*ids) || dst->ne[0] != ne0 || dst->ne[1] != frames || dst->ne[2] != 1 || dst->ne[3] != 1 ||
        ne0 > INT32_MAX) {
        return SHP_ERR_INVALID_ARG;
    }
    if (!i32_aligned(*ids)) {
        return SHP_ERR_UNSUPPORTED;
    }
    GatherSumArgs a{};
    bool          vec = rows_aligned(*dst, 16);
    for (int g = 0; g < n_tables; ++g) {
        const shp_tensor & t = tables[g];
        if (!well_formed(&t) || t.ne[0] != ne0 || t.ne[2] != 1 || t.ne[3] != 1) {
            return SHP_ERR_INVALID_ARG;
        }
        if (t.type != type) {
            return SHP_ERR_UNSUPPORTED;
        }
        a.tab[g]   = static_cast<const char *>(t.data);
        a.tnb1[g]  = static_cast<int64_t>(t.nb[1]);
        a.trows[g] = t.ne[1];
        vec        = vec && rows_aligned(t, block_type(type) ? 4 : 16);
    }
    // Q8_0 and Q5_K window paths: one row size for every table, 32-bit offsets.
    bool dense32 = type == SHP_TYPE_Q8_0 || type == SHP_TYPE_Q5_K;
    for (int g = 0; g < n_tables && dense32; ++g) {
        const shp_tensor & t = tables[g];
        dense32 = t.nb[1] == row_bytes(type, ne0) && t.ne[1] <= INT32_MAX &&
                  static_cast<uint64_t>(t.ne[1]) * t.nb[1] < (uint64_t{ 1 } << 31);
    }
    // Four waves per block; the window paths take one wave per 1024-element slab.
    const int64_t waves_per_frame = block_type(type) && ne0 % 1024 == 0 ? ne0 / 1024 : 1;
    if (frames > int64_t{ INT32_MAX } * 4 / waves_per_frame) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (dry_run()) {
        return SHP_OK;
    }
    // Slots past the last group (the kernels read whole chunks of slots):
    // a -0.0 row with a row stride of 0, group 0's row count (group 0's id is
    // read for them).
    const char * zero = neg_zero_row_address(type, as_stream(stream));
    if (zero == nullptr) {
        return SHP_ERR_BACKEND;
    }
    for (int g = n_tables; g < kMaxGroups; ++g) {
        a.tab[g]   = zero;
        a.tnb1[g]  = 0;
        a.trows[g] = a.trows[0];
    }
    if (dense32) {
        for (int g = 0; g < kMaxGroups; ++g) {
            const bool live = g < n_tables;
            a.rows32[g]     = static_cast<uint32_t>(tables[live ? g : 0].ne[1]);
            a.rstride[g]    = live ? static_cast<uint32_t>(row_bytes(type, ne0)) : 0u;
        }
    }
    a.ids         = static_cast<const int32_t *>(ids->data);
    a.ids_gstride = static_cast<int64_t>(ids->nb[1]);
    a.dst         = static_cast<float *>(dst->data);
    a.dnb1        = static_cast<int64_t>(dst->nb[1]);
    a.frames      = frames;
    a.ngroups     = n_tables;
    a.ne0         = static_cast<int32_t>(ne0);
    const hipStream_t st = as_stream(stream);
    switch (type) {
        case SHP_TYPE_F32:
            return launch_get_rows_sum<SHP_TYPE_F32>(a, vec && ne0 % 4 == 0 && ne0 <= kSumVecMaxNe0, st);
        case SHP_TYPE_F16:
            return launch_get_rows_sum<SHP_TYPE_F16>(a, vec && ne0 % 4 == 0 && ne0 <= kSumVecMaxNe0, st);
        case SHP_TYPE_BF16:
            return launch_get_rows_sum<SHP_TYPE_BF16>(a, vec && ne0 % 4 == 0 && ne0 <= kSumVecMaxNe0, st);
        case SHP_TYPE_Q5_K:
            return launch_get_rows_sum<SHP_TYPE_Q5_K>(a, vec && q5k_sum_width(ne0, dense32), st);
        default:
            return launch_get_rows_sum<SHP_TYPE_Q8_0>(a, vec && dense32, st);
    }
}

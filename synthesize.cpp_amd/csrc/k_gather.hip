// Row gather with dequant (F32 / F16 / BF16 / Q8_0 -> F32) and the
// multi-codebook gather->sum, for gfx950.
//
// Every conversion is exact, so results are bit-identical to ggml-CPU:
// F16 -> F32 uses the hardware conversion, BF16 is a 16-bit shift, and a Q8_0
// element is the single product qs*fp16(d), which needs at most 19 significant
// bits and therefore never rounds. The gather->sum adds group rows in group
// order in f32, exactly as the unfused ggml_add chain does.
//
// Q8_0 layout: 32-element blocks of {f16 d; int8 qs[32]} = 34 bytes. Two
// consecutive blocks are 68 bytes = 17 dwords, and a row of ne0 % 64 == 0
// elements starts every block pair on a 4-byte boundary. A lane therefore owns
// one block pair: it loads 17 aligned dwords with wide loads, shifts block
// 2k's bytes into place with v_alignbyte (they sit 2 bytes off), and decodes
// 64 outputs in registers without any LDS traffic.

#include "shp_internal.hpp"

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
    int64_t         total;
    int32_t         ne0;
    int32_t         batched;
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
};

template <int TYPE> constexpr int elems_per_chunk() {
    return TYPE == SHP_TYPE_F32 ? 4 : 8;
}

// Converts one 16-byte chunk of a row into EPC floats.
template <int TYPE> __device__ __forceinline__ void cvt_chunk(uint4 v, float * o) {
    if constexpr (TYPE == SHP_TYPE_F32) {
        o[0] = __uint_as_float(v.x);
        o[1] = __uint_as_float(v.y);
        o[2] = __uint_as_float(v.z);
        o[3] = __uint_as_float(v.w);
    } else {
        const uint32_t w[4] = { v.x, v.y, v.z, v.w };
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if constexpr (TYPE == SHP_TYPE_BF16) {
                o[2 * k]     = bf16_bits_to_f32(w[k] & 0xffffu);
                o[2 * k + 1] = bf16_bits_to_f32(w[k] >> 16);
            } else {
                o[2 * k]     = f16_bits_to_f32(w[k] & 0xffffu);
                o[2 * k + 1] = f16_bits_to_f32(w[k] >> 16);
            }
        }
    }
}

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

template <int TYPE> __device__ __forceinline__ float elem(const char * row, int e) {
    if constexpr (TYPE == SHP_TYPE_F32) {
        return reinterpret_cast<const float *>(row)[e];
    } else if constexpr (TYPE == SHP_TYPE_BF16) {
        return bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(row)[e]);
    } else if constexpr (TYPE == SHP_TYPE_F16) {
        return f16_bits_to_f32(reinterpret_cast<const uint16_t *>(row)[e]);
    } else {
        return q8_elem(row, e);
    }
}

__device__ __forceinline__ void gather_coords(const GatherArgs & a, int64_t R, int32_t & id, const char *& srow,
                                              float *& drow) {
    int64_t r = R, i11 = 0, i12 = 0;
    if (a.batched) {  // ids [n, ne11, ne12]: 64-bit divisions only for the batched form
        r             = R % a.n;
        const int64_t q = R / a.n;
        i11           = q % a.ne11;
        i12           = q / a.ne11;
    }
    id   = *reinterpret_cast<const int32_t *>(reinterpret_cast<const char *>(a.ids) + r * a.inb0 + i11 * a.inb1 +
                                            i12 * a.inb2);
    srow = a.src + static_cast<int64_t>(id) * a.snb1 + i11 * a.snb2 + i12 * a.snb3;
    drow = reinterpret_cast<float *>(reinterpret_cast<char *>(a.dst) + r * a.dnb1 + i11 * a.dnb2 + i12 * a.dnb3);
}

constexpr uint32_t kQNaN = 0x7fc00000u;

// F32/F16/BF16, 16-byte chunks, LPR lanes per row (up to 256: a 2048-wide
// BF16 row is one block with one chunk per lane). The id is read first; the
// row chunk load depends on it; the f32 output is streamed out with
// nontemporal stores. Table rows use ordinary loads so that rows gathered
// again (repeated tokens, a table that fits the Infinity Cache) can hit.
template <int TYPE, int LPR> __global__ __launch_bounds__(256) void k_get_rows_vec(const GatherArgs a) {
    constexpr int EPC = elems_per_chunk<TYPE>();
    const int     l   = threadIdx.x % LPR;
    const int64_t R   = static_cast<int64_t>(blockIdx.x) * (256 / LPR) + threadIdx.x / LPR;
    if (R >= a.total) {
        return;
    }
    int32_t      id;
    const char * srow;
    float *      drow;
    gather_coords(a, R, id, srow, drow);
    const int nch = a.ne0 / EPC;
    f32x4 *   out = reinterpret_cast<f32x4 *>(drow);
    if (id < 0 || id >= a.srows) {
        const float nan = __uint_as_float(kQNaN);
        for (int e = l; e < a.ne0 / 4; e += LPR) {
            st_stream(out + e, splat4(nan));
        }
        return;
    }
    for (int c = l; c < nch; c += LPR) {
        const uint4 v = reinterpret_cast<const uint4 *>(srow)[c];
        float       o[EPC];
        cvt_chunk<TYPE>(v, o);
#pragma unroll
        for (int k = 0; k < EPC / 4; ++k) {
            st_stream(out + c * (EPC / 4) + k, f32x4{ o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3] });
        }
    }
}

// Q8_0, one block pair per lane, LPR lanes per row.
template <int LPR> __global__ __launch_bounds__(256) void k_get_rows_q8(const GatherArgs a) {
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

__device__ __forceinline__ int32_t group_id(const GatherSumArgs & a, int g, int64_t f) {
    return *reinterpret_cast<const int32_t *>(reinterpret_cast<const char *>(a.ids) + g * a.ids_gstride + f * 4);
}

// Q8_0 sum: lane owns one block pair of the frame's output row (LPR = ne0/64),
// accumulates 64 floats over the groups in order. Two groups' loads are issued
// before either is decoded.
template <int LPR> __global__ __launch_bounds__(256) void k_get_rows_sum_q8(const GatherSumArgs a) {
    const int     l = threadIdx.x % LPR;
    const int64_t f = static_cast<int64_t>(blockIdx.x) * (256 / LPR) + threadIdx.x / LPR;
    if (f >= a.frames) {
        return;
    }
    float acc[64];
    bool  bad = false;
    int   g   = 0;
    for (; g + 1 < a.ngroups; g += 2) {
        const int32_t id0 = group_id(a, g, f);
        const int32_t id1 = group_id(a, g + 1, f);
        const bool    ok0 = id0 >= 0 && id0 < a.trows[g];
        const bool    ok1 = id1 >= 0 && id1 < a.trows[g + 1];
        bad               = bad || !ok0 || !ok1;
        uint32_t D0[17], D1[17];
        q8_load_pair(a.tab[g] + static_cast<int64_t>(ok0 ? id0 : 0) * a.tnb1[g], l, D0);
        q8_load_pair(a.tab[g + 1] + static_cast<int64_t>(ok1 ? id1 : 0) * a.tnb1[g + 1], l, D1);
        float o[64];
        q8_decode_pair(D0, o);
        if (g == 0) {
#pragma unroll
            for (int j = 0; j < 64; ++j) {
                acc[j] = o[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 64; ++j) {
                acc[j] = acc[j] + o[j];
            }
        }
        q8_decode_pair(D1, o);
#pragma unroll
        for (int j = 0; j < 64; ++j) {
            acc[j] = acc[j] + o[j];
        }
    }
    if (g < a.ngroups) {
        const int32_t id = group_id(a, g, f);
        const bool    ok = id >= 0 && id < a.trows[g];
        bad              = bad || !ok;
        uint32_t D[17];
        q8_load_pair(a.tab[g] + static_cast<int64_t>(ok ? id : 0) * a.tnb1[g], l, D);
        float o[64];
        q8_decode_pair(D, o);
        if (g == 0) {
#pragma unroll
            for (int j = 0; j < 64; ++j) {
                acc[j] = o[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 64; ++j) {
                acc[j] = acc[j] + o[j];
            }
        }
    }
    if (bad) {
#pragma unroll
        for (int j = 0; j < 64; ++j) {
            acc[j] = __uint_as_float(kQNaN);
        }
    }
    float4 * out = reinterpret_cast<float4 *>(reinterpret_cast<char *>(a.dst) + f * a.dnb1) + l * 16;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        out[k] = make_float4(acc[4 * k], acc[4 * k + 1], acc[4 * k + 2], acc[4 * k + 3]);
    }
}

// F32/F16/BF16 sum: lane owns CPL 16-byte chunks of the frame's row.
template <int TYPE, int CPL> __global__ __launch_bounds__(256) void k_get_rows_sum_vec(const GatherSumArgs a) {
    constexpr int EPC = elems_per_chunk<TYPE>();
    const int     l   = threadIdx.x % kWave;
    const int64_t f   = static_cast<int64_t>(blockIdx.x) * (256 / kWave) + threadIdx.x / kWave;
    if (f >= a.frames) {
        return;
    }
    const int nch = a.ne0 / EPC;
    float     acc[CPL][EPC];
    bool      bad = false;
    for (int g = 0; g < a.ngroups; ++g) {
        const int32_t id = group_id(a, g, f);
        const bool    ok = id >= 0 && id < a.trows[g];
        bad              = bad || !ok;
        const char * row = a.tab[g] + static_cast<int64_t>(ok ? id : 0) * a.tnb1[g];
        uint4        v[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = j * kWave + l;
            if (c < nch) {
                v[j] = reinterpret_cast<const uint4 *>(row)[c];
            }
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            float o[EPC];
            cvt_chunk<TYPE>(v[j], o);
#pragma unroll
            for (int k = 0; k < EPC; ++k) {
                acc[j][k] = g == 0 ? o[k] : acc[j][k] + o[k];
            }
        }
    }
    float * drow = reinterpret_cast<float *>(reinterpret_cast<char *>(a.dst) + f * a.dnb1);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = j * kWave + l;
        if (c < nch) {
#pragma unroll
            for (int k = 0; k < EPC / 4; ++k) {
                float4 o = make_float4(acc[j][4 * k], acc[j][4 * k + 1], acc[j][4 * k + 2], acc[j][4 * k + 3]);
                if (bad) {
                    const float nan = __uint_as_float(kQNaN);
                    o               = make_float4(nan, nan, nan, nan);
                }
                reinterpret_cast<float4 *>(drow + c * EPC)[k] = o;
            }
        }
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

template <int TYPE> shp_status_t launch_get_rows(const GatherArgs & a, bool vec, hipStream_t stream) {
    if (vec) {
        if constexpr (TYPE == SHP_TYPE_Q8_0) {
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
            const int64_t nch    = a.ne0 / elems_per_chunk<TYPE>();
            const int     lpr    = nch >= 256 ? 256 : (nch >= 128 ? 128 : lanes_for(nch));
            const int64_t blocks = (a.total * lpr + 255) / 256;
            if (lpr == 256) {
                hipLaunchKernelGGL((k_get_rows_vec<TYPE, 256>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                                   stream, a);
            } else if (lpr == 128) {
                hipLaunchKernelGGL((k_get_rows_vec<TYPE, 128>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                                   stream, a);
            } else if (lpr == 64) {
                hipLaunchKernelGGL((k_get_rows_vec<TYPE, 64>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                                   stream, a);
            } else if (lpr == 32) {
                hipLaunchKernelGGL((k_get_rows_vec<TYPE, 32>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                                   stream, a);
            } else {
                hipLaunchKernelGGL((k_get_rows_vec<TYPE, 16>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                                   stream, a);
            }
        }
        return launch_status();
    }
    const int64_t blocks = (a.total + 3) / 4;
    hipLaunchKernelGGL(k_get_rows_generic<TYPE>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
    return launch_status();
}

template <int TYPE> shp_status_t launch_get_rows_sum(const GatherSumArgs & a, bool vec, hipStream_t stream) {
    if (vec) {
        if constexpr (TYPE == SHP_TYPE_Q8_0) {
            const int     lpr    = a.ne0 / 64;
            const int64_t blocks = (a.frames * lpr + 255) / 256;
            if (lpr == 64) {
                hipLaunchKernelGGL(k_get_rows_sum_q8<64>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                                   a);
            } else if (lpr == 32) {
                hipLaunchKernelGGL(k_get_rows_sum_q8<32>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                                   a);
            } else {
                hipLaunchKernelGGL(k_get_rows_sum_q8<16>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                                   a);
            }
        } else {
            const int     cpl    = (a.ne0 / elems_per_chunk<TYPE>() + kWave - 1) / kWave;
            const int64_t blocks = (a.frames + 3) / 4;
            if (cpl <= 1) {
                hipLaunchKernelGGL((k_get_rows_sum_vec<TYPE, 1>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                                   stream, a);
            } else if (cpl <= 2) {
                hipLaunchKernelGGL((k_get_rows_sum_vec<TYPE, 2>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                                   stream, a);
            } else {
                hipLaunchKernelGGL((k_get_rows_sum_vec<TYPE, 4>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                                   stream, a);
            }
        }
        return launch_status();
    }
    const int64_t blocks = (a.frames + 3) / 4;
    hipLaunchKernelGGL(k_get_rows_sum_generic<TYPE>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
    return launch_status();
}

bool gather_type_ok(int32_t t) {
    return t == SHP_TYPE_F32 || t == SHP_TYPE_F16 || t == SHP_TYPE_BF16 || t == SHP_TYPE_Q8_0;
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
    a.batched = ids->ne[1] > 1 || ids->ne[2] > 1;
    a.ne0   = static_cast<int32_t>(src->ne[0]);
    if ((a.total + 3) / 4 > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    const bool dst16 = rows_aligned(*dst, 16);
    const hipStream_t st = as_stream(stream);
    switch (src->type) {
        case SHP_TYPE_F32:
            return launch_get_rows<SHP_TYPE_F32>(a, dst16 && rows_aligned(*src, 16) && src->ne[0] % 4 == 0, st);
        case SHP_TYPE_F16:
            return launch_get_rows<SHP_TYPE_F16>(a, dst16 && rows_aligned(*src, 16) && src->ne[0] % 8 == 0, st);
        case SHP_TYPE_BF16:
            return launch_get_rows<SHP_TYPE_BF16>(a, dst16 && rows_aligned(*src, 16) && src->ne[0] % 8 == 0, st);
        default:
            return launch_get_rows<SHP_TYPE_Q8_0>(a, dst16 && rows_aligned(*src, 4) && src->ne[0] % 64 == 0, st);
    }
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
        vec        = vec && rows_aligned(t, type == SHP_TYPE_Q8_0 ? 4 : 16);
    }
    a.ids         = static_cast<const int32_t *>(ids->data);
    a.ids_gstride = static_cast<int64_t>(ids->nb[1]);
    a.dst         = static_cast<float *>(dst->data);
    a.dnb1        = static_cast<int64_t>(dst->nb[1]);
    a.frames      = frames;
    a.ngroups     = n_tables;
    a.ne0         = static_cast<int32_t>(ne0);
    if ((frames + 3) / 4 > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    const hipStream_t st = as_stream(stream);
    switch (type) {
        case SHP_TYPE_F32:
            return launch_get_rows_sum<SHP_TYPE_F32>(a, vec && ne0 % 4 == 0 && ne0 <= 4 * 4 * kWave, st);
        case SHP_TYPE_F16:
            return launch_get_rows_sum<SHP_TYPE_F16>(a, vec && ne0 % 8 == 0 && ne0 <= 8 * 4 * kWave, st);
        case SHP_TYPE_BF16:
            return launch_get_rows_sum<SHP_TYPE_BF16>(a, vec && ne0 % 8 == 0 && ne0 <= 8 * 4 * kWave, st);
        default:
            return launch_get_rows_sum<SHP_TYPE_Q8_0>(
                a, vec && (ne0 == 16 * 64 || ne0 == 32 * 64 || ne0 == 64 * 64), st);
    }
}

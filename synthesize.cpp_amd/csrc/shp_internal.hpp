// Internal helpers shared by the libsynth_hip translation units: ggml-style row
// addressing, exact element conversions, wave64 reductions and the host-side
// argument checks every entry point applies before it launches anything.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "synth_hip.h"

namespace shp {

constexpr int kWave = 64;

// A native 4 x f32 vector: what the nontemporal builtins and 128-bit global
// loads/stores operate on.
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Streaming accesses. Activations are read or written exactly once per
// launch, so they are fetched and stored with the nontemporal hint: the lines
// are not kept in L2 / the Infinity Cache at the expense of data that is
// reused (gains, Snake alpha, positions, gathered table rows).
__device__ __forceinline__ f32x4 ld_stream(const f32x4 * p) {
    return __builtin_nontemporal_load(p);
}

__device__ __forceinline__ void st_stream(f32x4 * p, f32x4 v) {
    __builtin_nontemporal_store(v, p);
}

__device__ __forceinline__ float ld_stream(const float * p) {
    return __builtin_nontemporal_load(p);
}

__device__ __forceinline__ void st_stream(float * p, float v) {
    __builtin_nontemporal_store(v, p);
}

// Global-memory pointers. A pointer rebuilt from integer arithmetic has lost
// its address space, and accesses through it become flat ones (which also
// count against the LDS counter); casting it back keeps them global.
// (The host pass sees plain pointers.)
#if defined(__HIP_DEVICE_COMPILE__)
template <class T> using gptr = T __attribute__((address_space(1))) *;

__device__ __forceinline__ f32x4 ld_stream(gptr<const f32x4> p) {
    return __builtin_nontemporal_load(p);
}

__device__ __forceinline__ void st_stream(gptr<f32x4> p, f32x4 v) {
    __builtin_nontemporal_store(v, p);
}
#else
template <class T> using gptr = T *;
#endif

template <class T> __device__ __forceinline__ gptr<T> to_global(T * p) {
    return (gptr<T>) p;
}

// A load of data that no kernel writes while this one runs (ids, positions)
// through the constant address space: when the address is uniform over the
// wave it becomes one scalar load (s_load) instead of a vector load plus a
// readfirstlane, which is the shorter round trip in front of a gather's row
// loads. A non-uniform address still compiles to a vector load.
template <class T> __device__ __forceinline__ T ld_const(const T * p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return *(const T __attribute__((address_space(4))) *) p;
#else
    return *p;
#endif
}

__device__ __forceinline__ f32x4 splat4(float v) {
    return f32x4{ v, v, v, v };
}

// Index of this lane's LPR-lane group (a row) within its block. For LPR >= 64
// every lane of a wave has the same row, which readfirstlane makes visible to
// the compiler, so row bases, ids and bounds become scalar values.
template <int LPR> __device__ __forceinline__ int row_in_block() {
    const int r = static_cast<int>(threadIdx.x) / LPR;
    if constexpr (LPR >= kWave) {
        return __builtin_amdgcn_readfirstlane(r);
    } else {
        return r;
    }
}

// Kernel arguments arrive by scalar loads from the kernel-argument segment,
// and the compiler issues them where they are first needed: a bound checked
// before the first data load puts a branch -- and a full scalar round trip --
// between that bound and the pointers. Listing the values a wave needs before
// its first data load here makes them all live in SGPRs at this point, so
// their loads go out together and cost one round trip. Emits no instruction.
// Measured on MI355X: SwiGLU [3072,512] 4.58 us against 4.80-4.86 us.
// The statement counts as a side effect, so a later load of kernel data (not
// arguments) is no longer known to read unwritten memory and is not made a
// scalar load: the rope kernels, whose wave 0 reads its position with one,
// do not use it.
template <class T> __device__ __forceinline__ void arg_in_sgpr(const T & v) {
    asm volatile("" ::"s"(v));
}

template <class... T> __device__ __forceinline__ void args_in_sgprs(const T &... v) {
    (arg_in_sgpr(v), ...);
}

// Unsigned 32-bit division by a launch constant d >= 1 without an integer
// divide: q = (umulhi(n, m) + n) >> l, with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1 (Granlund & Montgomery, "Division by
// invariant integers using multiplication", 1994, section 4).
struct FastDiv {
    uint32_t d;
    uint32_t m;
    uint32_t l;
    uint32_t pad;
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f{};
    f.d = d;
    uint32_t l = 0;
    while (l < 32 && (uint64_t{ 1 } << l) < d) {
        ++l;
    }
    f.l = l;
    f.m = static_cast<uint32_t>(((uint64_t{ 1 } << 32) * ((uint64_t{ 1 } << l) - d)) / d + 1);
    return f;
}

__host__ __device__ __forceinline__ uint32_t fastdiv(uint32_t n, const FastDiv & f) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint64_t t = __umulhi(n, f.m);
#else
    const uint64_t t = (static_cast<uint64_t>(n) * f.m) >> 32;
#endif
    return static_cast<uint32_t>((t + n) >> f.l);
}

__host__ __device__ __forceinline__ uint32_t fastmod(uint32_t n, const FastDiv & f) {
    return n - fastdiv(n, f) * f.d;
}

// Addresses row r of a ggml tensor whose rows are the flattened dims 1..3
// (r = i1 + ne1*(i2 + ne2*i3)). When the rows are evenly strided the offset is
// r*rs, with no division; otherwise it is decomposed per dimension.
struct RowMap {
    int64_t ne1;
    int64_t ne2;
    int64_t nb1;
    int64_t nb2;
    int64_t nb3;
    int64_t rs;
    int32_t flat;
    int32_t pad;
};

__device__ __forceinline__ int64_t row_offset(const RowMap & m, int64_t r) {
    if (m.flat) {
        return r * m.rs;
    }
    const int64_t i1 = r % m.ne1;
    const int64_t q  = r / m.ne1;
    const int64_t i2 = q % m.ne2;
    const int64_t i3 = q / m.ne2;
    return i1 * m.nb1 + i2 * m.nb2 + i3 * m.nb3;
}

// bf16 -> f32 is a 16-bit shift; f16 -> f32 is the exact hardware conversion.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// Weight element loaders: WT 1 = F32, 2 = BF16, 3 = F16.
enum WeightKind { kWNone = 0, kWF32 = 1, kWBF16 = 2, kWF16 = 3 };

template <int WT> __device__ __forceinline__ float load_w1(const void * w, int64_t i) {
    if constexpr (WT == kWF32) {
        return static_cast<const float *>(w)[i];
    } else if constexpr (WT == kWBF16) {
        return bf16_bits_to_f32(static_cast<const uint16_t *>(w)[i]);
    } else if constexpr (WT == kWF16) {
        return f16_bits_to_f32(static_cast<const uint16_t *>(w)[i]);
    } else {
        return 1.0f;
    }
}

// Four consecutive weights starting at element e (e % 4 == 0, base 8-byte aligned).
template <int WT> __device__ __forceinline__ float4 load_w4(const void * w, int64_t e) {
    if constexpr (WT == kWF32) {
        return reinterpret_cast<const float4 *>(static_cast<const float *>(w) + e)[0];
    } else {
        const uint2 h = reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(w) + e)[0];
        if constexpr (WT == kWBF16) {
            return make_float4(bf16_bits_to_f32(h.x & 0xffffu), bf16_bits_to_f32(h.x >> 16),
                               bf16_bits_to_f32(h.y & 0xffffu), bf16_bits_to_f32(h.y >> 16));
        } else {
            return make_float4(f16_bits_to_f32(h.x & 0xffffu), f16_bits_to_f32(h.x >> 16), f16_bits_to_f32(h.y & 0xffffu),
                               f16_bits_to_f32(h.y >> 16));
        }
    }
}

// Two consecutive weights at element e (e % 2 == 0).
template <int WT> __device__ __forceinline__ float2 load_w2(const void * w, int64_t e) {
    if constexpr (WT == kWF32) {
        return reinterpret_cast<const float2 *>(static_cast<const float *>(w) + e)[0];
    } else {
        const uint32_t h = reinterpret_cast<const uint32_t *>(static_cast<const uint16_t *>(w) + e)[0];
        if constexpr (WT == kWBF16) {
            return make_float2(bf16_bits_to_f32(h & 0xffffu), bf16_bits_to_f32(h >> 16));
        } else {
            return make_float2(f16_bits_to_f32(h & 0xffffu), f16_bits_to_f32(h >> 16));
        }
    }
}

// Cross-lane moves inside a row of 16 lanes (DPP), no LDS round trip. Each
// pattern pairs lanes symmetrically, so `v op move(v)` gives both lanes of a
// pair the same two operands in swapped order: with a commutative op every
// lane ends with bit-identical results.
constexpr int kDppQuadXor1   = 0xB1;   // quad_perm(1,0,3,2): lane ^ 1
constexpr int kDppQuadXor2   = 0x4E;   // quad_perm(2,3,0,1): lane ^ 2
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror: lane i of each 8 <-> lane 7-i
constexpr int kDppMirror     = 0x140;  // row_mirror: lane i of each 16 <-> lane 15-i

template <int CTRL> __device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

template <int CTRL> __device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    return __builtin_bit_cast(double, static_cast<uint64_t>(dpp_u32<CTRL>(static_cast<uint32_t>(u))) |
                                          (static_cast<uint64_t>(dpp_u32<CTRL>(static_cast<uint32_t>(u >> 32))) << 32));
}

template <int CTRL> __device__ __forceinline__ float dpp_f32(float v) {
    return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v)));
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
    const uint64_t u  = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u), lane));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), lane));
    return __builtin_bit_cast(double, static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32));
}

// Sum of a double over groups of W consecutive lanes (W a power of two <= 64),
// the same bits in every lane of a group. Every lane of a group must be
// active. Groups of 16 and more: four DPP steps give each 16-lane row its
// sum; rows then combine by one shuffle (W = 32) or, for the whole wave, by
// reading the four row sums into scalars (the result is then wave-uniform).
template <int W> __device__ __forceinline__ double group_sum(double v) {
    if constexpr (W < 16) {
#pragma unroll
        for (int off = W / 2; off > 0; off >>= 1) {
            v += __shfl_xor(v, off, W);
        }
        return v;
    } else {
        v += dpp_f64<kDppQuadXor1>(v);
        v += dpp_f64<kDppQuadXor2>(v);
        v += dpp_f64<kDppHalfMirror>(v);
        v += dpp_f64<kDppMirror>(v);
        if constexpr (W == 32) {
            v += __shfl_xor(v, 16, 32);
        } else if constexpr (W == 64) {
            v = (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
        }
        return v;
    }
}

// Maximum of a float over the wave, wave-uniform (same order-free scheme).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<kDppQuadXor1>(v));
    v = fmaxf(v, dpp_f32<kDppQuadXor2>(v));
    v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f32<kDppMirror>(v));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

inline size_t type_size(int32_t type) {
    switch (type) {
        case SHP_TYPE_F32:
        case SHP_TYPE_I32:
            return 4;
        case SHP_TYPE_F16:
        case SHP_TYPE_BF16:
            return 2;
        default:
            return 0;
    }
}

// ggml's block types: elements and bytes per block (Q8_0: {f16 d; int8
// qs[32]}; Q5_K: {f16 d, dmin; u8 scales[12], qh[32], qs[128]}).
constexpr int64_t kQ8Elems = 32, kQ5KElems = 256;
constexpr size_t  kQ8Bytes = 34, kQ5KBytes = 176;

inline bool block_type(int32_t type) {
    return type == SHP_TYPE_Q8_0 || type == SHP_TYPE_Q5_K;
}

inline int64_t block_elems(int32_t type) {
    return type == SHP_TYPE_Q8_0 ? kQ8Elems : kQ5KElems;
}

inline size_t block_bytes(int32_t type) {
    return type == SHP_TYPE_Q8_0 ? kQ8Bytes : kQ5KBytes;
}

// Bytes of one ne0-long row; block types hold ne0/elems blocks.
inline size_t row_bytes(int32_t type, int64_t ne0) {
    if (block_type(type)) {
        return static_cast<size_t>(ne0 / block_elems(type)) * block_bytes(type);
    }
    return static_cast<size_t>(ne0) * type_size(type);
}

inline int64_t nrows(const shp_tensor & t) {
    return t.ne[1] * t.ne[2] * t.ne[3];
}

inline int64_t nelements(const shp_tensor & t) {
    return t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
}

inline bool same_shape(const shp_tensor & a, const shp_tensor & b) {
    return a.ne[0] == b.ne[0] && a.ne[1] == b.ne[1] && a.ne[2] == b.ne[2] && a.ne[3] == b.ne[3];
}

// A descriptor is well formed when its type is known, extents are positive,
// rows are contiguous (nb[0] is the element size, or the block size for Q8_0)
// and data is non-null.
inline bool well_formed(const shp_tensor * t) {
    if (t == nullptr || t->data == nullptr || t->reserved != 0) {
        return false;
    }
    for (int d = 0; d < 4; ++d) {
        if (t->ne[d] <= 0) {
            return false;
        }
    }
    if (block_type(t->type)) {
        return t->ne[0] % block_elems(t->type) == 0 && t->nb[0] == block_bytes(t->type);
    }
    const size_t ts = type_size(t->type);
    return ts != 0 && t->nb[0] == ts;
}

// An F32 view whose rows are not contiguous but one of dims 1..3 is: what
// ggml_permute / ggml_transpose leave in front of a ggml_cont. Returns that
// dimension (1..3), or 0 when t is not such a view. Every stride is a
// multiple of 4 bytes and every extent positive.
inline int f32_strided_view_dim(const shp_tensor * t) {
    if (t == nullptr || t->data == nullptr || t->reserved != 0 || t->type != SHP_TYPE_F32 ||
        reinterpret_cast<uintptr_t>(t->data) % 4 != 0) {
        return 0;
    }
    for (int d = 0; d < 4; ++d) {
        if (t->ne[d] <= 0 || t->nb[d] % 4 != 0 || t->nb[d] == 0) {
            return 0;
        }
    }
    if (t->nb[0] == 4) {
        return 0;
    }
    for (int d = 1; d < 4; ++d) {
        if (t->nb[d] == 4 && t->ne[d] > 1) {
            return d;
        }
    }
    return 0;
}

// b = [ne0, 1, 1, 1]: one row, repeated over every row of a. A b of ne0
// elements in another shape is not this: ggml repeats [1, ne0] as one value
// per row, for instance.
inline bool one_row_of(const shp_tensor & b, int64_t ne0) {
    return b.ne[0] == ne0 && b.ne[1] == 1 && b.ne[2] == 1 && b.ne[3] == 1;
}

// ggml_can_repeat(b, a): each of b's extents divides a's, and ggml's binary
// ops read b at (i0 % b.ne0, i1 % b.ne1, i2 % b.ne2, i3 % b.ne3).
inline bool can_repeat(const shp_tensor & b, const shp_tensor & a) {
    for (int d = 0; d < 4; ++d) {
        if (b.ne[d] < 1 || a.ne[d] % b.ne[d] != 0) {
            return false;
        }
    }
    return true;
}

// [lo, hi) of the bytes a descriptor can address: from data to the end of its
// last element (its last row, for a block type).
inline void byte_span(const shp_tensor & t, uintptr_t & lo, uintptr_t & hi) {
    size_t end = block_type(t.type) ? row_bytes(t.type, t.ne[0]) :
                                      type_size(t.type) + static_cast<size_t>(t.ne[0] - 1) * t.nb[0];
    for (int d = 1; d < 4; ++d) {
        end += static_cast<size_t>(t.ne[d] - 1) * t.nb[d];
    }
    lo = reinterpret_cast<uintptr_t>(t.data);
    hi = lo + end;
}

inline bool spans_overlap(const shp_tensor & a, const shp_tensor & b) {
    uintptr_t alo, ahi, blo, bhi;
    byte_span(a, alo, ahi);
    byte_span(b, blo, bhi);
    return alo < bhi && blo < ahi;
}

inline RowMap make_rowmap(const shp_tensor & t) {
    RowMap m{};
    m.ne1  = t.ne[1];
    m.ne2  = t.ne[2];
    m.nb1  = static_cast<int64_t>(t.nb[1]);
    m.nb2  = static_cast<int64_t>(t.nb[2]);
    m.nb3  = static_cast<int64_t>(t.nb[3]);
    m.flat = 1;
    m.rs   = 0;
    int64_t expect = -1;
    for (int d = 1; d < 4; ++d) {
        if (t.ne[d] == 1) {
            continue;
        }
        const int64_t nb = static_cast<int64_t>(t.nb[d]);
        if (expect < 0) {
            m.rs   = nb;
            expect = nb * t.ne[d];
        } else if (nb == expect) {
            expect *= t.ne[d];
        } else {
            m.flat = 0;
        }
    }
    return m;
}

// True when every row start of `t` is `align`-byte aligned.
inline bool rows_aligned(const shp_tensor & t, size_t align) {
    if (reinterpret_cast<uintptr_t>(t.data) % align != 0) {
        return false;
    }
    for (int d = 1; d < 4; ++d) {
        if (t.ne[d] > 1 && t.nb[d] % align != 0) {
            return false;
        }
    }
    return true;
}

// Fully contiguous (ggml_is_contiguous) in the element-size sense.
// An I32 index tensor (ids, positions, a cache slot or status word): the
// kernels read such values with scalar loads where they are wave-uniform, and
// a scalar load ignores an address's two low bits, so data and strides must
// be multiples of 4 (ggml's allocators always give that).
inline bool i32_aligned(const shp_tensor & t) {
    return rows_aligned(t, 4);
}

inline bool contiguous(const shp_tensor & t) {
    size_t expect = t.nb[0] * static_cast<size_t>(t.ne[0]);
    if (block_type(t.type)) {
        expect = row_bytes(t.type, t.ne[0]);
    }
    for (int d = 1; d < 4; ++d) {
        if (t.ne[d] > 1 && t.nb[d] != expect) {
            return false;
        }
        expect *= static_cast<size_t>(t.ne[d]);
    }
    return true;
}

inline int weight_kind(int32_t type) {
    switch (type) {
        case SHP_TYPE_F32:
            return kWF32;
        case SHP_TYPE_BF16:
            return kWBF16;
        case SHP_TYPE_F16:
            return kWF16;
        default:
            return -1;
    }
}

// Argument checks without launching. While a DryRun lives on a thread, every
// entry point called on that thread runs all of its argument checks and
// returns their status, but enqueues nothing and makes no HIP call: each
// launcher returns SHP_OK where it would launch. The node-run executor answers
// supports_op, and vets each fused run it plans, through the entry points
// themselves this way, so what it accepts is exactly what they accept.
inline bool & dry_run_flag() {
    static thread_local bool flag = false;
    return flag;
}

inline bool dry_run() {
    return dry_run_flag();
}

struct DryRun {
    bool prev;
    DryRun() : prev(dry_run_flag()) { dry_run_flag() = true; }
    ~DryRun() { dry_run_flag() = prev; }
    DryRun(const DryRun &)             = delete;
    DryRun & operator=(const DryRun &) = delete;
};

inline hipStream_t as_stream(shp_stream_t s) {
    return static_cast<hipStream_t>(s);
}

inline shp_status_t launch_status() {
    return hipGetLastError() == hipSuccess ? SHP_OK : SHP_ERR_BACKEND;
}

}  // namespace shp

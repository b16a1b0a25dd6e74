// RMSNorm x weight (optionally fed by a residual add), per-head QK-norm fused
// with NEOX rope, and bare NEOX rope, for gfx950.
//
// Arithmetic follows ggml-CPU exactly in operation order: squares are rounded
// in f32 and summed in double, the mean is rounded to f32, the scale is
// 1.0f/sqrtf(mean+eps) with correctly rounded divide and sqrt, and the result
// is (x*scale)*w in two f32 multiplies. Rope replays the f32 theta recurrence
// of the CPU cache. This file is compiled with -ffp-contract=off so nothing is
// fused into an FMA behind the formulas' back.
//
// Layout: a row (ne0 contiguous floats) is owned by a group of TPR lanes; each
// lane holds VPL float4 of it in registers between the reduction and the
// scaled store, so x is read from HBM once. Activations are streamed with
// nontemporal loads and stores; gains stay cacheable (every row reads them).

#include <cmath>

#include "shp_internal.hpp"
#include "shp_trig.hpp"

namespace shp {
namespace {

struct NormArgs {
    const float * x;
    RowMap        xm;
    const float * b;
    RowMap        bm;
    float *       s;
    RowMap        sm;
    float *       y;
    RowMap        ym;
    const void *  w;
    int64_t       nrows;
    int32_t       ne0;
    float         eps;
};

enum NormMode { kPlain = 0, kAdd = 1, kAddSum = 2 };

__device__ __forceinline__ float norm_scale(double sum, int32_t ne0, float eps) {
    const float mean = static_cast<float>(sum / static_cast<double>(ne0));
    return 1.0f / __builtin_sqrtf(mean + eps);
}

__device__ __forceinline__ f32x4 add4v(f32x4 a, f32x4 b) {
    return f32x4{ a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w };
}

// Each square is an f32 product; the accumulation is double, in element order.
__device__ __forceinline__ double sq4v(f32x4 v) {
    double acc = static_cast<double>(v.x * v.x);
    acc += static_cast<double>(v.y * v.y);
    acc += static_cast<double>(v.z * v.z);
    acc += static_cast<double>(v.w * v.w);
    return acc;
}

template <int WT> __device__ __forceinline__ f32x4 load_w4v(const void * w, int64_t e) {
    const float4 v = load_w4<WT>(w, e);
    return f32x4{ v.x, v.y, v.z, v.w };
}

// Four gains at element e as loaded (f32, or 16-bit patterns), converted later.
template <int WT> struct WRaw {
    uint32_t v[WT == kWF32 ? 4 : 2];
};

template <int WT> __device__ __forceinline__ WRaw<WT> load_wraw(const void * w, int64_t e) {
    WRaw<WT> r;
    if constexpr (WT == kWF32) {
        const uint4 u = *to_global(reinterpret_cast<const uint4 *>(static_cast<const float *>(w) + e));
        r.v[0] = u.x;
        r.v[1] = u.y;
        r.v[2] = u.z;
        r.v[3] = u.w;
    } else if constexpr (WT != kWNone) {
        const uint2 u = *to_global(reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(w) + e));
        r.v[0] = u.x;
        r.v[1] = u.y;
    }
    return r;
}

template <int WT> __device__ __forceinline__ f32x4 cvt_wraw(const WRaw<WT> & r) {
    if constexpr (WT == kWF32) {
        return f32x4{ __uint_as_float(r.v[0]), __uint_as_float(r.v[1]), __uint_as_float(r.v[2]), __uint_as_float(r.v[3]) };
    } else if constexpr (WT == kWBF16) {
        return f32x4{ bf16_bits_to_f32(r.v[0] & 0xffffu), bf16_bits_to_f32(r.v[0] >> 16), bf16_bits_to_f32(r.v[1] & 0xffffu),
                      bf16_bits_to_f32(r.v[1] >> 16) };
    } else if constexpr (WT == kWF16) {
        return f32x4{ f16_bits_to_f32(r.v[0] & 0xffffu), f16_bits_to_f32(r.v[0] >> 16), f16_bits_to_f32(r.v[1] & 0xffffu),
                      f16_bits_to_f32(r.v[1] >> 16) };
    } else {
        return splat4(1.0f);
    }
}

// Vector path (ne0 % 4 == 0, 16-byte aligned rows, ne0 <= 256*4*VPL).
//
// A row is spread over TPR lanes (16..256) so that each lane streams at most
// VPL float4 of it: a 1024-wide row is one 256-lane block with one float4 per
// lane, which keeps the most waves -- and so the most loads -- in flight per
// CU. Every load (x, the residual b, the gains) is issued before anything
// waits. The double sum of squares is reduced across the TPR lanes with
// shuffles, and across waves (TPR > 64) through LDS in a fixed order. Lanes
// past the end of the row or of the tensor still take part in the barrier.
template <int TPR, int VPL, int WT, int MODE, int BLOCK = 256>
__global__ __launch_bounds__(BLOCK) void k_rms_norm_vec(const NormArgs a) {
    constexpr int kRowsPerBlock = BLOCK / TPR;
    constexpr int kWavesPerRow  = TPR > kWave ? TPR / kWave : 1;
    __shared__ double s_part[TPR > kWave ? BLOCK / kWave : 1];

    args_in_sgprs(a.x, a.xm.flat, a.xm.rs, a.w, a.nrows, a.ne0, a.y, a.ym.flat, a.ym.rs);
    if constexpr (MODE != kPlain) {
        args_in_sgprs(a.b, a.bm.flat, a.bm.rs);
    }
    if constexpr (MODE == kAddSum) {
        args_in_sgprs(a.s, a.sm.flat, a.sm.rs);
    }
    const int     l     = threadIdx.x % TPR;
    const int64_t row   = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + row_in_block<TPR>();
    const bool    live  = row < a.nrows;
    const int     nvec  = a.ne0 / 4;
    const int64_t rrow  = live ? row : 0;
    const f32x4 * xp    = reinterpret_cast<const f32x4 *>(reinterpret_cast<const char *>(a.x) + row_offset(a.xm, rrow));
    f32x4         v[VPL];
    f32x4         bv[VPL];
    f32x4         wv[VPL];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int c = k * TPR + l;
        v[k]        = (live && c < nvec) ? ld_stream(xp + c) : splat4(0.0f);
    }
    if constexpr (MODE != kPlain) {
        const f32x4 * bp =
            reinterpret_cast<const f32x4 *>(reinterpret_cast<const char *>(a.b) + row_offset(a.bm, rrow));
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            const int c = k * TPR + l;
            bv[k]       = (live && c < nvec) ? ld_stream(bp + c) : splat4(0.0f);
        }
    }
    if constexpr (WT != kWNone) {
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            const int c = k * TPR + l;
            wv[k]       = c < nvec ? load_w4v<WT>(a.w, static_cast<int64_t>(c) * 4) : splat4(0.0f);
        }
    }
    if constexpr (MODE != kPlain) {
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            v[k] = add4v(v[k], bv[k]);
        }
        if constexpr (MODE == kAddSum) {
            f32x4 * sp = reinterpret_cast<f32x4 *>(reinterpret_cast<char *>(a.s) + row_offset(a.sm, rrow));
#pragma unroll
            for (int k = 0; k < VPL; ++k) {
                const int c = k * TPR + l;
                if (live && c < nvec) {
                    st_stream(sp + c, v[k]);
                }
            }
        }
    }
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        acc += sq4v(v[k]);
    }
    if constexpr (TPR <= kWave) {
        acc = group_sum<TPR>(acc);
    } else {
        acc             = group_sum<kWave>(acc);
        const int wave  = threadIdx.x / kWave;
        if (threadIdx.x % kWave == 0) {
            s_part[wave] = acc;
        }
        __syncthreads();
        const int first = (threadIdx.x / TPR) * kWavesPerRow;
        acc             = s_part[first];
#pragma unroll
        for (int k = 1; k < kWavesPerRow; ++k) {
            acc += s_part[first + k];
        }
    }
    if (!live) {
        return;
    }
    const float scale = norm_scale(acc, a.ne0, a.eps);
    f32x4 *     yp    = reinterpret_cast<f32x4 *>(reinterpret_cast<char *>(a.y) + row_offset(a.ym, row));
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int c = k * TPR + l;
        if (c < nvec) {
            f32x4 o = f32x4{ v[k].x * scale, v[k].y * scale, v[k].z * scale, v[k].w * scale };
            if constexpr (WT != kWNone) {
                o = f32x4{ o.x * wv[k].x, o.y * wv[k].y, o.z * wv[k].z, o.w * wv[k].w };
            }
            st_stream(yp + c, o);
        }
    }
}

// Any ne0 and alignment: one wave per row, two passes (the second re-reads the
// row, which is still in L1/L2).
template <int WT, int MODE> __global__ __launch_bounds__(256) void k_rms_norm_generic(const NormArgs a) {
    const int     lane = threadIdx.x % kWave;
    const int64_t row  = static_cast<int64_t>(blockIdx.x) * (256 / kWave) + threadIdx.x / kWave;
    if (row >= a.nrows) {
        return;
    }
    const float * xr = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.x) + row_offset(a.xm, row));
    const float * br = nullptr;
    float *       sr = nullptr;
    if constexpr (MODE != kPlain) {
        br = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.b) + row_offset(a.bm, row));
    }
    if constexpr (MODE == kAddSum) {
        sr = reinterpret_cast<float *>(reinterpret_cast<char *>(a.s) + row_offset(a.sm, row));
    }
    double acc = 0.0;
    for (int i = lane; i < a.ne0; i += kWave) {
        float v = xr[i];
        if constexpr (MODE != kPlain) {
            v = v + br[i];
        }
        if constexpr (MODE == kAddSum) {
            sr[i] = v;
        }
        acc += static_cast<double>(v * v);
    }
    acc               = group_sum<kWave>(acc);
    const float scale = norm_scale(acc, a.ne0, a.eps);
    float *     yr    = reinterpret_cast<float *>(reinterpret_cast<char *>(a.y) + row_offset(a.ym, row));
    for (int i = lane; i < a.ne0; i += kWave) {
        float v;
        if constexpr (MODE == kAddSum) {
            v = sr[i];
        } else if constexpr (MODE == kAdd) {
            v = xr[i] + br[i];
        } else {
            v = xr[i];
        }
        float o = v * scale;
        if constexpr (WT != kWNone) {
            o = o * load_w1<WT>(a.w, i);
        }
        yr[i] = o;
    }
}

// ggml_norm (LayerNorm without the affine part), one wave per row: the mean
// from a double sum, the variance from a double sum of the f32 centred values
// v = x - mean, scale = 1/sqrtf(variance + eps), y = v*scale (ggml-CPU's
// order of roundings; the sums' order differs, within the tolerance). The
// row is read three times, the later reads from cache. Sites:
// qwen3-tts/codec.cpp:216 (ConvNeXt), kokoro/operations.cpp:12,93.
__global__ __launch_bounds__(256) void k_layer_norm(const NormArgs a) {
    const int     lane = threadIdx.x % kWave;
    const int64_t row  = static_cast<int64_t>(blockIdx.x) * (256 / kWave) + threadIdx.x / kWave;
    if (row >= a.nrows) {
        return;
    }
    const float * xr  = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.x) + row_offset(a.xm, row));
    float *       yr  = reinterpret_cast<float *>(reinterpret_cast<char *>(a.y) + row_offset(a.ym, row));
    double        acc = 0.0;
    for (int i = lane; i < a.ne0; i += kWave) {
        acc += static_cast<double>(xr[i]);
    }
    const float mean = static_cast<float>(group_sum<kWave>(acc) / static_cast<double>(a.ne0));
    double      acc2 = 0.0;
    for (int i = lane; i < a.ne0; i += kWave) {
        const float v = xr[i] - mean;
        acc2 += static_cast<double>(v * v);
    }
    const float variance = static_cast<float>(group_sum<kWave>(acc2) / static_cast<double>(a.ne0));
    const float scale    = 1.0f / __builtin_sqrtf(variance + a.eps);
    for (int i = lane; i < a.ne0; i += kWave) {
        yr[i] = (xr[i] - mean) * scale;
    }
}

// ggml_sum_rows / ggml_mean, and the product-sum of ggml_mul then
// ggml_sum_rows (the speaker encoder's attention-weighted statistics,
// qwen3-tts/speaker-encoder.cpp:292-293,374): one wave per row, each lane
// accumulating its f32 values (or f32 products) into a double in element
// order, the lanes' doubles summed by DPP moves and rounded to f32 once; the
// mean divides that f32 by ne0 in f32. ggml-CPU accumulates the row in double
// in element order: the f32 results agree unless the two double sums fall on
// opposite sides of an f32 rounding boundary.
enum SumRowsMode { kSumRows = 0, kMeanRows = 1, kMulSumRows = 2 };

struct SumRowsArgs {
    const float * x;
    RowMap        xm;
    const float * w;
    RowMap        wm;
    float *       y;
    RowMap        ym;
    int64_t       nrows;
    int32_t       ne0;
    int32_t       pad;
};

template <int MODE, bool VEC> __global__ __launch_bounds__(256) void k_sum_rows(const SumRowsArgs a) {
    const int     lane = threadIdx.x % kWave;
    const int64_t row  = static_cast<int64_t>(blockIdx.x) * (256 / kWave) + threadIdx.x / kWave;
    if (row >= a.nrows) {
        return;
    }
    const float * xr  = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.x) + row_offset(a.xm, row));
    const float * wr  = MODE == kMulSumRows ?
                            reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.w) + row_offset(a.wm, row)) :
                            nullptr;
    double        acc = 0.0;
    if constexpr (VEC) {
        const int nvec = a.ne0 / 4;
        for (int i = lane; i < nvec; i += kWave) {
            f32x4 v = ld_stream(reinterpret_cast<const f32x4 *>(xr) + i);
            if constexpr (MODE == kMulSumRows) {
                const f32x4 u = ld_stream(reinterpret_cast<const f32x4 *>(wr) + i);
                v             = f32x4{ v.x * u.x, v.y * u.y, v.z * u.z, v.w * u.w };
            }
            acc += static_cast<double>(v.x);
            acc += static_cast<double>(v.y);
            acc += static_cast<double>(v.z);
            acc += static_cast<double>(v.w);
        }
    } else {
        for (int i = lane; i < a.ne0; i += kWave) {
            const float v = MODE == kMulSumRows ? xr[i] * wr[i] : xr[i];
            acc += static_cast<double>(v);
        }
    }
    acc = group_sum<kWave>(acc);
    if (lane == 0) {
        float v = static_cast<float>(acc);
        if constexpr (MODE == kMeanRows) {
            v = v / static_cast<float>(a.ne0);
        }
        *reinterpret_cast<float *>(reinterpret_cast<char *>(a.y) + row_offset(a.ym, row)) = v;
    }
}

template <int MODE> shp_status_t sum_rows_entry(const shp_tensor * x, const shp_tensor * w, shp_tensor * y,
                                                 hipStream_t stream) {
    if (!well_formed(x) || !well_formed(y) || (MODE == kMulSumRows && !well_formed(w))) {
        return SHP_ERR_INVALID_ARG;
    }
    if (x->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32 || (MODE == kMulSumRows && w->type != SHP_TYPE_F32)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (y->ne[0] != 1 || y->ne[1] != x->ne[1] || y->ne[2] != x->ne[2] || y->ne[3] != x->ne[3] ||
        x->ne[0] > INT32_MAX || (MODE == kMulSumRows && !same_shape(*x, *w))) {
        return SHP_ERR_INVALID_ARG;
    }
    if (spans_overlap(*x, *y) || (MODE == kMulSumRows && spans_overlap(*w, *y))) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (dry_run()) {
        return SHP_OK;
    }
    SumRowsArgs a{};
    a.x     = static_cast<const float *>(x->data);
    a.xm    = make_rowmap(*x);
    a.y     = static_cast<float *>(y->data);
    a.ym    = make_rowmap(*y);
    a.nrows = nrows(*x);
    a.ne0   = static_cast<int32_t>(x->ne[0]);
    bool vec = x->ne[0] % 4 == 0 && rows_aligned(*x, 16);
    if constexpr (MODE == kMulSumRows) {
        a.w  = static_cast<const float *>(w->data);
        a.wm = make_rowmap(*w);
        vec  = vec && rows_aligned(*w, 16);
    }
    const dim3 grid(static_cast<unsigned>((a.nrows + 3) / 4)), block(256);
    if (vec) {
        hipLaunchKernelGGL((k_sum_rows<MODE, true>), grid, block, 0, stream, a);
    } else {
        hipLaunchKernelGGL((k_sum_rows<MODE, false>), grid, block, 0, stream, a);
    }
    return launch_status();
}

template <int WT, int MODE> shp_status_t launch_norm(const NormArgs & a, bool vec, hipStream_t stream) {
    if (dry_run()) {
        return SHP_OK;
    }
    auto go = [&](auto kernel, int rows_per_block, int block = 256) {
        const int64_t blocks = (a.nrows + rows_per_block - 1) / rows_per_block;
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(block), 0, stream, a);
        return launch_status();
    };
    const int nvec = a.ne0 / 4;
    if (vec && nvec <= 256 * 8) {
        if (nvec <= 16) {
            return go(k_rms_norm_vec<16, 1, WT, MODE>, 16);
        }
        if (nvec <= 32) {
            return go(k_rms_norm_vec<32, 1, WT, MODE>, 8);
        }
        if (nvec <= 64) {
            return go(k_rms_norm_vec<64, 1, WT, MODE>, 4);
        }
        if (nvec <= 128) {
            return go(k_rms_norm_vec<128, 1, WT, MODE>, 2);
        }
        // Rows of 1024 / 2048: how many waves share a row, by row count.
        // Measured on MI355X (cold, us; 4 waves per row first, then the pick):
        //   plain 1024: 4 waves up to 2048 rows; two waves per row below
        //     6144 rows ([1024,3072] 6.37 -> 5.67, [1024,4096] 8.15 -> 6.68);
        //     one wave per row from 6144 ([1024,8192] 13.4 -> 11.5);
        //   plain 2048: 4 waves (2 float4 each) up to 2048 rows, then two
        //     waves per row ([2048,3072] 10.3 -> 9.65, [2048,8192] 25.1 ->
        //     22.9, at the same-size copy's speed);
        //   add forms 1024: 4 waves below 1024 rows (more loads in flight);
        //     two waves per row below 4096 ([1024,2048] 7.67 -> 6.51); one
        //     wave per row below 16384 ([1024,4096] 13.8 -> 11.4, [1024,8192]
        //     about even); 4 waves again from 16384 ([1024,16384] 44.0
        //     against 46.0 for one wave);
        //   add forms 2048: 4 waves below 2048 rows; two waves per row below
        //     4096 ([2048,2048] 13.5 -> 11.5); one wave per row from 4096
        //     ([2048,4096] 23.9 -> 21.9).
        const int64_t nr = a.nrows;
        if (nvec == 256 && MODE == kPlain && nr > 2048) {
            return nr < 6144 ? go(k_rms_norm_vec<128, 2, WT, MODE>, 2) : go(k_rms_norm_vec<64, 4, WT, MODE>, 4);
        }
        if (nvec == 256 && MODE != kPlain && nr >= 1024 && nr < 16384) {
            return nr < 4096 ? go(k_rms_norm_vec<128, 2, WT, MODE>, 2) : go(k_rms_norm_vec<64, 4, WT, MODE>, 4);
        }
        if (nvec == 512 && MODE == kPlain && nr > 2048) {
            return go(k_rms_norm_vec<128, 4, WT, MODE>, 2);
        }
        if (nvec == 512 && MODE != kPlain && nr >= 2048) {
            return nr < 4096 ? go(k_rms_norm_vec<128, 4, WT, MODE>, 2) : go(k_rms_norm_vec<64, 8, WT, MODE>, 4);
        }
        switch ((nvec + 255) / 256) {
            case 1:
                return go(k_rms_norm_vec<256, 1, WT, MODE>, 1);
            case 2:
                return go(k_rms_norm_vec<256, 2, WT, MODE>, 1);
            case 3:
                return go(k_rms_norm_vec<256, 3, WT, MODE>, 1);
            case 4:
                return go(k_rms_norm_vec<256, 4, WT, MODE>, 1);
            case 5:
            case 6:
                return go(k_rms_norm_vec<256, 6, WT, MODE>, 1);
            default:
                return go(k_rms_norm_vec<256, 8, WT, MODE>, 1);
        }
    }
    return go(k_rms_norm_generic<WT, MODE>, 4);
}

template <int MODE> shp_status_t dispatch_norm_w(const NormArgs & a, int wk, bool vec, hipStream_t stream) {
    switch (wk) {
        case kWNone:
            return launch_norm<kWNone, MODE>(a, vec, stream);
        case kWF32:
            return launch_norm<kWF32, MODE>(a, vec, stream);
        case kWBF16:
            return launch_norm<kWBF16, MODE>(a, vec, stream);
        case kWF16:
            return launch_norm<kWF16, MODE>(a, vec, stream);
        default:
            return SHP_ERR_UNSUPPORTED;
    }
}

// float4 gain loads: 16-byte aligned F32, 8-byte aligned BF16/F16.
bool gain_aligned(const shp_tensor * w) {
    return w == nullptr || reinterpret_cast<uintptr_t>(w->data) % (w->type == SHP_TYPE_F32 ? 16 : 8) == 0;
}

shp_status_t norm_entry(const shp_tensor * a,
                        const shp_tensor * b,
                        const shp_tensor * w,
                        float              eps,
                        shp_tensor *       sum,
                        shp_tensor *       y,
                        shp_stream_t       stream) {
    if (!well_formed(a) || !well_formed(y) || (b != nullptr && !well_formed(b)) ||
        (sum != nullptr && !well_formed(sum)) || (w != nullptr && !well_formed(w))) {
        return SHP_ERR_INVALID_ARG;
    }
    if (a->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32 || !same_shape(*a, *y)) {
        return a->type != SHP_TYPE_F32 ? SHP_ERR_UNSUPPORTED : SHP_ERR_INVALID_ARG;
    }
    if (b != nullptr && (b->type != SHP_TYPE_F32 || !same_shape(*a, *b))) {
        return SHP_ERR_INVALID_ARG;
    }
    if (sum != nullptr && (sum->type != SHP_TYPE_F32 || !same_shape(*a, *sum))) {
        return SHP_ERR_INVALID_ARG;
    }
    int wk = kWNone;
    if (w != nullptr) {
        wk = weight_kind(w->type);
        if (wk < 0) {
            return SHP_ERR_UNSUPPORTED;
        }
        // ggml_mul broadcasts a single row of ne0 gains over every row.
        if (nelements(*w) != a->ne[0] || !contiguous(*w)) {
            return SHP_ERR_UNSUPPORTED;
        }
    }
    if (a->ne[0] > INT32_MAX || !(eps >= 0.0f)) {
        return SHP_ERR_INVALID_ARG;
    }
    NormArgs args{};
    args.x     = static_cast<const float *>(a->data);
    args.xm    = make_rowmap(*a);
    args.y     = static_cast<float *>(y->data);
    args.ym    = make_rowmap(*y);
    args.nrows = nrows(*a);
    args.ne0   = static_cast<int32_t>(a->ne[0]);
    args.eps   = eps;
    args.w     = w != nullptr ? w->data : nullptr;
    bool vec   = a->ne[0] % 4 == 0 && rows_aligned(*a, 16) && rows_aligned(*y, 16) && gain_aligned(w);
    if (b != nullptr) {
        args.b  = static_cast<const float *>(b->data);
        args.bm = make_rowmap(*b);
        vec     = vec && rows_aligned(*b, 16);
    }
    if (sum != nullptr) {
        args.s  = static_cast<float *>(sum->data);
        args.sm = make_rowmap(*sum);
        vec     = vec && rows_aligned(*sum, 16);
    }
    const hipStream_t st = as_stream(stream);
    if (b == nullptr) {
        return dispatch_norm_w<kPlain>(args, wk, vec, st);
    }
    if (sum == nullptr) {
        return dispatch_norm_w<kAdd>(args, wk, vec, st);
    }
    return dispatch_norm_w<kAddSum>(args, wk, vec, st);
}

// ---------------------------------------------------------------------------
// NEOX rope, optionally preceded by the per-head RMSNorm x weight
// ---------------------------------------------------------------------------

struct RopePart {
    const float * x;
    float *       y;
    const void *  w;
    int64_t       xnb1;
    int64_t       xnb2;
    int64_t       ynb1;
    int64_t       ynb2;
    int32_t       heads;
    int32_t       pad;
};

struct RopeArgs {
    RopePart        part[3];  // q, k, then v (heads == 0 when absent); v rows are copied unchanged
    const int32_t * pos;
    const int32_t * slot;     // KV launches: first cache row from device memory, or null (then 0)
    int32_t *       status;   // with `slot`: set to 1 when the rows do not fit the cache (none written)
    int64_t         cap;      // with `slot`: cache rows
    int64_t         npos;
    int32_t         ne0;
    int32_t         n_dims;
    float           theta_scale;
    float           freq_scale;
    float           attn_factor;
    float           eps;
};

// Fields of head row hh (q rows first, then k rows, then v rows) as selects
// between the parts' kernel arguments, which stay in scalar registers.
// Indexing part[] with a per-lane value instead would read the argument block
// through vector memory and put a dependent round trip in front of every row
// load. KV: the launch has v rows (copied, no gain).
struct RowRef {
    const float * x;
    float *       y;      // the output row at position pi (k and v: before the cache slot)
    const void *  w;
    int64_t       ystep;  // k and v rows: bytes per cache row (the slot moves y by slot * ystep); q: 0
    bool          copy;   // a v row: stored unchanged
    bool          kv;     // a k or v row: lands in the cache

    __device__ __forceinline__ float * y_at(int64_t slot) const {
        return reinterpret_cast<float *>(reinterpret_cast<char *>(y) + slot * ystep);
    }
};

// One part's fields as scalars, for the per-lane selects of rope_row.
// Selecting among the kernel-argument fields themselves lets the compiler turn
// `isk ? k.x : q.x` into one load from a selected argument address, a
// vector-memory round trip in front of every row load; the fields are named
// members (not an array a lane indexes), so they stay in registers.
struct PartFields {
    const char * x;
    char *       y;
    const void * w;
    int64_t      xnb1;
    int64_t      xnb2;
    int64_t      ynb1;
    int64_t      ynb2;
    int32_t      heads;
};

struct RopeFields {
    PartFields q, k, v;
};

__device__ __forceinline__ PartFields part_fields(const RopePart & p) {
    PartFields f{ reinterpret_cast<const char *>(p.x), reinterpret_cast<char *>(p.y), p.w, p.xnb1, p.xnb2, p.ynb1,
                  p.ynb2, p.heads };
    args_in_sgprs(f.x, f.y, f.w, f.xnb1, f.xnb2, f.ynb1, f.ynb2, f.heads);
    return f;
}

template <bool KV> __device__ __forceinline__ RopeFields rope_fields(const RopeArgs & a) {
    RopeFields f;
    f.q = part_fields(a.part[0]);
    f.k = part_fields(a.part[1]);
    if constexpr (KV) {
        f.v = part_fields(a.part[2]);
    } else {
        f.v       = f.q;
        f.v.heads = 0;
    }
    return f;
}

// One of three scalars by masks (mk, mv: all ones or zero, not both), as
// bitwise arithmetic: a select the compiler cannot turn into a load from a
// selected address.
__device__ __forceinline__ uint64_t pick3(uint64_t mk, uint64_t mv, uint64_t q, uint64_t k, uint64_t v) {
    return (q & ~(mk | mv)) | (k & mk) | (v & mv);
}

template <class T> __device__ __forceinline__ uint64_t bits(T v) {
    if constexpr (sizeof(T) == 8) {
        return __builtin_bit_cast(uint64_t, v);
    } else {
        return static_cast<uint64_t>(static_cast<int64_t>(v));
    }
}

// Head row hh of position pi: q rows first, then k rows, then (KV) v rows.
template <bool KV> __device__ __forceinline__ RowRef rope_row(const RopeFields & a, int hh, int64_t pi) {
    const PartFields & q    = a.q;
    const PartFields & k    = a.k;
    const PartFields & v    = a.v;
    const int          qk   = q.heads + k.heads;
    const bool         isv  = KV && hh >= qk;
    const bool         isk  = !isv && hh >= q.heads;
    const uint64_t     mv   = isv ? ~uint64_t{ 0 } : 0;
    const uint64_t     mk   = isk ? ~uint64_t{ 0 } : 0;
    auto               sel  = [&](auto fq, auto fk, auto fv) { return pick3(mk, mv, bits(fq), bits(fk), bits(fv)); };
    const int64_t      h    = hh - static_cast<int64_t>(sel(0, q.heads, qk));
    const uint64_t     xb   = sel(q.x, k.x, v.x);
    const uint64_t     yb   = sel(q.y, k.y, v.y);
    const int64_t      xo   = h * static_cast<int64_t>(sel(q.xnb1, k.xnb1, v.xnb1)) +
                       pi * static_cast<int64_t>(sel(q.xnb2, k.xnb2, v.xnb2));
    const int64_t      ynb2 = static_cast<int64_t>(sel(q.ynb2, k.ynb2, v.ynb2));
    const int64_t      yo   = h * static_cast<int64_t>(sel(q.ynb1, k.ynb1, v.ynb1)) + pi * ynb2;
    return RowRef{ reinterpret_cast<const float *>(xb + xo), reinterpret_cast<float *>(yb + yo),
                   reinterpret_cast<const void *>(sel(q.w, k.w, static_cast<const void *>(nullptr))),
                   KV && (isk || isv) ? ynb2 : 0, isv, isk || isv };
}

// The KV launches' cache slot: 0 without a device slot; with one, its value,
// or -1 when the T rows from it do not fit the cache (block 0 then raises
// *status; no cache row is written).
template <bool KV> __device__ __forceinline__ int64_t rope_slot(const RopeArgs & a) {
    if constexpr (!KV) {
        return 0;
    } else {
        if (a.slot == nullptr) {
            return 0;
        }
        // a scalar load: a vector load here would be waited for (with every
        // row load before it) at the range check, ahead of the theta chain
        const int64_t sl = ld_const(a.slot);
        if (sl >= 0 && sl <= a.cap - a.npos) {
            return sl;
        }
        if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0 && a.status != nullptr) {
            *a.status = 1;
        }
        return -1;
    }
}

template <bool KV> __device__ __forceinline__ int rope_rows(const RopeArgs & a) {
    return a.part[0].heads + a.part[1].heads + (KV ? a.part[2].heads : 0);
}

template <bool KV> __device__ __forceinline__ int rope_rows(const RopeFields & f) {
    return f.q.heads + f.k.heads + (KV ? f.v.heads : 0);
}

// cos/sin of an f32 angle: evaluated in double and rounded once (the fast
// Cody-Waite path covers |angle| < 2^19 * pi/2; OCML's double sincos beyond).
__device__ __forceinline__ void rope_sincos(float th, float & s, float & c) {
    if (!sincos_f32_rn(th, s, c)) {
        double sd, cd;
        sincos(static_cast<double>(th), &sd, &cd);
        s = static_cast<float>(sd);
        c = static_cast<float>(cd);
    }
}

// theta_k = p * s * s * ... (k f32 multiplies, each rounded: the CPU cache's
// recurrence) in lane k of a full wave. One v_mul_f32 per step: before step i
// the exec mask drops lane i - 1 (s_bitset0_b64 leaves SCC alone), so lane k
// takes part in exactly the first k multiplies; the mask is restored after.
// Written out because the compiler's form of the same loop -- every lane
// multiplying and keeping its step's value by a compare and a select -- costs
// three vector instructions and a hazard wait per step: 0.5 us of a one-token
// QK-norm+RoPE launch. Plain v_mul_f32 under the kernel's float mode, so the
// values are the compiler's multiplies bit for bit.
#define SHP_THETA_STEP(i) "s_bitset0_b64 exec, " #i "\n\tv_mul_f32 %0, %1, %0\n\t"

__device__ __forceinline__ float theta_chain64(float p, float s) {
    float    th = p;
    uint64_t saved;
    asm volatile("s_mov_b64 %0, exec" : "=s"(saved));
    asm volatile(
                 SHP_THETA_STEP(0) SHP_THETA_STEP(1) SHP_THETA_STEP(2) SHP_THETA_STEP(3) SHP_THETA_STEP(4) SHP_THETA_STEP(5) SHP_THETA_STEP(6)
                 SHP_THETA_STEP(7) SHP_THETA_STEP(8) SHP_THETA_STEP(9) SHP_THETA_STEP(10) SHP_THETA_STEP(11) SHP_THETA_STEP(12) SHP_THETA_STEP(13)
                 SHP_THETA_STEP(14) SHP_THETA_STEP(15) SHP_THETA_STEP(16) SHP_THETA_STEP(17) SHP_THETA_STEP(18) SHP_THETA_STEP(19) SHP_THETA_STEP(20)
                 SHP_THETA_STEP(21) SHP_THETA_STEP(22) SHP_THETA_STEP(23) SHP_THETA_STEP(24) SHP_THETA_STEP(25) SHP_THETA_STEP(26) SHP_THETA_STEP(27)
                 SHP_THETA_STEP(28) SHP_THETA_STEP(29) SHP_THETA_STEP(30) SHP_THETA_STEP(31) SHP_THETA_STEP(32) SHP_THETA_STEP(33) SHP_THETA_STEP(34)
                 SHP_THETA_STEP(35) SHP_THETA_STEP(36) SHP_THETA_STEP(37) SHP_THETA_STEP(38) SHP_THETA_STEP(39) SHP_THETA_STEP(40) SHP_THETA_STEP(41)
                 SHP_THETA_STEP(42) SHP_THETA_STEP(43) SHP_THETA_STEP(44) SHP_THETA_STEP(45) SHP_THETA_STEP(46) SHP_THETA_STEP(47) SHP_THETA_STEP(48)
                 SHP_THETA_STEP(49) SHP_THETA_STEP(50) SHP_THETA_STEP(51) SHP_THETA_STEP(52) SHP_THETA_STEP(53) SHP_THETA_STEP(54) SHP_THETA_STEP(55)
                 SHP_THETA_STEP(56) SHP_THETA_STEP(57) SHP_THETA_STEP(58) SHP_THETA_STEP(59) SHP_THETA_STEP(60) SHP_THETA_STEP(61) SHP_THETA_STEP(62)
                 "s_mov_b64 exec, %2"
                 : "+v"(th)
                 : "s"(s), "s"(saved));
    return th;
}

#undef SHP_THETA_STEP

// cos/sin of the pair-k angle at position p: theta is replayed through the f32
// recurrence theta <- theta*theta_scale exactly k times (the CPU cache's order),
// then cos/sin are evaluated in double and rounded once to f32, then scaled by
// attn_factor in f32 as the CPU cache does.
__device__ __forceinline__ void rope_cs(int32_t p, int k, const RopeArgs & a, float & c, float & s) {
    float theta = static_cast<float>(p);
    for (int i = 0; i < k; ++i) {
        theta = theta * a.theta_scale;
    }
    float sf, cf;
    rope_sincos(a.freq_scale * theta, sf, cf);
    c = cf * a.attn_factor;
    s = sf * a.attn_factor;
}

// Fast path: head_dim == n_dims == 128, one block per position.
//
// A head row is owned by 16 lanes; lane j holds x[4j..4j+3] and
// x[64+4j..64+4j+3] as two float4, i.e. both halves of NEOX pairs 4j..4j+3,
// so the rotation needs no data exchange and every access is 128-bit. The
// block has one 16-lane group per head row of the position (q heads, then k
// heads; 24 rows = 384 lanes for Qwen3-TTS; with the KV-cache write, v heads
// follow and are stored unchanged), so every row load is issued at once.
// Meanwhile wave 0 builds the position's 64-entry cos/sin cache: it runs the
// serial f32 theta chain once, lane k leaving it after k multiplies
// (theta_chain64), evaluates its cos/sin in double and writes them to LDS;
// one barrier later every lane reads the 4 pairs it needs.
constexpr int kRopeLanes   = 16;
constexpr int kRopeMaxRows = 1024 / kRopeLanes;

template <bool NORM, int WT, bool KV> __global__ __launch_bounds__(1024) void k_rope128(const RopeArgs a) {
    __shared__ f32x4 s_cos[16];
    __shared__ f32x4 s_sin[16];

    const int64_t pi = blockIdx.x;
    // the position first: read before the field copies below, it stays one
    // scalar load
    const int32_t    p     = a.pos[pi];
    const RopeFields f     = rope_fields<KV>(a);
    const int        total = rope_rows<KV>(f);
    const int        slots = blockDim.x / kRopeLanes;
    const int        g     = threadIdx.x / kRopeLanes;
    const int        l     = threadIdx.x % kRopeLanes;

    // 1. this lane's first row, and its gains (both issued before any wait)
    const bool live = g < total;
    RowRef     r    = rope_row<KV>(f, live ? g : 0, pi);
    f32x4      lo   = splat4(0.0f);
    f32x4      hi   = splat4(0.0f);
    if (live) {
        lo = ld_stream(to_global(reinterpret_cast<const f32x4 *>(r.x)) + l);
        hi = ld_stream(to_global(reinterpret_cast<const f32x4 *>(r.x + 64)) + l);
    }
    // Gains stay raw until after the barrier: converting them here would make
    // wave 0 wait for every outstanding load before its theta chain.
    WRaw<WT> wlo_raw{}, whi_raw{};
    if constexpr (NORM && WT != kWNone) {
        if (live && !r.copy) {
            wlo_raw = load_wraw<WT>(r.w, 4 * l);
            whi_raw = load_wraw<WT>(r.w, 64 + 4 * l);
        }
    }

    // the cache slot (KV launches; read after the row loads went out, which do
    // not depend on it): -1 when the rows do not fit, then no k or v row is stored
    const int64_t slot = rope_slot<KV>(a);

    // 2. the cos/sin cache of this position (wave 0)
    if (threadIdx.x < 64) {
        const int   k   = threadIdx.x;
        const float mth = theta_chain64(static_cast<float>(p), a.theta_scale);
        float       sv, cv;
        rope_sincos(a.freq_scale * mth, sv, cv);
        reinterpret_cast<float *>(s_cos)[k] = cv * a.attn_factor;
        reinterpret_cast<float *>(s_sin)[k] = sv * a.attn_factor;
    }
    __syncthreads();
    const f32x4 cs = s_cos[l];
    const f32x4 sn = s_sin[l];

    // 3. normalise, rotate, store; rows beyond the first slot pass (more than
    //    64 heads) are loaded here
    for (int row = g; row < total; row += slots) {
        if (row != g) {
            r  = rope_row<KV>(f, row, pi);
            lo = ld_stream(to_global(reinterpret_cast<const f32x4 *>(r.x)) + l);
            hi = ld_stream(to_global(reinterpret_cast<const f32x4 *>(r.x + 64)) + l);
            if constexpr (NORM && WT != kWNone) {
                if (!r.copy) {
                    wlo_raw = load_wraw<WT>(r.w, 4 * l);
                    whi_raw = load_wraw<WT>(r.w, 64 + 4 * l);
                }
            }
        }
        const f32x4 rawlo = lo;
        const f32x4 rawhi = hi;
        if constexpr (NORM) {
            double acc        = sq4v(lo) + sq4v(hi);
            acc               = group_sum<kRopeLanes>(acc);
            const float scale = norm_scale(acc, 128, a.eps);
            lo                = f32x4{ lo.x * scale, lo.y * scale, lo.z * scale, lo.w * scale };
            hi                = f32x4{ hi.x * scale, hi.y * scale, hi.z * scale, hi.w * scale };
            if constexpr (WT != kWNone) {
                const f32x4 wlo = cvt_wraw<WT>(wlo_raw);
                const f32x4 whi = cvt_wraw<WT>(whi_raw);
                lo = f32x4{ lo.x * wlo.x, lo.y * wlo.y, lo.z * wlo.z, lo.w * wlo.w };
                hi = f32x4{ hi.x * whi.x, hi.y * whi.y, hi.z * whi.z, hi.w * whi.w };
            }
        }
        const f32x4 olo{ lo.x * cs.x - hi.x * sn.x, lo.y * cs.y - hi.y * sn.y, lo.z * cs.z - hi.z * sn.z,
                         lo.w * cs.w - hi.w * sn.w };
        const f32x4 ohi{ lo.x * sn.x + hi.x * cs.x, lo.y * sn.y + hi.y * cs.y, lo.z * sn.z + hi.z * cs.z,
                         lo.w * sn.w + hi.w * cs.w };
        // a v row (whole 16-lane group) stores its input unchanged
        if (!KV || slot >= 0 || !r.kv) {
            float * y = r.y_at(slot);
            st_stream(to_global(reinterpret_cast<f32x4 *>(y)) + l, KV && r.copy ? rawlo : olo);
            st_stream(to_global(reinterpret_cast<f32x4 *>(y + 64)) + l, KV && r.copy ? rawhi : ohi);
        }
    }
}

// The same for a few positions (a decode step). A position's head rows (q,
// then k, then v) are split into blocks of kRopeDecRows rows (the grid's y),
// and in each block the row waves take their whole row through the QK-norm
// (and gains) before the barrier, while one extra wave, wave 0, builds the
// position's cos/sin cache. The wave that runs the serial theta chain holds
// no rows, so the norm is not behind the chain on the block's critical path:
// after the barrier a row wave only rotates and stores. A block of v rows
// only (the KV-cache write) copies them, with no theta wave work and no
// barrier. Every block of a position runs the same theta chain, so a block
// waits for at most 8 rows' loads and norms instead of all of them. Measured
// on MI355X, one-token launch with the KV write (16 q + 8 k + 8 v rows, back
// to back): 2.83 us as one block with the theta wave after the rows, 2.63
// with it first and the slot a scalar load, 2.41 split over four blocks (4
// rows per block: the same). Same arithmetic as k_rope128, bit for bit.
constexpr int kRopeDecRows = 8;

template <bool NORM, int WT, bool KV>
__global__ __launch_bounds__(kWave + kRopeDecRows * kRopeLanes) void k_rope128_dec(const RopeArgs a) {
    __shared__ f32x4 s_cos[16];
    __shared__ f32x4 s_sin[16];

    const int64_t    pi    = blockIdx.x;
    const RopeFields f     = rope_fields<KV>(a);
    const int        total = rope_rows<KV>(f);
    const int        r0    = static_cast<int>(blockIdx.y) * kRopeDecRows;  // this block's first row
    const int        l     = static_cast<int>(threadIdx.x) % kRopeLanes;
    if (KV && r0 >= f.q.heads + f.k.heads) {
        // v rows only: the cache write, a plain copy
        const int     g    = r0 + static_cast<int>(threadIdx.x) / kRopeLanes;
        const int64_t slot = rope_slot<KV>(a);
        if (static_cast<int>(threadIdx.x) >= kRopeDecRows * kRopeLanes || g >= total || slot < 0) {
            return;
        }
        const RowRef r  = rope_row<KV>(f, g, pi);
        const f32x4  lo = ld_stream(to_global(reinterpret_cast<const f32x4 *>(r.x)) + l);
        const f32x4  hi = ld_stream(to_global(reinterpret_cast<const f32x4 *>(r.x + 64)) + l);
        float *      y  = r.y_at(slot);
        st_stream(to_global(reinterpret_cast<f32x4 *>(y)) + l, lo);
        st_stream(to_global(reinterpret_cast<f32x4 *>(y + 64)) + l, hi);
        return;
    }
    const int32_t p     = a.pos[pi];
    const int     tid   = static_cast<int>(threadIdx.x) - kWave;  // row thread index; < 0 in the theta wave
    const bool    theta = tid < 0;                                 // uniform over each wave
    const int     g     = r0 + (theta ? 0 : tid / kRopeLanes);
    const bool    live  = !theta & (g < total);

    RowRef r = rope_row<KV>(f, live ? g : 0, pi);
    f32x4  lo = splat4(0.0f), hi = splat4(0.0f), rawlo = lo, rawhi = hi;
    if (live) {
        lo = ld_stream(to_global(reinterpret_cast<const f32x4 *>(r.x)) + l);
        hi = ld_stream(to_global(reinterpret_cast<const f32x4 *>(r.x + 64)) + l);
    }
    WRaw<WT> wlo_raw{}, whi_raw{};
    if constexpr (NORM && WT != kWNone) {
        if (live && !r.copy) {
            wlo_raw = load_wraw<WT>(r.w, 4 * l);
            whi_raw = load_wraw<WT>(r.w, 64 + 4 * l);
        }
    }
    const int64_t slot = rope_slot<KV>(a);
    if (theta) {
        const int   k   = static_cast<int>(threadIdx.x);
        const float mth = theta_chain64(static_cast<float>(p), a.theta_scale);
        float       sv, cv;
        rope_sincos(a.freq_scale * mth, sv, cv);
        reinterpret_cast<float *>(s_cos)[k] = cv * a.attn_factor;
        reinterpret_cast<float *>(s_sin)[k] = sv * a.attn_factor;
    } else {
        rawlo = lo;
        rawhi = hi;
        if constexpr (NORM) {
            double acc        = sq4v(lo) + sq4v(hi);
            acc               = group_sum<kRopeLanes>(acc);
            const float scale = norm_scale(acc, 128, a.eps);
            lo                = f32x4{ lo.x * scale, lo.y * scale, lo.z * scale, lo.w * scale };
            hi                = f32x4{ hi.x * scale, hi.y * scale, hi.z * scale, hi.w * scale };
            if constexpr (WT != kWNone) {
                const f32x4 wlo = cvt_wraw<WT>(wlo_raw);
                const f32x4 whi = cvt_wraw<WT>(whi_raw);
                lo = f32x4{ lo.x * wlo.x, lo.y * wlo.y, lo.z * wlo.z, lo.w * wlo.w };
                hi = f32x4{ hi.x * whi.x, hi.y * whi.y, hi.z * whi.z, hi.w * whi.w };
            }
        }
    }
    __syncthreads();
    if (!live) {
        return;
    }
    const f32x4 cs = s_cos[l];
    const f32x4 sn = s_sin[l];
    const f32x4 olo{ lo.x * cs.x - hi.x * sn.x, lo.y * cs.y - hi.y * sn.y, lo.z * cs.z - hi.z * sn.z,
                     lo.w * cs.w - hi.w * sn.w };
    const f32x4 ohi{ lo.x * sn.x + hi.x * cs.x, lo.y * sn.y + hi.y * cs.y, lo.z * sn.z + hi.z * cs.z,
                     lo.w * sn.w + hi.w * cs.w };
    if (!KV || slot >= 0 || !r.kv) {
        float * y = r.y_at(slot);
        st_stream(to_global(reinterpret_cast<f32x4 *>(y)) + l, KV && r.copy ? rawlo : olo);
        st_stream(to_global(reinterpret_cast<f32x4 *>(y + 64)) + l, KV && r.copy ? rawhi : ohi);
    }
}

// Any head_dim / n_dims: one wave per head row; the theta recurrence is
// replayed per pair (fine for the small shapes that take this path).
template <bool NORM, int WT, bool KV> __global__ __launch_bounds__(256) void k_rope_generic(const RopeArgs a) {
    const int     lane  = threadIdx.x % kWave;
    const int     total = rope_rows<KV>(a);
    const int64_t row   = static_cast<int64_t>(blockIdx.x) * (256 / kWave) + threadIdx.x / kWave;
    if (row >= a.npos * total) {
        return;
    }
    const int64_t pi   = row / total;
    const int     hh   = static_cast<int>(row % total);
    const int64_t slot = rope_slot<KV>(a);
    const RowRef  rr   = rope_row<KV>(rope_fields<KV>(a), hh, pi);
    const float * xr   = rr.x;
    float *       yr   = rr.y_at(slot);
    if (KV && rr.kv && slot < 0) {
        return;  // the rows do not fit the cache: nothing written
    }
    if (KV && rr.copy) {  // a v row: the cache write, a plain copy (ggml_cpy F32 -> F32)
        for (int i = lane; i < a.ne0; i += kWave) {
            yr[i] = xr[i];
        }
        return;
    }
    const int32_t p = a.pos[pi];

    float scale = 1.0f;
    if constexpr (NORM) {
        double acc = 0.0;
        for (int i = lane; i < a.ne0; i += kWave) {
            acc += static_cast<double>(xr[i] * xr[i]);
        }
        acc   = group_sum<kWave>(acc);
        scale = norm_scale(acc, a.ne0, a.eps);
    }
    auto normed = [&](int i) {
        float v = xr[i];
        if constexpr (NORM) {
            v = v * scale;
            if constexpr (WT != kWNone) {
                v = v * load_w1<WT>(rr.w, i);
            }
        }
        return v;
    };
    const int half = a.n_dims / 2;
    for (int ic = lane; ic < half; ic += kWave) {
        float c, s;
        rope_cs(p, ic, a, c, s);
        const float x0  = normed(ic);
        const float x1  = normed(ic + half);
        yr[ic]          = x0 * c - x1 * s;
        yr[ic + half]   = x0 * s + x1 * c;
    }
    for (int i = a.n_dims + lane; i < a.ne0; i += kWave) {
        yr[i] = normed(i);
    }
}

// Up to this many positions a launch takes k_rope128_dec (a decode step of
// up to 64 streams); longer ones k_rope128, whose blocks hide the theta chain
// behind each other. Measured on MI355X (cold, 16 q + 8 k rows): one position
// 2.38 -> 2.18 us, 16: 2.52 -> 2.46, 64: 2.62 -> 2.55; at 128 k_rope128 is
// ahead (2.77 against 2.86).
constexpr int64_t kRopeDecMaxPos = 64;

template <bool NORM, int WT, bool KV> shp_status_t launch_rope(const RopeArgs & a, bool fast, hipStream_t stream) {
    if (dry_run()) {
        return SHP_OK;
    }
    const int total = a.part[0].heads + a.part[1].heads + a.part[2].heads;
    if (fast && a.npos <= kRopeDecMaxPos) {
        const int chunks = (total + kRopeDecRows - 1) / kRopeDecRows;
        hipLaunchKernelGGL((k_rope128_dec<NORM, WT, KV>), dim3(static_cast<unsigned>(a.npos), static_cast<unsigned>(chunks)),
                           dim3(kWave + kRopeDecRows * kRopeLanes), 0, stream, a);
        return launch_status();
    }
    if (fast) {
        const int rows    = total < kRopeMaxRows ? total : kRopeMaxRows;
        const int threads = ((rows * kRopeLanes + kWave - 1) / kWave) * kWave;
        hipLaunchKernelGGL((k_rope128<NORM, WT, KV>), dim3(static_cast<unsigned>(a.npos)), dim3(threads), 0, stream,
                           a);
        return launch_status();
    }
    const int64_t rows   = a.npos * total;
    const int64_t blocks = (rows + 3) / 4;
    hipLaunchKernelGGL((k_rope_generic<NORM, WT, KV>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
    return launch_status();
}

template <bool NORM, bool KV>
shp_status_t dispatch_rope_w(const RopeArgs & a, int wk, bool fast, hipStream_t stream) {
    switch (wk) {
        case kWNone:
            return launch_rope<NORM, kWNone, KV>(a, fast, stream);
        case kWF32:
            return launch_rope<NORM, kWF32, KV>(a, fast, stream);
        case kWBF16:
            return launch_rope<NORM, kWBF16, KV>(a, fast, stream);
        case kWF16:
            return launch_rope<NORM, kWF16, KV>(a, fast, stream);
        default:
            return SHP_ERR_UNSUPPORTED;
    }
}

// Validates one [head_dim, heads, T, 1] F32 part against its output.
bool rope_part_ok(const shp_tensor * x, const shp_tensor * y) {
    return well_formed(x) && well_formed(y) && x->type == SHP_TYPE_F32 && y->type == SHP_TYPE_F32 &&
           same_shape(*x, *y) && x->ne[3] == 1 && x->ne[1] <= INT32_MAX;
}

bool part_aligned(const shp_tensor & t) {
    return reinterpret_cast<uintptr_t>(t.data) % 16 == 0 && t.nb[1] % 16 == 0 && t.nb[2] % 16 == 0;
}

shp_status_t rope_entry(const shp_tensor * q,
                        const shp_tensor * k,
                        const shp_tensor * v,
                        const shp_tensor * wq,
                        const shp_tensor * wk,
                        bool               norm,
                        float              eps,
                        const shp_tensor * pos,
                        int32_t            n_dims,
                        float              freq_base,
                        float              freq_scale,
                        float              attn_factor,
                        shp_tensor *       q_out,
                        shp_tensor *       k_out,
                        shp_tensor *       v_out,
                        shp_stream_t       stream,
                        const int32_t *    slot   = nullptr,
                        int32_t *          status = nullptr,
                        int64_t            cap    = 0) {
    if (!rope_part_ok(q, q_out) || !well_formed(pos) || pos->type != SHP_TYPE_I32) {
        return SHP_ERR_INVALID_ARG;
    }
    if (!i32_aligned(*pos)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if ((k == nullptr) != (k_out == nullptr) || (v == nullptr) != (v_out == nullptr) || (v != nullptr && k == nullptr)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (k != nullptr && (!rope_part_ok(k, k_out) || k->ne[0] != q->ne[0] || k->ne[2] != q->ne[2])) {
        return SHP_ERR_INVALID_ARG;
    }
    if (v != nullptr && (!rope_part_ok(v, v_out) || !same_shape(*v, *k))) {
        return SHP_ERR_INVALID_ARG;
    }
    // ggml_rope_ext: positions are an I32 vector of ne[2] entries.
    if (nelements(*pos) != q->ne[2] || !contiguous(*pos)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (n_dims <= 0 || n_dims % 2 != 0 || n_dims > q->ne[0] || q->ne[0] > INT32_MAX) {
        return SHP_ERR_INVALID_ARG;
    }
    int wkind = kWNone;
    if (norm) {
        // Both heads carry a gain or neither does; without k there is no wk.
        if ((k != nullptr && (wq == nullptr) != (wk == nullptr)) || (k == nullptr && wk != nullptr)) {
            return SHP_ERR_INVALID_ARG;
        }
        if (wq != nullptr) {
            if (!well_formed(wq) || nelements(*wq) != q->ne[0] || !contiguous(*wq)) {
                return SHP_ERR_INVALID_ARG;
            }
            wkind = weight_kind(wq->type);
            if (wkind < 0) {
                return SHP_ERR_UNSUPPORTED;
            }
        }
        if (k != nullptr && wk != nullptr) {
            if (!well_formed(wk) || nelements(*wk) != k->ne[0] || !contiguous(*wk)) {
                return SHP_ERR_INVALID_ARG;
            }
            if (weight_kind(wk->type) != wkind) {
                return SHP_ERR_UNSUPPORTED;  // one launch reads both gains with one converter
            }
        }
        if (!(eps >= 0.0f)) {
            return SHP_ERR_INVALID_ARG;
        }
    }
    if (q->ne[1] + (k != nullptr ? k->ne[1] : 0) + (v != nullptr ? v->ne[1] : 0) > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }

    RopeArgs a{};
    auto     fill = [](RopePart & P, const shp_tensor * x, shp_tensor * y, const shp_tensor * w) {
        P.x     = static_cast<const float *>(x->data);
        P.y     = static_cast<float *>(y->data);
        P.w     = w != nullptr ? w->data : nullptr;
        P.xnb1  = static_cast<int64_t>(x->nb[1]);
        P.xnb2  = static_cast<int64_t>(x->nb[2]);
        P.ynb1  = static_cast<int64_t>(y->nb[1]);
        P.ynb2  = static_cast<int64_t>(y->nb[2]);
        P.heads = static_cast<int32_t>(x->ne[1]);
    };
    fill(a.part[0], q, q_out, norm ? wq : nullptr);
    if (k != nullptr) {
        fill(a.part[1], k, k_out, norm ? wk : nullptr);
    } else {
        a.part[1]       = a.part[0];
        a.part[1].heads = 0;
    }
    if (v != nullptr) {
        fill(a.part[2], v, v_out, nullptr);
    } else {
        a.part[2]       = a.part[0];
        a.part[2].heads = 0;
    }
    a.pos         = static_cast<const int32_t *>(pos->data);
    a.slot        = slot;
    a.status      = status;
    a.cap         = cap;
    a.npos        = q->ne[2];
    a.ne0         = static_cast<int32_t>(q->ne[0]);
    a.n_dims      = n_dims;
    a.theta_scale = powf(freq_base, -2.0f / static_cast<float>(n_dims));
    a.freq_scale  = freq_scale;
    a.attn_factor = attn_factor;
    a.eps         = eps;
    if (norm && wq == nullptr) {
        wkind = kWNone;
    }

    bool fast = q->ne[0] == 128 && n_dims == 128 && part_aligned(*q) && part_aligned(*q_out);
    if (k != nullptr) {
        fast = fast && part_aligned(*k) && part_aligned(*k_out);
    }
    if (v != nullptr) {
        fast = fast && part_aligned(*v) && part_aligned(*v_out);
    }
    if (norm) {
        fast = fast && gain_aligned(wq) && gain_aligned(wk);
    }
    if (a.npos > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    const hipStream_t st = as_stream(stream);
    if (v != nullptr) {
        return norm ? dispatch_rope_w<true, true>(a, wkind, fast, st) : dispatch_rope_w<false, true>(a, kWNone, fast, st);
    }
    return norm ? dispatch_rope_w<true, false>(a, wkind, fast, st) : dispatch_rope_w<false, false>(a, kWNone, fast, st);
}

// The rows [filled, filled + T) of a KV cache [head_dim, kv_heads, capacity, 1]
// as a [head_dim, kv_heads, T] view: ggml_view_3d(cache, hd, kv, T, nb1, nb2,
// filled*nb2) of qwen3-tts/operations.cpp:109-116.
bool cache_view(const shp_tensor * cache, const shp_tensor * src, int64_t filled, shp_tensor & view) {
    if (!well_formed(cache) || src == nullptr || cache->type != SHP_TYPE_F32 || cache->ne[0] != src->ne[0] ||
        cache->ne[1] != src->ne[1] || cache->ne[3] != 1 || filled < 0 || src->ne[2] > cache->ne[2] - filled) {
        return false;
    }
    view       = *cache;
    view.ne[2] = src->ne[2];
    view.data  = static_cast<char *>(cache->data) + static_cast<size_t>(filled) * cache->nb[2];
    return true;
}

}  // namespace
}  // namespace shp

extern "C" shp_status_t shp_norm(const shp_tensor * x, float eps, shp_tensor * y, shp_stream_t stream) {
    using namespace shp;
    if (!well_formed(x) || !well_formed(y) || !(eps >= 0.0f)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (x->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (!same_shape(*x, *y) || x->ne[0] > INT32_MAX) {
        return SHP_ERR_INVALID_ARG;
    }
    if (dry_run()) {
        return SHP_OK;
    }
    NormArgs a{};
    a.x                  = static_cast<const float *>(x->data);
    a.xm                 = make_rowmap(*x);
    a.y                  = static_cast<float *>(y->data);
    a.ym                 = make_rowmap(*y);
    a.nrows              = nrows(*x);
    a.ne0                = static_cast<int32_t>(x->ne[0]);
    a.eps                = eps;
    const int64_t blocks = (a.nrows + 3) / 4;
    hipLaunchKernelGGL(k_layer_norm, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream), a);
    return launch_status();
}

extern "C" shp_status_t shp_sum_rows(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return shp::sum_rows_entry<shp::kSumRows>(x, nullptr, y, shp::as_stream(stream));
}

extern "C" shp_status_t shp_mean(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return shp::sum_rows_entry<shp::kMeanRows>(x, nullptr, y, shp::as_stream(stream));
}

extern "C" shp_status_t shp_mul_sum_rows(const shp_tensor * x, const shp_tensor * w, shp_tensor * y,
                                         shp_stream_t stream) {
    return shp::sum_rows_entry<shp::kMulSumRows>(x, w, y, shp::as_stream(stream));
}

extern "C" shp_status_t shp_rms_norm_mul(const shp_tensor * x,
                                         const shp_tensor * w,
                                         float              eps,
                                         shp_tensor *       y,
                                         shp_stream_t       stream) {
    return shp::norm_entry(x, nullptr, w, eps, nullptr, y, stream);
}

extern "C" shp_status_t shp_add_rms_norm_mul(const shp_tensor * a,
                                             const shp_tensor * b,
                                             const shp_tensor * w,
                                             float              eps,
                                             shp_tensor *       sum,
                                             shp_tensor *       y,
                                             shp_stream_t       stream) {
    if (b == nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    return shp::norm_entry(a, b, w, eps, sum, y, stream);
}

extern "C" shp_status_t shp_rope_ext(const shp_tensor * x,
                                     const shp_tensor * pos,
                                     int32_t            n_dims,
                                     int32_t            mode,
                                     float              freq_base,
                                     float              freq_scale,
                                     float              ext_factor,
                                     float              attn_factor,
                                     shp_tensor *       y,
                                     shp_stream_t       stream) {
    if (mode != SHP_ROPE_TYPE_NEOX || ext_factor != 0.0f) {
        return SHP_ERR_UNSUPPORTED;
    }
    return shp::rope_entry(x, nullptr, nullptr, nullptr, nullptr, false, 0.0f, pos, n_dims, freq_base, freq_scale,
                           attn_factor, y, nullptr, nullptr, stream);
}

extern "C" shp_status_t shp_qk_norm_rope(const shp_tensor * q,
                                         const shp_tensor * k,
                                         const shp_tensor * wq,
                                         const shp_tensor * wk,
                                         float              eps,
                                         const shp_tensor * pos,
                                         int32_t            n_dims,
                                         float              freq_base,
                                         float              freq_scale,
                                         shp_tensor *       q_out,
                                         shp_tensor *       k_out,
                                         shp_stream_t       stream) {
    return shp::rope_entry(q, k, nullptr, wq, wk, true, eps, pos, n_dims, freq_base, freq_scale, 1.0f, q_out, k_out,
                           nullptr, stream);
}

extern "C" shp_status_t shp_qk_norm_rope_kv(const shp_tensor * q,
                                            const shp_tensor * k,
                                            const shp_tensor * v,
                                            const shp_tensor * wq,
                                            const shp_tensor * wk,
                                            float              eps,
                                            const shp_tensor * pos,
                                            int32_t            n_dims,
                                            float              freq_base,
                                            float              freq_scale,
                                            shp_tensor *       q_out,
                                            shp_tensor *       k_cache,
                                            shp_tensor *       v_cache,
                                            int64_t            filled,
                                            shp_stream_t       stream) {
    if (!shp::well_formed(k) || !shp::well_formed(v) || k_cache == nullptr || v_cache == nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    shp_tensor kview{}, vview{};
    if (!shp::cache_view(k_cache, k, filled, kview) || !shp::cache_view(v_cache, v, filled, vview)) {
        return SHP_ERR_INVALID_ARG;
    }
    return shp::rope_entry(q, k, v, wq, wk, true, eps, pos, n_dims, freq_base, freq_scale, 1.0f, q_out, &kview,
                           &vview, stream);
}

extern "C" shp_status_t shp_qk_norm_rope_kv_at(const shp_tensor * q,
                                               const shp_tensor * k,
                                               const shp_tensor * v,
                                               const shp_tensor * wq,
                                               const shp_tensor * wk,
                                               float              eps,
                                               const shp_tensor * pos,
                                               int32_t            n_dims,
                                               float              freq_base,
                                               float              freq_scale,
                                               shp_tensor *       q_out,
                                               shp_tensor *       k_cache,
                                               shp_tensor *       v_cache,
                                               const shp_tensor * slot,
                                               shp_tensor *       status,
                                               shp_stream_t       stream) {
    if (!shp::well_formed(k) || !shp::well_formed(v) || k_cache == nullptr || v_cache == nullptr ||
        !shp::well_formed(slot) || slot->type != SHP_TYPE_I32 || shp::nelements(*slot) != 1 ||
        (status != nullptr && (!shp::well_formed(status) || status->type != SHP_TYPE_I32 ||
                               shp::nelements(*status) != 1))) {
        return SHP_ERR_INVALID_ARG;
    }
    if (!shp::i32_aligned(*slot) || (status != nullptr && !shp::i32_aligned(*status))) {
        return SHP_ERR_UNSUPPORTED;
    }
    // The views start at row 0 and must fit T rows; the device slot moves them.
    shp_tensor kview{}, vview{};
    if (!shp::cache_view(k_cache, k, 0, kview) || !shp::cache_view(v_cache, v, 0, vview)) {
        return SHP_ERR_INVALID_ARG;
    }
    const int64_t cap = k_cache->ne[2] < v_cache->ne[2] ? k_cache->ne[2] : v_cache->ne[2];
    return shp::rope_entry(q, k, v, wq, wk, true, eps, pos, n_dims, freq_base, freq_scale, 1.0f, q_out, &kview, &vview,
                           stream, static_cast<const int32_t *>(slot->data),
                           status != nullptr ? static_cast<int32_t *>(status->data) : nullptr, cap);
}

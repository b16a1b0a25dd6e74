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
// Layout: a row (ne0 contiguous floats) is owned by a group of LPR lanes; each
// lane holds VPL float4 of it in registers between the reduction and the
// scaled store, so x is read from HBM once.

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

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__device__ __forceinline__ double sq4(float4 v) {
    // Each square is an f32 product; the accumulation is double, in element order.
    double acc = static_cast<double>(v.x * v.x);
    acc += static_cast<double>(v.y * v.y);
    acc += static_cast<double>(v.z * v.z);
    acc += static_cast<double>(v.w * v.w);
    return acc;
}

__device__ __forceinline__ float norm_scale(double sum, int32_t ne0, float eps) {
    const float mean = static_cast<float>(sum / static_cast<double>(ne0));
    return 1.0f / __builtin_sqrtf(mean + eps);
}

template <int LPR, int VPL, int WT, int MODE> __global__ __launch_bounds__(256) void k_rms_norm_vec(const NormArgs a) {
    constexpr int kRowsPerBlock = 256 / LPR;
    const int     l             = threadIdx.x % LPR;
    const int64_t row           = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / LPR;
    if (row >= a.nrows) {
        return;  // the whole LPR-lane group of this row leaves together
    }
    const float4 * xp = reinterpret_cast<const float4 *>(reinterpret_cast<const char *>(a.x) + row_offset(a.xm, row));
    float4         v[VPL];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        v[k] = xp[k * LPR + l];
    }
    // The gains are loaded with the row, not after the reduction, so the kernel
    // waits on one memory round trip, not two.
    float4 wv[VPL];
    if constexpr (WT != kWNone) {
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            wv[k] = load_w4<WT>(a.w, static_cast<int64_t>(k * LPR + l) * 4);
        }
    }
    if constexpr (MODE != kPlain) {
        const float4 * bp =
            reinterpret_cast<const float4 *>(reinterpret_cast<const char *>(a.b) + row_offset(a.bm, row));
        float4 bv[VPL];
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            bv[k] = bp[k * LPR + l];
        }
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            v[k] = add4(v[k], bv[k]);
        }
        if constexpr (MODE == kAddSum) {
            float4 * sp = reinterpret_cast<float4 *>(reinterpret_cast<char *>(a.s) + row_offset(a.sm, row));
#pragma unroll
            for (int k = 0; k < VPL; ++k) {
                sp[k * LPR + l] = v[k];
            }
        }
    }
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        acc += sq4(v[k]);
    }
    acc               = group_sum<LPR>(acc);
    const float scale = norm_scale(acc, a.ne0, a.eps);
    float4 *    yp    = reinterpret_cast<float4 *>(reinterpret_cast<char *>(a.y) + row_offset(a.ym, row));
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        float4 o = make_float4(v[k].x * scale, v[k].y * scale, v[k].z * scale, v[k].w * scale);
        if constexpr (WT != kWNone) {
            o = make_float4(o.x * wv[k].x, o.y * wv[k].y, o.z * wv[k].z, o.w * wv[k].w);
        }
        yp[k * LPR + l] = o;
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

template <int WT, int MODE> shp_status_t launch_norm(const NormArgs & a, bool vec, hipStream_t stream) {
    if (vec) {
        const int ne0 = a.ne0;
        auto      go  = [&](auto kernel, int rows_per_block) {
            const int64_t blocks = (a.nrows + rows_per_block - 1) / rows_per_block;
            hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
            return launch_status();
        };
        switch (ne0) {
            case 64:
                return go(k_rms_norm_vec<16, 1, WT, MODE>, 16);
            case 128:
                return go(k_rms_norm_vec<32, 1, WT, MODE>, 8);
            case 256:
                return go(k_rms_norm_vec<64, 1, WT, MODE>, 4);
            case 512:
                return go(k_rms_norm_vec<64, 2, WT, MODE>, 4);
            case 1024:
                return go(k_rms_norm_vec<64, 4, WT, MODE>, 4);
            case 2048:
                return go(k_rms_norm_vec<64, 8, WT, MODE>, 4);
            case 3072:
                return go(k_rms_norm_vec<64, 12, WT, MODE>, 4);
            case 4096:
                return go(k_rms_norm_vec<64, 16, WT, MODE>, 4);
            default:
                break;
        }
    }
    const int64_t blocks = (a.nrows + 3) / 4;
    hipLaunchKernelGGL((k_rms_norm_generic<WT, MODE>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
    return launch_status();
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
    bool vec   = a->ne[0] % 4 == 0 && rows_aligned(*a, 16) && rows_aligned(*y, 16) &&
               (w == nullptr || reinterpret_cast<uintptr_t>(w->data) % 8 == 0);
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
    RopePart        part[2];
    const int32_t * pos;
    int64_t         npos;
    int32_t         ne0;
    int32_t         n_dims;
    float           theta_scale;
    float           freq_scale;
    float           attn_factor;
    float           eps;
    int32_t         ppb;  // fast path: positions per block
    int32_t         pad;
};

// cos/sin of the pair-k angle at position p: theta is replayed through the f32
// recurrence theta <- theta*theta_scale exactly k times (the CPU cache's order),
// then cos/sin are evaluated in double and rounded once to f32, then scaled by
// attn_factor in f32 as the CPU cache does.
__device__ __forceinline__ void rope_cs(int32_t p, int k, const RopeArgs & a, float & c, float & s) {
    float theta = static_cast<float>(p);
    for (int i = 0; i < k; ++i) {
        theta = theta * a.theta_scale;
    }
    const float th = a.freq_scale * theta;
    float       sf, cf;
    if (!sincos_f32_rn(th, sf, cf)) {
        double sd, cd;  // beyond the fast reduction's range (|angle| > 2^19 pi/2)
        sincos(static_cast<double>(th), &sd, &cd);
        sf = static_cast<float>(sd);
        cf = static_cast<float>(cd);
    }
    c = cf * a.attn_factor;
    s = sf * a.attn_factor;
}

// Fast path: head_dim == n_dims == 128.
//
// A head row is owned by 16 lanes; lane j holds x[4j..4j+3] and
// x[64+4j..64+4j+3] as two float4, i.e. both halves of NEOX pairs 4j..4j+3,
// so the rotation needs no data exchange and every load is 128-bit. A block
// (16 row slots) covers `ppb` consecutive positions; each slot prefetches up
// to kRopeRows of its rows before anything waits, while the block builds the
// positions' 64-entry cos/sin caches in LDS.
constexpr int kRopeLanes    = 16;
constexpr int kRopeSlots    = 256 / kRopeLanes;
constexpr int kRopeRows     = 4;
constexpr int kRopeMaxPos   = 4;

template <bool NORM, int WT> __global__ __launch_bounds__(256) void k_rope128(const RopeArgs a) {
    __shared__ float s_cos[kRopeMaxPos][64];
    __shared__ float s_sin[kRopeMaxPos][64];

    const int64_t p0    = static_cast<int64_t>(blockIdx.x) * a.ppb;
    const int     np    = static_cast<int>(a.npos - p0 < a.ppb ? a.npos - p0 : a.ppb);
    const int     total = a.part[0].heads + a.part[1].heads;
    const int     nrows = np * total;
    const int     slot  = threadIdx.x / kRopeLanes;
    const int     l     = threadIdx.x % kRopeLanes;

    auto locate = [&](int row, int & pp, const float *& xr, float *& yr, int & t) {
        pp               = row / total;
        const int hh     = row - pp * total;
        t                = hh < a.part[0].heads ? 0 : 1;
        const int h      = t == 0 ? hh : hh - a.part[0].heads;
        const RopePart & P = a.part[t];
        const int64_t    pi = p0 + pp;
        xr = reinterpret_cast<const float *>(reinterpret_cast<const char *>(P.x) + h * P.xnb1 + pi * P.xnb2);
        yr = reinterpret_cast<float *>(reinterpret_cast<char *>(P.y) + h * P.ynb1 + pi * P.ynb2);
    };

    // Both heads' gains for this lane's eight elements, loaded once up front.
    float4 wlo[2] = { make_float4(1.f, 1.f, 1.f, 1.f), make_float4(1.f, 1.f, 1.f, 1.f) };
    float4 whi[2] = { wlo[0], wlo[0] };
    if constexpr (NORM && WT != kWNone) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (a.part[t].heads > 0) {
                wlo[t] = load_w4<WT>(a.part[t].w, 4 * l);
                whi[t] = load_w4<WT>(a.part[t].w, 64 + 4 * l);
            }
        }
    }

    auto finish = [&](int pp, float4 lo, float4 hi, float * yr, int t) {
        if constexpr (NORM) {
            double acc        = sq4(lo) + sq4(hi);
            acc               = group_sum<kRopeLanes>(acc);
            const float scale = norm_scale(acc, 128, a.eps);
            lo = make_float4(lo.x * scale, lo.y * scale, lo.z * scale, lo.w * scale);
            hi = make_float4(hi.x * scale, hi.y * scale, hi.z * scale, hi.w * scale);
            if constexpr (WT != kWNone) {
                const float4 wl = t == 0 ? wlo[0] : wlo[1];
                const float4 wh = t == 0 ? whi[0] : whi[1];
                lo = make_float4(lo.x * wl.x, lo.y * wl.y, lo.z * wl.z, lo.w * wl.w);
                hi = make_float4(hi.x * wh.x, hi.y * wh.y, hi.z * wh.z, hi.w * wh.w);
            }
        }
        const float * cs = s_cos[pp] + 4 * l;
        const float * sn = s_sin[pp] + 4 * l;
        float4        olo, ohi;
        olo.x = lo.x * cs[0] - hi.x * sn[0];
        ohi.x = lo.x * sn[0] + hi.x * cs[0];
        olo.y = lo.y * cs[1] - hi.y * sn[1];
        ohi.y = lo.y * sn[1] + hi.y * cs[1];
        olo.z = lo.z * cs[2] - hi.z * sn[2];
        ohi.z = lo.z * sn[2] + hi.z * cs[2];
        olo.w = lo.w * cs[3] - hi.w * sn[3];
        ohi.w = lo.w * sn[3] + hi.w * cs[3];
        reinterpret_cast<float4 *>(yr)[l]      = olo;
        reinterpret_cast<float4 *>(yr + 64)[l] = ohi;
    };

    // 1. issue every prefetched row load of this slot
    float4  lo[kRopeRows], hi[kRopeRows];
    int     pps[kRopeRows];
    int     ts[kRopeRows];
    float * yrs[kRopeRows];
#pragma unroll
    for (int r = 0; r < kRopeRows; ++r) {
        const int row = slot + r * kRopeSlots;
        pps[r]        = 0;
        ts[r]         = 0;
        yrs[r]        = nullptr;
        if (row < nrows) {
            const float * xr;
            locate(row, pps[r], xr, yrs[r], ts[r]);
            lo[r] = reinterpret_cast<const float4 *>(xr)[l];
            hi[r] = reinterpret_cast<const float4 *>(xr + 64)[l];
        }
    }
    // 2. the positions' cos/sin caches, meanwhile: lane 0 of wave pp replays
    //    position pp's f32 theta recurrence (inherently serial), then 64 lanes
    //    per position evaluate cos/sin in parallel.
    if (threadIdx.x % kWave == 0 && static_cast<int>(threadIdx.x / kWave) < np) {
        const int pp = threadIdx.x / kWave;
        float     th = static_cast<float>(a.pos[p0 + pp]);
#pragma unroll
        for (int k = 0; k < 64; ++k) {
            s_sin[pp][k] = a.freq_scale * th;  // angle k, overwritten by its sine below
            th           = th * a.theta_scale;
        }
    }
    __syncthreads();
    float cv = 0.0f, sv = 0.0f;
    const int epp = threadIdx.x / 64, ek = threadIdx.x % 64;
    if (epp < np) {
        const float th = s_sin[epp][ek];
        if (!sincos_f32_rn(th, sv, cv)) {
            double sd, cd;
            sincos(static_cast<double>(th), &sd, &cd);
            sv = static_cast<float>(sd);
            cv = static_cast<float>(cd);
        }
    }
    __syncthreads();
    if (epp < np) {
        s_cos[epp][ek] = cv * a.attn_factor;
        s_sin[epp][ek] = sv * a.attn_factor;
    }
    __syncthreads();
    // 3. normalise, rotate, store
#pragma unroll
    for (int r = 0; r < kRopeRows; ++r) {
        if (slot + r * kRopeSlots < nrows) {
            finish(pps[r], lo[r], hi[r], yrs[r], ts[r]);
        }
    }
    // rows past the prefetch window (only when a position has > 64 head rows)
    for (int row = slot + kRopeRows * kRopeSlots; row < nrows; row += kRopeSlots) {
        int           pp, t;
        const float * xr;
        float *       yr;
        locate(row, pp, xr, yr, t);
        finish(pp, reinterpret_cast<const float4 *>(xr)[l], reinterpret_cast<const float4 *>(xr + 64)[l], yr, t);
    }
}

// Any head_dim / n_dims: one wave per head row; the theta recurrence is
// replayed per pair (fine for the small shapes that take this path).
template <bool NORM, int WT> __global__ __launch_bounds__(256) void k_rope_generic(const RopeArgs a) {
    const int     lane  = threadIdx.x % kWave;
    const int     total = a.part[0].heads + a.part[1].heads;
    const int64_t row   = static_cast<int64_t>(blockIdx.x) * (256 / kWave) + threadIdx.x / kWave;
    if (row >= a.npos * total) {
        return;
    }
    const int64_t    pi = row / total;
    const int        hh = static_cast<int>(row % total);
    const int        t  = hh < a.part[0].heads ? 0 : 1;
    const int        h  = t == 0 ? hh : hh - a.part[0].heads;
    const RopePart & P  = a.part[t];
    const float *    xr = reinterpret_cast<const float *>(reinterpret_cast<const char *>(P.x) + h * P.xnb1 + pi * P.xnb2);
    float *          yr = reinterpret_cast<float *>(reinterpret_cast<char *>(P.y) + h * P.ynb1 + pi * P.ynb2);
    const int32_t    p  = a.pos[pi];

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
                v = v * load_w1<WT>(P.w, i);
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

template <bool NORM, int WT> shp_status_t launch_rope(const RopeArgs & a, bool fast, hipStream_t stream) {
    const int total = a.part[0].heads + a.part[1].heads;
    if (fast) {
        const int64_t blocks = (a.npos + a.ppb - 1) / a.ppb;
        hipLaunchKernelGGL((k_rope128<NORM, WT>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
        return launch_status();
    }
    const int64_t rows   = a.npos * total;
    const int64_t blocks = (rows + 3) / 4;
    hipLaunchKernelGGL((k_rope_generic<NORM, WT>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
    return launch_status();
}

template <bool NORM> shp_status_t dispatch_rope_w(const RopeArgs & a, int wk, bool fast, hipStream_t stream) {
    switch (wk) {
        case kWNone:
            return launch_rope<NORM, kWNone>(a, fast, stream);
        case kWF32:
            return launch_rope<NORM, kWF32>(a, fast, stream);
        case kWBF16:
            return launch_rope<NORM, kWBF16>(a, fast, stream);
        case kWF16:
            return launch_rope<NORM, kWF16>(a, fast, stream);
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

// float4 gain loads: 16-byte aligned F32, 8-byte aligned BF16/F16.
bool gain_aligned(const shp_tensor * w) {
    return w == nullptr || reinterpret_cast<uintptr_t>(w->data) % (w->type == SHP_TYPE_F32 ? 16 : 8) == 0;
}

shp_status_t rope_entry(const shp_tensor * q,
                        const shp_tensor * k,
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
                        shp_stream_t       stream) {
    if (!rope_part_ok(q, q_out) || !well_formed(pos) || pos->type != SHP_TYPE_I32) {
        return SHP_ERR_INVALID_ARG;
    }
    if ((k == nullptr) != (k_out == nullptr)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (k != nullptr && (!rope_part_ok(k, k_out) || k->ne[0] != q->ne[0] || k->ne[2] != q->ne[2])) {
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
    if (q->ne[1] + (k != nullptr ? k->ne[1] : 0) > INT32_MAX) {
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
    a.pos         = static_cast<const int32_t *>(pos->data);
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
    if (norm) {
        fast = fast && gain_aligned(wq) && gain_aligned(wk);
    }
    // Positions per block: fill the 16 row slots x kRopeRows prefetch window.
    // Short sequences are latency-bound: one position per block spreads them
    // over more CUs.
    const int total = static_cast<int>(a.part[0].heads + a.part[1].heads);
    a.ppb           = total > 0 ? (kRopeSlots * kRopeRows) / total : 1;
    a.ppb           = a.ppb < 1 ? 1 : (a.ppb > kRopeMaxPos ? kRopeMaxPos : a.ppb);
    if (a.npos < 2048) {
        a.ppb = 1;
    }
    if (a.npos > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    const hipStream_t st = as_stream(stream);
    return norm ? dispatch_rope_w<true>(a, wkind, fast, st) : dispatch_rope_w<false>(a, kWNone, fast, st);
}

}  // namespace
}  // namespace shp

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
    return shp::rope_entry(x, nullptr, nullptr, nullptr, false, 0.0f, pos, n_dims, freq_base, freq_scale, attn_factor,
                           y, nullptr, stream);
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
    return shp::rope_entry(q, k, wq, wk, true, eps, pos, n_dims, freq_base, freq_scale, 1.0f, q_out, k_out, stream);
}

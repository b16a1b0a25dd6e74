// ggml_soft_max_ext(a, mask, scale, max_bias = 0) for gfx950: the attention
// softmax of src/arch/qwen3-tts/operations.cpp:131-133 (scores over the cached
// keys, scaled by 1/sqrt(head_dim), causal mask).
//
// Per row, in ggml-CPU's rounding order:
//   w_i  = x_i*scale + 1*mask_i          (f32; the slope is 1 without ALiBi)
//   m    = max_i w_i
//   v_i  = exp(w_i - m)                  (f32 difference, exp rounded to f32)
//   sum  = sum_i (double) v_i            (double)
//   y_i  = v_i * (float)(1/sum)          (the reciprocal in double, rounded to f32)
// The exp is shp_expf.hpp's table-driven exp, within ~2^-44 before its f32
// rounding: it differs from the correctly rounded exp on 19 of the 2^32 f32
// inputs, glibc's expf (the CPU's) on 170,648. The double sum is added in a
// different order than the CPU's loop, which moves the f32 reciprocal only
// when the sum lies within ~1e-16 of a rounding boundary. A row holding a NaN
// or +inf (or only -inf) comes out NaN, as on the CPU: the max is then NaN or
// inf, or the NaN reaches the sum.
//
// Launch shapes: rows up to 2048 wide are held in registers. With float4
// rows, a row takes one wave (wave-level reductions only: no LDS, no barrier)
// when there are enough rows to fill the chip, else 2 or 4 waves (the decode
// step's 16 rows of ~512, a short prefill's 1024 rows of 2048); other rows
// take one wave each with scalar accesses. Wider rows take one 256-thread
// block per row and three passes over the row.

#include <cmath>

#include "shp_expf.hpp"
#include "shp_internal.hpp"

namespace shp {
namespace {

struct SoftMaxArgs {
    const float * x;
    RowMap        xm;
    const float * mask;  // null: no mask
    int64_t       mnb1;
    int64_t       mnb2;
    int64_t       mnb3;
    int64_t       mne2;  // mask heads (broadcast: head i2 reads mask head i2 % mne2)
    int64_t       mne3;
    float *       y;
    RowMap        ym;
    int64_t       nrows;
    int64_t       ne1;   // rows per head
    int64_t       ne2;   // heads
    int32_t       ne0;
    float         scale;
    // Every row index and mask extent below 2^32: the mask row's indices come
    // from multiply-shift divisions (FastDiv) instead of 64-bit divisions.
    int32_t       mfast;
    int32_t       pad;
    int64_t       n_past;  // causal form: element i of row r is masked when i > n_past + r % ne1
    FastDiv       fne1;
    FastDiv       fne2;
    FastDiv       fmne2;
    FastDiv       fmne3;
};

// Mask forms: none, a mask tensor added to the scaled scores, or the causal
// mask of ggml_diag_mask_inf in front of the softmax (the masked scores
// replaced by -inf before the scale, as the two nodes compute them: a masked
// +inf or NaN score drops out instead of turning the row into NaN).
enum MaskKind { kMaskNone = 0, kMaskTensor = 1, kMaskCausal = 2 };

constexpr int kSoftMaxWaveMax = 2048;  // widest row of the one-wave kernel
constexpr int kSoftMaxBlock   = 256;

// exp with the table read from memory (divergent loops).
__device__ __forceinline__ float exp_f32(float x) {
    return exp_f32_rn(x, [](int j) { return kExpTable[j]; });
}

// Mask row of score row r = (i1, i2, i3): ggml's i11 = i1, i12 = i2 % ne12,
// i13 = i3 % ne13.
__device__ __forceinline__ const float * mask_row(const SoftMaxArgs & a, int64_t r) {
    if (a.mfast) {
        const uint32_t q  = fastdiv(static_cast<uint32_t>(r), a.fne1);
        const uint32_t i1 = static_cast<uint32_t>(r) - q * a.fne1.d;
        const uint32_t i3 = fastdiv(q, a.fne2);
        const uint32_t i2 = q - i3 * a.fne2.d;
        return reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.mask) + i1 * a.mnb1 +
                                               fastmod(i2, a.fmne2) * a.mnb2 + fastmod(i3, a.fmne3) * a.mnb3);
    }
    const int64_t i1 = r % a.ne1;
    const int64_t q  = r / a.ne1;
    const int64_t i2 = q % a.ne2;
    const int64_t i3 = q / a.ne2;
    return reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.mask) + i1 * a.mnb1 +
                                           (i2 % a.mne2) * a.mnb2 + (i3 % a.mne3) * a.mnb3);
}

// The causal form's last unmasked element of row r: n_past + i1.
__device__ __forceinline__ int64_t causal_lim(const SoftMaxArgs & a, int64_t r) {
    if (a.mfast) {
        return a.n_past + fastmod(static_cast<uint32_t>(r), a.fne1);
    }
    return a.n_past + r % a.ne1;
}

// The kernel arguments a softmax wave needs before its first load.
template <int MK> __device__ __forceinline__ void softmax_args_in_sgprs(const SoftMaxArgs & a) {
    args_in_sgprs(a.x, a.xm.flat, a.xm.rs, a.y, a.ym.flat, a.ym.rs, a.nrows, a.ne0, a.scale);
    if constexpr (MK == kMaskTensor) {
        args_in_sgprs(a.mask, a.mfast, a.fne1.d, a.fne1.m, a.fne1.l, a.fne2.d, a.fne2.m, a.fne2.l, a.fmne2.d,
                      a.fmne2.m, a.fmne2.l, a.fmne3.d, a.fmne3.m, a.fmne3.l, a.mnb1, a.mnb2, a.mnb3);
    }
}

// One wave per row, element lane + 64k in register k (k < K, 64K >= ne0).
template <int K, int MK> __global__ __launch_bounds__(256) void k_soft_max_wave(const SoftMaxArgs a) {
    constexpr bool MASK = MK == kMaskTensor;
    __shared__ double s_tab[256 / kWave][64];
    softmax_args_in_sgprs<MK>(a);
    const int     lane = threadIdx.x % kWave;
    const int64_t r    = static_cast<int64_t>(blockIdx.x) * (256 / kWave) +
                      __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    if (r >= a.nrows) {
        return;  // whole wave
    }
    const float * xr = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.x) + row_offset(a.xm, r));
    float *       yr = reinterpret_cast<float *>(reinterpret_cast<char *>(a.y) + row_offset(a.ym, r));
    const float * mr  = MASK ? mask_row(a, r) : nullptr;
    const int64_t lim = MK == kMaskCausal ? causal_lim(a, r) : 0;
    float         w[K];
    float         mk[K];
    // The exp table's entry is loaded with the row. Loads are unconditional
    // (a lane past the row re-reads element 0) and out-of-row values are
    // zeroed by selects afterwards: a guarded load becomes a branch with a
    // wait of its own.
    const double entry = exp_table_entry(lane);
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = lane + kWave * k;
        w[k]        = xr[i < a.ne0 ? i : 0];
        mk[k]       = MASK ? mr[i < a.ne0 ? i : 0] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const bool in = lane + kWave * k < a.ne0;
        w[k]          = in ? w[k] : 0.0f;
        mk[k]         = in ? mk[k] : 0.0f;
    }
    const double * tab = wave_exp_table(s_tab, lane, entry);
    float          mx  = -INFINITY;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = lane + kWave * k;
        w[k]        = w[k] * a.scale;
        if constexpr (MASK) {
            w[k] = w[k] + mk[k];
        }
        if constexpr (MK == kMaskCausal) {
            w[k] = i > lim ? -INFINITY : w[k];
        }
        mx = i < a.ne0 ? fmaxf(mx, w[k]) : mx;
    }
    mx         = wave_max(mx);
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = lane + kWave * k;
        w[k]        = exp_f32_lds(w[k] - mx, tab);
        sum += i < a.ne0 ? static_cast<double>(w[k]) : 0.0;
    }
    sum             = group_sum<kWave>(sum);
    const float inv = static_cast<float>(1.0 / sum);
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = lane + kWave * k;
        if (i < a.ne0) {
            yr[i] = w[k] * inv;
        }
    }
}

// float4 rows (16-byte aligned rows, ne0 % 4 == 0), WPR waves per row: lane q
// of the row's 64*WPR lanes holds chunks q + 64*WPR*k in registers k (k < K4).
// The scores are read and the probabilities written once per launch, so both
// stream with the nontemporal hint (the mask, shared by heads, stays
// cacheable): 21 % faster than plain loads and stores at [512,512,16] on
// MI355X (9.65 -> 7.58 us).
// WPR > 1 spreads the few long rows of a decode or short prefill over more
// waves; the row's waves then combine their max and sum through LDS, in wave
// order.
template <int WPR, int K4, int MK, int BLOCK = 256>
__global__ __launch_bounds__(BLOCK) void k_soft_max_rows4(const SoftMaxArgs a) {
    constexpr bool MASK   = MK == kMaskTensor;
    constexpr int  kLanes = kWave * WPR;
    __shared__ float  s_max[BLOCK / kWave];
    __shared__ double s_sum[BLOCK / kWave];
    __shared__ double s_tab[BLOCK / kWave][64];
    softmax_args_in_sgprs<MK>(a);
    const int     lane = threadIdx.x % kWave;
    const int     q    = threadIdx.x % kLanes;
    const int     wv   = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int     slot = wv / WPR;  // row of this block
    const int64_t r    = static_cast<int64_t>(blockIdx.x) * (BLOCK / kLanes) + slot;
    const bool    live = r < a.nrows;
    if (WPR == 1 && !live) {
        return;  // whole wave; the one-wave form has no barrier
    }
    const int64_t rr = live ? r : 0;
    const f32x4 * xr =
        reinterpret_cast<const f32x4 *>(reinterpret_cast<const char *>(a.x) + row_offset(a.xm, rr));
    f32x4 *       yr    = reinterpret_cast<f32x4 *>(reinterpret_cast<char *>(a.y) + row_offset(a.ym, rr));
    const f32x4 * mr    = MASK ? reinterpret_cast<const f32x4 *>(mask_row(a, rr)) : nullptr;
    const int64_t lim   = MK == kMaskCausal ? causal_lim(a, rr) : 0;
    const int     n4 = live ? a.ne0 / 4 : 0;
    f32x4         w[K4];
    f32x4         mk[K4];
    // The exp table's entry is loaded with the row, so it is not a round trip
    // of its own. Loads are unconditional (a lane past the row re-reads chunk
    // 0 of row rr), zeroed by selects afterwards: a guarded load becomes a
    // branch with a wait of its own.
    const double entry = exp_table_entry(lane);
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        const int c = q + kLanes * k;
        w[k]        = ld_stream(xr + (c < n4 ? c : 0));
        mk[k]       = MASK ? mr[c < n4 ? c : 0] : splat4(0.0f);
    }
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        const bool in = q + kLanes * k < n4;
        w[k]          = in ? w[k] : splat4(0.0f);
        mk[k]         = in ? mk[k] : splat4(0.0f);
    }
    const double * tab = wave_exp_table(s_tab, lane, entry);
    float          mx  = -INFINITY;
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        const int c = q + kLanes * k;
        w[k]        = f32x4{ w[k].x * a.scale, w[k].y * a.scale, w[k].z * a.scale, w[k].w * a.scale };
        if constexpr (MASK) {
            w[k] = f32x4{ w[k].x + mk[k].x, w[k].y + mk[k].y, w[k].z + mk[k].z, w[k].w + mk[k].w };
        }
        if constexpr (MK == kMaskCausal) {
            const int64_t i = static_cast<int64_t>(c) * 4;
            w[k]            = f32x4{ i > lim ? -INFINITY : w[k].x, i + 1 > lim ? -INFINITY : w[k].y,
                                     i + 2 > lim ? -INFINITY : w[k].z, i + 3 > lim ? -INFINITY : w[k].w };
        }
        const float m4 = fmaxf(fmaxf(w[k].x, w[k].y), fmaxf(w[k].z, w[k].w));
        mx             = c < n4 ? fmaxf(mx, m4) : mx;
    }
    mx = wave_max(mx);
    if constexpr (WPR > 1) {
        if (lane == 0) {
            s_max[wv] = mx;
        }
        __syncthreads();
        mx = s_max[slot * WPR];
#pragma unroll
        for (int j = 1; j < WPR; ++j) {
            mx = fmaxf(mx, s_max[slot * WPR + j]);
        }
    }
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        const int c = q + kLanes * k;
        w[k] = f32x4{ exp_f32_lds(w[k].x - mx, tab), exp_f32_lds(w[k].y - mx, tab), exp_f32_lds(w[k].z - mx, tab),
                      exp_f32_lds(w[k].w - mx, tab) };
        const double s4 = (static_cast<double>(w[k].x) + static_cast<double>(w[k].y)) +
                          (static_cast<double>(w[k].z) + static_cast<double>(w[k].w));
        sum += c < n4 ? s4 : 0.0;
    }
    sum = group_sum<kWave>(sum);
    if constexpr (WPR > 1) {
        if (lane == 0) {
            s_sum[wv] = sum;
        }
        __syncthreads();
        sum = s_sum[slot * WPR];
#pragma unroll
        for (int j = 1; j < WPR; ++j) {
            sum += s_sum[slot * WPR + j];
        }
    }
    const float inv = static_cast<float>(1.0 / sum);
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        const int c = q + kLanes * k;
        if (c < n4) {
            st_stream(yr + c, f32x4{ w[k].x * inv, w[k].y * inv, w[k].z * inv, w[k].w * inv });
        }
    }
}

// One block per row, three passes: the max, the sum, the scaled exps.
template <int MK>
__device__ __forceinline__ float sm_w(const SoftMaxArgs & a, const float * xr, const float * mr, int64_t lim, int i) {
    float w = xr[i] * a.scale;
    if constexpr (MK == kMaskTensor) {
        w = w + mr[i];
    }
    if constexpr (MK == kMaskCausal) {
        w = i > lim ? -INFINITY : w;
    }
    return w;
}

template <int MK> __global__ __launch_bounds__(kSoftMaxBlock) void k_soft_max_block(const SoftMaxArgs a) {
    constexpr bool MASK = MK == kMaskTensor;
    __shared__ float  s_max[kSoftMaxBlock / kWave];
    __shared__ double s_sum[kSoftMaxBlock / kWave];
    const int64_t r    = blockIdx.x;
    const int     lane = threadIdx.x % kWave;
    const int     wv   = threadIdx.x / kWave;
    const float * xr   = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.x) + row_offset(a.xm, r));
    float *       yr   = reinterpret_cast<float *>(reinterpret_cast<char *>(a.y) + row_offset(a.ym, r));
    const float * mr   = MASK ? mask_row(a, r) : nullptr;
    const int64_t lim  = MK == kMaskCausal ? causal_lim(a, r) : 0;

    float mx = -INFINITY;
    for (int i = threadIdx.x; i < a.ne0; i += kSoftMaxBlock) {
        mx = fmaxf(mx, sm_w<MK>(a, xr, mr, lim, i));
    }
    mx = wave_max(mx);
    if (lane == 0) {
        s_max[wv] = mx;
    }
    __syncthreads();
    mx = s_max[0];
#pragma unroll
    for (int j = 1; j < kSoftMaxBlock / kWave; ++j) {
        mx = fmaxf(mx, s_max[j]);
    }

    double sum = 0.0;
    for (int i = threadIdx.x; i < a.ne0; i += kSoftMaxBlock) {
        sum += static_cast<double>(exp_f32(sm_w<MK>(a, xr, mr, lim, i) - mx));
    }
    sum = group_sum<kWave>(sum);
    if (lane == 0) {
        s_sum[wv] = sum;
    }
    __syncthreads();
    sum = s_sum[0];
#pragma unroll
    for (int j = 1; j < kSoftMaxBlock / kWave; ++j) {
        sum += s_sum[j];
    }
    const float inv = static_cast<float>(1.0 / sum);
    for (int i = threadIdx.x; i < a.ne0; i += kSoftMaxBlock) {
        yr[i] = exp_f32(sm_w<MK>(a, xr, mr, lim, i) - mx) * inv;
    }
}

template <int MK> shp_status_t launch_soft_max(const SoftMaxArgs & a, bool vec, hipStream_t stream) {
    if (dry_run()) {
        return SHP_OK;
    }
    if (a.ne0 > kSoftMaxWaveMax) {
        hipLaunchKernelGGL((k_soft_max_block<MK>), dim3(static_cast<unsigned>(a.nrows)), dim3(kSoftMaxBlock), 0,
                           stream, a);
        return launch_status();
    }
    const dim3 grid(static_cast<unsigned>((a.nrows + 3) / 4));
    if (vec) {
        // Few rows (under 8 waves per CU at one wave per row): 2 or 4 waves per
        // row. The decode step's 16 rows of 512 take one wave each (2.30 us
        // against 2.36 us with two waves and their LDS combine, MI355X), in
        // one-wave blocks: each row on its own CU (2.12 -> 1.99 us warm; the
        // 28-layer decode graph's layer with the softmax 9.62 -> 9.45 us).
        const int n4  = a.ne0 / 4;
        const int wpr = a.nrows >= 2048 ? 1 : (n4 >= 256 ? 4 : (n4 >= 128 && a.nrows > 64 ? 2 : 1));
        const int k4  = (n4 + kWave * wpr - 1) / (kWave * wpr);
        const dim3 g4(static_cast<unsigned>((a.nrows * wpr + 3) / 4));
        if (wpr == 4) {
            if (k4 <= 1) {
                hipLaunchKernelGGL((k_soft_max_rows4<4, 1, MK>), g4, dim3(256), 0, stream, a);
            } else {
                hipLaunchKernelGGL((k_soft_max_rows4<4, 2, MK>), g4, dim3(256), 0, stream, a);
            }
        } else if (wpr == 2) {
            if (k4 <= 1) {
                hipLaunchKernelGGL((k_soft_max_rows4<2, 1, MK>), g4, dim3(256), 0, stream, a);
            } else if (k4 <= 2) {
                hipLaunchKernelGGL((k_soft_max_rows4<2, 2, MK>), g4, dim3(256), 0, stream, a);
            } else {
                hipLaunchKernelGGL((k_soft_max_rows4<2, 4, MK>), g4, dim3(256), 0, stream, a);
            }
        } else if (k4 <= 1) {
            hipLaunchKernelGGL((k_soft_max_rows4<1, 1, MK>), g4, dim3(256), 0, stream, a);
        } else if (k4 <= 2 && a.nrows <= 64) {
            // a decode step's few rows: one one-wave block per row
            hipLaunchKernelGGL((k_soft_max_rows4<1, 2, MK, kWave>), dim3(static_cast<unsigned>(a.nrows)), dim3(kWave),
                               0, stream, a);
        } else if (k4 <= 2) {
            hipLaunchKernelGGL((k_soft_max_rows4<1, 2, MK>), g4, dim3(256), 0, stream, a);
        } else if (k4 <= 4) {
            hipLaunchKernelGGL((k_soft_max_rows4<1, 4, MK>), g4, dim3(256), 0, stream, a);
        } else {
            hipLaunchKernelGGL((k_soft_max_rows4<1, 8, MK>), g4, dim3(256), 0, stream, a);
        }
        return launch_status();
    }
    const int k = (a.ne0 + kWave - 1) / kWave;
    if (k <= 1) {
        hipLaunchKernelGGL((k_soft_max_wave<1, MK>), grid, dim3(256), 0, stream, a);
    } else if (k <= 2) {
        hipLaunchKernelGGL((k_soft_max_wave<2, MK>), grid, dim3(256), 0, stream, a);
    } else if (k <= 4) {
        hipLaunchKernelGGL((k_soft_max_wave<4, MK>), grid, dim3(256), 0, stream, a);
    } else if (k <= 8) {
        hipLaunchKernelGGL((k_soft_max_wave<8, MK>), grid, dim3(256), 0, stream, a);
    } else if (k <= 16) {
        hipLaunchKernelGGL((k_soft_max_wave<16, MK>), grid, dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL((k_soft_max_wave<32, MK>), grid, dim3(256), 0, stream, a);
    }
    return launch_status();
}

}  // namespace
}  // namespace shp

using namespace shp;

extern "C" shp_status_t shp_soft_max_ext(const shp_tensor * a,
                                         const shp_tensor * mask,
                                         float              scale,
                                         float              max_bias,
                                         shp_tensor *       y,
                                         shp_stream_t       stream) {
    if (!well_formed(a) || !well_formed(y) || (mask != nullptr && !well_formed(mask))) {
        return SHP_ERR_INVALID_ARG;
    }
    if (a->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32 || (mask != nullptr && mask->type != SHP_TYPE_F32)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (max_bias != 0.0f) {
        return SHP_ERR_UNSUPPORTED;  // ALiBi slopes: not on this path
    }
    if (!same_shape(*a, *y) || a->ne[0] > INT32_MAX || nrows(*a) > INT32_MAX) {
        return SHP_ERR_INVALID_ARG;
    }
    // ggml_soft_max_ext's mask contract: same row length, at least as many
    // rows, heads and batches broadcast by whole repeats.
    if (mask != nullptr && (mask->ne[0] != a->ne[0] || mask->ne[1] < a->ne[1] || a->ne[2] % mask->ne[2] != 0 ||
                            a->ne[3] % mask->ne[3] != 0)) {
        return SHP_ERR_INVALID_ARG;
    }
    SoftMaxArgs g{};
    g.x     = static_cast<const float *>(a->data);
    g.xm    = make_rowmap(*a);
    g.y     = static_cast<float *>(y->data);
    g.ym    = make_rowmap(*y);
    g.nrows = nrows(*a);
    g.ne1   = a->ne[1];
    g.ne2   = a->ne[2];
    g.ne0   = static_cast<int32_t>(a->ne[0]);
    g.scale = scale;
    if (mask != nullptr) {
        g.mask = static_cast<const float *>(mask->data);
        g.mnb1 = static_cast<int64_t>(mask->nb[1]);
        g.mnb2 = static_cast<int64_t>(mask->nb[2]);
        g.mnb3 = static_cast<int64_t>(mask->nb[3]);
        g.mne2 = mask->ne[2];
        g.mne3 = mask->ne[3];
        constexpr int64_t kU32 = int64_t{ UINT32_MAX };
        g.mfast = g.nrows <= kU32 && g.ne1 <= kU32 && g.ne2 <= kU32 && g.mne2 <= kU32 && g.mne3 <= kU32;
        if (g.mfast) {
            g.fne1  = make_fastdiv(static_cast<uint32_t>(g.ne1));
            g.fne2  = make_fastdiv(static_cast<uint32_t>(g.ne2));
            g.fmne2 = make_fastdiv(static_cast<uint32_t>(g.mne2));
            g.fmne3 = make_fastdiv(static_cast<uint32_t>(g.mne3));
        }
    }
    // float4 rows: every row start of the scores, the output and the mask
    // 16-byte aligned and whole float4s per row
    const bool vec = a->ne[0] % 4 == 0 && rows_aligned(*a, 16) && rows_aligned(*y, 16) &&
                     (mask == nullptr || rows_aligned(*mask, 16));
    return mask != nullptr ? launch_soft_max<kMaskTensor>(g, vec, as_stream(stream))
                           : launch_soft_max<kMaskNone>(g, vec, as_stream(stream));
}

// ggml_diag_mask_inf(x, n_past): every element past n_past + its row's index
// in the matrix (i0 > n_past + i1) becomes -inf, the rest copied.
struct DiagMaskArgs {
    const float * x;
    RowMap        xm;
    float *       y;
    RowMap        ym;
    int64_t       n_past;
    int64_t       ne1;
    int64_t       total;  // rows x ne0
    FastDiv       fne0;
    FastDiv       fne1;
};

__global__ __launch_bounds__(256) void k_diag_mask_inf(const DiagMaskArgs a) {
    const int64_t step = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; t < a.total; t += step) {
        const uint32_t r  = fastdiv(static_cast<uint32_t>(t), a.fne0);
        const uint32_t i0 = static_cast<uint32_t>(t) - r * a.fne0.d;
        const uint32_t i1 = fastmod(r, a.fne1);
        const float *  xr = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.x) + row_offset(a.xm, r));
        float *        yr = reinterpret_cast<float *>(reinterpret_cast<char *>(a.y) + row_offset(a.ym, r));
        yr[i0]            = static_cast<int64_t>(i0) > a.n_past + i1 ? -INFINITY : xr[i0];
    }
}

extern "C" shp_status_t shp_diag_mask_inf(const shp_tensor * x, int32_t n_past, shp_tensor * y, shp_stream_t stream) {
    if (!well_formed(x) || !well_formed(y) || n_past < 0) {
        return SHP_ERR_INVALID_ARG;
    }
    if (x->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (!same_shape(*x, *y) || nelements(*x) > INT32_MAX) {
        return SHP_ERR_INVALID_ARG;
    }
    const bool in_place = x->data == y->data && x->nb[1] == y->nb[1] && x->nb[2] == y->nb[2] && x->nb[3] == y->nb[3];
    if (!in_place && spans_overlap(*x, *y)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (dry_run()) {
        return SHP_OK;
    }
    DiagMaskArgs g{};
    g.x                  = static_cast<const float *>(x->data);
    g.xm                 = make_rowmap(*x);
    g.y                  = static_cast<float *>(y->data);
    g.ym                 = make_rowmap(*y);
    g.n_past             = n_past;
    g.ne1                = x->ne[1];
    g.total              = nelements(*x);
    g.fne0               = make_fastdiv(static_cast<uint32_t>(x->ne[0]));
    g.fne1               = make_fastdiv(static_cast<uint32_t>(x->ne[1]));
    const int64_t blocks = (g.total + 255) / 256;
    hipLaunchKernelGGL(k_diag_mask_inf, dim3(static_cast<unsigned>(blocks < (1 << 20) ? blocks : (1 << 20))),
                       dim3(256), 0, as_stream(stream), g);
    return launch_status();
}

extern "C" shp_status_t shp_soft_max_causal(const shp_tensor * a,
                                            int32_t            n_past,
                                            float              scale,
                                            shp_tensor *       y,
                                            shp_stream_t       stream) {
    if (!well_formed(a) || !well_formed(y) || n_past < 0) {
        return SHP_ERR_INVALID_ARG;
    }
    if (a->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    // -inf times the scale is -inf only for a positive finite scale
    if (!(scale > 0.0f) || !(scale < INFINITY)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (!same_shape(*a, *y) || a->ne[0] > INT32_MAX || nrows(*a) > INT32_MAX) {
        return SHP_ERR_INVALID_ARG;
    }
    SoftMaxArgs g{};
    g.x      = static_cast<const float *>(a->data);
    g.xm     = make_rowmap(*a);
    g.y      = static_cast<float *>(y->data);
    g.ym     = make_rowmap(*y);
    g.nrows  = nrows(*a);
    g.ne1    = a->ne[1];
    g.ne2    = a->ne[2];
    g.ne0    = static_cast<int32_t>(a->ne[0]);
    g.scale  = scale;
    g.n_past = n_past;
    g.mfast  = 1;  // rows below 2^31
    g.fne1   = make_fastdiv(static_cast<uint32_t>(g.ne1));
    const bool vec = a->ne[0] % 4 == 0 && rows_aligned(*a, 16) && rows_aligned(*y, 16);
    return launch_soft_max<kMaskCausal>(g, vec, as_stream(stream));
}

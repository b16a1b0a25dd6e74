// Elementwise primitives for gfx950: SwiGLU (silu(g)*u), bare silu, the
// single-tensor GLU, the Snake family (Kokoro's Snake, the guarded Snake and
// SnakeBeta), add->leaky-ReLU with the residual carried out, bare leaky-ReLU,
// the branch average sum->scale->leaky-ReLU, exp, scale/scale_bias and the
// plain residual add.
//
// Each fused op reproduces the f32 rounding sequence of the unfused ggml node
// run it replaces (compiled with -ffp-contract=off, IEEE divide), so the only
// difference from ggml-CPU can be the last ulp of a transcendental.
//
// Two launch shapes: a flat kernel for fully contiguous, 16-byte aligned
// tensors (the large vocoder and MLP tensors), one float4 per lane per operand;
// and a row kernel that follows ggml byte strides for any other view. Both
// stream activations with nontemporal loads and stores.

#include <cmath>
#include <type_traits>

#include "shp_div.hpp"
#include "shp_expf.hpp"
#include "shp_internal.hpp"
#include "shp_sinf.hpp"

namespace shp {
namespace {

enum EwOp {
    kSwiglu    = 0,
    kSilu      = 1,
    kAdd       = 2,
    kAddLeaky  = 3,
    kLeaky     = 4,
    kExp       = 5,
    kScale     = 6,
    kScaleBias = 7,
    kMul       = 8,
    kDiv       = 9,
    kSin       = 10,
    kSqr       = 11,
    kCopy      = 12,
    kSub       = 13,
    kTanh      = 14,
    kSigmoid   = 15,
    kElu       = 16,
    kGeluErf   = 17,
    kClamp     = 18,
    kRelu      = 19,
    kNeg       = 20,
    kStep      = 21,
    kSqrt      = 22
};

// Snake family: y = x + sin(x*al)^2 / den with per-channel al and den.
//   kSnakePlain   (kokoro/operations.cpp:137-147):   al = den = alpha
//   kSnakeGuarded (omnivoice/codec.cpp:51-68):        al = alpha, den = alpha + 1e-9
//   kSnakeBeta    (qwen3-tts/codec.cpp:184-199):      al = exp(log_alpha), den = exp(log_beta) + 1e-9
enum SnakeKind { kSnakePlain = 0, kSnakeGuarded = 1, kSnakeBeta = 2 };

// The fixed guard of Snake1d/SnakeBeta, added by ggml_scale_bias(c, 1.0f, 1e-9f).
constexpr float kSnakeGuard = 1e-9f;

struct EwArgs {
    const float * a;
    RowMap        am;
    const float * b;
    RowMap        bm;
    float *       y;
    RowMap        ym;
    float *       s;
    RowMap        sm;
    const float * alpha;   // Snake: first per-channel curve
    const float * beta;    // SnakeBeta: second per-channel curve
    int64_t       nrows;
    int64_t       n4;
    int32_t       ne0;
    FastDiv       period;  // flat path: row length, to index a broadcast row (alpha or b)
    FastDiv       quads;   // Snake flat path: float4 per row (ne0/4)
    int64_t       ntask;   // Snake flat path: lanes = row blocks x quads per row
    float         slope;
    float         scale;  // kScale / kScaleBias
    float         bias;   // kScaleBias
    int32_t       pad;
};

__device__ __forceinline__ float silu(float x) {
    return x / (1.0f + expf(-x));
}

// ggml's leaky: (x > 0 ? x : 0) + slope * (x < 0 ? x : 0), so -0 and NaN give +0.
__device__ __forceinline__ float leaky(float x, float slope) {
    const float pos = x > 0.0f ? x : 0.0f;
    const float neg = x < 0.0f ? x : 0.0f;
    return pos + slope * neg;
}

// e^x rounded to f32 from a double evaluation within ~2^-44 (shp_expf.hpp): it
// differs from the correctly rounded value for 19 of the 2^32 f32 inputs
// (host-checked over all of them), glibc's expf -- what ggml_exp calls per
// element -- for 170,648. The table is read from memory: these loops may run
// with part of the wave inactive, so no cross-lane lookup.
__device__ __forceinline__ float exp_f32(float x) {
    return exp_f32_rn(x, [](int j) { return kExpTable[j]; });
}

// One element of the op. `b` is the second input (or the broadcast row value);
// `s` receives the carried sum.
template <int OP> __device__ __forceinline__ float ew(float a, float b, const EwArgs & g, float & s) {
    if constexpr (OP == kSwiglu) {
        return silu(a) * b;
    } else if constexpr (OP == kSilu) {
        return silu(a);
    } else if constexpr (OP == kAdd) {
        return a + b;
    } else if constexpr (OP == kAddLeaky) {
        s = a + b;
        return leaky(s, g.slope);
    } else if constexpr (OP == kLeaky) {
        return leaky(a, g.slope);
    } else if constexpr (OP == kExp) {
        return exp_f32(a);
    } else if constexpr (OP == kScale) {
        // ggml_scale (bias 0): a plain multiply, so -0 stays -0.
        return a * g.scale;
    } else if constexpr (OP == kScaleBias) {
        // ggml_scale_bias with a non-zero bias: one fused multiply-add, as
        // ggml-CPU's vectorised path computes it on FMA hardware.
        return fmaf(a, g.scale, g.bias);
    } else if constexpr (OP == kMul) {
        return a * b;
    } else if constexpr (OP == kDiv) {
        return a / b;
    } else if constexpr (OP == kSin) {
        // The sine of the Snake kernels, so a Snake run and its nodes one by
        // one agree bit for bit. Its reduction turns -0 into +0 (-0 - 0*pi/2 is
        // +0); sinf keeps the sign of a zero, so zeros pass through (inside
        // Snake the sine is squared and the sign does not matter).
        return a == 0.0f ? a : (sin_fast_ok(a) ? sin_f32_fast(a) : sinf(a));
    } else if constexpr (OP == kSqr) {
        return a * a;
    } else if constexpr (OP == kSub) {
        return a - b;
    } else if constexpr (OP == kTanh) {
        // ggml's vec forms of the codec / vocoder activations, in f32 with the
        // device's math functions (vits/waveform-decoder.cpp:228,
        // kokoro/operations.cpp:133, qwen3-tts/codec.cpp:222,481)
        return tanhf(a);
    } else if constexpr (OP == kSigmoid) {
        return 1.0f / (1.0f + expf(-a));
    } else if constexpr (OP == kElu) {
        return a > 0.0f ? a : expm1f(a);
    } else if constexpr (OP == kGeluErf) {
        return 0.5f * a * (1.0f + erff(a * 0.70710678118654752440084436210484f));
    } else if constexpr (OP == kClamp) {
        // ggml's MAX(MIN(x, max), min): a NaN gives max
        const float m = a < g.bias ? a : g.bias;
        return m > g.scale ? m : g.scale;
    } else if constexpr (OP == kRelu) {
        // ggml's x > 0 ? x : 0 (vits/text-encoder.cpp:71, qwen3-tts/speaker-
        // encoder.cpp:184): -0 and NaN give +0
        return a > 0.0f ? a : 0.0f;
    } else if constexpr (OP == kNeg) {
        return -a;
    } else if constexpr (OP == kStep) {
        return a > 0.0f ? 1.0f : 0.0f;
    } else if constexpr (OP == kSqrt) {
        // correctly rounded, as sqrtf (qwen3-tts/speaker-encoder.cpp:294)
        return __builtin_sqrtf(a);
    } else {
        static_assert(OP == kCopy, "unknown elementwise op");
        return a;
    }
}

template <int OP> __device__ __forceinline__ f32x4 ew4(f32x4 a, f32x4 b, const EwArgs & g, f32x4 & s) {
    float       s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    const f32x4 o{ ew<OP>(a.x, b.x, g, s0), ew<OP>(a.y, b.y, g, s1), ew<OP>(a.z, b.z, g, s2),
                   ew<OP>(a.w, b.w, g, s3) };
    s = f32x4{ s0, s1, s2, s3 };
    return o;
}

// Flat path: the tensors are contiguous and 16-byte aligned, so element e of
// every operand sits at the same offset. Each lane streams exactly one float4
// of each input and output (more per lane measured slower on gfx950: fewer
// waves in flight per CU), with nontemporal loads and stores. The grid covers
// the tensor once; the loop only runs again for tensors beyond kMaxFlatBlocks.
// HAS_B: a second input; BCAST: b is one row of `period` elements repeated
// over rows; Snake reads alpha the same way; HAS_S: write the carried sum.
constexpr int64_t kMaxFlatBlocks = int64_t{ 1 } << 20;
// From this many float4 per operand (16 MB) the flat kernels launch 64-thread
// blocks, one wave each: measured on MI355X 1-3.5 % faster from [512,8192]
// up (SwiGLU [6144,8192] 93.0 -> 91.2 us, add->leaky+sum [128,131072] 44.2 ->
// 43.6 us), and 1-4 % slower below (a 512-token add, a decode step's SwiGLU),
// where 256-thread blocks stay. The Snake and RMSNorm kernels keep 256-thread
// blocks at every size: one-wave blocks measured 2 % (Snake [128,131072]) and
// 2-6 % (the [2048,8192] norms) slower.
constexpr int64_t kFlatWaveBlocksFrom = int64_t{ 1 } << 20;
// From 4 MB per operand up to that size, two float4 per lane
// (k_ew_flat2): SwiGLU [3072,512] 4.81 -> 4.66 us; at [1024,512] (2 MB per
// operand) it measured 1 % slower than one float4 per lane.
constexpr int64_t kFlat2From = int64_t{ 1 } << 18;

template <int OP, bool HAS_B, bool BCAST, bool HAS_S, int BLOCK>
__global__ __launch_bounds__(BLOCK) void k_ew_flat(const EwArgs a) {
    const f32x4 * A    = reinterpret_cast<const f32x4 *>(a.a);
    const f32x4 * B    = reinterpret_cast<const f32x4 *>(a.b);
    f32x4 *       Y    = reinterpret_cast<f32x4 *>(a.y);
    f32x4 *       S    = reinterpret_cast<f32x4 *>(a.s);
    const int64_t n4   = a.n4;
    const int64_t step = static_cast<int64_t>(gridDim.x) * BLOCK;
    args_in_sgprs(A, B, Y, n4, step);
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * BLOCK + threadIdx.x; i < n4; i += step) {
        const f32x4 av = ld_stream(A + i);
        f32x4       bv = splat4(0.0f);
        if constexpr (HAS_B) {
            if constexpr (BCAST) {
                bv = B[fastmod(static_cast<uint32_t>(i * 4), a.period) / 4];
            } else {
                bv = ld_stream(B + i);
            }
        }
        f32x4 sv = splat4(0.0f);
        st_stream(Y + i, ew4<OP>(av, bv, a, sv));
        if constexpr (HAS_S) {
            st_stream(S + i, sv);
        }
    }
}

// Per-channel coefficients of the Snake family from the stored curves c0
// (alpha or log alpha) and c1 (log beta). ggml_scale_bias(c, 1.0f, 1e-9f)
// is c*1 + 1e-9 with c*1 exact, so every evaluation order gives c + 1e-9
// rounded once.
struct SnakeCoef {
    float al;   // multiplier of x inside the sine
    float den;  // divisor of the squared sine
};

template <int K> __device__ __forceinline__ SnakeCoef snake_coef(float c0, float c1) {
    if constexpr (K == kSnakePlain) {
        return { c0, c0 };
    } else if constexpr (K == kSnakeGuarded) {
        return { c0, c0 + kSnakeGuard };
    } else {
        return { exp_f32(c0), exp_f32(c1) + kSnakeGuard };
    }
}

// The node run mul, sin, mul (or sqr), div, add, each rounded in f32, from
// t = x*al. FAST: t is known to be inside the fast sine's range. RCP: divide
// through the double reciprocal of den (IEEE quotient, shp_div.hpp).
template <bool FAST, bool RCP> __device__ __forceinline__ float snake_t(float x, float t, float den, double rcp) {
    // squared below, so the fast path may drop the sine's sign (bit-identical square)
    const float sn = FAST ? sin_f32_fast_unsigned(t) : (sin_fast_ok(t) ? sin_f32_fast(t) : sinf(t));
    const float q  = sn * sn;
    const float r  = RCP ? div_by_rcp(q, rcp) : q / den;
    return x + r;
}

template <bool RCP> __device__ __forceinline__ float snake1(float x, float al, float den, double rcp) {
    return snake_t<false, RCP>(x, x * al, den, rcp);
}

// Snake, flat path. The formula is ALU-heavy for a streaming op (a sine and
// a division per element, and for SnakeBeta two exps per channel), so its
// costs are cut without changing its result:
//   - a lane owns one quad of channels (4 consecutive coefficients) in R
//     consecutive rows (SnakeRows), so the per-channel work (the exps, the
//     guard and the 4 double reciprocals) is done once per R rows;
//   - the division: q / den becomes (float)((double)q * rcp), which is the
//     IEEE quotient (shp_div.hpp). Lanes whose den include 0, inf or NaN take
//     the f32 division;
//   - sinf: shp::sin_f32_fast, branch-free and within 1 ulp of the correctly
//     rounded sine for |t| < 2^15 (shp_sinf.hpp); OCML's sinf beyond that.
// The curves are loaded before the rows, so the per-channel work overlaps the
// row loads. Each of the wave's loads and stores is one contiguous 1 KB run
// (64 lanes, consecutive quads of one row). Measured on MI355X at
// [128,131072], plain Snake: ~6% faster than one float4 per lane with OCML's
// sinf and the f32 division.
// Rows per lane, measured on MI355X over the cfg4 shapes: 2 for Snake and the
// guarded Snake (3-6 % faster than 4), 8 for SnakeBeta, whose two exps per
// channel then spread over 32 elements (9-11 % faster than 4 at [256,32768]
// and [128,131072]).
template <int K> struct SnakeRows {
    static constexpr int R = K == kSnakeBeta ? 8 : 2;
};

// A lane's elements, two rows (8 elements) at a time: every t first, then one
// range test for the 8, so the common case is straight-line code whose
// independent sine/division chains the compiler interleaves (a test per
// element puts a branch between every pair of them; testing all R rows at
// once holds too many registers at R = 8).
constexpr int kSnakeSub = 2;

template <int K, int R, bool RCP>
__device__ __forceinline__ void snake_rows(const f32x4 (&xv)[R], f32x4 al, f32x4 den, const double (&rc)[4], int64_t i0,
                                           int64_t c4, int64_t n4, f32x4 * Y) {
    constexpr int SUB = R < kSnakeSub ? R : kSnakeSub;
    static_assert(R % SUB == 0, "rows per lane in whole sub-blocks");
#pragma unroll
    for (int r0 = 0; r0 < R; r0 += SUB) {
        f32x4    t[SUB];
        unsigned fast = 1u;  // bitwise: a short-circuit && would branch per element again
#pragma unroll
        for (int r = 0; r < SUB; ++r) {
            const f32x4 x = xv[r0 + r];
            t[r]          = f32x4{ x.x * al.x, x.y * al.y, x.z * al.z, x.w * al.w };
            fast &= static_cast<unsigned>(sin_fast_ok(t[r].x)) & static_cast<unsigned>(sin_fast_ok(t[r].y)) &
                    static_cast<unsigned>(sin_fast_ok(t[r].z)) & static_cast<unsigned>(sin_fast_ok(t[r].w));
        }
        f32x4 y[SUB];
        if (fast != 0u) {
#pragma unroll
            for (int r = 0; r < SUB; ++r) {
                const f32x4 x = xv[r0 + r];
                y[r]          = f32x4{ snake_t<true, RCP>(x.x, t[r].x, den.x, rc[0]),
                                       snake_t<true, RCP>(x.y, t[r].y, den.y, rc[1]),
                                       snake_t<true, RCP>(x.z, t[r].z, den.z, rc[2]),
                                       snake_t<true, RCP>(x.w, t[r].w, den.w, rc[3]) };
            }
        } else {
#pragma unroll
            for (int r = 0; r < SUB; ++r) {
                const f32x4 x = xv[r0 + r];
                y[r]          = f32x4{ snake_t<false, RCP>(x.x, t[r].x, den.x, rc[0]),
                                       snake_t<false, RCP>(x.y, t[r].y, den.y, rc[1]),
                                       snake_t<false, RCP>(x.z, t[r].z, den.z, rc[2]),
                                       snake_t<false, RCP>(x.w, t[r].w, den.w, rc[3]) };
            }
        }
#pragma unroll
        for (int r = 0; r < SUB; ++r) {
            const int64_t i = i0 + (r0 + r) * c4;
            if (i < n4) {
                st_stream(Y + i, y[r]);
            }
        }
    }
}

template <int K, int BLOCK, int R = SnakeRows<K>::R> __global__ __launch_bounds__(BLOCK) void k_snake_flat(const EwArgs a) {
    const f32x4 * X    = reinterpret_cast<const f32x4 *>(a.a);
    const f32x4 * C0   = reinterpret_cast<const f32x4 *>(a.alpha);
    const f32x4 * C1   = reinterpret_cast<const f32x4 *>(a.beta);
    f32x4 *       Y    = reinterpret_cast<f32x4 *>(a.y);
    const int64_t c4   = a.quads.d;
    const int64_t step = static_cast<int64_t>(gridDim.x) * BLOCK;
    args_in_sgprs(X, C0, C1, a.quads.d, a.quads.m, a.quads.l, a.ntask, a.n4, step);
    // A lane's task: its curves and its R rows, requested together, so the
    // per-channel work waits for one round trip, in parallel with the rows
    // (the loop runs once unless the grid is capped).
    int64_t  t = static_cast<int64_t>(blockIdx.x) * BLOCK + threadIdx.x;
    uint32_t q;
    int64_t  i0;
    f32x4    c0, c1, xv[R];
    auto     load = [&](int64_t tt) {
        const uint32_t rb = fastdiv(static_cast<uint32_t>(tt), a.quads);  // row block
        q                 = static_cast<uint32_t>(tt) - rb * a.quads.d;  // channel quad
        i0                = static_cast<int64_t>(rb) * R * c4 + q;
        const bool in     = tt < a.ntask;
        c0                = in ? C0[q] : splat4(1.0f);
        c1                = K == kSnakeBeta && in ? C1[q] : splat4(0.0f);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t i = i0 + r * c4;
            xv[r]           = (in & (i < a.n4)) ? ld_stream(X + i) : splat4(0.0f);
        }
    };
    load(t);
    while (t < a.ntask) {
        const SnakeCoef k0 = snake_coef<K>(c0.x, c1.x);
        const SnakeCoef k1 = snake_coef<K>(c0.y, c1.y);
        const SnakeCoef k2 = snake_coef<K>(c0.z, c1.z);
        const SnakeCoef k3 = snake_coef<K>(c0.w, c1.w);
        const f32x4     al{ k0.al, k1.al, k2.al, k3.al };
        const f32x4     den{ k0.den, k1.den, k2.den, k3.den };
        if (rcp_route_ok(den.x) && rcp_route_ok(den.y) && rcp_route_ok(den.z) && rcp_route_ok(den.w)) {
            const double rc[4] = { rcp_d(static_cast<double>(den.x)), rcp_d(static_cast<double>(den.y)),
                                   rcp_d(static_cast<double>(den.z)), rcp_d(static_cast<double>(den.w)) };
            snake_rows<K, R, true>(xv, al, den, rc, i0, c4, a.n4, Y);
        } else {
            const double rc[4] = { 0.0, 0.0, 0.0, 0.0 };
            snake_rows<K, R, false>(xv, al, den, rc, i0, c4, a.n4, Y);
        }
        t += step;
        if (t < a.ntask) {
            load(t);
        }
    }
}


// SnakeBeta with at most kSnakeLdsMaxC channels: each block evaluates every
// channel's exp curves, guard and double reciprocal once into LDS while its
// lanes' rows are in flight, and after one barrier each lane runs its task
// (R rows of one channel quad) from the table. One task per lane: R = 4 up to
// kSnakeLdsSmallTasks tasks, else R = 8 (the two exps per channel are spread
// over the block's 2048 or 4096 elements instead of 8 or 32 per lane).
// CF (the 4-row form): each thread requests its channels' log-curves and its
// lane's exp-table entry before the rows, so the exps wait for those loads
// alone (not for the rows queued ahead of them), and looks the table up in a
// per-wave LDS copy instead of memory; the same values bit for bit.
// Measured on MI355X against the 8-row flat kernel: [512,8192] 8.4 -> 7.4 us
// (7.8 without CF), [256,32768] 13.1 -> 12.7 us; [128,131072] 25.4 -> 24.7 us
// against 2-row tasks over 1024 persistent blocks. CF on the 8-row form is
// 11 % slower at the two larger shapes. Rejected at [128,131072]: 2048
// persistent blocks, 512- or 1024-thread blocks, 2-, 4- or 16-row tasks,
// each lane keeping its quad's curves in registers for all its tasks, and a
// table sized to 128 channels (4 KB of LDS instead of 18 KB, more blocks per
// CU: 25.6 against 24.9 us at [128,131072]). For
// plain Snake, whose per-channel work is only the reciprocal, a table does
// not pay.
constexpr int     kSnakeLdsMaxC       = 1024;
constexpr int64_t kSnakeLdsSmallTasks = int64_t{ 1024 } * 256;        // 4-row tasks, one per lane
constexpr int64_t kSnakeLdsMaxTasks   = int64_t{ 1 } << 20;          // 8-row tasks, one per lane
// Up to 128 channels (half a curve per thread to evaluate) the 4-row form with
// CF stays ahead at any length: [128,131072] 26.4 -> 25.4 us on MI355X, where
// at 256 channels the 8-row form is 2 % ahead ([256,32768] 14.2 against 14.6).
constexpr int64_t kSnakeLdsSmallQuads = 32;

template <int R, bool CF> __global__ __launch_bounds__(256) void k_snake_beta_lds(const EwArgs a) {
    constexpr int kPer = kSnakeLdsMaxC / 256;  // channels per thread at most
    __shared__ __align__(16) float  s_al[kSnakeLdsMaxC];
    __shared__ __align__(16) float  s_den[kSnakeLdsMaxC];
    __shared__ __align__(16) double s_rc[kSnakeLdsMaxC];
    __shared__ double               s_tab[CF ? 256 / kWave : 1][kWave];
    const f32x4 * X    = reinterpret_cast<const f32x4 *>(a.a);
    f32x4 *       Y    = reinterpret_cast<f32x4 *>(a.y);
    const int64_t c4   = a.quads.d;
    const int64_t step = static_cast<int64_t>(gridDim.x) * 256;
    args_in_sgprs(X, a.alpha, a.beta, a.quads.d, a.quads.m, a.quads.l, a.ntask, a.n4);
    const int nc   = static_cast<int>(a.quads.d) * 4;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    double    entry = 0.0;
    float     la[kPer], lb[kPer];
    if constexpr (CF) {
        entry = exp_table_entry(lane);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int c  = static_cast<int>(threadIdx.x) + 256 * j;
            const int cc = c < nc ? c : 0;  // past the channels: re-read channel 0, unused
            la[j]        = a.alpha[cc];
            lb[j]        = a.beta[cc];
        }
    }
    // The first task's rows are requested before the table of curves is
    // built, so their loads overlap its loads and exps.
    int64_t  t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    uint32_t q;
    int64_t  i0;
    f32x4    xv[R];
    auto     load = [&](int64_t tt) {
        const uint32_t rb = fastdiv(static_cast<uint32_t>(tt), a.quads);  // row block
        q                 = static_cast<uint32_t>(tt) - rb * a.quads.d;  // channel quad
        i0                = static_cast<int64_t>(rb) * R * c4 + q;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t i = i0 + r * c4;
            xv[r]           = ((tt < a.ntask) & (i < a.n4)) ? ld_stream(X + i) : splat4(0.0f);
        }
    };
    load(t);
    if constexpr (CF) {
        const double * tab = wave_exp_table(s_tab, lane, entry);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int c = static_cast<int>(threadIdx.x) + 256 * j;
            if (c < nc) {
                // snake_coef<kSnakeBeta> with the table in LDS
                const float al  = exp_f32_lds(la[j], tab);
                const float den = exp_f32_lds(lb[j], tab) + kSnakeGuard;
                s_al[c]         = al;
                s_den[c]        = den;
                s_rc[c]         = rcp_route_ok(den) ? rcp_d(static_cast<double>(den)) : 0.0;
            }
        }
    } else {
        for (int c = threadIdx.x; c < nc; c += 256) {
            const SnakeCoef k = snake_coef<kSnakeBeta>(a.alpha[c], a.beta[c]);
            s_al[c]           = k.al;
            s_den[c]          = k.den;
            s_rc[c]           = rcp_route_ok(k.den) ? rcp_d(static_cast<double>(k.den)) : 0.0;
        }
    }
    __syncthreads();
    while (t < a.ntask) {
        const f32x4  al    = reinterpret_cast<const f32x4 *>(s_al)[q];
        const f32x4  den   = reinterpret_cast<const f32x4 *>(s_den)[q];
        const double rc[4] = { s_rc[4 * q], s_rc[4 * q + 1], s_rc[4 * q + 2], s_rc[4 * q + 3] };
        if (rcp_route_ok(den.x) && rcp_route_ok(den.y) && rcp_route_ok(den.z) && rcp_route_ok(den.w)) {
            snake_rows<kSnakeBeta, R, true>(xv, al, den, rc, i0, c4, a.n4, Y);
        } else {
            snake_rows<kSnakeBeta, R, false>(xv, al, den, rc, i0, c4, a.n4, Y);
        }
        t += step;
        if (t < a.ntask) {
            load(t);
        }
    }
}

// Snake, row path: any byte strides for x and y (curves contiguous); rows
// grid-strided over blocks, channels over threads.
template <int K> __global__ __launch_bounds__(256) void k_snake_rows(const EwArgs a) {
    for (int64_t r = blockIdx.x; r < a.nrows; r += gridDim.x) {
        const float * xr = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.a) + row_offset(a.am, r));
        float *       yr = reinterpret_cast<float *>(reinterpret_cast<char *>(a.y) + row_offset(a.ym, r));
        for (int c = threadIdx.x; c < a.ne0; c += blockDim.x) {
            const SnakeCoef k = snake_coef<K>(a.alpha[c], K == kSnakeBeta ? a.beta[c] : 0.0f);
            yr[c]             = snake1<false>(xr[c], k.al, k.den, 0.0);
        }
    }
}

// Row path: any ggml byte strides; rows grid-strided over blocks, elements
// over threads. VEC uses float4 columns (ne0 % 4 == 0, rows 16-byte aligned).
template <int OP, bool HAS_B, bool BCAST, bool HAS_S, bool VEC>
__global__ __launch_bounds__(256) void k_ew_rows(const EwArgs a) {
    for (int64_t r = blockIdx.x; r < a.nrows; r += gridDim.x) {
        const char * ar = reinterpret_cast<const char *>(a.a) + row_offset(a.am, r);
        const char * br = nullptr;
        if constexpr (HAS_B) {
            br = reinterpret_cast<const char *>(a.b) + (BCAST ? 0 : row_offset(a.bm, r));
        }
        char * yr = reinterpret_cast<char *>(a.y) + row_offset(a.ym, r);
        char * sr = nullptr;
        if constexpr (HAS_S) {
            sr = reinterpret_cast<char *>(a.s) + row_offset(a.sm, r);
        }
        if constexpr (VEC) {
            for (int c = threadIdx.x; c < a.ne0 / 4; c += blockDim.x) {
                const f32x4 av = ld_stream(reinterpret_cast<const f32x4 *>(ar) + c);
                f32x4       bv = splat4(0.0f);
                if constexpr (HAS_B) {
                    bv = BCAST ? reinterpret_cast<const f32x4 *>(br)[c] : ld_stream(reinterpret_cast<const f32x4 *>(br) + c);
                }
                f32x4 sv = splat4(0.0f);
                st_stream(reinterpret_cast<f32x4 *>(yr) + c, ew4<OP>(av, bv, a, sv));
                if constexpr (HAS_S) {
                    st_stream(reinterpret_cast<f32x4 *>(sr) + c, sv);
                }
            }
        } else {
            for (int c = threadIdx.x; c < a.ne0; c += blockDim.x) {
                const float av = reinterpret_cast<const float *>(ar)[c];
                float       bv = 0.0f;
                if constexpr (HAS_B) {
                    bv = reinterpret_cast<const float *>(br)[c];
                }
                float sv                         = 0.0f;
                reinterpret_cast<float *>(yr)[c] = ew<OP>(av, bv, a, sv);
                if constexpr (HAS_S) {
                    reinterpret_cast<float *>(sr)[c] = sv;
                }
            }
        }
    }
}

// Branch average: summed = t0 + t1 + ... (in term order), current =
// summed * scale, y = leaky(current, slope). The node run add.., scale,
// leaky_relu of vits/waveform-decoder.cpp:214-225 and kokoro/generator.cpp:
// 165-179. Contiguous tensors only; VEC streams one float4 per lane per term.
constexpr int kMaxTerms = 8;

struct TermArgs {
    const float * t[kMaxTerms];
    float *       y;
    float *       m;  // the scaled sum (`current`), or null
    int64_t       n;  // elements, or float4s when VEC
    float         scale;
    float         slope;
};

template <int N, bool HAS_M, bool VEC> __global__ __launch_bounds__(256) void k_sum_scale_leaky(const TermArgs a) {
    using V            = typename std::conditional<VEC, f32x4, float>::type;
    const int64_t step = static_cast<int64_t>(gridDim.x) * 256;
    const int64_t n    = a.n;
    args_in_sgprs(n, step);
#pragma unroll
    for (int j = 0; j < N; ++j) {
        arg_in_sgpr(a.t[j]);
    }
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += step) {
        V v[N];
#pragma unroll
        for (int j = 0; j < N; ++j) {
            v[j] = ld_stream(reinterpret_cast<const V *>(a.t[j]) + i);
        }
        V s = v[0];
#pragma unroll
        for (int j = 1; j < N; ++j) {
            s = s + v[j];
        }
        const V cur = s * a.scale;
        if constexpr (HAS_M) {
            st_stream(reinterpret_cast<V *>(a.m) + i, cur);
        }
        if constexpr (VEC) {
            st_stream(reinterpret_cast<V *>(a.y) + i, f32x4{ leaky(cur.x, a.slope), leaky(cur.y, a.slope),
                                                          leaky(cur.z, a.slope), leaky(cur.w, a.slope) });
        } else {
            st_stream(reinterpret_cast<V *>(a.y) + i, leaky(cur, a.slope));
        }
    }
}

template <int N> shp_status_t launch_sum_scale_leaky(const TermArgs & a, bool vec, hipStream_t stream) {
    if (dry_run()) {
        return SHP_OK;
    }
    int64_t blocks = (a.n + 255) / 256;
    blocks         = blocks < kMaxFlatBlocks ? blocks : kMaxFlatBlocks;
    const dim3 grid(static_cast<unsigned>(blocks));
    if (a.m != nullptr) {
        if (vec) {
            hipLaunchKernelGGL((k_sum_scale_leaky<N, true, true>), grid, dim3(256), 0, stream, a);
        } else {
            hipLaunchKernelGGL((k_sum_scale_leaky<N, true, false>), grid, dim3(256), 0, stream, a);
        }
    } else if (vec) {
        hipLaunchKernelGGL((k_sum_scale_leaky<N, false, true>), grid, dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL((k_sum_scale_leaky<N, false, false>), grid, dim3(256), 0, stream, a);
    }
    return launch_status();
}

// Two float4 per lane and operand (a block covers 512 consecutive float4),
// every load issued before the first store; for mid-size tensors.
template <int OP, bool HAS_B, bool BCAST, bool HAS_S>
__global__ __launch_bounds__(256) void k_ew_flat2(const EwArgs a) {
    const f32x4 * A  = reinterpret_cast<const f32x4 *>(a.a);
    const f32x4 * B  = reinterpret_cast<const f32x4 *>(a.b);
    f32x4 *       Y  = reinterpret_cast<f32x4 *>(a.y);
    f32x4 *       S  = reinterpret_cast<f32x4 *>(a.s);
    const int64_t n4 = a.n4;
    args_in_sgprs(A, B, Y, n4);
    const int64_t i0 = static_cast<int64_t>(blockIdx.x) * 512 + threadIdx.x;
    f32x4         av[2], bv[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int64_t i = i0 + 256 * k < n4 ? i0 + 256 * k : n4 - 1;  // past the end: re-read the last chunk
        av[k]           = ld_stream(A + i);
        bv[k]           = splat4(0.0f);
        if constexpr (HAS_B) {
            if constexpr (BCAST) {
                bv[k] = B[fastmod(static_cast<uint32_t>(i * 4), a.period) / 4];
            } else {
                bv[k] = ld_stream(B + i);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int64_t i = i0 + 256 * k;
        if (i < n4) {
            f32x4 sv = splat4(0.0f);
            st_stream(Y + i, ew4<OP>(av[k], bv[k], a, sv));
            if constexpr (HAS_S) {
                st_stream(S + i, sv);
            }
        }
    }
}

template <int OP, bool HAS_B, bool BCAST, bool HAS_S>
shp_status_t launch_ew(const EwArgs & a, bool flat, bool vec, hipStream_t stream) {
    if (dry_run()) {
        return SHP_OK;
    }
    if (flat && a.n4 >= kFlat2From && a.n4 < kFlatWaveBlocksFrom) {
        hipLaunchKernelGGL((k_ew_flat2<OP, HAS_B, BCAST, HAS_S>), dim3(static_cast<unsigned>((a.n4 + 511) / 512)),
                           dim3(256), 0, stream, a);
        return launch_status();
    }
    if (flat) {
        const bool wave = a.n4 >= kFlatWaveBlocksFrom;
        const int  bs   = wave ? kWave : 256;
        int64_t    blocks = (a.n4 + bs - 1) / bs;
        blocks            = blocks < kMaxFlatBlocks ? blocks : kMaxFlatBlocks;
        if (wave) {
            hipLaunchKernelGGL((k_ew_flat<OP, HAS_B, BCAST, HAS_S, kWave>), dim3(static_cast<unsigned>(blocks)),
                               dim3(kWave), 0, stream, a);
        } else {
            hipLaunchKernelGGL((k_ew_flat<OP, HAS_B, BCAST, HAS_S, 256>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                               0, stream, a);
        }
        return launch_status();
    }
    const int64_t blocks = a.nrows < 65536 ? a.nrows : 65536;
    if (vec) {
        hipLaunchKernelGGL((k_ew_rows<OP, HAS_B, BCAST, HAS_S, true>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                           0, stream, a);
    } else {
        hipLaunchKernelGGL((k_ew_rows<OP, HAS_B, BCAST, HAS_S, false>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                           0, stream, a);
    }
    return launch_status();
}

// Common argument set-up. `b` may be null, may match `a`'s shape, or (when
// allow_bcast) be one row of ne0 elements.
struct EwPlan {
    EwArgs args{};
    bool   flat  = false;
    bool   vec   = false;
    bool   bcast = false;
};

shp_status_t plan_ew(const shp_tensor * a,
                     const shp_tensor * b,
                     bool               allow_bcast,
                     shp_tensor *       y,
                     shp_tensor *       s,
                     EwPlan &           plan) {
    if (!well_formed(a) || !well_formed(y) || (b != nullptr && !well_formed(b)) || (s != nullptr && !well_formed(s))) {
        return SHP_ERR_INVALID_ARG;
    }
    if (a->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32 || (b != nullptr && b->type != SHP_TYPE_F32) ||
        (s != nullptr && s->type != SHP_TYPE_F32)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (!same_shape(*a, *y) || (s != nullptr && !same_shape(*a, *s)) || a->ne[0] > INT32_MAX) {
        return SHP_ERR_INVALID_ARG;
    }
    if (b != nullptr && !same_shape(*a, *b)) {
        if (!allow_bcast || !one_row_of(*b, a->ne[0])) {
            return SHP_ERR_INVALID_ARG;
        }
        plan.bcast = true;
    }
    EwArgs & g = plan.args;
    g.a        = static_cast<const float *>(a->data);
    g.am       = make_rowmap(*a);
    g.y        = static_cast<float *>(y->data);
    g.ym       = make_rowmap(*y);
    g.nrows    = nrows(*a);
    g.ne0      = static_cast<int32_t>(a->ne[0]);
    if (b != nullptr) {
        g.b  = static_cast<const float *>(b->data);
        g.bm = make_rowmap(*b);
    }
    if (s != nullptr) {
        g.s  = static_cast<float *>(s->data);
        g.sm = make_rowmap(*s);
    }
    const int64_t n = nelements(*a);
    plan.vec        = a->ne[0] % 4 == 0 && rows_aligned(*a, 16) && rows_aligned(*y, 16) &&
               (b == nullptr || rows_aligned(*b, 16)) && (s == nullptr || rows_aligned(*s, 16));
    plan.flat = plan.vec && contiguous(*a) && contiguous(*y) && (b == nullptr || plan.bcast || contiguous(*b)) &&
                (s == nullptr || contiguous(*s)) && n < (int64_t{ 1 } << 32);
    g.n4     = n / 4;
    g.period = make_fastdiv(static_cast<uint32_t>(a->ne[0]));
    return SHP_OK;
}

}  // namespace
}  // namespace shp

using namespace shp;

extern "C" shp_status_t shp_swiglu(const shp_tensor * g, const shp_tensor * u, shp_tensor * y, shp_stream_t stream) {
    EwPlan             plan;
    const shp_status_t st = plan_ew(g, u, false, y, nullptr, plan);
    if (st != SHP_OK) {
        return st;
    }
    if (u == nullptr) {
        return launch_ew<kSilu, false, false, false>(plan.args, plan.flat, plan.vec, as_stream(stream));
    }
    return launch_ew<kSwiglu, true, false, false>(plan.args, plan.flat, plan.vec, as_stream(stream));
}

extern "C" shp_status_t shp_glu_swiglu(const shp_tensor * a, int32_t swapped, shp_tensor * y, shp_stream_t stream) {
    if (!well_formed(a) || !well_formed(y)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (a->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (a->ne[0] % 2 != 0 || y->ne[0] * 2 != a->ne[0] || y->ne[1] != a->ne[1] || y->ne[2] != a->ne[2] ||
        y->ne[3] != a->ne[3] || y->ne[0] > INT32_MAX) {
        return SHP_ERR_INVALID_ARG;
    }
    // The gate and up halves are two row views of `a` sharing its strides.
    const size_t half_bytes = static_cast<size_t>(y->ne[0]) * sizeof(float);
    shp_tensor   gate       = *a;
    shp_tensor   up         = *a;
    gate.ne[0]              = y->ne[0];
    up.ne[0]                = y->ne[0];
    gate.data = static_cast<char *>(a->data) + (swapped ? half_bytes : 0);
    up.data   = static_cast<char *>(a->data) + (swapped ? 0 : half_bytes);
    EwPlan             plan;
    const shp_status_t st = plan_ew(&gate, &up, false, y, nullptr, plan);
    if (st != SHP_OK) {
        return st;
    }
    return launch_ew<kSwiglu, true, false, false>(plan.args, false, plan.vec, as_stream(stream));
}

namespace shp {
namespace {

// A per-channel curve: F32, contiguous, exactly C elements (any of the
// [C], [C,1] or [1,C,1] shapes the builders store it in).
bool channel_curve(const shp_tensor * c, int64_t channels) {
    return nelements(*c) == channels && contiguous(*c);
}

template <int K>
shp_status_t launch_snake(const shp_tensor * x, const shp_tensor * c0, const shp_tensor * c1, shp_tensor * y,
                          hipStream_t stream) {
    if (!well_formed(x) || !well_formed(c0) || (K == kSnakeBeta && !well_formed(c1))) {
        return SHP_ERR_INVALID_ARG;
    }
    if (c0->type != SHP_TYPE_F32 || (K == kSnakeBeta && c1->type != SHP_TYPE_F32)) {
        return SHP_ERR_UNSUPPORTED;
    }
    // One coefficient per channel; channels are ne[0] (kokoro_decoder_test.cpp:46-49).
    if (!channel_curve(c0, x->ne[0]) || (K == kSnakeBeta && !channel_curve(c1, x->ne[0]))) {
        return SHP_ERR_INVALID_ARG;
    }
    EwPlan             plan;
    const shp_status_t st = plan_ew(x, nullptr, false, y, nullptr, plan);
    if (st != SHP_OK || dry_run()) {
        return st;
    }
    EwArgs & g = plan.args;
    g.alpha    = static_cast<const float *>(c0->data);
    g.beta     = K == kSnakeBeta ? static_cast<const float *>(c1->data) : nullptr;
    const bool c16 =
        reinterpret_cast<uintptr_t>(g.alpha) % 16 == 0 && reinterpret_cast<uintptr_t>(g.beta) % 16 == 0;
    if (K == kSnakeBeta && plan.flat && c16 && x->ne[0] <= kSnakeLdsMaxC) {
        const int64_t quads  = x->ne[0] / 4;
        const int64_t rows   = g.n4 / quads;
        const int64_t ntask4 = (rows + 3) / 4 * quads;
        const int64_t ntask8 = (rows + 7) / 8 * quads;
        g.quads              = make_fastdiv(static_cast<uint32_t>(quads));
        if (ntask4 <= kSnakeLdsSmallTasks || (quads <= kSnakeLdsSmallQuads && ntask4 <= kSnakeLdsMaxTasks)) {
            g.ntask = ntask4;
            hipLaunchKernelGGL((k_snake_beta_lds<4, true>), dim3(static_cast<unsigned>((ntask4 + 255) / 256)), dim3(256), 0,
                               stream, g);
            return launch_status();
        }
        if (ntask8 <= kSnakeLdsMaxTasks) {
            g.ntask = ntask8;
            hipLaunchKernelGGL((k_snake_beta_lds<8, false>), dim3(static_cast<unsigned>((ntask8 + 255) / 256)), dim3(256), 0,
                               stream, g);
            return launch_status();
        }
    }
    if (plan.flat && c16) {
        constexpr int R      = SnakeRows<K>::R;
        const int64_t quads  = x->ne[0] / 4;
        const int64_t rows   = g.n4 / quads;
        g.quads              = make_fastdiv(static_cast<uint32_t>(quads));
        g.ntask              = (rows + R - 1) / R * quads;
        int64_t       blocks = (g.ntask + 255) / 256;
        blocks               = blocks < kMaxFlatBlocks ? blocks : kMaxFlatBlocks;
        hipLaunchKernelGGL((k_snake_flat<K, 256>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, g);
        return launch_status();
    }
    const int64_t blocks = g.nrows < 65536 ? g.nrows : 65536;
    hipLaunchKernelGGL(k_snake_rows<K>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, g);
    return launch_status();
}

}  // namespace
}  // namespace shp

extern "C" shp_status_t shp_snake(const shp_tensor * x, const shp_tensor * alpha, shp_tensor * y, shp_stream_t stream) {
    return launch_snake<kSnakePlain>(x, alpha, nullptr, y, as_stream(stream));
}

extern "C" shp_status_t shp_snake_guarded(const shp_tensor * x,
                                          const shp_tensor * alpha,
                                          shp_tensor *       y,
                                          shp_stream_t       stream) {
    return launch_snake<kSnakeGuarded>(x, alpha, nullptr, y, as_stream(stream));
}

extern "C" shp_status_t shp_snake_beta(const shp_tensor * x,
                                       const shp_tensor * log_alpha,
                                       const shp_tensor * log_beta,
                                       shp_tensor *       y,
                                       shp_stream_t       stream) {
    return launch_snake<kSnakeBeta>(x, log_alpha, log_beta, y, as_stream(stream));
}

extern "C" shp_status_t shp_add_leaky_relu(const shp_tensor * a,
                                           const shp_tensor * b,
                                           float              slope,
                                           shp_tensor *       sum,
                                           shp_tensor *       y,
                                           shp_stream_t       stream) {
    if (b == nullptr && sum != nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    EwPlan             plan;
    const shp_status_t st = plan_ew(a, b, false, y, sum, plan);
    if (st != SHP_OK) {
        return st;
    }
    plan.args.slope      = slope;
    const hipStream_t ss = as_stream(stream);
    if (b == nullptr) {
        return launch_ew<kLeaky, false, false, false>(plan.args, plan.flat, plan.vec, ss);
    }
    if (sum == nullptr) {
        return launch_ew<kAddLeaky, true, false, false>(plan.args, plan.flat, plan.vec, ss);
    }
    return launch_ew<kAddLeaky, true, false, true>(plan.args, plan.flat, plan.vec, ss);
}

namespace shp {
namespace {

// ggml_add / ggml_mul / ggml_div with b repeated to a's shape in every other
// form ggml_can_repeat allows (each b->ne[d] divides a->ne[d]; ggml-CPU's
// binary ops read b at (i0 % b.ne0, i1 % b.ne1, i2 % b.ne2, i3 % b.ne3)). The
// graphs' per-channel bias and gain vectors reshaped to [1, C] against a
// time-major [T, C] activation are one value per row: vits/waveform-
// decoder.cpp:120,139, vits/operations.cpp:106,155, qwen3-tts/codec.cpp:180,
// omnivoice/codec.cpp:163, omnivoice/reference-encoder.cpp:135-136.
struct RepeatArgs {
    const float * a;
    RowMap        am;
    float *       y;
    RowMap        ym;
    const char *  b;
    int64_t       bnb1;
    int64_t       bnb2;
    int64_t       bnb3;
    int64_t       brs;    // kRepeatFlat: byte stride between b's values, one per row of a
    FastDiv       ne1;    // a's extents: row r = i1 + ne1*(i2 + ne2*i3)
    FastDiv       ne2;
    FastDiv       bne0;   // b's extents (the repeat periods)
    FastDiv       bne1;
    FastDiv       bne2;
    FastDiv       bne3;
    FastDiv       quads;  // flat kernel: float4 per row of a
    int64_t       nrows;
    int64_t       n4;
    int32_t       ne0;
    int32_t       pad;
};

template <int OP> __device__ __forceinline__ float binop(float a, float b) {
    if constexpr (OP == kAdd) {
        return a + b;
    } else if constexpr (OP == kMul) {
        return a * b;
    } else if constexpr (OP == kSub) {
        return a - b;
    } else {
        static_assert(OP == kDiv, "binary op");
        return a / b;
    }
}

// Byte offset of b's row for row r of a.
__device__ __forceinline__ int64_t repeat_row(const RepeatArgs & g, uint32_t r) {
    const uint32_t q  = fastdiv(r, g.ne1);
    const uint32_t i1 = r - q * g.ne1.d;
    const uint32_t i3 = fastdiv(q, g.ne2);
    const uint32_t i2 = q - i3 * g.ne2.d;
    return static_cast<int64_t>(fastmod(i1, g.bne1)) * g.bnb1 + static_cast<int64_t>(fastmod(i2, g.bne2)) * g.bnb2 +
           static_cast<int64_t>(fastmod(i3, g.bne3)) * g.bnb3;
}

// One value of b per row of a (b.ne0 == 1), a and y contiguous and 16-byte
// aligned with ne0 % 4 == 0: one float4 per lane, as the flat kernels. FLAT:
// b's rows are a's rows one for one at a fixed stride (b = [1, ne1, ne2,
// ne3]), so the row's value is at row * brs.
template <int OP, bool FLAT, int BLOCK> __global__ __launch_bounds__(BLOCK) void k_repeat_col(const RepeatArgs g) {
    const f32x4 * A    = reinterpret_cast<const f32x4 *>(g.a);
    f32x4 *       Y    = reinterpret_cast<f32x4 *>(g.y);
    const int64_t step = static_cast<int64_t>(gridDim.x) * BLOCK;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * BLOCK + threadIdx.x; e < g.n4; e += step) {
        const uint32_t r  = fastdiv(static_cast<uint32_t>(e), g.quads);
        const int64_t  bo = FLAT ? static_cast<int64_t>(r) * g.brs : repeat_row(g, r);
        const float    bv = *reinterpret_cast<const float *>(g.b + bo);
        const f32x4    av = ld_stream(A + e);
        st_stream(Y + e, f32x4{ binop<OP>(av.x, bv), binop<OP>(av.y, bv), binop<OP>(av.z, bv), binop<OP>(av.w, bv) });
    }
}

// Any repeat form and any row strides: rows over blocks, elements over threads.
template <int OP> __global__ __launch_bounds__(256) void k_repeat_rows(const RepeatArgs g) {
    for (int64_t r = blockIdx.x; r < g.nrows; r += gridDim.x) {
        const float * ar = reinterpret_cast<const float *>(reinterpret_cast<const char *>(g.a) + row_offset(g.am, r));
        float *       yr = reinterpret_cast<float *>(reinterpret_cast<char *>(g.y) + row_offset(g.ym, r));
        const float * br = reinterpret_cast<const float *>(g.b + repeat_row(g, static_cast<uint32_t>(r)));
        for (int i = static_cast<int>(threadIdx.x); i < g.ne0; i += 256) {
            yr[i] = binop<OP>(ar[i], br[fastmod(static_cast<uint32_t>(i), g.bne0)]);
        }
    }
}

template <int OP>
shp_status_t repeat_entry(const shp_tensor * a, const shp_tensor * b, shp_tensor * y, shp_stream_t stream) {
    if (!well_formed(a) || !well_formed(b) || !well_formed(y)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (a->type != SHP_TYPE_F32 || b->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (!same_shape(*a, *y) || !can_repeat(*b, *a)) {
        return SHP_ERR_INVALID_ARG;
    }
    const int64_t rows = nrows(*a);
    if (a->ne[0] > INT32_MAX || rows >= (int64_t{ 1 } << 32) || nelements(*a) >= (int64_t{ 1 } << 32)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (dry_run()) {
        return SHP_OK;
    }
    RepeatArgs g{};
    g.a     = static_cast<const float *>(a->data);
    g.am    = make_rowmap(*a);
    g.y     = static_cast<float *>(y->data);
    g.ym    = make_rowmap(*y);
    g.b     = static_cast<const char *>(b->data);
    g.bnb1  = static_cast<int64_t>(b->nb[1]);
    g.bnb2  = static_cast<int64_t>(b->nb[2]);
    g.bnb3  = static_cast<int64_t>(b->nb[3]);
    g.ne1   = make_fastdiv(static_cast<uint32_t>(a->ne[1]));
    g.ne2   = make_fastdiv(static_cast<uint32_t>(a->ne[2]));
    g.bne0  = make_fastdiv(static_cast<uint32_t>(b->ne[0]));
    g.bne1  = make_fastdiv(static_cast<uint32_t>(b->ne[1]));
    g.bne2  = make_fastdiv(static_cast<uint32_t>(b->ne[2]));
    g.bne3  = make_fastdiv(static_cast<uint32_t>(b->ne[3]));
    g.nrows = rows;
    g.ne0   = static_cast<int32_t>(a->ne[0]);
    g.n4    = nelements(*a) / 4;
    const hipStream_t ss   = as_stream(stream);
    const bool        flat = b->ne[0] == 1 && a->ne[0] % 4 == 0 && contiguous(*a) && contiguous(*y) &&
                      rows_aligned(*a, 16) && rows_aligned(*y, 16);
    if (flat) {
        g.quads = make_fastdiv(static_cast<uint32_t>(a->ne[0] / 4));
        // b's rows one for one with a's at a fixed stride: b = [1, ne1, ne2, ne3]
        const RowMap bm       = make_rowmap(*b);
        const bool   one_one  = b->ne[1] == a->ne[1] && b->ne[2] == a->ne[2] && b->ne[3] == a->ne[3] && bm.flat;
        g.brs                 = bm.rs;
        const bool    wave    = g.n4 >= kFlatWaveBlocksFrom;
        const int     bs      = wave ? kWave : 256;
        int64_t       blocks  = (g.n4 + bs - 1) / bs;
        blocks                = blocks < kMaxFlatBlocks ? blocks : kMaxFlatBlocks;
        const unsigned grid   = static_cast<unsigned>(blocks);
        if (one_one) {
            if (wave) {
                hipLaunchKernelGGL((k_repeat_col<OP, true, kWave>), dim3(grid), dim3(kWave), 0, ss, g);
            } else {
                hipLaunchKernelGGL((k_repeat_col<OP, true, 256>), dim3(grid), dim3(256), 0, ss, g);
            }
        } else {
            if (wave) {
                hipLaunchKernelGGL((k_repeat_col<OP, false, kWave>), dim3(grid), dim3(kWave), 0, ss, g);
            } else {
                hipLaunchKernelGGL((k_repeat_col<OP, false, 256>), dim3(grid), dim3(256), 0, ss, g);
            }
        }
        return launch_status();
    }
    const int64_t blocks = rows < 65536 ? rows : 65536;
    hipLaunchKernelGGL((k_repeat_rows<OP>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, ss, g);
    return launch_status();
}

// ggml_add / ggml_mul / ggml_div: b the same shape as a, one row of ne0
// elements repeated over every row, or any other shape that repeats to a's.
template <int OP>
shp_status_t binary_entry(const shp_tensor * a, const shp_tensor * b, shp_tensor * y, shp_stream_t stream) {
    if (b == nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    if (a != nullptr && well_formed(a) && well_formed(b) && !same_shape(*a, *b) && !one_row_of(*b, a->ne[0])) {
        return repeat_entry<OP>(a, b, y, stream);
    }
    EwPlan             plan;
    const shp_status_t st = plan_ew(a, b, true, y, nullptr, plan);
    if (st != SHP_OK) {
        return st;
    }
    const hipStream_t ss = as_stream(stream);
    if (plan.bcast) {
        const bool b16 = reinterpret_cast<uintptr_t>(b->data) % 16 == 0;
        return launch_ew<OP, true, true, false>(plan.args, plan.flat && b16, plan.vec && b16, ss);
    }
    return launch_ew<OP, true, false, false>(plan.args, plan.flat, plan.vec, ss);
}

template <int OP> shp_status_t unary_entry(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    EwPlan             plan;
    const shp_status_t st = plan_ew(x, nullptr, false, y, nullptr, plan);
    if (st != SHP_OK) {
        return st;
    }
    return launch_ew<OP, false, false, false>(plan.args, plan.flat, plan.vec, as_stream(stream));
}

// ggml_cpy / ggml_cast of an F16 or BF16 tensor into F32 of the same shape:
// one exact conversion per element, rows addressed through their byte strides.
// (The weight casts of as_f32, qwen3-tts/operations.cpp:20-25, when they are
// not folded into the norm that reads the gain.)
struct CastArgs {
    const void * x;
    RowMap       xm;
    float *      y;
    RowMap       ym;
    int64_t      nrows;
    int32_t      ne0;
    int32_t      pad;
};

template <int TYPE> __global__ __launch_bounds__(256) void k_cast_rows(const CastArgs a) {
    for (int64_t r = blockIdx.x; r < a.nrows; r += gridDim.x) {
        const uint16_t * xr =
            reinterpret_cast<const uint16_t *>(static_cast<const char *>(a.x) + row_offset(a.xm, r));
        float * yr = reinterpret_cast<float *>(reinterpret_cast<char *>(a.y) + row_offset(a.ym, r));
        for (int c = static_cast<int>(threadIdx.x); c < a.ne0; c += 256) {
            const uint32_t h = xr[c];
            yr[c]            = TYPE == SHP_TYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
        }
    }
}

// ggml_cont / ggml_cpy of an F32 view whose contiguous dimension is k in 1..3
// (what ggml_transpose and ggml_permute leave: the vocoder's time-major
// copies around each convolution, vits/operations.cpp:72,87,100,108) into a
// row-contiguous F32 tensor of the same shape. y[i0,i1,i2,i3] =
// x[i0,i1,i2,i3], one 64 (dim 0) x 128 (dim k) tile per block pass through
// LDS: the loads read 512-byte source lines along dim k, the stores write
// 256-byte destination lines along dim 0. Consecutive blocks take the tiles of
// one dim-0 range along dim k first; the other two dimensions (a, b) number
// the tiles last. V = 4: 16-byte accesses (every stride and both extents
// allow it); V = 1 otherwise.
// Measured on MI355X (cold inputs, the vocoder shapes [C,T] = [128,131072],
// [256,32768], [512,8192]): 25.2 / 13.6 / 6.4 us, against 29.6 / 13.7 / 7.5 us
// for 64 x 64 tiles with dim 0 first, 27.3 / 14.3 / 6.7 us with tiles spread
// over the XCDs in contiguous ranges, and 26.1-27.9 / 14.1-14.7 / 6.7-7.9 us
// with either access left cacheable.
struct TransposeArgs {
    const char * x;
    char *       y;
    int64_t      xnb0;  // source stride of dim 0 (dim k has stride 4)
    int64_t      xnba;
    int64_t      xnbb;
    int64_t      ynbk;  // destination strides (dim 0 has stride 4)
    int64_t      ynba;
    int64_t      ynbb;
    int64_t      ne0;
    int64_t      nek;
    FastDiv      tk;    // tiles along dim k
    FastDiv      t0;    // tiles along dim 0
    FastDiv      na;    // extent of dim a
    uint32_t     ntiles;
    uint32_t     pad;
    // epilogue (shp_cont_add_leaky_relu)
    const char * bias;   // one value per destination row, at row number * brs
    int64_t      brs;
    int64_t      rowk;   // destination row number per unit of dims k, a, b
    int64_t      rowa;
    int64_t      rowb;
    int64_t      rdelta;  // residual address - destination address (same layout)
    int64_t      sdelta;  // sum address - destination address (same layout)
    float        slope;
    int32_t      pad2;
};

constexpr int kTile0 = 64;
constexpr int kTileK = 128;

// Epilogue bits: add the bias -- the destination row's value (kEpiBias) or
// one value per destination column, a row of ne0 repeated over the rows
// (kEpiBias0) -- then the residual (a second rounding, in the node order),
// write that sum, apply leaky-ReLU.
enum TransposeEpi { kEpiBias = 1, kEpiResid = 2, kEpiLeaky = 4, kEpiSum = 8, kEpiBias0 = 16 };

// One tile: loads into registers, LDS, stores. FULL = the tile lies wholly
// inside the tensor: no guards, so each load's data goes to LDS as it arrives
// and the LDS reads of two passes issue before their stores. The epilogue's
// bias values and residual rows are requested with the tile's loads, before
// the barrier.
template <int V, bool FULL, int EPI>
__device__ __forceinline__ void transpose_tile(float (&tile)[kTile0][kTileK + 1], float (&s_bias)[kTileK],
                                               const TransposeArgs & a, const char * xb, char * yb, int64_t i0,
                                               int64_t row0, int n0, int nk) {
    typedef float vec __attribute__((ext_vector_type(V)));
    constexpr int RL = kTileK / V, RLINES = 256 / RL, RPASS = kTile0 / RLINES;  // loads: lines along dim k
    constexpr int WL = kTile0 / V, WLINES = 256 / WL, WPASS = kTileK / WLINES;  // stores: lines along dim 0
    const int     rc = (static_cast<int>(threadIdx.x) % RL) * V, rl = static_cast<int>(threadIdx.x) / RL;
    const int     wc = (static_cast<int>(threadIdx.x) % WL) * V, wl = static_cast<int>(threadIdx.x) / WL;
    vec           v[RPASS];
#pragma unroll
    for (int p = 0; p < RPASS; ++p) {
        const int r = rl + p * RLINES;
        if (FULL || (r < n0 && rc < nk)) {
            v[p] = __builtin_nontemporal_load(reinterpret_cast<const vec *>(xb + static_cast<int64_t>(r) * a.xnb0 + rc * 4));
        } else {
            v[p] = vec{};
        }
    }
    // The tile's 128 destination lines take one bias value each: one load per
    // line into LDS (8 loads per lane otherwise: measured 3-9 % slower).
    if constexpr ((EPI & kEpiBias) != 0) {
        const int r = static_cast<int>(threadIdx.x);
        if (r < kTileK) {
            const int rr = r < nk ? r : 0;  // a line past the tensor reads line 0's value, unused
            s_bias[r]    = *reinterpret_cast<const float *>(a.bias + (row0 + rr * a.rowk) * a.brs);
        }
    }
    // kEpiBias0: the lane's V columns are the same in every pass: one load
    // (b is one contiguous row of ne0 values).
    vec b0{};
    if constexpr ((EPI & kEpiBias0) != 0) {
        if (FULL || wc < n0) {
            b0 = *reinterpret_cast<const vec *>(a.bias + (i0 + wc) * 4);
        }
    }
    vec rv[WPASS];
#pragma unroll
    for (int p = 0; p < WPASS; ++p) {
        const int  r  = wl + p * WLINES;  // ik local
        const bool in = FULL || (r < nk && wc < n0);
        if constexpr ((EPI & kEpiResid) != 0) {
            rv[p] = in ? __builtin_nontemporal_load(
                             reinterpret_cast<const vec *>(yb + a.rdelta + static_cast<int64_t>(r) * a.ynbk + wc * 4)) :
                         vec{};
        }
    }
#pragma unroll
    for (int p = 0; p < RPASS; ++p) {
#pragma unroll
        for (int e = 0; e < V; ++e) {
            tile[rl + p * RLINES][rc + e] = v[p][e];
        }
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < WPASS; ++p) {
        const int   r  = wl + p * WLINES;  // ik local
        const float bv = (EPI & kEpiBias) != 0 ? s_bias[r] : 0.0f;
        vec         w;
#pragma unroll
        for (int e = 0; e < V; ++e) {
            w[e] = tile[wc + e][r];
            if constexpr ((EPI & kEpiBias) != 0) {
                w[e] = w[e] + bv;
            }
            if constexpr ((EPI & kEpiBias0) != 0) {
                w[e] = w[e] + b0[e];
            }
            if constexpr ((EPI & kEpiResid) != 0) {
                w[e] = w[e] + rv[p][e];
            }
        }
        if (FULL || (r < nk && wc < n0)) {
            char * yo = yb + static_cast<int64_t>(r) * a.ynbk + wc * 4;
            if constexpr ((EPI & kEpiSum) != 0) {
                __builtin_nontemporal_store(w, reinterpret_cast<vec *>(yo + a.sdelta));
            }
            if constexpr ((EPI & kEpiLeaky) != 0) {
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    w[e] = leaky(w[e], a.slope);
                }
            }
            __builtin_nontemporal_store(w, reinterpret_cast<vec *>(yo));
        }
    }
    __syncthreads();
}

template <int V, int EPI> __global__ __launch_bounds__(256) void k_transpose_tiles(const TransposeArgs a) {
    __shared__ float tile[kTile0][kTileK + 1];  // [i0 local][ik local]; the pad staggers a column's banks
    __shared__ float s_bias[kTileK];              // the epilogue's bias value per destination line
    for (uint32_t t = blockIdx.x; t < a.ntiles; t += gridDim.x) {
        const uint32_t q0   = fastdiv(t, a.tk);
        const uint32_t q1   = fastdiv(q0, a.t0);
        const uint32_t ib   = fastdiv(q1, a.na);
        const int64_t  ik   = static_cast<int64_t>(t - q0 * a.tk.d) * kTileK;
        const int64_t  i0   = static_cast<int64_t>(q0 - q1 * a.t0.d) * kTile0;
        const int64_t  ia   = q1 - ib * a.na.d;
        const char *   xb   = a.x + i0 * a.xnb0 + ik * 4 + ia * a.xnba + ib * a.xnbb;
        char *         yb   = a.y + i0 * 4 + ik * a.ynbk + ia * a.ynba + ib * a.ynbb;
        const int64_t  row0 = ik * a.rowk + ia * a.rowa + ib * a.rowb;  // destination row number at ik
        const int      n0   = static_cast<int>(a.ne0 - i0 < kTile0 ? a.ne0 - i0 : kTile0);
        const int      nk   = static_cast<int>(a.nek - ik < kTileK ? a.nek - ik : kTileK);
        if (n0 == kTile0 && nk == kTileK) {
            transpose_tile<V, true, EPI>(tile, s_bias, a, xb, yb, i0, row0, n0, nk);
        } else {
            transpose_tile<V, false, EPI>(tile, s_bias, a, xb, yb, i0, row0, n0, nk);
        }
    }
}

// The transposing copy's plan: dims, tiles, strides, and whether 16-byte
// accesses apply (every line start on both sides 16-byte aligned and both tile
// extents multiples of 4; the stride of a dimension of extent 1 is never
// used). SHP_ERR_UNSUPPORTED when x has no contiguous dimension or the tile
// count passes 2^31.
struct TransposePlan {
    TransposeArgs args{};
    bool          v4    = false;
    unsigned      grid  = 0;
    int           k     = 0;
    int           da    = 0;
    int           db    = 0;
};

shp_status_t plan_transpose(const shp_tensor * x, const shp_tensor * y, TransposePlan & pl) {
    const int k = f32_strided_view_dim(x);
    if (k == 0 || !well_formed(y) || y->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (!same_shape(*x, *y)) {
        return SHP_ERR_INVALID_ARG;
    }
    // A tile's stores land where other tiles still read: y must not overlap x.
    if (spans_overlap(*x, *y)) {
        return SHP_ERR_UNSUPPORTED;
    }
    int dims[2], n = 0;
    for (int d = 1; d < 4; ++d) {
        if (d != k) {
            dims[n++] = d;
        }
    }
    const int64_t t0 = (x->ne[0] + kTile0 - 1) / kTile0;
    const int64_t tk = (x->ne[k] + kTileK - 1) / kTileK;
    const int64_t nt = t0 * tk * x->ne[dims[0]] * x->ne[dims[1]];
    if (t0 > INT32_MAX || tk > INT32_MAX || nt > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    TransposeArgs & a = pl.args;
    a.x               = static_cast<const char *>(x->data);
    a.y               = static_cast<char *>(y->data);
    a.xnb0            = static_cast<int64_t>(x->nb[0]);
    a.xnba            = static_cast<int64_t>(x->nb[dims[0]]);
    a.xnbb            = static_cast<int64_t>(x->nb[dims[1]]);
    a.ynbk            = static_cast<int64_t>(y->nb[k]);
    a.ynba            = static_cast<int64_t>(y->nb[dims[0]]);
    a.ynbb            = static_cast<int64_t>(y->nb[dims[1]]);
    a.ne0             = x->ne[0];
    a.nek             = x->ne[k];
    a.t0              = make_fastdiv(static_cast<uint32_t>(t0));
    a.tk              = make_fastdiv(static_cast<uint32_t>(tk));
    a.na              = make_fastdiv(static_cast<uint32_t>(x->ne[dims[0]]));
    a.ntiles          = static_cast<uint32_t>(nt);
    const int64_t rownum[4] = { 0, 1, y->ne[1], y->ne[1] * y->ne[2] };  // row number per unit of dims 1..3
    a.rowk                  = rownum[k];
    a.rowa                  = rownum[dims[0]];
    a.rowb                  = rownum[dims[1]];
    const auto    a16 = [](int64_t ne, int64_t nb) { return ne == 1 || nb % 16 == 0; };
    const int64_t nea = x->ne[dims[0]], neb = x->ne[dims[1]];
    pl.v4             = reinterpret_cast<uintptr_t>(x->data) % 16 == 0 &&
             reinterpret_cast<uintptr_t>(y->data) % 16 == 0 && a16(a.ne0, a.xnb0) && a16(nea, a.xnba) &&
             a16(neb, a.xnbb) && a16(a.nek, a.ynbk) && a16(nea, a.ynba) && a16(neb, a.ynbb) && a.ne0 % 4 == 0 &&
             a.nek % 4 == 0;
    pl.grid = static_cast<unsigned>(nt < (1 << 20) ? nt : (1 << 20));
    pl.k    = k;
    pl.da   = dims[0];
    pl.db   = dims[1];
    return SHP_OK;
}

template <int EPI> shp_status_t launch_transpose(const TransposePlan & pl, hipStream_t stream) {
    if (pl.v4) {
        hipLaunchKernelGGL((k_transpose_tiles<4, EPI>), dim3(pl.grid), dim3(256), 0, stream, pl.args);
    } else {
        hipLaunchKernelGGL((k_transpose_tiles<1, EPI>), dim3(pl.grid), dim3(256), 0, stream, pl.args);
    }
    return launch_status();
}

shp_status_t transpose_entry(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    TransposePlan      pl;
    const shp_status_t st = plan_transpose(x, y, pl);
    if (st != SHP_OK || dry_run()) {
        return st;
    }
    return launch_transpose<0>(pl, as_stream(stream));
}

// ggml_concat: each destination row comes from a or b (dim >= 1) or is a's
// row followed by b's (dim 0); rows over blocks, elements over threads.
struct ConcatArgs {
    const char * a;
    const char * b;
    char *       y;
    int64_t      anb[4];
    int64_t      bnb[4];
    int64_t      ynb[4];
    int64_t      ane[4];
    int64_t      yne[4];
    int64_t      nrows;
    int32_t      dim;
    int32_t      pad;
};

__global__ __launch_bounds__(256) void k_concat_rows(const ConcatArgs g) {
    for (int64_t r = blockIdx.x; r < g.nrows; r += gridDim.x) {
        int64_t       i[4] = { 0, r % g.yne[1], (r / g.yne[1]) % g.yne[2], r / (g.yne[1] * g.yne[2]) };
        char *        yr   = g.y + i[1] * g.ynb[1] + i[2] * g.ynb[2] + i[3] * g.ynb[3];
        const int64_t ne0  = g.yne[0];
        if (g.dim == 0) {
            const float * ar = reinterpret_cast<const float *>(g.a + i[1] * g.anb[1] + i[2] * g.anb[2] + i[3] * g.anb[3]);
            const float * br = reinterpret_cast<const float *>(g.b + i[1] * g.bnb[1] + i[2] * g.bnb[2] + i[3] * g.bnb[3]);
            const int64_t na = g.ane[0];
            for (int64_t c = threadIdx.x; c < ne0; c += 256) {
                reinterpret_cast<float *>(yr)[c] = c < na ? ar[c] : br[c - na];
            }
            continue;
        }
        const bool   from_a = i[g.dim] < g.ane[g.dim];
        const char * src;
        if (from_a) {
            src = g.a + i[1] * g.anb[1] + i[2] * g.anb[2] + i[3] * g.anb[3];
        } else {
            i[g.dim] -= g.ane[g.dim];
            src = g.b + i[1] * g.bnb[1] + i[2] * g.bnb[2] + i[3] * g.bnb[3];
        }
        for (int64_t c = threadIdx.x; c < ne0; c += 256) {
            reinterpret_cast<float *>(yr)[c] = reinterpret_cast<const float *>(src)[c];
        }
    }
}

}  // namespace
}  // namespace shp

extern "C" shp_status_t shp_concat(const shp_tensor * a, const shp_tensor * b, int32_t dim, shp_tensor * y,
                                   shp_stream_t stream) {
    if (!well_formed(a) || !well_formed(b) || !well_formed(y) || dim < 0 || dim > 3) {
        return SHP_ERR_INVALID_ARG;
    }
    if (a->type != SHP_TYPE_F32 || b->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    for (int d = 0; d < 4; ++d) {
        const int64_t want = d == dim ? a->ne[d] + b->ne[d] : a->ne[d];
        if (y->ne[d] != want || (d != dim && b->ne[d] != a->ne[d])) {
            return SHP_ERR_INVALID_ARG;
        }
    }
    if (spans_overlap(*a, *y) || spans_overlap(*b, *y)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (dry_run()) {
        return SHP_OK;
    }
    ConcatArgs g{};
    g.a   = static_cast<const char *>(a->data);
    g.b   = static_cast<const char *>(b->data);
    g.y   = static_cast<char *>(y->data);
    g.dim = dim;
    for (int d = 0; d < 4; ++d) {
        g.anb[d] = static_cast<int64_t>(a->nb[d]);
        g.bnb[d] = static_cast<int64_t>(b->nb[d]);
        g.ynb[d] = static_cast<int64_t>(y->nb[d]);
        g.ane[d] = a->ne[d];
        g.yne[d] = y->ne[d];
    }
    g.nrows              = nrows(*y);
    const int64_t blocks = g.nrows < 65536 ? g.nrows : 65536;
    hipLaunchKernelGGL(k_concat_rows, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream), g);
    return launch_status();
}

extern "C" shp_status_t shp_add(const shp_tensor * a, const shp_tensor * b, shp_tensor * y, shp_stream_t stream) {
    return binary_entry<kAdd>(a, b, y, stream);
}

extern "C" shp_status_t shp_mul(const shp_tensor * a, const shp_tensor * b, shp_tensor * y, shp_stream_t stream) {
    return binary_entry<kMul>(a, b, y, stream);
}

extern "C" shp_status_t shp_div(const shp_tensor * a, const shp_tensor * b, shp_tensor * y, shp_stream_t stream) {
    return binary_entry<kDiv>(a, b, y, stream);
}

extern "C" shp_status_t shp_sub(const shp_tensor * a, const shp_tensor * b, shp_tensor * y, shp_stream_t stream) {
    return binary_entry<kSub>(a, b, y, stream);
}

extern "C" shp_status_t shp_tanh(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return unary_entry<kTanh>(x, y, stream);
}

extern "C" shp_status_t shp_sigmoid(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return unary_entry<kSigmoid>(x, y, stream);
}

extern "C" shp_status_t shp_elu(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return unary_entry<kElu>(x, y, stream);
}

extern "C" shp_status_t shp_gelu_erf(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return unary_entry<kGeluErf>(x, y, stream);
}

extern "C" shp_status_t shp_relu(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return unary_entry<kRelu>(x, y, stream);
}

extern "C" shp_status_t shp_neg(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return unary_entry<kNeg>(x, y, stream);
}

extern "C" shp_status_t shp_step(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return unary_entry<kStep>(x, y, stream);
}

extern "C" shp_status_t shp_sqrt(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return unary_entry<kSqrt>(x, y, stream);
}

extern "C" shp_status_t shp_clamp(const shp_tensor * x, float lo, float hi, shp_tensor * y, shp_stream_t stream) {
    EwPlan             plan;
    const shp_status_t st = plan_ew(x, nullptr, false, y, nullptr, plan);
    if (st != SHP_OK) {
        return st;
    }
    plan.args.scale = lo;
    plan.args.bias  = hi;
    return launch_ew<kClamp, false, false, false>(plan.args, plan.flat, plan.vec, as_stream(stream));
}

extern "C" shp_status_t shp_sin(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return unary_entry<kSin>(x, y, stream);
}

extern "C" shp_status_t shp_sqr(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return unary_entry<kSqr>(x, y, stream);
}

extern "C" shp_status_t shp_cpy(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    if (f32_strided_view_dim(x) != 0) {
        return transpose_entry(x, y, stream);
    }
    if (!well_formed(x) || !well_formed(y)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (y->type != SHP_TYPE_F32 || (x->type != SHP_TYPE_F32 && x->type != SHP_TYPE_F16 && x->type != SHP_TYPE_BF16)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (!same_shape(*x, *y) || x->ne[0] > INT32_MAX) {
        return SHP_ERR_INVALID_ARG;
    }
    if (x->type == SHP_TYPE_F32) {
        return unary_entry<kCopy>(x, y, stream);
    }
    if (dry_run()) {
        return SHP_OK;
    }
    CastArgs a{};
    a.x              = x->data;
    a.xm             = make_rowmap(*x);
    a.y              = static_cast<float *>(y->data);
    a.ym             = make_rowmap(*y);
    a.nrows          = nrows(*x);
    a.ne0            = static_cast<int32_t>(x->ne[0]);
    const int64_t bl = a.nrows < 65536 ? a.nrows : 65536;
    if (x->type == SHP_TYPE_BF16) {
        hipLaunchKernelGGL((k_cast_rows<SHP_TYPE_BF16>), dim3(static_cast<unsigned>(bl)), dim3(256), 0,
                           as_stream(stream), a);
    } else {
        hipLaunchKernelGGL((k_cast_rows<SHP_TYPE_F16>), dim3(static_cast<unsigned>(bl)), dim3(256), 0,
                           as_stream(stream), a);
    }
    return launch_status();
}

extern "C" shp_status_t shp_cont_add_leaky_relu(const shp_tensor * x,
                                                const shp_tensor * b,
                                                const shp_tensor * r,
                                                int32_t            apply_leaky,
                                                float              slope,
                                                shp_tensor *       sum,
                                                shp_tensor *       y,
                                                shp_stream_t       stream) {
    if (b == nullptr || !well_formed(b) || !well_formed(y) || (r != nullptr && !well_formed(r)) ||
        (sum != nullptr && !well_formed(sum)) || (sum != nullptr && !apply_leaky)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (b->type != SHP_TYPE_F32 || (r != nullptr && r->type != SHP_TYPE_F32) ||
        (sum != nullptr && sum->type != SHP_TYPE_F32)) {
        return SHP_ERR_UNSUPPORTED;
    }
    TransposePlan      pl;
    const shp_status_t st = plan_transpose(x, y, pl);
    if (st != SHP_OK) {
        return st;
    }
    // b: one value per row of y, b's rows one for one at a fixed stride
    // (ggml_add(cont, reshape_2d(bias, 1, C)), vits/waveform-decoder.cpp:118-121),
    // or one row of ne0 values repeated over y's rows (the channel bias of a
    // channel-major result, qwen3-tts/codec.cpp:58-59,134-140,179-181);
    // r and sum: y's shape and strides (the residual and the add's result).
    const RowMap bm      = make_rowmap(*b);
    const bool   per_row = b->ne[0] == 1 && b->ne[1] == y->ne[1] && b->ne[2] == y->ne[2] && b->ne[3] == y->ne[3] &&
                         bm.flat;
    const bool   per_col = !per_row && one_row_of(*b, y->ne[0]);
    if (!per_row && !per_col) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (per_col && reinterpret_cast<uintptr_t>(b->data) % 16 != 0) {
        pl.v4 = false;
    }
    const auto same_layout = [y](const shp_tensor * t) {
        return same_shape(*t, *y) && t->nb[1] == y->nb[1] && t->nb[2] == y->nb[2] && t->nb[3] == y->nb[3];
    };
    if ((r != nullptr && !same_layout(r)) || (sum != nullptr && !same_layout(sum))) {
        return SHP_ERR_UNSUPPORTED;
    }
    // Each element of r is read by the lane that writes that element of y and
    // sum, so r may be y or sum itself (an in-place add); any other overlap
    // among x, r, sum and y is refused.
    const auto apart = [](const shp_tensor * p, const shp_tensor * q) {
        return p == nullptr || q == nullptr || !spans_overlap(*p, *q);
    };
    if (!apart(x, r) || !apart(x, sum) || (sum != nullptr && !apart(sum, y)) ||
        (r != nullptr && r->data != y->data && !apart(r, y)) ||
        (r != nullptr && sum != nullptr && r->data != sum->data && !apart(r, sum))) {
        return SHP_ERR_UNSUPPORTED;
    }
    if ((r != nullptr && reinterpret_cast<uintptr_t>(r->data) % 16 != 0) ||
        (sum != nullptr && reinterpret_cast<uintptr_t>(sum->data) % 16 != 0)) {
        pl.v4 = false;
    }
    if (dry_run()) {
        return SHP_OK;
    }
    TransposeArgs & a = pl.args;
    a.bias            = static_cast<const char *>(b->data);
    a.brs             = bm.rs;
    a.slope           = slope;
    a.rdelta          = r != nullptr ? static_cast<const char *>(r->data) - static_cast<const char *>(y->data) : 0;
    a.sdelta          = sum != nullptr ? static_cast<const char *>(sum->data) - static_cast<const char *>(y->data) : 0;
    const hipStream_t ss = as_stream(stream);
    const int rest = (r != nullptr ? kEpiResid : 0) | (apply_leaky ? kEpiLeaky : 0) | (sum != nullptr ? kEpiSum : 0);
    if (per_col) {
        switch (rest) {
            case 0:
                return launch_transpose<kEpiBias0>(pl, ss);
            case kEpiLeaky:
                return launch_transpose<kEpiBias0 | kEpiLeaky>(pl, ss);
            case kEpiLeaky | kEpiSum:
                return launch_transpose<kEpiBias0 | kEpiLeaky | kEpiSum>(pl, ss);
            case kEpiResid:
                return launch_transpose<kEpiBias0 | kEpiResid>(pl, ss);
            case kEpiResid | kEpiLeaky:
                return launch_transpose<kEpiBias0 | kEpiResid | kEpiLeaky>(pl, ss);
            default:
                return launch_transpose<kEpiBias0 | kEpiResid | kEpiLeaky | kEpiSum>(pl, ss);
        }
    }
    const int epi = kEpiBias | rest;
    switch (epi) {
        case kEpiBias:
            return launch_transpose<kEpiBias>(pl, ss);
        case kEpiBias | kEpiLeaky:
            return launch_transpose<kEpiBias | kEpiLeaky>(pl, ss);
        case kEpiBias | kEpiLeaky | kEpiSum:
            return launch_transpose<kEpiBias | kEpiLeaky | kEpiSum>(pl, ss);
        case kEpiBias | kEpiResid:
            return launch_transpose<kEpiBias | kEpiResid>(pl, ss);
        case kEpiBias | kEpiResid | kEpiLeaky:
            return launch_transpose<kEpiBias | kEpiResid | kEpiLeaky>(pl, ss);
        default:
            return launch_transpose<kEpiBias | kEpiResid | kEpiLeaky | kEpiSum>(pl, ss);
    }
}

extern "C" shp_status_t shp_exp(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    return unary_entry<kExp>(x, y, stream);
}

extern "C" shp_status_t shp_scale_bias(const shp_tensor * x, float s, float b, shp_tensor * y, shp_stream_t stream) {
    EwPlan             plan;
    const shp_status_t st = plan_ew(x, nullptr, false, y, nullptr, plan);
    if (st != SHP_OK) {
        return st;
    }
    plan.args.scale      = s;
    plan.args.bias       = b;
    const hipStream_t ss = as_stream(stream);
    if (b == 0.0f) {
        return launch_ew<kScale, false, false, false>(plan.args, plan.flat, plan.vec, ss);
    }
    return launch_ew<kScaleBias, false, false, false>(plan.args, plan.flat, plan.vec, ss);
}

extern "C" shp_status_t shp_sum_scale_leaky_relu(const shp_tensor * terms,
                                                 int32_t            n_terms,
                                                 float              scale,
                                                 float              slope,
                                                 shp_tensor *       mean,
                                                 shp_tensor *       y,
                                                 shp_stream_t       stream) {
    if (terms == nullptr || n_terms < 1 || n_terms > kMaxTerms || !well_formed(y) ||
        (mean != nullptr && !well_formed(mean))) {
        return SHP_ERR_INVALID_ARG;
    }
    TermArgs a{};
    bool     vec = reinterpret_cast<uintptr_t>(y->data) % 16 == 0 && y->ne[0] % 4 == 0;
    for (int j = 0; j < n_terms; ++j) {
        const shp_tensor * t = &terms[j];
        if (!well_formed(t)) {
            return SHP_ERR_INVALID_ARG;
        }
        if (t->type != SHP_TYPE_F32) {
            return SHP_ERR_UNSUPPORTED;
        }
        if (!same_shape(*t, *y)) {
            return SHP_ERR_INVALID_ARG;
        }
        if (!contiguous(*t)) {
            return SHP_ERR_UNSUPPORTED;
        }
        a.t[j] = static_cast<const float *>(t->data);
        vec    = vec && reinterpret_cast<uintptr_t>(t->data) % 16 == 0;
    }
    if (y->type != SHP_TYPE_F32 || (mean != nullptr && mean->type != SHP_TYPE_F32)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (mean != nullptr && !same_shape(*mean, *y)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (!contiguous(*y) || (mean != nullptr && !contiguous(*mean))) {
        return SHP_ERR_UNSUPPORTED;
    }
    const int64_t n = nelements(*y);
    vec             = vec && (mean == nullptr || reinterpret_cast<uintptr_t>(mean->data) % 16 == 0);
    a.y     = static_cast<float *>(y->data);
    a.m     = mean != nullptr ? static_cast<float *>(mean->data) : nullptr;
    a.n     = vec ? n / 4 : n;
    a.scale = scale;
    a.slope = slope;
    const hipStream_t ss = as_stream(stream);
    switch (n_terms) {
        case 1: return launch_sum_scale_leaky<1>(a, vec, ss);
        case 2: return launch_sum_scale_leaky<2>(a, vec, ss);
        case 3: return launch_sum_scale_leaky<3>(a, vec, ss);
        case 4: return launch_sum_scale_leaky<4>(a, vec, ss);
        case 5: return launch_sum_scale_leaky<5>(a, vec, ss);
        case 6: return launch_sum_scale_leaky<6>(a, vec, ss);
        case 7: return launch_sum_scale_leaky<7>(a, vec, ss);
        default: return launch_sum_scale_leaky<8>(a, vec, ss);
    }
}

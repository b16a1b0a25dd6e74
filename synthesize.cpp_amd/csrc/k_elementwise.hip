// Elementwise primitives for gfx950: SwiGLU (silu(g)*u), bare silu, the
// single-tensor GLU, Snake, add->leaky-ReLU with the residual carried out, bare
// leaky-ReLU, and the plain residual add.
//
// Each fused op reproduces the f32 rounding sequence of the unfused ggml node
// run it replaces (compiled with -ffp-contract=off, IEEE divide, full-range
// OCML expf/sinf), so the only difference from ggml-CPU is the last ulp of the
// transcendental itself.
//
// Two launch shapes: a flat kernel for fully contiguous, 16-byte aligned
// tensors (the large vocoder and MLP tensors), one float4 per lane per operand;
// and a row kernel that follows ggml byte strides for any other view. Both
// stream activations with nontemporal loads and stores.

#include <cmath>

#include "shp_div.hpp"
#include "shp_internal.hpp"
#include "shp_sinf.hpp"

namespace shp {
namespace {

enum EwOp { kSwiglu = 0, kSilu = 1, kAdd = 2, kAddLeaky = 3, kLeaky = 4, kSnake = 5 };

struct EwArgs {
    const float * a;
    RowMap        am;
    const float * b;
    RowMap        bm;
    float *       y;
    RowMap        ym;
    float *       s;
    RowMap        sm;
    const float * alpha;
    int64_t       nrows;
    int64_t       n4;
    int32_t       ne0;
    FastDiv       period;  // flat path: row length, to index a broadcast row (alpha or b)
    FastDiv       quads;   // Snake flat path: float4 per row (ne0/4)
    int64_t       ntask;   // Snake flat path: lanes = row blocks x quads per row
    float         slope;
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

// One element of the op. `b` is the second input (or the broadcast row value),
// `al` the Snake channel coefficient; `s` receives the carried sum.
template <int OP> __device__ __forceinline__ float ew(float a, float b, float al, float slope, float & s) {
    if constexpr (OP == kSwiglu) {
        return silu(a) * b;
    } else if constexpr (OP == kSilu) {
        return silu(a);
    } else if constexpr (OP == kAdd) {
        return a + b;
    } else if constexpr (OP == kAddLeaky) {
        s = a + b;
        return leaky(s, slope);
    } else if constexpr (OP == kLeaky) {
        return leaky(a, slope);
    } else {
        // Snake, kokoro/operations.cpp:143-146: mul, sin, mul, div, add.
        const float t  = a * al;
        const float sn = sinf(t);
        const float q  = sn * sn;
        const float r  = q / al;
        return a + r;
    }
}

template <int OP> __device__ __forceinline__ f32x4 ew4(f32x4 a, f32x4 b, f32x4 al, float slope, f32x4 & s) {
    float       s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    const f32x4 o{ ew<OP>(a.x, b.x, al.x, slope, s0), ew<OP>(a.y, b.y, al.y, slope, s1),
                   ew<OP>(a.z, b.z, al.z, slope, s2), ew<OP>(a.w, b.w, al.w, slope, s3) };
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

template <int OP, bool HAS_B, bool BCAST, bool HAS_S>
__global__ __launch_bounds__(256) void k_ew_flat(const EwArgs a) {
    const f32x4 * A    = reinterpret_cast<const f32x4 *>(a.a);
    const f32x4 * B    = reinterpret_cast<const f32x4 *>(a.b);
    const f32x4 * AL   = reinterpret_cast<const f32x4 *>(a.alpha);
    f32x4 *       Y    = reinterpret_cast<f32x4 *>(a.y);
    f32x4 *       S    = reinterpret_cast<f32x4 *>(a.s);
    const int64_t step = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < a.n4; i += step) {
        const f32x4 av  = ld_stream(A + i);
        f32x4       bv  = splat4(0.0f);
        f32x4       alv = splat4(1.0f);
        if constexpr (HAS_B) {
            if constexpr (BCAST) {
                bv = B[fastmod(static_cast<uint32_t>(i * 4), a.period) / 4];
            } else {
                bv = ld_stream(B + i);
            }
        }
        if constexpr (OP == kSnake) {
            alv = AL[fastmod(static_cast<uint32_t>(i * 4), a.period) / 4];
        }
        f32x4 sv = splat4(0.0f);
        st_stream(Y + i, ew4<OP>(av, bv, alv, a.slope, sv));
        if constexpr (HAS_S) {
            st_stream(S + i, sv);
        }
    }
}

// Snake, flat path. The five-node formula is ALU-heavy for a streaming op
// (a sine and a division per element), so two of its costs are cut without
// changing its result:
//   - the division by alpha: a lane owns one quad of channels (4 consecutive
//     alphas) in kSnakeRows consecutive rows, forms the 4 double reciprocals
//     once, and q / alpha becomes (float)((double)q * rcp), which is the IEEE
//     quotient (shp_div.hpp). Lanes whose alphas include 0, inf or NaN take
//     the f32 division.
//   - sinf: shp::sin_f32_fast, branch-free and within 1 ulp of the correctly
//     rounded sine for |t| < 2^15 (shp_sinf.hpp); OCML's sinf beyond that.
// Each of the wave's loads and stores is still one contiguous 1 KB run (64
// lanes, consecutive quads of one row). Measured on MI355X at [128,131072]:
// ~6% faster than one float4 per lane with OCML's sinf and the f32 division.
constexpr int kSnakeRows = 4;

// kokoro/operations.cpp:143-146: mul, sin, mul, div, add, each rounded in f32.
template <bool RCP> __device__ __forceinline__ float snake1(float x, float al, double rcp) {
    const float t  = x * al;
    const float sn = sin_fast_ok(t) ? sin_f32_fast(t) : sinf(t);
    const float q  = sn * sn;
    const float r  = RCP ? div_by_rcp(q, rcp) : q / al;
    return x + r;
}

template <bool RCP>
__device__ __forceinline__ void snake_rows(const f32x4 (&xv)[kSnakeRows], f32x4 al, const double (&rc)[4], int64_t i0,
                                           int64_t c4, int64_t n4, f32x4 * Y) {
#pragma unroll
    for (int r = 0; r < kSnakeRows; ++r) {
        const int64_t i = i0 + r * c4;
        if (i < n4) {
            const f32x4 v = xv[r];
            st_stream(Y + i, f32x4{ snake1<RCP>(v.x, al.x, rc[0]), snake1<RCP>(v.y, al.y, rc[1]),
                                    snake1<RCP>(v.z, al.z, rc[2]), snake1<RCP>(v.w, al.w, rc[3]) });
        }
    }
}

__global__ __launch_bounds__(256) void k_snake_flat(const EwArgs a) {
    const f32x4 * X    = reinterpret_cast<const f32x4 *>(a.a);
    const f32x4 * AL   = reinterpret_cast<const f32x4 *>(a.alpha);
    f32x4 *       Y    = reinterpret_cast<f32x4 *>(a.y);
    const int64_t c4   = a.quads.d;
    const int64_t step = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; t < a.ntask; t += step) {
        const uint32_t rb = fastdiv(static_cast<uint32_t>(t), a.quads);  // row block
        const uint32_t q  = static_cast<uint32_t>(t) - rb * a.quads.d;  // channel quad
        const int64_t  i0 = static_cast<int64_t>(rb) * kSnakeRows * c4 + q;
        f32x4          xv[kSnakeRows];
#pragma unroll
        for (int r = 0; r < kSnakeRows; ++r) {
            const int64_t i = i0 + r * c4;
            xv[r]           = i < a.n4 ? ld_stream(X + i) : splat4(0.0f);
        }
        const f32x4 al = AL[q];
        if (rcp_route_ok(al.x) && rcp_route_ok(al.y) && rcp_route_ok(al.z) && rcp_route_ok(al.w)) {
            const double rc[4] = { rcp_d(static_cast<double>(al.x)), rcp_d(static_cast<double>(al.y)),
                                   rcp_d(static_cast<double>(al.z)), rcp_d(static_cast<double>(al.w)) };
            snake_rows<true>(xv, al, rc, i0, c4, a.n4, Y);
        } else {
            const double rc[4] = { 0.0, 0.0, 0.0, 0.0 };
            snake_rows<false>(xv, al, rc, i0, c4, a.n4, Y);
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
                const f32x4 av  = ld_stream(reinterpret_cast<const f32x4 *>(ar) + c);
                f32x4       bv  = splat4(0.0f);
                f32x4       alv = splat4(1.0f);
                if constexpr (HAS_B) {
                    bv = BCAST ? reinterpret_cast<const f32x4 *>(br)[c] : ld_stream(reinterpret_cast<const f32x4 *>(br) + c);
                }
                if constexpr (OP == kSnake) {
                    alv = reinterpret_cast<const f32x4 *>(a.alpha)[c];
                }
                f32x4 sv = splat4(0.0f);
                st_stream(reinterpret_cast<f32x4 *>(yr) + c, ew4<OP>(av, bv, alv, a.slope, sv));
                if constexpr (HAS_S) {
                    st_stream(reinterpret_cast<f32x4 *>(sr) + c, sv);
                }
            }
        } else {
            for (int c = threadIdx.x; c < a.ne0; c += blockDim.x) {
                const float av  = reinterpret_cast<const float *>(ar)[c];
                float       bv  = 0.0f;
                float       alv = 1.0f;
                if constexpr (HAS_B) {
                    bv = reinterpret_cast<const float *>(br)[c];
                }
                if constexpr (OP == kSnake) {
                    alv = a.alpha[c];
                }
                float sv                            = 0.0f;
                reinterpret_cast<float *>(yr)[c]    = ew<OP>(av, bv, alv, a.slope, sv);
                if constexpr (HAS_S) {
                    reinterpret_cast<float *>(sr)[c] = sv;
                }
            }
        }
    }
}

template <int OP, bool HAS_B, bool BCAST, bool HAS_S>
shp_status_t launch_ew(const EwArgs & a, bool flat, bool vec, hipStream_t stream) {
    if (flat) {
        int64_t blocks = (a.n4 + 255) / 256;
        blocks         = blocks < kMaxFlatBlocks ? blocks : kMaxFlatBlocks;
        hipLaunchKernelGGL((k_ew_flat<OP, HAS_B, BCAST, HAS_S>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                           stream, a);
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
// allow_bcast) be a single contiguous row of ne0 elements.
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
        if (!allow_bcast || nelements(*b) != a->ne[0] || !contiguous(*b)) {
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

extern "C" shp_status_t shp_snake(const shp_tensor * x, const shp_tensor * alpha, shp_tensor * y, shp_stream_t stream) {
    if (!well_formed(alpha) || !well_formed(x)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (alpha->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    // One coefficient per channel; channels are ne[0] (kokoro_decoder_test.cpp:46-49).
    if (nelements(*alpha) != x->ne[0] || !contiguous(*alpha)) {
        return SHP_ERR_INVALID_ARG;
    }
    EwPlan             plan;
    const shp_status_t st = plan_ew(x, nullptr, false, y, nullptr, plan);
    if (st != SHP_OK) {
        return st;
    }
    plan.args.alpha = static_cast<const float *>(alpha->data);
    const bool al16 = reinterpret_cast<uintptr_t>(alpha->data) % 16 == 0;
    if (plan.flat && al16) {
        EwArgs &      g      = plan.args;
        const int64_t quads  = x->ne[0] / 4;
        const int64_t rows   = g.n4 / quads;
        g.quads              = make_fastdiv(static_cast<uint32_t>(quads));
        g.ntask              = (rows + kSnakeRows - 1) / kSnakeRows * quads;
        int64_t       blocks = (g.ntask + 255) / 256;
        blocks               = blocks < kMaxFlatBlocks ? blocks : kMaxFlatBlocks;
        hipLaunchKernelGGL(k_snake_flat, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream), g);
        return launch_status();
    }
    return launch_ew<kSnake, false, false, false>(plan.args, false, plan.vec && al16, as_stream(stream));
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

extern "C" shp_status_t shp_add(const shp_tensor * a, const shp_tensor * b, shp_tensor * y, shp_stream_t stream) {
    if (b == nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    EwPlan             plan;
    const shp_status_t st = plan_ew(a, b, true, y, nullptr, plan);
    if (st != SHP_OK) {
        return st;
    }
    const hipStream_t ss = as_stream(stream);
    if (plan.bcast) {
        const bool b16 = reinterpret_cast<uintptr_t>(b->data) % 16 == 0;
        return launch_ew<kAdd, true, true, false>(plan.args, plan.flat && b16, plan.vec && b16, ss);
    }
    return launch_ew<kAdd, true, false, false>(plan.args, plan.flat, plan.vec, ss);
}

// The padding and tiling copies of the vocoders, codecs and encoders, for
// gfx950: every destination element is one source element or zero.
//   ggml_pad / ggml_pad_ext: zeros before and after each dimension
//     (kokoro/operations.cpp:192,196,255,260 -- the transposed convolution's
//     zero-stuffed "spread" and its edge widening --, vits/text-encoder.cpp:36,50,
//     omnivoice/reference-encoder.cpp:482, qwen3-tts/codec-encoder.cpp:351)
//   ggml_pad_reflect_1d: reflection about the row's edge samples
//     (qwen3-tts/speaker-encoder.cpp:164)
//   ggml_repeat / ggml_repeat_4d: the source tiled over a larger shape
//     (kokoro/operations.cpp:23,118 -- the frame doubling of
//     upsample_nearest_2x --, qwen3-tts/speaker-encoder.cpp:356-357,
//     codec-encoder.cpp:183,188)
// One lane per four consecutive destination values of a row, one 16-byte
// nontemporal store: from the row's start when the destination's rows are
// 16-byte aligned, else from its first 16-byte boundary, with the few values
// before it stored one by one (four values per lane at the row's own start
// made every store instruction a 16-byte-strided scatter: 15 % of HBM peak for
// a row padded by 3 + 4). The four source values come in one 16-byte load
// where they are contiguous and aligned. A destination row the padding puts outside the source is stored as
// zeros without loads.

#include "shp_internal.hpp"

namespace shp {
namespace {

enum PadMode { kPadZero = 0, kPadReflect = 1, kPadRepeat = 2 };

struct PadArgs {
    const char * x;
    char *       y;
    int64_t      xnb[4];
    int64_t      ynb[4];
    int64_t      xne[4];
    int64_t      off[4];   // left pads (zero pad), {p0} (reflect)
    int64_t      yne0;
    FastDiv      quads;    // units (V values) per destination row
    FastDiv      yne1;
    FastDiv      yne2;
    FastDiv      xne0;     // repeat: source extents
    FastDiv      xne1;
    FastDiv      xne2;
    FastDiv      xne3;
    int64_t      total;    // units in all
};

template <int MODE> __device__ __forceinline__ int64_t src_index0(const PadArgs & a, int64_t i0, bool & in) {
    if constexpr (MODE == kPadZero) {
        const int64_t j = i0 - a.off[0];
        in              = j >= 0 && j < a.xne[0];
        return j;
    } else if constexpr (MODE == kPadReflect) {
        in = true;
        const int64_t p0 = a.off[0];
        return i0 < p0 ? p0 - i0 : (i0 < p0 + a.xne[0] ? i0 - p0 : 2 * (a.xne[0] - 1) + p0 - i0);
    } else {
        in = true;
        return fastmod(static_cast<uint32_t>(i0), a.xne0);
    }
}

// V values per lane: 4 (consecutive, one 16-byte store: the destination's rows
// are 16-byte aligned) or 1 (consecutive lanes on consecutive values, so each
// store instruction is one contiguous run). V4LOAD: the four source values are
// contiguous and 16-byte aligned whenever they are all inside the source (zero
// pad with lp0 and x's rows multiples of 4 values; repeat with x's rows so).
// SHIFT (V = 4, rows not 16-byte aligned): unit 0 of a row is its first h
// values, up to the first 16-byte boundary (scalar stores), unit u >= 1 the
// four from h + 4(u-1) (one 16-byte store when whole).
template <int MODE, int V, bool V4LOAD, bool SHIFT> __global__ __launch_bounds__(256) void k_pad(const PadArgs a) {
    const int64_t step = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; t < a.total; t += step) {
        const uint32_t r  = fastdiv(static_cast<uint32_t>(t), a.quads);  // destination row (quads: units per row)
        const int64_t  u  = t - static_cast<int64_t>(r) * a.quads.d;
        const uint32_t q1 = fastdiv(r, a.yne1);
        const uint32_t i1 = r - q1 * a.yne1.d;
        const uint32_t i3 = fastdiv(q1, a.yne2);
        const uint32_t i2 = q1 - i3 * a.yne2.d;
        // the source row, or none (a padded row)
        int64_t s1, s2, s3;
        bool    rin = true;
        if constexpr (MODE == kPadZero) {
            s1  = static_cast<int64_t>(i1) - a.off[1];
            s2  = static_cast<int64_t>(i2) - a.off[2];
            s3  = static_cast<int64_t>(i3) - a.off[3];
            rin = s1 >= 0 && s1 < a.xne[1] && s2 >= 0 && s2 < a.xne[2] && s3 >= 0 && s3 < a.xne[3];
        } else if constexpr (MODE == kPadReflect) {
            s1 = i1;
            s2 = i2;
            s3 = i3;
        } else {
            s1 = fastmod(i1, a.xne1);
            s2 = fastmod(i2, a.xne2);
            s3 = fastmod(i3, a.xne3);
        }
        const char * xr = a.x + s1 * a.xnb[1] + s2 * a.xnb[2] + s3 * a.xnb[3];
        char *       yr = a.y + static_cast<int64_t>(i1) * a.ynb[1] + static_cast<int64_t>(i2) * a.ynb[2] +
                    static_cast<int64_t>(i3) * a.ynb[3];
        int64_t i0;
        if constexpr (SHIFT) {
            const int h = static_cast<int>(((16 - reinterpret_cast<uintptr_t>(yr) % 16) % 16) / 4);
            if (u == 0) {  // the head: h values, scalar
                for (int e = 0; e < h && e < a.yne0; ++e) {
                    bool          in = false;
                    const int64_t j  = src_index0<MODE>(a, e, in);
                    __builtin_nontemporal_store((rin && in) ? reinterpret_cast<const float *>(xr)[j] : 0.0f,
                                                reinterpret_cast<float *>(yr) + e);
                }
                continue;
            }
            i0 = h + (u - 1) * 4;
            if (i0 >= a.yne0) {
                continue;
            }
        } else {
            i0 = u * V;
        }
        float        v[V];
        bool         done = false;
        if constexpr (V4LOAD && V == 4) {
            bool          in = false;
            const int64_t j  = src_index0<MODE>(a, i0, in);
            if (rin && in && j + 3 < a.xne[0] && i0 + 3 < a.yne0) {
                const f32x4 w = *reinterpret_cast<const f32x4 *>(xr + j * 4);
                v[0] = w.x;
                v[1] = w.y;
                v[2] = w.z;
                v[3] = w.w;
                done = true;
            }
        }
        if (!done) {
#pragma unroll
            for (int e = 0; e < V; ++e) {
                bool          in = false;
                const int64_t j  = src_index0<MODE>(a, i0 + e, in);
                v[e]             = (rin && in && i0 + e < a.yne0) ? reinterpret_cast<const float *>(xr)[j] : 0.0f;
            }
        }
        if constexpr (V == 4) {
            if (i0 + 3 < a.yne0) {
                __builtin_nontemporal_store(f32x4{ v[0], v[1], v[2], v[3] }, reinterpret_cast<f32x4 *>(yr + i0 * 4));
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (i0 + e < a.yne0) {
                        __builtin_nontemporal_store(v[e], reinterpret_cast<float *>(yr) + i0 + e);
                    }
                }
            }
        } else {
            __builtin_nontemporal_store(v[0], reinterpret_cast<float *>(yr) + i0);
        }
    }
}

// Checks common to the three ops, the argument block, and the launch.
template <int MODE>
shp_status_t pad_entry(const shp_tensor * x, const int64_t (&off)[4], shp_tensor * y, shp_stream_t stream) {
    if (!well_formed(x) || !well_formed(y)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (x->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (spans_overlap(*x, *y)) {
        return SHP_ERR_UNSUPPORTED;
    }
    const bool    v4    = rows_aligned(*y, 16);
    const bool    shift = !v4 && reinterpret_cast<uintptr_t>(y->data) % 4 == 0 && y->nb[1] % 4 == 0 &&
                       y->nb[2] % 4 == 0 && y->nb[3] % 4 == 0;
    const int64_t rows  = nrows(*y);
    const int64_t quads = v4 ? (y->ne[0] + 3) / 4 : (shift ? (y->ne[0] + 3) / 4 + 1 : y->ne[0]);
    if (quads > INT32_MAX || rows > INT32_MAX || y->ne[0] > INT32_MAX || x->ne[0] > INT32_MAX ||
        quads * rows > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (dry_run()) {
        return SHP_OK;
    }
    PadArgs a{};
    a.x = static_cast<const char *>(x->data);
    a.y = static_cast<char *>(y->data);
    for (int d = 0; d < 4; ++d) {
        a.xnb[d] = static_cast<int64_t>(x->nb[d]);
        a.ynb[d] = static_cast<int64_t>(y->nb[d]);
        a.xne[d] = x->ne[d];
        a.off[d] = off[d];
    }
    a.yne0  = y->ne[0];
    a.quads = make_fastdiv(static_cast<uint32_t>(quads));
    a.yne1  = make_fastdiv(static_cast<uint32_t>(y->ne[1]));
    a.yne2  = make_fastdiv(static_cast<uint32_t>(y->ne[2]));
    a.xne0  = make_fastdiv(static_cast<uint32_t>(x->ne[0]));
    a.xne1  = make_fastdiv(static_cast<uint32_t>(x->ne[1]));
    a.xne2  = make_fastdiv(static_cast<uint32_t>(x->ne[2]));
    a.xne3  = make_fastdiv(static_cast<uint32_t>(x->ne[3]));
    a.total = quads * rows;
    const bool v4load = MODE != kPadReflect && rows_aligned(*x, 16) && x->ne[0] % 4 == 0 && off[0] % 4 == 0;
    const int64_t  blocks = (a.total + 255) / 256;
    const unsigned grid   = static_cast<unsigned>(blocks < (1 << 20) ? blocks : (1 << 20));
    const dim3     g(grid), b(256);
    if (v4 && v4load) {
        hipLaunchKernelGGL((k_pad<MODE, 4, true, false>), g, b, 0, as_stream(stream), a);
    } else if (v4) {
        hipLaunchKernelGGL((k_pad<MODE, 4, false, false>), g, b, 0, as_stream(stream), a);
    } else if (shift) {
        hipLaunchKernelGGL((k_pad<MODE, 4, false, true>), g, b, 0, as_stream(stream), a);
    } else {
        hipLaunchKernelGGL((k_pad<MODE, 1, false, false>), g, b, 0, as_stream(stream), a);
    }
    return launch_status();
}

}  // namespace
}  // namespace shp

using namespace shp;

extern "C" shp_status_t shp_pad(const shp_tensor * x, const int32_t * lpad, shp_tensor * y, shp_stream_t stream) {
    if (x == nullptr || y == nullptr || lpad == nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    int64_t off[4];
    for (int d = 0; d < 4; ++d) {
        off[d] = lpad[d];
        if (lpad[d] < 0 || y->ne[d] < x->ne[d] + lpad[d]) {  // a negative right pad: y too small
            return SHP_ERR_INVALID_ARG;
        }
    }
    return pad_entry<kPadZero>(x, off, y, stream);
}

extern "C" shp_status_t shp_pad_reflect_1d(const shp_tensor * x, int32_t p0, int32_t p1, shp_tensor * y,
                                           shp_stream_t stream) {
    if (x == nullptr || y == nullptr || p0 < 0 || p1 < 0 || p0 >= x->ne[0] || p1 >= x->ne[0] ||
        y->ne[0] != x->ne[0] + p0 + p1 || y->ne[1] != x->ne[1] || y->ne[2] != x->ne[2] || y->ne[3] != x->ne[3]) {
        return SHP_ERR_INVALID_ARG;
    }
    const int64_t off[4] = { p0, 0, 0, 0 };
    return pad_entry<kPadReflect>(x, off, y, stream);
}

extern "C" shp_status_t shp_repeat(const shp_tensor * x, shp_tensor * y, shp_stream_t stream) {
    if (x == nullptr || y == nullptr || !can_repeat(*x, *y)) {
        return SHP_ERR_INVALID_ARG;
    }
    const int64_t off[4] = { 0, 0, 0, 0 };
    return pad_entry<kPadRepeat>(x, off, y, stream);
}

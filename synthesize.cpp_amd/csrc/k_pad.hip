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
// One lane per four consecutive destination values of a row: one 16-byte
// nontemporal store when the destination's rows allow; a destination row
// that the padding puts outside the source is stored as zeros without loads.
// Source loads are per value, coalesced across lanes (the ops are write-bound:
// the spread writes stride x its input, the repeat reads a small source many
// times from cache).

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
    FastDiv      quads;    // quads per destination row
    FastDiv      yne1;
    FastDiv      yne2;
    FastDiv      xne0;     // repeat: source extents
    FastDiv      xne1;
    FastDiv      xne2;
    FastDiv      xne3;
    int64_t      total;    // quads in all
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

template <int MODE, bool V4> __global__ __launch_bounds__(256) void k_pad(const PadArgs a) {
    const int64_t step = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; t < a.total; t += step) {
        const uint32_t r  = fastdiv(static_cast<uint32_t>(t), a.quads);  // destination row
        const int64_t  i0 = (t - static_cast<int64_t>(r) * a.quads.d) * 4;
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
        float        v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            bool          in = false;
            const int64_t j  = src_index0<MODE>(a, i0 + e, in);
            v[e]             = (rin && in && i0 + e < a.yne0) ? reinterpret_cast<const float *>(xr)[j] : 0.0f;
        }
        char * yr = a.y + static_cast<int64_t>(i1) * a.ynb[1] + static_cast<int64_t>(i2) * a.ynb[2] +
                    static_cast<int64_t>(i3) * a.ynb[3];
        if (V4 && i0 + 3 < a.yne0) {
            __builtin_nontemporal_store(f32x4{ v[0], v[1], v[2], v[3] }, reinterpret_cast<f32x4 *>(yr + i0 * 4));
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (i0 + e < a.yne0) {
                    __builtin_nontemporal_store(v[e], reinterpret_cast<float *>(yr) + i0 + e);
                }
            }
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
    const int64_t rows = nrows(*y), quads = (y->ne[0] + 3) / 4;
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
    const bool     v4     = rows_aligned(*y, 16);
    const int64_t  blocks = (a.total + 255) / 256;
    const unsigned grid   = static_cast<unsigned>(blocks < (1 << 20) ? blocks : (1 << 20));
    if (v4) {
        hipLaunchKernelGGL((k_pad<MODE, true>), dim3(grid), dim3(256), 0, as_stream(stream), a);
    } else {
        hipLaunchKernelGGL((k_pad<MODE, false>), dim3(grid), dim3(256), 0, as_stream(stream), a);
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

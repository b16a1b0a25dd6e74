// ggml_acc for gfx950: a copy of a with b added into a view of it, the
// talker's prefill input (qwen3-tts/talker.cpp:31,90,109,112,115: the codec
// stream, the x-vector's slot and the ICL acoustic block added into the text
// stream at a row offset).
//
// The view is ggml's: element (i0, i1, i2, i3) of b lands at byte offset +
// 4*i0 + i1*nb1 + i2*nb2 + i3*nb3 of the destination, and is added to a at
// the same byte. Its rows must not overlap (each extent times its stride at
// most the next stride, after dropping unit dimensions), so a destination
// element has at most one b element and its index follows from mixed-radix
// division by the strides.
//
//   out of place (y apart from a): one lane per four consecutive destination
//     values, a 16-byte load of a and a 16-byte store of y (nontemporal); the
//     four values' window position comes from three multiply-shift divisions
//     of the first, and when all four sit in one window row their b values
//     are one load (16 bytes when aligned), else each is located alone.
//   in place (y is a, ggml's inplace form): only the window is touched; one
//     lane per four consecutive values of a b row, read-add-write (16-byte
//     nontemporal accesses where the row allows).

#include "shp_internal.hpp"

namespace shp {
namespace {

struct AccArgs {
    const float * a;
    float *       y;
    const char *  b;
    int64_t       bnb[4];  // b's byte strides (bnb[0] = 4)
    int64_t       vs[4];   // the view's strides in elements (vs[0] = 1)
    int32_t       bne[4];
    FastDiv       s1;      // the view's strides with unit dimensions dropped
    FastDiv       s2;      // (a unit dimension takes the next one's stride),
    FastDiv       s3;      // in elements
    FastDiv       bq;      // quads per b row (in place)
    FastDiv       bne1;
    FastDiv       bne2;
    int64_t       off;     // the view's offset in elements
    int64_t       span;    // elements from off to one past the window's last
    int64_t       n;       // elements of a and y
    int64_t       total;   // units of the launch
};

// The window element at E = e - off (0 <= E < span), or false.
__device__ __forceinline__ bool locate(const AccArgs & a, uint32_t E, int64_t & boff, uint32_t & i0) {
    const uint32_t i3 = fastdiv(E, a.s3);
    uint32_t       r  = E - i3 * a.s3.d;
    const uint32_t i2 = fastdiv(r, a.s2);
    r -= i2 * a.s2.d;
    const uint32_t i1 = fastdiv(r, a.s1);
    i0                = r - i1 * a.s1.d;
    boff              = i1 * a.bnb[1] + i2 * a.bnb[2] + i3 * a.bnb[3] + static_cast<int64_t>(i0) * 4;
    return i0 < static_cast<uint32_t>(a.bne[0]) && i1 < static_cast<uint32_t>(a.bne[1]) &&
           i2 < static_cast<uint32_t>(a.bne[2]) && i3 < static_cast<uint32_t>(a.bne[3]);
}

// V = 4: a and y 16-byte aligned; V = 1 otherwise. An element outside the
// window adds nothing: a + 0.0f would turn -0.0 into +0.0, so it is copied.
template <int V> __global__ __launch_bounds__(256) void k_acc_copy(const AccArgs a) {
    const int64_t step = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; t < a.total; t += step) {
        const int64_t e0 = t * V;
        if constexpr (V == 4) {
            const bool whole = e0 + 3 < a.n;
            f32x4      v;
            if (whole) {
                v = ld_stream(reinterpret_cast<const f32x4 *>(a.a) + t);
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    v[k] = e0 + k < a.n ? a.a[e0 + k] : 0.0f;
                }
            }
            const int64_t E = e0 - a.off;
            if (E + 3 >= 0 && E < a.span) {  // the quad meets the window's range
                int64_t  boff = 0;
                uint32_t i0   = 0;
                if (E >= 0 && locate(a, static_cast<uint32_t>(E), boff, i0) && i0 + 3 < static_cast<uint32_t>(a.bne[0])) {
                    const char * p = a.b + boff;
                    f32x4        w;
                    if (reinterpret_cast<uintptr_t>(p) % 16 == 0) {
                        w = *reinterpret_cast<const f32x4 *>(p);
                    } else {
                        const float * q = reinterpret_cast<const float *>(p);
                        w               = f32x4{ q[0], q[1], q[2], q[3] };
                    }
                    v = f32x4{ v.x + w.x, v.y + w.y, v.z + w.z, v.w + w.w };
                } else {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int64_t Ek = E + k;
                        if (Ek >= 0 && Ek < a.span && e0 + k < a.n) {
                            int64_t  bo;
                            uint32_t j0;
                            if (locate(a, static_cast<uint32_t>(Ek), bo, j0)) {
                                v[k] = v[k] + *reinterpret_cast<const float *>(a.b + bo);
                            }
                        }
                    }
                }
            }
            if (whole) {
                st_stream(reinterpret_cast<f32x4 *>(a.y) + t, v);
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (e0 + k < a.n) {
                        a.y[e0 + k] = v[k];
                    }
                }
            }
        } else {
            const int64_t E = e0 - a.off;
            float         v = a.a[e0];
            if (E >= 0 && E < a.span) {
                int64_t  bo;
                uint32_t j0;
                if (locate(a, static_cast<uint32_t>(E), bo, j0)) {
                    v = v + *reinterpret_cast<const float *>(a.b + bo);
                }
            }
            a.y[e0] = v;
        }
    }
}

// In place: unit t is quad q of b row r (r = i1 + bne1*(i2 + bne2*i3)).
__global__ __launch_bounds__(256) void k_acc_inplace(const AccArgs a) {
    const int64_t step = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; t < a.total; t += step) {
        const uint32_t r  = fastdiv(static_cast<uint32_t>(t), a.bq);
        const uint32_t i0 = (static_cast<uint32_t>(t) - r * a.bq.d) * 4;
        const uint32_t q1 = fastdiv(r, a.bne1);
        const uint32_t i1 = r - q1 * a.bne1.d;
        const uint32_t i3 = fastdiv(q1, a.bne2);
        const uint32_t i2 = q1 - i3 * a.bne2.d;
        const float *  br = reinterpret_cast<const float *>(a.b + i1 * a.bnb[1] + i2 * a.bnb[2] + i3 * a.bnb[3]);
        float *        yr = a.y + a.off + i1 * a.vs[1] + i2 * a.vs[2] + i3 * a.vs[3];
        const int      m  = a.bne[0] - static_cast<int>(i0) < 4 ? a.bne[0] - static_cast<int>(i0) : 4;
        if (m == 4 && reinterpret_cast<uintptr_t>(yr + i0) % 16 == 0 && reinterpret_cast<uintptr_t>(br + i0) % 16 == 0) {
            const f32x4 w = ld_stream(reinterpret_cast<const f32x4 *>(br + i0));
            f32x4 *     p = reinterpret_cast<f32x4 *>(yr + i0);
            const f32x4 v = ld_stream(p);
            st_stream(p, f32x4{ v.x + w.x, v.y + w.y, v.z + w.z, v.w + w.w });
        } else {
            for (int k = 0; k < m; ++k) {
                yr[i0 + k] = yr[i0 + k] + br[i0 + k];
            }
        }
    }
}

}  // namespace
}  // namespace shp

using namespace shp;

extern "C" shp_status_t shp_acc(const shp_tensor * a, const shp_tensor * b, int64_t nb1, int64_t nb2, int64_t nb3,
                                int64_t offset, shp_tensor * y, shp_stream_t stream) {
    if (!well_formed(a) || !well_formed(b) || !well_formed(y)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (a->type != SHP_TYPE_F32 || b->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32 || !contiguous(*a) ||
        !contiguous(*y) || !same_shape(*a, *y)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (nb1 < 0 || nb2 < 0 || nb3 < 0 || offset < 0 || nb1 % 4 != 0 || nb2 % 4 != 0 || nb3 % 4 != 0 ||
        offset % 4 != 0 || reinterpret_cast<uintptr_t>(a->data) % 4 != 0 || reinterpret_cast<uintptr_t>(y->data) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(b->data) % 4 != 0 || b->nb[1] % 4 != 0 || b->nb[2] % 4 != 0 || b->nb[3] % 4 != 0) {
        return SHP_ERR_UNSUPPORTED;
    }
    const int64_t n = nelements(*a);
    if (n >= (int64_t{ 1 } << 31) || nelements(*b) >= (int64_t{ 1 } << 31)) {
        return SHP_ERR_UNSUPPORTED;
    }
    const int64_t vs[4]  = { 1, nb1 / 4, nb2 / 4, nb3 / 4 };
    const int64_t off    = offset / 4;
    int64_t       last   = off + (b->ne[0] - 1);
    for (int d = 1; d < 4; ++d) {
        last += (b->ne[d] - 1) * vs[d];
    }
    if (last >= n) {  // the view runs past a's end (ggml asserts)
        return SHP_ERR_INVALID_ARG;
    }
    // strides with unit dimensions dropped; rows that do not overlap
    int64_t s[5];
    s[4] = int64_t{ 1 } << 31;
    for (int d = 3; d >= 1; --d) {
        s[d] = b->ne[d] > 1 ? vs[d] : s[d + 1];
    }
    s[0] = 1;
    if (b->ne[0] > s[1] || b->ne[1] * s[1] > s[2] || b->ne[2] * s[2] > s[3]) {
        return SHP_ERR_UNSUPPORTED;
    }
    const bool inplace = a->data == y->data;
    if ((!inplace && spans_overlap(*a, *y)) || spans_overlap(*b, *y)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (dry_run()) {
        return SHP_OK;
    }
    AccArgs g{};
    g.a    = static_cast<const float *>(a->data);
    g.y    = static_cast<float *>(y->data);
    g.b    = static_cast<const char *>(b->data);
    for (int d = 0; d < 4; ++d) {
        g.bnb[d] = static_cast<int64_t>(b->nb[d]);
        g.vs[d]  = vs[d];
        g.bne[d] = static_cast<int32_t>(b->ne[d]);
    }
    g.s1   = make_fastdiv(static_cast<uint32_t>(s[1]));
    g.s2   = make_fastdiv(static_cast<uint32_t>(s[2]));
    g.s3   = make_fastdiv(static_cast<uint32_t>(s[3]));
    g.off  = off;
    g.span = last - off + 1;
    g.n    = n;
    const hipStream_t st = as_stream(stream);
    if (inplace) {
        const int64_t quads = (b->ne[0] + 3) / 4;
        const int64_t rows  = b->ne[1] * b->ne[2] * b->ne[3];
        g.bq                = make_fastdiv(static_cast<uint32_t>(quads));
        g.bne1              = make_fastdiv(static_cast<uint32_t>(b->ne[1]));
        g.bne2              = make_fastdiv(static_cast<uint32_t>(b->ne[2]));
        g.total             = quads * rows;
        const int64_t blocks = (g.total + 255) / 256;
        hipLaunchKernelGGL(k_acc_inplace, dim3(static_cast<unsigned>(blocks < (1 << 20) ? blocks : (1 << 20))), dim3(256),
                           0, st, g);
        return launch_status();
    }
    const bool v4 = reinterpret_cast<uintptr_t>(a->data) % 16 == 0 && reinterpret_cast<uintptr_t>(y->data) % 16 == 0;
    g.total       = v4 ? (n + 3) / 4 : n;
    const int64_t blocks = (g.total + 255) / 256;
    const dim3    grid(static_cast<unsigned>(blocks < (1 << 20) ? blocks : (1 << 20)));
    if (v4) {
        hipLaunchKernelGGL(k_acc_copy<4>, grid, dim3(256), 0, st, g);
    } else {
        hipLaunchKernelGGL(k_acc_copy<1>, grid, dim3(256), 0, st, g);
    }
    return launch_status();
}

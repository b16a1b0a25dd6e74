// ggml_im2col, 1-D (is_2D = false), for gfx950: the column matrix every
// convolution of the vocoders, codecs and speech encoders feeds its GEMM
// (vits/waveform-decoder.cpp:104, vits/operations.cpp:40,103,
// kokoro/operations.cpp:76, omnivoice/codec.cpp:114,
// omnivoice/reference-encoder.cpp:190, qwen3-tts/codec.cpp:96,129,
// qwen3-tts/speaker-encoder.cpp:174, qwen3-tts/codec-encoder.cpp:359).
//
//   x [IW, IC, N] (F32)  ->  y [IC*K, OW, N] (F32 or F16)
//   y[n][ow][ic*K + k] = x[n][ic][ow*s0 + k*d0 - p0], 0 outside [0, IW)
//
// A pure gather: every output is one input element (or 0), rounded to nearest
// even for an F16 y, so the result is bit-exact. The write of K copies of the
// input is the traffic (HBM-bound, no arithmetic to hide).
//
// One block per tile of OWT output positions x ICT channels of one batch
// entry:
//   1. the tile's input window (ICT channel rows of (OWT-1)*s0 + (K-1)*d0 + 1
//      samples, zeros where the window passes the input's ends) is loaded into
//      LDS, consecutive lanes on consecutive addresses: along time for a
//      time-contiguous x, along channels for a channel-contiguous x (the
//      transposed view of a channel-major activation, so the ggml_cont that
//      the reference puts in front of im2col is not needed);
//   2. the tile's outputs are written in y's order (for each position, ICT*K
//      consecutive values), each lane four values per store, from LDS.
// ICT = 32 channels makes a position's run 128*K bytes of F32: whole,
// aligned cache lines whenever IC is a multiple of 32. Tiles with every
// channel (IC <= 32) cover one contiguous range of y, written in 4-value
// stores whatever its alignment (scalar stores at its two ends).

#include "shp_internal.hpp"

namespace shp {
namespace {

constexpr int kIm2colBlock = 256;
constexpr int kIm2colLds   = 8192;   // floats of LDS window per block (32 KB)
constexpr int kIm2colIct   = 32;     // channels per tile
constexpr int kIm2colElems = 16384;  // target outputs per tile

// Write forms: SEG1 = per-position runs, one value per store; SEG4 = the same,
// four per store (IC*K a multiple of 4 and y aligned to four values); FLAT4 =
// the tile's one contiguous range (ICT == IC), four per store between scalar
// ends.
enum Im2colForm { kSeg1 = 0, kSeg4 = 1, kFlat4 = 2 };

struct Im2colArgs {
    const char * x;
    char *       y;
    int64_t      xnb0;  // byte strides of x: time, channel, batch
    int64_t      xnb1;
    int64_t      xnb2;
    int64_t      iw;    // IW
    int64_t      ic;    // IC
    int64_t      ow;    // OW
    int64_t      row;   // IC*K: y values per (n, ow)
    int32_t      k;
    int32_t      s0;
    int32_t      p0;
    int32_t      d0;
    int32_t      ict;   // tile extents
    int32_t      owt;
    int32_t      wt;    // window samples of a full tile
    int32_t      wtp;   // LDS row stride (wt, odd)
    FastDiv      tic;   // channel tiles
    FastDiv      tow;   // position tiles
    FastDiv      kdiv;  // K
    FastDiv      wdiv;  // wt (time-contiguous loader)
    FastDiv      cdiv;  // ict (channel-contiguous loader)
    FastDiv      vfull; // SEG forms: stores per position run, full channel tile
    FastDiv      vlast; // ... the last channel tile
    FastDiv      rdiv;  // FLAT form: row
    uint32_t     ntiles;
    uint32_t     pad;
};

template <bool F16> __device__ __forceinline__ void put1(char * y, int64_t e, float v) {
    if constexpr (F16) {
        __builtin_nontemporal_store(static_cast<_Float16>(v), reinterpret_cast<_Float16 *>(y) + e);
    } else {
        __builtin_nontemporal_store(v, reinterpret_cast<float *>(y) + e);
    }
}

template <bool F16> __device__ __forceinline__ void put4(char * y, int64_t e, const float (&v)[4]) {
    if constexpr (F16) {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        const h4 h{ static_cast<_Float16>(v[0]), static_cast<_Float16>(v[1]), static_cast<_Float16>(v[2]),
                    static_cast<_Float16>(v[3]) };
        __builtin_nontemporal_store(h, reinterpret_cast<h4 *>(y) + e / 4);
    } else {
        __builtin_nontemporal_store(f32x4{ v[0], v[1], v[2], v[3] }, reinterpret_cast<f32x4 *>(y) + e / 4);
    }
}

// The value at (position owl, channel icl, tap k) of the tile, from LDS.
__device__ __forceinline__ float tap(const float * lds, const Im2colArgs & a, int owl, int icl, int k) {
    return lds[icl * a.wtp + owl * a.s0 + k * a.d0];
}

template <int FORM, bool F16, bool CHFAST> __global__ __launch_bounds__(kIm2colBlock) void k_im2col(const Im2colArgs a) {
    __shared__ float lds[kIm2colLds];
    const int        tid = static_cast<int>(threadIdx.x);
    for (uint32_t t = blockIdx.x; t < a.ntiles; t += gridDim.x) {
        const uint32_t q    = fastdiv(t, a.tic);
        const uint32_t n    = fastdiv(q, a.tow);
        const int64_t  ic0  = static_cast<int64_t>(t - q * a.tic.d) * a.ict;
        const int64_t  ow0  = static_cast<int64_t>(q - n * a.tow.d) * a.owt;
        const int      nic  = static_cast<int>(a.ic - ic0 < a.ict ? a.ic - ic0 : a.ict);
        const int      now  = static_cast<int>(a.ow - ow0 < a.owt ? a.ow - ow0 : a.owt);
        const int64_t  iw0  = ow0 * a.s0 - a.p0;
        const char *   xb   = a.x + static_cast<int64_t>(n) * a.xnb2 + ic0 * a.xnb1;
        // 1. the window, zero-filled past the input's ends (channels past IC
        //    are never read)
        const int      nwin = a.ict * a.wt;
        for (int idx = tid; idx < nwin; idx += kIm2colBlock) {
            int icl, w;
            if constexpr (CHFAST) {
                w   = static_cast<int>(fastdiv(static_cast<uint32_t>(idx), a.cdiv));
                icl = idx - w * a.ict;
            } else {
                icl = static_cast<int>(fastdiv(static_cast<uint32_t>(idx), a.wdiv));
                w   = idx - icl * a.wt;
            }
            const int64_t iw = iw0 + w;
            float         v  = 0.0f;
            if (icl < nic && iw >= 0 && iw < a.iw) {
                v = *reinterpret_cast<const float *>(xb + icl * a.xnb1 + iw * a.xnb0);
            }
            lds[icl * a.wtp + w] = v;
        }
        __syncthreads();
        // 2. the outputs, in y's order
        const int64_t ybase = (static_cast<int64_t>(n) * a.ow + ow0) * a.row + ic0 * a.k;  // first value's index
        if constexpr (FORM == kFlat4) {
            // ICT == IC: positions ow0 .. ow0+now-1 are one range of now*row values
            const int64_t len  = static_cast<int64_t>(now) * a.row;
            const int     head0 = static_cast<int>((4 - ybase % 4) % 4);
            const int     head = static_cast<int>(head0 < len ? head0 : len);
            const int64_t nvec = (len - head) / 4;
            const int64_t tail = head + nvec * 4;
            auto          one  = [&](int64_t f) {
                const uint32_t owl = fastdiv(static_cast<uint32_t>(f), a.rdiv);
                const uint32_t j   = static_cast<uint32_t>(f) - owl * a.rdiv.d;
                const uint32_t icl = fastdiv(j, a.kdiv);
                put1<F16>(a.y, ybase + f, tap(lds, a, static_cast<int>(owl), static_cast<int>(icl),
                                               static_cast<int>(j - icl * a.kdiv.d)));
            };
            if (tid < head) {
                one(tid);
            }
            for (int64_t v = tid; v < nvec; v += kIm2colBlock) {
                const int64_t f   = head + v * 4;
                uint32_t      owl = fastdiv(static_cast<uint32_t>(f), a.rdiv);
                const uint32_t j  = static_cast<uint32_t>(f) - owl * a.rdiv.d;
                uint32_t      icl = fastdiv(j, a.kdiv);
                int           k   = static_cast<int>(j - icl * a.kdiv.d);
                float         vals[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    vals[e] = tap(lds, a, static_cast<int>(owl), static_cast<int>(icl), k);
                    if (++k == a.k) {
                        k = 0;
                        if (++icl == static_cast<uint32_t>(nic)) {
                            icl = 0;
                            ++owl;
                        }
                    }
                }
                put4<F16>(a.y, ybase + f, vals);
            }
            if (tail + tid < len) {
                one(tail + tid);
            }
        } else {
            constexpr int V    = FORM == kSeg4 ? 4 : 1;
            const int     seg  = nic * a.k;  // values per position in this tile
            const FastDiv vd   = nic == a.ict ? a.vfull : a.vlast;
            const int     nv   = seg / V;
            const int     tot  = now * nv;
            for (int v = tid; v < tot; v += kIm2colBlock) {
                const uint32_t owl = fastdiv(static_cast<uint32_t>(v), vd);
                const int      j   = (v - static_cast<int>(owl * vd.d)) * V;
                int            icl = static_cast<int>(fastdiv(static_cast<uint32_t>(j), a.kdiv));
                int            k   = j - icl * a.k;
                const int64_t  e   = ybase + static_cast<int64_t>(owl) * a.row + j;
                if constexpr (V == 1) {
                    put1<F16>(a.y, e, tap(lds, a, static_cast<int>(owl), icl, k));
                } else {
                    float vals[4];
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) {
                        vals[q4] = tap(lds, a, static_cast<int>(owl), icl, k);
                        if (++k == a.k) {
                            k = 0;
                            ++icl;
                        }
                    }
                    put4<F16>(a.y, e, vals);
                }
            }
        }
        __syncthreads();
    }
}

template <int FORM, bool F16> void launch_form(const Im2colArgs & a, bool chfast, unsigned grid, hipStream_t s) {
    if (chfast) {
        hipLaunchKernelGGL((k_im2col<FORM, F16, true>), dim3(grid), dim3(kIm2colBlock), 0, s, a);
    } else {
        hipLaunchKernelGGL((k_im2col<FORM, F16, false>), dim3(grid), dim3(kIm2colBlock), 0, s, a);
    }
}

inline int64_t window(int64_t owt, int64_t s0, int64_t k, int64_t d0) {
    return (owt - 1) * s0 + (k - 1) * d0 + 1;
}

inline int64_t padded(int64_t w) {
    return w | 1;  // an odd row stride spreads a column of the window over the banks
}

}  // namespace

// ggml_calc_conv_output_size with C's truncating division; < 1: no output.
int64_t im2col_out_len(int64_t iw, int64_t k, int64_t s0, int64_t p0, int64_t d0) {
    return (iw + 2 * p0 - d0 * (k - 1) - 1) / s0 + 1;
}

// The launch plan. chfast: x's channel stride is 4 bytes and its time stride is
// not (the transposed view of a channel-major activation).
struct Im2colPlan {
    Im2colArgs args{};
    int        form   = kSeg1;
    bool       f16    = false;
    bool       chfast = false;
    unsigned   grid   = 0;
};

shp_status_t plan_im2col(const shp_tensor * kernel, const shp_tensor * x, int32_t s0, int32_t p0, int32_t d0,
                         const shp_tensor * y, Im2colPlan & pl) {
    if (kernel == nullptr || x == nullptr || y == nullptr || x->data == nullptr || x->reserved != 0 ||
        kernel->reserved != 0) {
        return SHP_ERR_INVALID_ARG;
    }
    for (int d = 0; d < 4; ++d) {
        if (kernel->ne[d] < 1 || x->ne[d] < 1) {
            return SHP_ERR_INVALID_ARG;
        }
    }
    if (s0 < 1 || d0 < 1 || p0 < 0) {
        return SHP_ERR_INVALID_ARG;
    }
    if (x->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    // ggml_im2col (1-D): the kernel's channel extent is x's; x has no 4th dim
    if (kernel->ne[1] != x->ne[1] || x->ne[3] != 1) {
        return SHP_ERR_INVALID_ARG;
    }
    if (reinterpret_cast<uintptr_t>(x->data) % 4 != 0 || x->nb[0] % 4 != 0 || x->nb[1] % 4 != 0 ||
        x->nb[2] % 4 != 0) {
        return SHP_ERR_UNSUPPORTED;
    }
    const int64_t K = kernel->ne[0], IW = x->ne[0], IC = x->ne[1], N = x->ne[2];
    if (K > INT32_MAX / 4 || static_cast<int64_t>(d0) * (K - 1) > INT32_MAX / 4) {
        return SHP_ERR_UNSUPPORTED;
    }
    const int64_t OW = im2col_out_len(IW, K, s0, p0, d0);
    if (OW < 1) {
        return SHP_ERR_INVALID_ARG;
    }
    if (!well_formed(y) || !contiguous(*y)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (y->type != SHP_TYPE_F32 && y->type != SHP_TYPE_F16) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (y->ne[0] != IC * K || y->ne[1] != OW || y->ne[2] != N || y->ne[3] != 1) {
        return SHP_ERR_INVALID_ARG;
    }
    if (spans_overlap(*x, *y)) {
        return SHP_ERR_UNSUPPORTED;
    }
    // tile: ICT channels, OWT positions, the window in LDS
    int64_t ict = IC < kIm2colIct ? IC : kIm2colIct;
    int64_t owt = kIm2colElems / (ict * K);
    owt         = owt < 1 ? 1 : (owt >= 16 ? owt / 16 * 16 : owt);
    owt         = owt < OW ? owt : OW;
    while (owt > 1 && ict * padded(window(owt, s0, K, d0)) > kIm2colLds) {
        owt = (owt + 1) / 2;
    }
    while (ict > 1 && ict * padded(window(owt, s0, K, d0)) > kIm2colLds) {
        ict = (ict + 1) / 2;
    }
    if (ict * padded(window(owt, s0, K, d0)) > kIm2colLds) {
        return SHP_ERR_UNSUPPORTED;  // one channel's receptive field alone passes the window
    }
    const int64_t tic = (IC + ict - 1) / ict, tow = (OW + owt - 1) / owt;
    if (IC * K > INT32_MAX || OW > INT32_MAX || N > INT32_MAX || tic * tow * N > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    Im2colArgs & a = pl.args;
    a.x            = static_cast<const char *>(x->data);
    a.y            = static_cast<char *>(y->data);
    a.xnb0         = static_cast<int64_t>(x->nb[0]);
    a.xnb1         = static_cast<int64_t>(x->nb[1]);
    a.xnb2         = static_cast<int64_t>(x->nb[2]);
    a.iw           = IW;
    a.ic           = IC;
    a.ow           = OW;
    a.row          = IC * K;
    a.k            = static_cast<int32_t>(K);
    a.s0           = s0;
    a.p0           = p0;
    a.d0           = d0;
    a.ict          = static_cast<int32_t>(ict);
    a.owt          = static_cast<int32_t>(owt);
    a.wt           = static_cast<int32_t>(window(owt, s0, K, d0));
    a.wtp          = static_cast<int32_t>(padded(a.wt));
    a.tic          = make_fastdiv(static_cast<uint32_t>(tic));
    a.tow          = make_fastdiv(static_cast<uint32_t>(tow));
    a.kdiv         = make_fastdiv(static_cast<uint32_t>(K));
    a.wdiv         = make_fastdiv(static_cast<uint32_t>(a.wt));
    a.cdiv         = make_fastdiv(static_cast<uint32_t>(ict));
    a.rdiv         = make_fastdiv(static_cast<uint32_t>(IC * K));
    a.ntiles       = static_cast<uint32_t>(tic * tow * N);
    pl.f16         = y->type == SHP_TYPE_F16;
    const size_t esz = pl.f16 ? 2 : 4;
    if (ict == IC) {
        pl.form = kFlat4;
    } else if ((IC * K) % 4 == 0 && (ict * K) % 4 == 0 && reinterpret_cast<uintptr_t>(y->data) % (4 * esz) == 0) {
        pl.form = kSeg4;
    } else {
        pl.form = kSeg1;
    }
    const int64_t vdiv = pl.form == kSeg4 ? 4 : 1;
    const int64_t last = IC - (tic - 1) * ict;
    a.vfull            = make_fastdiv(static_cast<uint32_t>(ict * K / vdiv));
    a.vlast            = make_fastdiv(static_cast<uint32_t>(last * K / vdiv));
    if (pl.form == kFlat4 && reinterpret_cast<uintptr_t>(y->data) % (4 * esz) != 0) {
        pl.form = kSeg1;  // FLAT4 finds its ends from value indices, which needs an aligned y
    }
    pl.chfast = x->nb[1] == 4 && x->nb[0] != 4 && IC > 1;
    pl.grid   = a.ntiles < (1u << 20) ? a.ntiles : (1u << 20);
    return SHP_OK;
}

shp_status_t launch_im2col(const Im2colPlan & pl, hipStream_t s) {
    const Im2colArgs & a = pl.args;
    switch (pl.form) {
        case kFlat4:
            pl.f16 ? launch_form<kFlat4, true>(a, pl.chfast, pl.grid, s) :
                     launch_form<kFlat4, false>(a, pl.chfast, pl.grid, s);
            break;
        case kSeg4:
            pl.f16 ? launch_form<kSeg4, true>(a, pl.chfast, pl.grid, s) :
                     launch_form<kSeg4, false>(a, pl.chfast, pl.grid, s);
            break;
        default:
            pl.f16 ? launch_form<kSeg1, true>(a, pl.chfast, pl.grid, s) :
                     launch_form<kSeg1, false>(a, pl.chfast, pl.grid, s);
            break;
    }
    return launch_status();
}

}  // namespace shp

using namespace shp;

extern "C" shp_status_t shp_im2col(const shp_tensor * kernel, const shp_tensor * x, int32_t s0, int32_t p0, int32_t d0,
                                   shp_tensor * y, shp_stream_t stream) {
    Im2colPlan         pl;
    const shp_status_t st = plan_im2col(kernel, x, s0, p0, d0, y, pl);
    if (st != SHP_OK || dry_run()) {
        return st;
    }
    return launch_im2col(pl, as_stream(stream));
}

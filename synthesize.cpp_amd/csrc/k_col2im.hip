// ggml_col2im_1d for gfx950: the scatter-back of a transposed convolution
// computed as a matrix product -- the upsampling layers of the vocoders and
// codecs (vits/operations.cpp:118-140, omnivoice/codec.cpp:150-159,
// qwen3-tts/codec.cpp:163-171).
//
//   columns [K*OC, L] (column l: the K*OC taps of input sample l, out-channel
//   major, tap minor)  ->  y [T, OC], T = (L-1)*stride + K - 2*padding
//   y[oc][t] = sum of columns[l][oc*K + k] over l*stride + k = t + padding
//
// Each output sums its terms in ascending l from +0.0f, the order of a
// zero-initialised scatter in column order (the op belongs to the reference's
// pinned ggml, absent here). With K <= 2*stride -- every upsampling layer of
// the vocoders and codecs -- an output has at most two terms, and a two-term
// f32 sum from +0 does not depend on the order.
//
// One 256-thread block per tile of OCT out-channels x TT output samples:
//   1. the column rows the tile needs (l from the tile's first to its last
//      contributing sample), OCT*K contiguous values each, go to LDS with
//      consecutive lanes on consecutive addresses (16-byte loads when
//      aligned);
//   2. each wave takes one channel of the tile at a time, each lane four
//      consecutive samples (a 16-byte store when y's rows allow), each value
//      its <= ceil(K/stride) terms from LDS.
// Reads are the columns once (plus the rows two neighbouring tiles share),
// writes the output once: HBM-bound.

#include "shp_internal.hpp"

namespace shp {
namespace {

constexpr int kC2iBlock = 256;
constexpr int kC2iLds   = 4608;  // floats of column rows per block at most (18 KB)
constexpr int kC2iTt    = 256;   // output samples per tile (64 lanes x 4)

struct Col2imArgs {
    const char * c;     // columns, rows of K*OC values
    char *       y;
    int64_t      cnb1;  // byte stride of a column row
    int64_t      ynb1;  // byte stride of an output row (one out-channel)
    int32_t      k;
    int32_t      oc;
    int32_t      l;     // L
    int32_t      t;     // T
    int32_t      s;     // stride
    int32_t      p;     // padding
    int32_t      oct;   // channels per tile
    int32_t      tt;    // samples per tile
    int32_t      nlmax; // column rows per tile at most
    int32_t      pad;
    FastDiv      sdiv;  // stride
    FastDiv      toc;   // channel tiles
    FastDiv      rdiv;  // OCT*K (the loader's row length)
};

template <bool V4LOAD, bool V4STORE> __global__ __launch_bounds__(kC2iBlock) void k_col2im_1d(const Col2imArgs a) {
    extern __shared__ float lds[];
    const int      tid = static_cast<int>(threadIdx.x);
    const uint32_t q   = fastdiv(blockIdx.x, a.toc);
    const int      oc0 = static_cast<int>(blockIdx.x - q * a.toc.d) * a.oct;
    const int      t0  = static_cast<int>(q) * a.tt;
    const int      noc = a.oc - oc0 < a.oct ? a.oc - oc0 : a.oct;
    const int      ntt = a.t - t0 < a.tt ? a.t - t0 : a.tt;
    // column rows [lb, le]: the first contributes to sample t0 (l*s + K-1 >=
    // t0 + p), the last to sample t0 + ntt - 1 (l*s <= t0 + ntt - 1 + p)
    const int u0 = t0 + a.p;
    const int lb = u0 >= a.k ? static_cast<int>(fastdiv(static_cast<uint32_t>(u0 - a.k), a.sdiv)) + 1 : 0;
    int       le = static_cast<int>(fastdiv(static_cast<uint32_t>(u0 + ntt - 1), a.sdiv));
    le           = le < a.l - 1 ? le : a.l - 1;
    const int rw = a.oct * a.k;  // LDS row length
    // 1. the rows
    const char * cb  = a.c + static_cast<int64_t>(oc0) * a.k * 4;
    const int    nrw = noc * a.k;  // values of a row this tile reads
    if (le >= lb) {
        const int nrows = le - lb + 1;
        if constexpr (V4LOAD) {
            const int q4  = nrw / 4;  // this tile's 16-byte pieces per row (nrw % 4 == 0)
            const int tot = nrows * static_cast<int>(a.rdiv.d);
            for (int i = tid; i < tot; i += kC2iBlock) {
                const int r = static_cast<int>(fastdiv(static_cast<uint32_t>(i), a.rdiv));  // rdiv: a full tile's pieces
                const int j = i - r * static_cast<int>(a.rdiv.d);
                if (j < q4) {
                    const f32x4 v = *reinterpret_cast<const f32x4 *>(cb + static_cast<int64_t>(lb + r) * a.cnb1 + j * 16);
                    *reinterpret_cast<f32x4 *>(lds + r * rw + j * 4) = v;
                }
            }
        } else {
            const int tot = nrows * rw;
            for (int i = tid; i < tot; i += kC2iBlock) {
                const int r = static_cast<int>(fastdiv(static_cast<uint32_t>(i), a.rdiv));  // rdiv: rw
                const int j = i - r * rw;
                if (j < nrw) {
                    lds[r * rw + j] = *reinterpret_cast<const float *>(cb + static_cast<int64_t>(lb + r) * a.cnb1 + j * 4);
                }
            }
        }
    }
    __syncthreads();
    // 2. the outputs: wave w, channels w, w+4, ...; lane: samples 4*lane..+3
    const int wave = tid / kWave, lane = tid % kWave;
    for (int ocl = wave; ocl < noc; ocl += kC2iBlock / kWave) {
        char * yrow = a.y + static_cast<int64_t>(oc0 + ocl) * a.ynb1;
        for (int tl = lane * 4; tl < ntt; tl += kWave * 4) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int u  = u0 + tl + e;  // t + p
                int       hi = static_cast<int>(fastdiv(static_cast<uint32_t>(u), a.sdiv));
                hi           = hi < a.l - 1 ? hi : a.l - 1;
                const int lo = u >= a.k ? static_cast<int>(fastdiv(static_cast<uint32_t>(u - a.k), a.sdiv)) + 1 : 0;
                float     acc = 0.0f;
                for (int l = lo; l <= hi; ++l) {
                    acc += lds[(l - lb) * rw + ocl * a.k + (u - l * a.s)];
                }
                v[e] = acc;
            }
            if (V4STORE && tl + 3 < ntt) {
                __builtin_nontemporal_store(f32x4{ v[0], v[1], v[2], v[3] },
                                            reinterpret_cast<f32x4 *>(yrow + static_cast<int64_t>(t0 + tl) * 4));
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (tl + e < ntt) {
                        __builtin_nontemporal_store(v[e], reinterpret_cast<float *>(yrow) + t0 + tl + e);
                    }
                }
            }
        }
    }
}

}  // namespace

struct Col2imPlan {
    Col2imArgs args{};
    bool       v4load  = false;
    bool       v4store = false;
    unsigned   grid    = 0;
    size_t     shmem   = 0;
};

shp_status_t plan_col2im_1d(const shp_tensor * cols, int32_t stride, int32_t oc, int32_t padding, const shp_tensor * y,
                            Col2imPlan & pl) {
    if (!well_formed(cols) || !well_formed(y) || stride < 1 || oc < 1 || padding < 0) {
        return SHP_ERR_INVALID_ARG;
    }
    if (cols->type != SHP_TYPE_F32 || y->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (cols->ne[0] % oc != 0 || cols->ne[2] != 1 || cols->ne[3] != 1) {
        return SHP_ERR_INVALID_ARG;
    }
    const int64_t K = cols->ne[0] / oc, L = cols->ne[1];
    const int64_t T = (L - 1) * stride + K - 2 * static_cast<int64_t>(padding);
    if (T < 1 || y->ne[0] != T || y->ne[1] != oc || y->ne[2] != 1 || y->ne[3] != 1) {
        return SHP_ERR_INVALID_ARG;
    }
    if (spans_overlap(*cols, *y)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (L > INT32_MAX / 2 || T > INT32_MAX / 2 || K > INT32_MAX / 2 || (L - 1) * stride + K > INT32_MAX / 2) {
        return SHP_ERR_UNSUPPORTED;
    }
    // tile: TT samples (fewer when one channel's rows pass the LDS), OCT channels
    int64_t tt = kC2iTt, nl = 0, oct = 0;
    for (;; tt /= 2) {
        nl  = (tt - 1 + K - 1) / stride + 2;  // column rows a tile can need
        oct = kC2iLds / (nl * K);
        if (oct >= 1 || tt <= 4) {
            break;
        }
    }
    if (oct < 1) {
        return SHP_ERR_UNSUPPORTED;  // K alone passes the LDS
    }
    oct = oct < oc ? oct : oc;
    oct = oct < 64 ? oct : 64;
    const int64_t toc = (oc + oct - 1) / oct, tts = (T + tt - 1) / tt;
    if (toc * tts > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    Col2imArgs & a = pl.args;
    a.c            = static_cast<const char *>(cols->data);
    a.y            = static_cast<char *>(y->data);
    a.cnb1         = static_cast<int64_t>(cols->nb[1]);
    a.ynb1         = static_cast<int64_t>(y->nb[1]);
    a.k            = static_cast<int32_t>(K);
    a.oc           = oc;
    a.l            = static_cast<int32_t>(L);
    a.t            = static_cast<int32_t>(T);
    a.s            = stride;
    a.p            = padding;
    a.oct          = static_cast<int32_t>(oct);
    a.tt           = static_cast<int32_t>(tt);
    a.nlmax        = static_cast<int32_t>(nl);
    a.sdiv         = make_fastdiv(static_cast<uint32_t>(stride));
    a.toc          = make_fastdiv(static_cast<uint32_t>(toc));
    // 16-byte loads: every tile's row piece starts and ends on 16 bytes
    pl.v4load = reinterpret_cast<uintptr_t>(cols->data) % 16 == 0 && (L == 1 || a.cnb1 % 16 == 0) &&
                (oct * K) % 4 == 0 && (oc * K) % 4 == 0;
    a.rdiv     = make_fastdiv(static_cast<uint32_t>(pl.v4load ? oct * K / 4 : oct * K));
    pl.v4store = reinterpret_cast<uintptr_t>(y->data) % 16 == 0 && (oc == 1 || a.ynb1 % 16 == 0);
    pl.grid    = static_cast<unsigned>(toc * tts);
    pl.shmem   = static_cast<size_t>(nl * oct * K) * sizeof(float);
    return SHP_OK;
}

shp_status_t launch_col2im_1d(const Col2imPlan & pl, hipStream_t s) {
    const dim3 g(pl.grid), b(kC2iBlock);
    if (pl.v4load && pl.v4store) {
        hipLaunchKernelGGL((k_col2im_1d<true, true>), g, b, pl.shmem, s, pl.args);
    } else if (pl.v4load) {
        hipLaunchKernelGGL((k_col2im_1d<true, false>), g, b, pl.shmem, s, pl.args);
    } else if (pl.v4store) {
        hipLaunchKernelGGL((k_col2im_1d<false, true>), g, b, pl.shmem, s, pl.args);
    } else {
        hipLaunchKernelGGL((k_col2im_1d<false, false>), g, b, pl.shmem, s, pl.args);
    }
    return launch_status();
}

}  // namespace shp

using namespace shp;

extern "C" shp_status_t shp_col2im_1d(const shp_tensor * cols, int32_t stride, int32_t out_channels, int32_t padding,
                                      shp_tensor * y, shp_stream_t stream) {
    Col2imPlan         pl;
    const shp_status_t st = plan_col2im_1d(cols, stride, out_channels, padding, y, pl);
    if (st != SHP_OK || dry_run()) {
        return st;
    }
    return launch_col2im_1d(pl, as_stream(stream));
}

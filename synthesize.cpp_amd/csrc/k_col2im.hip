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
// With K <= 4*stride each lane locates its four samples' terms once per tile
// (the offsets depend on the sample, not on the channel), so a channel costs
// its LDS reads, adds and one store: no division in the channel loop (per-value
// divisions held an earlier form to 35-49 % of HBM peak at the vocoder shapes).
// Reads are the columns once (plus the rows two neighbouring tiles share),
// writes the output once: HBM-bound.

#include "shp_internal.hpp"

namespace shp {
namespace {

constexpr int kC2iBlock = 256;
constexpr int kC2iLds   = 4608;  // floats of column rows per block at most (18 KB)
constexpr int kC2iTt    = 256;   // output samples per tile, a power of two from 16 to 1024
constexpr int kC2iBatch = 8;     // column-row loads a lane issues before its LDS writes

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
    int32_t      rwp;   // LDS row stride: OCT*K, odd (consecutive rows on different banks)
    FastDiv      sdiv;  // stride
    FastDiv      toc;   // channel tiles
    FastDiv      rdiv;  // OCT*K (the loader's row length)
};

// NT: the most terms an output can take (ceil(K / stride) <= 4); 0: any.
template <int NT, bool V4LOAD, bool V4STORE>
__global__ __launch_bounds__(kC2iBlock) void k_col2im_1d(const Col2imArgs a) {
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
    const int rw = a.rwp;  // LDS row stride: OCT*K rounded up to odd
    // 1. the rows, walked by running sums: lane tid starts at (tid / w, tid %
    //    w) of the nrows x w pieces and steps 256 pieces (w = a full tile's
    //    pieces per row; pieces past this tile's channels are skipped)
    {
        constexpr int VL  = V4LOAD ? 4 : 1;
        const int     w   = static_cast<int>(a.rdiv.d);
        const int     nrw = noc * a.k / VL;  // this tile's pieces per row
        int           r   = static_cast<int>(fastdiv(static_cast<uint32_t>(tid), a.rdiv));
        int           j   = tid - r * w;
        const int     dr = kC2iBlock / w, dj = kC2iBlock % w;
        const char *  cb = a.c + static_cast<int64_t>(oc0) * a.k * 4 + static_cast<int64_t>(lb) * a.cnb1;
        typedef float vl __attribute__((ext_vector_type(VL)));
        while (lb + r <= le) {
            // kC2iBatch loads in flight per lane, then their LDS writes (one
            // load, wait, write per step leaves each lane's loads serialised
            // behind HBM latency: 35-49 % of peak at the vocoder shapes)
            vl  v[kC2iBatch];
            int at[kC2iBatch];
#pragma unroll
            for (int b = 0; b < kC2iBatch; ++b) {
                const bool in = lb + r <= le && j < nrw;
                at[b]         = in ? r * rw + j * VL : -1;
                if (in) {
                    v[b] = *reinterpret_cast<const vl *>(cb + static_cast<int64_t>(r) * a.cnb1 + j * VL * 4);
                }
                r += dr;
                j += dj;
                if (j >= w) {
                    j -= w;
                    ++r;
                }
            }
#pragma unroll
            for (int b = 0; b < kC2iBatch; ++b) {
                if (at[b] >= 0) {
#pragma unroll
                    for (int i = 0; i < VL; ++i) {  // the odd row stride leaves rows unaligned
                        lds[at[b] + i] = v[b][i];
                    }
                }
            }
        }
    }
    __syncthreads();
    // 2. the outputs: the tile's tt/4 quads of four samples x its channels,
    //    256 at a time; with tt/4 dividing 256 a thread keeps one quad (its
    //    terms' offsets are found once) and steps channels by 256 / (tt/4)
    const int nq = a.tt / 4;
    for (int tl = (tid % nq) * 4; tl < ntt; tl += kC2iBlock * 4) {
        // each value's terms (ascending column order), channel offset aside
        int      off[4][NT > 0 ? NT : 1];
        uint32_t ok = 0;  // bit e*4 + j: term j of value e exists
        if constexpr (NT > 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int u  = u0 + tl + e;
                const int qh = static_cast<int>(fastdiv(static_cast<uint32_t>(u), a.sdiv));  // the latest column
                const int r  = u - qh * a.s;
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    const int  l  = qh - (NT - 1 - j);  // ascending
                    const int  k  = r + (NT - 1 - j) * a.s;
                    const bool in = tl + e < ntt && k < a.k && l >= 0 && l <= a.l - 1;
                    off[e][j]     = in ? (l - lb) * rw + k : 0;  // a term that does not exist reads slot 0, unused
                    ok |= static_cast<uint32_t>(in) << (e * 4 + j);
                }
            }
        }
        for (int ocl = tid / nq; ocl < noc; ocl += kC2iBlock / nq) {
            char *    yrow = a.y + static_cast<int64_t>(oc0 + ocl) * a.ynb1;
            const int cko  = ocl * a.k;
            float     v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float acc = 0.0f;
                if constexpr (NT > 0) {
#pragma unroll
                    for (int j = 0; j < NT; ++j) {
                        const float x = lds[cko + off[e][j]];
                        acc           = (ok >> (e * 4 + j)) & 1u ? acc + x : acc;
                    }
                } else {
                    const int u  = u0 + tl + e;
                    int       hi = static_cast<int>(fastdiv(static_cast<uint32_t>(u), a.sdiv));
                    hi           = hi < a.l - 1 ? hi : a.l - 1;
                    const int lo = u >= a.k ? static_cast<int>(fastdiv(static_cast<uint32_t>(u - a.k), a.sdiv)) + 1 : 0;
                    for (int l = lo; l <= hi && tl + e < ntt; ++l) {
                        acc += lds[(l - lb) * rw + cko + (u - l * a.s)];
                    }
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

// The persistent, double-buffered form (16-byte column loads: a tile's row
// pieces are at most kC2iLds/4 = 1152, so each lane's share, five at most,
// fits one batch of registers): a block walks tiles blockIdx.x, +gridDim.x,
// ...; the next tile's loads are issued before the current tile's outputs
// are written from the other LDS buffer, so the two overlap within a block;
// one barrier per tile.
constexpr int kC2iPersist = 1024;  // blocks: four per CU at 2 x 18 KB of LDS

struct C2iTile {
    int oc0, t0, noc, ntt, u0, lb, le;
};

__device__ __forceinline__ C2iTile c2i_tile(const Col2imArgs & a, uint32_t tile) {
    C2iTile       g;
    const uint32_t q = fastdiv(tile, a.toc);
    g.oc0            = static_cast<int>(tile - q * a.toc.d) * a.oct;
    g.t0             = static_cast<int>(q) * a.tt;
    g.noc            = a.oc - g.oc0 < a.oct ? a.oc - g.oc0 : a.oct;
    g.ntt            = a.t - g.t0 < a.tt ? a.t - g.t0 : a.tt;
    g.u0             = g.t0 + a.p;
    g.lb             = g.u0 >= a.k ? static_cast<int>(fastdiv(static_cast<uint32_t>(g.u0 - a.k), a.sdiv)) + 1 : 0;
    g.le             = static_cast<int>(fastdiv(static_cast<uint32_t>(g.u0 + g.ntt - 1), a.sdiv));
    g.le             = g.le < a.l - 1 ? g.le : a.l - 1;
    return g;
}

template <int NT, bool V4STORE>
__global__ __launch_bounds__(kC2iBlock) void k_col2im_1d_pipe(const Col2imArgs a, uint32_t ntiles) {
    extern __shared__ float lds2[];
    const int    tid  = static_cast<int>(threadIdx.x);
    const int    rw   = a.rwp;
    const int    bufn = a.nlmax * rw;
    const int    w    = static_cast<int>(a.rdiv.d);
    f32x4        v[kC2iBatch];
    int          at[kC2iBatch];
    // issue tile's row-piece loads into v / at (LDS offsets, -1 for none)
    auto issue = [&](const C2iTile & g) {
        const int    nrw = g.noc * a.k / 4;
        int          r   = static_cast<int>(fastdiv(static_cast<uint32_t>(tid), a.rdiv));
        int          j   = tid - r * w;
        const int    dr = kC2iBlock / w, dj = kC2iBlock % w;
        const char * cb = a.c + static_cast<int64_t>(g.oc0) * a.k * 4 + static_cast<int64_t>(g.lb) * a.cnb1;
#pragma unroll
        for (int b = 0; b < kC2iBatch; ++b) {
            const bool in = g.lb + r <= g.le && j < nrw;
            at[b]         = in ? r * rw + j * 4 : -1;
            if (in) {
                v[b] = *reinterpret_cast<const f32x4 *>(cb + static_cast<int64_t>(r) * a.cnb1 + j * 16);
            }
            r += dr;
            j += dj;
            if (j >= w) {
                j -= w;
                ++r;
            }
        }
    };
    auto write = [&](float * buf) {
#pragma unroll
        for (int b = 0; b < kC2iBatch; ++b) {
            if (at[b] >= 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    buf[at[b] + i] = v[b][i];
                }
            }
        }
    };
    uint32_t tile = blockIdx.x;
    if (tile >= ntiles) {
        return;
    }
    C2iTile g = c2i_tile(a, tile);
    issue(g);
    write(lds2);
    __syncthreads();
    int cur = 0;
    for (; tile < ntiles; tile += gridDim.x) {
        const uint32_t next = tile + gridDim.x;
        C2iTile        gn{};
        if (next < ntiles) {
            gn = c2i_tile(a, next);
            issue(gn);  // in flight while this tile's outputs are written
        }
        const float * lds = lds2 + cur * bufn;
        const int     nq  = a.tt / 4;
        for (int tl = (tid % nq) * 4; tl < g.ntt; tl += kC2iBlock * 4) {
            int      off[4][NT];
            uint32_t ok = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int u  = g.u0 + tl + e;
                const int qh = static_cast<int>(fastdiv(static_cast<uint32_t>(u), a.sdiv));
                const int r  = u - qh * a.s;
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    const int  l  = qh - (NT - 1 - j);
                    const int  k  = r + (NT - 1 - j) * a.s;
                    const bool in = tl + e < g.ntt && k < a.k && l >= 0 && l <= a.l - 1;
                    off[e][j]     = in ? (l - g.lb) * rw + k : 0;
                    ok |= static_cast<uint32_t>(in) << (e * 4 + j);
                }
            }
            for (int ocl = tid / nq; ocl < g.noc; ocl += kC2iBlock / nq) {
                char *    yrow = a.y + static_cast<int64_t>(g.oc0 + ocl) * a.ynb1;
                const int cko  = ocl * a.k;
                float     o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float acc = 0.0f;
#pragma unroll
                    for (int j = 0; j < NT; ++j) {
                        const float x = lds[cko + off[e][j]];
                        acc           = (ok >> (e * 4 + j)) & 1u ? acc + x : acc;
                    }
                    o[e] = acc;
                }
                if (V4STORE && tl + 3 < g.ntt) {
                    __builtin_nontemporal_store(f32x4{ o[0], o[1], o[2], o[3] },
                                                reinterpret_cast<f32x4 *>(yrow + static_cast<int64_t>(g.t0 + tl) * 4));
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (tl + e < g.ntt) {
                            __builtin_nontemporal_store(o[e], reinterpret_cast<float *>(yrow) + g.t0 + tl + e);
                        }
                    }
                }
            }
        }
        if (next < ntiles) {
            write(lds2 + (cur ^ 1) * bufn);
        }
        __syncthreads();
        cur ^= 1;
        g = gn;
    }
}

}  // namespace

struct Col2imPlan {
    Col2imArgs args{};
    bool       v4load  = false;
    bool       v4store = false;
    int        nt      = 0;  // ceil(K / stride) when at most 4, else 0 (any)
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
        oct = (kC2iLds / nl - 1) / K;         // rows of OCT*K values, stride rounded up to odd
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
    a.rwp          = static_cast<int32_t>((oct * K) | 1);
    a.sdiv         = make_fastdiv(static_cast<uint32_t>(stride));
    a.toc          = make_fastdiv(static_cast<uint32_t>(toc));
    // 16-byte loads: every tile's row piece starts and ends on 16 bytes
    pl.v4load = reinterpret_cast<uintptr_t>(cols->data) % 16 == 0 && (L == 1 || a.cnb1 % 16 == 0) &&
                (oct * K) % 4 == 0 && (oc * K) % 4 == 0;
    a.rdiv     = make_fastdiv(static_cast<uint32_t>(pl.v4load ? oct * K / 4 : oct * K));
    pl.v4store = reinterpret_cast<uintptr_t>(y->data) % 16 == 0 && (oc == 1 || a.ynb1 % 16 == 0);
    const int64_t nt = (K + stride - 1) / stride;
    pl.nt            = nt <= 4 ? static_cast<int>(nt) : 0;
    pl.grid          = static_cast<unsigned>(toc * tts);
    pl.shmem   = static_cast<size_t>(nl * a.rwp) * sizeof(float);
    return SHP_OK;
}

template <int NT> void launch_nt(const Col2imPlan & pl, hipStream_t s) {
    const dim3 g(pl.grid), b(kC2iBlock);
    if constexpr (NT > 0) {
        // the persistent double-buffered form, with four tiles or more per block
        // (at [128,131072] K=4: 47.6 -> 45.8 us; [256,32768] K=16: 25.6 -> 25.1;
        // with two per block, [512,8192] K=16, 12.2 -> 13.2: not taken)
        if (pl.v4load && pl.grid >= 4u * kC2iPersist) {
            const dim3 gp(pl.grid < kC2iPersist ? pl.grid : kC2iPersist);
            if (pl.v4store) {
                hipLaunchKernelGGL((k_col2im_1d_pipe<NT, true>), gp, b, 2 * pl.shmem, s, pl.args, pl.grid);
            } else {
                hipLaunchKernelGGL((k_col2im_1d_pipe<NT, false>), gp, b, 2 * pl.shmem, s, pl.args, pl.grid);
            }
            return;
        }
    }
    if (pl.v4load && pl.v4store) {
        hipLaunchKernelGGL((k_col2im_1d<NT, true, true>), g, b, pl.shmem, s, pl.args);
    } else if (pl.v4load) {
        hipLaunchKernelGGL((k_col2im_1d<NT, true, false>), g, b, pl.shmem, s, pl.args);
    } else if (pl.v4store) {
        hipLaunchKernelGGL((k_col2im_1d<NT, false, true>), g, b, pl.shmem, s, pl.args);
    } else {
        hipLaunchKernelGGL((k_col2im_1d<NT, false, false>), g, b, pl.shmem, s, pl.args);
    }
}

shp_status_t launch_col2im_1d(const Col2imPlan & pl, hipStream_t s) {
    switch (pl.nt) {
        case 1:
            launch_nt<1>(pl, s);
            break;
        case 2:
            launch_nt<2>(pl, s);
            break;
        case 3:
            launch_nt<3>(pl, s);
            break;
        case 4:
            launch_nt<4>(pl, s);
            break;
        default:
            launch_nt<0>(pl, s);
            break;
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

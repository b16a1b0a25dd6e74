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
// input is the traffic (HBM-bound).
//
// One block per tile of OWT output positions x ICT channels of one batch
// entry (no loop: a block's stores never wait at a barrier):
//   1. the tile's input window (ICT channel rows of (OWT-1)*s0 + (K-1)*d0 + 1
//      samples, zeros past the input's ends) goes to LDS, consecutive lanes on
//      consecutive addresses: along time for a time-contiguous x, along
//      channels for a channel-contiguous x (the transposed view of a
//      channel-major activation, so the ggml_cont the reference puts in front
//      of im2col is not needed);
//   2. the tile's outputs are written in y's order, V values (16 bytes) per
//      store. The LDS offsets of the values a store takes repeat with a short
//      period -- one position's run of ICT*K values, or for a tile of every
//      channel (one contiguous range of y) lcm(IC*K, V) values -- so each tile
//      first tabulates one period's offsets in LDS; a store is then one table
//      read, V window reads and running sums, with no division.
// Both phases step their indices by running sums: the kernel is bound by its
// stores, not by address arithmetic (per-value divisions held an earlier form
// to ~65 % of HBM peak at [128,131072], K = 3).

#include "shp_internal.hpp"

namespace shp {
namespace {

constexpr int kIm2colBlock = 256;
constexpr int kIm2colLds   = 4480;   // floats of LDS window per block at most (17.5 KB; with the table, 8 blocks per CU)
constexpr int kIm2colBatch = 8;      // window loads a lane issues before its LDS writes
constexpr int kIm2colTab   = 1024;   // int16 LDS offsets of the store table (one period)

// Tile shape: ict channels; at least owt positions, or enough for `elems`
// outputs; fewer positions when the window passes kIm2colLds. Measured on
// MI355X over K = 3 / 7 / 11, dilations 1-5, [128,131072] and [512,8192],
// F32 and F16 columns, both input layouts (% of HBM peak at [128,131072];
// the same-run copy reaches 75 %):
//   - runs shorter than a 128-byte line per position (ict*K*esize) cost
//     2-3x (8 channels: 21-38 %);
//   - time-contiguous x, F32, K <= 4: 16 x 64 (4096 outputs) 76 %, against
//     69 % for 32 x 128;
//   - time-contiguous x otherwise: 32 x 64, K = 11 d = 5 75 % (66-68 % for
//     16 or 64 channels, or 128 positions); F16 K = 7: 32 x 128 69 %;
//   - channel-contiguous x: 32 x 128, 76 % (63 % for 16 channels);
//   - one channel (the depthwise form): 4096 outputs 63 %, 8192 56 %.
struct TileRule {
    int ict;
    int owt;
    int elems;
};

inline TileRule tile_rule(bool chfast, bool f16, int64_t ic, int64_t k) {
    if (ic == 1) {
        return { 1, 64, 4096 };
    }
    if (chfast) {
        return { 32, 128, 8192 };
    }
    if (!f16 && k <= 4) {
        return { 16, 64, 4096 };
    }
    return f16 ? TileRule{ 32, 128, 8192 } : TileRule{ 32, 64, 8192 };
}

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
    FastDiv      rdiv;  // IC*K
    FastDiv      segf;  // ICT*K: a full channel tile's run per position
    FastDiv      segl;  // the last channel tile's run
    // window walk: ns rows of nf values (time-contiguous x: ICT channel rows of
    // wt samples; channel-contiguous x: wt sample rows of ICT channels); lane
    // tid starts at (tid / nf, tid % nf) and steps 256 values at a time
    FastDiv      fdiv;  // nf
    int32_t      ns;
    int32_t      ds;    // 256 / nf
    int32_t      df;    // 256 % nf
    int32_t      nbs;   // x byte strides of a row and of a value of the walk
    int32_t      nbf;
    int32_t      ls;    // LDS strides of the same
    int32_t      lf;
    int32_t      pad;
};

// V consecutive values of y from index e (e % V == 0 for V > 1), nontemporal.
template <int V, bool F16> __device__ __forceinline__ void put(char * y, int64_t e, const float (&v)[V]) {
    if constexpr (F16) {
        typedef _Float16 hv __attribute__((ext_vector_type(V)));
        hv h;
#pragma unroll
        for (int i = 0; i < V; ++i) {
            h[i] = static_cast<_Float16>(v[i]);
        }
        if constexpr (V == 1) {
            __builtin_nontemporal_store(h[0], reinterpret_cast<_Float16 *>(y) + e);
        } else {
            __builtin_nontemporal_store(h, reinterpret_cast<hv *>(y) + e / V);
        }
    } else {
        if constexpr (V == 1) {
            __builtin_nontemporal_store(v[0], reinterpret_cast<float *>(y) + e);
        } else {
            typedef float fv __attribute__((ext_vector_type(V)));
            fv f;
#pragma unroll
            for (int i = 0; i < V; ++i) {
                f[i] = v[i];
            }
            __builtin_nontemporal_store(f, reinterpret_cast<fv *>(y) + e / V);
        }
    }
}

// LDS offset of value f of the tile, whose values run (position, channel, tap)
// with rd.d values per position.
__device__ __forceinline__ int tap_offset(const Im2colArgs & a, uint32_t f, const FastDiv & rd) {
    const uint32_t owl = fastdiv(f, rd);
    const uint32_t j   = f - owl * rd.d;
    const uint32_t icl = fastdiv(j, a.kdiv);
    return static_cast<int>(icl) * a.wtp + static_cast<int>(owl) * a.s0 + static_cast<int>(j - icl * a.kdiv.d) * a.d0;
}

// FLAT: the tile holds every channel (ICT == IC): its outputs are one range of
// y, written in V-value stores between scalar ends (table period lcm(row, V)
// values). Otherwise each position has a run of ICT*K values, a multiple of V,
// starting V-aligned (table period: one run). V == 1: no table, one value per
// lane and step, located by division (layouts the others cannot take).
template <bool FLAT, int V, bool F16, bool CHFAST>
__global__ __launch_bounds__(kIm2colBlock) void k_im2col(const Im2colArgs a) {
    typedef int16_t         tv __attribute__((ext_vector_type(V > 1 ? V : 2)));  // one store's offsets
    extern __shared__ float lds[];
    __shared__ tv           tabv[V > 1 ? kIm2colTab / V : 1];
    int16_t *               tab = reinterpret_cast<int16_t *>(tabv);
    const int               tid = static_cast<int>(threadIdx.x);
    const uint32_t          t   = blockIdx.x;
    const uint32_t          q   = fastdiv(t, a.tic);
    const uint32_t          n   = fastdiv(q, a.tow);
    const int64_t           ic0 = static_cast<int64_t>(t - q * a.tic.d) * a.ict;
    const int64_t           ow0 = static_cast<int64_t>(q - n * a.tow.d) * a.owt;
    const int               nic = static_cast<int>(a.ic - ic0 < a.ict ? a.ic - ic0 : a.ict);
    const int               now = static_cast<int>(a.ow - ow0 < a.owt ? a.ow - ow0 : a.owt);
    const int64_t           iw0 = ow0 * a.s0 - a.p0;
    // the window's first sample (may lie before x: only in-range samples are read)
    const char *            xw  = a.x + static_cast<int64_t>(n) * a.xnb2 + ic0 * a.xnb1 + iw0 * a.xnb0;
    const int               wlo = static_cast<int>(iw0 < 0 ? -iw0 : 0);                      // first sample in x
    const int               whi = static_cast<int>(a.iw - iw0 < a.wt ? a.iw - iw0 : a.wt);  // past the last
    // 1. the window, by running sums; zeros outside [wlo, whi) and for
    //    channels past IC (never read)
    {
        const int nf = static_cast<int>(a.fdiv.d);
        int       s  = static_cast<int>(fastdiv(static_cast<uint32_t>(tid), a.fdiv));
        int       f  = tid - s * nf;
        int       ox = s * a.nbs + f * a.nbf;
        int       ol = s * a.ls + f * a.lf;
        const int sx = a.ds * a.nbs + a.df * a.nbf, cx = a.nbs - nf * a.nbf;
        const int sl = a.ds * a.ls + a.df * a.lf, cl = a.ls - nf * a.lf;
        while (s < a.ns) {
            float v[kIm2colBatch];
            int   at[kIm2colBatch];
#pragma unroll
            for (int u = 0; u < kIm2colBatch; ++u) {
                const int icl = CHFAST ? f : s;
                const int w   = CHFAST ? s : f;
                at[u]         = s < a.ns ? ol : -1;
                v[u]          = 0.0f;
                if (s < a.ns && icl < nic && w >= wlo && w < whi) {
                    v[u] = *reinterpret_cast<const float *>(xw + ox);
                }
                s += a.ds;
                f += a.df;
                ox += sx;
                ol += sl;
                if (f >= nf) {
                    f -= nf;
                    ++s;
                    ox += cx;
                    ol += cl;
                }
            }
#pragma unroll
            for (int u = 0; u < kIm2colBatch; ++u) {
                if (at[u] >= 0) {
                    lds[at[u]] = v[u];
                }
            }
        }
    }
    const int64_t ybase = (static_cast<int64_t>(n) * a.ow + ow0) * a.row + ic0 * a.k;  // first value's index
    const FastDiv sd    = nic == a.ict ? a.segf : a.segl;                              // run per position
    // the store pattern (V > 1): FLAT ranges start V-aligned after `head`
    // scalar values; P stores per period, covering cpos positions and cst
    // values of y
    int64_t       len  = 0;
    int           head = 0;
    int           P = 1, cpos = 1;
    int64_t       cst  = 0;
    int64_t       nvec = 0;
    if constexpr (V > 1) {
        if constexpr (FLAT) {
            len              = static_cast<int64_t>(now) * a.row;
            const int head0  = static_cast<int>((V - ybase % V) % V);
            head             = static_cast<int>(head0 < len ? head0 : len);
            const int64_t rw = a.row;
            const int     g  = rw % V == 0 ? V : (rw % (V / 2) == 0 ? V / 2 : (rw % 2 == 0 ? 2 : 1));  // gcd(row, V)
            P                = static_cast<int>(rw / g);  // lcm(row, V) / V
            cpos             = V / g;                     // lcm(row, V) / row
            cst              = static_cast<int64_t>(P) * V;
            nvec             = (len - head) / V;
            for (int r = tid; r < P * V; r += kIm2colBlock) {
                tab[r] = static_cast<int16_t>(tap_offset(a, static_cast<uint32_t>(head + r), a.rdiv));
            }
        } else {
            const int seg = static_cast<int>(sd.d);
            P             = seg / V;
            cst           = a.row;
            nvec          = static_cast<int64_t>(now) * P;
            for (int r = tid; r < seg; r += kIm2colBlock) {
                const uint32_t icl = fastdiv(static_cast<uint32_t>(r), a.kdiv);
                tab[r]             = static_cast<int16_t>(static_cast<int>(icl) * a.wtp +
                                                          (r - static_cast<int>(icl * a.kdiv.d)) * a.d0);
            }
        }
    }
    __syncthreads();
    // 2. the outputs, in y's order
    if constexpr (V == 1) {
        const FastDiv rd   = FLAT ? a.rdiv : sd;
        const int64_t nval = static_cast<int64_t>(now) * rd.d;
        for (int64_t f = tid; f < nval; f += kIm2colBlock) {
            const uint32_t owl   = fastdiv(static_cast<uint32_t>(f), rd);
            const float    v1[1] = { lds[tap_offset(a, static_cast<uint32_t>(f), rd)] };
            put<1, F16>(a.y, ybase + static_cast<int64_t>(owl) * a.row + (static_cast<uint32_t>(f) - owl * rd.d), v1);
        }
    } else {
        if constexpr (FLAT) {
            // the scalar ends of the range
            const int64_t tail = head + nvec * V;
            if (tid < head) {
                const float v1[1] = { lds[tap_offset(a, static_cast<uint32_t>(tid), a.rdiv)] };
                put<1, F16>(a.y, ybase + tid, v1);
            }
            if (tail + tid < len) {
                const float v1[1] = { lds[tap_offset(a, static_cast<uint32_t>(tail + tid), a.rdiv)] };
                put<1, F16>(a.y, ybase + tail + tid, v1);
            }
        }
        // store vi: period c = vi / P, entry r = vi % P, by running sums (the
        // block's 256 lanes step 256 stores: dc periods and dr entries)
        int           c      = tid / P;
        int           r      = tid - c * P;
        const int     dc     = kIm2colBlock / P, dr = kIm2colBlock % P;
        const int     lstep  = cpos * a.s0;  // window offset per period
        int           lb     = c * lstep;
        int64_t       ye     = ybase + head + static_cast<int64_t>(c) * cst + static_cast<int64_t>(r) * V;
        const int64_t ystep  = static_cast<int64_t>(dc) * cst + static_cast<int64_t>(dr) * V;
        const int64_t ycarry = cst - static_cast<int64_t>(P) * V;
        for (int64_t vi = tid; vi < nvec; vi += kIm2colBlock) {
            const tv o = tabv[r];  // one LDS read for the V offsets
            float    vals[V];
#pragma unroll
            for (int e = 0; e < V; ++e) {
                vals[e] = lds[lb + o[e]];
            }
            put<V, F16>(a.y, ye, vals);
            r += dr;
            lb += dc * lstep;
            ye += ystep;
            if (r >= P) {
                r -= P;
                lb += lstep;
                ye += ycarry;
            }
        }
    }
}

template <bool FLAT, int V, bool F16>
void launch_form(const Im2colArgs & a, bool chfast, unsigned grid, size_t shmem, hipStream_t s) {
    if (chfast) {
        hipLaunchKernelGGL((k_im2col<FLAT, V, F16, true>), dim3(grid), dim3(kIm2colBlock), shmem, s, a);
    } else {
        hipLaunchKernelGGL((k_im2col<FLAT, V, F16, false>), dim3(grid), dim3(kIm2colBlock), shmem, s, a);
    }
}

inline int64_t window(int64_t owt, int64_t s0, int64_t k, int64_t d0) {
    return (owt - 1) * s0 + (k - 1) * d0 + 1;
}

inline int64_t padded(int64_t w) {
    return w | 1;  // an odd row stride spreads a column of the window over the banks
}

inline int64_t gcd64(int64_t a, int64_t b) {
    while (b != 0) {
        const int64_t r = a % b;
        a               = b;
        b               = r;
    }
    return a;
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
    bool       flat   = false;
    int        v      = 1;   // values per store: 1, 4 (F32 or F16) or 8 (F16)
    bool       f16    = false;
    bool       chfast = false;
    unsigned   grid   = 0;   // one block per tile
    size_t     shmem  = 0;
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
    // tile: ICT channels, OWT positions, the window in LDS: as many positions
    // as wanted and fit (window + 1 for the odd row stride <= kIm2colLds /
    // ICT), fewer channels when not one position fits
    const int64_t  nb0 = static_cast<int64_t>(x->nb[0]), nb1 = static_cast<int64_t>(x->nb[1]);
    pl.chfast          = nb1 == 4 && nb0 != 4 && IC > 1;
    pl.f16             = y->type == SHP_TYPE_F16;
    const TileRule rule = tile_rule(pl.chfast, pl.f16, IC, K);
    int64_t        ict  = IC < rule.ict ? IC : rule.ict;
    int64_t owt = 0;
    for (;; ict = (ict + 1) / 2) {
        const int64_t room = kIm2colLds / ict - 1 - (K - 1) * d0 - 1;  // (owt - 1) * s0 at most
        owt                = room < 0 ? 0 : room / s0 + 1;
        if (owt >= 1 || ict == 1) {
            break;
        }
    }
    if (owt < 1) {
        return SHP_ERR_UNSUPPORTED;  // one channel's receptive field alone passes the window
    }
    const int64_t want = rule.elems / (ict * K) > rule.owt ? rule.elems / (ict * K) : rule.owt;
    owt                = owt < want ? owt : want;
    owt                = owt < OW ? owt : OW;
    const int64_t tic = (IC + ict - 1) / ict, tow = (OW + owt - 1) / owt;
    if (IC * K > INT32_MAX || OW > INT32_MAX || N > INT32_MAX || tic * tow * N > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    const int64_t wt = window(owt, s0, K, d0);
    // the window walk's byte offsets are 32-bit
    if ((ict - 1) * nb1 + (wt - 1) * nb0 + kIm2colBlock * (nb0 + nb1) > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    const int64_t last = IC - (tic - 1) * ict;  // channels of the last channel tile
    Im2colArgs &  a    = pl.args;
    a.x                = static_cast<const char *>(x->data);
    a.y                = static_cast<char *>(y->data);
    a.xnb0             = nb0;
    a.xnb1             = nb1;
    a.xnb2             = static_cast<int64_t>(x->nb[2]);
    a.iw               = IW;
    a.ic               = IC;
    a.ow               = OW;
    a.row              = IC * K;
    a.k                = static_cast<int32_t>(K);
    a.s0               = s0;
    a.p0               = p0;
    a.d0               = d0;
    a.ict              = static_cast<int32_t>(ict);
    a.owt              = static_cast<int32_t>(owt);
    a.wt               = static_cast<int32_t>(wt);
    a.wtp              = static_cast<int32_t>(padded(wt));
    a.tic              = make_fastdiv(static_cast<uint32_t>(tic));
    a.tow              = make_fastdiv(static_cast<uint32_t>(tow));
    a.kdiv             = make_fastdiv(static_cast<uint32_t>(K));
    a.rdiv             = make_fastdiv(static_cast<uint32_t>(IC * K));
    a.segf             = make_fastdiv(static_cast<uint32_t>(ict * K));
    a.segl             = make_fastdiv(static_cast<uint32_t>(last * K));
    const int64_t nf   = pl.chfast ? ict : wt;
    a.fdiv             = make_fastdiv(static_cast<uint32_t>(nf));
    a.ns               = static_cast<int32_t>(pl.chfast ? wt : ict);
    a.ds               = static_cast<int32_t>(kIm2colBlock / nf);
    a.df               = static_cast<int32_t>(kIm2colBlock % nf);
    a.nbs              = static_cast<int32_t>(pl.chfast ? nb0 : nb1);
    a.nbf              = static_cast<int32_t>(pl.chfast ? nb1 : nb0);
    a.ls               = pl.chfast ? 1 : a.wtp;
    a.lf               = pl.chfast ? a.wtp : 1;
    // Stores of 16 bytes where the layout allows (8 values of F16, 4 of F32),
    // else 8 bytes of F16, else one value. One table period must fit.
    const size_t    esz   = pl.f16 ? 2 : 4;
    const uintptr_t yaddr = reinterpret_cast<uintptr_t>(y->data);
    pl.flat               = ict == IC;
    pl.v                  = 1;
    for (int v : { pl.f16 ? 8 : 4, 4 }) {
        const bool    aligned = yaddr % (v * esz) == 0;
        const bool    runs    = (IC * K) % v == 0 && (ict * K) % v == 0;
        const int64_t per     = pl.flat ? IC * K * v / gcd64(IC * K, v) : ict * K;  // table entries
        if (aligned && (pl.flat || runs) && per <= kIm2colTab) {
            pl.v = v;
            break;
        }
    }
    pl.grid  = static_cast<unsigned>(tic * tow * N);
    pl.shmem = static_cast<size_t>(ict * a.wtp) * sizeof(float);
    return SHP_OK;
}

shp_status_t launch_im2col(const Im2colPlan & pl, hipStream_t s) {
    const Im2colArgs & a = pl.args;
    const bool         c = pl.chfast;
    if (pl.f16) {
        if (pl.flat) {
            pl.v == 8 ? launch_form<true, 8, true>(a, c, pl.grid, pl.shmem, s) :
            pl.v == 4 ? launch_form<true, 4, true>(a, c, pl.grid, pl.shmem, s) :
                        launch_form<true, 1, true>(a, c, pl.grid, pl.shmem, s);
        } else {
            pl.v == 8 ? launch_form<false, 8, true>(a, c, pl.grid, pl.shmem, s) :
            pl.v == 4 ? launch_form<false, 4, true>(a, c, pl.grid, pl.shmem, s) :
                        launch_form<false, 1, true>(a, c, pl.grid, pl.shmem, s);
        }
    } else if (pl.flat) {
        pl.v == 4 ? launch_form<true, 4, false>(a, c, pl.grid, pl.shmem, s) :
                    launch_form<true, 1, false>(a, c, pl.grid, pl.shmem, s);
    } else {
        pl.v == 4 ? launch_form<false, 4, false>(a, c, pl.grid, pl.shmem, s) :
                    launch_form<false, 1, false>(a, c, pl.grid, pl.shmem, s);
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

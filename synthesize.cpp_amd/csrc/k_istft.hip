// Kokoro's inverse short-time transform for gfx950 (kokoro/decoder-host.cpp:
// 28-100; the host runs it on the generator's output at kokoro/model.cpp:1056,
// after copying the spectrum off the device): from frames of n_fft/2 + 1
// log-magnitudes and as many raw phases, the waveform, in double as the host
// code computes it.
//
// One block per run of output samples. (1) The block's twiddles cos/sin(2 pi
// k / n_fft) go to LDS, and the complex bins of every frame its samples
// overlap -- exp(log-magnitude) * (cos, sin)(sin(raw phase)) -- are formed
// once each into LDS (a frame's bins serve its n_fft samples). (2) Each lane
// takes output samples t: position P = t + n_fft/2 is covered by the frames f
// with f*hop <= P < f*hop + n_fft; for each, in frame order, the sample
// s = P - f*hop is the real inverse DFT of the frame's bins (bin 0 and the
// Nyquist bin once, the others twice, in bin order, over n_fft), added times
// the window value, and the squared window added to the envelope; the output
// is their quotient rounded to f32, or 0 where the envelope is below 1e-11.
// The window is the periodic Hann window rounded to f32, the value the host
// code tabulates. The turn of bin b at sample s is taken from the twiddle of
// (b*s) mod n_fft: the host computes cos(2 pi b s / n_fft) of the unreduced
// product, which differs in the last bits of the double.

#include <cmath>

#include "shp_internal.hpp"

namespace shp {
namespace {

constexpr int    kIstftBlock = 256;
constexpr size_t kIstftLds   = 48 * 1024;  // bytes of LDS a block may take
constexpr double kIstftPi    = 3.14159265358979323846;

struct IstftArgs {
    const char * spec;
    int64_t      snb1;    // bytes between frames
    float *      y;
    int64_t      frames;
    int64_t      kept;    // output samples, (frames - 1) * hop
    int32_t      nfft;
    int32_t      hop;
    int32_t      bins;
    int32_t      bt;      // output samples per block
    int32_t      nf_max;  // frames a block's samples overlap, at most
    int32_t      pad;
};

__device__ __forceinline__ int64_t floor_div(int64_t a, int64_t b) {
    return a >= 0 ? a / b : -((-a + b - 1) / b);
}

__global__ __launch_bounds__(kIstftBlock) void k_istft(const IstftArgs a) {
    extern __shared__ double2 sm[];  // [nfft] twiddles, then [nf][bins] frame bins
    double2 *     tw   = sm;
    double2 *     fb   = sm + a.nfft;
    const int     tid  = static_cast<int>(threadIdx.x);
    const int64_t t0   = static_cast<int64_t>(blockIdx.x) * a.bt;
    const int64_t t1   = t0 + a.bt < a.kept ? t0 + a.bt : a.kept;
    const int     half = a.nfft / 2;
    // frames overlapping positions [t0 + half, t1 - 1 + half]
    int64_t       flo  = floor_div(t0 + half - (a.nfft - 1) + a.hop - 1, a.hop);
    flo                = flo < 0 ? 0 : flo;
    int64_t fhi        = (t1 - 1 + half) / a.hop;
    fhi                = fhi > a.frames - 1 ? a.frames - 1 : fhi;
    const int nf       = static_cast<int>(fhi - flo + 1);  // <= nf_max (host-checked bound)
    for (int k = tid; k < a.nfft; k += kIstftBlock) {
        const double turn = 2.0 * kIstftPi * static_cast<double>(k) / static_cast<double>(a.nfft);
        double       sn, cs;
        sincos(turn, &sn, &cs);
        tw[k] = double2{ cs, sn };
    }
    for (int i = tid; i < nf * a.bins; i += kIstftBlock) {
        const int     f   = i / a.bins;
        const int     b   = i - f * a.bins;
        const float * row = reinterpret_cast<const float *>(a.spec + (flo + f) * a.snb1);
        const double  mag = exp(static_cast<double>(row[b]));
        const double  ang = sin(static_cast<double>(row[a.bins + b]));
        double        sn, cs;
        sincos(ang, &sn, &cs);
        fb[i] = double2{ mag * cs, mag * sn };
    }
    __syncthreads();
    for (int64_t t = t0 + tid; t < t1; t += kIstftBlock) {
        const int64_t P  = t + half;
        int64_t       fa = floor_div(P - (a.nfft - 1) + a.hop - 1, a.hop);
        fa               = fa < flo ? flo : fa;
        int64_t fz       = P / a.hop;
        fz               = fz > fhi ? fhi : fz;
        double acc = 0.0, env = 0.0;
        for (int64_t f = fa; f <= fz; ++f) {
            const int       s   = static_cast<int>(P - f * a.hop);
            const double2 * bf  = fb + (f - flo) * a.bins;
            double          v   = 0.0;
            int             k   = 0;  // (b * s) mod nfft
            for (int b = 0; b < a.bins; ++b) {
                const double  w  = (b == 0 || b == a.bins - 1) ? 1.0 : 2.0;
                const double2 c  = tw[k];
                const double2 z  = bf[b];
                v += w * (z.x * c.x - z.y * c.y);
                k += s;
                k = k >= a.nfft ? k - a.nfft : k;
            }
            v                 = v / static_cast<double>(a.nfft);
            const double  win = static_cast<double>(static_cast<float>(0.5 * (1.0 - tw[s].x)));
            acc += v * win;
            env += win * win;
        }
        a.y[t] = fabs(env) < static_cast<double>(1e-11f) ? 0.0f : static_cast<float>(acc / env);
    }
}

}  // namespace
}  // namespace shp

using namespace shp;

extern "C" shp_status_t shp_inverse_stft(const shp_tensor * spectrum,
                                         int32_t            n_fft,
                                         int32_t            hop,
                                         shp_tensor *       audio,
                                         shp_stream_t       stream) {
    if (!well_formed(spectrum) || !well_formed(audio) || n_fft < 2 || n_fft % 2 != 0 || hop <= 0) {
        return SHP_ERR_INVALID_ARG;
    }
    if (spectrum->type != SHP_TYPE_F32 || audio->type != SHP_TYPE_F32) {
        return SHP_ERR_UNSUPPORTED;
    }
    const int64_t frames = spectrum->ne[1];
    if (spectrum->ne[0] != n_fft + 2 || spectrum->ne[2] != 1 || spectrum->ne[3] != 1 || frames < 2 ||
        audio->ne[0] != (frames - 1) * hop || audio->ne[1] != 1 || audio->ne[2] != 1 || audio->ne[3] != 1) {
        return SHP_ERR_INVALID_ARG;
    }
    if (spans_overlap(*spectrum, *audio) || frames > INT32_MAX || audio->ne[0] > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    // Output samples per block: the most (256, 128 or 64) whose frames' bins
    // and the twiddles fit the LDS budget.
    const int64_t bins = n_fft / 2 + 1;
    int64_t       bt = 0, nf_max = 0;
    for (int64_t cand : { 256, 128, 64 }) {
        const int64_t nf = (cand - 1 + n_fft - 1) / hop + 2;
        if (static_cast<size_t>(nf * bins + n_fft) * sizeof(double2) <= kIstftLds) {
            bt     = cand;
            nf_max = nf;
            break;
        }
    }
    if (bt == 0) {
        return SHP_ERR_UNSUPPORTED;  // windows too long for their hop to stage a block's frames
    }
    if (dry_run()) {
        return SHP_OK;
    }
    IstftArgs a{};
    a.spec       = static_cast<const char *>(spectrum->data);
    a.snb1       = static_cast<int64_t>(spectrum->nb[1]);
    a.y          = static_cast<float *>(audio->data);
    a.frames     = frames;
    a.kept       = audio->ne[0];
    a.nfft       = n_fft;
    a.hop        = hop;
    a.bins       = static_cast<int32_t>(bins);
    a.bt         = static_cast<int32_t>(bt);
    a.nf_max     = static_cast<int32_t>(nf_max);
    const size_t lds    = static_cast<size_t>(nf_max * bins + n_fft) * sizeof(double2);
    const int64_t blocks = (a.kept + bt - 1) / bt;
    hipLaunchKernelGGL(k_istft, dim3(static_cast<unsigned>(blocks)), dim3(kIstftBlock), lds, as_stream(stream), a);
    return launch_status();
}

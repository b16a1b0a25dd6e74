// The Qwen3-TTS speaker encoder's log-mel front end for gfx950
// (qwen3-tts/mel.cpp:63-299, compute_log_mel; the reference runs it on the
// host before the ECAPA graph): PCM to [mel_bins, frames] log energies.
//
// One 256-thread block per frame: the frame's reflect-padded samples times the
// periodic Hann window go to LDS at their bit-reversed places; the FFT's
// n_fft - 1 twiddles cos/sin((-2 pi / len) * k) are tabulated in LDS in
// double, as the host code evaluates them; log2(n_fft) radix-2 stages run
// with a barrier between them, each butterfly's products and sums in double
// and its two results rounded to f32 -- the host code's in-place transform,
// stage for stage; then the amplitudes sqrt(re^2 + im^2 + 1e-9) (double,
// rounded), and per mel bin the filterbank-weighted sum in double in
// frequency order and log(max(energy, 1e-5)). The device's double cos, sin,
// sqrt and log replace the host library's; sqrt is correctly rounded on both.
//
// shp_mel_filterbank is the Slaney filterbank the transform is weighted with
// (mel.cpp:96-170), computed on the host once per model.

#include <cmath>
#include <vector>

#include "shp_internal.hpp"

namespace shp {
namespace {

constexpr double kMelPi      = 3.14159265358979323846;
constexpr int    kMelMaxNfft = 2048;

struct MelArgs {
    const float * pcm;
    const float * fb;  // [bins][n_fft/2 + 1]
    float *       y;   // [frames][bins]
    int64_t       ns;
    int64_t       frames;
    int32_t       nfft;
    int32_t       log2n;
    int32_t       hop;
    int32_t       win;
    int32_t       pad;
    int32_t       bins;
};

__global__ __launch_bounds__(256) void k_log_mel(const MelArgs a) {
    extern __shared__ double2 s_tw[];  // [nfft - 1] twiddles, then re, im (f32), then amplitudes
    float *       s_re  = reinterpret_cast<float *>(s_tw + (a.nfft - 1));
    float *       s_im  = s_re + a.nfft;
    float *       s_mag = s_im + a.nfft;
    const int     tid   = static_cast<int>(threadIdx.x);
    const int64_t f     = blockIdx.x;
    const int     n     = a.nfft;
    const int     nf    = n / 2 + 1;
    // twiddle idx = len/2 - 1 + k for stage length len and butterfly offset k
    for (int idx = tid; idx < n - 1; idx += 256) {
        const int    half  = 1 << (31 - __clz(idx + 1));  // len / 2
        const int    len   = half * 2;
        const int    k     = idx - (half - 1);
        const double angle = -2.0 * kMelPi / static_cast<double>(len);
        double       sn, cs;
        sincos(angle * static_cast<double>(k), &sn, &cs);
        s_tw[idx] = double2{ cs, sn };
    }
    const int wpl = (n - a.win) / 2;
    for (int i = tid; i < n; i += 256) {
        // the padded signal at frame start + i: reflect-padded by `pad`
        const int64_t p = f * a.hop + i;
        float         x;
        if (p < a.pad) {
            x = a.pcm[a.pad - p];
        } else if (p < a.pad + a.ns) {
            x = a.pcm[p - a.pad];
        } else {
            x = a.pcm[a.ns - 2 - (p - a.pad - a.ns)];
        }
        float w = 0.0f;
        if (i >= wpl && i < wpl + a.win) {
            const double phase = 2.0 * kMelPi * static_cast<double>(i - wpl) / static_cast<double>(a.win);
            w                  = static_cast<float>(0.5 - 0.5 * cos(phase));
        }
        const int r = static_cast<int>(__brev(static_cast<unsigned>(i)) >> (32 - a.log2n));
        s_re[r]     = x * w;
        s_im[r]     = 0.0f;
    }
    __syncthreads();
    for (int half = 1; half < n; half *= 2) {
        for (int t = tid; t < n / 2; t += 256) {
            const int     k   = t & (half - 1);
            const int     ia  = (t - k) * 2 + k;  // start + k, start = (t / half) * 2 * half
            const int     ib  = ia + half;
            const double2 tw  = s_tw[half - 1 + k];
            const double  xr  = static_cast<double>(s_re[ib]) * tw.x - static_cast<double>(s_im[ib]) * tw.y;
            const double  xi  = static_cast<double>(s_re[ib]) * tw.y + static_cast<double>(s_im[ib]) * tw.x;
            const double  ar  = s_re[ia];
            const double  ai  = s_im[ia];
            s_re[ib]          = static_cast<float>(ar - xr);
            s_im[ib]          = static_cast<float>(ai - xi);
            s_re[ia]          = static_cast<float>(ar + xr);
            s_im[ia]          = static_cast<float>(ai + xi);
        }
        __syncthreads();
    }
    for (int k = tid; k < nf; k += 256) {
        const double sq = static_cast<double>(s_re[k]) * static_cast<double>(s_re[k]) +
                          static_cast<double>(s_im[k]) * static_cast<double>(s_im[k]);
        s_mag[k]        = static_cast<float>(sqrt(sq + 1e-9));
    }
    __syncthreads();
    for (int b = tid; b < a.bins; b += 256) {
        const float * row = a.fb + static_cast<int64_t>(b) * nf;
        double        e   = 0.0;
        for (int k = 0; k < nf; ++k) {
            e += static_cast<double>(row[k]) * static_cast<double>(s_mag[k]);
        }
        a.y[f * a.bins + b] = static_cast<float>(log(e < 1e-5 ? 1e-5 : e));  // std::max(e, 1e-5)
    }
}

double slaney_step() {
    return std::log(6.4) / 27.0;
}

double hz_to_mel(double hz) {
    const double min_log_mel = 1000.0 / (200.0 / 3.0);
    return hz >= 1000.0 ? min_log_mel + std::log(hz / 1000.0) / slaney_step() : hz / (200.0 / 3.0);
}

double mel_to_hz(double mel) {
    const double min_log_mel = 1000.0 / (200.0 / 3.0);
    return mel >= min_log_mel ? 1000.0 * std::exp(slaney_step() * (mel - min_log_mel)) : (200.0 / 3.0) * mel;
}

bool pow2(int64_t v) {
    return v > 0 && (v & (v - 1)) == 0;
}

}  // namespace
}  // namespace shp

using namespace shp;

extern "C" shp_status_t shp_mel_filterbank(int32_t sample_rate, int32_t n_fft, int32_t mel_bins, float fmin, float fmax,
                                           float * out) {
    if (out == nullptr || sample_rate < 1 || n_fft < 2 || mel_bins < 1) {
        return SHP_ERR_INVALID_ARG;
    }
    const int64_t       nf = n_fft / 2 + 1;
    std::vector<double> edges(static_cast<size_t>(mel_bins) + 2);
    const double        lo = hz_to_mel(static_cast<double>(fmin)), hi = hz_to_mel(static_cast<double>(fmax));
    for (size_t i = 0; i < edges.size(); ++i) {
        edges[i] = mel_to_hz(lo + (hi - lo) * static_cast<double>(i) / static_cast<double>(mel_bins + 1));
    }
    for (int64_t b = 0; b < mel_bins; ++b) {
        const double enorm = 2.0 / (edges[b + 2] - edges[b]);
        for (int64_t k = 0; k < nf; ++k) {
            const double hz    = static_cast<double>(k) * static_cast<double>(sample_rate) / static_cast<double>(n_fft);
            const double lower = (hz - edges[b]) / (edges[b + 1] - edges[b]);
            const double upper = (edges[b + 2] - hz) / (edges[b + 2] - edges[b + 1]);
            const double v     = upper < lower ? upper : lower;  // std::min(lower, upper)
            out[b * nf + k]    = static_cast<float>((0.0 < v ? v : 0.0) * enorm);
        }
    }
    return SHP_OK;
}

extern "C" shp_status_t shp_log_mel(const shp_tensor * pcm,
                                    const shp_tensor * filterbank,
                                    int32_t            n_fft,
                                    int32_t            hop,
                                    int32_t            win_length,
                                    shp_tensor *       mel,
                                    shp_stream_t       stream) {
    if (!well_formed(pcm) || !well_formed(filterbank) || !well_formed(mel)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (pcm->type != SHP_TYPE_F32 || filterbank->type != SHP_TYPE_F32 || mel->type != SHP_TYPE_F32 ||
        !contiguous(*pcm) || !contiguous(*filterbank) || !contiguous(*mel)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (!pow2(n_fft) || hop < 1 || win_length < 1 || win_length > n_fft || hop > n_fft) {
        return SHP_ERR_INVALID_ARG;
    }
    const int64_t ns   = nelements(*pcm);
    const int64_t pad  = (n_fft - hop) / 2;
    const int64_t plen = ns + 2 * pad;
    const int64_t bins = filterbank->ne[1];
    // upstream's reflect pad needs more samples than the pad
    if (ns <= pad || plen < n_fft || filterbank->ne[0] != n_fft / 2 + 1 || nelements(*filterbank) != bins * (n_fft / 2 + 1)) {
        return SHP_ERR_INVALID_ARG;
    }
    const int64_t frames = 1 + (plen - n_fft) / hop;
    if (mel->ne[0] != bins || nelements(*mel) != bins * frames) {
        return SHP_ERR_INVALID_ARG;
    }
    if (n_fft > kMelMaxNfft || frames > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (spans_overlap(*pcm, *mel) || spans_overlap(*filterbank, *mel)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (dry_run()) {
        return SHP_OK;
    }
    MelArgs a{};
    a.pcm    = static_cast<const float *>(pcm->data);
    a.fb     = static_cast<const float *>(filterbank->data);
    a.y      = static_cast<float *>(mel->data);
    a.ns     = ns;
    a.frames = frames;
    a.nfft   = n_fft;
    a.log2n  = 31 - __builtin_clz(static_cast<unsigned>(n_fft));
    a.hop    = hop;
    a.win    = win_length;
    a.pad    = static_cast<int32_t>(pad);
    a.bins   = static_cast<int32_t>(bins);
    const size_t lds = static_cast<size_t>(n_fft - 1) * sizeof(double2) + static_cast<size_t>(2 * n_fft + n_fft / 2 + 1) * sizeof(float);
    hipLaunchKernelGGL(k_log_mel, dim3(static_cast<unsigned>(frames)), dim3(256), lds, as_stream(stream), a);
    return launch_status();
}

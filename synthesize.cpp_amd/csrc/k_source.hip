// Kokoro's harmonic-plus-noise source and its short-time spectrum for gfx950
// (kokoro/source.cpp:60-184, build_harmonic_source; the host runs it between
// the prosody and generator graphs). Four launches on one stream:
//
//   k_source_coarse (a lane per frame and harmonic): the phase increments
//     frac(f0 * (h+1) / rate) of the upsampled grid, resampled linearly to the
//     f0 grid (PyTorch's align_corners=false mapping, in double, the weight
//     rounded to f32), staged in the spectrum output's own memory until the
//     excitation launch has read them;
//   k_source_phase (one block): each harmonic's running f32 sum in frame
//     order -- one lane per harmonic, the order the host code adds in, so the
//     sums are bit for bit its own -- over LDS chunks, and the phase
//     running * 2 pi * scale (double, rounded) in place of the increment;
//   k_source_excite (a lane per upsampled sample): the phase resampled back,
//     sin(phase) * amp for voiced samples plus the noise at its gain, merged
//     with the weights in harmonic order from the bias, tanh;
//   k_source_stft (a lane per frame and bin): torch.stft's centred framing --
//     reflect padding by n_fft/2, the periodic Hann window rounded to f32 --
//     and the DFT in double with the host code's twiddles (the angle
//     -2 pi b k / n_fft as it computes it), the magnitude by hypot and the
//     phase by atan2, each rounded to f32.
// The f32 sine and tanh are the device's, within an ulp or two of the host
// library's; everything else is the host code's arithmetic in its order.

#include <cmath>

#include "shp_internal.hpp"

namespace shp {
namespace {

constexpr double kSrcPi       = 3.14159265358979323846;
constexpr int    kSrcMaxH     = 64;    // harmonics
constexpr int    kSrcMaxNfft  = 64;    // window (the twiddle table holds (n_fft/2 + 1) x n_fft entries)
constexpr int    kSrcChunk    = 8192;  // coarse values per LDS chunk

struct SourceArgs {
    const float * f0;
    const float * mw;     // merge weights
    const float * ri;     // initial phases
    const float * noise;  // [U][H]
    float *       exc;    // [U]
    float *       har;    // [frames][2*bins]; first L*H floats stage the phase
    int64_t       L;
    int64_t       U;
    int64_t       frames;
    float         bias;
    float         amp;
    float         noise_std;
    float         threshold;
    float         rate;
    int32_t       H;
    int32_t       scale;
    int32_t       nfft;
    int32_t       hop;
    int32_t       bins;
};

// The increment of harmonic h at upsampled sample u.
__device__ __forceinline__ float increment(const SourceArgs & a, int64_t u, int h) {
    const float v = a.f0[u / a.scale] * static_cast<float>(h + 1) / a.rate;
    float       r = v - floorf(v);
    if (u == 0) {
        r += a.ri[h];
    }
    return r;
}

// PyTorch's align_corners=false source position for output o, clamped at 0:
// its lower index, upper index and f32 weight.
__device__ __forceinline__ void linear_at(int64_t o, double ratio, int64_t in_len, int64_t & lo, int64_t & hi,
                                          float & w) {
    double position = (static_cast<double>(o) + 0.5) * ratio - 0.5;
    position        = position < 0.0 ? 0.0 : position;
    lo              = static_cast<int64_t>(position);
    hi              = lo + 1 < in_len ? lo + 1 : in_len - 1;
    w               = static_cast<float>(position - static_cast<double>(lo));
}

// The coarse increments, one lane per (frame, harmonic), staged in har.
__global__ __launch_bounds__(256) void k_source_coarse(const SourceArgs a) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= a.L * a.H) {
        return;
    }
    const int64_t j = i / a.H;
    const int     h = static_cast<int>(i - j * a.H);
    int64_t       lo, hi;
    float         w;
    linear_at(j, static_cast<double>(a.U) / static_cast<double>(a.L), a.U, lo, hi, w);
    a.har[i] = increment(a, lo, h) * (1.0f - w) + increment(a, hi, h) * w;
}

// The running sums, one lane per harmonic in frame order, over LDS chunks of
// the staged increments (each chunk read and written back in one coalesced
// pass); the phase replaces the increment in place.
__global__ __launch_bounds__(256) void k_source_phase(const SourceArgs a) {
    extern __shared__ float s_run[];  // [chunk][H]
    const int     tid   = static_cast<int>(threadIdx.x);
    const int     H     = a.H;
    const int64_t chunk = kSrcChunk / H;
    float         run   = 0.0f;  // lane h < H: harmonic h's running sum
    for (int64_t j0 = 0; j0 < a.L; j0 += chunk) {
        const int64_t nj = a.L - j0 < chunk ? a.L - j0 : chunk;
        const int64_t n = nj * H;
        for (int64_t i0 = tid; i0 < n; i0 += 256 * 8) {  // eight loads in flight per lane
            float v[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int64_t i = i0 + q * 256;
                v[q]            = i < n ? a.har[j0 * H + i] : 0.0f;
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int64_t i = i0 + q * 256;
                if (i < n) {
                    s_run[i] = v[q];
                }
            }
        }
        __syncthreads();
        if (tid < H) {
            constexpr int kAhead = 16;  // reads ahead of their adds; the sums stay in frame order
            int64_t       j      = 0;
            for (; j + kAhead <= nj; j += kAhead) {
                float v[kAhead];
#pragma unroll
                for (int q = 0; q < kAhead; ++q) {
                    v[q] = s_run[(j + q) * H + tid];
                }
#pragma unroll
                for (int q = 0; q < kAhead; ++q) {
                    run = run + v[q];
                    v[q] = run;
                }
#pragma unroll
                for (int q = 0; q < kAhead; ++q) {
                    s_run[(j + q) * H + tid] = v[q];
                }
            }
            for (; j < nj; ++j) {
                run                = run + s_run[j * H + tid];
                s_run[j * H + tid] = run;
            }
        }
        __syncthreads();
        for (int64_t i = tid; i < nj * H; i += 256) {
            a.har[j0 * H + i] = static_cast<float>(static_cast<double>(s_run[i]) * 2.0 * kSrcPi *
                                                   static_cast<double>(a.scale));
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void k_source_excite(const SourceArgs a) {
    const int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (u >= a.U) {
        return;
    }
    int64_t lo, hi;
    float   w;
    linear_at(u, static_cast<double>(a.L) / static_cast<double>(a.U), a.L, lo, hi, w);
    const float   f0u    = a.f0[u / a.scale];
    const float   uv     = f0u > a.threshold ? 1.0f : 0.0f;
    const float   gain   = uv * a.noise_std + (1.0f - uv) * a.amp / 3.0f;
    const float * plo    = a.har + lo * a.H;
    const float * phi    = a.har + hi * a.H;
    const float * nz     = a.noise + u * a.H;
    float         merged = a.bias;
    for (int h = 0; h < a.H; ++h) {
        const float fine  = plo[h] * (1.0f - w) + phi[h] * w;
        const float sine  = sinf(fine) * a.amp;
        const float value = sine * uv + gain * nz[h];
        merged            = merged + a.mw[h] * value;
    }
    a.exc[u] = tanhf(merged);
}

__global__ __launch_bounds__(256) void k_source_stft(const SourceArgs a) {
    __shared__ double2 s_tw[(kSrcMaxNfft / 2 + 1) * kSrcMaxNfft];
    __shared__ float   s_win[kSrcMaxNfft];
    const int tid = static_cast<int>(threadIdx.x);
    for (int i = tid; i < a.bins * a.nfft; i += 256) {
        const int    b     = i / a.nfft;
        const int    k     = i - b * a.nfft;
        const double angle = -2.0 * kSrcPi * static_cast<double>(b) * static_cast<double>(k) / static_cast<double>(a.nfft);
        s_tw[i]            = double2{ cos(angle), sin(angle) };
    }
    for (int k = tid; k < a.nfft; k += 256) {
        s_win[k] = static_cast<float>(0.5 * (1.0 - cos(2.0 * kSrcPi * static_cast<double>(k) / static_cast<double>(a.nfft))));
    }
    __syncthreads();
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + tid;
    if (i >= a.frames * a.bins) {
        return;
    }
    const int64_t f    = i / a.bins;
    const int     b    = static_cast<int>(i - f * a.bins);
    const int     half = a.nfft / 2;
    const int64_t last = a.U - 1;
    double        re = 0.0, im = 0.0;
    for (int k = 0; k < a.nfft; ++k) {
        int64_t src = f * a.hop + k - half;
        while (src < 0 || src > last) {  // reflection without repeating the edge sample
            src = src < 0 ? -src : 2 * last - src;
        }
        const float   seg = a.exc[src] * s_win[k];
        const double2 t   = s_tw[b * a.nfft + k];
        re += static_cast<double>(seg) * t.x;
        im += static_cast<double>(seg) * t.y;
    }
    float * row       = a.har + f * 2 * a.bins;
    row[b]            = static_cast<float>(hypot(re, im));
    row[a.bins + b]   = static_cast<float>(atan2(im, re));
}

bool contiguous_f32(const shp_tensor * t) {
    return well_formed(t) && t->type == SHP_TYPE_F32 && contiguous(*t) && reinterpret_cast<uintptr_t>(t->data) % 4 == 0;
}

}  // namespace
}  // namespace shp

using namespace shp;

extern "C" shp_status_t shp_harmonic_source(const shp_tensor * f0,
                                            const shp_tensor * merge_weight,
                                            float              merge_bias,
                                            const shp_tensor * rand_ini,
                                            const shp_tensor * noise,
                                            int32_t            sampling_rate,
                                            int32_t            upsample_scale,
                                            float              sine_amp,
                                            float              noise_std,
                                            float              voiced_threshold,
                                            int32_t            n_fft,
                                            int32_t            hop,
                                            shp_tensor *       excitation,
                                            shp_tensor *       har,
                                            shp_stream_t       stream) {
    if (!contiguous_f32(f0) || !contiguous_f32(merge_weight) || !contiguous_f32(rand_ini) || !contiguous_f32(noise) ||
        !contiguous_f32(excitation) || !contiguous_f32(har)) {
        return SHP_ERR_INVALID_ARG;
    }
    const int64_t L = nelements(*f0), H = nelements(*merge_weight);
    if (sampling_rate < 1 || upsample_scale < 1 || n_fft < 2 || n_fft % 2 != 0 || hop < 1 || nelements(*rand_ini) != H) {
        return SHP_ERR_INVALID_ARG;
    }
    const int64_t U = L * upsample_scale, bins = n_fft / 2 + 1, frames = U / hop + 1;
    // one sample cannot be reflect-padded (the host code's reflection loop
    // would not end)
    if (U < 2 || noise->ne[0] != H || nelements(*noise) != U * H || nelements(*excitation) != U || har->ne[0] != 2 * bins ||
        nelements(*har) != frames * 2 * bins) {
        return SHP_ERR_INVALID_ARG;
    }
    // the kernel limits; the spectrum's memory stages the L*H coarse phases
    if (H > kSrcMaxH || n_fft > kSrcMaxNfft || L * H > frames * 2 * bins || U > INT32_MAX ||
        frames * bins > INT32_MAX) {
        return SHP_ERR_UNSUPPORTED;
    }
    const shp_tensor * ins[] = { f0, merge_weight, rand_ini, noise };
    for (const shp_tensor * t : ins) {
        if (spans_overlap(*t, *excitation) || spans_overlap(*t, *har)) {
            return SHP_ERR_UNSUPPORTED;
        }
    }
    if (spans_overlap(*excitation, *har)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (dry_run()) {
        return SHP_OK;
    }
    SourceArgs a{};
    a.f0        = static_cast<const float *>(f0->data);
    a.mw        = static_cast<const float *>(merge_weight->data);
    a.ri        = static_cast<const float *>(rand_ini->data);
    a.noise     = static_cast<const float *>(noise->data);
    a.exc       = static_cast<float *>(excitation->data);
    a.har       = static_cast<float *>(har->data);
    a.L         = L;
    a.U         = U;
    a.frames    = frames;
    a.bias      = merge_bias;
    a.amp       = sine_amp;
    a.noise_std = noise_std;
    a.threshold = voiced_threshold;
    a.rate      = static_cast<float>(sampling_rate);
    a.H         = static_cast<int32_t>(H);
    a.scale     = upsample_scale;
    a.nfft      = n_fft;
    a.hop       = hop;
    a.bins      = static_cast<int32_t>(bins);
    const hipStream_t st    = as_stream(stream);
    const int64_t     chunk = kSrcChunk / H;
    hipLaunchKernelGGL(k_source_coarse, dim3(static_cast<unsigned>((L * H + 255) / 256)), dim3(256), 0, st, a);
    shp_status_t s = launch_status();
    if (s != SHP_OK) {
        return s;
    }
    hipLaunchKernelGGL(k_source_phase, dim3(1), dim3(256), static_cast<size_t>(chunk * H) * sizeof(float), st, a);
    s = launch_status();
    if (s != SHP_OK) {
        return s;
    }
    hipLaunchKernelGGL(k_source_excite, dim3(static_cast<unsigned>((U + 255) / 256)), dim3(256), 0, st, a);
    s = launch_status();
    if (s != SHP_OK) {
        return s;
    }
    hipLaunchKernelGGL(k_source_stft, dim3(static_cast<unsigned>((frames * bins + 255) / 256)), dim3(256), 0, st, a);
    return launch_status();
}

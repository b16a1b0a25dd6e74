// TEST INFRASTRUCTURE ONLY: a C entry point over the reference's own
// synth::kokoro::build_harmonic_source (kokoro/source.cpp:60-184), compiled from
// the reference checkout by `make -C oracle ref` into oracle/_ref/. Only the
// tests load it, to hold the restatement (op_harmonic_source in
// ggml_cpu_ref.c) to the reference's compiled host code.
#include "source.h"
#include "weights.h"

#include <cstdint>
#include <cstring>
#include <vector>

extern "C" int ref_harmonic_source(const float * f0, uint64_t f0_len, const float * merge_weight, float merge_bias,
                                   const float * rand_ini, const float * noise, uint32_t harmonics, uint32_t rate,
                                   uint32_t scale, float sine_amp, float noise_std, float voiced_threshold,
                                   uint32_t n_fft, uint32_t hop, float * excitation, uint64_t excitation_len,
                                   float * har, uint64_t har_len) {
    synth::kokoro::HParams h;
    h.source.sampling_rate        = rate;
    h.source.harmonic_num         = harmonics - 1;
    h.source.upsample_scale       = scale;
    h.source.sine_amp             = sine_amp;
    h.source.noise_std            = noise_std;
    h.source.voiced_threshold     = voiced_threshold;
    h.istftnet.gen_istft_n_fft    = n_fft;
    h.istftnet.gen_istft_hop_size = hop;
    synth::kokoro::SourceRandomInputs random;
    random.rand_ini.assign(rand_ini, rand_ini + harmonics);
    random.noise.assign(noise, noise + f0_len * scale * harmonics);
    synth::kokoro::SourceResult out;
    const synth_status_t st = synth::kokoro::build_harmonic_source(
        h, std::vector<float>(f0, f0 + f0_len), std::vector<float>(merge_weight, merge_weight + harmonics),
        merge_bias, random, out);
    if (st != SYNTH_OK) {
        return static_cast<int>(st);
    }
    if (out.har_source.size() != excitation_len || out.har.size() != har_len) {
        return -1000;
    }
    std::memcpy(excitation, out.har_source.data(), excitation_len * sizeof(float));
    std::memcpy(har, out.har.data(), har_len * sizeof(float));
    return 0;
}

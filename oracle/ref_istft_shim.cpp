// TEST INFRASTRUCTURE ONLY: a C entry point over the reference's own
// synth::kokoro::inverse_stft (kokoro/decoder-host.cpp:28-100), compiled from
// the reference checkout by `make -C oracle ref` into oracle/_ref/. Only the
// tests load it, to hold the restatement (op_istft in ggml_cpu_ref.c) to the
// reference's compiled host code.
#include "decoder-host.h"
#include "weights.h"

#include <cstdint>
#include <cstring>
#include <vector>

extern "C" int ref_inverse_stft(const float * spectrum, uint64_t frames, uint32_t n_fft, uint32_t hop, float * audio,
                                uint64_t audio_len) {
    synth::kokoro::HParams h;
    h.istftnet.gen_istft_n_fft    = n_fft;
    h.istftnet.gen_istft_hop_size = hop;
    const std::vector<float> spec(spectrum, spectrum + frames * (uint64_t(n_fft) + 2));
    std::vector<float>       out;
    const synth_status_t     st = synth::kokoro::inverse_stft(h, spec, frames, out);
    if (st != SYNTH_OK) {
        return static_cast<int>(st);
    }
    if (out.size() != audio_len) {
        return -1000;
    }
    std::memcpy(audio, out.data(), out.size() * sizeof(float));
    return 0;
}

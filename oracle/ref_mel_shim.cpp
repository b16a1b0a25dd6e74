// TEST INFRASTRUCTURE ONLY: a C entry point over the reference's own
// synth::qwen3tts::compute_log_mel (qwen3-tts/mel.cpp:174-299), compiled from
// the reference checkout by `make -C oracle ref` into oracle/_ref/. Only the
// tests load it, to hold the restatement (op_log_mel and orc_mel_filterbank in
// ggml_cpu_ref.c) to the reference's compiled host code.
#include "mel.h"
#include "weights.h"

#include <cstdint>
#include <cstring>
#include <vector>

extern "C" int ref_log_mel(const float * pcm, uint64_t samples, uint32_t sample_rate, uint32_t n_fft, uint32_t hop,
                           uint32_t win_length, uint32_t mel_bins, float fmin, float fmax, float * out,
                           uint64_t out_len, uint64_t * frames) {
    synth::qwen3tts::SpeakerEncoderParams p;
    p.sample_rate = sample_rate;
    p.n_fft       = n_fft;
    p.hop_length  = hop;
    p.win_length  = win_length;
    p.mel_bins    = mel_bins;
    p.fmin        = fmin;
    p.fmax        = fmax;
    synth::qwen3tts::MelSpectrogram mel;
    const synth_status_t st = synth::qwen3tts::compute_log_mel(p, std::vector<float>(pcm, pcm + samples), mel);
    if (st != SYNTH_OK) {
        return static_cast<int>(st);
    }
    *frames = mel.frames;
    if (mel.values.size() > out_len) {
        return -1000;
    }
    std::memcpy(out, mel.values.data(), mel.values.size() * sizeof(float));
    return 0;
}

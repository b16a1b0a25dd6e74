"""shp_log_mel against the restatement of the Qwen3-TTS speaker encoder's
compute_log_mel (qwen3-tts/mel.cpp:174-299), which equals the reference's
own compiled code bit for bit: one-second and ten-second clips of noise and
tones at the production parameters (n_fft 1024, hop 256, 128 Slaney bins to
12 kHz), hop 512, a shorter zero-padded window with fewer bins, the
shortest clip the reflect pad allows; the upstream frame counts (93, 46).
The FFT is the host code's, stage for stage, with f32 results; the device's
double cos/sin/log move a twiddle or a log in its last bit, so the log
energies are held within 1e-5 and > 99 % identical."""
import numpy as np
import pytest

from test_gpu_parity import _np, _t
from test_oracle_goldens import MEL, oracle_log_mel

pytestmark = pytest.mark.gpu

SEED = 20261218


def _gpu_mel(gpu, pcm, p):
    fb = gpu.mel_filterbank(p["sample_rate"], p["n_fft"], p["mel_bins"], p["fmin"], p["fmax"])
    return _np(gpu.log_mel(_t(gpu, pcm), _t(gpu, fb), p["n_fft"], p["hop"], p["win_length"]))


def _close(got, ref):
    assert got.shape == ref.shape
    assert np.abs(got - ref).max() <= 1e-5
    assert (got == ref).mean() > 0.99


@pytest.mark.parametrize("kind,seconds,p", [("noise", 1, MEL), ("tone", 1, MEL), ("noise", 10, MEL),
                                            ("tone", 1, dict(MEL, hop=512)),
                                            ("noise", 1, dict(MEL, n_fft=512, win_length=400, hop=160, mel_bins=80)),
                                            ("noise", 1, dict(MEL, n_fft=2048, win_length=2048, hop=512))])
def test_log_mel_matches_restatement(gpu, kind, seconds, p):
    ns = 24000 * seconds
    rng = np.random.default_rng([SEED, ns, p["n_fft"], p["hop"]])
    pcm = (rng.standard_normal(ns) * 0.2).astype(np.float32) if kind == "noise" else \
        (0.4 * np.sin(2 * np.pi * 440 * np.arange(ns) / 24000)).astype(np.float32)
    _close(_gpu_mel(gpu, pcm, p), oracle_log_mel(pcm, p))


def test_log_mel_frame_counts_and_short_clips(gpu):
    """93 frames at hop 256 and 46 at hop 512 for one second (the upstream
    counts); 385 samples are the fewest the reflect pad takes, 384 refused."""
    pcm = np.full(24000, 0.5, np.float32)
    assert _gpu_mel(gpu, pcm, MEL).shape == (93, 128)
    assert _gpu_mel(gpu, pcm, dict(MEL, hop=512)).shape == (46, 128)
    short = (np.random.default_rng(SEED).standard_normal(385) * 0.3).astype(np.float32)
    _close(_gpu_mel(gpu, short, MEL), oracle_log_mel(short, MEL))
    with pytest.raises(gpu.ShpError):
        _gpu_mel(gpu, short[:384], MEL)


def test_log_mel_refusals(gpu):
    import torch
    fb = _t(gpu, gpu.mel_filterbank(24000, 1024, 128, 0.0, 12000.0))
    pcm = torch.zeros(24000, device="cuda")
    with pytest.raises(gpu.ShpError):       # not a power of two
        gpu.log_mel(pcm, _t(gpu, gpu.mel_filterbank(24000, 1000, 128, 0.0, 12000.0)), 1000, 250, 1000)
    with pytest.raises(gpu.ShpError):       # window wider than the transform
        gpu.log_mel(pcm, fb, 1024, 256, 1100)
    with pytest.raises(gpu.ShpError):       # a filterbank of another transform
        gpu.log_mel(pcm, fb, 512, 128, 512)

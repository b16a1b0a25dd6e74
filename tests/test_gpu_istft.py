"""shp_inverse_stft against the restatement of Kokoro's inverse_stft
(kokoro/decoder-host.cpp:28-100): the reference test's torch.istft vector
(G7, tests/kokoro_istft_test.cpp) at its 1e-5, and random spectra at Kokoro's
n_fft 20 / hop 5 and other windows, hops that leave gaps, strided frames and
a 5-second utterance, within 2 f32 ulp of the output's scale (both compute in
double: the device's exp/sin/cos and the twiddles of (b*s) mod n_fft move
only the last bits of the double before the single f32 rounding)."""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t
from test_oracle_goldens import _load

pytestmark = pytest.mark.gpu

SEED = 20261216


def _close(got, ref):
    assert got.shape == ref.shape
    assert np.abs(got - ref).max() <= 2 * np.spacing(np.float32(np.abs(ref).max()))
    assert (got == ref).mean() > 0.99


def test_golden_kokoro_istft_on_the_gpu(gpu):
    d = _load("kokoro_istft.json")
    n, hop, frames = d["n_fft"], d["hop"], d["frames"]
    spec = np.array(d["spectrum"], np.float32).reshape(frames, n + 2)
    exp = np.array(d["expected_audio"], np.float32)
    got = _np(gpu.inverse_stft(_t(gpu, spec), n, hop))
    assert np.abs(got - exp).max() < d["tolerance"]
    _close(got, R.run(lambda g: g.inverse_stft(spec, n, hop)))


@pytest.mark.parametrize("n_fft,hop,frames", [(20, 5, 4001), (20, 5, 2), (16, 4, 333), (8, 3, 200), (6, 8, 50),
                                              (64, 16, 300), (256, 64, 100), (20, 2, 500)])
def test_istft_matches_restatement(gpu, n_fft, hop, frames):
    rng = np.random.default_rng([SEED, n_fft, hop, frames])
    spec = rng.uniform(-3, 2, (frames, n_fft + 2)).astype(np.float32)
    _close(_np(gpu.inverse_stft(_t(gpu, spec), n_fft, hop)), R.run(lambda g: g.inverse_stft(spec, n_fft, hop)))


def test_istft_strided_frames(gpu):
    """Frames at a row stride past n_fft + 2 values (a view of a wider
    tensor)."""
    rng = np.random.default_rng(SEED + 1)
    wide = rng.uniform(-3, 2, (700, 29)).astype(np.float32)
    spec = wide[:, 3:25]
    got = _np(gpu.inverse_stft(_t(gpu, wide)[:, 3:25], 20, 5))
    _close(got, R.run(lambda g: g.inverse_stft(np.ascontiguousarray(spec), 20, 5)))


def test_istft_kokoro_utterance(gpu):
    """A 5-second utterance at 24 kHz: 24001 frames of n_fft 20, hop 5."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(SEED + 2)
    spec = torch.rand((24001, 22), generator=g, device="cuda") * 5 - 3
    _close(_np(gpu.inverse_stft(spec, 20, 5)), R.run(lambda gr: gr.inverse_stft(_np(spec), 20, 5)))


def test_istft_refusals(gpu):
    import torch
    spec = torch.zeros((9, 10), device="cuda")
    with pytest.raises(gpu.ShpError):       # odd window
        gpu.inverse_stft(torch.zeros((9, 9), device="cuda"), 7, 2)
    with pytest.raises(gpu.ShpError):       # no hop
        gpu.inverse_stft(spec, 8, 0)
    with pytest.raises(gpu.ShpError):       # one frame: no samples
        gpu.inverse_stft(torch.zeros((1, 10), device="cuda"), 8, 2, out=torch.empty((1,), device="cuda"))
    with pytest.raises(gpu.ShpError):       # wrong output length
        gpu.inverse_stft(spec, 8, 2, out=torch.empty((15,), device="cuda"))
    with pytest.raises(gpu.ShpError):       # a block's frames past the LDS budget
        gpu.inverse_stft(torch.zeros((40, 1026), device="cuda"), 1024, 1)

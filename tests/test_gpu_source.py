"""shp_harmonic_source against the restatement of Kokoro's
build_harmonic_source (kokoro/source.cpp:60-184), which equals the
reference's own compiled code bit for bit: the upstream module's values (G8,
tests/kokoro_source_test.cpp) at the test's bounds, and random f0 curves at
Kokoro's 9 harmonics, upsampling 300, n_fft 20 and hop 5 up to a 5-second
utterance. The excitation is held within 8 f32 ulp of 1 (the device's f32
sine and tanh against the host library's), the spectrum's bins as complex
values within 2e-5 (the DFT of that excitation)."""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t
from test_oracle_goldens import _load, check_source_golden, random_source_case, source_inputs

pytestmark = pytest.mark.gpu

SEED = 20261217


def _run_gpu(gpu, args, kw):
    f0, mw, bias, ri, noise = args
    exc, har = gpu.harmonic_source(_t(gpu, f0), _t(gpu, mw), bias, _t(gpu, ri), _t(gpu, noise), **kw)
    return _np(exc), _np(har)


def _run_ref(args, kw):
    g = R.Graph()
    exc, har = g.harmonic_source(*args, **kw)
    g.compute()
    return exc, har


def _close(got, ref, bins):
    (e, h), (er, hr) = got, ref
    assert e.shape == er.shape and h.shape == hr.shape
    assert np.abs(e - er).max() <= 8 * np.spacing(np.float32(1))
    z = h[:, :bins].astype(np.float64) * np.exp(1j * h[:, bins:].astype(np.float64))
    zr = hr[:, :bins].astype(np.float64) * np.exp(1j * hr[:, bins:].astype(np.float64))
    assert np.abs(z - zr).max() <= 2e-5
    assert np.abs(h[:, :bins] - hr[:, :bins]).max() <= 2e-5


def test_golden_kokoro_source_on_the_gpu(gpu):
    d = _load("kokoro_source.json")
    args, kw = source_inputs(d)
    got = _run_gpu(gpu, args, kw)
    check_source_golden(*got, d)
    _close(got, _run_ref(args, kw), d["n_fft"] // 2 + 1)


@pytest.mark.parametrize("L,H,scale,n_fft,hop", [(50, 9, 300, 20, 5), (400, 9, 300, 20, 5), (37, 3, 4, 8, 2),
                                                 (20, 5, 16, 16, 4), (3, 1, 7, 64, 3), (2000, 9, 12, 20, 5)])
def test_source_matches_restatement(gpu, L, H, scale, n_fft, hop):
    """Random voiced and unvoiced f0 at Kokoro's dimensions (400 frames: a
    5-second utterance at 24 kHz), other harmonic counts, windows and hops, and
    2000 frames (the running sums over more than one LDS chunk)."""
    args, kw = random_source_case(SEED + L + H, L, H, scale, n_fft, hop)
    _close(_run_gpu(gpu, args, kw), _run_ref(args, kw), n_fft // 2 + 1)


def test_source_refusals(gpu):
    import torch
    d = _load("kokoro_source.json")
    (f0, mw, bias, ri, noise), kw = source_inputs(d)
    tf0, tmw, tri, tnz = _t(gpu, f0), _t(gpu, mw), _t(gpu, ri), _t(gpu, noise)
    with pytest.raises(gpu.ShpError):        # noise of the wrong size
        gpu.harmonic_source(tf0, tmw, bias, tri, tnz[:-1], **kw)
    with pytest.raises(gpu.ShpError):        # an odd window
        gpu.harmonic_source(tf0, tmw, bias, tri, tnz, **dict(kw, n_fft=7))
    with pytest.raises(gpu.ShpError):        # one sample: nothing to reflect
        gpu.harmonic_source(tf0[:1], tmw, bias, tri, tnz[:1, :].contiguous(), **dict(kw, scale=1))
    with pytest.raises(gpu.ShpError):        # more harmonics than the kernel takes
        big = torch.zeros(65, device="cuda")
        gpu.harmonic_source(tf0, big, bias, big, torch.zeros((20, 65), device="cuda"), **kw)

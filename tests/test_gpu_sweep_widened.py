"""Seeded random sweep over the widened rows' entry points, against the
ggml-CPU restatement on the same inputs:
- acc: windows of random extent at random row, plane and element offsets
  (aligned and not), out of place and ggml's inplace form;
- pad_ext, pad_reflect_1d and repeat over 1-4-D shapes, pads on every
  dimension (rows landing on and off 16 bytes), reflections up to the row's
  length minus one, every tiling factor up to 4;
- relu, neg, step, sqrt with signed zeros, infinities and NaN planted;
- sum_rows, mean and the fused mul→sum_rows over row lengths either side of
  the wave's width, values spread over 16 binary orders of magnitude;
- diag_mask_inf at random n_past, and the fused causal softmax against the
  two nodes it replaces;
- the host-seam ports (inverse_stft, harmonic_source, log_mel) at random
  windows, hops, harmonic counts, upsampling factors and bin counts, held to
  their focused tests' bars.
The bars are the focused tests': bit-exact for every copy, add, mask, unary
op and row sum (the restatement accumulates in double and rounds once, as
ggml does); the fused softmax bit-identical to the two GPU nodes and within
2 ulp of the restatement (the share of identical elements is row-granular, so
the sweep holds the bar only). SWEEP_SEED fixes the case list, so a failure names
a shape that reruns the same way.
"""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t, _ulps_apart
from test_gpu_sweep import _gen, _pick

pytestmark = pytest.mark.gpu

SWEEP_SEED = 616161
MAX_ELEMS = 1 << 22


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _eq(got, ref):
    got = _np(got)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.array_equal(_bits(got), _bits(ref))


# ---------------------------------------------------------------------------
# acc
# ---------------------------------------------------------------------------

def _acc_case(rng):
    """a of ggml shape [n0, n1, n2] (numpy reversed), b a window of it that
    starts at (e0, e1, e2) with a's own strides, so the view never overlaps
    itself and stays inside a."""
    n0 = _pick(rng, [1, 3, 4, 7, 64, 100, 1001, 2048])
    n1 = _pick(rng, [1, 2, 5, 33, 300])
    n2 = _pick(rng, [1, 1, 3])
    if n0 * n1 * n2 > MAX_ELEMS:
        return None
    b0, b1, b2 = int(rng.integers(1, n0 + 1)), int(rng.integers(1, n1 + 1)), int(rng.integers(1, n2 + 1))
    e0, e1, e2 = int(rng.integers(0, n0 - b0 + 1)), int(rng.integers(0, n1 - b1 + 1)), int(rng.integers(0, n2 - b2 + 1))
    return ((n2, n1, n0), (b2, b1, b0), (e2, e1, e0))


@pytest.mark.parametrize("ashape,bshape,start", _gen("acc", _acc_case))
def test_sweep_acc(gpu, ashape, bshape, start):
    rng = np.random.default_rng([SWEEP_SEED, *ashape, *bshape, *start])
    a = rng.standard_normal(ashape).astype(np.float32)
    b = rng.standard_normal(bshape).astype(np.float32)
    n2, n1, n0 = ashape
    nb = (4 * n0, 4 * n0 * n1, 4 * n0 * n1 * n2)
    offset = 4 * (start[2] + start[1] * n0 + start[0] * n0 * n1)
    ref = R.run(lambda g: g.acc(a, b, *nb, offset))
    _eq(gpu.acc(_t(gpu, a), _t(gpu, b), *nb, offset), ref)
    ta = _t(gpu, a)
    gpu.acc(ta, _t(gpu, b), *nb, offset, inplace=True)
    _eq(ta, ref)


# ---------------------------------------------------------------------------
# the pad family
# ---------------------------------------------------------------------------

def _pad_case(rng):
    nd = int(rng.integers(1, 5))
    shape = [_pick(rng, [1, 2, 3, 5, 8, 64, 129, 1024, 4096]) for _ in range(nd)]
    lp = [int(rng.integers(0, 9)) for _ in range(nd)]
    rp = [int(rng.integers(0, 9)) for _ in range(nd)]
    out = 1
    for s, l, r in zip(shape, lp, rp):
        out *= s + l + r
    if out > MAX_ELEMS or int(np.prod(shape)) > MAX_ELEMS:
        return None
    return (tuple(shape), tuple(lp[::-1]), tuple(rp[::-1]))


@pytest.mark.parametrize("shape,lp,rp", _gen("pad_ext", _pad_case))
def test_sweep_pad_ext(gpu, shape, lp, rp):
    x = np.random.default_rng([SWEEP_SEED, *shape, *lp, *rp]).standard_normal(shape).astype(np.float32)
    _eq(gpu.pad_ext(_t(gpu, x), list(lp), list(rp)), R.run(lambda g: g.pad_ext(x, list(lp), list(rp)), n_threads=8))


def _reflect_case(rng):
    n0 = _pick(rng, [2, 3, 5, 16, 100, 1000, 8193])
    rows = _pick(rng, [1, 3, 64, 257])
    if n0 * rows > MAX_ELEMS:
        return None
    return ((rows, n0), int(rng.integers(0, n0)), int(rng.integers(0, n0)))


@pytest.mark.parametrize("shape,p0,p1", _gen("pad_reflect_1d", _reflect_case))
def test_sweep_pad_reflect_1d(gpu, shape, p0, p1):
    x = np.random.default_rng([SWEEP_SEED, *shape, p0, p1]).standard_normal(shape).astype(np.float32)
    _eq(gpu.pad_reflect_1d(_t(gpu, x), p0, p1), R.run(lambda g: g.pad_reflect_1d(x, p0, p1), n_threads=8))


def _repeat_case(rng):
    nd = int(rng.integers(1, 5))
    shape = [_pick(rng, [1, 2, 3, 7, 64, 128, 1000]) for _ in range(nd)]
    target = [s * int(rng.integers(1, 5)) for s in shape]
    if int(np.prod(target)) > MAX_ELEMS:
        return None
    return (tuple(shape), tuple(target))


@pytest.mark.parametrize("shape,target", _gen("repeat", _repeat_case))
def test_sweep_repeat(gpu, shape, target):
    x = np.random.default_rng([SWEEP_SEED, *shape, *target]).standard_normal(shape).astype(np.float32)
    _eq(gpu.repeat(_t(gpu, x), target), R.run(lambda g: g.repeat(x, target), n_threads=8))


# ---------------------------------------------------------------------------
# unary ops and row sums
# ---------------------------------------------------------------------------

SPECIALS = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.4e38, -3.4e38], np.float32)


def _rows_case(rng):
    ne0 = _pick(rng, [1, 2, 3, 4, 5, 31, 63, 64, 65, 127, 128, 400, 1024, 4099])
    rows = _pick(rng, [1, 2, 7, 64, 65, 1000, 1536])
    if ne0 * rows > MAX_ELEMS:
        return None
    return (rows, ne0)


@pytest.mark.parametrize("rows,ne0", _gen("unary", _rows_case))
def test_sweep_unary(gpu, rows, ne0):
    rng = np.random.default_rng([SWEEP_SEED, 1, rows, ne0])
    x = (rng.standard_normal((rows, ne0)) * 10).astype(np.float32)
    k = min(x.size, SPECIALS.size)
    x.reshape(-1)[:k] = SPECIALS[:k]
    tx = _t(gpu, x)
    for op in ("relu", "neg", "step", "sqrt"):
        _eq(getattr(gpu, op)(tx), R.run(lambda g: getattr(g, op)(x)))


@pytest.mark.parametrize("rows,ne0", _gen("row_sums", _rows_case))
def test_sweep_row_sums(gpu, rows, ne0):
    rng = np.random.default_rng([SWEEP_SEED, 2, rows, ne0])
    x = (rng.standard_normal((rows, ne0)) * np.exp(rng.uniform(-8, 8, (rows, ne0)))).astype(np.float32)
    w = rng.random((rows, ne0)).astype(np.float32)
    g = R.Graph()
    s, m, ws = g.sum_rows(x), g.mean(x), g.sum_rows(g.mul(x, w))
    g.compute()
    tx, tw = _t(gpu, x), _t(gpu, w)
    _eq(gpu.sum_rows(tx), s)
    _eq(gpu.mean(tx), m)
    _eq(gpu.mul_sum_rows(tx, tw), ws)


# ---------------------------------------------------------------------------
# causal masking
# ---------------------------------------------------------------------------

def _causal_case(rng):
    H = _pick(rng, [1, 2, 8, 16])
    T = _pick(rng, [1, 2, 7, 64, 65, 300])
    n_past = _pick(rng, [0, 0, 1, 5, 37, 200])
    N = T + n_past + _pick(rng, [0, 0, 1, 3, 64])
    if H * T * N > MAX_ELEMS:
        return None
    return (H, T, N, n_past)


@pytest.mark.parametrize("H,T,N,n_past", _gen("causal", _causal_case))
def test_sweep_diag_mask_and_causal_softmax(gpu, H, T, N, n_past):
    rng = np.random.default_rng([SWEEP_SEED, 3, H, T, N, n_past])
    x = (rng.standard_normal((H, T, N)) * 4).astype(np.float32)
    tx = _t(gpu, x)
    masked = gpu.diag_mask_inf(tx, n_past)
    _eq(masked, R.run(lambda g: g.diag_mask_inf(x, n_past)))
    scale = float(1.0 / np.sqrt(128.0))
    fused = _np(gpu.soft_max_causal(tx, n_past, scale))
    two = _np(gpu.soft_max_ext(masked, None, scale))
    assert np.array_equal(_bits(fused), _bits(two))
    g = R.Graph()
    ref = g.soft_max_ext(g.diag_mask_inf(x, n_past), None, scale)
    g.compute()
    # the bar only, as for soft_max_ext's sweep: a row's sum that rounds to
    # the neighbouring float moves the whole row by one ulp, so the share of
    # identical elements over a few rows says little
    assert _ulps_apart(fused, ref).max() <= 2


# ---------------------------------------------------------------------------
# the host seams: inverse STFT, harmonic source, log-mel
# ---------------------------------------------------------------------------

def _istft_case(rng):
    n_fft = 2 * int(rng.integers(1, 33))
    hop = int(rng.integers(1, n_fft + 5))
    frames = _pick(rng, [2, 3, 17, 64, 65, 500, 3001])
    nf = (63 + n_fft - 1) // hop + 2  # the kernel's smallest tile's frames must fit its LDS budget
    if (nf * (n_fft // 2 + 1) + n_fft) * 16 > 48 * 1024:
        return None
    return (n_fft, hop, frames)


@pytest.mark.parametrize("n_fft,hop,frames", _gen("istft", _istft_case))
def test_sweep_inverse_stft(gpu, n_fft, hop, frames):
    from test_gpu_istft import _close as istft_close
    rng = np.random.default_rng([SWEEP_SEED, 4, n_fft, hop, frames])
    spec = rng.uniform(-3, 2, (frames, n_fft + 2)).astype(np.float32)
    istft_close(_np(gpu.inverse_stft(_t(gpu, spec), n_fft, hop)), R.run(lambda g: g.inverse_stft(spec, n_fft, hop)))


def _source_case(rng):
    L = _pick(rng, [1, 2, 5, 37, 200])
    H = _pick(rng, [1, 2, 9, 16, 64])
    scale = _pick(rng, [2, 3, 8, 60, 300])
    n_fft = 2 * int(rng.integers(1, 33))
    hop = int(rng.integers(1, n_fft + 1))
    n = L * scale
    if n < 2 or (n_fft + 2) * (n // hop) < L * H or n * H > MAX_ELEMS:
        return None
    return (L, H, scale, n_fft, hop)


@pytest.mark.parametrize("L,H,scale,n_fft,hop", _gen("source", _source_case, n=16))
def test_sweep_harmonic_source(gpu, L, H, scale, n_fft, hop):
    from test_gpu_source import _close as source_close, _run_gpu, _run_ref
    from test_oracle_goldens import random_source_case
    args, kw = random_source_case(SWEEP_SEED + L * 7 + H * 13 + scale + n_fft + hop, L, H, scale, n_fft, hop)
    source_close(_run_gpu(gpu, args, kw), _run_ref(args, kw), n_fft // 2 + 1)


def _mel_case(rng):
    n_fft = _pick(rng, [64, 128, 256, 512, 1024, 2048])
    hop = int(rng.integers(1, n_fft + 1)) if rng.random() < 0.3 else n_fft // _pick(rng, [1, 2, 4, 8])
    win = int(rng.integers(n_fft // 2, n_fft + 1))
    bins = _pick(rng, [1, 8, 40, 80, 128, 256])
    ns = _pick(rng, [n_fft, 3000, 24000])
    pad = (n_fft - hop) // 2
    if ns <= pad or ns + 2 * pad < n_fft or (ns + 2 * pad - n_fft) // hop + 1 > 3000:
        return None
    return (n_fft, hop, win, bins, ns)


@pytest.mark.parametrize("n_fft,hop,win,bins,ns", _gen("log_mel", _mel_case, n=16))
def test_sweep_log_mel(gpu, n_fft, hop, win, bins, ns):
    """Random windows, hops, window lengths (zero-padded Hann) and bin
    counts; within 1e-5 of the restatement, > 95 % identical (short clips and
    few bins leave few values to share)."""
    from test_oracle_goldens import MEL, oracle_log_mel
    p = dict(MEL, n_fft=n_fft, hop=hop, win_length=win, mel_bins=bins)
    pcm = (np.random.default_rng([SWEEP_SEED, 5, n_fft, hop, win, bins, ns]).standard_normal(ns) * 0.2).astype(np.float32)
    fb = gpu.mel_filterbank(p["sample_rate"], n_fft, bins, p["fmin"], p["fmax"])
    got = _np(gpu.log_mel(_t(gpu, pcm), _t(gpu, fb), n_fft, hop, win))
    ref = oracle_log_mel(pcm, p)
    assert got.shape == ref.shape
    assert np.abs(got - ref).max() <= 1e-5
    assert (got == ref).mean() > 0.95

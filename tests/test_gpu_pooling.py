"""shp_relu, shp_neg, shp_step, shp_sqrt, shp_sum_rows, shp_mean and
shp_mul_sum_rows against the restatement, bit for bit; the speaker encoder's
attentive statistics pooling (qwen3-tts/speaker-encoder.cpp:284-295,340-376)
as the node list its builder emits, through the executor."""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t

pytestmark = pytest.mark.gpu

SEED = 20261214

SPECIALS = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.4e38, -3.4e38, 1.0, -1.0], np.float32)


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("shape", [(64, 65), (8, 4096), (3, 5, 7)])
@pytest.mark.parametrize("op", ["relu", "neg", "step", "sqrt"])
def test_unary_matches_restatement(gpu, op, shape):
    x = (np.random.default_rng([SEED, *shape]).standard_normal(shape) * 10).astype(np.float32)
    x.reshape(-1)[:SPECIALS.size] = SPECIALS
    ref = R.run(lambda g: getattr(g, op)(x))
    got = _np(getattr(gpu, op)(_t(gpu, x)))
    assert np.array_equal(_bits(got), _bits(ref))


def test_unary_strided_rows(gpu):
    import torch
    x = np.random.default_rng(SEED).standard_normal((40, 100)).astype(np.float32)
    tx = _t(gpu, x)[:, 3:90]
    out = torch.empty((40, 87), device="cuda")
    gpu.relu(tx, out=out)
    assert np.array_equal(_bits(_np(out)), _bits(R.run(lambda g: g.relu(x[:, 3:90]))))


def _wide(rng, shape):
    return (rng.standard_normal(shape) * np.exp(rng.uniform(-8, 8, shape))).astype(np.float32)


@pytest.mark.parametrize("shape", [(1536, 400), (7, 33), (2, 3, 129), (64, 4096), (5, 1)])
def test_row_sums_match_restatement(gpu, shape):
    rng = np.random.default_rng([SEED, *shape])
    x, w = _wide(rng, shape), rng.random(shape).astype(np.float32)
    g = R.Graph()
    s, m, ws = g.sum_rows(x), g.mean(x), g.sum_rows(g.mul(x, w))
    g.compute()
    tx, tw = _t(gpu, x), _t(gpu, w)
    assert np.array_equal(_bits(_np(gpu.sum_rows(tx))), _bits(s))
    assert np.array_equal(_bits(_np(gpu.mean(tx))), _bits(m))
    assert np.array_equal(_bits(_np(gpu.mul_sum_rows(tx, tw))), _bits(ws))


def test_row_sums_unaligned_and_strided(gpu):
    """Rows starting off 16 bytes (the scalar path) and rows of a column slice."""
    import torch
    rng = np.random.default_rng(SEED + 1)
    x = _wide(rng, (30, 202))
    ref = R.run(lambda g: g.sum_rows(x[:, 1:201]))
    got = _np(gpu.sum_rows(_t(gpu, x)[:, 1:201]))
    assert np.array_equal(_bits(got), _bits(ref))
    buf = torch.zeros(31, device="cuda")
    out = buf[1:].view(30, 1)
    gpu.mean(_t(gpu, x), out=out)
    assert np.array_equal(_bits(_np(out)), _bits(R.run(lambda g: g.mean(x))))


def test_row_sum_refusals(gpu):
    import torch
    x = torch.zeros((4, 8), device="cuda")
    with pytest.raises(gpu.ShpError):       # y of the wrong shape
        gpu.sum_rows(x, out=torch.empty((4, 2), device="cuda"))
    with pytest.raises(gpu.ShpError):       # w of another shape
        gpu.mul_sum_rows(x, torch.zeros((4, 7), device="cuda"))
    with pytest.raises(gpu.ShpError):       # y over x
        gpu.sum_rows(x, out=x[:, :1])


VARIANCE_FLOOR = 1e-12   # kVarianceFloor, speaker-encoder.cpp:96


def _oracle_pooling(features, logits):
    """The pooling's statistics on the restatement: features and logits are
    numpy (T, C) = ggml [C, T]."""
    g = R.Graph()
    tm = np.ascontiguousarray(features.T)                     # cont(transpose): ggml [T, C]
    mean = g.mean(tm)

    def deviation(m, w):
        d = g.sqr(g.sub(tm, m))
        var = g.mean(d) if w is None else g.sum_rows(g.mul(d, w))
        return g.sqrt(g.clamp(var, VARIANCE_FLOOR, np.inf))
    dev = deviation(mean, None)
    att = g.soft_max_ext(np.ascontiguousarray(logits.T), None, 1.0)
    wmean = g.sum_rows(g.mul(tm, att))
    wscale = deviation(wmean, att)
    g.compute()
    return mean, dev, wmean, wscale


def test_attentive_statistics_pooling_through_the_executor(gpu):
    """speaker-encoder.cpp:340-376 with weighted_deviation (:284-295): the
    transposing copy, the mean and deviation over time, the softmax over
    time of the attention logits, then the attention-weighted mean and
    deviation -- each mul -> sum_rows one launch. The unweighted statistics
    are bit-exact; the weighted ones take the softmax's last-ulp
    differences (within 1e-5 relative)."""
    T, C = 600, 192
    rng = np.random.default_rng(SEED + 2)
    features = rng.standard_normal((T, C)).astype(np.float32)
    logits = (rng.standard_normal((T, C)) * 3).astype(np.float32)
    ref = _oracle_pooling(features, logits)
    g = gpu.Graph()
    tf, tl = _t(gpu, features), _t(gpu, logits)
    tm = g.cont(g.view(tf, tf.t()))
    mean = g.mean(tm)

    def deviation(m, w):
        d = g.sqr(g.sub(tm, m))
        var = g.mean(d) if w is None else g.sum_rows(g.mul(d, w))
        return g.sqrt(g.clamp(var, VARIANCE_FLOOR, float("inf")))
    dev = deviation(mean, None)
    att = g.soft_max_ext(g.cont(g.view(tl, tl.t())), None, 1.0)
    wmean = g.sum_rows(g.mul(tm, att))
    wscale = deviation(wmean, att)
    kinds = [k for k, *_ in g.plan(mean, dev, wmean, wscale) if k != "nop"]
    assert kinds.count("mul_sum_rows") == 2, kinds
    g.compute(mean, dev, wmean, wscale)
    assert np.array_equal(_bits(_np(mean.t)), _bits(ref[0]))
    assert np.array_equal(_bits(_np(dev.t)), _bits(ref[1]))
    for got, exp in ((wmean, ref[2]), (wscale, ref[3])):
        got = _np(got.t)
        assert np.abs(got - exp).max() <= 1e-5 * np.abs(exp).max()

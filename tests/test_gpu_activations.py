"""The codec / vocoder / encoder ops between GEMMs: ggml_sub, tanh, sigmoid,
elu, gelu_erf, clamp and norm, against the oracle's restatement of ggml-CPU's
vec forms. sub and clamp are bit-exact; the others use the device's
tanhf / expf / expm1f / erff, so they are held to 1e-5 relative (gelu_erf: plus
|x| * 2^-22 absolute, for ggml's 1 + erff(.) cancels for x < 0, where one ulp
of erff between libraries is a large relative change of a tiny result)."""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t, assert_bitexact

pytestmark = pytest.mark.gpu
SEED = 20261205


def _inputs(rng, shape):
    x = (rng.standard_normal(shape) * 3).astype(np.float32)
    flat = x.reshape(-1)
    sp = np.float32([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 88.0, -104.0, 1e30, -1e30, 20.0, -20.0])
    n = min(sp.size, flat.size)
    flat[:n] = sp[:n]
    return x


def _close(got, ref, x=None, rel=1e-5):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = np.isfinite(ref)
    assert np.array_equal(got[~fin & ~np.isnan(ref)], ref[~fin & ~np.isnan(ref)])
    tol = rel * np.abs(ref[fin]) + 1e-30
    if x is not None:
        tol = tol + np.abs(np.asarray(x, np.float64)[fin]) * 2.0 ** -22
    bad = np.abs(got[fin] - ref[fin]) > tol
    assert not bad.any(), (bad.sum(), got[fin][bad][:4], ref[fin][bad][:4])


@pytest.mark.parametrize("shape", [(64, 1000), (3, 37), (128, 4096)])
@pytest.mark.parametrize("op", ["tanh", "sigmoid", "elu", "gelu_erf"])
def test_activation_matches_oracle(gpu, shape, op):
    rng = np.random.default_rng(SEED + sum(shape) + len(op))
    x = _inputs(rng, shape)
    y = getattr(gpu, op)(_t(gpu, x))
    ref = R.run(lambda g: getattr(g, op)(x))
    _close(_np(y), ref, x if op == "gelu_erf" else None)


@pytest.mark.parametrize("shape", [(64, 1000), (3, 37)])
def test_clamp_and_sub_bit_exact(gpu, shape):
    rng = np.random.default_rng(SEED + sum(shape))
    x = _inputs(rng, shape)
    assert_bitexact(_np(gpu.clamp(_t(gpu, x), -1.0, 1.0)), R.run(lambda g: g.clamp(x, -1.0, 1.0)))
    b = rng.standard_normal(shape).astype(np.float32)
    row = rng.standard_normal(shape[-1]).astype(np.float32)
    col = rng.standard_normal((shape[0], 1)).astype(np.float32)
    assert_bitexact(_np(gpu.sub(_t(gpu, x), _t(gpu, b))), x - b)
    assert_bitexact(_np(gpu.sub(_t(gpu, x), _t(gpu, row))), x - row)
    assert_bitexact(_np(gpu.sub(_t(gpu, x), _t(gpu, col))), R.run(lambda g: g.binbcast(R.OP_SUB, x, col)))


@pytest.mark.parametrize("rows,ne0", [(64, 1024), (7, 37), (300, 512), (2, 4096)])
def test_norm_matches_oracle(gpu, rows, ne0):
    rng = np.random.default_rng(SEED + rows + ne0)
    x = (rng.standard_normal((rows, ne0)) * 2 + 3).astype(np.float32)
    x[0] = 5.0                               # a constant row: exactly 0
    y = gpu.norm(_t(gpu, x), 1e-6)
    ref = R.run(lambda g: g.norm(x, 1e-6))
    got = _np(y)
    assert (got[0] == 0).all()
    assert np.abs(got - ref).max() <= 1e-5


def test_convnext_tail_in_a_node_list(gpu):
    """codec_convnext_block's norm, affine and GELU (qwen3-tts/codec.cpp:
    216-222) as a node list: every node alone, against the restatement."""
    rng = np.random.default_rng(SEED + 21)
    x = rng.standard_normal((256, 1024)).astype(np.float32)
    w = rng.normal(1, 0.1, 1024).astype(np.float32)
    b = rng.normal(0, 0.1, 1024).astype(np.float32)
    g = gpu.Graph()
    y = g.gelu_erf(g.add(g.mul(g.norm(_t(gpu, x), 1e-6), _t(gpu, w)), _t(gpu, b)))
    assert [k for k, *_ in g.plan(y) if k != "nop"] == ["single"] * 4
    g.compute(y)
    ref = R.run(lambda og: og.gelu_erf(og.add(og.mul(og.norm(x, 1e-6), w), b)))
    assert np.abs(_np(y.t) - ref).max() <= 1e-4

"""ggml_add / ggml_mul / ggml_div with b repeated to a's shape (ggml_can_repeat)
through shp_add / shp_mul / shp_div: the time-major vocoder's per-channel
[1, C] bias (vits/waveform-decoder.cpp:120,139; qwen3-tts/codec.cpp:180;
omnivoice/codec.cpp:163) and gains (omnivoice/reference-encoder.cpp:135-136),
and every other repeat form. Bit-exact against the oracle's restatement of
ggml-CPU's repeat (op_binbcast)."""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t, assert_bitexact

pytestmark = pytest.mark.gpu
SEED = 20261203
OPS = (("add", R.OP_ADD), ("mul", R.OP_MUL), ("div", R.OP_DIV))


def _oracle(op, a, b):
    g = R.Graph()
    y = g.binbcast(op, a, b)
    g.compute(8)
    return y


# (torch shape of a, torch shape of b): torch (ne3, ne2, ne1, ne0)
CASES = [
    ((128, 4096), (128, 1)),        # time-major [T, C] + [1, C] bias: one value per row, flat kernel
    ((96, 1000), (96, 1)),          # the same, 1000 % 4 == 0
    ((37, 1001), (37, 1)),          # ne0 odd: the row kernel
    ((4, 8, 64), (1, 8, 1)),        # b's rows repeat over dim 2: flat kernel, decomposed rows
    ((4, 8, 64), (4, 1, 1)),
    ((3, 6, 40), (3, 2, 20)),       # every dim repeated by a divisor: row kernel
    ((2, 3, 5, 8), (1, 3, 1, 8)),
    ((2, 3, 5, 8), (1, 1, 1, 1)),   # one scalar
    ((16, 256), (2, 1)),
]


@pytest.mark.parametrize("ashape,bshape", CASES)
@pytest.mark.parametrize("name,op", OPS)
def test_repeat_matches_oracle(gpu, ashape, bshape, name, op):
    rng = np.random.default_rng(SEED + sum(ashape) + 3 * sum(bshape))
    a = rng.standard_normal(ashape).astype(np.float32)
    b = (rng.standard_normal(bshape) + 2.5).astype(np.float32)
    print("case", name, ashape, bshape, flush=True)
    y = getattr(gpu, name)(_t(gpu, a), _t(gpu, b))
    assert_bitexact(_np(y), _oracle(op, a, b))


def test_repeat_row_strided_and_in_place(gpu):
    """a as a row-strided view (the row kernel), and the flat kernel writing
    over its own input (ggml's in-place adds): each element is read and
    written by one lane."""
    import torch
    rng = np.random.default_rng(SEED + 5)
    big = rng.standard_normal((64, 300)).astype(np.float32)
    bias = rng.standard_normal((64, 1)).astype(np.float32)
    ta = _t(gpu, big)
    view = ta[:, 10:266]
    y = gpu.add(view, _t(gpu, bias))
    assert_bitexact(_np(y), _oracle(R.OP_ADD, big[:, 10:266], bias))
    x = rng.standard_normal((32, 2048)).astype(np.float32)
    tx = _t(gpu, x)
    gpu.mul(tx, _t(gpu, bias[:32]), out=tx)
    assert_bitexact(_np(tx), _oracle(R.OP_MUL, x, bias[:32]))
    assert torch.isfinite(tx).all()


def test_repeat_large_time_major_bias(gpu):
    """The vocoder shape: ggml [131072, 128] + [1, 128]."""
    rng = np.random.default_rng(SEED + 9)
    a = rng.standard_normal((128, 131072)).astype(np.float32)
    b = rng.standard_normal((128, 1)).astype(np.float32)
    y = gpu.add(_t(gpu, a), _t(gpu, b))
    assert_bitexact(_np(y), _oracle(R.OP_ADD, a, b))


def test_repeat_in_a_node_list(gpu):
    """conv1d_time_major's tail (vits/waveform-decoder.cpp:111,118-121): the
    transposing copy of the convolution's output, then the [1, C] bias add,
    then the next leaky-ReLU, as one launch (the biased value written, being
    an output too), equal to the restatement; and with the copy read
    elsewhere, every node alone."""
    rng = np.random.default_rng(SEED + 11)
    out = rng.standard_normal((2048, 96)).astype(np.float32)   # ggml [C_out=96, T=2048] (GEMM output)
    bias = rng.standard_normal((96, 1)).astype(np.float32)      # ggml [1, 96]
    g = gpu.Graph()
    to = _t(gpu, out)
    tm = g.cont(g.view(to, to.t()))                              # ggml [2048, 96]
    biased = g.add(tm, _t(gpu, bias))
    act = g.leaky_relu(biased, 0.1)
    kinds = [k for k, *_ in g.plan(biased, act) if k != "nop"]
    assert kinds == ["cont_add_leaky"], kinds
    g.compute(biased, act)
    ref = _oracle(R.OP_ADD, np.ascontiguousarray(out.T), bias)
    assert_bitexact(_np(biased.t), ref)
    lk = R.Graph()
    ref_act = lk.leaky_relu(ref, 0.1)
    lk.compute(1)
    assert_bitexact(_np(act.t), ref_act)
    g = gpu.Graph()
    tm = g.cont(g.view(to, to.t()))
    biased = g.add(tm, _t(gpu, bias))
    kinds = [k for k, *_ in g.plan(biased, tm) if k != "nop"]
    assert kinds == ["single", "single"], kinds
    g.compute(biased, tm)
    assert_bitexact(_np(biased.t), ref)
    assert_bitexact(_np(tm.t), np.ascontiguousarray(out.T))

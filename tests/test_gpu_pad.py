"""shp_pad, shp_pad_reflect_1d and shp_repeat against the restatement, bit for
bit (pure copies): zero padding on every dimension, reflection, tiling; the
Kokoro decoder's zero-stuffed spread, edge widening and frame doubling at the
vocoder sizes, alone and as the node list its transposed convolution builds
(kokoro/operations.cpp:189-196)."""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t

pytestmark = pytest.mark.gpu

SEED = 20261211


def _eq(got, ref):
    got = _np(got)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("shape,lp,rp", [
    ((7,), [2], [3]), ((4, 9), [0, 1], [5, 2]), ((3, 1, 5), [1, 0, 0], [0, 7, 2]), ((2, 3, 4, 5), [1, 2, 0, 1], [2, 0, 3, 0]),
    ((1000, 256), [3, 0], [5, 0]),            # a codec encoder's edge padding on time (ggml dim 0 here)
    ((4096, 1, 256), [0, 0], [0, 7]),         # the Kokoro spread: [C, 1, L] padded to [C, 8, L]
    ((8191, 129), [0, 6], [0, 1]),            # edge widening along time of a [C, T] activation
])
def test_pad_ext_matches(gpu, shape, lp, rp):
    x = np.random.default_rng([SEED, *shape]).standard_normal(shape).astype(np.float32)
    _eq(gpu.pad_ext(_t(gpu, x), lp, rp), R.run(lambda g: g.pad_ext(x, lp, rp), n_threads=8))


@pytest.mark.parametrize("shape,p0,p1", [((3, 10), 2, 3), ((16,), 1, 1), ((2, 3, 8), 7, 0), ((4, 5), 0, 4),
                                         ((512, 2000), 3, 3)])
def test_pad_reflect_1d_matches(gpu, shape, p0, p1):
    x = np.random.default_rng([SEED, *shape, p0, p1]).standard_normal(shape).astype(np.float32)
    _eq(gpu.pad_reflect_1d(_t(gpu, x), p0, p1), R.run(lambda g: g.pad_reflect_1d(x, p0, p1), n_threads=8))


@pytest.mark.parametrize("shape,target", [((1, 7), (5, 7)), ((3, 1, 4), (3, 2, 4)), ((2, 3), (4, 9)), ((5,), (2, 3, 10)),
                                          ((1, 1, 1, 2), (2, 3, 2, 6)),
                                          ((1, 512), (8192, 512)),           # broadcast_over_time (kokoro :21-24)
                                          ((16384, 1, 256), (16384, 2, 256))])  # upsample_nearest_2x (:113-120)
def test_repeat_matches(gpu, shape, target):
    x = np.random.default_rng([SEED, *target]).standard_normal(shape).astype(np.float32)
    _eq(gpu.repeat(_t(gpu, x), target), R.run(lambda g: g.repeat(x, target), n_threads=8))


@pytest.mark.parametrize("shift,pad_rows", [(1, 0), (0, 3)])
def test_pad_into_strided_and_unaligned_destination(gpu, shift, pad_rows):
    import torch
    x = np.random.default_rng(SEED + shift).standard_normal((50, 37)).astype(np.float32)
    buf = torch.zeros(60 * (45 + pad_rows) + shift, device="cuda")
    out = buf[shift:].view(60, 45 + pad_rows)[:, :45]
    gpu.pad_ext(_t(gpu, x), [3, 4], [5, 6], out=out)
    _eq(out, R.run(lambda g: g.pad_ext(x, [3, 4], [5, 6])))
    assert (_np(buf[shift:].view(60, 45 + pad_rows)[:, 45:]) == 0).all()


def test_pad_family_refusals(gpu):
    import torch
    x = torch.zeros((4, 5), device="cuda")
    with pytest.raises(gpu.ShpError):  # reflection by the row's length
        gpu.pad_reflect_1d(x, 5, 0)
    with pytest.raises(gpu.ShpError):  # not a multiple
        gpu.repeat(x, (6, 5))
    with pytest.raises(gpu.ShpError):  # y smaller than x plus the left pad
        gpu.pad_ext(x, [2, 0], [0, 0], out=torch.empty((4, 6), device="cuda"))
    with pytest.raises(gpu.ShpError):  # y over x
        buf = torch.zeros(64, device="cuda")
        gpu.repeat(buf[:20].view(4, 5), (8, 5), out=buf[10:50].view(8, 5))


def test_kokoro_spread_node_list(gpu):
    """The front of kokoro's transpose_conv1d (:189-196) as the node list it
    builds: the reshape to [C, 1, L], ggml_pad of the unit axis by stride - 1,
    ggml_cont, the reshape to [C, stride*L], ggml_pad_ext by (left, right) on
    time; through the executor, against the restatement's nodes."""
    C, L, S, K, P = 128, 2048, 4, 8, 2
    left, right = K - 1 - P, K - S - P
    rng = np.random.default_rng(SEED + 5)
    x = rng.standard_normal((L, C)).astype(np.float32)            # ggml [C, L]
    tx = _t(gpu, x)
    g = gpu.Graph()
    spread = g.pad(g.view(tx, tx.view(L, 1, C)), [0, S - 1, 0, 0])
    flat = g.cont(spread)
    padded = g.pad_ext(g.view(flat, flat.t.view(L * S, C)), [0, left], [0, right])
    kinds = [k for k, *_ in g.plan(padded) if k != "nop"]
    assert kinds == ["single"] * 3, kinds
    g.compute(padded)
    gr = R.Graph()
    sp = gr.pad(x.reshape(L, 1, C), [0, S - 1, 0, 0])
    pd = gr.pad_ext(sp.reshape(L * S, C), [0, left], [0, right])
    gr.compute(8)
    _eq(padded.t, pd)

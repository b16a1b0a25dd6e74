"""shp_col2im_1d against the restatement's ggml_col2im_1d, bit for bit: the
vocoders' and codecs' upsampling shapes (K = 2*stride: two terms per output,
order-free) and other kernels (three terms per output with K = 3 at stride 1,
zero gaps with K < stride), both load forms, strided and unaligned outputs; the
reference's transposed-convolution known answers and the codec's transposed
convolution golden with the scatter on the GPU."""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t

pytestmark = pytest.mark.gpu

SEED = 20261209

# (K, OC, L, stride, padding)
CASES = [
    (16, 256, 1024, 8, 4),   # vits ups stage (kernel 16, stride 8, padding 4)
    (20, 64, 300, 10, 5),    # kokoro-like (kernel 20, stride 10)
    (4, 96, 1001, 2, 1),     # kernel 4, stride 2
    (4, 6, 7, 2, 0),         # the codec ops test's transposed shape (K = 2*stride, no padding)
    (3, 2, 6, 1, 0),         # K = 3 at stride 1: three terms per output
    (2, 7, 33, 5, 0),        # K < stride: zero gaps
    (12, 37, 129, 6, 3),     # K*OC 444, 37 channels over tiles
    (5, 3, 50, 2, 1),        # K*OC 15: one-value loads
    (8, 1, 1, 4, 0),         # one column
    (16, 3, 5, 8, 4),        # the reference test's multichannel case
]


def _ref(cols, s, oc, p):
    return R.run(lambda g: g.col2im_1d(cols, s, oc, p), n_threads=8)


@pytest.mark.parametrize("K,OC,L,S,P", CASES)
def test_col2im_matches_restatement(gpu, K, OC, L, S, P):
    rng = np.random.default_rng([SEED, K, OC, L, S, P])
    cols = rng.standard_normal((L, K * OC)).astype(np.float32)
    got = _np(gpu.col2im_1d(_t(gpu, cols), S, OC, P))
    ref = _ref(cols, S, OC, P)
    assert got.shape == ref.shape
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("shift,row_pad", [(1, 0), (0, 3), (2, 5)])
def test_col2im_strided_and_unaligned_output(gpu, shift, row_pad):
    """y rows at a stride other than T, starting off 16 bytes."""
    import torch
    K, OC, L, S, P = 16, 24, 200, 8, 4
    rng = np.random.default_rng(SEED + shift + 10 * row_pad)
    cols = rng.standard_normal((L, K * OC)).astype(np.float32)
    T = (L - 1) * S + K - 2 * P
    buf = torch.zeros(OC * (T + row_pad) + shift, device="cuda")
    out = buf[shift:].view(OC, T + row_pad)[:, :T]
    gpu.col2im_1d(_t(gpu, cols), S, OC, P, out=out)
    assert np.array_equal(_np(out), _ref(cols, S, OC, P))
    assert (_np(buf[shift:].view(OC, T + row_pad)[:, T:]) == 0).all()  # the gaps stay untouched


def test_col2im_refusals(gpu):
    import torch
    cols = torch.zeros((1, 12), device="cuda")
    with pytest.raises(gpu.ShpError):  # the crop takes the whole signal
        gpu.col2im_1d(cols, 2, 3, 2, out=torch.empty((3, 1), device="cuda"))
    with pytest.raises(gpu.ShpError):  # K*OC not a multiple of OC
        gpu.col2im_1d(torch.zeros((3, 10), device="cuda"), 2, 3, 0)
    with pytest.raises(gpu.ShpError):  # wrong output length
        gpu.col2im_1d(cols, 2, 3, 0, out=torch.empty((3, 5), device="cuda"))
    with pytest.raises(gpu.ShpError):  # y over cols
        buf = torch.zeros(64, device="cuda")
        gpu.col2im_1d(buf[:12].view(1, 12), 2, 3, 0, out=buf[4:16].view(3, 4))


def test_transpose_conv_known_answers_on_the_gpu(gpu):
    """tests/vits_transpose_conv_test.cpp:237-264 with the scatter as a node
    of a list run by the executor (exact, as the test compares)."""
    from test_oracle_goldens import _definition, _load, transpose_conv
    d = _load("vits_transpose_conv.json")

    def col2im_on_gpu(stride, oc, padding):
        def run(cols):
            g = gpu.Graph()
            y = g.col2im_1d(_t(gpu, cols), stride, oc, padding)
            assert [k for k, *_ in g.plan(y)] == ["single"]
            g.compute(y)
            return _np(y.t)
        return run
    for c in d["single_channel"]:
        x = np.array(c["input"], np.float32).reshape(-1, 1)
        w = np.array(c["kernel"], np.float32).reshape(1, 1, -1)
        got = transpose_conv(x, w, c["stride"], c["padding"], col2im_on_gpu(c["stride"], 1, c["padding"]))
        assert np.array_equal(got.reshape(-1), np.array(c["expected"], np.float32))
    km, kb = d["kernel_fill"]
    im, ib = d["input_fill"]
    for c in d["multichannel"]:
        K, OC, IC, L = c["kernel"], c["out_channels"], c["in_channels"], c["length"]
        w = (np.arange(K * OC * IC) % km + kb).astype(np.float32).reshape(IC, OC, K)
        x = (np.arange(IC * L) % im + ib).astype(np.float32).reshape(L, IC)
        got = transpose_conv(x, w, c["stride"], c["padding"], col2im_on_gpu(c["stride"], OC, c["padding"]))
        assert np.array_equal(got, _definition(x, w, c["stride"], c["padding"]).astype(np.float32))


def test_codec_transposed_convolution_golden_through_the_executor(gpu):
    """tests/qwen3_tts_codec_ops_test.cpp:57-70: the node list after the
    codec's matrix product (qwen3-tts/codec.cpp:171-181) -- col2im_1d, the
    causal crop's copy, the channel bias, the transposing copy -- on the GPU,
    the product in double on the host; at the test's 1e-4."""
    from test_oracle_goldens import _load, codec_conv_inputs
    d = _load("qwen3_codec_convs.json")
    x, v = codec_conv_inputs(d)
    C, OC, S = d["channels"], d["out_channels"], d["stride"]
    K = 2 * S
    w = v["transposed_weight"].reshape(C, OC, K)
    cols = R.mul_mat(w.reshape(C, OC * K).T.copy(), x)       # (L, K*OC)
    g = gpu.Graph()
    wide = g.col2im_1d(_t(gpu, cols), S, OC, 0)               # (OC, T)
    kept = wide.t.shape[1] - (K - S)
    crop = g.cont(g.view(wide, wide.t[:, :kept]))
    biased = g.add(crop, _t(gpu, v["transposed_bias"].reshape(OC, 1)))
    out = g.cont(g.view(biased, biased.t.t()))
    kinds = [k for k, *_ in g.plan(out) if k != "nop"]
    assert kinds[0] == "single" and len(kinds) <= 3, kinds
    g.compute(out)
    exp = np.array(d["expected_transposed"], np.float32)
    assert np.abs(_np(out.t).reshape(-1) - exp).max() < d["tolerance_cpu"]


@pytest.mark.parametrize("K,OC,L,S,P", [(16, 256, 4096, 8, 4), (16, 128, 8192, 8, 4), (4, 64, 65536, 2, 1)])
def test_col2im_full_size(gpu, K, OC, L, S, P):
    """The vocoders' upsampling stages at configs[3]'s sizes (T = 32768 /
    65536 / 131072 samples)."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(SEED + K + OC)
    cols = torch.randn((L, K * OC), generator=g, device="cuda")
    got = _np(gpu.col2im_1d(cols, S, OC, P))
    ref = _ref(_np(cols), S, OC, P)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))

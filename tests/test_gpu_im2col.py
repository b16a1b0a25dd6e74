"""shp_im2col against the restatement's ggml_im2col (1-D), bit for bit: F32
and F16 columns, every write form of the kernel (whole-tile ranges with
unaligned ends, 4-value runs, 1-value runs), time-contiguous and transposed
channel-major inputs, strides, dilations, paddings past the receptive field,
and the vocoder / codec shapes at full size against torch's strided gather."""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t

pytestmark = pytest.mark.gpu

SEED = 20261207

# (N, IC, IW, K, s0, p0, d0): the call sites' forms and the kernel's tilings
CASES = [
    (1, 128, 1000, 3, 1, 1, 1),     # a resblock conv (4-value runs, 32-channel tiles)
    (1, 128, 777, 11, 1, 25, 5),    # K = 11 at dilation 5 (vits resblock)
    (1, 96, 515, 7, 1, 9, 3),       # K = 7 at dilation 3
    (1, 37, 300, 3, 1, 1, 1),       # IC*K not a multiple of 4, channel tiles: 1-value runs
    (1, 32, 4099, 3, 1, 1, 1),      # whole-channel tiles, one range per tile
    (1, 5, 1001, 7, 1, 3, 1),       # whole-channel tiles, ranges with unaligned ends
    (64, 1, 333, 7, 1, 6, 1),       # the depthwise form: each channel a batch entry (codec.cpp:124-129)
    (3, 16, 200, 4, 2, 1, 1),       # stride 2 (kokoro / omnivoice encoders)
    (2, 40, 97, 5, 3, 0, 2),        # stride 3, dilation 2, no padding
    (1, 8, 6, 7, 3, 0, 1),          # kernel wider than the input: OW = 1 by C's truncation
    (1, 1, 1, 1, 1, 0, 1),          # one value
    (1, 512, 64, 3, 1, 40, 1),      # padding far past both ends
]


def _cols_ref(x, k, s0, p0, d0, dtype):
    return R.run(lambda g: g.im2col(x, k, s0, p0, d0, dst_type=dtype), n_threads=8)


def _check(got, ref, dtype):
    got = _np(got)
    if dtype == R.F16:
        assert np.array_equal(got.view(np.uint16), ref)
    else:
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("N,IC,IW,K,s0,p0,d0", CASES)
@pytest.mark.parametrize("f16", [False, True])
def test_im2col_time_contiguous(gpu, N, IC, IW, K, s0, p0, d0, f16):
    import torch
    rng = np.random.default_rng([SEED, N, IC, IW, K, s0, p0, d0])
    x = rng.standard_normal((N, IC, IW)).astype(np.float32)
    dt = torch.float16 if f16 else torch.float32
    got = gpu.im2col(_t(gpu, x), K, s0, p0, d0, dtype=dt)
    _check(got, _cols_ref(x, K, s0, p0, d0, R.F16 if f16 else R.F32), R.F16 if f16 else R.F32)


@pytest.mark.parametrize("N,IC,IW,K,s0,p0,d0", [c for c in CASES if c[0] == 1])
@pytest.mark.parametrize("f16", [False, True])
def test_im2col_reads_the_transposed_channel_major_view(gpu, N, IC, IW, K, s0, p0, d0, f16):
    """x is ggml_transpose of a channel-major [IC, IW] activation (channels
    contiguous): the columns equal those of its ggml_cont."""
    import torch
    rng = np.random.default_rng([SEED + 1, IC, IW, K])
    cm = rng.standard_normal((IW, IC)).astype(np.float32)  # ggml [IC, IW]
    view = _t(gpu, cm).t()                                   # ggml [IW, IC], nb0 = 4*IC, nb1 = 4
    dt = torch.float16 if f16 else torch.float32
    got = gpu.im2col(view, K, s0, p0, d0, dtype=dt)
    ref = _cols_ref(np.ascontiguousarray(cm.T), K, s0, p0, d0, R.F16 if f16 else R.F32)
    _check(got, ref, R.F16 if f16 else R.F32)


@pytest.mark.parametrize("shift_x,shift_y", [(1, 0), (0, 1), (3, 2)])
def test_im2col_unaligned_input_and_output(gpu, shift_x, shift_y):
    """x and y starting off 16 bytes: the same bits (y off its alignment takes
    the 1-value form)."""
    import torch
    rng = np.random.default_rng(SEED + 7 * shift_x + shift_y)
    IC, IW, K = 64, 301, 3
    base = rng.standard_normal(IC * IW + shift_x).astype(np.float32)
    x = _t(gpu, base)[shift_x:].view(IC, IW)
    ow = R.conv_out_len(IW, K, 1, 1, 1)
    ybuf = torch.empty(ow * IC * K + shift_y, dtype=torch.float32, device="cuda")
    out = ybuf[shift_y:].view(1, ow, IC * K)
    gpu.im2col(x, K, 1, 1, 1, out=out)
    _check(out, _cols_ref(base[shift_x:].reshape(IC, IW), K, 1, 1, 1, R.F32), R.F32)


def _torch_cols(x, k, s0, p0, d0):
    """The columns by torch's strided view of the zero-padded input: (N, OW, IC*k)."""
    import torch
    n_, ic, iw = x.shape
    ow = R.conv_out_len(iw, k, s0, p0, d0)
    xp = torch.nn.functional.pad(x, (p0, p0 + s0 + k * d0))
    cols = xp.as_strided((n_, ow, ic, k), (xp.stride(0), s0, xp.stride(1), d0))
    return cols.reshape(n_, ow, ic * k)


@pytest.mark.parametrize("IC,T,K,d0,f16,chmajor", [
    (128, 131072, 3, 1, False, False),   # configs[3]'s last vocoder stage, resblock K=3
    (128, 131072, 11, 5, False, False),  # K = 11 at dilation 5
    (512, 8192, 7, 3, True, False),      # F16 columns of an F16 kernel (vits/operations.cpp:40)
    (1024, 8192, 3, 1, False, True),     # the codec's causal conv from the channel-major activation
])
def test_im2col_full_size(gpu, IC, T, K, d0, f16, chmajor):
    import torch
    g = torch.Generator(device="cuda").manual_seed(SEED + IC + K)
    if chmajor:
        x = torch.randn((T, IC), generator=g, device="cuda").t()
        p0 = (K - 1) * d0
    else:
        x = torch.randn((IC, T), generator=g, device="cuda")
        p0 = (K - 1) * d0 // 2
    dt = torch.float16 if f16 else torch.float32
    got = gpu.im2col(x, K, 1, p0, d0, dtype=dt)
    ref = _torch_cols(x.contiguous().unsqueeze(0), K, 1, p0, d0).to(dt)
    assert got.shape == ref.shape
    assert torch.equal(got.view(torch.int16 if f16 else torch.int32), ref.view(torch.int16 if f16 else torch.int32))


def test_im2col_refusals(gpu):
    import torch
    x = torch.zeros((4, 100), device="cuda")
    ow = R.conv_out_len(100, 3, 1, 1, 1)
    with pytest.raises(gpu.ShpError):  # wrong output length
        gpu.im2col(x, 3, 1, 1, 1, out=torch.empty((1, ow + 1, 12), device="cuda"))
    with pytest.raises(gpu.ShpError):  # no output position
        gpu.im2col(x, 50, 1, 0, 3)
    with pytest.raises(gpu.ShpError):  # F16 input
        gpu.im2col(x.half(), 3, 1, 1, 1)
    with pytest.raises(gpu.ShpError):  # y over x
        buf = torch.zeros(4 * 100 * 3 + 400, device="cuda")
        gpu.im2col(buf[:400].view(4, 100), 3, 1, 1, 1, out=buf[:1200].view(1, ow, 12))
    with pytest.raises(gpu.ShpError):  # stride 0
        gpu.im2col(x, 3, 0, 1, 1, out=torch.empty((1, ow, 12), device="cuda"))


# ---------------------------------------------------------------------------
# through the node-run executor
# ---------------------------------------------------------------------------

def _golden_inputs():
    from test_oracle_goldens import _load, codec_conv_inputs
    d = _load("qwen3_codec_convs.json")
    x, v = codec_conv_inputs(d)
    return d, x, v


def test_codec_convolutions_golden_through_the_executor(gpu):
    """tests/qwen3_tts_codec_ops_test.cpp:43-56 with the columns built on the
    GPU from the node list codec_causal_conv1d and codec_causal_depthwise_conv1d
    emit (codec.cpp:94-96,124-129): the causal convolution's copy and im2col
    as one launch (the copy never written), the depthwise form's copy then
    im2col. The products, crop and bias in double on the host, at the test's
    1e-4."""
    d, x, v = _golden_inputs()
    C, L, OC, K, dil = d["channels"], d["length"], d["out_channels"], d["kernel"], d["dilation"]
    w = v["conv_weight"].reshape(OC, C, K)
    wd = v["depthwise_weight"].reshape(C, 1, K)
    tx = _t(gpu, x)                                    # ggml [C, L]
    g = gpu.Graph()
    tm = g.cont(g.view(tx, tx.t()))
    cols = g.im2col(_t(gpu, w), tm, 1, (K - 1) * dil, dil)
    assert [k for k, *_ in g.plan(cols) if k != "nop"] == ["cont_im2col"]
    g.compute(cols)
    wide = _np(cols.t)[0].astype(np.float64) @ w.reshape(OC, C * K).astype(np.float64).T
    got = (wide[:L] + v["conv_bias"][None, :]).astype(np.float32)
    assert np.abs(got.reshape(-1) - np.array(d["expected_causal_conv"], np.float32)).max() < d["tolerance_cpu"]
    g = gpu.Graph()
    tm = g.cont(g.view(tx, tx.t()))
    dcols = g.im2col(_t(gpu, wd), g.view(tm, tm.t.view(C, 1, L)), 1, K - 1, 1)
    assert [k for k, *_ in g.plan(dcols) if k != "nop"] == ["single", "single"]
    g.compute(dcols)
    wide = np.einsum("cok,ck->oc", _np(dcols.t).astype(np.float64), wd.reshape(C, K).astype(np.float64))
    got = (wide[:L] + v["depthwise_bias"][None, :]).astype(np.float32)
    assert np.abs(got.reshape(-1) - np.array(d["expected_depthwise"], np.float32)).max() < d["tolerance_cpu"]


@pytest.mark.parametrize("C,T,K,d0,f16", [(1024, 2000, 7, 1, False), (512, 3001, 3, 3, True), (96, 777, 5, 2, False)])
def test_cont_im2col_run_equals_its_nodes(gpu, C, T, K, d0, f16):
    """The fused run against the same list with the copy written (read again
    after the graph), bit for bit, and against the restatement's im2col of the
    time-major copy."""
    import torch
    rng = np.random.default_rng([SEED, C, T, K])
    x = rng.standard_normal((T, C)).astype(np.float32)  # ggml [C, T]
    w = torch.zeros((8, C, K), device="cuda")
    dt = torch.float16 if f16 else torch.float32
    outs = []
    for keep_copy in (False, True):
        tx = _t(gpu, x)
        g = gpu.Graph()
        tm = g.cont(g.view(tx, tx.t()))
        cols = g.im2col(w, tm, 1, (K - 1) * d0, d0, dtype=dt)
        kinds = [k for k, *_ in g.plan(*((cols, tm) if keep_copy else (cols,))) if k != "nop"]
        assert kinds == (["single", "single"] if keep_copy else ["cont_im2col"])
        g.compute(*((cols, tm) if keep_copy else (cols,)))
        outs.append(_np(cols.t))
    assert np.array_equal(outs[0].view(np.uint16 if f16 else np.uint32), outs[1].view(np.uint16 if f16 else np.uint32))
    ref = _cols_ref(np.ascontiguousarray(x.T), K, 1, (K - 1) * d0, d0, R.F16 if f16 else R.F32)
    _check(torch.from_numpy(outs[0]), ref, R.F16 if f16 else R.F32)

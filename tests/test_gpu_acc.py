"""shp_acc against the restatement's ggml_acc, bit for bit (one f32 add per
element in the window, a copy elsewhere): row windows at a row offset, narrower
and 3-D windows, unaligned destinations, ggml's inplace form; the talker's
prefill input (qwen3-tts/talker.cpp:86-118) as the node list its builder emits,
the codec embeddings gathered on the GPU, through the executor."""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t
from test_oracle_closed_forms import prefill_input

pytestmark = pytest.mark.gpu

SEED = 20261213

CASES = [
    # (a shape, b shape, (nb1, nb2, nb3), offset)
    ((10, 8), (4, 8), (32, 128, 128), 3 * 32),
    ((10, 8), (1, 8), (32, 32, 32), 9 * 32),
    ((10, 8), (3, 5), (32, 96, 96), 1 * 32 + 2 * 4),
    ((6, 5, 12), (2, 3, 4), (48, 240, 480), 4 + 48),
    ((40,), (6,), (24, 24, 24), 7 * 4),
    ((9, 7), (3, 2), (56, 112, 112), 4),
    ((37, 1001), (30, 1001), (4004, 4004 * 37, 4004 * 37), 7 * 4004),   # rows of 1001: quads across rows
    ((300, 2048), (297, 2048), (8192, 8192 * 300, 8192 * 300), 3 * 8192),  # the talker's codec run
]


def _ref(a, b, nb, offset):
    return R.run(lambda g: g.acc(a, b, *nb, offset))


@pytest.mark.parametrize("ashape,bshape,nb,offset", CASES)
def test_acc_matches_restatement(gpu, ashape, bshape, nb, offset):
    rng = np.random.default_rng([SEED, *ashape, offset])
    a = rng.standard_normal(ashape).astype(np.float32)
    b = rng.standard_normal(bshape).astype(np.float32)
    ref = _ref(a, b, nb, offset)
    got = _np(gpu.acc(_t(gpu, a), _t(gpu, b), *nb, offset))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    ta = _t(gpu, a)                                         # ggml's inplace form: the window only
    gpu.acc(ta, _t(gpu, b), *nb, offset, inplace=True)
    assert np.array_equal(_np(ta).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("shift", [1, 2, 3])
def test_acc_unaligned_and_strided_b(gpu, shift):
    """a and y off 16 bytes; b a column slice (rows strided)."""
    import torch
    rng = np.random.default_rng(SEED + shift)
    a = rng.standard_normal((50, 37)).astype(np.float32)
    wide = rng.standard_normal((20, 40)).astype(np.float32)
    b = wide[:, 3:33]
    nb = (4 * 37, 4 * 37 * 50, 4 * 37 * 50)
    ref = _ref(a, np.ascontiguousarray(b), nb, 5 * 4 * 37 + 4)
    abuf = torch.zeros(a.size + shift, device="cuda")
    abuf[shift:] = torch.from_numpy(a.reshape(-1)).cuda()
    ybuf = torch.zeros(a.size + shift, device="cuda")
    out = ybuf[shift:].view(50, 37)
    gpu.acc(abuf[shift:].view(50, 37), _t(gpu, wide)[:, 3:33], *nb, 5 * 4 * 37 + 4, out=out)
    assert np.array_equal(_np(out).view(np.uint32), ref.view(np.uint32))


def test_acc_negative_zero_outside_the_window(gpu):
    """Elements outside the window are copied, not added to 0 (-0.0 stays)."""
    a = np.full((4, 8), -0.0, np.float32)
    b = np.ones((1, 8), np.float32)
    got = _np(gpu.acc(_t(gpu, a), _t(gpu, b), 32, 32, 32, 32))
    assert np.array_equal(got.view(np.uint32), _ref(a, b, (32, 32, 32), 32).view(np.uint32))
    assert np.signbit(got[0]).all()


def test_acc_refusals(gpu):
    import torch
    a = torch.zeros((4, 8), device="cuda")
    b = torch.zeros((2, 8), device="cuda")
    with pytest.raises(gpu.ShpError):     # past a's end
        gpu.acc(a, b, 32, 64, 64, 3 * 32)
    with pytest.raises(gpu.ShpError):     # overlapping rows
        gpu.acc(a, b, 16, 64, 64, 0)
    with pytest.raises(gpu.ShpError):     # an offset inside an element
        gpu.acc(a, b, 32, 64, 64, 2)
    with pytest.raises(gpu.ShpError):     # y over b
        buf = torch.zeros(64, device="cuda")
        gpu.acc(a, buf[:16].view(2, 8), 32, 64, 64, 0, out=buf[8:40].view(4, 8))


@pytest.mark.parametrize("speaker_index,codec_offset,acoustic", [(0, 0, False), (2, 3, False), (5, 3, True),
                                                                  (None, 4, True)])
def test_talker_prefill_input_through_the_executor(gpu, speaker_index, codec_offset, acoustic):
    """build_talker_prefill_input's accumulation (talker.cpp:86-118): the
    codec embeddings gathered from a BF16-valued table on the GPU, viewed as
    head and tail around the x-vector's slot, each added into the text stream
    with ggml_acc, then the ICL acoustic block; against the restatement's
    nodes, exactly."""
    rng = np.random.default_rng(SEED + (speaker_index or 0) + 10 * codec_offset)
    H, n, V = 1024, 6, 64
    N = codec_offset + n
    text = rng.standard_normal((N, H)).astype(np.float32)
    table = rng.standard_normal((V, H)).astype(np.float32)
    ids = rng.integers(0, V, n).astype(np.int32)
    speaker = rng.standard_normal(H).astype(np.float32)
    m = 4
    ac = rng.standard_normal((m, H)).astype(np.float32) if acoustic else None
    codec_np = table[ids]
    ref = R.run(lambda g: prefill_input(g, text, codec_np, codec_offset, None if speaker_index is None else speaker,
                                        -1 if speaker_index is None else speaker_index, ac, N - m if acoustic else -1))
    g = gpu.Graph()
    tt, sp = _t(gpu, text), _t(gpu, speaker)
    codec = g.get_rows(_t(gpu, table), _t(gpu, ids))
    nb1, nb2 = 4 * H, 4 * H * N
    if speaker_index is None:
        out = g.acc(tt, codec, nb1, nb2, nb2, codec_offset * nb1)
    else:
        out = tt
        if speaker_index > 0:
            out = g.acc(out, g.view(codec, codec.t[:speaker_index]), nb1, nb2, nb2, codec_offset * nb1)
        out = g.acc(out, g.view(sp, sp.view(1, H)), nb1, nb2, nb2, (codec_offset + speaker_index) * nb1)
        if n - speaker_index - 1 > 0:
            out = g.acc(out, g.view(codec, codec.t[speaker_index + 1:]), nb1, nb2, nb2,
                        (codec_offset + speaker_index + 1) * nb1)
    if acoustic:
        out = g.acc(out, _t(gpu, ac), nb1, nb2, nb2, (N - m) * nb1)
    kinds = [k for k, *_ in g.plan(out) if k != "nop"]
    assert set(kinds) == {"single"}, kinds
    g.compute(out)
    assert np.array_equal(_np(out.t).view(np.uint32), ref.view(np.uint32))


def test_acc_inplace_node(gpu):
    """GGML_OP_ACC with inplace set: the node's result is a's own memory."""
    rng = np.random.default_rng(SEED + 99)
    a = rng.standard_normal((12, 64)).astype(np.float32)
    b = rng.standard_normal((5, 64)).astype(np.float32)
    ref = _ref(a, b, (256, 256 * 12, 256 * 12), 256 * 4)
    g = gpu.Graph()
    ta = _t(gpu, a)
    out = g.acc(ta, _t(gpu, b), 256, 256 * 12, 256 * 12, 256 * 4, inplace=True)
    g.compute(out)
    assert out.t.data_ptr() == ta.data_ptr()
    assert np.array_equal(_np(ta).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("inplace", [False, True])
def test_acc_full_size(gpu, inplace):
    """The bench's shape: a [2048, 8192] stream with an 8176-position block
    added from position 16."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(SEED + inplace)
    a = torch.randn((8192, 2048), generator=g, device="cuda")
    b = torch.randn((8176, 2048), generator=g, device="cuda")
    ref = _ref(_np(a), _np(b), (8192, 8192 * 8192, 8192 * 8192), 16 * 8192)
    got = gpu.acc(a, b, 8192, 8192 * 8192, 8192 * 8192, 16 * 8192, inplace=inplace)
    assert np.array_equal(_np(got).view(np.uint32), ref.view(np.uint32))

"""ggml_cont / ggml_cpy of transposed and permuted F32 views through shp_cpy:
the vocoder's time-major copies around each convolution (vits/operations.cpp:
72,87,100,108) and the attention's permute(1,0,2,3) copy (qwen3-tts/
operations.cpp:136). Every result must equal the oracle's ggml_cont
restatement bit for bit, and torch's own permuted copy too."""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t, assert_bitexact

pytestmark = pytest.mark.gpu
SEED = 20261202


def _oracle_cont(gpu, base, v):
    """The oracle's ggml_cont of the torch view v of the contiguous tensor
    base, read through the same ggml extents and byte strides the library
    sees."""
    d = gpu.desc(v)
    g = R.Graph()
    y = g.cont_f32(_np(base), list(d.ne), list(d.nb), offset=v.data_ptr() - base.data_ptr())
    g.compute(8)
    return y.reshape(tuple(v.shape))


def _source(rng, shape):
    import torch
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).cuda()


# (torch shape of the contiguous source, permutation of its axes)
CASES = [
    ((37, 70), (1, 0)),            # ragged tiles; ne0 = 37: element-wide path
    ((64, 64), (1, 0)),            # one full tile
    ((128, 256), (1, 0)),          # full tiles, 16-byte path
    ((200, 196), (1, 0)),          # 16-byte path with partial tiles along both dims
    ((130, 7), (1, 0)),
    ((1, 33), (1, 0)),             # ne0 = 1
    ((1000, 3), (1, 0)),
    ((4, 4096), (1, 0)),
    ((5, 9, 130), (1, 2, 0)),      # contiguous dim lands on ggml dim 1
    ((2, 16, 7, 128), (0, 3, 1, 2)),  # contiguous dim lands on ggml dim 2
    ((7, 9, 11, 12), (3, 0, 1, 2)),   # contiguous dim lands on ggml dim 3
    ((2, 3, 5, 7), (3, 2, 1, 0)),
    ((37, 16, 128), (0, 2, 1)),    # ggml permute(x, 1, 0, 2, 3) of x = [128, 16, 37]
]


@pytest.mark.parametrize("shape,perm", CASES)
def test_transposed_copy_matches_oracle(gpu, shape, perm):
    rng = np.random.default_rng(SEED + sum(shape))
    x = _source(rng, shape)
    v = x.permute(perm)
    d = gpu.desc(v)
    print("case", shape, perm, list(d.ne), list(d.nb), flush=True)
    assert d.nb[0] != 4
    y = gpu.cpy(v)
    assert_bitexact(_np(y), _oracle_cont(gpu, x, v))
    assert_bitexact(_np(y), _np(v.contiguous()))


@pytest.mark.parametrize("shift", [0, 1, 2, 3])
def test_unaligned_views_take_the_narrow_path(gpu, shift):
    """A view starting 1-3 floats past a 16-byte boundary, or with strides
    that are not multiples of 16 bytes, is copied element by element; the
    result is the same."""
    import torch
    rng = np.random.default_rng(SEED + 40 + shift)
    x = _source(rng, (300, 258))
    v = x[:, shift:shift + 200].t()  # ggml [300, 200] over rows of 258 floats
    print("shift", shift, flush=True)
    y = gpu.cpy(v)
    assert_bitexact(_np(y), _oracle_cont(gpu, x, v))
    out = torch.empty((200, 300), dtype=torch.float32, device="cuda")
    gpu.cpy(v, out)
    assert_bitexact(_np(out), _np(v.contiguous()))


def test_into_a_row_strided_destination(gpu):
    """The destination may be a slice of a wider buffer (rows contiguous, row
    stride larger): only its own elements are written."""
    import torch
    rng = np.random.default_rng(SEED + 60)
    x = _source(rng, (96, 160))
    big = torch.full((160, 128), 7.0, dtype=torch.float32, device="cuda")
    dst = big[:, 16:112]
    gpu.cpy(x.t(), dst)
    host = _np(big)
    assert_bitexact(host[:, 16:112], _np(x.t().contiguous()))
    assert (host[:, :16] == 7.0).all() and (host[:, 112:] == 7.0).all()


@pytest.mark.parametrize("C,T", [(512, 8192), (256, 32768), (128, 131072)])
def test_vocoder_time_major_copy_full_size(gpu, C, T):
    """ggml_cont(ggml_transpose(x)) of a vocoder activation x = ggml [C, T]
    (vits/operations.cpp:72) at the Snake shapes: x stored as torch (T, C)."""
    rng = np.random.default_rng(SEED + C)
    x = _source(rng, (T, C))
    v = x.t()
    print("C", C, "T", T, flush=True)
    y = gpu.cpy(v)
    assert_bitexact(_np(y), _oracle_cont(gpu, x, v))
    back = gpu.cpy(y.t())  # and back: the depthwise branch's final transpose (:108)
    assert_bitexact(_np(back), _np(x))


def test_transposed_copy_in_a_node_list(gpu):
    """The executor runs ggml_cont(ggml_transpose(x)) as a copy node between
    the vocoder's leaky-ReLU and the next consumer, each node on its own."""
    rng = np.random.default_rng(SEED + 80)
    x = _source(rng, (1024, 192))  # ggml [192, 1024]
    g = gpu.Graph()
    act = g.leaky_relu(x, 0.1)
    tm = g.cont(g.view(act, act.t.t()))
    out = g.exp(tm)
    kinds = [k for k, *_ in g.plan(act, out) if k != "nop"]
    assert kinds == ["single", "single", "single"], kinds
    g.compute(act, out)
    assert_bitexact(_np(tm.t), np.ascontiguousarray(_np(act.t).T))


def _oracle_tail(out, bias, r, slope):
    """The restatement of the tail node by node: ggml_cont of out^T, the
    [1, C] bias add, the residual add, the leaky-ReLU. out: numpy (T, C) =
    ggml [C, T]; bias (C, 1); r (C, T) or None. Returns (sum, y)."""
    g = R.Graph()
    T, C = out.shape
    tm = g.cont_f32(out, [T, C], [4 * C, 4])
    s = g.binbcast(R.OP_ADD, tm.reshape(C, T), bias)
    if r is not None:
        s = g.add(s, r)
    y = g.leaky_relu(s, slope) if slope is not None else s
    g.compute(8)
    return s.reshape(C, T), y.reshape(C, T)


TAIL_SHAPES = [(2048, 96), (4096, 512), (1000, 37), (130, 64)]


@pytest.mark.parametrize("T,C", TAIL_SHAPES)
@pytest.mark.parametrize("resid,leaky,with_sum", [(False, False, False), (False, True, False), (False, True, True),
                                                  (True, False, False), (True, True, False), (True, True, True)])
def test_cont_add_leaky_matches_nodes(gpu, T, C, resid, leaky, with_sum):
    """shp_cont_add_leaky_relu against the restatement's nodes one by one,
    bit-exact, for every form (vits/waveform-decoder.cpp:111,118-121,146-150)."""
    import torch
    rng = np.random.default_rng(SEED + T + C + 7 * resid + 3 * leaky + with_sum)
    out = rng.standard_normal((T, C)).astype(np.float32)
    bias = rng.standard_normal((C, 1)).astype(np.float32)
    r = rng.standard_normal((C, T)).astype(np.float32) if resid else None
    slope = 0.1 if leaky else None
    to = _t(gpu, out)
    s_out = torch.empty((C, T), dtype=torch.float32, device="cuda") if with_sum else None
    print("tail", T, C, resid, leaky, with_sum, flush=True)
    y = gpu.cont_add_leaky_relu(to.t(), _t(gpu, bias), _t(gpu, r) if resid else None, slope, sum_out=s_out)
    ref_s, ref_y = _oracle_tail(out, bias, r, slope)
    assert_bitexact(_np(y), ref_y)
    if with_sum:
        assert_bitexact(_np(s_out), ref_s)


def test_cont_add_leaky_in_place_residual_and_unaligned(gpu):
    """The residual's buffer reused for the sum (ggml's in-place add), and a
    source view 1 float off a 16-byte boundary (dword path)."""
    import torch
    rng = np.random.default_rng(SEED + 91)
    T, C = 1024, 64
    out = rng.standard_normal((T, C + 1)).astype(np.float32)
    bias = rng.standard_normal((C, 1)).astype(np.float32)
    r = rng.standard_normal((C, T)).astype(np.float32)
    to = _t(gpu, out)
    tr = _t(gpu, r)
    view = to[:, 1:].t()                                  # ggml [T, C], rows 1 float in
    y = gpu.cont_add_leaky_relu(view, _t(gpu, bias), tr, 0.2, sum_out=tr)
    ref_s, ref_y = _oracle_tail(np.ascontiguousarray(out[:, 1:]), bias, r, 0.2)
    assert_bitexact(_np(y), ref_y)
    assert_bitexact(_np(tr), ref_s)


def test_transposing_copy_refuses_an_overlapping_destination(gpu):
    """A destination overlapping the transposed source would be read after
    being written by another tile: refused, nothing launched."""
    import torch
    x = torch.zeros((64, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(gpu.ShpError):
        gpu.cpy(x.t(), x)
    with pytest.raises(gpu.ShpError):
        gpu.cont_add_leaky_relu(x.t(), torch.zeros((64, 1), device="cuda"), None, 0.1, out=x)


def test_conv_tail_refuses_a_contiguous_view(gpu):
    """One channel: the transpose of ggml [1, T] has ne[0] contiguous, so its
    ggml_cont is a plain copy, not this entry point's form: refused, nothing
    launched."""
    import torch
    x = torch.zeros((256, 1), dtype=torch.float32, device="cuda")
    with pytest.raises(gpu.ShpError):
        gpu.cont_add_leaky_relu(x.t(), torch.zeros((1, 1), device="cuda"), None, 0.1)


def test_conv_tail_in_a_node_list(gpu):
    """Two resblock convolutions' tails in one list (:146-150): copy, bias,
    leaky into the next GEMM's input; copy, bias, residual add, the next
    layer's leaky with the sum carried. Two launches, bit-identical to the
    list run with every result written, and to the restatement."""
    import torch
    rng = np.random.default_rng(SEED + 93)
    T, C = 4096, 128
    host = {n: rng.standard_normal(sh).astype(np.float32) for n, sh in
            (("o1", (T, C)), ("o2", (T, C)), ("b1", (C, 1)), ("b2", (C, 1)), ("res", (C, T)))}
    dev = {n: _t(gpu, a) for n, a in host.items()}

    def build(every):
        g = gpu.Graph()
        t1 = g.cont(g.view(dev["o1"], dev["o1"].t()))
        act = g.leaky_relu(g.add(t1, dev["b1"]), 0.1)
        t2 = g.cont(g.view(dev["o2"], dev["o2"].t()))
        state = g.add(g.add(t2, dev["b2"]), dev["res"])
        nxt = g.leaky_relu(state, 0.1)
        outs = [act, state, nxt]
        return g, outs, (outs + [n["val"] for n in g.order(*outs)]) if every else outs

    g, outs, every = build(False)
    assert [k for k, *_ in g.plan(*every) if k != "nop"] == ["cont_add_leaky", "cont_add_leaky"]
    g.compute(*every)
    fused = [_np(o.t).copy() for o in outs]
    g, outs, every = build(True)
    assert "cont_add_leaky" not in [k for k, *_ in g.plan(*every)]  # every copy is written: no tail runs
    g.compute(*every)
    for a, b in zip(fused, [_np(o.t) for o in outs]):
        assert_bitexact(a, b)
    _, act = _oracle_tail(host["o1"], host["b1"], None, 0.1)
    state, nxt = _oracle_tail(host["o2"], host["b2"], host["res"], 0.1)
    for a, b in zip(fused, (act, state, nxt)):
        assert_bitexact(a, b)


@pytest.mark.parametrize("T,C", [(4096, 96), (1000, 37), (130, 64)])
@pytest.mark.parametrize("resid,leaky,with_sum", [(False, False, False), (True, True, True), (False, True, False)])
def test_cont_add_leaky_column_bias(gpu, T, C, resid, leaky, with_sum):
    """The bias as one row of ne0 values repeated over y's rows (the channel
    bias of a channel-major result, qwen3-tts/codec.cpp:58-59,179-181): y =
    cont(x) + b [+ r], leaky; against the restatement's nodes."""
    import torch
    rng = np.random.default_rng(SEED + 2 * T + C + resid)
    src = rng.standard_normal((C, T)).astype(np.float32)       # ggml [T, C]; y = its transpose, ggml [C, T]
    bias = rng.standard_normal(C).astype(np.float32)           # ggml [C]
    r = rng.standard_normal((T, C)).astype(np.float32) if resid else None
    slope = 0.1 if leaky else None
    ts = _t(gpu, src)
    s_out = torch.empty((T, C), dtype=torch.float32, device="cuda") if with_sum else None
    y = gpu.cont_add_leaky_relu(ts.t(), _t(gpu, bias), _t(gpu, r) if resid else None, slope, sum_out=s_out)
    g = R.Graph()
    tm = g.cont_f32(src, [C, T], [4 * T, 4]).reshape(T, C)
    s_ = g.add(tm, bias)
    if resid:
        s_ = g.add(s_, r)
    yr = g.leaky_relu(s_, slope) if leaky else s_
    g.compute(4)
    assert_bitexact(_np(y), yr)
    if with_sum:
        assert_bitexact(_np(s_out), s_)

"""The node-run executor on the GPU: node lists in the order the reference's
graphs reach a backend (ggml_build_forward_expand order), run by
shp_graph_compute, against the restatement and against the same lists run node
by node (an intermediate marked as a graph output keeps a run from fusing).

Bars as in test_gpu_parity: bit-exact for adds, products, quotients, squares,
casts, gathers and sums; 1e-5 for norms, SwiGLU and Snake; rope bit-exact
against the restatement with correctly rounded cos/sin. Fused and node-by-node
runs of one list are bit-identical.
"""
import numpy as np
import pytest

import formats as F
import ggml_ref as R
from test_gpu_parity import (SEED, _np, _positions, _t, assert_bitexact, assert_close, assert_rope_close,
                              assert_snake_close)

pytestmark = pytest.mark.gpu


def _bf16(gpu, bits):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def test_single_node_entry_points(gpu):
    """shp_mul / shp_div (same shape and a broadcast row), shp_sin, shp_sqr and
    shp_cpy (F32 copy into a strided view, BF16 and F16 casts) against the
    restatement's nodes."""
    import torch
    rng = np.random.default_rng(SEED + 201)
    a = rng.standard_normal((37, 1024)).astype(np.float32)
    b = rng.standard_normal((37, 1024)).astype(np.float32)
    row = rng.standard_normal(1024).astype(np.float32)
    row[:4] = [0.0, -0.0, 1e-40, np.inf]
    for op in ("mul", "div"):
        for bb in (b, row):
            with np.errstate(all="ignore"):
                ref = R.run(lambda g: getattr(g, op)(a, bb))
            got = _np(getattr(gpu, op)(_t(gpu, a), _t(gpu, bb)))
            assert np.array_equal(np.isnan(got), np.isnan(ref))
            assert_bitexact(np.where(np.isnan(ref), 0, got), np.where(np.isnan(ref), 0, ref))
    x = (rng.standard_normal((64, 512)) * 20).astype(np.float32)
    x[0, :8] = [0.0, -0.0, 1e5, -3e4, 40000.0, 1e-30, -1e-30, -1e-45]
    assert_bitexact(_np(gpu.sqr(_t(gpu, x))), R.run(lambda g: g.sqr(x)))
    ref = R.run(lambda g: g.sin(x))
    got = _np(gpu.sin(_t(gpu, x)))
    ulps = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    # libm's sinf and the kernel's sine (the Snake kernels' own) are each within
    # 1 ulp of the exact sine; they agree on the sign of zeros
    assert ulps.max() <= 1
    assert (ulps == 0).mean() > 0.8
    cache = torch.zeros(16, 8, 64, device="cuda")
    k = rng.standard_normal((5, 8, 64)).astype(np.float32)
    gpu.cpy(_t(gpu, k), out=cache[3:8])
    assert_bitexact(_np(cache[3:8]), k)
    assert (_np(cache[:3]) == 0).all() and (_np(cache[8:]) == 0).all()
    w = rng.normal(1, 0.1, 3000).astype(np.float32)
    bits = F.f32_to_bf16_bits(w)
    assert_bitexact(_np(gpu.cpy(_bf16(gpu, bits))), R.run(lambda g: g.cast_f32(bits, R.BF16)))
    h = F.f32_to_f16_bits(w)
    got = _np(gpu.cpy(torch.from_numpy(h.view(np.int16)).cuda().view(torch.float16)))
    assert_bitexact(got, R.run(lambda g: g.cast_f32(h, R.F16)))


def _layer_inputs(rng, T, H=1024, heads=16, kv=8, hd=128, cap=64):
    d = dict(x=rng.standard_normal((T, H)), attn=rng.standard_normal((T, H)), mlp=rng.standard_normal((T, H)),
             q=rng.standard_normal((T, heads, hd)), k=rng.standard_normal((T, kv, hd)))
    d = {n: a.astype(np.float32) for n, a in d.items()}
    for n, size in (("w_in", H), ("w_post", H), ("wq", hd), ("wk", hd)):
        d[n] = F.f32_to_bf16_bits(rng.normal(1.0, 0.1, size).astype(np.float32))
    d["pos"] = _positions(rng, T, 8192)
    return d


@pytest.mark.parametrize("T", [1, 37])
def test_qwen3_layer_graph(gpu, T):
    """The non-GEMM nodes of a Qwen3 layer (operations.cpp:80-147) in expand
    order, with BF16 gains through ggml_cast: 4 fused runs and one add, every
    output as the restatement computes it; the same list with every
    intermediate marked as an output runs node by node, bit-identical."""
    import torch
    rng = np.random.default_rng(SEED + 300 + T)
    d = _layer_inputs(rng, T)
    eps, theta, hd, filled = np.float32(1e-6), np.float32(1e6), 128, 5
    dev = {n: (_bf16(gpu, a) if n.startswith("w") else _t(gpu, a)) for n, a in d.items()}

    def build(keep_all):
        g = gpu.Graph()
        cache = torch.zeros(64, 8, hd, device="cuda")
        mids = []

        def m(v):
            mids.append(v)
            return v
        normed = g.mul(m(g.rms_norm(dev["x"], eps)), m(g.cast(dev["w_in"])))
        qr = g.rope_ext(m(g.mul(m(g.rms_norm(dev["q"], eps)), m(g.cast(dev["wq"])))), dev["pos"], hd,
                        gpu.ROPE_TYPE_NEOX, theta)
        kr = m(g.rope_ext(m(g.mul(m(g.rms_norm(dev["k"], eps)), m(g.cast(dev["wk"])))), dev["pos"], hd,
                          gpu.ROPE_TYPE_NEOX, theta))
        kc = g.cpy(kr, cache[filled:filled + T])
        after = g.add(dev["x"], dev["attn"])
        mlp_in = g.mul(m(g.rms_norm(after, eps)), m(g.cast(dev["w_post"])))
        out = g.add(after, dev["mlp"])
        outs = [kc, normed, qr, mlp_in, out, after]
        return g, outs + (mids if keep_all else []), cache

    g, outs, cache = build(False)
    kinds = [k for k, *_ in g.plan(*outs) if k != "nop"]
    assert kinds == ["qk_norm_rope", "norm_mul", "add_norm_mul", "single"]
    g.compute(*outs)
    _, normed, qr, mlp_in, out, after = [_np(v.t) for v in outs]
    kc = _np(cache)
    g2, outs2, cache2 = build(True)
    assert all(k in ("single", "nop") for k, *_ in g2.plan(*outs2))
    g2.compute(*outs2)
    for a, b in zip(outs[1:6], outs2[1:6]):
        assert_bitexact(_np(a.t), _np(b.t))
    assert_bitexact(_np(cache2), kc)

    x, q, k = d["x"], d["q"], d["k"]
    assert_close(normed, R.run(lambda gr: R.rms_norm_w(gr, x, d["w_in"], eps, R.BF16)))
    qc, kc_ref = R.run(lambda gr: R.qk_norm_rope(gr, q, k, d["wq"], d["wk"], eps, d["pos"], hd, theta, R.BF16,
                                                 cs_rounded=True))
    assert_bitexact(qr, qc)
    assert_bitexact(kc[filled:filled + T], kc_ref)
    assert (kc[:filled] == 0).all() and (kc[filled + T:] == 0).all()
    s_ref, y_ref = R.run(lambda gr: R.add_rms_norm_w(gr, x, d["attn"], d["w_post"], eps, R.BF16))
    assert_bitexact(after, s_ref)
    assert_close(mlp_in, y_ref)
    assert_bitexact(out, R.run(lambda gr: gr.add(s_ref, d["mlp"])))


def _reference_layer_leaves(gpu, rng, T, total, H=1024, heads=16, kv=8, hd=128, ffn=3072):
    import torch
    d = _layer_inputs(rng, T, H, heads, kv, hd)
    d.update(v=rng.standard_normal((T, kv, hd)).astype(np.float32),
             scores=(4 * rng.standard_normal((heads, T, total))).astype(np.float32),
             gate=rng.standard_normal((T, ffn)).astype(np.float32),
             up=rng.standard_normal((T, ffn)).astype(np.float32))
    dev = {n: (_bf16(gpu, a) if n.startswith("w") else _t(gpu, a)) for n, a in d.items()}
    return d, dev, lambda: {"kcache": torch.zeros(total, kv, hd, device="cuda"),
                            "vcache": torch.zeros(total, kv, hd, device="cuda")}


@pytest.mark.parametrize("T", [1, 37])
def test_reference_order_layer_graph(gpu, T):
    """decoder_layer's non-GEMM nodes (operations.cpp:56-147) in expand order:
    the input norm, k's path and the k and v cache copies (:106-116) before
    the q path, then the softmax, the residual add, the post-attention norm,
    SwiGLU and the output add. The q run is moved up into k's launch with v's
    copy: five launches and the add. Every output is bit-identical to the same
    list run node by node and matches the restatement at the usual bars (rope
    bit-exact with correctly rounded cos/sin, the cache rows bit-exact, the
    softmax within 2 ulp)."""
    import torch
    from test_graph_plan import reference_layer
    rng = np.random.default_rng(SEED + 320 + T)
    hd, total, eps, theta = 128, 64, np.float32(1e-6), np.float32(1e6)
    filled = total - T
    d, dev, caches = _reference_layer_leaves(gpu, rng, T, total)

    def build(node_by_node):
        g = gpu.Graph()
        leaves = dict(dev, **caches())
        outs, leaves = reference_layer(g, dev["x"], T=T, H=1024, heads=16, kv=8, hd=hd, ffn=3072, total=total,
                                       leaves=leaves)
        if node_by_node:
            outs = outs + [n["val"] for n in g.order(*outs)]
        return g, outs, leaves

    g, outs, lv = build(False)
    assert [k for k, *_ in g.plan(*outs) if k != "nop"] == ["norm_mul", "qk_norm_rope_kv", "single",
                                                             "add_norm_mul", "silu_mul", "single"]
    g.compute(*outs)
    g2, outs2, lv2 = build(True)
    assert all(k in ("single", "nop") for k, *_ in g2.plan(*outs2))
    g2.compute(*outs2)
    for a, b in zip(outs, outs2):
        assert_bitexact(_np(a.t), _np(b.t))
    assert_bitexact(_np(lv["kcache"]), _np(lv2["kcache"]))
    assert_bitexact(_np(lv["vcache"]), _np(lv2["vcache"]))

    normed, _, _, qr, probs, mlp_in, act, out = [_np(v.t) for v in outs]
    kc, vc = _np(lv["kcache"]), _np(lv["vcache"])
    x, q, k = d["x"], d["q"], d["k"]
    assert_close(normed, R.run(lambda gr: R.rms_norm_w(gr, x, d["w_in"], eps, R.BF16)))
    q_ref, k_ref = R.run(lambda gr: R.qk_norm_rope(gr, q, k, d["wq"], d["wk"], eps, d["pos"], hd, theta, R.BF16,
                                                   cs_rounded=True))
    assert_bitexact(qr, q_ref)
    assert_bitexact(kc[filled:], k_ref)
    assert_bitexact(vc[filled:], d["v"])
    assert (kc[:filled] == 0).all() and (vc[:filled] == 0).all()
    p_ref = R.run(lambda gr: gr.soft_max_ext(d["scores"], None, np.float32(hd ** -0.5)))
    assert np.abs(probs.view(np.int32).astype(np.int64) - p_ref.view(np.int32).astype(np.int64)).max() <= 2
    s_ref, y_ref = R.run(lambda gr: R.add_rms_norm_w(gr, x, d["attn"], d["w_post"], eps, R.BF16))
    assert_bitexact(_np(outs[-1].node["srcs"][0].t), s_ref)
    assert_close(mlp_in, y_ref)
    assert_close(act, R.run(lambda gr: R.swiglu(gr, d["gate"], d["up"])))
    assert_bitexact(out, R.run(lambda gr: gr.add(s_ref, d["mlp"])))


def test_cont_of_permuted_views_graph(gpu):
    """ggml_cont(ggml_permute(x, 0, 2, 1, 3)) as a copy node (operations.cpp:
    123-125, 139): the contiguous result equals torch's permuted copy bit for
    bit, after q's rope run in the same list."""
    import torch
    rng = np.random.default_rng(SEED + 350)
    T, heads, hd = 37, 16, 128
    q = rng.standard_normal((T, heads, hd)).astype(np.float32)
    wq = rng.normal(1, 0.1, hd).astype(np.float32)
    pos = _positions(rng, T, 8192)
    g = gpu.Graph()
    qr = g.rope_ext(g.mul(g.rms_norm(_t(gpu, q), 1e-6), _t(gpu, wq)), _t(gpu, pos), hd, gpu.ROPE_TYPE_NEOX, 1e6)
    q_hd = g.cont(g.view(qr, qr.t.permute(1, 0, 2)))
    assert [k for k, *_ in g.plan(q_hd, qr) if k != "nop"] == ["norm_mul_rope", "single"]
    g.compute(q_hd, qr)
    assert q_hd.t.is_contiguous() and tuple(q_hd.t.shape) == (heads, T, hd)
    assert_bitexact(_np(q_hd.t), _np(qr.t.permute(1, 0, 2).contiguous()))


def test_reference_order_layers_chained(gpu):
    """Three decoder layers in one list, each layer's output add feeding the
    next layer's input norm (:147 -> :86): the add and the next norm are one
    launch that writes the sum, and the whole list is bit-identical to the
    same list run node by node."""
    from test_graph_plan import reference_layer
    rng = np.random.default_rng(SEED + 340)
    T, total, layers = 1, 38, 3

    def build(node_by_node, per):
        g = gpu.Graph()
        x, outs, caches = per[0][1]["x"], [], []
        for l in range(layers):
            d, dev, mk = per[l]
            leaves = dict(dev, **mk())
            o, leaves = reference_layer(g, x, T=T, H=1024, heads=16, kv=8, hd=128, ffn=3072, total=total,
                                        leaves=leaves)
            outs += o
            caches += [leaves["kcache"], leaves["vcache"]]
            x = o[-1]
        if node_by_node:
            outs = outs + [n["val"] for n in g.order(*outs)]
        return g, outs, caches

    per = [_reference_layer_leaves(gpu, rng, T, total) for _ in range(layers)]
    g, outs, caches = build(False, per)
    kinds = [k for k, *_ in g.plan(*outs) if k != "nop"]
    assert kinds == ["norm_mul"] + ["qk_norm_rope_kv", "single", "add_norm_mul", "silu_mul", "add_norm_mul"] * 2 + \
        ["qk_norm_rope_kv", "single", "add_norm_mul", "silu_mul", "single"]
    g.compute(*outs)
    g2, outs2, caches2 = build(True, per)
    g2.compute(*outs2)
    for a, b in zip(outs, outs2):
        assert_bitexact(_np(a.t), _np(b.t))
    for a, b in zip(caches, caches2):
        assert_bitexact(_np(a), _np(b))


@pytest.mark.parametrize("kind", ["plain", "guarded", "beta"])
def test_snake_family_graph(gpu, kind):
    """Kokoro Snake, the guarded Snake and SnakeBeta as their node lists: one
    fused run each, equal to the node-by-node run (sine marked as an output)
    bit for bit and to the restatement within the Snake bar (1e-5 of the
    closing add's operands)."""
    from test_graph_plan import snake_graph
    rng = np.random.default_rng(SEED + 400)
    T, C = 300, 256
    x = rng.standard_normal((T, C)).astype(np.float32)
    if kind == "beta":
        la = rng.uniform(-1, 1, C).astype(np.float32)
        lb = rng.uniform(-1, 1, C).astype(np.float32)
        alpha = (_t(gpu, la), _t(gpu, lb))
        ref = R.run(lambda g: R.snake_beta(g, x, la, lb))
    else:
        al = np.exp(rng.uniform(np.log(0.1), np.log(10.0), C)).astype(np.float32)
        alpha = _t(gpu, al.reshape(1, C, 1))
        ref = R.run(lambda g: (R.snake if kind == "plain" else R.snake_guarded)(g, x, al))
    g = gpu.Graph()
    y = snake_graph(g, _t(gpu, x), alpha, kind)
    assert [k for k, *_ in g.plan(y) if k != "nop"] == [{"plain": "snake", "guarded": "snake_guarded",
                                                          "beta": "snake_beta"}[kind]]
    fused = _np(g.compute(y).t)
    # the same list with the sine read outside: every node alone
    g2 = gpu.Graph()
    y2 = snake_graph(g2, _t(gpu, x), alpha, kind)
    sine = [v for v in _walk(y2) if v.node["op"] == gpu.NODE_SIN][0]
    assert all(k in ("single", "nop") for k, *_ in g2.plan(y2, sine))
    g2.compute(y2, sine)
    assert_bitexact(fused, _np(y2.t))
    assert_snake_close(fused, ref, x)


def _walk(v):
    out, stack, seen = [], [v], set()
    while stack:
        u = stack.pop()
        if u is None or u.node is None or id(u.node) in seen:
            continue
        seen.add(id(u.node))
        out.append(u)
        stack.extend(u.node["srcs"])
    return out


def test_gather_sum_graph(gpu):
    """sum_code_embeddings (code-predictor.cpp:82-107) as 16 get_rows over the
    column views of one codes tensor and 15 adds: one fused run, bit-exact; the
    list cut by an intermediate output runs as a 2-group run plus nodes, with
    the same bits."""
    import torch
    rng = np.random.default_rng(SEED + 500)
    groups, rows, ne0, frames = 16, 2048, 1024, 333
    tabs = [F.q8_0_synthetic(rng, rows, ne0) for _ in range(groups)]
    codes = rng.integers(0, rows, (groups, frames)).astype(np.int32)
    ref = R.run(lambda g: R.sum_code_embeddings(g, tabs, R.Q8_0, ne0, codes))
    dt = [gpu.Q8Tensor(_t(gpu, t), ne0) for t in tabs]
    dc = _t(gpu, codes)

    def build(cut):
        g = gpu.Graph()
        total, mid = None, None
        for t in range(groups):
            r = g.get_rows(dt[t], g.view(dc, dc[t]))
            total = r if total is None else g.add(total, r)
            if t == 1:
                mid = total
        return g, ([total, mid] if cut else [total])
    g, outs = build(False)
    assert [k for k, *_ in g.plan(*outs) if k != "nop"] == ["gather_sum"]
    g.compute(*outs)
    assert_bitexact(_np(outs[0].t), ref)
    g, outs = build(True)
    assert [k for k, *_ in g.plan(*outs) if k != "nop"] == ["gather_sum"] + ["single"] * 28
    g.compute(*outs)
    assert_bitexact(_np(outs[0].t), ref)
    torch.cuda.synchronize()


def test_vits_runs_graph(gpu):
    """The residual carry (waveform-decoder.cpp:150-158, the sum read by the
    next layer's add) and the branch average (:214-225): bit-exact."""
    rng = np.random.default_rng(SEED + 600)
    sh = (4096, 192)
    a, b, c, b0, b1, b2 = [rng.standard_normal(sh).astype(np.float32) for _ in range(6)]
    s_ref, y_ref = R.run(lambda g: R.add_leaky(g, a, b, 0.1))
    nxt_ref = R.run(lambda g: g.add(c, s_ref))
    cur_ref, avg_ref = R.run(lambda g: R.sum_scale_leaky(g, [b0, b1, b2], np.float32(1.0 / 3), 0.1))
    g = gpu.Graph()
    s = g.add(_t(gpu, a), _t(gpu, b))
    y = g.leaky_relu(s, 0.1)
    nxt = g.add(_t(gpu, c), s)
    summed = g.add(g.add(_t(gpu, b0), _t(gpu, b1)), _t(gpu, b2))
    avg = g.leaky_relu(g.scale(summed, np.float32(1.0 / 3)), 0.1)
    assert [k for k, *_ in g.plan(y, nxt, avg) if k != "nop"] == ["add_leaky", "single", "add_scale_leaky"]
    g.compute(y, nxt, avg)
    assert_bitexact(_np(y.t), y_ref)
    assert_bitexact(_np(s.t), s_ref)
    assert_bitexact(_np(nxt.t), nxt_ref)
    assert_bitexact(_np(avg.t), avg_ref)


def test_single_nodes_graph(gpu):
    """Nodes that run alone: rope, soft_max_ext with a causal mask, the
    single-tensor GLU, exp, and an unfused silu then mul (an up-projection
    between them in the reference's order)."""
    rng = np.random.default_rng(SEED + 700)
    x = rng.standard_normal((9, 4, 64)).astype(np.float32)
    pos = _positions(rng, 9, 1000)
    sc = rng.standard_normal((2, 9, 12)).astype(np.float32)
    mask = np.zeros((9, 12), np.float32)
    mask[np.triu_indices(9, 4, 12)] = -np.inf
    glu = rng.standard_normal((5, 96)).astype(np.float32)
    e = rng.uniform(-80, 80, (7, 33)).astype(np.float32)
    gate, up = rng.standard_normal((2, 7, 300)).astype(np.float32)
    g = gpu.Graph()
    r = g.rope_ext(_t(gpu, x), _t(gpu, pos), 64, gpu.ROPE_TYPE_NEOX, 1e4)
    p = g.soft_max_ext(_t(gpu, sc), _t(gpu, mask), 0.125)
    gl = g.glu_swiglu(_t(gpu, glu))
    ex = g.exp(_t(gpu, e))
    si = g.silu(_t(gpu, gate))
    between = g.add(_t(gpu, up), _t(gpu, up))  # stands for the up-projection
    mu = g.mul(si, between)
    outs = [r, p, gl, ex, mu]
    assert [k for k, *_ in g.plan(*outs) if k != "nop"] == ["single"] * 7
    g.compute(*outs)
    assert_bitexact(_np(r.t), R.run(lambda gr: gr.rope_neox(x, pos, 64, np.float32(1e4), cs_rounded=True)))
    assert_rope_close(_np(r.t), R.run(lambda gr: gr.rope_neox(x, pos, 64, np.float32(1e4))), 64)
    ref = R.run(lambda gr: gr.soft_max_ext(sc, mask, np.float32(0.125)))
    got = _np(p.t)
    assert np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64)).max() <= 2
    assert_close(_np(gl.t), R.run(lambda gr: gr.glu_swiglu(glu)))
    ref = R.run(lambda gr: gr.exp(e))
    assert np.abs(_np(ex.t).view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64)).max() <= 1
    assert_close(_np(mu.t), R.run(lambda gr: gr.mul(gr.silu(gate), gr.add(up, up))))


def test_executor_inside_a_captured_hip_graph(gpu):
    """A layer list run by shp_graph_compute inside a HIP graph capture: three
    replays, with eager work and a synchronisation between them and new inputs
    copied in before each, every replay bit-equal to the eager run of the same
    list on the same inputs."""
    import torch
    rng = np.random.default_rng(SEED + 800)
    T, hd = 3, 128
    d = _layer_inputs(rng, T)
    dev = {n: (_bf16(gpu, a) if n.startswith("w") else _t(gpu, a)) for n, a in d.items()}
    g = gpu.Graph()
    normed = g.mul(g.rms_norm(dev["x"], 1e-6), g.cast(dev["w_in"]))
    qr = g.rope_ext(g.mul(g.rms_norm(dev["q"], 1e-6), g.cast(dev["wq"])), dev["pos"], hd, gpu.ROPE_TYPE_NEOX, 1e6)
    after = g.add(dev["x"], dev["attn"])
    mlp_in = g.mul(g.rms_norm(after, 1e-6), g.cast(dev["w_post"]))
    outs = (normed, qr, mlp_in, after)
    arr, n, keep = g.nodes(*outs)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        g.compute(*outs)  # warm-up on the capture stream
        with torch.cuda.graph(graph, stream=stream):
            assert gpu.load().shp_graph_compute(arr, n, gpu._stream()) == gpu.OK
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for rep in range(3):
        new = {k: rng.standard_normal(dev[k].shape).astype(np.float32) for k in ("x", "q", "attn")}
        for k, a in new.items():
            dev[k].copy_(torch.from_numpy(a).cuda())
        junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [_np(v.t).copy() for v in outs]
        g.compute(*outs)  # eager, same list, same inputs
        want = [_np(v.t) for v in outs]
        for a, b in zip(got, want):
            assert_bitexact(a, b)
        assert bool(torch.isfinite(junk))


def test_codec_crop_bias_snake_beta_graph(gpu):
    """codec_causal_conv1d's tail and the next SnakeBeta (qwen3-tts/codec.cpp:
    64-71,100-104,184-199): the crop's copy of the GEMM output's first
    columns, the channel bias add (one launch that reads the view), then the
    SnakeBeta run. Bit-identical to the nodes one by one, and the biased crop
    bit-exact against the restatement."""
    rng = np.random.default_rng(SEED + 360)
    C, L, keep = 256, 1030, 1024
    wide = rng.standard_normal((L, C)).astype(np.float32)          # ggml [C, L]
    bias = rng.standard_normal(C).astype(np.float32)
    la = rng.uniform(-3, 3, C).astype(np.float32)
    lb = rng.uniform(-3, 3, C).astype(np.float32)
    tw, tb, tla, tlb = _t(gpu, wide), _t(gpu, bias), _t(gpu, la), _t(gpu, lb)

    def build(every):
        g = gpu.Graph()
        crop = g.cont(g.view(tw, tw[:keep]))
        biased = g.add(crop, tb)
        a = g.exp(g.view(tla, tla.reshape(1, -1)))
        b = g.exp(g.view(tlb, tlb.reshape(1, -1)))
        y = g.add(biased, g.div(g.sqr(g.sin(g.mul(biased, a))), g.scale_bias(b, 1.0, 1e-9)))
        outs = [biased, y]
        return g, outs, (outs + [n["val"] for n in g.order(*outs)]) if every else outs

    g, outs, every = build(False)
    assert [k for k, *_ in g.plan(*every) if k != "nop"] == ["view_binary", "snake_beta"]
    g.compute(*every)
    fused = [_np(o.t).copy() for o in outs]
    g, outs, every = build(True)
    assert "view_binary" not in [k for k, *_ in g.plan(*every)]
    g.compute(*every)
    for a, b in zip(fused, [_np(o.t) for o in outs]):
        assert_bitexact(a, b)
    ref = R.run(lambda og: og.add(wide[:keep], bias))
    assert_bitexact(fused[0], ref)


def test_codec_transpose_bias_graphs(gpu):
    """qwen3-tts/codec.cpp's channel-major tails as one launch each: the
    transposed convolution's crop, [1, C] bias and return (:179-181), and the
    depthwise convolution's return, crop and [C] bias (:134-140).
    Bit-identical to the nodes with every result written, and to the
    restatement."""
    rng = np.random.default_rng(SEED + 370)
    C, Lw, kept = 96, 2056, 2048
    wide = rng.standard_normal((C, Lw)).astype(np.float32)       # col2im's ggml [Lw, C]
    b1 = rng.standard_normal((C, 1)).astype(np.float32)          # ggml [1, C]
    mm = rng.standard_normal((C, Lw)).astype(np.float32)         # depthwise GEMM output ggml [Lw, C] (:133)
    b2 = rng.standard_normal(C).astype(np.float32)               # ggml [C]
    tw, tb1, tmm, tb2 = _t(gpu, wide), _t(gpu, b1), _t(gpu, mm), _t(gpu, b2)

    def build(every):
        g = gpu.Graph()
        crop = g.cont(g.view(tw, tw[:, :kept]))
        s1 = g.add(crop, tb1)
        y1 = g.cont(g.view(s1, s1.t.t()))                        # ggml [C, kept]
        cm = g.cont(g.view(tmm, tmm.t()))                        # channel-major ggml [C, Lw]
        crop2 = g.cont(g.view(cm, cm.t[:kept]))
        y2 = g.add(crop2, tb2)
        outs = [y1, y2]
        return g, outs, (outs + [n["val"] for n in g.order(*outs)]) if every else outs

    g, outs, every = build(False)
    assert [k for k, *_ in g.plan(*every) if k != "nop"] == ["cont_add_leaky", "cont_add_leaky"]
    g.compute(*every)
    fused = [_np(o.t).copy() for o in outs]
    g, outs, every = build(True)
    assert "cont_add_leaky" not in [k for k, *_ in g.plan(*every)]
    g.compute(*every)
    for a, b in zip(fused, [_np(o.t) for o in outs]):
        assert_bitexact(a, b)
    ref1 = R.run(lambda og: og.binbcast(R.OP_ADD, np.ascontiguousarray(wide[:, :kept]), b1))
    assert_bitexact(fused[0], np.ascontiguousarray(ref1.T))
    ref2 = R.run(lambda og: og.add(np.ascontiguousarray(mm.T[:kept]), b2))
    assert_bitexact(fused[1], ref2)

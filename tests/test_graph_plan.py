"""The node-run executor's planner on the CPU (include/synth_graph.h): which
runs it finds in node lists ordered as ggml_build_forward_expand orders the
reference's graphs, and when it must not fuse. Host code only: the tensors are
CPU tensors whose pointers are never dereferenced, and nothing is launched."""
import ctypes

import pytest
import torch

import qwen3_layer as Q
import synth_hip as S

F32 = torch.float32


def z(*shape, dtype=F32):
    return torch.zeros(shape, dtype=dtype)


def kinds(plan):
    return [k for k, _, _, _ in plan if k != "nop"]


def qwen3_layer(g, T=5, H=64, heads=4, kv=2, hd=16, ffn=96, cast=True, cache_rows=32):
    """The non-GEMM nodes of decoder_layer (src/arch/qwen3-tts/operations.cpp:
    80-147) with the GEMM outputs as leaves: returns the results a backend
    hands back to the GEMMs and the cache write."""
    wt = torch.bfloat16 if cast else F32
    x, attn, mlp = z(T, H), z(T, H), z(T, H)
    q, k = z(T, heads, hd), z(T, kv, hd)
    w_in, w_post, wq, wk = z(H, dtype=wt), z(H, dtype=wt), z(hd, dtype=wt), z(hd, dtype=wt)
    pos = z(T, dtype=torch.int32)
    cache = z(cache_rows, kv, hd)
    f = (lambda w: g.cast(w)) if cast else (lambda w: w)
    normed = g.mul(g.rms_norm(x, 1e-6), f(w_in))
    qr = g.rope_ext(g.mul(g.rms_norm(q, 1e-6), f(wq)), pos, hd, S.ROPE_TYPE_NEOX, 1e6)
    kr = g.rope_ext(g.mul(g.rms_norm(k, 1e-6), f(wk)), pos, hd, S.ROPE_TYPE_NEOX, 1e6)
    kc = g.cpy(kr, cache[3:3 + T])
    after = g.add(x, attn)
    mlp_in = g.mul(g.rms_norm(after, 1e-6), f(w_post))
    out = g.add(after, mlp)
    return kc, normed, qr, mlp_in, out


def test_qwen3_layer_runs():
    g = S.Graph()
    kc, normed, qr, mlp_in, out = qwen3_layer(g)
    plan = g.plan(kc, normed, qr, mlp_in, out)
    # expand order: the k path first (the cache write), then the input norm, q, the add+norm, the output add;
    # q's run is taken into k's launch across the input norm (which touches neither)
    assert kinds(plan) == ["qk_norm_rope", "norm_mul", "add_norm_mul", "single"]
    nodes = [n for k, _, _, n in plan if k != "nop"]
    assert nodes == [9, 3, 4, 1]
    g = S.Graph()
    res = qwen3_layer(g, cast=False)
    assert kinds(g.plan(*res)) == ["qk_norm_rope", "norm_mul", "add_norm_mul", "single"]
    assert [n for k, _, _, n in g.plan(*res) if k != "nop"] == [7, 2, 3, 1]


def reference_layer(g, x, T=1, H=64, heads=4, kv=2, hd=16, ffn=96, total=8, cast=True, leaves=None):
    """decoder_layer's non-GEMM nodes in expand order, small shapes by default
    (qwen3_layer.decoder_layer_nodes: the GEMM and attention-product outputs
    are leaves). Returns (outputs in expand order, leaves)."""
    return Q.decoder_layer_nodes(g, x, {} if leaves is None else leaves, T=T, H=H, heads=heads, kv=kv, hd=hd,
                                 ffn=ffn, total=total, cast=cast)


def test_reference_order_layer_is_five_launches():
    """The q run comes after k's and v's cache copies in expand order; the
    planner moves it up into k's launch with v's copy: input norm, one
    QK-norm+RoPE+KV launch, softmax, add+norm, SwiGLU, add."""
    g = S.Graph()
    outs, _ = reference_layer(g, z(1, 64))
    plan = g.plan(*outs)
    assert kinds(plan) == ["norm_mul", "qk_norm_rope_kv", "single", "add_norm_mul", "silu_mul", "single"]
    run = [r for r in plan if r[0] == "qk_norm_rope_kv"][0]
    assert run[3] == 5 + 1 + 4  # k's run with its copy, v's copy, q's run
    # the launch sits where k's run starts; the parts that followed it are gone from later windows
    order = g.order(*outs)
    assert order[run[1]]["op"] == S.NODE_RMS_NORM and order[run[2]]["op"] == S.NODE_ROPE
    # 28 chained layers (each layer's output add feeds the next input norm): 5 launches per layer, + the last add
    g = S.Graph()
    x, outs = z(1, 64), []
    for _ in range(28):
        o, _ = reference_layer(g, x)
        outs += o
        x = o[-1]
    assert kinds(g.plan(*outs)) == ["norm_mul"] + ["qk_norm_rope_kv", "single", "add_norm_mul", "silu_mul",
                                                   "add_norm_mul"] * 27 + \
        ["qk_norm_rope_kv", "single", "add_norm_mul", "silu_mul", "single"]


def test_cont_of_permuted_views():
    """ggml_cont of the attention's permute(0,2,1,3) views (operations.cpp:
    123-125, 139) keeps rows contiguous and runs as a copy; so does the
    transposing permute(1,0,2,3) (:136), whose ne[0] is strided, and the
    vocoder's ggml_cont(ggml_transpose(x)) (vits/operations.cpp:72); q's rope
    run still plans as its own launch before the copy. A view with no
    contiguous dimension, an F16 transposed view and a copy into a
    non-contiguous destination row stay unsupported."""
    g = S.Graph()
    q = z(5, 4, 16)  # ggml [16, 4, 5]
    qr = g.rope_ext(g.mul(g.rms_norm(q, 1e-6), z(16)), z(5, dtype=torch.int32), 16, S.ROPE_TYPE_NEOX, 1e6)
    q_hd = g.cont(g.view(qr, qr.t.permute(1, 0, 2)))  # ggml permute(q, 0, 2, 1, 3): [16, 5, 4]
    assert kinds(g.plan(q_hd)) == ["norm_mul_rope", "single"]
    v_hd = z(2, 7, 16)  # ggml [16, 7, 2]
    g = S.Graph()
    v_t = g.cont(g.view(v_hd, v_hd.permute(0, 2, 1)))  # ggml permute(v_hd, 1, 0, 2, 3): ne[0] strided
    assert kinds(g.plan(v_t)) == ["single"]
    x = z(512, 96)  # ggml [96, 512]
    g = S.Graph()
    assert kinds(g.plan(g.cont(g.view(x, x.t())))) == ["single"]
    g = S.Graph()
    assert kinds(g.plan(g.cont(g.view(x, x[:, ::2].t())))) == ["unsupported"]  # ggml nb [384, 8]: no dim contiguous
    h = z(64, 96, dtype=torch.float16)
    g = S.Graph()
    assert kinds(g.plan(g.cont(g.view(h, h.t())))) == ["unsupported"]
    g = S.Graph()
    assert kinds(g.plan(g.cpy(g.view(x, x.t()), z(96, 1024)[:, ::2]))) == ["unsupported"]


def test_sibling_runs_stay_apart_when_moving_one_up_is_visible():
    """A part that sits later is moved up only when nothing between reads
    what it writes, writes what it reads or writes, or produces its input."""
    hd, T = 16, 3
    pos, wq, wk = z(T, dtype=torch.int32), z(hd), z(hd)

    def runs(between, q_first=True, eps_k=1e-6, pos_k=None, kcache=None):
        g = S.Graph()
        q, k = z(T, 4, hd), z(T, 2, hd)
        kcache = z(8, 2, hd) if kcache is None else kcache
        qrun = lambda: g.rope_ext(g.mul(g.rms_norm(q, 1e-6), wq), pos, hd, S.ROPE_TYPE_NEOX, 1e6)
        krun = lambda: g.cpy(g.rope_ext(g.mul(g.rms_norm(k, eps_k), wk), pos if pos_k is None else pos_k, hd,
                                        S.ROPE_TYPE_NEOX, 1e6), kcache[5:])
        first = qrun() if q_first else krun()
        mid = between(g, q, k, kcache, first)
        second = krun() if q_first else qrun()
        return kinds(g.plan(first, mid, second))

    read_cache = lambda g, q, k, kc, first: g.add(kc, kc)
    # q first: k's cache write would move above a read of the cache
    assert runs(read_cache) == ["norm_mul_rope", "single", "norm_mul_rope"]
    # k first: q moves up over the read; the cache was written before it either way
    assert runs(read_cache, q_first=False) == ["qk_norm_rope", "single"]
    # a node between writes q's input: q cannot move up
    assert runs(lambda g, q, k, kc, first: g.cpy(z(T, 4, hd), q), q_first=False) == \
        ["norm_mul_rope", "single", "norm_mul_rope"]
    # a node between reads the first run's result: fine, the first run does not move
    assert runs(lambda g, q, k, kc, first: g.add(first, first)) == ["qk_norm_rope", "single"]
    # unrelated work between: fused
    assert runs(lambda g, q, k, kc, first: g.exp(z(4, 4))) == ["qk_norm_rope", "single"]
    # different eps or positions: two launches
    assert runs(lambda g, q, k, kc, first: g.exp(z(4, 4)), eps_k=1e-5) == \
        ["norm_mul_rope", "single", "norm_mul_rope"]
    assert runs(lambda g, q, k, kc, first: g.exp(z(4, 4)), pos_k=z(T, dtype=torch.int32)) == \
        ["norm_mul_rope", "single", "norm_mul_rope"]


def test_v_copy_joins_only_when_it_can_move_up():
    """v's cache copy joins the q/k launch unless a node between writes its
    source; the q/k part still fuses."""
    g = S.Graph()
    outs, d = reference_layer(g, z(1, 64))
    assert "qk_norm_rope_kv" in kinds(g.plan(*outs))
    # a cast into v's source placed between k's run and v's copy (a cast, so
    # that it cannot itself be taken as the F32 copy of v)
    g2 = S.Graph()
    hd, T = 16, 1
    q, k, v, pos = z(T, 4, hd), z(T, 2, hd), z(T, 2, hd), z(T, dtype=torch.int32)
    kcache, vcache = z(8, 2, hd), z(8, 2, hd)
    kc = g2.cpy(g2.rope_ext(g2.mul(g2.rms_norm(k, 1e-6), z(hd)), pos, hd, S.ROPE_TYPE_NEOX, 1e6), kcache[7:])
    clobber = g2.cpy(z(T, 2, hd, dtype=torch.float16), v)
    vc = g2.cpy(v, vcache[7:])
    qr = g2.rope_ext(g2.mul(g2.rms_norm(q, 1e-6), z(hd)), pos, hd, S.ROPE_TYPE_NEOX, 1e6)
    assert kinds(g2.plan(kc, clobber, vc, qr)) == ["qk_norm_rope", "single", "single"]


def test_a_read_in_a_later_split_keeps_a_result_written():
    """after_attention (operations.cpp:143) is read by the post-attention norm
    in this split and by the layer's output add after the MLP's GEMMs, in a
    later split: its ggml use count (2) exceeds the reads in the list (1), so
    the add+norm run writes the sum; the same holds for a skipped gain cast or
    norm, which then run as nodes."""
    g = S.Graph()
    x, attn, w = z(4, 64), z(4, 64), z(64)
    after = g.add(x, attn)
    mlp_in = g.mul(g.rms_norm(after, 1e-6), w)
    arr, n, _ = g.nodes(mlp_in)
    runs = (S.ShpGraphRun * 4)()
    count = ctypes.c_int32()
    L = S.load()
    assert L.shp_graph_plan(arr, n, runs, 4, ctypes.byref(count)) == S.OK
    assert [runs[i].kind for i in range(count.value)] == [4]  # add_norm_mul
    g = S.Graph()
    after = g.read_later(g.add(x, attn), 2)
    nrm = g.rms_norm(after, 1e-6)
    mlp_in = g.mul(nrm, w)
    assert kinds(g.plan(mlp_in)) == ["add_norm_mul"]
    g = S.Graph()
    nrm = g.read_later(g.rms_norm(x, 1e-6), 2)
    assert kinds(g.plan(g.mul(nrm, w))) == ["single", "single"]


def test_layer_output_add_fuses_into_the_next_input_norm():
    """:147 -> :86: the layer output add followed by the next layer's input
    norm is one add+norm run that writes the sum (the next residual)."""
    g = S.Graph()
    after, mlp, w = z(4, 64), z(4, 64), z(64, dtype=torch.bfloat16)
    out = g.add(after, mlp)
    nxt = g.mul(g.rms_norm(out, 1e-6), g.cast(w))
    resid = g.add(out, z(4, 64))
    assert kinds(g.plan(nxt, resid)) == ["add_norm_mul", "single"]


def test_swiglu_fuses_only_when_adjacent():
    g = S.Graph()
    gate, up = z(3, 96), z(3, 96)
    assert kinds(g.plan(g.mul(g.silu(gate), up))) == ["silu_mul"]
    g = S.Graph()
    assert kinds(g.plan(g.mul(up, g.silu(gate)))) == ["silu_mul"]
    g = S.Graph()
    s = g.silu(gate)
    other = g.add(s, up)  # the silu is read twice
    assert kinds(g.plan(g.mul(s, up), other)) == ["single", "single", "single"]


def snake_graph(g, x, alpha, kind):
    per = g.view(alpha, alpha.reshape(-1)) if kind != "beta" else None
    if kind == "plain":
        sq = g.sin(g.mul(x, per))
        return g.add(x, g.div(g.mul(sq, sq), per))
    if kind == "guarded":
        sq = g.sin(g.mul(x, per))
        return g.add(x, g.div(g.mul(sq, sq), g.scale_bias(per, 1.0, 1e-9)))
    la, lb = alpha
    # ggml_reshape_2d(alpha, ne0, 1) (codec.cpp:193-194): ggml [C, 1], torch (1, C)
    a = g.exp(g.view(la, la.reshape(1, -1)))
    b = g.exp(g.view(lb, lb.reshape(1, -1)))
    sq = g.sqr(g.sin(g.mul(x, a)))
    return g.add(x, g.div(sq, g.scale_bias(b, 1.0, 1e-9)))


@pytest.mark.parametrize("kind,run,n", [("plain", "snake", 5), ("guarded", "snake_guarded", 6),
                                        ("beta", "snake_beta", 8)])
def test_snake_family_runs(kind, run, n):
    """kokoro/operations.cpp:137-147, omnivoice/codec.cpp:51-68 and
    qwen3-tts/codec.cpp:184-200 in expand order (the curves' reshapes are view
    nodes inside the span)."""
    g = S.Graph()
    x = z(7, 32)
    alpha = (z(32), z(32)) if kind == "beta" else z(1, 32, 1)
    plan = g.plan(snake_graph(g, x, alpha, kind))
    assert kinds(plan) == [run]
    assert [p[3] for p in plan if p[0] == run] == [n]


def test_snake_not_fused_when_an_intermediate_is_read_elsewhere():
    g = S.Graph()
    x, alpha = z(7, 32), z(32)
    t = g.mul(x, alpha)
    sn = g.sin(t)
    y = g.add(x, g.div(g.mul(sn, sn), alpha))
    assert kinds(g.plan(y, sn)) == ["single"] * 5  # the sine is a graph output
    g = S.Graph()
    t = g.mul(x, alpha)
    sn = g.sin(t)
    y = g.add(x, g.div(g.mul(sn, sn), z(32)))  # another tensor as the divisor
    assert kinds(g.plan(y)) == ["single"] * 5
    g = S.Graph()
    sn = g.sin(g.mul(x, alpha))
    y = g.add(x, g.div(g.mul(sn, sn), g.scale_bias(alpha, 1.0, 1e-8)))  # not Snake1d's guard
    assert kinds(g.plan(y)) == ["single"] * 6


def test_gather_sum_runs():
    """code-predictor.cpp:82-107: one view per group column of codes, a get_rows
    per group, added in group order."""
    groups, frames = 16, 9
    tables = [S.Q8Tensor(z(64, 2 * 34, dtype=torch.uint8), 64) for _ in range(groups)]
    codes = z(groups, frames, dtype=torch.int32)
    g = S.Graph()
    total = None
    for t in range(groups):
        rows = g.get_rows(tables[t], g.view(codes, codes[t]))
        total = rows if total is None else g.add(total, rows)
    plan = g.plan(total)
    assert kinds(plan) == ["gather_sum"]
    assert [p[3] for p in plan if p[0] == "gather_sum"] == [2 * groups - 1]
    # ids from two separate tensors are not columns of one codes tensor
    other = z(groups, frames, dtype=torch.int32)
    g = S.Graph()
    r0 = g.get_rows(tables[0], codes[0])
    r1 = g.get_rows(tables[1], other[1])
    assert kinds(g.plan(g.add(r0, r1))) == ["single"] * 3
    # an intermediate sum read elsewhere stops the run after it
    g = S.Graph()
    acc = g.get_rows(tables[0], codes[0])
    acc = g.add(acc, g.get_rows(tables[1], codes[1]))
    mid = acc
    acc = g.add(acc, g.get_rows(tables[2], codes[2]))
    assert kinds(g.plan(acc, mid)) == ["gather_sum", "single", "single"]


def test_vits_residual_and_branch_average_runs():
    """waveform-decoder.cpp:150-158 (the add's sum is the next residual) and
    :214-225 (the last branch add, the scale by 1/n, the stage's leaky)."""
    g = S.Graph()
    a, b = z(16, 8), z(16, 8)
    s = g.add(a, b)
    y = g.leaky_relu(s, 0.1)
    nxt = g.add(z(16, 8), s)
    assert kinds(g.plan(y, nxt)) == ["add_leaky", "single"]
    g = S.Graph()
    b0, b1, b2 = z(16, 8), z(16, 8), z(16, 8)
    summed = g.add(g.add(b0, b1), b2)
    y = g.leaky_relu(g.scale(summed, 1.0 / 3), 0.1)
    plan = g.plan(y)
    assert kinds(plan) == ["add_scale_leaky"]
    assert [p[3] for p in plan if p[0] != "nop"] == [4]


def test_singles_and_support():
    g = S.Graph()
    x = z(4, 2, 8)
    pos = z(4, dtype=torch.int32)
    outs = [g.rope_ext(x, pos, 8, S.ROPE_TYPE_NEOX, 1e4), g.soft_max_ext(z(3, 5), None, 0.5),
            g.glu_swiglu(z(3, 8)), g.exp(z(3, 4)), g.cast(z(8, dtype=torch.float16))]
    assert kinds(g.plan(*outs)) == ["single"] * 5
    g = S.Graph()
    normal = g.rope_ext(x, pos, 8, 0, 1e4)  # GPT-J pairing: not here
    assert kinds(g.plan(normal)) == ["unsupported"]
    arr, n, _ = g.nodes(normal)
    assert S.load().shp_graph_node_supported(ctypes.byref(arr[0])) == 0
    assert S.load().shp_graph_compute(arr, n, None) == S.ERR_UNSUPPORTED  # nothing launched
    g = S.Graph()
    alibi = g.soft_max_ext(z(3, 5), None, 0.5, max_bias=8.0)
    assert kinds(g.plan(alibi)) == ["unsupported"]
    g = S.Graph()
    empty = g.exp(z(0, 4))  # no rows: ggml keeps the node (a no-op there)
    assert kinds(g.plan(empty)) == ["unsupported"]
    arr, n, _ = g.nodes(empty)
    assert S.load().shp_graph_node_supported(ctypes.byref(arr[n - 1])) == 0


def test_support_is_the_entry_points_own_answer():
    """supports_op (shp_graph_node_supported) runs the node's entry point with
    its argument checks only, so a node the structural checks pass but the
    entry point refuses is reported unsupported and planned as such: a batched
    get_rows whose ids batch (ne[1]) differs from the table's ne[2], and a
    softmax mask whose head count does not divide the scores' (ggml broadcasts
    masks by whole repeats). The well-formed neighbours stay supported, and the
    same operands through the entry points give the same statuses."""
    L = S.load()

    def support(g, v):
        arr, n, _ = g.nodes(v)
        return L.shp_graph_node_supported(ctypes.byref(arr[n - 1]))

    g = S.Graph()
    table, ids_bad, ids_ok = z(2, 10, 8), z(3, 4, dtype=torch.int32), z(2, 4, dtype=torch.int32)
    bad, ok = g.get_rows(table, ids_bad), g.get_rows(table, ids_ok)
    bad.t = z(3, 4, 8)
    ok.t = z(2, 4, 8)
    assert (support(g, bad), support(g, ok)) == (0, 1)
    assert kinds(g.plan(bad)) == ["unsupported"] and kinds(g.plan(ok)) == ["single"]
    r = ctypes.byref
    assert L.shp_get_rows(r(S.desc(table)), r(S.desc(ids_bad)), r(S.desc(z(3, 4, 8))), None) == S.ERR_INVALID_ARG

    g = S.Graph()
    scores = z(1, 3, 2, 5)  # ggml [5, 2, 3, 1]: 3 heads
    sm_bad = g.soft_max_ext(scores, z(2, 2, 5), 0.5)  # 2 mask heads do not divide 3
    sm_ok = g.soft_max_ext(scores, z(1, 2, 5), 0.5)
    assert (support(g, sm_bad), support(g, sm_ok)) == (0, 1)
    assert kinds(g.plan(sm_bad)) == ["unsupported"] and kinds(g.plan(sm_ok)) == ["single"]
    assert L.shp_soft_max_ext(r(S.desc(scores)), r(S.desc(z(2, 2, 5))), ctypes.c_float(0.5), ctypes.c_float(0.0),
                              r(S.desc(z(1, 3, 2, 5))), None) == S.ERR_INVALID_ARG


def test_malformed_lists_are_rejected():
    g = S.Graph()
    y = g.add(g.add(z(4, 8), z(4, 8)), z(4, 8))
    arr, n, _ = g.nodes(y)
    count = ctypes.c_int32()
    L = S.load()
    assert L.shp_graph_plan(arr, n, None, 0, ctypes.byref(count)) == S.OK and count.value == 2
    arr[1].src_node[0] = 1  # not an earlier node
    assert L.shp_graph_plan(arr, n, None, 0, ctypes.byref(count)) == S.ERR_INVALID_ARG
    arr[1].src_node[0] = 0
    arr[0].uses = -1
    assert L.shp_graph_compute(arr, n, None) == S.ERR_INVALID_ARG
    arr[0].uses = 1  # read once by the list: consistent
    assert L.shp_graph_plan(arr, n, None, 0, ctypes.byref(count)) == S.OK
    arr[0].uses = 0
    g2 = S.Graph()
    s = g2.add(z(4, 8), z(4, 8))
    y2 = g2.mul(s, s)
    arr2, n2, _ = g2.nodes(y2)
    arr2[0].uses = 1  # below the two reads the list makes
    assert L.shp_graph_plan(arr2, n2, None, 0, ctypes.byref(count)) == S.ERR_INVALID_ARG
    arr[1].op = 99
    assert L.shp_graph_plan(arr, n, None, 0, ctypes.byref(count)) == S.ERR_INVALID_ARG
    arr[1].op = S.NODE_ADD
    runs = (S.ShpGraphRun * 1)()
    assert L.shp_graph_plan(arr, n, runs, 1, ctypes.byref(count)) == S.ERR_INVALID_ARG  # capacity
    assert L.shp_graph_plan(arr, 0, None, 0, ctypes.byref(count)) == S.OK and count.value == 0


def test_repeated_operands_follow_ggml():
    """A single add/mul/div takes every b that repeats to a's shape
    (ggml_can_repeat), such as the time-major vocoder's [1, C] bias
    (vits/waveform-decoder.cpp:120); a shape that does not repeat is
    unsupported. A fused run takes only the forms it computes: a gain or a
    Snake curve of n values is fused only as [n, 1, 1, 1]; as [1, n] ggml
    repeats it as one value per row, so the nodes run alone."""
    T, C = 64, 16
    x = z(C, T)  # ggml [T, C], time-major
    for b in (z(C, 1), z(1, 1), z(C, T // 2), z(1, T), z(2, T)):
        g = S.Graph()
        assert kinds(g.plan(g.add(x, b))) == (["single"] if C % b.shape[0] == 0 else ["unsupported"]), b.shape
    g = S.Graph()
    assert kinds(g.plan(g.mul(x, z(3, 1)))) == ["unsupported"]  # 16 rows do not repeat 3
    # norm -> mul with the gain as ggml [1, n]: not the fused form
    h = z(4, 32)
    g = S.Graph()
    assert kinds(g.plan(g.mul(g.rms_norm(h, 1e-6), z(32)))) == ["norm_mul"]
    g = S.Graph()
    assert "norm_mul" not in kinds(g.plan(g.mul(g.rms_norm(h, 1e-6), z(32, 1))))
    # SnakeBeta with its curves as ggml [1, C]
    g = S.Graph()
    xs = z(32, 32)
    la, lb = z(32), z(32)
    a = g.exp(g.view(la, la.reshape(-1, 1)))
    bb = g.exp(g.view(lb, lb.reshape(-1, 1)))
    sq = g.sqr(g.sin(g.mul(xs, a)))
    assert "snake_beta" not in kinds(g.plan(g.add(xs, g.div(sq, g.scale_bias(bb, 1.0, 1e-9)))))


def _conv_tail(g, T=64, C=16, residual=None, leaky=True, extra_read=None):
    """conv1d_time_major's tail (vits/waveform-decoder.cpp:111,118-121) and
    what follows it: the transposing copy of the GEMM output [C, T], the
    [1, C] bias add, optionally the residual add (:150) and the next
    leaky-ReLU (:146)."""
    out = z(T, C)                       # ggml [C, T] (the GEMM's output)
    tm = g.cont(g.view(out, out.t()))   # ggml [T, C]
    s = g.add(tm, z(C, 1))              # + ggml [1, C]
    if residual is not None:
        s = g.add(s, residual)
    y = g.leaky_relu(s, 0.1) if leaky else s
    return tm, s, y


def test_conv_tail_runs():
    """The copy, the bias add, the residual add and the leaky-ReLU run as one
    shp_cont_add_leaky_relu launch in each form the decoder emits; the
    copy's result must be read by the bias add alone."""
    T, C = 64, 16
    for resid, leaky, n in ((False, True, 3), (True, True, 4), (True, False, 3), (False, False, 2)):
        g = S.Graph()
        r = z(C, T) if resid else None
        tm, s, y = _conv_tail(g, T, C, r, leaky)
        plan = g.plan(y)
        assert kinds(plan) == ["cont_add_leaky"], (resid, leaky, kinds(plan))
        assert [p[3] for p in plan if p[0] == "cont_add_leaky"] == [n]
    # the sum read later (the next layer's residual): still one launch
    g = S.Graph()
    tm, s, y = _conv_tail(g, T, C, z(C, T), True)
    assert kinds(g.plan(y, g.add(s, s))) == ["cont_add_leaky", "single"]
    # the copy read elsewhere: it must be written, so the nodes run alone
    g = S.Graph()
    tm, s, y = _conv_tail(g, T, C, None, True)
    assert kinds(g.plan(y, g.exp(tm))) == ["single", "single", "single", "single"]
    # a plain (untransposed) copy is not this run
    g = S.Graph()
    x = z(C, T)
    assert "cont_add_leaky" not in kinds(g.plan(g.leaky_relu(g.add(g.cont(x), z(C, 1)), 0.1)))
    # a bias that is one row [T] repeated over the rows: the same run
    g = S.Graph()
    out = z(T, C)
    tm = g.cont(g.view(out, out.t()))
    assert kinds(g.plan(g.leaky_relu(g.add(tm, z(T)), 0.1))) == ["cont_add_leaky"]
    # a bias that tiles along the row ([T/2]): the nodes alone
    g = S.Graph()
    tm = g.cont(g.view(out, out.t()))
    assert "cont_add_leaky" not in kinds(g.plan(g.leaky_relu(g.add(tm, z(T // 2)), 0.1)))
    # one channel: the transpose of [1, T] has ne[0] contiguous, so its copy is
    # a plain copy of a row-contiguous view, which the bias add reads in place
    g = S.Graph()
    out1 = z(T, 1)
    tm = g.cont(g.view(out1, out1.t()))
    assert kinds(g.plan(g.leaky_relu(g.add(tm, z(1, 1)), 0.1))) == ["view_binary", "single"]


def test_view_copy_then_binary():
    """keep_prefix's copy of a row-contiguous view, then the channel bias
    (qwen3-tts/codec.cpp:64-71,100-104): the add reads the view, one launch;
    kept apart when the copy is read elsewhere, when it is a cast, when the
    add's result would overlap the view, or for a transposed view (that is
    the conv-tail run's)."""
    C, L, keep = 32, 70, 64
    wide = z(L, C)                                  # ggml [C, L]
    view = wide[:keep]                              # the first `keep` columns
    g = S.Graph()
    crop = g.cont(g.view(wide, view))
    assert kinds(g.plan(g.add(crop, z(C)))) == ["view_binary"]
    g = S.Graph()
    crop = g.cont(g.view(wide, view))
    assert kinds(g.plan(g.mul(crop, z(keep, C)))) == ["view_binary"]
    g = S.Graph()
    crop = g.cont(g.view(wide, view))
    assert kinds(g.plan(g.add(crop, z(C)), g.exp(crop))) == ["single", "single", "single"]
    h = z(L, C, dtype=torch.float16)
    g = S.Graph()
    crop = g.cont(g.view(h, h[:keep]))
    assert kinds(g.plan(g.add(crop, z(C)))) == ["single", "single"]
    # the add's result placed over the view's own memory (shifted one row): apart
    g = S.Graph()
    crop = g.cont(g.view(wide, view))
    added = g._op(S.NODE_ADD, wide[1:keep + 1], [crop, z(C)])
    assert kinds(g.plan(added)) == ["single", "single"]


def test_cont_then_im2col():
    """The codec's causal convolution (qwen3-tts/codec.cpp:94-96): the
    time-major copy of a channel-major activation, then its im2col, one launch
    reading the activation through the transposed view, for F32 and F16
    columns. Kept apart: the depthwise form (each channel a batch entry,
    :124-129), the copy read elsewhere, a plain copy, and columns placed over
    the activation."""
    C, T, OC, K, d = 64, 300, 32, 3, 2
    x = z(T, C)                                     # ggml [C, T], channels fastest
    w = z(OC, C, K)                                 # ggml [K, C, OC]
    g = S.Graph()
    tm = g.cont(g.view(x, x.t()))
    plan = g.plan(g.im2col(w, tm, 1, (K - 1) * d, d))
    assert kinds(plan) == ["cont_im2col"] and plan[-1][3] == 2
    g = S.Graph()
    tm = g.cont(g.view(x, x.t()))
    assert kinds(g.plan(g.im2col(w, tm, 1, 2, 1, dtype=torch.float16))) == ["cont_im2col"]
    # depthwise: [T, 1, C] batches; the view would be batch-contiguous
    g = S.Graph()
    tm = g.cont(g.view(x, x.t()))
    batched = g.view(tm, tm.t.view(C, 1, T))
    assert kinds(g.plan(g.im2col(z(C, 1, 7), batched, 1, 6, 1))) == ["single", "single"]
    # the copy read elsewhere must be written
    g = S.Graph()
    tm = g.cont(g.view(x, x.t()))
    assert kinds(g.plan(g.im2col(w, tm, 1, 2, 1), g.exp(tm))) == ["single", "single", "single"]
    # a plain (time-contiguous) copy is not this run
    g = S.Graph()
    tm = g.cont(z(C, T))
    assert kinds(g.plan(g.im2col(w, tm, 1, 2, 1))) == ["single", "single"]
    # columns over the activation's memory: apart
    big = z(T * C * K + T * C)
    xs = big[:T * C].view(T, C)
    g = S.Graph()
    tm = g.cont(g.view(xs, xs.t()))
    cols = g._op(S.NODE_IM2COL, big[:T * C * K].view(1, T, C * K), [w, tm], ints={0: 1, 2: 1, 4: 1})
    assert "cont_im2col" not in kinds(g.plan(cols))


def test_im2col_node_forms():
    """supports_op for IM2COL: the 1-D form only (is_2D 0, p1 0), F32 input,
    F32 or F16 columns of the shape ggml_im2col gives."""
    w, x = z(8, 4, 3), z(4, 50)
    g = S.Graph()
    ok = g.im2col(w, x, 1, 1, 1)
    arr, n, keep = g.nodes(ok)
    assert S.load().shp_graph_node_supported(ctypes.byref(arr[0])) == 1
    for k, v in ((6, 1), (3, 1)):  # is_2D, p1
        arr[0].op_params[k] = v
        assert S.load().shp_graph_node_supported(ctypes.byref(arr[0])) == 0
        arr[0].op_params[k] = 0
    g = S.Graph()
    bad = g._op(S.NODE_IM2COL, z(1, 49, 12), [w, x], ints={0: 1, 2: 1, 4: 1})  # OW is 50
    arr, n, keep = g.nodes(bad)
    assert S.load().shp_graph_node_supported(ctypes.byref(arr[0])) == 0


def test_runs_keep_outputs_apart_from_inputs():
    """A fused run reads its inputs while it writes its outputs, so an output
    the allocator placed over an input at another offset keeps the nodes
    apart; the output written exactly over its input (in place) is fused."""
    big = z(9, 64)
    x = big[:8]
    w = z(64)
    g = S.Graph()
    nrm = g.rms_norm(x, 1e-6)
    y = g._op(S.NODE_MUL, big[1:9], [nrm, w])      # over x, one row on
    assert kinds(g.plan(y)) == ["single", "single"]
    g = S.Graph()
    nrm = g.rms_norm(x, 1e-6)
    y = g._op(S.NODE_MUL, x, [nrm, w])              # exactly over x
    assert kinds(g.plan(y)) == ["norm_mul"]
    # add -> leaky with the leaky result over b shifted
    a, b2 = z(8, 64), z(9, 64)
    g = S.Graph()
    s_ = g.add(a, b2[:8])
    y = g._op(S.NODE_LEAKY_RELU, b2[1:9], [s_], floats={0: 0.1})
    assert kinds(g.plan(y)) == ["single", "single"]


def test_codec_transpose_bias_runs():
    """The channel-major convolutions' tails in qwen3-tts/codec.cpp as one
    transposing launch: the transposed convolution's crop, [1, C] bias and
    return (:179-181), with or without the crop's copy; the depthwise
    convolution's return, crop and [C] bias (:134-140). A transpose read
    elsewhere, or a bias of another shape, keeps the nodes apart."""
    C, Lw, kept = 32, 80, 64
    wide = z(C, Lw)                                 # ggml [Lw, C]: col2im's [out_length, out_channels]
    g = S.Graph()
    crop = g.cont(g.view(wide, wide[:, :kept]))     # ggml [kept, C]
    s_ = g.add(crop, z(C, 1))                       # + ggml [1, C]
    y = g.cont(g.view(s_, s_.t.t()))                # ggml [C, kept]
    plan = g.plan(y)
    assert kinds(plan) == ["cont_add_leaky"] and [p[3] for p in plan if p[0] != "nop"] == [3]
    g = S.Graph()
    x = z(C, kept)
    s_ = g.add(x, z(C, 1))
    y = g.cont(g.view(s_, s_.t.t()))
    assert kinds(g.plan(y)) == ["cont_add_leaky"]
    g = S.Graph()
    s_ = g.add(x, z(C, 1))
    y = g.cont(g.view(s_, s_.t.t()))
    assert kinds(g.plan(y, g.exp(s_))) == ["single", "single", "single"]   # the sum read elsewhere
    # depthwise: GEMM output ggml [out_length, C] -> channel-major, first `kept` rows, + bias [C]
    mm = z(C, Lw)
    g = S.Graph()
    cm = g.cont(g.view(mm, mm.t()))                 # ggml [C, Lw]
    crop = g.cont(g.view(cm, cm.t[:kept]))          # ggml [C, kept]
    y = g.add(crop, z(C))
    plan = g.plan(y)
    assert kinds(plan) == ["cont_add_leaky"] and [p[3] for p in plan if p[0] != "nop"] == [3]
    g = S.Graph()
    cm = g.cont(g.view(mm, mm.t()))
    crop = g.cont(g.view(cm, cm.t[:kept]))
    assert "cont_add_leaky" not in kinds(g.plan(g.add(crop, z(kept, 1)), g.exp(cm)))


def test_concat_node():
    """ggml_concat as a single node (src/arch/qwen3-tts/model.cpp:1450: the
    talker's hidden state and the code embedding as one two-position block)."""
    g = S.Graph()
    assert kinds(g.plan(g.concat(z(1, 1024), z(1, 1024), 1))) == ["single"]
    g = S.Graph()
    assert kinds(g.plan(g.concat(z(3, 8), z(3, 5), 0))) == ["single"]
    g = S.Graph()
    h = z(3, 8, dtype=torch.float16)
    assert kinds(g.plan(g.concat(h, h, 1))) == ["unsupported"]


def test_codec_activation_nodes():
    """ggml_sub, tanh, sigmoid, elu, gelu_erf, clamp and norm run as single
    nodes (qwen3-tts/codec.cpp:216-222,481, vits/waveform-decoder.cpp:228,
    kokoro/operations.cpp:12,133)."""
    x = z(8, 64)
    for build in (lambda g: g.sub(x, z(64)), lambda g: g.tanh(x), lambda g: g.sigmoid(x), lambda g: g.elu(x),
                  lambda g: g.gelu_erf(x), lambda g: g.clamp(x, -1.0, 1.0), lambda g: g.norm(x, 1e-6)):
        g = S.Graph()
        assert kinds(g.plan(build(g))) == ["single"]
    g = S.Graph()
    assert kinds(g.plan(g.norm(x, -1.0))) == ["unsupported"]


def test_acc_node_forms():
    """supports_op for ACC is the entry point's own answer: a row window at a
    row offset and ggml's inplace form are taken; overlapping rows, a view
    past a's end and an offset inside an element are not."""
    a, b = z(10, 8), z(4, 8)
    for params, ok in (((32, 128, 128, 3 * 32), 1), ((16, 128, 128, 0), 0), ((32, 128, 128, 7 * 32), 0),
                       ((32, 128, 128, 2), 0)):
        g = S.Graph()
        y = g.acc(a, b, *params)
        arr, n, keep = g.nodes(y)
        assert S.load().shp_graph_node_supported(ctypes.byref(arr[0])) == ok, params
    g = S.Graph()
    y = g.acc(a, b, 32, 128, 128, 32, inplace=True)
    assert kinds(g.plan(y)) == ["single"]
    assert y.t.data_ptr() == a.data_ptr()


def test_talker_prefill_accumulation_plans_as_singles():
    """talker.cpp:86-118 with the x-vector in the middle of the codec run:
    get_rows, then three ggml_acc over views of its result, then the ICL
    block's: one launch each."""
    H, n, N = 64, 5, 8
    text, table, ids, sp, ac = z(N, H), z(30, H), z(n, dtype=torch.int32), z(H), z(3, H)
    g = S.Graph()
    codec = g.get_rows(table, ids)
    nb1, nb2 = 4 * H, 4 * H * N
    out = g.acc(text, g.view(codec, codec.t[:2]), nb1, nb2, nb2, 3 * nb1)
    out = g.acc(out, g.view(sp, sp.view(1, H)), nb1, nb2, nb2, 5 * nb1)
    out = g.acc(out, g.view(codec, codec.t[3:]), nb1, nb2, nb2, 6 * nb1)
    out = g.acc(out, ac, nb1, nb2, nb2, 5 * nb1)
    assert [k for k in kinds(g.plan(out)) if k != "nop"] == ["single"] * 5


def test_row_sum_nodes_and_the_weighted_sum_run():
    """SUM_ROWS and MEAN take [1, ne1, ne2, ne3] results; MUL then SUM_ROWS of
    the product is one launch unless the product is read elsewhere."""
    x, w = z(6, 40), z(6, 40)
    g = S.Graph()
    s = g.sum_rows(g.mul(x, w))
    assert kinds(g.plan(s)) == ["mul_sum_rows"]
    g = S.Graph()
    p = g.mul(x, w)
    s = g.sum_rows(p)
    assert kinds(g.plan(s, p)) == ["single", "single"]
    g = S.Graph()
    bad = g._op(S.NODE_MEAN, z(6, 2), [x])
    arr, n, keep = g.nodes(bad)
    assert S.load().shp_graph_node_supported(ctypes.byref(arr[0])) == 0
    g = S.Graph()
    y = g.sqrt(g.relu(g.neg(g.step(x))))
    assert kinds(g.plan(y)) == ["single"] * 4


def test_causal_soft_max_run():
    """DIAG_MASK_INF then a maskless SOFT_MAX is one launch; not with a mask
    tensor, a zero scale, or the masked scores read elsewhere."""
    x = z(4, 16, 16)
    g = S.Graph()
    p = g.soft_max_ext(g.diag_mask_inf(x, 0), None, 0.125)
    assert kinds(g.plan(p)) == ["diag_mask_soft_max"]
    g = S.Graph()
    p = g.soft_max_ext(g.diag_mask_inf(x, 0), None, 0.0)
    assert kinds(g.plan(p)) == ["single", "single"]
    g = S.Graph()
    m = g.diag_mask_inf(x, 0)
    p = g.soft_max_ext(m, None, 0.125)
    assert kinds(g.plan(p, m)) == ["single", "single"]
    g = S.Graph()
    p = g.soft_max_ext(g.diag_mask_inf(x, 0), z(16, 16), 0.125)
    assert kinds(g.plan(p)) == ["single", "single"]


def test_mel_filterbank_is_the_restatement():
    """shp_mel_filterbank (host code of the library) against the oracle's
    restated Slaney filterbank, bit for bit, at the production parameters
    and another rate, window and band."""
    import numpy as np
    import ggml_ref as R
    for args in ((24000, 1024, 128, 0.0, 12000.0), (16000, 512, 80, 20.0, 7600.0), (24000, 2048, 64, 50.0, 8000.0)):
        a, b = S.mel_filterbank(*args), R.mel_filterbank(*args)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), args
    with pytest.raises(S.ShpError):
        S.mel_filterbank(24000, 1, 128, 0.0, 12000.0)

"""Seeded random node lists for the executor's q/k/v launch (include/synth_graph.h):
an attention block's q and k rope runs (src/arch/qwen3-tts/operations.cpp:
98-104) and the k and v cache copies (:109-116), in a random order, among
nodes that touch the same memory or not:
  - a read of the whole k or v cache (the attention's ggml_cont of the cache
    view, :121-123, stands here as an add of the view to itself);
  - a cast written into the whole k or v cache;
  - a cast written into q's or v's input tensor (a node between that changes
    what the moved part reads);
  - a read of q's rotated output (what the scores' permute/cont does, :120);
  - unrelated work (an exp of another tensor).
The executor may move a later part up into the first part's launch only
where that is invisible. Each list runs twice from the same starting memory:
once as planned, once with every node's result marked as an output (so every
node runs alone, in list order, as ggml-CPU runs them). Every output, both
caches and every input the list writes must be bit-identical between the two.
"""
import numpy as np
import pytest

import formats as F
from test_gpu_parity import _np, _t, assert_bitexact

pytestmark = pytest.mark.gpu
SEED = 20260728
CASES = 64


def _case(gpu, seed):
    """(build(outputs_all) -> (graph, outputs, written tensors), restore())"""
    import torch
    rng = np.random.default_rng(SEED + 9000 + seed)
    T = int(rng.choice([1, 3, 8]))
    heads, kv, hd, cap = 4, 2, 128, 16
    filled = int(rng.integers(0, cap - T + 1))
    cast = bool(rng.integers(0, 2))
    host = {"q": rng.standard_normal((T, heads, hd)), "k": rng.standard_normal((T, kv, hd)),
            "v": rng.standard_normal((T, kv, hd)), "kc": rng.standard_normal((cap, kv, hd)),
            "vc": rng.standard_normal((cap, kv, hd)), "a": rng.standard_normal((T, 64)),
            "qf16": rng.standard_normal((T, heads, hd)), "vf16": rng.standard_normal((T, kv, hd)),
            "kcf16": rng.standard_normal((cap, kv, hd)), "vcf16": rng.standard_normal((cap, kv, hd))}
    host = {n: a.astype(np.float32) for n, a in host.items()}
    wq = rng.normal(1, 0.1, hd).astype(np.float32)
    wk = rng.normal(1, 0.1, hd).astype(np.float32)
    pos = rng.integers(0, 4096, T).astype(np.int32)
    dev = {n: _t(gpu, a) for n, a in host.items()}
    dev["qf16"] = dev["qf16"].to(torch.float16)
    for n in ("vf16", "kcf16", "vcf16"):
        dev[n] = dev[n].to(torch.float16)
    if cast:
        dev["wq"] = torch.from_numpy(F.f32_to_bf16_bits(wq).view(np.int16)).cuda().view(torch.bfloat16)
        dev["wk"] = torch.from_numpy(F.f32_to_bf16_bits(wk).view(np.int16)).cuda().view(torch.bfloat16)
    else:
        dev["wq"], dev["wk"] = _t(gpu, wq), _t(gpu, wk)
    dev["pos"] = _t(gpu, pos)

    # the parts, each a list of items; an item builds its nodes and returns its results
    parts = ["q", "k", "v"]
    extras = list(rng.choice(["read_cache", "read_vcache", "write_kcache", "write_vcache", "clobber_q", "clobber_v",
                              "read_q", "unrelated"], size=int(rng.integers(0, 4))))
    order = parts + extras
    rng.shuffle(order)

    def restore():
        for n in ("q", "k", "v", "kc", "vc", "a"):
            dev[n].copy_(torch.from_numpy(host[n]).cuda())
        torch.cuda.synchronize()

    def build(all_outputs):
        g = gpu.Graph()
        w = (lambda x: g.cast(x)) if cast else (lambda x: x)
        outs, made = [], {}

        def rope(name, wname):
            return g.rope_ext(g.mul(g.rms_norm(g.view(dev[name], dev[name]), 1e-6), w(dev[wname])), dev["pos"],
                              hd, gpu.ROPE_TYPE_NEOX, 1e6)
        for item in order:
            if item == "q":
                made["q"] = rope("q", "wq")
                outs.append(made["q"])
            elif item == "k":
                outs.append(g.cpy(rope("k", "wk"), dev["kc"][filled:filled + T]))
            elif item == "v":
                outs.append(g.cpy(g.view(dev["v"], dev["v"]), dev["vc"][filled:filled + T]))
            elif item == "read_cache":
                full = g.view(dev["kc"], dev["kc"])
                outs.append(g.add(full, full))
            elif item == "read_vcache":
                full = g.view(dev["vc"], dev["vc"])
                outs.append(g.add(full, full))
            elif item == "write_kcache":
                outs.append(g.cpy(dev["kcf16"], dev["kc"]))
            elif item == "write_vcache":
                outs.append(g.cpy(dev["vcf16"], dev["vc"]))
            elif item == "clobber_q":
                outs.append(g.cpy(dev["qf16"], dev["q"]))
            elif item == "clobber_v":
                outs.append(g.cpy(dev["vf16"], dev["v"]))
            elif item == "read_q":
                if "q" in made:
                    outs.append(g.add(made["q"], made["q"]))
            else:
                outs.append(g.exp(dev["a"]))
        every = outs + [n["val"] for n in g.order(*outs)] if all_outputs else outs
        return g, outs, every

    return build, restore, dev, order


@pytest.mark.parametrize("seed", range(CASES))
def test_qkv_launch_equals_node_by_node(gpu, seed):
    import torch
    build, restore, dev, order = _case(gpu, seed)
    print("case", seed, list(order), flush=True)
    results = []
    for every_node in (False, True):
        restore()
        g, outs, every = build(every_node)
        kinds = [k for k, *_ in g.plan(*every) if k != "nop"]
        if every_node:
            assert all(k == "single" for k in kinds), kinds
        else:
            print("plan", kinds, flush=True)
        g.compute(*every)
        torch.cuda.synchronize()
        results.append(([_np(o.t).copy() for o in outs], [_np(dev[x]).copy() for x in ("q", "v", "kc", "vc")]))
    (fo, fm), (so, sm) = results
    assert len(fo) == len(so)
    for a, b in zip(fo, so):
        assert_bitexact(a, b)
    for a, b in zip(fm, sm):
        assert_bitexact(a, b)


def test_sweep_exercises_the_moved_launch(gpu):
    """Across the cases, the q/k/v launch is taken where nothing stands in the
    way, including with k's part or v's copy moved up past other nodes, and
    kept apart in others."""
    taken = apart = 0
    for seed in range(CASES):
        build, restore, dev, order = _case(gpu, seed)
        g, outs, _ = build(False)
        kinds = [k for k, *_ in g.plan(*outs)]
        if "qk_norm_rope_kv" in kinds or "qk_norm_rope" in kinds:
            taken += 1
        else:
            apart += 1
    assert taken >= CASES // 3 and apart >= 1, (taken, apart)


# ---------------------------------------------------------------------------
# the vocoder / codec tails: the conv-tail, codec transpose-bias and
# view -> binary runs, with readers of the intermediates, outputs flagged,
# and outputs placed over the source's memory
# ---------------------------------------------------------------------------

TAIL_CASES = 48


def _tail_case(gpu, seed):
    import torch
    rng = np.random.default_rng(SEED + 20000 + seed)
    kind = str(rng.choice(["conv_tail", "codec_tconv", "codec_dw", "crop_bias"]))
    T = int(rng.choice([64, 130, 1000, 2048]))
    C = int(rng.choice([8, 37, 64, 96]))
    kept = T - int(rng.integers(0, 9))
    resid = bool(rng.integers(0, 2))
    leaky = bool(rng.integers(0, 2))
    crop_copy = bool(rng.integers(0, 2))
    extra = str(rng.choice(["none", "none", "read_first", "read_mid", "flag_mid", "over_source"]))
    host = {"src": rng.standard_normal((C, T)).astype(np.float32),       # ggml [T, C]
            "srcT": rng.standard_normal((T, C)).astype(np.float32),      # ggml [C, T]
            "bC1": rng.standard_normal((C, 1)).astype(np.float32),       # ggml [1, C]
            "bC": rng.standard_normal(C).astype(np.float32),             # ggml [C]
            "r": rng.standard_normal((C, T)).astype(np.float32)}
    dev = {n: _t(gpu, a) for n, a in host.items()}

    def restore():
        for n in ("src", "srcT", "r"):
            dev[n].copy_(torch.from_numpy(host[n]).cuda())
        torch.cuda.synchronize()

    def build(all_outputs):
        g = gpu.Graph()
        outs, first, mid = [], None, None
        if kind == "conv_tail":                      # vits: cont(transpose(out)) + bias [+ r] [-> leaky]
            o = dev["srcT"]
            first = g.cont(g.view(o, o.t()))          # ggml [T, C]
            mid = g.add(first, dev["bC1"])
            last = g.add(mid, dev["r"]) if resid else mid
            if leaky:
                if extra == "over_source":            # the result over the source's bytes, other layout
                    last = g._op(gpu.NODE_LEAKY_RELU, dev["srcT"].view(C, T), [last], floats={0: 0.1})
                else:
                    last = g.leaky_relu(last, 0.1)
        elif kind == "codec_tconv":                   # qwen3 codec: [cont(crop)] + bias [1, C] -> cont(transpose)
            w = dev["src"]
            first = g.cont(g.view(w, w[:, :kept])) if crop_copy else g.view(w, w[:, :kept])
            mid = g.add(first, dev["bC1"])
            if extra == "over_source":
                last = g._op(gpu.NODE_CPY, dev["src"].view(-1)[:kept * C].view(kept, C), [g.view(mid, mid.t.t())])
            else:
                last = g.cont(g.view(mid, mid.t.t()))
        elif kind == "codec_dw":                      # cont(transpose(mm)), cont(first rows), + bias [C]
            m = dev["src"]
            first = g.cont(g.view(m, m.t()))          # ggml [C, T]
            mid = g.cont(g.view(first, first.t[:kept]))
            last = g.add(mid, dev["bC"])
        else:                                         # crop, + row bias (view -> binary)
            w = dev["srcT"]
            first = g.cont(g.view(w, w[:kept]))
            mid = first
            last = g.add(first, dev["bC"])
        outs.append(last)
        if extra == "read_first" and isinstance(first, gpu.GVal) and first.node["op"] != gpu.NODE_NOP:
            outs.append(g.exp(first))
        elif extra == "read_mid" and mid is not None:
            outs.append(g.exp(mid))
        elif extra == "flag_mid" and mid is not None:
            outs.append(mid)
        every = outs + [n["val"] for n in g.order(*outs)] if all_outputs else outs
        return g, outs, every

    return build, restore, dev, (kind, T, C, kept, resid, leaky, crop_copy, extra)


@pytest.mark.parametrize("seed", range(TAIL_CASES))
def test_tail_runs_equal_node_by_node(gpu, seed):
    import torch
    build, restore, dev, desc_ = _tail_case(gpu, seed)
    print("tail case", seed, desc_, flush=True)
    results = []
    for every_node in (False, True):
        restore()
        g, outs, every = build(every_node)
        kinds = [k for k, *_ in g.plan(*every) if k != "nop"]
        print("plan", every_node, kinds, flush=True)
        g.compute(*every)
        torch.cuda.synchronize()
        results.append(([_np(o.t).copy() for o in outs], [_np(dev[n]).copy() for n in ("src", "srcT", "r")]))
    (fo, fm), (so, sm) = results
    for a, b in zip(fo, so):
        assert_bitexact(a, b)
    for a, b in zip(fm, sm):
        assert_bitexact(a, b)


def test_tail_sweep_exercises_the_runs(gpu):
    """Across the cases, each tail run is taken somewhere and kept apart
    somewhere (by a reader, a flag or an overlapping output)."""
    seen, apart = set(), 0
    for seed in range(TAIL_CASES):
        build, restore, dev, d_ = _tail_case(gpu, seed)
        g, outs, _ = build(False)
        kinds = [k for k, *_ in g.plan(*outs) if k != "nop"]
        seen.update(k for k in kinds if k in ("cont_add_leaky", "view_binary"))
        if d_[-1] != "none" and "cont_add_leaky" not in kinds and "view_binary" not in kinds:
            apart += 1
    assert seen == {"cont_add_leaky", "view_binary"} and apart >= 1, (seen, apart)

#!/usr/bin/env python3
"""Benchmark of the fused non-GEMM layer primitives on one MI355X.

Default workload: the non-GEMM work of one
Qwen3-TTS-0.6B talker layer at prefill -- 512 tokens x hidden 1024, f32
activations ~N(0,1), BF16 norm gains, 16 q / 8 kv heads x 128, NEOX rope theta
1e6 at positions 0..511, SwiGLU 3072 -- plus the BF16 text-embedding gather
from a 151936 x 2048 table ~N(0, 0.02) with 512 uniform ids. One step is six
launches through the C ABI, in graph order:

    get_rows(bf16 table)        talker.cpp:44
    rms_norm_mul (input norm)   operations.cpp:86
    qk_norm_rope (q and k)      operations.cpp:98-104
    add_rms_norm_mul (+sum)     operations.cpp:143-145
    swiglu                      operations.cpp:39-41
    add (layer output)          operations.cpp:147

Each step is replayed from a HIP graph (captured once per input set), the way
a decode loop would issue it. Cold-cache protocol: inputs rotate over enough
sets that the working set exceeds 512 MB (twice the 256 MB MALL), so every
step reads from HBM. value = algorithmic bytes per step x steps / elapsed.

Also reported: per-op launch durations (each op replayed alone over the same
rotation), the dominant kernel's roofline, the 28-layer decode step's non-GEMM
time per layer (config 1 shape), and the CPU restatement of the same step
timed on this host (ggml-style thread split), as a baseline only.
"""
import argparse
import json
import math
import os
import statistics
import sys

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "synthesize.cpp_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

PEAK_GBS = 8000.0
METRIC = "achieved HBM GB/s (% of peak) per fused op; µs/talker-layer non-GEMM step"
SEED = 20260728
COLD_BYTES = 512 << 20
CALIB_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_configs1_step.txt")


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=40)
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU-baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--suite", metavar="JSON", help="instead: measure every op on every BASELINE config "
                   "(cold-cache protocol), print a markdown table and write the figures to JSON")
    p.add_argument("--only", default="", help="with --suite: comma-separated config names to run")
    p.add_argument("--pmc-pass", action="store_true", help="instead: run each op of the step eagerly over every "
                   "input set a few times, plus a %d MiB device copy of known size, for rocprofv3 --pmc "
                   "FETCH_SIZE / WRITE_SIZE passes (few dispatches, no graphs)" % (CALIB_BYTES >> 20))
    p.add_argument("--pmc-large", action="store_true", help="instead: run one launch of each op at the large "
                   "configs' shapes, three times, for rocprofv3 --pmc occupancy / VALU passes")
    return p.parse_args()


# ---------------------------------------------------------------------------
# the step
# ---------------------------------------------------------------------------

class PrefillStep:
    T, HIDDEN, HEADS, KV_HEADS, HEAD_DIM, FFN = 512, 1024, 16, 8, 128, 3072
    VOCAB, TEXT_HIDDEN = 151936, 2048
    EPS, THETA = 1e-6, 1e6

    def __init__(self, S, torch):
        self.S, self.torch = S, torch
        T, H, D = self.T, self.HIDDEN, self.HEAD_DIM
        f32 = 4
        self.op_bytes = {
            "get_rows_bf16": T * (4 + self.TEXT_HIDDEN * 2 + self.TEXT_HIDDEN * f32),
            "rms_norm_mul": 2 * T * H * f32 + H * 2,
            "qk_norm_rope": 2 * (self.HEADS + self.KV_HEADS) * D * T * f32 + T * 4 + 2 * D * 2,
            "add_rms_norm_mul": 4 * T * H * f32 + H * 2,
            "swiglu": 3 * T * self.FFN * f32,
            "add": 3 * T * H * f32,
        }
        self.step_bytes = sum(self.op_bytes.values())
        per_set = self.step_bytes
        self.nsets = max(2, -(-COLD_BYTES // per_set) + 1)
        g = torch.Generator(device="cuda")
        g.manual_seed(SEED)
        dev = "cuda"
        randn = lambda *shape: torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
        gain = lambda n: (1.0 + 0.1 * randn(n)).to(torch.bfloat16)
        self.table = (0.02 * randn(self.VOCAB, self.TEXT_HIDDEN)).to(torch.bfloat16)
        self.w_in, self.w_post = gain(H), gain(H)
        self.wq, self.wk = gain(D), gain(D)
        self.pos = torch.arange(T, dtype=torch.int32, device=dev)
        self.sets = []
        for _ in range(self.nsets):
            s = dict(
                ids=torch.randint(0, self.VOCAB, (T,), generator=g, device=dev, dtype=torch.int32),
                x=randn(T, H), q=randn(T, self.HEADS, D), k=randn(T, self.KV_HEADS, D), proj=randn(T, H),
                gate=randn(T, self.FFN), up=randn(T, self.FFN), mlp=randn(T, H),
            )
            s.update(emb=torch.empty(T, self.TEXT_HIDDEN, device=dev), normed=torch.empty(T, H, device=dev),
                     qo=torch.empty_like(s["q"]), ko=torch.empty_like(s["k"]), resid=torch.empty(T, H, device=dev),
                     mlp_in=torch.empty(T, H, device=dev), act=torch.empty(T, self.FFN, device=dev),
                     out=torch.empty(T, H, device=dev))
            self.sets.append(s)
        torch.cuda.synchronize()

    def ops(self, s):
        S, c = self.S, self.sets[s]
        return [
            ("get_rows_bf16", lambda: S.get_rows(self.table, c["ids"], out=c["emb"])),
            ("rms_norm_mul", lambda: S.rms_norm_mul(c["x"], self.w_in, self.EPS, out=c["normed"])),
            ("qk_norm_rope", lambda: S.qk_norm_rope(c["q"], c["k"], self.wq, self.wk, self.EPS, self.pos,
                                                    self.HEAD_DIM, self.THETA, q_out=c["qo"], k_out=c["ko"])),
            ("add_rms_norm_mul", lambda: S.add_rms_norm_mul(c["x"], c["proj"], self.w_post, self.EPS,
                                                            out=c["mlp_in"], sum_out=c["resid"])),
            ("swiglu", lambda: S.swiglu(c["gate"], c["up"], out=c["act"])),
            ("add", lambda: S.add(c["resid"], c["mlp"], out=c["out"])),
        ]


def capture(torch, fns):
    """One HIP graph replaying `fns` in order (each already run eagerly once)."""
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for f in fns:
                f()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    return graph


def time_graphs(torch, graphs, reps):
    """Replays graphs round-robin `reps` times between two events; returns ms."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(reps):
        graphs[i % len(graphs)].replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end)


# ---------------------------------------------------------------------------
# decode step: 28 layers x (add+norm, qk-norm+rope, add+norm, swiglu) at T=1
# ---------------------------------------------------------------------------

def decode_layer_us(S, torch, layers=28, reps=50, kv=False, total=512, streams=1):
    """µs per talker layer of the decode step's non-GEMM ops, replayed as one
    graph of `layers` layers. kv: qk-norm+rope also writes this step's k and v
    into the layer's cache (slot total-1) and the step adds the attention
    softmax over `total` keys for the 16 heads (5 launches per layer).
    streams: concurrent decode streams batched into each op (one token each)."""
    assert not (kv and streams != 1), "the KV variant models one stream"
    g = torch.Generator(device="cuda")
    g.manual_seed(SEED + 1)
    randn = lambda *shape: torch.randn(shape, generator=g, device="cuda", dtype=torch.float32)
    gain = lambda n: (1.0 + 0.1 * randn(n)).to(torch.bfloat16)
    L = []
    for _ in range(layers):
        n = streams
        c = dict(a=randn(n, 1024), b=randn(n, 1024), w1=gain(1024), w2=gain(1024), wq=gain(128),
                 wk=gain(128), q=randn(n, 16, 128), k=randn(n, 8, 128), proj=randn(n, 1024),
                 gate=randn(n, 3072), up=randn(n, 3072), s1=torch.empty(n, 1024, device="cuda"),
                 y1=torch.empty(n, 1024, device="cuda"), s2=torch.empty(n, 1024, device="cuda"),
                 y2=torch.empty(n, 1024, device="cuda"), qo=torch.empty(n, 16, 128, device="cuda"),
                 ko=torch.empty(n, 8, 128, device="cuda"), act=torch.empty(n, 3072, device="cuda"))
        if kv:
            c.update(v=randn(1, 8, 128), kc=randn(total, 8, 128), vc=randn(total, 8, 128),
                     sc=randn(16, 1, total), p=torch.empty(16, 1, total, device="cuda"))
        L.append(c)
    pos = torch.full((streams,), total - 1, dtype=torch.int32, device="cuda")
    scale = 1.0 / math.sqrt(128.0)

    def layer_fns(c):
        if kv:
            rope = lambda: S.qk_norm_rope_kv(c["q"], c["k"], c["v"], c["wq"], c["wk"], 1e-6, pos, 128, 1e6, c["kc"],
                                             c["vc"], total - 1, q_out=c["qo"])
        else:
            rope = lambda: S.qk_norm_rope(c["q"], c["k"], c["wq"], c["wk"], 1e-6, pos, 128, 1e6, q_out=c["qo"],
                                          k_out=c["ko"])
        fns = [lambda: S.add_rms_norm_mul(c["a"], c["b"], c["w1"], 1e-6, out=c["y1"], sum_out=c["s1"]), rope]
        if kv:
            fns.append(lambda: S.soft_max_ext(c["sc"], None, scale, out=c["p"]))
        return fns + [lambda: S.add_rms_norm_mul(c["s1"], c["proj"], c["w2"], 1e-6, out=c["y2"], sum_out=c["s2"]),
                      lambda: S.swiglu(c["gate"], c["up"], out=c["act"])]

    fns = [f for c in L for f in layer_fns(c)]
    for f in fns:
        f()
    graph = capture(torch, fns)
    time_graphs(torch, [graph], 5)
    ms = time_graphs(torch, [graph], reps)
    return ms * 1e3 / (reps * layers)


def decode_layer_bytes(streams=1, kv=False, total=512):
    """Algorithmic bytes of one layer of decode_layer_us's graph, every operand
    once: add+norm (a, b read; sum, y written; BF16 gain), qk-norm+rope (q, k
    read and written; two BF16 gains; one I32 position per stream), add+norm
    again, SwiGLU 3072 (gate, up read; act written). kv adds this step's v row
    (read, and written with k into the caches) and the 16-head softmax over
    `total` keys (read and written)."""
    f32 = 4
    per_stream = 2 * (4 * 1024 * f32) + 2 * (24 * 128 * f32) + 3 * 3072 * f32 + 4
    fixed = 2 * 1024 * 2 + 2 * 128 * 2
    if kv:
        per_stream += 2 * 8 * 128 * f32
        fixed += 2 * 16 * total * f32
    return streams * per_stream + fixed


# ---------------------------------------------------------------------------
# CPU baseline: the same step as ggml node runs on the restatement
# ---------------------------------------------------------------------------

def cpu_baseline(step, torch, seconds):
    import numpy as np
    import ggml_ref as R

    c = step.sets[0]
    h = lambda t: t.detach().cpu().contiguous().numpy()
    bits = lambda t: h(t.view(torch.int16)).view(np.uint16)
    table, ids = bits(step.table), h(c["ids"])
    x, q, k, proj, gate, up, mlp = (h(c[n]) for n in ("x", "q", "k", "proj", "gate", "up", "mlp"))
    w_in, w_post, wq, wk = bits(step.w_in), bits(step.w_post), bits(step.wq), bits(step.wk)
    pos = h(step.pos)
    eps, theta = np.float32(step.EPS), np.float32(step.THETA)

    def build(g):
        g.get_rows(table, R.BF16, step.TEXT_HIDDEN, ids)
        R.rms_norm_w(g, x, w_in, eps, R.BF16)
        R.qk_norm_rope(g, q, k, wq, wk, eps, pos, step.HEAD_DIM, theta, R.BF16)
        s, _ = R.add_rms_norm_w(g, x, proj, w_post, eps, R.BF16)
        R.swiglu(g, gate, up)
        g.add(s, mlp)

    g = R.Graph()
    build(g)
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    nth = max(1, min(cores, 16))
    probe = g.time(nth, 1, 1)[0]
    reps = int(max(3, min(400, 0.5 * seconds / max(probe, 1e-6))))
    t_many = statistics.median(g.time(nth, 2, reps))
    # max(1, N/2) threads is the reference's default CPU parallelism
    # (cpu-parallelism.h:21-39); N and 1 bracket it.
    half = max(1, nth // 2)
    t_half = statistics.median(g.time(half, 1, max(3, reps // 2)))
    probe1 = g.time(1, 0, 1)[0]
    reps1 = int(max(2, min(100, 0.25 * seconds / max(probe1, 1e-6))))
    t_one = statistics.median(g.time(1, 1, reps1))
    gbs = lambda t: step.step_bytes / t / 1e9
    return {
        "value": round(gbs(t_many), 2), "unit": "GB/s", "cores": nth, "kind": "port",
        "sample": "the same configs[1] prefill step (gather + norm + qk-norm/rope + add/norm + swiglu + add, "
                  "%d ggml nodes) on the ggml-CPU restatement, median of %d reps at %d threads; "
                  "%d threads (the reference's default, N/2): %.2f GB/s; 1 thread: %.2f GB/s (median of %d)" % (
                      len(g.nodes), reps, nth, half, gbs(t_half), gbs(t_one), reps1),
        "ms_per_step": round(t_many * 1e3, 3), "value_half_threads": round(gbs(t_half), 3), "half_threads": half,
        "value_1thread": round(gbs(t_one), 3),
    }


# ---------------------------------------------------------------------------
# --suite: every op on every BASELINE config
# ---------------------------------------------------------------------------

def measure_op(torch, make, nbytes, reps_target=200, cold=True):
    """Average launch duration (µs) of the op built by make() -> callable, over
    enough rotating input sets to exceed COLD_BYTES (cold=False: one set,
    cache resident), replayed from one graph."""
    nsets = 1 if (nbytes >= COLD_BYTES or not cold) else -(-COLD_BYTES // nbytes) + 1
    nsets = min(nsets, 4096)
    fns = [make() for _ in range(nsets)]
    for f in fns:
        f()
    if nsets == 1:
        fns = fns * (4 if cold else 256)  # warm: enough nodes to amortise the graph launch
    graph = capture(torch, fns)
    time_graphs(torch, [graph], 2)
    reps = max(2, reps_target // len(fns))
    us = time_graphs(torch, [graph], reps) * 1e3 / (reps * len(fns))
    del graph, fns
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return us, nsets


def suite(args, S, torch):
    g = torch.Generator(device="cuda")
    g.manual_seed(SEED + 7)
    randn = lambda *shape: torch.randn(shape, generator=g, device="cuda", dtype=torch.float32)
    empty = lambda *shape: torch.empty(shape, device="cuda", dtype=torch.float32)
    bf16 = lambda n: (1.0 + 0.1 * randn(n)).to(torch.bfloat16)
    f32 = 4
    rows = []

    def run(cfg, name, nbytes, make, note="", cold=True):
        us, nsets = measure_op(torch, make, nbytes, cold=cold)
        if not cold:
            note = ("warm " + note).strip()
        gbs = nbytes / (us * 1e-6) / 1e9
        rows.append({"config": cfg, "op": name, "bytes": nbytes, "us": round(us, 3), "GB/s": round(gbs, 1),
                     "frac": round(gbs / PEAK_GBS, 4), "sets": nsets, "note": note})
        print("%-5s %-38s %12d B %9.3f us %8.1f GB/s %6.1f%%  sets=%d %s" % (cfg, name, nbytes, us, gbs,
                                                                            100 * gbs / PEAK_GBS, nsets, note),
              flush=True)

    want = set(filter(None, args.only.split(",")))
    on = lambda c: not want or c in want

    if on("calib"):
        # what a plain device copy, a read-only reduction and this library's
        # copy-like kernel (bare leaky-ReLU: one read, one write) reach on this box
        n = (1 << 30) // 4
        src, dst = randn(n), empty(n)
        acc = torch.empty((), device="cuda", dtype=torch.float32)
        run("calib", "torch copy_ 1 GiB (read+write)", 2 * n * 4, lambda: (lambda: dst.copy_(src)))
        run("calib", "torch sum 1 GiB (read only)", n * 4, lambda: (lambda: torch.sum(src, dim=0, out=acc)))
        del src, dst

        def make_floor():
            x, y = randn(8192, 2048), empty(8192, 2048)
            return lambda: S.leaky_relu(x, 0.1, out=y)
        run("calib", "copy-like floor: bare leaky [2048,8192]", 8 * 8192 * 2048, make_floor)

    def norm_case(cfg, T, H, add=False, wsum=True, cold=True):
        def make():
            a, b, w, y, s = randn(T, H), randn(T, H), bf16(H), empty(T, H), empty(T, H)
            if add:
                return lambda: S.add_rms_norm_mul(a, b, w, 1e-6, out=y, sum_out=s if wsum else None,
                                                  want_sum=wsum)
            return lambda: S.rms_norm_mul(a, w, 1e-6, out=y)
        n = (4 if wsum else 3) if add else 2
        run(cfg, ("add_rms_norm_mul%s [%d,%d]" % ("+sum" if wsum else "", H, T)) if add else
            "rms_norm_mul [%d,%d]" % (H, T), n * T * H * f32 + H * 2, make, cold=cold)

    def qk_case(cfg, T, hi, cold=True):
        def make():
            q, k = randn(T, 16, 128), randn(T, 8, 128)
            qo, ko = torch.empty_like(q), torch.empty_like(k)
            wq, wk = bf16(128), bf16(128)
            pos = torch.randint(0, hi, (T,), generator=g, device="cuda", dtype=torch.int32)
            return lambda: S.qk_norm_rope(q, k, wq, wk, 1e-6, pos, 128, 1e6, q_out=qo, k_out=ko)
        run(cfg, "qk_norm_rope q[128,16,%d] k[128,8,%d]" % (T, T), 2 * 24 * 128 * T * f32 + T * 4 + 512, make,
            cold=cold)

    def swiglu_case(cfg, T, F_, cold=True):
        def make():
            a, b, y = randn(T, F_), randn(T, F_), empty(T, F_)
            return lambda: S.swiglu(a, b, out=y)
        run(cfg, "swiglu [%d,%d]" % (F_, T), 3 * T * F_ * f32, make, cold=cold)

    def add_case(cfg, T, H, cold=True):
        def make():
            a, b, y = randn(T, H), randn(T, H), empty(T, H)
            return lambda: S.add(a, b, out=y)
        run(cfg, "add [%d,%d]" % (H, T), 3 * T * H * f32, make, cold=cold)

    if on("cfg1"):
        def make_tiny():
            a, b = randn(1), empty(1)
            return lambda: torch.add(a, a, out=b)
        run("cfg1", "graph launch floor (torch 1-element add)", 12, make_tiny, cold=False)
        for cold in (True, False):
            norm_case("cfg1", 1, 1024, cold=cold)
            norm_case("cfg1", 1, 1024, add=True, cold=cold)
            qk_case("cfg1", 1, 64, cold=cold)
            swiglu_case("cfg1", 1, 3072, cold=cold)
            add_case("cfg1", 1, 1024, cold=cold)
        us = decode_layer_us(S, torch)
        b1 = decode_layer_bytes()
        rows.append({"config": "cfg1", "op": "talker layer non-GEMM step (28-layer graph, 4 launches/layer)",
                     "us": round(us, 3), "bytes": b1, "GB/s": round(b1 / (us * 1e3), 1), "note": "per layer"})
        print("cfg1  decode layer non-GEMM step: %.3f us/layer (%d B, %.1f GB/s)" % (us, b1, b1 / (us * 1e3)),
              flush=True)
        us_kv = decode_layer_us(S, torch, kv=True)
        bkv = decode_layer_bytes(kv=True)
        rows.append({"config": "cfg1", "op": "talker layer non-GEMM step + KV-cache write + soft_max over 512 keys "
                     "(28-layer graph, 5 launches/layer)", "us": round(us_kv, 3), "bytes": bkv,
                     "GB/s": round(bkv / (us_kv * 1e3), 1), "note": "per layer"})
        print("cfg1  decode layer + KV write + soft_max: %.3f us/layer (%d B, %.1f GB/s)" % (us_kv, bkv,
                                                                                        bkv / (us_kv * 1e3)), flush=True)

        def make_kv():
            q, k, v = randn(1, 16, 128), randn(1, 8, 128), randn(1, 8, 128)
            kc, vc, qo = randn(512, 8, 128), randn(512, 8, 128), empty(1, 16, 128)
            w = bf16(128)
            pos = torch.tensor([511], dtype=torch.int32, device="cuda")
            return lambda: S.qk_norm_rope_kv(q, k, v, w, w, 1e-6, pos, 128, 1e6, kc, vc, 511, q_out=qo)
        run("cfg1", "qk_norm_rope_kv [128,16+8(+8 v),1]", (2 * 32) * 128 * f32 + 4 + 2 * 128 * 2, make_kv, cold=False)

        def make_sm(T=1, N=512):
            sc, p = randn(16, T, N), empty(16, T, N)
            return lambda: S.soft_max_ext(sc, None, 1.0 / math.sqrt(128.0), out=p)
        run("cfg1", "soft_max_ext [512,1,16]", 2 * 16 * 512 * f32, make_sm, cold=False)
        run("cfg2", "soft_max_ext causal-size [512,512,16]", 2 * 16 * 512 * 512 * f32, lambda: make_sm(512, 512))

    if on("cfg2"):
        norm_case("cfg2", 512, 1024)
        qk_case("cfg2", 512, 512)
        norm_case("cfg2", 512, 1024, add=True)
        swiglu_case("cfg2", 512, 3072)
        add_case("cfg2", 512, 1024)
        table = (0.02 * randn(151936, 2048)).to(torch.bfloat16)

        def make_gather():
            ids = torch.randint(0, 151936, (512,), generator=g, device="cuda", dtype=torch.int32)
            out = empty(512, 2048)
            return lambda: S.get_rows(table, ids, out=out)
        run("cfg2", "get_rows bf16 [2048,151936] x512", 512 * (4 + 2048 * 2 + 2048 * f32), make_gather)
        del table

    if on("cfg3"):
        import numpy as np
        import formats as F
        rng = np.random.default_rng(SEED + 3)
        row = 1024 // 32 * 34
        # Each input set has its own 16 tables (35.7 MB), so the rotation (8+ sets)
        # exceeds the Infinity Cache and every launch fetches its tables from HBM.
        table_sets = []

        def tables(n=16):
            raw = torch.from_numpy(np.stack([F.q8_0_synthetic(rng, 2048, 1024) for _ in range(n)])).cuda()
            table_sets.append(raw)
            return [S.Q8Tensor(raw[t], 1024) for t in range(n)]

        def make_sum():
            tabs = tables()
            codes = torch.randint(0, 2048, (16, 4096), generator=g, device="cuda", dtype=torch.int32)
            out = empty(4096, 1024)
            return lambda: S.get_rows_sum(tabs, codes, out=out)
        logical = 4096 * (16 * (row + 4) + 1024 * f32)
        touched = 16 * 2048 * (1.0 - (1.0 - 1.0 / 2048) ** 4096)  # expected distinct rows touched
        compulsory = int(touched * row) + 4096 * (16 * 4 + 1024 * f32)
        run("cfg3", "get_rows_sum q8_0 16x[1024,2048] x4096", compulsory, make_sum, "compulsory bytes")
        rows[-1]["logical_bytes"] = logical
        rows[-1]["logical_GB/s"] = round(logical / (rows[-1]["us"] * 1e-6) / 1e9, 1)
        rows[-1]["note"] = "compulsory bytes (distinct rows once + ids + out); logical %.1f GB/s" % rows[-1]["logical_GB/s"]
        table_sets.clear()

        def make_q8():
            tabs = tables(1)
            ids = torch.randint(0, 2048, (4096,), generator=g, device="cuda", dtype=torch.int32)
            out = empty(4096, 1024)
            return lambda: S.get_rows(tabs[0], ids, out=out)
        touched1 = 2048 * (1.0 - (1.0 - 1.0 / 2048) ** 4096)
        compulsory1 = int(touched1 * row) + 4096 * (4 + 1024 * f32)
        run("cfg3", "get_rows q8_0 [1024,2048] x4096", compulsory1, make_q8,
            "compulsory bytes; logical %d B" % (4096 * (row + 4 + 1024 * f32)))
        table_sets.clear()

    if on("cfg4"):
        for C, T in ((512, 8192), (256, 32768), (128, 131072)):
            n = C * T

            def make_snake(C=C, T=T):
                x, y = randn(T, C), empty(T, C)
                al = torch.exp(torch.empty(C, device="cuda").uniform_(math.log(0.1), math.log(10.0), generator=g))
                return lambda: S.snake(x, al, out=y)
            run("cfg4", "snake [%d,%d]" % (C, T), 8 * n + 4 * C, make_snake)

            def make_leaky(C=C, T=T, with_s=False):
                a, b, y, s = randn(T, C), randn(T, C), empty(T, C), empty(T, C)
                return lambda: S.add_leaky_relu(a, b, 0.1, out=y, sum_out=s if with_s else None)
            run("cfg4", "add_leaky_relu [%d,%d]" % (C, T), 12 * n, make_leaky)
            run("cfg4", "add_leaky_relu+sum [%d,%d]" % (C, T), 16 * n, lambda: make_leaky(with_s=True))

            def make_snake_var(C=C, T=T, beta=False):
                x, y = randn(T, C), empty(T, C)
                la = torch.empty(C, device="cuda").uniform_(-3.0, 3.0, generator=g)
                if beta:
                    lb = torch.empty(C, device="cuda").uniform_(-3.0, 3.0, generator=g)
                    return lambda: S.snake_beta(x, la, lb, out=y)
                al = torch.exp(la)
                return lambda: S.snake_guarded(x, al, out=y)
            run("cfg4", "snake_guarded [%d,%d]" % (C, T), 8 * n + 4 * C, make_snake_var)
            run("cfg4", "snake_beta [%d,%d]" % (C, T), 8 * n + 8 * C, lambda: make_snake_var(beta=True))

            def make_branch(C=C, T=T):
                ts, y = [randn(T, C) for _ in range(3)], empty(T, C)
                return lambda: S.sum_scale_leaky_relu(ts, 1.0 / 3.0, 0.1, out=y)
            run("cfg4", "branch mean 3->scale->leaky [%d,%d]" % (C, T), 16 * n, make_branch)

    if on("cfg5"):
        norm_case("cfg5", 8192, 2048)
        norm_case("cfg5", 8192, 2048, add=True)
        qk_case("cfg5", 8192, 8192)
        swiglu_case("cfg5", 8192, 6144)
        norm_case("cfg5", 64, 1024, add=True)
        qk_case("cfg5", 64, 8192)
        swiglu_case("cfg5", 64, 3072)
        us64 = decode_layer_us(S, torch, streams=64)
        b64 = decode_layer_bytes(streams=64)
        rows.append({"config": "cfg5", "op": "64 concurrent decode streams: talker layer non-GEMM step "
                     "(28-layer graph, 4 launches/layer, 64 rows per launch)", "us": round(us64, 3), "bytes": b64,
                     "GB/s": round(b64 / (us64 * 1e3), 1),
                     "note": "per layer; per 28-layer step %.1f us, %d B" % (28 * us64, 28 * b64)})
        print("cfg5  64-stream decode layer non-GEMM step: %.3f us/layer (%d B, %.1f GB/s; 28-layer step %.1f us)"
              % (us64, b64, b64 / (us64 * 1e3), 28 * us64), flush=True)

    if on("gguf"):
        # A package's lookup tables streamed file -> HBM by shp_gguf_load_tensor
        # (page cache warm after the first pass): the BF16 text embedding of
        # configs[1] and the 16 Q8_0 codebooks of configs[2], those one call
        # per tensor and in one shp_gguf_load_tensors call.
        import tempfile
        import time
        import numpy as np
        import formats as F
        from gguf_write import write_gguf
        rng = np.random.default_rng(SEED + 5)
        with tempfile.TemporaryDirectory() as tmp:
            path = os.path.join(tmp, "tables.gguf")
            bf = F.f32_to_bf16_bits(rng.standard_normal((151936, 2048), dtype=np.float32) * 0.02)
            q8 = F.q8_0_synthetic(rng, 2048, 1024)
            tensors = [("talker.model.text_embedding.weight", 30, [2048, 151936], bf.tobytes())]
            del bf
            tensors += [("talker.code_predictor.model.codec_embedding.%d.weight" % k, 8, [1024, 2048],
                         q8.tobytes()) for k in range(16)]
            write_gguf(path, tensors)
            del tensors
            with S.GgufFile(path) as f:
                codecs = ["talker.code_predictor.model.codec_embedding.%d.weight" % k for k in range(16)]
                for label, names, many in (
                        ("gguf load BF16 [2048,151936] file->HBM", ["talker.model.text_embedding.weight"], False),
                        ("gguf load 16 x Q8_0 [1024,2048] file->HBM", codecs, False),
                        ("gguf load 16 x Q8_0 [1024,2048] file->HBM, one call", codecs, True)):
                    nbytes = sum(f.info(n)[1] for n in names)
                    best = None
                    for _ in range(3):
                        torch.cuda.synchronize()
                        t0 = time.perf_counter()
                        out = f.load_many(names) if many else [f.load(n) for n in names]
                        torch.cuda.synchronize()
                        dt = time.perf_counter() - t0
                        best = dt if best is None else min(best, dt)
                        del out
                    gbs = nbytes / best / 1e9
                    rows.append({"config": "gguf", "op": label, "bytes": nbytes, "us": round(best * 1e6, 1),
                                 "GB/s": round(gbs, 2), "note": "page cache warm; PCIe host->device bound"})
                    print("gguf  %-44s %12d B %11.1f us %8.2f GB/s" % (label, nbytes, best * 1e6, gbs), flush=True)

    with open(args.suite, "w") as f:
        json.dump({"peak_GBps": PEAK_GBS, "cold_bytes": COLD_BYTES, "rows": rows}, f, indent=1)


def pmc_pass(step, torch):
    """Each op of the step, eagerly, 3 times over every input set, between two
    copies of CALIB_BYTES (a plain device-to-device copy: CALIB_BYTES read and
    CALIB_BYTES written), for counter collection."""
    n = CALIB_BYTES // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    for _ in range(3):
        for s in range(step.nsets):
            for _, f in step.ops(s):
                f()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_pass": "done", "sets": step.nsets, "calib_bytes": CALIB_BYTES, "op_bytes": step.op_bytes}))


def pmc_large(S, torch):
    """One launch each of the ops at the large configs' shapes, three times
    (rocprofv3 --pmc occupancy and VALU passes read them per dispatch)."""
    import numpy as np
    import formats as F
    g = torch.Generator(device="cuda")
    g.manual_seed(SEED + 9)
    randn = lambda *shape: torch.randn(shape, generator=g, device="cuda", dtype=torch.float32)
    bf16 = lambda n: (1.0 + 0.1 * randn(n)).to(torch.bfloat16)
    rng = np.random.default_rng(SEED + 9)
    x2, w2 = randn(8192, 2048), bf16(2048)
    q, k, wq, wk = randn(8192, 16, 128), randn(8192, 8, 128), bf16(128), bf16(128)
    pos = torch.arange(8192, dtype=torch.int32, device="cuda")
    gt, up = randn(8192, 6144), randn(8192, 6144)
    xs, al = randn(131072, 128), torch.exp(torch.empty(128, device="cuda").uniform_(-2.3, 2.3, generator=g))
    la, lb = torch.empty(128, device="cuda").uniform_(-3, 3, generator=g), torch.empty(128, device="cuda").uniform_(
        -3, 3, generator=g)
    a4, b4 = randn(131072, 128), randn(131072, 128)
    tabs = [S.Q8Tensor(torch.from_numpy(F.q8_0_synthetic(rng, 2048, 1024)).cuda(), 1024) for _ in range(16)]
    codes = torch.randint(0, 2048, (16, 4096), generator=g, device="cuda", dtype=torch.int32)
    sc = randn(16, 512, 512)
    ops = [("rms_norm_mul [2048,8192]", lambda: S.rms_norm_mul(x2, w2, 1e-6)),
           ("add_rms_norm_mul [2048,8192]", lambda: S.add_rms_norm_mul(x2, x2, w2, 1e-6)),
           ("qk_norm_rope [128,16+8,8192]", lambda: S.qk_norm_rope(q, k, wq, wk, 1e-6, pos, 128, 1e6)),
           ("swiglu [6144,8192]", lambda: S.swiglu(gt, up)),
           ("snake [128,131072]", lambda: S.snake(xs, al)),
           ("snake_beta [128,131072]", lambda: S.snake_beta(xs, la, lb)),
           ("add_leaky_relu [128,131072]", lambda: S.add_leaky_relu(a4, b4, 0.1)),
           ("get_rows_sum q8_0 16x4096", lambda: S.get_rows_sum(tabs, codes)),
           ("get_rows q8_0 x4096", lambda: S.get_rows(tabs[0], codes[0])),
           ("soft_max_ext [512,512,16]", lambda: S.soft_max_ext(sc, None, 0.0884))]
    torch.cuda.synchronize()
    for _ in range(3):
        for _, f in ops:
            f()
    torch.cuda.synchronize()
    print(json.dumps({"pmc_large": [name for name, _ in ops]}))


def read_traffic(op):
    """HBM bytes per launch of `op` from the committed counter summary (two
    rocprofv3 --pmc passes, FETCH_SIZE then WRITE_SIZE, each scaled by what the
    counter reads for the calibration copy), or None when it has no line."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        fields = dict(kv.split("=", 1) for kv in line.split() if "=" in kv)
        if fields.get("op") == op and "hbm_bytes" in fields:
            return int(float(fields["hbm_bytes"]))
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build is single-GPU by design. The primitives are "
              "row-independent, so G GPUs would each run the same kernels on 1/G of the tokens or streams "
              "with no exchange. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    import synth_hip as S

    torch.cuda.set_device(0)
    S.load()
    if args.suite:
        suite(args, S, torch)
        return
    if args.pmc_large:
        pmc_large(S, torch)
        return
    step = PrefillStep(S, torch)
    if args.pmc_pass:
        pmc_pass(step, torch)
        return

    # eager run of every op of every set (loads the code objects before capture)
    per_set_ops = [step.ops(s) for s in range(step.nsets)]
    for ops in per_set_ops:
        for _, f in ops:
            f()
    torch.cuda.synchronize()
    ref_out = step.sets[0]["out"].clone()
    ref_q = step.sets[0]["qo"].clone()

    # The timed region runs exactly `steps` steps, the sets in rotation. A
    # model's prefill replays its layers' steps from one graph (as the decode
    # measurement below replays 28 layers), so the steps are captured
    # back to back: one graph of all nsets steps, replayed steps // nsets
    # times, and one graph of the first steps % nsets steps for the rest.
    # ms_per_step_one_graph_each keeps the time with one graph launch per step.
    def run_steps(k, full, rem):
        for _ in range(k // step.nsets):
            full.replay()
        if rem is not None:
            rem.replay()

    full = capture(torch, [f for ops in per_set_ops for _, f in ops])
    rems = {k % step.nsets: capture(torch, [f for ops in per_set_ops[:k % step.nsets] for _, f in ops])
            for k in (args.warmup, args.steps) if k % step.nsets}
    run_steps(args.warmup, full, rems.get(args.warmup % step.nsets))
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    run_steps(args.steps, full, rems.get(args.steps % step.nsets))
    end.record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps
    value = step.step_bytes / (ms_per_step * 1e-3) / 1e9
    step_graphs = [capture(torch, [f for _, f in ops]) for ops in per_set_ops]
    time_graphs(torch, step_graphs, args.warmup)
    ms_one_graph_each = time_graphs(torch, step_graphs, args.steps) / args.steps

    # replays must reproduce the eager results bit for bit
    assert torch.equal(step.sets[0]["out"], ref_out) and torch.equal(step.sets[0]["qo"], ref_q)

    # per-op launch durations: each op alone, one graph over all sets
    names = [n for n, _ in per_set_ops[0]]
    per_op = {}
    reps = max(args.steps // step.nsets, 4)
    for i, name in enumerate(names):
        graph = capture(torch, [per_set_ops[s][i][1] for s in range(step.nsets)])
        time_graphs(torch, [graph], 2)
        us = time_graphs(torch, [graph], reps) * 1e3 / (reps * step.nsets)
        gbs = step.op_bytes[name] / (us * 1e-6) / 1e9
        per_op[name] = {"us": round(us, 3), "bytes": step.op_bytes[name], "GB/s": round(gbs, 1),
                        "frac": round(gbs / PEAK_GBS, 4)}
    dom = max(per_op, key=lambda n: per_op[n]["us"])
    # What a one-read-one-write stream of the same bytes reaches at this size in
    # the same run (this library's bare leaky-ReLU over the same rotation
    # protocol): a 19 MB launch cannot approach the HBM peak, and this says how
    # close the dominant kernel is to what its size allows.
    floor_elems = step.op_bytes[dom] // 8
    floor_us, _ = measure_op(torch, lambda: (lambda x, y: (lambda: S.leaky_relu(x, 0.1, out=y)))(
        torch.randn(floor_elems, device="cuda"), torch.empty(floor_elems, device="cuda")), 8 * floor_elems)
    roof = {"bound": "hbm", "kernel": dom, "achieved": per_op[dom]["GB/s"], "peak": PEAK_GBS, "unit": "GB/s",
            "frac": per_op[dom]["frac"], "traffic": read_traffic(dom),
            "algorithmic_bytes": step.op_bytes[dom], "us_per_launch": per_op[dom]["us"],
            "same_bytes_copy_like_us": round(floor_us, 3),
            "frac_of_same_bytes_copy_like": round(floor_us / per_op[dom]["us"], 4)}

    layer_us = decode_layer_us(S, torch)

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
        "ms_per_step_one_graph_each": round(ms_one_graph_each, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "configs[1]: Qwen3-TTS-0.6B talker layer non-GEMM prefill step, 512 tokens x hidden "
                               "1024, 16/8 heads x 128, SwiGLU 3072, BF16 gains + BF16 151936x2048 text-embedding "
                               "gather of 512 ids; the %d rotating input sets' steps (cold cache) replayed "
                               "back to back from one HIP graph" % step.nsets,
                   "tokens": step.T, "hidden": step.HIDDEN, "bytes_per_step": step.step_bytes,
                   "frac_of_peak": round(value / PEAK_GBS, 4)},
        "ops": per_op,
        "decode_layer_us": round(layer_us, 3),
        "decode_layer_GB/s": round(decode_layer_bytes() / (layer_us * 1e3), 1),
        "roofline": roof,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(step, torch, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

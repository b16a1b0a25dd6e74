#!/usr/bin/env python3
"""Benchmark of the fused non-GEMM layer primitives on one MI355X.

Default workload (the largest single-GPU config):
the non-GEMM work of one Qwen3-TTS-1.7B-shaped talker layer at an 8192-token
prefill -- hidden 2048, f32 activations ~N(0,1), BF16 norm gains, 16 q / 8 kv
heads x 128, NEOX rope theta 1e6 at positions 0..8191, SwiGLU 6144. One step
is five launches through the C ABI, in graph order:

    rms_norm_mul (input norm)           operations.cpp:86
    qk_norm_rope (q and k)              operations.cpp:94-104
    add_rms_norm_mul (+sum)             operations.cpp:143-145
    swiglu                              operations.cpp:39-41
    add (layer output)                  operations.cpp:147

The step moves 1.41 GB, so two input sets alternate and every step reads from
HBM (the Infinity Cache is 256 MB). Steps are captured back to back in one
HIP graph, as a model replays its layers; value = algorithmic bytes per step x
steps / elapsed, inputs resident in HBM before the timed region.

The same line carries, each op timed alone from a HIP graph over rotating
input sets whose total exceeds 512 MB (cold cache):
  - every op of the configs[4] step, and its roofline (the dominant kernel);
  - the 16-codebook Q8_0 gather->sum and the plain Q8_0 get_rows
    (logical bytes, every looked-up row per lookup; compulsory bytes beside),
    and the same two over Q5_K tables (the Q5_K_MIXED profile's);
  - Snake, SnakeBeta, add->leaky-ReLU and add->leaky-ReLU with the
    sum carried, the time-major ggml_cont(ggml_transpose(x)) copy of each
    vocoder convolution's output, the [1, C] bias add behind it, and the
    whole tail (copy, bias, residual, leaky) as one launch, and the
    convolution's im2col columns (K = 3 from the time-major input and from the
    channel-major activation's transposed view; at [128,131072] also K = 11
    dilation 5 and F16 columns of K = 7 dilation 3), the upsampling
    transposed convolution's col2im_1d scatter into each shape, and Kokoro's
    zero-stuffed spread, frame doubling and a time-axis edge padding, on
    [512,8192], [256,32768] and [128,131072];
  - the talker's prefill input assembly at configs[4]'s shape: ggml_acc of
    an 8176-position codec run into the [2048, 8192] text stream, out of
    place and in ggml's inplace form;
  - Kokoro's harmonic source and its spectrum, and the inverse short-time
    transform, of a 5-second utterance (9 harmonics, upsampling 300, n_fft 20,
    hop 5, 24 kHz): host code in the reference, between and after its graphs;
  - the Qwen3-TTS speaker encoder's log-mel of a 10-second reference clip
    (n_fft 1024, hop 256, 128 Slaney bins): host code in the reference too;
  - the decode step's non-GEMM work per talker layer (28-layer
    graph), without and with the KV-cache write and the attention softmax;
  - the 512-token prefill step of the 0.6B talker (with the BF16
    text-embedding gather) in GB/s and us per step;
  - configs[4]'s 64-stream decode: us per 28-layer step;
  - the CPU restatement of the configs[4] step timed on this host's cores, as
    a baseline only.

Every timed region is wrapped in a ROCTx range ("row:<config>|<op>|<bytes>"),
so `rocprofv3 --kernel-trace --marker-trace --stats` of this command can be
turned into per-row kernel durations with --trace-summary.
"""
import argparse
import ctypes
import csv
import glob
import json
import math
import os
import platform
import re
import statistics
import sys
from collections import defaultdict

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "synthesize.cpp_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

PEAK_GBS = 8000.0
METRIC = "achieved HBM GB/s (% of peak) per fused op; µs/talker-layer non-GEMM step"
SEED = 20260728
COLD_BYTES = 512 << 20
CALIB_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_large_configs.txt")
# Worker threads one GPU's share of a GPU box allows (the pool's per-GPU CPU
# allotment); the CPU baseline never uses more.
BOX_CPU_SHARE = 16


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU-baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--suite", metavar="JSON", help="instead: every op on every BASELINE config, smaller "
                   "shapes included (cold-cache protocol); a table on stdout, the rows as JSON")
    p.add_argument("--only", default="", help="with --suite: comma-separated config names (calib,configs0..4,gguf)")
    p.add_argument("--pmc-large", action="store_true", help="instead: three launches of each large-config op "
                   "on one input set, plus a %d MiB device copy of known size before and after, for "
                   "rocprofv3 --pmc passes (few dispatches, no graphs)" % (CALIB_BYTES >> 20))
    p.add_argument("--trace-summary", nargs=2, metavar=("ROCPROF_DIR", "BENCH_JSON"),
                   help="instead: summarise a rocprofv3 --kernel-trace --marker-trace run of this command "
                   "(per-row kernel durations against the bench line in BENCH_JSON, the stdout of an "
                   "unprofiled run on the same box); no GPU used")
    p.add_argument("--occ-summary", nargs="+", metavar="DIR",
                   help="instead: occupancy, VALU and memory-stall per --pmc-large op from rocprofv3 --pmc passes "
                   "of OccupancyPercent, MeanOccupancyPerCU, VALUBusy, MemUnitStalled (one DIR each, that order); "
                   "no GPU used")
    p.add_argument("--pmc-summary", nargs=3, metavar=("FETCH_DIR", "WRITE_DIR", "LOG"),
                   help="instead: HBM bytes per launch from FETCH_SIZE and WRITE_SIZE passes over --pmc-large "
                   "(LOG: that run's output, for the op list); no GPU used")
    return p.parse_args()


# ---------------------------------------------------------------------------
# ROCTx ranges (no-ops unless a profiler listens)
# ---------------------------------------------------------------------------

class Roctx:
    def __init__(self):
        self.lib = None
        for name in ("librocprofiler-sdk-roctx.so.1", "/opt/rocm/lib/librocprofiler-sdk-roctx.so.1"):
            try:
                self.lib = ctypes.CDLL(name)
                break
            except OSError:
                continue

    def push(self, label):
        if self.lib is not None:
            self.lib.roctxRangePushA(label.encode())

    def pop(self):
        if self.lib is not None:
            self.lib.roctxRangePop()


ROCTX = Roctx()


def row_label(cfg, op, nbytes):
    return "row:%s|%s|%d" % (cfg, op, nbytes)


# ---------------------------------------------------------------------------
# graphs and timing
# ---------------------------------------------------------------------------

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


def time_graphs(torch, graphs, reps, label=None):
    """Replays graphs round-robin `reps` times between two HIP events recorded
    on the stream the graphs are launched on; returns ms. `label`: a ROCTx
    range around the timed replays."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    if label:
        ROCTX.push(label)
    start.record()
    for i in range(reps):
        graphs[i % len(graphs)].replay()
    end.record()
    torch.cuda.synchronize()
    if label:
        ROCTX.pop()
    return start.elapsed_time(end)


def time_chunks(torch, graph, replays, chunks, label=None):
    """Replays `graph` chunks x replays times back to back, with a HIP event
    recorded on the launching stream between chunks; returns each chunk's ms."""
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(chunks + 1)]
    torch.cuda.synchronize()
    if label:
        ROCTX.push(label)
    evs[0].record()
    for c in range(chunks):
        for _ in range(replays):
            graph.replay()
        evs[c + 1].record()
    torch.cuda.synchronize()
    if label:
        ROCTX.pop()
    return [evs[c].elapsed_time(evs[c + 1]) for c in range(chunks)]


CHUNKS = 10


def measure_op(torch, make, nbytes, reps_target=200, cold=True, label=None):
    """Launch duration (us) of the op built by make() -> callable, over enough
    rotating input sets to exceed COLD_BYTES (cold=False: one set, cache
    resident), replayed from one graph: the graph is replayed in CHUNKS timed
    chunks of at least reps_target / CHUNKS launches each, and the result is
    the median over chunks of the mean launch duration in a chunk (the mean
    over all launches is returned beside it)."""
    nsets = 1 if (nbytes >= COLD_BYTES or not cold) else -(-COLD_BYTES // nbytes) + 1
    nsets = min(nsets, 4096)
    fns = [make() for _ in range(nsets)]
    for f in fns:
        f()
    if nsets == 1:
        fns = fns * (4 if cold else 256)  # enough nodes to amortise the graph launch
    graph = capture(torch, fns)
    time_graphs(torch, [graph], 2)
    replays = max(1, -(-reps_target // (CHUNKS * len(fns))))
    ms = time_chunks(torch, graph, replays, CHUNKS, label)
    nf = len(fns)
    per = [m * 1e3 / (replays * nf) for m in ms]
    del graph, fns
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return statistics.median(per), nsets, statistics.mean(per), CHUNKS * replays * nf


class Rows:
    """Per-op rows: each op timed alone (measure_op) under a ROCTx range."""

    def __init__(self, torch):
        self.torch, self.rows = torch, []

    def run(self, cfg, name, nbytes, make, cold=True, extra=None, quiet=False):
        us, nsets, mean, launches = measure_op(self.torch, make, nbytes, cold=cold,
                                               label=row_label(cfg, name, nbytes))
        gbs = nbytes / (us * 1e-6) / 1e9
        row = {"config": cfg, "op": name, "bytes": nbytes, "us": round(us, 3), "GB/s": round(gbs, 1),
               "frac": round(gbs / PEAK_GBS, 4), "sets": nsets, "us_mean": round(mean, 3), "launches": launches}
        if not cold:
            row["note"] = "warm (one input set)"
        for k, v in (extra or {}).items():
            row[k] = v(us) if callable(v) else v
        self.rows.append(row)
        if not quiet:
            print("%-10s %-40s %12d B %9.3f us %8.1f GB/s %6.1f%%  sets=%d" % (
                cfg, name, nbytes, us, gbs, 100 * gbs / PEAK_GBS, nsets), file=sys.stderr, flush=True)
        return row


def gen(torch, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    randn = lambda *shape: torch.randn(shape, generator=g, device="cuda", dtype=torch.float32)
    empty = lambda *shape: torch.empty(shape, device="cuda", dtype=torch.float32)
    bf16 = lambda n: (1.0 + 0.1 * randn(n)).to(torch.bfloat16)
    return g, randn, empty, bf16


# ---------------------------------------------------------------------------
# the layer step (configs[4]; configs[1] with the text-embedding gather)
# ---------------------------------------------------------------------------

class LayerStep:
    HEADS, KV_HEADS, HEAD_DIM = 16, 8, 128
    VOCAB, TEXT_HIDDEN = 151936, 2048
    EPS, THETA = 1e-6, 1e6

    def __init__(self, S, torch, T, hidden, ffn, gather, nsets=None):
        self.S, self.torch = S, torch
        self.T, self.HIDDEN, self.FFN, self.gather = T, hidden, ffn, gather
        H, D, f32 = hidden, self.HEAD_DIM, 4
        self.op_bytes = {}
        if gather:
            self.op_bytes["get_rows_bf16"] = T * (4 + self.TEXT_HIDDEN * 2 + self.TEXT_HIDDEN * f32)
        self.op_bytes.update({
            "rms_norm_mul": 2 * T * H * f32 + H * 2,
            "qk_norm_rope": 2 * (self.HEADS + self.KV_HEADS) * D * T * f32 + T * 4 + 2 * D * 2,
            "add_rms_norm_mul": 4 * T * H * f32 + H * 2,
            "swiglu": 3 * T * ffn * f32,
            "add": 3 * T * H * f32,
        })
        self.step_bytes = sum(self.op_bytes.values())
        self.nsets = nsets or max(2, -(-COLD_BYTES // self.step_bytes) + 1)
        g, randn, empty, bf16 = gen(torch, SEED)
        dev = "cuda"
        if gather:
            self.table = (0.02 * randn(self.VOCAB, self.TEXT_HIDDEN)).to(torch.bfloat16)
        self.w_in, self.w_post = bf16(H), bf16(H)
        self.wq, self.wk = bf16(D), bf16(D)
        self.pos = torch.arange(T, dtype=torch.int32, device=dev)
        self.sets = []
        for _ in range(self.nsets):
            s = dict(x=randn(T, H), q=randn(T, self.HEADS, D), k=randn(T, self.KV_HEADS, D), proj=randn(T, H),
                     gate=randn(T, ffn), up=randn(T, ffn), mlp=randn(T, H))
            if gather:
                s.update(ids=torch.randint(0, self.VOCAB, (T,), generator=g, device=dev, dtype=torch.int32),
                         emb=empty(T, self.TEXT_HIDDEN))
            s.update(normed=empty(T, H), qo=torch.empty_like(s["q"]), ko=torch.empty_like(s["k"]),
                     resid=empty(T, H), mlp_in=empty(T, H), act=empty(T, ffn), out=empty(T, H))
            self.sets.append(s)
        torch.cuda.synchronize()

    def ops(self, s):
        S, c = self.S, self.sets[s]
        ops = [("get_rows_bf16", lambda: S.get_rows(self.table, c["ids"], out=c["emb"]))] if self.gather else []
        return ops + [
            ("rms_norm_mul", lambda: S.rms_norm_mul(c["x"], self.w_in, self.EPS, out=c["normed"])),
            ("qk_norm_rope", lambda: S.qk_norm_rope(c["q"], c["k"], self.wq, self.wk, self.EPS, self.pos,
                                                    self.HEAD_DIM, self.THETA, q_out=c["qo"], k_out=c["ko"])),
            ("add_rms_norm_mul", lambda: S.add_rms_norm_mul(c["x"], c["proj"], self.w_post, self.EPS,
                                                            out=c["mlp_in"], sum_out=c["resid"])),
            ("swiglu", lambda: S.swiglu(c["gate"], c["up"], out=c["act"])),
            ("add", lambda: S.add(c["resid"], c["mlp"], out=c["out"])),
        ]

    def time_steps(self, steps, warmup, label=None):
        """ms per step over exactly `steps` steps, the sets in rotation: a graph
        of all nsets steps back to back replayed steps // nsets times, then a
        graph of the first steps % nsets. Checks that replays reproduce the
        eager results bit for bit."""
        torch = self.torch
        per_set = [self.ops(s) for s in range(self.nsets)]
        for ops in per_set:
            for _, f in ops:
                f()
        torch.cuda.synchronize()
        ref_out, ref_q = self.sets[0]["out"].clone(), self.sets[0]["qo"].clone()
        full = capture(torch, [f for ops in per_set for _, f in ops])
        rems = {k % self.nsets: capture(torch, [f for ops in per_set[:k % self.nsets] for _, f in ops])
                for k in (warmup, steps) if k % self.nsets}

        def run(k):
            for _ in range(k // self.nsets):
                full.replay()
            if k % self.nsets:
                rems[k % self.nsets].replay()

        run(warmup)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        if label:
            ROCTX.push(label)
        start.record()
        run(steps)
        end.record()
        torch.cuda.synchronize()
        if label:
            ROCTX.pop()
        assert torch.equal(self.sets[0]["out"], ref_out) and torch.equal(self.sets[0]["qo"], ref_q)
        del full, rems
        return start.elapsed_time(end) / steps


def step_op_rows(R, S, torch, cfg, T, H, F_, seed):
    """The configs[4] step's ops alone, each on its own rotating sets."""
    g, randn, empty, bf16 = gen(torch, seed)
    f32 = 4

    def norm(add):
        def make():
            a, b, w, y, s = randn(T, H), randn(T, H), bf16(H), empty(T, H), empty(T, H)
            if add:
                return lambda: S.add_rms_norm_mul(a, b, w, 1e-6, out=y, sum_out=s)
            return lambda: S.rms_norm_mul(a, w, 1e-6, out=y)
        return make

    def qk():
        q, k = randn(T, 16, 128), randn(T, 8, 128)
        qo, ko, wq, wk = torch.empty_like(q), torch.empty_like(k), bf16(128), bf16(128)
        pos = torch.arange(T, dtype=torch.int32, device="cuda")
        return lambda: S.qk_norm_rope(q, k, wq, wk, 1e-6, pos, 128, 1e6, q_out=qo, k_out=ko)

    def sw():
        a, b, y = randn(T, F_), randn(T, F_), empty(T, F_)
        return lambda: S.swiglu(a, b, out=y)

    def add():
        a, b, y = randn(T, H), randn(T, H), empty(T, H)
        return lambda: S.add(a, b, out=y)

    return {
        "rms_norm_mul": R.run(cfg, "rms_norm_mul [%d,%d]" % (H, T), 2 * T * H * f32 + H * 2, norm(False)),
        "qk_norm_rope": R.run(cfg, "qk_norm_rope q[128,16,%d] k[128,8,%d]" % (T, T),
                              2 * 24 * 128 * T * f32 + T * 4 + 512, qk),
        "add_rms_norm_mul": R.run(cfg, "add_rms_norm_mul+sum [%d,%d]" % (H, T), 4 * T * H * f32 + H * 2,
                                  norm(True)),
        "swiglu": R.run(cfg, "swiglu [%d,%d]" % (F_, T), 3 * T * F_ * f32, sw),
        "add": R.run(cfg, "add [%d,%d]" % (H, T), 3 * T * H * f32, add),
    }


# ---------------------------------------------------------------------------
# Q8_0 gather->sum and get_rows; configs[3]: vocoder activations
# ---------------------------------------------------------------------------

def q8_rows(R, S, torch, cfg, seed, kind="q8_0"):
    """configs[2]'s gathers; kind "q5_k": the same shapes over Q5_K tables (the
    Q5_K_MIXED profile's)."""
    import numpy as np
    import formats as F
    g, randn, empty, bf16 = gen(torch, seed)
    rng = np.random.default_rng(seed)
    f32 = 4
    if kind == "q5_k":
        row, synth, wrap = 1024 // 256 * 176, F.q5_k_synthetic, S.Q5KTensor
    else:
        row, synth, wrap = 1024 // 32 * 34, F.q8_0_synthetic, S.Q8Tensor
    # Each input set has its own tables, so the rotation exceeds the Infinity
    # Cache and every launch fetches its rows from HBM.
    keep = []

    def tables(n):
        raw = torch.from_numpy(np.stack([synth(rng, 2048, 1024) for _ in range(n)])).cuda()
        keep.append(raw)
        return [wrap(raw[t], 1024) for t in range(n)]

    def make_sum():
        tabs = tables(16)
        codes = torch.randint(0, 2048, (16, 4096), generator=g, device="cuda", dtype=torch.int32)
        out = empty(4096, 1024)
        return lambda: S.get_rows_sum(tabs, codes, out=out)

    def make_q8():
        tabs = tables(1)
        ids = torch.randint(0, 2048, (4096,), generator=g, device="cuda", dtype=torch.int32)
        out = empty(4096, 1024)
        return lambda: S.get_rows(tabs[0], ids, out=out)

    def compulsory(groups):
        touched = groups * 2048 * (1.0 - (1.0 - 1.0 / 2048) ** 4096)  # expected distinct rows
        return int(touched * row) + 4096 * (groups * 4 + 1024 * f32)

    out = []
    for name, groups, make in (("get_rows_sum %s 16x[1024,2048] x4096" % kind, 16, make_sum),
                               ("get_rows %s [1024,2048] x4096" % kind, 1, make_q8)):
        logical = 4096 * (groups * (row + 4) + 1024 * f32)
        cb = compulsory(groups)
        out.append(R.run(cfg, name, logical, make, extra={
            "bytes_kind": "logical (every looked-up row per lookup)", "compulsory_bytes": cb,
            "compulsory_GB/s": lambda us, cb=cb: round(cb / (us * 1e-6) / 1e9, 1)}))
        keep.clear()
    return out


def vocoder_rows(R, S, torch, cfg, seed, shapes=((512, 8192), (256, 32768), (128, 131072)), variants=False):
    g, randn, empty, bf16 = gen(torch, seed)
    out = []
    for C, T in shapes:
        n = C * T

        def make_snake(C=C, T=T):
            x, y = randn(T, C), empty(T, C)
            al = torch.exp(torch.empty(C, device="cuda").uniform_(math.log(0.1), math.log(10.0), generator=g))
            return lambda: S.snake(x, al, out=y)

        def make_beta(C=C, T=T):
            x, y = randn(T, C), empty(T, C)
            la = torch.empty(C, device="cuda").uniform_(-3.0, 3.0, generator=g)
            lb = torch.empty(C, device="cuda").uniform_(-3.0, 3.0, generator=g)
            return lambda: S.snake_beta(x, la, lb, out=y)

        def make_guarded(C=C, T=T):
            x, y = randn(T, C), empty(T, C)
            al = torch.exp(torch.empty(C, device="cuda").uniform_(-3.0, 3.0, generator=g))
            return lambda: S.snake_guarded(x, al, out=y)

        def make_leaky(C=C, T=T, with_s=False):
            a, b, y, s = randn(T, C), randn(T, C), empty(T, C), empty(T, C)
            return lambda: S.add_leaky_relu(a, b, 0.1, out=y, sum_out=s if with_s else None)

        def make_branch(C=C, T=T):
            ts, y = [randn(T, C) for _ in range(3)], empty(T, C)
            return lambda: S.sum_scale_leaky_relu(ts, 1.0 / 3.0, 0.1, out=y)

        def make_bare(C=C, T=T):
            x, y = randn(T, C), empty(T, C)
            return lambda: S.leaky_relu(x, 0.1, out=y)

        def make_bias(C=C, T=T):
            # the time-major vocoder's conv bias: ggml [T, C] + [1, C], one
            # value per row (vits/waveform-decoder.cpp:118-121)
            x, y, b = randn(C, T), empty(C, T), randn(C, 1)
            return lambda: S.add(x, b, out=y)

        def make_tail(C=C, T=T, resid=False):
            # the time-major conv's tail in one launch (vits/waveform-
            # decoder.cpp:111,118-121,146-150): the GEMM output ggml [C, T]
            # transposed, + the [1, C] bias (+ the residual), leaky-ReLU
            x, y, b = randn(T, C), empty(C, T), randn(C, 1)
            r, s_ = (randn(C, T), empty(C, T)) if resid else (None, None)
            v = x.t()
            return lambda: S.cont_add_leaky_relu(v, b, r, 0.1, out=y, sum_out=s_)

        def make_cont(C=C, T=T):
            # ggml_cont(ggml_transpose(x)), x = ggml [C, T] (torch (T, C)):
            # the time-major copy in front of each vocoder convolution
            x, y = randn(T, C), empty(C, T)
            v = x.t()
            return lambda: S.cpy(v, out=y)

        def make_im2col(C=C, T=T, K=3, d0=1, chmajor=False, f16=False):
            # the column matrix in front of a convolution GEMM: x ggml [T, C]
            # time-contiguous (vits/waveform-decoder.cpp:104, same-length
            # padding), or the transposed view of a channel-major [C, T]
            # activation, causal padding (qwen3-tts/codec.cpp:94-96)
            x = randn(T, C).t() if chmajor else randn(C, T)
            p0 = (K - 1) * d0 if chmajor else (K - 1) * d0 // 2
            y = torch.empty((1, S.conv_out_len(T, K, 1, p0, d0), C * K), device="cuda",
                            dtype=torch.float16 if f16 else torch.float32)
            return lambda: S.im2col(x, K, 1, p0, d0, out=y)

        def make_col2im(C=C, T=T):
            # the upsampling transposed convolution's scatter-back into this
            # shape (vits/operations.cpp:118-140): kernel 2*stride, padding
            # stride/2; stride 8 into [512,8192] and [256,32768], 2 into
            # [128,131072] (the VITS decoder's upsampling stages)
            st = 2 if T >= 131072 else 8
            K, P = 2 * st, st // 2
            L = (T + 2 * P - K) // st + 1
            c, y = randn(L, K * C), empty(C, T)
            return lambda: S.col2im_1d(c, st, C, P, out=y)

        def make_spread(C=C, T=T):
            # kokoro's transposed convolution front (kokoro/operations.cpp:
            # 190-196): stride - 1 zero frames after every frame of [C, 1, L]
            st = 2 if T >= 131072 else 8
            x, y = randn(T // st, 1, C), empty(T // st, st, C)
            return lambda: S.pad_ext(x, [0, 0], [0, st - 1], out=y)

        def make_double(C=C, T=T):
            # kokoro's upsample_nearest_2x (:113-120): [C, 1, T/2] to [C, 2, T/2]
            x, y = randn(T // 2, 1, C), empty(T // 2, 2, C)
            return lambda: S.repeat(x, (T // 2, 2, C), out=y)

        def make_edge(C=C, T=T):
            # edge padding along time of a time-contiguous activation
            # (codec-encoder.cpp:351): rows of T + 7 values, not 16-byte aligned
            x, y = randn(C, T), empty(C, T + 7)
            return lambda: S.pad_ext(x, [3], [4], out=y)

        out.append(R.run(cfg, "snake [%d,%d]" % (C, T), 8 * n + 4 * C, make_snake))
        out.append(R.run(cfg, "snake_beta [%d,%d]" % (C, T), 8 * n + 8 * C, make_beta))
        out.append(R.run(cfg, "add_leaky_relu [%d,%d]" % (C, T), 12 * n, make_leaky))
        out.append(R.run(cfg, "add_leaky_relu+sum [%d,%d]" % (C, T), 16 * n, lambda: make_leaky(with_s=True)))
        out.append(R.run(cfg, "cont(transpose) [%d,%d]" % (C, T), 8 * n, make_cont))
        out.append(R.run(cfg, "add bias[1,C] time-major [%d,%d]" % (C, T), 8 * n + 4 * C, make_bias))
        out.append(R.run(cfg, "conv tail: cont(transpose)+bias->leaky [%d,%d]" % (C, T), 8 * n + 4 * C,
                         make_tail))
        out.append(R.run(cfg, "conv tail: cont(transpose)+bias+residual->leaky, sum [%d,%d]" % (C, T),
                         16 * n + 4 * C, lambda: make_tail(resid=True)))
        out.append(R.run(cfg, "im2col K=3 [%d,%d]" % (C, T), 4 * n + 4 * 3 * n, make_im2col))
        out.append(R.run(cfg, "im2col K=3 channel-major view [%d,%d]" % (C, T),
                         4 * n + 4 * 3 * (T + 2) * C, lambda: make_im2col(chmajor=True)))
        st = 2 if T >= 131072 else 8
        out.append(R.run(cfg, "pad: spread x%d [%d,1,%d]" % (st, C, T // st), 4 * n // st * (1 + st), make_spread))
        out.append(R.run(cfg, "repeat: frames x2 [%d,1,%d]" % (C, T // 2), 6 * n, make_double))
        out.append(R.run(cfg, "pad_ext: time +3/+4 [%d,%d]" % (T, C), 4 * n + 4 * C * (T + 7), make_edge))
        out.append(R.run(cfg, "col2im_1d K=%d s=%d [%d,%d]" % (2 * st, st, C, T),
                         4 * 2 * st * C * ((T + st - 2 * st) // st + 1) + 4 * n, make_col2im))
        if (C, T) == (128, 131072):
            out.append(R.run(cfg, "im2col K=11 d=5 [%d,%d]" % (C, T), 4 * n + 4 * 11 * n,
                             lambda: make_im2col(K=11, d0=5)))
            out.append(R.run(cfg, "im2col K=7 d=3 f16 [%d,%d]" % (C, T), 4 * n + 2 * 7 * n,
                             lambda: make_im2col(K=7, d0=3, f16=True)))
        if variants:
            # the size's streaming floor: one read and one write with no work
            out.append(R.run(cfg, "copy-like floor: bare leaky [%d,%d]" % (C, T), 8 * n, make_bare))
            out.append(R.run(cfg, "snake_guarded [%d,%d]" % (C, T), 8 * n + 4 * C, make_guarded))
            out.append(R.run(cfg, "branch mean 3->scale->leaky [%d,%d]" % (C, T), 16 * n, make_branch))
    return out


def talker_input_rows(R, S, torch, cfg, seed, T=8192, H=2048, at=16):
    """The talker's prefill input assembly (qwen3-tts/talker.cpp:86-118):
    ggml_acc of a codec run of T - at positions into the [H, T] text stream
    from position `at`, out of place (a's copy with the run added: a read,
    the run read, y written) and in ggml's inplace form (the window alone)."""
    g, randn, empty, bf16 = gen(torch, seed)
    nb1 = 4 * H

    def make(inplace):
        def build():
            a, b, y = randn(T, H), randn(T - at, H), empty(T, H)
            if inplace:
                return lambda: S.acc(a, b, nb1, nb1 * T, nb1 * T, at * nb1, inplace=True)
            return lambda: S.acc(a, b, nb1, nb1 * T, nb1 * T, at * nb1, out=y)
        return build
    n, m = T * H, (T - at) * H
    R.run(cfg, "acc: codec run +%d@%d into text [%d,%d]" % (T - at, at, H, T), 4 * (2 * n + m), make(False))
    R.run(cfg, "acc inplace: codec run +%d@%d [%d,%d]" % (T - at, at, H, T), 12 * m, make(True))


def istft_rows(R, S, torch, cfg, seed, seconds=5, rate=24000, n_fft=20, hop=5):
    """Kokoro's inverse short-time transform (kokoro/decoder-host.cpp:28-100) of
    a `seconds`-long utterance at Kokoro's n_fft 20 / hop 5: the generator's
    spectrum (n_fft + 2 values per frame) read, the waveform written."""
    g, randn, empty, bf16 = gen(torch, seed)
    frames = seconds * rate // hop + 1

    def make():
        spec = torch.rand((frames, n_fft + 2), generator=g, device="cuda") * 5 - 3
        y = empty((frames - 1) * hop)
        return lambda: S.inverse_stft(spec, n_fft, hop, out=y)
    R.run(cfg, "inverse_stft n_fft %d hop %d, %d s at %d Hz" % (n_fft, hop, seconds, rate),
          4 * frames * (n_fft + 2) + 4 * (frames - 1) * hop, make)


def source_rows(R, S, torch, cfg, seed, seconds=5, rate=24000, H=9, scale=300, n_fft=20, hop=5):
    """Kokoro's harmonic source and its spectrum (kokoro/source.cpp:60-184) for
    a `seconds`-long utterance at Kokoro's dimensions: f0 and the noise draws
    read, the excitation and the spectrum written."""
    g, randn, empty, bf16 = gen(torch, seed)
    L = seconds * rate // scale
    U, frames = L * scale, L * scale // hop + 1

    def make():
        f0 = torch.rand((L,), generator=g, device="cuda") * 300 + 60
        mw, ri = randn(H) * 0.5, torch.rand((H,), generator=g, device="cuda")
        noise = randn(U, H)
        out = (empty(U), empty(frames, n_fft + 2))
        return lambda: S.harmonic_source(f0, mw, 0.1, ri, noise, rate=rate, scale=scale, sine_amp=0.1,
                                         noise_std=0.003, voiced_threshold=10.0, n_fft=n_fft, hop=hop, out=out)
    R.run(cfg, "harmonic_source %d harmonics, %d s at %d Hz" % (H, seconds, rate),
          4 * (L + U * H + U + frames * (n_fft + 2)), make)


def mel_rows(R, S, torch, cfg, seed, seconds=10, rate=24000):
    """The Qwen3-TTS speaker encoder's log-mel (qwen3-tts/mel.cpp:174-299) of a
    `seconds`-long reference clip at the production parameters: the PCM read,
    [128, frames] log energies written (the filterbank, 263 KB, cache-resident)."""
    g, randn, empty, bf16 = gen(torch, seed)
    ns = seconds * rate
    frames = 1 + (ns + 2 * 384 - 1024) // 256

    def make():
        pcm = randn(ns) * 0.2
        fb = torch.from_numpy(S.mel_filterbank(rate, 1024, 128, 0.0, 12000.0)).cuda()
        y = empty(frames, 128)
        return lambda: S.log_mel(pcm, fb, 1024, 256, 1024, out=y)
    R.run(cfg, "log_mel n_fft 1024 hop 256 128 bins, %d s at %d Hz" % (seconds, rate), 4 * ns + 4 * frames * 128,
          make)


def floor_rows(R, S, torch, seed=SEED + 8):
    """Same-run floors the op rows are read against, each timed as the op rows
    are (cold rotating sets, HIP graph, median of chunks):
      - copy [C,T]: shp_cpy of an F32 tensor (one read and one write of every
        element, no arithmetic) at each configs[3] shape and at [2048,8192];
      - write-only [1024,4096]: torch's fill_ of the gathers' output tensor
        (no reads at all);
      - id-then-write: shp_get_rows of 4096 ids from an 8-row Q8_0 table
        [1024,8] (8.7 KB, cache-resident), i.e. the gather's id load, row
        address and dequantised store with the table fetch taken away.
    Returns {name: row}."""
    import numpy as np
    import formats as F
    g, randn, empty, bf16 = gen(torch, seed)
    out = {}
    for C, T in ((512, 8192), (256, 32768), (128, 131072), (2048, 8192)):
        def make_copy(C=C, T=T):
            x, y = randn(T, C), empty(T, C)
            return lambda: S.cpy(x, out=y)
        name = "copy [%d,%d]" % (C, T)
        out[name] = R.run("floor", name, 8 * C * T, make_copy)

    def make_fill():
        y = empty(4096, 1024)
        return lambda: y.fill_(1.0)
    out["write-only [1024,4096]"] = R.run("floor", "write-only [1024,4096]", 4 * 4096 * 1024, make_fill)
    rng = np.random.default_rng(seed)

    def make_idw():
        tab = S.Q8Tensor(torch.from_numpy(F.q8_0_synthetic(rng, 8, 1024)).cuda(), 1024)
        ids = torch.randint(0, 8, (4096,), generator=g, device="cuda", dtype=torch.int32)
        y = empty(4096, 1024)
        return lambda: S.get_rows(tab, ids, out=y)
    name = "id-then-write: get_rows q8_0 [1024,8] x4096"
    out[name] = R.run("floor", name, 4096 * (4 + 1024 * 4), make_idw)
    return out


def link_floors(rows, floors):
    """Adds to each op row the floor it is read against: 'of_floor' = the
    row's GB/s over the floor's (streams: the copy of the same shape), or for
    the plain gathers 'of_floor_time' = floor us / row us (the row's own
    launch against the write-only and id-then-write launches)."""
    for row in rows:
        op, cfg = row["op"], row["config"]
        m = re.search(r"\[(\d+),(\d+)\]$", op)
        m3 = re.search(r"\[(\d+),1,(\d+)\]$", op)
        if cfg == "configs[3]" and m3 and op.startswith(("pad: spread", "repeat: frames")):
            # [C, 1, L] spread or doubled into [C, k, L]: the copy of the output's shape
            k = int(re.search(r"x(\d+)", op).group(1))
            f = floors.get("copy [%s,%d]" % (m3.group(1), k * int(m3.group(2))))
            if f is not None:
                row["floor"] = f["op"]
                row["of_floor"] = round(row["GB/s"] / f["GB/s"], 4)
        elif cfg in ("configs[3]", "configs[4]") and m and not op.startswith(("swiglu", "add [", "qk_")):
            # ggml [T, C] names (the time-axis padding) take the copy of [C, T]
            f = floors.get("copy [%s,%s]" % m.groups()) or floors.get("copy [%s,%s]" % m.groups()[::-1])
            if f is not None:
                row["floor"] = f["op"]
                row["of_floor"] = round(row["GB/s"] / f["GB/s"], 4)
        elif cfg == "configs[2]" and op.startswith("get_rows "):
            row["floor"] = "write-only [1024,4096]; id-then-write: get_rows q8_0 [1024,8] x4096"
            row["of_floor_time"] = [round(floors["write-only [1024,4096]"]["us"] / row["us"], 4),
                                    round(floors["id-then-write: get_rows q8_0 [1024,8] x4096"]["us"] / row["us"], 4)]


# ---------------------------------------------------------------------------
# decode step: 28 layers x (add+norm, qk-norm+rope, add+norm, swiglu) at T=1
# ---------------------------------------------------------------------------

DECODE_TOTAL = 38  # configs[0]: the token at position 37 attends over 38 keys


def decode_layer_us(S, torch, layers=28, reps=50, kv=False, total=DECODE_TOTAL, streams=1, label=None):
    """us per talker layer of the decode step's non-GEMM ops, replayed as one
    graph of `layers` layers (median over CHUNKS timed chunks of replays).
    kv: qk-norm+rope also writes this step's k and v into the layer's cache
    (slot total-1) and the step adds the attention softmax over `total` keys
    for the 16 heads (5 launches per layer). streams: concurrent decode
    streams batched into each op (one token each), each at position total-1."""
    assert not (kv and streams != 1), "the KV variant models one stream"
    g, randn, empty, bf16 = gen(torch, SEED + 1)
    L = []
    for _ in range(layers):
        n = streams
        c = dict(a=randn(n, 1024), b=randn(n, 1024), w1=bf16(1024), w2=bf16(1024), wq=bf16(128),
                 wk=bf16(128), q=randn(n, 16, 128), k=randn(n, 8, 128), proj=randn(n, 1024),
                 gate=randn(n, 3072), up=randn(n, 3072), s1=empty(n, 1024), y1=empty(n, 1024),
                 s2=empty(n, 1024), y2=empty(n, 1024), qo=empty(n, 16, 128), ko=empty(n, 8, 128),
                 act=empty(n, 3072))
        if kv:
            c.update(v=randn(1, 8, 128), kc=randn(total, 8, 128), vc=randn(total, 8, 128),
                     sc=randn(16, 1, total), p=empty(16, 1, total))
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
    ms = time_chunks(torch, graph, max(1, reps // CHUNKS), CHUNKS, label)
    return statistics.median(ms) * 1e3 / (max(1, reps // CHUNKS) * layers)


def decode_layer_graph_us(S, torch, layers=28, reps=50, total=DECODE_TOTAL, label=None):
    """us per talker layer of the one-token decode step run through the
    node-run executor: `layers` chained copies of decoder_layer's non-GEMM node
    list in the reference's expand order (qwen3_layer.decoder_layer_nodes: the
    projections, attention scores and outputs as leaves, the KV cache written
    at slot total-1, the softmax over `total` keys, each layer's output add
    feeding the next layer's input norm), planned by shp_graph_compute inside
    one HIP graph capture and replayed (median over CHUNKS timed chunks).
    Returns (us per layer, the plan's launch count)."""
    import qwen3_layer as Q
    g_, randn, empty, bf16 = gen(torch, SEED + 2)
    g = S.Graph()
    x, outs = randn(1, 1024), []
    for _ in range(layers):
        leaves = dict(q=randn(1, 16, 128), k=randn(1, 8, 128), v=randn(1, 8, 128), scores=randn(16, 1, total),
                      attn=randn(1, 1024), gate=randn(1, 3072), up=randn(1, 3072), mlp=randn(1, 1024),
                      w_in=bf16(1024), w_post=bf16(1024), wq=bf16(128), wk=bf16(128),
                      pos=torch.full((1,), total - 1, dtype=torch.int32, device="cuda"),
                      kcache=randn(total, 8, 128), vcache=randn(total, 8, 128))
        o, _ = Q.decoder_layer_nodes(g, x, leaves, total=total)
        outs += o
        x = o[-1]
    launches = sum(1 for k, *_ in g.plan(*outs) if k not in ("nop", "unsupported"))
    arr, n, keep = g.nodes(*outs)
    lib, fns = S.load(), [lambda: S._check(S.load().shp_graph_compute(arr, n, S._stream()), "graph_compute")]
    fns[0]()
    graph = capture(torch, fns)
    time_graphs(torch, [graph], 5)
    ms = time_chunks(torch, graph, max(1, reps // CHUNKS), CHUNKS, label)
    del graph, keep, lib
    return statistics.median(ms) * 1e3 / (max(1, reps // CHUNKS) * layers), launches


def decode_layer_bytes(streams=1, kv=False, total=DECODE_TOTAL):
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

def cpu_share():
    """CPUs this process may run on: the affinity mask, the cgroup v2 quota
    (as the reference's available_cpu_parallelism, cpu-parallelism.h:8-21),
    and the per-GPU CPU share of the GPU box."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
            if q != "max":
                quota = max(1, math.ceil(int(q) / int(period)))
    except (OSError, ValueError):
        pass
    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    n = min(affinity, quota or affinity)
    return {"affinity_cpus": affinity, "cgroup_quota_cpus": quota, "available_cpus": n,
            "threads_used": max(1, min(n, BOX_CPU_SHARE)), "cpu_model": model}


def cpu_baseline(step, torch, seconds):
    import numpy as np
    import ggml_ref as R

    c = step.sets[0]
    h = lambda t: t.detach().cpu().contiguous().numpy()
    bits = lambda t: h(t.view(torch.int16)).view(np.uint16)
    x, q, k, proj, gate, up, mlp = (h(c[n]) for n in ("x", "q", "k", "proj", "gate", "up", "mlp"))
    w_in, w_post, wq, wk = bits(step.w_in), bits(step.w_post), bits(step.wq), bits(step.wk)
    pos = h(step.pos)
    eps, theta = np.float32(step.EPS), np.float32(step.THETA)

    g = R.Graph()
    R.rms_norm_w(g, x, w_in, eps, R.BF16)
    R.qk_norm_rope(g, q, k, wq, wk, eps, pos, step.HEAD_DIM, theta, R.BF16)
    s, _ = R.add_rms_norm_w(g, x, proj, w_post, eps, R.BF16)
    R.swiglu(g, gate, up)
    g.add(s, mlp)

    share = cpu_share()
    nth = share["threads_used"]
    probe = g.time(nth, 1, 1)[0]
    reps = int(max(3, min(200, 0.5 * seconds / max(probe, 1e-6))))
    t_many = statistics.median(g.time(nth, 0, reps))
    # max(1, N/2) threads is the reference's default CPU parallelism
    # (cpu-parallelism.h:24-44); N and 1 bracket it.
    half = max(1, nth // 2)
    t_half = statistics.median(g.time(half, 0, max(3, reps // 2)))
    probe1 = g.time(1, 0, 1)[0]
    reps1 = int(max(1, min(50, 0.25 * seconds / max(probe1, 1e-6))))
    t_one = statistics.median(g.time(1, 0, reps1))
    gbs = lambda t: step.step_bytes / t / 1e9
    out = {
        "value": round(gbs(t_many), 2), "unit": "GB/s", "cores": nth, "kind": "port",
        "sample": "the configs[4] step (norm, qk-norm+rope, add+norm, swiglu, add; %d ggml nodes, %d B) on the "
                  "ggml-CPU restatement (oracle/ggml_cpu_ref.c, -O3, ggml's ith/nth row split), median of %d reps "
                  "at %d threads; %d threads (the reference's default, N/2): %.2f GB/s; 1 thread: %.2f GB/s "
                  "(median of %d). This box: %s, %d CPUs in the affinity mask, cgroup quota %s; one GPU's share "
                  "of the box is %d CPUs, so at most %d threads are used" % (
                      len(g.nodes), step.step_bytes, reps, nth, half, gbs(t_half), gbs(t_one), reps1,
                      share["cpu_model"], share["affinity_cpus"], share["cgroup_quota_cpus"], BOX_CPU_SHARE,
                      BOX_CPU_SHARE),
        "ms_per_step": round(t_many * 1e3, 3), "value_half_threads": round(gbs(t_half), 3), "half_threads": half,
        "value_1thread": round(gbs(t_one), 3),
    }
    out.update(share)
    return out


# ---------------------------------------------------------------------------
# CPU baseline per op: each row's node run on the restatement
# ---------------------------------------------------------------------------

def _time_cpu(g, nth, budget):
    """Seconds per run of the restatement graph `g` at `nth` threads: one
    warm-up run and one timed run, then the median of as many more as fit in
    `budget` seconds (at most 20)."""
    t = g.time(nth, 1, 1)[0]
    reps = int(min(20, budget / max(t, 1e-7)))
    if reps >= 3:
        t = statistics.median(g.time(nth, 0, reps))
    return t


def cpu_op_builders(seed=SEED + 9):
    """[(config, op name, algorithmic bytes, build(g))] for every row the bench
    line carries, named as its GPU row: the same node runs over host inputs of
    the same shapes (one pool of N(0,1) values, each operand a differently
    offset window of it), as the reference's graphs build them for ggml-CPU."""
    import numpy as np
    import formats as F
    import ggml_ref as R
    rng = np.random.default_rng(seed)
    pool = rng.standard_normal(8192 * 6144 + 4096, dtype=np.float32)
    cursor = [0]

    def take(*shape):
        n = math.prod(shape)
        o = (cursor[0] * 61) % 4096
        cursor[0] += 1
        return pool[o:o + n].reshape(shape)

    bf16 = lambda n: F.f32_to_bf16_bits(rng.normal(1.0, 0.1, n).astype(np.float32))
    eps, theta, f32 = np.float32(1e-6), np.float32(1e6), 4
    out = []
    T, H, F_ = 8192, 2048, 6144
    cfg = "configs[4]"
    out.append((cfg, "rms_norm_mul [%d,%d]" % (H, T), 2 * T * H * f32 + H * 2,
                lambda g: R.rms_norm_w(g, take(T, H), bf16(H), eps, R.BF16)))
    out.append((cfg, "qk_norm_rope q[128,16,%d] k[128,8,%d]" % (T, T), 2 * 24 * 128 * T * f32 + T * 4 + 512,
                lambda g: R.qk_norm_rope(g, take(T, 16, 128), take(T, 8, 128), bf16(128), bf16(128), eps,
                                         np.arange(T, dtype=np.int32), 128, theta, R.BF16)))
    out.append((cfg, "add_rms_norm_mul+sum [%d,%d]" % (H, T), 4 * T * H * f32 + H * 2,
                lambda g: R.add_rms_norm_w(g, take(T, H), take(T, H), bf16(H), eps, R.BF16)))
    out.append((cfg, "swiglu [%d,%d]" % (F_, T), 3 * T * F_ * f32, lambda g: R.swiglu(g, take(T, F_), take(T, F_))))
    out.append((cfg, "add [%d,%d]" % (H, T), 3 * T * H * f32, lambda g: g.add(take(T, H), take(T, H))))
    nm = 10 * 24000
    fbm = R.mel_filterbank(24000, 1024, 128, 0.0, 12000.0)
    out.append(("configs[3]", "log_mel n_fft 1024 hop 256 128 bins, 10 s at 24000 Hz",
                4 * nm + 4 * (1 + (nm + 768 - 1024) // 256) * 128,
                lambda g: g.log_mel((rng.standard_normal(nm) * 0.2).astype(np.float32), fbm, 1024, 256, 1024)))
    Ls, Us = 5 * 24000 // 300, 5 * 24000
    out.append(("configs[3]", "harmonic_source 9 harmonics, 5 s at 24000 Hz",
                4 * (Ls + Us * 9 + Us + (Us // 5 + 1) * 22),
                lambda g: g.harmonic_source(rng.uniform(60, 360, Ls).astype(np.float32),
                                            rng.normal(0, 0.5, 9).astype(np.float32), np.float32(0.1),
                                            rng.uniform(0, 1, 9).astype(np.float32),
                                            rng.standard_normal((Us, 9)).astype(np.float32), rate=24000, scale=300,
                                            sine_amp=np.float32(0.1), noise_std=np.float32(0.003),
                                            voiced_threshold=np.float32(10.0), n_fft=20, hop=5)))
    fr = 5 * 24000 // 5 + 1
    out.append(("configs[3]", "inverse_stft n_fft 20 hop 5, 5 s at 24000 Hz", 4 * fr * 22 + 4 * (fr - 1) * 5,
                lambda g: g.inverse_stft(rng.uniform(-3, 2, (fr, 22)).astype(np.float32), 20, 5)))
    at = 16
    out.append((cfg, "acc: codec run +%d@%d into text [%d,%d]" % (T - at, at, H, T), 4 * (2 * T * H + (T - at) * H),
                lambda g: g.acc(take(T, H), take(T - at, H), 4 * H, 4 * H * T, 4 * H * T, at * 4 * H)))

    for kind, synth, rb, typ in (("q8_0", F.q8_0_synthetic, 1024 // 32 * 34, R.Q8_0),
                                 ("q5_k", F.q5_k_synthetic, 1024 // 256 * 176, R.Q5_K)):
        def gsum(g, synth=synth, typ=typ):
            tabs = [synth(rng, 2048, 1024) for _ in range(16)]
            codes = rng.integers(0, 2048, (16, 4096)).astype(np.int32)
            return R.sum_code_embeddings(g, tabs, typ, 1024, codes)

        def gone(g, synth=synth, typ=typ):
            return g.get_rows(synth(rng, 2048, 1024), typ, 1024, rng.integers(0, 2048, 4096).astype(np.int32))
        out.append(("configs[2]", "get_rows_sum %s 16x[1024,2048] x4096" % kind, 4096 * (16 * (rb + 4) + 1024 * f32),
                    gsum))
        out.append(("configs[2]", "get_rows %s [1024,2048] x4096" % kind, 4096 * (rb + 4 + 1024 * f32), gone))

    for C, Tv in ((512, 8192), (256, 32768), (128, 131072)):
        n = C * Tv
        al = lambda C=C: np.exp(rng.uniform(math.log(0.1), math.log(10.0), C)).astype(np.float32)
        lg = lambda C=C: rng.uniform(-3.0, 3.0, C).astype(np.float32)
        cfg = "configs[3]"
        out.append((cfg, "snake [%d,%d]" % (C, Tv), 8 * n + 4 * C,
                    lambda g, C=C, Tv=Tv, al=al: R.snake(g, take(Tv, C), al())))
        out.append((cfg, "snake_beta [%d,%d]" % (C, Tv), 8 * n + 8 * C,
                    lambda g, C=C, Tv=Tv, lg=lg: R.snake_beta(g, take(Tv, C), lg(), lg())))
        # ggml-CPU's add node always writes the sum, so one CPU run serves both rows
        for name, nbytes in (("add_leaky_relu [%d,%d]" % (C, Tv), 12 * n),
                             ("add_leaky_relu+sum [%d,%d]" % (C, Tv), 16 * n)):
            out.append((cfg, name, nbytes,
                        lambda g, C=C, Tv=Tv: R.add_leaky(g, take(Tv, C), take(Tv, C), np.float32(0.1))))
        out.append((cfg, "cont(transpose) [%d,%d]" % (C, Tv), 8 * n,
                    lambda g, C=C, Tv=Tv: g.cont_f32(take(Tv, C), [Tv, C], [4 * C, 4])))
        out.append((cfg, "add bias[1,C] time-major [%d,%d]" % (C, Tv), 8 * n + 4 * C,
                    lambda g, C=C, Tv=Tv: g.binbcast(R.OP_ADD, take(C, Tv), take(C, 1))))

        def tail(g, C=C, Tv=Tv, resid=False):
            t = g.cont_f32(take(Tv, C), [Tv, C], [4 * C, 4]).reshape(C, Tv)
            s_ = g.binbcast(R.OP_ADD, t, take(C, 1))
            if resid:
                s_ = g.add(s_, take(C, Tv))
            return g.leaky_relu(s_, np.float32(0.1))
        out.append((cfg, "conv tail: cont(transpose)+bias->leaky [%d,%d]" % (C, Tv), 8 * n + 4 * C, tail))
        out.append((cfg, "conv tail: cont(transpose)+bias+residual->leaky, sum [%d,%d]" % (C, Tv), 16 * n + 4 * C,
                    lambda g, tail=tail: tail(g, resid=True)))
        # im2col: ggml-CPU's column gather; the channel-major form is the
        # reference's ggml_cont of the transpose, then im2col
        out.append((cfg, "im2col K=3 [%d,%d]" % (C, Tv), 16 * n,
                    lambda g, C=C, Tv=Tv: g.im2col(take(C, Tv), 3, 1, 1, 1)))
        out.append((cfg, "im2col K=3 channel-major view [%d,%d]" % (C, Tv), 4 * n + 12 * (Tv + 2) * C,
                    lambda g, C=C, Tv=Tv: g.im2col(g.cont_f32(take(Tv, C), [Tv, C], [4 * C, 4]).reshape(C, Tv),
                                                   3, 1, 2, 1)))
        st = 2 if Tv >= 131072 else 8
        out.append((cfg, "pad: spread x%d [%d,1,%d]" % (st, C, Tv // st), 4 * n // st * (1 + st),
                    lambda g, C=C, Tv=Tv, st=st: g.pad(take(Tv // st, 1, C), [0, st - 1, 0, 0])))
        out.append((cfg, "repeat: frames x2 [%d,1,%d]" % (C, Tv // 2), 6 * n,
                    lambda g, C=C, Tv=Tv: g.repeat(take(Tv // 2, 1, C), (Tv // 2, 2, C))))
        out.append((cfg, "pad_ext: time +3/+4 [%d,%d]" % (Tv, C), 4 * n + 4 * C * (Tv + 7),
                    lambda g, C=C, Tv=Tv: g.pad_ext(take(C, Tv), [3], [4])))
        Lc = (Tv + st - 2 * st) // st + 1
        out.append((cfg, "col2im_1d K=%d s=%d [%d,%d]" % (2 * st, st, C, Tv), 4 * 2 * st * C * Lc + 4 * n,
                    lambda g, C=C, st=st, Lc=Lc: g.col2im_1d(take(Lc, 2 * st * C), st, C, st // 2)))
        if (C, Tv) == (128, 131072):
            out.append((cfg, "im2col K=11 d=5 [%d,%d]" % (C, Tv), 48 * n,
                        lambda g, C=C, Tv=Tv: g.im2col(take(C, Tv), 11, 1, 25, 5)))
            out.append((cfg, "im2col K=7 d=3 f16 [%d,%d]" % (C, Tv), 18 * n,
                        lambda g, C=C, Tv=Tv: g.im2col(take(C, Tv), 7, 1, 9, 3, dst_type=R.F16)))
    return out


def cpu_decode_layers(g, layers=28, total=DECODE_TOTAL, seed=SEED + 10):
    """The configs[0] decode step's non-GEMM nodes on the restatement, as
    ggml-CPU runs them for the talker today (src/arch/qwen3-tts/model.cpp:
    99-126), decoder_layer's list per layer (operations.cpp:84-147): the
    input norm, QK-norm and rope of q and k, the k and v cache copies at slot
    total-1, the softmax over `total` keys, the residual add and the
    post-attention norm, SwiGLU and the output add; `layers` layers chained
    in one node list (the projections' outputs as inputs)."""
    import numpy as np
    import formats as F
    import ggml_ref as R
    rng = np.random.default_rng(seed)
    r = lambda *shape: rng.standard_normal(shape).astype(np.float32)
    bf16 = lambda n: F.f32_to_bf16_bits(rng.normal(1.0, 0.1, n).astype(np.float32))
    eps, theta = np.float32(1e-6), np.float32(1e6)
    pos = np.full(1, total - 1, np.int32)
    x = r(1, 1024)
    for _ in range(layers):
        R.rms_norm_w(g, x, bf16(1024), eps, R.BF16)
        qr, kr = R.qk_norm_rope(g, r(1, 16, 128), r(1, 8, 128), bf16(128), bf16(128), eps, pos, 128, theta, R.BF16)
        kc, vc, v = r(total, 8, 128), r(total, 8, 128), r(1, 8, 128)
        g._node(R.OP_CAST_F32, kc[total - 1:], kr, type0=R.F32, ne0=128, nrows=8)
        g._node(R.OP_CAST_F32, vc[total - 1:], v, type0=R.F32, ne0=128, nrows=8)
        g.soft_max_ext(r(16, 1, total), None, np.float32(1.0 / math.sqrt(128.0)))
        after, _ = R.add_rms_norm_w(g, x, r(1, 1024), bf16(1024), eps, R.BF16)
        R.swiglu(g, r(1, 3072), r(1, 3072))
        x = g.add(after, r(1, 1024))
    return g


def cpu_op_baselines(seconds):
    """Each row's node run on the restatement at N, max(1, N/2) and 1 threads
    (N: this process's CPU share, as cpu_share), within about `seconds` in
    all. Returns ({(config, op): entry}, decode-layer entry)."""
    import ggml_ref as R
    share = cpu_share()
    nth = share["threads_used"]
    threads = [nth, max(1, nth // 2), 1]
    builders = cpu_op_builders()
    budget = seconds / (3 * (len(builders) + 1))
    by_row = {}
    for cfg, name, nbytes, build in builders:
        g = R.Graph()
        build(g)
        ts = [_time_cpu(g, t, budget) for t in threads]
        by_row[(cfg, name)] = {"threads": threads, "us": [round(t * 1e6, 1) for t in ts],
                               "GB/s": [round(nbytes / t / 1e9, 2) for t in ts], "nodes": len(g.nodes)}
        del g
    g = cpu_decode_layers(R.Graph())
    ts = [_time_cpu(g, t, budget) / 28 for t in threads]
    nb = decode_layer_bytes(kv=True)
    dec = {"threads": threads, "us_per_layer": [round(t * 1e6, 2) for t in ts],
           "GB/s": [round(nb / t / 1e9, 3) for t in ts], "nodes_per_layer": len(g.nodes) // 28}
    return by_row, dec


# ---------------------------------------------------------------------------
# --suite: every op on every BASELINE config, small shapes included
# ---------------------------------------------------------------------------

def suite(args, S, torch):
    R = Rows(torch)
    g, randn, empty, bf16 = gen(torch, SEED + 7)
    f32 = 4
    want = set(filter(None, args.only.split(",")))
    on = lambda c: not want or c in want

    def per_layer(cfg, name, us, nbytes, note):
        R.rows.append({"config": cfg, "op": name, "us": round(us, 3), "bytes": nbytes,
                       "GB/s": round(nbytes / (us * 1e3), 1), "note": note})
        print("%-10s %-40s %9.3f us/layer  %d B  %s" % (cfg, name, us, nbytes, note), file=sys.stderr, flush=True)

    if on("calib"):
        n = (1 << 30) // 4
        src, dst = randn(n), empty(n)
        acc = torch.empty((), device="cuda", dtype=torch.float32)
        R.run("calib", "torch copy_ 1 GiB (read+write)", 2 * n * 4, lambda: (lambda: dst.copy_(src)))
        R.run("calib", "torch sum 1 GiB (read only)", n * 4, lambda: (lambda: torch.sum(src, dim=0, out=acc)))
        del src, dst

        def make_floor():
            x, y = randn(8192, 2048), empty(8192, 2048)
            return lambda: S.leaky_relu(x, 0.1, out=y)
        R.run("calib", "copy-like floor: bare leaky [2048,8192]", 8 * 8192 * 2048, make_floor)

    def norm_case(cfg, T, H, add=False, cold=True):
        def make():
            a, b, w, y, s = randn(T, H), randn(T, H), bf16(H), empty(T, H), empty(T, H)
            if add:
                return lambda: S.add_rms_norm_mul(a, b, w, 1e-6, out=y, sum_out=s)
            return lambda: S.rms_norm_mul(a, w, 1e-6, out=y)
        R.run(cfg, ("add_rms_norm_mul+sum [%d,%d]" if add else "rms_norm_mul [%d,%d]") % (H, T),
              (4 if add else 2) * T * H * f32 + H * 2, make, cold=cold)

    def qk_case(cfg, T, hi, cold=True):
        def make():
            q, k = randn(T, 16, 128), randn(T, 8, 128)
            qo, ko, wq, wk = torch.empty_like(q), torch.empty_like(k), bf16(128), bf16(128)
            pos = torch.randint(0, hi, (T,), generator=g, device="cuda", dtype=torch.int32)
            return lambda: S.qk_norm_rope(q, k, wq, wk, 1e-6, pos, 128, 1e6, q_out=qo, k_out=ko)
        R.run(cfg, "qk_norm_rope q[128,16,%d] k[128,8,%d]" % (T, T), 2 * 24 * 128 * T * f32 + T * 4 + 512, make,
              cold=cold)

    def swiglu_case(cfg, T, F_, cold=True):
        def make():
            a, b, y = randn(T, F_), randn(T, F_), empty(T, F_)
            return lambda: S.swiglu(a, b, out=y)
        R.run(cfg, "swiglu [%d,%d]" % (F_, T), 3 * T * F_ * f32, make, cold=cold)

    def add_case(cfg, T, H, cold=True):
        def make():
            a, b, y = randn(T, H), randn(T, H), empty(T, H)
            return lambda: S.add(a, b, out=y)
        R.run(cfg, "add [%d,%d]" % (H, T), 3 * T * H * f32, make, cold=cold)

    def make_sm(T=1, N=512):
        sc, p = randn(16, T, N), empty(16, T, N)
        return lambda: S.soft_max_ext(sc, None, 1.0 / math.sqrt(128.0), out=p)

    if on("configs0"):
        def make_tiny():
            a, b = randn(1), empty(1)
            return lambda: torch.add(a, a, out=b)
        R.run("configs[0]", "graph launch floor (torch 1-element add)", 12, make_tiny, cold=False)
        for cold in (True, False):
            norm_case("configs[0]", 1, 1024, cold=cold)
            norm_case("configs[0]", 1, 1024, add=True, cold=cold)
            qk_case("configs[0]", 1, 64, cold=cold)
            swiglu_case("configs[0]", 1, 3072, cold=cold)
            add_case("configs[0]", 1, 1024, cold=cold)

        def make_kv():
            q, k, v = randn(1, 16, 128), randn(1, 8, 128), randn(1, 8, 128)
            kc, vc, qo = randn(DECODE_TOTAL, 8, 128), randn(DECODE_TOTAL, 8, 128), empty(1, 16, 128)
            w = bf16(128)
            pos = torch.tensor([DECODE_TOTAL - 1], dtype=torch.int32, device="cuda")
            return lambda: S.qk_norm_rope_kv(q, k, v, w, w, 1e-6, pos, 128, 1e6, kc, vc, DECODE_TOTAL - 1, q_out=qo)
        R.run("configs[0]", "qk_norm_rope_kv [128,16+8(+8 v),1] at position 37", 64 * 128 * f32 + 4 + 2 * 128 * 2,
              make_kv, cold=False)
        R.run("configs[0]", "soft_max_ext [38,1,16]", 2 * 16 * DECODE_TOTAL * f32, lambda: make_sm(1, DECODE_TOTAL),
              cold=False)
        per_layer("configs[0]", "talker layer non-GEMM step (28-layer graph, 4 launches/layer)",
                  decode_layer_us(S, torch), decode_layer_bytes(), "per layer")
        per_layer("configs[0]", "talker layer non-GEMM step + KV-cache write + soft_max over 38 keys "
                  "(28-layer graph, 5 launches/layer)", decode_layer_us(S, torch, kv=True),
                  decode_layer_bytes(kv=True), "per layer")
        per_layer("configs[0]", "talker layer non-GEMM node list through shp_graph_compute (28 layers)",
                  decode_layer_graph_us(S, torch)[0], decode_layer_bytes(kv=True), "per layer")

    if on("configs1"):
        norm_case("configs[1]", 512, 1024)
        qk_case("configs[1]", 512, 512)
        norm_case("configs[1]", 512, 1024, add=True)
        swiglu_case("configs[1]", 512, 3072)
        add_case("configs[1]", 512, 1024)
        R.run("configs[1]", "soft_max_ext causal-size [512,512,16]", 2 * 16 * 512 * 512 * f32,
              lambda: make_sm(512, 512))
        table = (0.02 * randn(151936, 2048)).to(torch.bfloat16)

        def make_gather():
            ids = torch.randint(0, 151936, (512,), generator=g, device="cuda", dtype=torch.int32)
            out = empty(512, 2048)
            return lambda: S.get_rows(table, ids, out=out)
        R.run("configs[1]", "get_rows bf16 [2048,151936] x512", 512 * (4 + 2048 * 2 + 2048 * f32), make_gather)
        del table

    if on("configs2"):
        q8_rows(R, S, torch, "configs[2]", SEED + 3)
        q8_rows(R, S, torch, "configs[2]", SEED + 6, kind="q5_k")

    if on("configs3"):
        vocoder_rows(R, S, torch, "configs[3]", SEED + 4, variants=True)

    if on("configs4"):
        step_op_rows(R, S, torch, "configs[4]", 8192, 2048, 6144, SEED + 5)
        norm_case("configs[4]", 64, 1024, add=True)
        qk_case("configs[4]", 64, 8192)
        swiglu_case("configs[4]", 64, 3072)
        us64 = decode_layer_us(S, torch, streams=64)
        per_layer("configs[4]", "64 concurrent decode streams: talker layer non-GEMM step (28-layer graph, "
                  "4 launches/layer, 64 rows per launch)", us64, decode_layer_bytes(streams=64),
                  "per layer; per 28-layer step %.1f us" % (28 * us64))

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
                    R.rows.append({"config": "gguf", "op": label, "bytes": nbytes, "us": round(best * 1e6, 1),
                                   "GB/s": round(gbs, 2), "note": "page cache warm; PCIe host->device bound"})
                    print("gguf       %-44s %12d B %11.1f us %8.2f GB/s" % (label, nbytes, best * 1e6, gbs),
                          file=sys.stderr, flush=True)

    with open(args.suite, "w") as f:
        json.dump({"peak_GBps": PEAK_GBS, "cold_bytes": COLD_BYTES, "rows": R.rows}, f, indent=1)


# ---------------------------------------------------------------------------
# counter passes and profile summaries
# ---------------------------------------------------------------------------

PMC_OPS = [
    ("rms_norm_mul [2048,8192]", 134221824), ("add_rms_norm_mul+sum [2048,8192]", 268439552),
    ("qk_norm_rope q[128,16,8192] k[128,8,8192]", 201359872), ("swiglu [6144,8192]", 603979776),
    ("add [2048,8192]", 201326592), ("snake [128,131072]", 134218240), ("snake_beta [128,131072]", 134218752),
    ("add_leaky_relu [128,131072]", 201326592), ("get_rows_sum q8_0 16x[1024,2048] x4096", 88342528),
    ("get_rows q8_0 [1024,2048] x4096", 21250048), ("soft_max_ext causal-size [512,512,16]", 33554432),
    ("get_rows_sum q5_k 16x[1024,2048] x4096", 63176704), ("get_rows q5_k [1024,2048] x4096", 19677184),
    ("cont(transpose) [128,131072]", 134217728), ("add bias[1,C] time-major [128,131072]", 134218240),
    ("conv tail: cont(transpose)+bias+residual->leaky, sum [128,131072]", 268435968),
    ("im2col K=3 [128,131072]", 268435456), ("im2col K=3 channel-major view [128,131072]", 268439552),
    ("im2col K=7 d=3 f16 [128,131072]", 301989888), ("col2im_1d K=4 s=2 [128,131072]", 201326592),
    ("pad: spread x2 [128,1,65536]", 100663296), ("repeat: frames x2 [128,1,65536]", 100663296),
    ("pad_ext: time +3/+4 [131072,128]", 134221312),
    ("acc: codec run +8176@16 into text [2048,8192]", 201195520)]


def pmc_large(S, torch):
    """Three launches of each large-config op on one input set, between two
    CALIB_BYTES device copies (CALIB_BYTES read and written), for rocprofv3
    --pmc passes. The op order is PMC_OPS'."""
    import numpy as np
    import formats as F
    g, randn, empty, bf16 = gen(torch, SEED + 9)
    rng = np.random.default_rng(SEED + 9)
    x2, x2b, w2 = randn(8192, 2048), randn(8192, 2048), bf16(2048)
    q, k, wq, wk = randn(8192, 16, 128), randn(8192, 8, 128), bf16(128), bf16(128)
    pos = torch.arange(8192, dtype=torch.int32, device="cuda")
    gt, up = randn(8192, 6144), randn(8192, 6144)
    xs, al = randn(131072, 128), torch.exp(torch.empty(128, device="cuda").uniform_(-2.3, 2.3, generator=g))
    la = torch.empty(128, device="cuda").uniform_(-3, 3, generator=g)
    lb = torch.empty(128, device="cuda").uniform_(-3, 3, generator=g)
    a4, b4 = randn(131072, 128), randn(131072, 128)
    tabs = [S.Q8Tensor(torch.from_numpy(F.q8_0_synthetic(rng, 2048, 1024)).cuda(), 1024) for _ in range(16)]
    codes = torch.randint(0, 2048, (16, 4096), generator=g, device="cuda", dtype=torch.int32)
    tabs5 = [S.Q5KTensor(torch.from_numpy(F.q5_k_synthetic(rng, 2048, 1024)).cuda(), 1024) for _ in range(16)]
    sc = randn(16, 512, 512)
    xt, tb, tr = randn(131072, 128), randn(128, 1), randn(128, 131072)   # GEMM output ggml [128, T], bias, residual
    ty, ts = empty(128, 131072), empty(128, 131072)
    cols3, cols3c = empty(1, 131072, 384), empty(1, 131074, 384)   # im2col columns of tr (ggml [T, C]) and of xt^T
    cols7 = torch.empty((1, 131072, 896), dtype=torch.float16, device="cuda")
    c2i = randn(65536, 512)   # col2im_1d columns: K 4 x 128 channels, 65536 samples in, 131072 out
    sp_x, sp_y = randn(65536, 1, 128), empty(65536, 2, 128)   # the spread and the frame doubling
    ed_x, ed_y = randn(128, 131072), empty(128, 131079)        # edge padding +3/+4 along time
    ac_a, ac_b, ac_y = randn(8192, 2048), randn(8176, 2048), empty(8192, 2048)
    fns = [lambda: S.rms_norm_mul(x2, w2, 1e-6), lambda: S.add_rms_norm_mul(x2, x2b, w2, 1e-6),
           lambda: S.qk_norm_rope(q, k, wq, wk, 1e-6, pos, 128, 1e6), lambda: S.swiglu(gt, up),
           lambda: S.add(x2, x2b), lambda: S.snake(xs, al), lambda: S.snake_beta(xs, la, lb),
           lambda: S.add_leaky_relu(a4, b4, 0.1), lambda: S.get_rows_sum(tabs, codes),
           lambda: S.get_rows(tabs[0], codes[0]), lambda: S.soft_max_ext(sc, None, 0.0884),
           lambda: S.get_rows_sum(tabs5, codes), lambda: S.get_rows(tabs5[0], codes[0]),
           lambda: S.cpy(xt.t(), out=ty), lambda: S.add(tr, tb, out=ty),
           lambda: S.cont_add_leaky_relu(xt.t(), tb, tr, 0.1, out=ty, sum_out=ts),
           lambda: S.im2col(tr, 3, 1, 1, 1, out=cols3), lambda: S.im2col(xt.t(), 3, 1, 2, 1, out=cols3c),
           lambda: S.im2col(tr, 7, 1, 9, 3, out=cols7), lambda: S.col2im_1d(c2i, 2, 128, 1, out=ty),
           lambda: S.pad_ext(sp_x, [0, 0], [0, 1], out=sp_y), lambda: S.repeat(sp_x, (65536, 2, 128), out=sp_y),
           lambda: S.pad_ext(ed_x, [3], [4], out=ed_y),
           lambda: S.acc(ac_a, ac_b, 8192, 8192 * 8192, 8192 * 8192, 16 * 8192, out=ac_y)]
    n = CALIB_BYTES // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    for f in fns:
        for _ in range(3):
            f()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_large": [name for name, _ in PMC_OPS], "calib_bytes": CALIB_BYTES}))


def short_kernel(name):
    m = re.search(r"(k_[A-Za-z0-9_]+(?:<[^()]*>)?)\(", name)
    if m:
        return m.group(1).replace(" ", "")
    if "copyBuffer" in name:
        return "__amd_rocclr_copyBuffer"
    return re.sub(r"<.*", "", name.replace("void ", "", 1)).split("::")[-1].split("(")[0][:40]


def _one(pattern):
    hits = sorted(glob.glob(pattern, recursive=True))
    if not hits:
        raise SystemExit("no file matches %s" % pattern)
    return hits[0]


def _grid(r):
    if "Grid_Size" in r:
        return int(r["Grid_Size"])
    return int(r["Grid_Size_X"]) * int(r.get("Grid_Size_Y", 1)) * int(r.get("Grid_Size_Z", 1))


def trace_summary(rocdir, log):
    """Per-row kernel durations of a `rocprofv3 --kernel-trace --marker-trace
    --stats` run of this command: every dispatch that starts inside a row's
    ROCTx range belongs to that row."""
    kt = list(csv.DictReader(open(_one(os.path.join(rocdir, "**", "*kernel_trace.csv")))))
    mk = list(csv.DictReader(open(_one(os.path.join(rocdir, "**", "*marker_api_trace.csv")))))
    line = json.loads([l for l in open(log).read().splitlines() if l.startswith("{")][-1])
    bench_us = {}
    for r in line.get("ops", {}).values():
        bench_us[(r["config"], r["op"])] = r["us"]
    for r in line.get("rows", []):
        bench_us[(r["config"], r["op"])] = r["us"]
    text_col = next(c for c in ("Message", "Function", "Name") if c in mk[0])
    ranges = [(int(m["Start_Timestamp"]), int(m["End_Timestamp"]), m[text_col]) for m in mk
              if m[text_col].startswith(("row:", "step:"))]
    kern = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), short_kernel(r["Kernel_Name"]), _grid(r))
                  for r in kt)
    out = ["# kernel durations per bench row, from rocprofv3's kernel trace (End-Start per dispatch) and the",
           "# ROCTx range bench.py puts around each row's timed replays; bytes = the row's algorithmic bytes;",
           "# trace_GB/s = bytes / avg_ns; frac = trace_GB/s / 8000; bench_us = bench.py's HIP-event time per",
           "# launch for the row in the JSON line given: an unprofiled run on the same box just before (graph",
           "# replay, events on the replay stream).",
           "# made by (from /tmp with TMPDIR=/tmp, R the repository root): python3 -u $R/bench.py > bench.json (unprofiled);",
           "#   rocprofv3 --kernel-trace --marker-trace --stats --output-format csv -d prof -o bench -- python3 -u $R/bench.py;",
           "#   python3 $R/bench.py --trace-summary prof bench.json",
           "%-11s %-44s %-36s %9s %6s %9s %9s %9s %9s %9s %6s" % (
               "config", "op", "kernel", "grid", "calls", "avg_ns", "med_ns", "min_ns", "bench_us", "trace_GB/s",
               "frac")]
    import bisect
    starts = [k[0] for k in kern]
    for t0, t1, text in ranges:
        lo, hi = bisect.bisect_left(starts, t0), bisect.bisect_right(starts, t1)
        by = defaultdict(list)
        for s, e, name, grid in kern[lo:hi]:
            by[(name, grid)].append(e - s)
        if text.startswith("step:"):
            out.append("# %s: %d dispatches inside the timed steps" % (text, hi - lo))
            for (name, grid), d in sorted(by.items(), key=lambda kv: -sum(kv[1])):
                out.append("#   %-36s %9d %6d avg %9.0f ns" % (name, grid, len(d), statistics.mean(d)))
            continue
        cfg, op, nbytes = text.split(":", 1)[1].rsplit("|", 2)
        nbytes = int(nbytes)
        if not by:
            out.append("%-11s %-44s (no dispatch traced)" % (cfg, op))
            continue
        (name, grid), d = max(by.items(), key=lambda kv: sum(kv[1]))
        avg = statistics.mean(d)
        bu = bench_us.get((cfg, op))
        gbs = nbytes / avg
        out.append("%-11s %-44s %-36s %9d %6d %9.0f %9.0f %9.0f %9s %9.1f %6.3f" % (
            cfg, op[:44], name[:36], grid, len(d), avg, statistics.median(d), min(d),
            "%.3f" % bu if bu is not None else "-", gbs, gbs / PEAK_GBS))
    stats = glob.glob(os.path.join(rocdir, "**", "*kernel_stats.csv"), recursive=True)
    if stats:
        out += ["", "# rocprofv3 --stats (kernel_stats.csv) of the whole run, by kernel name over every shape it ran",
                "%-44s %7s %12s %10s %6s" % ("kernel", "calls", "total_ns", "avg_ns", "pct")]
        for r in list(csv.DictReader(open(sorted(stats)[0])))[:20]:
            out.append("%-44s %7s %12s %10.0f %6s" % (short_kernel(r["Name"])[:44], r["Calls"], r["TotalDurationNs"],
                                                     float(r["AverageNs"]), r["Percentage"]))
    print("\n".join(out))


def pmc_summary(fetch_dir, write_dir, log):
    """HBM bytes per launch of each --pmc-large op from a FETCH_SIZE and a
    WRITE_SIZE pass, each scaled by what the counter reads for the
    CALIB_BYTES device copy."""
    meta = json.loads([l for l in open(log).read().splitlines() if l.startswith("{") and "pmc_large" in l][-1])

    def load(d):
        rows = list(csv.DictReader(open(_one(os.path.join(d, "**", "*counter_collection.csv")))))
        rows.sort(key=lambda r: int(r["Dispatch_Id"]))
        return [(short_kernel(r["Kernel_Name"]), _grid(r), float(r["Counter_Value"])) for r in rows]

    F, W = load(fetch_dir), load(write_dir)
    copies = [i for i, (k, g, v) in enumerate(F) if k == "__amd_rocclr_copyBuffer" and v > 1e5]
    first, last = copies[0], copies[-1]
    cal_f = statistics.mean([F[first][2], F[last][2]])
    cal_w = statistics.mean([W[first][2], W[last][2]])
    kib = meta["calib_bytes"] / 1024
    fs, ws = kib / cal_f, kib / cal_w
    ours = [i for i in range(first + 1, last) if F[i][0].startswith("k_")]
    out = ["# HBM bytes per launch of the large-config kernels: two rocprofv3 --pmc passes (FETCH_SIZE, then",
           "# WRITE_SIZE) over `bench.py --pmc-large`, three launches per op on one input set; each counter is",
           "# scaled by what it reads for the %d MiB device copy before and after (%d KiB read and written):" % (
               meta["calib_bytes"] >> 20, kib),
           "# FETCH_SIZE %.1f KiB -> scale %.4f; WRITE_SIZE %.1f KiB -> scale %.4f." % (cal_f, fs, cal_w, ws),
           "# hbm_bytes = (FETCH_KiB * fetch_scale + WRITE_KiB * write_scale) * 1024, averaged over the 3 launches;",
           "# ratio = hbm_bytes / algorithmic bytes (gathers: logical, every looked-up row per lookup). FETCH_SIZE",
           "# counts what L2 fetches from beyond it (Infinity Cache or HBM).",
           "# made by (from /tmp with TMPDIR=/tmp, R the repository root), for M in FETCH_SIZE WRITE_SIZE:",
           "#   rocprofv3 --pmc $M --output-format csv -d pmc_$M -o x -- python3 -u $R/bench.py --pmc-large > pmc_$M.log;",
           "#   python3 $R/bench.py --pmc-summary pmc_FETCH_SIZE pmc_WRITE_SIZE pmc_FETCH_SIZE.log"]
    assert len(ours) == 3 * len(PMC_OPS), (len(ours), len(PMC_OPS))
    for j, (op, nbytes) in enumerate(PMC_OPS):
        idx = ours[3 * j:3 * j + 3]
        fk = statistics.mean(F[i][2] for i in idx)
        wk = statistics.mean(W[i][2] for i in idx)
        hb = (fk * fs + wk * ws) * 1024
        out.append("op=%s kernel=%s grid=%d fetch_kib=%.1f write_kib=%.1f hbm_bytes=%d algorithmic_bytes=%d "
                   "ratio=%.4f" % (op.replace(" ", "_"), F[idx[0]][0], F[idx[0]][1], fk, wk, hb, nbytes,
                                    hb / nbytes))
    print("\n".join(out))


OCC_METRICS = ("OccupancyPercent", "MeanOccupancyPerCU", "VALUBusy", "MemUnitStalled")


def occ_summary(dirs):
    """Per --pmc-large op: the average over its three launches of each derived
    metric (one rocprofv3 --pmc pass per metric), with the dispatch's register
    and LDS use from the same records."""
    if len(dirs) != len(OCC_METRICS):
        raise SystemExit("--occ-summary takes %d directories: %s" % (len(OCC_METRICS), ", ".join(OCC_METRICS)))
    passes = []
    for d in dirs:
        rows = list(csv.DictReader(open(_one(os.path.join(d, "**", "*counter_collection.csv")))))
        rows.sort(key=lambda r: int(r["Dispatch_Id"]))
        passes.append([r for r in rows if short_kernel(r["Kernel_Name"]).startswith("k_")])
    n = len(passes[0])
    assert all(len(p) == n for p in passes) and n == 3 * len(PMC_OPS), ([len(p) for p in passes], len(PMC_OPS))
    out = ["# Occupancy, VALU and memory-unit stall per large-config kernel, MI355X gfx950: one rocprofv3 --pmc",
           "# pass per derived metric over `bench.py --pmc-large` (three launches per op, one input set), averaged",
           "# over the three. occ% = resident waves as a % of the maximum (OccupancyPercent); w/CU = waves resident",
           "# per CU, time-averaged (MeanOccupancyPerCU); valu% = % of time a CU issues VALU (VALUBusy); mstl% =",
           "# % of time the memory unit is stalled on data (MemUnitStalled); vgpr/sgpr/lds from the dispatch",
           "# records (lds in bytes per workgroup).",
           "# made by (from /tmp with TMPDIR=/tmp, R the repository root), for M in OccupancyPercent",
           "# MeanOccupancyPerCU VALUBusy MemUnitStalled: rocprofv3 --pmc $M --output-format csv -d occ_$M -o o --",
           "#   python3 -u $R/bench.py --pmc-large; then python3 $R/bench.py --occ-summary occ_OccupancyPercent",
           "#   occ_MeanOccupancyPerCU occ_VALUBusy occ_MemUnitStalled",
           "%-44s %-34s %9s %7s %7s %7s %7s %5s %5s %6s" % ("op", "kernel", "grid", "occ%", "w/CU", "valu%", "mstl%",
                                                          "vgpr", "sgpr", "lds")]
    for j, (op, _) in enumerate(PMC_OPS):
        vals = [statistics.mean(float(p[i]["Counter_Value"]) for i in range(3 * j, 3 * j + 3)) for p in passes]
        r = passes[0][3 * j]
        out.append("%-44s %-34s %9d %7.1f %7.2f %7.1f %7.1f %5s %5s %6s" % (
            op[:44], short_kernel(r["Kernel_Name"])[:34], _grid(r), vals[0], vals[1], vals[2], vals[3],
            r.get("VGPR_Count", "-"), r.get("SGPR_Count", "-"), r.get("LDS_Block_Size", "-")))
    print("\n".join(out))


def read_traffic(op):
    """HBM bytes per launch of `op` from the committed counter summary, or None."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        fields = dict(kv.split("=", 1) for kv in line.split() if "=" in kv)
        if fields.get("op") == op.replace(" ", "_") and "hbm_bytes" in fields:
            return int(float(fields["hbm_bytes"]))
    return None


# ---------------------------------------------------------------------------
# the bench line
# ---------------------------------------------------------------------------

def main():
    args = parse()
    if args.trace_summary:
        trace_summary(*args.trace_summary)
        return
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.occ_summary:
        occ_summary(args.occ_summary)
        return
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

    # the 8192-token step of the 1.7B-shaped talker layer
    step = LayerStep(S, torch, T=8192, hidden=2048, ffn=6144, gather=False, nsets=2)
    ms_per_step = step.time_steps(args.steps, args.warmup, label="step:configs[4]")
    step_bytes = step.step_bytes
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    cpu = None if args.no_cpu else cpu_baseline(step, torch, args.cpu_seconds)
    del step
    torch.cuda.empty_cache()

    ops4 = step_op_rows(Rows(torch), S, torch, "configs[4]", 8192, 2048, 6144, SEED + 5)
    R = Rows(torch)
    q8_rows(R, S, torch, "configs[2]", SEED + 3)
    q8_rows(R, S, torch, "configs[2]", SEED + 6, kind="q5_k")
    vocoder_rows(R, S, torch, "configs[3]", SEED + 4)
    talker_input_rows(R, S, torch, "configs[4]", SEED + 7)
    istft_rows(R, S, torch, "configs[3]", SEED + 11)
    source_rows(R, S, torch, "configs[3]", SEED + 12)
    mel_rows(R, S, torch, "configs[3]", SEED + 13)
    floors = floor_rows(R, S, torch)
    link_floors(list(ops4.values()) + R.rows, floors)

    if not args.no_cpu:
        cpu_rows, cpu_dec = cpu_op_baselines(args.cpu_seconds)
        for row in list(ops4.values()) + R.rows:
            c = cpu_rows.get((row["config"], row["op"]))
            if c is not None:
                row["cpu"] = c

    dom = max(ops4, key=lambda n: ops4[n]["us"])
    d = ops4[dom]
    roof = {"bound": "hbm", "kernel": d["op"], "achieved": d["GB/s"], "peak": PEAK_GBS, "unit": "GB/s",
            "frac": d["frac"], "traffic": read_traffic(d["op"]), "algorithmic_bytes": d["bytes"],
            "us_per_launch": d["us"], "us_per_launch_mean": d["us_mean"],
            "achieved_from_mean": round(d["bytes"] / (d["us_mean"] * 1e-6) / 1e9, 1),
            "timing": "achieved = algorithmic bytes / us_per_launch, the median over 10 timed chunks of the "
                      "mean launch duration in a chunk (HIP events on the replay stream); achieved_from_mean "
                      "uses the mean over all the launches",
            "traffic_source": "read from the committed counter summary profiles/traffic_large_configs.txt "
                              "(rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of this kernel at this shape, scaled "
                              "by the same counters over a device copy of known size), not measured in this run"}

    # one decode token per layer (position 37), 28 layers in one graph
    dec = decode_layer_us(S, torch, label="step:configs[0] decode, 28 layers x 4 launches")
    dec_full = decode_layer_us(S, torch, kv=True, label="step:configs[0] decode + kv + softmax, 28 layers x 5 launches")
    dec_graph, dec_graph_launches = decode_layer_graph_us(
        S, torch, label="step:configs[0] decode through shp_graph_compute, 28 layers")
    # 64 concurrent decode streams
    dec64 = decode_layer_us(S, torch, streams=64, label="step:configs[4] 64-stream decode, 28 layers x 4 launches")
    # the 0.6B talker's 512-token prefill step with the text-embedding gather
    step1 = LayerStep(S, torch, T=512, hidden=1024, ffn=3072, gather=True)
    ms1 = step1.time_steps(max(args.steps, 200), args.warmup, label="step:configs[1]")
    b1 = step1.step_bytes
    del step1
    torch.cuda.empty_cache()

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "configs[4]: Qwen3-TTS-1.7B-shaped talker layer non-GEMM prefill step, 8192 tokens "
                               "x hidden 2048, 16/8 heads x 128 (NEOX rope theta 1e6, positions 0..8191), SwiGLU "
                               "6144, BF16 gains, f32 activations ~N(0,1): rms_norm_mul, qk_norm_rope, "
                               "add_rms_norm_mul+sum, swiglu, add; two input sets alternating (1.41 GB per "
                               "step, cold), steps replayed back to back from one HIP graph",
                   "tokens": 8192, "hidden": 2048, "bytes_per_step": step_bytes,
                   "frac_of_peak": round(value / PEAK_GBS, 4)},
        "ops": {k: v for k, v in ops4.items()},
        "rows": R.rows,
        "roofline": roof,
        "decode_layer_us": round(dec, 3),
        "decode_layer_full_us": round(dec_full, 3),
        "decode_layer_graph_us": round(dec_graph, 3),
        "decode_layer_note": "configs[0]: us per talker layer of a 28-layer one-token decode graph at position 37 "
                             "(median of %d timed chunks); _us: add+norm, qk-norm+rope, add+norm, swiglu "
                             "(4 launches, %d B); _full_us: with the KV-cache write fused into qk-norm+rope and "
                             "the 16-head softmax over 38 keys (5 launches, %d B), entry points called directly; "
                             "_graph_us: the same work as decoder_layer's non-GEMM node list in the reference's "
                             "expand order (operations.cpp:84-147; GEMM outputs as leaves, 28 chained layers), "
                             "planned and launched by shp_graph_compute inside one HIP graph capture: %d launches "
                             "for 28 layers" % (CHUNKS, decode_layer_bytes(), decode_layer_bytes(kv=True),
                                                dec_graph_launches),
        "decode64_step_us": round(28 * dec64, 2),
        "decode64_note": "configs[4]: 64 concurrent decode streams, us per 28-layer step (%d B per step)" % (
            28 * decode_layer_bytes(streams=64)),
        "configs1_step": {"GB/s": round(b1 / (ms1 * 1e-3) / 1e9, 1), "us_per_step": round(ms1 * 1e3, 3),
                          "bytes": b1, "note": "0.6B talker layer, 512-token prefill incl. the BF16 gather "
                          "from the 151936x2048 table; rotating sets, back to back from one HIP graph"},
    }
    if cpu is not None:
        line["cpu_baseline"] = cpu
    if not args.no_cpu:
        line["decode_layer_cpu"] = dict(cpu_dec, note="configs[0]: the same decode layer's non-GEMM nodes (28 "
                                        "chained layers, %d B per layer) on the ggml-CPU restatement, us per "
                                        "layer at the threads listed" % decode_layer_bytes(kv=True))
        line["cpu_rows_note"] = ("each ops/rows entry's 'cpu': its node run on the ggml-CPU restatement "
                                 "(oracle/ggml_cpu_ref.c, ggml's row split) over host inputs of the same shapes, "
                                 "at N, max(1, N/2) and 1 threads (N = threads_used); median of up to 20 runs after "
                                 "a warm-up, within --cpu-seconds in all; a reported baseline only")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

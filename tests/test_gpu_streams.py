"""The boundary's threading contract: entry points are stream-ordered and
re-entrant, so calls from several host threads on distinct streams run
concurrently and give the same bits as the same calls made one at a time.
ctypes releases the GIL around each call, so the calls do overlap inside the
library, including the first-use lookups it keeps per device."""
import threading

import numpy as np
import pytest

import formats as F

pytestmark = pytest.mark.gpu


def _ops(gpu, torch):
    rng = np.random.default_rng(20260728 + 7)
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    randn = lambda *shape: torch.randn(shape, generator=g, device="cuda")
    bf16 = lambda n: (1 + 0.1 * randn(n)).to(torch.bfloat16)
    x, b, w = randn(64, 1024), randn(64, 1024), bf16(1024)
    q, k, wq, wk = randn(64, 16, 128), randn(64, 8, 128), bf16(128), bf16(128)
    pos = torch.randint(0, 4096, (64,), generator=g, device="cuda", dtype=torch.int32)
    gate, up = randn(64, 3072), randn(64, 3072)
    xs, la, lb = randn(256, 512), randn(512), randn(512)
    sc = randn(16, 33, 512) * 3
    mask = torch.zeros(33, 512, device="cuda").masked_fill(
        torch.ones(33, 512, device="cuda", dtype=torch.bool).triu(480), float("-inf"))
    table = (0.02 * randn(5000, 2048)).to(torch.bfloat16)
    ids = torch.randint(0, 5000, (77,), generator=g, device="cuda", dtype=torch.int32)
    q8 = torch.from_numpy(np.stack([F.q8_0_synthetic(rng, 300, 1024) for _ in range(15)])).cuda()
    q8tabs = [gpu.Q8Tensor(q8[t], 1024) for t in range(15)]
    codes = torch.randint(0, 300, (15, 101), generator=g, device="cuda", dtype=torch.int32)
    bftabs = [(0.02 * randn(300, 1024)).to(torch.bfloat16) for _ in range(9)]
    bcodes = torch.randint(0, 300, (9, 101), generator=g, device="cuda", dtype=torch.int32)
    return [
        lambda: gpu.rms_norm_mul(x, w, 1e-6),
        lambda: gpu.add_rms_norm_mul(x, b, w, 1e-6)[1],
        lambda: gpu.qk_norm_rope(q, k, wq, wk, 1e-6, pos, 128, 1e6)[0],
        lambda: gpu.swiglu(gate, up),
        lambda: gpu.snake_beta(xs, la, lb),
        lambda: gpu.soft_max_ext(sc, mask, 0.0884),
        lambda: gpu.get_rows(table, ids),
        lambda: gpu.get_rows_sum(q8tabs, codes),
        lambda: gpu.get_rows_sum(bftabs, bcodes),
    ]


def test_concurrent_streams_match_serial(gpu):
    import torch
    ops = _ops(gpu, torch)
    ref = [op().clone() for op in ops]
    torch.cuda.synchronize()
    errors = []

    def worker(tid):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for it in range(10):
                    outs = [op() for op in (ops[tid:] + ops[:tid])]  # each thread starts elsewhere
                    s.synchronize()
                    for j, o in enumerate(outs):
                        r = ref[(tid + j) % len(ops)]
                        if not torch.equal(o.view(torch.int32), r.view(torch.int32)):
                            errors.append((tid, it, (tid + j) % len(ops)))
        except Exception as e:  # surfaced in the main thread
            errors.append((tid, repr(e)))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads)
    torch.cuda.synchronize()
    assert not errors, errors[:5]

"""shp_diag_mask_inf against the restatement, bit for bit; shp_soft_max_causal
against the GPU's own two nodes (diag_mask_inf, then soft_max_ext), bit for
bit, and against the restatement within the softmax's bound; the codec
encoder's causal attention softmax (qwen3-tts/codec-encoder.cpp:482-483) as
its two nodes through the executor."""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t, _ulps_apart

pytestmark = pytest.mark.gpu

SEED = 20261215


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("shape,n_past", [((8, 375, 375), 0), ((3, 7, 9), 2), ((2, 5, 33), 40), ((1, 1), 0)])
def test_diag_mask_inf_matches_restatement(gpu, shape, n_past):
    x = np.random.default_rng([SEED, *shape, n_past]).standard_normal(shape).astype(np.float32)
    ref = R.run(lambda g: g.diag_mask_inf(x, n_past))
    assert np.array_equal(_bits(_np(gpu.diag_mask_inf(_t(gpu, x), n_past))), _bits(ref))
    tx = _t(gpu, x)
    gpu.diag_mask_inf(tx, n_past, out=tx)           # ggml's inplace form
    assert np.array_equal(_bits(_np(tx)), _bits(ref))


# (heads, rows, row length, n_past): float4 rows of one and several waves,
# scalar rows (odd length), block rows (> 2048)
CASES = [(8, 375, 376, 0), (8, 375, 375, 0), (4, 64, 64, 0), (2, 16, 512, 3), (2, 7, 2500, 100), (16, 1, 37, 36),
         (1, 250, 250, 0)]


@pytest.mark.parametrize("H,T,N,n_past", CASES)
def test_soft_max_causal_is_the_two_nodes(gpu, H, T, N, n_past):
    """Bit-identical to diag_mask_inf then soft_max_ext on the GPU, with +inf
    and NaN scores at masked positions (masked away, as the two nodes do),
    and within 2 ulp (> 99 % identical) of the restatement's two nodes."""
    rng = np.random.default_rng([SEED, H, T, N, n_past])
    x = (rng.standard_normal((H, T, N)) * 4).astype(np.float32)
    if N > n_past + 1:
        x[:, 0, -1] = np.inf
        x[:, 0, n_past + 1] = np.nan
    scale = 1.0 / np.sqrt(64.0)
    tx = _t(gpu, x)
    fused = _np(gpu.soft_max_causal(tx, n_past, scale))
    two = _np(gpu.soft_max_ext(gpu.diag_mask_inf(tx, n_past), None, scale))
    assert np.array_equal(_bits(fused), _bits(two))
    assert np.isfinite(fused).all()
    g = R.Graph()
    ref = g.soft_max_ext(g.diag_mask_inf(x, n_past), None, scale)
    g.compute()
    d = _ulps_apart(fused, ref)
    assert d.max() <= 2 and (d == 0).mean() > 0.99


def test_soft_max_causal_refusals(gpu):
    import torch
    x = torch.zeros((4, 8), device="cuda")
    for bad in (0.0, -1.0, float("inf")):
        with pytest.raises(gpu.ShpError):
            gpu.soft_max_causal(x, 0, bad)
    with pytest.raises(gpu.ShpError):
        gpu.soft_max_causal(x, -1, 1.0)


def test_codec_encoder_attention_softmax_through_the_executor(gpu):
    """codec-encoder.cpp:482-483: the inplace causal mask over the scores,
    then soft_max_ext with 1/sqrt(head_dim): one launch, bit-identical to
    running the two nodes one by one."""
    H, T = 8, 300
    rng = np.random.default_rng(SEED + 1)
    x = rng.standard_normal((H, T, T)).astype(np.float32) * 3
    scale = 1.0 / np.sqrt(64.0)
    g = gpu.Graph()
    ts = _t(gpu, x)
    masked = g.diag_mask_inf(ts, 0, inplace=True)
    probs = g.soft_max_ext(masked, None, scale)
    assert [k for k, *_ in g.plan(probs) if k != "nop"] == ["diag_mask_soft_max"]
    g.compute(probs)
    two = _np(gpu.soft_max_ext(gpu.diag_mask_inf(_t(gpu, x), 0), None, scale))
    assert np.array_equal(_bits(_np(probs.t)), _bits(two))

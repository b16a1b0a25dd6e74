"""GPU parity at BASELINE.json's full configuration sizes.

The parity tests in test_gpu_parity.py cover every entry point, its launch
variants and its edge cases at small and mid sizes; this module runs each op
of the hot path once at the exact shapes the benchmark configurations name,
with their input distributions, against the ggml-CPU restatement (which is
threaded C, so a full-size reference takes well under a second per op):

  configs[0]  one decode token through a whole talker layer's non-GEMM work
  configs[1]  512-token prefill ops with BF16 gains, and the BF16 gather from
              the full 151936 x 2048 text-embedding table
  configs[2]  the 16-codebook Q8_0 gather->sum over 4096 frames and the plain
              Q8_0 get_rows
  configs[3]  Snake (and its guarded and SnakeBeta forms) and add->leaky on
              [512,8192], [256,32768] and [128,131072]
  configs[4]  the 8192-token 1.7B-shaped prefill ops, and 64 decode streams
              through 28 chained layers

Bars as in test_gpu_parity.py: bit-exact for gathers, sums, adds and leaky;
1e-5 relative (floored at 1e-3 of the row RMS) for the norms, SwiGLU and the
Snake family; rope bit-exact against the restatement with correctly rounded
cos/sin and within 1e-5 of each NEOX pair against libm's.
"""
import os

import numpy as np
import pytest

import formats as F
import ggml_ref as R
from test_gpu_parity import (SEED, _dev_w, _np, _t, _weights, assert_bitexact, assert_close, assert_rope_close,
                             assert_snake_close)

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))
EPS, THETA = np.float32(1e-6), np.float32(1e6)


def ref(build):
    return R.run(build, THREADS)


def _normal(rng, shape, scale=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)


def _check_qk(gpu, T, hi_pos, wkind, seed):
    rng = np.random.default_rng(seed)
    q = _normal(rng, (T, 16, 128))
    k = _normal(rng, (T, 8, 128))
    wq, wt = _weights(rng, 128, wkind)
    wk, _ = _weights(rng, 128, wkind)
    pos = np.arange(T, dtype=np.int32) if hi_pos is None else np.array(hi_pos, np.int32)
    qo, ko = gpu.qk_norm_rope(_t(gpu, q), _t(gpu, k), _dev_w(gpu, wq, wkind), _dev_w(gpu, wk, wkind), EPS,
                              _t(gpu, pos), 128, THETA)
    qo, ko = _np(qo), _np(ko)
    qc, kc = ref(lambda g: R.qk_norm_rope(g, q, k, wq, wk, EPS, pos, 128, THETA, wt, cs_rounded=True))
    assert_bitexact(qo, qc)
    assert_bitexact(ko, kc)
    qr, kr = ref(lambda g: R.qk_norm_rope(g, q, k, wq, wk, EPS, pos, 128, THETA, wt))
    assert_rope_close(qo, qr, 128)
    assert_rope_close(ko, kr, 128)


# ---------------------------------------------------------------------------
# one decode token
# ---------------------------------------------------------------------------

def test_cfg0_decode_token_layer_ops(gpu):
    """hidden 1024 ~N(0,1), weight ~N(1,0.1); QK-norm over 16 q + 8 kv heads x
    128; NEOX rope theta 1e6 at position 37; SwiGLU 3072."""
    rng = np.random.default_rng(SEED)
    x = _normal(rng, (1, 1024))
    w, wt = _weights(rng, 1024, "f32")
    assert_close(_np(gpu.rms_norm_mul(_t(gpu, x), _t(gpu, w), EPS)), ref(lambda g: R.rms_norm_w(g, x, w, EPS, wt)))
    _check_qk(gpu, 1, [37], "f32", SEED + 1)
    gate, up = _normal(rng, (1, 3072)), _normal(rng, (1, 3072))
    assert_close(_np(gpu.swiglu(_t(gpu, gate), _t(gpu, up))), ref(lambda g: R.swiglu(g, gate, up)))


# ---------------------------------------------------------------------------
# 512-token prefill, BF16 gains, BF16 text-embedding gather
# ---------------------------------------------------------------------------

def test_cfg1_prefill_norms_and_swiglu(gpu):
    rng = np.random.default_rng(SEED + 2)
    x, r = _normal(rng, (512, 1024)), _normal(rng, (512, 1024))
    w, wt = _weights(rng, 1024, "bf16")
    dw = _dev_w(gpu, w, "bf16")
    assert_close(_np(gpu.rms_norm_mul(_t(gpu, x), dw, EPS)), ref(lambda g: R.rms_norm_w(g, x, w, EPS, wt)))
    s, y = gpu.add_rms_norm_mul(_t(gpu, x), _t(gpu, r), dw, EPS)
    s_ref, y_ref = ref(lambda g: R.add_rms_norm_w(g, x, r, w, EPS, wt))
    assert_bitexact(_np(s), s_ref)
    assert_close(_np(y), y_ref)
    gate, up = _normal(rng, (512, 3072)), _normal(rng, (512, 3072))
    assert_close(_np(gpu.swiglu(_t(gpu, gate), _t(gpu, up))), ref(lambda g: R.swiglu(g, gate, up)))


def test_cfg1_prefill_qk_norm_rope_positions_0_to_511(gpu):
    _check_qk(gpu, 512, None, "bf16", SEED + 3)


def test_cfg1_bf16_text_embedding_gather_full_table(gpu):
    """BF16 [2048, 151936] table ~N(0, 0.02), 512 uniform ids (the ids also hit
    the first and the last row)."""
    rng = np.random.default_rng(SEED + 4)
    rows, ne0 = 151936, 2048
    table = np.empty((rows, ne0), np.uint16)
    for r0 in range(0, rows, 16384):
        r1 = min(rows, r0 + 16384)
        table[r0:r1] = F.f32_to_bf16_bits(_normal(rng, (r1 - r0, ne0), 0.02))
    ids = rng.integers(0, rows, 512).astype(np.int32)
    ids[:2] = [0, rows - 1]
    import torch
    dev = torch.from_numpy(table.view(np.int16)).cuda().view(torch.bfloat16)
    got = _np(gpu.get_rows(dev, _t(gpu, ids)))
    exp = ref(lambda g: g.get_rows(table, R.BF16, ne0, ids))
    assert_bitexact(got, exp)
    assert_bitexact(exp, F.bf16_bits_to_f32(table[ids]))  # the closed form: bits << 16


# ---------------------------------------------------------------------------
# 16 Q8_0 codebooks [1024, 2048], 4096 frames
# ---------------------------------------------------------------------------

def test_cfg2_q8_0_codebook_sum_and_get_rows(gpu):
    """qs ~ U{-127..127}, d ~ U[1e-3, 1e-2] rounded to f16; ids uniform. The
    ordered f32 sum of 16 dequantized rows and the plain get_rows of table 0
    are both bit-exact."""
    rng = np.random.default_rng(SEED + 5)
    groups, rows, ne0, frames = 16, 2048, 1024, 4096
    tabs = [F.q8_0_synthetic(rng, rows, ne0) for _ in range(groups)]
    codes = rng.integers(0, rows, (groups, frames)).astype(np.int32)
    codes[:, 0] = rows - 1
    dev = [gpu.Q8Tensor(_t(gpu, t), ne0) for t in tabs]
    got = _np(gpu.get_rows_sum(dev, _t(gpu, codes)))
    assert_bitexact(got, ref(lambda g: R.sum_code_embeddings(g, tabs, R.Q8_0, ne0, codes)))
    rows0 = _np(gpu.get_rows(dev[0], _t(gpu, codes[0])))
    exp = ref(lambda g: g.get_rows(tabs[0], R.Q8_0, ne0, codes[0]))
    assert_bitexact(rows0, exp)
    assert_bitexact(exp, F.q8_0_dequant(tabs[0], ne0)[codes[0]])


# ---------------------------------------------------------------------------
# vocoder activations
# ---------------------------------------------------------------------------

CFG3 = [(512, 8192), (256, 32768), (128, 131072)]  # ggml [C, T]


@pytest.mark.parametrize("C,T", CFG3)
def test_cfg3_snake_family(gpu, C, T):
    """Kokoro Snake with alpha log-uniform in [0.1, 10]; the guarded form with
    the same alpha; SnakeBeta with log curves log-uniform over the same range."""
    rng = np.random.default_rng(SEED + C)
    x = _normal(rng, (T, C))
    alpha = np.exp(rng.uniform(np.log(0.1), np.log(10.0), C)).astype(np.float32)
    dx, da = _t(gpu, x), _t(gpu, alpha)
    assert_close(_np(gpu.snake(dx, da)), ref(lambda g: R.snake(g, x, alpha)))
    assert_snake_close(_np(gpu.snake_guarded(dx, da)), ref(lambda g: R.snake_guarded(g, x, alpha)), x)
    la = np.log(alpha).astype(np.float32)
    lb = rng.uniform(np.log(0.1), np.log(10.0), C).astype(np.float32)
    assert_snake_close(_np(gpu.snake_beta(dx, _t(gpu, la), _t(gpu, lb))), ref(lambda g: R.snake_beta(g, x, la, lb)), x)


@pytest.mark.parametrize("C,T", CFG3)
def test_cfg3_add_leaky_relu(gpu, C, T):
    """VITS residual carry: s = a + b, y = leaky(s, 0.1), both bit-exact."""
    rng = np.random.default_rng(SEED + 3 * C)
    a, b = _normal(rng, (T, C)), _normal(rng, (T, C))
    s, y = gpu.add_leaky_relu(_t(gpu, a), _t(gpu, b), 0.1, want_sum=True)
    s_ref, y_ref = ref(lambda g: R.add_leaky(g, a, b, np.float32(0.1)))
    assert_bitexact(_np(s), s_ref)
    assert_bitexact(_np(y), y_ref)
    _, y_only = gpu.add_leaky_relu(_t(gpu, a), _t(gpu, b), 0.1)
    assert_bitexact(_np(y_only), y_ref)


# ---------------------------------------------------------------------------
# 1.7B-shaped 8192-token prefill, and 64 decode streams x 28 layers
# ---------------------------------------------------------------------------

def test_cfg4_prefill_norms(gpu):
    rng = np.random.default_rng(SEED + 6)
    x, r = _normal(rng, (8192, 2048)), _normal(rng, (8192, 2048))
    w, wt = _weights(rng, 2048, "bf16")
    dw = _dev_w(gpu, w, "bf16")
    assert_close(_np(gpu.rms_norm_mul(_t(gpu, x), dw, EPS)), ref(lambda g: R.rms_norm_w(g, x, w, EPS, wt)))
    s, y = gpu.add_rms_norm_mul(_t(gpu, x), _t(gpu, r), dw, EPS)
    s_ref, y_ref = ref(lambda g: R.add_rms_norm_w(g, x, r, w, EPS, wt))
    assert_bitexact(_np(s), s_ref)
    assert_close(_np(y), y_ref)


def test_cfg4_prefill_qk_norm_rope_positions_0_to_8191(gpu):
    _check_qk(gpu, 8192, None, "bf16", SEED + 7)


def test_cfg4_prefill_swiglu_6144(gpu):
    rng = np.random.default_rng(SEED + 8)
    gate, up = _normal(rng, (8192, 6144)), _normal(rng, (8192, 6144))
    assert_close(_np(gpu.swiglu(_t(gpu, gate), _t(gpu, up))), ref(lambda g: R.swiglu(g, gate, up)))


def test_cfg4_64_decode_streams_through_28_layers(gpu):
    """64 streams at 64 distinct positions, hidden 1024, 16/8 heads x 128,
    SwiGLU 3072, BF16 gains: 28 layers chained through the layer-step entry
    point, each layer's GEMM outputs standing in as fresh random inputs. The
    residual stream (adds only) stays bit-exact across all 28 layers."""
    rng = np.random.default_rng(SEED + 9)
    T, hidden, ffn, hd = 64, 1024, 3072, 128
    pos = rng.choice(8192, T, replace=False).astype(np.int32)
    x = _normal(rng, (T, hidden))
    dx = _t(gpu, x)
    for layer in range(28):
        (w_in, wt), (w_post, _), (wq, _), (wk, _) = [_weights(rng, n, "bf16") for n in (hidden, hidden, hd, hd)]
        q, k = _normal(rng, (T, 16, hd)), _normal(rng, (T, 8, hd))
        attn, mlp = _normal(rng, (T, hidden)), _normal(rng, (T, hidden))
        gate, up = _normal(rng, (T, ffn)), _normal(rng, (T, ffn))
        outs = gpu.layer_nongemm_step(dx, _dev_w(gpu, w_in, "bf16"), _t(gpu, q), _t(gpu, k), _dev_w(gpu, wq, "bf16"),
                                      _dev_w(gpu, wk, "bf16"), _t(gpu, pos), _t(gpu, attn), _dev_w(gpu, w_post, "bf16"),
                                      _t(gpu, gate), _t(gpu, up), _t(gpu, mlp), EPS, hd, THETA)
        got = {n: _np(t) for n, t in outs.items()}
        assert_close(got["normed"], ref(lambda g: R.rms_norm_w(g, x, w_in, EPS, wt)))
        qc, kc = ref(lambda g: R.qk_norm_rope(g, q, k, wq, wk, EPS, pos, hd, THETA, wt, cs_rounded=True))
        assert_bitexact(got["q_out"], qc)
        assert_bitexact(got["k_out"], kc)
        s_ref, y_ref = ref(lambda g: R.add_rms_norm_w(g, x, attn, w_post, EPS, wt))
        assert_bitexact(got["resid"], s_ref)
        assert_close(got["mlp_in"], y_ref)
        assert_close(got["act"], ref(lambda g: R.swiglu(g, gate, up)))
        x = ref(lambda g: g.add(s_ref, mlp))
        assert_bitexact(got["out"], x)
        dx = outs["out"]

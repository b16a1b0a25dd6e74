"""Pins the ggml-CPU restatement against the reference's own golden vectors.

G1: tests/qwen3_tts_decoder_layer_test.cpp:42-47 (a whole Qwen3 block, prefill
    then cached step) -- pins rms_norm eps placement, QK-norm before rope, NEOX
    half pairing, theta, silu*up and both residual adds.
G2: tests/qwen3_tts_code_predictor_test.cpp:46-61 (two-layer predictor logits,
    greedy codes, and the ordered multi-codebook embedding sum).
G3: tests/qwen3_tts_codec_ops_test.cpp:77-82 (SnakeBeta: the sin^2 Snake family
    through exp, sin, sqr, scale_bias, div and add nodes).
G4: tests/kokoro_decoder_test.cpp:81-90 (double-precision host Snake, layout
    t*C + c).
G5: tests/qwen3_tts_codec_ops_test.cpp:43-94 (the codec's causal convolution
    at dilation 2, its depthwise convolution, its causal transposed
    convolution and the ConvNeXt block) -- pins ggml_im2col's column order,
    padding, dilation and batching, ggml_col2im_1d's scatter and crop, and
    ggml_norm and ggml_gelu_erf inside the block.
G6: tests/vits_transpose_conv_test.cpp:237-265 (the transposed convolution's
    exact known answers and multichannel cases) -- pins ggml_col2im_1d's
    tap placement, padding and channel order.
Each test also plants a plausible mistake in the restatement's composition and
checks that the golden rejects it, so the golden is shown to constrain the
part it is claimed to pin.
"""
import json
import os

import numpy as np
import pytest

import ggml_ref as R

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def _shape(d):
    return {"head_dim": d["head_dim"], "heads": d["heads"], "kv_heads": d["kv_heads"],
            "rms_norm_eps": np.float32(d["rms_norm_eps"]), "rope_theta": np.float32(d["rope_theta"])}


def _causal(n):
    m = np.zeros((n, n), dtype=np.float32)
    m[np.triu_indices(n, 1)] = -np.inf
    return m


def run_decoder_golden(d, ops=None):
    s = R.LcgStream(d["seed"])
    W = R.layer_weights(s, d["hidden"], d["heads"], d["kv_heads"], d["head_dim"], d["intermediate"])
    P, pre, H = d["positions"], d["prefill"], d["hidden"]
    hidden = s.fill(P * H, 0.5, 0.0).reshape(P, H)
    cache = {"k": np.zeros((P, d["kv_heads"], d["head_dim"]), np.float32),
             "v": np.zeros((P, d["kv_heads"], d["head_dim"]), np.float32)}
    shape = _shape(d)
    out_pre = R.decoder_layer(hidden[:pre], np.arange(pre, dtype=np.int32), _causal(pre), W, shape, cache, 0, ops)
    out_step = R.decoder_layer(hidden[pre:], np.array([pre], np.int32), None, W, shape, cache, pre, ops)
    return np.concatenate([out_pre, out_step]).reshape(-1)


def test_g1_decoder_layer():
    d = _load("qwen3_decoder_layer.json")
    got = run_decoder_golden(d)
    diff = np.abs(got - np.array(d["expected_hidden"], np.float32)).max()
    assert diff < d["tolerance_cpu"], diff


class _GptjRope(R.OracleOps):
    """Planted mistake: interleaved (GPT-J) pairing instead of NEOX halves."""

    def qk_norm_rope(self, q, k, wq, wk, eps, pos, n_dims, theta):
        qn = R.run(lambda g: R.rms_norm_w(g, q, wq, eps))
        kn = R.run(lambda g: R.rms_norm_w(g, k, wk, eps))

        def gptj(x):
            y = x.copy()
            ts = np.float32(theta) ** np.float32(-2.0 / n_dims)
            for t, p in enumerate(pos):
                th = np.float32(p)
                for i in range(n_dims // 2):
                    c, s_ = np.float32(np.cos(th)), np.float32(np.sin(th))
                    x0, x1 = x[t, :, 2 * i], x[t, :, 2 * i + 1]
                    y[t, :, 2 * i], y[t, :, 2 * i + 1] = x0 * c - x1 * s_, x0 * s_ + x1 * c
                    th = np.float32(th * ts)
            return y
        return gptj(qn), gptj(kn)


class _NormAfterRope(R.OracleOps):
    """Planted mistake: rope before the per-head norm."""

    def qk_norm_rope(self, q, k, wq, wk, eps, pos, n_dims, theta):
        qr = R.run(lambda g: g.rope_neox(q, pos, n_dims, theta))
        kr = R.run(lambda g: g.rope_neox(k, pos, n_dims, theta))
        return (R.run(lambda g: R.rms_norm_w(g, qr, wq, eps)), R.run(lambda g: R.rms_norm_w(g, kr, wk, eps)))


class _EpsOutsideSqrt(R.OracleOps):
    """Planted mistake: eps added after the square root (1/(sqrt(mean)+eps))."""

    def rms_norm_w(self, x, w, eps):
        ms = (x.astype(np.float64) ** 2).mean(axis=-1, keepdims=True)
        return (x / (np.sqrt(ms) + 1e-2)).astype(np.float32) * w


class _SiluOnUp(R.OracleOps):
    """Planted mistake: silu applied to the up projection instead of the gate."""

    def swiglu(self, gate, up):
        return R.run(lambda g: R.swiglu(g, up, gate))


@pytest.mark.parametrize("ops", [_GptjRope(), _NormAfterRope(), _EpsOutsideSqrt(), _SiluOnUp()],
                         ids=["gptj-pairing", "norm-after-rope", "eps-outside-sqrt", "silu-on-up"])
def test_g1_rejects_planted_mistakes(ops):
    d = _load("qwen3_decoder_layer.json")
    got = run_decoder_golden(d, ops)
    diff = np.abs(got - np.array(d["expected_hidden"], np.float32)).max()
    assert diff > 10 * d["tolerance_cpu"], diff


def run_code_predictor(d, reverse_sum=False):
    s = R.LcgStream(d["seed"])
    H, V, G = d["hidden"], d["vocab"], d["code_groups"]
    layers = [R.layer_weights(s, H, d["heads"], d["kv_heads"], d["head_dim"], d["intermediate"])
              for _ in range(d["layers"])]
    norm = s.fill(H, 0.25, 1.0)
    tables = [s.fill(V * H, 0.5, 0.0).reshape(V, H) for _ in range(G - 1)]
    heads = [s.fill(V * H, 0.5, 0.0).reshape(V, H) for _ in range(G - 1)]
    prefill = s.fill(2 * H, 0.5, 0.0).reshape(2, H)
    shape = _shape(d)
    caches = [{"k": np.zeros((G, d["kv_heads"], d["head_dim"]), np.float32),
               "v": np.zeros((G, d["kv_heads"], d["head_dim"]), np.float32)} for _ in layers]
    logits_all, codes, filled = [], [], 0
    # code_predictor_schedule, src/arch/qwen3-tts/code-predictor-host.cpp:15-42
    schedule = [(None, 0, 0, 2)] + [(g - 1, g, g + 1, 1) for g in range(1, G - 1)]
    for table, head, first, count in schedule:
        if table is None:
            x, pos, mask = prefill, np.array([0, 1], np.int32), _causal(2)
        else:
            x = R.OracleOps().get_rows(tables[table], np.array([codes[-1]], np.int32))
            pos, mask = np.array([first], np.int32), None
        assert first == filled
        for W, cache in zip(layers, caches):
            x = R.decoder_layer(x, pos, mask, W, shape, cache, filled)
        x = R.run(lambda g: R.rms_norm_w(g, x, norm, shape["rms_norm_eps"]))
        logits = R.mul_mat(heads[head], x[-1:])[0]
        logits_all.append(logits)
        codes.append(int(np.argmax(logits)))
        filled += count
    order = list(range(G - 1))
    if reverse_sum:
        order = order[::-1]
    code_ids = np.array([[codes[t]] for t in order], np.int32)
    summed = R.run(lambda g: R.sum_code_embeddings(g, [tables[t] for t in order], R.F32, H, code_ids))
    return np.concatenate(logits_all), codes, summed.reshape(-1), tables


def test_g2_code_predictor_logits_codes_and_sum():
    d = _load("qwen3_code_predictor.json")
    logits, codes, summed, _ = run_code_predictor(d)
    assert codes == d["expected_codes"]
    assert np.abs(logits - np.array(d["expected_logits"], np.float32)).max() < d["tolerance_cpu"]
    assert np.abs(summed - np.array(d["expected_summed_embedding"], np.float32)).max() < d["tolerance_cpu"]


def test_g2_sum_is_ordered_and_table_specific():
    """The summed embedding pins which table each group reads: reading every
    code through table 0 misses the golden."""
    d = _load("qwen3_code_predictor.json")
    _, codes, _, tables = run_code_predictor(d)
    wrong = R.run(lambda g: R.sum_code_embeddings(g, [tables[0]] * len(codes), R.F32, d["hidden"],
                                                  np.array([[c] for c in codes], np.int32)))
    assert np.abs(wrong.reshape(-1) - np.array(d["expected_summed_embedding"], np.float32)).max() > 1e-2


def snake_beta_inputs(d):
    s = R.LcgStream(d["seed"])
    C, L = d["channels"], d["length"]
    raw = s.fill(C * L, 0.5, 0.0)
    x = np.ascontiguousarray(raw.reshape(C, L).T)  # [C, L] channels fastest = numpy (L, C)
    for name, count in d["draws_before_alpha"].items():
        if name != "signal":
            s.fill(count, 1.0, 0.0)
    alpha = s.fill(C, 0.5, 0.0)
    beta = s.fill(C, 0.5, 0.0)
    return x, alpha, beta


def test_g3_snake_beta():
    d = _load("qwen3_codec_snake_beta.json")
    x, a, b = snake_beta_inputs(d)
    got = R.run(lambda g: R.snake_beta(g, x, a, b)).reshape(-1)
    assert np.abs(got - np.array(d["expected_snake_beta"], np.float32)).max() < d["tolerance_cpu"]


def test_g3_rejects_guard_and_layout_mistakes():
    d = _load("qwen3_codec_snake_beta.json")
    x, a, b = snake_beta_inputs(d)
    exp = np.array(d["expected_snake_beta"], np.float32)
    # alpha in the denominator instead of beta
    wrong = R.run(lambda g: g.add(x, g.div(g.sqr(g.sin(g.mul(x, g.exp(a)))), g.exp(a)))).reshape(-1)
    assert np.abs(wrong - exp).max() > 1e-2
    # time-fastest layout (coefficients applied along the wrong axis)
    xt = np.ascontiguousarray(x.T)
    wrong = R.run(lambda g: R.snake_beta(g, xt, np.resize(a, xt.shape[1]), np.resize(b, xt.shape[1])))
    assert np.abs(wrong.T.reshape(-1) - exp).max() > 1e-2


def test_g4_kokoro_snake_matches_double_host_reference():
    """reference_snake, tests/kokoro_decoder_test.cpp:81-90: y = x + sin(a x)^2 / a in
    double on [C, T] (element (c, t) at t*C + c); compared at the test's 1e-4."""
    rng = np.random.default_rng(20260728)
    C, T = 16, 37
    x = rng.standard_normal((T, C)).astype(np.float32)
    alpha = np.exp(rng.uniform(np.log(0.1), np.log(10.0), C)).astype(np.float32)
    got = R.run(lambda g: R.snake(g, x, alpha))
    a = alpha.astype(np.float64)
    ref = x + np.sin(a * x) ** 2 / a
    assert np.abs(got - ref).max() < 1e-4
    # f32 node-by-node rounding stays within a few ulp of the double form
    assert np.abs(got - ref).max() < 8 * np.finfo(np.float32).eps * np.abs(ref).max()


# ---------------------------------------------------------------------------
# G5: the codec's convolutions through ggml_im2col
# ---------------------------------------------------------------------------

def codec_conv_inputs(d):
    """The fixture's tensors in LCG fill order; the signal as ggml [C, L] =
    numpy (L, C) (drawn channel-major, laid out channels fastest)."""
    s = R.LcgStream(d["seed"])
    v = {name: s.fill(count, scale, offset) for name, count, scale, offset in d["fill_order"]}
    C, L = d["channels"], d["length"]
    return np.ascontiguousarray(v["signal"].reshape(C, L).T), v


def causal_conv(x, w, b, dilation, im2col=None):
    """codec_causal_conv1d (qwen3-tts/codec.cpp:76-106): the time-major copy,
    ggml_im2col padded by the whole receptive field on both sides, the matrix
    product, the first L columns, the channel bias. x numpy (L, C); w numpy
    (OC, C, K) = ggml [K, C, OC]."""
    L, C = x.shape
    OC, _, K = w.shape
    cols = (im2col or R.run)(lambda g: g.im2col(np.ascontiguousarray(x.T), K, 1, (K - 1) * dilation, dilation))[0]
    return R.mul_mat(w.reshape(OC, C * K), cols)[:L] + b[None, :]


def depthwise_conv(x, w, b):
    """codec_causal_depthwise_conv1d (:108-137): each channel its own batch
    entry of ggml_im2col ([L, 1, C]), one K-tap product per channel, the first
    L columns, the channel bias. w numpy (C, 1, K)."""
    L, C = x.shape
    K = w.shape[-1]
    cols = R.run(lambda g: g.im2col(np.ascontiguousarray(x.T).reshape(C, 1, L), K, 1, K - 1, 1))  # (C, OW, K)
    wide = np.einsum("cok,ck->oc", cols.astype(np.float64), w.reshape(C, K).astype(np.float64)).astype(np.float32)
    return wide[:L] + b[None, :]


def convnext(x, v, d):
    """codec_convnext_block (:201-221)."""
    C = d["channels"]
    h = depthwise_conv(x, v["dwconv_weight"].reshape(C, 1, d["convnext_kernel"]), v["dwconv_bias"])
    h = R.run(lambda g: g.norm(h, np.float32(d["norm_eps"])))
    h = h * v["norm_weight"][None, :] + v["norm_bias"][None, :]
    h = R.mul_mat(v["pwconv1_weight"].reshape(4 * C, C), h) + v["pwconv1_bias"][None, :]
    h = R.run(lambda g: g.gelu_erf(h))
    h = R.mul_mat(v["pwconv2_weight"].reshape(C, 4 * C), h) + v["pwconv2_bias"][None, :]
    return x + h * v["gamma"][None, :]


def _dev(got, exp):
    return np.abs(np.asarray(got, np.float32).reshape(-1) - np.array(exp, np.float32)).max()


def test_g5_codec_convolutions():
    d = _load("qwen3_codec_convs.json")
    x, v = codec_conv_inputs(d)
    C, OC, K = d["channels"], d["out_channels"], d["kernel"]
    tol = d["tolerance_cpu"]
    assert _dev(causal_conv(x, v["conv_weight"].reshape(OC, C, K), v["conv_bias"], d["dilation"]),
                d["expected_causal_conv"]) < tol
    assert _dev(depthwise_conv(x, v["depthwise_weight"].reshape(C, 1, K), v["depthwise_bias"]),
                d["expected_depthwise"]) < tol
    assert _dev(convnext(x, v, d), d["expected_convnext"]) < tol


def test_g5_rejects_im2col_mistakes():
    """Reversed taps, dilation 1, padding on the left only (the port pads both
    sides and keeps the prefix) and the taps channel-minor in the column: each
    misses the causal golden."""
    d = _load("qwen3_codec_convs.json")
    x, v = codec_conv_inputs(d)
    C, OC, K, dil = d["channels"], d["out_channels"], d["kernel"], d["dilation"]
    w, b, exp = v["conv_weight"].reshape(OC, C, K), v["conv_bias"], d["expected_causal_conv"]
    assert _dev(causal_conv(x, w[:, :, ::-1].copy(), b, dil), exp) > 1e-2
    assert _dev(causal_conv(x, w, b, 1), exp) > 1e-2
    # left padding only: drop the right padding's columns, keep the first L
    L = x.shape[0]
    cols = R.run(lambda g: g.im2col(np.ascontiguousarray(x.T), K, 1, (K - 1) * dil, dil))[0]
    shifted = np.vstack([cols[(K - 1) * dil:], np.zeros_like(cols[:(K - 1) * dil])])
    assert _dev(R.mul_mat(w.reshape(OC, C * K), shifted)[:L] + b[None, :], exp) > 1e-2
    # column index k*C + ic instead of ic*K + k
    swapped = cols.reshape(-1, C, K).transpose(0, 2, 1).reshape(-1, C * K)
    assert _dev(R.mul_mat(w.reshape(OC, C * K), swapped)[:L] + b[None, :], exp) > 1e-2


def _direct_conv(x, w, s0, p0, d0):
    """The convolution's definition, summed in double: x (N, IC, IW), w (OC, IC,
    K); y[n, oc, ow] = sum over ic, k of w[oc, ic, k] * x[n, ic, ow*s0 + k*d0 - p0]
    (0 outside the input)."""
    N, IC, IW = x.shape
    OC, _, K = w.shape
    OW = R.conv_out_len(IW, K, s0, p0, d0)
    y = np.zeros((N, OC, OW))
    for ow in range(OW):
        for k in range(K):
            iw = ow * s0 + k * d0 - p0
            if 0 <= iw < IW:
                y[:, :, ow] += x[:, :, iw].astype(np.float64) @ w[:, :, k].T.astype(np.float64)
    return y


@pytest.mark.parametrize("N,IC,IW,K,s0,p0,d0", [(1, 3, 17, 3, 1, 1, 1), (2, 5, 40, 7, 1, 9, 3), (1, 4, 33, 11, 1, 25, 5),
                                                (3, 2, 29, 4, 2, 1, 1), (1, 1, 9, 5, 3, 0, 2), (2, 6, 8, 3, 1, 0, 3),
                                                (1, 2, 6, 7, 3, 0, 1)])
def test_im2col_products_equal_the_convolution(N, IC, IW, K, s0, p0, d0):
    """im2col then one K*IC product per output equals the direct convolution
    sum for strides, paddings and dilations, including kernels wider than the
    input (no tap in range: zero columns) and an output length that C's
    truncating division sets to 1."""
    rng = np.random.default_rng(N * 1000 + IC * 100 + IW + K + s0 + p0 + d0)
    x = rng.standard_normal((N, IC, IW)).astype(np.float32)
    w = rng.standard_normal((3, IC, K)).astype(np.float32)
    cols = R.run(lambda g: g.im2col(x, K, s0, p0, d0))
    assert cols.shape == (N, R.conv_out_len(IW, K, s0, p0, d0), IC * K)
    got = np.einsum("nok,ck->nco", cols.astype(np.float64), w.reshape(3, IC * K).astype(np.float64))
    np.testing.assert_allclose(got, _direct_conv(x, w, s0, p0, d0), rtol=0, atol=1e-9)


def test_im2col_without_an_output_position_is_refused():
    """ggml_im2col asserts OW > 0: (8 - 8 - 1)/1 + 1 = 0 and (5 - 6 - 1)/2 + 1 = 0."""
    assert R.conv_out_len(8, 3, 1, 0, 4) == 0 and R.conv_out_len(5, 7, 2, 0, 1) == 0
    assert R.conv_out_len(6, 7, 3, 0, 1) == 1  # (-1)/3 truncates to 0
    for args in ((8, 3, 1, 0, 4), (5, 7, 2, 0, 1)):
        with pytest.raises(ValueError):
            R.Graph().im2col(np.zeros((1, 2, args[0]), np.float32), *args[1:])


def test_im2col_f16_columns_round_to_nearest_even():
    """An F16 destination holds numpy's (IEEE round-to-nearest-even) half of
    each F32 column value, ties, subnormals, overflow and zeros included."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((2, 3, 50)) * 10.0 ** rng.integers(-8, 6, (2, 3, 50))).astype(np.float32)
    x.reshape(-1)[:6] = [65520.0, 65519.0, 2.0 ** -25, -(2.0 ** -24) * 1.5, -0.0, 1.0 + 2.0 ** -11]
    f32 = R.run(lambda g: g.im2col(x, 5, 2, 3, 2))
    f16 = R.run(lambda g: g.im2col(x, 5, 2, 3, 2, dst_type=R.F16))
    assert np.array_equal(f16, f32.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------------------
# G6 and G5's transposed convolution: ggml_col2im_1d
# ---------------------------------------------------------------------------

def transpose_conv(x, w, stride, padding, col2im=None):
    """vits transpose_conv1d with a zero bias (vits/operations.cpp:118-157):
    the kernel's (K, OC) pair merged out-channel-major, the product with the
    input, ggml_col2im_1d, then the transpose back. x numpy (L, IC) = ggml
    [IC, L]; w numpy (IC, OC, K) = ggml [K, OC, IC]. Returns (T, OC)."""
    ic, oc, k = w.shape
    cols = R.mul_mat(w.reshape(ic, oc * k).T.copy(), x)           # (L, K*OC) = ggml [K*OC, L]
    wide = (col2im or (lambda c: R.run(lambda g: g.col2im_1d(c, stride, oc, padding))))(cols)
    return np.ascontiguousarray(wide.T)


def _definition(x, w, stride, padding):
    """The transposed convolution from its definition (each input sample
    spreads its kernel taps), summed in double: (T, OC)."""
    L, ic = x.shape
    _, oc, k = w.shape
    raw = np.zeros((oc, (L - 1) * stride + k))
    for l in range(L):
        raw[:, l * stride:l * stride + k] += np.einsum("i,iok->ok", x[l].astype(np.float64), w.astype(np.float64))
    return raw[:, padding:raw.shape[1] - padding].T


def test_g6_transpose_conv_known_answers():
    """tests/vits_transpose_conv_test.cpp:237-246: exact, as the test compares."""
    d = _load("vits_transpose_conv.json")
    for c in d["single_channel"]:
        x = np.array(c["input"], np.float32).reshape(-1, 1)
        w = np.array(c["kernel"], np.float32).reshape(1, 1, -1)
        got = transpose_conv(x, w, c["stride"], c["padding"]).reshape(-1)
        assert np.array_equal(got, np.array(c["expected"], np.float32)), (got, c["expected"])


def test_g6_transpose_conv_multichannel_cases():
    """:255-264 with the test's fill (:126-134), against the definition,
    exactly (small integers: exact in every order). The third case (K 3,
    stride 1) sums three terms per output."""
    d = _load("vits_transpose_conv.json")
    km, kb = d["kernel_fill"]
    im, ib = d["input_fill"]
    for c in d["multichannel"]:
        K, OC, IC, L = c["kernel"], c["out_channels"], c["in_channels"], c["length"]
        w = (np.arange(K * OC * IC) % km + kb).astype(np.float32).reshape(IC, OC, K)
        x = (np.arange(IC * L) % im + ib).astype(np.float32).reshape(L, IC)
        got = transpose_conv(x, w, c["stride"], c["padding"])
        assert np.array_equal(got, _definition(x, w, c["stride"], c["padding"]).astype(np.float32)), c


def test_g5_codec_transposed_convolution():
    """tests/qwen3_tts_codec_ops_test.cpp:57-70: codec_causal_transpose_conv1d
    (qwen3-tts/codec.cpp:146-181): columns, col2im_1d without padding, the
    trailing K - stride samples dropped, the channel bias, back to channels
    fastest; at the test's 1e-4. The kernel's taps reversed, or the columns
    read tap-major, miss it."""
    d = _load("qwen3_codec_convs.json")
    x, v = codec_conv_inputs(d)
    C, OC, S = d["channels"], d["out_channels"], d["stride"]
    K = 2 * S
    w = v["transposed_weight"].reshape(C, OC, K)
    exp = np.array(d["expected_transposed"], np.float32)

    def causal(out):
        return out[:out.shape[0] - (K - S)] + v["transposed_bias"][None, :]
    assert np.abs(causal(transpose_conv(x, w, S, 0)).reshape(-1) - exp).max() < d["tolerance_cpu"]
    flipped = transpose_conv(x, w[:, :, ::-1].copy(), S, 0)
    assert np.abs(causal(flipped).reshape(-1) - exp).max() > 1e-2
    cols = R.mul_mat(w.reshape(C, OC * K).T.copy(), x)
    tap_major = cols.reshape(-1, OC, K).transpose(0, 2, 1).reshape(-1, OC * K).copy()
    wrong = R.run(lambda g: g.col2im_1d(tap_major, S, OC, 0)).T
    assert np.abs(causal(wrong).reshape(-1) - exp).max() > 1e-2


def test_col2im_refuses_empty_outputs():
    """vits/operations.cpp:134-137: a crop of the whole signal has no output
    (ggml_col2im_1d asserts); one sample less still builds."""
    with pytest.raises(ValueError):
        R.Graph().col2im_1d(np.zeros((1, 4 * 3), np.float32), 2, 3, 2)
    assert R.run(lambda g: g.col2im_1d(np.ones((1, 4 * 3), np.float32), 2, 3, 1)).shape == (3, 2)


# ---------------------------------------------------------------------------
# G7: Kokoro's inverse short-time transform (tests/kokoro_istft_test.cpp)
# ---------------------------------------------------------------------------

def istft_numpy(spec, n_fft, hop, *, phase=np.sin, weights_nyquist=1.0, normalise=True, offset=None):
    """An independent restatement through numpy's FFT: each frame is numpy's
    irfft of exp(log-magnitude) * e^(i phase(raw)) (irfft takes bin 0 and the
    Nyquist bin once and the rest twice, over n_fft), overlap-added with the
    periodic Hann window rounded to f32 and divided by the overlap-added
    squared window, trimmed by n_fft/2 at the front (torch.istft's centred
    form). The keyword arguments plant the mistakes a restatement could make."""
    frames = spec.shape[0]
    bins = n_fft // 2 + 1
    mag = np.exp(spec[:, :bins].astype(np.float64))
    ph = phase(spec[:, bins:].astype(np.float64))
    X = mag * np.exp(1j * ph)
    if weights_nyquist != 1.0:
        X[:, -1] *= weights_nyquist
    fr = np.fft.irfft(X, n=n_fft, axis=1)
    win = (0.5 * (1.0 - np.cos(2.0 * np.pi * np.arange(n_fft) / n_fft))).astype(np.float32).astype(np.float64)
    total = n_fft + hop * (frames - 1)
    acc, env = np.zeros(total), np.zeros(total)
    for f in range(frames):
        acc[f * hop:f * hop + n_fft] += fr[f] * win
        env[f * hop:f * hop + n_fft] += win * win
    off = n_fft // 2 if offset is None else offset
    kept = (frames - 1) * hop
    a, e = acc[off:off + kept], env[off:off + kept]
    out = np.where(np.abs(e) < np.float32(1e-11), 0.0, a / np.where(e == 0, 1, e) if normalise else a)
    return out.astype(np.float32)


def test_golden_kokoro_istft():
    """G7: the restatement against tests/kokoro_istft_test.cpp's torch.istft
    vector at the test's 1e-5; numpy's irfft restatement agrees with it to
    within an f32 ulp; the phase taken raw instead of through sin, the
    Nyquist bin counted twice, the window sum left undivided and the trim at
    0 instead of n_fft/2 each miss the vector by more than 1e-3."""
    d = _load("kokoro_istft.json")
    n, hop, frames = d["n_fft"], d["hop"], d["frames"]
    spec = np.array(d["spectrum"], np.float32).reshape(frames, n + 2)
    exp = np.array(d["expected_audio"], np.float32)
    got = R.run(lambda g: g.inverse_stft(spec, n, hop))
    assert got.shape == exp.shape and np.abs(got - exp).max() < d["tolerance"]
    ref = istft_numpy(spec, n, hop)
    assert np.abs(got - ref).max() <= 2 * np.spacing(np.abs(exp).max())
    for bad in (dict(phase=lambda p: p), dict(weights_nyquist=2.0), dict(normalise=False), dict(offset=0)):
        assert np.abs(istft_numpy(spec, n, hop, **bad) - exp).max() > 1e-3, bad


@pytest.mark.parametrize("n_fft,hop,frames", [(20, 5, 400), (16, 4, 33), (8, 3, 20), (6, 8, 10), (64, 16, 50)])
def test_istft_against_numpy_irfft(n_fft, hop, frames):
    """The direct double DFT of the restatement against numpy's irfft path on
    random spectra, Kokoro's n_fft 20 / hop 5 among them, and hops that do
    not divide n_fft or leave gaps (a window sum of 0 gives 0): within an f32
    ulp of the output's scale, > 99 % identical."""
    rng = np.random.default_rng(n_fft * 100 + hop)
    spec = rng.uniform(-2, 2, (frames, n_fft + 2)).astype(np.float32)
    got = R.run(lambda g: g.inverse_stft(spec, n_fft, hop))
    ref = istft_numpy(spec, n_fft, hop)
    assert got.shape == ((frames - 1) * hop,)
    assert np.abs(got - ref).max() <= 2 * np.spacing(np.abs(ref).max())
    assert (got == ref).mean() > 0.99
    with pytest.raises(ValueError):
        R.Graph().inverse_stft(spec, n_fft + 1, hop)


def _ref_istft_lib():
    """oracle/_ref's build of the reference's own inverse_stft, or None."""
    import ctypes
    path = os.path.join(R.HERE, "_ref", "libkokoro_istft_ref.so")
    if not os.path.exists(path):
        return None
    L = ctypes.CDLL(path)
    L.ref_inverse_stft.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                   ctypes.c_void_p, ctypes.c_uint64]
    L.ref_inverse_stft.restype = ctypes.c_int
    return L


@pytest.mark.parametrize("n_fft,hop,frames", [(8, 2, 9), (20, 5, 2401), (16, 4, 33), (8, 3, 20), (6, 8, 10),
                                              (64, 16, 50)])
def test_istft_restatement_is_the_reference_build(n_fft, hop, frames):
    """The restatement against the reference's own inverse_stft compiled from
    the checkout (oracle/_ref, `make -C oracle ref`): bit for bit on G7's
    spectrum and on random spectra (both double code in the same order over
    glibc's exp/sin/cos); the reference's refusals (odd window, no hop, a
    spectrum of the wrong size) returned as errors. Skipped where the
    reference checkout was not there to build it."""
    L = _ref_istft_lib()
    if L is None:
        pytest.skip("oracle/_ref not built (no reference checkout)")
    if (n_fft, hop, frames) == (8, 2, 9):
        spec = np.array(_load("kokoro_istft.json")["spectrum"], np.float32).reshape(frames, n_fft + 2)
    else:
        spec = np.random.default_rng(n_fft * 7 + hop).uniform(-3, 2, (frames, n_fft + 2)).astype(np.float32)
    out = np.empty((frames - 1) * hop, np.float32)
    assert L.ref_inverse_stft(spec.ctypes.data, frames, n_fft, hop, out.ctypes.data, out.size) == 0
    got = R.run(lambda g: g.inverse_stft(spec, n_fft, hop))
    assert np.array_equal(got.view(np.uint32), out.view(np.uint32))
    if (n_fft, hop, frames) == (8, 2, 9):
        assert L.ref_inverse_stft(spec.ctypes.data, frames, 7, hop, out.ctypes.data, out.size) != 0
        assert L.ref_inverse_stft(spec.ctypes.data, frames, n_fft, 0, out.ctypes.data, out.size) != 0


# ---------------------------------------------------------------------------
# G8: Kokoro's harmonic source (tests/kokoro_source_test.cpp)
# ---------------------------------------------------------------------------

def source_inputs(d):
    """G8's inputs and constants as harmonic_source's arguments."""
    H, S = d["harmonics"], d["scale"]
    f0 = np.array(d["f0"], np.float32)
    noise = np.array(d["noise"], np.float32).reshape(f0.size * S, H)
    kw = dict(rate=d["rate"], scale=S, sine_amp=np.float32(d["sine_amp"]), noise_std=np.float32(d["noise_std"]),
              voiced_threshold=np.float32(d["voiced_threshold"]), n_fft=d["n_fft"], hop=d["hop"])
    return (f0, np.array(d["merge_weight"], np.float32), np.float32(d["merge_bias"]),
            np.array(d["rand_ini"], np.float32), noise), kw


def phase_gap(a, b):
    """Distance on the circle."""
    return np.abs(np.arctan2(np.sin(a - b), np.cos(a - b)))


def check_source_golden(exc, har, d):
    bins = d["n_fft"] // 2 + 1
    exp_s = np.array(d["expected_source"], np.float32)
    exp_h = np.array(d["expected_har"], np.float32).reshape(-1, 2 * bins)
    assert exc.shape == exp_s.shape and har.shape == exp_h.shape
    assert np.abs(exc - exp_s).max() < d["tolerance_source"]
    assert np.abs(har[:, :bins] - exp_h[:, :bins]).max() < d["tolerance_magnitude"]
    assert phase_gap(har[:, bins:].astype(np.float64), exp_h[:, bins:].astype(np.float64)).max() < d["tolerance_phase"]


def test_golden_kokoro_source():
    """G8: the restatement against the upstream module's values at the test's
    bounds (excitation 1e-5, magnitudes 1e-5, phases 1e-4 on the circle);
    the phase accumulated on the sample grid instead of the coarse one, the
    resampling's half-sample offset dropped, the voiced threshold ignored, and
    the STFT without its reflect padding each miss."""
    d = _load("kokoro_source.json")
    args, kw = source_inputs(d)
    g = R.Graph()
    exc, har = g.harmonic_source(*args, **kw)
    g.compute()
    check_source_golden(exc, har, d)
    exp_s = np.array(d["expected_source"], np.float32)
    # planted mistakes, each on a copy of the numpy restatement below
    for bad in ("fine_grid", "no_half", "all_voiced", "no_reflect"):
        e, h = source_numpy(*args, **kw, mistake=bad)
        miss = np.abs(e - exp_s).max() > 1e-3 or np.abs(h[:, :d["n_fft"] // 2 + 1] -
                                                        np.array(d["expected_har"], np.float32).reshape(h.shape)[:, :d["n_fft"] // 2 + 1]).max() > 1e-3
        assert miss, bad
    e, h = source_numpy(*args, **kw)
    check_source_golden(e, h, d)


def source_numpy(f0, mw, bias, ri, noise, *, rate, scale, sine_amp, noise_std, voiced_threshold, n_fft, hop,
                 mistake=None):
    """An independent numpy restatement of the source (vectorised; the STFT by
    numpy's rfft over reflect-padded frames), with planted mistakes."""
    L, H = f0.size, mw.size
    U = L * scale
    f0u = np.repeat(f0, scale)
    rad = f0u[:, None] * np.arange(1, H + 1, dtype=np.float32)[None, :] / np.float32(rate)
    rad = (rad - np.floor(rad)).astype(np.float32)
    rad[0] += ri

    def resample(x, n_out):
        n_in = x.shape[0]
        o = np.arange(n_out, dtype=np.float64)
        pos = (o + 0.5) * (n_in / n_out) - (0.0 if mistake == "no_half" else 0.5)
        pos = np.maximum(pos, 0.0)
        lo = pos.astype(np.int64)
        hi = np.minimum(lo + 1, n_in - 1)
        w = (pos - lo).astype(np.float32)[:, None]
        return (x[lo] * (np.float32(1) - w) + x[hi] * w).astype(np.float32)
    if mistake == "fine_grid":
        run = np.cumsum(rad, axis=0, dtype=np.float32)
        fine = (run.astype(np.float64) * 2 * np.pi).astype(np.float32)
    else:
        crs = resample(rad, L)
        run = np.zeros_like(crs)
        acc = np.zeros(H, np.float32)
        for j in range(L):
            acc = (acc + crs[j]).astype(np.float32)
            run[j] = acc
        ph = (run.astype(np.float64) * 2.0 * np.pi * scale).astype(np.float32)
        fine = resample(ph, U)
    uv = (f0u > voiced_threshold).astype(np.float32) if mistake != "all_voiced" else np.ones(U, np.float32)
    gain = uv * np.float32(noise_std) + (np.float32(1) - uv) * (np.float32(sine_amp) / np.float32(3))
    vals = np.sin(fine.astype(np.float64)).astype(np.float32) * np.float32(sine_amp) * uv[:, None] + \
        gain[:, None] * noise
    merged = np.full(U, np.float32(bias), np.float32)
    for h in range(H):
        merged = (merged + mw[h] * vals[:, h]).astype(np.float32)
    exc = np.tanh(merged.astype(np.float64)).astype(np.float32)
    half = n_fft // 2
    padded = np.pad(exc, half, mode="reflect" if mistake != "no_reflect" else "constant")
    win = (0.5 * (1.0 - np.cos(2.0 * np.pi * np.arange(n_fft) / n_fft))).astype(np.float32)
    frames = U // hop + 1
    segs = np.stack([padded[f * hop:f * hop + n_fft] * win for f in range(frames)]).astype(np.float64)
    X = np.fft.rfft(segs, axis=1)
    return exc, np.concatenate([np.abs(X), np.angle(X)], axis=1).astype(np.float32)


def _ref_source_lib():
    import ctypes
    path = os.path.join(R.HERE, "_ref", "libkokoro_source_ref.so")
    if not os.path.exists(path):
        return None
    L = ctypes.CDLL(path)
    f, u32, u64, vp = ctypes.c_float, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p
    L.ref_harmonic_source.argtypes = [vp, u64, vp, f, vp, vp, u32, u32, u32, f, f, f, u32, u32, vp, u64, vp, u64]
    L.ref_harmonic_source.restype = ctypes.c_int
    return L


def random_source_case(seed, L, H, scale, n_fft, hop):
    rng = np.random.default_rng(seed)
    f0 = np.where(rng.random(L) < 0.2, rng.uniform(0, 8, L), rng.uniform(60, 400, L)).astype(np.float32)
    mw = rng.normal(0, 0.5, H).astype(np.float32)
    ri = np.concatenate([[0.0], rng.uniform(0, 1, H - 1)]).astype(np.float32)
    noise = rng.standard_normal((L * scale, H)).astype(np.float32)
    kw = dict(rate=24000, scale=scale, sine_amp=np.float32(0.1), noise_std=np.float32(0.003),
              voiced_threshold=np.float32(10.0), n_fft=n_fft, hop=hop)
    return (f0, mw, np.float32(rng.normal(0, 0.3)), ri, noise), kw


@pytest.mark.parametrize("case", ["golden", (50, 9, 300, 20, 5), (37, 3, 4, 8, 2), (20, 5, 16, 16, 4)])
def test_source_restatement_is_the_reference_build(case):
    """The restatement against the reference's own build_harmonic_source
    compiled from the checkout (oracle/_ref): bit for bit, excitation and
    spectrum, on G8's inputs and on random ones at Kokoro's 9 harmonics,
    upsampling 300, n_fft 20 and hop 5. Skipped where the reference checkout
    was not there to build it."""
    L = _ref_source_lib()
    if L is None:
        pytest.skip("oracle/_ref not built (no reference checkout)")
    if case == "golden":
        args, kw = source_inputs(_load("kokoro_source.json"))
    else:
        args, kw = random_source_case(sum(case), *case)
    f0, mw, bias, ri, noise = args
    g = R.Graph()
    exc, har = g.harmonic_source(*args, **kw)
    g.compute()
    e2, h2 = np.empty_like(exc), np.empty_like(har)
    assert L.ref_harmonic_source(f0.ctypes.data, f0.size, mw.ctypes.data, bias, ri.ctypes.data, noise.ctypes.data,
                                 mw.size, kw["rate"], kw["scale"], kw["sine_amp"], kw["noise_std"],
                                 kw["voiced_threshold"], kw["n_fft"], kw["hop"], e2.ctypes.data, e2.size,
                                 h2.ctypes.data, h2.size) == 0
    assert np.array_equal(exc.view(np.uint32), e2.view(np.uint32))
    assert np.array_equal(har.view(np.uint32), h2.view(np.uint32))


# ---------------------------------------------------------------------------
# The Qwen3-TTS speaker encoder's log-mel front end (qwen3-tts/mel.cpp)
# ---------------------------------------------------------------------------

MEL = dict(sample_rate=24000, n_fft=1024, hop=256, win_length=1024, mel_bins=128, fmin=0.0, fmax=12000.0)


def _ref_mel_lib():
    import ctypes
    path = os.path.join(R.HERE, "_ref", "libqwen3_mel_ref.so")
    if not os.path.exists(path):
        return None
    L = ctypes.CDLL(path)
    u32, u64, f, vp = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p
    L.ref_log_mel.argtypes = [vp, u64, u32, u32, u32, u32, u32, f, f, vp, u64, ctypes.POINTER(u64)]
    L.ref_log_mel.restype = ctypes.c_int
    return L


def oracle_log_mel(pcm, p):
    fb = R.mel_filterbank(p["sample_rate"], p["n_fft"], p["mel_bins"], p["fmin"], p["fmax"])
    return R.run(lambda g: g.log_mel(pcm, fb, p["n_fft"], p["hop"], p["win_length"]))


def test_log_mel_frame_counts_and_slaney_scale():
    """tests/qwen3_tts_mel_test.cpp:21-60: one second at 24 kHz gives the
    upstream 93 frames at hop 256 and 46 at hop 512 (what neither a centred
    nor a plain uncentred STFT gives: 94/47 and 89/44); the Slaney scale's
    closed forms -- 1 kHz at mel 15, linear below (f / (200/3)), a ratio of
    6.4 per 27 mels above -- placed through the filterbank's band edges; each
    filter's weights peak where its centre frequency falls and are
    area-normalised (2 / band width in Hz times the triangle's height 1)."""
    pcm = np.full(24000, 0.5, np.float32)
    assert oracle_log_mel(pcm, MEL).shape == (93, 128)
    assert oracle_log_mel(pcm, dict(MEL, hop=512)).shape == (46, 128)
    n, hop = 1024, 256
    assert (1 + 24000 // hop, 1 + (24000 - n) // hop) != (93, 93)
    fb = R.mel_filterbank(24000, 1024, 128, 0.0, 12000.0).astype(np.float64)
    hz = np.arange(513) * 24000 / 1024

    def mel_to_hz(m):
        return np.where(m >= 15, 1000 * 6.4 ** ((m - 15) / 27), m * 200 / 3)
    def hz_to_mel(f):
        return np.where(f >= 1000, 15 + 27 * np.log(f / 1000) / np.log(6.4), f * 3 / 200)
    edges = mel_to_hz(np.linspace(0, hz_to_mel(12000.0), 130))
    for b in (0, 10, 64, 127):
        w = fb[b]
        inside = (hz > edges[b]) & (hz < edges[b + 2])
        assert (w[~inside] == 0).all()
        tri = np.maximum(0, np.minimum((hz - edges[b]) / (edges[b + 1] - edges[b]),
                                       (edges[b + 2] - hz) / (edges[b + 2] - edges[b + 1])))
        assert np.allclose(w, (tri * 2 / (edges[b + 2] - edges[b])).astype(np.float32), rtol=1e-6, atol=1e-9)


def test_log_mel_tone_and_silence():
    """A 1 kHz tone puts its largest energy in the filter whose band centre
    is nearest 1 kHz, in every interior frame; digital silence gives the log
    floor, log(max(sqrt(1e-9) * filter sum, 1e-5))."""
    t = np.arange(24000) / 24000
    tone = (0.5 * np.sin(2 * np.pi * 1000 * t)).astype(np.float32)
    y = oracle_log_mel(tone, MEL)
    centres = np.where(np.linspace(0, 15 + 27 * np.log(12) / np.log(6.4), 130)[1:-1] >= 15,
                       1000 * 6.4 ** ((np.linspace(0, 15 + 27 * np.log(12) / np.log(6.4), 130)[1:-1] - 15) / 27),
                       np.linspace(0, 15 + 27 * np.log(12) / np.log(6.4), 130)[1:-1] * 200 / 3)
    assert (np.argmax(y[5:-5], axis=1) == np.argmin(np.abs(centres - 1000))).all()
    z = oracle_log_mel(np.zeros(24000, np.float32), MEL)
    fb = R.mel_filterbank(24000, 1024, 128, 0.0, 12000.0).astype(np.float64)
    floor = np.log(np.maximum(np.float32(np.sqrt(1e-9)) * fb.sum(axis=1), 1e-5)).astype(np.float32)
    assert np.allclose(z, floor[None, :], atol=1e-6)


@pytest.mark.parametrize("case", [("noise", 24000, MEL), ("tone", 7000, dict(MEL, hop=512)),
                                  ("noise", 3000, dict(MEL, n_fft=512, win_length=400, hop=160, mel_bins=80)),
                                  ("noise", 385, MEL)])
def test_log_mel_restatement_is_the_reference_build(case):
    """The restatement against the reference's own compute_log_mel compiled
    from the checkout (oracle/_ref): bit for bit, at the production
    parameters, at hop 512, with a shorter zero-padded window and fewer bins,
    and at the shortest clip upstream's reflect pad allows (385 samples);
    384 samples are refused by both. Skipped where the reference checkout
    was not there to build it."""
    import ctypes
    L = _ref_mel_lib()
    if L is None:
        pytest.skip("oracle/_ref not built (no reference checkout)")
    kind, ns, p = case
    rng = np.random.default_rng(ns)
    pcm = (rng.standard_normal(ns) * 0.2).astype(np.float32) if kind == "noise" else \
        (0.3 * np.sin(2 * np.pi * 440 * np.arange(ns) / 24000)).astype(np.float32)
    got = oracle_log_mel(pcm, p)
    out = np.empty(got.size + 16, np.float32)
    frames = ctypes.c_uint64()
    assert L.ref_log_mel(pcm.ctypes.data, ns, p["sample_rate"], p["n_fft"], p["hop"], p["win_length"],
                         p["mel_bins"], p["fmin"], p["fmax"], out.ctypes.data, out.size, ctypes.byref(frames)) == 0
    assert frames.value == got.shape[0]
    assert np.array_equal(got.reshape(-1).view(np.uint32), out[:got.size].view(np.uint32))
    if ns == 385:
        short = pcm[:384].copy()
        assert L.ref_log_mel(short.ctypes.data, 384, p["sample_rate"], p["n_fft"], p["hop"], p["win_length"],
                             p["mel_bins"], p["fmin"], p["fmax"], out.ctypes.data, out.size,
                             ctypes.byref(frames)) != 0
        with pytest.raises(ValueError):
            oracle_log_mel(short, p)

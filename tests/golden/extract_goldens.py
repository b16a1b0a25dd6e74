"""Writes the reference's golden vectors for this path as JSON fixtures.

Run in the build container, where the synthesize.cpp checkout is mounted read
only; it reads the reference's test sources as text and copies out only the
numeric literals (the expected outputs) plus the fixture configuration they
were produced under. Nothing from the reference is executed or imported.

    python tests/golden/extract_goldens.py [/path/to/synthesize.cpp]

Sources:
  G1 tests/qwen3_tts_decoder_layer_test.cpp:30-47   (kExpectedHidden, config)
  G2 tests/qwen3_tts_code_predictor_test.cpp:33-61  (logits, codes, summed embedding)
  G3 tests/qwen3_tts_codec_ops_test.cpp:34-82       (kExpectedSnakeBeta, config)
  G5 tests/qwen3_tts_codec_ops_test.cpp:34-94,184-210 (kExpectedCausalConv,
     kExpectedDepthwise, kExpectedTransposed, kExpectedConvNeXt, fill order)
  G6 tests/vits_transpose_conv_test.cpp:237-265 (the transposed convolution's
     known answers and the multichannel cases' shapes and fill rule)
  G7 tests/kokoro_istft_test.cpp:15-62 (Kokoro's inverse short-time transform
     against torch.istft: the raw spectrum, n_fft, hop, frames, the audio)
  G8 tests/kokoro_source_test.cpp:18-88 (Kokoro's harmonic source against the
     upstream module: f0, the merge, the random draws, the excitation and its
     spectrum, at reduced dimensions)
"""
import json
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def literal_array(text, name):
    m = re.search(r"%s\[\]\s*=\s*\{(.*?)\};" % re.escape(name), text, re.S)
    if m is None:
        raise SystemExit("array %s not found" % name)
    body = m.group(1)
    out = []
    for tok in body.replace("\n", " ").split(","):
        tok = tok.strip()
        if not tok:
            continue
        out.append(float(tok.rstrip("fF")) if ("." in tok or "e" in tok.lower()) else int(tok))
    return out


def constant(text, name):
    m = re.search(r"constexpr\s+\w+\s+%s\s*=\s*([-0-9.eEfu]+)\s*;" % re.escape(name), text)
    if m is None:
        raise SystemExit("constant %s not found" % name)
    tok = m.group(1).rstrip("fFuU")
    return float(tok) if ("." in tok or "e" in tok.lower()) else int(tok)


def call_args(text, name):
    """The argument lists of every call `name(...)` in text, split at top-level
    commas (braces and parentheses nest)."""
    out = []
    for m in re.finditer(re.escape(name) + r"\(", text):
        i, depth, args, cur = m.end(), 1, [], ""
        while depth:
            ch = text[i]
            if ch in "({":
                depth += 1
            elif ch in ")}":
                depth -= 1
            if depth == 1 and ch == ",":
                args.append(cur.strip())
                cur = ""
            elif depth:
                cur += ch
            i += 1
        args.append(cur.strip())
        out.append(args)
    return out


def float_list(arg):
    """A float vector argument: `{ a, b, ... }` or `std::vector<float>(n, v)`."""
    m = re.fullmatch(r"std::vector<float>\((\d+),\s*([-0-9.eE]+)f?\)", arg)
    if m:
        return [float(m.group(2))] * int(m.group(1))
    return [float(t.strip().rstrip("fF")) for t in arg.strip("{} ").split(",") if t.strip()]


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    read = lambda rel: open(os.path.join(root, rel), encoding="utf-8").read()

    t = read("tests/qwen3_tts_decoder_layer_test.cpp")
    g1 = {
        "source": "tests/qwen3_tts_decoder_layer_test.cpp:30-47,146-172",
        "hidden": constant(t, "kHidden"), "heads": constant(t, "kHeads"), "kv_heads": constant(t, "kKvHeads"),
        "head_dim": constant(t, "kHeadDim"), "intermediate": constant(t, "kIntermediate"),
        "positions": constant(t, "kPositions"), "prefill": constant(t, "kPrefill"),
        "rms_norm_eps": constant(t, "kRmsNormEps"), "rope_theta": constant(t, "kRopeTheta"),
        "seed": constant(t, "kSeed"),
        # (tensor, scale, offset) in LCG fill order, :146-158; hidden state last, :165.
        "fill_order": [["input_layernorm", 0.25, 1.0], ["q_proj", 0.5, 0.0], ["k_proj", 0.5, 0.0],
                       ["v_proj", 0.5, 0.0], ["o_proj", 0.5, 0.0], ["q_norm", 0.25, 1.0], ["k_norm", 0.25, 1.0],
                       ["post_attention_layernorm", 0.25, 1.0], ["gate_proj", 0.5, 0.0], ["up_proj", 0.5, 0.0],
                       ["down_proj", 0.5, 0.0], ["hidden", 0.5, 0.0]],
        "tolerance_cpu": 1e-4, "tolerance_gpu": 5e-3,
        "expected_hidden": literal_array(t, "kExpectedHidden"),
    }

    t = read("tests/qwen3_tts_code_predictor_test.cpp")
    g2 = {
        "source": "tests/qwen3_tts_code_predictor_test.cpp:33-61,159-214",
        "hidden": constant(t, "kHidden"), "heads": constant(t, "kHeads"), "kv_heads": constant(t, "kKvHeads"),
        "head_dim": constant(t, "kHeadDim"), "intermediate": constant(t, "kIntermediate"),
        "layers": constant(t, "kLayers"), "vocab": constant(t, "kVocab"), "code_groups": constant(t, "kCodeGroups"),
        "rms_norm_eps": constant(t, "kRmsNormEps"), "rope_theta": constant(t, "kRopeTheta"),
        "seed": constant(t, "kSeed"),
        "tolerance_cpu": 1e-4, "tolerance_gpu": 5e-3,
        "expected_logits": literal_array(t, "kExpectedLogits"),
        "expected_codes": literal_array(t, "kExpectedCodes"),
        "expected_summed_embedding": literal_array(t, "kExpectedSummedEmbedding"),
    }

    t = read("tests/qwen3_tts_codec_ops_test.cpp")
    g3 = {
        "source": "tests/qwen3_tts_codec_ops_test.cpp:34-82,184-234",
        "length": constant(t, "kLength"), "channels": constant(t, "kChannels"),
        "out_channels": constant(t, "kOutChannels"), "kernel": constant(t, "kKernel"),
        "stride": constant(t, "kStride"), "seed": constant(t, "kSeed"),
        # element counts drawn before alpha/beta, in fill order (:185-196)
        "draws_before_alpha": {
            "signal": constant(t, "kChannels") * constant(t, "kLength"),
            "conv_weight": constant(t, "kKernel") * constant(t, "kChannels") * constant(t, "kOutChannels"),
            "conv_bias": constant(t, "kOutChannels"),
            "depthwise_weight": constant(t, "kKernel") * constant(t, "kChannels"),
            "depthwise_bias": constant(t, "kChannels"),
            "transposed_weight": 2 * constant(t, "kStride") * constant(t, "kOutChannels") * constant(t, "kChannels"),
            "transposed_bias": constant(t, "kOutChannels"),
        },
        "tolerance_cpu": 1e-4, "tolerance_gpu": 5e-3,
        "expected_snake_beta": literal_array(t, "kExpectedSnakeBeta"),
    }

    C, L, OC, K, S = (constant(t, n) for n in ("kChannels", "kLength", "kOutChannels", "kKernel", "kStride"))
    g5 = {
        "source": "tests/qwen3_tts_codec_ops_test.cpp:34-94,184-210,249-251",
        "length": L, "channels": C, "out_channels": OC, "kernel": K, "stride": S,
        "dilation": constant(t, "kDilation"), "seed": constant(t, "kSeed"),
        # (tensor, element count, scale, offset) in LCG fill order (:185-210);
        # the signal is drawn channel-major and laid out channels fastest (:216-226)
        "fill_order": [["signal", C * L, 0.5, 0.0], ["conv_weight", K * C * OC, 0.5, 0.0],
                       ["conv_bias", OC, 0.25, 0.0], ["depthwise_weight", K * C, 0.5, 0.0],
                       ["depthwise_bias", C, 0.25, 0.0], ["transposed_weight", 2 * S * OC * C, 0.5, 0.0],
                       ["transposed_bias", OC, 0.25, 0.0], ["snake_alpha", C, 0.5, 0.0],
                       ["snake_beta", C, 0.5, 0.0], ["dwconv_weight", 7 * C, 0.5, 0.0],
                       ["dwconv_bias", C, 0.25, 0.0], ["norm_weight", C, 0.25, 1.0], ["norm_bias", C, 0.25, 0.0],
                       ["pwconv1_weight", C * 4 * C, 0.5, 0.0], ["pwconv1_bias", 4 * C, 0.25, 0.0],
                       ["pwconv2_weight", 4 * C * C, 0.5, 0.0], ["pwconv2_bias", C, 0.25, 0.0],
                       ["gamma", C, 0.5, 1.0]],
        "convnext_kernel": 7, "norm_eps": 1e-6,
        "tolerance_cpu": 1e-4, "tolerance_gpu": 5e-3,
        "expected_causal_conv": literal_array(t, "kExpectedCausalConv"),
        "expected_depthwise": literal_array(t, "kExpectedDepthwise"),
        "expected_transposed": literal_array(t, "kExpectedTransposed"),
        "expected_convnext": literal_array(t, "kExpectedConvNeXt"),
    }

    t = read("tests/vits_transpose_conv_test.cpp")
    single = []
    for a in call_args(t, "run_transpose_conv_case")[1:]:  # [0] is the definition
        if len(a) > 6:
            continue  # the F16-weight repeat of a case (same values)
        single.append({"kernel": float_list(a[1]), "input": float_list(a[2]), "stride": int(a[3]),
                       "padding": int(a[4]), "expected": float_list(a[5])})
    multi = []
    for a in call_args(t, "run_transpose_conv_multichannel_case")[1:]:
        if a[1].isdigit():
            multi.append({k: int(v) for k, v in zip(("kernel", "out_channels", "in_channels", "length", "stride",
                                                     "padding"), a[1:7])})
    g6 = {
        "source": "tests/vits_transpose_conv_test.cpp:82-110,126-134,237-265",
        # single-channel cases: kernel [K, 1, 1], input [1, L], bias 0, expected [1, T]
        "single_channel": [dict(c) for c in {tuple(sorted((k, tuple(v) if isinstance(v, list) else v)
                                                          for k, v in c.items())): c for c in single}.values()],
        # multichannel cases: kernel [K, OC, IC] with kernel[i] = i % 7 + 1 over its flat
        # (ic*OC + oc)*K + k order, input [IC, L] with input[i] = i % 5 + 1 (l*IC + ic),
        # bias 0; the test compares exactly against the definition (:82-110)
        "multichannel": multi, "kernel_fill": [7, 1], "input_fill": [5, 1],
    }

    t = read("tests/kokoro_istft_test.cpp")
    g7 = {
        "source": "tests/kokoro_istft_test.cpp:15-62",
        # frames rows of n_fft + 2 values (n_fft/2 + 1 log-magnitudes, then the raw
        # phases), frame-major; audio (frames - 1) * hop samples; the test's bound
        "n_fft": constant(t, "kNfft"), "hop": constant(t, "kHop"), "frames": constant(t, "kFrames"),
        "spectrum": literal_array(t, "kSpectrum"), "expected_audio": literal_array(t, "kExpectedAudio"),
        "tolerance": 1e-5,
    }

    t = read("tests/kokoro_source_test.cpp")

    def assigned(name):
        m = re.search(r"%s\s*=\s*([-0-9.eE]+)f?\s*;" % re.escape(name), t)
        if m is None:
            raise SystemExit("assignment %s not found" % name)
        return float(m.group(1))
    g8 = {
        "source": "tests/kokoro_source_test.cpp:18-88",
        "scale": constant(t, "kScale"), "harmonics": constant(t, "kHarmonics"), "n_fft": constant(t, "kNfft"),
        "hop": constant(t, "kHop"), "rate": constant(t, "kRate"),
        "sine_amp": assigned("h.source.sine_amp"), "noise_std": assigned("h.source.noise_std"),
        "voiced_threshold": assigned("h.source.voiced_threshold"),
        "merge_weight": literal_array(t, "kMergeWeight"), "merge_bias": assigned("kMergeBias"),
        "rand_ini": literal_array(t, "kRandIni"), "noise": literal_array(t, "kNoise"), "f0": literal_array(t, "kF0"),
        # the excitation (upsampled samples) and the spectrum, frame-major rows of
        # n_fft/2 + 1 magnitudes then as many phases; the test's bounds (phases on the circle)
        "expected_source": literal_array(t, "kExpectedSource"), "expected_har": literal_array(t, "kExpectedHar"),
        "tolerance_source": 1e-5, "tolerance_magnitude": 1e-5, "tolerance_phase": 1e-4,
    }

    for name, obj in (("qwen3_decoder_layer", g1), ("qwen3_code_predictor", g2), ("qwen3_codec_snake_beta", g3),
                      ("qwen3_codec_convs", g5), ("vits_transpose_conv", g6), ("kokoro_istft", g7),
                      ("kokoro_source", g8)):
        with open(os.path.join(HERE, name + ".json"), "w") as f:
            json.dump(obj, f, indent=1)
            f.write("\n")
        print("wrote", name)


if __name__ == "__main__":
    main()

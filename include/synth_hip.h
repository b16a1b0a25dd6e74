/*
 * synth_hip.h -- C ABI of libsynth_hip, the MI355X (gfx950) kernels for the
 * memory-bound non-GEMM primitives that synthesize.cpp's graph builders emit.
 *
 * Every entry point keeps the semantics of the ggml op (or the ggml op run)
 * the reference graphs build today, so a ggml backend module can map nodes
 * onto these calls without changing any graph. Citations name the reference
 * call site (paths relative to the synthesize.cpp checkout) whose node or
 * node run each entry point replaces.
 *
 * Conventions (all entry points):
 *   - Tensors are described by shp_tensor, which mirrors ggml_tensor's
 *     ne[4]/nb[4]/type/data: ne[0] is the fastest dimension, nb[] are byte
 *     strides, type is a ggml type id. data is a DEVICE pointer owned by
 *     the caller.
 *   - Rows (the ne[0] extent) must be contiguous (nb[0] == element size);
 *     rows may be strided in dims 1..3 exactly as ggml views allow.
 *   - `stream` is a hipStream_t (NULL = the null stream). Every call is
 *     asynchronous and ordered on that stream; nothing is allocated,
 *     nothing synchronises, and no exception crosses this boundary.
 *   - Return value is a shp_status_t. SHP_ERR_UNSUPPORTED means "valid for
 *     ggml, not implemented here": a backend module should report
 *     supports_op == false for such a node so it falls back, as
 *     docs/backends.md:269-274 describes.
 *   - Calls on distinct streams may run concurrently from different host
 *     threads (no global mutable state in the launch path).
 */
#ifndef SYNTH_HIP_H
#define SYNTH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SHP_ABI_VERSION 1u

typedef int32_t shp_status_t;
#define SHP_OK              ((shp_status_t) 0)
#define SHP_ERR_INVALID_ARG ((shp_status_t) 1)  /* where ggml would assert: null, shape/type mismatch */
#define SHP_ERR_UNSUPPORTED ((shp_status_t) 2)  /* legal ggml, not handled here: fall back */
#define SHP_ERR_BACKEND     ((shp_status_t) 17) /* HIP launch failure; same value as SYNTH_ERR_BACKEND */

/* ggml_type values (upstream enum ggml_type). */
#define SHP_TYPE_F32  0
#define SHP_TYPE_F16  1
#define SHP_TYPE_Q8_0 8
#define SHP_TYPE_Q5_K 13
#define SHP_TYPE_I32  26
#define SHP_TYPE_BF16 30

/* ggml rope mode bit (GGML_ROPE_TYPE_NEOX); src/arch/qwen3-tts/operations.cpp:16. */
#define SHP_ROPE_TYPE_NEOX 2

/*
 * Every extent must be at least 1: a tensor with a zero extent is
 * SHP_ERR_INVALID_ARG at every entry point, and shp_graph_node_supported
 * reports a node with one unsupported, so ggml keeps it (an empty node is a
 * no-op there). The graph builders never emit one on this path: the hosts
 * reject zero frames and groups first (qwen3-tts/profile.cpp:325,1485).
 */
typedef struct shp_tensor {
    int32_t type;     /* SHP_TYPE_* */
    int32_t reserved; /* must be 0 */
    int64_t ne[4];    /* extents, ne[0] fastest; each >= 1 */
    size_t  nb[4];    /* byte strides */
    void *  data;     /* device pointer */
} shp_tensor;

typedef void * shp_stream_t; /* hipStream_t */

uint32_t     shp_abi_version(void);
const char * shp_status_string(shp_status_t status);

/*
 * ggml_get_rows(src, ids): dst[:, r, i11, i12] = to_f32(src[:, ids[r, i11, i12], i11, i12]).
 * src F32/F16/BF16/Q8_0/Q5_K; ids I32 [n, ne11, ne12]; dst F32 [ne00, n, ne11, ne12].
 * Conversions are exact (Q8_0: one product q*d per element), so results are
 * bit-identical to ggml-CPU. Q5_K (256-element super-blocks of 176 bytes,
 * the Matrix-role tables of Q5_K_MIXED packages, qwen3-tts/catalog.cpp:
 * 165-192): y = (d*sc)*q - dmin*m, whose products are exact in f32, so its
 * one rounding (the subtraction) is ggml-CPU's dequantize_row_q5_K's too. An id outside [0, src.ne[1]) is never read:
 * its output row is filled with quiet NaN (ggml-CPU aborts instead; callers
 * pre-validate ids on the host, src/arch/qwen3-tts/talker-host.cpp:42).
 * Replaces: src/arch/qwen3-tts/talker.cpp:44 and :86,
 *           src/arch/qwen3-tts/code-predictor.cpp:31,
 *           src/arch/qwen3-tts/model.cpp:1347,1449.
 */
shp_status_t shp_get_rows(const shp_tensor * src, const shp_tensor * ids, shp_tensor * dst, shp_stream_t stream);

/*
 * Multi-codebook gather->sum: the node run of sum_code_embeddings,
 * src/arch/qwen3-tts/code-predictor.cpp:82-107 (one ggml_get_rows per group,
 * then ggml_add in group order). tables[g] are [ne0, rows_g] of one common
 * type (F32/F16/BF16/Q8_0/Q5_K); ids is I32 [frames, n_tables] contiguous, frames
 * fastest (code-predictor.cpp:86-99); dst is F32 [ne0, frames].
 * dst[:, f] = ((row_0 + row_1) + row_2) + ... in f32, in group order, so the
 * result is bit-identical to the unfused node run. Out-of-range ids give a
 * NaN row as in shp_get_rows. n_tables in [1, 64].
 */
shp_status_t shp_get_rows_sum(const shp_tensor * tables,
                              int32_t            n_tables,
                              const shp_tensor * ids,
                              shp_tensor *       dst,
                              shp_stream_t       stream);

/*
 * ggml_rms_norm(x, eps) followed by ggml_mul(., w): the rms_norm() helper,
 * src/arch/qwen3-tts/operations.cpp:27-32 (with as_f32's BF16->F32 cast of
 * the gain folded in, :20-25). Per row: sum of f32 squares accumulated in
 * double, mean = (float)(sum/ne0), scale = 1.0f/sqrtf(mean+eps),
 * y = (x*scale)*w. x, y F32 of one shape; w F32/BF16/F16 with exactly ne0
 * elements (broadcast over rows), or NULL for a bare ggml_rms_norm.
 * Also replaces talker.cpp:168, code-predictor.cpp:68 and the per-head
 * QK-norm at operations.cpp:98-99 when called on the [head_dim, heads, T] view.
 */
shp_status_t shp_rms_norm_mul(const shp_tensor * x,
                              const shp_tensor * w,
                              float              eps,
                              shp_tensor *       y,
                              shp_stream_t       stream);

/*
 * ggml_add(a, b) followed by rms_norm()*w: the residual add feeding the
 * post-attention norm (operations.cpp:143-145) and the layer-output add
 * feeding the next layer's input norm (:147 -> :86). s = a + b (f32) is
 * written to `sum` when it is non-NULL (the residual the graph carries on);
 * y = rms_norm(s)*w. a, b, sum, y F32 of one shape.
 */
shp_status_t shp_add_rms_norm_mul(const shp_tensor * a,
                                  const shp_tensor * b,
                                  const shp_tensor * w,
                                  float              eps,
                                  shp_tensor *       sum,
                                  shp_tensor *       y,
                                  shp_stream_t       stream);

/*
 * ggml_rope_ext(x, pos, NULL, n_dims, mode, n_ctx_orig, freq_base,
 * freq_scale, ext_factor, attn_factor, beta_fast, beta_slow) in NEOX mode,
 * as at src/arch/qwen3-tts/operations.cpp:101-104. x, y F32
 * [head_dim, heads, T, 1]; pos I32 [T]. theta for pair i at position p is
 * the ggml-CPU recurrence theta_0 = p, theta_{i+1} = theta_i * powf(base,
 * -2/n_dims) in f32 (replayed exactly), rotated by cos/sin of
 * freq_scale*theta times attn_factor. Elements >= n_dims are copied.
 * Supported: mode == SHP_ROPE_TYPE_NEOX, ext_factor == 0 (beta_* unused).
 */
shp_status_t shp_rope_ext(const shp_tensor * x,
                          const shp_tensor * pos,
                          int32_t            n_dims,
                          int32_t            mode,
                          float              freq_base,
                          float              freq_scale,
                          float              ext_factor,
                          float              attn_factor,
                          shp_tensor *       y,
                          shp_stream_t       stream);

/*
 * Fused per-head QK-norm then NEOX rope for q and k in one launch: the node
 * run rms_norm(q)*w_q -> rope_ext(q) and rms_norm(k)*w_k -> rope_ext(k) of
 * src/arch/qwen3-tts/operations.cpp:98-104. q [head_dim, q_heads, T],
 * k [head_dim, kv_heads, T] F32 (k may be NULL with k_out/wk NULL); wq, wk
 * [head_dim] F32/BF16/F16; pos I32 [T]. Same arithmetic, in the same order,
 * as the two unfused node runs (norm, mul, rope each rounded in f32).
 */
shp_status_t shp_qk_norm_rope(const shp_tensor * q,
                              const shp_tensor * k,
                              const shp_tensor * wq,
                              const shp_tensor * wk,
                              float              eps,
                              const shp_tensor * pos,
                              int32_t            n_dims,
                              float              freq_base,
                              float              freq_scale,
                              shp_tensor *       q_out,
                              shp_tensor *       k_out,
                              shp_stream_t       stream);

/*
 * shp_qk_norm_rope plus this step's KV-cache write, in one launch: the node
 * runs of src/arch/qwen3-tts/operations.cpp:98-116, i.e. q and k normalised
 * and rotated as in shp_qk_norm_rope, then ggml_cpy(k) and ggml_cpy(v) into
 * the cache views ggml_view_3d(cache, head_dim, kv_heads, T, nb1, nb2,
 * filled*nb2). q_out receives q; the rotated k goes straight to rows
 * [filled, filled + T) of k_cache and v (copied unchanged) to the same rows
 * of v_cache. k_cache, v_cache: F32 [head_dim, kv_heads, capacity, 1] with
 * capacity >= filled + T (operations.cpp:71-76); v F32 of k's shape. No other
 * cache row is touched.
 */
shp_status_t shp_qk_norm_rope_kv(const shp_tensor * q,
                                 const shp_tensor * k,
                                 const shp_tensor * v,
                                 const shp_tensor * wq,
                                 const shp_tensor * wk,
                                 float              eps,
                                 const shp_tensor * pos,
                                 int32_t            n_dims,
                                 float              freq_base,
                                 float              freq_scale,
                                 shp_tensor *       q_out,
                                 shp_tensor *       k_cache,
                                 shp_tensor *       v_cache,
                                 int64_t            filled,
                                 shp_stream_t       stream);

/*
 * shp_qk_norm_rope_kv with the cache slot in device memory, so that one
 * captured HIP graph of a decode step can be replayed step after step (the
 * reference rebuilds its graph every step, src/arch/qwen3-tts/model.cpp:1311,
 * 1437): slot is an I32 tensor of one element holding `filled`, read by the
 * kernel when it runs. If slot < 0 or slot + T > the caches' rows, no cache
 * row is written (q_out still is) and, when status (an I32 tensor of one
 * element, or NULL) is given, *status is set to 1; the library never clears
 * it. k_cache and v_cache as in shp_qk_norm_rope_kv, with at least T rows.
 */
shp_status_t shp_qk_norm_rope_kv_at(const shp_tensor * q,
                                    const shp_tensor * k,
                                    const shp_tensor * v,
                                    const shp_tensor * wq,
                                    const shp_tensor * wk,
                                    float              eps,
                                    const shp_tensor * pos,
                                    int32_t            n_dims,
                                    float              freq_base,
                                    float              freq_scale,
                                    shp_tensor *       q_out,
                                    shp_tensor *       k_cache,
                                    shp_tensor *       v_cache,
                                    const shp_tensor * slot,
                                    shp_tensor *       status,
                                    shp_stream_t       stream);

/*
 * ggml_silu(g) followed by ggml_mul(., u): the SwiGLU of
 * src/arch/qwen3-tts/operations.cpp:39-41 (== ggml_swiglu_split(g, u)).
 * y = (g / (1 + expf(-g))) * u in f32. g, u, y F32 of one shape.
 * u == NULL gives a bare ggml_silu (talker.cpp:47).
 */
shp_status_t shp_swiglu(const shp_tensor * g, const shp_tensor * u, shp_tensor * y, shp_stream_t stream);

/*
 * ggml_swiglu(a) / ggml_swiglu_swapped(a): single-tensor GLU. a is F32
 * [2n, rows...]; gate is the first half of each row (second when swapped),
 * up the other half; y is F32 [n, rows...].
 */
shp_status_t shp_glu_swiglu(const shp_tensor * a, int32_t swapped, shp_tensor * y, shp_stream_t stream);

/*
 * Snake: the five-node run of src/arch/kokoro/operations.cpp:137-147,
 * t = x*alpha_c; s = sinf(t); q = s*s; r = q/alpha_c; y = x + r (each
 * rounded in f32, in this order). x, y F32 [C, T] channels fastest
 * (ne[0] == C); alpha F32 with exactly C elements ([1, C, 1] or [C]).
 */
shp_status_t shp_snake(const shp_tensor * x, const shp_tensor * alpha, shp_tensor * y, shp_stream_t stream);

/*
 * Guarded Snake (Snake1d): codec_snake of src/arch/omnivoice/codec.cpp:51-68,
 * t = x*alpha_c; s = sinf(t); q = s*s; g = alpha_c*1 + 1e-9 (ggml_scale_bias);
 * r = q/g; y = x + r, each rounded in f32. Shapes as shp_snake.
 */
shp_status_t shp_snake_guarded(const shp_tensor * x, const shp_tensor * alpha, shp_tensor * y, shp_stream_t stream);

/*
 * SnakeBeta: codec_snake_beta of src/arch/qwen3-tts/codec.cpp:184-199,
 * a_c = expf(log_alpha_c); b_c = expf(log_beta_c); t = x*a_c; s = sinf(t);
 * q = s*s (ggml_sqr); g = b_c*1 + 1e-9 (ggml_scale_bias); r = q/g; y = x + r,
 * each rounded in f32. x, y F32 [C, T]; log_alpha and log_beta F32 with
 * exactly C elements each ([C] or [C, 1]).
 */
shp_status_t shp_snake_beta(const shp_tensor * x,
                            const shp_tensor * log_alpha,
                            const shp_tensor * log_beta,
                            shp_tensor *       y,
                            shp_stream_t       stream);

/*
 * ggml_add(a, b) then ggml_leaky_relu(., slope, false): the residual carry
 * of src/arch/vits/waveform-decoder.cpp:150-158 (layer l's closing add and
 * layer l+1's opening leaky) and kokoro/generator.cpp:115,180.
 * s = a + b; y = (s > 0 ? s : 0) + slope*(s < 0 ? s : 0) (so -0 -> +0,
 * NaN -> 0), bit-identical to the two ggml nodes. b == NULL gives a bare
 * leaky_relu of a (waveform-decoder.cpp:205,225). sum == NULL skips the
 * residual output. All F32 of one shape.
 */
shp_status_t shp_add_leaky_relu(const shp_tensor * a,
                                const shp_tensor * b,
                                float              slope,
                                shp_tensor *       sum,
                                shp_tensor *       y,
                                shp_stream_t       stream);

/*
 * ggml_add(a, b) with b the same shape as a or any shape that repeats to it
 * (ggml_can_repeat: each b->ne[d] divides a->ne[d], and b is read at
 * (i0 % b.ne0, i1 % b.ne1, i2 % b.ne2, i3 % b.ne3) as ggml-CPU does): one row
 * broadcast over rows, and the per-channel [1, C] bias of a time-major
 * [T, C] activation, one value per row (vits/waveform-decoder.cpp:118-121,
 * qwen3-tts/codec.cpp:180). The plain residual add at
 * src/arch/qwen3-tts/operations.cpp:143,147 when it is not fused into a norm.
 */
shp_status_t shp_add(const shp_tensor * a, const shp_tensor * b, shp_tensor * y, shp_stream_t stream);

/*
 * Single nodes of the runs above, for graphs where a run does not stay
 * together (the node executor in synth_graph.h falls back to them), each
 * bit-identical to its ggml-CPU node except where noted:
 *   shp_mul  ggml_mul, b as in shp_add: SwiGLU's mul when an up-projection
 *            sits between it and the silu (qwen3-tts/operations.cpp:39-41),
 *            the Snake multiplies (kokoro/operations.cpp:143,145)
 *   shp_div  ggml_div, b as in shp_add (kokoro/operations.cpp:146), IEEE
 *   shp_sin  ggml_sin (kokoro/operations.cpp:144): the Snake kernels' sine,
 *            within 1 ulp of the correctly rounded one as libm's sinf is
 *            (so a Snake run and its nodes one by one agree bit for bit)
 *   shp_sqr  ggml_sqr (qwen3-tts/codec.cpp:196)
 *   shp_cpy  ggml_cpy / ggml_cast into F32 of the same shape from F32, F16
 *            or BF16 (qwen3-tts/operations.cpp:20-25, the KV-cache writes
 *            :109-116); rows may be strided on either side. An F32 x may
 *            also be a transposed or permuted view, ne[0] strided and one of
 *            dims 1..3 contiguous (nb = 4): ggml_cont(ggml_transpose(x)),
 *            the vocoder's time-major copies (vits/operations.cpp:72,87,100,
 *            108), and ggml_cont(ggml_permute(v, 1, 0, 2, 3))
 *            (qwen3-tts/operations.cpp:136); y's rows contiguous. Such a view
 *            with no contiguous dimension, or of another type, is
 *            SHP_ERR_UNSUPPORTED
 * All F32 unless stated; y has a's shape.
 */
shp_status_t shp_mul(const shp_tensor * a, const shp_tensor * b, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_div(const shp_tensor * a, const shp_tensor * b, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_sin(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_sqr(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_cpy(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);

/*
 * The activations and arithmetic the codec, vocoder and speech encoders put
 * between their GEMMs, as ggml-CPU's vec forms compute them in f32 (the
 * device's tanhf / expf / expm1f / erff, within the tolerance of glibc's):
 *   shp_sub      ggml_sub, b as in shp_add (bit-identical)
 *   shp_tanh     ggml_tanh (vits/waveform-decoder.cpp:228, kokoro/operations.cpp:133)
 *   shp_sigmoid  ggml_sigmoid, 1 / (1 + expf(-x))
 *   shp_elu      ggml_elu, x > 0 ? x : expm1f(x)
 *   shp_gelu_erf ggml_gelu_erf, 0.5 x (1 + erff(x / sqrt 2)) (qwen3-tts/codec.cpp:222)
 *   shp_clamp    ggml_clamp, MAX(MIN(x, hi), lo) with ggml's macros, so a NaN
 *                gives hi (qwen3-tts/codec.cpp:481; bit-identical)
 *   shp_norm     ggml_norm: (x - mean) / sqrtf(variance + eps) per row, mean
 *                and variance summed in double (qwen3-tts/codec.cpp:216,
 *                kokoro/operations.cpp:12,93)
 * All F32; y has x's (a's) shape; rows contiguous, any row strides.
 */
shp_status_t shp_sub(const shp_tensor * a, const shp_tensor * b, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_tanh(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_sigmoid(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_elu(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_gelu_erf(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_clamp(const shp_tensor * x, float lo, float hi, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_norm(const shp_tensor * x, float eps, shp_tensor * y, shp_stream_t stream);

/*
 * The speaker encoder's and the VITS text encoder / duration predictor's
 * remaining element and row ops, as ggml-CPU's vec forms compute them:
 *   shp_relu   ggml_relu, x > 0 ? x : 0 (-0 and NaN give +0; vits/text-encoder.cpp:71,
 *              qwen3-tts/speaker-encoder.cpp:184)
 *   shp_neg    ggml_neg, -x (vits/duration-predictor.cpp:113,117,205)
 *   shp_step   ggml_step, x > 0 ? 1 : 0 (vits/duration-predictor.cpp:89-90)
 *   shp_sqrt   ggml_sqrt, correctly rounded (qwen3-tts/speaker-encoder.cpp:294)
 *   shp_sum_rows  ggml_sum_rows: y [1, ne1, ne2, ne3] = each row's sum,
 *              accumulated in double and rounded to f32 once
 *              (qwen3-tts/speaker-encoder.cpp:293,374, vits/duration-predictor.cpp:47,93)
 *   shp_mean   ggml_mean: that sum divided by ne0 in f32 (speaker-encoder.cpp:195,350)
 *   shp_mul_sum_rows  ggml_mul(x, w) then ggml_sum_rows as one launch: each
 *              row's f32 products summed as shp_sum_rows sums (the attention-
 *              weighted statistics, speaker-encoder.cpp:293,374); w x's shape
 * All F32, rows contiguous, any row strides; the element ops' y has x's shape;
 * the row sums' y may not overlap x or w. The row sums agree with ggml-CPU's
 * element-order double sum unless the two double sums fall on opposite sides
 * of an f32 rounding boundary.
 */
shp_status_t shp_relu(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_neg(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_step(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_sqrt(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_sum_rows(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_mean(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);
shp_status_t shp_mul_sum_rows(const shp_tensor * x, const shp_tensor * w, shp_tensor * y, shp_stream_t stream);

/*
 * Kokoro's inverse short-time transform (kokoro/decoder-host.cpp:28-100,
 * inverse_stft; run by the host at kokoro/model.cpp:1056 on the generator's
 * output): spectrum F32 [n_fft + 2, frames] -- per frame n_fft/2 + 1
 * log-magnitudes, then as many raw phases (the phase is their sine) -- into
 * audio F32 [(frames - 1) * hop]: per frame the real inverse DFT of
 * exp(log-magnitude) * e^(i sin(phase)), weighted by the periodic Hann window
 * (rounded to f32) and overlap-added at hop, divided by the overlap-added
 * squared window (0 where that is below 1e-11), trimmed by n_fft/2; in
 * double, rounded to f32 once. n_fft even >= 2, hop >= 1, frames >= 2;
 * frames may sit at any row stride. SHP_ERR_UNSUPPORTED when a block's frames
 * do not fit the kernel's LDS (n_fft/2 + 1 complex bins per frame; Kokoro's
 * n_fft 20, hop 5 use 37 KB).
 */
shp_status_t shp_inverse_stft(const shp_tensor * spectrum, int32_t n_fft, int32_t hop, shp_tensor * audio,
                              shp_stream_t stream);

/*
 * Kokoro's harmonic-plus-noise source and its short-time spectrum
 * (kokoro/source.cpp:60-184, build_harmonic_source; run by the host between
 * the prosody and generator graphs): f0 F32 [L] (the prosody curve),
 * merge_weight and rand_ini F32 [H] (the 9-to-1 merge and the initial phases),
 * noise F32 [H, L*upsample_scale] (the additive draws, frame-major) into
 * excitation F32 [L*upsample_scale] (tanh of the merged harmonics) and har F32
 * [n_fft + 2, frames] (frames = L*upsample_scale/hop + 1; per frame n_fft/2 + 1
 * magnitudes, then as many phases): the phase increments accumulated on the
 * f0 grid in f32 in frame order (bit for bit the host code's sums), resampled
 * with PyTorch's align_corners=false mapping, sin(phase) * sine_amp for voiced
 * samples (f0 > voiced_threshold) plus the noise at noise_std (unvoiced:
 * sine_amp/3), merged in harmonic order from merge_bias; then torch.stft's
 * centred, reflect-padded framing with the periodic Hann window, the DFT in
 * double, hypot and atan2. The sine and tanh are the device's f32 ones (an ulp
 * or two from the host library's). All contiguous; H <= 64, n_fft even in
 * 2..64, at least two samples; har's memory stages the L*H coarse phases
 * between the launches (SHP_ERR_UNSUPPORTED when it is smaller).
 */
shp_status_t shp_harmonic_source(const shp_tensor * f0, const shp_tensor * merge_weight, float merge_bias,
                                 const shp_tensor * rand_ini, const shp_tensor * noise, int32_t sampling_rate,
                                 int32_t upsample_scale, float sine_amp, float noise_std, float voiced_threshold,
                                 int32_t n_fft, int32_t hop, shp_tensor * excitation, shp_tensor * har,
                                 shp_stream_t stream);

/*
 * The Qwen3-TTS speaker encoder's log-mel front end (qwen3-tts/mel.cpp:
 * 174-299, compute_log_mel; run by the host before the ECAPA graph): pcm F32
 * [samples] reflect-padded by (n_fft - hop)/2 on each side and framed
 * without centring (frames = 1 + (samples + 2*pad - n_fft)/hop), the periodic
 * Hann window of win_length centred in n_fft, the host code's radix-2 FFT on
 * f32 values with double twiddles and butterflies (stage for stage), the
 * amplitude sqrt(re^2 + im^2 + 1e-9), the filterbank F32 [n_fft/2 + 1,
 * mel_bins] weighted sum in double, log(max(energy, 1e-5)), into mel F32
 * [mel_bins, frames]. n_fft a power of two up to 2048, win_length and hop at
 * most n_fft, more samples than the pad; all contiguous. Non-finite samples
 * are not screened here (the reference refuses them; its audio normaliser
 * does so before this stage on the synthesis path).
 */
shp_status_t shp_log_mel(const shp_tensor * pcm, const shp_tensor * filterbank, int32_t n_fft, int32_t hop,
                         int32_t win_length, shp_tensor * mel, shp_stream_t stream);

/*
 * The Slaney mel filterbank shp_log_mel weights the amplitudes with
 * (qwen3-tts/mel.cpp:96-170, librosa's filters.mel with htk=False and
 * norm='slaney'): mel_bins rows of n_fft/2 + 1 f32 weights into the host
 * array out. Host code, no device work: computed once per model and
 * uploaded.
 */
shp_status_t shp_mel_filterbank(int32_t sample_rate, int32_t n_fft, int32_t mel_bins, float fmin, float fmax,
                                float * out);

/*
 * ggml_concat(a, b, dim): y of a's shape except y->ne[dim] = a->ne[dim] +
 * b->ne[dim]; y(i) = a(i) where i[dim] < a->ne[dim], else b(i) with
 * i[dim] - a->ne[dim]. All F32, rows contiguous (any row strides). The code
 * predictor's prefill input, the talker's hidden state and its code embedding
 * as one two-position block (src/arch/qwen3-tts/model.cpp:1450), and the
 * encoders' feature joins (qwen3-tts/speaker-encoder.cpp:236,335,358).
 */
shp_status_t shp_concat(const shp_tensor * a, const shp_tensor * b, int32_t dim, shp_tensor * y, shp_stream_t stream);

/*
 * ggml_im2col(kernel, x, s0, 0, p0, 0, d0, 0, false, y->type): the 1-D column
 * matrix in front of every convolution GEMM of the vocoders, codecs and
 * speech encoders (vits/waveform-decoder.cpp:104, vits/operations.cpp:40,103,
 * kokoro/operations.cpp:76, omnivoice/codec.cpp:114,
 * omnivoice/reference-encoder.cpp:190, qwen3-tts/codec.cpp:96,129,
 * qwen3-tts/speaker-encoder.cpp:174, qwen3-tts/codec-encoder.cpp:359).
 *   kernel: only its extents are read: K = ne[0], ne[1] = x's channel count
 *           (data may be NULL, as for the shape-only kernel of a packed
 *           weight, vits/waveform-decoder.cpp:102-103)
 *   x:      F32 [IW, IC, N, 1], any 4-byte strides: time-contiguous rows, or
 *           the transposed view of a channel-major [IC, IW] activation (read
 *           directly, so the ggml_cont in front of the reference's im2col,
 *           qwen3-tts/codec.cpp:94,125, is not needed)
 *   y:      F32 or F16 [IC*K, OW, N, 1], contiguous, not overlapping x, with
 *           OW = (IW + 2*p0 - d0*(K-1) - 1)/s0 + 1 (C division) >= 1:
 *           y[n][ow][ic*K + k] = x[n][ic][ow*s0 + k*d0 - p0], 0 outside the
 *           input; an F16 y holds each value rounded to nearest even.
 * s0, d0 >= 1, p0 >= 0. Bit-exact (a gather). SHP_ERR_INVALID_ARG for shapes
 * that do not match, SHP_ERR_UNSUPPORTED for other types or an overlap.
 */
/*
 * ggml_col2im_1d(cols, stride, out_channels, padding): the scatter-back of a
 * transposed convolution computed as a matrix product, the upsampling layers
 * of the vocoders and codecs (vits/operations.cpp:118-140,
 * omnivoice/codec.cpp:150-159, qwen3-tts/codec.cpp:163-171).
 *   cols: F32 [K*OC, L, 1, 1], rows contiguous (any row stride): column l
 *         holds the K*OC taps of input sample l, out-channel major, tap minor
 *   y:    F32 [T, OC, 1, 1], T = (L-1)*stride + K - 2*padding >= 1, rows
 *         contiguous (any row stride), not overlapping cols:
 *         y[oc][t] = sum of cols[l][oc*K + k] over l*stride + k = t + padding,
 *         accumulated from +0.0f in ascending l
 * stride, out_channels >= 1, padding >= 0, K = cols->ne[0] / out_channels.
 * With K <= 2*stride (every upsampling layer of the reference's models) each
 * output is a sum of at most two terms, the same in any order.
 */
shp_status_t shp_col2im_1d(const shp_tensor * cols,
                           int32_t            stride,
                           int32_t            out_channels,
                           int32_t            padding,
                           shp_tensor *       y,
                           shp_stream_t       stream);

/*
 * ggml_pad_ext(x, lp0, rp0, lp1, rp1, lp2, rp2, lp3, rp3) (and ggml_pad, all
 * left pads 0): y[i] = x[i - lpad] where every i_d - lpad_d lies inside x,
 * else 0; the right pads are what y's extents leave (y->ne[d] >= x->ne[d] +
 * lpad[d]). The transposed convolution's zero-stuffed spread and its edge
 * widening (kokoro/operations.cpp:190-196,253-260), the text encoder's
 * relative-position tables (vits/text-encoder.cpp:36,50), the encoders' edge
 * padding (omnivoice/reference-encoder.cpp:482, qwen3-tts/codec-encoder.cpp:351).
 * x, y F32, rows contiguous (any row strides), not overlapping; lpad[4] >= 0.
 */
shp_status_t shp_pad(const shp_tensor * x, const int32_t * lpad, shp_tensor * y, shp_stream_t stream);

/*
 * ggml_pad_reflect_1d(x, p0, p1): rows widened by p0 and p1 samples mirrored
 * about the edge samples (not repeating them), as PyTorch's reflect padding
 * (qwen3-tts/speaker-encoder.cpp:164). 0 <= p0, p1 < x->ne[0]; y F32 [ne0 + p0
 * + p1, ne1, ne2, ne3].
 */
shp_status_t shp_pad_reflect_1d(const shp_tensor * x, int32_t p0, int32_t p1, shp_tensor * y, shp_stream_t stream);

/*
 * ggml_repeat(x, y's shape) / ggml_repeat_4d: y[i] = x[i_d mod x->ne_d], each
 * of y's extents a multiple of x's: the vector broadcast over time and the
 * frame doubling of the Kokoro decoder (kokoro/operations.cpp:21-24,113-120),
 * the speaker encoder's statistics broadcast (qwen3-tts/speaker-encoder.cpp:
 * 356-357), the codec encoder's edge replication (codec-encoder.cpp:183,188).
 */
shp_status_t shp_repeat(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);

/*
 * ggml_acc(a, b, nb1, nb2, nb3, offset): y = a with b added into the view of
 * y at byte `offset` with byte strides nb1..nb3 (b's extents, element stride
 * 4): y[offset + 4*i0 + i1*nb1 + i2*nb2 + i3*nb3] = a[same] + b[i0, i1, i2, i3],
 * every other element a's. The talker's prefill input: the codec stream, the
 * x-vector's slot and the ICL acoustic block added into the text stream at a
 * row offset (qwen3-tts/talker.cpp:31,90,109,112,115). a, y F32 contiguous,
 * same shape; y == a (the same data) is ggml's inplace form and touches the
 * window only, any other overlap of y with a or b is refused. b F32, rows
 * contiguous (any row strides). The strides and offset are multiples of 4 and
 * the view's rows do not overlap (each extent times its stride at most the
 * next stride, unit dimensions aside); a view past a's end is refused.
 */
shp_status_t shp_acc(const shp_tensor * a,
                     const shp_tensor * b,
                     int64_t            nb1,
                     int64_t            nb2,
                     int64_t            nb3,
                     int64_t            offset,
                     shp_tensor *       y,
                     shp_stream_t       stream);

shp_status_t shp_im2col(const shp_tensor * kernel,
                        const shp_tensor * x,
                        int32_t            s0,
                        int32_t            p0,
                        int32_t            d0,
                        shp_tensor *       y,
                        shp_stream_t       stream);

/*
 * The tail of the time-major vocoder convolution, in one pass
 * (vits/waveform-decoder.cpp:111,118-121, then :147,150 or the next layer's
 * :146): s = ggml_add(ggml_cont(ggml_transpose(out)), reshape_2d(bias, 1, C)),
 * then s = ggml_add(s, r) when r is given, then y = ggml_leaky_relu(s, slope)
 * when apply_leaky (sum, if given, receives s), else y = s (sum must be NULL).
 * Each add is one f32 rounding, in that order, so y and sum are bit-identical
 * to the nodes one by one.
 *   x:   an F32 transposed or permuted view as shp_cpy takes it, ne[0]
 *        strided; a view with nb[0] == 4 (the transpose of a one-channel
 *        [1, T] result) is SHP_ERR_UNSUPPORTED: its ggml_cont is a plain
 *        copy, and such a tail runs as its nodes
 *   b:   F32 [1, ne1, ne2, ne3]: one value per row of y, rows evenly
 *        strided; or F32 [ne0]: one row repeated over y's rows (the channel
 *        bias of a channel-major result, qwen3-tts/codec.cpp:58-59,134-140,
 *        179-181, where the add precedes the transpose: the add is exact per
 *        element, so adding after the transposing copy gives the same bits)
 *   r:   NULL or F32 of y's shape and strides (the residual)
 *   sum: NULL or F32 of y's shape and strides
 *   y:   F32 of x's shape, rows contiguous
 * Replaces the CPY, ADD(, ADD)(, LEAKY_RELU) nodes of that tail; no
 * counterpart entry point in the reference (ggml runs them as nodes).
 */
shp_status_t shp_cont_add_leaky_relu(const shp_tensor * x,
                                     const shp_tensor * b,
                                     const shp_tensor * r,
                                     int32_t            apply_leaky,
                                     float              slope,
                                     shp_tensor *       sum,
                                     shp_tensor *       y,
                                     shp_stream_t       stream);

/*
 * The non-GEMM node runs of one Qwen3 decoder layer,
 * src/arch/qwen3-tts/operations.cpp:84-147, in the layer's order. The
 * layer's matrix products and its attention run between these node runs in
 * a model, so their outputs are inputs here:
 *   normed       = rms_norm(x)*w_in                        (:85-86)
 *   q_out, k_out = rope(rms_norm(q)*wq), rope(rms_norm(k)*wk)  (:98-104)
 *   resid        = x + attn_out                            (:143)
 *   mlp_in       = rms_norm(resid)*w_post                  (:145)
 *   act          = silu(gate)*up                           (:39-41 via :146)
 *   out          = resid + mlp_out                         (:147)
 * Five launches on `stream`, each the launch of shp_rms_norm_mul,
 * shp_qk_norm_rope, shp_add_rms_norm_mul, shp_swiglu and shp_add, with the
 * same results. Every tensor's presence, type and shape is checked first:
 * a malformed step returns SHP_ERR_INVALID_ARG with nothing enqueued.
 * x, normed, attn_out, resid, mlp_in, mlp_out, out: F32 [hidden, T];
 * q, q_out: F32 [head_dim, q_heads, T]; k, k_out: F32 [head_dim, kv_heads, T];
 * gate, up, act: F32 [ffn, T]; pos: I32 [T]; w_in, w_post: [hidden] and
 * wq, wk: [head_dim], each F32, BF16 or F16. NEOX rope over n_dims, with
 * freq_scale 1.
 */
typedef struct shp_layer_step {
    const shp_tensor * x;
    const shp_tensor * w_in;
    shp_tensor *       normed;
    const shp_tensor * q;
    const shp_tensor * k;
    const shp_tensor * wq;
    const shp_tensor * wk;
    const shp_tensor * pos;
    shp_tensor *       q_out;
    shp_tensor *       k_out;
    const shp_tensor * attn_out;
    const shp_tensor * w_post;
    shp_tensor *       resid;
    shp_tensor *       mlp_in;
    const shp_tensor * gate;
    const shp_tensor * up;
    shp_tensor *       act;
    const shp_tensor * mlp_out;
    shp_tensor *       out;
    float              eps;
    float              freq_base;
    int32_t            n_dims;
    int32_t            reserved; /* must be 0 */
} shp_layer_step;

shp_status_t shp_layer_nongemm_step(const shp_layer_step * step, shp_stream_t stream);

/*
 * ggml_soft_max_ext(a, mask, scale, max_bias): the attention softmax of
 * src/arch/qwen3-tts/operations.cpp:131-133. Per row: w = a*scale + mask
 * (f32), v = expf(w - max w), y = v * (float)(1/sum v) with the sum in
 * double. a, y F32 [ne0, ne1, ne2, ne3] (y may alias a); mask NULL or F32
 * [ne0, >= ne1, ne2 | divisor, ne3 | divisor], row i1 of head i2 reading mask
 * row i1 of mask head i2 % mask->ne[2]. max_bias != 0 (ALiBi) gives
 * SHP_ERR_UNSUPPORTED.
 */
shp_status_t shp_soft_max_ext(const shp_tensor * a,
                              const shp_tensor * mask,
                              float              scale,
                              float              max_bias,
                              shp_tensor *       y,
                              shp_stream_t       stream);

/*
 * ggml_diag_mask_inf(x, n_past) (and its inplace form, y == x): element i0
 * of row i1 of each matrix becomes -inf when i0 > n_past + i1, the rest are
 * copied; the codec encoder's causal attention scores
 * (qwen3-tts/codec-encoder.cpp:482). x, y F32 of one shape, rows contiguous.
 */
shp_status_t shp_diag_mask_inf(const shp_tensor * x, int32_t n_past, shp_tensor * y, shp_stream_t stream);

/*
 * ggml_diag_mask_inf(a, n_past) then ggml_soft_max_ext(., NULL, scale, 0) as
 * one launch (qwen3-tts/codec-encoder.cpp:482-483): the masked scores are
 * replaced by -inf and the rest scaled, then the softmax of
 * shp_soft_max_ext; bit-identical to the two nodes. scale positive and
 * finite (-inf times it stays -inf).
 */
shp_status_t shp_soft_max_causal(const shp_tensor * a, int32_t n_past, float scale, shp_tensor * y,
                                 shp_stream_t stream);

/*
 * ggml_exp: y = expf(x) per element, F32 of one shape
 * (src/arch/qwen3-tts/codec.cpp:193-194, vits/latent-sampling.cpp:30).
 */
shp_status_t shp_exp(const shp_tensor * x, shp_tensor * y, shp_stream_t stream);

/*
 * ggml_scale_bias(x, s, b) and ggml_scale(x, s) (b == 0): y = x*s when
 * b == 0 (one multiply, so -0 stays -0), else y = fma(x, s, b) rounded once,
 * as ggml-CPU's vectorised path computes it. With s == 1 (the guards of
 * omnivoice/codec.cpp:68 and qwen3-tts/codec.cpp:197) every evaluation order
 * gives the same f32. F32 of one shape.
 */
shp_status_t shp_scale_bias(const shp_tensor * x, float s, float b, shp_tensor * y, shp_stream_t stream);

/*
 * The branch average of src/arch/vits/waveform-decoder.cpp:214-225 and
 * src/arch/kokoro/generator.cpp:165-179: summed = ((t0 + t1) + t2) + ...
 * (ggml_add in term order), current = summed*scale (ggml_scale, a plain
 * multiply), y = leaky_relu(current, slope) as in shp_add_leaky_relu. Pass
 * scale = 1/n as the builders compute it (1.0f/(float)n); a single term with
 * scale 1 is the bare leaky_relu, as the builders skip the scale there and
 * x*1 is exact. terms points to n_terms (1..8) F32 tensors of y's shape;
 * mean (optional) receives current. All tensors contiguous (a strided view
 * gives SHP_ERR_UNSUPPORTED).
 */
shp_status_t shp_sum_scale_leaky_relu(const shp_tensor * terms,
                                      int32_t            n_terms,
                                      float              scale,
                                      float              slope,
                                      shp_tensor *       mean,
                                      shp_tensor *       y,
                                      shp_stream_t       stream);

#ifdef __cplusplus
}
#endif

#endif /* SYNTH_HIP_H */

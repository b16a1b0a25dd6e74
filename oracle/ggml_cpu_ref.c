/*
 * ggml_cpu_ref.c -- TEST INFRASTRUCTURE ONLY (see ggml_cpu_ref.h).
 *
 * A restatement of ggml-CPU op arithmetic for the nodes synthesize.cpp's graph
 * builders emit on the fused-primitive path. The upstream ggml-cpu sources
 * (ops.cpp, vec.h, ggml-quants.c) are not present in the reference checkout
 * (its ggml/ submodule is empty), so each op states the published algorithm
 * and cites the reference site that builds the node. Built with
 * -ffp-contract=off so that every f32 operation is rounded on its own, which
 * is the order the formulas below are written in.
 *
 * Last-ulp points this restatement fixes by choice (ggml's own build may
 * differ there, and the tests absorb that in tolerance):
 *   - silu uses libm expf for every element (ggml vectorises it with its own
 *     SIMD expf, within ~1 ulp of libm);
 *   - rope is computed without fused multiply-add;
 *   - scale_bias with a non-zero bias is one fused multiply-add (ggml's
 *     vectorised path on FMA hardware; its scalar tail may round twice).
 *
 * Parity unpinned, because no golden vector, closed form or build of the real
 * ggml fixes these last-ulp questions (ggml is absent from this environment):
 *   - ggml's SIMD silu exp, against the libm expf used here;
 *   - libm sinf/cosf as ggml links them;
 *   - the pinned commit's RMS accumulation in double and its cached theta
 *     recurrence for rope (both restated as upstream ggml-CPU does them);
 *   - leaky-ReLU's NaN and -0 handling at that commit.
 * Each op's arithmetic is otherwise pinned by the reference's goldens and by
 * closed forms (tests/test_oracle_goldens.py, tests/test_oracle_closed_forms.py).
 */
#define _GNU_SOURCE
#include "ggml_cpu_ref.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------ */
/* conversions                                                         */
/* ------------------------------------------------------------------ */

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e    = (h >> 10) & 0x1fu;
    const uint32_t m    = h & 0x3ffu;
    uint32_t       bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            /* subnormal half: m * 2^-24, exact in f32 */
            const float v = (float) m * 5.9604644775390625e-8f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

float orc_bf16_to_fp32(uint16_t h) {
    const uint32_t bits = (uint32_t) h << 16;
    float          out;
    memcpy(&out, &bits, 4);
    return out;
}

uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax   = x & 0x7fffffffu;
    if (ax > 0x7f800000u) {
        return (uint16_t) (sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) { /* >= 65520 rounds to infinity */
        return (uint16_t) (sign | 0x7c00u);
    }
    if (ax < 0x38800000u) { /* below the smallest normal half, 2^-14 */
        float v;
        memcpy(&v, &ax, 4);
        const uint32_t m = (uint32_t) rintf(v * 16777216.0f); /* v / 2^-24, round half even */
        return (uint16_t) (sign | m);
    }
    const uint32_t e    = (ax >> 23) - 112u;
    const uint32_t mant = ax & 0x7fffffu;
    uint32_t       h    = (e << 10) | (mant >> 13);
    const uint32_t rem  = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
        h += 1u;
    }
    return (uint16_t) (sign | h);
}

/* ggml's fp32 -> bf16: round half to even, NaN forced quiet. */
uint16_t orc_fp32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return (uint16_t) ((u >> 16) | 64u);
    }
    return (uint16_t) ((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
}

static float to_f32(int type, const void * row, int64_t i) {
    switch (type) {
        case ORC_F32:
            return ((const float *) row)[i];
        case ORC_F16:
            return orc_fp16_to_fp32(((const uint16_t *) row)[i]);
        case ORC_BF16:
            return orc_bf16_to_fp32(((const uint16_t *) row)[i]);
        default:
            return NAN;
    }
}

static size_t row_bytes(int type, int64_t ne0) {
    switch (type) {
        case ORC_F32:
            return (size_t) ne0 * 4u;
        case ORC_F16:
        case ORC_BF16:
            return (size_t) ne0 * 2u;
        case ORC_Q8_0:
            return (size_t) (ne0 / 32) * 34u;
        case ORC_Q5_K:
            return (size_t) (ne0 / 256) * 176u;
        default:
            return 0;
    }
}

/* dequantize_row_q8_0: y[32b + j] = qs[j] * fp16(d), one rounding (exact). */
static void dequantize_row_q8_0(const uint8_t * x, float * y, int64_t k) {
    const int64_t nb = k / 32;
    for (int64_t b = 0; b < nb; ++b) {
        const uint8_t * blk = x + b * 34;
        uint16_t        dh;
        memcpy(&dh, blk, 2);
        const float    d  = orc_fp16_to_fp32(dh);
        const int8_t * qs = (const int8_t *) (blk + 2);
        for (int j = 0; j < 32; ++j) {
            y[b * 32 + j] = (float) qs[j] * d;
        }
    }
}

/* dequantize_row_q5_K with get_scale_min_k4 (upstream ggml's ggml-quants.c;
 * the tables of the reference's Q5_K_MIXED packages,
 * src/arch/qwen3-tts/catalog.cpp:165-192). A 176-byte super-block holds 256
 * elements: f16 d, f16 dmin, scales[12], qh[32], qs[128]. Sub-block s
 * (0..7, 32 elements each) has a 6-bit scale and min packed in scales -- for
 * s < 4 the low six bits of scales[s] and scales[s + 4]; for s >= 4 the
 * nibbles of scales[s + 4] topped with the high two bits of scales[s - 4]
 * (scale) and scales[s] (min). Its element i takes the low (s even) or high
 * (s odd) nibble of qs[32*(s/2) + i] and bit s of qh[i] as bit 4. The value
 * is (d*sc)*q - dmin*m. */
static void q5k_scale_min(const uint8_t * scales, int s, int * sc, int * m) {
    if (s < 4) {
        *sc = scales[s] & 63;
        *m  = scales[s + 4] & 63;
    } else {
        *sc = (scales[s + 4] & 15) | ((scales[s - 4] >> 6) << 4);
        *m  = (scales[s + 4] >> 4) | ((scales[s] >> 6) << 4);
    }
}

static void dequantize_row_q5_k(const uint8_t * x, float * y, int64_t k) {
    for (int64_t b = 0; b < k / 256; ++b) {
        const uint8_t * blk = x + b * 176;
        uint16_t        dh, mh;
        memcpy(&dh, blk, 2);
        memcpy(&mh, blk + 2, 2);
        const float     d    = orc_fp16_to_fp32(dh);
        const float     dmin = orc_fp16_to_fp32(mh);
        const uint8_t * qh   = blk + 16;
        const uint8_t * qs   = blk + 48;
        for (int s = 0; s < 8; ++s) {
            int sc, m;
            q5k_scale_min(blk + 4, s, &sc, &m);
            const float d1 = d * (float) sc;
            const float m1 = dmin * (float) m;
            for (int i = 0; i < 32; ++i) {
                const int q = ((qs[32 * (s / 2) + i] >> (4 * (s & 1))) & 15) | (((qh[i] >> s) & 1) << 4);
                y[b * 256 + 32 * s + i] = d1 * (float) q - m1;
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* ops: each runs thread ith's share of rows, as ggml-CPU splits them  */
/* ------------------------------------------------------------------ */

static atomic_int g_node_error;

static void chunk(int64_t nr, int ith, int nth, int64_t * r0, int64_t * r1) {
    const int64_t dr = (nr + nth - 1) / nth;
    *r0              = dr * ith;
    *r1              = *r0 + dr < nr ? *r0 + dr : nr;
}

/* ggml_add / ggml_mul / ggml_div, src1 repeated over rows or along a row.
 * Sites: qwen3-tts/operations.cpp:31,41,143,147; kokoro/operations.cpp:143-146;
 * code-predictor.cpp:104; vits/waveform-decoder.cpp:157. */
static void op_binary(const orc_node * n, int ith, int nth) {
    int64_t r0, r1;
    chunk(n->nrows, ith, nth, &r0, &r1);
    const int64_t ne0 = n->ne0;
    for (int64_t r = r0; r < r1; ++r) {
        const float * a = (const float *) n->src0 + r * ne0;
        const float * b;
        int           scalar = 0;
        const int64_t brow   = n->src1_rows == 1 ? 0 : r;
        if (n->src1_ne0 == 1) {
            b      = (const float *) n->src1 + brow;
            scalar = 1;
        } else {
            b = (const float *) n->src1 + brow * ne0;
        }
        float * d = (float *) n->dst + r * ne0;
        for (int64_t i = 0; i < ne0; ++i) {
            const float bv = scalar ? b[0] : b[i];
            switch (n->op) {
                case ORC_OP_ADD:
                    d[i] = a[i] + bv;
                    break;
                case ORC_OP_MUL:
                    d[i] = a[i] * bv;
                    break;
                case ORC_OP_SUB:
                    d[i] = a[i] - bv;
                    break;
                default:
                    d[i] = a[i] / bv;
                    break;
            }
        }
    }
}

/* ggml_add / ggml_mul / ggml_div with src1 repeated to src0's shape
 * (ggml_can_repeat: each src1 extent divides src0's): ggml-CPU's binary ops
 * take src0's rows in thread chunks and read src1's row (i1 % ne11,
 * i2 % ne12, i3 % ne13); when ne10 < ne00 that row is applied ne00/ne10
 * times along the row. Sites: the per-channel [1, C] bias and gain vectors,
 * vits/waveform-decoder.cpp:120,139, qwen3-tts/codec.cpp:180,
 * omnivoice/codec.cpp:163, omnivoice/reference-encoder.cpp:135-136.
 * src0, src1 and dst contiguous; src1 points at int64_t[8]: src0's ne[0..3],
 * src1's ne[0..3], then the src1 data pointer as int64_t; i[0] = the op
 * (ORC_OP_ADD, ORC_OP_MUL or ORC_OP_DIV). */
static void op_binbcast(const orc_node * n, int ith, int nth) {
    const int64_t * v    = (const int64_t *) n->src1;
    const int64_t   ne00 = v[0], ne01 = v[1], ne02 = v[2], ne03 = v[3];
    const int64_t   ne10 = v[4], ne11 = v[5], ne12 = v[6], ne13 = v[7];
    const float *   b    = (const float *) (intptr_t) v[8];
    int64_t         r0, r1;
    chunk(ne01 * ne02 * ne03, ith, nth, &r0, &r1);
    for (int64_t r = r0; r < r1; ++r) {
        const int64_t i1 = r % ne01, i2 = (r / ne01) % ne02, i3 = r / (ne01 * ne02);
        const float * a  = (const float *) n->src0 + r * ne00;
        const float * br = b + ((i3 % ne13) * ne12 * ne11 + (i2 % ne12) * ne11 + (i1 % ne11)) * ne10;
        float *       d  = (float *) n->dst + r * ne00;
        for (int64_t k = 0; k < ne00 / ne10; ++k) {
            for (int64_t i = 0; i < ne10; ++i) {
                const float av = a[k * ne10 + i], bv = br[i];
                d[k * ne10 + i] = n->i[0] == ORC_OP_ADD ? av + bv :
                                  n->i[0] == ORC_OP_MUL ? av * bv :
                                  n->i[0] == ORC_OP_SUB ? av - bv :
                                                          av / bv;
            }
        }
    }
}

/* ggml_norm (LayerNorm without the affine part): per row, the mean from a
 * double sum, the centred values v = x - mean in f32, the variance from a
 * double sum of v*v, scale = 1/sqrtf(variance + eps), y = v*scale; rows
 * interleaved over threads. Sites: qwen3-tts/codec.cpp:216 (ConvNeXt),
 * kokoro/operations.cpp:12,93. */
static void op_norm(const orc_node * n, int ith, int nth) {
    const int64_t ne0 = n->ne0;
    const float   eps = n->f[0];
    for (int64_t r = ith; r < n->nrows; r += nth) {
        const float * x   = (const float *) n->src0 + r * ne0;
        float *       y   = (float *) n->dst + r * ne0;
        double        sum = 0.0;
        for (int64_t i = 0; i < ne0; ++i) {
            sum += (double) x[i];
        }
        const float mean = (float) (sum / (double) ne0);
        double      sum2 = 0.0;
        for (int64_t i = 0; i < ne0; ++i) {
            const float v = x[i] - mean;
            y[i]          = v;
            sum2 += (double) (v * v);
        }
        const float variance = (float) (sum2 / (double) ne0);
        const float scale    = 1.0f / sqrtf(variance + eps);
        for (int64_t i = 0; i < ne0; ++i) {
            y[i] *= scale;
        }
    }
}

/* ggml_rms_norm: rows interleaved over threads; f32 squares summed in double,
 * mean rounded to f32, scale = 1/sqrtf(mean + eps), y = x*scale.
 * Sites: qwen3-tts/operations.cpp:31 (via rms_norm :27-32), :86, :98-99, :145. */
static void op_rms_norm(const orc_node * n, int ith, int nth) {
    const int64_t ne0 = n->ne0;
    const float   eps = n->f[0];
    for (int64_t r = ith; r < n->nrows; r += nth) {
        const float * x   = (const float *) n->src0 + r * ne0;
        float *       y   = (float *) n->dst + r * ne0;
        double        sum = 0.0;
        for (int64_t i = 0; i < ne0; ++i) {
            sum += (double) (x[i] * x[i]);
        }
        const float mean = (float) (sum / (double) ne0);
        if (y != x) {
            memmove(y, x, (size_t) ne0 * sizeof(float));
        }
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t i = 0; i < ne0; ++i) {
            y[i] = y[i] * scale;
        }
    }
}

/* ggml_rope_ext, NEOX mode, ext_factor 0: per position a cos/sin cache built
 * from theta_0 = p, theta_{i+1} = theta_i * powf(base, -2/n_dims) (f32), each
 * entry cosf/sinf(freq_scale*theta) * attn_factor; pair (ic, ic + n_dims/2)
 * rotated; elements >= n_dims copied. Site: qwen3-tts/operations.cpp:101-104.
 * i[1] = 1 evaluates cos/sin in double and rounds once (correctly rounded
 * almost always) instead of libm cosf/sinf; everything else is unchanged. */
static void op_rope_neox(const orc_node * n, int ith, int nth) {
    const int64_t   ne0         = n->ne0;
    const int64_t   ne1         = n->ne1;
    const int       n_dims      = n->i[0];
    const int       cs_mode     = n->i[1];
    const float     freq_base   = n->f[0];
    const float     freq_scale  = n->f[1];
    const float     attn_factor = n->f[2];
    const float     theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    const int32_t * pos         = (const int32_t *) n->src1;
    const int64_t   half        = n_dims / 2;

    int64_t r0, r1;
    chunk(n->nrows, ith, nth, &r0, &r1);
    if (r0 >= r1) {
        return;
    }
    float * cache = (float *) malloc((size_t) (ne0 + 2) * sizeof(float));
    if (cache == NULL) {
        atomic_store(&g_node_error, -3);
        return;
    }
    const int64_t p_first = r0 / ne1;
    const int64_t p_last  = (r1 - 1) / ne1;
    for (int64_t pi = p_first; pi <= p_last; ++pi) {
        float theta = (float) pos[pi];
        for (int64_t i0 = 0; i0 < ne0; i0 += 2) {
            const float th = freq_scale * theta;
            if (cs_mode == 0) {
                cache[i0 + 0] = cosf(th) * attn_factor;
                cache[i0 + 1] = sinf(th) * attn_factor;
            } else {
                cache[i0 + 0] = (float) cos((double) th) * attn_factor;
                cache[i0 + 1] = (float) sin((double) th) * attn_factor;
            }
            theta = theta * theta_scale;
        }
        for (int64_t h = 0; h < ne1; ++h) {
            const int64_t r = pi * ne1 + h;
            if (r < r0 || r >= r1) {
                continue;
            }
            const float * src = (const float *) n->src0 + r * ne0;
            float *       dst = (float *) n->dst + r * ne0;
            for (int64_t i0 = 0; i0 < n_dims; i0 += 2) {
                const int64_t ic = i0 / 2;
                const float   c  = cache[i0 + 0];
                const float   s  = cache[i0 + 1];
                const float   x0 = src[ic];
                const float   x1 = src[ic + half];
                dst[ic]          = x0 * c - x1 * s;
                dst[ic + half]   = x0 * s + x1 * c;
            }
            for (int64_t i0 = n_dims; i0 < ne0; ++i0) {
                dst[i0] = src[i0];
            }
        }
    }
    free(cache);
}

static inline float silu_f32(float x) {
    return x / (1.0f + expf(-x));
}

/* Unary ops, rows chunked over threads. silu: qwen3-tts/operations.cpp:39,
 * talker.cpp:47; sin: kokoro/operations.cpp:144; sqr/exp: qwen3-tts/codec.cpp:
 * 192-195; leaky: vits/waveform-decoder.cpp:152,155,205,225; scale_bias:
 * qwen3-tts/codec.cpp:197, omnivoice/codec.cpp:66. */
static void op_unary(const orc_node * n, int ith, int nth) {
    int64_t r0, r1;
    chunk(n->nrows, ith, nth, &r0, &r1);
    const int64_t ne0 = n->ne0;
    for (int64_t r = r0; r < r1; ++r) {
        const float * x = (const float *) n->src0 + r * ne0;
        float *       y = (float *) n->dst + r * ne0;
        switch (n->op) {
            case ORC_OP_SILU:
                for (int64_t i = 0; i < ne0; ++i) {
                    y[i] = silu_f32(x[i]);
                }
                break;
            case ORC_OP_SIN:
                for (int64_t i = 0; i < ne0; ++i) {
                    y[i] = sinf(x[i]);
                }
                break;
            case ORC_OP_SQR:
                for (int64_t i = 0; i < ne0; ++i) {
                    y[i] = x[i] * x[i];
                }
                break;
            case ORC_OP_EXP:
                for (int64_t i = 0; i < ne0; ++i) {
                    y[i] = expf(x[i]);
                }
                break;
            /* ggml-CPU's vec forms: ggml_vec_tanh_f32, _sigmoid_f32, _elu_f32,
             * _gelu_erf_f32 and forward_clamp (MAX(MIN(x, max), min) with
             * ggml's macros, so a NaN gives max). Sites: vits/waveform-
             * decoder.cpp:228, kokoro/operations.cpp:133, qwen3-tts/codec.cpp:
             * 222,481. */
            case ORC_OP_TANH:
                for (int64_t i = 0; i < ne0; ++i) {
                    y[i] = tanhf(x[i]);
                }
                break;
            case ORC_OP_SIGMOID:
                for (int64_t i = 0; i < ne0; ++i) {
                    y[i] = 1.0f / (1.0f + expf(-x[i]));
                }
                break;
            case ORC_OP_ELU:
                for (int64_t i = 0; i < ne0; ++i) {
                    y[i] = (x[i] > 0.0f) ? x[i] : expm1f(x[i]);
                }
                break;
            case ORC_OP_GELU_ERF: {
                const float sqrt_2_inv = 0.70710678118654752440084436210484f;
                for (int64_t i = 0; i < ne0; ++i) {
                    const float v = x[i];
                    y[i]          = 0.5f * v * (1.0f + erff(v * sqrt_2_inv));
                }
                break;
            }
            /* ggml-CPU's vec forms ggml_vec_relu_f32, _neg_f32, _step_f32 and
             * _sqrt_f32 (vits/text-encoder.cpp:71, qwen3-tts/speaker-
             * encoder.cpp:184,294, vits/duration-predictor.cpp:89-117): a NaN
             * or -0 gives +0 from relu and 0 from step. */
            case ORC_OP_RELU:
                for (int64_t i = 0; i < ne0; ++i) {
                    y[i] = x[i] > 0.0f ? x[i] : 0.0f;
                }
                break;
            case ORC_OP_NEG:
                for (int64_t i = 0; i < ne0; ++i) {
                    y[i] = -x[i];
                }
                break;
            case ORC_OP_STEP:
                for (int64_t i = 0; i < ne0; ++i) {
                    y[i] = x[i] > 0.0f ? 1.0f : 0.0f;
                }
                break;
            case ORC_OP_SQRT:
                for (int64_t i = 0; i < ne0; ++i) {
                    y[i] = sqrtf(x[i]);
                }
                break;
            case ORC_OP_CLAMP: {
                const float lo = n->f[0], hi = n->f[1];
                for (int64_t i = 0; i < ne0; ++i) {
                    const float m = x[i] < hi ? x[i] : hi;
                    y[i]          = m > lo ? m : lo;
                }
                break;
            }
            case ORC_OP_LEAKY_RELU: {
                const float ns = n->f[0];
                for (int64_t i = 0; i < ne0; ++i) {
                    y[i] = ((x[i] > 0.0f) ? x[i] : 0.0f) + ns * ((x[i] < 0.0f) ? x[i] : 0.0f);
                }
                break;
            }
            case ORC_OP_SCALE_BIAS: {
                /* ggml-CPU's forward_scale: with b == 0 a plain multiply
                 * (ggml_vec_scale_f32, so -0 stays -0), else the vectorised
                 * x*s + b, one fused multiply-add on FMA hardware. */
                const float s = n->f[0];
                const float b = n->f[1];
                if (b == 0.0f) {
                    for (int64_t i = 0; i < ne0; ++i) {
                        y[i] = x[i] * s;
                    }
                } else {
                    for (int64_t i = 0; i < ne0; ++i) {
                        y[i] = fmaf(x[i], s, b);
                    }
                }
                break;
            }
            default:
                break;
        }
    }
}

/* ggml_get_rows: ids chunked over threads; each row converted to f32.
 * Sites: qwen3-tts/talker.cpp:44,86; code-predictor.cpp:31; model.cpp:1347,1449. */
static void op_get_rows(const orc_node * n, int ith, int nth) {
    int64_t r0, r1;
    chunk(n->nrows, ith, nth, &r0, &r1);
    const int64_t   ne0 = n->ne0;
    const size_t    rb  = row_bytes(n->type0, ne0);
    const int32_t * ids = (const int32_t *) n->src1;
    for (int64_t r = r0; r < r1; ++r) {
        const int32_t id = ids[r];
        float *       y  = (float *) n->dst + r * ne0;
        if (id < 0 || id >= n->src1_rows) {
            atomic_store(&g_node_error, -2); /* ggml-CPU asserts here */
            continue;
        }
        const uint8_t * row = (const uint8_t *) n->src0 + (size_t) id * rb;
        if (n->type0 == ORC_Q8_0) {
            dequantize_row_q8_0(row, y, ne0);
        } else if (n->type0 == ORC_Q5_K) {
            dequantize_row_q5_k(row, y, ne0);
        } else {
            for (int64_t i = 0; i < ne0; ++i) {
                y[i] = to_f32(n->type0, row, i);
            }
        }
    }
}

/* ggml_cast to F32 (as_f32, qwen3-tts/operations.cpp:20-25). */
static void op_cast(const orc_node * n, int ith, int nth) {
    int64_t r0, r1;
    chunk(n->nrows, ith, nth, &r0, &r1);
    const int64_t ne0 = n->ne0;
    const size_t  rb  = row_bytes(n->type0, ne0);
    for (int64_t r = r0; r < r1; ++r) {
        const uint8_t * row = (const uint8_t *) n->src0 + (size_t) r * rb;
        float *         y   = (float *) n->dst + r * ne0;
        for (int64_t i = 0; i < ne0; ++i) {
            y[i] = to_f32(n->type0, row, i);
        }
    }
}

/* ggml_cont of an F32 view with arbitrary byte strides into a contiguous F32
 * tensor of the same shape (ggml-CPU's dup into a contiguous destination: per
 * (i2, i3) plane each thread takes its share of the ne1 rows and walks each
 * row's ne0 elements through nb0). Sites: the vocoder's time-major copies,
 * vits/operations.cpp:72,87,100,108; the attention's permuted copies,
 * qwen3-tts/operations.cpp:120-125,136,139. src1 holds the view's
 * int64_t ne[4] then nb[4]. */
static void op_cont_f32(const orc_node * n, int ith, int nth) {
    const int64_t * v   = (const int64_t *) n->src1;
    const int64_t   ne0 = v[0], ne1 = v[1], ne2 = v[2], ne3 = v[3];
    const int64_t   nb0 = v[4], nb1 = v[5], nb2 = v[6], nb3 = v[7];
    int64_t         r0, r1;
    chunk(ne1, ith, nth, &r0, &r1);
    for (int64_t i3 = 0; i3 < ne3; ++i3) {
        for (int64_t i2 = 0; i2 < ne2; ++i2) {
            for (int64_t i1 = r0; i1 < r1; ++i1) {
                const uint8_t * row = (const uint8_t *) n->src0 + i1 * nb1 + i2 * nb2 + i3 * nb3;
                float *         y   = (float *) n->dst + ((i3 * ne2 + i2) * ne1 + i1) * ne0;
                for (int64_t i0 = 0; i0 < ne0; ++i0) {
                    memcpy(&y[i0], row + i0 * nb0, sizeof(float));
                }
            }
        }
    }
}

/* ggml_im2col(kernel, x, s0, 0, p0, 0, d0, 0, is_2D = false, dst_type), the
 * 1-D form every call site uses (vits/waveform-decoder.cpp:104,
 * vits/operations.cpp:40,103, kokoro/operations.cpp:76,
 * omnivoice/codec.cpp:114, omnivoice/reference-encoder.cpp:190,
 * qwen3-tts/codec.cpp:96,129, qwen3-tts/speaker-encoder.cpp:174,
 * qwen3-tts/codec-encoder.cpp:359). The kernel tensor gives only its extent K.
 * With x F32 [IW, IC, N] (rows contiguous) and OW = (IW + 2*p0 - d0*(K-1) -
 * 1)/s0 + 1 (ggml_calc_conv_output_size, C division), the dst [IC*K, OW, N]
 * holds dst[n][ow][ic*K + k] = x[n][ic][ow*s0 + k*d0 - p0], and 0 where that
 * index falls outside [0, IW): a pure gather, no arithmetic. An F16 dst holds
 * each value rounded to nearest even. ggml-CPU hands thread ith the channels
 * ith, ith + nth, ... of every (n, ow). */
static void op_im2col(const orc_node * n, int ith, int nth) {
    const int64_t * v  = (const int64_t *) n->src1;
    const int64_t   IW = v[0], IC = v[1], N = v[2], K = v[3], s0 = v[4], p0 = v[5], d0 = v[6];
    const int64_t   OW = (IW + 2 * p0 - d0 * (K - 1) - 1) / s0 + 1;
    const float *   x  = (const float *) n->src0;
    for (int64_t in = 0; in < N; ++in) {
        for (int64_t ow = 0; ow < OW; ++ow) {
            for (int64_t ic = ith; ic < IC; ic += nth) {
                const float * row = x + (in * IC + ic) * IW;
                const int64_t o   = ((in * OW + ow) * IC + ic) * K;
                for (int64_t k = 0; k < K; ++k) {
                    const int64_t iw  = ow * s0 + k * d0 - p0;
                    const float   val = (iw < 0 || iw >= IW) ? 0.0f : row[iw];
                    if (n->type0 == ORC_F16) {
                        ((uint16_t *) n->dst)[o + k] = orc_fp32_to_fp16(val);
                    } else {
                        ((float *) n->dst)[o + k] = val;
                    }
                }
            }
        }
    }
}

/* ggml_col2im_1d(columns, stride, OC, padding): the scatter-back of a
 * transposed convolution computed as a matrix product (columns[l] = the
 * kernel's K*OC taps times input column l, out-channel-major, tap-minor), at
 * vits/operations.cpp:118-140, omnivoice/codec.cpp:150-159 and
 * qwen3-tts/codec.cpp:163-171. Output [T, OC], T = (L-1)*stride + K -
 * 2*padding:
 *   dst[oc][t] = sum of columns[l][oc*K + k] over l*stride + k = t + padding,
 * 0 <= l < L, 0 <= k < K: each column l adds its taps at t = l*stride + k -
 * padding. The op belongs to the reference's pinned ggml, which is absent;
 * the sum is accumulated into +0.0f in ascending l (a zero-initialised
 * scatter in column order). For K <= 2*stride -- every upsampling layer of the
 * vocoders and codecs -- an output takes at most two terms, and the f32 sum of
 * two terms from +0 is the same in either order. Threads take channels. */
static void op_col2im_1d(const orc_node * n, int ith, int nth) {
    const int64_t * v  = (const int64_t *) n->src1;
    const int64_t   K = v[0], OC = v[1], L = v[2], S = v[3], P = v[4];
    const int64_t   T  = (L - 1) * S + K - 2 * P;
    const float *   c  = (const float *) n->src0;
    for (int64_t oc = ith; oc < OC; oc += nth) {
        float * y = (float *) n->dst + oc * T;
        for (int64_t t = 0; t < T; ++t) {
            y[t] = 0.0f;
        }
        for (int64_t l = 0; l < L; ++l) {
            for (int64_t k = 0; k < K; ++k) {
                const int64_t t = l * S + k - P;
                if (t >= 0 && t < T) {
                    y[t] += c[l * K * OC + oc * K + k];
                }
            }
        }
    }
}

/* The padding and tiling copies (no arithmetic): each destination element is
 * one source element or zero. src1 holds the source and destination extents
 * and the op's offsets (ggml_cpu_ref.h). Threads take destination rows.
 *   PAD (ggml_pad / ggml_pad_ext; kokoro/operations.cpp:192,196,
 *        vits/text-encoder.cpp:36, omnivoice/reference-encoder.cpp:482,
 *        qwen3-tts/codec-encoder.cpp:351): dst[i] = src[i - lp] where every
 *        i_d - lp_d lies in [0, src.ne_d), else 0 (the right pads are what
 *        the destination's extents leave).
 *   PAD_REFLECT_1D (qwen3-tts/speaker-encoder.cpp:164): along dim 0, i < p0
 *        reads src[p0 - i], the middle src[i - p0], the right end
 *        src[2*(ne0 - 1) + p0 - i]: reflection about the edge samples, which
 *        are not repeated.
 *   REPEAT (ggml_repeat / ggml_repeat_4d; kokoro/operations.cpp:23,118,
 *        qwen3-tts/speaker-encoder.cpp:356-357, codec-encoder.cpp:183,188):
 *        dst[i] = src[i_d mod src.ne_d]. */
static void op_pad_family(const orc_node * n, int ith, int nth) {
    const int64_t * v = (const int64_t *) n->src1;
    const int64_t * sne = v, *dne = v + 4, *off = v + 8;
    const float *   src = (const float *) n->src0;
    float *         dst = (float *) n->dst;
    const int64_t   rows = dne[1] * dne[2] * dne[3];
    for (int64_t r = ith; r < rows; r += nth) {
        const int64_t i1 = r % dne[1], i2 = (r / dne[1]) % dne[2], i3 = r / (dne[1] * dne[2]);
        const int64_t i[4] = { 0, i1, i2, i3 };
        int64_t       s[4];
        int           in = 1;
        for (int d = 1; d < 4; ++d) {
            if (n->op == ORC_OP_REPEAT) {
                s[d] = i[d] % sne[d];
            } else if (n->op == ORC_OP_PAD) {
                s[d] = i[d] - off[d];
                in &= s[d] >= 0 && s[d] < sne[d];
            } else {
                s[d] = i[d];
            }
        }
        float *       y  = dst + r * dne[0];
        const float * xr = in ? src + ((s[3] * sne[2] + s[2]) * sne[1] + s[1]) * sne[0] : NULL;
        for (int64_t i0 = 0; i0 < dne[0]; ++i0) {
            float val = 0.0f;
            if (xr != NULL) {
                if (n->op == ORC_OP_REPEAT) {
                    val = xr[i0 % sne[0]];
                } else if (n->op == ORC_OP_PAD) {
                    const int64_t j = i0 - off[0];
                    val             = (j >= 0 && j < sne[0]) ? xr[j] : 0.0f;
                } else {
                    const int64_t p0 = off[0];
                    const int64_t j  = i0 < p0 ? p0 - i0 : (i0 < p0 + sne[0] ? i0 - p0 : 2 * (sne[0] - 1) + p0 - i0);
                    val              = xr[j];
                }
            }
            y[i0] = val;
        }
    }
}

/* The Qwen3-TTS speaker encoder's log-mel front end (qwen3-tts/mel.cpp:
 * 63-94, 131-299), restated: librosa's Slaney mel scale (linear below
 * 1 kHz, log above) and area-normalised triangular filters in double, rounded
 * to f32; the PCM reflect-padded by (n_fft - hop)/2 on each side and framed
 * without centring; the periodic Hann window of win_length (f32), centred in
 * n_fft; per frame an in-place iterative radix-2 FFT on f32 buffers (the
 * bit-reversal swap, then butterflies with double twiddles cos/sin((-2 pi /
 * len) * k), each result rounded to f32); the amplitude sqrt(re^2 + im^2 +
 * 1e-9) in double rounded to f32; each mel energy summed in double in bin
 * order; log(max(energy, 1e-5)) rounded to f32. */
static double mel_slaney_step(void) {
    return log(6.4) / 27.0;
}

static double mel_hz_to_mel(double hz) {
    const double min_log_mel = 1000.0 / (200.0 / 3.0);
    if (hz >= 1000.0) {
        return min_log_mel + log(hz / 1000.0) / mel_slaney_step();
    }
    return hz / (200.0 / 3.0);
}

static double mel_mel_to_hz(double mel) {
    const double min_log_mel = 1000.0 / (200.0 / 3.0);
    if (mel >= min_log_mel) {
        return 1000.0 * exp(mel_slaney_step() * (mel - min_log_mel));
    }
    return (200.0 / 3.0) * mel;
}

void orc_mel_filterbank(uint32_t sample_rate, uint32_t n_fft, uint32_t mel_bins, float fmin, float fmax, float * out) {
    const uint32_t nf = n_fft / 2 + 1;
    double *       mf = (double *) malloc(sizeof(double) * (mel_bins + 2));
    if (mf == NULL) {
        return;
    }
    const double lo = mel_hz_to_mel((double) fmin), hi = mel_hz_to_mel((double) fmax);
    for (uint32_t i = 0; i < mel_bins + 2; ++i) {
        mf[i] = mel_mel_to_hz(lo + (hi - lo) * (double) i / (double) (mel_bins + 1));
    }
    for (uint32_t b = 0; b < mel_bins; ++b) {
        const double enorm = 2.0 / (mf[b + 2] - mf[b]);
        for (uint32_t k = 0; k < nf; ++k) {
            const double f     = (double) k * (double) sample_rate / (double) n_fft;
            const double lower = (f - mf[b]) / (mf[b + 1] - mf[b]);
            const double upper = (mf[b + 2] - f) / (mf[b + 2] - mf[b + 1]);
            const double v     = lower < upper ? lower : upper;
            out[(size_t) b * nf + k] = (float) ((v > 0.0 ? v : 0.0) * enorm);
        }
    }
    free(mf);
}

static void fft_radix2_f32(float * re, float * im, size_t n) {
    const double pi = 3.14159265358979323846;
    for (size_t i = 1, j = 0; i < n; ++i) {
        size_t bit = n >> 1;
        for (; j & bit; bit >>= 1) {
            j ^= bit;
        }
        j ^= bit;
        if (i < j) {
            float t = re[i];
            re[i]   = re[j];
            re[j]   = t;
            t       = im[i];
            im[i]   = im[j];
            im[j]   = t;
        }
    }
    for (size_t len = 2; len <= n; len <<= 1) {
        const double angle = -2.0 * pi / (double) len;
        for (size_t start = 0; start < n; start += len) {
            for (size_t k = 0; k < len / 2; ++k) {
                const double theta = angle * (double) k;
                const double wr = cos(theta), wi = sin(theta);
                const size_t a = start + k, b = a + len / 2;
                const double xr = re[b] * wr - im[b] * wi;
                const double xi = re[b] * wi + im[b] * wr;
                re[b]           = (float) (re[a] - xr);
                im[b]           = (float) (im[a] - xi);
                re[a]           = (float) (re[a] + xr);
                im[a]           = (float) (im[a] + xi);
            }
        }
    }
}

static void op_log_mel(const orc_node * n, int ith, int nth) {
    (void) nth;
    if (ith != 0) {
        return;
    }
    const double   pi   = 3.14159265358979323846;
    const float *  pcm  = (const float *) n->src0;
    const float *  fb   = (const float *) n->src1;
    const int64_t  ns   = n->ne0;
    const int64_t  nfft = n->i[0], hop = n->i[1], win = n->i[2], bins = n->i[3];
    const int64_t  pad  = (nfft - hop) / 2;
    const int64_t  plen = ns + 2 * pad;
    if (nfft < 2 || (nfft & (nfft - 1)) != 0 || hop < 1 || win < 1 || win > nfft || hop > nfft || ns <= pad ||
        plen < nfft) {
        atomic_store(&g_node_error, -2);
        return;
    }
    const int64_t frames = 1 + (plen - nfft) / hop;
    const int64_t nf     = nfft / 2 + 1;
    float *       padded = (float *) malloc(sizeof(float) * (size_t) plen);
    float *       w      = (float *) calloc((size_t) nfft, sizeof(float));
    float *       re     = (float *) malloc(sizeof(float) * (size_t) nfft);
    float *       im     = (float *) malloc(sizeof(float) * (size_t) nfft);
    float *       mag    = (float *) malloc(sizeof(float) * (size_t) nf);
    if (!padded || !w || !re || !im || !mag) {
        atomic_store(&g_node_error, -3);
        goto done;
    }
    for (int64_t i = 0; i < ns; ++i) {
        padded[pad + i] = pcm[i];
    }
    for (int64_t j = 0; j < pad; ++j) {
        padded[j]            = pcm[pad - j];
        padded[pad + ns + j] = pcm[ns - 2 - j];
    }
    for (int64_t i = 0; i < win; ++i) {
        w[(nfft - win) / 2 + i] = (float) (0.5 - 0.5 * cos(2.0 * pi * (double) i / (double) win));
    }
    for (int64_t f = 0; f < frames; ++f) {
        for (int64_t i = 0; i < nfft; ++i) {
            re[i] = padded[f * hop + i] * w[i];
            im[i] = 0.0f;
        }
        fft_radix2_f32(re, im, (size_t) nfft);
        for (int64_t k = 0; k < nf; ++k) {
            const double sq = (double) re[k] * (double) re[k] + (double) im[k] * (double) im[k];
            mag[k]          = (float) sqrt(sq + 1e-9);
        }
        float * y = (float *) n->dst + f * bins;
        for (int64_t b = 0; b < bins; ++b) {
            double e = 0.0;
            for (int64_t k = 0; k < nf; ++k) {
                e += (double) fb[b * nf + k] * (double) mag[k];
            }
            y[b] = (float) log(e < 1e-5 ? 1e-5 : e);  /* std::max(e, 1e-5): a NaN passes */
        }
    }
done:
    free(padded);
    free(w);
    free(re);
    free(im);
    free(mag);
}

/* Kokoro's harmonic-plus-noise source and its short-time spectrum
 * (kokoro/source.cpp:60-184, build_harmonic_source), restated step by step:
 * f0 repeated `scale` times; per sample and harmonic h the phase increment
 * frac(f0 * (h+1) / rate) in f32, the random initial phase added on sample 0;
 * the increments resampled linearly to the f0 grid (PyTorch's
 * align_corners=false: position (o + 0.5) * in/out - 0.5 in double, clamped
 * at 0, the weight rounded to f32, a*(1-w) + b*w); a running f32 sum per
 * harmonic in frame order, scaled by 2*pi*scale in double and rounded; that
 * phase resampled back to the sample grid; per sample the voiced flag (f0 >
 * threshold), sin(phase) * amp * uv + gain * noise merged with the weights in
 * harmonic order from the bias, tanh; then torch.stft's centred framing:
 * reflect padding by n_fft/2, the periodic Hann window rounded to f32, the
 * DFT in double, magnitude by hypot and phase by atan2, each rounded to f32. */
static void resample_linear_f32(const float * in, int64_t in_len, int64_t out_len, int64_t ch, float * out) {
    const double ratio = (double) in_len / (double) out_len;
    for (int64_t o = 0; o < out_len; ++o) {
        double position = ((double) o + 0.5) * ratio - 0.5;
        if (position < 0.0) {
            position = 0.0;
        }
        const int64_t low  = (int64_t) position;
        const int64_t high = low + 1 < in_len ? low + 1 : in_len - 1;
        const float   w    = (float) (position - (double) low);
        for (int64_t c = 0; c < ch; ++c) {
            const float a  = in[low * ch + c];
            const float b  = in[high * ch + c];
            out[o * ch + c] = a * (1.0f - w) + b * w;
        }
    }
}

static void op_harmonic_source(const orc_node * n, int ith, int nth) {
    (void) nth;
    if (ith != 0) {
        return;
    }
    const orc_source_args * a  = (const orc_source_args *) n->src1;
    const double            pi = 3.14159265358979323846;
    const int64_t           L  = n->nrows;
    const int64_t           H  = a->harmonics, S = a->scale, N = a->n_fft, hop = a->hop;
    if (L < 1 || H < 1 || S < 1 || N < 2 || hop < 1 || a->sampling_rate < 1) {
        atomic_store(&g_node_error, -2);
        return;
    }
    const int64_t U    = L * S;
    const float * f0   = (const float *) n->src0;
    float *       f0u  = (float *) malloc((size_t) U * sizeof(float));
    float *       rad  = (float *) malloc((size_t) (U * H) * sizeof(float));
    float *       crs  = (float *) malloc((size_t) (L * H) * sizeof(float));
    float *       ph   = (float *) malloc((size_t) (L * H) * sizeof(float));
    float *       fine = (float *) malloc((size_t) (U * H) * sizeof(float));
    float *       run  = (float *) calloc((size_t) H, sizeof(float));
    const int64_t half = N / 2, bins = half + 1, frames = U / hop + 1;
    float *       pad  = (float *) malloc((size_t) (U + 2 * half) * sizeof(float));
    float *       win  = (float *) malloc((size_t) N * sizeof(float));
    float *       seg  = (float *) malloc((size_t) N * sizeof(float));
    if (!f0u || !rad || !crs || !ph || !fine || !run || !pad || !win || !seg) {
        atomic_store(&g_node_error, -3);
        goto done;
    }
    for (int64_t i = 0; i < L; ++i) {
        for (int64_t k = 0; k < S; ++k) {
            f0u[i * S + k] = f0[i];
        }
    }
    {
        const float rate = (float) a->sampling_rate;
        for (int64_t u = 0; u < U; ++u) {
            for (int64_t h = 0; h < H; ++h) {
                const float v  = f0u[u] * (float) (h + 1) / rate;
                rad[u * H + h] = v - floorf(v);
            }
        }
    }
    for (int64_t h = 0; h < H; ++h) {
        rad[h] += a->rand_ini[h];
    }
    resample_linear_f32(rad, U, L, H, crs);
    for (int64_t j = 0; j < L; ++j) {
        for (int64_t h = 0; h < H; ++h) {
            run[h] += crs[j * H + h];
            ph[j * H + h] = (float) ((double) run[h] * 2.0 * pi * (double) S);
        }
    }
    resample_linear_f32(ph, L, U, H, fine);
    {
        float * exc = (float *) n->dst;
        for (int64_t u = 0; u < U; ++u) {
            const int   voiced = f0u[u] > a->voiced_threshold;
            const float uv     = voiced ? 1.0f : 0.0f;
            const float gain   = uv * a->noise_std + (1.0f - uv) * a->sine_amp / 3.0f;
            float       merged = a->merge_bias;
            for (int64_t h = 0; h < H; ++h) {
                const float sine  = sinf(fine[u * H + h]) * a->sine_amp;
                const float value = sine * uv + gain * a->noise[u * H + h];
                merged += a->merge_weight[h] * value;
            }
            exc[u] = tanhf(merged);
        }
        for (int64_t i = 0; i < U + 2 * half; ++i) {
            int64_t       src  = i - half;
            const int64_t last = U - 1;
            while (src < 0 || src > last) {
                src = src < 0 ? -src : 2 * last - src;
            }
            pad[i] = exc[src];
        }
    }
    for (int64_t k = 0; k < N; ++k) {
        win[k] = (float) (0.5 * (1.0 - cos(2.0 * pi * (double) k / (double) N)));
    }
    for (int64_t f = 0; f < frames; ++f) {
        for (int64_t k = 0; k < N; ++k) {
            seg[k] = pad[f * hop + k] * win[k];
        }
        for (int64_t b = 0; b < bins; ++b) {
            double re = 0.0, im = 0.0;
            for (int64_t k = 0; k < N; ++k) {
                const double angle = -2.0 * pi * (double) b * (double) k / (double) N;
                re += (double) seg[k] * cos(angle);
                im += (double) seg[k] * sin(angle);
            }
            a->har[f * 2 * bins + b]        = (float) hypot(re, im);
            a->har[f * 2 * bins + bins + b] = (float) atan2(im, re);
        }
    }
done:
    free(f0u);
    free(rad);
    free(crs);
    free(ph);
    free(fine);
    free(run);
    free(pad);
    free(win);
    free(seg);
}

/* Kokoro's inverse short-time transform (kokoro/decoder-host.cpp:28-100,
 * called at kokoro/model.cpp:1056 on the generator's output), restated as the
 * host code computes it, in double: a periodic Hann window rounded to f32;
 * per frame, the bins' complex values exp(log-magnitude) * e^(i sin(raw
 * phase)), and each of the frame's n_fft samples as the real inverse DFT (bin
 * 0 and the Nyquist bin once, the others twice, over n_fft), in bin order;
 * overlap-add of sample * window and of window^2 in frame order; output
 * sample t = the sums at t + n_fft/2, their quotient rounded to f32, or 0
 * where the window sum is below 1e-11. Serial, as the host code is. */
static void op_istft(const orc_node * n, int ith, int nth) {
    (void) nth;
    if (ith != 0) {
        return;
    }
    const double   pi     = 3.14159265358979323846;
    const int64_t  frames = n->nrows;
    const int64_t  nfft   = n->i[0];
    const int64_t  hop    = n->i[1];
    const int64_t  bins   = nfft / 2 + 1;
    if (frames < 2 || nfft < 2 || nfft % 2 != 0 || hop <= 0 || n->ne0 != nfft + 2) {
        atomic_store(&g_node_error, -2);
        return;
    }
    const int64_t total = nfft + hop * (frames - 1);
    const int64_t kept  = (frames - 1) * hop;
    float *       win   = (float *) malloc((size_t) nfft * sizeof(float));
    double *      acc   = (double *) calloc((size_t) total, sizeof(double));
    double *      env   = (double *) calloc((size_t) total, sizeof(double));
    double *      frame = (double *) malloc((size_t) nfft * sizeof(double));
    if (win == NULL || acc == NULL || env == NULL || frame == NULL) {
        atomic_store(&g_node_error, -3);
        free(win);
        free(acc);
        free(env);
        free(frame);
        return;
    }
    for (int64_t k = 0; k < nfft; ++k) {
        win[k] = (float) (0.5 * (1.0 - cos(2.0 * pi * (double) k / (double) nfft)));
    }
    for (int64_t f = 0; f < frames; ++f) {
        const float * row = (const float *) n->src0 + f * n->ne0;
        for (int64_t s = 0; s < nfft; ++s) {
            double value = 0.0;
            for (int64_t b = 0; b < bins; ++b) {
                const double mag    = exp((double) row[b]);
                const double angle  = sin((double) row[bins + b]);
                const double turn   = 2.0 * pi * (double) b * (double) s / (double) nfft;
                const double re     = mag * cos(angle);
                const double im     = mag * sin(angle);
                const double weight = (b == 0 || b == bins - 1) ? 1.0 : 2.0;
                value += weight * (re * cos(turn) - im * sin(turn));
            }
            frame[s] = value / (double) nfft;
        }
        for (int64_t s = 0; s < nfft; ++s) {
            acc[f * hop + s] += frame[s] * (double) win[s];
            env[f * hop + s] += (double) win[s] * (double) win[s];
        }
    }
    float * y = (float *) n->dst;
    for (int64_t t = 0; t < kept; ++t) {
        const double d = env[t + nfft / 2];
        y[t]           = fabs(d) < (double) 1e-11f ? 0.0f : (float) (acc[t + nfft / 2] / d);
    }
    free(win);
    free(acc);
    free(env);
    free(frame);
}

/* ggml_diag_mask_inf(x, n_past) (qwen3-tts/codec-encoder.cpp:482): x copied,
 * then in row j of every matrix each element i >= n_past with i > n_past + j
 * set to -inf, as ggml-CPU's forward_diag_mask writes them. */
static void op_diag_mask_inf(const orc_node * n, int ith, int nth) {
    int64_t r0, r1;
    chunk(n->nrows, ith, nth, &r0, &r1);
    const int64_t n_past = n->i[0];
    for (int64_t r = r0; r < r1; ++r) {
        const int64_t j = r % n->ne1;
        const float * x = (const float *) n->src0 + r * n->ne0;
        float *       y = (float *) n->dst + r * n->ne0;
        memcpy(y, x, (size_t) n->ne0 * sizeof(float));
        for (int64_t i = n_past; i < n->ne0; ++i) {
            if (i > n_past + j) {
                y[i] = -INFINITY;
            }
        }
    }
}

/* ggml_sum_rows and ggml_mean (qwen3-tts/speaker-encoder.cpp:195,292-293,
 * 350,374, the speaker encoder's statistics pooling; vits/duration-
 * predictor.cpp:47,93): ggml_vec_sum_f32 accumulates a row's f32 values into
 * a double in element order and rounds the sum to f32 once; the mean then
 * divides that f32 by ne0 converted to f32. */
static void op_sum_rows(const orc_node * n, int ith, int nth) {
    int64_t r0, r1;
    chunk(n->nrows, ith, nth, &r0, &r1);
    for (int64_t r = r0; r < r1; ++r) {
        const float * x   = (const float *) n->src0 + r * n->ne0;
        double        sum = 0.0;
        for (int64_t i = 0; i < n->ne0; ++i) {
            sum += (double) x[i];
        }
        float v = (float) sum;
        if (n->op == ORC_OP_MEAN) {
            v /= (float) n->ne0;
        }
        ((float *) n->dst)[r] = v;
    }
}

/* ggml_acc(a, b, nb1, nb2, nb3, offset) (qwen3-tts/talker.cpp:31,90,109,112,
 * 115: the talker's prefill input, the codec stream, the x-vector's slot and
 * the ICL acoustic block added into the text stream at a row offset): dst is a
 * copy of a, then every row (i1, i2, i3) of b is added to dst at byte
 * i1*nb1 + i2*nb2 + i3*nb3 + offset, reading a at the same byte: dst[v] =
 * a[v] + b[row][i0], one f32 add per element. ggml-CPU copies on thread 0,
 * waits, then splits b's rows over the threads; a window whose rows do not
 * overlap (every use in the reference) gives the same values in any split, so
 * thread 0 does it all here. A window past a's end is refused (ggml asserts). */
static void op_acc(const orc_node * n, int ith, int nth) {
    (void) nth;
    if (ith != 0) {
        return;
    }
    const int64_t * v   = (const int64_t *) n->src1;
    const int64_t * bne = v;
    const int64_t   nb1 = v[4], nb2 = v[5], nb3 = v[6], off = v[7];
    const float *   b   = (const float *) (intptr_t) v[8];
    const int64_t   nbytes = n->ne0 * n->nrows * (int64_t) sizeof(float);
    if (bne[0] * bne[1] * bne[2] * bne[3] > 0 &&
        off + (bne[0] - 1) * 4 + (bne[1] - 1) * nb1 + (bne[2] - 1) * nb2 + (bne[3] - 1) * nb3 >= nbytes) {
        atomic_store(&g_node_error, -2);
        return;
    }
    memcpy(n->dst, n->src0, (size_t) nbytes);
    for (int64_t i3 = 0; i3 < bne[3]; ++i3) {
        for (int64_t i2 = 0; i2 < bne[2]; ++i2) {
            for (int64_t i1 = 0; i1 < bne[1]; ++i1) {
                const int64_t at = i3 * nb3 + i2 * nb2 + i1 * nb1 + off;
                float *       d  = (float *) ((char *) n->dst + at);
                const float * s  = (const float *) ((const char *) n->src0 + at);
                const float * br = b + ((i3 * bne[2] + i2) * bne[1] + i1) * bne[0];
                for (int64_t i0 = 0; i0 < bne[0]; ++i0) {
                    d[i0] = s[i0] + br[i0];
                }
            }
        }
    }
}

/* ggml_swiglu (single tensor): gate = first half of each row (second when
 * swapped), y = silu(gate) * other half. */
static void op_glu_swiglu(const orc_node * n, int ith, int nth) {
    int64_t r0, r1;
    chunk(n->nrows, ith, nth, &r0, &r1);
    const int64_t nc      = n->ne0;
    const int     swapped = n->i[0];
    for (int64_t r = r0; r < r1; ++r) {
        const float * row  = (const float *) n->src0 + r * 2 * nc;
        const float * gate = row + (swapped ? nc : 0);
        const float * up   = row + (swapped ? 0 : nc);
        float *       y    = (float *) n->dst + r * nc;
        for (int64_t i = 0; i < nc; ++i) {
            y[i] = silu_f32(gate[i]) * up[i];
        }
    }
}

/* ggml_soft_max_ext(x, mask, scale, max_bias = 0), ggml-CPU's per-row order:
 * w = x*scale, then w += 1*mask (slope 1 without ALiBi); max over the row by
 * the sequential (max > w ? max : w); v = expf(w - max) with each v added to a
 * double sum; y = v * (float)(1.0/sum). Rows interleaved over threads.
 * Site: qwen3-tts/operations.cpp:131-133 (scale 1/sqrt(head_dim), causal mask
 * of tests/qwen3_tts_decoder_layer_test.cpp:174-181). */
static void op_soft_max(const orc_node * n, int ith, int nth) {
    const int64_t ne0    = n->ne0;
    const int64_t ne1    = n->ne1;
    const int64_t mrows  = n->src1_rows;
    const int64_t mheads = n->i[0] > 0 ? n->i[0] : 1;
    const float   scale  = n->f[0];
    float *       w      = (float *) malloc((size_t) ne0 * sizeof(float));
    if (w == NULL) {
        atomic_store(&g_node_error, -2);
        return;
    }
    for (int64_t r = ith; r < n->nrows; r += nth) {
        const float * x = (const float *) n->src0 + r * ne0;
        float *       y = (float *) n->dst + r * ne0;
        for (int64_t i = 0; i < ne0; ++i) {
            w[i] = x[i] * scale;
        }
        if (n->src1 != NULL) {
            const int64_t i1 = r % ne1;
            const int64_t h  = r / ne1;
            const float * m  = (const float *) n->src1 + ((h % mheads) * mrows + i1) * ne0;
            for (int64_t i = 0; i < ne0; ++i) {
                w[i] += 1.0f * m[i];
            }
        }
        float mx = -INFINITY;
        for (int64_t i = 0; i < ne0; ++i) {
            mx = mx > w[i] ? mx : w[i];
        }
        double sum = 0.0;
        for (int64_t i = 0; i < ne0; ++i) {
            const float v = expf(w[i] - mx);
            sum += (double) v;
            y[i] = v;
        }
        const float inv = (float) (1.0 / sum);
        for (int64_t i = 0; i < ne0; ++i) {
            y[i] *= inv;
        }
    }
    free(w);
}

static void run_node(const orc_node * n, int ith, int nth) {
    switch (n->op) {
        case ORC_OP_ADD:
        case ORC_OP_MUL:
        case ORC_OP_DIV:
        case ORC_OP_SUB:
            op_binary(n, ith, nth);
            break;
        case ORC_OP_TANH:
        case ORC_OP_SIGMOID:
        case ORC_OP_ELU:
        case ORC_OP_GELU_ERF:
        case ORC_OP_CLAMP:
            op_unary(n, ith, nth);
            break;
        case ORC_OP_NORM:
            op_norm(n, ith, nth);
            break;
        case ORC_OP_RMS_NORM:
            op_rms_norm(n, ith, nth);
            break;
        case ORC_OP_ROPE_NEOX:
            op_rope_neox(n, ith, nth);
            break;
        case ORC_OP_SILU:
        case ORC_OP_SIN:
        case ORC_OP_SQR:
        case ORC_OP_EXP:
        case ORC_OP_LEAKY_RELU:
        case ORC_OP_SCALE_BIAS:
            op_unary(n, ith, nth);
            break;
        case ORC_OP_GET_ROWS:
            op_get_rows(n, ith, nth);
            break;
        case ORC_OP_CAST_F32:
            op_cast(n, ith, nth);
            break;
        case ORC_OP_GLU_SWIGLU:
            op_glu_swiglu(n, ith, nth);
            break;
        case ORC_OP_SOFT_MAX:
            op_soft_max(n, ith, nth);
            break;
        case ORC_OP_CONT_F32:
            op_cont_f32(n, ith, nth);
            break;
        case ORC_OP_BINBCAST:
            op_binbcast(n, ith, nth);
            break;
        case ORC_OP_IM2COL:
            op_im2col(n, ith, nth);
            break;
        case ORC_OP_COL2IM_1D:
            op_col2im_1d(n, ith, nth);
            break;
        case ORC_OP_PAD:
        case ORC_OP_PAD_REFLECT_1D:
        case ORC_OP_REPEAT:
            op_pad_family(n, ith, nth);
            break;
        case ORC_OP_ACC:
            op_acc(n, ith, nth);
            break;
        case ORC_OP_RELU:
        case ORC_OP_NEG:
        case ORC_OP_STEP:
        case ORC_OP_SQRT:
            op_unary(n, ith, nth);
            break;
        case ORC_OP_SUM_ROWS:
        case ORC_OP_MEAN:
            op_sum_rows(n, ith, nth);
            break;
        case ORC_OP_DIAG_MASK_INF:
            op_diag_mask_inf(n, ith, nth);
            break;
        case ORC_OP_ISTFT:
            op_istft(n, ith, nth);
            break;
        case ORC_OP_HARMONIC_SOURCE:
            op_harmonic_source(n, ith, nth);
            break;
        case ORC_OP_LOG_MEL:
            op_log_mel(n, ith, nth);
            break;
        default:
            atomic_store(&g_node_error, -1);
            break;
    }
}

/* ------------------------------------------------------------------ */
/* persistent thread pool with a spin barrier between nodes (as ggml)  */
/* ------------------------------------------------------------------ */

#define ORC_MAX_THREADS 512

static inline void cpu_relax(void) {
#if defined(__x86_64__) || defined(__i386__)
    __builtin_ia32_pause();
#else
    sched_yield();
#endif
}

static struct {
    int              n;
    pthread_t        th[ORC_MAX_THREADS];
    atomic_int       gen;
    atomic_int       stop;
    atomic_int       bar_count;
    atomic_int       bar_sense;
    const orc_node * nodes;
    int              n_nodes;
} g_pool;

static pthread_mutex_t g_pool_lock = PTHREAD_MUTEX_INITIALIZER;
static _Thread_local int t_sense   = 0;

static void barrier(int nth) {
    const int s = !t_sense;
    t_sense     = s;
    if (atomic_fetch_add(&g_pool.bar_count, 1) == nth - 1) {
        atomic_store(&g_pool.bar_count, 0);
        atomic_store(&g_pool.bar_sense, s);
    } else {
        while (atomic_load(&g_pool.bar_sense) != s) {
            cpu_relax();
        }
    }
}

static void run_job(int ith, int nth) {
    const orc_node * nodes   = g_pool.nodes;
    const int        n_nodes = g_pool.n_nodes;
    for (int k = 0; k < n_nodes; ++k) {
        run_node(&nodes[k], ith, nth);
        barrier(nth);
    }
}

static void * worker_main(void * arg) {
    const int ith  = (int) (intptr_t) arg;
    int       seen = 0;
    t_sense        = atomic_load(&g_pool.bar_sense);
    for (;;) {
        long spins = 0;
        int  g;
        while ((g = atomic_load(&g_pool.gen)) == seen) {
            if (++spins < (1L << 18)) {
                cpu_relax();
            } else {
                struct timespec ts = { 0, 50000 };
                nanosleep(&ts, NULL);
            }
        }
        seen = g;
        if (atomic_load(&g_pool.stop)) {
            break;
        }
        run_job(ith, g_pool.n);
    }
    return NULL;
}

static void pool_shutdown(void) {
    if (g_pool.n > 1) {
        atomic_store(&g_pool.stop, 1);
        atomic_fetch_add(&g_pool.gen, 1);
        for (int i = 1; i < g_pool.n; ++i) {
            pthread_join(g_pool.th[i], NULL);
        }
    }
    g_pool.n = 0;
    atomic_store(&g_pool.stop, 0);
}

static int pool_ensure(int n) {
    if (g_pool.n == n) {
        return 0;
    }
    pool_shutdown();
    atomic_store(&g_pool.bar_count, 0);
    t_sense = atomic_load(&g_pool.bar_sense);
    atomic_store(&g_pool.gen, 0);
    g_pool.n = n;
    for (int i = 1; i < n; ++i) {
        if (pthread_create(&g_pool.th[i], NULL, worker_main, (void *) (intptr_t) i) != 0) {
            g_pool.n = i;
            pool_shutdown();
            return -4;
        }
    }
    return 0;
}

static int compute_locked(const orc_node * nodes, int32_t n_nodes, int32_t n_threads) {
    atomic_store(&g_node_error, 0);
    if (n_threads <= 1) {
        for (int k = 0; k < n_nodes; ++k) {
            run_node(&nodes[k], 0, 1);
        }
        return atomic_load(&g_node_error);
    }
    const int rc = pool_ensure(n_threads);
    if (rc != 0) {
        return rc;
    }
    g_pool.nodes   = nodes;
    g_pool.n_nodes = n_nodes;
    atomic_fetch_add(&g_pool.gen, 1);
    run_job(0, n_threads);
    return atomic_load(&g_node_error);
}

int orc_compute(const orc_node * nodes, int32_t n_nodes, int32_t n_threads) {
    if (nodes == NULL || n_nodes < 0 || n_threads < 1 || n_threads > ORC_MAX_THREADS) {
        return -1;
    }
    pthread_mutex_lock(&g_pool_lock);
    const int rc = compute_locked(nodes, n_nodes, n_threads);
    pthread_mutex_unlock(&g_pool_lock);
    return rc;
}

double orc_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double) ts.tv_sec + 1e-9 * (double) ts.tv_nsec;
}

int orc_time_nodes(const orc_node * nodes, int32_t n_nodes, int32_t n_threads, int32_t warmup, int32_t reps,
                   double * times) {
    if (nodes == NULL || times == NULL || reps < 1 || n_threads < 1 || n_threads > ORC_MAX_THREADS) {
        return -1;
    }
    pthread_mutex_lock(&g_pool_lock);
    int rc = 0;
    for (int i = 0; i < warmup && rc == 0; ++i) {
        rc = compute_locked(nodes, n_nodes, n_threads);
    }
    for (int i = 0; i < reps && rc == 0; ++i) {
        const double t0 = orc_now();
        rc              = compute_locked(nodes, n_nodes, n_threads);
        times[i]        = orc_now() - t0;
    }
    pthread_mutex_unlock(&g_pool_lock);
    return rc;
}

__attribute__((destructor)) static void orc_fini(void) {
    pool_shutdown();
}

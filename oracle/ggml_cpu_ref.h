/*
 * ggml_cpu_ref.h -- TEST INFRASTRUCTURE ONLY. A CPU restatement of the
 * ggml-CPU arithmetic for the ops synthesize.cpp's graph builders emit on the
 * fused-primitive path. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker or as the timed CPU
 * baseline; the product (libsynth_hip) never links or calls it.
 *
 * The upstream ggml sources are not available (the reference's ggml/ is an
 * uninitialised submodule), so each op restates the published ggml-CPU
 * algorithm and cites the reference call site that emits the node. The
 * restatement is pinned against the reference's own golden vectors and
 * against closed forms in tests/.
 *
 * Execution mirrors ggml's CPU graph compute: a persistent pool of n_threads
 * threads runs every node, thread ith taking its ggml share of rows, with a
 * barrier between nodes.
 */
#ifndef GGML_CPU_REF_H
#define GGML_CPU_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum orc_type { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_Q5_K = 13, ORC_I32 = 26, ORC_BF16 = 30 };

enum orc_op {
    ORC_OP_ADD = 1,      /* dst = src0 + src1                       ggml_add            */
    ORC_OP_MUL,          /* dst = src0 * src1                       ggml_mul            */
    ORC_OP_DIV,          /* dst = src0 / src1                       ggml_div            */
    ORC_OP_RMS_NORM,     /* dst = x * 1/sqrt(mean(x^2)+eps)         ggml_rms_norm       */
    ORC_OP_ROPE_NEOX,    /* NEOX rotary                             ggml_rope_ext       */
    ORC_OP_SILU,         /* x/(1+exp(-x))                           ggml_silu           */
    ORC_OP_SIN,          /* sinf(x)                                 ggml_sin            */
    ORC_OP_SQR,          /* x*x                                     ggml_sqr            */
    ORC_OP_EXP,          /* expf(x)                                 ggml_exp            */
    ORC_OP_LEAKY_RELU,   /* (x>0?x:0) + slope*(x<0?x:0)             ggml_leaky_relu     */
    ORC_OP_SCALE_BIAS,   /* b==0: x*s; else fma(x, s, b)            ggml_scale_bias     */
    ORC_OP_GET_ROWS,     /* dst[:, r] = to_f32(src0[:, ids[r]])     ggml_get_rows       */
    ORC_OP_CAST_F32,     /* BF16/F16/F32 -> F32                     ggml_cast           */
    ORC_OP_GLU_SWIGLU,   /* single-tensor swiglu                    ggml_swiglu         */
    ORC_OP_SOFT_MAX,     /* softmax(x*scale + mask) per row         ggml_soft_max_ext   */
    ORC_OP_CONT_F32,     /* strided F32 view -> contiguous          ggml_cont           */
    ORC_OP_BINBCAST,     /* add/mul/div, src1 repeated (can_repeat) ggml_add ...        */
    ORC_OP_SUB,          /* dst = src0 - src1                       ggml_sub            */
    ORC_OP_TANH,         /* tanhf(x)                                ggml_tanh           */
    ORC_OP_SIGMOID,      /* 1/(1+expf(-x))                          ggml_sigmoid        */
    ORC_OP_ELU,          /* x > 0 ? x : expm1f(x)                   ggml_elu            */
    ORC_OP_GELU_ERF,     /* 0.5*x*(1+erff(x/sqrt(2)))               ggml_gelu_erf       */
    ORC_OP_CLAMP,        /* MAX(MIN(x, f[1]), f[0])                 ggml_clamp          */
    ORC_OP_NORM,         /* (x-mean)/sqrt(var+eps), f[0] = eps      ggml_norm           */
    ORC_OP_IM2COL,       /* 1-D convolution columns                 ggml_im2col         */
    ORC_OP_COL2IM_1D,    /* transposed-convolution scatter-back     ggml_col2im_1d      */
    ORC_OP_PAD,          /* zero padding, left and right per dim    ggml_pad_ext        */
    ORC_OP_PAD_REFLECT_1D, /* reflect padding along dim 0           ggml_pad_reflect_1d */
    ORC_OP_REPEAT,       /* tile to a larger shape                  ggml_repeat         */
    ORC_OP_ACC,          /* a copy of src0, src1 added into a view  ggml_acc            */
    ORC_OP_RELU,         /* x > 0 ? x : 0                           ggml_relu           */
    ORC_OP_NEG,          /* -x                                      ggml_neg            */
    ORC_OP_STEP,         /* x > 0 ? 1 : 0                           ggml_step           */
    ORC_OP_SQRT,         /* sqrtf(x)                                ggml_sqrt           */
    ORC_OP_SUM_ROWS,     /* dst[r] = (float) double sum of row r    ggml_sum_rows       */
    ORC_OP_MEAN,         /* dst[r] = sum_rows / (float) ne0         ggml_mean           */
    ORC_OP_DIAG_MASK_INF, /* -inf past n_past + row, else x         ggml_diag_mask_inf  */
    ORC_OP_ISTFT,        /* Kokoro's inverse STFT (host code)      kokoro inverse_stft */
    ORC_OP_HARMONIC_SOURCE, /* Kokoro's harmonic source (host code) build_harmonic_source */
    ORC_OP_LOG_MEL,      /* Qwen3-TTS speaker encoder's log-mel      compute_log_mel     */
};

/*
 * One graph node. All tensors are contiguous row-major: `nrows` rows of `ne0`
 * elements. Binary ops take src1 either with `nrows` rows or with one row that
 * is broadcast over every row (src1_rows == 1), which is ggml's
 * ggml_can_repeat_rows case, or with one element per row (src1_ne0 == 1,
 * broadcast along the row).
 *
 *   ROPE_NEOX : src0 [ne0=head_dim, ne1=heads, nrows/ne1 positions], src1 = I32
 *               positions; i[0] = n_dims; f[0] = freq_base, f[1] = freq_scale,
 *               f[2] = attn_factor; i[1] = 0: cos/sin from libm cosf/sinf (as
 *               ggml-CPU), 1: from double cos/sin rounded once to f32.
 *   RMS_NORM  : f[0] = eps.
 *   LEAKY_RELU: f[0] = negative slope.
 *   SCALE_BIAS: f[0] = scale, f[1] = bias.
 *   GET_ROWS  : src0 is a table of `src1_rows` rows of ne0 elements of type
 *               `type0`; src1 = I32 ids (nrows of them); dst F32.
 *   CAST_F32  : src0 of type `type0`.
 *   GLU_SWIGLU: src0 rows of 2*ne0 elements; i[0] = swapped.
 *   SOFT_MAX  : src0 rows of ne0 scores, ne1 rows per head; src1 = F32 mask or
 *               NULL, with src1_rows rows per mask head and i[0] mask heads
 *               (head h reads mask head h % i[0]); f[0] = scale.
 *   BINBCAST  : src1 = int64_t[9]: src0's ne[0..3], src1's ne[0..3], the
 *               src1 data pointer; i[0] = ORC_OP_ADD, _MUL or _DIV. Every
 *               src1 extent divides src0's; all contiguous.
 *   CONT_F32  : src0 = the first element of an F32 view, src1 = int64_t[8]
 *               (the view's ne[0..3], then its byte strides nb[0..3]); dst
 *               contiguous. The only op whose src0 is not contiguous.
 *   IM2COL    : src0 = F32 x [IW, IC, N]; src1 = int64_t[7] {IW, IC, N, K,
 *               s0, p0, d0}; type0 = the dst type, ORC_F32 or ORC_F16; dst
 *               [IC*K, OW, N], OW = (IW + 2*p0 - d0*(K-1) - 1)/s0 + 1 (C
 *               division).
 *   COL2IM_1D : src0 = F32 columns [K*OC, L]; src1 = int64_t[5] {K, OC, L,
 *               stride, padding}; dst F32 [T, OC], T = (L-1)*stride + K -
 *               2*padding.
 *   PAD, PAD_REFLECT_1D, REPEAT : src0 contiguous F32; src1 = int64_t[12]:
 *               src0's ne[0..3], dst's ne[0..3], then the left pads lp[0..3]
 *               (PAD), {p0, p1, 0, 0} (PAD_REFLECT_1D) or zeros (REPEAT);
 *               dst contiguous F32.
 *   SUM_ROWS, MEAN : src0 nrows rows of ne0; dst one value per row.
 *   DIAG_MASK_INF : src0 nrows rows of ne0, ne1 rows per matrix; i[0] = n_past.
 *   LOG_MEL   : src0 = PCM (ne0 samples); src1 = the Slaney filterbank
 *               (i[3] mel bins of n_fft/2 + 1); i[0] = n_fft, i[1] = hop,
 *               i[2] = win_length; dst frames of i[3] log energies.
 *   HARMONIC_SOURCE : src0 = f0 (nrows values); src1 = orc_source_args; dst =
 *               the excitation (nrows * scale values); the spectrum into
 *               args->har ((nrows*scale/hop + 1) frames of 2*(n_fft/2 + 1)).
 *   ISTFT     : src0 = the generator's spectrum, nrows frames of ne0 = n_fft + 2
 *               values (n_fft/2 + 1 log-magnitudes, then as many raw phases);
 *               i[0] = n_fft, i[1] = hop; dst (nrows - 1) * hop samples.
 *   ACC       : src0 = a, contiguous F32 of nrows*ne0 elements; src1 =
 *               int64_t[9]: b's ne[0..3], the view's byte strides nb1, nb2,
 *               nb3, its byte offset, then the b data pointer (contiguous F32);
 *               dst contiguous F32 of a's size.
 */
/* Kokoro's harmonic source (kokoro/source.cpp): the learned merge, the random
 * draws and the module's constants. */
typedef struct orc_source_args {
    const float * merge_weight;  /* harmonics */
    const float * rand_ini;      /* harmonics */
    const float * noise;         /* nrows*scale frames of harmonics */
    float *       har;           /* out: frames of 2*bins (magnitudes, then phases) */
    float         merge_bias;
    float         sine_amp;
    float         noise_std;
    float         voiced_threshold;
    int32_t       sampling_rate;
    int32_t       harmonics;
    int32_t       scale;
    int32_t       n_fft;
    int32_t       hop;
    int32_t       pad;
} orc_source_args;

typedef struct orc_node {
    int32_t      op;
    int32_t      type0;
    int64_t      ne0;
    int64_t      nrows;
    int64_t      ne1;
    int64_t      src1_rows;
    int64_t      src1_ne0;
    const void * src0;
    const void * src1;
    void *       dst;
    float        f[4];
    int32_t      i[4];
} orc_node;

/* The Qwen3-TTS speaker encoder's Slaney mel filterbank (qwen3-tts/mel.cpp:
 * 131-170): mel_bins rows of n_fft/2 + 1 weights into out. */
void orc_mel_filterbank(uint32_t sample_rate, uint32_t n_fft, uint32_t mel_bins, float fmin, float fmax, float * out);

/* Runs the nodes in order on n_threads threads (1 = inline). Returns 0, or a
 * negative value for an unknown op / bad argument. */
int orc_compute(const orc_node * nodes, int32_t n_nodes, int32_t n_threads);

/* Scalar conversions (exact), and the ggml data-generation roundings. */
float    orc_fp16_to_fp32(uint16_t h);
float    orc_bf16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16(float f);
uint16_t orc_fp32_to_bf16(float f);

/* Wall-clock helper for the CPU baseline (CLOCK_MONOTONIC, seconds). */
double orc_now(void);

/* Times `reps` repetitions of the node list on n_threads threads after
 * `warmup` untimed ones; writes each repetition's seconds into times[]. */
int orc_time_nodes(const orc_node * nodes, int32_t n_nodes, int32_t n_threads, int32_t warmup, int32_t reps,
                   double * times);

#ifdef __cplusplus
}
#endif

#endif

/*
 * synth_graph.h -- node-run executor of libsynth_hip: the graph_compute core
 * of a ggml backend module, without ggml's headers.
 *
 * A ggml backend receives the nodes the scheduler placed on it as an ordered
 * list (ggml_cgraph, topological, the order ggml_build_forward_expand visits
 * them: src[0] before src[1]) and must run them in that order; a fusing
 * backend runs a recognised node run as one launch when the run's
 * intermediate tensors are read nowhere else (no other node of the list, no
 * later split, not a graph output). This file is that logic over
 * plain descriptors: the module's glue turns each ggml_tensor node into an
 * shp_node (op kind, op_params words, dst and src descriptors, and for each
 * src the index of the node that produced it) and calls shp_graph_compute
 * from its graph_compute, and shp_graph_node_supported from supports_op
 * (src/backend-plan.cpp:120-131 builds the scheduler that asks both).
 *
 * Runs recognised (each one launch, bit-identical to running its nodes one by
 * one, which is what the reference's graphs compute today):
 *   RMS_NORM [CPY] MUL [ROPE [CPY]]  rms_norm()*w, with the gain cast and a
 *        following NEOX rope and cache copy folded in
 *        (src/arch/qwen3-tts/operations.cpp:20-32, 98-116)
 *   two such rope runs + [CPY]        the q and k runs of one attention block
 *        (:98-104) with k's cache copy and v's (:109-116) in one launch: the
 *        sibling run and the v copy may sit later in the list with other
 *        nodes between (ggml expands the k and v copies before the q path);
 *        they are moved up to the first run only when no node between them
 *        reads or writes what they read or write (byte ranges of the
 *        descriptors) and none produces what they read
 *   ADD RMS_NORM [CPY] MUL           residual add + post-attention norm
 *        (:143-145, :147 -> :86); the sum is written when read elsewhere
 *   SILU MUL                         SwiGLU (:39-41)
 *   ADD LEAKY_RELU                   residual carry
 *        (src/arch/vits/waveform-decoder.cpp:150-158)
 *   ADD.. SCALE LEAKY_RELU           branch average (:214-225)
 *   MUL SIN MUL|SQR DIV ADD          Snake (src/arch/kokoro/operations.cpp:137-147)
 *   MUL SIN MUL|SQR SCALE DIV ADD    guarded Snake (src/arch/omnivoice/codec.cpp:51-68)
 *   EXP MUL SIN SQR|MUL EXP SCALE DIV ADD  SnakeBeta (src/arch/qwen3-tts/codec.cpp:184-200)
 *   GET_ROWS (GET_ROWS ADD)+         multi-codebook gather->sum
 *        (src/arch/qwen3-tts/code-predictor.cpp:82-107)
 *   CPY ADD [ADD] [LEAKY_RELU]       a time-major convolution's tail: the
 *        transposing copy, the [1, C] bias, the residual, the next leaky-ReLU
 *        (src/arch/vits/waveform-decoder.cpp:111,118-121,146-150); also the
 *        codec's channel bias before or after its transposing copy
 *        (src/arch/qwen3-tts/codec.cpp:134-140,179-181)
 *   CPY ADD|MUL|DIV                  a crop's copy of a row-contiguous view,
 *        then the op on the copy (codec.cpp:64-71,100-104): the op reads the view
 *   CPY [views] IM2COL               the causal convolution's time-major copy
 *        and its column matrix (src/arch/qwen3-tts/codec.cpp:94-96): im2col
 *        reads the channel-major activation through the transposed view
 *   DIAG_MASK_INF SOFT_MAX           the codec encoder's causal attention softmax
 *        (src/arch/qwen3-tts/codec-encoder.cpp:482-483)
 *   MUL SUM_ROWS                     the attention-weighted sums of the speaker
 *        encoder's statistics pooling (src/arch/qwen3-tts/speaker-encoder.cpp:
 *        292-293,374): the product is summed as it is formed
 * Any other supported node runs alone through its entry point in
 * synth_hip.h. View-like nodes (NONE, VIEW, RESHAPE, PERMUTE, TRANSPOSE)
 * are SHP_NODE_NOP: no work.
 */
#ifndef SYNTH_GRAPH_H
#define SYNTH_GRAPH_H

#include "synth_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Node kinds, named for the ggml op (and unary/GLU op) each stands for. The
 * values are this library's own; the glue maps ggml's enums by name. op_params
 * hold the words ggml's op constructor stored, in its layout. */
typedef enum shp_node_op {
    SHP_NODE_NOP = 0,    /* GGML_OP_NONE, VIEW, RESHAPE, PERMUTE, TRANSPOSE */
    SHP_NODE_ADD,        /* GGML_OP_ADD */
    SHP_NODE_MUL,        /* GGML_OP_MUL */
    SHP_NODE_DIV,        /* GGML_OP_DIV */
    SHP_NODE_SQR,        /* GGML_OP_SQR */
    SHP_NODE_SIN,        /* GGML_OP_SIN */
    SHP_NODE_SCALE,      /* GGML_OP_SCALE: f32 {s, b} */
    SHP_NODE_CPY,        /* GGML_OP_CPY (ggml_cpy, ggml_cast): src[0] into dst; also
                            GGML_OP_CONT (ggml_cont: src[0] into a contiguous dst of
                            its shape), e.g. of a permute(0,2,1,3) view, or of an F32
                            transpose / permute whose ne[0] is strided and one of dims
                            1..3 contiguous; a view with no contiguous dimension is
                            unsupported */
    SHP_NODE_GET_ROWS,   /* GGML_OP_GET_ROWS: src[0] table, src[1] ids */
    SHP_NODE_RMS_NORM,   /* GGML_OP_RMS_NORM: f32 {eps} */
    SHP_NODE_SOFT_MAX,   /* GGML_OP_SOFT_MAX: f32 {scale, max_bias}; src[1] mask or absent */
    SHP_NODE_ROPE,       /* GGML_OP_ROPE: i32 {n_past, n_dims, mode, n_ctx, n_ctx_orig},
                            f32 [5..10] {freq_base, freq_scale, ext_factor, attn_factor,
                            beta_fast, beta_slow}; src[1] positions, src[2] freq factors */
    SHP_NODE_LEAKY_RELU, /* GGML_OP_LEAKY_RELU: f32 {negative_slope} */
    SHP_NODE_SILU,       /* GGML_OP_UNARY, GGML_UNARY_OP_SILU */
    SHP_NODE_EXP,        /* GGML_OP_UNARY, GGML_UNARY_OP_EXP */
    SHP_NODE_GLU_SWIGLU, /* GGML_OP_GLU, GGML_GLU_OP_SWIGLU: i32 [1] swapped; src[1] absent
                            (single tensor) or the second half (split form) */
    SHP_NODE_CONCAT,     /* GGML_OP_CONCAT: i32 {dim}; src[0], src[1] */
    SHP_NODE_SUB,        /* GGML_OP_SUB */
    SHP_NODE_TANH,       /* GGML_OP_UNARY, GGML_UNARY_OP_TANH */
    SHP_NODE_SIGMOID,    /* GGML_OP_UNARY, GGML_UNARY_OP_SIGMOID */
    SHP_NODE_ELU,        /* GGML_OP_UNARY, GGML_UNARY_OP_ELU */
    SHP_NODE_GELU_ERF,   /* GGML_OP_UNARY, GGML_UNARY_OP_GELU_ERF */
    SHP_NODE_CLAMP,      /* GGML_OP_CLAMP: f32 {min, max} */
    SHP_NODE_NORM,       /* GGML_OP_NORM: f32 {eps} */
    SHP_NODE_IM2COL,     /* GGML_OP_IM2COL: i32 {s0, s1, p0, p1, d0, d1, is_2D}; src[0] the
                            kernel (its extents only), src[1] the input; the 1-D form
                            (is_2D 0, p1 0) every src/arch call site builds */
    SHP_NODE_COL2IM_1D,  /* ggml_col2im_1d (an op of the reference's pinned ggml): i32
                            {stride, out_channels, padding}, which the module's glue fills
                            from the node's own parameters; src[0] the columns */
    SHP_NODE_PAD,        /* GGML_OP_PAD (ggml_pad, ggml_pad_ext): i32 {lp0, rp0, lp1, rp1,
                            lp2, rp2, lp3, rp3} (a ninth word, circular padding, must be 0) */
    SHP_NODE_PAD_REFLECT_1D, /* GGML_OP_PAD_REFLECT_1D: i32 {p0, p1} */
    SHP_NODE_REPEAT,     /* GGML_OP_REPEAT (ggml_repeat, ggml_repeat_4d): dst's shape */
    SHP_NODE_ACC,        /* GGML_OP_ACC: i32 {nb1, nb2, nb3, offset, inplace} (bytes); src[0]
                            a, src[1] b; dst a's shape (the same data when inplace) */
    SHP_NODE_RELU,       /* GGML_OP_UNARY, GGML_UNARY_OP_RELU */
    SHP_NODE_NEG,        /* GGML_OP_UNARY, GGML_UNARY_OP_NEG */
    SHP_NODE_STEP,       /* GGML_OP_UNARY, GGML_UNARY_OP_STEP */
    SHP_NODE_SQRT,       /* GGML_OP_SQRT */
    SHP_NODE_SUM_ROWS,   /* GGML_OP_SUM_ROWS: dst [1, ne1, ne2, ne3] */
    SHP_NODE_MEAN,       /* GGML_OP_MEAN: dst [1, ne1, ne2, ne3] */
    SHP_NODE_DIAG_MASK_INF, /* GGML_OP_DIAG_MASK_INF: i32 {n_past} (dst may be src[0]: inplace) */
    SHP_NODE_OP_COUNT
} shp_node_op;

#define SHP_NODE_MAX_SRC     3
#define SHP_NODE_FLAG_OUTPUT 1u /* dst is read after this graph (GGML_TENSOR_FLAG_OUTPUT) */

typedef struct shp_node {
    int32_t    op;                         /* shp_node_op */
    uint32_t   flags;                      /* SHP_NODE_FLAG_* */
    int32_t    src_node[SHP_NODE_MAX_SRC]; /* index in this list of the node whose dst
                                              src[i] is, or -1 (a leaf, a tensor from
                                              outside the list, or no src) */
    int32_t    uses;                       /* reads of dst in the whole graph (ggml's use
                                              count, later splits included), or 0 when
                                              this list holds every read */
    int32_t    op_params[16];
    shp_tensor dst;
    shp_tensor src[SHP_NODE_MAX_SRC]; /* data == NULL: no such src */
} shp_node;

typedef enum shp_run_kind {
    SHP_RUN_UNSUPPORTED = -1, /* the node cannot run here */
    SHP_RUN_NOP         = 0,  /* view-like node */
    SHP_RUN_SINGLE,           /* one node through its own entry point */
    SHP_RUN_NORM_MUL,
    SHP_RUN_NORM_MUL_ROPE,
    SHP_RUN_ADD_NORM_MUL,
    SHP_RUN_SILU_MUL,
    SHP_RUN_ADD_LEAKY,
    SHP_RUN_ADD_SCALE_LEAKY,
    SHP_RUN_SNAKE,
    SHP_RUN_SNAKE_GUARDED,
    SHP_RUN_SNAKE_BETA,
    SHP_RUN_GATHER_SUM,
    SHP_RUN_QK_NORM_ROPE,     /* q and k rope runs (the k sink may be a cache copy) */
    SHP_RUN_QK_NORM_ROPE_KV,  /* the same plus the v cache copy */
    SHP_RUN_CONT_ADD_LEAKY,   /* CPY of a transposed view, ADD of the per-row bias,
                                 [ADD of a residual], [LEAKY_RELU]:
                                 shp_cont_add_leaky_relu */
    SHP_RUN_VIEW_BINARY,      /* CPY of a row-contiguous F32 view, then ADD, MUL or
                                 DIV of the copy: the binary op reads the view */
    SHP_RUN_CONT_IM2COL,      /* CPY of a transposed channel-major F32 activation,
                                 [views], IM2COL of the copy: shp_im2col reads the
                                 activation in place of the copy */
    SHP_RUN_MUL_SUM_ROWS,     /* MUL whose product only SUM_ROWS reads, then that
                                 SUM_ROWS: shp_mul_sum_rows */
    SHP_RUN_DIAG_MASK_SOFT_MAX /* DIAG_MASK_INF whose result only a maskless SOFT_MAX
                                 reads, then that SOFT_MAX: shp_soft_max_causal */
} shp_run_kind;

typedef struct shp_graph_run {
    int32_t kind;  /* shp_run_kind */
    int32_t first; /* index of the run's first node, where it is launched */
    int32_t last;  /* index of its last node (the run's result; for the q/k
                      runs, the last of their nodes); view-like nodes between
                      first and last belong to no run, and for the q/k runs
                      so do the other nodes between their parts */
    int32_t nodes; /* nodes the run executes */
} shp_graph_run;

/* 1 when the node can run here on its own (supports_op), else 0. */
int32_t shp_graph_node_supported(const shp_node * node);

/*
 * Splits the list into runs, in order, without launching anything (host code
 * only). runs may be NULL to count them; *n_runs receives the count.
 * SHP_ERR_INVALID_ARG for a malformed list: a src_node not naming an earlier
 * node, a src_node without its src, a negative uses or one below the reads
 * the list itself makes, an unknown op.
 */
shp_status_t shp_graph_plan(const shp_node * nodes,
                            int32_t          n_nodes,
                            shp_graph_run *  runs,
                            int32_t          capacity,
                            int32_t *        n_runs);

/*
 * Runs the list on `stream`, run by run. A list holding an unsupported node
 * returns SHP_ERR_UNSUPPORTED with nothing enqueued (ggml's scheduler never
 * hands a backend such a node when supports_op said no). Otherwise the first
 * failing launch's status is returned (runs before it have been enqueued),
 * as graph_compute's ggml_status is.
 */
shp_status_t shp_graph_compute(const shp_node * nodes, int32_t n_nodes, shp_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SYNTH_GRAPH_H */

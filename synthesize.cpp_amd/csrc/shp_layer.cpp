// shp_layer_nongemm_step: the non-GEMM node runs of one Qwen3 decoder layer
// (src/arch/qwen3-tts/operations.cpp:84-147) enqueued in the layer's order on
// one stream, after every tensor of the step has been checked.
//
// The five launches are the ones the single entry points make; the value of
// this entry point is the contract (one call per layer, with the GEMM and
// attention outputs as inputs, and no partial enqueue on a malformed step),
// not a different kernel.
#include <cstdint>

#include "shp_internal.hpp"
#include "synth_hip.h"

namespace shp {
namespace {

// An F32 activation of ggml shape [ne0, t, 1, 1].
bool act2d(const shp_tensor * a, int64_t ne0, int64_t t) {
    return well_formed(a) && a->type == SHP_TYPE_F32 && a->ne[0] == ne0 && a->ne[1] == t && a->ne[2] == 1 &&
           a->ne[3] == 1;
}

// An F32 activation of ggml shape [head_dim, heads, t, 1].
bool act3d(const shp_tensor * a, int64_t head_dim, int64_t heads, int64_t t) {
    return well_formed(a) && a->type == SHP_TYPE_F32 && a->ne[0] == head_dim && a->ne[1] == heads &&
           a->ne[2] == t && a->ne[3] == 1;
}

// A gain vector of n elements: one contiguous row, F32, BF16 or F16.
bool gain(const shp_tensor * w, int64_t n) {
    return well_formed(w) && weight_kind(w->type) >= 0 && nelements(*w) == n && contiguous(*w);
}

shp_status_t check_step(const shp_layer_step & s) {
    if (s.reserved != 0 || s.x == nullptr || s.q == nullptr || s.k == nullptr || s.gate == nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    const int64_t hidden   = s.x->ne[0];
    const int64_t t        = s.x->ne[1];
    const int64_t head_dim = s.q->ne[0];
    const int64_t q_heads  = s.q->ne[1];
    const int64_t kv_heads = s.k->ne[1];
    const int64_t ffn      = s.gate->ne[0];
    if (hidden > INT32_MAX || head_dim > INT32_MAX || ffn > INT32_MAX || t > INT32_MAX ||
        q_heads + kv_heads > INT32_MAX) {
        return SHP_ERR_INVALID_ARG;
    }
    for (const shp_tensor * a : { s.x, static_cast<const shp_tensor *>(s.normed), s.attn_out,
                                  static_cast<const shp_tensor *>(s.resid), static_cast<const shp_tensor *>(s.mlp_in),
                                  s.mlp_out, static_cast<const shp_tensor *>(s.out) }) {
        if (!act2d(a, hidden, t)) {
            return SHP_ERR_INVALID_ARG;
        }
    }
    for (const shp_tensor * a : { s.gate, s.up, static_cast<const shp_tensor *>(s.act) }) {
        if (!act2d(a, ffn, t)) {
            return SHP_ERR_INVALID_ARG;
        }
    }
    if (!act3d(s.q, head_dim, q_heads, t) || !act3d(s.q_out, head_dim, q_heads, t) ||
        !act3d(s.k, head_dim, kv_heads, t) || !act3d(s.k_out, head_dim, kv_heads, t)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (!well_formed(s.pos) || s.pos->type != SHP_TYPE_I32 || nelements(*s.pos) != t || !contiguous(*s.pos)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (!i32_aligned(*s.pos)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (!gain(s.w_in, hidden) || !gain(s.w_post, hidden) || !gain(s.wq, head_dim) || !gain(s.wk, head_dim)) {
        return SHP_ERR_INVALID_ARG;
    }
    if (s.wq->type != s.wk->type) {
        return SHP_ERR_UNSUPPORTED;  // one rope launch converts both head gains
    }
    if (!(s.eps >= 0.0f) || s.n_dims <= 0 || s.n_dims % 2 != 0 || s.n_dims > head_dim) {
        return SHP_ERR_INVALID_ARG;
    }
    return SHP_OK;
}

}  // namespace
}  // namespace shp

extern "C" shp_status_t shp_layer_nongemm_step(const shp_layer_step * step, shp_stream_t stream) {
    if (step == nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    const shp_layer_step & s  = *step;
    shp_status_t           st = shp::check_step(s);
    if (st != SHP_OK) {
        return st;
    }
    // operations.cpp:85-86, the input norm.
    if ((st = shp_rms_norm_mul(s.x, s.w_in, s.eps, s.normed, stream)) != SHP_OK) {
        return st;
    }
    // :98-104, per-head q/k norm and NEOX rope (freq_scale 1: no rope scaling in this model).
    if ((st = shp_qk_norm_rope(s.q, s.k, s.wq, s.wk, s.eps, s.pos, s.n_dims, s.freq_base, 1.0f, s.q_out, s.k_out,
                               stream)) != SHP_OK) {
        return st;
    }
    // :143-145, residual add and the post-attention norm.
    if ((st = shp_add_rms_norm_mul(s.x, s.attn_out, s.w_post, s.eps, s.resid, s.mlp_in, stream)) != SHP_OK) {
        return st;
    }
    // :39-41 through :146, the MLP's gate activation.
    if ((st = shp_swiglu(s.gate, s.up, s.act, stream)) != SHP_OK) {
        return st;
    }
    // :147, the layer output.
    return shp_add(s.resid, s.mlp_out, s.out, stream);
}

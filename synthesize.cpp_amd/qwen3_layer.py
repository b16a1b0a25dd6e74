"""The non-GEMM node list of one Qwen3-TTS decoder layer, as a ggml backend
receives it.

decoder_layer (src/arch/qwen3-tts/operations.cpp:47-147) builds, per layer:
the input rms_norm()*w (:85-86), the q/k/v projections (:90-92), per-head
QK-norm (:98-99) and NEOX rope (:101-104), the k and v cache copies expanded
into the graph at once (:106-116), attention over the cache (:118-140), the
residual add (:143), the post-attention norm (:145), the SwiGLU MLP
(:34-42 via :146) and the output add (:147). ggml_build_forward_expand
orders the nodes depth first, src[0] first: the input norm (reached through
the k projection), k's path and its copy, v's copy, then -- from the layer
output -- the q path (reached through the attention scores), the softmax, the
residual add, the post-attention norm, SwiGLU and the output add.

decoder_layer_nodes appends exactly those nodes to a synth_hip.Graph in that
order, with the matrix products (projections, scores, attention output, MLP
projections) as leaves: their outputs are inputs here, as a backend without
GEMMs sees them. Chaining layers (x of layer l+1 = the output of layer l)
gives the non-GEMM list of a whole talker step.
"""

import torch

import synth_hip as S

F32 = torch.float32


def decoder_layer_nodes(g, x, leaves, T=1, H=1024, heads=16, kv=8, hd=128, ffn=3072, total=38, cast=True,
                        eps=1e-6, theta=1e6):
    """Appends one layer's non-GEMM nodes to `g`. `leaves` maps names to
    tensors; missing ones are created as zeros on x's device: q [T, heads, hd],
    k and v [T, kv, hd] (projections), scores [heads, T, total] (k.q), attn
    [T, H] (o_proj output), gate and up [T, ffn], mlp [T, H] (down_proj
    output), w_in, w_post [H] and wq, wk [hd] (BF16 when `cast`, the gains
    going through ggml_cast as as_f32 does, :20-25), pos I32 [T], and the
    caches kcache, vcache [total, kv, hd] whose last T rows this step writes.
    Returns ([normed, k copy, v copy, q rope, softmax, mlp_in, act, out], leaves)
    in expand order."""
    dev = x.t.device if isinstance(x, S.GVal) else x.device
    wt = torch.bfloat16 if cast else F32

    def mk(name, *shape, dtype=F32):
        if name not in leaves:
            leaves[name] = torch.zeros(shape, dtype=dtype, device=dev)
        return leaves[name]

    q, k, v = mk("q", T, heads, hd), mk("k", T, kv, hd), mk("v", T, kv, hd)
    scores, attn = mk("scores", heads, T, total), mk("attn", T, H)
    gate, up, mlp = mk("gate", T, ffn), mk("up", T, ffn), mk("mlp", T, H)
    w_in, w_post = mk("w_in", H, dtype=wt), mk("w_post", H, dtype=wt)
    wq, wk = mk("wq", hd, dtype=wt), mk("wk", hd, dtype=wt)
    pos = mk("pos", T, dtype=torch.int32)
    kcache, vcache = mk("kcache", total, kv, hd), mk("vcache", total, kv, hd)
    f = (lambda w: g.cast(w)) if cast else (lambda w: w)
    filled = total - T
    normed = g.mul(g.rms_norm(x, eps), f(w_in))
    # reshape_3d of the projections (:94-96) and the cache views (:109-116) are view nodes
    kr = g.rope_ext(g.mul(g.rms_norm(g.view(k, k), eps), f(wk)), pos, hd, S.ROPE_TYPE_NEOX, theta)
    kc = g.cpy(kr, kcache[filled:])
    vc = g.cpy(g.view(v, v), vcache[filled:])
    qr = g.rope_ext(g.mul(g.rms_norm(g.view(q, q), eps), f(wq)), pos, hd, S.ROPE_TYPE_NEOX, theta)
    probs = g.soft_max_ext(scores, None, hd ** -0.5)
    after = g.add(x, attn)
    mlp_in = g.mul(g.rms_norm(after, eps), f(w_post))
    act = g.mul(g.silu(gate), up)
    out = g.add(after, mlp)
    return [normed, kc, vc, qr, probs, mlp_in, act, out], leaves

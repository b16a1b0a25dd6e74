"""Python host binding of libsynth_hip (ctypes over the C ABI in include/synth_hip.h).

The functions mirror the ggml op (or node run) each C entry point replaces --
same names, same argument meaning, ggml [ne0, ne1, ...] shapes expressed as
torch tensors of shape (..., ne1, ne0) -- and raise ShpError on a non-zero
status, which is how the reference's builders report a node they cannot build.

torch is used only as device-memory plumbing: tensors carry the device
pointers and every call is enqueued on torch's current HIP stream. torch must
be imported before the library is loaded, because torch ships its own copy of
libamdhip64.so.7 and one process must run one HIP runtime.

There is no CPU fallback: without the built library every call raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# SHP_LIB selects another build of the library (the sanitized one of `make asan`).
LIB_PATH = os.environ.get("SHP_LIB") or os.path.join(HERE, "libsynth_hip.so")

OK, ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_BACKEND = 0, 1, 2, 17
TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_Q5_K, TYPE_I32, TYPE_BF16 = 0, 1, 8, 13, 26, 30
ROPE_TYPE_NEOX = 2
Q8_0_BLOCK_BYTES, Q8_0_BLOCK_ELEMS = 34, 32
Q5_K_BLOCK_BYTES, Q5_K_BLOCK_ELEMS = 176, 256


class ShpTensor(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int32), ("reserved", ctypes.c_int32), ("ne", ctypes.c_int64 * 4),
                ("nb", ctypes.c_size_t * 4), ("data", ctypes.c_void_p)]


class ShpLayerStep(ctypes.Structure):
    _fields_ = [(n, ctypes.POINTER(ShpTensor)) for n in (
        "x", "w_in", "normed", "q", "k", "wq", "wk", "pos", "q_out", "k_out", "attn_out", "w_post", "resid",
        "mlp_in", "gate", "up", "act", "mlp_out", "out")] + [
        ("eps", ctypes.c_float), ("freq_base", ctypes.c_float), ("n_dims", ctypes.c_int32),
        ("reserved", ctypes.c_int32)]


class ShpError(RuntimeError):
    def __init__(self, status, what):
        super().__init__("%s failed: %s (%d)" % (what, status_string(status), status))
        self.status = status


_lib = None
_PT = ctypes.POINTER(ShpTensor)


def load(path=None):
    """Loads the built library once (raises if it is missing)."""
    global _lib
    if _lib is not None:
        return _lib
    try:
        import torch  # noqa: F401  -- share torch's HIP runtime (see module docstring)
    except ImportError:
        pass
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError("libsynth_hip.so is not built (%s); run __graft_entry__.build() or make -C "
                           "synthesize.cpp_amd" % path)
    L = ctypes.CDLL(path)
    vp, f, i32, i64 = ctypes.c_void_p, ctypes.c_float, ctypes.c_int32, ctypes.c_int64
    sigs = {
        "shp_get_rows": [_PT, _PT, _PT, vp],
        "shp_get_rows_sum": [_PT, i32, _PT, _PT, vp],
        "shp_rms_norm_mul": [_PT, _PT, f, _PT, vp],
        "shp_add_rms_norm_mul": [_PT, _PT, _PT, f, _PT, _PT, vp],
        "shp_rope_ext": [_PT, _PT, i32, i32, f, f, f, f, _PT, vp],
        "shp_qk_norm_rope": [_PT, _PT, _PT, _PT, f, _PT, i32, f, f, _PT, _PT, vp],
        "shp_swiglu": [_PT, _PT, _PT, vp],
        "shp_glu_swiglu": [_PT, i32, _PT, vp],
        "shp_snake": [_PT, _PT, _PT, vp],
        "shp_add_leaky_relu": [_PT, _PT, f, _PT, _PT, vp],
        "shp_add": [_PT, _PT, _PT, vp],
        "shp_qk_norm_rope_kv": [_PT, _PT, _PT, _PT, _PT, f, _PT, i32, f, f, _PT, _PT, _PT, ctypes.c_int64, vp],
        "shp_qk_norm_rope_kv_at": [_PT, _PT, _PT, _PT, _PT, f, _PT, i32, f, f, _PT, _PT, _PT, _PT, _PT, vp],
        "shp_snake_guarded": [_PT, _PT, _PT, vp],
        "shp_snake_beta": [_PT, _PT, _PT, _PT, vp],
        "shp_exp": [_PT, _PT, vp],
        "shp_soft_max_ext": [_PT, _PT, f, f, _PT, vp],
        "shp_scale_bias": [_PT, f, f, _PT, vp],
        "shp_sum_scale_leaky_relu": [_PT, i32, f, f, _PT, _PT, vp],
        "shp_layer_nongemm_step": [ctypes.POINTER(ShpLayerStep), vp],
        "shp_mul": [_PT, _PT, _PT, vp],
        "shp_div": [_PT, _PT, _PT, vp],
        "shp_sin": [_PT, _PT, vp],
        "shp_sqr": [_PT, _PT, vp],
        "shp_cpy": [_PT, _PT, vp],
        "shp_cont_add_leaky_relu": [_PT, _PT, _PT, i32, f, _PT, _PT, vp],
        "shp_concat": [_PT, _PT, i32, _PT, vp],
        "shp_im2col": [_PT, _PT, i32, i32, i32, _PT, vp],
        "shp_col2im_1d": [_PT, i32, i32, i32, _PT, vp],
        "shp_pad": [_PT, ctypes.POINTER(ctypes.c_int32), _PT, vp],
        "shp_pad_reflect_1d": [_PT, i32, i32, _PT, vp],
        "shp_repeat": [_PT, _PT, vp],
        "shp_acc": [_PT, _PT, i64, i64, i64, i64, _PT, vp],
        "shp_sub": [_PT, _PT, _PT, vp],
        "shp_tanh": [_PT, _PT, vp],
        "shp_relu": [_PT, _PT, vp],
        "shp_neg": [_PT, _PT, vp],
        "shp_step": [_PT, _PT, vp],
        "shp_sqrt": [_PT, _PT, vp],
        "shp_sum_rows": [_PT, _PT, vp],
        "shp_mean": [_PT, _PT, vp],
        "shp_mul_sum_rows": [_PT, _PT, _PT, vp],
        "shp_diag_mask_inf": [_PT, i32, _PT, vp],
        "shp_soft_max_causal": [_PT, i32, f, _PT, vp],
        "shp_inverse_stft": [_PT, i32, i32, _PT, vp],
        "shp_harmonic_source": [_PT, _PT, f, _PT, _PT, i32, i32, f, f, f, i32, i32, _PT, _PT, vp],
        "shp_log_mel": [_PT, _PT, i32, i32, i32, _PT, vp],
        "shp_mel_filterbank": [i32, i32, i32, f, f, vp],
        "shp_sigmoid": [_PT, _PT, vp],
        "shp_elu": [_PT, _PT, vp],
        "shp_gelu_erf": [_PT, _PT, vp],
        "shp_clamp": [_PT, f, f, _PT, vp],
        "shp_norm": [_PT, f, _PT, vp],
        "shp_graph_compute": [ctypes.POINTER(ShpNode), i32, vp],
        "shp_graph_plan": [ctypes.POINTER(ShpNode), i32, ctypes.POINTER(ShpGraphRun), i32, ctypes.POINTER(i32)],
    }
    for name, args in sigs.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int32
    vpp, u64p = ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_uint64)
    gsigs = {
        "shp_gguf_open": ([ctypes.c_char_p, vpp], ctypes.c_int32),
        "shp_gguf_close": ([vp], None),
        "shp_gguf_version": ([vp], ctypes.c_uint32),
        "shp_gguf_tensor_count": ([vp], ctypes.c_int64),
        "shp_gguf_tensor_name": ([vp, ctypes.c_int64], ctypes.c_char_p),
        "shp_gguf_tensor_info": ([vp, ctypes.c_char_p, _PT, u64p, u64p], ctypes.c_int32),
        "shp_gguf_kv_u32": ([vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)], ctypes.c_int32),
        "shp_gguf_kv_string": ([vp, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t], ctypes.c_int32),
        "shp_gguf_load_tensor": ([vp, ctypes.c_char_p, vp, ctypes.c_size_t, _PT, vp], ctypes.c_int32),
        "shp_gguf_load_tensors": ([vp, ctypes.POINTER(ctypes.c_char_p), ctypes.c_int32, ctypes.POINTER(vp),
                                   ctypes.POINTER(ctypes.c_size_t), _PT, vp], ctypes.c_int32),
        "shp_table_type_for_profile": ([ctypes.c_char_p, ctypes.POINTER(ctypes.c_int32)], ctypes.c_int32),
    }
    for name, (args, res) in gsigs.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    L.shp_graph_node_supported.argtypes = [ctypes.POINTER(ShpNode)]
    L.shp_graph_node_supported.restype = ctypes.c_int32
    L.shp_abi_version.restype = ctypes.c_uint32
    L.shp_abi_version.argtypes = []
    L.shp_status_string.restype = ctypes.c_char_p
    L.shp_status_string.argtypes = [ctypes.c_int32]
    _lib = L
    return L


def status_string(status):
    return load().shp_status_string(int(status)).decode()


def abi_version():
    return int(load().shp_abi_version())


# ---------------------------------------------------------------------------
# descriptors
# ---------------------------------------------------------------------------

class BlockTensor:
    """A block-quantized tensor held as raw blocks: `data` is a uint8 torch
    tensor of shape (..., rows, ne0/ELEMS*BYTES); ne0 is the logical row length."""
    TYPE = ELEMS = BYTES = None

    def __init__(self, data, ne0):
        assert ne0 % self.ELEMS == 0
        assert data.shape[-1] == ne0 // self.ELEMS * self.BYTES
        self.data, self.ne0 = data, ne0

    @property
    def rows(self):
        return self.data.shape[-2]


class Q8Tensor(BlockTensor):
    """Q8_0: 32-element blocks {f16 d; int8 qs[32]}."""
    TYPE, ELEMS, BYTES = TYPE_Q8_0, Q8_0_BLOCK_ELEMS, Q8_0_BLOCK_BYTES


class Q5KTensor(BlockTensor):
    """Q5_K: 256-element super-blocks of 176 bytes."""
    TYPE, ELEMS, BYTES = TYPE_Q5_K, Q5_K_BLOCK_ELEMS, Q5_K_BLOCK_BYTES


def _torch_type(t):
    import torch
    return {torch.float32: TYPE_F32, torch.float16: TYPE_F16, torch.bfloat16: TYPE_BF16,
            torch.int32: TYPE_I32}[t.dtype]


def desc(t):
    """shp_tensor for a torch tensor (or BlockTensor); None stays None."""
    if t is None:
        return None
    d = ShpTensor()
    if isinstance(t, BlockTensor):
        raw = t.data
        shape = list(raw.shape[::-1])
        strides = list(raw.stride()[::-1])
        d.type = t.TYPE
        shape[0] = t.ne0
        strides[0] = t.BYTES
        item = 1
    else:
        shape = list(t.shape[::-1]) or [1]
        strides = list(t.stride()[::-1]) or [1]
        d.type = _torch_type(t)
        item = t.element_size()
        strides = [s * item for s in strides]
        raw = t
    if len(shape) > 4:
        raise ValueError("at most 4 dimensions")
    while len(shape) < 4:
        strides.append(strides[-1] * shape[-1] if item else 0)
        shape.append(1)
    d.reserved = 0
    for k in range(4):
        d.ne[k] = int(shape[k])
        d.nb[k] = int(strides[k])
    d.data = raw.data_ptr()
    return d


def _ref(d):
    return ctypes.byref(d) if d is not None else None


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check(status, what):
    if status != OK:
        raise ShpError(status, what)


def _empty_like_f32(shape, device):
    import torch
    return torch.empty(shape, dtype=torch.float32, device=device)


# ---------------------------------------------------------------------------
# ops (ggml names)
# ---------------------------------------------------------------------------

def get_rows(src, ids, out=None):
    """ggml_get_rows(src, ids) -> f32. src (rows, ne0) torch F32/F16/BF16, Q8Tensor or Q5KTensor;
    ids int32 (n,). Batched forms follow ggml's [ne0, rows, ne2, ne3] x [n, ne2, ne3]."""
    raw = src.data if isinstance(src, BlockTensor) else src
    ne0 = src.ne0 if isinstance(src, BlockTensor) else src.shape[-1]
    if out is None:
        out = _empty_like_f32(tuple(ids.shape) + (ne0,), raw.device)
    _check(load().shp_get_rows(_ref(desc(src)), _ref(desc(ids)), _ref(desc(out)), _stream()), "get_rows")
    return out


def get_rows_sum(tables, codes, out=None):
    """sum_code_embeddings: codes int32 (groups, frames) (ggml [frames, groups]); tables
    one per group; returns f32 (frames, ne0) = ordered sum of the gathered rows."""
    n = len(tables)
    arr = (ShpTensor * n)(*[desc(t) for t in tables])
    first = tables[0]
    ne0 = first.ne0 if isinstance(first, BlockTensor) else first.shape[-1]
    raw = first.data if isinstance(first, BlockTensor) else first
    if out is None:
        out = _empty_like_f32((codes.shape[-1], ne0), raw.device)
    _check(load().shp_get_rows_sum(arr, n, _ref(desc(codes)), _ref(desc(out)), _stream()), "get_rows_sum")
    return out


def rms_norm_mul(x, w, eps, out=None):
    """rms_norm() of src/arch/qwen3-tts/operations.cpp:27-32 (w None: bare ggml_rms_norm)."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_rms_norm_mul(_ref(desc(x)), _ref(desc(w)), float(eps), _ref(desc(out)), _stream()),
           "rms_norm_mul")
    return out


def add_rms_norm_mul(a, b, w, eps, out=None, sum_out=None, want_sum=True):
    """ggml_add(a, b) then rms_norm()*w; returns (sum or None, y)."""
    out = a.new_empty(a.shape) if out is None else out
    if sum_out is None and want_sum:
        sum_out = a.new_empty(a.shape)
    _check(load().shp_add_rms_norm_mul(_ref(desc(a)), _ref(desc(b)), _ref(desc(w)), float(eps), _ref(desc(sum_out)),
                                       _ref(desc(out)), _stream()), "add_rms_norm_mul")
    return sum_out, out


def rope_ext(x, pos, n_dims, mode, freq_base, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0, out=None):
    """ggml_rope_ext on x (T, heads, head_dim) with I32 positions (T,)."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_rope_ext(_ref(desc(x)), _ref(desc(pos)), int(n_dims), int(mode), float(freq_base),
                               float(freq_scale), float(ext_factor), float(attn_factor), _ref(desc(out)), _stream()),
           "rope_ext")
    return out


def qk_norm_rope(q, k, wq, wk, eps, pos, n_dims, freq_base, freq_scale=1.0, q_out=None, k_out=None):
    """Per-head rms_norm()*w then NEOX rope for q (T, H, hd) and k (T, KVH, hd)."""
    q_out = q.new_empty(q.shape) if q_out is None else q_out
    if k is not None and k_out is None:
        k_out = k.new_empty(k.shape)
    _check(load().shp_qk_norm_rope(_ref(desc(q)), _ref(desc(k)), _ref(desc(wq)), _ref(desc(wk)), float(eps),
                                   _ref(desc(pos)), int(n_dims), float(freq_base), float(freq_scale),
                                   _ref(desc(q_out)), _ref(desc(k_out)), _stream()), "qk_norm_rope")
    return q_out, k_out


def qk_norm_rope_kv(q, k, v, wq, wk, eps, pos, n_dims, freq_base, k_cache, v_cache, filled, freq_scale=1.0,
                    q_out=None):
    """qk_norm_rope plus the step's cache write: the rotated k and v land in rows
    [filled, filled + T) of k_cache / v_cache (T, ...) = torch (capacity, kv_heads,
    head_dim); returns q_out."""
    q_out = q.new_empty(q.shape) if q_out is None else q_out
    _check(load().shp_qk_norm_rope_kv(_ref(desc(q)), _ref(desc(k)), _ref(desc(v)), _ref(desc(wq)), _ref(desc(wk)),
                                      float(eps), _ref(desc(pos)), int(n_dims), float(freq_base), float(freq_scale),
                                      _ref(desc(q_out)), _ref(desc(k_cache)), _ref(desc(v_cache)), int(filled),
                                      _stream()), "qk_norm_rope_kv")
    return q_out


def qk_norm_rope_kv_at(q, k, v, wq, wk, eps, pos, n_dims, freq_base, k_cache, v_cache, slot, status=None,
                       freq_scale=1.0, q_out=None):
    """qk_norm_rope_kv with the first cache row read from the int32 device tensor
    `slot` when the kernel runs (graph-replayable); `status` (int32, one element)
    is set to 1 when the rows do not fit the cache."""
    q_out = q.new_empty(q.shape) if q_out is None else q_out
    _check(load().shp_qk_norm_rope_kv_at(_ref(desc(q)), _ref(desc(k)), _ref(desc(v)), _ref(desc(wq)), _ref(desc(wk)),
                                         float(eps), _ref(desc(pos)), int(n_dims), float(freq_base), float(freq_scale),
                                         _ref(desc(q_out)), _ref(desc(k_cache)), _ref(desc(v_cache)), _ref(desc(slot)),
                                         _ref(desc(status)), _stream()), "qk_norm_rope_kv_at")
    return q_out


def swiglu(g, u=None, out=None):
    """ggml_silu(g) then ggml_mul(., u) (u None: bare silu)."""
    out = g.new_empty(g.shape) if out is None else out
    _check(load().shp_swiglu(_ref(desc(g)), _ref(desc(u)), _ref(desc(out)), _stream()), "swiglu")
    return out


def glu_swiglu(a, swapped=False, out=None):
    """ggml_swiglu(a) / ggml_swiglu_swapped(a) on a (..., 2n) -> (..., n)."""
    out = a.new_empty(tuple(a.shape[:-1]) + (a.shape[-1] // 2,)) if out is None else out
    _check(load().shp_glu_swiglu(_ref(desc(a)), 1 if swapped else 0, _ref(desc(out)), _stream()), "glu_swiglu")
    return out


def snake(x, alpha, out=None):
    """Kokoro Snake on x (T, C) (ggml [C, T], channels fastest), alpha (C,)."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_snake(_ref(desc(x)), _ref(desc(alpha)), _ref(desc(out)), _stream()), "snake")
    return out


def snake_guarded(x, alpha, out=None):
    """codec_snake (omnivoice): x + sin(x*alpha)^2 / (alpha + 1e-9), x (T, C), alpha C values."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_snake_guarded(_ref(desc(x)), _ref(desc(alpha)), _ref(desc(out)), _stream()), "snake_guarded")
    return out


def snake_beta(x, log_alpha, log_beta, out=None):
    """codec_snake_beta (qwen3-tts): x + sin(x*exp(la))^2 / (exp(lb) + 1e-9), x (T, C)."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_snake_beta(_ref(desc(x)), _ref(desc(log_alpha)), _ref(desc(log_beta)), _ref(desc(out)),
                                 _stream()), "snake_beta")
    return out


def soft_max_ext(a, mask, scale, max_bias=0.0, out=None):
    """ggml_soft_max_ext over the last axis of a (..., ne1, ne0); mask None or
    (ne1', ne0) / (heads', ne1', ne0) broadcast as ggml does."""
    out = a.new_empty(a.shape) if out is None else out
    _check(load().shp_soft_max_ext(_ref(desc(a)), _ref(desc(mask)), float(scale), float(max_bias), _ref(desc(out)),
                                   _stream()), "soft_max_ext")
    return out


def exp(x, out=None):
    """ggml_exp."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_exp(_ref(desc(x)), _ref(desc(out)), _stream()), "exp")
    return out


def scale_bias(x, s, b=0.0, out=None):
    """ggml_scale_bias(x, s, b); b == 0 is ggml_scale(x, s)."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_scale_bias(_ref(desc(x)), float(s), float(b), _ref(desc(out)), _stream()), "scale_bias")
    return out


def sum_scale_leaky_relu(terms, scale, slope, out=None, mean_out=None, want_mean=False):
    """Branch average: leaky_relu((t0 + t1 + ...) * scale, slope); returns (mean or None, y)."""
    n = len(terms)
    arr = (ShpTensor * n)(*[desc(t) for t in terms])
    out = terms[0].new_empty(terms[0].shape) if out is None else out
    if mean_out is None and want_mean:
        mean_out = terms[0].new_empty(terms[0].shape)
    _check(load().shp_sum_scale_leaky_relu(arr, n, float(scale), float(slope), _ref(desc(mean_out)),
                                           _ref(desc(out)), _stream()), "sum_scale_leaky_relu")
    return mean_out, out


def add_leaky_relu(a, b, slope, out=None, sum_out=None, want_sum=False):
    """ggml_add(a, b) then ggml_leaky_relu(., slope); returns (sum or None, y)."""
    out = a.new_empty(a.shape) if out is None else out
    if sum_out is None and want_sum:
        sum_out = a.new_empty(a.shape)
    _check(load().shp_add_leaky_relu(_ref(desc(a)), _ref(desc(b)), float(slope), _ref(desc(sum_out)),
                                     _ref(desc(out)), _stream()), "add_leaky_relu")
    return sum_out, out


def leaky_relu(a, slope, out=None):
    return add_leaky_relu(a, None, slope, out=out)[1]


def add(a, b, out=None):
    """ggml_add(a, b), b of a's shape or any shape that repeats to it
    (ggml_can_repeat: each ggml extent of b divides a's)."""
    out = a.new_empty(a.shape) if out is None else out
    _check(load().shp_add(_ref(desc(a)), _ref(desc(b)), _ref(desc(out)), _stream()), "add")
    return out


LAYER_OUTPUTS = ("normed", "q_out", "k_out", "resid", "mlp_in", "act", "out")


def layer_nongemm_step(x, w_in, q, k, wq, wk, pos, attn_out, w_post, gate, up, mlp_out, eps, n_dims, freq_base,
                       outs=None):
    """The non-GEMM node runs of one Qwen3 decoder layer
    (src/arch/qwen3-tts/operations.cpp:84-147) in one call: x, attn_out, mlp_out
    (T, hidden); q (T, heads, hd); k (T, kv_heads, hd); gate, up (T, ffn); pos
    int32 (T,). Returns a dict of the outputs named in LAYER_OUTPUTS (`outs`
    may supply any of them)."""
    outs = dict(outs or {})
    like = {"normed": x, "q_out": q, "k_out": k, "resid": x, "mlp_in": x, "act": gate, "out": x}
    for name in LAYER_OUTPUTS:
        if outs.get(name) is None:
            outs[name] = like[name].new_empty(like[name].shape)
    ins = dict(x=x, w_in=w_in, q=q, k=k, wq=wq, wk=wk, pos=pos, attn_out=attn_out, w_post=w_post, gate=gate, up=up,
               mlp_out=mlp_out)
    descs = {n: desc(t) for n, t in list(ins.items()) + list(outs.items())}
    step = ShpLayerStep()
    for n, d in descs.items():
        setattr(step, n, ctypes.pointer(d) if d is not None else None)
    step.eps, step.freq_base, step.n_dims, step.reserved = float(eps), float(freq_base), int(n_dims), 0
    _check(load().shp_layer_nongemm_step(ctypes.byref(step), _stream()), "layer_nongemm_step")
    return outs


def mul(a, b, out=None):
    """ggml_mul(a, b), b as in add."""
    out = a.new_empty(a.shape) if out is None else out
    _check(load().shp_mul(_ref(desc(a)), _ref(desc(b)), _ref(desc(out)), _stream()), "mul")
    return out


def div(a, b, out=None):
    """ggml_div(a, b), b as in add."""
    out = a.new_empty(a.shape) if out is None else out
    _check(load().shp_div(_ref(desc(a)), _ref(desc(b)), _ref(desc(out)), _stream()), "div")
    return out


def sin(x, out=None):
    """ggml_sin."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_sin(_ref(desc(x)), _ref(desc(out)), _stream()), "sin")
    return out


def sqr(x, out=None):
    """ggml_sqr."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_sqr(_ref(desc(x)), _ref(desc(out)), _stream()), "sqr")
    return out


def cont_add_leaky_relu(x, b, r=None, slope=None, out=None, sum_out=None):
    """s = ggml_cont(x) + b (+ r), y = leaky_relu(s, slope) when slope is not
    None (sum_out receives s), else y = s; x a transposed F32 view, b one
    value per row of y. Returns y."""
    import torch
    out = torch.empty(x.shape, dtype=torch.float32, device=x.device) if out is None else out
    leaky = slope is not None
    _check(load().shp_cont_add_leaky_relu(_ref(desc(x)), _ref(desc(b)), _ref(desc(r)), int(leaky),
                                          float(slope if leaky else 0.0), _ref(desc(sum_out)), _ref(desc(out)),
                                          _stream()), "cont_add_leaky_relu")
    return out


def sub(a, b, out=None):
    """ggml_sub(a, b), b as in add."""
    out = a.new_empty(a.shape) if out is None else out
    _check(load().shp_sub(_ref(desc(a)), _ref(desc(b)), _ref(desc(out)), _stream()), "sub")
    return out


def _unary_call(name, x, out):
    out = x.new_empty(x.shape) if out is None else out
    _check(getattr(load(), "shp_" + name)(_ref(desc(x)), _ref(desc(out)), _stream()), name)
    return out


def tanh(x, out=None):
    """ggml_tanh."""
    return _unary_call("tanh", x, out)


def sigmoid(x, out=None):
    """ggml_sigmoid."""
    return _unary_call("sigmoid", x, out)


def elu(x, out=None):
    """ggml_elu."""
    return _unary_call("elu", x, out)


def gelu_erf(x, out=None):
    """ggml_gelu_erf."""
    return _unary_call("gelu_erf", x, out)


def relu(x, out=None):
    """ggml_relu."""
    return _unary_call("relu", x, out)


def neg(x, out=None):
    """ggml_neg."""
    return _unary_call("neg", x, out)


def step(x, out=None):
    """ggml_step."""
    return _unary_call("step", x, out)


def sqrt(x, out=None):
    """ggml_sqrt."""
    return _unary_call("sqrt", x, out)


def _row_sums(name, x, w, out):
    import torch
    out = torch.empty(tuple(x.shape[:-1]) + (1,), dtype=torch.float32, device=x.device) if out is None else out
    args = [_ref(desc(x))] + ([_ref(desc(w))] if w is not None else []) + [_ref(desc(out)), _stream()]
    _check(getattr(load(), "shp_" + name)(*args), name)
    return out


def sum_rows(x, out=None):
    """ggml_sum_rows: (..., ne0) -> (..., 1)."""
    return _row_sums("sum_rows", x, None, out)


def mean(x, out=None):
    """ggml_mean: (..., ne0) -> (..., 1)."""
    return _row_sums("mean", x, None, out)


def mul_sum_rows(x, w, out=None):
    """ggml_mul(x, w) then ggml_sum_rows, one launch."""
    return _row_sums("mul_sum_rows", x, w, out)


def diag_mask_inf(x, n_past, out=None):
    """ggml_diag_mask_inf(x, n_past); out=x for the inplace form."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_diag_mask_inf(_ref(desc(x)), int(n_past), _ref(desc(out)), _stream()), "diag_mask_inf")
    return out


def soft_max_causal(x, n_past, scale, out=None):
    """ggml_diag_mask_inf(x, n_past) then ggml_soft_max_ext(., NULL, scale, 0), one launch."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_soft_max_causal(_ref(desc(x)), int(n_past), float(scale), _ref(desc(out)), _stream()),
           "soft_max_causal")
    return out


def inverse_stft(spectrum, n_fft, hop, out=None):
    """Kokoro's inverse_stft: spectrum (frames, n_fft + 2) -> ((frames - 1) * hop,)."""
    import torch
    frames = spectrum.shape[0]
    out = torch.empty(((frames - 1) * hop,), dtype=torch.float32, device=spectrum.device) if out is None else out
    _check(load().shp_inverse_stft(_ref(desc(spectrum)), int(n_fft), int(hop), _ref(desc(out)), _stream()),
           "inverse_stft")
    return out


def harmonic_source(f0, merge_weight, merge_bias, rand_ini, noise, *, rate, scale, sine_amp, noise_std,
                    voiced_threshold, n_fft, hop, out=None):
    """Kokoro's build_harmonic_source: f0 (L,), merge_weight and rand_ini (H,),
    noise (L*scale, H) -> (excitation (L*scale,), spectrum (frames, n_fft + 2))."""
    import torch
    U = f0.numel() * scale
    frames = U // hop + 1
    if out is None:
        out = (torch.empty((U,), dtype=torch.float32, device=f0.device),
               torch.empty((frames, n_fft + 2), dtype=torch.float32, device=f0.device))
    exc, har = out
    _check(load().shp_harmonic_source(_ref(desc(f0)), _ref(desc(merge_weight)), float(merge_bias), _ref(desc(rand_ini)),
                                      _ref(desc(noise)), int(rate), int(scale), float(sine_amp), float(noise_std),
                                      float(voiced_threshold), int(n_fft), int(hop), _ref(desc(exc)), _ref(desc(har)),
                                      _stream()), "harmonic_source")
    return exc, har


def mel_filterbank(sample_rate, n_fft, mel_bins, fmin, fmax):
    """The Slaney filterbank (host code): a numpy (mel_bins, n_fft/2 + 1) f32 array."""
    import numpy as np
    out = np.empty((mel_bins, n_fft // 2 + 1), np.float32)
    _check(load().shp_mel_filterbank(int(sample_rate), int(n_fft), int(mel_bins), float(fmin), float(fmax),
                                     out.ctypes.data_as(ctypes.c_void_p)), "mel_filterbank")
    return out


def log_mel(pcm, filterbank, n_fft, hop, win_length, out=None):
    """The speaker encoder's log-mel: pcm (samples,), filterbank (mel_bins,
    n_fft/2 + 1) on the device -> (frames, mel_bins)."""
    import torch
    pad = (n_fft - hop) // 2
    frames = 1 + (pcm.numel() + 2 * pad - n_fft) // hop
    out = torch.empty((max(frames, 1), filterbank.shape[0]), dtype=torch.float32, device=pcm.device) if out is None \
        else out
    _check(load().shp_log_mel(_ref(desc(pcm)), _ref(desc(filterbank)), int(n_fft), int(hop), int(win_length),
                              _ref(desc(out)), _stream()), "log_mel")
    return out


def clamp(x, lo, hi, out=None):
    """ggml_clamp(x, lo, hi)."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_clamp(_ref(desc(x)), float(lo), float(hi), _ref(desc(out)), _stream()), "clamp")
    return out


def norm(x, eps, out=None):
    """ggml_norm(x, eps)."""
    out = x.new_empty(x.shape) if out is None else out
    _check(load().shp_norm(_ref(desc(x)), float(eps), _ref(desc(out)), _stream()), "norm")
    return out


def concat(a, b, dim, out=None):
    """ggml_concat(a, b, dim) (dim a ggml dimension)."""
    import torch
    ax = a.dim() - 1 - dim
    shape = list(a.shape)
    shape[ax] += b.shape[ax]
    out = torch.empty(shape, dtype=torch.float32, device=a.device) if out is None else out
    _check(load().shp_concat(_ref(desc(a)), _ref(desc(b)), int(dim), _ref(desc(out)), _stream()), "concat")
    return out


def conv_out_len(iw, k, s0, p0, d0):
    """ggml_calc_conv_output_size: (iw + 2*p0 - d0*(k-1) - 1)/s0 + 1, C division."""
    num = iw + 2 * p0 - d0 * (k - 1) - 1
    return (num // s0 if num >= 0 else -((-num) // s0)) + 1


def kernel_shape(k, ic, oc=1):
    """A shape-only kernel descriptor [k, ic, oc] (no data), as ggml_im2col reads
    its kernel operand."""
    d = ShpTensor()
    d.type, d.reserved, d.data = TYPE_F32, 0, None
    for i, n in enumerate((k, ic, oc, 1)):
        d.ne[i] = n
    d.nb[0] = 4
    for i in range(1, 4):
        d.nb[i] = d.nb[i - 1] * d.ne[i - 1]
    return d


def im2col(x, k, s0=1, p0=0, d0=1, dtype=None, out=None):
    """ggml_im2col(kernel [k, IC], x, s0, 0, p0, 0, d0, 0, false, dtype): x a
    torch F32 tensor (N, IC, IW) or (IC, IW) = ggml [IW, IC, N], any strides;
    returns (N, OW, IC*k) of dtype (float32 or float16)."""
    import torch
    if out is None:
        n_, ic, iw = (1,) + tuple(x.shape) if x.dim() == 2 else tuple(x.shape)
        ow = conv_out_len(iw, k, s0, p0, d0)
        out = torch.empty((n_, max(ow, 1), ic * k), dtype=dtype or torch.float32, device=x.device)
    ic = x.shape[-2]
    _check(load().shp_im2col(ctypes.byref(kernel_shape(k, ic)), _ref(desc(x)), int(s0), int(p0), int(d0),
                             _ref(desc(out)), _stream()), "im2col")
    return out


def col2im_1d(cols, stride, out_channels, padding=0, out=None):
    """ggml_col2im_1d(cols, stride, out_channels, padding): cols a torch F32
    tensor (L, K*OC) = ggml [K*OC, L]; returns (OC, T) = ggml [T, OC]."""
    import torch
    L, ko = cols.shape
    t = (L - 1) * stride + ko // out_channels - 2 * padding
    out = torch.empty((out_channels, max(t, 1)), dtype=torch.float32, device=cols.device) if out is None else out
    _check(load().shp_col2im_1d(_ref(desc(cols)), int(stride), int(out_channels), int(padding), _ref(desc(out)),
                                _stream()), "col2im_1d")
    return out


def pad_ext(x, lp, rp, out=None):
    """ggml_pad_ext(x, lp0, rp0, ...): lp, rp per ggml dimension (up to 4)."""
    import torch
    lp = list(lp) + [0] * (4 - len(lp))
    rp = list(rp) + [0] * (4 - len(rp))
    if out is None:
        ne = list(x.shape[::-1]) + [1] * (4 - x.dim())
        nd = max(x.dim(), max([d + 1 for d in range(4) if lp[d] or rp[d]] + [1]))
        out = torch.empty([ne[d] + lp[d] + rp[d] for d in range(nd)][::-1], dtype=torch.float32, device=x.device)
    _check(load().shp_pad(_ref(desc(x)), (ctypes.c_int32 * 4)(*lp), _ref(desc(out)), _stream()), "pad")
    return out


def pad_reflect_1d(x, p0, p1, out=None):
    """ggml_pad_reflect_1d(x, p0, p1)."""
    import torch
    out = torch.empty(tuple(x.shape[:-1]) + (x.shape[-1] + p0 + p1,), dtype=torch.float32,
                      device=x.device) if out is None else out
    _check(load().shp_pad_reflect_1d(_ref(desc(x)), int(p0), int(p1), _ref(desc(out)), _stream()), "pad_reflect_1d")
    return out


def repeat(x, shape, out=None):
    """ggml_repeat(x, a tensor of torch shape `shape`)."""
    import torch
    out = torch.empty(tuple(shape), dtype=torch.float32, device=x.device) if out is None else out
    _check(load().shp_repeat(_ref(desc(x)), _ref(desc(out)), _stream()), "repeat")
    return out


def acc(a, b, nb1, nb2, nb3, offset, out=None, inplace=False):
    """ggml_acc(a, b, nb1, nb2, nb3, offset): a with b added into the view at
    byte `offset` with byte strides nb1..nb3 (b's extents). inplace: into a
    itself (ggml's inplace form)."""
    import torch
    if inplace:
        out = a
    elif out is None:
        out = torch.empty(a.shape, dtype=torch.float32, device=a.device)
    _check(load().shp_acc(_ref(desc(a)), _ref(desc(b)), int(nb1), int(nb2), int(nb3), int(offset), _ref(desc(out)),
                          _stream()), "acc")
    return out


def cpy(x, out=None):
    """ggml_cpy / ggml_cast into F32 of x's shape (x F32, F16 or BF16)."""
    import torch
    out = torch.empty(x.shape, dtype=torch.float32, device=x.device) if out is None else out
    _check(load().shp_cpy(_ref(desc(x)), _ref(desc(out)), _stream()), "cpy")
    return out


# ---------------------------------------------------------------------------
# node-run executor (include/synth_graph.h)
# ---------------------------------------------------------------------------

(NODE_NOP, NODE_ADD, NODE_MUL, NODE_DIV, NODE_SQR, NODE_SIN, NODE_SCALE, NODE_CPY, NODE_GET_ROWS, NODE_RMS_NORM,
 NODE_SOFT_MAX, NODE_ROPE, NODE_LEAKY_RELU, NODE_SILU, NODE_EXP, NODE_GLU_SWIGLU, NODE_CONCAT, NODE_SUB, NODE_TANH,
 NODE_SIGMOID, NODE_ELU, NODE_GELU_ERF, NODE_CLAMP, NODE_NORM, NODE_IM2COL, NODE_COL2IM_1D, NODE_PAD,
 NODE_PAD_REFLECT_1D, NODE_REPEAT, NODE_ACC, NODE_RELU, NODE_NEG, NODE_STEP, NODE_SQRT, NODE_SUM_ROWS,
 NODE_MEAN, NODE_DIAG_MASK_INF) = range(37)
NODE_FLAG_OUTPUT = 1
RUN_KINDS = {-1: "unsupported", 0: "nop", 1: "single", 2: "norm_mul", 3: "norm_mul_rope", 4: "add_norm_mul",
             5: "silu_mul", 6: "add_leaky", 7: "add_scale_leaky", 8: "snake", 9: "snake_guarded", 10: "snake_beta",
             11: "gather_sum", 12: "qk_norm_rope", 13: "qk_norm_rope_kv", 14: "cont_add_leaky",
             15: "view_binary", 16: "cont_im2col", 17: "mul_sum_rows", 18: "diag_mask_soft_max"}


class ShpNode(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int32), ("flags", ctypes.c_uint32), ("src_node", ctypes.c_int32 * 3),
                ("uses", ctypes.c_int32), ("op_params", ctypes.c_int32 * 16), ("dst", ShpTensor),
                ("src", ShpTensor * 3)]


class ShpGraphRun(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("first", ctypes.c_int32), ("last", ctypes.c_int32),
                ("nodes", ctypes.c_int32)]


class GVal:
    """A tensor of a Graph: `t` (torch tensor or BlockTensor) and the node that
    computes it (None for a leaf: weights, inputs, outputs of other graphs)."""

    def __init__(self, t, node=None):
        self.t, self.node = t, node


def _f32_bits(v):
    import struct
    return struct.unpack("<i", struct.pack("<f", float(v)))[0]


class Graph:
    """A ggml-style graph over torch tensors, run by shp_graph_compute.

    Each op method mirrors the ggml constructor of the same name: it appends a
    node, allocates the node's F32 result on the device of its first operand
    and returns it as a GVal. order() lists the nodes reachable from the given
    results as ggml_build_forward_expand does (depth first, src[0] first, each
    node once), which is the order a ggml backend receives them in; compute()
    runs that list, plan() shows the runs the executor splits it into."""

    def __init__(self):
        self._outputs = []

    @staticmethod
    def _v(x):
        return x if isinstance(x, GVal) or x is None else GVal(x)

    @staticmethod
    def _t(x):
        return x.t if isinstance(x, GVal) else x

    def _op(self, op, dst, srcs, ints=None, floats=None):
        params = [0] * 16
        for k, v in (ints or {}).items():
            params[k] = int(v)
        for k, v in (floats or {}).items():
            params[k] = _f32_bits(v)
        node = {"op": op, "srcs": [self._v(s) for s in srcs], "params": params}
        val = GVal(dst, node)
        node["val"] = val
        return val

    def _like(self, x, shape=None):
        import torch
        t = self._t(x)
        raw = t.data if isinstance(t, BlockTensor) else t
        return torch.empty(tuple(t.shape) if shape is None else shape, dtype=torch.float32, device=raw.device)

    # binary and unary nodes -------------------------------------------------
    def add(self, a, b):
        return self._op(NODE_ADD, self._like(a), [a, b])

    def mul(self, a, b):
        return self._op(NODE_MUL, self._like(a), [a, b])

    def div(self, a, b):
        return self._op(NODE_DIV, self._like(a), [a, b])

    def sqr(self, x):
        return self._op(NODE_SQR, self._like(x), [x])

    def sin(self, x):
        return self._op(NODE_SIN, self._like(x), [x])

    def silu(self, x):
        return self._op(NODE_SILU, self._like(x), [x])

    def exp(self, x):
        return self._op(NODE_EXP, self._like(x), [x])

    def scale(self, x, s):
        return self._op(NODE_SCALE, self._like(x), [x], floats={0: s, 1: 0.0})

    def scale_bias(self, x, s, b):
        return self._op(NODE_SCALE, self._like(x), [x], floats={0: s, 1: b})

    def leaky_relu(self, x, slope):
        return self._op(NODE_LEAKY_RELU, self._like(x), [x], floats={0: slope})

    def rms_norm(self, x, eps):
        return self._op(NODE_RMS_NORM, self._like(x), [x], floats={0: eps})

    def rope_ext(self, x, pos, n_dims, mode, freq_base, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0):
        return self._op(NODE_ROPE, self._like(x), [x, pos], ints={1: n_dims, 2: mode},
                        floats={5: freq_base, 6: freq_scale, 7: ext_factor, 8: attn_factor})

    def soft_max_ext(self, x, mask, scale, max_bias=0.0):
        return self._op(NODE_SOFT_MAX, self._like(x), [x, mask], floats={0: scale, 1: max_bias})

    def get_rows(self, table, ids):
        t = self._t(table)
        ne0 = t.ne0 if isinstance(t, BlockTensor) else t.shape[-1]
        return self._op(NODE_GET_ROWS, self._like(ids, tuple(self._t(ids).shape) + (ne0,)), [table, ids])

    def cast(self, x):
        """ggml_cast(x, F32)."""
        return self._op(NODE_CPY, self._like(x), [x])

    def cpy(self, x, dst):
        """ggml_cpy(x, dst): dst a torch tensor (a view of a cache, say)."""
        return self._op(NODE_CPY, dst, [x])

    def cont(self, x):
        """ggml_cont(x): x (typically a permuted view) copied into a new
        contiguous tensor of its shape; the same node kind as ggml_cpy."""
        return self._op(NODE_CPY, self._like(x), [x])

    def sub(self, a, b):
        return self._op(NODE_SUB, self._like(a), [a, b])

    def tanh(self, x):
        return self._op(NODE_TANH, self._like(x), [x])

    def sigmoid(self, x):
        return self._op(NODE_SIGMOID, self._like(x), [x])

    def elu(self, x):
        return self._op(NODE_ELU, self._like(x), [x])

    def gelu_erf(self, x):
        return self._op(NODE_GELU_ERF, self._like(x), [x])

    def relu(self, x):
        return self._op(NODE_RELU, self._like(x), [x])

    def neg(self, x):
        return self._op(NODE_NEG, self._like(x), [x])

    def step(self, x):
        return self._op(NODE_STEP, self._like(x), [x])

    def sqrt(self, x):
        return self._op(NODE_SQRT, self._like(x), [x])

    def diag_mask_inf(self, x, n_past, inplace=False):
        return self._op(NODE_DIAG_MASK_INF, self._t(x) if inplace else self._like(x), [x], ints={0: n_past})

    def sum_rows(self, x):
        t = self._t(x)
        return self._op(NODE_SUM_ROWS, self._like(x, tuple(t.shape[:-1]) + (1,)), [x])

    def mean(self, x):
        t = self._t(x)
        return self._op(NODE_MEAN, self._like(x, tuple(t.shape[:-1]) + (1,)), [x])

    def clamp(self, x, lo, hi):
        return self._op(NODE_CLAMP, self._like(x), [x], floats={0: lo, 1: hi})

    def norm(self, x, eps):
        return self._op(NODE_NORM, self._like(x), [x], floats={0: eps})

    def concat(self, a, b, dim):
        """ggml_concat(a, b, dim) (dim a ggml dimension)."""
        import torch
        ta, tb = self._t(a), self._t(b)
        ax = ta.dim() - 1 - dim
        shape = list(ta.shape)
        shape[ax] += tb.shape[ax]
        return self._op(NODE_CONCAT, torch.empty(shape, dtype=torch.float32, device=ta.device), [a, b],
                        ints={0: dim})

    def im2col(self, kernel, x, s0=1, p0=0, d0=1, dtype=None):
        """ggml_im2col(kernel, x, s0, 0, p0, 0, d0, 0, false, dtype): kernel a
        torch tensor (OC, IC, K) = ggml [K, IC, OC] (only its extents are
        read), x (N, IC, IW) or (IC, IW); the result (N, OW, IC*K)."""
        import torch
        k, ic = self._t(kernel).shape[-1], self._t(kernel).shape[-2]
        t = self._t(x)
        n_, iw = (t.shape[0] if t.dim() == 3 else 1), t.shape[-1]
        ow = conv_out_len(iw, k, s0, p0, d0)
        dst = torch.empty((n_, max(ow, 1), ic * k), dtype=dtype or torch.float32, device=t.device)
        return self._op(NODE_IM2COL, dst, [kernel, x], ints={0: s0, 2: p0, 4: d0})

    def col2im_1d(self, cols, stride, out_channels, padding=0):
        """ggml_col2im_1d: cols (L, K*OC) = ggml [K*OC, L]; the result (OC, T)."""
        import torch
        t = self._t(cols)
        L, ko = t.shape
        n = (L - 1) * stride + ko // out_channels - 2 * padding
        dst = torch.empty((out_channels, max(n, 1)), dtype=torch.float32, device=t.device)
        return self._op(NODE_COL2IM_1D, dst, [cols], ints={0: stride, 1: out_channels, 2: padding})

    def pad_ext(self, x, lp, rp):
        """ggml_pad_ext (ggml_pad: lp all 0)."""
        import torch
        t = self._t(x)
        lp = list(lp) + [0] * (4 - len(lp))
        rp = list(rp) + [0] * (4 - len(rp))
        ne = list(t.shape[::-1]) + [1] * (4 - t.dim())
        nd = max(t.dim(), max([d + 1 for d in range(4) if lp[d] or rp[d]] + [1]))
        dst = torch.empty([ne[d] + lp[d] + rp[d] for d in range(nd)][::-1], dtype=torch.float32, device=t.device)
        return self._op(NODE_PAD, dst, [x], ints={2 * d + k: (lp, rp)[k][d] for d in range(4) for k in range(2)})

    def pad(self, x, p):
        return self.pad_ext(x, [0, 0, 0, 0], p)

    def pad_reflect_1d(self, x, p0, p1):
        t = self._t(x)
        return self._op(NODE_PAD_REFLECT_1D, self._like(x, tuple(t.shape[:-1]) + (t.shape[-1] + p0 + p1,)), [x],
                        ints={0: p0, 1: p1})

    def repeat(self, x, shape):
        return self._op(NODE_REPEAT, self._like(x, tuple(shape)), [x])

    def acc(self, a, b, nb1, nb2, nb3, offset, inplace=False):
        """ggml_acc (byte strides and offset of the view of a's copy; inplace:
        the result is a's own memory)."""
        t = self._t(a)
        dst = t if inplace else self._like(a)
        return self._op(NODE_ACC, dst, [a, b], ints={0: nb1, 1: nb2, 2: nb3, 3: offset, 4: 1 if inplace else 0})

    def glu_swiglu(self, a, b=None, swapped=False):
        t = self._t(a)
        shape = tuple(t.shape) if b is not None else tuple(t.shape[:-1]) + (t.shape[-1] // 2,)
        return self._op(NODE_GLU_SWIGLU, self._like(a, shape), [a, b], ints={1: 1 if swapped else 0})

    @staticmethod
    def read_later(v, uses):
        """Declares that v is read `uses` times in the whole graph (ggml's use
        count), some of them by nodes outside this list (a later split)."""
        v.node["uses"] = int(uses)
        return v

    def view(self, x, t):
        """A view-like node (ggml_view/reshape/permute): `t` is the torch view of x's memory."""
        return self._op(NODE_NOP, t, [x])

    # ordering and running ---------------------------------------------------
    def order(self, *outputs):
        """The nodes reachable from `outputs`, in ggml_build_forward_expand order."""
        seen, out = set(), []
        for o in outputs:
            stack = [(o, False)]
            while stack:
                v, done = stack.pop()
                n = v.node if isinstance(v, GVal) else None
                if n is None:
                    continue
                if done:
                    out.append(n)
                    continue
                if id(n) in seen:
                    continue
                seen.add(id(n))
                stack.append((v, True))
                for s in reversed(n["srcs"]):
                    if s is not None:
                        stack.append((s, False))
        return out

    def nodes(self, *outputs, flag_outputs=True):
        """The shp_node array for order(*outputs); the results in `outputs`
        carry SHP_NODE_FLAG_OUTPUT. Returns (array, keep-alive list)."""
        order = self.order(*outputs)
        index = {id(n): i for i, n in enumerate(order)}
        outs = {id(o.node) for o in outputs if isinstance(o, GVal) and o.node is not None}
        arr = (ShpNode * max(1, len(order)))()
        keep = []
        for i, n in enumerate(order):
            c = arr[i]
            c.op = n["op"]
            c.flags = NODE_FLAG_OUTPUT if flag_outputs and id(n) in outs else 0
            c.uses = n.get("uses", 0)
            for k in range(16):
                c.op_params[k] = n["params"][k]
            c.dst = desc(n["val"].t)
            for k in range(3):
                c.src_node[k] = -1
                s = n["srcs"][k] if k < len(n["srcs"]) else None
                if s is not None:
                    c.src[k] = desc(s.t)
                    if s.node is not None:
                        c.src_node[k] = index[id(s.node)]
            keep.append(n)
        return arr, len(order), keep

    def plan(self, *outputs):
        """[(run kind, first node, last node, nodes executed)] for order(*outputs)."""
        arr, n, _ = self.nodes(*outputs)
        count = ctypes.c_int32()
        _check(load().shp_graph_plan(arr, n, None, 0, ctypes.byref(count)), "graph_plan")
        runs = (ShpGraphRun * max(1, count.value))()
        _check(load().shp_graph_plan(arr, n, runs, count.value, ctypes.byref(count)), "graph_plan")
        return [(RUN_KINDS[r.kind], r.first, r.last, r.nodes) for r in runs[:count.value]]

    def compute(self, *outputs):
        arr, n, _ = self.nodes(*outputs)
        _check(load().shp_graph_compute(arr, n, _stream()), "graph_compute")
        return outputs[0] if len(outputs) == 1 else outputs


# ---------------------------------------------------------------------------
# GGUF packages (include/synth_gguf.h)
# ---------------------------------------------------------------------------

class GgufFile:
    """A GGUF package opened by libsynth_hip's reader. info() and the metadata
    getters run host code only; load() streams a tensor into a new device
    buffer and returns it as a torch tensor (or BlockTensor) the gathers take."""

    def __init__(self, path):
        self._h = ctypes.c_void_p()
        _check(load().shp_gguf_open(os.fsencode(path), ctypes.byref(self._h)), "gguf_open")

    def close(self):
        if self._h:
            load().shp_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def version(self):
        return int(load().shp_gguf_version(self._h))

    def tensor_names(self):
        L = load()
        # names are UTF-8 by the format; undecodable bytes round-trip through surrogateescape
        return [L.shp_gguf_tensor_name(self._h, i).decode("utf-8", "surrogateescape")
                for i in range(L.shp_gguf_tensor_count(self._h))]

    def info(self, name):
        """(shp_tensor with data NULL, nbytes, absolute file offset)."""
        d, nbytes, off = ShpTensor(), ctypes.c_uint64(), ctypes.c_uint64()
        _check(load().shp_gguf_tensor_info(self._h, name.encode("utf-8", "surrogateescape"), ctypes.byref(d),
                                           ctypes.byref(nbytes),
                                           ctypes.byref(off)), "gguf_tensor_info")
        return d, int(nbytes.value), int(off.value)

    def kv_u32(self, key):
        v = ctypes.c_uint32()
        _check(load().shp_gguf_kv_u32(self._h, key.encode(), ctypes.byref(v)), "gguf_kv_u32")
        return int(v.value)

    def kv_string(self, key, capacity=4096):
        buf = ctypes.create_string_buffer(capacity)
        _check(load().shp_gguf_kv_string(self._h, key.encode(), buf, capacity), "gguf_kv_string")
        return buf.value.decode()

    def load(self, name, device="cuda"):
        import torch
        d, nbytes, _ = self.info(name)
        raw = torch.empty(nbytes, dtype=torch.uint8, device=device)
        out = ShpTensor()
        _check(load().shp_gguf_load_tensor(self._h, name.encode("utf-8", "surrogateescape"),
                                           ctypes.c_void_p(raw.data_ptr()), nbytes,
                                           ctypes.byref(out), _stream()), "gguf_load_tensor")
        return _typed_view(raw, out)

    def load_many(self, names, device="cuda"):
        """Several tensors in one pass (shp_gguf_load_tensors), in the order of
        `names`; each as load() returns it."""
        import torch
        names = list(names)
        raws = [torch.empty(self.info(n)[1], dtype=torch.uint8, device=device) for n in names]
        n = len(names)
        descs = (ShpTensor * max(n, 1))()
        _check(load().shp_gguf_load_tensors(
            self._h, (ctypes.c_char_p * max(n, 1))(*[x.encode("utf-8", "surrogateescape") for x in names]), n,
            (ctypes.c_void_p * max(n, 1))(*[r.data_ptr() for r in raws]),
            (ctypes.c_size_t * max(n, 1))(*[r.numel() for r in raws]), descs, _stream()), "gguf_load_tensors")
        return [_typed_view(r, descs[i]) for i, r in enumerate(raws)]


def _typed_view(raw, desc):
    """A loaded tensor's device bytes as the torch tensor (or BlockTensor) its
    descriptor names."""
    import torch
    ne = [int(desc.ne[k]) for k in range(4)]
    nd = max([k + 1 for k in range(4) if ne[k] != 1] or [1])
    for cls in (Q8Tensor, Q5KTensor):
        if desc.type == cls.TYPE:
            rows = ne[1] * ne[2] * ne[3]
            return cls(raw.view(rows, ne[0] // cls.ELEMS * cls.BYTES), ne[0])
    dt = {TYPE_F32: torch.float32, TYPE_F16: torch.float16, TYPE_BF16: torch.bfloat16,
          TYPE_I32: torch.int32}[desc.type]
    return raw.view(dt).view(tuple(reversed(ne[:nd])))


def table_type_for_profile(profile):
    """The table type the catalog requires under a quantization profile
    (ShpError(ERR_INVALID_ARG) for an unknown profile)."""
    t = ctypes.c_int32()
    _check(load().shp_table_type_for_profile(profile.encode(), ctypes.byref(t)), "table_type_for_profile")
    return int(t.value)

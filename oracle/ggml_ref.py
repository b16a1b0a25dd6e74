"""TEST INFRASTRUCTURE ONLY: Python face of the ggml-CPU restatement.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker or the timed CPU baseline. The product
(libsynth_hip and its binding) never imports it.

The arithmetic of every hot-path op lives in ggml_cpu_ref.c (built into
libggml_cpu_ref.so by oracle/Makefile). This module builds node lists for it in
the order the reference graph builders emit them, and adds what the tiny golden
configurations also need around the hot ops (mul_mat, soft_max_ext, the KV
cache), written with numpy.

Layout: a ggml tensor [ne0, ne1, ne2] is a C-contiguous numpy array of shape
(ne2, ne1, ne0); e.g. a Qwen3 activation [hidden, T] is np.float32 (T, hidden).
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libggml_cpu_ref.so")

F32, F16, Q8_0, Q5_K, I32, BF16 = 0, 1, 8, 13, 26, 30

(OP_ADD, OP_MUL, OP_DIV, OP_RMS_NORM, OP_ROPE_NEOX, OP_SILU, OP_SIN, OP_SQR, OP_EXP, OP_LEAKY_RELU, OP_SCALE_BIAS,
 OP_GET_ROWS, OP_CAST_F32, OP_GLU_SWIGLU, OP_SOFT_MAX, OP_CONT_F32, OP_BINBCAST, OP_SUB, OP_TANH, OP_SIGMOID,
 OP_ELU, OP_GELU_ERF, OP_CLAMP, OP_NORM, OP_IM2COL, OP_COL2IM_1D, OP_PAD, OP_PAD_REFLECT_1D,
 OP_REPEAT, OP_ACC, OP_RELU, OP_NEG, OP_STEP, OP_SQRT, OP_SUM_ROWS, OP_MEAN, OP_DIAG_MASK_INF,
 OP_ISTFT, OP_HARMONIC_SOURCE, OP_LOG_MEL) = range(1, 41)


class OrcNode(ctypes.Structure):
    _fields_ = [
        ("op", ctypes.c_int32), ("type0", ctypes.c_int32),
        ("ne0", ctypes.c_int64), ("nrows", ctypes.c_int64), ("ne1", ctypes.c_int64),
        ("src1_rows", ctypes.c_int64), ("src1_ne0", ctypes.c_int64),
        ("src0", ctypes.c_void_p), ("src1", ctypes.c_void_p), ("dst", ctypes.c_void_p),
        ("f", ctypes.c_float * 4), ("i", ctypes.c_int32 * 4),
    ]


class OrcSourceArgs(ctypes.Structure):
    _fields_ = [
        ("merge_weight", ctypes.c_void_p), ("rand_ini", ctypes.c_void_p), ("noise", ctypes.c_void_p),
        ("har", ctypes.c_void_p), ("merge_bias", ctypes.c_float), ("sine_amp", ctypes.c_float),
        ("noise_std", ctypes.c_float), ("voiced_threshold", ctypes.c_float), ("sampling_rate", ctypes.c_int32),
        ("harmonics", ctypes.c_int32), ("scale", ctypes.c_int32), ("n_fft", ctypes.c_int32), ("hop", ctypes.c_int32),
        ("pad", ctypes.c_int32),
    ]


_lib = None


def mel_filterbank(sample_rate, n_fft, mel_bins, fmin, fmax):
    """The restated Slaney filterbank, (mel_bins, n_fft/2 + 1) f32."""
    out = np.empty((mel_bins, n_fft // 2 + 1), np.float32)
    lib().orc_mel_filterbank(int(sample_rate), int(n_fft), int(mel_bins), float(fmin), float(fmax), _ptr(out))
    return out


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("oracle not built: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        L.orc_compute.argtypes = [ctypes.POINTER(OrcNode), ctypes.c_int32, ctypes.c_int32]
        L.orc_compute.restype = ctypes.c_int
        L.orc_time_nodes.argtypes = [ctypes.POINTER(OrcNode), ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                     ctypes.c_int32, ctypes.POINTER(ctypes.c_double)]
        L.orc_time_nodes.restype = ctypes.c_int
        L.orc_mel_filterbank.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float,
                                         ctypes.c_float, ctypes.c_void_p]
        L.orc_mel_filterbank.restype = None
        for name in ("orc_fp16_to_fp32", "orc_bf16_to_fp32"):
            getattr(L, name).argtypes = [ctypes.c_uint16]
            getattr(L, name).restype = ctypes.c_float
        for name in ("orc_fp32_to_fp16", "orc_fp32_to_bf16"):
            getattr(L, name).argtypes = [ctypes.c_float]
            getattr(L, name).restype = ctypes.c_uint16
        _lib = L
    return _lib


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def _rows(a):
    return int(a.size // a.shape[-1]) if a.ndim else 1


class Graph:
    """An ordered node list over numpy buffers, run by the C restatement.

    Each method appends one ggml node, allocates its output and returns it; the
    values are only valid after compute(). Inputs must stay alive (the graph
    keeps references)."""

    def __init__(self):
        self.nodes = []
        self.keep = []

    def _node(self, op, dst, src0, src1=None, **kw):
        n = OrcNode()
        n.op = op
        n.type0 = kw.get("type0", F32)
        n.ne0 = kw.get("ne0", dst.shape[-1])
        n.nrows = kw.get("nrows", _rows(dst))
        n.ne1 = kw.get("ne1", 0)
        n.src1_rows = kw.get("src1_rows", 0)
        n.src1_ne0 = kw.get("src1_ne0", 0)
        n.src0 = _ptr(src0)
        n.src1 = _ptr(src1) if src1 is not None else None
        n.dst = _ptr(dst)
        for k, v in enumerate(kw.get("f", ())):
            n.f[k] = v
        for k, v in enumerate(kw.get("i", ())):
            n.i[k] = v
        self.nodes.append(n)
        self.keep += [dst, src0] + ([src1] if src1 is not None else [])
        return dst

    @staticmethod
    def _f32(a):
        a = np.ascontiguousarray(a, dtype=np.float32)
        return a

    def _binary(self, op, a, b):
        a = self._f32(a)
        b = self._f32(b)
        dst = np.empty_like(a)
        ne0 = a.shape[-1]
        if b.shape == a.shape:
            src1_rows, src1_ne0 = _rows(a), ne0
        elif b.size == ne0:
            src1_rows, src1_ne0 = 1, ne0          # one row repeated over rows
        elif b.size == _rows(a) and b.shape[-1] == 1:
            src1_rows, src1_ne0 = _rows(a), 1     # one value per row
        else:
            raise ValueError("unsupported broadcast %s vs %s" % (a.shape, b.shape))
        return self._node(op, dst, a, b, src1_rows=src1_rows, src1_ne0=src1_ne0)

    def add(self, a, b):
        return self._binary(OP_ADD, a, b)

    def mul(self, a, b):
        return self._binary(OP_MUL, a, b)

    def div(self, a, b):
        return self._binary(OP_DIV, a, b)

    def _unary(self, op, x, f=()):
        x = self._f32(x)
        return self._node(op, np.empty_like(x), x, f=f)

    def rms_norm(self, x, eps):
        return self._unary(OP_RMS_NORM, x, f=(eps,))

    def silu(self, x):
        return self._unary(OP_SILU, x)

    def sin(self, x):
        return self._unary(OP_SIN, x)

    def sqr(self, x):
        return self._unary(OP_SQR, x)

    def exp(self, x):
        return self._unary(OP_EXP, x)

    def leaky_relu(self, x, slope):
        return self._unary(OP_LEAKY_RELU, x, f=(slope,))

    def tanh(self, x):
        return self._unary(OP_TANH, x)

    def sigmoid(self, x):
        return self._unary(OP_SIGMOID, x)

    def elu(self, x):
        return self._unary(OP_ELU, x)

    def gelu_erf(self, x):
        return self._unary(OP_GELU_ERF, x)

    def relu(self, x):
        return self._unary(OP_RELU, x)

    def neg(self, x):
        return self._unary(OP_NEG, x)

    def step(self, x):
        return self._unary(OP_STEP, x)

    def sqrt(self, x):
        return self._unary(OP_SQRT, x)

    def diag_mask_inf(self, x, n_past):
        """ggml_diag_mask_inf: x (..., ne1, ne0)."""
        x = self._f32(x)
        return self._node(OP_DIAG_MASK_INF, np.empty_like(x), x, ne1=x.shape[-2] if x.ndim > 1 else 1,
                          i=(int(n_past),))

    def harmonic_source(self, f0, merge_weight, merge_bias, rand_ini, noise, *, rate, scale, sine_amp, noise_std,
                        voiced_threshold, n_fft, hop):
        """Kokoro's build_harmonic_source: f0 (L,), merge_weight and rand_ini
        (H,), noise (L*scale, H) -> (excitation (L*scale,), spectrum (frames,
        2*(n_fft/2 + 1)), magnitudes then phases per frame)."""
        f0 = self._f32(f0)
        mw, ri, nz = self._f32(merge_weight), self._f32(rand_ini), self._f32(noise)
        L, H = f0.size, mw.size
        U = L * scale
        if ri.size != H or nz.shape != (U, H) or n_fft < 2 or hop < 1 or scale < 1:
            raise ValueError("harmonic_source: bad shapes or parameters")
        bins = n_fft // 2 + 1
        exc = np.empty(U, np.float32)
        har = np.empty((U // hop + 1, 2 * bins), np.float32)
        args = OrcSourceArgs(mw.ctypes.data, ri.ctypes.data, nz.ctypes.data, har.ctypes.data, merge_bias, sine_amp,
                             noise_std, voiced_threshold, int(rate), int(H), int(scale), int(n_fft), int(hop), 0)
        n = OrcNode()
        n.op, n.type0, n.ne0, n.nrows = OP_HARMONIC_SOURCE, F32, 1, L
        n.src0, n.src1, n.dst = _ptr(f0), ctypes.cast(ctypes.pointer(args), ctypes.c_void_p), _ptr(exc)
        self.nodes.append(n)
        self.keep += [exc, har, f0, mw, ri, nz, args]
        return exc, har

    def log_mel(self, pcm, filterbank, n_fft, hop, win_length):
        """The speaker encoder's compute_log_mel given the filterbank (mel_bins,
        n_fft/2 + 1): pcm (samples,) -> (frames, mel_bins)."""
        x = self._f32(pcm)
        fb = self._f32(filterbank)
        bins = fb.shape[0]
        pad = (n_fft - hop) // 2
        plen = x.size + 2 * pad
        if n_fft < 2 or n_fft & (n_fft - 1) or hop < 1 or win_length > n_fft or hop > n_fft or x.size <= pad \
                or plen < n_fft or fb.shape != (bins, n_fft // 2 + 1):
            raise ValueError("log_mel: bad input or parameters")
        frames = 1 + (plen - n_fft) // hop
        return self._node(OP_LOG_MEL, np.empty((frames, bins), np.float32), x, fb, ne0=x.size, nrows=1,
                          i=(int(n_fft), int(hop), int(win_length), int(bins)))

    def inverse_stft(self, spectrum, n_fft, hop):
        """Kokoro's inverse_stft: spectrum (frames, n_fft + 2) -> ((frames - 1) * hop,)."""
        x = self._f32(spectrum)
        frames = x.shape[0]
        if x.ndim != 2 or x.shape[1] != n_fft + 2 or frames < 2 or n_fft < 2 or n_fft % 2 or hop <= 0:
            raise ValueError("inverse_stft: bad spectrum or parameters")
        return self._node(OP_ISTFT, np.empty((frames - 1) * hop, np.float32), x, ne0=n_fft + 2, nrows=frames,
                          i=(int(n_fft), int(hop)))

    def sum_rows(self, x):
        """ggml_sum_rows: (..., ne0) -> (..., 1)."""
        x = self._f32(x)
        return self._node(OP_SUM_ROWS, np.empty(x.shape[:-1] + (1,), np.float32), x, ne0=x.shape[-1], nrows=_rows(x))

    def mean(self, x):
        """ggml_mean: (..., ne0) -> (..., 1)."""
        x = self._f32(x)
        return self._node(OP_MEAN, np.empty(x.shape[:-1] + (1,), np.float32), x, ne0=x.shape[-1], nrows=_rows(x))

    def clamp(self, x, lo, hi):
        return self._unary(OP_CLAMP, x, f=(lo, hi))

    def norm(self, x, eps):
        """ggml_norm: x (rows, ne0)."""
        x = self._f32(x)
        dst = np.empty(x.shape, dtype=np.float32)
        return self._node(OP_NORM, dst, x, f=(eps,))

    def sub(self, a, b):
        return self._binary(OP_SUB, a, b)

    def scale_bias(self, x, s, b):
        return self._unary(OP_SCALE_BIAS, x, f=(s, b))

    def scale(self, x, s):
        """ggml_scale: ggml_scale_bias with bias 0."""
        return self._unary(OP_SCALE_BIAS, x, f=(s, 0.0))

    def rope_neox(self, x, pos, n_dims, freq_base, freq_scale=1.0, attn_factor=1.0, cs_rounded=False):
        """x: (T, heads, head_dim) f32; pos: (T,) int32. cs_rounded: cos/sin from
        double rounded once to f32 instead of libm cosf/sinf (ggml-CPU's)."""
        x = self._f32(x)
        pos = np.ascontiguousarray(pos, dtype=np.int32)
        assert x.ndim == 3 and pos.shape == (x.shape[0],)
        return self._node(OP_ROPE_NEOX, np.empty_like(x), x, pos, ne1=x.shape[1], nrows=x.shape[0] * x.shape[1],
                          f=(freq_base, freq_scale, attn_factor), i=(n_dims, 1 if cs_rounded else 0))

    def get_rows(self, table, type0, ne0, ids):
        """table: numpy array of raw rows (any dtype, C-contiguous, one row per
        leading index: (rows, row_elems) for F32/F16(bits)/BF16(bits), (rows,
        row_bytes) uint8 for Q8_0 and Q5_K); ids: (n,) int32 -> (n, ne0) f32."""
        table = np.ascontiguousarray(table)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        dst = np.empty((ids.size, ne0), dtype=np.float32)
        return self._node(OP_GET_ROWS, dst, table, ids, type0=type0, ne0=ne0, nrows=ids.size,
                          src1_rows=table.shape[0])

    def cast_f32(self, x, type0):
        x = np.ascontiguousarray(x)
        dst = np.empty(x.shape, dtype=np.float32)
        return self._node(OP_CAST_F32, dst, x, type0=type0)

    def binbcast(self, op, a, b):
        """ggml_add / ggml_mul / ggml_div (op = OP_ADD, OP_MUL, OP_DIV) with b
        repeated to a's shape: a and b are numpy arrays in the module's
        layout (ggml [ne0, ne1, ne2, ne3] = numpy (ne3, ne2, ne1, ne0), up to
        4 axes); every ggml extent of b must divide a's."""
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        ane = list(a.shape[::-1]) + [1] * (4 - a.ndim)
        bne = list(b.shape[::-1]) + [1] * (4 - b.ndim)
        if any(x < 1 or y % x for x, y in zip(bne, ane)):
            raise ValueError("b does not repeat to a's shape")
        view = np.array(ane + bne + [b.ctypes.data], dtype=np.int64)
        dst = np.empty(a.shape, dtype=np.float32)
        n = OrcNode()
        n.op, n.type0, n.ne0, n.nrows = OP_BINBCAST, F32, ane[0], ane[1] * ane[2] * ane[3]
        n.src0, n.src1, n.dst = _ptr(a), _ptr(view), _ptr(dst)
        n.i[0] = op
        self.nodes.append(n)
        self.keep += [dst, a, b, view]
        return dst

    def cont_f32(self, buf, ne, nb, offset=0):
        """ggml_cont of an F32 view of `buf` (any C-contiguous numpy array,
        read as raw bytes): the view starts `offset` bytes in, with ggml
        extents ne[0..3] and byte strides nb[0..3]. Returns the contiguous
        result as a numpy array of shape (ne3, ne2, ne1, ne0)."""
        buf = np.ascontiguousarray(buf)
        ne = [int(v) for v in ne] + [1] * (4 - len(ne))
        nb = [int(v) for v in nb] + [0] * (4 - len(nb))
        last = offset + 4 + sum((n - 1) * b for n, b in zip(ne, nb))
        if offset < 0 or last > buf.nbytes or min(ne) < 1 or min(nb) < 0:
            raise ValueError("view outside the buffer")
        view = np.array(ne + nb, dtype=np.int64)
        dst = np.empty((ne[3], ne[2], ne[1], ne[0]), dtype=np.float32)
        n = OrcNode()
        n.op, n.type0, n.ne0, n.nrows, n.ne1 = OP_CONT_F32, F32, ne[0], ne[1] * ne[2] * ne[3], ne[1]
        n.src0 = ctypes.c_void_p(buf.ctypes.data + offset)
        n.src1 = _ptr(view)
        n.dst = _ptr(dst)
        self.nodes.append(n)
        self.keep += [dst, buf, view]
        return dst

    def im2col(self, x, k, s0, p0, d0, dst_type=F32):
        """ggml_im2col(kernel [k, IC, ...], x, s0, 0, p0, 0, d0, 0, false,
        dst_type): x numpy (N, IC, IW) or (IC, IW) = ggml [IW, IC, N]. Returns
        numpy (N, OW, IC*k) = ggml [IC*k, OW, N]: float32, or uint16 F16 bits
        for dst_type F16."""
        x = self._f32(x)
        x = x.reshape((1,) * (3 - x.ndim) + x.shape)
        n_, ic, iw = x.shape
        ow = conv_out_len(iw, k, s0, p0, d0)
        if ow < 1 or dst_type not in (F32, F16):
            raise ValueError("im2col: no output position, or a dst type other than F32/F16")
        view = np.array([iw, ic, n_, k, s0, p0, d0], dtype=np.int64)
        dst = np.empty((n_, ow, ic * k), dtype=np.float32 if dst_type == F32 else np.uint16)
        nd = OrcNode()
        nd.op, nd.type0, nd.ne0, nd.nrows = OP_IM2COL, dst_type, ic * k, n_ * ow
        nd.src0, nd.src1, nd.dst = _ptr(x), _ptr(view), _ptr(dst)
        self.nodes.append(nd)
        self.keep += [dst, x, view]
        return dst

    def col2im_1d(self, cols, stride, oc, padding):
        """ggml_col2im_1d(columns, stride, oc, padding): cols numpy (L, K*OC) =
        ggml [K*OC, L]; returns (OC, T) = ggml [T, OC], T = (L-1)*stride + K -
        2*padding."""
        cols = self._f32(cols)
        L, ko = cols.shape
        if ko % oc or stride < 1 or padding < 0:
            raise ValueError("col2im_1d: K*OC not a multiple of OC, or a bad stride / padding")
        k = ko // oc
        t = (L - 1) * stride + k - 2 * padding
        if t < 1:
            raise ValueError("col2im_1d: no output sample")
        view = np.array([k, oc, L, stride, padding], dtype=np.int64)
        dst = np.empty((oc, t), dtype=np.float32)
        nd = OrcNode()
        nd.op, nd.type0, nd.ne0, nd.nrows = OP_COL2IM_1D, F32, t, oc
        nd.src0, nd.src1, nd.dst = _ptr(cols), _ptr(view), _ptr(dst)
        self.nodes.append(nd)
        self.keep += [dst, cols, view]
        return dst

    def _pad_family(self, op, x, dshape, offs):
        """x numpy (up to 4 axes, this module's layout); dshape the result's
        numpy shape; offs the op's ggml-order offsets."""
        x = self._f32(x)
        nd = max(x.ndim, len(dshape))
        sne = list(x.shape[::-1]) + [1] * (4 - x.ndim)
        dne = list(dshape[::-1]) + [1] * (4 - len(dshape))
        view = np.array(sne + dne + list(offs) + [0] * (4 - len(offs)), dtype=np.int64)
        dst = np.empty(tuple(dshape), dtype=np.float32)
        n = OrcNode()
        n.op, n.type0, n.ne0, n.nrows = op, F32, dne[0], dne[1] * dne[2] * dne[3]
        n.src0, n.src1, n.dst = _ptr(x), _ptr(view), _ptr(dst)
        self.nodes.append(n)
        self.keep += [dst, x, view]
        return dst

    def pad_ext(self, x, lp, rp):
        """ggml_pad_ext(x, lp0, rp0, lp1, rp1, ...): lp, rp per ggml dim (up to 4)."""
        x = self._f32(x)
        lp = list(lp) + [0] * (4 - len(lp))
        rp = list(rp) + [0] * (4 - len(rp))
        sne = list(x.shape[::-1]) + [1] * (4 - x.ndim)
        dne = [sne[d] + lp[d] + rp[d] for d in range(4)]
        nd = max(x.ndim, max([d + 1 for d in range(4) if lp[d] or rp[d]] + [1]))
        return self._pad_family(OP_PAD, x, tuple(dne[:nd][::-1]), lp)

    def pad(self, x, p):
        """ggml_pad(x, p0, p1, p2, p3): zeros after the end of each dim."""
        return self.pad_ext(x, [0, 0, 0, 0], p)

    def pad_reflect_1d(self, x, p0, p1):
        """ggml_pad_reflect_1d(x, p0, p1) (p0, p1 < ne0)."""
        x = self._f32(x)
        if p0 >= x.shape[-1] or p1 >= x.shape[-1] or p0 < 0 or p1 < 0:
            raise ValueError("pad_reflect_1d: a pad of the row's length or more")
        return self._pad_family(OP_PAD_REFLECT_1D, x, x.shape[:-1] + (x.shape[-1] + p0 + p1,), [p0, 0, 0, 0])

    def repeat(self, x, shape):
        """ggml_repeat(x, b) with b of numpy shape `shape` (every extent a multiple of x's)."""
        x = self._f32(x)
        xs = (1,) * (len(shape) - x.ndim) + x.shape
        if any(d % s for d, s in zip(shape, xs)):
            raise ValueError("repeat: an extent not a multiple of the source's")
        return self._pad_family(OP_REPEAT, x.reshape(xs), tuple(shape), [0, 0, 0, 0])

    def acc(self, a, b, nb1, nb2, nb3, offset):
        """ggml_acc(a, b, nb1, nb2, nb3, offset): a copy of a with b added into
        the view of it at byte `offset` with byte strides nb1..nb3 (b's shape,
        b's element stride 4). a and b in this module's layout; b may be the
        output of an earlier node (a contiguous slice of one)."""
        a = self._f32(a)
        b = self._f32(b)
        bne = list(b.shape[::-1]) + [1] * (4 - b.ndim)
        if b.size and offset + (bne[0] - 1) * 4 + (bne[1] - 1) * nb1 + (bne[2] - 1) * nb2 + \
                (bne[3] - 1) * nb3 >= a.nbytes:
            raise ValueError("acc: the view runs past a's end")
        view = np.array(bne + [nb1, nb2, nb3, offset, b.ctypes.data], dtype=np.int64)
        dst = np.empty_like(a)
        n = OrcNode()
        n.op, n.type0, n.ne0, n.nrows = OP_ACC, F32, a.shape[-1], _rows(a)
        n.src0, n.src1, n.dst = _ptr(a), _ptr(view), _ptr(dst)
        self.nodes.append(n)
        self.keep += [dst, a, b, view]
        return dst

    def glu_swiglu(self, a, swapped=False):
        a = self._f32(a)
        nc = a.shape[-1] // 2
        dst = np.empty(a.shape[:-1] + (nc,), dtype=np.float32)
        return self._node(OP_GLU_SWIGLU, dst, a, ne0=nc, nrows=_rows(dst), i=(1 if swapped else 0,))

    def soft_max_ext(self, x, mask, scale):
        """x (heads, rows, cols) or (rows, cols) = ggml [cols, rows, heads]; mask None,
        (mrows, cols) or (mheads, mrows, cols) with mrows >= rows and heads % mheads == 0."""
        x = self._f32(x)
        x3 = x.reshape((-1,) + x.shape[-2:])
        ne1 = x3.shape[1]
        mheads, mrows = 1, 0
        if mask is not None:
            mask = self._f32(mask)
            m3 = mask.reshape((-1,) + mask.shape[-2:])
            mheads, mrows = m3.shape[0], m3.shape[1]
            assert m3.shape[2] == x.shape[-1] and mrows >= ne1 and x3.shape[0] % mheads == 0
        return self._node(OP_SOFT_MAX, np.empty_like(x), x, mask, ne1=ne1, src1_rows=mrows, i=(mheads,),
                          f=(scale,))

    def _array(self):
        arr = (OrcNode * len(self.nodes))(*self.nodes)
        return arr

    def compute(self, n_threads=1):
        arr = self._array()
        rc = lib().orc_compute(arr, len(self.nodes), int(n_threads))
        if rc != 0:
            raise RuntimeError("oracle compute failed (%d)" % rc)

    def time(self, n_threads, warmup, reps):
        arr = self._array()
        times = (ctypes.c_double * reps)()
        rc = lib().orc_time_nodes(arr, len(self.nodes), int(n_threads), int(warmup), int(reps), times)
        if rc != 0:
            raise RuntimeError("oracle timing failed (%d)" % rc)
        return list(times)


# ---------------------------------------------------------------------------
# node runs the reference graph builders emit
# ---------------------------------------------------------------------------

def conv_out_len(iw, k, s0, p0, d0):
    """ggml_calc_conv_output_size: (iw + 2*p0 - d0*(k-1) - 1)/s0 + 1 with C's
    truncating division."""
    num = iw + 2 * p0 - d0 * (k - 1) - 1
    return (num // s0 if num >= 0 else -((-num) // s0)) + 1


def concat(a, b, dim):
    """ggml_concat(a, b, dim) restated (data movement only: every element of
    the result is a's where its index along ggml dimension dim is below a's
    extent, else b's at that index minus a's extent). a, b: numpy arrays in
    this module's layout; ggml dim d is numpy axis ndim - 1 - d. Sites:
    src/arch/qwen3-tts/model.cpp:1450, qwen3-tts/speaker-encoder.cpp:236,335,358."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    nd = max(a.ndim, b.ndim, dim + 1)
    a = a.reshape((1,) * (nd - a.ndim) + a.shape)
    b = b.reshape((1,) * (nd - b.ndim) + b.shape)
    return np.concatenate([a, b], axis=nd - 1 - dim)


def as_f32(g, w, wtype=F32):
    """as_f32, src/arch/qwen3-tts/operations.cpp:20-25 (ggml_cast when not F32)."""
    return w if wtype == F32 else g.cast_f32(w, wtype)


def rms_norm_w(g, x, w, eps, wtype=F32):
    """rms_norm(), src/arch/qwen3-tts/operations.cpp:27-32: ggml_rms_norm then ggml_mul."""
    return g.mul(g.rms_norm(x, eps), as_f32(g, w, wtype))


def swiglu(g, gate, up):
    """src/arch/qwen3-tts/operations.cpp:39-41: ggml_silu(gate) then ggml_mul(., up)."""
    return g.mul(g.silu(gate), up)


def qk_norm_rope(g, q, k, wq, wk, eps, pos, n_dims, theta, wtype=F32, cs_rounded=False):
    """src/arch/qwen3-tts/operations.cpp:98-104: per-head rms_norm()*w then NEOX rope,
    for q (T, heads, hd) and k (T, kv_heads, hd)."""
    qn = rms_norm_w(g, q, wq, eps, wtype)
    kn = rms_norm_w(g, k, wk, eps, wtype)
    return (g.rope_neox(qn, pos, n_dims, theta, cs_rounded=cs_rounded),
            g.rope_neox(kn, pos, n_dims, theta, cs_rounded=cs_rounded))


def add_rms_norm_w(g, a, b, w, eps, wtype=F32):
    """src/arch/qwen3-tts/operations.cpp:143-145: residual ggml_add then rms_norm()."""
    s = g.add(a, b)
    return s, rms_norm_w(g, s, w, eps, wtype)


def snake(g, x, alpha):
    """src/arch/kokoro/operations.cpp:137-147: mul, sin, mul(s, s), div, add. x (T, C)."""
    scaled = g.mul(x, alpha)
    sine = g.sin(scaled)
    squared = g.mul(sine, sine)
    return g.add(x, g.div(squared, alpha))


def snake_beta(g, x, log_alpha, log_beta):
    """codec_snake_beta, src/arch/qwen3-tts/codec.cpp:184-199:
    x + sin(x*exp(a))^2 / (exp(b) + 1e-9)."""
    alpha = g.exp(log_alpha)
    beta = g.exp(log_beta)
    squared = g.sqr(g.sin(g.mul(x, alpha)))
    guard = g.scale_bias(beta, 1.0, 1e-9)
    return g.add(x, g.div(squared, guard))


def snake_guarded(g, x, alpha):
    """codec_snake, src/arch/omnivoice/codec.cpp:51-68: mul, sin, mul(s, s),
    scale_bias(alpha, 1, 1e-9), div, add. x (T, C)."""
    scaled = g.mul(x, alpha)
    sine = g.sin(scaled)
    squared = g.mul(sine, sine)
    guard = g.scale_bias(alpha, 1.0, 1e-9)
    return g.add(x, g.div(squared, guard))


def sum_scale_leaky(g, terms, scale, slope):
    """The branch average of src/arch/vits/waveform-decoder.cpp:214-225 and
    src/arch/kokoro/generator.cpp:165-179: ggml_add over the terms in order,
    ggml_scale (skipped for one term), then ggml_leaky_relu. Returns (current, y)."""
    summed = None
    for t in terms:
        summed = t if summed is None else g.add(summed, t)
    current = summed if len(terms) == 1 else g.scale(summed, scale)
    return current, g.leaky_relu(current, slope)


def add_leaky(g, a, b, slope):
    """src/arch/vits/waveform-decoder.cpp:150-158: layer l's closing ggml_add, then layer
    l+1's ggml_leaky_relu. Returns (sum, y)."""
    s = g.add(a, b)
    return s, g.leaky_relu(s, slope)


def sum_code_embeddings(g, tables, type0, ne0, codes):
    """src/arch/qwen3-tts/code-predictor.cpp:82-107: get_rows per group, added in group
    order. codes: (groups, frames) int32 (ggml [frames, groups], frames fastest)."""
    total = None
    for t, table in enumerate(tables):
        rows = g.get_rows(table, type0, ne0, codes[t])
        total = rows if total is None else g.add(total, rows)
    return total


def run(build, n_threads=1):
    """Builds a graph with `build(g)` and computes it; returns build's result."""
    g = Graph()
    out = build(g)
    g.compute(n_threads)
    return out


# ---------------------------------------------------------------------------
# the rest of a Qwen3 block, for the tiny golden configurations
# ---------------------------------------------------------------------------

def mul_mat(w, x):
    """ggml_mul_mat(w, x) with w [in, out] (numpy (out, in)) and x (T, in): (T, out).
    Accumulated in double and rounded once, which is within the goldens' 1e-4 of
    ggml's f32 SIMD dot products."""
    return (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)


def soft_max_ext(scores, mask, scale):
    """ggml_soft_max_ext(scores, mask, scale, 0) over the last axis, through the
    C restatement (ggml-CPU's rounding order)."""
    return run(lambda g: g.soft_max_ext(scores, mask, np.float32(scale)))


class LcgStream:
    """The reference tests' weight stream: 64-bit LCG, float(state>>40)/2^23 - 1
    (tests/qwen3_tts_decoder_layer_test.cpp:51-70)."""

    MUL = 6364136223846793005
    INC = 1442695040888963407
    MASK = (1 << 64) - 1

    def __init__(self, seed):
        self.state = seed & self.MASK

    def fill(self, count, scale, offset):
        out = np.empty(count, dtype=np.float32)
        s = self.state
        for k in range(count):
            s = (s * self.MUL + self.INC) & self.MASK
            out[k] = np.float32(s >> 40) / np.float32(8388608.0) - np.float32(1.0)
        self.state = s
        return out * np.float32(scale) + np.float32(offset)


def decoder_layer(x, pos, mask, W, shape, cache, filled, ops=None):
    """decoder_layer, src/arch/qwen3-tts/operations.cpp:44-148, over x (T, hidden).

    W holds numpy weights in ggml memory order ((out, in) for projections).
    cache = {"k": (cap, kv_heads, hd), "v": ...} is written in place at
    [filled, filled+T). `ops` replaces the hot-path node runs (default: this
    restatement); the GPU parity tests pass the HIP versions here."""
    ops = ops or OracleOps()
    T = x.shape[0]
    hd, H, KVH = shape["head_dim"], shape["heads"], shape["kv_heads"]
    eps, theta = shape["rms_norm_eps"], shape["rope_theta"]
    residual = x
    normed = ops.rms_norm_w(x, W["input_layernorm"], eps)
    q = mul_mat(W["q_proj"], normed).reshape(T, H, hd)
    k = mul_mat(W["k_proj"], normed).reshape(T, KVH, hd)
    v = mul_mat(W["v_proj"], normed).reshape(T, KVH, hd)
    q = ops.qk_norm_rope_kv(q, k, v, W["q_norm"], W["k_norm"], eps, pos, hd, theta, cache, filled)
    total = filled + T
    kc, vc = cache["k"][:total], cache["v"][:total]
    group = H // KVH
    attended = np.empty((T, H, hd), dtype=np.float32)
    for h in range(H):
        kv = h // group  # ggml_mul_mat's broadcast: blocked grouping (operations.cpp:127-131)
        scores = (q[:, h, :].astype(np.float64) @ kc[:, kv, :].astype(np.float64).T).astype(np.float32)
        p = ops.soft_max_ext(scores, mask, np.float32(1.0) / np.sqrt(np.float32(hd)))
        attended[:, h, :] = (p.astype(np.float64) @ vc[:, kv, :].astype(np.float64)).astype(np.float32)
    projected = mul_mat(W["o_proj"], attended.reshape(T, H * hd))
    after_attention, mlp_in = ops.add_rms_norm_w(residual, projected, W["post_attention_layernorm"], eps)
    gate = mul_mat(W["gate_proj"], mlp_in)
    up = mul_mat(W["up_proj"], mlp_in)
    mlp = mul_mat(W["down_proj"], ops.swiglu(gate, up))
    return ops.add(after_attention, mlp)


class OracleOps:
    """The hot-path node runs of decoder_layer, evaluated by the restatement."""

    def rms_norm_w(self, x, w, eps):
        return run(lambda g: rms_norm_w(g, x, w, eps))

    def qk_norm_rope(self, q, k, wq, wk, eps, pos, n_dims, theta):
        return run(lambda g: qk_norm_rope(g, q, k, wq, wk, eps, pos, n_dims, theta))

    def qk_norm_rope_kv(self, q, k, v, wq, wk, eps, pos, n_dims, theta, cache, filled):
        """operations.cpp:98-116: q and k normalised and rotated, then k and v
        copied (ggml_cpy) into cache rows [filled, filled + T); returns q."""
        q, k = self.qk_norm_rope(q, k, wq, wk, eps, pos, n_dims, theta)
        T = q.shape[0]
        cache["k"][filled:filled + T] = k
        cache["v"][filled:filled + T] = v
        return q

    def soft_max_ext(self, scores, mask, scale):
        return soft_max_ext(scores, mask, scale)

    def add_rms_norm_w(self, a, b, w, eps):
        return run(lambda g: add_rms_norm_w(g, a, b, w, eps))

    def swiglu(self, gate, up):
        return run(lambda g: swiglu(g, gate, up))

    def add(self, a, b):
        return run(lambda g: g.add(a, b))

    def get_rows(self, table, ids):
        return run(lambda g: g.get_rows(table, F32, table.shape[-1], ids))


def layer_weights(stream, hidden, heads, kv_heads, head_dim, intermediate):
    """One decoder layer's weights in the reference tests' fill order
    (tests/qwen3_tts_decoder_layer_test.cpp:146-158), numpy (out, in)."""
    spec = [("input_layernorm", (hidden,), 0.25, 1.0), ("q_proj", (heads * head_dim, hidden), 0.5, 0.0),
            ("k_proj", (kv_heads * head_dim, hidden), 0.5, 0.0), ("v_proj", (kv_heads * head_dim, hidden), 0.5, 0.0),
            ("o_proj", (hidden, heads * head_dim), 0.5, 0.0), ("q_norm", (head_dim,), 0.25, 1.0),
            ("k_norm", (head_dim,), 0.25, 1.0), ("post_attention_layernorm", (hidden,), 0.25, 1.0),
            ("gate_proj", (intermediate, hidden), 0.5, 0.0), ("up_proj", (intermediate, hidden), 0.5, 0.0),
            ("down_proj", (hidden, intermediate), 0.5, 0.0)]
    W = {}
    for name, shp, scale, offset in spec:
        W[name] = stream.fill(int(np.prod(shp)), scale, offset).reshape(shp)
    return W

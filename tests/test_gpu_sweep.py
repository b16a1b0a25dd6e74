"""Seeded random sweep: each entry point over shapes drawn across its launch
forms, against the ggml-CPU restatement on the same inputs:
- norm row counts either side of the 2048 / 4096 / 16384 boundaries;
- QK-norm+RoPE head counts that straddle the decode kernel's blocks of 8
  rows, with and without the KV-cache write (slots that fit exactly or not);
- softmax rows either side of 256 / 512 / 2048 elements;
- gathers of 1..4099 ids (F32/F16/BF16/Q8_0/Q5_K) and sums of 1..20
  codebooks (1..33 for Q5_K);
- Snake channel counts that are and are not multiples of 4, ragged last
  blocks everywhere;
- the one-call layer step at 1..513 positions;
- the transposing copy over 2-4-D permutations and unaligned starts, the
  fused conv tail with either bias form, every repeat form of
  add/sub/mul/div, concat along every dimension, LayerNorm and the
  activations.
The bars are test_gpu_parity.py's: bit-exact for gathers, sums of gathers,
adds and leaky-ReLU; 1e-5 relative for the norms, SwiGLU and the Snake
family; rope to 1e-5 of its NEOX pair against libm and bit-exact against the
restatement with correctly rounded cos/sin; softmax within 2 ulp. The case
list is fixed by SWEEP_SEED, so a failure names a shape that reruns the same
way.
"""
import numpy as np
import pytest

import formats as F
from test_gpu_activations import _close as _act_close, _inputs as _act_inputs
import ggml_ref as R
from test_gpu_parity import (_dev_table, _dev_w, _np, _positions, _specials, _t, _table, _ulps_apart, _weights,
                             assert_bitexact, assert_close, assert_rope_close, assert_snake_close)

pytestmark = pytest.mark.gpu

SWEEP_SEED = 515151
N_CASES = 24
MAX_ELEMS = 1 << 23


def _gen(name, draw, n=N_CASES):
    rng = np.random.default_rng([SWEEP_SEED, sum(map(ord, name))])
    out = []
    while len(out) < n:
        c = draw(rng)
        if c is not None and c not in out:
            out.append(c)
    return out


def _pick(rng, xs):
    return xs[int(rng.integers(0, len(xs)))]


# ---------------------------------------------------------------------------
# norms
# ---------------------------------------------------------------------------

_NORM_NE0 = [4, 8, 12, 64, 100, 128, 256, 512, 768, 1000, 1024, 2048, 3072, 4096, 5000, 8192]
_NORM_ROWS = [1, 2, 3, 7, 64, 65, 511, 1023, 1025, 2047, 2049, 4095, 4097, 6145, 16385]


def _norm_case(rng, kinds):
    ne0, rows = _pick(rng, _NORM_NE0), _pick(rng, _NORM_ROWS)
    if ne0 * rows > MAX_ELEMS:
        return None
    return (rows, ne0, _pick(rng, kinds))


@pytest.mark.parametrize("rows,ne0,wkind", _gen("rms_norm_mul", lambda r: _norm_case(r, ["f32", "bf16", "f16", "none"])))
def test_sweep_rms_norm_mul(gpu, rows, ne0, wkind):
    rng = np.random.default_rng([SWEEP_SEED, rows, ne0])
    x = (rng.standard_normal((rows, ne0)) * rng.uniform(0.01, 100)).astype(np.float32)
    eps = np.float32(1e-6)
    if wkind == "none":
        ref = R.run(lambda g: g.rms_norm(x, eps))
        got = gpu.rms_norm_mul(_t(gpu, x), None, eps)
    else:
        w, wt = _weights(rng, ne0, wkind)
        ref = R.run(lambda g: R.rms_norm_w(g, x, w, eps, wt))
        got = gpu.rms_norm_mul(_t(gpu, x), _dev_w(gpu, w, wkind), eps)
    assert_close(_np(got), ref)


@pytest.mark.parametrize("rows,ne0,wkind", _gen("add_rms_norm_mul", lambda r: _norm_case(r, ["f32", "bf16", "f16"])))
def test_sweep_add_rms_norm_mul(gpu, rows, ne0, wkind):
    rng = np.random.default_rng([SWEEP_SEED, 2, rows, ne0])
    a = rng.standard_normal((rows, ne0)).astype(np.float32)
    b = rng.standard_normal((rows, ne0)).astype(np.float32)
    w, wt = _weights(rng, ne0, wkind)
    eps = np.float32(1e-6)
    s_ref, y_ref = R.run(lambda g: R.add_rms_norm_w(g, a, b, w, eps, wt))
    s, y = gpu.add_rms_norm_mul(_t(gpu, a), _t(gpu, b), _dev_w(gpu, w, wkind), eps)
    assert_bitexact(_np(s), s_ref)
    assert_close(_np(y), y_ref)


# ---------------------------------------------------------------------------
# QK-norm + RoPE
# ---------------------------------------------------------------------------

def _rope_case(rng):
    T = _pick(rng, [1, 2, 7, 63, 64, 65, 128, 300])
    H = int(rng.integers(1, 25))
    KVH = int(rng.integers(1, H + 1))
    if T * (H + KVH) * 128 > MAX_ELEMS:
        return None
    return (T, H, KVH, _pick(rng, [8, 512, 8192, 100000]), _pick(rng, ["f32", "bf16", "f16"]))


@pytest.mark.parametrize("T,H,KVH,hi,wkind", _gen("qk_norm_rope", _rope_case))
def test_sweep_qk_norm_rope(gpu, T, H, KVH, hi, wkind):
    rng = np.random.default_rng([SWEEP_SEED, T, H, KVH])
    q = rng.standard_normal((T, H, 128)).astype(np.float32)
    k = rng.standard_normal((T, KVH, 128)).astype(np.float32)
    wq, wt = _weights(rng, 128, wkind)
    wk, _ = _weights(rng, 128, wkind)
    pos = _positions(rng, T, hi)
    eps, theta = np.float32(1e-6), np.float32(1e6)
    qo, ko = gpu.qk_norm_rope(_t(gpu, q), _t(gpu, k), _dev_w(gpu, wq, wkind), _dev_w(gpu, wk, wkind), eps,
                              _t(gpu, pos), 128, theta)
    qo, ko = _np(qo), _np(ko)
    qr, kr = R.run(lambda g: R.qk_norm_rope(g, q, k, wq, wk, eps, pos, 128, theta, wt))
    assert_rope_close(qo, qr, 128)
    assert_rope_close(ko, kr, 128)
    qc, kc = R.run(lambda g: R.qk_norm_rope(g, q, k, wq, wk, eps, pos, 128, theta, wt, cs_rounded=True))
    assert_bitexact(qo, qc)
    assert_bitexact(ko, kc)


def _rope_kv_case(rng):
    T = _pick(rng, [1, 1, 2, 5, 16, 63, 64, 65, 128])
    H = int(rng.integers(1, 25))
    KVH = int(rng.integers(1, H + 1))
    filled = int(rng.integers(0, 200))
    cap = filled + T + _pick(rng, [0, 1, 37])
    return (T, H, KVH, filled, cap, _pick(rng, ["f32", "bf16", "f16"]))


@pytest.mark.parametrize("T,H,KVH,filled,cap,wkind", _gen("qk_norm_rope_kv", _rope_kv_case))
def test_sweep_qk_norm_rope_kv(gpu, T, H, KVH, filled, cap, wkind):
    """The fused cache write: the same bits as the unfused kernel for q and
    the cache's k rows, v copied, every other cache row untouched."""
    from test_gpu_parity import test_qk_norm_rope_kv
    test_qk_norm_rope_kv(gpu, T, filled, cap, 128, wkind, H=H, KVH=KVH)


def _layer_case(rng):
    return (_pick(rng, [1, 2, 3, 17, 64, 65, 127, 300, 513]), _pick(rng, [128, 128, 64]),
            _pick(rng, ["f32", "bf16", "f16"]))


@pytest.mark.parametrize("T,hd,wkind", _gen("layer_nongemm_step", _layer_case, n=12))
def test_sweep_layer_nongemm_step(gpu, T, hd, wkind):
    """One call for a layer's non-GEMM node runs: each output the single
    entry points' bits and the oracle's, at the talker's widths."""
    from test_gpu_parity import test_layer_nongemm_step
    test_layer_nongemm_step(gpu, T, hd, wkind)


# ---------------------------------------------------------------------------
# gathers
# ---------------------------------------------------------------------------

def _gather_case(rng):
    kind = _pick(rng, ["f32", "f16", "bf16", "q8_0"])
    ne0s = [32, 64, 96, 160, 256, 512, 1024, 2048, 3072, 4096, 8192]
    if kind != "q8_0":
        ne0s = ne0s + [4, 12, 100, 1000, 6000]
    return (kind, _pick(rng, ne0s), _pick(rng, [1, 5, 300, 2048]), _pick(rng, [1, 2, 63, 64, 65, 257, 1000, 4099]))


@pytest.mark.parametrize("kind,ne0,rows,n", _gen("get_rows", _gather_case))
def test_sweep_get_rows(gpu, kind, ne0, rows, n):
    rng = np.random.default_rng([SWEEP_SEED, ne0, rows, n])
    raw, otype = _table(rng, kind, rows, ne0)
    ids = rng.integers(0, rows, n).astype(np.int32)
    ids[-1] = rows - 1
    ref = R.run(lambda g: g.get_rows(raw, otype, ne0, ids))
    assert_bitexact(_np(gpu.get_rows(_dev_table(gpu, raw, kind, ne0), _t(gpu, ids))), ref)


def _gather_sum_case(rng):
    kind = _pick(rng, ["f32", "f16", "bf16", "q8_0", "q8_0"])
    ne0s = [32, 96, 256, 512, 1024, 2048, 4096]
    if kind != "q8_0":
        ne0s = ne0s + [8, 100, 3000]
    return (kind, _pick(rng, ne0s), int(rng.integers(1, 21)), _pick(rng, [1, 3, 64, 301, 1025]))


@pytest.mark.parametrize("kind,ne0,groups,frames", _gen("get_rows_sum", _gather_sum_case))
def test_sweep_get_rows_sum(gpu, kind, ne0, groups, frames):
    rng = np.random.default_rng([SWEEP_SEED, ne0, groups, frames])
    rows = 200
    tabs = [_table(rng, kind, rows, ne0) for _ in range(groups)]
    codes = rng.integers(0, rows, (groups, frames)).astype(np.int32)
    ref = R.run(lambda g: R.sum_code_embeddings(g, [t for t, _ in tabs], tabs[0][1], ne0, codes))
    got = gpu.get_rows_sum([_dev_table(gpu, t, kind, ne0) for t, _ in tabs], _t(gpu, codes))
    assert_bitexact(_np(got), ref)


def _q5k_case(rng):
    return (256 * _pick(rng, [1, 2, 3, 4, 5, 8, 12, 16]), _pick(rng, [1, 7, 60, 2048]),
            _pick(rng, [1, 2, 63, 64, 65, 257, 1000, 4099]))


@pytest.mark.parametrize("ne0,rows,n", _gen("get_rows_q5k", _q5k_case))
def test_sweep_get_rows_q5k(gpu, ne0, rows, n):
    rng = np.random.default_rng([SWEEP_SEED, 29, ne0, rows, n])
    raw = F.q5_k_synthetic(rng, rows, ne0)
    ids = rng.integers(0, rows, n).astype(np.int32)
    ids[-1] = rows - 1
    ref = R.run(lambda g: g.get_rows(raw, R.Q5_K, ne0, ids))
    assert_bitexact(_np(gpu.get_rows(gpu.Q5KTensor(_t(gpu, raw), ne0), _t(gpu, ids))), ref)


def _q5k_sum_case(rng):
    return (256 * _pick(rng, [1, 2, 3, 4, 8, 12, 16]), int(rng.integers(1, 34)), _pick(rng, [1, 3, 64, 301, 1025]))


@pytest.mark.parametrize("ne0,groups,frames", _gen("get_rows_sum_q5k", _q5k_sum_case))
def test_sweep_get_rows_sum_q5k(gpu, ne0, groups, frames):
    rng = np.random.default_rng([SWEEP_SEED, 31, ne0, groups, frames])
    rows = 60
    tabs = [F.q5_k_synthetic(rng, rows, ne0) for _ in range(groups)]
    codes = rng.integers(0, rows, (groups, frames)).astype(np.int32)
    ref = R.run(lambda g: R.sum_code_embeddings(g, tabs, R.Q5_K, ne0, codes))
    got = gpu.get_rows_sum([gpu.Q5KTensor(_t(gpu, t), ne0) for t in tabs], _t(gpu, codes))
    assert_bitexact(_np(got), ref)


# ---------------------------------------------------------------------------
# softmax
# ---------------------------------------------------------------------------

def _softmax_case(rng):
    H, T = int(rng.integers(1, 17)), _pick(rng, [1, 1, 2, 5, 33, 64, 70])
    N = _pick(rng, [1, 2, 33, 64, 255, 256, 257, 300, 512, 513, 1024, 2048, 2049, 3000])
    masks = ["none", "rows+"] + (["causal"] if T <= N else []) + (["heads2"] if H % 2 == 0 else [])
    if H * T * N > MAX_ELEMS:
        return None
    return (H, T, N, _pick(rng, masks))


@pytest.mark.parametrize("H,T,N,mask", _gen("soft_max_ext", _softmax_case))
def test_sweep_soft_max_ext(gpu, H, T, N, mask):
    rng = np.random.default_rng([SWEEP_SEED, H, T, N])
    x = (rng.standard_normal((H, T, N)) * 3).astype(np.float32)
    m = None
    if mask == "causal":
        m = np.zeros((T, N), np.float32)
        m[np.triu_indices(T, N - T + 1, N)] = -np.inf
    elif mask == "heads2":
        m = rng.uniform(-5, 0, (2, T, N)).astype(np.float32)
    elif mask == "rows+":
        m = rng.uniform(-5, 0, (T + 3, N)).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    ref = R.run(lambda g: g.soft_max_ext(x, m, scale))
    got = _np(gpu.soft_max_ext(_t(gpu, x), None if m is None else _t(gpu, m), scale))
    # The bar only: a row whose double sum rounds to the other neighbouring
    # float moves every element of that row by one ulp, so the share of
    # identical elements is row-granular and says little over a few rows.
    assert _ulps_apart(got, ref).max() <= 2


# ---------------------------------------------------------------------------
# elementwise: SwiGLU, the Snake family, add, add -> leaky-ReLU
# ---------------------------------------------------------------------------

def _flat_case(rng):
    rows, ne0 = _pick(rng, [1, 3, 16, 257, 1000, 4099]), _pick(rng, [4, 7, 64, 1001, 1024, 3072, 3071, 8192])
    return None if rows * ne0 > MAX_ELEMS else (rows, ne0)


@pytest.mark.parametrize("rows,ne0", _gen("swiglu", _flat_case))
def test_sweep_swiglu(gpu, rows, ne0):
    rng = np.random.default_rng([SWEEP_SEED, 7, rows, ne0])
    gt = (rng.standard_normal((rows, ne0)) * 4).astype(np.float32)
    up = rng.standard_normal((rows, ne0)).astype(np.float32)
    assert_close(_np(gpu.swiglu(_t(gpu, gt), _t(gpu, up))), R.run(lambda g: R.swiglu(g, gt, up)))


def _snake_case(rng):
    T, C = _pick(rng, [1, 2, 3, 9, 37, 256, 1001, 4099]), _pick(rng, [4, 8, 30, 64, 100, 128, 260, 512, 1024, 1028, 2048])
    return None if T * C > MAX_ELEMS else (T, C)


@pytest.mark.parametrize("T,C", _gen("snake", _snake_case))
def test_sweep_snake(gpu, T, C):
    rng = np.random.default_rng([SWEEP_SEED, 11, T, C])
    x = rng.standard_normal((T, C)).astype(np.float32)
    alpha = np.exp(rng.uniform(np.log(0.1), np.log(10.0), C)).astype(np.float32)
    assert_close(_np(gpu.snake(_t(gpu, x), _t(gpu, alpha))), R.run(lambda g: R.snake(g, x, alpha)))


@pytest.mark.parametrize("T,C", _gen("snake_guarded", _snake_case))
def test_sweep_snake_guarded(gpu, T, C):
    rng = np.random.default_rng([SWEEP_SEED, 13, T, C])
    x = rng.standard_normal((T, C)).astype(np.float32)
    alpha = np.exp(rng.uniform(np.log(1e-9), np.log(10.0), C)).astype(np.float32)
    alpha[0] = 0.0
    got = _np(gpu.snake_guarded(_t(gpu, x), _t(gpu, alpha)))
    assert_snake_close(got, R.run(lambda g: R.snake_guarded(g, x, alpha)), x)


@pytest.mark.parametrize("T,C", _gen("snake_beta", _snake_case))
def test_sweep_snake_beta(gpu, T, C):
    rng = np.random.default_rng([SWEEP_SEED, 17, T, C])
    x = rng.standard_normal((T, C)).astype(np.float32)
    la = rng.uniform(-3, 3, C).astype(np.float32)
    lb = rng.uniform(-3, 3, C).astype(np.float32)
    got = _np(gpu.snake_beta(_t(gpu, x), _t(gpu, la), _t(gpu, lb)))
    assert_snake_close(got, R.run(lambda g: R.snake_beta(g, x, la, lb)), x)


@pytest.mark.parametrize("rows,ne0", _gen("add", _flat_case))
def test_sweep_add_and_row_broadcast(gpu, rows, ne0):
    rng = np.random.default_rng([SWEEP_SEED, 19, rows, ne0])
    a = rng.standard_normal((rows, ne0)).astype(np.float32)
    b = rng.standard_normal((rows, ne0)).astype(np.float32)
    assert_bitexact(_np(gpu.add(_t(gpu, a), _t(gpu, b))), R.run(lambda g: g.add(a, b)))
    brow = b[0].copy()
    assert_bitexact(_np(gpu.add(_t(gpu, a), _t(gpu, brow))), R.run(lambda g: g.add(a, brow)))


@pytest.mark.parametrize("rows,ne0", _gen("add_leaky_relu", _flat_case))
def test_sweep_add_leaky_relu(gpu, rows, ne0):
    rng = np.random.default_rng([SWEEP_SEED, 23, rows, ne0])
    a = _specials(rows * ne0, rng).reshape(rows, ne0)
    b = rng.standard_normal((rows, ne0)).astype(np.float32)
    slope = np.float32(_pick(rng, [0.1, 0.01, 0.2]))
    s_ref, y_ref = R.run(lambda g: R.add_leaky(g, a, b, slope))
    s, y = gpu.add_leaky_relu(_t(gpu, a), _t(gpu, b), float(slope), want_sum=True)
    assert_bitexact(_np(s), s_ref)
    assert_bitexact(_np(y), y_ref)


# ---------------------------------------------------------------------------
# the vocoder / codec neighbours: the transposing copy and the fused tail,
# repeated operands, concat, LayerNorm, the activations
# ---------------------------------------------------------------------------

_PERMS = {2: [(1, 0)], 3: [(1, 2, 0), (0, 2, 1), (2, 0, 1), (2, 1, 0)],
          4: [(0, 3, 1, 2), (3, 0, 1, 2), (0, 1, 3, 2), (3, 2, 1, 0), (1, 0, 3, 2)]}


def _transpose_case(rng):
    nd = int(rng.integers(2, 5))
    shape = tuple(int(_pick(rng, [1, 2, 3, 5, 17, 64, 100, 128, 255, 1000])) for _ in range(nd))
    shape = shape[:-1] + (max(shape[-1], 2),)      # the contiguous axis has extent > 1
    perm = _pick(rng, _PERMS[nd])
    if perm[-1] == nd - 1 or int(np.prod(shape)) > MAX_ELEMS:
        return None
    return (shape, perm, int(rng.integers(0, 4)))


@pytest.mark.parametrize("shape,perm,shift", _gen("transpose", _transpose_case))
def test_sweep_transposing_copy(gpu, shape, perm, shift):
    rng = np.random.default_rng([SWEEP_SEED, 29, *shape, shift])
    base = rng.standard_normal(int(np.prod(shape)) + shift).astype(np.float32)
    tb = _t(gpu, base)
    x = tb[shift:].view(shape)
    v = x.permute(perm)
    d = gpu.desc(v)
    g = R.Graph()
    ref = g.cont_f32(base, list(d.ne), list(d.nb), offset=4 * shift)
    g.compute(8)
    assert_bitexact(_np(gpu.cpy(v)), ref.reshape(tuple(v.shape)))


def _tail_case(rng):
    T, C = _pick(rng, [3, 64, 130, 1000, 2048, 4099]), _pick(rng, [2, 4, 37, 64, 96, 256])
    if T * C > MAX_ELEMS:
        return None
    leaky = int(rng.integers(0, 2))
    return (T, C, _pick(rng, ["row", "col"]), int(rng.integers(0, 2)), leaky,
            leaky * int(rng.integers(0, 2)), int(rng.integers(0, 2)))


@pytest.mark.parametrize("T,C,form,resid,leaky,with_sum,shift", _gen("cont_add_leaky", _tail_case))
def test_sweep_cont_add_leaky(gpu, T, C, form, resid, leaky, with_sum, shift):
    """y = cont(out^T) + b [+ r] [-> leaky], b one value per row ([1, C]) or
    one row ([ne0]) of y, out ggml [C, T] starting 0 or 1 float off 16 bytes."""
    import torch
    rng = np.random.default_rng([SWEEP_SEED, 31, T, C, resid, leaky, with_sum, shift])
    base = rng.standard_normal(T * C + shift).astype(np.float32)
    out = base[shift:].reshape(T, C)
    b = rng.standard_normal((C, 1) if form == "row" else (T,)).astype(np.float32)
    r = rng.standard_normal((C, T)).astype(np.float32) if resid else None
    tb = _t(gpu, base)
    view = tb[shift:].view(T, C).t()
    s_out = torch.empty((C, T), dtype=torch.float32, device="cuda") if with_sum else None
    y = gpu.cont_add_leaky_relu(view, _t(gpu, b), _t(gpu, r) if resid else None, 0.1 if leaky else None,
                                sum_out=s_out)
    g = R.Graph()
    tm = g.cont_f32(out, [T, C], [4 * C, 4]).reshape(C, T)
    s_ = g.binbcast(R.OP_ADD, tm, b if form == "row" else b.reshape(1, T))
    if resid:
        s_ = g.add(s_, r)
    yr = g.leaky_relu(s_, 0.1) if leaky else s_
    g.compute(4)
    assert_bitexact(_np(y), yr)
    if with_sum:
        assert_bitexact(_np(s_out), s_)


def _repeat_case(rng):
    nd = int(rng.integers(2, 5))
    ashape = [int(_pick(rng, [1, 2, 3, 4, 6, 12, 37, 64, 100, 1000])) for _ in range(nd)]
    bshape = []
    for n in ashape:
        divs = [d for d in (1, 2, 3, 4, 6, n) if n % d == 0]
        bshape.append(int(_pick(rng, divs)))
    if int(np.prod(ashape)) > MAX_ELEMS or ashape == bshape:
        return None
    return (tuple(ashape), tuple(bshape), _pick(rng, ["add", "sub", "mul", "div"]))


@pytest.mark.parametrize("ashape,bshape,op", _gen("repeat", _repeat_case))
def test_sweep_repeated_operand(gpu, ashape, bshape, op):
    rng = np.random.default_rng([SWEEP_SEED, 37, *ashape, *bshape])
    a = rng.standard_normal(ashape).astype(np.float32)
    b = (rng.standard_normal(bshape) + 2.5).astype(np.float32)
    code = {"add": R.OP_ADD, "sub": R.OP_SUB, "mul": R.OP_MUL, "div": R.OP_DIV}[op]
    assert_bitexact(_np(getattr(gpu, op)(_t(gpu, a), _t(gpu, b))), R.run(lambda g: g.binbcast(code, a, b)))


def _concat_case(rng):
    nd = int(rng.integers(1, 5))
    shape = [int(_pick(rng, [1, 2, 3, 7, 64, 100, 1024])) for _ in range(nd)]
    dim = int(rng.integers(0, nd))
    other = list(shape)
    other[nd - 1 - dim] = int(_pick(rng, [1, 2, 5, 64]))
    if int(np.prod(shape)) + int(np.prod(other)) > MAX_ELEMS:
        return None
    return (tuple(shape), tuple(other), dim)


@pytest.mark.parametrize("ashape,bshape,dim", _gen("concat", _concat_case))
def test_sweep_concat(gpu, ashape, bshape, dim):
    rng = np.random.default_rng([SWEEP_SEED, 41, *ashape, *bshape, dim])
    a = rng.standard_normal(ashape).astype(np.float32)
    b = rng.standard_normal(bshape).astype(np.float32)
    ref = R.concat(a, b, dim)
    got = _np(gpu.concat(_t(gpu, a), _t(gpu, b), dim))
    assert_bitexact(got.reshape(ref.shape), ref)


@pytest.mark.parametrize("rows,ne0,wkind", _gen("norm", lambda r: _norm_case(r, ["none"])))
def test_sweep_layer_norm(gpu, rows, ne0, wkind):
    rng = np.random.default_rng([SWEEP_SEED, 43, rows, ne0])
    x = (rng.standard_normal((rows, ne0)) * 2 + 1).astype(np.float32)
    got = _np(gpu.norm(_t(gpu, x), 1e-5))
    assert np.abs(got - R.run(lambda g: g.norm(x, 1e-5))).max() <= 1e-5


@pytest.mark.parametrize("rows,ne0", _gen("activations", _flat_case))
def test_sweep_activations(gpu, rows, ne0):
    rng = np.random.default_rng([SWEEP_SEED, 47, rows, ne0])
    x = _act_inputs(rng, (rows, ne0))
    tx = _t(gpu, x)
    for op in ("tanh", "sigmoid", "elu", "gelu_erf"):
        _act_close(_np(getattr(gpu, op)(tx)), R.run(lambda g: getattr(g, op)(x)), x if op == "gelu_erf" else None)
    assert_bitexact(_np(gpu.clamp(tx, -2.0, 2.0)), R.run(lambda g: g.clamp(x, -2.0, 2.0)))

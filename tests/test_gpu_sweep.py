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
- the one-call layer step at 1..513 positions.
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

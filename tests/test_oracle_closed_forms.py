"""Pins the ggml-CPU restatement where the reference's goldens leave it open:
exact conversions (all 65536 half/bf16 patterns), the Q8_0 closed form and a
pure-Python brute force, RMSNorm invariants, rope identities and a
double-precision closed form at large positions, SwiGLU / Snake against double
closed forms, leaky-ReLU's signed-zero and NaN behaviour, and thread-count
invariance of the ggml-style row split. Planted mistakes check that each test
can fail."""
import math
import struct

import numpy as np
import pytest

import formats as F
import ggml_ref as R

ULP = np.finfo(np.float32).eps


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------------------
# conversions and gathers
# ---------------------------------------------------------------------------

def test_half_and_bf16_conversions_all_patterns():
    # Through get_rows, so results stay in f32 buffers (a ctypes float return
    # would pass through a Python double and quiet signalling NaNs).
    allp = np.arange(65536, dtype=np.uint16).reshape(512, 128)
    ids = np.arange(512, dtype=np.int32)
    h = R.run(lambda g: g.get_rows(allp, R.F16, 128, ids))
    np.testing.assert_array_equal(bits(h), bits(allp.view(np.float16).astype(np.float32)))
    b = R.run(lambda g: g.get_rows(allp, R.BF16, 128, ids))
    np.testing.assert_array_equal(bits(b), (allp.astype(np.uint32) << 16))


def test_fp32_to_half_and_bf16_rounding():
    L = R.lib()
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 4000),
                        np.array([65504, 65519.99, 65520, 1e-8, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, -0.0, np.inf,
                                  -np.inf], np.float32)]).astype(np.float32)
    got = np.array([L.orc_fp32_to_fp16(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(got, x.astype(np.float16).view(np.uint16))
    got = np.array([L.orc_fp32_to_bf16(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(got, F.f32_to_bf16_bits(x))
    # round half to even at the bf16 boundary: 1 + 2^-8 ties to 1, 1 + 3*2^-8 ties up
    np.testing.assert_array_equal(F.f32_to_bf16_bits(np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8], np.float32)),
                                  [0x3F80, 0x3F82])


def q8_brute(raw, ne0, ids):
    """Pure-Python dequant of Q8_0 rows: d from the f16 bit pattern by its
    definition, each element q*d (exact), no numpy arithmetic."""
    out = []
    nb = ne0 // 32
    for i in ids:
        row = bytes(raw[i])
        vals = []
        for b in range(nb):
            blk = row[34 * b: 34 * b + 34]
            (dh,) = struct.unpack("<H", blk[:2])
            sign = -1.0 if dh & 0x8000 else 1.0
            e, m = (dh >> 10) & 31, dh & 1023
            d = sign * (m * 2.0 ** -24 if e == 0 else (1 + m / 1024.0) * 2.0 ** (e - 15))
            for q in struct.unpack("<32b", blk[2:]):
                vals.append(q * d)
        out.append(vals)
    return np.array(out, np.float32)


@pytest.mark.parametrize("kind", ["f32", "f16", "bf16", "q8_0"])
def test_get_rows_closed_form(kind):
    rng = np.random.default_rng(2)
    rows, ne0 = 40, 128
    ids = rng.integers(0, rows, 23).astype(np.int32)
    if kind == "f32":
        tab = rng.standard_normal((rows, ne0)).astype(np.float32)
        ref, t = tab[ids], R.F32
    elif kind == "f16":
        tab = F.f32_to_f16_bits(rng.standard_normal((rows, ne0)))
        ref, t = F.f16_bits_to_f32(tab[ids]), R.F16
    elif kind == "bf16":
        tab = F.f32_to_bf16_bits(rng.standard_normal((rows, ne0)))
        ref, t = F.bf16_bits_to_f32(tab[ids]), R.BF16
    else:
        d, qs = F.q8_0_unpack(F.q8_0_synthetic(rng, rows, ne0), ne0)
        d = d.copy()
        d[3], d[4], d[5] = 0x0000, 0x8001, 0xBC00  # zero, negative subnormal, -1
        ids[:3] = [3, 4, 5]
        tab = F.q8_0_pack(d, qs)
        ref, t = q8_brute(tab, ne0, ids), R.Q8_0
        np.testing.assert_array_equal(bits(F.q8_0_dequant(tab, ne0)[ids]), bits(ref))
    got = R.run(lambda g: g.get_rows(tab, t, ne0, ids))
    np.testing.assert_array_equal(bits(got), bits(ref))


def test_get_rows_rejects_out_of_range():
    tab = np.zeros((4, 32), np.float32)
    with pytest.raises(RuntimeError):
        R.run(lambda g: g.get_rows(tab, R.F32, 32, np.array([4], np.int32)))


def test_q8_0_pack_roundtrip_and_quantizer():
    rng = np.random.default_rng(3)
    raw = F.q8_0_synthetic(rng, 7, 256)
    d, qs = F.q8_0_unpack(raw, 256)
    np.testing.assert_array_equal(F.q8_0_pack(d, qs), raw)
    x = rng.standard_normal((5, 256)).astype(np.float32)
    qraw = F.q8_0_quantize(x)
    deq = F.q8_0_dequant(qraw, 256)
    dd = F.f16_bits_to_f32(F.q8_0_unpack(qraw, 256)[0])
    assert (np.abs(deq - x).reshape(5, 8, 32) <= 0.51 * dd[:, :, None] + 1e-3 * np.abs(x).max()).all()


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------

def test_rms_norm_invariants():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((64, 1024)).astype(np.float32)
    y = R.run(lambda g: g.rms_norm(x, np.float32(0.0)))
    # unit mean square
    assert np.abs((y.astype(np.float64) ** 2).mean(axis=1) - 1).max() < 1e-6
    # with eps = 0 a power-of-two rescale of the row changes nothing, bit for bit
    y4 = R.run(lambda g: g.rms_norm(x * np.float32(4.0), np.float32(0.0)))
    np.testing.assert_array_equal(bits(y), bits(y4))
    # against the textbook double form: within 2 ulp
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True))
    assert (np.abs(y - ref) <= 2 * ULP * np.abs(ref) + 1e-30).all()
    # zero row: scale 1/sqrt(eps) times 0; constant row: c / sqrt(c^2 + eps)
    z = R.run(lambda g: g.rms_norm(np.zeros((1, 64), np.float32), np.float32(1e-6)))
    assert (z == 0).all()
    c = np.full((1, 64), 0.5, np.float32)
    yc = R.run(lambda g: g.rms_norm(c, np.float32(1e-6)))
    assert abs(float(yc[0, 0]) - 0.5 / math.sqrt(0.25 + 1e-6)) < 2 * ULP


def test_rms_norm_eps_is_inside_the_sqrt():
    x = np.full((1, 16), 1e-3, np.float32)
    eps = np.float32(1e-6)
    y = R.run(lambda g: g.rms_norm(x, eps))[0, 0]
    inside = 1e-3 / math.sqrt(1e-6 + 1e-6)
    outside = 1e-3 / (math.sqrt(1e-6) + 1e-6)
    assert abs(y - inside) < 1e-5 < abs(y - outside)


# ---------------------------------------------------------------------------
# rope
# ---------------------------------------------------------------------------

def _theta_recurrence(p, i, base, n_dims):
    ts = np.float32(base) ** np.float32(-2.0 / n_dims)
    ts = np.float32(math.pow(np.float32(base), np.float32(-2.0) / np.float32(n_dims)))
    th = np.float32(p)
    for _ in range(i):
        th = np.float32(th * ts)
    return th, ts


def test_rope_identities_and_double_closed_form():
    rng = np.random.default_rng(6)
    T, H, hd = 24, 3, 128
    x = rng.standard_normal((T, H, hd)).astype(np.float32)
    pos = np.concatenate([[0], rng.integers(1, 8192, T - 1)]).astype(np.int32)
    y = R.run(lambda g: g.rope_neox(x, pos, hd, np.float32(1e6)))
    np.testing.assert_array_equal(bits(y[0]), bits(x[0]))  # p = 0 is the identity
    half = hd // 2
    n_in = np.hypot(x[..., :half].astype(np.float64), x[..., half:])
    n_out = np.hypot(y[..., :half].astype(np.float64), y[..., half:])
    assert np.abs(n_out - n_in).max() <= 4 * ULP * n_in.max()  # rotation keeps each pair's length
    for t in range(1, T):
        for i in (0, 1, 7, 31, 63):
            th, _ = _theta_recurrence(int(pos[t]), i, 1e6, hd)
            c, s = math.cos(float(th)), math.sin(float(th))
            x0, x1 = x[t, :, i].astype(np.float64), x[t, :, i + half].astype(np.float64)
            scale = np.maximum(np.abs(x0), np.abs(x1))
            assert (np.abs(y[t, :, i] - (x0 * c - x1 * s)) <= 4 * ULP * scale).all()
            assert (np.abs(y[t, :, i + half] - (x0 * s + x1 * c)) <= 4 * ULP * scale).all()


def test_rope_recurrence_is_not_the_pow_form_at_large_positions():
    """ggml-CPU's cache multiplies theta by theta_scale once per pair in f32; a
    pos*theta_scale^i evaluation drifts from it by ~1 ulp per step, which at
    p = 8191 is far outside 1e-5 -- so the restatement (and the kernel) must
    replay the recurrence."""
    p, n_dims, base = 8191, 128, 1e6
    half = n_dims // 2
    x = np.zeros((half, 1, n_dims), np.float32)
    for i in range(half):
        x[i, 0, i] = 1.0  # row i probes pair i: y[i] = cos(theta_i)
    y = R.run(lambda g: g.rope_neox(x, np.full(half, p, np.int32), n_dims, np.float32(base)))
    gap = 0.0
    for i in range(half):
        th_rec, ts = _theta_recurrence(p, i, base, n_dims)
        th_pow = np.float32(np.float32(p) * np.float32(math.pow(float(ts), i)))
        assert abs(y[i, 0, i] - math.cos(float(th_rec))) < 1e-6
        gap = max(gap, abs(math.cos(float(th_rec)) - math.cos(float(th_pow))))
    assert gap > 1e-5


# ---------------------------------------------------------------------------
# SwiGLU, Snake, leaky
# ---------------------------------------------------------------------------

def test_swiglu_double_closed_form():
    rng = np.random.default_rng(8)
    g_ = (rng.standard_normal((16, 3072)) * 5).astype(np.float32)
    u = rng.standard_normal((16, 3072)).astype(np.float32)
    y = R.run(lambda g: R.swiglu(g, g_, u))
    gd = g_.astype(np.float64)
    ref = gd / (1 + np.exp(-gd)) * u
    assert (np.abs(y - ref) <= 4 * ULP * np.abs(ref) + 1e-37).all()
    yg = R.run(lambda g: g.glu_swiglu(np.concatenate([g_, u], axis=1), False))
    np.testing.assert_array_equal(bits(yg), bits(y))
    ys = R.run(lambda g: g.glu_swiglu(np.concatenate([u, g_], axis=1), True))
    np.testing.assert_array_equal(bits(ys), bits(y))


def test_snake_double_closed_form():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((100, 64)).astype(np.float32)
    a = np.exp(rng.uniform(np.log(0.1), np.log(10), 64)).astype(np.float32)
    y = R.run(lambda g: R.snake(g, x, a))
    ad = a.astype(np.float64)
    ref = x + np.sin(ad * x) ** 2 / ad
    assert (np.abs(y - ref) <= 8 * ULP * np.maximum(np.abs(ref), 1e-3)).all()


def test_guarded_snake_double_closed_form_and_guard():
    """codec_snake (omnivoice/codec.cpp:51-68) against x + sin(a x)^2 / (a + 1e-9) in
    double. The guard shows where the Snake term is visible next to x: alpha = 0
    (0/0 without it) and alphas near 1e-9 with |x| ~ 1e4. Dropping it (the
    Kokoro form) fails the same check."""
    rng = np.random.default_rng(21)
    C = 64
    x = rng.standard_normal((50, C)).astype(np.float32)
    a = np.exp(rng.uniform(np.log(1e-9), np.log(10), C)).astype(np.float32)
    a[:5] = np.array([0.0, 1e-9, 3e-9, 1e-7, 1e-4], np.float32)
    x[:, :5] *= 1e4
    y = R.run(lambda g: R.snake_guarded(g, x, a))
    ad = a.astype(np.float64)
    den = np.float32(a + np.float32(1e-9)).astype(np.float64)  # the guard add is one f32 rounding

    def ok(v, d):
        with np.errstate(invalid="ignore", divide="ignore"):
            ref = x + np.sin(ad * x) ** 2 / d
            return (np.abs(v - ref) <= 8 * ULP * np.maximum(np.abs(ref), 1e-3)).all()
    assert ok(y, den)
    with np.errstate(invalid="ignore"):
        assert not ok(R.run(lambda g: R.snake(g, x, a)), den)
    assert not ok(y, ad)
    np.testing.assert_array_equal(y[:, 0], x[:, 0])  # alpha = 0: sin(0)^2 / 1e-9 = 0


def test_snake_beta_double_closed_form():
    """codec_snake_beta against x + sin(t)^2 / (e^lb + 1e-9), t = x e^la, in double
    after the f32 roundings of the two exps, the guard and the product t (a
    large alpha over a small beta amplifies t's rounding far beyond y's ulp,
    so t is rounded as ggml rounds it). Tolerance: 8 ulp of the larger of |x|
    and the Snake term. Swapping the curves fails."""
    rng = np.random.default_rng(22)
    C = 48
    x = rng.standard_normal((40, C)).astype(np.float32)
    la = rng.uniform(-3, 3, C).astype(np.float32)
    lb = rng.uniform(-3, 3, C).astype(np.float32)
    y = R.run(lambda g: R.snake_beta(g, x, la, lb))

    def close(ca, cb):
        a = np.exp(ca.astype(np.float64)).astype(np.float32)
        b = np.float32(np.exp(cb.astype(np.float64)).astype(np.float32) + np.float32(1e-9)).astype(np.float64)
        t = (x * a).astype(np.float64)  # one f32 rounding, as ggml_mul
        r = np.sin(t) ** 2 / b
        scale = np.maximum(np.maximum(np.abs(x), r), 1e-3)
        return (np.abs(y - (x + r)) <= 8 * ULP * scale).all()
    assert close(la, lb)
    assert not close(lb, la)


def test_exp_is_correctly_rounded_almost_everywhere():
    """ggml_exp: glibc expf against e^x in double rounded once to f32 (the
    correctly rounded value unless e^x lies within ~2^-52 of a rounding
    boundary): every result within one ulp, nearly all identical (glibc's
    expf is documented at 0.502 ulp and lands on the other side of a
    midpoint for ~0.06% of arguments). Overflow to inf, underflow to
    subnormals and zero, and exp(0) = 1 exactly."""
    rng = np.random.default_rng(23)
    x = np.concatenate([rng.uniform(-104, 89, 200000), [0.0, -0.0, 88.8, -104.0, -87.5, 1e-30, np.inf, -np.inf]])
    x = x.astype(np.float32).reshape(-1, 8)
    y = R.run(lambda g: g.exp(x)).reshape(-1)
    with np.errstate(over="ignore"):
        ref = np.exp(x.astype(np.float64)).astype(np.float32).reshape(-1)
    same = bits(y) == bits(ref)
    assert same.mean() > 0.999
    diff = np.abs(bits(y).astype(np.int64) - bits(ref).astype(np.int64))
    assert diff.max() <= 1
    xs = x.reshape(-1)
    assert y[xs == 0].tolist() == [1.0, 1.0] and y[xs == np.inf][0] == np.inf and y[xs == -np.inf][0] == 0
    assert y[xs == np.float32(88.8)][0] == np.inf and 0 < y[xs == np.float32(-87.5)][0] < 2 ** -126


def test_scale_bias_rounding():
    """ggml_scale (b == 0) is one multiply, so -0 stays -0; ggml_scale_bias with
    b != 0 rounds x*s + b once. Checked against numpy's f32 multiply and against
    the exact value: x*s is exact in double, so double(x*s) + b rounds once in
    double and once more to f32, which is the single rounding except when the
    double sum lands on an f32 midpoint (excluded). A two-rounding mul+add is
    planted and fails."""
    rng = np.random.default_rng(24)
    x = rng.standard_normal((1000, 16)).astype(np.float32)
    x[0, :4] = [-0.0, 0.0, np.inf, np.nan]
    s, b = np.float32(0.7853982), np.float32(-0.3183099)
    y0 = R.run(lambda g: g.scale(x, s))
    np.testing.assert_array_equal(bits(y0), bits(x * s))
    assert np.signbit(y0[0, 0])
    y = R.run(lambda g: g.scale_bias(x, s, b)).reshape(-1)
    d = x.reshape(-1).astype(np.float64) * np.float64(s) + np.float64(b)
    ref = d.astype(np.float32)
    lo = np.nextafter(ref, np.float32(-np.inf)).astype(np.float64)
    hi = np.nextafter(ref, np.float32(np.inf)).astype(np.float64)
    mid = (d == (ref.astype(np.float64) + lo) / 2) | (d == (ref.astype(np.float64) + hi) / 2)
    fin = np.isfinite(d) & ~mid
    np.testing.assert_array_equal(bits(y[fin]), bits(ref[fin]))
    two = (x.reshape(-1) * s + b).astype(np.float32)
    assert (bits(two[fin]) != bits(ref[fin])).any()
    # with s == 1 (the Snake guards) every evaluation order agrees
    np.testing.assert_array_equal(bits(R.run(lambda g: g.scale_bias(x, np.float32(1.0), np.float32(1e-9)))),
                                  bits(x + np.float32(1e-9)))


def test_branch_average_order_and_invariants():
    """sum_scale_leaky (waveform-decoder.cpp:214-225): the terms are added in
    order, so (1e8 + 1) - 1e8 is 0 where another order gives 1; two equal
    terms scaled by 0.5 give back the term exactly (doubling and halving are
    exact), so y = leaky(t) bit for bit; one term is the bare leaky."""
    big = np.array([[1e8, 3.0, -2.0, 5.0]], np.float32)
    one = np.array([[1.0, 1.0, 1.0, 1.0]], np.float32)
    cur, y = R.run(lambda g: R.sum_scale_leaky(g, [big, one, -big], np.float32(1 / 3), np.float32(0.1)))
    assert cur[0, 0] == 0.0 and cur[0, 1] == np.float32(np.float32(3.0 + 1.0 - 3.0) * np.float32(1 / 3))
    cur2, _ = R.run(lambda g: R.sum_scale_leaky(g, [big, -big, one], np.float32(1 / 3), np.float32(0.1)))
    assert cur2[0, 0] == np.float32(1 / 3)
    rng = np.random.default_rng(25)
    t = rng.standard_normal((30, 64)).astype(np.float32)
    t[0, :4] = [-0.0, np.nan, 1e-45, -3e-39]
    c, y = R.run(lambda g: R.sum_scale_leaky(g, [t, t], np.float32(0.5), np.float32(0.1)))
    np.testing.assert_array_equal(bits(c[np.isfinite(t)]), bits(t[np.isfinite(t)]))
    ly = R.run(lambda g: g.leaky_relu(t, np.float32(0.1)))
    np.testing.assert_array_equal(bits(y), bits(ly))
    c1, y1 = R.run(lambda g: R.sum_scale_leaky(g, [t], np.float32(1.0), np.float32(0.1)))
    np.testing.assert_array_equal(bits(y1), bits(ly))


def _softmax_double(w):
    e = np.exp(w.astype(np.float64) - w.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def test_soft_max_closed_form_and_exact_cases():
    """soft_max_ext against the double softmax of the same f32 w = x*scale + mask:
    within 3 ulp (one expf, the f32 reciprocal, one multiply). A uniform row
    gives exactly (float)(1/n); -inf mask entries give exactly 0; every row
    sums to 1 within n ulp; scaling after adding the mask is planted and fails."""
    rng = np.random.default_rng(26)
    H, T, N = 4, 9, 300
    x = rng.standard_normal((H, T, N)).astype(np.float32) * 4
    mask = rng.uniform(-3, 0, (T, N)).astype(np.float32)
    mask[:, -50:] = -np.inf
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    y = R.run(lambda g: g.soft_max_ext(x, mask, scale))
    w = x * scale + mask
    ref = _softmax_double(w)
    assert (np.abs(y - ref) <= 3 * ULP * ref + 1e-45).all()
    assert (y[..., -50:] == 0).all()
    assert np.abs(y.astype(np.float64).sum(-1) - 1).max() <= N * ULP
    wrong = _softmax_double((x + mask) * scale)
    assert not (np.abs(y - wrong) <= 3 * ULP * wrong + 1e-45).all()
    u = R.run(lambda g: g.soft_max_ext(np.full((2, 37), 0.3, np.float32), None, np.float32(1.0)))
    assert (u == np.float32(1.0 / 37)).all()


def test_soft_max_mask_head_broadcast():
    """Head h reads mask head h % mask_heads (ggml's i12 = i02 % ne12) and score
    row i1 reads mask row i1 (the mask may have more rows)."""
    rng = np.random.default_rng(27)
    H, T, N = 6, 5, 40
    x = rng.standard_normal((H, T, N)).astype(np.float32)
    mask = rng.uniform(-4, 0, (2, T + 3, N)).astype(np.float32)
    y = R.run(lambda g: g.soft_max_ext(x, mask, np.float32(0.5)))
    for h in range(H):
        one = R.run(lambda g: g.soft_max_ext(x[h], mask[h % 2, :T], np.float32(0.5)))
        np.testing.assert_array_equal(bits(y[h]), bits(one))
    other = R.run(lambda g: g.soft_max_ext(x[1], mask[0, :T], np.float32(0.5)))
    assert (bits(y[1]) != bits(other)).any()


def test_leaky_relu_signed_zero_and_nan():
    x = np.array([[-0.0, 0.0, np.nan, -np.nan, np.inf, -np.inf, -1e-45, 2.5, -2.5, -3e-39]], np.float32)
    y = R.run(lambda g: g.leaky_relu(x, np.float32(0.1)))[0]
    assert y[0] == 0 and not np.signbit(y[0])  # -0 -> +0
    assert y[2] == 0 and y[3] == 0  # NaN -> 0
    assert y[4] == np.inf and y[5] == -np.inf
    assert y[6] == 0 and not np.signbit(y[6])  # 0.1 * -1e-45 underflows to -0, then 0 + -0 = +0
    assert y[7] == np.float32(2.5) and y[8] == np.float32(-0.25)
    assert y[9] == np.float32(np.float32(0.1) * np.float32(-3e-39))
    # a max(x, slope*x) formulation differs exactly on those cases
    alt = np.maximum(x[0], np.float32(0.1) * x[0])
    assert np.signbit(alt[0]) or np.isnan(alt[2])


# ---------------------------------------------------------------------------
# the ggml-style thread split does not change results
# ---------------------------------------------------------------------------

def _step_graph(rng, T=64):
    x = rng.standard_normal((T, 1024)).astype(np.float32)
    w = F.f32_to_bf16_bits(rng.normal(1, 0.1, 1024))
    q = rng.standard_normal((T, 16, 128)).astype(np.float32)
    k = rng.standard_normal((T, 8, 128)).astype(np.float32)
    wq = F.f32_to_bf16_bits(rng.normal(1, 0.1, 128))
    pos = rng.integers(0, 8192, T).astype(np.int32)
    gt = rng.standard_normal((T, 3072)).astype(np.float32)
    tab = F.q8_0_synthetic(rng, 100, 1024)
    codes = rng.integers(0, 100, (3, T)).astype(np.int32)
    a = rng.standard_normal((T, 512)).astype(np.float32)
    al = np.exp(rng.uniform(-2, 2, 512)).astype(np.float32)

    def build(g):
        return [R.rms_norm_w(g, x, w, np.float32(1e-6), R.BF16),
                *R.qk_norm_rope(g, q, k, wq, wq, np.float32(1e-6), pos, 128, np.float32(1e6), R.BF16),
                R.swiglu(g, gt, gt), R.sum_code_embeddings(g, [tab] * 3, R.Q8_0, 1024, codes),
                R.snake(g, a, al), R.add_leaky(g, a, a, np.float32(0.1))[1]]
    return build


def test_thread_split_invariance():
    build = _step_graph(np.random.default_rng(10))
    one = R.run(build, n_threads=1)
    for nth in (3, 8):
        many = R.run(build, n_threads=nth)
        for a, b in zip(one, many):
            np.testing.assert_array_equal(bits(a), bits(b))


# ---------------------------------------------------------------------------
# ggml_cont of strided views
# ---------------------------------------------------------------------------

def _ggml_view(a, perm):
    """(ne, nb) of the ggml view that numpy's a.transpose(perm) is: numpy axis
    order reversed into ggml dims."""
    t = a.transpose(perm)
    return list(t.shape[::-1]), list(t.strides[::-1]), t


@pytest.mark.parametrize("shape,perm", [((37, 70), (1, 0)), ((5, 9, 130), (1, 2, 0)), ((3, 4, 66, 7), (0, 3, 2, 1)),
                                        ((2, 3, 5, 7), (3, 2, 1, 0)), ((64, 64), (1, 0)), ((1, 33), (1, 0))])
def test_cont_against_numpy_transpose(shape, perm):
    """ggml_cont of a transposed/permuted view equals numpy's own transposed
    copy (an independent implementation), on non-square extents so that a
    swapped index or stride cannot pass, at 1 and several threads."""
    rng = np.random.default_rng(sum(shape))
    a = rng.standard_normal(shape).astype(np.float32)
    ne, nb, t = _ggml_view(a, perm)
    for nth in (1, 3, 8):
        g = R.Graph()
        y = g.cont_f32(a, ne, nb)
        g.compute(nth)
        np.testing.assert_array_equal(bits(y.reshape(t.shape)), bits(np.ascontiguousarray(t)))


def test_cont_identities():
    """A contiguous view copies to itself; transposing twice gives back the
    source; a view at an offset equals numpy's slice; and a planted mistake
    (extents and strides of dims 0 and 1 both left unswapped: the transpose
    dropped) does not equal the transposed copy."""
    rng = np.random.default_rng(7)
    a = rng.standard_normal((6, 11, 40)).astype(np.float32)
    g = R.Graph()
    same = g.cont_f32(a, [40, 11, 6], [4, 160, 1760])
    ne, nb, _ = _ggml_view(a, (0, 2, 1))
    once = g.cont_f32(a, ne, nb)
    g.compute(2)
    np.testing.assert_array_equal(bits(same.reshape(a.shape)), bits(a))
    g = R.Graph()
    twice = g.cont_f32(once, [40, 11, 6], [44, 4, 1760])
    sub = g.cont_f32(a, [7, 3, 2], [8, 160, 1760 * 3], offset=4 * (1 + 40 * 2 + 440 * 1))
    planted = g.cont_f32(a, [ne[1], ne[0]] + ne[2:], [nb[1], nb[0]] + nb[2:])
    g.compute(1)
    np.testing.assert_array_equal(bits(twice.reshape(a.shape)), bits(a))
    np.testing.assert_array_equal(bits(sub.reshape(2, 3, 7)), bits(a[1::3, 2:5, 1:15:2]))
    assert not np.array_equal(bits(planted), bits(once))
    with pytest.raises(ValueError):
        R.Graph().cont_f32(a, [41, 11, 6], [4, 160, 1760])


# ---------------------------------------------------------------------------
# binary ops with b repeated to a's shape
# ---------------------------------------------------------------------------

def _tile_to(b, shape):
    """numpy's own tiling of b to `shape` (ggml's repeat: index modulo b's extent)."""
    b = b.reshape((1,) * (len(shape) - b.ndim) + b.shape)
    return np.tile(b, [s // t for s, t in zip(shape, b.shape)])


@pytest.mark.parametrize("ashape,bshape", [((6, 37), (6, 1)), ((2, 3, 40), (1, 3, 1)), ((4, 6, 12), (2, 3, 4)),
                                           ((3, 5, 7, 8), (1, 5, 1, 8)), ((3, 5, 7, 8), (1, 1, 1, 1)),
                                           ((9, 16), (1, 16)), ((9, 16), (3, 8))])
def test_binbcast_against_numpy_tile(ashape, bshape):
    """ggml's repeat semantics against numpy's tile, for every op, at 1 and
    several threads; the same-shape and one-row forms agree with the plain
    binary node; and block repetition (a planted mistake: b's index i // r
    instead of i % n) differs wherever b has more than one value along a
    repeated dim."""
    rng = np.random.default_rng(sum(ashape) + 7 * sum(bshape))
    a = rng.standard_normal(ashape).astype(np.float32)
    b = (rng.standard_normal(bshape) + 3.0).astype(np.float32)
    bt = _tile_to(b, ashape)
    for op, f in ((R.OP_ADD, np.add), (R.OP_MUL, np.multiply), (R.OP_DIV, np.divide)):
        for nth in (1, 4):
            g = R.Graph()
            y = g.binbcast(op, a, b)
            g.compute(nth)
            np.testing.assert_array_equal(bits(y), bits(f(a, bt)))
    block = b
    for axis, (s_, t_) in enumerate(zip(ashape, bshape)):
        block = np.repeat(block, s_ // t_, axis=axis)
    if any(t_ > 1 and s_ > t_ for s_, t_ in zip(ashape, bshape)):
        assert not np.array_equal(bits(a + block), bits(a + bt))


def test_binbcast_reduces_to_the_plain_forms():
    rng = np.random.default_rng(11)
    a = rng.standard_normal((5, 64)).astype(np.float32)
    row = rng.standard_normal(64).astype(np.float32)
    col = rng.standard_normal((5, 1)).astype(np.float32)
    g = R.Graph()
    y1 = g.binbcast(R.OP_ADD, a, row.reshape(1, 64))
    y2 = g.add(a, row)
    y3 = g.binbcast(R.OP_MUL, a, col)
    y4 = g.mul(a, col)
    g.compute(2)
    np.testing.assert_array_equal(bits(y1), bits(y2))
    np.testing.assert_array_equal(bits(y3), bits(y4))
    with pytest.raises(ValueError):
        R.Graph().binbcast(R.OP_ADD, a, np.zeros((3, 64), np.float32))


@pytest.mark.parametrize("dim", [0, 1, 2, 3])
def test_concat_against_an_element_loop(dim):
    """concat along each ggml dimension against the definition, element by
    element (tiny shapes), and a planted mistake (the operands swapped)
    rejected."""
    rng = np.random.default_rng(dim)
    ashape = [2, 3, 4, 5]            # numpy (ne3, ne2, ne1, ne0)
    bshape = list(ashape)
    bshape[3 - dim] = 2
    a = rng.standard_normal(ashape).astype(np.float32)
    b = rng.standard_normal(bshape).astype(np.float32)
    y = R.concat(a, b, dim)
    na = ashape[3 - dim]
    for idx in np.ndindex(*y.shape):
        k = idx[3 - dim]
        want = a[idx] if k < na else b[tuple(k - na if j == 3 - dim else v for j, v in enumerate(idx))]
        assert bits(y[idx]) == bits(want)
    assert not np.array_equal(bits(R.concat(b, a, dim)), bits(y))


# ---------------------------------------------------------------------------
# the codec / vocoder elementwise ops, sub and LayerNorm
# ---------------------------------------------------------------------------

def _ulps(got, want):
    """Distance in f32 ulps of `want`'s binade (want in double)."""
    want = np.asarray(want, np.float64)
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    return np.abs(np.asarray(got, np.float64) - want) / ulp


def _grid():
    rng = np.random.default_rng(77)
    return np.concatenate([rng.standard_normal(4000) * 3, rng.uniform(-30, 30, 2000),
                           np.linspace(-1e-3, 1e-3, 100)]).astype(np.float32).reshape(61, -1)


def test_tanh_sigmoid_elu_gelu_against_double_closed_forms():
    x = _grid()
    g = R.Graph()
    t, s, e, ge = g.tanh(x), g.sigmoid(x), g.elu(x), g.gelu_erf(x)
    g.compute(2)
    xd = x.astype(np.float64)
    assert _ulps(t, np.tanh(xd)).max() <= 2
    assert _ulps(s, 1.0 / (1.0 + np.exp(-xd))).max() <= 4
    pos = x > 0
    assert np.array_equal(bits(e[pos]), bits(x[pos]))
    assert _ulps(e[~pos], np.expm1(xd[~pos])).max() <= 2
    import math
    gd = 0.5 * xd * (1.0 + np.vectorize(math.erf)(xd / math.sqrt(2.0)))
    # ggml's formula adds erff's result to 1 in f32, so for x < 0 the error is
    # absolute: about |x|/2 times an ulp of 1 (the cancellation), plus a few
    # ulps of the result
    bound = 2.0 * np.abs(xd) * 2.0 ** -24 + 4 * np.spacing(np.abs(gd).astype(np.float32))
    assert (np.abs(ge - gd) <= bound).all()
    # a planted mistake: the tanh approximation of GELU is not this op
    ga = 0.5 * xd * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.abs(ge - ga).max() > 1e-4


def test_elementwise_special_values():
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 88.0, -104.0, 1e30, -1e30, 3.0],
                  dtype=np.float32).reshape(1, -1)
    g = R.Graph()
    t, s, e, c = g.tanh(sp), g.sigmoid(sp), g.elu(sp), g.clamp(sp, -1.0, 1.0)
    g.compute(1)
    assert bits(t[0, 0]) == bits(np.float32(0.0)) and bits(t[0, 1]) == bits(np.float32(-0.0))
    assert t[0, 2] == 1.0 and t[0, 3] == -1.0 and np.isnan(t[0, 4])
    assert s[0, 0] == 0.5 and s[0, 2] == 1.0 and s[0, 3] == 0.0 and np.isnan(s[0, 4])
    assert bits(e[0, 1]) == bits(np.float32(-0.0)) and e[0, 3] == -1.0 and np.isnan(e[0, 4])
    # ggml's clamp is MAX(MIN(x, max), min): NaN gives max; fminf/fmaxf would give min or max differently
    assert c[0, 4] == 1.0
    np.testing.assert_array_equal(c[0, [0, 2, 3, 9, 10, 11]], np.float32([0.0, 1.0, -1.0, 1.0, -1.0, 1.0]))


def test_sub_and_its_repeat_forms():
    rng = np.random.default_rng(5)
    a = rng.standard_normal((6, 40)).astype(np.float32)
    b = rng.standard_normal((6, 40)).astype(np.float32)
    row = rng.standard_normal(40).astype(np.float32)
    col = rng.standard_normal((6, 1)).astype(np.float32)
    g = R.Graph()
    y1, y2, y3 = g.sub(a, b), g.sub(a, row), g.sub(a, col)
    y4 = g.binbcast(R.OP_SUB, a, rng.standard_normal((3, 20)).astype(np.float32))
    g.compute(2)
    np.testing.assert_array_equal(bits(y1), bits(a - b))
    np.testing.assert_array_equal(bits(y2), bits(a - row))
    np.testing.assert_array_equal(bits(y3), bits(a - col))
    assert not np.array_equal(bits(y1), bits(b - a))


def test_norm_against_double_and_invariants():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((16, 1024)) * 3 + 5).astype(np.float32)
    g = R.Graph()
    y = g.norm(x, 1e-6)
    const = g.norm(np.full((2, 64), 7.0, np.float32), 1e-5)
    tiny = g.norm((rng.standard_normal((2, 64)) * 1e-4).astype(np.float32), 1e-5)
    g.compute(3)
    xd = x.astype(np.float64)
    m = xd.mean(axis=1, keepdims=True)
    want = (xd - m) / np.sqrt(((xd - m) ** 2).mean(axis=1, keepdims=True) + 1e-6)
    assert np.abs(y - want).max() <= 1e-5
    assert np.abs(y.mean(axis=1)).max() < 1e-5 and np.abs(y.var(axis=1) - 1).max() < 1e-4
    assert (const == 0).all()
    # eps is inside the sqrt: with variance ~1e-8 the result is far below 1 in size
    assert np.abs(tiny).max() < 0.1


# ---------------------------------------------------------------------------
# ggml_pad / ggml_pad_ext, ggml_pad_reflect_1d, ggml_repeat
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape,lp,rp", [((7,), [2], [3]), ((4, 9), [0, 1], [5, 2]), ((3, 1, 5), [1, 0, 0], [0, 7, 2]),
                                         ((2, 3, 4, 5), [1, 2, 0, 1], [2, 0, 3, 0]), ((6, 10), [0, 0], [0, 0])])
def test_pad_ext_is_numpy_constant_pad(shape, lp, rp):
    """ggml_pad_ext: numpy's zero pad, ggml's (lp_d, rp_d) per dim d on the
    reversed numpy axis; lp and rp swapped differ."""
    x = np.random.default_rng(len(shape) + sum(lp)).standard_normal(shape).astype(np.float32) + 3
    nd = len(shape)
    ref = np.pad(x, [(lp[nd - 1 - a], rp[nd - 1 - a]) for a in range(nd)])
    got = R.run(lambda g: g.pad_ext(x, lp, rp))
    assert got.shape == ref.shape and np.array_equal(got, ref)
    if lp != rp:
        assert not np.array_equal(R.run(lambda g: g.pad_ext(x, rp, lp)), ref)


def test_pad_spreads_frames_with_zeros():
    """kokoro/operations.cpp:190-193: padding the unit axis of [C, 1, L] by
    stride - 1 puts stride - 1 zero frames after every frame."""
    C, L, S = 5, 6, 4
    x = np.random.default_rng(3).standard_normal((L, 1, C)).astype(np.float32)   # ggml [C, 1, L]
    got = R.run(lambda g: g.pad(x, [0, S - 1, 0, 0])).reshape(L * S, C)
    ref = np.zeros((L * S, C), np.float32)
    ref[::S] = x[:, 0]
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("shape,p0,p1", [((3, 10), 2, 3), ((16,), 1, 1), ((2, 3, 8), 7, 0), ((4, 5), 0, 4)])
def test_pad_reflect_1d_is_numpy_reflect(shape, p0, p1):
    """ggml_pad_reflect_1d: numpy's 'reflect' (the edge sample not repeated),
    which its 'symmetric' mode (edge repeated) is not; pads of the row's
    length are refused."""
    x = np.random.default_rng(p0 * 10 + p1).standard_normal(shape).astype(np.float32)
    pads = [(0, 0)] * (len(shape) - 1) + [(p0, p1)]
    got = R.run(lambda g: g.pad_reflect_1d(x, p0, p1))
    assert np.array_equal(got, np.pad(x, pads, mode="reflect"))
    if p0 or p1:
        assert not np.array_equal(got, np.pad(x, pads, mode="symmetric"))
    with pytest.raises(ValueError):
        R.Graph().pad_reflect_1d(x, shape[-1], 0)


@pytest.mark.parametrize("shape,target", [((1, 7), (5, 7)), ((3, 1, 4), (3, 2, 4)), ((2, 3), (4, 9)), ((5,), (2, 3, 10)),
                                          ((1, 1, 1, 2), (2, 3, 2, 6))])
def test_repeat_is_numpy_tile(shape, target):
    """ggml_repeat: numpy's tile of x to the target shape (kokoro's
    broadcast_over_time and upsample_nearest_2x, :21-24,113-120)."""
    x = np.random.default_rng(sum(target)).standard_normal(shape).astype(np.float32)
    xs = x.reshape((1,) * (len(target) - x.ndim) + x.shape)
    ref = np.tile(xs, [t // s for t, s in zip(target, xs.shape)])
    assert np.array_equal(R.run(lambda g: g.repeat(x, target)), ref)


def test_repeat_doubles_frames():
    """upsample_nearest_2x (kokoro/operations.cpp:113-120): repeating [C, 1, L]
    to [C, 2, L] duplicates every frame."""
    x = np.random.default_rng(4).standard_normal((6, 1, 5)).astype(np.float32)   # ggml [5, 1, 6]
    got = R.run(lambda g: g.repeat(x, (6, 2, 5))).reshape(12, 5)
    assert np.array_equal(got, np.repeat(x[:, 0], 2, axis=0))


# ---------------------------------------------------------------------------
# ggml_acc (the talker's prefill input)
# ---------------------------------------------------------------------------

def _acc_numpy(a, b, nb1, nb2, nb3, offset):
    """numpy's own strided view of a's copy (ggml's view: byte strides 4, nb1,
    nb2, nb3 from byte `offset`), b added through it."""
    out = a.copy()
    flat = out.reshape(-1)[offset // 4:]
    strides = (nb3, nb2, nb1, 4)[4 - b.ndim:]
    view = np.lib.stride_tricks.as_strided(flat, shape=b.shape, strides=strides)
    view += b
    return out


def _acc_span(b, nb, offset):
    """The byte just past the view's last element."""
    bne = list(b.shape[::-1]) + [1] * (4 - b.ndim)
    return offset + 4 * bne[0] + sum((bne[d] - 1) * nb[d - 1] for d in (1, 2, 3))


@pytest.mark.parametrize("ashape,bshape,nb,offset", [
    ((10, 8), (4, 8), (32, 128, 128), 3 * 32),          # whole rows at a row offset (the codec tail)
    ((10, 8), (1, 8), (32, 32, 32), 9 * 32),            # one row, the last (the x-vector's slot)
    ((10, 8), (3, 5), (32, 96, 96), 1 * 32 + 2 * 4),    # a narrower window at a column offset
    ((6, 5, 12), (2, 3, 4), (48, 240, 480), 4 + 48),    # a 3-D window
    ((40,), (6,), (24, 24, 24), 7 * 4),                 # one row anywhere in a vector
    ((9, 7), (3, 2), (56, 112, 112), 4),                # rows two apart
])
def test_acc_is_numpy_strided_view_add(ashape, bshape, nb, offset):
    """ggml_acc: a's copy with b added through the byte-strided view; an
    offset one element off misses."""
    rng = np.random.default_rng(sum(ashape) + offset)
    a = rng.standard_normal(ashape).astype(np.float32)
    b = rng.standard_normal(bshape).astype(np.float32)
    got = R.run(lambda g: g.acc(a, b, *nb, offset))
    assert np.array_equal(got, _acc_numpy(a, b, *nb, offset))
    shifted = offset + 4 if _acc_span(b, nb, offset + 4) <= a.nbytes else offset - 4
    assert not np.array_equal(R.run(lambda g: g.acc(a, b, *nb, shifted)), got)
    with pytest.raises(ValueError):   # past a's end
        R.Graph().acc(a, b, *nb, a.nbytes)


def prefill_input(g, text, codec, codec_offset, speaker=None, speaker_index=-1, acoustic=None, acoustic_offset=-1,
                  tail_slip=0):
    """The accumulation nodes of build_talker_prefill_input
    (qwen3-tts/talker.cpp:86-118, accumulate_acoustic :23-32) on an oracle
    graph: text (N, H) and codec (n, H) are the projected text stream and the
    codec embeddings (the get_rows output), speaker (H,) the x-vector.
    tail_slip moves the tail's offset (a planted off-by-one)."""
    N, H = text.shape
    nb1, nb2 = 4 * H, 4 * H * N
    if speaker is None:
        out = g.acc(text, codec, nb1, nb2, nb2, codec_offset * nb1)
    else:
        out = text
        if speaker_index > 0:
            out = g.acc(out, codec[:speaker_index], nb1, nb2, nb2, codec_offset * nb1)
        out = g.acc(out, speaker.reshape(1, H), nb1, nb2, nb2, (codec_offset + speaker_index) * nb1)
        if codec.shape[0] - speaker_index - 1 > 0:
            out = g.acc(out, codec[speaker_index + 1:], nb1, nb2, nb2,
                        (codec_offset + speaker_index + 1 + tail_slip) * nb1)
    if acoustic is not None:
        out = g.acc(out, acoustic, nb1, nb2, nb2, acoustic_offset * nb1)
    return out


@pytest.mark.parametrize("codec_offset", [0, 3])
def test_acc_prefill_speaker_slot_rule(codec_offset):
    """tests/qwen3_tts_prompt_slot_test.cpp:356-420 (offset 0) and :527-600
    (a codec run after a text-only prefix): with the x-vector at every slot of
    the codec run, each position is text + (the x-vector at the slot, else its
    codec row), the positions before the run bare text, exactly as the plain
    accumulation; a tail accumulated one row early misses the rule."""
    rng = np.random.default_rng(11 + codec_offset)
    n, H = 5, 16
    N = codec_offset + n
    text = rng.standard_normal((N, H)).astype(np.float32)
    codec = rng.standard_normal((n, H)).astype(np.float32)
    speaker = rng.standard_normal(H).astype(np.float32)
    plain = R.run(lambda g: prefill_input(g, text, codec, codec_offset))
    for si in range(n):
        got = R.run(lambda g: prefill_input(g, text, codec, codec_offset, speaker, si))
        exp = text.copy()
        for j in range(n):
            exp[codec_offset + j] = text[codec_offset + j] + (speaker if j == si else codec[j])
        assert np.array_equal(got, exp)
        keep = np.ones(N, bool)
        keep[codec_offset + si] = False
        assert np.array_equal(got[keep], plain[keep])
        if si < n - 2:
            slipped = R.run(lambda g: prefill_input(g, text, codec, codec_offset, speaker, si, tail_slip=-1))
            assert not np.array_equal(slipped, exp)


def test_acc_prefill_acoustic_block_after_the_codec_sum():
    """accumulate_acoustic (talker.cpp:23-32): the ICL block's summed groups
    are added to the already accumulated streams: (text + codec) + acoustic in
    f32, which the other association misses for some position."""
    rng = np.random.default_rng(12)
    N, n, H, m = 9, 6, 64, 4
    text = rng.standard_normal((N, H)).astype(np.float32)
    codec = rng.standard_normal((n, H)).astype(np.float32)
    acoustic = rng.standard_normal((m, H)).astype(np.float32) * 3
    got = R.run(lambda g: prefill_input(g, text, codec, N - n, acoustic=acoustic, acoustic_offset=N - m))
    exp = text.copy()
    exp[N - n:] = exp[N - n:] + codec
    exp[N - m:] = exp[N - m:] + acoustic
    assert np.array_equal(got, exp)
    other = text.copy()
    other[N - m:] = text[N - m:] + (codec[n - m:] + acoustic)
    other[N - n:N - m] = text[N - n:N - m] + codec[:n - m]
    assert not np.array_equal(got, other)


# ---------------------------------------------------------------------------
# ggml_relu, ggml_neg, ggml_step, ggml_sqrt; ggml_sum_rows, ggml_mean
# ---------------------------------------------------------------------------

_SPECIALS = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.4e38, -3.4e38, 1.0, -1.0],
                     np.float32)


def test_relu_neg_step_sqrt_against_numpy():
    """relu is numpy's maximum with 0 and step its heaviside at 0 on ordered
    values, with ggml's x > 0 forms at the rest (-0 and NaN give +0); neg
    flips exactly the sign bit (zeros and NaN included); sqrt is numpy's
    correctly rounded f32 square root (NaN below zero)."""
    x = np.random.default_rng(21).standard_normal((64, 65)).astype(np.float32) * 10
    x.reshape(-1)[:_SPECIALS.size] = _SPECIALS
    g = R.Graph()
    outs = g.relu(x), g.neg(x), g.step(x), g.sqrt(x)
    g.compute()
    relu, neg, step, sq = outs
    ok = ~np.isnan(x) & (x != 0)
    assert np.array_equal(relu[ok], np.maximum(x[ok], 0))
    assert (relu[~ok].view(np.uint32) == 0).all()
    assert np.array_equal(neg.view(np.uint32), x.view(np.uint32) ^ np.uint32(0x80000000))
    assert np.array_equal(step[~np.isnan(x)], np.heaviside(x[~np.isnan(x)], 0).astype(np.float32))
    assert (step[np.isnan(x)] == 0).all()
    with np.errstate(invalid="ignore"):
        ref = np.sqrt(x)
    assert np.array_equal(sq.view(np.uint32)[x >= 0], ref.view(np.uint32)[x >= 0])
    assert np.isnan(sq[(x < 0) | np.isnan(x)]).all()


def test_sum_rows_and_mean_are_the_rounded_exact_sum():
    """ggml_vec_sum_f32's double accumulation of f32 values: the f32 rounding
    of the exact sum (math.fsum) for every row, over rows with a wide spread
    of magnitudes, which a running f32 sum misses; the mean is that f32 sum
    divided by ne0 in f32, which rounding the exact mean once misses."""
    import math
    rng = np.random.default_rng(22)
    x = (rng.standard_normal((512, 300)) * np.exp(rng.uniform(-8, 8, (512, 300)))).astype(np.float32)
    g = R.Graph()
    s, m = g.sum_rows(x), g.mean(x)
    g.compute()
    exact = np.array([math.fsum(map(float, row)) for row in x])
    assert s.shape == (512, 1) and np.array_equal(s[:, 0], exact.astype(np.float32))
    running = np.cumsum(x, axis=1, dtype=np.float32)[:, -1]
    assert not np.array_equal(s[:, 0], running)
    assert np.array_equal(m[:, 0], exact.astype(np.float32) / np.float32(300))
    assert not np.array_equal(m[:, 0], (exact / 300).astype(np.float32))


# ---------------------------------------------------------------------------
# ggml_diag_mask_inf (the codec encoder's causal attention)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n_past", [0, 2])
def test_diag_mask_inf_is_numpy_triu(n_past):
    """ggml_diag_mask_inf: -inf exactly on numpy's upper triangle above the
    diagonal shifted by n_past (np.triu with k = n_past + 1), x elsewhere;
    k = n_past misses. Followed by the softmax, row 0 at n_past 0 is one-hot
    and every row sums to 1 with zeros where masked."""
    x = np.random.default_rng(23 + n_past).standard_normal((3, 7, 9)).astype(np.float32)
    got = R.run(lambda g: g.diag_mask_inf(x, n_past))
    up = np.triu(np.ones((7, 9), bool), k=n_past + 1)
    assert np.array_equal(got, np.where(up, np.float32(-np.inf), x))
    assert not np.array_equal(got, np.where(np.triu(np.ones((7, 9), bool), k=n_past), np.float32(-np.inf), x))
    g = R.Graph()
    p = g.soft_max_ext(g.diag_mask_inf(x, n_past), None, 0.25)
    g.compute()
    assert (p[:, up] == 0).all() and np.allclose(p.sum(-1), 1, atol=1e-6)
    if n_past == 0:
        assert (p[:, 0, 0] == 1).all()

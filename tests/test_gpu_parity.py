"""GPU parity: every libsynth_hip entry point against the ggml-CPU restatement on
the same seeded inputs, through the C ABI.

Bars: bit-exact for gathers, sums of gathers, adds, leaky-ReLU, scale and the
branch average (compared as raw 32-bit patterns, NaN payloads included); for
RMSNorm, SwiGLU and Snake an elementwise relative error <= 1e-5 with the
denominator floored at 1e-3 * RMS of the reference row (so near-zero outputs do
not blow the ratio up). The guarded Snake and SnakeBeta, whose closing add
x + r can cancel, take the same 1e-5 relative to max(|y|, |x|); exp is held to
one ulp.

Rope: the kernel evaluates cos/sin in double and rounds once (correctly
rounded), while ggml-CPU calls glibc cosf/sinf, which land one ulp away in
about 1.3% of arguments. A rotated component that nearly cancels
(x0*c - x1*s ~ 0) then differs by ~1e-7 of the pair's length, which an
elementwise ratio reports as a large relative error of a tiny number. So rope
outputs are held to 1e-5 relative to the length of their NEOX pair (which the
rotation preserves), AND the kernel is checked bit-exact against the
restatement run with correctly rounded cos/sin -- which isolates libm's last
ulp as the only difference.
"""
import json
import os

import numpy as np
import pytest

import formats as F
import ggml_ref as R

pytestmark = pytest.mark.gpu

REL_TOL = 1e-5
SEED = 20260728


def _t(gpu, a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bits16(gpu, bits, dtype):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(dtype)


def _np(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def assert_bitexact(got, ref):
    got = np.ascontiguousarray(got, np.float32)
    ref = np.ascontiguousarray(ref, np.float32)
    assert got.shape == ref.shape
    bad = got.view(np.uint32) != ref.view(np.uint32)
    assert not bad.any(), "%d of %d differ; first at %s: %r vs %r" % (
        bad.sum(), bad.size, np.argwhere(bad)[0], got[bad][0], ref[bad][0])


def assert_close(got, ref, tol=REL_TOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    rows = ref.reshape(-1, ref.shape[-1])
    rms = np.sqrt((rows ** 2).mean(axis=-1, keepdims=True))
    floor = np.broadcast_to(1e-3 * rms, rows.shape).reshape(ref.shape)
    den = np.maximum(np.abs(ref), floor)
    den = np.where(den == 0, 1.0, den)
    rel = np.abs(got - ref) / den
    worst = rel.max()
    assert worst <= tol, "max rel err %.3g at %s (got %r ref %r)" % (
        worst, np.unravel_index(rel.argmax(), rel.shape), got.flat[rel.argmax()], ref.flat[rel.argmax()])
    assert normwise(got, ref) <= tol
    return float(worst), float((got == ref).mean())


def normwise(got, ref):
    """||got - ref|| / ||ref|| (2-norms over the whole tensor, in double)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    n = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (n if n > 0 else 1.0))


def assert_snake_close(got, ref, x, tol=REL_TOL):
    """Snake family: y = x + r ends in an add whose operands can cancel (a large
    term over a small beta against an x of the opposite sign), so the error is
    measured relative to the operands of that add, max(|y|, |x|) >= |r| / 2,
    floored as in assert_close. A last-ulp difference of the sine or the exp
    then stays a last-ulp difference."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    rows = ref.reshape(-1, ref.shape[-1])
    rms = np.sqrt((rows ** 2).mean(axis=-1, keepdims=True))
    floor = np.broadcast_to(1e-3 * rms, rows.shape).reshape(ref.shape)
    den = np.maximum(np.maximum(np.abs(ref), np.abs(np.asarray(x, np.float64))), floor)
    den = np.where(den == 0, 1.0, den)
    rel = np.abs(got - ref) / den
    assert rel.max() <= tol, "max rel err %.3g at %s (got %r ref %r)" % (
        rel.max(), np.unravel_index(rel.argmax(), rel.shape), got.flat[rel.argmax()], ref.flat[rel.argmax()])


def assert_rope_close(got, ref, n_dims, tol=REL_TOL):
    """|got - ref| <= tol * |(ref_i, ref_{i+n_dims/2})| per NEOX pair; elements
    past n_dims (copied) elementwise."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    half = n_dims // 2
    pair = np.hypot(ref[..., :half], ref[..., half:n_dims])
    den = np.concatenate([pair, pair], axis=-1)
    den = np.where(den == 0, 1.0, den)
    rel = np.abs(got[..., :n_dims] - ref[..., :n_dims]) / den
    assert rel.max() <= tol, "max pair-relative err %.3g" % rel.max()
    if n_dims < ref.shape[-1]:
        assert_close(got[..., n_dims:], ref[..., n_dims:], tol)
    return float(rel.max())


# ---------------------------------------------------------------------------
# gathers
# ---------------------------------------------------------------------------

def _table(rng, kind, rows, ne0):
    """Returns (oracle raw rows, oracle type, torch tensor or Q8Tensor builder input)."""
    if kind == "f32":
        a = rng.standard_normal((rows, ne0)).astype(np.float32)
        return a, R.F32
    if kind == "bf16":
        return F.f32_to_bf16_bits(rng.standard_normal((rows, ne0)).astype(np.float32) * 0.02), R.BF16
    if kind == "f16":
        return F.f32_to_f16_bits(rng.standard_normal((rows, ne0)).astype(np.float32)), R.F16
    return F.q8_0_synthetic(rng, rows, ne0), R.Q8_0


def _dev_table(gpu, raw, kind, ne0):
    import torch
    if kind == "f32":
        return _t(gpu, raw)
    if kind == "bf16":
        return _bits16(gpu, raw, torch.bfloat16)
    if kind == "f16":
        return _bits16(gpu, raw, torch.float16)
    return gpu.Q8Tensor(_t(gpu, raw), ne0)


@pytest.mark.parametrize("kind", ["f32", "f16", "bf16", "q8_0"])
@pytest.mark.parametrize("ne0", [64, 1024, 2048, 96, 4096])
def test_get_rows_bitexact(gpu, kind, ne0):
    if kind == "q8_0" and ne0 % 32:
        pytest.skip("Q8_0 rows are whole blocks")
    rng = np.random.default_rng(SEED + ne0)
    rows, n = 300, 257
    raw, otype = _table(rng, kind, rows, ne0)
    ids = rng.integers(0, rows, n).astype(np.int32)
    ids[:2] = [0, rows - 1]
    ref = R.run(lambda g: g.get_rows(raw, otype, ne0, ids))
    got = gpu.get_rows(_dev_table(gpu, raw, kind, ne0), _t(gpu, ids))
    assert_bitexact(_np(got), ref)


def test_get_rows_special_values(gpu):
    """BF16 NaN/Inf payloads and -0, F16 subnormals/Inf/NaN, Q8_0 with d = 0,
    negative d, subnormal f16 d and qs = +-127/-128: all exact, as the closed
    forms say."""
    import torch
    specials = np.array([0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC1, 0xFFA5, 0x0001, 0x807F, 0x3F80, 0xC2F7] * 13,
                        np.uint16)[:128]
    bf = np.tile(specials, (4, 1))
    ref = R.run(lambda g: g.get_rows(bf, R.BF16, 128, np.array([3, 0, 2], np.int32)))
    got = gpu.get_rows(_bits16(gpu, bf, torch.bfloat16), _t(gpu, np.array([3, 0, 2], np.int32)))
    assert_bitexact(_np(got), ref)
    assert_bitexact(ref, F.bf16_bits_to_f32(bf[[3, 0, 2]]))

    h = np.array([0x0001, 0x03FF, 0x8001, 0x7C00, 0xFC00, 0x7E01, 0x0000, 0x8000, 0x3C00, 0x7BFF] * 13,
                 np.uint16)[:128]
    hf = np.tile(h, (2, 1))
    ref = R.run(lambda g: g.get_rows(hf, R.F16, 128, np.array([1, 0], np.int32)))
    got = gpu.get_rows(_bits16(gpu, hf, torch.float16), _t(gpu, np.array([1, 0], np.int32)))
    assert_bitexact(_np(got), ref)
    assert_bitexact(ref, F.f16_bits_to_f32(hf[[1, 0]]))

    rng = np.random.default_rng(5)
    nb = 4
    d = np.array([[0x0000, 0x8C00, 0x0003, 0x2E66]], np.uint16).repeat(3, 0)  # 0, negative, subnormal, ~0.1
    qs = rng.integers(-128, 128, (3, nb, 32), dtype=np.int8)
    qs[:, :, 0], qs[:, :, 1], qs[:, :, 2] = 127, -127, -128
    raw = F.q8_0_pack(d, qs)
    ids = np.array([2, 1, 0], np.int32)
    ref = R.run(lambda g: g.get_rows(raw, R.Q8_0, 128, ids))
    got = gpu.get_rows(gpu.Q8Tensor(_t(gpu, raw), 128), _t(gpu, ids))
    assert_bitexact(_np(got), ref)
    assert_bitexact(ref, F.q8_0_dequant(raw, 128)[ids])


def test_get_rows_batched_and_out_of_range(gpu):
    import torch
    rng = np.random.default_rng(7)
    # ggml_get_rows batch form: src [ne0, rows, 2], ids [n, 2] -> [ne0, n, 2]
    src = rng.standard_normal((2, 50, 256)).astype(np.float32)
    ids = rng.integers(0, 50, (2, 9)).astype(np.int32)
    got = _np(gpu.get_rows(_t(gpu, src), _t(gpu, ids)))
    for b in range(2):
        assert_bitexact(got[b], src[b][ids[b]])
    # An id outside the table is never read; its row comes back as NaN.
    tab = _t(gpu, rng.standard_normal((10, 1024)).astype(np.float32))
    bad = _t(gpu, np.array([3, 10, -1, 9], np.int32))
    out = _np(gpu.get_rows(tab, bad))
    assert np.isnan(out[1]).all() and np.isnan(out[2]).all()
    assert_bitexact(out[[0, 3]], _np(tab)[[3, 9]])
    for ne0 in (1024, 2048, 4096):  # the LDS-staged widths: row 0 is read for a bad id, NaN stored
        raw = F.q8_0_synthetic(rng, 10, ne0)
        out = _np(gpu.get_rows(gpu.Q8Tensor(_t(gpu, raw), ne0), bad))
        assert np.isnan(out[1]).all() and np.isnan(out[2]).all()
        assert_bitexact(out[[0, 3]], F.q8_0_dequant(raw, ne0)[[3, 9]])
    # the staged Q8_0 kernel in ggml's batch form: table [1024, 12, 2], ids [7, 2]
    raw2 = np.stack([F.q8_0_synthetic(rng, 12, 1024) for _ in range(2)])
    ids2 = rng.integers(0, 12, (2, 7)).astype(np.int32)
    ids2[1, 3] = 12
    got2 = _np(gpu.get_rows(gpu.Q8Tensor(_t(gpu, raw2), 1024), _t(gpu, ids2)))
    for b in range(2):
        ok = ids2[b] < 12
        assert_bitexact(got2[b][ok], F.q8_0_dequant(raw2[b], 1024)[ids2[b][ok]])
        assert np.isnan(got2[b][~ok]).all()
    del torch


@pytest.mark.parametrize("kind,ne0,groups", [("q8_0", 1024, 16), ("q8_0", 2048, 15), ("q8_0", 4096, 3),
                                             ("q8_0", 1024, 20), ("q8_0", 4096, 5), ("q8_0", 512, 7),
                                             ("q8_0", 96, 5), ("bf16", 1024, 16), ("f16", 2048, 4),
                                             ("f32", 1024, 15), ("f32", 8, 4), ("f32", 3000, 2)])
def test_get_rows_sum_bitexact(gpu, kind, ne0, groups):
    rng = np.random.default_rng(SEED + ne0 + groups)
    rows, frames = 200, 301
    tabs = [_table(rng, kind, rows, ne0) for _ in range(groups)]
    codes = rng.integers(0, rows, (groups, frames)).astype(np.int32)
    ref = R.run(lambda g: R.sum_code_embeddings(g, [t for t, _ in tabs], tabs[0][1], ne0, codes))
    got = gpu.get_rows_sum([_dev_table(gpu, t, kind, ne0) for t, _ in tabs], _t(gpu, codes))
    assert_bitexact(_np(got), ref)


@pytest.mark.parametrize("kind,groups", [("q8_0", 57), ("q8_0", 63), ("q8_0", 64), ("bf16", 64)])
def test_get_rows_sum_up_to_64_groups(gpu, kind, groups):
    """The most groups a sum takes (64) and counts just under it, at ne0 =
    1024 (the Q8_0 windows' chunks fill every slot at 64 and leave slots past
    the last group at 57 and 63); an out-of-range id in the last group makes
    its frame's row NaN, every other frame is the ordered sum bit for bit."""
    rng = np.random.default_rng(SEED + 71 + groups)
    ne0, rows, frames = 1024, 40, 200
    tabs = [_table(rng, kind, rows, ne0) for _ in range(groups)]
    codes = rng.integers(0, rows, (groups, frames)).astype(np.int32)
    codes[groups - 1, 11] = rows
    got = _np(gpu.get_rows_sum([_dev_table(gpu, t, kind, ne0) for t, _ in tabs], _t(gpu, codes)))
    assert np.isnan(got[11]).all()
    ok = [f for f in range(frames) if f != 11]
    ref = R.run(lambda g: R.sum_code_embeddings(g, [t for t, _ in tabs], tabs[0][1], ne0,
                                                np.minimum(codes, rows - 1)))
    assert_bitexact(got[ok], ref[ok])


def test_get_rows_sum_order_matters_and_nan_on_bad_id(gpu):
    rng = np.random.default_rng(11)
    tabs = [(rng.standard_normal((64, 1024)) * 10.0 ** rng.integers(-3, 3, (64, 1))).astype(np.float32)
            for _ in range(4)]
    codes = rng.integers(0, 64, (4, 100)).astype(np.int32)
    dev = [_t(gpu, t) for t in tabs]
    fwd = _np(gpu.get_rows_sum(dev, _t(gpu, codes)))
    rev = _np(gpu.get_rows_sum(dev[::-1], _t(gpu, np.ascontiguousarray(codes[::-1]))))
    assert not np.array_equal(fwd.view(np.uint32), rev.view(np.uint32))  # f32 addition is not associative
    bad = codes.copy()
    bad[2, 5] = 64
    out = _np(gpu.get_rows_sum(dev, _t(gpu, bad)))
    assert np.isnan(out[5]).all()
    assert_bitexact(np.delete(out, 5, 0), np.delete(fwd, 5, 0))


@pytest.mark.parametrize("kind,ne0,groups", [("bf16", 1024, 16), ("bf16", 2048, 15), ("f16", 1024, 3),
                                             ("f32", 1024, 17), ("f32", 2048, 2), ("bf16", 64, 5),
                                             ("f16", 12, 40), ("f32", 1020, 9)])
def test_get_rows_sum_float_tables_special_values(gpu, kind, ne0, groups):
    """F32/F16/BF16 gather->sum over +-0, subnormals, +inf and ordinary
    values, bit for bit against the ordered f32 sum (-inf is left out: inf -
    inf is a NaN whose bits the CPU and the GPU choose differently). Row 0 of
    every table is
    all -0.0, so frame 0 (every group on row 0) must stay -0.0: a +0 slipped
    into the chain (from a slot past the last group, or a sum started at +0)
    flips it. The group counts leave slots past the last group in every chunk
    size the kernel picks; widths 12 and 1020 leave lanes past the row."""
    rng = np.random.default_rng(SEED + 91 + ne0 + groups)
    rows = 30
    if kind == "f32":
        pool = np.array([0.0, -0.0, 1e-40, -3e-42, np.inf, 1.5, -2.25, 3e38], np.float32).view(np.uint32)
        tabs = [rng.standard_normal((rows, ne0)).astype(np.float32) for _ in range(groups)]
        for t in tabs:
            t.view(np.uint32)[:, ::3] = pool[rng.integers(0, len(pool), (rows, len(range(0, ne0, 3))))]
            t[0] = -0.0
    else:
        pool = np.array([0x0000, 0x8000, 0x0001, 0x8003, 0x7C00 if kind == "f16" else 0x7F80,
                         0x3C00 if kind == "f16" else 0x3F80], np.uint16)
        conv = F.f32_to_f16_bits if kind == "f16" else F.f32_to_bf16_bits
        tabs = [conv(rng.standard_normal((rows, ne0)).astype(np.float32)) for _ in range(groups)]
        for t in tabs:
            t[:, ::3] = pool[rng.integers(0, len(pool), (rows, len(range(0, ne0, 3))))]
            t[0] = 0x8000
    otype = {"f32": R.F32, "f16": R.F16, "bf16": R.BF16}[kind]
    codes = rng.integers(0, rows, (groups, 41)).astype(np.int32)
    codes[:, 0] = 0
    with np.errstate(all="ignore"):
        ref = R.run(lambda g: R.sum_code_embeddings(g, tabs, otype, ne0, codes))
    assert (ref[0].view(np.uint32) == 0x80000000).all()
    got = _np(gpu.get_rows_sum([_dev_table(gpu, t, kind, ne0) for t in tabs], _t(gpu, codes)))
    assert_bitexact(got, ref)


def test_get_rows_sum_one_group_is_a_copy(gpu):
    """One group: ggml's sum is rows_0 itself, so BF16 NaN payloads, signalling
    NaNs included, come through bit for bit (an add would quiet them)."""
    rng = np.random.default_rng(SEED + 93)
    t = F.f32_to_bf16_bits(rng.standard_normal((20, 1024)).astype(np.float32))
    t[:, :8] = [0x7F81, 0xFF81, 0x7FC1, 0xFFFF, 0x7F80, 0x8000, 0x0001, 0x7FA5]
    codes = rng.integers(0, 20, (1, 33)).astype(np.int32)
    got = _np(gpu.get_rows_sum([_dev_table(gpu, t, "bf16", 1024)], _t(gpu, codes)))
    assert_bitexact(got, F.bf16_bits_to_f32(t[codes[0]]))


@pytest.mark.parametrize("ne0,groups", [(1024, 16), (1024, 15), (2048, 9), (4096, 3), (512, 7), (1024, 20)])
def test_get_rows_sum_q8_special_scales_and_signed_zero(gpu, ne0, groups):
    """Q8_0 gather->sum over scales -0, +0, negative, f16-subnormal and the
    largest f16, with quants +-127/-128/0, bit for bit against the ordered f32
    sum. Row 0 of every table is all-zero quants under d = -0, so frame 0
    (every group on row 0) sums to -0.0 in every element: one +0 slipped into
    the chain (say, from a slot past the last group) would flip it to +0. The
    group counts leave 0, 1, 7, 5 and 12 slots past the last group."""
    rng = np.random.default_rng(SEED + 77 + ne0 + groups)
    rows, nb = 40, ne0 // 32
    specials = np.array([0x8000, 0x0000, 0x8C00, 0x0003, 0x7BFF, 0x2E66, 0xBC00, 0x0400], np.uint16)
    tabs = []
    for _ in range(groups):
        d = specials[rng.integers(0, len(specials), (rows, nb))]
        qs = rng.integers(-128, 128, (rows, nb, 32)).astype(np.int8)
        qs[:, :, :3] = [127, -128, 0]
        d[0], qs[0] = 0x8000, 0
        tabs.append(F.q8_0_pack(d, qs))
    codes = rng.integers(0, rows, (groups, 33)).astype(np.int32)
    codes[:, 0] = 0
    ref = R.run(lambda g: R.sum_code_embeddings(g, tabs, R.Q8_0, ne0, codes))
    assert (ref[0].view(np.uint32) == 0x80000000).all()
    got = _np(gpu.get_rows_sum([gpu.Q8Tensor(_t(gpu, t), ne0) for t in tabs], _t(gpu, codes)))
    assert_bitexact(got, ref)


# ---------------------------------------------------------------------------
# norms and rope
# ---------------------------------------------------------------------------

def _weights(rng, n, kind):
    w = rng.normal(1.0, 0.1, n).astype(np.float32)
    if kind == "bf16":
        return F.f32_to_bf16_bits(w), R.BF16
    if kind == "f16":
        return F.f32_to_f16_bits(w), R.F16
    return w, R.F32


def _dev_w(gpu, w, kind):
    import torch
    if kind == "bf16":
        return _bits16(gpu, w, torch.bfloat16)
    if kind == "f16":
        return _bits16(gpu, w, torch.float16)
    return _t(gpu, w)


@pytest.mark.parametrize("shape,wkind", [((512, 1024), "bf16"), ((64, 2048), "f32"), ((7, 24, 128), "f16"),
                                         ((33, 1000), "f32"), ((5, 8), "f32"), ((3, 4096), "bf16"),
                                         ((40, 3072), "f32"), ((9, 64), "none"), ((4, 256), "bf16"),
                                         ((6, 512), "f32"), ((4101, 1024), "bf16"), ((4098, 2048), "f32"),
                                         ((3073, 1024), "bf16"), ((6147, 1024), "f32"), ((2049, 2048), "f16")])
def test_rms_norm_mul(gpu, shape, wkind):
    """Row counts past each launch-shape boundary, with a partly empty last
    block: (3073, 1024) and (2049, 2048) two waves per row, (4101, 1024) two
    waves and (6147, 1024) one wave per row, (4098, 2048) two waves."""
    rng = np.random.default_rng(SEED + sum(shape))
    x = rng.standard_normal(shape).astype(np.float32)
    x[0] = 0.0  # an all-zero row: scale = 1/sqrt(eps), output exactly 0
    eps = np.float32(1e-6)
    if wkind == "none":
        ref = R.run(lambda g: g.rms_norm(x, eps))
        got = gpu.rms_norm_mul(_t(gpu, x), None, eps)
    else:
        w, wt = _weights(rng, shape[-1], wkind)
        ref = R.run(lambda g: R.rms_norm_w(g, x, w, eps, wt))
        got = gpu.rms_norm_mul(_t(gpu, x), _dev_w(gpu, w, wkind), eps)
    got = _np(got)
    assert (got[0] == 0).all()
    _, same = assert_close(got, ref)
    assert same > 0.999  # double-accumulated squares: the GPU lands on the CPU's bits


@pytest.mark.parametrize("shape", [(64, 1024), (4100, 1024), (8, 2048)])
def test_rms_norm_mul_f32_gain_8_byte_aligned(gpu, shape):
    """An F32 gain vector that starts 8 bytes past a 16-byte boundary (a view
    into a larger buffer) is read element by element, not with 16-byte loads:
    same results as the aligned copy of the same gains."""
    import torch
    rng = np.random.default_rng(SEED + 11 + shape[0])
    x = rng.standard_normal(shape).astype(np.float32)
    w, _ = _weights(rng, shape[-1], "f32")
    eps = np.float32(1e-6)
    buf = torch.zeros(shape[-1] + 4, dtype=torch.float32, device="cuda")
    wv = buf[2:2 + shape[-1]]
    wv.copy_(_t(gpu, w))
    assert wv.data_ptr() % 16 == 8
    ref = R.run(lambda g: R.rms_norm_w(g, x, w, eps, R.F32))
    got = _np(gpu.rms_norm_mul(_t(gpu, x), wv, eps))
    _, same = assert_close(got, ref)
    assert same > 0.999
    s, y = gpu.add_rms_norm_mul(_t(gpu, x), _t(gpu, x), wv, eps)
    s_ref, y_ref = R.run(lambda g: R.add_rms_norm_w(g, x, x, w, eps, R.F32))
    assert_bitexact(_np(s), s_ref)
    assert_close(_np(y), y_ref)


@pytest.mark.parametrize("shape,wkind", [((512, 1024), "bf16"), ((64, 2048), "f32"), ((3, 1000), "f32"),
                                         ((4099, 1024), "f16"), ((4096, 2048), "bf16"), ((1025, 1024), "bf16"),
                                         ((2051, 2048), "f32"), ((4097, 2048), "bf16"), ((16385, 1024), "bf16")])
def test_add_rms_norm_mul(gpu, shape, wkind):
    """Row counts on each side of the launch-shape boundaries, most with a
    partly empty last block: (1025, 1024) and (2051, 2048) two waves per row,
    (4099, 1024) and (4097, 2048) one wave per row, (16385, 1024) four."""
    rng = np.random.default_rng(SEED + 3 * sum(shape))
    a = rng.standard_normal(shape).astype(np.float32)
    b = rng.standard_normal(shape).astype(np.float32)
    w, wt = _weights(rng, shape[-1], wkind)
    eps = np.float32(1e-6)
    s_ref, y_ref = R.run(lambda g: R.add_rms_norm_w(g, a, b, w, eps, wt))
    s, y = gpu.add_rms_norm_mul(_t(gpu, a), _t(gpu, b), _dev_w(gpu, w, wkind), eps)
    assert_bitexact(_np(s), s_ref)
    assert_close(_np(y), y_ref)
    _, y2 = gpu.add_rms_norm_mul(_t(gpu, a), _t(gpu, b), _dev_w(gpu, w, wkind), eps, want_sum=False)
    assert_bitexact(_np(y2), _np(y))


def _positions(rng, T, hi):
    p = rng.integers(0, hi, T).astype(np.int32)
    p[0] = 0
    return p


@pytest.mark.parametrize("T,H,hd,n_dims,hi", [(512, 16, 128, 128, 512), (64, 8, 128, 128, 8192),
                                              (17, 4, 96, 64, 8192), (3, 4, 4, 4, 4), (9, 2, 128, 64, 1000)])
def test_rope_ext_neox(gpu, T, H, hd, n_dims, hi):
    rng = np.random.default_rng(SEED + T + hd)
    x = rng.standard_normal((T, H, hd)).astype(np.float32)
    pos = _positions(rng, T, hi)
    theta = np.float32(1e6)
    ref = R.run(lambda g: g.rope_neox(x, pos, n_dims, theta))
    got = _np(gpu.rope_ext(_t(gpu, x), _t(gpu, pos), n_dims, gpu.ROPE_TYPE_NEOX, theta))
    assert_rope_close(got, ref, n_dims)
    assert_bitexact(got, R.run(lambda g: g.rope_neox(x, pos, n_dims, theta, cs_rounded=True)))
    assert_bitexact(got[0], x[0])  # position 0 is the identity rotation (cos 0 = 1, sin 0 = 0)
    if n_dims < hd:
        assert_bitexact(got[..., n_dims:], x[..., n_dims:])


def test_rope_in_place_and_scaled(gpu):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((40, 16, 128)).astype(np.float32)
    pos = _positions(rng, 40, 8192)
    ref = R.run(lambda g: g.rope_neox(x, pos, 128, np.float32(1e4), np.float32(0.5), np.float32(1.25)))
    xt = _t(gpu, x)
    gpu.rope_ext(xt, _t(gpu, pos), 128, gpu.ROPE_TYPE_NEOX, 1e4, 0.5, 0.0, 1.25, out=xt)
    assert_rope_close(_np(xt), ref, 128)
    assert_bitexact(_np(xt), R.run(lambda g: g.rope_neox(x, pos, 128, np.float32(1e4), np.float32(0.5),
                                                          np.float32(1.25), cs_rounded=True)))


@pytest.mark.parametrize("T,hi,wkind", [(1, 64, "bf16"), (512, 512, "bf16"), (300, 8192, "f32"), (64, 8192, "f16"),
                                        (16, 8192, "f32"), (7, 32768, "f16"), (3, 8192, "bf16")])
def test_qk_norm_rope(gpu, T, hi, wkind, H=16, KVH=8):
    """T <= 64 takes the decode-step kernel (blocks of 8 head rows, each with a
    separate wave building the cos/sin cache), longer runs the one whose wave
    0 does; both bit-exact against the restatement with correctly rounded
    cos/sin."""
    rng = np.random.default_rng(SEED + T)
    q = rng.standard_normal((T, H, 128)).astype(np.float32)
    k = rng.standard_normal((T, KVH, 128)).astype(np.float32)
    wq, wt = _weights(rng, 128, wkind)
    wk, _ = _weights(rng, 128, wkind)
    pos = _positions(rng, T, hi)
    eps, theta = np.float32(1e-6), np.float32(1e6)
    qr, kr = R.run(lambda g: R.qk_norm_rope(g, q, k, wq, wk, eps, pos, 128, theta, wt))
    qo, ko = gpu.qk_norm_rope(_t(gpu, q), _t(gpu, k), _dev_w(gpu, wq, wkind), _dev_w(gpu, wk, wkind), eps,
                              _t(gpu, pos), 128, theta)
    assert_rope_close(_np(qo), qr, 128)
    assert_rope_close(_np(ko), kr, 128)
    qc, kc = R.run(lambda g: R.qk_norm_rope(g, q, k, wq, wk, eps, pos, 128, theta, wt, cs_rounded=True))
    assert_bitexact(_np(qo), qc)
    assert_bitexact(_np(ko), kc)


@pytest.mark.parametrize("T,H,KVH", [(1, 6, 3), (3, 9, 7), (16, 20, 4)])
def test_qk_norm_rope_head_counts(gpu, T, H, KVH):
    """Decode-size launches in blocks of 8 head rows: 6 + 3 (one block with q
    and k), 9 + 7 (blocks straddling q and k), 20 + 4 (three blocks)."""
    test_qk_norm_rope(gpu, T, 8192, "bf16", H=H, KVH=KVH)


def test_qk_norm_rope_generic_head_dim(gpu):
    rng = np.random.default_rng(13)
    q = rng.standard_normal((6, 4, 64)).astype(np.float32)
    k = rng.standard_normal((6, 2, 64)).astype(np.float32)
    wq = rng.normal(1, 0.1, 64).astype(np.float32)
    wk = rng.normal(1, 0.1, 64).astype(np.float32)
    pos = _positions(rng, 6, 100)
    qr, kr = R.run(lambda g: R.qk_norm_rope(g, q, k, wq, wk, np.float32(1e-6), pos, 64, np.float32(1e6)))
    qo, ko = gpu.qk_norm_rope(_t(gpu, q), _t(gpu, k), _t(gpu, wq), _t(gpu, wk), 1e-6, _t(gpu, pos), 64, 1e6)
    assert_rope_close(_np(qo), qr, 64)
    assert_rope_close(_np(ko), kr, 64)


@pytest.mark.parametrize("T,filled,cap,hd,wkind", [(1, 37, 64, 128, "bf16"), (16, 0, 16, 128, "f32"),
                                                     (5, 10, 32, 64, "f32"), (3, 4, 8, 128, "f16")])
def test_qk_norm_rope_kv(gpu, T, filled, cap, hd, wkind, H=16, KVH=8):
    """The fused cache write (operations.cpp:98-116): q_out and the cache rows
    [filled, filled + T) of k equal the unfused qk_norm_rope's outputs bit for
    bit and the oracle's within the rope bar (and bit-exact against the oracle
    with correctly rounded cos/sin); v lands in the same rows unchanged; every
    other cache row keeps its sentinel. hd = 64 takes the generic kernel."""
    rng = np.random.default_rng(SEED + 3 * T + filled)
    q = rng.standard_normal((T, H, hd)).astype(np.float32)
    k = rng.standard_normal((T, KVH, hd)).astype(np.float32)
    v = rng.standard_normal((T, KVH, hd)).astype(np.float32)
    wq, wt = _weights(rng, hd, wkind)
    wk, _ = _weights(rng, hd, wkind)
    pos = (filled + np.arange(T)).astype(np.int32)
    eps, theta = np.float32(1e-6), np.float32(1e6)
    sentinel = np.full((cap, KVH, hd), 7.25, np.float32)
    sentinel[:, :, 1::3] = np.nan
    kc, vc = _t(gpu, sentinel), _t(gpu, sentinel)
    qo = gpu.qk_norm_rope_kv(_t(gpu, q), _t(gpu, k), _t(gpu, v), _dev_w(gpu, wq, wkind), _dev_w(gpu, wk, wkind), eps,
                             _t(gpu, pos), hd, theta, kc, vc, filled)
    qo, kc, vc = _np(qo), _np(kc), _np(vc)
    qu, ku = gpu.qk_norm_rope(_t(gpu, q), _t(gpu, k), _dev_w(gpu, wq, wkind), _dev_w(gpu, wk, wkind), eps,
                              _t(gpu, pos), hd, theta)
    rows = slice(filled, filled + T)
    assert_bitexact(qo, _np(qu))
    assert_bitexact(kc[rows], _np(ku))
    qr, kr = R.run(lambda g: R.qk_norm_rope(g, q, k, wq, wk, eps, pos, hd, theta, wt))
    assert_rope_close(qo, qr, hd)
    assert_rope_close(kc[rows], kr, hd)
    qcr, kcr = R.run(lambda g: R.qk_norm_rope(g, q, k, wq, wk, eps, pos, hd, theta, wt, cs_rounded=True))
    assert_bitexact(kc[rows], kcr)
    assert_bitexact(vc[rows], v)
    outside = np.ones(cap, bool)
    outside[rows] = False
    assert_bitexact(kc[outside], sentinel[outside])
    assert_bitexact(vc[outside], sentinel[outside])


@pytest.mark.parametrize("T,H,KVH", [(1, 6, 3), (5, 12, 4), (2, 16, 8), (16, 9, 7)])
def test_qk_norm_rope_kv_head_counts(gpu, T, H, KVH):
    """Decode-size launches split a position's q, k and v rows into blocks of
    8 rows: 6 + 3 + 3 puts k and v rows in one block, 12 + 4 + 4 a q/k block
    and a v block of 4, 16 + 8 + 8 one block of v rows only, 9 + 7 + 7 blocks
    that straddle every part. Same checks as above."""
    test_qk_norm_rope_kv(gpu, T, 20, 64, 128, "bf16", H=H, KVH=KVH)


def _kv_inputs(rng, T, hd=128, H=16, KVH=8):
    q = rng.standard_normal((T, H, hd)).astype(np.float32)
    k = rng.standard_normal((T, KVH, hd)).astype(np.float32)
    v = rng.standard_normal((T, KVH, hd)).astype(np.float32)
    wq = F.f32_to_bf16_bits(rng.normal(1, 0.1, hd))
    wk = F.f32_to_bf16_bits(rng.normal(1, 0.1, hd))
    return q, k, v, wq, wk


@pytest.mark.parametrize("T,filled,cap", [(1, 37, 64), (4, 60, 64), (3, 5, 16)])
def test_qk_norm_rope_kv_device_slot_matches_host_slot(gpu, T, filled, cap):
    """shp_qk_norm_rope_kv_at with `filled` in device memory writes exactly what
    shp_qk_norm_rope_kv writes with it as an argument (q_out and both caches,
    bit for bit); a slot whose rows do not fit (cap - T + 1, and -1) writes no
    cache row, still writes q_out, and raises the status word."""
    import torch
    rng = np.random.default_rng(SEED + 17 * T + filled)
    q, k, v, wq, wk = _kv_inputs(rng, T)
    pos = (filled + np.arange(T)).astype(np.int32)
    sentinel = rng.standard_normal((cap, 8, 128)).astype(np.float32)
    args = lambda kc, vc: (_t(gpu, q), _t(gpu, k), _t(gpu, v), _bits16(gpu, wq, torch.bfloat16),
                           _bits16(gpu, wk, torch.bfloat16), 1e-6, _t(gpu, pos), 128, 1e6, kc, vc)
    kc0, vc0 = _t(gpu, sentinel), _t(gpu, sentinel)
    q0 = gpu.qk_norm_rope_kv(*args(kc0, vc0), filled)
    kc1, vc1 = _t(gpu, sentinel), _t(gpu, sentinel)
    slot = torch.tensor([filled], dtype=torch.int32, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    q1 = gpu.qk_norm_rope_kv_at(*args(kc1, vc1), slot, status)
    for a, b in ((q0, q1), (kc0, kc1), (vc0, vc1)):
        assert_bitexact(_np(b), _np(a))
    assert int(_np(status)[0]) == 0
    for bad in (cap - T + 1, -1):
        kc2, vc2 = _t(gpu, sentinel), _t(gpu, sentinel)
        status.zero_()
        q2 = gpu.qk_norm_rope_kv_at(*args(kc2, vc2), torch.tensor([bad], dtype=torch.int32, device="cuda"), status)
        assert_bitexact(_np(q2), _np(q0))
        assert_bitexact(_np(kc2), sentinel)
        assert_bitexact(_np(vc2), sentinel)
        assert int(_np(status)[0]) == 1


def test_decode_steps_replay_one_captured_graph(gpu):
    """One HIP graph holding [qk-norm+rope+cache write at the device slot,
    slot += 1, position += 1] is captured once and replayed for 5 decode steps;
    after every replay (with eager work and a synchronisation in between) the
    caches equal those of 5 eager steps with `filled` passed from the host."""
    import torch
    rng = np.random.default_rng(SEED + 23)
    cap, steps = 16, 5
    q, k, v, wq, wk = _kv_inputs(rng, 1)
    dq, dk, dv = _t(gpu, q), _t(gpu, k), _t(gpu, v)
    dwq, dwk = _bits16(gpu, wq, torch.bfloat16), _bits16(gpu, wk, torch.bfloat16)
    sentinel = np.full((cap, 8, 128), -3.5, np.float32)
    # eager reference: steps with filled and the position from the host
    ek, ev, eq = _t(gpu, sentinel), _t(gpu, sentinel), []
    expect = []
    for n in range(steps):
        p = torch.tensor([n], dtype=torch.int32, device="cuda")
        eq.append(_np(gpu.qk_norm_rope_kv(dq, dk, dv, dwq, dwk, 1e-6, p, 128, 1e6, ek, ev, n)))
        expect.append((_np(ek).copy(), _np(ev).copy()))
    # the graph
    gk, gv = _t(gpu, sentinel), _t(gpu, sentinel)
    slot = torch.zeros(1, dtype=torch.int32, device="cuda")
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    qo = torch.empty_like(dq)

    def step():
        gpu.qk_norm_rope_kv_at(dq, dk, dv, dwq, dwk, 1e-6, pos, 128, 1e6, gk, gv, slot, status, q_out=qo)
        slot.add_(1)
        pos.add_(1)

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    # capture ran nothing: the caches are still the sentinel and the slot 0
    assert_bitexact(_np(gk), sentinel)
    assert int(_np(slot)[0]) == 0
    for n in range(steps):
        graph.replay()
        torch.cuda.synchronize()
        junk = torch.randn(1024, device="cuda").sum()  # eager work between the replays
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        assert_bitexact(_np(gk), expect[n][0])
        assert_bitexact(_np(gv), expect[n][1])
        assert_bitexact(_np(qo), eq[n])
        assert int(_np(slot)[0]) == n + 1
    assert int(_np(status)[0]) == 0


def _ulps_apart(got, ref):
    g = np.ascontiguousarray(got, np.float32).view(np.int32).astype(np.int64)
    r = np.ascontiguousarray(ref, np.float32).view(np.int32).astype(np.int64)
    return np.abs(g - r)


@pytest.mark.parametrize("H,T,N,mask", [(16, 1, 37, "none"), (16, 64, 64, "causal"), (4, 7, 2500, "heads2"),
                                        (3, 5, 64, "rows+"), (2, 3, 1, "none"), (8, 33, 2048, "causal"),
                                        (2, 2, 4097, "none"), (16, 1, 512, "none"), (3, 1, 512, "rows+"),
                                        (6, 3, 1024, "heads2"), (16, 512, 512, "causal"), (6, 4, 300, "heads2")])
def test_soft_max_ext(gpu, H, T, N, mask):
    """ggml_soft_max_ext with scale 1/sqrt(128): decode rows (1 x 37, 1 x 512;
    up to 64 rows of 260-512 take one-wave blocks, as 24 rows of 300 do),
    causal prefills, a mask broadcast over 2 heads, a mask with more rows than
    the scores, a one-element row, rows spread over 2 waves (512 wide; 3 rows
    leave the last block half empty) and 4 waves (1024, 2048 wide), and rows
    past the register kernels (2500, 4097).
    The kernel's exp is the correctly rounded one and its double sum runs in
    another order, so: at most 2 ulp from the oracle, and > 99% identical."""
    rng = np.random.default_rng(SEED + H * T + N)
    x = (rng.standard_normal((H, T, N)) * 3).astype(np.float32)
    m = None
    if mask == "causal":
        m = np.zeros((T, N), np.float32)
        m[np.triu_indices(T, N - T + 1, N)] = -np.inf
    elif mask == "heads2":
        m = rng.uniform(-5, 0, (2, T, N)).astype(np.float32)
        m[1, :, :100] = -np.inf
    elif mask == "rows+":
        m = rng.uniform(-5, 0, (T + 4, N)).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    ref = R.run(lambda g: g.soft_max_ext(x, m, scale))
    got = _np(gpu.soft_max_ext(_t(gpu, x), None if m is None else _t(gpu, m), scale))
    d = _ulps_apart(got, ref)
    assert d.max() <= 2 and (d == 0).mean() > 0.99


def test_soft_max_ext_special_rows(gpu):
    """A fully masked row (all -inf) and a row holding NaN or +inf come out NaN,
    as on the CPU; -inf entries next to finite ones give exact zeros."""
    x = np.zeros((4, 8), np.float32)
    x[1, 3] = np.nan
    x[2, 5] = np.inf
    m = np.zeros((4, 8), np.float32)
    m[0, :] = -np.inf
    m[3, :4] = -np.inf
    with np.errstate(invalid="ignore"):
        ref = R.run(lambda g: g.soft_max_ext(x, m, np.float32(1.0)))
    got = _np(gpu.soft_max_ext(_t(gpu, x), _t(gpu, m), 1.0))
    assert np.isnan(ref[:3]).all() and np.isnan(got[:3]).all()
    assert_bitexact(got[3], ref[3])
    assert (got[3, :4] == 0).all()


# ---------------------------------------------------------------------------
# elementwise
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(512, 3072), (3, 6144), (7, 1001), (1, 3072), (16, 4), (401, 3071)])
def test_swiglu_and_silu(gpu, shape):
    """Every flat launch form: one float4 per lane in 256-lane blocks, two per
    lane from 4 MB per operand ((512, 3072), and (401, 3071) with a partial
    last block), one-wave blocks from 16 MB (the configs[4] shape in
    test_gpu_full_configs.py)."""
    rng = np.random.default_rng(SEED + sum(shape))
    gt = (rng.standard_normal(shape) * 4).astype(np.float32)
    up = rng.standard_normal(shape).astype(np.float32)
    ref = R.run(lambda g: R.swiglu(g, gt, up))
    assert_close(_np(gpu.swiglu(_t(gpu, gt), _t(gpu, up))), ref)
    ref = R.run(lambda g: g.silu(gt))
    assert_close(_np(gpu.swiglu(_t(gpu, gt))), ref)


def assert_same_specials(got, ref):
    """NaN where the oracle has NaN, the same signed infinities and the same
    sign on zeros; returns the mask of the oracle's finite entries."""
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    assert got.shape == ref.shape
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    inf = np.isinf(ref)
    assert np.array_equal(np.isinf(got), inf) and np.array_equal(got[inf], ref[inf])
    zero = ref == 0
    assert np.array_equal(got[zero] == 0, np.ones(zero.sum(), bool))
    assert np.array_equal(np.signbit(got[zero]), np.signbit(ref[zero]))
    return np.isfinite(ref)


def test_norms_special_rows(gpu):
    """RMSNorm (plain, x gain, after an add) on rows holding NaN, +-inf, a value
    whose f32 square overflows (2e19: sum inf, scale 0), subnormals (squares
    that underflow to 0, so scale = 1/sqrt(eps)) and zeros: every such row is
    bit-identical to the oracle (NaN compared as NaN), the ordinary row within
    the float bar."""
    rng = np.random.default_rng(SEED + 41)
    x = rng.standard_normal((9, 1024)).astype(np.float32)
    x[0] = 0.0
    x[1, 5] = np.nan
    x[2, 7] = np.inf
    x[3, 9] = -np.inf
    x[4, 11] = 2e19
    x[5] = np.float32(1e-41) * np.sign(x[5])
    x[6] = 3e-20
    x[7, :3] = [np.inf, -np.inf, 1.0]
    b = rng.standard_normal((9, 1024)).astype(np.float32)
    b[1:8] = 0.0  # the add keeps the special rows as they are
    w, wt = _weights(rng, 1024, "bf16")
    eps = np.float32(1e-6)
    ref = R.run(lambda g: R.rms_norm_w(g, x, w, eps, wt))
    got = _np(gpu.rms_norm_mul(_t(gpu, x), _dev_w(gpu, w, "bf16"), eps))
    fin = assert_same_specials(got, ref)
    assert_bitexact(np.where(fin, got, 0)[:8], np.where(fin, ref, 0)[:8])
    assert_close(got[8:], ref[8:])
    ref = R.run(lambda g: g.rms_norm(x, eps))
    got = _np(gpu.rms_norm_mul(_t(gpu, x), None, eps))
    fin = assert_same_specials(got, ref)
    assert_bitexact(np.where(fin, got, 0)[:8], np.where(fin, ref, 0)[:8])
    s_ref, y_ref = R.run(lambda g: R.add_rms_norm_w(g, x, b, w, eps, wt))
    s, y = gpu.add_rms_norm_mul(_t(gpu, x), _t(gpu, b), _dev_w(gpu, w, "bf16"), eps)
    assert_same_specials(_np(s), s_ref)
    fin = assert_same_specials(_np(y), y_ref)
    assert_bitexact(np.where(fin, _np(y), 0)[1:8], np.where(fin, y_ref, 0)[1:8])


def test_rope_and_qk_norm_rope_special_values(gpu):
    """NaN and +-inf components through the NEOX rotation (inf * sin 0 is NaN
    at position 0, as in the CPU formula; no identity shortcut), on the
    128-wide fast path and the generic one: NaN and inf where the oracle has
    them, everything else bit-exact against the restatement with correctly
    rounded cos/sin."""
    rng = np.random.default_rng(SEED + 43)
    for hd in (128, 64):
        x = rng.standard_normal((4, 4, hd)).astype(np.float32)
        x[0, 0, 1] = np.inf
        x[0, 1, hd // 2 + 2] = -np.inf
        x[1, 2, 3] = np.nan
        x[2, 3, :] = 0.0
        x[3, 0, 0] = 3e38
        x[3, 0, hd // 2] = -3e38
        pos = np.array([0, 37, 8191, 5], np.int32)
        theta = np.float32(1e6)
        ref = R.run(lambda g: g.rope_neox(x, pos, hd, theta, cs_rounded=True))
        got = _np(gpu.rope_ext(_t(gpu, x), _t(gpu, pos), hd, gpu.ROPE_TYPE_NEOX, theta))
        fin = assert_same_specials(got, ref)
        assert_bitexact(np.where(fin, got, 0), np.where(fin, ref, 0))
        k = rng.standard_normal((4, 2, hd)).astype(np.float32)
        k[1, 1, 4] = np.inf
        wq = rng.normal(1, 0.1, hd).astype(np.float32)
        wk = rng.normal(1, 0.1, hd).astype(np.float32)
        eps = np.float32(1e-6)
        qr, kr = R.run(lambda g: R.qk_norm_rope(g, x, k, wq, wk, eps, pos, hd, theta, cs_rounded=True))
        qo, ko = gpu.qk_norm_rope(_t(gpu, x), _t(gpu, k), _t(gpu, wq), _t(gpu, wk), eps, _t(gpu, pos), hd, theta)
        for a, b in ((_np(qo), qr), (_np(ko), kr)):
            fin = assert_same_specials(a, b)
            assert_bitexact(np.where(fin, a, 0), np.where(fin, b, 0))


def test_swiglu_special_values(gpu):
    """silu(g)*u with g over zeros, +-inf, NaN, subnormals, values where
    exp(-g) overflows or underflows, and u over zeros, inf and NaN: NaN, inf
    and signed zeros where the oracle has them, finite values within 1e-5."""
    gp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -100.0, 100.0, 88.7, -88.7, -103.0, 1e-45, -1e-45,
                   1e-38, 20.0, -20.0, 0.5], np.float32)
    up = np.array([1.0, -1.0, 0.0, -0.0, np.inf, -np.inf, np.nan, 2.5], np.float32)
    g = np.repeat(gp, up.size).reshape(1, -1)
    u = np.tile(up, gp.size).reshape(1, -1)
    g = np.tile(g, (3, 8))
    u = np.tile(u, (3, 8))
    ref = R.run(lambda gr: R.swiglu(gr, g, u))
    got = _np(gpu.swiglu(_t(gpu, g), _t(gpu, u)))
    fin = assert_same_specials(got, ref)
    nz = fin & (ref != 0)
    rel = np.abs(got[nz].astype(np.float64) - ref[nz]) / np.abs(ref[nz].astype(np.float64))
    assert rel.max() <= REL_TOL
    ref = R.run(lambda gr: gr.silu(g))
    got = _np(gpu.swiglu(_t(gpu, g)))
    fin = assert_same_specials(got, ref)
    nz = fin & (ref != 0)
    rel = np.abs(got[nz].astype(np.float64) - ref[nz]) / np.abs(ref[nz].astype(np.float64))
    assert rel.max() <= REL_TOL


@pytest.mark.parametrize("swapped", [False, True])
def test_glu_swiglu_single_tensor(gpu, swapped):
    rng = np.random.default_rng(17)
    a = rng.standard_normal((33, 2 * 384)).astype(np.float32)
    ref = R.run(lambda g: g.glu_swiglu(a, swapped))
    assert_close(_np(gpu.glu_swiglu(_t(gpu, a), swapped)), ref)


@pytest.mark.parametrize("T,C", [(256, 512), (64, 128), (31, 30), (5, 1024), (9, 2048), (3, 1028)])
def test_snake(gpu, T, C):
    """C % 4 == 0: the flat kernel (2 rows per lane, division through a double
    reciprocal; odd T leaves a partial group); C % 4 != 0: the row kernel.
    Row 0 holds large x, so |alpha*x| crosses 2^15 and those elements take
    OCML's sine instead of the fast one."""
    rng = np.random.default_rng(SEED + T + C)
    x = rng.standard_normal((T, C)).astype(np.float32)
    x[0, ::3] *= 20000.0
    alpha = np.exp(rng.uniform(np.log(0.1), np.log(10.0), C)).astype(np.float32)
    ref = R.run(lambda g: R.snake(g, x, alpha))
    assert_close(_np(gpu.snake(_t(gpu, x), _t(gpu, alpha))), ref)


def test_snake_special_alphas(gpu):
    """Channels whose alpha is 0, -0, +-inf or NaN take the f32 division, the
    others the reciprocal route; power-of-two, negative, subnormal and extreme
    alphas exercise exact ties, overflow to inf and underflow. NaN and inf land
    where the oracle puts them; finite outputs meet the Snake tolerance. 37 rows
    also leave a partial group of the kernel's 2 rows per lane. Rows 1-2 hold
    special x: +-inf and NaN (sin gives NaN), +-3e38, subnormals, and
    arguments on both sides of the fast sine's |a*x| < 2^15 range, up to 1e30
    (the full-range sine)."""
    rng = np.random.default_rng(SEED + 99)
    T, C = 37, 64
    x = rng.standard_normal((T, C)).astype(np.float32)
    x[0, :] = 0.0
    xs = np.array([np.inf, -np.inf, np.nan, 3e38, -3e38, 1e-45, -1e-40, 40000.0, -1e6, 1e30, 32767.99, 32768.0,
                   -32768.0, 12345.678, 3276.8, 1e-3], np.float32)
    x[1, :] = np.tile(xs, C // xs.size)
    x[2, :] = np.roll(x[1, :], 5)
    alpha = np.exp(rng.uniform(np.log(0.1), np.log(10.0), C)).astype(np.float32)
    alpha[:16] = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 2.0, 0.125, -4.0, 1e-39, -1e-30, 3e38, 1e-45,
                           2.0 ** -126, 2.0 ** 100, -0.5, 1.0], np.float32)
    with np.errstate(all="ignore"):
        ref = R.run(lambda g: R.snake(g, x, alpha))
    got = _np(gpu.snake(_t(gpu, x), _t(gpu, alpha)))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    inf = np.isinf(ref)
    assert np.array_equal(np.isinf(got), inf) and np.array_equal(got[inf], ref[inf])
    fin = np.isfinite(ref)
    den = np.maximum(np.abs(ref[fin]).astype(np.float64), 1e-3)
    assert (np.abs(got[fin].astype(np.float64) - ref[fin]) / den).max() <= REL_TOL


@pytest.mark.parametrize("T,C", [(256, 512), (37, 64), (31, 30), (3, 1028)])
def test_snake_guarded(gpu, T, C):
    """codec_snake (omnivoice): alpha = 0 and alphas near 1e-9 next to |x| ~ 1e4
    are where the 1e-9 guard changes the result; row 0's large x crosses the
    fast sine's range. C % 4 != 0 takes the row kernel."""
    rng = np.random.default_rng(SEED + 7 * T + C)
    x = rng.standard_normal((T, C)).astype(np.float32)
    x[0, ::3] *= 20000.0
    alpha = np.exp(rng.uniform(np.log(1e-9), np.log(10.0), C)).astype(np.float32)
    alpha[:4] = np.array([0.0, 1e-9, 1e-7, 1e-4], np.float32)
    x[:, :4] *= 1e4
    ref = R.run(lambda g: R.snake_guarded(g, x, alpha))
    got = _np(gpu.snake_guarded(_t(gpu, x), _t(gpu, alpha)))
    assert_snake_close(got, ref, x)
    assert_bitexact(got[:, 0], x[:, 0])  # alpha = 0: the guard keeps sin(0)^2 / 1e-9 = 0


@pytest.mark.parametrize("T,C", [(256, 512), (37, 64), (31, 30), (9, 2048), (4, 1028), (1001, 1024), (77, 260),
                                 (32771, 128)])
def test_snake_beta(gpu, T, C):
    """codec_snake_beta (qwen3-tts): log curves over [-3, 3], so alpha/beta span
    e^+-3 and the two exps, the guard and the division all matter. Up to 1024
    channels the 4-row LDS-table kernel runs (1024 channels: four per thread
    in its table; 260: one or two; 128 channels at any length up to 2^20
    tasks); past 1024 the flat kernel, 8 rows per lane: T = 37, 9 and 4 leave
    partial groups, as 1001, 77 and 32771 do for 4-row tasks."""
    rng = np.random.default_rng(SEED + 11 * T + C)
    x = rng.standard_normal((T, C)).astype(np.float32)
    la = rng.uniform(-3, 3, C).astype(np.float32)
    lb = rng.uniform(-3, 3, C).astype(np.float32)
    ref = R.run(lambda g: R.snake_beta(g, x, la, lb))
    assert_snake_close(_np(gpu.snake_beta(_t(gpu, x), _t(gpu, la), _t(gpu, lb))), ref, x)


def test_snake_beta_large_channel_table(gpu):
    """[128, 131072] takes the kernel that evaluates each channel's curves
    once per block into LDS, one 4-row task per lane (2^20 tasks: at 128
    channels the 4-row form runs at every length it covers); rows 0 and 1
    carry large x, so some sines leave the fast range, and channels 0-3 hold
    extreme curves."""
    rng = np.random.default_rng(SEED + 131)
    T, C = 131072, 128
    x = rng.standard_normal((T, C), dtype=np.float32)
    x[:2, ::5] *= 30000.0
    la = rng.uniform(-3, 3, C).astype(np.float32)
    lb = rng.uniform(-3, 3, C).astype(np.float32)
    la[:4] = [-30.0, 30.0, 0.0, -3.0]
    lb[:4] = [-30.0, 3.0, 30.0, -25.0]
    ref = R.run(lambda g: R.snake_beta(g, x, la, lb))
    assert_snake_close(_np(gpu.snake_beta(_t(gpu, x), _t(gpu, la), _t(gpu, lb))), ref, x)


@pytest.mark.parametrize("T,C", [(16387, 256), (8197, 1024)])
def test_snake_beta_eight_row_tasks_ragged(gpu, T, C):
    """Shapes of more than 128 channels just past 2^18 4-row tasks take the
    8-row LDS kernel; T is not a multiple of 8, so the last task of each
    channel quad is partial."""
    rng = np.random.default_rng(SEED + 137 + C)
    x = rng.standard_normal((T, C), dtype=np.float32)
    la = rng.uniform(-3, 3, C).astype(np.float32)
    lb = rng.uniform(-3, 3, C).astype(np.float32)
    ref = R.run(lambda g: R.snake_beta(g, x, la, lb))
    assert_snake_close(_np(gpu.snake_beta(_t(gpu, x), _t(gpu, la), _t(gpu, lb))), ref, x)


def test_golden_g3_snake_beta_on_gpu(gpu):
    """kExpectedSnakeBeta, tests/qwen3_tts_codec_ops_test.cpp:77-82, at the
    test's CPU tolerance (1e-4, tighter than its 5e-3 for accelerators)."""
    import test_oracle_goldens as G
    d = _golden("qwen3_codec_snake_beta.json")
    x, a, b = G.snake_beta_inputs(d)
    got = _np(gpu.snake_beta(_t(gpu, x), _t(gpu, a), _t(gpu, b)))
    exp = np.array(d["expected_snake_beta"], np.float32)
    assert np.abs(got.reshape(-1) - exp).max() < d["tolerance_cpu"]
    assert_snake_close(got, R.run(lambda g: R.snake_beta(g, x, a, b)), x)


@pytest.mark.parametrize("shape", [(333, 256), (17, 75)])
def test_exp(gpu, shape):
    """ggml_exp: the kernel rounds the double exp once (correctly rounded but for
    arguments within ~2^-52 of a rounding boundary); glibc's expf lands one ulp
    away for ~0.06% of arguments. So: at most one ulp apart everywhere, >99.9%
    identical; inf, 0, subnormal and NaN results where the oracle has them."""
    rng = np.random.default_rng(SEED + shape[1])
    x = rng.uniform(-104, 89, shape).astype(np.float32)
    x.reshape(-1)[:8] = [0.0, -0.0, np.inf, -np.inf, np.nan, 88.8, -87.5, -103.9]
    with np.errstate(over="ignore"):
        ref = R.run(lambda g: g.exp(x))
    got = _np(gpu.exp(_t(gpu, x)))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    d = np.abs(got[ok].view(np.int32).astype(np.int64) - ref[ok].view(np.int32).astype(np.int64))
    assert d.max() <= 1 and (d == 0).mean() > 0.999


@pytest.mark.parametrize("shape", [(37, 1024), (33, 77)])
@pytest.mark.parametrize("s,b", [(0.7853982, 0.0), (-1.5, 0.0), (0.7853982, -0.3183099), (1.0, 1e-9)])
def test_scale_bias_bitexact(gpu, shape, s, b):
    rng = np.random.default_rng(SEED + shape[1])
    x = _specials(int(np.prod(shape)), rng).reshape(shape)
    s, b = np.float32(s), np.float32(b)
    with np.errstate(all="ignore"):
        ref = R.run(lambda g: g.scale_bias(x, s, b))
    assert_bitexact(_np(gpu.scale_bias(_t(gpu, x), s, b)), ref)


@pytest.mark.parametrize("n", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("shape", [(64, 4096), (33, 77)])
def test_sum_scale_leaky_relu_bitexact(gpu, n, shape):
    """The branch average: terms added in order, scaled by 1/n (skipped for one
    term), then leaky; the scaled sum too. (33, 77) takes the scalar kernel."""
    rng = np.random.default_rng(SEED + 13 * n + shape[1])
    terms = [rng.standard_normal(shape).astype(np.float32) for _ in range(n)]
    terms[0] = _specials(int(np.prod(shape)), rng).reshape(shape)
    scale, slope = np.float32(1.0 / n), np.float32(0.1)
    with np.errstate(all="ignore"):
        cur_ref, y_ref = R.run(lambda g: R.sum_scale_leaky(g, terms, scale, slope))
    cur, y = gpu.sum_scale_leaky_relu([_t(gpu, t) for t in terms], scale, slope, want_mean=True)
    assert_bitexact(_np(cur), cur_ref)
    assert_bitexact(_np(y), y_ref)
    _, y_only = gpu.sum_scale_leaky_relu([_t(gpu, t) for t in terms], scale, slope)
    assert_bitexact(_np(y_only), y_ref)


def _specials(n, rng):
    v = rng.standard_normal(n).astype(np.float32)
    sp = np.array([0.0, -0.0, np.nan, -np.nan, np.inf, -np.inf, 1e-45, -1e-45, 1e-38, -3e-39, 3.4e38, -3.4e38],
                  np.float32)
    m = min(n, sp.size)
    v[:m] = sp[:m]
    return v


@pytest.mark.parametrize("shape", [(128, 8192), (33, 77), (1, 4), (301, 3500), (512, 8192)])
@pytest.mark.parametrize("slope", [0.1, 0.01])
def test_add_leaky_relu_bitexact(gpu, shape, slope):
    rng = np.random.default_rng(SEED + shape[1])
    a = _specials(int(np.prod(shape)), rng).reshape(shape)
    b = rng.standard_normal(shape).astype(np.float32)
    b.reshape(-1)[:12] = 0.0  # the specials reach the leaky unchanged
    s_ref, y_ref = R.run(lambda g: R.add_leaky(g, a, b, np.float32(slope)))
    s, y = gpu.add_leaky_relu(_t(gpu, a), _t(gpu, b), slope, want_sum=True)
    assert_bitexact(_np(s), s_ref)
    assert_bitexact(_np(y), y_ref)
    # -0 -> +0 and NaN -> +0, exactly as ggml's (x>0?x:0) + slope*(x<0?x:0)
    yv = _np(y).reshape(-1)
    assert yv[1] == 0 and not np.signbit(yv[1]) and yv[2] == 0 and yv[3] == 0
    y_only = gpu.leaky_relu(_t(gpu, a), slope)
    assert_bitexact(_np(y_only), R.run(lambda g: g.leaky_relu(a, np.float32(slope))))


@pytest.mark.parametrize("bshape", ["full", "row"])
@pytest.mark.parametrize("shape", [(37, 1024), (1001, 1100), (4099, 1028)])
def test_add(gpu, bshape, shape):
    """A full second operand or one broadcast row, in each flat launch form
    (2, 4.4 and 16.9 MB per operand)."""
    rng = np.random.default_rng(19 + shape[0])
    a = rng.standard_normal(shape).astype(np.float32)
    b = rng.standard_normal(shape if bshape == "full" else (shape[1],)).astype(np.float32)
    assert_bitexact(_np(gpu.add(_t(gpu, a), _t(gpu, b))), R.run(lambda g: g.add(a, b)))


@pytest.mark.parametrize("T,hd,wkind", [(1, 128, "bf16"), (37, 128, "f32"), (5, 64, "f16")])
def test_layer_nongemm_step(gpu, T, hd, wkind):
    """One call for a Qwen3 layer's non-GEMM node runs
    (qwen3-tts/operations.cpp:84-147): every output equals the single entry
    points' bit for bit, and the oracle's -- adds bit-exact, norms and SwiGLU
    within 1e-5, q/k bit-exact against the restatement with correctly rounded
    cos/sin. hidden 1024, 16 q and 8 kv heads, ffn 3072 (the talker's shape)."""
    rng = np.random.default_rng(SEED + 7 * T + hd)
    hidden, heads, kv_heads, ffn = 1024, 16, 8, 3072
    eps, theta = np.float32(1e-6), np.float32(1e6)
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    q = rng.standard_normal((T, heads, hd)).astype(np.float32)
    k = rng.standard_normal((T, kv_heads, hd)).astype(np.float32)
    attn = rng.standard_normal((T, hidden)).astype(np.float32)
    gate = (rng.standard_normal((T, ffn)) * 4).astype(np.float32)
    up = rng.standard_normal((T, ffn)).astype(np.float32)
    mlp = rng.standard_normal((T, hidden)).astype(np.float32)
    pos = _positions(rng, T, 8192)
    (w_in, wt), (w_post, _), (wq, _), (wk, _) = [_weights(rng, n, wkind) for n in (hidden, hidden, hd, hd)]
    d = {n: _t(gpu, a) for n, a in dict(x=x, q=q, k=k, attn=attn, gate=gate, up=up, mlp=mlp, pos=pos).items()}
    dw = {n: _dev_w(gpu, a, wkind) for n, a in dict(w_in=w_in, w_post=w_post, wq=wq, wk=wk).items()}

    outs = gpu.layer_nongemm_step(d["x"], dw["w_in"], d["q"], d["k"], dw["wq"], dw["wk"], d["pos"], d["attn"],
                                  dw["w_post"], d["gate"], d["up"], d["mlp"], eps, hd, theta)
    got = {n: _np(t) for n, t in outs.items()}

    normed = gpu.rms_norm_mul(d["x"], dw["w_in"], eps)
    qo, ko = gpu.qk_norm_rope(d["q"], d["k"], dw["wq"], dw["wk"], eps, d["pos"], hd, theta)
    resid, mlp_in = gpu.add_rms_norm_mul(d["x"], d["attn"], dw["w_post"], eps)
    act = gpu.swiglu(d["gate"], d["up"])
    out = gpu.add(resid, d["mlp"])
    single = dict(normed=normed, q_out=qo, k_out=ko, resid=resid, mlp_in=mlp_in, act=act, out=out)
    assert sorted(single) == sorted(gpu.LAYER_OUTPUTS)
    for n, t in single.items():
        assert_bitexact(got[n], _np(t))

    assert_close(got["normed"], R.run(lambda g: R.rms_norm_w(g, x, w_in, eps, wt)))
    qc, kc = R.run(lambda g: R.qk_norm_rope(g, q, k, wq, wk, eps, pos, hd, theta, wt, cs_rounded=True))
    assert_bitexact(got["q_out"], qc)
    assert_bitexact(got["k_out"], kc)
    s_ref, y_ref = R.run(lambda g: R.add_rms_norm_w(g, x, attn, w_post, eps, wt))
    assert_bitexact(got["resid"], s_ref)
    assert_close(got["mlp_in"], y_ref)
    assert_close(got["act"], R.run(lambda g: R.swiglu(g, gate, up)))
    assert_bitexact(got["out"], R.run(lambda g: g.add(s_ref, mlp)))


def test_strided_views(gpu):
    """ggml views: rows strided in dims 1..3 (a q/k head view of a fused qkv
    buffer) go through the row path with the same results."""
    import torch
    rng = np.random.default_rng(23)
    qkv = rng.standard_normal((10, 32, 128)).astype(np.float32)  # T, heads(16 q + 8 k + 8 v), hd
    dev = _t(gpu, qkv)
    q, k = dev[:, :16, :], dev[:, 16:24, :]
    pos = _positions(rng, 10, 500)
    wq = rng.normal(1, 0.1, 128).astype(np.float32)
    wk = rng.normal(1, 0.1, 128).astype(np.float32)
    qr, kr = R.run(lambda g: R.qk_norm_rope(g, qkv[:, :16], qkv[:, 16:24], wq, wk, np.float32(1e-6), pos, 128,
                                            np.float32(1e6)))
    qo, ko = gpu.qk_norm_rope(q, k, _t(gpu, wq), _t(gpu, wk), 1e-6, _t(gpu, pos), 128, 1e6)
    assert_rope_close(_np(qo), qr, 128)
    assert_rope_close(_np(ko), kr, 128)
    x = dev.reshape(10, 32 * 128)[:, :1024]  # strided rows
    w = rng.normal(1, 0.1, 1024).astype(np.float32)
    ref = R.run(lambda g: R.rms_norm_w(g, qkv.reshape(10, -1)[:, :1024], w, np.float32(1e-6)))
    assert_close(_np(gpu.rms_norm_mul(x, _t(gpu, w), 1e-6)), ref)
    out = torch.empty((10, 4096), device="cuda")
    y = out[:, 1000:2024]
    gpu.swiglu(x, x, out=y)
    assert_close(_np(y), R.run(lambda g: R.swiglu(g, qkv.reshape(10, -1)[:, :1024], qkv.reshape(10, -1)[:, :1024])))


def test_strided_views_newer_ops(gpu):
    """Views for the Snake variants, exp, scale_bias and soft_max_ext (the row
    kernels; float4 rows with a strided RowMap, and scalar rows with a
    non-flat one), and the fused cache write fed by q, k, v head views of one
    qkv buffer, as the attention's projection leaves them."""
    import torch
    rng = np.random.default_rng(29)
    buf = rng.standard_normal((10, 32, 128)).astype(np.float32)
    dev = _t(gpu, buf)
    flat = buf.reshape(10, -1)
    xv = dev.reshape(10, 4096)[:, 8:1032]            # rows 16 KB apart, 32 B in
    xr = flat[:, 8:1032]
    out = torch.full((10, 4096), 7.0, device="cuda")
    yv = out[:, 2048:3072]
    la = rng.uniform(-3, 3, 1024).astype(np.float32)
    lb = rng.uniform(-3, 3, 1024).astype(np.float32)
    gpu.snake_beta(xv, _t(gpu, la), _t(gpu, lb), out=yv)
    assert_snake_close(_np(yv), R.run(lambda g: R.snake_beta(g, xr, la, lb)), xr)
    al = np.exp(rng.uniform(np.log(1e-3), np.log(10.0), 1024)).astype(np.float32)
    assert_snake_close(_np(gpu.snake_guarded(xv, _t(gpu, al))), R.run(lambda g: R.snake_guarded(g, xr, al)), xr)
    with np.errstate(over="ignore"):
        e_ref = R.run(lambda g: g.exp(xr))
    d = _ulps_apart(_np(gpu.exp(xv)), e_ref)
    assert d.max() <= 1 and (d == 0).mean() > 0.99
    assert_bitexact(_np(gpu.scale_bias(xv, 0.75, -0.25)), R.run(lambda g: g.scale_bias(xr, np.float32(0.75),
                                                                                     np.float32(-0.25))))
    assert (_np(out)[:, :2048] == 7.0).all() and (_np(out)[:, 3072:] == 7.0).all()  # only the view written
    for cols in (100, 97):  # float4 rows (strided, flat map) and scalar rows (non-flat map)
        sv = dev[:, :16, :cols] if cols == 97 else dev[:, :, :cols]
        sr = buf[:, :16, :cols] if cols == 97 else buf[:, :, :cols]
        m = rng.uniform(-2, 0, (sr.shape[1], cols)).astype(np.float32)
        ref = R.run(lambda g: g.soft_max_ext(sr, m, np.float32(0.125)))
        got = _np(gpu.soft_max_ext(sv, _t(gpu, m), 0.125))
        d = _ulps_apart(got, ref)
        assert d.max() <= 2 and (d == 0).mean() > 0.99
    # q, k, v as head views of one [T, 16 + 8 + 8, 128] qkv buffer
    q, k, v = dev[:, :16, :], dev[:, 16:24, :], dev[:, 24:32, :]
    wq = F.f32_to_bf16_bits(rng.normal(1, 0.1, 128))
    wk = F.f32_to_bf16_bits(rng.normal(1, 0.1, 128))
    pos = (20 + np.arange(10)).astype(np.int32)
    kc, vc = torch.zeros(40, 8, 128, device="cuda"), torch.zeros(40, 8, 128, device="cuda")
    qo = gpu.qk_norm_rope_kv(q, k, v, _bits16(gpu, wq, torch.bfloat16), _bits16(gpu, wk, torch.bfloat16), 1e-6,
                             _t(gpu, pos), 128, 1e6, kc, vc, 20)
    qr, kr = R.run(lambda g: R.qk_norm_rope(g, buf[:, :16], buf[:, 16:24], wq, wk, np.float32(1e-6), pos, 128,
                                            np.float32(1e6), R.BF16))
    assert_rope_close(_np(qo), qr, 128)
    assert_rope_close(_np(kc)[20:30], kr, 128)
    assert_bitexact(_np(vc)[20:30], buf[:, 24:32])
    assert (_np(kc)[:20] == 0).all() and (_np(vc)[30:] == 0).all()


# ---------------------------------------------------------------------------
# the reference's goldens through the HIP kernels
# ---------------------------------------------------------------------------

class HipOps(R.OracleOps):
    """decoder_layer's hot-path node runs on the GPU through the C ABI."""

    def __init__(self, gpu):
        self.g = gpu

    def rms_norm_w(self, x, w, eps):
        return _np(self.g.rms_norm_mul(_t(self.g, x), _t(self.g, w), eps))

    def qk_norm_rope(self, q, k, wq, wk, eps, pos, n_dims, theta):
        qo, ko = self.g.qk_norm_rope(_t(self.g, q), _t(self.g, k), _t(self.g, wq), _t(self.g, wk), eps,
                                     _t(self.g, pos), n_dims, theta)
        return _np(qo), _np(ko)

    def qk_norm_rope_kv(self, q, k, v, wq, wk, eps, pos, n_dims, theta, cache, filled):
        kc, vc = _t(self.g, cache["k"]), _t(self.g, cache["v"])
        qo = self.g.qk_norm_rope_kv(_t(self.g, q), _t(self.g, k), _t(self.g, v), _t(self.g, wq), _t(self.g, wk), eps,
                                    _t(self.g, pos), n_dims, theta, kc, vc, filled)
        cache["k"][...] = _np(kc)
        cache["v"][...] = _np(vc)
        return _np(qo)

    def soft_max_ext(self, scores, mask, scale):
        return _np(self.g.soft_max_ext(_t(self.g, scores), None if mask is None else _t(self.g, mask), scale))

    def add_rms_norm_w(self, a, b, w, eps):
        s, y = self.g.add_rms_norm_mul(_t(self.g, a), _t(self.g, b), _t(self.g, w), eps)
        return _np(s), _np(y)

    def swiglu(self, gate, up):
        return _np(self.g.swiglu(_t(self.g, gate), _t(self.g, up)))

    def add(self, a, b):
        return _np(self.g.add(_t(self.g, a), _t(self.g, b)))

    def get_rows(self, table, ids):
        return _np(self.g.get_rows(_t(self.g, table), _t(self.g, ids)))


def _golden(name):
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name)) as f:
        return json.load(f)


def test_golden_g1_decoder_layer_on_gpu(gpu):
    import test_oracle_goldens as G
    d = _golden("qwen3_decoder_layer.json")
    got = G.run_decoder_golden(d, HipOps(gpu))
    exp = np.array(d["expected_hidden"], np.float32)
    assert np.abs(got - exp).max() < d["tolerance_gpu"]
    assert np.abs(got - exp).max() < d["tolerance_cpu"]
    assert_close(got.reshape(4, -1), G.run_decoder_golden(d).reshape(4, -1))


def test_golden_g2_summed_embedding_on_gpu(gpu):
    import test_oracle_goldens as G
    d = _golden("qwen3_code_predictor.json")
    _, codes, summed_ref, tables = G.run_code_predictor(d)
    got = _np(gpu.get_rows_sum([_t(gpu, t) for t in tables], _t(gpu, np.array([[c] for c in codes], np.int32))))
    assert_bitexact(got.reshape(-1), summed_ref)
    assert np.abs(got.reshape(-1) - np.array(d["expected_summed_embedding"], np.float32)).max() < d["tolerance_cpu"]


@pytest.mark.parametrize("C,T", [(16, 37), (512, 257)])
def test_golden_g4_kokoro_snake_on_gpu(gpu, C, T):
    """reference_snake, tests/kokoro_decoder_test.cpp:81-90: y = x + sin(a x)^2
    / a in double on [C, T] (element (c, t) at t*C + c), at the test's 1e-4;
    the f32 node-by-node form stays within a few ulp of it."""
    rng = np.random.default_rng(20260728 + C)
    x = rng.standard_normal((T, C)).astype(np.float32)
    alpha = np.exp(rng.uniform(np.log(0.1), np.log(10.0), C)).astype(np.float32)
    got = _np(gpu.snake(_t(gpu, x), _t(gpu, alpha))).astype(np.float64)
    a = alpha.astype(np.float64)
    ref = x + np.sin(a * x) ** 2 / a
    assert np.abs(got - ref).max() < 1e-4
    assert np.abs(got - ref).max() < 8 * np.finfo(np.float32).eps * np.abs(ref).max()


def test_q8_last_row_at_end_of_allocation(gpu):
    """Regression: 16 Q8_0 tables stacked in one allocation of exactly 34 MiB (a
    multiple of the allocator's 2 MiB granularity, so nothing follows the last
    row of table 15). Gathering that last row, alone and in the gather->sum,
    must read only inside the row and match the oracle bit for bit."""
    import torch
    rng = np.random.default_rng(SEED + 34)
    groups, rows, ne0 = 16, 2048, 1024
    raw = np.stack([F.q8_0_synthetic(rng, rows, ne0) for _ in range(groups)])
    assert raw.nbytes == 34 << 20
    dev = torch.from_numpy(raw).cuda()
    tabs = [gpu.Q8Tensor(dev[t], ne0) for t in range(groups)]
    ids = np.array([rows - 1, 0, rows - 1, 17], np.int32)
    got = _np(gpu.get_rows(tabs[-1], _t(gpu, ids)))
    assert_bitexact(got, F.q8_0_dequant(raw[-1], ne0)[ids])
    codes = rng.integers(0, rows, (groups, 64)).astype(np.int32)
    codes[:, :3] = rows - 1
    ref = R.run(lambda g: R.sum_code_embeddings(g, list(raw), R.Q8_0, ne0, codes))
    assert_bitexact(_np(gpu.get_rows_sum(tabs, _t(gpu, codes))), ref)


@pytest.mark.parametrize("ne0", [1024, 2048])
def test_q8_unaligned_table_and_bad_id_in_sum(gpu, ne0):
    """A Q8_0 table view that starts 4 bytes into its allocation (4-byte but not
    16-byte aligned rows) takes the register-decode get_rows instead of the
    LDS-staged one, and the gather->sum's windows at 4-byte alignment, and
    still matches bit for bit; an out-of-range id in one
    group of a Q8_0 gather->sum turns that frame into NaN and leaves the
    others exact."""
    import torch
    rng = np.random.default_rng(SEED + ne0 + 4)
    rows, rb = 64, ne0 // 32 * 34
    raw = F.q8_0_synthetic(rng, rows, ne0)
    buf = torch.zeros(rows * rb + 16, dtype=torch.uint8, device="cuda")
    buf[4:4 + rows * rb] = torch.from_numpy(raw.reshape(-1)).cuda()
    view = gpu.Q8Tensor(buf[4:4 + rows * rb].view(rows, rb), ne0)
    ids = rng.integers(0, rows, 40).astype(np.int32)
    assert_bitexact(_np(gpu.get_rows(view, _t(gpu, ids))), F.q8_0_dequant(raw, ne0)[ids])
    tabs = [F.q8_0_synthetic(rng, rows, ne0) for _ in range(6)]
    codes = rng.integers(0, rows, (6, 50)).astype(np.int32)
    ref = R.run(lambda g: R.sum_code_embeddings(g, tabs, R.Q8_0, ne0, codes))
    dev = [gpu.Q8Tensor(_t(gpu, t), ne0) for t in tabs]
    assert_bitexact(_np(gpu.get_rows_sum(dev, _t(gpu, codes))), ref)
    mixed = [view] + dev[1:]
    ref_mixed = R.run(lambda g: R.sum_code_embeddings(g, [raw] + tabs[1:], R.Q8_0, ne0, codes))
    assert_bitexact(_np(gpu.get_rows_sum(mixed, _t(gpu, codes))), ref_mixed)
    bad = codes.copy()
    bad[3, 7] = rows
    bad[1, 9] = -1
    out = _np(gpu.get_rows_sum(dev, _t(gpu, bad)))
    assert np.isnan(out[7]).all() and np.isnan(out[9]).all()
    keep = [f for f in range(50) if f not in (7, 9)]
    assert_bitexact(out[keep], ref[keep])


def test_float_parity_report(gpu):
    """The floating-point ops at their configs[1]/[3] shapes: the worst
    elementwise relative error (floored as in assert_close, or pair-relative for
    rope), the normwise error ||got - ref|| / ||ref|| and the share of outputs
    bit-identical to the ggml-CPU restatement, each held to the 1e-5 bar. With
    SHP_PARITY_REPORT set, the figures are also written there as JSON."""
    rng = np.random.default_rng(SEED + 4242)
    eps, theta = np.float32(1e-6), np.float32(1e6)
    rows = []

    def record(op, shape, got, ref, pair_dims=None):
        if pair_dims:
            worst = assert_rope_close(got, ref, pair_dims)
        else:
            worst, _ = assert_close(got, ref)
        nw = normwise(got, ref)
        assert nw <= REL_TOL
        rows.append({"op": op, "shape": list(shape), "max_rel": worst, "normwise": nw,
                     "bit_identical": float((np.asarray(got, np.float32).view(np.uint32) ==
                                             np.asarray(ref, np.float32).view(np.uint32)).mean())})

    x = rng.standard_normal((512, 1024)).astype(np.float32)
    w, wt = _weights(rng, 1024, "bf16")
    record("rms_norm_mul", x.shape, _np(gpu.rms_norm_mul(_t(gpu, x), _dev_w(gpu, w, "bf16"), eps)),
           R.run(lambda g: R.rms_norm_w(g, x, w, eps, wt)))
    b = rng.standard_normal((512, 1024)).astype(np.float32)
    _, y_ref = R.run(lambda g: R.add_rms_norm_w(g, x, b, w, eps, wt))
    _, y = gpu.add_rms_norm_mul(_t(gpu, x), _t(gpu, b), _dev_w(gpu, w, "bf16"), eps)
    record("add_rms_norm_mul", x.shape, _np(y), y_ref)
    q = rng.standard_normal((512, 16, 128)).astype(np.float32)
    k = rng.standard_normal((512, 8, 128)).astype(np.float32)
    wq, _ = _weights(rng, 128, "bf16")
    wk, _ = _weights(rng, 128, "bf16")
    pos = np.arange(512, dtype=np.int32)
    qr, kr = R.run(lambda g: R.qk_norm_rope(g, q, k, wq, wk, eps, pos, 128, theta, R.BF16))
    qo, ko = gpu.qk_norm_rope(_t(gpu, q), _t(gpu, k), _dev_w(gpu, wq, "bf16"), _dev_w(gpu, wk, "bf16"), eps,
                              _t(gpu, pos), 128, theta)
    record("qk_norm_rope q", q.shape, _np(qo), qr, 128)
    record("qk_norm_rope k", k.shape, _np(ko), kr, 128)
    gt = rng.standard_normal((512, 3072)).astype(np.float32)
    up = rng.standard_normal((512, 3072)).astype(np.float32)
    record("swiglu", gt.shape, _np(gpu.swiglu(_t(gpu, gt), _t(gpu, up))), R.run(lambda g: R.swiglu(g, gt, up)))
    xs = rng.standard_normal((8192, 512)).astype(np.float32)
    alpha = np.exp(rng.uniform(np.log(0.1), np.log(10.0), 512)).astype(np.float32)
    record("snake", xs.shape, _np(gpu.snake(_t(gpu, xs), _t(gpu, alpha))), R.run(lambda g: R.snake(g, xs, alpha)))
    s_ = rng.standard_normal((16, 512, 512)).astype(np.float32) * 3
    m = np.zeros((512, 512), np.float32)
    m[np.triu_indices(512, 1, 512)] = -np.inf
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    record("soft_max_ext causal", s_.shape, _np(gpu.soft_max_ext(_t(gpu, s_), _t(gpu, m), scale)),
           R.run(lambda g: g.soft_max_ext(s_, m, scale)))
    out = os.environ.get("SHP_PARITY_REPORT")
    if out:
        with open(out, "w") as f:
            json.dump(rows, f, indent=1)


"""GPU parity of the Q5_K gathers (shp_get_rows and shp_get_rows_sum over
ggml block_q5_K tables, the talker's embedding tables under the reference's
Q5_K_MIXED profile, src/arch/qwen3-tts/catalog.cpp:165-192), through the C
ABI, bit for bit against the oracle's dequantize_row_q5_K restatement (itself
pinned by the hand-assembled block and the exact formula of
tests/test_q5k_format.py). Every value is one rounding of exact products, so
there is no tolerance: raw 32-bit patterns are compared."""
import numpy as np
import pytest

import formats as F
import ggml_ref as R
from test_gpu_parity import _np, _t, assert_bitexact
from test_q5k_format import hand_block, hand_block2, hand_values, hand_values2

pytestmark = pytest.mark.gpu
SEED = 20260728


def _table(gpu, raw, ne0):
    return gpu.Q5KTensor(_t(gpu, raw), ne0)


@pytest.mark.parametrize("ne0,rows,n", [(256, 50, 77), (512, 30, 64), (768, 20, 40), (1024, 2048, 4096),
                                        (2048, 300, 512), (4096, 9, 33)])
def test_get_rows_q5k_bitexact(gpu, ne0, rows, n):
    """Widths of 1..16 super-blocks (768: three, a chunk left part-full);
    (1024, 2048, 4096) is a codec table of configs[2]'s shape."""
    rng = np.random.default_rng(SEED + ne0 + rows)
    raw = F.q5_k_synthetic(rng, rows, ne0)
    ids = rng.integers(0, rows, n).astype(np.int32)
    ids[:2] = [0, rows - 1]
    ref = R.run(lambda g: g.get_rows(raw, R.Q5_K, ne0, ids))
    got = _np(gpu.get_rows(_table(gpu, raw, ne0), _t(gpu, ids)))
    assert_bitexact(got, ref)
    assert_bitexact(got, F.q5_k_values(*F.q5_k_fields(np.random.default_rng(SEED + ne0 + rows), rows, ne0))[ids])


def test_get_rows_q5k_hand_block_and_bad_ids(gpu):
    raw = np.frombuffer(hand_block() * 3, np.uint8).reshape(3, 176).copy()
    ids = np.array([2, 0, -1, 3, 1, 1 << 30], np.int32)
    got = _np(gpu.get_rows(_table(gpu, raw, 256), _t(gpu, ids)))
    for r in (0, 1, 4):
        assert_bitexact(got[r], hand_values())
    for r in (2, 3, 5):  # out of range: a quiet-NaN row, nothing read
        assert np.isnan(got[r]).all()


def test_get_rows_q5k_second_hand_block(gpu):
    """The second hand-assembled block (every sub-block, every qh bit, both
    nibbles of every scales[8..11] byte) through the 256-wide kernel and, as
    the four super-blocks of 1024-wide rows, through the staged one: the
    worked-out values bit for bit, +0.0 included."""
    b1, b2 = hand_block(), hand_block2()
    raw = np.frombuffer(b2 + b1, np.uint8).reshape(2, 176).copy()
    got = _np(gpu.get_rows(_table(gpu, raw, 256), _t(gpu, np.array([0, 1, 0], np.int32))))
    for r, want in ((0, hand_values2()), (1, hand_values()), (2, hand_values2())):
        assert_bitexact(got[r], want)
    wide = np.frombuffer(b1 + b2 + b2 + b1 + b2 + b1 + b1 + b2, np.uint8).reshape(2, 4 * 176).copy()
    got = _np(gpu.get_rows(_table(gpu, wide, 1024), _t(gpu, np.array([1, 0, 1, 5], np.int32))))
    rows = {0: [hand_values(), hand_values2(), hand_values2(), hand_values()],
            1: [hand_values2(), hand_values(), hand_values(), hand_values2()]}
    for r, rid in enumerate([1, 0, 1]):
        assert_bitexact(got[r], np.concatenate(rows[rid]))
    assert np.isnan(got[3]).all()


def test_get_rows_q5k_special_scales(gpu):
    """d and dmin over -0, +0, f16 subnormals, the largest f16 and ordinary
    values (no inf or NaN scale: inf*0 makes a NaN whose sign differs between
    CPU and GPU arithmetic)."""
    rng = np.random.default_rng(SEED + 3)
    rows, ne0 = 64, 1024
    d, dmin, sc, m, q = F.q5_k_fields(rng, rows, ne0)
    specials = np.array([0x8000, 0x0000, 0x0001, 0x03FF, 0x7BFF, 0x3C00, 0xBC00, 0x1400], np.uint16)
    d[:] = specials[rng.integers(0, len(specials), d.shape)]
    dmin[:] = specials[rng.integers(0, len(specials), dmin.shape)]
    sc[0], m[0], q[0] = 63, 63, 31
    sc[1], m[1], q[1] = 0, 0, 0
    raw = F.q5_k_pack(d, dmin, sc, m, q)
    ids = np.arange(rows, dtype=np.int32)
    ref = R.run(lambda g: g.get_rows(raw, R.Q5_K, ne0, ids))
    assert_bitexact(_np(gpu.get_rows(_table(gpu, raw, ne0), _t(gpu, ids))), ref)


def test_get_rows_q5k_batched_and_misaligned(gpu):
    """ggml's batched form (table [ne0, rows, 2], ids [n, 2]); a table at a
    2-byte offset and an output at a 4-byte offset take the element-wise
    kernel, with the same bits."""
    import torch
    rng = np.random.default_rng(SEED + 9)
    ne0, rows = 512, 25
    raw = np.stack([F.q5_k_synthetic(rng, rows, ne0) for _ in range(2)])
    ids = rng.integers(0, rows, (2, 31)).astype(np.int32)
    ref = np.stack([R.run(lambda g, b=b: g.get_rows(raw[b], R.Q5_K, ne0, ids[b])) for b in range(2)])
    got = _np(gpu.get_rows(gpu.Q5KTensor(_t(gpu, raw), ne0), _t(gpu, ids)))
    assert_bitexact(got, ref)
    flat = raw[0]
    buf = torch.zeros(flat.size + 2, dtype=torch.uint8, device="cuda")
    buf[2:].copy_(torch.from_numpy(flat.reshape(-1)).cuda())
    view = buf[2:].view(rows, flat.shape[1])
    assert view.data_ptr() % 4 == 2
    out_buf = torch.empty(31 * ne0 + 1, dtype=torch.float32, device="cuda")
    out = out_buf[1:].view(31, ne0)
    gpu.get_rows(gpu.Q5KTensor(view, ne0), _t(gpu, ids[0]), out=out)
    assert_bitexact(_np(out), ref[0])


@pytest.mark.parametrize("ne0", [1024, 2048, 4096])
def test_get_rows_q5k_staged_bad_ids_and_4_byte_table(gpu, ne0):
    """The LDS-staged widths: ids out of range give a quiet-NaN row while the
    rows around them stay exact; the same table 4 bytes off a 16-byte boundary
    takes the per-super-block kernel, with the same bits."""
    import torch
    rng = np.random.default_rng(SEED + 11 + ne0)
    rows = 40
    raw = F.q5_k_synthetic(rng, rows, ne0)
    ids = rng.integers(0, rows, 37).astype(np.int32)
    ids[[3, 17, 36]] = [-1, rows, -(1 << 31)]
    ok = (ids >= 0) & (ids < rows)
    ref = R.run(lambda g: g.get_rows(raw, R.Q5_K, ne0, np.where(ok, ids, 0).astype(np.int32)))
    got = _np(gpu.get_rows(_table(gpu, raw, ne0), _t(gpu, ids)))
    assert np.isnan(got[~ok]).all()
    assert_bitexact(got[ok], ref[ok])
    buf = torch.zeros(raw.size + 4, dtype=torch.uint8, device="cuda")
    buf[4:].copy_(torch.from_numpy(raw.reshape(-1)).cuda())
    view = buf[4:].view(rows, raw.shape[1])
    assert view.data_ptr() % 16 == 4
    got4 = _np(gpu.get_rows(gpu.Q5KTensor(view, ne0), _t(gpu, ids)))
    assert np.isnan(got4[~ok]).all()
    assert_bitexact(got4[ok], ref[ok])


@pytest.mark.parametrize("ne0,groups,frames", [(1024, 16, 4096), (1024, 15, 64), (256, 1, 33), (512, 3, 100),
                                               (2048, 9, 50), (4096, 4, 20), (1024, 33, 40), (1024, 1, 7),
                                               (3072, 2, 9)])
def test_get_rows_sum_q5k_bitexact(gpu, ne0, groups, frames):
    """sum_code_embeddings over Q5_K tables (code-predictor.cpp:82-107): the
    ordered f32 sum of the dequantized rows, bit for bit. (1024, 16, 4096) is
    configs[2]'s shape with Q5_K codebooks. Widths 1024, 2048 and 4096 take
    the 1024-element slab windows (groups in chunks of 8: 15, 9, 33 and 1
    leave slots past the last group), 256 and 512 the narrow kernel, 3072 the
    element-wise one."""
    rng = np.random.default_rng(SEED + 17 + ne0 + groups)
    rows = 2048 if frames >= 4096 else 60
    tabs = [F.q5_k_synthetic(rng, rows, ne0) for _ in range(groups)]
    codes = rng.integers(0, rows, (groups, frames)).astype(np.int32)
    ref = R.run(lambda g: R.sum_code_embeddings(g, tabs, R.Q5_K, ne0, codes))
    got = _np(gpu.get_rows_sum([_table(gpu, t, ne0) for t in tabs], _t(gpu, codes)))
    assert_bitexact(got, ref)


@pytest.mark.parametrize("groups", [57, 63, 64])
def test_get_rows_sum_q5k_many_groups(gpu, groups):
    """57 to 64 groups over 1024-wide Q5_K tables: the slab windows take
    groups in chunks of 8, so 57 and 63 leave slots past the last group and 64
    fills every chunk (the prefetch past the last chunk clamps its slot); one
    frame holds an out-of-range id in the last group, whose row is NaN, and
    every other frame equals the restatement's ordered sum bit for bit."""
    rng = np.random.default_rng(SEED + 53 + groups)
    ne0, rows, frames = 1024, 40, 300
    tabs = [F.q5_k_synthetic(rng, rows, ne0) for _ in range(groups)]
    codes = rng.integers(0, rows, (groups, frames)).astype(np.int32)
    codes[groups - 1, 17] = rows + 3
    got = _np(gpu.get_rows_sum([_table(gpu, t, ne0) for t in tabs], _t(gpu, codes)))
    assert np.isnan(got[17]).all()
    ok = [f for f in range(frames) if f != 17]
    ref = R.run(lambda g: R.sum_code_embeddings(g, tabs, R.Q5_K, ne0, np.minimum(codes, rows - 1)))
    assert_bitexact(got[ok], ref[ok])


def test_get_rows_sum_q5k_order_and_bad_id(gpu):
    """The sum is order-dependent in f32 (it is one chain of adds), and an id
    out of range in any group makes the frame's row NaN."""
    rng = np.random.default_rng(SEED + 29)
    ne0, rows, groups = 1024, 30, 5
    tabs = [F.q5_k_synthetic(rng, rows, ne0, 1e-2, 5e-2) for _ in range(groups)]
    codes = rng.integers(0, rows, (groups, 40)).astype(np.int32)
    codes[3, 7] = rows
    codes[0, 9] = -5
    dev = [_table(gpu, t, ne0) for t in tabs]
    got = _np(gpu.get_rows_sum(dev, _t(gpu, codes)))
    assert np.isnan(got[7]).all() and np.isnan(got[9]).all()
    ok = [f for f in range(40) if f not in (7, 9)]
    ref = R.run(lambda g: R.sum_code_embeddings(g, tabs, R.Q5_K, ne0, np.where(codes < 0, 0, np.minimum(codes, rows - 1))))
    assert_bitexact(got[ok], ref[ok])
    rev = _np(gpu.get_rows_sum(dev[::-1], _t(gpu, np.ascontiguousarray(codes[::-1]))))
    assert not np.array_equal(rev[ok].view(np.uint32), got[ok].view(np.uint32))


def test_get_rows_sum_q5k_padded_rows(gpu):
    """Tables whose rows are padded past the 704 bytes of a 1024-wide row (row
    stride 720) cannot take the windows' 32-bit dense offsets; they take the
    element-wise kernel, with the same bits."""
    import torch
    rng = np.random.default_rng(SEED + 41)
    ne0, rows, groups, frames = 1024, 50, 4, 64
    tabs = [F.q5_k_synthetic(rng, rows, ne0) for _ in range(groups)]
    codes = rng.integers(0, rows, (groups, frames)).astype(np.int32)
    ref = R.run(lambda g: R.sum_code_embeddings(g, tabs, R.Q5_K, ne0, codes))
    dev = []
    for t in tabs:
        buf = torch.zeros((rows, 720), dtype=torch.uint8, device="cuda")
        buf[:, :704].copy_(torch.from_numpy(t).cuda())
        dev.append(gpu.Q5KTensor(buf[:, :704], ne0))
    assert dev[0].data.stride(0) == 720
    assert_bitexact(_np(gpu.get_rows_sum(dev, _t(gpu, codes))), ref)

"""GGUF tables streamed into device memory (shp_gguf_load_tensor) and read in
place by the gathers: the device bytes equal the file's, and get_rows /
get_rows_sum over the loaded tables equal the restatement on the same bytes,
bit for bit. The BF16 table is 41 MB, so its load crosses the 32 MiB staging
chunk and ends on a partial one."""
import numpy as np
import pytest

import formats as F
import gguf_ref as G
import ggml_ref as R

pytestmark = pytest.mark.gpu

TEXT = "talker.model.text_embedding.weight"
CODEC = "talker.code_predictor.model.codec_embedding.%d.weight"


def _package(tmp_path, rng):
    bf = F.f32_to_bf16_bits(rng.standard_normal((10000, 2048)) * 0.02)
    q8 = [F.q8_0_synthetic(rng, 2048, 1024) for _ in range(15)]
    tensors = [(TEXT, G.GGML_BF16, [2048, 10000], bf.tobytes())]
    tensors += [(CODEC % g, G.GGML_Q8_0, [1024, 2048], t.tobytes()) for g, t in enumerate(q8)]
    tensors.append(("talker.model.norm.weight", G.GGML_F32, [1024], rng.standard_normal(1024).astype(np.float32)
                    .tobytes()))
    p = tmp_path / "pkg-Q8_MIXED.gguf"
    G.write(p, [("general.architecture", G.STRING, "qwen3-tts"),
                ("synthesize.quantization.profile", G.STRING, "Q8_MIXED")], tensors, alignment=64)
    return p, bf, q8


def test_tables_load_and_gather_in_place(gpu, tmp_path):
    import torch
    rng = np.random.default_rng(41)
    p, bf, q8 = _package(tmp_path, rng)
    raw = p.read_bytes()
    with gpu.GgufFile(p) as f:
        assert gpu.table_type_for_profile(f.kv_string("synthesize.quantization.profile")) == gpu.TYPE_Q8_0
        text = f.load(TEXT)
        assert text.dtype == torch.bfloat16 and tuple(text.shape) == (10000, 2048)
        _, nbytes, off = f.info(TEXT)
        assert bytes(text.view(torch.uint8).cpu().numpy().tobytes()) == raw[off:off + nbytes]
        codec = [f.load(CODEC % g) for g in range(15)]
        for g, t in enumerate(codec):
            _, nbytes, off = f.info(CODEC % g)
            assert t.ne0 == 1024 and t.rows == 2048
            assert bytes(t.data.cpu().numpy().tobytes()) == raw[off:off + nbytes]
        norm = f.load("talker.model.norm.weight")
        assert tuple(norm.shape) == (1024,)

    ids = rng.integers(0, 10000, 300).astype(np.int32)
    ids[:2] = [0, 9999]
    got = gpu.get_rows(text, torch.from_numpy(ids).cuda())
    ref = R.run(lambda g: g.get_rows(bf, R.BF16, 2048, ids))
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))

    codes = rng.integers(0, 2048, (15, 64)).astype(np.int32)
    got = gpu.get_rows_sum(codec, torch.from_numpy(codes).cuda())
    ref = R.run(lambda g: R.sum_code_embeddings(g, q8, R.Q8_0, 1024, codes))
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_load_into_a_smaller_buffer_is_refused(gpu, tmp_path):
    import ctypes
    import torch
    p = tmp_path / "small.gguf"
    G.write(p, [], [("t", G.GGML_F32, [256], np.arange(256, dtype=np.float32).tobytes())])
    dst = torch.zeros(1024, dtype=torch.uint8, device="cuda")
    with gpu.GgufFile(p) as f:
        d = gpu.ShpTensor()
        L = gpu.load()
        assert L.shp_gguf_load_tensor(f._h, b"t", ctypes.c_void_p(dst.data_ptr()), 1023, ctypes.byref(d),
                                      None) == gpu.ERR_INVALID_ARG
        assert L.shp_gguf_load_tensor(f._h, b"t", ctypes.c_void_p(dst.data_ptr()), 1024, ctypes.byref(d),
                                      None) == gpu.OK
        torch.cuda.synchronize()
        np.testing.assert_array_equal(dst.cpu().numpy().view(np.float32), np.arange(256, dtype=np.float32))
        assert d.data == dst.data_ptr() and d.ne[0] == 256


def test_load_many_matches_the_file_across_chunk_boundaries(gpu, tmp_path):
    """shp_gguf_load_tensors over the whole package in a shuffled order: the
    41 MB BF16 table spans two 32 MiB staging chunks and the small tensors
    share chunks with it and with each other; every device tensor equals the
    file's bytes, and the gathers read the loaded tables as before."""
    import torch
    rng = np.random.default_rng(43)
    p, bf, q8 = _package(tmp_path, rng)
    raw = p.read_bytes()
    with gpu.GgufFile(p) as f:
        names = list(f.tensor_names())
        order = [names[i] for i in rng.permutation(len(names))]
        loaded = f.load_many(order)
        for name, t in zip(order, loaded):
            _, nbytes, off = f.info(name)
            data = t.data if isinstance(t, gpu.Q8Tensor) else t
            assert bytes(data.contiguous().view(torch.uint8).cpu().numpy().tobytes()) == raw[off:off + nbytes], name
        assert f.load_many([]) == []
        one = f.load_many([TEXT])[0]
        assert torch.equal(one.view(torch.int16), loaded[order.index(TEXT)].view(torch.int16))
    codec = [loaded[order.index(CODEC % g)] for g in range(15)]
    codes = rng.integers(0, 2048, (15, 64)).astype(np.int32)
    got = gpu.get_rows_sum(codec, torch.from_numpy(codes).cuda())
    ref = R.run(lambda g: R.sum_code_embeddings(g, q8, R.Q8_0, 1024, codes))
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))

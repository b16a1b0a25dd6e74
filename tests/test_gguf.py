"""GGUF package reader (include/synth_gguf.h) without a GPU: header parsing,
tensor descriptions and metadata against the format restatement
(oracle/gguf_ref.py), whose writer is pinned by a file assembled by hand, field
by field; every malformed-file rule; and the quantization-profile table rule of
src/arch/qwen3-tts/catalog.cpp:155-196. Device loading is in
tests/test_gpu_gguf.py."""
import struct

import numpy as np
import pytest

import gguf_ref as G
import synth_hip as S


def known_answer_bytes():
    """One F32 tensor "t" of 4 elements, alignment 32, one key: spelled out."""
    b = b"GGUF"                                   # magic
    b += struct.pack("<I", 3)                     # version
    b += struct.pack("<Q", 1)                     # tensor count
    b += struct.pack("<Q", 1)                     # key/value count
    b += struct.pack("<Q", 17) + b"general.alignment"
    b += struct.pack("<I", 4)                     # value type u32
    b += struct.pack("<I", 32)                    # alignment
    b += struct.pack("<Q", 1) + b"t"              # tensor name
    b += struct.pack("<I", 1)                     # n_dims
    b += struct.pack("<Q", 4)                     # ne[0]
    b += struct.pack("<I", 0)                     # ggml type F32
    b += struct.pack("<Q", 0)                     # offset
    assert len(b) == 4 + 4 + 8 + 8 + 25 + 4 + 4 + 9 + 4 + 8 + 4 + 8 == 90
    b += b"\0" * (96 - len(b))                    # pad to the alignment
    b += struct.pack("<4f", 1.0, -2.0, 0.5, 3.0)  # data
    b += b"\0" * 16                               # each tensor padded to the alignment, the last included
    return b


def test_writer_matches_hand_assembled_file(tmp_path):
    p = tmp_path / "kat.gguf"
    data = struct.pack("<4f", 1.0, -2.0, 0.5, 3.0)
    start = G.write(p, [], [("t", G.GGML_F32, [4], data)], alignment=32)
    assert start == 96
    assert p.read_bytes() == known_answer_bytes()


def test_reader_on_hand_assembled_file(tmp_path):
    p = tmp_path / "kat.gguf"
    p.write_bytes(known_answer_bytes())
    with S.GgufFile(p) as f:
        assert f.version == 3
        assert f.tensor_names() == ["t"]
        d, nbytes, off = f.info("t")
        assert (d.type, list(d.ne), list(d.nb), nbytes, off) == (S.TYPE_F32, [4, 1, 1, 1], [4, 16, 16, 16], 16, 96)
        assert d.data is None
        assert f.kv_u32("general.alignment") == 32


def _tables(rng):
    import formats as F
    bf = F.f32_to_bf16_bits(rng.standard_normal((100, 2048)) * 0.02)
    q8 = F.q8_0_synthetic(rng, 50, 1024)
    q5 = F.q5_k_synthetic(rng, 20, 1024)
    f16 = F.f32_to_f16_bits(rng.standard_normal((3, 5, 64)))
    f32 = rng.standard_normal(7).astype(np.float32)
    i32 = np.arange(12, dtype=np.int32).reshape(3, 4)
    return [("talker.model.text_embedding.weight", G.GGML_BF16, [2048, 100], bf.tobytes()),
            ("talker.code_predictor.model.codec_embedding.0.weight", G.GGML_Q8_0, [1024, 50], q8.tobytes()),
            ("talker.code_predictor.model.codec_embedding.1.weight", G.GGML_Q5_K, [1024, 20], q5.tobytes()),
            ("conv.weight", G.GGML_F16, [64, 5, 3], f16.tobytes()),
            ("bias", G.GGML_F32, [7], f32.tobytes()),
            ("ids", G.GGML_I32, [4, 3], i32.tobytes())]


KV = [("general.architecture", G.STRING, "qwen3-tts"),
      ("synthesize.quantization.profile", G.STRING, "Q8_MIXED"),
      ("synthesize.quantization.profile_version", G.U32, 1),
      ("synthesize.capabilities.max_output_frames", G.U64, 15728640),
      ("synthesize.capabilities.min_speaking_rate", G.F32, 0.5),
      ("a.u8", G.U8, 200), ("a.i8", G.I8, -5), ("a.u16", G.U16, 60000), ("a.i16", G.I16, -30000),
      ("a.i32", G.I32, -7), ("a.bool", G.BOOL, True), ("a.i64", G.I64, -(1 << 40)), ("a.f64", G.F64, 2.5),
      ("tokenizer.tokens", G.ARRAY, (G.STRING, ["a", "bb", "", "音声"])),
      ("a.array_u32", G.ARRAY, (G.U32, [1, 2, 3]))]


@pytest.mark.parametrize("alignment", [None, 64, 4096])
def test_round_trip_against_the_restatement(tmp_path, alignment):
    rng = np.random.default_rng(31)
    p = tmp_path / "pkg.gguf"
    tensors = _tables(rng)
    G.write(p, KV, tensors, alignment=alignment)
    version, kv, infos, data_start = G.read(p)
    assert data_start % (alignment or 32) == 0
    raw = p.read_bytes()
    with S.GgufFile(p) as f:
        assert f.version == version == 3
        assert f.tensor_names() == [t[0] for t in tensors]
        for name, gtype, ne, data in tensors:
            d, nbytes, off = f.info(name)
            rtype, rne, roff, rbytes = infos[name]
            assert d.type == gtype == rtype
            assert list(d.ne) == rne + [1] * (4 - len(rne))
            assert (nbytes, off) == (rbytes, roff) and raw[off:off + nbytes] == data
            be, bb = G.BLOCKS[gtype]
            assert d.nb[0] == bb and d.nb[1] == ne[0] // be * bb
            assert d.nb[2] == d.nb[1] * d.ne[1] and d.nb[3] == d.nb[2] * d.ne[2]
        assert f.kv_string("general.architecture") == "qwen3-tts"
        assert f.kv_string("synthesize.quantization.profile") == "Q8_MIXED"
        assert f.kv_u32("synthesize.quantization.profile_version") == 1
        with pytest.raises(S.ShpError):
            f.kv_u32("synthesize.capabilities.max_output_frames")  # a u64, not a u32
        with pytest.raises(S.ShpError):
            f.kv_string("general.architecture", capacity=9)  # no room for the terminator
        with pytest.raises(S.ShpError):
            f.info("missing.weight")


def _expect_open(path, status):
    with pytest.raises(S.ShpError) as e:
        S.GgufFile(path)
    assert e.value.status == status


def test_every_truncation_is_refused(tmp_path):
    """Each prefix of a valid file that cuts the header or a tensor's bytes is
    refused; one that cuts only the last tensor's trailing alignment padding
    opens (the tensor is whole), as does the whole file."""
    p = tmp_path / "full.gguf"
    G.write(p, KV[:3], [("t", G.GGML_F32, [4], struct.pack("<4f", 1, 2, 3, 4))])
    full = p.read_bytes()
    _, _, infos, _ = G.read(p)
    _, _, off, nbytes = infos["t"]
    need = off + nbytes
    assert need < len(full)
    q = tmp_path / "cut.gguf"
    for n in range(len(full) + 1):
        q.write_bytes(full[:n])
        if n < need:
            _expect_open(q, S.ERR_INVALID_ARG)
        else:
            S.GgufFile(q).close()


def _patched(tmp_path, mutate, tensors=None, kv=None, alignment=None):
    p = tmp_path / "bad.gguf"
    G.write(p, kv if kv is not None else KV[:2], tensors or [("t", G.GGML_F32, [8], bytes(32))], alignment=alignment)
    b = bytearray(p.read_bytes())
    mutate(b)
    p.write_bytes(bytes(b))
    return p


def _find(b, s):
    i = bytes(b).find(s)
    assert i >= 0
    return i


def test_malformed_files_are_refused(tmp_path):
    inv, uns = S.ERR_INVALID_ARG, S.ERR_UNSUPPORTED

    def magic(b):
        b[0:4] = b"GGUG"
    _expect_open(_patched(tmp_path, magic), inv)

    def version1(b):
        b[4:8] = struct.pack("<I", 1)
    _expect_open(_patched(tmp_path, version1), inv)

    # the tensor info sits after the name "t" (u64 len 1 + b"t")
    def tinfo(b):
        return _find(b, struct.pack("<Q", 1) + b"t") + 9  # -> n_dims

    def ndims5(b):
        b[tinfo(b):tinfo(b) + 4] = struct.pack("<I", 5)
    _expect_open(_patched(tmp_path, ndims5), inv)

    def zero_dim(b):
        b[tinfo(b) + 4:tinfo(b) + 12] = struct.pack("<Q", 0)
    _expect_open(_patched(tmp_path, zero_dim), inv)

    def unknown_type(b):
        b[tinfo(b) + 12:tinfo(b) + 16] = struct.pack("<I", 99)
    _expect_open(_patched(tmp_path, unknown_type), uns)

    def misaligned(b):
        b[tinfo(b) + 16:tinfo(b) + 24] = struct.pack("<Q", 4)
    _expect_open(_patched(tmp_path, misaligned), inv)

    def past_end(b):
        b[tinfo(b) + 16:tinfo(b) + 24] = struct.pack("<Q", 32)
    _expect_open(_patched(tmp_path, past_end), inv)

    # Dimensions each within 2^62 whose product wraps 64 (and 128) bits: the
    # byte count is built one factor at a time and refused once past 2^62.
    four_d = [("t", G.GGML_F32, [4, 1, 1, 1], bytes(16))]
    for dims in ([4, 1 << 62, 1 << 62, 16], [4, 1 << 62, 2, 1], [1 << 61, 2, 1, 1], [4, 1 << 30, 1 << 30, 1 << 2]):
        def huge(b, dims=dims):
            b[tinfo(b) + 4:tinfo(b) + 36] = struct.pack("<4Q", *dims)
        _expect_open(_patched(tmp_path, huge, tensors=four_d), inv)

    q8_odd = [("t", G.GGML_Q8_0, [32], bytes(34))]

    def q8_partial_block(b):
        b[tinfo(b) + 4:tinfo(b) + 12] = struct.pack("<Q", 48)
    _expect_open(_patched(tmp_path, q8_partial_block, tensors=q8_odd), inv)

    dup_t = [("t", G.GGML_F32, [8], bytes(32)), ("t", G.GGML_F32, [8], bytes(32))]
    _expect_open(_patched(tmp_path, lambda b: None, tensors=dup_t), inv)
    dup_k = [("k", G.U32, 1), ("k", G.U32, 2)]
    _expect_open(_patched(tmp_path, lambda b: None, kv=dup_k), inv)
    _expect_open(_patched(tmp_path, lambda b: None, kv=[("general.alignment", G.U32, 48)]), inv)
    _expect_open(_patched(tmp_path, lambda b: None, kv=[("general.alignment", G.U64, 64)]), inv)

    def bad_bool(b):
        b[_find(b, b"flag") + 4 + 4] = 2
    _expect_open(_patched(tmp_path, bad_bool, kv=[("flag", G.BOOL, True)]), inv)

    def nested_array(b):
        i = _find(b, b"arr") + 3 + 4  # past the key and the value type
        b[i:i + 4] = struct.pack("<I", G.ARRAY)
    _expect_open(_patched(tmp_path, nested_array, kv=[("arr", G.ARRAY, (G.U32, [1, 2]))]), inv)
    _expect_open(tmp_path / "does-not-exist.gguf", inv)
    _expect_open(tmp_path, inv)  # a directory


def test_load_rejects_without_touching_the_device(tmp_path):
    """Argument checks of shp_gguf_load_tensor happen before any HIP call."""
    import ctypes
    p = tmp_path / "k.gguf"
    G.write(p, [], [("q", 12, [256, 2], bytes(288)), ("t", G.GGML_F32, [8], bytes(32))])  # Q4_K: not loadable
    L = S.load()
    with S.GgufFile(p) as f:
        d = S.ShpTensor()
        assert f.info("q")[0].type == 12
        fake = ctypes.c_void_p(0x10000)
        assert L.shp_gguf_load_tensor(f._h, b"q", fake, 1 << 20, ctypes.byref(d), None) == S.ERR_UNSUPPORTED
        assert L.shp_gguf_load_tensor(f._h, b"t", fake, 31, ctypes.byref(d), None) == S.ERR_INVALID_ARG
        assert L.shp_gguf_load_tensor(f._h, b"nope", fake, 64, ctypes.byref(d), None) == S.ERR_INVALID_ARG
        assert L.shp_gguf_load_tensor(f._h, b"t", None, 64, ctypes.byref(d), None) == S.ERR_INVALID_ARG

        # The list form checks every entry before it reads or copies anything.
        def many(names, dsts, caps):
            n = len(names)
            descs = (S.ShpTensor * max(n, 1))()
            return L.shp_gguf_load_tensors(f._h, (ctypes.c_char_p * max(n, 1))(*names), n,
                                           (ctypes.c_void_p * max(n, 1))(*dsts),
                                           (ctypes.c_size_t * max(n, 1))(*caps), descs, None)
        assert many([b"t", b"q"], [0x10000, 0x20000], [64, 1 << 20]) == S.ERR_UNSUPPORTED
        assert many([b"t", b"t"], [0x10000, 0x20000], [64, 31]) == S.ERR_INVALID_ARG
        assert many([b"t", b"nope"], [0x10000, 0x20000], [64, 64]) == S.ERR_INVALID_ARG
        assert many([b"t", b"t"], [0x10000, None], [64, 64]) == S.ERR_INVALID_ARG
        assert many([b"t", None], [0x10000, 0x20000], [64, 64]) == S.ERR_INVALID_ARG
        assert many([], [], []) == S.OK
        assert L.shp_gguf_load_tensors(f._h, None, 1, None, None, None, None) == S.ERR_INVALID_ARG
        assert L.shp_gguf_load_tensors(None, None, 0, None, None, None, None) == S.ERR_INVALID_ARG
        assert L.shp_gguf_load_tensors(f._h, None, -1, None, None, None, None) == S.ERR_INVALID_ARG


def test_table_type_for_profile():
    assert S.table_type_for_profile("BF16") == S.TYPE_BF16
    assert S.table_type_for_profile("F16") == S.TYPE_F16
    assert S.table_type_for_profile("Q8_MIXED") == S.TYPE_Q8_0
    assert S.table_type_for_profile("Q5_K_MIXED") == S.TYPE_Q5_K
    with pytest.raises(S.ShpError) as e:
        S.table_type_for_profile("Q4_K")
    assert e.value.status == S.ERR_INVALID_ARG


FUZZ_SCRIPT = r"""
import random, sys, struct
sys.path[:0] = sys.argv[1:4]
import gguf_ref as G, synth_hip as S
path, out = sys.argv[4], sys.argv[5]
G.write(path, [("general.architecture", G.STRING, "qwen3-tts"), ("a", G.ARRAY, (G.STRING, ["x", "yy"])),
               ("b", G.U32, 7)],
        [("t", G.GGML_BF16, [64, 3], bytes(384)), ("q", G.GGML_Q8_0, [64, 2], bytes(136))])
base = open(path, "rb").read()
rng = random.Random(7)
seen = set()
for i in range(3000):
    b = bytearray(base)
    for _ in range(rng.randint(1, 4)):
        k = rng.randrange(min(len(b), 200))
        b[k] = rng.randrange(256)
    if rng.random() < 0.3:
        b = b[:rng.randrange(len(b))]
    open(out, "wb").write(bytes(b))
    try:
        with S.GgufFile(out) as f:
            for n in f.tensor_names():
                f.info(n)
        seen.add(0)
    except S.ShpError as e:
        seen.add(e.status)
print(sorted(seen))
"""


def test_mutated_headers_never_crash(tmp_path):
    """3000 random byte mutations and truncations of a small package: every one
    opens or is refused with a status; the process survives (run in a child so
    a memory error would fail this test instead of the session)."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    r = subprocess.run([sys.executable, "-c", FUZZ_SCRIPT, root, os.path.join(root, "synthesize.cpp_amd"),
                        os.path.join(root, "oracle"), str(tmp_path / "base.gguf"), str(tmp_path / "m.gguf")],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    seen = eval(r.stdout.strip().splitlines()[-1])
    assert S.ERR_INVALID_ARG in seen and 0 in seen


def test_package_writer_matches_the_restatement(tmp_path):
    """synthesize.cpp_amd/gguf_write.py (what tools and the benchmark cut
    packages with) writes the same bytes as the restatement's writer."""
    from gguf_write import write_gguf
    rng = np.random.default_rng(33)
    tensors = [t for t in _tables(rng) if t[1] in (G.GGML_BF16, G.GGML_Q8_0, G.GGML_F16, G.GGML_F32, G.GGML_I32)]
    strings = [("general.architecture", "qwen3-tts"), ("synthesize.quantization.profile", "Q8_MIXED")]
    for align in (32, 256):
        a, b = tmp_path / "a.gguf", tmp_path / "b.gguf"
        write_gguf(a, tensors, strings, alignment=align)
        G.write(b, [(k, G.STRING, v) for k, v in strings], tensors, alignment=align)
        assert a.read_bytes() == b.read_bytes()
    with pytest.raises(ValueError):
        write_gguf(tmp_path / "c.gguf", [("t", G.GGML_Q8_0, [32, 2], bytes(67))])

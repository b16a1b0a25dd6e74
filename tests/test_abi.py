"""The C ABI without a GPU: the library loads, exports every entry point the
header declares, and rejects malformed arguments before launching anything
(argument checks are host code; no device pointer is dereferenced)."""
import ctypes
import os
import re

import pytest

import synth_hip as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("synth_hip.h", "synth_gguf.h", "synth_graph.h")]


def declared_symbols():
    text = "".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(shp_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = S.load()
    names = declared_symbols()
    assert len(names) >= 30
    for name in names:
        assert hasattr(lib, name), name


def test_headers_compile_and_link_from_plain_c(tmp_path):
    """The headers are plain C11 (a C caller, such as a ggml backend module
    written in C, includes them with -pedantic and no warning), and a C
    program links libsynth_hip.so and gets statuses back through it."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "consumer.c"
    src.write_text(
        '#include "synth_hip.h"\n#include "synth_graph.h"\n#include "synth_gguf.h"\n#include <stdio.h>\n'
        "int main(void) {\n"
        "    shp_tensor y = {0};\n"
        '    printf("%u %s\\n", shp_abi_version(), shp_status_string(SHP_ERR_INVALID_ARG));\n'
        "    return shp_rms_norm_mul(NULL, NULL, 1e-6f, &y, NULL) == SHP_ERR_INVALID_ARG ? 0 : 1;\n"
        "}\n")
    # A sanitizer build (make asan) needs clang's sanitizer runtime at link
    # time, which a plain gcc link does not bring: the program links the
    # product library then.
    lib_path = S.LIB_PATH
    if "_asan" in os.path.basename(lib_path):
        lib_path = os.path.join(ROOT, "synthesize.cpp_amd", "libsynth_hip.so")
    lib_dir = os.path.dirname(lib_path)
    exe = tmp_path / "consumer"
    build = subprocess.run([cc, "-std=c11", "-Wall", "-Wextra", "-pedantic", "-Werror", "-I", os.path.join(ROOT, "include"),
                            str(src), "-L" + lib_dir, "-l:" + os.path.basename(lib_path), "-Wl,-rpath," + lib_dir,
                            "-o", str(exe)], capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, run.stderr
    assert run.stdout.split()[0] == str(S.load().shp_abi_version())


def test_abi_version_and_status_strings():
    assert S.abi_version() == 1
    assert S.status_string(S.OK) == "ok"
    assert "invalid" in S.status_string(S.ERR_INVALID_ARG)
    assert "unsupported" in S.status_string(S.ERR_UNSUPPORTED)
    assert "HIP" in S.status_string(S.ERR_BACKEND)


FAKE = 0x10000  # never dereferenced: every call below fails validation first


def mk(type_, ne, nb=None, data=FAKE):
    t = S.ShpTensor()
    t.type = type_
    size = {S.TYPE_F32: 4, S.TYPE_I32: 4, S.TYPE_F16: 2, S.TYPE_BF16: 2, S.TYPE_Q8_0: 34}[type_]
    ne = list(ne) + [1] * (4 - len(ne))
    if nb is None:
        nb = [size]
        row = size * (ne[0] // 32 if type_ == S.TYPE_Q8_0 else ne[0])
        nb.append(row)
        nb.append(row * ne[1])
        nb.append(row * ne[1] * ne[2])
    for k in range(4):
        t.ne[k], t.nb[k] = ne[k], nb[k]
    t.data = data
    return t


def R(x):
    return ctypes.byref(x) if x is not None else None


def test_argument_validation():
    L = S.load()
    x = mk(S.TYPE_F32, [1024, 8])
    y = mk(S.TYPE_F32, [1024, 8])
    w = mk(S.TYPE_F32, [1024])
    bad_w = mk(S.TYPE_F32, [512])
    assert L.shp_rms_norm_mul(None, R(w), 1e-6, R(y), None) == S.ERR_INVALID_ARG
    assert L.shp_rms_norm_mul(R(x), R(w), 1e-6, R(mk(S.TYPE_F32, [1024, 7])), None) == S.ERR_INVALID_ARG
    assert L.shp_rms_norm_mul(R(x), R(bad_w), 1e-6, R(y), None) == S.ERR_UNSUPPORTED
    assert L.shp_rms_norm_mul(R(mk(S.TYPE_F16, [1024, 8])), R(w), 1e-6, R(y), None) == S.ERR_UNSUPPORTED
    assert L.shp_rms_norm_mul(R(mk(S.TYPE_F32, [1024, 8], data=0)), R(w), 1e-6, R(y), None) == S.ERR_INVALID_ARG
    assert L.shp_add_rms_norm_mul(R(x), None, R(w), 1e-6, None, R(y), None) == S.ERR_INVALID_ARG
    xt = mk(S.TYPE_F32, [1024, 8])
    xt.nb[0] = 8  # non-contiguous rows
    assert L.shp_rms_norm_mul(R(xt), R(w), 1e-6, R(y), None) == S.ERR_INVALID_ARG
    xr = mk(S.TYPE_F32, [1024, 8])
    xr.reserved = 1
    assert L.shp_rms_norm_mul(R(xr), R(w), 1e-6, R(y), None) == S.ERR_INVALID_ARG

    q = mk(S.TYPE_F32, [128, 16, 5])
    k = mk(S.TYPE_F32, [128, 8, 5])
    pos = mk(S.TYPE_I32, [5])
    assert L.shp_rope_ext(R(q), R(pos), 128, 0, 1e6, 1, 0, 1, R(q), None) == S.ERR_UNSUPPORTED  # normal mode
    assert L.shp_rope_ext(R(q), R(pos), 128, 2, 1e6, 1, 0.5, 1, R(q), None) == S.ERR_UNSUPPORTED  # yarn
    assert L.shp_rope_ext(R(q), R(mk(S.TYPE_I32, [4])), 128, 2, 1e6, 1, 0, 1, R(q), None) == S.ERR_INVALID_ARG
    assert L.shp_rope_ext(R(q), R(pos), 130, 2, 1e6, 1, 0, 1, R(q), None) == S.ERR_INVALID_ARG
    assert L.shp_rope_ext(R(q), R(pos), 127, 2, 1e6, 1, 0, 1, R(q), None) == S.ERR_INVALID_ARG
    wq = mk(S.TYPE_BF16, [128])
    wk = mk(S.TYPE_F32, [128])
    assert L.shp_qk_norm_rope(R(q), R(k), R(wq), R(wk), 1e-6, R(pos), 128, 1e6, 1, R(q), R(k), None) == \
        S.ERR_UNSUPPORTED  # mixed gain types
    assert L.shp_qk_norm_rope(R(q), R(k), R(wq), None, 1e-6, R(pos), 128, 1e6, 1, R(q), R(k), None) == \
        S.ERR_INVALID_ARG
    assert L.shp_qk_norm_rope(R(q), R(k), R(wq), R(wq), 1e-6, R(pos), 128, 1e6, 1, R(q), None, None) == \
        S.ERR_INVALID_ARG

    tab = mk(S.TYPE_Q8_0, [1024, 100])
    ids = mk(S.TYPE_I32, [7])
    out = mk(S.TYPE_F32, [1024, 7])
    assert L.shp_get_rows(R(tab), R(mk(S.TYPE_F32, [7])), R(out), None) == S.ERR_INVALID_ARG
    assert L.shp_get_rows(R(tab), R(ids), R(mk(S.TYPE_F32, [1024, 6])), None) == S.ERR_INVALID_ARG
    assert L.shp_get_rows(R(tab), R(ids), R(mk(S.TYPE_F16, [1024, 7])), None) == S.ERR_UNSUPPORTED
    odd = mk(S.TYPE_Q8_0, [1024, 100])
    odd.ne[0] = 1000  # not whole blocks
    assert L.shp_get_rows(R(odd), R(ids), R(out), None) == S.ERR_INVALID_ARG
    tabs = (S.ShpTensor * 2)(mk(S.TYPE_Q8_0, [1024, 100]), mk(S.TYPE_BF16, [1024, 100]))
    codes = mk(S.TYPE_I32, [7, 2])
    assert L.shp_get_rows_sum(tabs, 2, R(codes), R(out), None) == S.ERR_UNSUPPORTED  # mixed table types
    assert L.shp_get_rows_sum(tabs, 0, R(codes), R(out), None) == S.ERR_INVALID_ARG
    assert L.shp_get_rows_sum(tabs, 65, R(codes), R(out), None) == S.ERR_INVALID_ARG
    assert L.shp_get_rows_sum(tabs, 1, R(codes), R(out), None) == S.ERR_INVALID_ARG  # codes has 2 groups

    a = mk(S.TYPE_F32, [256, 4])
    assert L.shp_snake(R(a), R(mk(S.TYPE_F32, [255])), R(a), None) == S.ERR_INVALID_ARG
    assert L.shp_add_leaky_relu(R(a), None, 0.1, R(a), R(a), None) == S.ERR_INVALID_ARG
    assert L.shp_add(R(a), R(mk(S.TYPE_F32, [256, 3])), R(a), None) == S.ERR_INVALID_ARG
    assert L.shp_glu_swiglu(R(a), 0, R(a), None) == S.ERR_INVALID_ARG
    assert L.shp_swiglu(R(a), R(mk(S.TYPE_F32, [256, 5])), R(a), None) == S.ERR_INVALID_ARG

    c = mk(S.TYPE_F32, [256])
    assert L.shp_snake_guarded(R(a), R(mk(S.TYPE_F32, [128])), R(a), None) == S.ERR_INVALID_ARG
    assert L.shp_snake_guarded(R(a), R(mk(S.TYPE_F16, [256])), R(a), None) == S.ERR_UNSUPPORTED
    assert L.shp_snake_beta(R(a), R(c), None, R(a), None) == S.ERR_INVALID_ARG
    assert L.shp_snake_beta(R(a), R(c), R(mk(S.TYPE_F32, [255])), R(a), None) == S.ERR_INVALID_ARG
    assert L.shp_snake_beta(R(a), R(c), R(mk(S.TYPE_F32, [256, 2])), R(a), None) == S.ERR_INVALID_ARG
    assert L.shp_exp(R(a), R(mk(S.TYPE_F32, [256, 5])), None) == S.ERR_INVALID_ARG
    assert L.shp_scale_bias(R(mk(S.TYPE_F16, [256, 4])), 1.0, 0.0, R(a), None) == S.ERR_UNSUPPORTED
    terms = (S.ShpTensor * 3)(mk(S.TYPE_F32, [256, 4]), mk(S.TYPE_F32, [256, 4]), mk(S.TYPE_F32, [256, 3]))
    assert L.shp_sum_scale_leaky_relu(terms, 3, 1 / 3, 0.1, None, R(a), None) == S.ERR_INVALID_ARG  # shape
    assert L.shp_sum_scale_leaky_relu(terms, 2, 0.5, 0.1, R(mk(S.TYPE_F32, [256, 5])), R(a), None) == \
        S.ERR_INVALID_ARG
    assert L.shp_sum_scale_leaky_relu(terms, 0, 1.0, 0.1, None, R(a), None) == S.ERR_INVALID_ARG
    assert L.shp_sum_scale_leaky_relu(terms, 9, 1.0, 0.1, None, R(a), None) == S.ERR_INVALID_ARG
    assert L.shp_sum_scale_leaky_relu(None, 1, 1.0, 0.1, None, R(a), None) == S.ERR_INVALID_ARG
    kc = mk(S.TYPE_F32, [128, 8, 64])
    v = mk(S.TYPE_F32, [128, 8, 5])
    args = lambda filled, cache=kc, vv=v: (R(q), R(k), R(vv), R(wk), R(wk), 1e-6, R(pos), 128, 1e6, 1.0, R(q),
                                           R(cache), R(kc), filled, None)
    assert L.shp_qk_norm_rope_kv(*args(60)) == S.ERR_INVALID_ARG  # 60 + 5 rows > capacity 64
    assert L.shp_qk_norm_rope_kv(*args(-1)) == S.ERR_INVALID_ARG
    assert L.shp_qk_norm_rope_kv(*args(0, cache=mk(S.TYPE_F32, [128, 4, 64]))) == S.ERR_INVALID_ARG  # kv heads
    assert L.shp_qk_norm_rope_kv(*args(0, vv=mk(S.TYPE_F32, [128, 8, 4]))) == S.ERR_INVALID_ARG  # v shape
    assert L.shp_qk_norm_rope_kv(*args(0, cache=mk(S.TYPE_F16, [128, 8, 64]))) == S.ERR_INVALID_ARG  # cache type
    slot, st = mk(S.TYPE_I32, [1]), mk(S.TYPE_I32, [1])
    at = lambda cache=kc, sl=slot, stt=st: (R(q), R(k), R(v), R(wk), R(wk), 1e-6, R(pos), 128, 1e6, 1.0, R(q),
                                             R(cache), R(kc), R(sl), R(stt), None)
    assert L.shp_qk_norm_rope_kv_at(*at(sl=mk(S.TYPE_F32, [1]))) == S.ERR_INVALID_ARG  # slot type
    assert L.shp_qk_norm_rope_kv_at(*at(sl=mk(S.TYPE_I32, [2]))) == S.ERR_INVALID_ARG  # one element
    assert L.shp_qk_norm_rope_kv_at(*at(stt=mk(S.TYPE_F32, [1]))) == S.ERR_INVALID_ARG  # status type
    assert L.shp_qk_norm_rope_kv_at(*at(cache=mk(S.TYPE_F32, [128, 8, 4]))) == S.ERR_INVALID_ARG  # < T rows
    assert L.shp_qk_norm_rope_kv_at(R(q), R(k), R(v), R(wk), R(wk), 1e-6, R(pos), 128, 1e6, 1.0, R(q), R(kc), R(kc),
                                    None, None, None) == S.ERR_INVALID_ARG  # no slot
    sc = mk(S.TYPE_F32, [37, 1, 16])
    assert L.shp_soft_max_ext(R(sc), None, 0.1, 0.5, R(sc), None) == S.ERR_UNSUPPORTED  # ALiBi
    assert L.shp_soft_max_ext(R(sc), R(mk(S.TYPE_F32, [36, 1])), 0.1, 0.0, R(sc), None) == S.ERR_INVALID_ARG
    assert L.shp_soft_max_ext(R(sc), R(mk(S.TYPE_F32, [37, 1, 3])), 0.1, 0.0, R(sc), None) == S.ERR_INVALID_ARG
    assert L.shp_soft_max_ext(R(sc), R(mk(S.TYPE_F16, [37, 1])), 0.1, 0.0, R(sc), None) == S.ERR_UNSUPPORTED
    assert L.shp_soft_max_ext(R(sc), None, 0.1, 0.0, R(mk(S.TYPE_F32, [37, 2, 16])), None) == S.ERR_INVALID_ARG
    strided = (S.ShpTensor * 1)(mk(S.TYPE_F32, [256, 4], nb=[4, 2048, 8192, 8192]))
    assert L.shp_sum_scale_leaky_relu(strided, 1, 1.0, 0.1, None, R(a), None) == S.ERR_UNSUPPORTED


def test_index_tensors_must_be_four_byte_aligned():
    """ids, positions, the cache slot and the status word are read with
    scalar loads where wave-uniform, which need 4-byte aligned addresses: a
    misaligned index tensor is UNSUPPORTED (ggml keeps the node), before any
    launch (no GPU here)."""
    L = S.load()
    odd = FAKE + 2
    tab = mk(S.TYPE_Q8_0, [1024, 100])
    out = mk(S.TYPE_F32, [1024, 7])
    assert L.shp_get_rows(R(tab), R(mk(S.TYPE_I32, [7], data=odd)), R(out), None) == S.ERR_UNSUPPORTED
    ids_nb = mk(S.TYPE_I32, [7, 2], nb=[4, 30, 60, 60])  # a row stride that is not a multiple of 4
    tab2 = mk(S.TYPE_Q8_0, [1024, 100, 2])
    assert L.shp_get_rows(R(tab2), R(ids_nb), R(mk(S.TYPE_F32, [1024, 7, 2])), None) == S.ERR_UNSUPPORTED
    tabs = (S.ShpTensor * 2)(mk(S.TYPE_Q8_0, [1024, 100]), mk(S.TYPE_Q8_0, [1024, 100]))
    assert L.shp_get_rows_sum(tabs, 2, R(mk(S.TYPE_I32, [7, 2], data=odd)), R(out), None) == S.ERR_UNSUPPORTED
    q = mk(S.TYPE_F32, [128, 16, 5])
    k = mk(S.TYPE_F32, [128, 8, 5])
    pos = mk(S.TYPE_I32, [5], data=odd)
    assert L.shp_rope_ext(R(q), R(pos), 128, 2, 1e6, 1, 0, 1, R(q), None) == S.ERR_UNSUPPORTED
    w = mk(S.TYPE_F32, [128])
    assert L.shp_qk_norm_rope(R(q), R(k), R(w), R(w), 1e-6, R(pos), 128, 1e6, 1, R(q), R(k), None) == \
        S.ERR_UNSUPPORTED
    kc = mk(S.TYPE_F32, [128, 8, 64])
    v = mk(S.TYPE_F32, [128, 8, 5])
    good_pos, i1 = mk(S.TYPE_I32, [5]), mk(S.TYPE_I32, [1])
    at = lambda sl, stt: L.shp_qk_norm_rope_kv_at(R(q), R(k), R(v), R(w), R(w), 1e-6, R(good_pos), 128, 1e6, 1.0,
                                                  R(q), R(kc), R(kc), R(sl), R(stt) if stt is not None else None, None)
    assert at(mk(S.TYPE_I32, [1], data=odd), i1) == S.ERR_UNSUPPORTED  # slot
    assert at(i1, mk(S.TYPE_I32, [1], data=odd)) == S.ERR_UNSUPPORTED  # status word


def test_zero_extents_are_rejected_before_any_launch():
    """A tensor with a zero extent (no rows, no ids, no positions) is
    INVALID_ARG at the entry points, with nothing launched (no GPU here)."""
    L = S.load()
    w = mk(S.TYPE_F32, [1024])
    empty = mk(S.TYPE_F32, [1024, 0])
    assert L.shp_rms_norm_mul(R(empty), R(w), 1e-6, R(empty), None) == S.ERR_INVALID_ARG
    assert L.shp_add_rms_norm_mul(R(empty), R(empty), R(w), 1e-6, None, R(empty), None) == S.ERR_INVALID_ARG
    assert L.shp_swiglu(R(empty), R(empty), R(empty), None) == S.ERR_INVALID_ARG
    assert L.shp_add(R(empty), R(empty), R(empty), None) == S.ERR_INVALID_ARG
    tab = mk(S.TYPE_Q8_0, [1024, 100])
    assert L.shp_get_rows(R(tab), R(mk(S.TYPE_I32, [0])), R(empty), None) == S.ERR_INVALID_ARG
    q0, k0 = mk(S.TYPE_F32, [128, 16, 0]), mk(S.TYPE_F32, [128, 8, 0])
    wq = mk(S.TYPE_F32, [128])
    assert L.shp_qk_norm_rope(R(q0), R(k0), R(wq), R(wq), 1e-6, R(mk(S.TYPE_I32, [0])), 128, 1e6, 1, R(q0), R(k0),
                              None) == S.ERR_INVALID_ARG
    c = mk(S.TYPE_F32, [256])
    e2 = mk(S.TYPE_F32, [256, 0])
    assert L.shp_snake(R(e2), R(c), R(e2), None) == S.ERR_INVALID_ARG
    assert L.shp_add_leaky_relu(R(e2), R(e2), 0.1, None, R(e2), None) == S.ERR_INVALID_ARG


def test_binding_fails_loudly_without_library(tmp_path):
    with pytest.raises(RuntimeError):
        import importlib
        mod = importlib.reload(S)
        mod._lib = None
        mod.load(str(tmp_path / "missing.so"))
    import importlib
    importlib.reload(S)


def layer_step(**over):
    """A well-formed step of 5 positions (hidden 256, 4+2 heads of 64, ffn 512)
    with fake pointers; keyword arguments replace a field."""
    t = 5
    f = dict(x=mk(S.TYPE_F32, [256, t]), w_in=mk(S.TYPE_BF16, [256]), normed=mk(S.TYPE_F32, [256, t]),
             q=mk(S.TYPE_F32, [64, 4, t]), k=mk(S.TYPE_F32, [64, 2, t]), wq=mk(S.TYPE_BF16, [64]),
             wk=mk(S.TYPE_BF16, [64]), pos=mk(S.TYPE_I32, [t]), q_out=mk(S.TYPE_F32, [64, 4, t]),
             k_out=mk(S.TYPE_F32, [64, 2, t]), attn_out=mk(S.TYPE_F32, [256, t]), w_post=mk(S.TYPE_BF16, [256]),
             resid=mk(S.TYPE_F32, [256, t]), mlp_in=mk(S.TYPE_F32, [256, t]), gate=mk(S.TYPE_F32, [512, t]),
             up=mk(S.TYPE_F32, [512, t]), act=mk(S.TYPE_F32, [512, t]), mlp_out=mk(S.TYPE_F32, [256, t]),
             out=mk(S.TYPE_F32, [256, t]))
    scal = dict(eps=1e-6, freq_base=1e6, n_dims=64, reserved=0)
    for key, val in over.items():
        (scal if key in scal else f)[key] = val
    step = S.ShpLayerStep()
    for key, val in f.items():
        setattr(step, key, ctypes.pointer(val) if val is not None else None)
    for key, val in scal.items():
        setattr(step, key, val)
    step._keep = f
    return step


LAYER_TENSORS = ("x", "w_in", "normed", "q", "k", "wq", "wk", "pos", "q_out", "k_out", "attn_out", "w_post",
                 "resid", "mlp_in", "gate", "up", "act", "mlp_out", "out")


def test_layer_step_rejects_a_malformed_step_before_any_launch():
    """Every tensor of the step is checked before the first of its five
    launches: each case below changes one field of a well-formed step."""
    L = S.load()
    call = lambda **over: L.shp_layer_nongemm_step(ctypes.byref(layer_step(**over)), None)
    assert L.shp_layer_nongemm_step(None, None) == S.ERR_INVALID_ARG
    assert call(reserved=1) == S.ERR_INVALID_ARG
    for name in LAYER_TENSORS:
        assert call(**{name: None}) == S.ERR_INVALID_ARG, name
    # one wrong extent per tensor, in the last (position) dimension or the row
    for name in ("normed", "attn_out", "resid", "mlp_in", "mlp_out", "out"):
        assert call(**{name: mk(S.TYPE_F32, [256, 4])}) == S.ERR_INVALID_ARG, name
        assert call(**{name: mk(S.TYPE_F32, [252, 5])}) == S.ERR_INVALID_ARG, name
    for name in ("up", "act"):
        assert call(**{name: mk(S.TYPE_F32, [512, 6])}) == S.ERR_INVALID_ARG, name
        assert call(**{name: mk(S.TYPE_F32, [508, 5])}) == S.ERR_INVALID_ARG, name
    assert call(q_out=mk(S.TYPE_F32, [64, 2, 5])) == S.ERR_INVALID_ARG
    assert call(k_out=mk(S.TYPE_F32, [64, 4, 5])) == S.ERR_INVALID_ARG
    assert call(k=mk(S.TYPE_F32, [32, 2, 5])) == S.ERR_INVALID_ARG  # head_dim differs from q's
    assert call(q=mk(S.TYPE_F32, [64, 4, 4])) == S.ERR_INVALID_ARG  # positions differ from x's
    assert call(x=mk(S.TYPE_F32, [256, 5, 2])) == S.ERR_INVALID_ARG  # a 3-d hidden state
    assert call(out=mk(S.TYPE_F16, [256, 5])) == S.ERR_INVALID_ARG
    assert call(pos=mk(S.TYPE_I32, [4])) == S.ERR_INVALID_ARG
    assert call(pos=mk(S.TYPE_F32, [5])) == S.ERR_INVALID_ARG
    assert call(w_in=mk(S.TYPE_BF16, [255])) == S.ERR_INVALID_ARG
    assert call(w_post=mk(S.TYPE_Q8_0, [256])) == S.ERR_INVALID_ARG
    assert call(wq=mk(S.TYPE_BF16, [32])) == S.ERR_INVALID_ARG
    assert call(wk=mk(S.TYPE_F32, [64])) == S.ERR_UNSUPPORTED  # q and k gains of two types
    assert call(n_dims=63) == S.ERR_INVALID_ARG
    assert call(n_dims=66) == S.ERR_INVALID_ARG
    assert call(n_dims=0) == S.ERR_INVALID_ARG
    assert call(eps=-1e-6) == S.ERR_INVALID_ARG
    assert call(eps=float("nan")) == S.ERR_INVALID_ARG
    bad_nb = mk(S.TYPE_F32, [256, 5])
    bad_nb.nb[0] = 8
    assert call(resid=bad_nb) == S.ERR_INVALID_ARG
    assert call(pos=mk(S.TYPE_I32, [5], data=FAKE + 2)) == S.ERR_UNSUPPORTED  # positions read by scalar loads

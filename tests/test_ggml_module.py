"""libggml-hip-synth.so, the ggml backend-module face of the library, found the
way synthesize.cpp finds backend modules. No GPU: the module reads the KFD
topology from sysfs, and these tests point it at topology trees laid out like
/sys/class/kfd/kfd/topology (SHP_KFD_TOPOLOGY).

Without the pinned ggml's headers the module has no registry
(ggml_backend_init returns NULL), so its ggml_backend_score is 0: the
discovery passes it over for any working libggml-hip-*.so and for the bare
libggml-hip.so. The gfx950 detection a registry build would score with is
exported as shp_module_gfx950_score and checked here on its own.

The discovery below restates src/backend-module.cpp:
  module_score (:99-127): dlopen(path, RTLD_NOW | RTLD_LOCAL), dlsym
    "ggml_backend_score", call it (0 when the file does not load or has no
    such symbol), dlclose;
  load_best_module (:145-177): among the regular files of the directory whose
    name starts with "libggml-" + name + "-" and ends in ".so", keep the first
    with the highest score, which must be above 0; with none, fall back to
    "libggml-" + name + ".so" when that file exists.
"""
import _ctypes
import ctypes
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MODULE = os.path.join(ROOT, "synthesize.cpp_amd", "libggml-hip-synth.so")


def module_score(path, symbol="ggml_backend_score"):
    try:
        lib = ctypes.CDLL(str(path), mode=os.RTLD_NOW | os.RTLD_LOCAL)
    except OSError:
        return 0
    try:
        fn = getattr(lib, symbol, None)
        if fn is None:
            return 0
        fn.restype, fn.argtypes = ctypes.c_int, []
        return fn()
    finally:
        _ctypes.dlclose(lib._handle)


def load_best_module(directory, backend_name):
    """The file synthesize.cpp would hand to ggml_backend_load, or None."""
    prefix, best_score, best = "libggml-%s-" % backend_name, 0, None
    for entry in sorted(os.scandir(directory), key=lambda e: e.name):
        if entry.is_file() and entry.name.startswith(prefix) and os.path.splitext(entry.name)[1] == ".so":
            score = module_score(entry.path)
            if score > best_score:
                best_score, best = score, entry.path
    if best_score == 0:
        bare = os.path.join(directory, "libggml-%s.so" % backend_name)
        return bare if os.path.isfile(bare) else None
    return best


def topology(tmp_path, targets, name="topo"):
    """A KFD topology tree: node 0 a CPU, then one node per GPU target."""
    root = tmp_path / name
    for i, t in enumerate([0] + list(targets)):
        node = root / "nodes" / str(i)
        node.mkdir(parents=True)
        (node / "properties").write_text("cpu_cores_count %d\nsimd_count %d\ngfx_target_version %d\nmax_waves_per_simd 8\n"
                                         % (0 if t else 64, 1024 if t else 0, t))
    return str(root)


@pytest.fixture
def env(monkeypatch):
    for k in ("ROCR_VISIBLE_DEVICES", "HIP_VISIBLE_DEVICES"):
        monkeypatch.delenv(k, raising=False)
    return monkeypatch


def score_with(env, topo, **visible):
    """The gfx950 detection's score (what a registry build reports)."""
    env.setenv("SHP_KFD_TOPOLOGY", topo)
    for k, v in visible.items():
        env.setenv(k, v)
    return module_score(MODULE, "shp_module_gfx950_score")


def test_detection_is_nonzero_exactly_when_a_gfx950_is_visible(tmp_path, env):
    mi355x, mi300x = 90500, 90402
    assert score_with(env, topology(tmp_path, [mi355x], "one")) == 2
    assert score_with(env, topology(tmp_path, [mi355x] * 8, "eight")) == 9
    assert score_with(env, topology(tmp_path, [mi300x, mi300x], "gfx942")) == 0
    assert score_with(env, topology(tmp_path, [], "cpu_only")) == 0
    assert score_with(env, str(tmp_path / "missing")) == 0
    mixed = topology(tmp_path, [mi300x, mi355x], "mixed")
    assert score_with(env, mixed) == 2
    assert score_with(env, mixed, HIP_VISIBLE_DEVICES="0") == 0  # only the gfx942 left
    assert score_with(env, mixed, HIP_VISIBLE_DEVICES="1") == 2
    assert score_with(env, mixed, ROCR_VISIBLE_DEVICES="1", HIP_VISIBLE_DEVICES="0") == 2  # HIP indexes ROCR's list
    assert score_with(env, mixed, ROCR_VISIBLE_DEVICES="") == 0
    assert score_with(env, mixed, HIP_VISIBLE_DEVICES="-1") == 0
    env.delenv("ROCR_VISIBLE_DEVICES")
    assert score_with(env, mixed, HIP_VISIBLE_DEVICES="GPU-1234abcd") == 2  # UUIDs: no index filtering


def test_without_a_registry_the_module_scores_zero(tmp_path, env):
    """ggml_backend_init has no registry to return, so ggml_backend_score is 0
    even with gfx950s visible."""
    lib = ctypes.CDLL(MODULE, mode=os.RTLD_NOW | os.RTLD_LOCAL)
    try:
        lib.ggml_backend_init.restype = ctypes.c_void_p
        assert lib.ggml_backend_init() is None
    finally:
        _ctypes.dlclose(lib._handle)
    env.setenv("SHP_KFD_TOPOLOGY", topology(tmp_path, [90500] * 8))
    assert module_score(MODULE) == 0
    assert module_score(MODULE, "shp_module_gfx950_score") == 9


def _decoy(path, body):
    src = str(path) + ".c"
    with open(src, "w") as f:
        f.write(body)
    subprocess.run(["gcc", "-shared", "-fPIC", "-o", str(path), src], check=True)
    os.remove(src)


def test_discovery_keeps_the_working_hip_module(tmp_path, env):
    """Next to a working ggml HIP build -- a scored libggml-hip-*.so, or only
    the bare libggml-hip.so fallback -- this build is never the file handed to
    ggml_backend_load (src/backend-module.cpp:145-177)."""
    mods = tmp_path / "backends"
    mods.mkdir()
    shutil.copy(MODULE, mods / "libggml-hip-synth.so")
    _decoy(mods / "libggml-hip.so", "int ggml_backend_score(void) { return 0; }\n")  # the bare fallback name
    _decoy(mods / "libggml-hip-zero.so", "int ggml_backend_score(void) { return 0; }\n")
    _decoy(mods / "libggml-hip-nosym.so", "int unrelated(void) { return 7; }\n")
    _decoy(mods / "libggml-cuda-x.so", "int ggml_backend_score(void) { return 50; }\n")  # another backend
    shutil.copy(MODULE, mods / "libggml-hip-synth.so.bak")  # wrong extension
    (mods / "libggml-hip-broken.so").write_bytes(b"not an ELF file")  # fails to load: score 0
    env.setenv("SHP_KFD_TOPOLOGY", topology(tmp_path, [90500]))
    # a gfx950 is visible, yet the bare ggml HIP build is the one loaded
    assert load_best_module(mods, "hip") == str(mods / "libggml-hip.so")
    assert load_best_module(mods, "cuda") == str(mods / "libggml-cuda-x.so")
    # a scored ggml HIP module in the same directory is loaded
    _decoy(mods / "libggml-hip-gfx950.so", "int ggml_backend_score(void) { return 1; }\n")
    assert load_best_module(mods, "hip") == str(mods / "libggml-hip-gfx950.so")
    # with nothing else there, no hip module is loaded at all (the CPU path stays)
    for f in ("libggml-hip.so", "libggml-hip-gfx950.so"):
        os.remove(mods / f)
    assert load_best_module(mods, "hip") is None


@pytest.mark.gpu
def test_the_box_gpu_is_found(monkeypatch, tmp_path):
    """On an MI355X box the live topology (under the box's own visibility
    settings) holds a visible gfx950: the detection finds it, while the
    module itself still scores 0 and the discovery keeps a bare
    libggml-hip.so beside it."""
    monkeypatch.delenv("SHP_KFD_TOPOLOGY", raising=False)
    assert module_score(MODULE, "shp_module_gfx950_score") >= 2
    assert module_score(MODULE) == 0
    shutil.copy(MODULE, tmp_path / "libggml-hip-synth.so")
    _decoy(tmp_path / "libggml-hip.so", "int ggml_backend_score(void) { return 0; }\n")
    assert load_best_module(tmp_path, "hip") == str(tmp_path / "libggml-hip.so")

"""ggml_concat through shp_concat, bit-exact against the oracle's restatement:
the code predictor's prefill input (src/arch/qwen3-tts/model.cpp:1450) and
every dimension, with ragged extents and row-strided operands."""
import numpy as np
import pytest

import ggml_ref as R
from test_gpu_parity import _np, _t, assert_bitexact

pytestmark = pytest.mark.gpu
SEED = 20261204


@pytest.mark.parametrize("ashape,bshape,dim", [
    ((1, 1024), (1, 1024), 1),          # [1024, 1] + [1024, 1] -> [1024, 2]
    ((3, 37), (3, 29), 0),
    ((2, 5, 64), (2, 3, 64), 1),
    ((4, 2, 6, 33), (4, 3, 6, 33), 2),
    ((2, 3, 4, 5), (1, 3, 4, 5), 3),
    ((513, 300), (7, 300), 1),
])
def test_concat_matches_oracle(gpu, ashape, bshape, dim):
    rng = np.random.default_rng(SEED + sum(ashape) + dim)
    a = rng.standard_normal(ashape).astype(np.float32)
    b = rng.standard_normal(bshape).astype(np.float32)
    print("concat", ashape, bshape, dim, flush=True)
    y = gpu.concat(_t(gpu, a), _t(gpu, b), dim)
    assert_bitexact(_np(y), R.concat(a, b, dim))


def test_concat_of_views_and_in_a_node_list(gpu):
    """Row-strided operands (column slices of wider buffers), and the node in
    a list between a gather and a norm, as the code predictor's prefill has
    it (model.cpp:1449-1450, code-predictor.cpp:68)."""
    rng = np.random.default_rng(SEED + 5)
    wa = rng.standard_normal((6, 80)).astype(np.float32)
    wb = rng.standard_normal((6, 90)).astype(np.float32)
    ta, tb = _t(gpu, wa), _t(gpu, wb)
    y = gpu.concat(ta[:, 8:72], tb[:, 2:66], 1)
    assert_bitexact(_np(y), R.concat(wa[:, 8:72], wb[:, 2:66], 1))
    table = rng.standard_normal((50, 256)).astype(np.float32)
    hidden = rng.standard_normal((1, 256)).astype(np.float32)
    ids = np.array([17], dtype=np.int32)
    w = rng.normal(1, 0.1, 256).astype(np.float32)
    g = gpu.Graph()
    emb = g.get_rows(_t(gpu, table), _t(gpu, ids))
    both = g.concat(_t(gpu, hidden), emb, 1)
    out = g.mul(g.rms_norm(both, 1e-6), _t(gpu, w))
    assert [k for k, *_ in g.plan(out) if k != "nop"] == ["single", "single", "norm_mul"]
    g.compute(out)
    ref = R.run(lambda og: og.mul(og.rms_norm(R.concat(hidden, table[17:18], 1), 1e-6), w))
    np.testing.assert_allclose(_np(out.t), ref, rtol=1e-5, atol=1e-6)

"""CPU: known answers for the chain-stage oracle (``oracle/chain.py``)."""

import numpy as np

from oracle.chain import SLICE, SWIGLU, stage_input, stage_ref
from oracle.matvec import linear_ref

from _util import layer_np, table
from eptq_amd.synthetic import make_layer


def test_slice_is_identity():
    src = np.arange(32, dtype=np.float16) / 8
    assert np.array_equal(stage_input(src, 8, 16, SLICE), src[8:24].astype(np.float64))


def test_swiglu_known_answers():
    N = 8
    gate = np.array([0, 0, 0, 0, 20, 20, -20, 1], dtype=np.float16)
    up = np.array([1, -2, 3, 0, 1.5, -0.25, 7, 2], dtype=np.float16)
    x = stage_input(np.concatenate([gate, up]), 0, N, SWIGLU)
    assert np.all(x[:4] == 0)                                 # silu(0) = 0
    assert np.allclose(x[4:6], 20 * up[4:6].astype(np.float64), rtol=1e-3)   # silu(20) = 20 to fp32
    assert abs(x[6]) < 1e-6                                   # silu(-20) ~ 0
    assert abs(x[7] - 2 / (1 + np.exp(-1.0))) < 2e-3          # silu(1)·2, fp16-rounded


def test_rmsnorm_of_constant_vector_is_the_weight():
    src = np.full(64, 3.0, dtype=np.float16)
    w = (np.arange(64) % 7 - 3).astype(np.float16)
    x = stage_input(src, 0, 64, SLICE, norm_weight=w, eps=0.0)
    assert np.allclose(x, w.astype(np.float64), atol=1e-12)


def test_stage_ref_is_the_layers_side_by_side():
    tab = table("e8_d4", 1.75)
    ls = [layer_np(make_layer(o, 64, seed=o, percmask=0.02, bias=o == 16)) for o in (16, 24)]
    x = np.random.default_rng(0).standard_normal(64)
    y = stage_ref(x, ls, tab)
    want = np.concatenate([linear_ref(x[None], L["Q"], L["g"], L["h"], L["O"], tab, "e8_d4", L["bias"])[0]
                           for L in ls])
    assert y.shape == (40,) and np.array_equal(y, want)

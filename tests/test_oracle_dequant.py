"""Oracle dequantizer and fused-Linear reference on the CPU: known answers and
independent checks (no GPU).

* Known answers: with g = h = 1 and no S the weight is the fp16 table, block by
  block (rows 0..3 from codes[t, i], rows 4..7 from codes[t, j] for E8-D4); an
  index sweep over all 65,535 codes dumps the whole table through the decode.
* The vectorized restatement against the element-by-element brute force on
  tiny layers (with S_group, markers at the edges, fp16 subnormal outputs).
* The critical-block overwrite order is row-major (Q's mask.nonzero()).
* The fused-Linear references: fp32 reconstruct + matmul vs the float64 fused
  math, linearity, x = 0 gives the bias, g-scaling.
"""

from __future__ import annotations

import numpy as np
import pytest

from eptq_amd.synthetic import make_layer
from oracle.codebooks import e8_raw_points_shells, e8d4_raw_codes_heap, scale_table
from oracle.dequant import build_csr, dequantize_layer, dequantize_scalar
from oracle.matvec import fused_ref64, linear_ref, rel_l2


def _tab(kind, r=1.75):
    if kind == "e8_d4":
        return scale_table(e8d4_raw_codes_heap(), r).reshape(512, 4)
    return _E8[r] if r in _E8 else _E8.setdefault(r, scale_table(e8_raw_points_shells(), r))


_E8 = {}


def _np(qd):
    return (qd.Q.numpy(), qd.g.numpy(), qd.h.numpy(), qd.O.numpy(),
            None if qd.S_group is None else qd.S_group.numpy())


def test_known_answer_e8d4_unit_scales():
    tab = _tab("e8_d4")
    rng = np.random.default_rng(0)
    u = rng.integers(0, 65535, size=(3, 5))
    Q = (u - 32768).astype(np.int16)
    W = dequantize_layer(Q, np.ones(24, np.float16), np.ones(5, np.float16),
                         np.zeros((0, 8), np.float16), tab, "e8_d4")
    for m in range(3):
        for n in range(5):
            t, i, j = (u[m, n] >> 14) & 3, (u[m, n] >> 7) & 127, u[m, n] & 127
            want = np.concatenate([tab[t * 128 + i], tab[t * 128 + j]]).astype(np.float16)
            assert np.array_equal(W[8 * m:8 * m + 8, n], want)


def test_index_sweep_dumps_every_table_row():
    for kind in ("e8_d4", "e8_lattice"):
        tab = _tab(kind, 1.75 if kind == "e8_d4" else 1.6)
        u = np.arange(65535)
        Q = (u - 32768).astype(np.int16).reshape(1, -1)
        W = dequantize_layer(Q, np.ones(8, np.float16), np.ones(65535, np.float16),
                             np.zeros((0, 8), np.float16), tab, kind)
        if kind == "e8_lattice":
            assert np.array_equal(W.T, tab.astype(np.float16))
        else:
            t, i, j = (u >> 14) & 3, (u >> 7) & 127, u & 127
            want = np.concatenate([tab[t * 128 + i], tab[t * 128 + j]], axis=1).astype(np.float16)
            assert np.array_equal(W.T, want)


@pytest.mark.parametrize("kind", ["e8_d4", "e8_lattice"])
@pytest.mark.parametrize("qb", [None, 8, 16])
def test_vectorized_equals_bruteforce(kind, qb):
    qd = make_layer(32, 24, seed=7 + (qb or 0), percmask=0.08, qb_size=qb)
    Q, g, h, O, S = _np(qd)
    # markers in the first and last block of the layer
    Q = Q.copy()
    tab = _tab(kind, 1.75 if kind == "e8_d4" else 1.6)
    a = dequantize_layer(Q, g, h, O, tab, kind, S)
    b = dequantize_scalar(Q, g, h, O, tab, kind, S)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_edge_markers_and_row_major_overwrite_order():
    qd = make_layer(24, 16, seed=3, percmask=0.0)
    Q, g, h, _, _ = _np(qd)
    Q = Q.copy()
    pos = [(0, 0), (0, 15), (1, 3), (2, 0), (2, 15)]
    for m, n in pos:
        Q[m, n] = 32767
    O = (np.arange(len(pos) * 8, dtype=np.float32).reshape(-1, 8) + 1).astype(np.float16)
    W = dequantize_layer(Q, np.ones_like(g), np.ones_like(h), O, _tab("e8_d4"), "e8_d4")
    for k, (m, n) in enumerate(pos):   # k-th marker in row-major order gets O[k]
        assert np.array_equal(W[8 * m:8 * m + 8, n], O[k])
    cols, rp = build_csr(Q)
    assert cols.tolist() == [0, 15, 3, 0, 15] and rp.tolist() == [0, 2, 3, 5]


def test_subnormal_outputs_round_like_numpy():
    qd = make_layer(16, 32, seed=9, percmask=0.05)
    Q, g, h, O, _ = _np(qd)
    g = (g.astype(np.float32) * 1e-5).astype(np.float16)
    W = dequantize_layer(Q, g, h, O, _tab("e8_d4"), "e8_d4")
    assert (np.abs(W.astype(np.float32)) < 6.1e-5).mean() > 0.3
    b = dequantize_scalar(Q, g, h, O, _tab("e8_d4"), "e8_d4")
    assert np.array_equal(W.view(np.uint16), b.view(np.uint16))


@pytest.mark.parametrize("kind,qb,bias", [("e8_d4", None, True), ("e8_d4", 16, False),
                                          ("e8_lattice", None, False)])
def test_linear_references_agree(kind, qb, bias):
    qd = make_layer(64, 96, seed=21, percmask=0.02, qb_size=qb, bias=bias)
    Q, g, h, O, S = _np(qd)
    tab = _tab(kind, 1.75 if kind == "e8_d4" else 1.6)
    b = None if qd.bias is None else qd.bias.numpy()
    x = np.random.default_rng(1).standard_normal((3, 96)).astype(np.float16)
    y32 = linear_ref(x, Q, g, h, O, tab, kind, b, S)
    y64 = fused_ref64(x, Q, g, h, O, tab, kind, b, S)
    assert rel_l2(y32, y64) < 2e-3          # only the fp16 rounding of W differs
    # linearity and x = 0
    x2 = np.random.default_rng(2).standard_normal((3, 96)).astype(np.float16)
    ya = fused_ref64(x.astype(np.float32) + x2.astype(np.float32), Q, g, h, O, tab, kind, None, S)
    yb = fused_ref64(x, Q, g, h, O, tab, kind, None, S) + fused_ref64(x2, Q, g, h, O, tab, kind, None, S)
    assert np.allclose(ya, yb, rtol=1e-9, atol=1e-9)
    y0 = fused_ref64(np.zeros((2, 96), np.float16), Q, g, h, O, tab, kind, b, S)
    assert np.allclose(y0, 0.0 if b is None else np.broadcast_to(b.astype(np.float64), y0.shape))
    # g scales the outputs row by row
    g2 = (g.astype(np.float32) * 2).astype(np.float16)
    assert np.allclose(fused_ref64(x, Q, g2, h, O, tab, kind, None, S),
                       2 * fused_ref64(x, Q, g, h, O, tab, kind, None, S), rtol=1e-9)


def test_rel_l2():
    assert rel_l2(np.ones(4), np.ones(4)) == 0.0
    assert abs(rel_l2(np.array([1.0, 0.0]), np.array([2.0, 0.0])) - 0.5) < 1e-12

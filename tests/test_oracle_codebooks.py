"""Codebook tables: the oracle's restatements pinned against independent constructions.

CPU only.  Two constructions of each table (the reference's own procedure
restated in ``oracle.codebooks`` and the package's closed-form enumeration in
``eptq_amd.quantizers``) must agree bit for bit, and both must satisfy the
lattice facts that fix them independently of either: theta-series shell sizes,
coset sizes and membership, distinctness, sort order, the reserved marker slot.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from eptq_amd.quantizers import E8D4Quantizer, E8LatticeQuantizer
from eptq_amd.quantizers.e8_d4 import e8d4_raw_codes
from eptq_amd.quantizers.e8_lattice import e8_raw_points
from oracle.codebooks import e8_raw_points_shells, e8_roots, e8d4_raw_codes_heap, scale_table


@pytest.fixture(scope="module")
def d4_heap():
    return e8d4_raw_codes_heap()


@pytest.fixture(scope="module")
def e8_shells():
    return e8_raw_points_shells()


# ---------------------------------------------------------------- E8-D4 -----

def test_e8d4_heap_walk_equals_closed_form(d4_heap):
    closed = e8d4_raw_codes()
    assert d4_heap.shape == (4, 128, 4) and d4_heap.dtype == np.float32
    assert np.array_equal(d4_heap, closed)


def test_e8d4_coset_membership(d4_heap):
    # [even-int, even-half, odd-int, odd-half]: integrality and coordinate-sum parity
    for t in range(4):
        pts = d4_heap[t].astype(np.float64)
        integral = np.all(pts == np.round(pts), axis=1)
        half = np.all(np.abs(pts - np.round(pts)) == 0.5, axis=1)
        parity = np.round(pts.sum(axis=1)).astype(int) % 2
        assert (integral if t in (0, 2) else half).all()
        assert (parity == (0 if t < 2 else 1)).all()


def test_e8d4_sorted_by_norm_then_tuple_and_distinct(d4_heap):
    for t in range(4):
        keys = [(float((p * p).sum()), tuple(p.tolist())) for p in d4_heap[t]]
        assert keys == sorted(keys)
        assert len(set(k[1] for k in keys)) == 128
        assert max(k[0] for k in keys) <= 7.0


def test_e8d4_coset_truncation_counts(d4_heap):
    # Points of each coset with norm² <= 7 (counted by brute force): 145/152/152/152;
    # the kept 128 are every point below the last norm shell plus a prefix of it.
    grid = np.arange(-6, 7) / 2.0
    full = {0: [], 1: [], 2: [], 3: []}
    for p in np.array(np.meshgrid(grid, grid, grid, grid, indexing="ij")).reshape(4, -1).T:
        n2 = float((p * p).sum())
        integral = np.all(p == np.round(p))
        half = np.all(np.abs(p - np.round(p)) == 0.5)
        if n2 > 7 or not (integral or half):
            continue
        par = int(round(p.sum())) % 2
        full[2 * par + (0 if integral else 1)].append((n2, tuple(p.tolist())))
    assert [len(full[t]) for t in range(4)] == [145, 152, 152, 152]
    for t in range(4):
        want = [pt for _, pt in sorted(full[t])[:128]]
        assert [tuple(p.tolist()) for p in d4_heap[t]] == want


def test_e8d4_marker_slot_is_last_row(d4_heap):
    # u = 65535 decodes to (t, i, j) = (3, 127, 127): the last row of the odd-half coset.
    u = 65535
    assert ((u >> 14) & 3, (u >> 7) & 127, u & 127) == (3, 127, 127)
    assert tuple(d4_heap[3, 127].tolist()) == sorted((float((p * p).sum()), tuple(p.tolist()))
                                              for p in d4_heap[3])[-1][1]


def test_e8d4_quantizer_table_scaling():
    q = E8D4Quantizer(radius=1.75)
    raw = e8d4_raw_codes()
    assert np.array_equal(q.codes.numpy(), scale_table(raw, 1.75, "divide"))
    assert np.array_equal(q.flat_table().numpy(), scale_table(raw, 1.75).reshape(512, 4))
    q.set_radius(2.0)
    assert np.array_equal(q.codes.numpy(), raw / np.float32(2.0))


# ----------------------------------------------------------------- E8 -------

def test_e8_roots():
    r = e8_roots()
    assert r.shape == (240, 8)
    assert np.all((r * r).sum(axis=1) == 2.0)
    assert len({tuple(v) for v in r.tolist()}) == 240
    # every root is in E8: all-integer or all-half-integer with an even coordinate sum
    s = r.sum(axis=1)
    assert np.all(s == np.round(s)) and np.all(np.round(s).astype(int) % 2 == 0)


def _sigma3(k):
    return sum(d ** 3 for d in range(1, k + 1) if k % d == 0)


def test_e8_shell_expansion_equals_closed_form(e8_shells):
    closed = e8_raw_points()
    assert e8_shells.shape == (65535, 8) and closed.shape == (65535, 8)
    assert np.array_equal(e8_shells, closed)


def test_e8_shell_sizes_follow_theta_series(e8_shells):
    n2 = (e8_shells.astype(np.float64) ** 2).sum(axis=1)
    counts = [int((n2 == 2 * k).sum()) for k in range(7)]
    want = [1] + [240 * _sigma3(k) for k in range(1, 6)]
    assert counts[:6] == want == [1, 240, 2160, 6720, 17520, 30240]
    assert counts[6] == 65535 - sum(want) == 8654
    assert np.all(np.diff(n2) >= 0)           # shells in increasing norm


def test_e8_rows_lexicographic_within_shell_and_distinct(e8_shells):
    n2 = (e8_shells.astype(np.float64) ** 2).sum(axis=1)
    for k in range(7):
        sh = e8_shells[n2 == 2 * k]
        order = np.lexsort([sh[:, c] for c in range(7, -1, -1)])
        assert np.array_equal(order, np.arange(len(sh)))
    assert len(np.unique(e8_shells, axis=0)) == 65535


def test_e8_truncated_shell_is_prefix_of_full_norm12_shell(e8_shells):
    # Independent enumeration of the whole norm² = 12 shell (60480 = 240·σ₃(6)).
    vals_i = np.arange(-3, 4, dtype=np.int8) * 2
    vals_h = np.arange(-7, 8, 2, dtype=np.int8)
    vals_h = vals_h[np.abs(vals_h) <= 7]
    shell = []
    for vals in (vals_i, vals_h):
        grids = np.stack(np.meshgrid(*([vals] * 4), indexing="ij"), -1).reshape(-1, 4).astype(np.int32)
        sq = (grids ** 2).sum(1)
        for a in range(len(grids)):
            rest = 48 - sq[a]
            if rest < 0:
                continue
            sel = grids[sq == rest]
            if len(sel):
                v = np.concatenate([np.repeat(grids[a][None], len(sel), 0), sel], 1)
                shell.append(v[(v.sum(1) % 4) == 0])
    shell = np.concatenate(shell)
    assert len(shell) == 240 * _sigma3(6) == 60480
    order = np.lexsort([shell[:, c] for c in range(7, -1, -1)])
    first = shell[order][:8654].astype(np.float32) / 2.0
    n2 = (e8_shells.astype(np.float64) ** 2).sum(axis=1)
    assert np.array_equal(e8_shells[n2 == 12], first)


def test_e8_quantizer_table_scaling():
    q = E8LatticeQuantizer(radius=1.6)
    assert np.array_equal(q.flat_table().numpy(), scale_table(e8_raw_points(), 1.6))


def test_scale_modes_differ_only_by_rounding():
    raw = e8d4_raw_codes()
    a = scale_table(raw, 1.75, "divide")
    b = scale_table(raw, 1.75, "reciprocal")
    assert np.max(np.abs(a.astype(np.float64) - b.astype(np.float64))) <= np.spacing(np.float32(2.0))
    # torch on the CPU divides: the oracle's "divide" mode is its rounding.
    t = (torch.from_numpy(raw) / 1.75).numpy()
    assert np.array_equal(t, a)

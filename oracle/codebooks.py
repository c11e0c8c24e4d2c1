"""Oracle codebooks: the reference's own table procedures, restated on the CPU.

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import heapq
from itertools import combinations, product

import numpy as np

# quantizers/e8_d4.py:40-50 — the 24 unit vectors of the Hurwitz lattice.
_D4_STEPS = (
    [tuple(s if k == a else 0 for k in range(4)) for a in range(4) for s in (1, -1)]
    + [tuple(0.5 * (1 - 2 * ((m >> k) & 1)) for k in range(4)) for m in range(16)]
)


def e8d4_raw_codes_heap() -> np.ndarray:
    """Restates ``quantizers/e8_d4.py:50-86``: heap walk from the origin,
    points popped by (norm², tuple), filed by coordinate-sum parity and
    integrality, the first 128 of each coset kept, order [ef, eh, of, oh]."""
    heap = [(0, (0, 0, 0, 0))]
    seen = {(0, 0, 0, 0)}
    ef, eh, of, oh = [], [], [], []
    while True:
        d, top = heapq.heappop(heap)
        if d > 7:
            break
        integral = all((c * 2) % 2 == 0 for c in top)
        if sum(top) % 2 == 0:
            (ef if integral else eh).append(top)
        else:
            (of if integral else oh).append(top)
        for st in _D4_STEPS:
            nv = tuple(top[k] + st[k] for k in range(4))
            if nv not in seen:
                seen.add(nv)
                heapq.heappush(heap, (sum(c * c for c in nv), nv))
    return np.asarray([ef[:128], eh[:128], of[:128], oh[:128]], dtype=np.float32)


def e8_roots() -> np.ndarray:
    """Restates ``quantizers/e8_lattice.py:54-67``: 112 integer roots ±e_a±e_b
    and 128 half-integer roots with an even number of minus signs."""
    roots = []
    for a, b in combinations(range(8), 2):
        for s1, s2 in ((1, 1), (1, -1), (-1, 1), (-1, -1)):
            v = [0.0] * 8
            v[a], v[b] = float(s1), float(s2)
            roots.append(v)
    for signs in product([0.5, -0.5], repeat=7):
        v = list(signs) + [0.5]
        v[-1] -= sum(v) % 2   # Python float modulo, as torch.remainder
        roots.append(v)
    return np.asarray(roots, dtype=np.float32)


def e8_raw_points_shells() -> np.ndarray:
    """Restates ``quantizers/e8_lattice.py:69-81`` + ``remove_last``
    (``quantize.py:178-181``): six shell expansions with rows deduplicated in
    lexicographic order, concatenated, first 65,536 rows, last row dropped."""
    roots = e8_roots()
    shells = [np.zeros((1, 8), dtype=np.float32)]
    for i in range(6):
        cur = shells[-1]
        cand = (cur[:, None, :] + roots[None, :, :]).reshape(-1, 8)
        keep = (cand * cand).sum(axis=1) == 2 * (i + 1)
        shells.append(np.unique(cand[keep], axis=0))
    book = np.concatenate(shells, axis=0)[:65536]
    return book[:-1].copy()


def scale_table(raw: np.ndarray, radius: float, mode: str = "divide") -> np.ndarray:
    """``raw / radius`` in fp32 as torch evaluates it (``reconstruct.py:52-62``).

    ``mode="divide"``: CPU tensors, a true fp32 division by fp32(radius).
    ``mode="reciprocal"``: GPU tensors, where torch multiplies by the fp32
    reciprocal of a host scalar divisor.
    """
    raw = np.asarray(raw, dtype=np.float32)
    r = np.float32(radius)
    if mode == "divide":
        return (raw / r).astype(np.float32)
    if mode == "reciprocal":
        inv = np.float32(np.float32(1.0) / r)
        return (raw * inv).astype(np.float32)
    raise ValueError(mode)

"""E8-lattice codebook: 65,535 points of the first six E8 shells, decode side only.

The reference builds its table by shell expansion (``quantizers/e8_lattice.py:54-81``):
shell k+1 is ``{s + r : s in shell k, r in roots, |s + r|² = 2(k+1)}`` with rows
deduplicated and ordered by ``torch.unique(dim=0)`` (lexicographic), shells 0..6
concatenated, truncated to 65,536 rows, and the last row dropped by
``remove_last`` (``quantize.py:178-181``) so index 65535 can mark critical blocks.

Here the same table comes from direct enumeration: every E8 vector
(D8 ∪ D8+½, even coordinate sum) with norm² ≤ 12 is listed, grouped by norm²,
each group sorted lexicographically.  Shell sizes are 1, 240, 2160, 6720,
17520, 30240 (= 240·σ₃(k)) for norm² 0..10, so the table holds all of them
(56,881 points) plus the first 8,654 points of the norm²-12 shell.

Index decode (``quantizers/e8_lattice.py:111-122``): rows 8m..8m+7 of column n
are ``points[u]``.
"""

from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from .base import BaseQuantizer

CODEBOOK_ROWS = 65535
MAX_NORM2 = 12


def _doubled_vectors(values: np.ndarray, lim2: int) -> np.ndarray:
    """All 8-vectors over ``values`` (doubled coordinates) with sum of squares
    ≤ lim2, built one coordinate at a time with pruning."""
    vecs = np.zeros((1, 0), dtype=np.int8)
    n2 = np.zeros(1, dtype=np.int32)
    vsq = values.astype(np.int32) ** 2
    min_sq = int(vsq.min())
    for dim in range(8):
        remaining = 7 - dim
        new_n2 = n2[:, None] + vsq[None, :]
        ok = new_n2 + remaining * min_sq <= lim2
        rows, cols = np.nonzero(ok)
        vecs = np.concatenate([vecs[rows], values[cols, None].astype(np.int8)], axis=1)
        n2 = new_n2[rows, cols]
    return vecs


def e8_raw_points() -> np.ndarray:
    """Unscaled E8 table, float32 of shape (65535, 8) (closed form)."""
    lim2 = 4 * MAX_NORM2  # doubled coordinates: |2v|² = 4|v|²
    ints = np.arange(-6, 7, 2, dtype=np.int8)      # 2v for v in {-3..3}
    halves = np.arange(-5, 6, 2, dtype=np.int8)    # 2v for v in {±½, ±3/2, ±5/2}
    pts = np.concatenate([_doubled_vectors(ints, lim2), _doubled_vectors(halves, lim2)])
    s = pts.astype(np.int32).sum(axis=1)
    pts = pts[(s % 4) == 0]                       # coordinate sum s/2 must be even
    n2 = (pts.astype(np.int32) ** 2).sum(axis=1)
    # Primary key norm², then the coordinates lexicographically.
    keys = [pts[:, c] for c in range(7, -1, -1)] + [n2]
    order = np.lexsort(keys)
    table = pts[order][:CODEBOOK_ROWS + 1][:CODEBOOK_ROWS]
    return (table.astype(np.float32) / 2.0)


class E8LatticeQuantizer(BaseQuantizer):
    """Decode-side E8-lattice quantizer with the reference's table semantics.

    ``points`` is the fp32 (65535, 8) table divided by ``_radius``.
    """

    RAW_ATTR = "_raw_points"
    DEFAULT_RADIUS = 1.6

    def __init__(self, device: str = "cpu", codebook: Optional[torch.Tensor] = None,
                 radius: Optional[float] = None):
        if codebook is not None:
            # quantizers/e8_lattice.py:29-33
            self.points = codebook
            self._raw_points = None
            self._radius = self.DEFAULT_RADIUS
            return
        raw = torch.from_numpy(e8_raw_points()).to(device)
        self._raw_points = raw.clone()
        self._radius = radius if radius is not None else self.DEFAULT_RADIUS
        self.points = raw / self._radius

    def set_radius(self, new_radius: float) -> None:
        """quantizers/e8_lattice.py:41-52."""
        if self._raw_points is not None:
            self.points = self._raw_points / new_radius
        else:
            self.points *= (self._radius / new_radius)
        self._radius = new_radius

    def dequant(self, indices: torch.Tensor, scale) -> torch.Tensor:
        """quantizers/e8_lattice.py:111-122."""
        return self.points[indices.T.long()].reshape(indices.shape[1], -1).T * scale

    def flat_table(self) -> torch.Tensor:
        """The fp32 table as the kernels consume it: (65535, 8), contiguous."""
        return self.points.float().contiguous()

    def remove_last(self) -> None:
        """No-op: tables built here already exclude the reserved last row."""

"""E8-D4 codebook: four 128-point D4-coset tables, decode side only.

The table is defined by the reference's heap walk over the Hurwitz lattice
(``quantizers/e8_d4.py:40-77``): starting at the origin and stepping by the 24
unit-norm vectors, points are popped in increasing ``(norm², coordinates)``
order and filed into four cosets, keeping the first 128 of each.  Because every
non-zero lattice point has a neighbour strictly closer to the origin, that walk
pops points in exactly sorted ``(norm², tuple)`` order, so the same table is
built here directly: enumerate every point of Z⁴ ∪ (Z+½)⁴ with norm² ≤ 7, split
by (coordinate-sum parity, integer/half-integer), sort, truncate.

Coset order is the reference's ``[even-int, even-half, odd-int, odd-half]``
(``quantizers/e8_d4.py:80``).  Index packing (``quantizers/e8_d4.py:237-255``):
``t = (u >> 14) & 3``, ``i = (u >> 7) & 127``, ``j = u & 127``; rows 0..3 of an
8-row block come from ``codes[t, i]`` and rows 4..7 from ``codes[t, j]``.

The offline encoder (``quant``/``quant_block``) is not part of this package.
"""

from __future__ import annotations

from itertools import product
from typing import Optional

import numpy as np
import torch

from .base import BaseQuantizer

NORM2_LIMIT = 7
CODES_PER_COSET = 128


def e8d4_raw_codes() -> np.ndarray:
    """Unscaled E8-D4 table, float32 of shape (4, 128, 4) (closed form)."""
    # Work in doubled coordinates so every value is an integer: integer points
    # have even doubled coordinates, half-integer points odd ones.
    lim2 = 4 * NORM2_LIMIT
    even = [v for v in range(-6, 7) if v % 2 == 0]
    odd = [v for v in range(-5, 6) if v % 2 != 0]
    cosets = {0: [], 1: [], 2: [], 3: []}
    for vals, half in ((even, False), (odd, True)):
        for p in product(vals, repeat=4):
            n2 = sum(c * c for c in p)
            if n2 > lim2:
                continue
            parity = (sum(p) // 2) % 2          # coordinate sum is sum(p)/2
            t = 2 * parity + (1 if half else 0)  # ef=0, eh=1, of=2, oh=3
            cosets[t].append((n2, p))
    out = np.empty((4, CODES_PER_COSET, 4), dtype=np.float32)
    for t in range(4):
        pts = sorted(cosets[t])[:CODES_PER_COSET]
        if len(pts) < CODES_PER_COSET:
            raise RuntimeError("E8-D4 coset too small")
        out[t] = np.asarray([p for _, p in pts], dtype=np.float32) / 2.0
    return out


class E8D4Quantizer(BaseQuantizer):
    """Decode-side E8-D4 quantizer with the reference's table semantics.

    ``codes`` is the fp32 (4, 128, 4) table divided by ``_radius``;
    ``_raw_codes`` is the unscaled table when known (fresh tables and the
    ``raw_codes`` on-disk format), else ``None``.
    """

    RAW_ATTR = "_raw_codes"
    DEFAULT_RADIUS = 1.875

    def __init__(self, device: str = "cpu", codebook: Optional[torch.Tensor] = None,
                 radius: Optional[float] = None):
        if codebook is not None:
            # Matches quantizers/e8_d4.py:30-35: a pre-divided table whose
            # radius is unknown falls back to DEFAULT_RADIUS.
            self.codes = codebook
            self._raw_codes = None
            self._radius = self.DEFAULT_RADIUS
            return
        raw = torch.from_numpy(e8d4_raw_codes()).to(device)
        self._raw_codes = raw.clone()
        self._radius = radius if radius is not None else self.DEFAULT_RADIUS
        self.codes = raw / self._radius

    def set_radius(self, new_radius: float) -> None:
        """quantizers/e8_d4.py:90-102: exact ``raw / r`` when raw is known,
        else an in-place rescale by ``r_old / r_new``."""
        if self._raw_codes is not None:
            self.codes = self._raw_codes / new_radius
        else:
            self.codes *= (self._radius / new_radius)
        self._radius = new_radius

    def dequant(self, indices: torch.Tensor, scale) -> torch.Tensor:
        """quantizers/e8_d4.py:237-255: (M, N) indices -> (8M, N) weights."""
        t = (indices >> 14) & 0x03
        i = (indices >> 7) & 0x7F
        j = indices & 0x7F
        a1 = self.codes[t.T, i.T]
        a2 = self.codes[t.T, j.T]
        return torch.stack((a1, a2), dim=-2).reshape(j.shape[-1], -1).T * scale

    def warp_codebook(self, alpha: float) -> None:
        """quantizers/e8_d4.py:282-298: radial warp of the 4-D codes.

        Uses the same torch operations in the same order so that, on the same
        device, the warped table carries the reference's bits.
        """
        flat = self.codes.view(-1, 4)
        norms = flat.norm(dim=1)
        max_norm = norms.max()
        r_norm = norms / max_norm.clamp(min=1e-8)
        new_norms = r_norm.pow(alpha) * max_norm
        scale = torch.where(norms > 1e-8, new_norms / norms, torch.zeros_like(norms))
        self.codes = (flat * scale.unsqueeze(1)).view(4, 128, 4)
        self._warp_alpha = alpha
        self._warp_max_norm = max_norm.item()

    def flat_table(self) -> torch.Tensor:
        """The fp32 table as the kernels consume it: (512, 4), contiguous."""
        return self.codes.reshape(512, 4).float().contiguous()

    def remove_last(self) -> None:
        """No-op: index 65535 = (3, 127, 127) is reserved by the encoder."""

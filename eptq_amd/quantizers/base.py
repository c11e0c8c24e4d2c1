"""Minimal quantizer interface (decode side), mirroring ``quantizers/base.py:8-25``."""

from abc import ABC, abstractmethod

import torch


class BaseQuantizer(ABC):
    """A codebook that maps 16-bit indices to 8-row weight blocks."""

    # Attribute that holds the unscaled table (None when only a pre-divided
    # table is known); subclasses name theirs.
    RAW_ATTR = "_raw"

    @classmethod
    def from_raw(cls, raw: torch.Tensor, radius: float) -> "BaseQuantizer":
        """A quantizer whose table is ``raw / radius``, divided on ``raw``'s
        device, that keeps ``raw`` for later radius switches."""
        q = cls(device=str(raw.device), codebook=raw / radius)
        setattr(q, cls.RAW_ATTR, raw)
        q._radius = radius
        return q

    @abstractmethod
    def dequant(self, indices: torch.Tensor, scale) -> torch.Tensor:
        """(M, N) indices -> (8M, N) fp32 weights, times ``scale``."""

    @abstractmethod
    def set_radius(self, new_radius: float) -> None:
        """Make the table's divisor ``new_radius``."""

    @abstractmethod
    def flat_table(self) -> torch.Tensor:
        """fp32 table in the layout the HIP kernels read."""

    def remove_last(self) -> None:
        """Drop the last codebook entry (reserved as the critical-block marker)."""

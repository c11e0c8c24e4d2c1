"""Minimal quantizer interface (decode side), mirroring ``quantizers/base.py:8-25``."""

from abc import ABC, abstractmethod

import torch


class BaseQuantizer(ABC):
    """A codebook that maps 16-bit indices to 8-row weight blocks."""

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

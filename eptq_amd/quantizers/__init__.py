"""Codebooks (decode side): E8-lattice and E8-D4."""

from .base import BaseQuantizer
from .e8_d4 import E8D4Quantizer, e8d4_raw_codes
from .e8_lattice import E8LatticeQuantizer, e8_raw_points

__all__ = ["BaseQuantizer", "E8D4Quantizer", "E8LatticeQuantizer",
           "e8d4_raw_codes", "e8_raw_points"]

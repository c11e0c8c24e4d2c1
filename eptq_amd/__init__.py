"""EPTQ quantized-Linear inference on AMD Instinct MI355X (gfx950).

Public surface (drop-in for the reference's inference path):

* ``eptq_amd.kernels.patch.load_quantized_model`` — quantized HF model loader;
* ``eptq_amd.kernels.linear.EPTQLinear`` / ``QuantizedLinear``;
* ``torch.ops.eptq.e8_forward`` / ``e8d4_forward`` (+ grouped and dequant ops);
* ``eptq_amd.config.QuantizedLayerData`` — the on-disk layer format;
* ``eptq_amd.quantizers`` — E8-lattice / E8-D4 codebooks (decode side);
* ``eptq_amd.reconstruct`` — directory loaders.

The compute runs in ``libeptq_hip.so`` (C ABI, ``include/eptq_hip.h``).
"""

from .config import QuantizedLayerData
from .quantizers import E8D4Quantizer, E8LatticeQuantizer

__all__ = ["QuantizedLayerData", "E8D4Quantizer", "E8LatticeQuantizer"]

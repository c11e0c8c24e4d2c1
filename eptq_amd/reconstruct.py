"""Loaders for a quantized-model directory (``reconstruct.py:32-108`` of the reference).

Directory layout (``README.md:127-152``): ``quant_config.json``,
``quantizer.pt``, ``config.json`` + ``tokenizer/``, ``non_quantized_params.pt``,
``layer_<i>/<linear name>.pt`` (``QuantizedLayerData``) and
``layer_<i>/non_quantized.pt``.  Every file is read with
``torch.load(weights_only=True)``.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Dict, Optional

import torch

from .config import QuantizedLayerData
from .quantizers import BaseQuantizer, E8D4Quantizer, E8LatticeQuantizer


def load_quantization_config(quantized_dir) -> Dict:
    """``reconstruct.py:32-36``."""
    with open(Path(quantized_dir) / "quant_config.json", "r") as f:
        return json.load(f)


_QUANTIZER_CLASSES = {"e8_lattice": E8LatticeQuantizer, "e8_d4": E8D4Quantizer}


def _legacy_radius(blob: Dict, quantized_dir: Path) -> Optional[float]:
    """Radius of a pre-divided table: ``saved_radius`` in the mid format,
    else ``codebook_radius`` from ``quant_config.json`` (old format), else
    unknown (the quantizer's default stays)."""
    if "saved_radius" in blob:
        return float(blob["saved_radius"])
    if not (quantized_dir / "quant_config.json").exists():
        return None
    r = load_quantization_config(quantized_dir).get("codebook_radius")
    return None if r is None else float(r)


def load_quantizer(quantized_dir, device: str = "cuda") -> BaseQuantizer:
    """The codebook of a quantized directory (``reconstruct.py:39-90``).

    Three ``quantizer.pt`` formats:

    * ``raw_codes`` + ``radius`` (+ ``warp_alpha``): the table is
      ``raw / radius`` divided on ``device`` — so its fp32 bits are those
      the reference computes on the same device — then warped when
      ``warp_alpha != 1``; the raw codes stay for per-layer ``chosen_r``.  A
      type other than ``e8_lattice`` reads as E8-D4, as in the reference;
    * ``codebook`` + ``saved_radius``: a pre-divided table and its radius;
    * ``codebook`` alone: a pre-divided table, radius from
      ``quant_config.json``.
    """
    quantized_dir = Path(quantized_dir)
    blob = torch.load(quantized_dir / "quantizer.pt", weights_only=True, map_location="cpu")
    kind = blob.get("quantizer_type", "e8_lattice")
    if "raw_codes" in blob:
        cls = E8LatticeQuantizer if kind == "e8_lattice" else E8D4Quantizer
        q = cls.from_raw(blob["raw_codes"].float().to(device), float(blob["radius"]))
        alpha = float(blob.get("warp_alpha", 1.0))
        if alpha != 1.0:
            q.warp_codebook(alpha)
        return q
    cls = _QUANTIZER_CLASSES.get(kind)
    if cls is None:
        raise ValueError(f"{quantized_dir / 'quantizer.pt'}: unsupported quantizer type {kind!r} "
                         f"(expected one of {sorted(_QUANTIZER_CLASSES)})")
    q = cls(device=device, codebook=blob["codebook"].float().to(device))
    radius = _legacy_radius(blob, quantized_dir)
    if radius is not None:
        q._radius = radius
    return q


def save_quantizer(eq: BaseQuantizer, output_dir, quantizer_type: str) -> None:
    """Writer of the new format (``quantize.py:43-60``), for synthetic models."""
    raw = eq._raw_points if quantizer_type == "e8_lattice" else eq._raw_codes
    torch.save({"quantizer_type": quantizer_type, "raw_codes": raw.float().cpu(),
                "radius": eq._radius, "warp_alpha": getattr(eq, "_warp_alpha", 1.0)},
               Path(output_dir) / "quantizer.pt")


def load_quantized_layer(layer_dir, layer_name: str) -> QuantizedLayerData:
    """``reconstruct.py:93-96``."""
    return QuantizedLayerData.load(Path(layer_dir) / f"{layer_name}.pt")


def load_global_non_quantized_params(quantized_dir) -> Dict[str, torch.Tensor]:
    """``reconstruct.py:99-102``."""
    return torch.load(Path(quantized_dir) / "non_quantized_params.pt", weights_only=True,
                      map_location="cpu")


def load_layer_non_quantized_params(layer_dir) -> Dict[str, torch.Tensor]:
    """``reconstruct.py:105-108``."""
    return torch.load(Path(layer_dir) / "non_quantized.pt", weights_only=True, map_location="cpu")

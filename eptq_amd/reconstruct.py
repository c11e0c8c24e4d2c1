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
from typing import Dict

import torch

from .config import QuantizedLayerData
from .quantizers import BaseQuantizer, E8D4Quantizer, E8LatticeQuantizer


def load_quantization_config(quantized_dir) -> Dict:
    """``reconstruct.py:32-36``."""
    with open(Path(quantized_dir) / "quant_config.json", "r") as f:
        return json.load(f)


def load_quantizer(quantized_dir, device: str = "cuda") -> BaseQuantizer:
    """``reconstruct.py:39-90``: the three ``quantizer.pt`` formats.

    * new: ``raw_codes`` + ``radius`` (+ ``warp_alpha``) -> table ``raw / radius``
      computed on ``device`` (so its fp32 bits are the reference's on the same
      device), raw codes kept for per-layer ``chosen_r``;
    * mid: pre-divided ``codebook`` + ``saved_radius``;
    * old: pre-divided ``codebook``, radius from ``quant_config.json``.
    """
    quantized_dir = Path(quantized_dir)
    data = torch.load(quantized_dir / "quantizer.pt", weights_only=True, map_location="cpu")
    qtype = data.get("quantizer_type", "e8_lattice")
    if "raw_codes" in data:
        raw = data["raw_codes"].float().to(device)
        radius = float(data["radius"])
        if qtype == "e8_lattice":
            eq = E8LatticeQuantizer(device=device, codebook=raw / radius)
            eq._raw_points = raw
        else:
            eq = E8D4Quantizer(device=device, codebook=raw / radius)
            eq._raw_codes = raw
        eq._radius = radius
        warp_alpha = float(data.get("warp_alpha", 1.0))
        if warp_alpha != 1.0:
            eq.warp_codebook(warp_alpha)
        return eq
    codebook = data["codebook"].float().to(device)
    if qtype == "e8_lattice":
        eq = E8LatticeQuantizer(device=device, codebook=codebook)
    elif qtype == "e8_d4":
        eq = E8D4Quantizer(device=device, codebook=codebook)
    else:
        raise ValueError(f"Unknown quantizer type: {qtype}")
    if "saved_radius" in data:
        eq._radius = float(data["saved_radius"])
    else:
        cfg_path = quantized_dir / "quant_config.json"
        if cfg_path.exists():
            with open(cfg_path) as f:
                actual = json.load(f).get("codebook_radius")
            if actual is not None:
                eq._radius = float(actual)
    return eq


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

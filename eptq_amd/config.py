"""On-disk layer format: ``QuantizedLayerData`` (``config.py:98-159`` of the reference).

One ``torch.save`` dict per Linear with keys ``Q`` (int16 (M, N), index − 32768,
32767 = critical block), ``g`` (out,), ``h`` (in,), ``O`` (nnz, 8), and the
optional ``bias``, ``chosen_r`` and ``S_group`` ((out/qb, in)).  The quantizer
writes g/h/O/S_group as fp16 (``algorithms/eptq.py:395-403``).  Read and written
unchanged here.
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path
from typing import Any, Dict, Optional

import torch


@dataclass
class QuantizedLayerData:
    """One quantized Linear (``config.py:98-159``)."""

    Q: torch.Tensor
    g: torch.Tensor
    h: torch.Tensor
    O: torch.Tensor
    bias: Optional[torch.Tensor] = None
    chosen_r: Optional[float] = None
    S_group: Optional[torch.Tensor] = None

    def to_dict(self) -> Dict[str, Any]:
        out = {"Q": self.Q, "g": self.g, "h": self.h, "O": self.O}
        if self.bias is not None:
            out["bias"] = self.bias
        if self.chosen_r is not None:
            out["chosen_r"] = self.chosen_r
        if self.S_group is not None:
            out["S_group"] = self.S_group
        return out

    @classmethod
    def from_dict(cls, d: Dict[str, Any]) -> "QuantizedLayerData":
        return cls(Q=d["Q"], g=d["g"], h=d["h"], O=d["O"], bias=d.get("bias"),
                   chosen_r=d.get("chosen_r"), S_group=d.get("S_group"))

    def save(self, path: Path) -> None:
        torch.save(self.to_dict(), path)

    @classmethod
    def load(cls, path: Path) -> "QuantizedLayerData":
        data = torch.load(path, weights_only=True, map_location="cpu")
        return cls.from_dict(data)

    @property
    def out_features(self) -> int:
        return int(self.Q.shape[0]) * 8

    @property
    def in_features(self) -> int:
        return int(self.Q.shape[1])

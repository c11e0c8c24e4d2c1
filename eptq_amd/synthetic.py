"""Seeded synthetic quantized layers at real LLaMA/OPT shapes.

Distributions follow the benchmark configurations: indices uniform over the
valid 0..65534, exactly ``round(p·M·N)`` critical blocks at distinct
positions, ``O ~ N(0,1)``, ``g ~ |N(0.02, 0.005)|``, ``h ~ lognormal(0, 0.3)``,
optional ``bias ~ N(0, 0.01)`` and ``S_group ~ lognormal(0, 0.2)``,
``x ~ N(0, 1)``; everything fp16 except Q (int16).
"""

from __future__ import annotations

from typing import Optional

import torch

from .config import QuantizedLayerData

# (out_features, in_features) per benchmark configuration.
SHAPES = {
    "opt125m_fc1": (3072, 768),
    "llama2_7b": {"q": (4096, 4096), "k": (4096, 4096), "v": (4096, 4096), "o": (4096, 4096),
                  "gate": (11008, 4096), "up": (11008, 4096), "down": (4096, 11008)},
    "llama3_8b": {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
                  "gate": (14336, 4096), "up": (14336, 4096), "down": (4096, 14336)},
    "llama2_13b": {"qkvo": (5120, 5120), "gate_up": (13824, 5120), "down": (5120, 13824)},
}


def make_layer(out_features: int, in_features: int, *, seed: int, percmask: float,
               bias: bool = False, qb_size: Optional[int] = None,
               chosen_r: Optional[float] = None, device="cpu") -> QuantizedLayerData:
    """One synthetic ``QuantizedLayerData`` (generated on ``device``)."""
    if out_features % 8:
        raise ValueError("out_features must be a multiple of 8")
    M, N = out_features // 8, in_features
    gen = torch.Generator(device=device).manual_seed(seed)
    u = torch.randint(0, 65535, (M, N), generator=gen, device=device, dtype=torch.int32)
    Q = (u - 32768).to(torch.int16)
    nnz = int(round(percmask * M * N))
    if nnz:
        pos = torch.randperm(M * N, generator=gen, device=device)[:nnz]
        Q.view(-1)[pos] = 32767
    O = torch.randn((nnz, 8), generator=gen, device=device).half()
    g = (torch.randn(out_features, generator=gen, device=device) * 0.005 + 0.02).abs().half()
    h = torch.exp(torch.randn(N, generator=gen, device=device) * 0.3).half()
    b = (torch.randn(out_features, generator=gen, device=device) * 0.01).half() if bias else None
    S = None
    if qb_size is not None:
        if out_features % qb_size or qb_size % 8:
            raise ValueError("qb_size must divide out_features and be a multiple of 8")
        S = torch.exp(torch.randn((out_features // qb_size, N), generator=gen, device=device) * 0.2).half()
    return QuantizedLayerData(Q=Q, g=g, h=h, O=O, bias=b, chosen_r=chosen_r, S_group=S)


def make_x(batch: int, in_features: int, *, seed: int, device="cpu") -> torch.Tensor:
    gen = torch.Generator(device=device).manual_seed(seed)
    return torch.randn((batch, in_features), generator=gen, device=device).half()

"""Seeded synthetic quantized layers at real LLaMA/OPT shapes.

Distributions follow the benchmark configurations: indices uniform over the
valid 0..65534, exactly ``round(p·M·N)`` critical blocks at distinct
positions, ``O ~ N(0,1)``, ``g ~ |N(0.02, 0.005)|``, ``h ~ lognormal(0, 0.3)``,
optional ``bias ~ N(0, 0.01)`` and ``S_group ~ lognormal(0, 0.2)``,
``x ~ N(0, 1)``; everything fp16 except Q (int16).
"""

from __future__ import annotations

from typing import Optional, Sequence

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


def write_quantized_model(out_dir, hf_config, quantizer_type: str = "e8_d4", radius: float = 1.75,
                          percmask: float = 0.01, seed: int = 0, tokenizer=None,
                          qb_size: Optional[int] = None, warp_alpha: float = 1.0,
                          chosen_r: Optional[Sequence[Optional[float]]] = None) -> None:
    """Write a synthetic quantized-model directory in the reference layout
    (``README.md:127-152``; writers ``quantize.py:36-105,425-433``).

    ``hf_config`` is a ``transformers`` config (Llama or OPT architecture);
    every decoder ``nn.Linear`` becomes a seeded ``QuantizedLayerData``, the
    remaining parameters are random.  ``tokenizer``, if given, is saved under
    ``tokenizer/``.  ``warp_alpha`` is stored in ``quantizer.pt`` (the loader
    warps the table, ``reconstruct.py:63-65``); ``chosen_r``, if given, is
    cycled over the quantized Linears in load order as their ``chosen_r``.
    """
    import json
    from pathlib import Path

    from accelerate import init_empty_weights
    from transformers import AutoModelForCausalLM

    from .handlers import ModelHandler, get_model_handler_by_type
    from .quantizers import E8D4Quantizer, E8LatticeQuantizer
    from .reconstruct import save_quantizer

    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    with open(out / "quant_config.json", "w") as f:
        json.dump({"quantizer_type": quantizer_type, "codebook_radius": radius,
                   "model_name": None}, f, indent=2)
    q = E8D4Quantizer(radius=radius) if quantizer_type == "e8_d4" else E8LatticeQuantizer(radius=radius)
    if warp_alpha != 1.0:
        q._warp_alpha = warp_alpha      # recorded only: the file keeps the raw codes
    save_quantizer(q, out, quantizer_type)
    hf_config.save_pretrained(out)
    if tokenizer is not None:
        tokenizer.save_pretrained(out / "tokenizer")

    with init_empty_weights():
        model = AutoModelForCausalLM.from_config(hf_config)
    handler = get_model_handler_by_type(ModelHandler.detect_model_type(model))
    gen = torch.Generator().manual_seed(seed)
    quantized = set()
    n_lin = 0
    for lid, layer in enumerate(handler.get_layers(model)):
        layer_dir = out / f"layer_{lid}"
        layer_dir.mkdir(exist_ok=True)
        for k, (name, lin) in enumerate(handler.get_linear_layers(layer).items()):
            cr = chosen_r[n_lin % len(chosen_r)] if chosen_r else None
            n_lin += 1
            qd = make_layer(lin.out_features, lin.in_features, seed=seed + 1000 * lid + k,
                            percmask=percmask, bias=lin.bias is not None, qb_size=qb_size, chosen_r=cr)
            qd.save(layer_dir / f"{name}.pt")
            quantized.update({f"{name}.weight", f"{name}.bias"})
        other = {n: (torch.randn(p.shape, generator=gen) * 0.02 + (1.0 if "norm" in n else 0.0)).half()
                 for n, p in layer.named_parameters() if n not in quantized}
        torch.save(other, layer_dir / "non_quantized.pt")
    layer_prefix = {id(p) for l in handler.get_layers(model) for p in l.parameters()}
    glob = {n: (torch.randn(p.shape, generator=gen) * 0.02 + (1.0 if "norm" in n else 0.0)).half()
            for n, p in model.named_parameters() if id(p) not in layer_prefix}
    torch.save(glob, out / "non_quantized_params.pt")

"""``load_quantized_model``: a HuggingFace model whose decoder Linears are ``EPTQLinear``.

Drop-in for the reference's ``kernels/patch.py:24-142`` (same signature and
return value ``(model, tokenizer)``).  One change, towards the reference's own
reconstruct semantics: the codebook comes from ``load_quantizer``
(``reconstruct.py:39-90``), so ``warp_alpha`` and each layer's ``chosen_r`` are
honoured, and the fp32 table used for bit-exact dequantization is computed on
``device`` as ``eptq.reconstruct`` computes it.
"""

from __future__ import annotations

import sys
from pathlib import Path
from typing import Tuple

import torch
import torch.nn as nn

from ..handlers import ModelHandler, get_model_handler_by_type
from ..reconstruct import (load_global_non_quantized_params, load_layer_non_quantized_params,
                           load_quantization_config, load_quantized_layer, load_quantizer)
from .linear import EPTQLinear


def _set_param(root: nn.Module, dotted: str, value: torch.Tensor) -> None:
    parts, target = dotted.split("."), root
    for p in parts[:-1]:
        target = getattr(target, p)
    setattr(target, parts[-1], nn.Parameter(value, requires_grad=False))


def load_quantized_model(quantized_dir: str, device: str = "cuda") -> Tuple[nn.Module, object]:
    """Build the model skeleton, swap every decoder ``nn.Linear`` for an
    ``EPTQLinear`` holding the compressed layer, load the remaining params."""
    from accelerate import init_empty_weights
    from transformers import AutoConfig, AutoModelForCausalLM, AutoTokenizer

    quantized_dir = Path(quantized_dir)
    quant_config = load_quantization_config(quantized_dir)
    quantizer_type = quant_config.get("quantizer_type", "e8_lattice")

    print(f"eptq_amd: reading the codebook of {quantized_dir}", file=sys.stderr)
    quantizer = load_quantizer(quantized_dir, device=device)

    print("eptq_amd: building the model skeleton", file=sys.stderr)
    config = AutoConfig.from_pretrained(quantized_dir)
    model_dtype = getattr(config, "torch_dtype", None) or torch.float16
    with init_empty_weights():
        try:
            model = AutoModelForCausalLM.from_config(config, dtype=model_dtype)
        except TypeError:
            model = AutoModelForCausalLM.from_config(config, torch_dtype=model_dtype)

    tokenizer_dir = quantized_dir / "tokenizer"
    try:
        tokenizer = AutoTokenizer.from_pretrained(tokenizer_dir)
    except Exception:
        model_name = quant_config.get("model_name")
        if not model_name:
            raise ValueError(f"no tokenizer under {tokenizer_dir}, and quant_config.json names "
                             "no model_name to fetch one by")
        print(f"eptq_amd: no tokenizer under {tokenizer_dir}; using the one of {model_name}", file=sys.stderr)
        tokenizer = AutoTokenizer.from_pretrained(model_name)

    handler = get_model_handler_by_type(ModelHandler.detect_model_type(model))
    global_params = load_global_non_quantized_params(quantized_dir)
    layers = handler.get_layers(model)
    print(f"eptq_amd: swapping in {len(layers)} quantized decoder layers", file=sys.stderr)
    for lid, layer in enumerate(layers):
        layer_dir = quantized_dir / f"layer_{lid}"
        for name in list(handler.get_linear_layers(layer).keys()):
            qd = load_quantized_layer(layer_dir, name)
            lin = EPTQLinear.from_quantized_data(qd, quantizer, quantizer_type)
            parts, parent = name.split("."), layer
            for p in parts[:-1]:
                parent = getattr(parent, p)
            setattr(parent, parts[-1], lin)
        for pname, param in load_layer_non_quantized_params(layer_dir).items():
            _set_param(layer, pname, param)
    for name, param in global_params.items():
        _set_param(model, name, param)

    unloaded = [n for n, p in model.named_parameters() if p.is_meta]
    if unloaded:
        print(f"eptq_amd: {len(unloaded)} parameters still on the meta device after loading "
              f"(first: {', '.join(unloaded[:5])})", file=sys.stderr)
    model = model.to(device=device)
    model.eval()
    print("eptq_amd: model ready", file=sys.stderr)
    return model, tokenizer

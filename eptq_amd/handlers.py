"""The three loader-facing model-handler methods (``models/base.py:126-143``,
``models/llama.py:13-15,62-68``, ``models/opt.py:13-15,49-55``)."""

from __future__ import annotations

from typing import Dict

from torch import nn


class ModelHandler:
    def get_layers(self, model: nn.Module) -> nn.ModuleList:
        raise NotImplementedError

    def get_linear_layers(self, layer: nn.Module) -> Dict[str, nn.Module]:
        """Every ``nn.Linear`` inside one decoder layer, by dotted name."""
        return {name: mod for name, mod in layer.named_modules() if isinstance(mod, nn.Linear)}

    @staticmethod
    def detect_model_type(model: nn.Module) -> str:
        name = model.__class__.__name__.lower()
        if "opt" in name:
            return "opt"
        if "llama" in name:
            return "llama"
        return "unknown"


class LlamaHandler(ModelHandler):
    def get_layers(self, model: nn.Module) -> nn.ModuleList:
        return model.model.layers


class OPTHandler(ModelHandler):
    def get_layers(self, model: nn.Module) -> nn.ModuleList:
        return model.model.decoder.layers


def get_model_handler_by_type(model_type: str) -> ModelHandler:
    """``reconstruct.py:22-29``."""
    if model_type == "opt":
        return OPTHandler()
    if model_type == "llama":
        return LlamaHandler()
    raise ValueError(f"Unsupported model type: {model_type}")

"""Which nn.Linear layers become W8A8 modules.

Restates the selection rule of QuantLayerConfig.should_quantize
(x_base/x_base/config/config_loader.py:182-232) and the per-model layer
exclusions of x_base/x_base/config/quant_config.yaml (default :14-29,
hunyuan :74-90, minimax_h3 :146-171, model mapping :191-199) for the W8A8
(int8 / fp8) path:

  1. the layer must be one of layer_types (nn.Linear);
  2. a name matching any exclude pattern is skipped (glob or substring);
  3. if include patterns are given, the name must match one;
  4. dtype patterns: None = every layer that passed, [] = none, else must match.
"""
from __future__ import annotations

import fnmatch
from dataclasses import dataclass, field
from typing import Dict, List, Optional

from torch import nn

_LAYER_TYPES = {"Linear": nn.Linear, "Conv2d": nn.Conv2d, "Conv3d": nn.Conv3d}


@dataclass
class QuantLayerConfig:
    include_patterns: Optional[List[str]] = None
    exclude_patterns: List[str] = field(default_factory=list)
    layer_types: List[str] = field(default_factory=lambda: ["Linear"])
    int8_patterns: Optional[List[str]] = None
    fp8_patterns: Optional[List[str]] = None

    def __post_init__(self):
        self._types = tuple(_LAYER_TYPES.get(t, nn.Linear) for t in self.layer_types)

    @classmethod
    def from_dict(cls, d: Dict) -> "QuantLayerConfig":
        return cls(include_patterns=d.get("include_patterns"),
                   exclude_patterns=list(d.get("exclude_patterns", [])),
                   layer_types=list(d.get("layer_types", ["Linear"])),
                   int8_patterns=d.get("int8_patterns"),
                   fp8_patterns=d.get("fp8_patterns"))

    @staticmethod
    def _matches(name: str, patterns: List[str]) -> bool:
        return any(fnmatch.fnmatch(name, p) or p in name for p in patterns)

    def should_quantize(self, layer_name: str, layer: nn.Module, dtype: str = 'int8') -> bool:
        if not isinstance(layer, self._types):
            return False
        if self._matches(layer_name, self.exclude_patterns):
            return False
        if self.include_patterns:
            if not self._matches(layer_name, self.include_patterns):
                return False
        patterns = getattr(self, f"{dtype}_patterns", None)
        if patterns is None:
            return True
        if len(patterns) == 0:
            return False
        return self._matches(layer_name, patterns)


_COMMON_EXCLUDE = ["timesteps_proj", "time_embedder", "lora"]

MODEL_CONFIGS: Dict[str, Dict] = {
    "default": {"exclude_patterns": _COMMON_EXCLUDE},
    "hunyuan": {"exclude_patterns": _COMMON_EXCLUDE},
    "cogvideox": {"exclude_patterns": _COMMON_EXCLUDE},
    "wan": {"exclude_patterns": _COMMON_EXCLUDE},
    "minimax_h3": {"exclude_patterns": [
        "proj_in", "audio_proj_in", "context_embedder", "time_embedder", "time_proj", "token_refiner",
        "adaln_proj.linear", "norm_out", "proj_out", "audio_proj_out", "rope", "lora"]},
}

MODEL_TYPE_MAPPING = {
    "WanTransformer3DModel": "wan",
    "HunyuanVideoTransformer3DModel": "hunyuan",
    "CogVideoXTransformer3DModel": "cogvideox",
    "MiniMaxH3Transformer3DModel": "minimax_h3",
}


def detect_config_name(transformer: nn.Module) -> str:
    """Class name, then base classes, then name keywords (config_loader.py:295-325)."""
    for cls in type(transformer).__mro__:
        if cls.__name__ in MODEL_TYPE_MAPPING:
            return MODEL_TYPE_MAPPING[cls.__name__]
    lower = type(transformer).__name__.lower()
    for key in ("wan", "hunyuan", "cogvideo"):
        if key in lower:
            return "cogvideox" if key == "cogvideo" else key
    return "default"


def get_config(name: str) -> QuantLayerConfig:
    return QuantLayerConfig.from_dict(MODEL_CONFIGS.get(name, MODEL_CONFIGS["default"]))


def get_config_for_model(transformer: nn.Module) -> QuantLayerConfig:
    return get_config(detect_config_name(transformer))

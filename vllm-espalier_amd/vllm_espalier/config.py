"""The vLLM quantisation config for Espalier checkpoints, quant_method "espalier" (the interface of
vllm_espalier/config.py: EspalierConfig, text_key, PACKED).

Which modules are trellis-coded is decided by the checkpoint itself: every weight-map key ending in ".esp_trellis"
names one coded matrix (maybe_update_config scans model.safetensors.index.json). A vLLM layer that fuses several
checkpoint matrices (PACKED) is coded when all of them are; a fused layer with only some of them coded is refused.
Routed experts are coded when any tensor under their prefix is. Everything else (router, norms, embeddings, vision
tower) stays unquantised.

vLLM is optional here: with vLLM importable the class registers itself with vLLM and derives from its
QuantizationConfig; without it the same class works stand-alone (checkpoint scan, layer decisions), which is how the
tests drive it. Layer kinds are recognised by the class names in the layer's type hierarchy (RoutedExperts or
FusedMoE, ParallelLMHead, LinearBase), so vLLM's own layers and stand-ins are treated alike.
"""
from __future__ import annotations

import json
import re
from pathlib import Path
from typing import Any

import torch

try:                                                   # vLLM present: register the method with it
    from vllm.model_executor.layers.quantization import register_quantization_config as _register
    from vllm.model_executor.layers.quantization.base_config import QuantizationConfig as _Base
    HAVE_VLLM = True
except ImportError:                                    # stand-alone
    _Base = object
    HAVE_VLLM = False

    def _register(name):
        return lambda cls: cls

NAME = "espalier"
TRELLIS_SUFFIX = ".esp_trellis"
# a vLLM fused layer -> the checkpoint matrices it holds, in vLLM's output order (config.py:25-30)
PACKED = {
    "qkv_proj": ["q_proj", "k_proj", "v_proj"],
    "gate_up_proj": ["gate_proj", "up_proj"],
    "in_proj_qkvz": ["in_proj_qkv", "in_proj_z"],
    "in_proj_ba": ["in_proj_b", "in_proj_a"],
}
_LAYER_PATH = re.compile(r"(?:^|\.)(mtp\.)?(layers\.\d+\..+)$")


def text_key(name: str) -> str | None:
    """A checkpoint key or vLLM prefix -> its text-model key: "layers.N.<rest>", "mtp.layers.N.<rest>" (the MTP
    head's layers keep their own namespace, never aliasing decoder layer N) or "lm_head"; None for the vision tower
    and for names outside the layer stack (config.py:33-42)."""
    if "visual" in name or "vision" in name:
        return None
    if name == "lm_head" or name.endswith(".lm_head") or ".lm_head." in name:
        return "lm_head"
    m = _LAYER_PATH.search(name)
    if m is None:
        return None
    return (m.group(1) or "") + m.group(2)


def checkpoint_dir(model: str, revision: str | None = None) -> Path:
    """A local checkpoint directory as given, else the hub snapshot of its json files (which needs the network)."""
    p = Path(model)
    if p.is_dir():
        return p
    from huggingface_hub import snapshot_download
    return Path(snapshot_download(model, revision=revision, allow_patterns=["*.json"]))


def _layer_kind(layer) -> str | None:
    names = {c.__name__ for c in type(layer).__mro__}
    if names & {"RoutedExperts", "FusedMoE"}:
        return "experts"
    if "ParallelLMHead" in names:
        return "lm_head"
    if "LinearBase" in names:
        return "linear"
    return None


def _unquantized_linear():
    if HAVE_VLLM:
        from vllm.model_executor.layers.linear import UnquantizedLinearMethod
        return UnquantizedLinearMethod()
    return None


@_register(NAME)
class EspalierConfig(_Base):
    def __init__(self, raw: dict[str, Any] | None = None):
        if HAVE_VLLM:
            super().__init__()
        self.raw = dict(raw or {})
        self.coded: set[str] = set()          # text keys of the checkpoint's trellis-coded matrices
        self.packed_modules_mapping = {k: list(v) for k, v in PACKED.items()}
        self.checkpoint: Path | None = None

    # ---- QuantizationConfig surface (config.py:56-90)
    def get_name(self) -> str:
        return NAME

    def get_supported_act_dtypes(self) -> list:
        return [torch.bfloat16, torch.float16]

    @classmethod
    def get_min_capability(cls) -> int:
        return 80

    @staticmethod
    def get_config_filenames() -> list[str]:
        return []

    @classmethod
    def from_config(cls, config: dict[str, Any]) -> "EspalierConfig":
        method = str(config.get("quant_method", "")).lower()
        if method != NAME:
            raise ValueError(f"quant_method {config.get('quant_method')!r} is not {NAME!r}")
        return cls(config)

    @classmethod
    def override_quantization_method(cls, hf_quant_cfg, user_quant, hf_config=None):
        method = str((hf_quant_cfg or {}).get("quant_method", "")).lower()
        return NAME if method == NAME else None

    # ---- the checkpoint scan (config.py:92-104)
    def maybe_update_config(self, model_name: str, hf_config=None, revision: str | None = None) -> None:
        d = checkpoint_dir(model_name, revision)
        index = json.loads((d / "model.safetensors.index.json").read_text())
        self.scan(index["weight_map"])
        self.checkpoint = d

    def scan(self, weight_map) -> None:
        """Record every trellis-coded matrix of a weight map (its keys)."""
        for key in weight_map:
            if key.endswith(TRELLIS_SUFFIX):
                t = text_key(key[:-len(TRELLIS_SUFFIX)])
                if t is not None:
                    self.coded.add(t)
        if not self.coded:
            raise ValueError("the checkpoint holds no .esp_trellis tensors")

    # ---- per-layer decisions (config.py:106-133)
    def is_exl3(self, prefix: str) -> bool:
        """Whether the vLLM layer at `prefix` is trellis-coded: every checkpoint matrix it fuses is (an error when
        only some are)."""
        t = text_key(prefix)
        if t is None:
            return False
        if t == "lm_head":
            return t in self.coded
        parent, _, leaf = t.rpartition(".")
        parts = [f"{parent}.{m}" if parent else m for m in PACKED.get(leaf, [leaf])]
        found = {p: p in self.coded for p in parts}
        if any(found.values()) and not all(found.values()):
            raise ValueError(f"{prefix}: a fused layer only partly trellis-coded: {found}")
        return all(found.values())

    def experts_exl3(self, prefix: str) -> bool:
        t = text_key(prefix)
        return t is not None and any(k.startswith(t + ".") for k in self.coded)

    def get_quant_method(self, layer, prefix: str):
        from .linear import EspLinearMethod
        from .moe import EspMoEMethod
        kind = _layer_kind(layer)
        if kind == "experts":
            if not self.experts_exl3(prefix):
                raise ValueError(f"{prefix}: routed experts without trellis-coded tensors")
            return EspMoEMethod(getattr(layer, "moe_config", None))
        if kind == "lm_head":
            return EspLinearMethod(prefix) if self.is_exl3(prefix) else None
        if kind == "linear":
            return EspLinearMethod(prefix) if self.is_exl3(prefix) else _unquantized_linear()
        return None

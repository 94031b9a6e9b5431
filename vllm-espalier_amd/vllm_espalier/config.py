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

    # ---- QuantizationConfig surface (the reference's config.py:56-90)
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

    # ---- the checkpoint scan (the reference's config.py:92-104)
    def maybe_update_config(self, model_name: str, hf_config=None, revision: str | None = None) -> None:
        d = checkpoint_dir(model_name, revision)
        index = json.loads((d / "model.safetensors.index.json").read_text())
        self.scan(index["weight_map"])
        self.checkpoint = d

    def scan(self, weight_map) -> None:
        """Record every trellis-coded matrix of a weight map (its keys)."""
        self.coded |= coded_matrices(weight_map)
        if not self.coded:
            raise ValueError("the checkpoint holds no .esp_trellis tensors")

    # ---- per-layer decisions (the reference's config.py:106-133)
    def is_exl3(self, prefix: str) -> bool:
        """Whether the vLLM layer at `prefix` is trellis-coded: every checkpoint matrix it fuses is (ValueError when
        only some are)."""
        members = fused_members(text_key(prefix))
        coded = [m for m in members if m in self.coded]
        if coded and len(coded) != len(members):
            raise ValueError(f"{prefix}: a fused layer only partly trellis-coded: coded {coded} of {members}")
        return bool(members) and len(coded) == len(members)

    def experts_exl3(self, prefix: str) -> bool:
        """Whether any matrix under the routed experts at `prefix` is trellis-coded."""
        t = text_key(prefix)
        return t is not None and any(k.startswith(t + ".") for k in self.coded)

    def get_quant_method(self, layer, prefix: str):
        from .linear import EspLinearMethod
        from .moe import EspMoEMethod
        kind = _layer_kind(layer)
        if kind is None:
            return None
        if kind == "experts":
            if not self.experts_exl3(prefix):
                raise ValueError(f"{prefix}: routed experts without trellis-coded tensors")
            return EspMoEMethod(getattr(layer, "moe_config", None))
        if self.is_exl3(prefix):
            return EspLinearMethod(prefix)
        # an uncoded head keeps vLLM's default; an uncoded linear layer runs unquantised
        return None if kind == "lm_head" else _unquantized_linear()


def coded_matrices(weight_map) -> set[str]:
    """Text keys of the trellis-coded matrices a checkpoint's weight map names (keys ending in .esp_trellis)."""
    keys = (text_key(k[:-len(TRELLIS_SUFFIX)]) for k in weight_map if k.endswith(TRELLIS_SUFFIX))
    return {k for k in keys if k is not None}


def fused_members(text: str | None) -> list[str]:
    """The checkpoint matrices a vLLM layer holds, by text key: the PACKED members of a fused layer, else the layer
    itself; none outside the text model."""
    if text is None:
        return []
    parent, _, leaf = text.rpartition(".")
    return [f"{parent}.{m}" if parent else m for m in PACKED.get(leaf, [leaf])]

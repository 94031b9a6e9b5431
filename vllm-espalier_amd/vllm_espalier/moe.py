"""The vLLM fused-MoE method for trellis-coded routed experts (the interface of vllm_espalier/moe.py: EspMoEMethod,
GROUPED, GROUPED_ROWS, ROUTE).

Up to GROUPED_ROWS tokens (ESPALIER_GROUPED_EXPERTS=1, default) the whole layer runs as the grouped pipeline of
experts.py. The shared expert is one more slot of it: the method reports mk_can_overlap_shared_experts, so vLLM's
runner leaves the shared expert to apply(), which stores its gated output where the runner reads it
(shared_experts._output). vLLM is asked for int32 top-k ids, so no cast kernels run around the layer.

With ESPALIER_FUSED_ROUTING=1 (default) the method is monolithic: the router GEMV, softmax / top-k /
renormalisation and the grouping are one launch (esp_route_group), fed the hidden states by a pass-through that
replaces the runner's gate. More tokens (prefill) follow ESPALIER_PREFILL_MODE: chunk, the pipeline over 32-token
windows (a token gets its decode bits); tile, the whole prompt at once (experts.prefill: one routing launch, one
grouping, each picked expert decoded once); gemm (or ESPALIER_GROUPED_EXPERTS=0), expert by expert through
espalier::matmul.

Each expert keeps its own gate / up / down EspMatrix (its own width and codebook), so nothing is stacked. The layer's
load_weights is replaced: vLLM's expert loader takes any 3-D tensor for an all-experts tensor, and a trellis is 3-D
per expert.

vLLM is optional: with it the method derives from FusedMoEMethodBase and finds the layer's runner through vLLM's
forward context; without it the same code runs on stand-in layers (the runner then comes from layer._esp_runner).
"""
from __future__ import annotations

import enum
import re
import types

import torch
import torch.nn.functional as F
from torch.nn import Parameter

from . import experts as grouped
from ._env import env
from .linear import single_process
from .matrix import SUFFIXES, EspMatrix

try:
    from vllm.model_executor.layers.fused_moe.fused_moe_method_base import FusedMoEMethodBase as _Base
    from vllm.model_executor.layers.fused_moe.runner.shared_experts import SharedExpertsOrder
    HAVE_VLLM = True
except ImportError:
    _Base = object
    HAVE_VLLM = False

    class SharedExpertsOrder(enum.Enum):
        """The orders vLLM's runner can give a layer's shared experts (only this one matters here)."""
        MK_INTERNAL_OVERLAPPED = "mk_internal_overlapped"
        EXTERNAL = "external"

GROUPED = env("ESPALIER_GROUPED_EXPERTS", "1") != "0"
GROUPED_ROWS = 32
# routing in the plugin's own launch; its picks match exact routing (fp64 logits rounded to bf16), where a bf16
# router GEMM can differ on near-ties. ESPALIER_FUSED_ROUTING=0 keeps vLLM's router.
ROUTE = GROUPED and env("ESPALIER_FUSED_ROUTING", "1") != "0"

_EXPERT_KEY = re.compile(r"(?:^|\.)(\d+)\.(gate_proj|up_proj|down_proj)\.(\w+)$")
_PROJ = ("gate_proj", "up_proj", "down_proj")


def _prefill_mode() -> str:
    from . import ops
    return ops.PREFILL


class _PassThroughGate(torch.nn.Module):
    """Takes the place of the runner's router gate under ROUTE: hands the hidden states on as the "logits", so
    apply_monolithic runs the GEMV inside esp_route_group. Keeps the original gate (and its weight)."""

    def __init__(self, gate):
        super().__init__()
        self.inner = gate
        self.weight = gate.weight

    def forward(self, x):
        return x, None


def _runner(layer):
    """The layer's MoE runner: from vLLM's forward context, else (stand-alone) the one the layer carries."""
    if HAVE_VLLM:
        from vllm.forward_context import get_forward_context
        return get_forward_context().no_compile_layers[layer.layer_name]
    return layer._esp_runner


class EspMoEMethod(_Base):
    def __init__(self, moe_config=None):
        if HAVE_VLLM:
            super().__init__(moe_config)
        self.moe_config = moe_config

    @property
    def topk_indices_dtype(self):
        return torch.int32

    @property
    def is_monolithic(self) -> bool:
        return ROUTE

    @property
    def mk_can_overlap_shared_experts(self) -> bool:
        return GROUPED

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition, params_dtype,
                       **extra_weight_attrs):
        single_process()
        layer._esp_num_experts = num_experts
        layer._esp_parts = {}                       # (expert, projection) -> {suffix: tensor}
        for group in ("w13", "w2"):
            for suffix in SUFFIXES:
                layer.register_parameter(f"{group}_{suffix}", Parameter(torch.empty(0), requires_grad=False))
        device = layer.w13_esp_trellis.device

        def load_weights(self_, weights):
            for name, tensor in weights:
                m = _EXPERT_KEY.search(name)
                if m is None:
                    raise ValueError(f"{getattr(self_, 'layer_name', '?')}: unexpected expert tensor {name!r}")
                e, proj, suffix = int(m.group(1)), m.group(2), m.group(3)
                if suffix not in SUFFIXES:
                    raise ValueError(f"{getattr(self_, 'layer_name', '?')}: unknown suffix in {name!r}")
                self_._esp_parts.setdefault((e, proj), {})[suffix] = tensor.to(device).clone()
                yield f"{'w2' if proj == 'down_proj' else 'w13'}_{suffix}"

        layer.load_weights = types.MethodType(load_weights, layer)

    def process_weights_after_loading(self, layer) -> None:
        E = layer._esp_num_experts
        mats = {key: EspMatrix(t) for key, t in layer._esp_parts.items()}
        missing = [(e, p) for e in range(E) for p in _PROJ if (e, p) not in mats]
        if missing:
            raise RuntimeError(f"{getattr(layer, 'layer_name', '?')}: {len(missing)} expert matrices missing, "
                               f"first {missing[:3]}")
        layer._esp_experts = [tuple(mats[(e, p)] for p in _PROJ) for e in range(E)]
        del layer._esp_parts
        act = str(getattr(layer, "activation", "silu")).lower()
        if "silu" not in act:
            raise NotImplementedError(f"{getattr(layer, 'layer_name', '?')}: activation {act}")
        layer._esp_grouped = None                   # built at the first apply, once the shared expert is known

    def get_fused_moe_quant_config(self, layer):
        return None

    # ---- the grouped pipeline
    @staticmethod
    def _same_input(layer) -> bool:
        """True when the layer's runner applies no routed-input transform, so the routed input and the shared
        experts' input are the same value and the shared slot may read x."""
        try:
            runner = _runner(layer)
        except Exception:
            return False
        return runner is not None and getattr(runner, "routed_input_transform", "missing") is None

    @staticmethod
    def _shared_from(shared_experts):
        """(gate, up, down) EspMatrix and the sigmoid gate's weight of vLLM's shared-expert MLP, or (None, None)
        when it is not a trellis-coded gate_up / down pair with a one-output gate."""
        if shared_experts is None:
            return None, None
        mlp = shared_experts._layer
        gu = getattr(mlp.gate_up_proj, "_esp_mats", None)
        dn = getattr(mlp.down_proj, "_esp_mats", None)
        gate = getattr(mlp, "expert_gate", None)
        if gu and dn and len(gu) == 2 and len(dn) == 1 and gate is not None and gate.weight.shape[0] == 1:
            return (gu[0], gu[1], dn[0]), gate.weight.detach()
        return None, None

    def _layer_tables(self, layer, shared_experts, internal: bool):
        """The grouped tables (built once) and whether the shared expert is folded into them for this call."""
        if layer._esp_grouped is None:
            layer._esp_same_input = self._same_input(layer)
            shared, gate_w = self._shared_from(shared_experts if internal and layer._esp_same_input else None)
            layer._esp_grouped = grouped.prepare(layer._esp_experts, shared, gate_w)
        L = layer._esp_grouped
        return L, internal and L.shared_id >= 0 and layer._esp_same_input

    @staticmethod
    def _finish_shared(shared_experts, shared_input, sh, fold: bool, internal: bool) -> None:
        if fold:
            shared_experts._output[shared_experts._output_idx] = sh
        elif internal:
            shared_experts.forward(shared_input, SharedExpertsOrder.MK_INTERNAL_OVERLAPPED)

    @staticmethod
    def _grouped_run(L, x, pick, wts, k: int, gate=None):
        """The grouped layer over x's rows: one pipeline up to GROUPED_ROWS rows, else the prefill mode's."""
        T = x.shape[0]
        slots = k + (L.shared_id >= 0)
        if T <= GROUPED_ROWS:
            s = grouped.scratch(L, GROUPED_ROWS, slots, x.device)
            if pick is None:
                grouped.route(x, gate, k, L, s)
            return grouped.routed2(x, pick, wts, L, s, k=k)
        if _prefill_mode() == "tile":
            ps = grouped.prefill_scratch(L, T, slots, x.device)
            return grouped.prefill(x, pick, wts, L, ps, k, gate=gate)
        s = grouped.scratch(L, GROUPED_ROWS, slots, x.device)
        return grouped.windows(x, pick, wts, L, s, k=k, gate=gate)

    def _expert_loop(self, layer, x, topk_weights, topk_ids):
        """Expert by expert (no grouped kernels): each picked expert's rows through its three matrices, the weighted
        sum in fp32."""
        T, k = topk_ids.shape
        acc = torch.zeros(x.shape, dtype=torch.float32, device=x.device)
        ids = topk_ids.reshape(-1).long()
        rows = torch.arange(T, device=x.device).repeat_interleave(k)
        w = topk_weights.reshape(-1).float()
        for e in torch.unique(ids).tolist():
            hit = ids == e
            r = rows[hit]
            gate, up, down = layer._esp_experts[e]
            xr = x[r]
            h = F.silu(gate.forward(xr).float()) * up.forward(xr).float()
            acc.index_add_(0, r, down.forward(h.to(x.dtype)).float() * w[hit, None])
        return acc.to(x.dtype)

    def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None, shared_experts_input=None):
        T, k = topk_ids.shape
        internal = (shared_experts is not None and shared_experts._determine_shared_experts_order(
            shared_experts_input) == SharedExpertsOrder.MK_INTERNAL_OVERLAPPED)
        if GROUPED and (T <= GROUPED_ROWS or _prefill_mode() in ("chunk", "tile")):
            L, fold = self._layer_tables(layer, shared_experts, internal)
            out, sh = self._grouped_run(L, x.contiguous(), topk_ids.to(torch.int32).contiguous(),
                                        topk_weights.float().contiguous(), k)
            self._finish_shared(shared_experts, shared_experts_input, sh, fold, internal)
            return out
        if internal:
            shared_experts.forward(shared_experts_input, SharedExpertsOrder.MK_INTERNAL_OVERLAPPED)
        return self._expert_loop(layer, x, topk_weights, topk_ids)

    def apply_monolithic(self, layer, x, router_logits, input_ids=None):
        """Routing inside the plugin (ROUTE). On the first call the runner's gate gives way to a pass-through (its
        weight kept here), so router_logits is the hidden states from then on; that first call's real logits go
        through vLLM's router."""
        runner = _runner(layer)
        if getattr(layer, "_esp_gate_w", None) is None:
            r = runner.router
            if not (getattr(r, "renormalize", True) and getattr(r, "scoring_func", "softmax") == "softmax"):
                raise NotImplementedError("the fused routing implements softmax top-k with renormalisation only")
            layer._esp_gate_w = runner.gate.weight.detach()
            runner.gate = _PassThroughGate(runner.gate)
        shared = runner._shared_experts
        logits_given = router_logits.shape[-1] == layer._esp_num_experts != x.shape[-1]
        k = runner.router.top_k if hasattr(runner.router, "top_k") else layer.top_k
        internal = shared is not None and shared._determine_shared_experts_order(x) == \
            SharedExpertsOrder.MK_INTERNAL_OVERLAPPED
        T = x.shape[0]
        if not logits_given and (T <= GROUPED_ROWS or _prefill_mode() in ("chunk", "tile")):
            L, fold = self._layer_tables(layer, shared, internal)
            out, sh = self._grouped_run(L, x.contiguous(), None, None, k, gate=layer._esp_gate_w)
            self._finish_shared(shared, x, sh, fold, internal)
            return out
        logits = router_logits if logits_given else F.linear(x, layer._esp_gate_w)
        topk_weights, topk_ids = runner.router.select_experts(hidden_states=x, router_logits=logits,
                                                              topk_indices_dtype=self.topk_indices_dtype,
                                                              input_ids=input_ids)
        return self.apply(layer, x, topk_weights, topk_ids, shared, x)

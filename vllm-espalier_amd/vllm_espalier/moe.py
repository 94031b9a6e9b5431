"""The vLLM fused-MoE method for trellis-coded routed experts: EspMoEMethod, written against vLLM's FusedMoEMethodBase
contract (create_weights, process_weights_after_loading, apply, apply_monolithic, topk_indices_dtype, is_monolithic,
mk_can_overlap_shared_experts), with the switches GROUPED (ESPALIER_GROUPED_EXPERTS), ROUTE
(ESPALIER_FUSED_ROUTING) and GROUPED_ROWS of the plugin's interface (the reference's vllm_espalier/moe.py:40-47).

Loading. Each expert keeps its own gate / up / down EspMatrix (its own width and codebook), so nothing is stacked.
vLLM's expert loader would take any 3-D tensor for an all-experts tensor, and a trellis is 3-D for one expert, so
the layer's load_weights is an ExpertStore's: it files each tensor by (expert, projection, suffix) and reports the
layer parameter it stands for (w13_<suffix> for gate and up, w2_<suffix> for down), as vLLM's loader expects.

Running. Every path ends in run_grouped, the kernels of experts.py:
  * up to GROUPED_ROWS tokens, the decode pipeline (routed2), with the routing launch first when the plugin routes;
  * more tokens (prefill) as ESPALIER_PREFILL_MODE says: chunk, the pipeline over 32-token windows (a token gets its
    decode bits); tile, the whole prompt at once (experts.prefill); gemm, or ESPALIER_GROUPED_EXPERTS=0, each
    picked expert's rows through espalier::matmul (expert_loop).
The shared expert is one more slot of the grouped launches when vLLM hands it to the method (the order
MK_INTERNAL_OVERLAPPED, which mk_can_overlap_shared_experts asks for), the runner transforms no routed input, and it
is a trellis-coded gate_up / down pair with a one-output sigmoid gate; its gated output is then stored where the
runner reads it. Otherwise the runner's own shared-expert forward runs.

Routing. With ROUTE the method is monolithic: the first apply_monolithic call replaces the runner's gate by a
HiddenStatesGate, so router_logits is the hidden states from then on, and one launch does the router GEMV, softmax /
top-k / renormalisation and the grouping (its picks match exact routing: fp64 logits rounded to bf16). That first
call's logits are real, and go through vLLM's router, as do prompts in the gemm mode.

vLLM is optional: with it the method derives from FusedMoEMethodBase and finds the runner in vLLM's forward context;
without it the same code runs on stand-in layers, whose runner is layer.espalier_runner.
"""
from __future__ import annotations

import enum
import weakref
from dataclasses import dataclass

import torch
import torch.nn.functional as F

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
        """vLLM's orders for a layer's shared experts (the method distinguishes only the first)."""
        MK_INTERNAL_OVERLAPPED = "mk_internal_overlapped"
        EXTERNAL = "external"

GROUPED = env("ESPALIER_GROUPED_EXPERTS", "1") != "0"
GROUPED_ROWS = 32
ROUTE = GROUPED and env("ESPALIER_FUSED_ROUTING", "1") != "0"

# projection -> the layer parameter group its tensors stand for
_GROUP_OF = {"gate_proj": "w13", "up_proj": "w13", "down_proj": "w2"}
_PROJECTIONS = tuple(_GROUP_OF)
_INTERNAL = SharedExpertsOrder.MK_INTERNAL_OVERLAPPED


def split_expert_name(name: str) -> tuple[int, str, str]:
    """'<...>.<expert>.<projection>.<suffix>' -> (expert, projection, suffix); ValueError for anything else."""
    parts = name.rsplit(".", 3)
    if len(parts) < 3 or not parts[-3].isdigit() or parts[-2] not in _GROUP_OF:
        raise ValueError(f"unexpected expert tensor {name!r}")
    if parts[-1] not in SUFFIXES:
        raise ValueError(f"unknown suffix in expert tensor {name!r}")
    return int(parts[-3]), parts[-2], parts[-1]


class ExpertStore:
    """One MoE layer's expert tensors as they arrive, on the layer's device; load() is the layer's load_weights."""

    def __init__(self, layer, num_experts: int, device):
        self._layer = weakref.ref(layer)
        self.num_experts, self.device = num_experts, device
        self.tensors: dict[tuple[int, str], dict[str, torch.Tensor]] = {}

    @property
    def layer_name(self) -> str:
        return getattr(self._layer(), "layer_name", "?")

    def load(self, weights):
        for name, tensor in weights:
            try:
                expert, proj, suffix = split_expert_name(name)
            except ValueError as err:
                raise ValueError(f"{self.layer_name}: {err}") from None
            self.tensors.setdefault((expert, proj), {})[suffix] = tensor.to(self.device).clone()
            yield f"{_GROUP_OF[proj]}_{suffix}"

    def experts(self) -> list[tuple[EspMatrix, EspMatrix, EspMatrix]]:
        """(gate, up, down) of every expert, in id order; RuntimeError if any matrix never arrived."""
        absent = [(e, p) for e in range(self.num_experts) for p in _PROJECTIONS if (e, p) not in self.tensors]
        if absent:
            raise RuntimeError(f"{self.layer_name}: {len(absent)} expert matrices missing, first {absent[:3]}")
        return [tuple(EspMatrix(self.tensors[(e, p)]) for p in _PROJECTIONS) for e in range(self.num_experts)]


class HiddenStatesGate(torch.nn.Module):
    """Takes the runner's router gate's place under ROUTE: returns the hidden states unchanged as the "logits", so the
    router GEMV runs inside the routing launch. The replaced gate and its weight stay reachable."""

    def __init__(self, replaced: torch.nn.Module):
        super().__init__()
        self.replaced = replaced
        self.weight = replaced.weight

    def forward(self, hidden_states):
        return hidden_states, None


@dataclass
class MoEState:
    """What the method keeps on a layer (layer.espalier) once its weights are loaded."""
    experts: list
    tables: grouped.Layer | None = None        # built on the first grouped call, once the shared expert is known
    shares_input: bool = False                 # the runner hands the routed and shared experts the same input
    router_weight: torch.Tensor | None = None  # the runner's gate weight, once ROUTE has taken the gate over


def runner_of(layer):
    """The layer's MoE runner: vLLM's, from its forward context; a stand-in layer carries its own."""
    if HAVE_VLLM:
        from vllm.forward_context import get_forward_context
        return get_forward_context().no_compile_layers[layer.layer_name]
    return layer.espalier_runner


def shared_trellis(shared_experts):
    """((gate, up, down) EspMatrix, sigmoid-gate weight [1, D]) of vLLM's shared-expert MLP when it can be a slot of
    the grouped launches (trellis-coded gate_up and down, one-output expert gate), else None."""
    mlp = getattr(shared_experts, "_layer", None)
    gate_up = getattr(getattr(mlp, "gate_up_proj", None), "espalier", None)
    down = getattr(getattr(mlp, "down_proj", None), "espalier", None)
    expert_gate = getattr(mlp, "expert_gate", None)
    if gate_up is None or down is None or expert_gate is None:
        return None
    if len(gate_up.mats) != 2 or len(down.mats) != 1 or expert_gate.weight.shape[0] != 1:
        return None
    return (*gate_up.mats, down.mats[0]), expert_gate.weight.detach()


def run_grouped(L: grouped.Layer, x: torch.Tensor, pick, wts, k: int, router_weight=None):
    """The grouped kernels over x's rows: (routed sum, shared output or None). pick / wts are vLLM's top-k (int32,
    fp32), or None with router_weight given, when the plugin routes."""
    T = x.shape[0]
    slots = k + (L.shared_id >= 0)
    if T <= GROUPED_ROWS:
        s = grouped.scratch(L, GROUPED_ROWS, slots, x.device)
        if pick is None:
            grouped.route(x, router_weight, k, L, s)
        return grouped.routed2(x, pick, wts, L, s, k=k)
    if prefill_mode() == "tile":
        return grouped.prefill(x, pick, wts, L, grouped.prefill_scratch(L, min(T, grouped.PREFILL_MAX_ROWS), slots,
                                                                        x.device), k, gate=router_weight)
    return grouped.windows(x, pick, wts, L, grouped.scratch(L, GROUPED_ROWS, slots, x.device), k=k,
                           gate=router_weight)


def expert_loop(experts, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor) -> torch.Tensor:
    """The MoE without the grouped kernels: the picks sorted by expert, each picked expert's rows through its gate,
    up and down matrices (espalier::matmul), weighted and summed in fp32 in expert order."""
    T, k = topk_ids.shape
    flat = topk_ids.reshape(-1).long()
    order = torch.argsort(flat, stable=True)
    ids, counts = torch.unique_consecutive(flat[order], return_counts=True)
    rows = order // k
    weights = topk_weights.reshape(-1).float()[order]
    acc = torch.zeros(x.shape, dtype=torch.float32, device=x.device)
    start = 0
    for e, n in zip(ids.tolist(), counts.tolist()):
        seg = slice(start, start + n)
        start += n
        gate, up, down = experts[e]
        xr = x[rows[seg]]
        act = F.silu(gate.forward(xr).float()) * up.forward(xr).float()
        acc.index_add_(0, rows[seg], down.forward(act.to(x.dtype)).float() * weights[seg, None])
    return acc.to(x.dtype)


def prefill_mode() -> str:
    from . import ops
    return ops.PREFILL


def _grouped_fits(T: int) -> bool:
    return GROUPED and (T <= GROUPED_ROWS or prefill_mode() in ("chunk", "tile"))


class EspMoEMethod(_Base):
    def __init__(self, moe_config=None):
        if HAVE_VLLM:
            super().__init__(moe_config)
        self.moe_config = moe_config

    @property
    def topk_indices_dtype(self):
        return torch.int32                     # the grouping reads int32 picks: no cast kernels around the layer

    @property
    def is_monolithic(self) -> bool:
        return ROUTE

    @property
    def mk_can_overlap_shared_experts(self) -> bool:
        return GROUPED                         # the shared expert runs as a slot of the grouped launches

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition, params_dtype,
                       **extra_weight_attrs):
        single_process()
        for group in sorted(set(_GROUP_OF.values())):
            for suffix in SUFFIXES:
                layer.register_parameter(f"{group}_{suffix}", torch.nn.Parameter(torch.empty(0), requires_grad=False))
        store = ExpertStore(layer, num_experts, layer.w13_esp_trellis.device)
        layer.espalier_store = store
        layer.load_weights = store.load

    def process_weights_after_loading(self, layer) -> None:
        store = layer.espalier_store
        activation = str(getattr(layer, "activation", "silu")).lower()
        if "silu" not in activation:
            raise NotImplementedError(f"{store.layer_name}: activation {activation} (the kernels run SwiGLU)")
        layer.espalier = MoEState(store.experts())
        store.tensors.clear()                  # the matrices hold the tensors now

    def get_fused_moe_quant_config(self, layer):
        return None

    # ---- running
    @staticmethod
    def _tables(layer, shared_experts) -> tuple[grouped.Layer, bool]:
        """The layer's grouped tables and whether the shared expert is a slot of them for this call (shared_experts
        is None when vLLM does not hand it to the method)."""
        state: MoEState = layer.espalier
        if state.tables is None:
            try:
                state.shares_input = getattr(runner_of(layer), "routed_input_transform", "absent") is None
            except Exception:
                state.shares_input = False
            slot = shared_trellis(shared_experts) if shared_experts is not None and state.shares_input else None
            state.tables = grouped.prepare(state.experts, *(slot or (None, None)))
        return state.tables, shared_experts is not None and state.shares_input and state.tables.shared_id >= 0

    def _grouped(self, layer, x, pick, wts, k, shared_experts, shared_input, router_weight=None):
        handed = shared_experts is not None and \
            shared_experts._determine_shared_experts_order(shared_input) == _INTERNAL
        L, folded = self._tables(layer, shared_experts if handed else None)
        out, shared_out = run_grouped(L, x.contiguous(), pick, wts, k, router_weight)
        if folded:
            shared_experts._output[shared_experts._output_idx] = shared_out
        elif handed:
            shared_experts.forward(shared_input, _INTERNAL)
        return out

    def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None, shared_experts_input=None):
        if _grouped_fits(topk_ids.shape[0]):
            return self._grouped(layer, x, topk_ids.to(torch.int32).contiguous(), topk_weights.float().contiguous(),
                                 topk_ids.shape[1], shared_experts, shared_experts_input)
        if shared_experts is not None and \
                shared_experts._determine_shared_experts_order(shared_experts_input) == _INTERNAL:
            shared_experts.forward(shared_experts_input, _INTERNAL)
        return expert_loop(layer.espalier.experts, x, topk_weights, topk_ids)

    def apply_monolithic(self, layer, x, router_logits, input_ids=None):
        runner = runner_of(layer)
        state: MoEState = layer.espalier
        took_over_now = state.router_weight is None
        if took_over_now:
            router = runner.router
            if not getattr(router, "renormalize", True) or getattr(router, "scoring_func", "softmax") != "softmax":
                raise NotImplementedError("the fused routing implements softmax top-k with renormalisation only")
            state.router_weight = runner.gate.weight.detach()
            runner.gate = HiddenStatesGate(runner.gate)
        # the call that took the gate over was handed the replaced gate's logits; later calls get hidden states
        real_logits = took_over_now or router_logits.shape[-1] != x.shape[-1]
        k = getattr(runner.router, "top_k", None) or layer.top_k
        shared = runner._shared_experts
        if not real_logits and _grouped_fits(x.shape[0]):
            return self._grouped(layer, x, None, None, k, shared, x, router_weight=state.router_weight)
        logits = router_logits if real_logits else F.linear(x, state.router_weight)
        topk_weights, topk_ids = runner.router.select_experts(hidden_states=x, router_logits=logits,
                                                              topk_indices_dtype=self.topk_indices_dtype,
                                                              input_ids=input_ids)
        return self.apply(layer, x, topk_weights, topk_ids, shared, x)

"""The vLLM linear method for trellis-coded dense layers and the LM head (the interface of vllm_espalier/linear.py:
EspLinearMethod, shard_order, single_process, DENSE).

A vLLM layer can fuse several checkpoint matrices (q/k/v, gate/up, in_proj_qkv/z); each keeps its own suh / svh, so
they are never concatenated into one trellis. The layer holds one EspMatrix per shard, in vLLM's shard order, and
concatenates their outputs. Shapes are only known once the checkpoint's tensors arrive, so create_weights registers
empty placeholder parameters whose loader keeps each tensor by (shard, suffix).

With DENSE (default; ESPALIER_FUSED_DENSE=0 turns it off) the whole layer is one espalier::dense call: at most 32 rows
a launch of esp_dense for all its matrices, rows beyond that as ESPALIER_PREFILL_MODE says (ops.py); else each
matrix through espalier::matmul.

vLLM is optional: with it, the method derives from vLLM's LinearMethodBase and checks the tensor-parallel size; the
same code runs on stand-in layers without it.
"""
from __future__ import annotations

import weakref

import torch
import torch.nn.functional as F
from torch.nn import Parameter

from ._env import env
from .matrix import SUFFIXES, EspMatrix

try:
    from vllm.model_executor.layers.linear import LinearMethodBase as _Base
    HAVE_VLLM = True
except ImportError:
    _Base = object
    HAVE_VLLM = False

DENSE = env("ESPALIER_FUSED_DENSE", "1") != "0"
_QKV_ORDER = {"q": 0, "k": 1, "v": 2}


def shard_order(shard) -> int:
    """Sort key of a loaded shard id: None (an unfused layer), "q" / "k" / "v", an int, or a tuple / list of ints
    (a merged shard, placed by its first index) (linear.py:27-34)."""
    if shard is None:
        return 0
    if isinstance(shard, str):
        return _QKV_ORDER[shard]
    if isinstance(shard, (tuple, list)):
        return min(shard)
    return int(shard)


def single_process() -> None:
    """The kernels serve one GPU's whole layer (tensor-parallel size 1, linear.py:37-41)."""
    if not HAVE_VLLM:
        return
    from vllm.distributed import get_tensor_model_parallel_world_size
    if get_tensor_model_parallel_world_size() != 1:
        raise NotImplementedError("vllm_espalier runs at tensor-parallel size 1")


class EspLinearMethod(_Base):
    def __init__(self, prefix: str):
        self.prefix = prefix

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size, output_size,
                       params_dtype, **extra_weight_attrs):
        single_process()
        layer._esp_parts = {}                       # shard -> {suffix: tensor}
        layer._esp_in = input_size_per_partition
        layer._esp_out = sum(output_partition_sizes)

        def weight_loader(param, loaded_weight, shard_id=None, *args, **kwargs):
            shard = getattr(loaded_weight, "shard_id", shard_id)
            if isinstance(shard, list):
                shard = tuple(shard)
            layer._esp_parts.setdefault(shard, {})[param._esp_suffix] = loaded_weight.to(param.device).clone()

        for suffix in SUFFIXES:
            p = Parameter(torch.empty(0), requires_grad=False)
            p._esp_suffix = suffix
            p.weight_loader = weight_loader
            layer.register_parameter(suffix, p)

    def process_weights_after_loading(self, layer) -> None:
        if not layer._esp_parts:
            if self.prefix.endswith("lm_head"):
                # a drafter's own head, never loaded (the target's replaces it)
                layer._esp_mats, layer._esp_dense, layer._esp_pad = [], None, 0
                return
            raise RuntimeError(f"{self.prefix}: no trellis-coded tensors were loaded")
        shards = sorted(layer._esp_parts.items(), key=lambda kv: shard_order(kv[0]))
        layer._esp_mats = [EspMatrix(tensors) for _, tensors in shards]
        del layer._esp_parts
        # module buffers, so a compiled graph receives the packed tensors as inputs
        for i, m in enumerate(layer._esp_mats):
            layer.register_buffer(f"_esp_t{i}", m.trellis, persistent=False)
            layer.register_buffer(f"_esp_s{i}", m.suh, persistent=False)
            layer.register_buffer(f"_esp_v{i}", m.svh, persistent=False)
        widths = {m.in_features for m in layer._esp_mats}
        n = sum(m.out_features for m in layer._esp_mats)
        if widths != {layer._esp_in} or n > layer._esp_out:
            raise RuntimeError(f"{self.prefix}: matrices of input widths {sorted(widths)} and {n} outputs do not "
                               f"fit the layer ({layer._esp_in} in, {layer._esp_out} out)")
        layer._esp_pad = layer._esp_out - n        # the LM head's vocabulary padding
        layer._esp_dense = None
        if DENSE and all(m.in_features % 128 == 0 and m.out_features % 128 == 0 for m in layer._esp_mats):
            from . import dense, ops
            key = next(ops.DENSE_KEYS)
            ops.DENSE_LAYERS[key] = dense.Dense(layer._esp_mats, layer._esp_out)
            layer._esp_dense = key
            # a layer vLLM drops after loading (a drafter's own head) leaves the registry with it
            weakref.finalize(layer, ops.DENSE_LAYERS.pop, key, None)

    def _tensors(self, layer, i: int):
        return getattr(layer, f"_esp_t{i}"), getattr(layer, f"_esp_s{i}"), getattr(layer, f"_esp_v{i}")

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        from . import ops  # noqa: F401  (registers the custom ops)
        n = len(layer._esp_mats)
        if layer._esp_dense is not None:
            lead = x.shape[:-1]
            ts = [self._tensors(layer, i) for i in range(n)]
            y = torch.ops.espalier.dense(x.reshape(-1, x.shape[-1]), [t[0] for t in ts], [t[1] for t in ts],
                                         [t[2] for t in ts], layer._esp_dense)
            y = y.reshape(*lead, y.shape[-1])
        else:
            parts = [m.forward_with(x, *self._tensors(layer, i)) for i, m in enumerate(layer._esp_mats)]
            y = parts[0] if n == 1 else torch.cat(parts, dim=-1)
            if layer._esp_pad:
                y = F.pad(y, (0, layer._esp_pad))
        return y + bias if bias is not None else y

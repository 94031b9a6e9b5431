"""The vLLM linear method for trellis-coded dense layers and the LM head: EspLinearMethod, written against vLLM's
LinearMethodBase contract (create_weights / process_weights_after_loading / apply), with the switch DENSE
(ESPALIER_FUSED_DENSE) and the helpers shard_order and single_process of the plugin's interface (the reference's
vllm_espalier/linear.py:27-41).

How a layer is held here:
  * create_weights gives the layer one empty placeholder parameter per checkpoint suffix (esp_trellis, suh, svh, ...:
    vLLM's loader finds parameters by these names), each with a ShardCollector as its weight_loader. Matrix shapes
    are only known once the tensors arrive, and a fused layer (q/k/v, gate/up, ...) receives one tensor per suffix
    per shard, so the collector files every tensor under its shard.
  * process_weights_after_loading turns the collection into a TrellisLinear child module, `layer.espalier`: the
    shards' EspMatrix objects in vLLM's output order, their tensors as non-persistent buffers (a compiled graph then
    takes them as inputs rather than constants), and the output padding (a vocabulary padded past the matrix).
    Each shard keeps its own suh / svh, so the matrices are never concatenated into one trellis.
  * apply runs layer.espalier: with DENSE the whole layer is one espalier::dense call (one esp_dense launch for all
    its matrices up to 32 rows, more rows as ESPALIER_PREFILL_MODE says); without it each matrix goes through
    espalier::matmul and the outputs are joined.

vLLM is optional: with it the method derives from LinearMethodBase and checks the tensor-parallel size; without it
the same code runs on stand-in layers.
"""
from __future__ import annotations

import weakref

import torch

from ._env import env
from .matrix import SUFFIXES, EspMatrix

try:
    from vllm.model_executor.layers.linear import LinearMethodBase as _Base
    HAVE_VLLM = True
except ImportError:
    _Base = object
    HAVE_VLLM = False

DENSE = env("ESPALIER_FUSED_DENSE", "1") != "0"
_NAMED_SHARDS = {None: 0, "q": 0, "k": 1, "v": 2}


def shard_order(shard) -> int:
    """Where a loaded shard goes in the layer's output: an unfused layer's single shard (None) first, q / k / v in
    that order, an integer shard at its index, a merged shard (tuple or list of indices) at its first index."""
    if isinstance(shard, (tuple, list)):
        return min(int(s) for s in shard)
    if shard is None or isinstance(shard, str):
        return _NAMED_SHARDS[shard]
    return int(shard)


def single_process() -> None:
    """The kernels serve one GPU's whole layer: refuse a tensor-parallel size other than 1 (a no-op without vLLM)."""
    if HAVE_VLLM:
        from vllm.distributed import get_tensor_model_parallel_world_size
        size = get_tensor_model_parallel_world_size()
        if size != 1:
            raise NotImplementedError(f"vllm_espalier serves a layer on one GPU; tensor-parallel size is {size}")


class ShardCollector:
    """The weight_loader of every placeholder parameter of one layer: files each arriving tensor under (shard,
    suffix), a copy on the placeholder's device. vLLM passes the shard as an argument or, for some loaders, as an
    attribute of the tensor; a list-valued shard (a merged one) is kept as a tuple."""

    def __init__(self):
        self.shards: dict = {}

    def __call__(self, param, loaded_weight, shard_id=None, *args, **kwargs):
        shard = getattr(loaded_weight, "shard_id", shard_id)
        key = tuple(shard) if isinstance(shard, list) else shard
        self.shards.setdefault(key, {})[param.esp_suffix] = loaded_weight.to(param.device).clone()

    def matrices(self) -> list[EspMatrix]:
        """The collected shards as matrices, in the layer's output order."""
        return [EspMatrix(self.shards[s]) for s in sorted(self.shards, key=shard_order)]


class TrellisLinear(torch.nn.Module):
    """The trellis-coded matrices of one vLLM linear layer, ready to run.

    Its buffers (trellis_i, suh_i, svh_i for shard i) are what the custom ops receive, so under torch.compile they
    are graph inputs. With a dense key, forward is one espalier::dense call over all shards (registered in
    ops.DENSE_LAYERS and dropped from it with this module); otherwise each shard goes through espalier::matmul."""

    def __init__(self, mats: list[EspMatrix], out_features: int, fused: bool):
        super().__init__()
        self.mats = mats
        self.out_features = out_features
        self.pad = out_features - sum(m.out_features for m in mats)
        for i, m in enumerate(mats):
            self.register_buffer(f"trellis_{i}", m.trellis, persistent=False)
            self.register_buffer(f"suh_{i}", m.suh, persistent=False)
            self.register_buffer(f"svh_{i}", m.svh, persistent=False)
        self.dense_key = None
        if fused and mats and all(m.in_features % 128 == 0 and m.out_features % 128 == 0 for m in mats):
            from . import dense, ops
            self.dense_key = next(ops.DENSE_KEYS)
            ops.DENSE_LAYERS[self.dense_key] = dense.Dense(mats, out_features)
            weakref.finalize(self, ops.DENSE_LAYERS.pop, self.dense_key, None)

    def tensors(self, name: str) -> list[torch.Tensor]:
        return [getattr(self, f"{name}_{i}") for i in range(len(self.mats))]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from . import ops  # noqa: F401  (registers the espalier::* ops)
        if not self.mats:
            raise RuntimeError("this layer's matrices were never loaded (a drafter's head, replaced by the target's)")
        trellis, suh, svh = self.tensors("trellis"), self.tensors("suh"), self.tensors("svh")
        if self.dense_key is not None:
            rows = x.reshape(-1, x.shape[-1])
            y = torch.ops.espalier.dense(rows, trellis, suh, svh, self.dense_key)
            return y.reshape(*x.shape[:-1], self.out_features)
        outs = [m.forward_with(x, t, s, v) for m, t, s, v in zip(self.mats, trellis, suh, svh)]
        if self.pad:
            outs.append(x.new_zeros((*x.shape[:-1], self.pad)))
        return torch.cat(outs, dim=-1) if len(outs) > 1 else outs[0]


class EspLinearMethod(_Base):
    def __init__(self, prefix: str):
        self.prefix = prefix

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size, output_size,
                       params_dtype, **extra_weight_attrs):
        single_process()
        collector = ShardCollector()
        layer.espalier_shape = (input_size_per_partition, sum(output_partition_sizes))
        layer.espalier_collector = collector
        for suffix in SUFFIXES:
            placeholder = torch.nn.Parameter(torch.empty(0), requires_grad=False)
            placeholder.esp_suffix = suffix
            placeholder.weight_loader = collector
            layer.register_parameter(suffix, placeholder)

    def process_weights_after_loading(self, layer) -> None:
        collector = layer.espalier_collector
        del layer.espalier_collector
        k_in, n_out = layer.espalier_shape
        if not collector.shards:
            # an MTP drafter's own LM head is never loaded: vLLM installs the target's head in its place
            if not self.prefix.endswith("lm_head"):
                raise RuntimeError(f"{self.prefix}: no trellis-coded tensors were loaded")
            layer.espalier = TrellisLinear([], n_out, fused=False)
            return
        mats = collector.matrices()
        widths = sorted({m.in_features for m in mats})
        total = sum(m.out_features for m in mats)
        if widths != [k_in] or total > n_out:
            raise RuntimeError(f"{self.prefix}: matrices of input widths {widths} and {total} outputs do not fit "
                               f"the layer ({k_in} in, {n_out} out)")
        layer.espalier = TrellisLinear(mats, n_out, fused=DENSE)

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        y = layer.espalier(x)
        return y if bias is None else y + bias

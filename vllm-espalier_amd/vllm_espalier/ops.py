"""The plugin's torch custom ops (the interface of vllm_espalier/ops.py): opaque to torch.compile and safe under
HIP-graph capture, since nothing in them allocates from the host's point of view beyond the output.

espalier::matmul(x, trellis, suh, svh, K, cb) -> fp16 [m, out]
    one trellis matrix, x fp16 [m, in] contiguous; K is the bit width, cb the checkpoint grid code.
espalier::dense(x, trellis[], suh[], svh[], key) -> [m, n_out] in x's dtype
    every matrix of one vLLM layer, the Dense registered under `key` in DENSE_LAYERS.

Rows beyond one launch (prefill) follow ESPALIER_PREFILL_MODE:
    chunk  (default) the decode kernels over windows of MAX_ROWS rows, so a row gets exactly its decode bits;
    gemm   each matrix decoded once (dequant kernel), both Hadamards by the had kernel, and an fp16 matmul
           (hipBLASLt) between them. A layer of HUGE weights or more (the LM head) stays windowed: its decoded weight
           would not fit beside the model;
    tile   the prompt launch (esp_dense_tile): every weight decoded once for each 128 rows, inside the GEMM; a row's
           bits are its own (the same for any prompt), not its decode bits. No counterpart in the reference.
The fake implementations give only the output shapes.
"""
from __future__ import annotations

import itertools

import torch

from ._env import env

PREFILL_MODES = ("chunk", "gemm", "tile")
PREFILL = env("ESPALIER_PREFILL_MODE", "chunk")
if PREFILL not in PREFILL_MODES:
    raise ValueError(f"ESPALIER_PREFILL_MODE={PREFILL}: expected one of {PREFILL_MODES}")

DENSE_LAYERS: dict = {}       # key -> dense.Dense, filled by the linear method
DENSE_KEYS = itertools.count()
HUGE = 1 << 28                 # K * N at or above which a layer is never decoded whole
_SINGLE: dict = {}             # trellis address -> a one-matrix dense.Dense for espalier::matmul


class _Single:
    """The fields dense.Dense reads from a matrix, for a matrix that reaches matmul as bare tensors."""

    def __init__(self, trellis, suh, svh, bits: int, grid: int):
        self.trellis, self.suh, self.svh = trellis, suh, svh
        self.K, self.cb = bits, grid
        self.in_features, self.out_features = suh.numel(), svh.numel()


def windowed(layer, x: torch.Tensor, *tensors) -> torch.Tensor:
    """layer.forward over consecutive windows of layer.MAX_ROWS rows of x, into one output."""
    step = layer.MAX_ROWS
    if x.shape[0] <= step:
        return layer.forward(x, *tensors)
    y = x.new_empty((x.shape[0], layer.n_out))
    for r0 in range(0, x.shape[0], step):
        rows = slice(r0, r0 + step)
        layer.forward(x[rows], *tensors, out=y[rows])
    return y


def _decoded_matmul(x: torch.Tensor, trellis, suh, svh, bits: int, grid: int) -> torch.Tensor:
    """The gemm prefill path of one matrix: W decoded, x rotated by H(x * suh), the fp16 product, then H(.) * svh."""
    from . import experts
    e = experts.ext()
    w = experts.dequant(trellis, bits, grid)
    rotated = torch.empty_like(x)
    e.had(x, suh, None, rotated)
    y = rotated @ w
    e.had(y, None, svh, y)
    return y


def _single(trellis, suh, svh, bits: int, grid: int):
    from . import dense
    layer = _SINGLE.get(trellis.data_ptr())
    if layer is None:
        layer = _SINGLE[trellis.data_ptr()] = dense.Dense([_Single(trellis, suh, svh, bits, grid)])
    return layer


@torch.library.custom_op("espalier::matmul", mutates_args=())
def matmul(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
           K: int, cb: int) -> torch.Tensor:
    from .dense import MAX_ROWS
    if PREFILL == "gemm" and x.shape[0] > MAX_ROWS:
        return _decoded_matmul(x, trellis, suh, svh, K, cb)
    layer = _single(trellis, suh, svh, K, cb)
    if PREFILL == "tile" and x.shape[0] > MAX_ROWS and _tileable(layer):
        return layer.forward_tile(x)
    return windowed(layer, x)


def _tileable(layer) -> bool:
    """Whether a layer runs as prompt launches: 128-wide input and output blocks."""
    return layer.K % 128 == 0 and all(m.out_features % 128 == 0 for m in layer.mats)


@torch.library.custom_op("espalier::dense", mutates_args=())
def dense(x: torch.Tensor, trellis: list[torch.Tensor], suh: list[torch.Tensor], svh: list[torch.Tensor],
          key: int) -> torch.Tensor:
    layer = DENSE_LAYERS[key]
    if PREFILL == "tile" and x.shape[0] > layer.MAX_ROWS:
        return layer.forward_tile(x.contiguous(), trellis, suh, svh)
    decode_whole = PREFILL == "gemm" and x.shape[0] > layer.MAX_ROWS and layer.K * layer.N < HUGE
    if not decode_whole:
        return windowed(layer, x.contiguous(), trellis, suh, svh)
    x16 = x.to(torch.float16).contiguous()
    parts = [matmul(x16, t, s, v, m.K, m.cb) for t, s, v, m in zip(trellis, suh, svh, layer.mats)]
    y = torch.cat(parts, dim=-1) if len(parts) > 1 else parts[0]
    y = y.to(x.dtype)
    if layer.n_out > layer.N:
        y = torch.nn.functional.pad(y, (0, layer.n_out - layer.N))
    return y


@matmul.register_fake
def _matmul_shape(x, trellis, suh, svh, K, cb):
    return x.new_empty((x.shape[0], svh.shape[0]), dtype=torch.float16)


@dense.register_fake
def _dense_shape(x, trellis, suh, svh, key):
    return x.new_empty((x.shape[0], DENSE_LAYERS[key].n_out))

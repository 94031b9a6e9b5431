"""EspMatrix: one trellis-coded weight matrix as the checkpoint stores it (the interface of vllm_espalier/matrix.py).

A matrix arrives as tensors named by suffix:
    esp_trellis  int16 [in/16, out/16, 16 * bits]   the 16x16 tiles' code words
    suh          fp16 [in]                          input signs / scales
    svh          fp16 [out]                         output signs / scales
    mcg          marker (required)
    mul1         marker (optional): the E2M1 grid when no esp_grid is given
    esp_grid     int32 code: 1 E2M1, 2 E4M3, 3 int5, 4 int6
The grid code (`cb`) is esp_grid's value, else 1 with mul1, else 0 (the plain mcg codebook).

y = H(H(x * suh) @ W) * svh, H the 128-wide normalised Walsh-Hadamard transform along rows, W decoded from the tiles;
forward() runs it through the espalier::matmul custom op.
"""
from __future__ import annotations

import torch

SUFFIXES = ("esp_trellis", "suh", "svh", "mcg", "mul1", "esp_grid")
_REQUIRED = SUFFIXES[:4]
GRID_CODES = (1, 2, 3, 4)             # esp_grid values a checkpoint may carry


def grid_code(tensors: dict) -> int:
    """The matrix's grid code from its marker tensors."""
    if "esp_grid" not in tensors:
        return 1 if "mul1" in tensors else 0
    code = int(tensors["esp_grid"].reshape(-1)[0].item())
    if code not in GRID_CODES:
        raise ValueError(f"esp_grid code {code} is not one of {GRID_CODES}")
    return code


class EspMatrix:
    def __init__(self, tensors: dict[str, torch.Tensor]):
        absent = [name for name in _REQUIRED if name not in tensors]
        if absent:
            raise ValueError(f"Espalier matrix is missing {absent}")
        codes = tensors["esp_trellis"]
        if codes.dtype != torch.int16 or codes.dim() != 3:
            raise ValueError(f"esp_trellis must be int16 [in/16, out/16, 16 * bits], got {codes.dtype} "
                             f"{tuple(codes.shape)}")
        self.trellis = codes.contiguous()
        self.suh = tensors["suh"].to(torch.float16).contiguous()
        self.svh = tensors["svh"].to(torch.float16).contiguous()
        self.in_features, self.out_features = self.suh.numel(), self.svh.numel()
        k_tiles, n_tiles, words = self.trellis.shape
        if (16 * k_tiles, 16 * n_tiles) != (self.in_features, self.out_features):
            raise ValueError(f"trellis {tuple(self.trellis.shape)} does not match in {self.in_features}, "
                             f"out {self.out_features}")
        self.K = words // 16                  # bits per weight
        self.cb = grid_code(tensors)

    def to(self, device):
        self.trellis = self.trellis.to(device)
        self.suh = self.suh.to(device)
        self.svh = self.svh.to(device)
        return self

    def weight(self) -> torch.Tensor:
        """The decoded W [in, out] fp16 (before either Hadamard), from the dequantisation kernel."""
        from .experts import dequant
        return dequant(self.trellis, self.K, self.cb)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x [..., in] in any float dtype -> [..., out] in x's dtype."""
        return self.forward_with(x, self.trellis, self.suh, self.svh)

    def forward_with(self, x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor) -> torch.Tensor:
        """forward() with the tensors passed in, as a compiled graph hands over module buffers."""
        from . import ops  # noqa: F401  (registers espalier::matmul)
        lead = x.shape[:-1]
        rows = x.reshape(-1, self.in_features).to(torch.float16).contiguous()
        y = torch.ops.espalier.matmul(rows, trellis, suh, svh, self.K, self.cb)
        return y.reshape(*lead, self.out_features).to(x.dtype)

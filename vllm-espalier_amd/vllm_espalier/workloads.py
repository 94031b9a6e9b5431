"""Synthetic Espalier layers for benchmarks and tests: random trellis codes of the checkpoint format, seeded.

Generator (one torch.Generator per call, on the CPU, so the bytes do not depend on the device):
  trellis  uniform 16-bit words, int16 [K/16, N/16, 16 * bits] (uniform random states per 16x16 tile)
  suh      random +-1, fp16 [K]
  svh      random +-1 times lognormal(0, 0.25), fp16 [N] (the per-output-channel scale)
Activations are N(0, 1) cast to the model dtype by the caller.
"""
from __future__ import annotations

import torch

from .matrix import EspMatrix

# checkpoint grid codes (EspMatrix.cb): 0 mcg, 1 E2M1, 3 int5, 4 int6
GRID = {"mcg": 0, "e2m1": 1, "int5": 3, "int6": 4}


def matrix_tensors(K: int, N: int, bits: int, grid: str, gen: torch.Generator) -> dict[str, torch.Tensor]:
    """The tensors on gen's device (a CPU generator gives device-independent bytes; a device generator is fast for
    the benchmarks' gigabyte weight stacks)."""
    if K % 16 or N % 16:
        raise ValueError("K and N must be multiples of 16")
    dev = gen.device
    t = torch.randint(-32768, 32768, (K // 16, N // 16, 16 * bits), dtype=torch.int32, generator=gen, device=dev)
    trellis = t.to(torch.int16)
    suh = (torch.randint(0, 2, (K,), generator=gen, device=dev) * 2 - 1).to(torch.float16)
    sign = (torch.randint(0, 2, (N,), generator=gen, device=dev) * 2 - 1).to(torch.float32)
    scale = torch.exp(torch.randn((N,), generator=gen, device=dev) * 0.25)
    svh = (sign * scale).to(torch.float16)
    d = {"esp_trellis": trellis, "suh": suh, "svh": svh, "mcg": torch.zeros(1, dtype=torch.int32, device=dev)}
    code = GRID[grid]
    if code:
        d["esp_grid"] = torch.tensor([code], dtype=torch.int32, device=dev)
    return d


def matrix(K: int, N: int, bits: int, grid: str, gen: torch.Generator, device) -> EspMatrix:
    return EspMatrix({k: v.to(device) for k, v in matrix_tensors(K, N, bits, grid, gen).items()})


def nbytes(mats) -> int:
    """Algorithmic bytes of matrices: trellis + suh + svh."""
    return sum(m.trellis.numel() * 2 + (m.suh.numel() + m.svh.numel()) * 2 for m in mats)

"""The HIP kernels against the committed golden fixtures (tests/golden/oracle_vectors.npz), bit for bit: the same
vectors the CPU oracle is held to in test_golden.py."""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
G = np.load(Path(__file__).resolve().parent / "golden" / "oracle_vectors.npz")


def t16(a: np.ndarray, dtype=torch.int16) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("cb,k2", sorted(O.COMPILED))
def test_golden_dequant(dev, ext, cb, k2):
    tr = torch.from_numpy(G[f"dequant_cb{cb}_k{k2}_trellis"]).to(dev)
    out = torch.empty((tr.shape[0] * 16, tr.shape[1] * 16), dtype=torch.float16, device=dev)
    ext.dequant(tr, out, k2, cb)
    assert np.array_equal(bits(out), G[f"dequant_cb{cb}_k{k2}_w"])


def test_golden_had(dev, ext):
    x = t16(G["had_x"], torch.float16).to(dev)
    y = torch.empty_like(x)
    ext.had(x, t16(G["had_pre"], torch.float16).to(dev), t16(G["had_post"], torch.float16).to(dev), y)
    assert np.array_equal(bits(y), G["had_out"])


def test_golden_route(dev, ext):
    x = t16(G["route_x"], torch.bfloat16).to(dev)
    gate = t16(G["route_gate"], torch.bfloat16).to(dev)
    sg = t16(G["route_sgate"], torch.bfloat16).to(dev)
    R, k, E = x.shape[0], 8, gate.shape[0]
    slots, C = k + 1, E + 1
    maxu = min(R * slots, C)
    logits = torch.zeros(R * C, dtype=torch.float32, device=dev)
    counter = torch.zeros(1, dtype=torch.int32, device=dev)
    pick = torch.zeros(R * slots, dtype=torch.int32, device=dev)
    wts = torch.zeros(R * slots, dtype=torch.float32, device=dev)
    uids = torch.zeros(maxu, dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    members = torch.full((maxu, R), -7, dtype=torch.int32, device=dev)
    ext.route_group(x, gate, sg, k, E, logits, counter, pick, wts, uids, count, members)
    torch.cuda.synchronize()
    assert np.array_equal(pick.view(R, slots).cpu().numpy(), G["route_pick"])
    assert np.array_equal(O.f32_to_bf16(logits.view(R, C)[:, :E].cpu().numpy()), G["route_logits"])
    assert np.abs(wts.view(R, slots).cpu().numpy().astype(np.float64) - G["route_wts"]).max() < 1e-6


def test_golden_group(dev, ext):
    pick = torch.from_numpy(G["group_pick"]).to(dev)
    uids = torch.full((10,), -7, dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    members = torch.full((10, 45), -7, dtype=torch.int32, device=dev)
    ext.group(pick, uids, count, members, 5, 9, 10)
    n = int(count.item())
    assert n == len(G["group_uids"])
    assert np.array_equal(uids[:n].cpu().numpy(), G["group_uids"])
    assert np.array_equal(members[:n].cpu().numpy(), G["group_members"])

"""Grouped routed experts: one MoE layer for up to ROWS tokens in six launches, whatever the experts' widths
(the surface of vllm_espalier/experts.py:1-268, over the gfx950 kernels of csrc/):

  group_shared / route_group   pick / weight tables with the shared expert as one more slot, then the grouping
                               (distinct experts in id order, member rows in pick order), all on the device
  rot_in                       H(x * suh) for gate and up of every slot, read straight from the model's bf16/fp16 x
  grouped (mats=2)             gate and up of all distinct experts in one launch, W decoded in registers
  gateup_epilogue              splits summed, H, * svh, SwiGLU in fp32, * suh_d, H -> the down input
  grouped (mats=1)             down
  down_combine2                splits summed, H, * svh_d, routing-weighted sum over the routed slots (slot order),
                               and the gated shared slot, both written in the model's dtype

Every sum runs in a fixed order, so a token's output never depends on the other tokens in the window, and nothing
allocates, so HIP graphs capture it. The trellises are read in place through pointer tables; suh/svh are stacked per
projection and each EspMatrix's suh/svh become views of the stacks.

The extension (espalier_ext, csrc/binding.cpp over libespalier_hip.so) is built in-tree by csrc/build.py;
ESPALIER_PREBUILT_EXTENSION points at a prebuilt espalier_ext .so instead.
"""
from __future__ import annotations

import importlib.machinery
import importlib.util
import math
import os
from dataclasses import dataclass, field
from functools import lru_cache
from pathlib import Path

import torch

from ._env import env

# Espalier grid code (EspMatrix.cb) -> the kernels' codebook id (exllamav3's: 1 mcg, 3 E2M1, 6 int5, 7 int6)
KERNEL_CB = {0: 1, 1: 3, 3: 6, 4: 7}
# (codebook id, half-bits) pairs with kernels (csrc/trellis.hpp ESP_CASES)
COMPILED = {(1, k2) for k2 in range(2, 17, 2)} | {(3, 2), (3, 4), (3, 6), (6, 4), (6, 6), (6, 8), (7, 6), (7, 8),
                                                   (7, 10)}
ACT_F32 = 1
# routed2 with rot_in, the gate/up GEMM and its epilogue in one launch (esp_moe_gateup) for windows of up to
# FUSED_ROWS rows: one launch less than two hand-offs cost (MI355X, 1 token: 2.2 us a layer less). Wider windows keep
# the reference's sequence, since each (expert, 128 columns) program rotates its rows again. Same bits either way.
# ESPALIER_MOE_FUSED=0 turns it off.
FUSED = env("ESPALIER_MOE_FUSED", "1") != "0"
FUSED_ROWS = 4
PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"


def _ext_path() -> Path | None:
    for p in sorted(PKG.glob("espalier_ext*.so")):
        return p
    return None


def _load(path: str):
    loader = importlib.machinery.ExtensionFileLoader("espalier_ext", path)
    spec = importlib.util.spec_from_loader("espalier_ext", loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    return mod


@lru_cache(1)
def ext():
    """The espalier_ext module. Raises when it cannot be found or built: there is no other implementation."""
    path = os.environ.get("ESPALIER_PREBUILT_EXTENSION")
    if path:
        return _load(path)
    p = _ext_path()
    if p is None or not (PKG / "libespalier_hip.so").exists():
        import subprocess
        import sys
        subprocess.run([sys.executable, str(CSRC / "build.py")], check=True)
        p = _ext_path()
    if p is None:
        raise RuntimeError("espalier_ext is not built (run vllm-espalier_amd/vllm_espalier/csrc/build.py)")
    return _load(str(p))


def tile_config(K: int, N: int, gateup: bool) -> tuple[int, int, int, int]:
    """(n tiles a block, waves a workgroup, K splits, tiles in flight) for a K -> N projection, from the shape alone so
    a row's bits never depend on the batch. A gfx950 workgroup is 4 * KW waves on 128 columns. From cold sweeps of
    the BASELINE MoE layer on MI355X (1 and 32 tokens): K splits of 256 (8 32-k steps a workgroup; 128 below K = 1024)
    and 4 waves. That keeps the handful of experts one token picks spread over the CUs and, at 32 tokens, beats 8
    waves by a fifth: the decode is VALU-bound, so more workgroups in flight win over fewer wider ones. The
    reference's sm89 choices are experts.py:59-68. ESPALIER_GROUPED_TILE_PLAN="w,sk" (both projections) or
    "w,sk;w,sk" (gate/up; down) forces."""
    if N % 128 or K % 32:
        raise ValueError(f"no tile setting divides K={K}, N={N}")
    forced = env("ESPALIER_GROUPED_TILE_PLAN")
    if forced:
        parts = forced.split(";")
        w, sk = (int(v) for v in parts[0 if gateup or len(parts) == 1 else 1].split(","))
        return 8, w, sk, 2
    min_kr = 256 if K >= 1024 else 128                   # 8 steps a workgroup, 4 for the narrow down projection
    sk = 1
    while K % (32 * sk * 2) == 0 and K // (sk * 2) >= min_kr:
        sk *= 2
    return 8, 4, sk, 2


@dataclass
class Layer:
    """One layer's routed experts as the kernels read them."""

    ptr: tuple            # int64 [E] trellis pointers: gate, up, down
    k2: tuple             # int32 [E] half-bits: gate, up, down
    cb: tuple             # int32 [E] kernel codebook ids: gate, up, down
    suh_g: torch.Tensor   # fp16 [E, D]
    suh_u: torch.Tensor
    svh_g: torch.Tensor   # fp16 [E, I]
    svh_u: torch.Tensor
    suh_d: torch.Tensor   # fp16 [E, I]
    svh_d: torch.Tensor   # fp16 [E, D]
    E: int                # matrices in the tables: routed experts, plus the shared expert at index E-1 if any
    D: int
    I: int
    k2_gu: tuple          # (min, max) over gate and up
    k2_d: tuple
    shared_id: int = -1   # index of the shared expert in the tables, -1 without one
    gate_w: torch.Tensor | None = None   # the shared expert's sigmoid-gate weight [D], the model's dtype
    keep: list = field(default_factory=list, repr=False)


def prepare(experts, shared=None, gate_w=None) -> Layer:
    """experts: [(gate, up, down) EspMatrix] in expert order; shared: the shared expert's (gate, up, down), appended as
    the last table entry, with gate_w its sigmoid-gate weight [D]. Rebinds each matrix's suh/svh to stack rows."""
    if shared is not None:
        experts = list(experts) + [tuple(shared)]
    E = len(experts)
    g0 = experts[0][0]
    D, I = g0.in_features, g0.out_features
    dev = g0.trellis.device

    def tables(j, k, n):
        ptrs, k2s, cbs = [], [], []
        for e, mats in enumerate(experts):
            m = mats[j]
            if (m.in_features, m.out_features) != (k, n):
                raise ValueError(f"expert {e} projection {j}: {m.in_features}x{m.out_features}, expected {k}x{n}")
            if m.cb not in KERNEL_CB:
                raise NotImplementedError(f"expert {e}: grid code {m.cb} has no grouped kernel")
            k2, cb = 2 * m.K, KERNEL_CB[m.cb]
            if (cb, k2) not in COMPILED:
                raise NotImplementedError(f"expert {e}: no grouped instance for codebook {cb} at {m.K} bits")
            if not (m.trellis.is_contiguous() and m.trellis.dtype == torch.int16):
                raise ValueError(f"expert {e} projection {j}: trellis must be contiguous int16")
            ptrs.append(m.trellis.data_ptr())
            k2s.append(k2)
            cbs.append(cb)
        return (torch.tensor(ptrs, dtype=torch.int64, device=dev), torch.tensor(k2s, dtype=torch.int32, device=dev),
                torch.tensor(cbs, dtype=torch.int32, device=dev), k2s)

    gp, gk, gc, gks = tables(0, D, I)
    up, uk, uc, uks = tables(1, D, I)
    dp, dk, dc, dks = tables(2, I, D)

    def stack(j, attr, n):
        out = torch.empty((E, n), dtype=torch.float16, device=dev)
        for e, mats in enumerate(experts):
            out[e].copy_(getattr(mats[j], attr).reshape(-1))
            setattr(mats[j], attr, out[e])
        return out

    return Layer((gp, up, dp), (gk, uk, dk), (gc, uc, dc), stack(0, "suh", D), stack(1, "suh", D),
                 stack(0, "svh", I), stack(1, "svh", I), stack(2, "suh", I), stack(2, "svh", D), E, D, I,
                 (min(gks + uks), max(gks + uks)), (min(dks), max(dks)),
                 E - 1 if shared is not None else -1,
                 None if gate_w is None else gate_w.reshape(-1).contiguous(),
                 [m.trellis for mats in experts for m in mats])


class Scratch:
    """Buffers for up to `rows` tokens of `slots` picks, shared by every layer of one shape (layers run in turn)."""

    def __init__(self, E: int, D: int, I: int, rows: int, slots: int, device):
        self.cfg_gu = tile_config(D, I, True)
        self.cfg_d = tile_config(I, D, False)
        P = rows * slots
        self.xg = torch.zeros((P, D), dtype=torch.float16, device=device)
        self.xu = torch.zeros((P, D), dtype=torch.float16, device=device)
        self.xd = torch.zeros((P, I), dtype=torch.float16, device=device)
        self.z = torch.zeros((max(2 * self.cfg_gu[2] * I, self.cfg_d[2] * D) * P,), dtype=torch.float32,
                             device=device)
        self.y = torch.zeros((P, D), dtype=torch.float32, device=device)
        self.route_counter = torch.zeros((1,), dtype=torch.int32, device=device)       # route_group's arrivals
        self.logits = torch.zeros((rows * E,), dtype=torch.float32, device=device)     # route_group's logits
        maxu = min(P, E)
        self.pick = torch.zeros((P,), dtype=torch.int32, device=device)      # with the shared slot
        self.wts = torch.zeros((P,), dtype=torch.float32, device=device)
        self.ids = torch.zeros((maxu,), dtype=torch.int32, device=device)
        self.count = torch.zeros((1,), dtype=torch.int32, device=device)
        self.members = torch.full((maxu * rows,), -1, dtype=torch.int32, device=device)
        # arrival counters of the fused gate/up launch, one per (expert, 128 columns), 32 ints apart, zero between
        # launches
        self.counters = torch.zeros((maxu * (I // 128) * 32,), dtype=torch.int32, device=device)
        self.rows, self.slots, self.E = rows, slots, E

    def window(self, R: int):
        maxu = min(R * self.slots, self.E)
        return self.ids[:maxu], self.members[:maxu * R].view(maxu, R)


_SCRATCH: dict = {}


def scratch(layer: Layer, rows: int, slots: int, device) -> Scratch:
    """slots counts the shared slot when the layer has one."""
    key = (layer.E, layer.D, layer.I, rows, slots, str(device))
    if key not in _SCRATCH:
        _SCRATCH[key] = Scratch(layer.E, layer.D, layer.I, rows, slots, device)
    return _SCRATCH[key]


def routed(x: torch.Tensor, pick: torch.Tensor, wts: torch.Tensor, L: Layer, s: Scratch,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """x [R, D] fp16/bf16, pick int32 [R, slots], wts fp32 [R, slots] -> fp32 [R, D], the weighted sum of the
    routed experts' outputs (picks outside [0, E) are skipped)."""
    e = ext()
    R, slots = pick.shape
    D, I, E = L.D, L.I, L.E
    P = R * slots
    if R > s.rows or slots != s.slots:
        raise ValueError(f"{R}x{slots} picks but the scratch holds {s.rows}x{s.slots}")
    ids, members = s.window(R)
    e.group(pick, ids, s.count, members, R, slots, E)
    e.rot_in(x, x.stride(0), pick, L.suh_g, L.suh_u, s.xg, s.xu, R, D, slots, E)
    nt, w, sk, pf = s.cfg_gu
    e.grouped(s.xg, s.xu, L.ptr[0], L.ptr[1], L.k2[0], L.k2[1], L.cb[0], L.cb[1], ids, s.count, members, s.z, 2,
              D, I, P, sk, slots, nt, w, pf, L.k2_gu[0], L.k2_gu[1])
    e.gateup_epilogue(s.z, pick, L.svh_g, L.svh_u, L.suh_d, s.xd, R, P, I, sk, slots, E, math.inf, ACT_F32)
    nt, w, sk, pf = s.cfg_d
    e.grouped(s.xd, s.xd, L.ptr[2], L.ptr[2], L.k2[2], L.k2[2], L.cb[2], L.cb[2], ids, s.count, members, s.z, 1,
              I, D, P, sk, slots, nt, w, pf, L.k2_d[0], L.k2_d[1])
    if out is None:
        out = torch.empty((R, D), dtype=torch.float32, device=x.device)
    e.down_combine(s.z, pick, L.svh_d, s.y, wts, out, R, P, D, sk, slots, E)
    return out


def route(x: torch.Tensor, gate: torch.Tensor, k: int, L: Layer, s: Scratch):
    """Router logits (x @ gate.T, plus the shared gate), softmax / top-k / renormalisation and grouping in one launch
    (csrc/moe.hip route_group), into the scratch's pick / wts / ids / count / members; then routed2(..., pick=None)."""
    R = x.shape[0]
    ids, members = s.window(R)
    ext().route_group(x, gate, L.gate_w, k, L.shared_id, s.logits, s.route_counter, s.pick[:R * s.slots],
                      s.wts[:R * s.slots], ids, s.count, members)


def route_rmsnorm(h: torch.Tensor, d1: torch.Tensor | None, norm_w: torch.Tensor, eps: float, h_out: torch.Tensor,
                  a_out: torch.Tensor, gate: torch.Tensor, k: int, L: Layer, s: Scratch):
    """route() of a_out = RMSNorm(h + d1) * norm_w, the norm made inside the routing launch (bit-identical to
    add_rmsnorm then route); stores a_out and the residual h + d1 to h_out. At most 4 rows."""
    R = h.shape[0]
    ids, members = s.window(R)
    ext().route_group_rmsnorm(h, d1, norm_w, eps, h_out, a_out, gate, L.gate_w, k, L.shared_id, s.logits,
                              s.route_counter, s.pick[:R * s.slots], s.wts[:R * s.slots], ids, s.count, members)


def windows(x: torch.Tensor, pick: torch.Tensor | None, wts: torch.Tensor | None, L: Layer, s: Scratch,
            k: int | None = None, gate: torch.Tensor | None = None):
    """routed2 over windows of s.rows tokens (prefill), each window as in decode; with gate (and pick=None) route()
    first in each window. Returns (routed sum, shared expert output or None)."""
    R = x.shape[0]
    out = torch.empty_like(x)
    sh = torch.empty_like(x) if L.shared_id >= 0 else None
    for r in range(0, R, s.rows):
        w = slice(r, r + s.rows)
        if gate is not None:
            route(x[w], gate, k, L, s)
        routed2(x[w], None if pick is None else pick[w], None if wts is None else wts[w], L, s, out=out[w],
                out_shared=None if sh is None else sh[w], k=k)
    return out, sh


def routed2(x: torch.Tensor, pick: torch.Tensor | None, wts: torch.Tensor | None, L: Layer, s: Scratch,
            out: torch.Tensor | None = None, out_shared: torch.Tensor | None = None, k: int | None = None):
    """x [R, D] in the model's dtype, pick int32 [R, k] (vLLM's routed ids), wts fp32 [R, k]. Returns (routed sum,
    shared expert output or None), both [R, D] in x's dtype; the shared output is gated by sigmoid(x . gate_w).
    pick=None: the scratch already holds the grouping (route()), for k routed slots a row."""
    e = ext()
    R, k = (x.shape[0], k) if pick is None else pick.shape
    D, I, E = L.D, L.I, L.E
    slots = k + (L.shared_id >= 0)
    P = R * slots
    if R > s.rows or slots != s.slots:
        raise ValueError(f"{R}x{slots} slots but the scratch holds {s.rows}x{s.slots}")
    ids, members = s.window(R)
    pk, wt = s.pick[:P], s.wts[:P]
    if pick is not None:
        e.group_shared(pick, wts, x, x.stride(0), L.gate_w, L.shared_id, pk, wt, ids, s.count, members, R, k, E)
    if out is None:
        out = torch.empty((R, D), dtype=x.dtype, device=x.device)
    if L.shared_id >= 0 and out_shared is None:
        out_shared = torch.empty((R, D), dtype=x.dtype, device=x.device)
    osh = out_shared if L.shared_id >= 0 else None
    nt, w, sk, pf = s.cfg_gu
    if FUSED and R <= FUSED_ROWS and (D // sk) % 128 == 0:
        # rot_in + gate/up + its epilogue in one launch (the same arithmetic in the same order: the same bits)
        e.moe_gateup(x, x.stride(0), L.suh_g, L.suh_u, L.ptr[0], L.ptr[1], L.k2[0], L.k2[1], L.cb[0], L.cb[1], ids,
                     s.count, members, s.z, s.counters, L.svh_g, L.svh_u, L.suh_d, s.xd, D, I, P, sk, slots, w,
                     L.k2_gu[0], L.k2_gu[1], math.inf, ACT_F32)
    else:
        e.rot_in(x, x.stride(0), pk, L.suh_g, L.suh_u, s.xg, s.xu, R, D, slots, E)
        e.grouped(s.xg, s.xu, L.ptr[0], L.ptr[1], L.k2[0], L.k2[1], L.cb[0], L.cb[1], ids, s.count, members, s.z, 2,
                  D, I, P, sk, slots, nt, w, pf, L.k2_gu[0], L.k2_gu[1])
        e.gateup_epilogue(s.z, pk, L.svh_g, L.svh_u, L.suh_d, s.xd, R, P, I, sk, slots, E, math.inf, ACT_F32)
    nt, w, sk, pf = s.cfg_d
    e.grouped(s.xd, s.xd, L.ptr[2], L.ptr[2], L.k2[2], L.k2[2], L.cb[2], L.cb[2], ids, s.count, members, s.z, 1,
              I, D, P, sk, slots, nt, w, pf, L.k2_d[0], L.k2_d[1])
    e.down_combine2(s.z, pk, L.svh_d, s.y, wt, out, osh, R, P, D, sk, slots, E, k)
    return out, osh


def dequant(trellis: torch.Tensor, K: int, grid: int) -> torch.Tensor:
    """W [in, out] fp16 through the kernels' lane decode (bit-exact with the reference dequantisation)."""
    out = torch.empty((trellis.shape[0] * 16, trellis.shape[1] * 16), dtype=torch.float16, device=trellis.device)
    ext().dequant(trellis.contiguous(), out, 2 * K, KERNEL_CB[grid])
    return out

"""Routed and shared experts of one MoE layer through the grouped trellis kernels (the interface of
vllm_espalier/experts.py: Layer, prepare, Scratch, scratch, route, routed, routed2, windows, dequant, ext).

One layer, up to Scratch.rows tokens, whatever the experts' widths, in six launches:
  group_shared | route_group   the pick and weight tables with the shared expert as one more slot, then the grouping
                               (distinct experts in id order, their member rows in pick order), all on the device
  rot_in                       H(x * suh) of every slot for gate and up, from the model's bf16 / fp16 rows
  grouped, 2 matrices          gate and up of every distinct expert in one launch, the weights decoded in registers
  gateup_epilogue              splits summed, H, * svh, SwiGLU in fp32, * suh of down, H: the fp16 down input
  grouped, 1 matrix            down
  down_combine2                splits summed, H, * svh of down; the routing-weighted sum over the routed slots in slot
                               order, and the gated shared slot, each in the model's dtype
(Up to FUSED_ROWS tokens the rot_in / gate-up / epilogue trio is one launch, esp_moe_gateup, with the same bits.)

Sums run in a fixed order, so a token's output does not depend on the other tokens of its window, and nothing
allocates, so a HIP graph can hold the whole layer. Trellises are read in place through device address tables; the
matrices' suh / svh become rows of per-projection stacks.

The extension (espalier_ext: csrc/binding.cpp over libespalier_hip.so) is built in-tree by csrc/build.py;
ESPALIER_PREBUILT_EXTENSION names a prebuilt espalier_ext .so instead.
"""
from __future__ import annotations

import importlib.machinery
import importlib.util
import math
import os
from dataclasses import dataclass
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
# up to CHAIN_ROWS tokens the fused gate/up launch, the down launch and the combine run as one chained launch
# (esp_moe_chain: the down programs decode their weights while gate/up runs; the same bits); ESPALIER_MOE_CHAIN=0 off
CHAIN = env("ESPALIER_MOE_CHAIN", "1") != "0"
CHAIN_ROWS = 4
PREFILL_WAVES = 4          # waves a workgroup of the whole-prompt (prefill) grouped launches
PREFILL_SK_GU = 1          # K splits of the whole-prompt gate/up launch
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


_PROJECTIONS = ("gate", "up", "down")


@dataclass(frozen=True)
class ExpertTable:
    """One projection over a layer's expert matrices, as the grouped kernels read it: device tables indexed by
    expert, and the range of half-bits the launch's shared-memory stages must hold."""
    ptr: torch.Tensor        # int64 [E] trellis addresses
    k2: torch.Tensor         # int32 [E] half-bits (2 * bits)
    cb: torch.Tensor         # int32 [E] kernel codebook ids
    k2_lo: int
    k2_hi: int


def _expert_table(mats, in_f: int, out_f: int, proj: str, device) -> ExpertTable:
    addrs, half_bits, books = [], [], []
    for e, m in enumerate(mats):
        where = f"expert {e} {proj}"
        if (m.in_features, m.out_features) != (in_f, out_f):
            raise ValueError(f"{where}: {m.in_features}x{m.out_features}, expected {in_f}x{out_f}")
        if m.cb not in KERNEL_CB:
            raise NotImplementedError(f"{where}: grid code {m.cb} has no grouped kernel")
        pair = (KERNEL_CB[m.cb], 2 * m.K)
        if pair not in COMPILED:
            raise NotImplementedError(f"{where}: no grouped kernel for codebook {pair[0]} at {m.K} bits")
        if m.trellis.dtype != torch.int16 or not m.trellis.is_contiguous():
            raise ValueError(f"{where}: the trellis must be contiguous int16")
        addrs.append(m.trellis.data_ptr())
        books.append(pair[0])
        half_bits.append(pair[1])

    def dev(values, dtype):
        return torch.tensor(values, dtype=dtype, device=device)
    return ExpertTable(dev(addrs, torch.int64), dev(half_bits, torch.int32), dev(books, torch.int32),
                       min(half_bits), max(half_bits))


def _stack_rows(mats, attr: str, width: int, device) -> torch.Tensor:
    """fp16 [E, width] holding each matrix's `attr` (suh or svh) as a row; the matrix then refers to its row."""
    stack = torch.empty((len(mats), width), dtype=torch.float16, device=device)
    for row, m in zip(stack, mats):
        row.copy_(getattr(m, attr).reshape(-1))
        setattr(m, attr, row)
    return stack


class Layer:
    """One layer's experts as the kernels read them: three ExpertTables (gate, up, down), the suh / svh stacks, and
    the shared expert (if any) as the last entry, with its sigmoid-gate weight."""

    def __init__(self, experts, shared=None, gate_w=None):
        entries = [tuple(mats) for mats in experts]
        if shared is not None:
            entries.append(tuple(shared))
        gate0 = entries[0][0]
        self.E, self.D, self.I = len(entries), gate0.in_features, gate0.out_features
        device = gate0.trellis.device
        by_proj = list(zip(*entries))                        # [gate mats], [up mats], [down mats]
        shapes = ((self.D, self.I), (self.D, self.I), (self.I, self.D))
        self.tables = tuple(_expert_table(mats, k, n, name, device)
                            for mats, (k, n), name in zip(by_proj, shapes, _PROJECTIONS))
        gate_m, up_m, down_m = by_proj
        self.suh_g = _stack_rows(gate_m, "suh", self.D, device)
        self.suh_u = _stack_rows(up_m, "suh", self.D, device)
        self.svh_g = _stack_rows(gate_m, "svh", self.I, device)
        self.svh_u = _stack_rows(up_m, "svh", self.I, device)
        self.suh_d = _stack_rows(down_m, "suh", self.I, device)
        self.svh_d = _stack_rows(down_m, "svh", self.D, device)
        self.shared_id = self.E - 1 if shared is not None else -1
        self.gate_w = None if gate_w is None else gate_w.reshape(-1).contiguous()
        self.keep = [m.trellis for mats in entries for m in mats]     # the tables hold raw addresses

    @property
    def ptr(self) -> tuple:
        return tuple(t.ptr for t in self.tables)

    @property
    def k2(self) -> tuple:
        return tuple(t.k2 for t in self.tables)

    @property
    def cb(self) -> tuple:
        return tuple(t.cb for t in self.tables)

    @property
    def k2_gu(self) -> tuple:
        """(lowest, highest) half-bits over gate and up: one launch runs both."""
        g, u = self.tables[0], self.tables[1]
        return min(g.k2_lo, u.k2_lo), max(g.k2_hi, u.k2_hi)

    @property
    def k2_d(self) -> tuple:
        return self.tables[2].k2_lo, self.tables[2].k2_hi


# The bits of the device status word (include/espalier.h, ESP_STATUS_*)
STATUS_BITS = ((1, "a grouped launch met an expert whose (codebook, K2) has no kernel"),
               (2, "a grouped launch met an expert whose K2 lies outside the launch's range"),
               (4, "a launch gave up waiting (~20 ms) for another part of the launch"),
               (8, "a tile list held more member tiles than its bound, or a list launch's grid was shorter than it"))


def check_status(clear: bool = True) -> None:
    """Raise RuntimeError naming every bit set in the device status word (esp_status: what the kernels met in
    device-resident tables or in-launch hand-offs, which the host cannot see without reading it back), clearing the
    word first if asked. The read synchronises the current stream, so call it outside graph capture: after a prefill,
    between decode steps, in tests."""
    v = int(ext().status(clear))
    if v:
        raise RuntimeError(f"espalier device status {v:#x}: " + "; ".join(t for b, t in STATUS_BITS if v & b))


def prepare(experts, shared=None, gate_w=None) -> Layer:
    """experts: [(gate, up, down) EspMatrix] in expert order; shared: the shared expert's (gate, up, down), appended as
    the last table entry, with gate_w its sigmoid-gate weight [D]. Each matrix's suh / svh become rows of the layer's
    stacks."""
    return Layer(experts, shared, gate_w)


class Scratch:
    """Every buffer of the pipeline for up to `rows` tokens of `slots` picks each, shared by all layers of one shape
    (layers run one after another, so no two use it at once)."""

    def __init__(self, E: int, D: int, I: int, rows: int, slots: int, device):
        self.rows, self.slots, self.E = rows, slots, E
        self.cfg_gu = tile_config(D, I, True)
        self.cfg_d = tile_config(I, D, False)
        P = rows * slots
        maxu = min(P, E)
        partials = P * max(2 * self.cfg_gu[2] * I, self.cfg_d[2] * D)
        f16, f32, i32 = torch.float16, torch.float32, torch.int32
        layout = {
            "xg": ((P, D), f16, 0), "xu": ((P, D), f16, 0),          # rotated gate / up inputs, a row a slot
            "xd": ((P, I), f16, 0),                                   # the down input
            "z": ((partials,), f32, 0),                               # K-split partial sums of either projection
            "y": ((P, D), f32, 0),                                    # per-slot down outputs
            "route_counter": ((1,), i32, 0),                          # route_group's arrival count
            "pick": ((P,), i32, 0), "wts": ((P,), f32, 0),            # with the shared slot
            "ids": ((maxu,), i32, 0), "count": ((1,), i32, 0),        # distinct experts, in id order
            "members": ((maxu * rows,), i32, -1),                     # their member rows, -1 padded
            # esp_moe_gateup's arrival counters, one a (expert, 128 columns) on its own 128-byte line
            "counters": ((maxu * (I // 128) * 32,), i32, 0),
            # esp_moe_chain: its reader counts (zero between uses)
            "flags": ((2 * (maxu * (I // 128) + D // 128) * 32,), i32, 0),
        }
        for name, (shape, dtype, fill) in layout.items():
            setattr(self, name, torch.full(shape, fill, dtype=dtype, device=device))
        # esp_moe_chain's own hand-off buffers, xd and the down partials: every bit set between uses (the launch reads
        # a piece once no word of it is all-ones, then puts the all-ones back)
        self.xdc = torch.full((P, I), -1, dtype=torch.int16, device=device).view(f16)
        self.zd = torch.full((P * D * (I // 128),), -1, dtype=i32, device=device).view(f32)
        # the logits of esp_route_group_own and esp_route_group_rmsnorm (the shared gate's after each row's E): all-ones
        # between uses
        self.logits_n = torch.full((rows * (E + 1),), -1, dtype=i32, device=device).view(f32)

    def window(self, R: int):
        """(ids, members [maxu, R]) views for a window of R tokens."""
        maxu = min(R * self.slots, self.E)
        return self.ids[:maxu], self.members[:maxu * R].view(maxu, R)

    def fit(self, R: int, slots: int) -> None:
        if R > self.rows or slots != self.slots:
            raise ValueError(f"{R}x{slots} slots but the scratch holds {self.rows}x{self.slots}")


_SCRATCH: dict = {}


def scratch(layer: Layer, rows: int, slots: int, device) -> Scratch:
    """The Scratch shared by every layer of this layer's shape; slots counts the shared slot when there is one."""
    key = (layer.E, layer.D, layer.I, rows, slots, str(device))
    found = _SCRATCH.get(key)
    if found is None:
        found = _SCRATCH[key] = Scratch(layer.E, layer.D, layer.I, rows, slots, device)
    return found


def _gate_up(e, x, L: Layer, s: Scratch, R: int, P: int, slots: int, pick, ids, members) -> None:
    """xd (the down input) of every valid slot: rot_in, the gate/up GEMM and its epilogue, fused into one launch for
    up to FUSED_ROWS rows (the same arithmetic in the same order)."""
    nt, w, sk, pf = s.cfg_gu
    lo, hi = L.k2_gu
    (tg, tu), (bg, bu), (cg, cu) = L.ptr[:2], L.k2[:2], L.cb[:2]
    if FUSED and R <= FUSED_ROWS and (L.D // sk) % 128 == 0:
        e.moe_gateup(x, x.stride(0), L.suh_g, L.suh_u, tg, tu, bg, bu, cg, cu, ids, s.count, members, s.z,
                     s.counters, L.svh_g, L.svh_u, L.suh_d, s.xd, L.D, L.I, P, sk, slots, w, lo, hi, math.inf,
                     ACT_F32)
        return
    e.rot_in(x, x.stride(0), pick, L.suh_g, L.suh_u, s.xg, s.xu, R, L.D, slots, L.E)
    e.grouped(s.xg, s.xu, tg, tu, bg, bu, cg, cu, ids, s.count, members, s.z, 2, L.D, L.I, P, sk, slots, nt, w, pf,
              lo, hi)
    e.gateup_epilogue(s.z, pick, L.svh_g, L.svh_u, L.suh_d, s.xd, R, P, L.I, sk, slots, L.E, math.inf, ACT_F32)


def _down(e, L: Layer, s: Scratch, P: int, slots: int, ids, members) -> int:
    """The down GEMM's partials into s.z; returns its K splits."""
    nt, w, sk, pf = s.cfg_d
    t, b, c = L.ptr[2], L.k2[2], L.cb[2]
    e.grouped(s.xd, s.xd, t, t, b, b, c, c, ids, s.count, members, s.z, 1, L.I, L.D, P, sk, slots, nt, w, pf,
              *L.k2_d)
    return sk


def routed(x: torch.Tensor, pick: torch.Tensor, wts: torch.Tensor, L: Layer, s: Scratch,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """x [R, D] fp16/bf16, pick int32 [R, slots] (every slot a routed expert; picks outside [0, E) skipped), wts fp32
    [R, slots] -> fp32 [R, D], the weighted sum of the experts' outputs (the legacy fp32 pipeline: group, rot_in,
    grouped, gateup_epilogue, grouped, down_combine)."""
    e = ext()
    R, slots = pick.shape
    s.fit(R, slots)
    P = R * slots
    ids, members = s.window(R)
    e.group(pick, ids, s.count, members, R, slots, L.E)
    nt, w, sk, pf = s.cfg_gu
    e.rot_in(x, x.stride(0), pick, L.suh_g, L.suh_u, s.xg, s.xu, R, L.D, slots, L.E)
    e.grouped(s.xg, s.xu, L.ptr[0], L.ptr[1], L.k2[0], L.k2[1], L.cb[0], L.cb[1], ids, s.count, members, s.z, 2,
              L.D, L.I, P, sk, slots, nt, w, pf, *L.k2_gu)
    e.gateup_epilogue(s.z, pick, L.svh_g, L.svh_u, L.suh_d, s.xd, R, P, L.I, sk, slots, L.E, math.inf, ACT_F32)
    sk_d = _down(e, L, s, P, slots, ids, members)
    out = torch.empty((R, L.D), dtype=torch.float32, device=x.device) if out is None else out
    e.down_combine(s.z, pick, L.svh_d, s.y, wts, out, R, P, L.D, sk_d, slots, L.E)
    return out


def route(x: torch.Tensor, gate: torch.Tensor, k: int, L: Layer, s: Scratch):
    """The router GEMV (plus the shared gate), softmax / top-k / renormalisation and the grouping in one launch
    (route_group, over the scratch's all-ones logits buffer: esp_route_group_own, the same bits) into the scratch's
    tables; routed2(..., pick=None) then runs the experts."""
    R = x.shape[0]
    ids, members = s.window(R)
    P = R * s.slots
    ext().route_group_own(x, gate, L.gate_w, k, L.shared_id, s.logits_n, s.route_counter, s.pick[:P], s.wts[:P], ids,
                          s.count, members)


def route_rmsnorm(h: torch.Tensor, d1: torch.Tensor | None, norm_w: torch.Tensor, eps: float, h_out: torch.Tensor,
                  a_out: torch.Tensor, gate: torch.Tensor, k: int, L: Layer, s: Scratch):
    """route() of a_out = RMSNorm(h + d1) * norm_w, the norm made inside the routing launch (bit-identical to
    add_rmsnorm then route); stores a_out and the residual h + d1 to h_out. At most 4 rows. Its logits go through the
    scratch's all-ones buffer (logits_n), which the launch leaves all-ones."""
    R = h.shape[0]
    ids, members = s.window(R)
    P = R * s.slots
    ext().route_group_rmsnorm(h, d1, norm_w, eps, h_out, a_out, gate, L.gate_w, k, L.shared_id, s.logits_n,
                              s.route_counter, s.pick[:P], s.wts[:P], ids, s.count, members)


def routed2(x: torch.Tensor, pick: torch.Tensor | None, wts: torch.Tensor | None, L: Layer, s: Scratch,
            out: torch.Tensor | None = None, out_shared: torch.Tensor | None = None, k: int | None = None):
    """x [R, D] in the model's dtype; pick int32 [R, k] (vLLM's routed ids) and wts fp32 [R, k], or pick=None when
    route() has already filled the scratch's tables for k routed slots a row. Returns (routed sum, the shared expert's
    gated output or None), [R, D] in x's dtype."""
    e = ext()
    R = x.shape[0]
    k = k if pick is None else pick.shape[1]
    has_shared = L.shared_id >= 0
    slots = k + has_shared
    s.fit(R, slots)
    P = R * slots
    ids, members = s.window(R)
    pick_p, wts_p = s.pick[:P], s.wts[:P]
    if pick is not None:
        e.group_shared(pick, wts, x, x.stride(0), L.gate_w, L.shared_id, pick_p, wts_p, ids, s.count, members, R, k,
                       L.E)
    out = torch.empty((R, L.D), dtype=x.dtype, device=x.device) if out is None else out
    if has_shared and out_shared is None:
        out_shared = torch.empty((R, L.D), dtype=x.dtype, device=x.device)
    shared_out = out_shared if has_shared else None
    sk_gu, sk_d = s.cfg_gu[2], s.cfg_d[2]
    if CHAIN and FUSED and R <= CHAIN_ROWS and (L.D // sk_gu) % 128 == 0 and sk_d * 128 == L.I and L.I <= 1024:
        (tg, tu, td), (bg, bu, bd), (cg, cu, cd) = L.ptr, L.k2, L.cb
        e.moe_chain(x, x.stride(0), L.suh_g, L.suh_u, tg, tu, td, bg, bu, bd, cg, cu, cd, ids, s.count, members,
                    pick_p, wts_p, L.svh_g, L.svh_u, L.suh_d, L.svh_d, s.xdc, s.z, s.zd, s.y, out, shared_out,
                    s.counters, s.flags, L.D, L.I, sk_gu, slots, L.E, k, *L.k2_gu, *L.k2_d, math.inf, ACT_F32)
        return out, shared_out
    _gate_up(e, x, L, s, R, P, slots, pick_p, ids, members)
    sk_d = _down(e, L, s, P, slots, ids, members)
    e.down_combine2(s.z, pick_p, L.svh_d, s.y, wts_p, out, shared_out, R, P, L.D, sk_d, slots, L.E, k)
    return out, shared_out


def windows(x: torch.Tensor, pick: torch.Tensor | None, wts: torch.Tensor | None, L: Layer, s: Scratch,
            k: int | None = None, gate: torch.Tensor | None = None):
    """routed2 over consecutive windows of s.rows tokens (prefill), each exactly as in decode; with gate (and
    pick=None), route() first in each window. Returns (routed sum, shared output or None)."""
    out = torch.empty_like(x)
    shared_out = torch.empty_like(x) if L.shared_id >= 0 else None
    for r0 in range(0, x.shape[0], s.rows):
        rows = slice(r0, r0 + s.rows)
        if gate is not None:
            route(x[rows], gate, k, L, s)
        routed2(x[rows], None if pick is None else pick[rows], None if wts is None else wts[rows], L, s,
                out=out[rows], out_shared=None if shared_out is None else shared_out[rows], k=k)
    return out, shared_out


class PrefillScratch:
    """The buffers of one whole-prompt MoE pass (prefill) for up to `rows` tokens of `slots` picks: the pipeline's
    tables and activations for P = rows * slots slot rows, the grouping over the whole prompt (members [maxu][rows]),
    and route_rows' logits."""

    def __init__(self, E: int, D: int, I: int, rows: int, slots: int, device, window: int = 32):
        self.rows, self.slots, self.E, self.window = rows, slots, E, window
        P = rows * slots
        maxu = min(P, E)
        f16, f32, i32 = torch.float16, torch.float32, torch.int32
        layout = {
            "xg": ((P, D), f16, 0), "xu": ((P, D), f16, 0), "xd": ((P, I), f16, 0),
            "z": ((P * max(2 * I * PREFILL_SK_GU, D),), f32, 0),     # the gate/up splits' partials, or down's sums
            "pick": ((P,), i32, 0), "wts": ((P,), f32, 0),
            "ids": ((maxu,), i32, 0), "count": ((1,), i32, 0), "members": ((maxu * rows,), i32, -1),
            "tiles": ((1 + tile_list_cap(maxu, rows, P),), i32, 0),
            "logits": ((rows * E,), f32, 0),
        }
        for name, (shape, dtype, fill) in layout.items():
            setattr(self, name, torch.full(shape, fill, dtype=dtype, device=device))

    def grouping(self, T: int):
        maxu = min(T * self.slots, self.E)
        return self.ids[:maxu], self.members[:maxu * T].view(maxu, T)


_PREFILL: dict = {}
TILE_LIST_PAIRS = 32768      # esp_tile_list's limit on (expert slot, member tile) pairs


def tile_list_cap(maxu: int, maxm: int, P: int) -> int:
    """Entries esp_tile_list may write for a grouping of P picks over maxu expert slots, maxm members a row."""
    return min(maxu * -(-maxm // 32), -(-P // 32) + maxu)


def prefill_scratch(layer: Layer, rows: int, slots: int, device) -> PrefillScratch:
    """The PrefillScratch shared by every layer of this layer's shape, for prompts of up to `rows` tokens."""
    key = (layer.E, layer.D, layer.I, slots, str(device))
    found = _PREFILL.get(key)
    if found is None or found.rows < rows:
        found = _PREFILL[key] = PrefillScratch(layer.E, layer.D, layer.I, rows, slots, device)
    return found


PREFILL_MAX_ROWS = 16384    # tokens one whole-prompt grouping takes (the wide grouping's members an expert)


def prefill(x: torch.Tensor, pick: torch.Tensor | None, wts: torch.Tensor | None, L: Layer, s: PrefillScratch,
            k: int, gate: torch.Tensor | None = None, out: torch.Tensor | None = None,
            out_shared: torch.Tensor | None = None):
    """The MoE layer over a whole prompt (ESPALIER_PREFILL_MODE=tile): the picks of every token (vLLM's, or route_rows
    over the whole prompt, the bits decode's route_group gives them), ONE grouping of all of them, and the expert GEMMs
    over that grouping with one K split, so each picked expert's weights are decoded once for all its member rows
    (in tiles of 32) instead of once a 32-token window. Returns (routed sum, shared output or None), [T, D] in x's
    dtype; a token's output depends on its own picks and rows only (the K split is fixed), not on the other tokens.
    A prompt of more than PREFILL_MAX_ROWS tokens runs as consecutive chunks of that many (the same bits a row)."""
    T = x.shape[0]
    if T <= PREFILL_MAX_ROWS:
        return _prefill(x, pick, wts, L, s, k, gate, out, out_shared)
    out = torch.empty((T, L.D), dtype=x.dtype, device=x.device) if out is None else out
    if L.shared_id >= 0 and out_shared is None:
        out_shared = torch.empty((T, L.D), dtype=x.dtype, device=x.device)
    for r0 in range(0, T, PREFILL_MAX_ROWS):
        rows = slice(r0, r0 + PREFILL_MAX_ROWS)
        _prefill(x[rows], None if pick is None else pick[rows], None if wts is None else wts[rows], L, s, k, gate,
                 out[rows], None if out_shared is None else out_shared[rows])
    return out, (out_shared if L.shared_id >= 0 else None)


def _prefill(x, pick, wts, L: Layer, s: PrefillScratch, k: int, gate, out, out_shared):
    e = ext()
    T = x.shape[0]
    has_shared = L.shared_id >= 0
    slots = k + has_shared
    if T > s.rows or slots != s.slots:
        raise ValueError(f"{T}x{slots} slots but the prefill scratch holds {s.rows}x{s.slots}")
    P = T * slots
    ids, members = s.grouping(T)
    pick_p, wts_p = s.pick[:P], s.wts[:P]
    if pick is None:
        if gate is None:
            raise ValueError("prefill needs the picks or the router weight")
        e.route_rows(x, gate, L.gate_w, k, L.shared_id, s.logits, pick_p, wts_p)
        e.group(pick_p, ids, s.count, members, T, slots, L.E)
    else:
        e.group_shared(pick, wts, x, x.stride(0), L.gate_w, L.shared_id, pick_p, wts_p, ids, s.count, members, T, k,
                       L.E)
    e.rot_in(x, x.stride(0), pick_p, L.suh_g, L.suh_u, s.xg, s.xu, T, L.D, slots, L.E)
    sk = PREFILL_SK_GU
    t, b, c = L.ptr[2], L.k2[2], L.cb[2]
    # the grouped launches over the grouping's non-empty (expert, member tile) pairs only: a grid of every expert slot
    # times every member tile is mostly empty workgroups (the same programs either way, the same bits)
    if ids.numel() * -(-T // 32) <= TILE_LIST_PAIRS:
        e.tile_list(s.count, members, ids.numel(), P, s.tiles)
        e.grouped_list(s.xg, s.xu, L.ptr[0], L.ptr[1], L.k2[0], L.k2[1], L.cb[0], L.cb[1], ids, s.count, members,
                       s.tiles, s.z, 2, L.D, L.I, P, sk, slots, PREFILL_WAVES, *L.k2_gu)
        e.gateup_epilogue(s.z, pick_p, L.svh_g, L.svh_u, L.suh_d, s.xd, T, P, L.I, sk, slots, L.E, math.inf, ACT_F32)
        e.grouped_list(s.xd, s.xd, t, t, b, b, c, c, ids, s.count, members, s.tiles, s.z, 1, L.I, L.D, P, 1, slots,
                       PREFILL_WAVES, *L.k2_d)
    else:
        e.grouped(s.xg, s.xu, L.ptr[0], L.ptr[1], L.k2[0], L.k2[1], L.cb[0], L.cb[1], ids, s.count, members, s.z, 2,
                  L.D, L.I, P, sk, slots, 8, PREFILL_WAVES, 2, *L.k2_gu)
        e.gateup_epilogue(s.z, pick_p, L.svh_g, L.svh_u, L.suh_d, s.xd, T, P, L.I, sk, slots, L.E, math.inf, ACT_F32)
        e.grouped(s.xd, s.xd, t, t, b, b, c, c, ids, s.count, members, s.z, 1, L.I, L.D, P, 1, slots, 8,
                  PREFILL_WAVES, 2, *L.k2_d)
    out = torch.empty((T, L.D), dtype=x.dtype, device=x.device) if out is None else out
    if has_shared and out_shared is None:
        out_shared = torch.empty((T, L.D), dtype=x.dtype, device=x.device)
    shared_out = out_shared if has_shared else None
    # no per-slot outputs: nothing reads them, and every pick of route_rows / the caller's tables is valid
    e.down_combine2(s.z, pick_p, L.svh_d, None, wts_p, out, shared_out, T, P, L.D, 1, slots, L.E, k)
    return out, shared_out


def dequant(trellis: torch.Tensor, K: int, grid: int) -> torch.Tensor:
    """W [in, out] fp16 decoded by the kernels' lane decode (bit-exact with the reference dequantisation). K is the
    bit width, grid the checkpoint grid code."""
    w = torch.empty((16 * trellis.shape[0], 16 * trellis.shape[1]), dtype=torch.float16, device=trellis.device)
    ext().dequant(trellis.contiguous(), w, 2 * K, KERNEL_CB[grid])
    return w

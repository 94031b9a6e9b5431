"""A synthetic Espalier decoder for whole-model decode / prefill throughput on random weights (the BASELINE decoder
step: 40 layers of the dense block and the grouped MoE block, an mcg LM head, greedy decode).

Per layer, on rows h (bf16 [T, 2048], the residual stream):
  a   = RMSNorm(h + the previous layer's MoE outputs)     add_rmsnorm (csrc/step.hip)
  qkv = [q | k | v](a)                                    one dense launch (2048 -> 4096 + 512 + 512, int6)
        attention is not part of this layer set: o reads q itself (qkv[:, :4096]) as a placeholder
  o   = o(q)                                              one dense launch (4096 -> 2048, int6)
  a   = RMSNorm(h + o)                                    add_rmsnorm
  route_group, then the grouped launches                  256 routed experts (top-8) + the gated shared expert
then RMSNorm, the LM head (one dense launch, 2048 -> vocab, 6-bit mcg) and the argmax, which writes the next ids on
the device. The shared expert of the dense block is the MoE's shared slot, counted once. Every op is a kernel of this
package, nothing allocates after construction, so a HIP graph holds a whole step.

For up to 4 rows (decode) each norm runs inside its consumer's launch instead (dense_rmsnorm for qkv and the head,
route_group_rmsnorm for the router), with the same arithmetic in the same order, so the bits do not change: the qkv
launch stores the residual to a second buffer, which the routing launch reads and adds o to, back into h. qkv and o
run as one chained launch (dense.DenseMulti: o's workgroups land and decode their weights, then wait for qkv's column
blocks), with the bits of the two launches apart (MULTI_ATTN = False runs them apart). Both run at ATTN_W waves a
workgroup: at 8, a CU holds a qkv and an o workgroup at once, so o's decode overlaps qkv (decode step 2,152 -> 2,122
us on MI355X; at 16 waves the chain was slower than the launches apart, 2,214 against 2,146 us). Up to 4 rows the
MoE after the routing is one chained launch too (experts.routed2: esp_moe_chain).

Rows never interact (the dense and grouped kernels keep rows apart, norms are per row), so a window of T rows
gives each row the bits it gets alone.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import dense as Dn
from . import experts as G
from . import workloads as WL
from .experts import ext

D_MODEL = 2048
Q_OUT, KV_OUT = 4096, 512
EXPERT_I = 512
VOCAB = 151936
TOPK = 8
EPS = 1e-6
FUSE_NORMS = True            # the norms inside their consumers' launches for up to 4 rows (same bits)
MULTI_ATTN = True             # qkv and o as one chained launch (same bits)
ATTN_W = 8                    # waves a workgroup of the qkv and o launches, chained or apart (the same bits either way)


@dataclass
class DecoderLayer:
    norm1: torch.Tensor          # bf16 [D]
    qkv: Dn.Dense
    o: Dn.Dense
    attn: Dn.DenseMulti          # qkv then o (reading q) in one launch
    norm2: torch.Tensor
    router: torch.Tensor         # bf16 [E, D]
    moe: G.Layer
    experts: list                # [(gate, up, down) EspMatrix] routed, in id order
    shared: tuple                # the shared expert's (gate, up, down)


def _norm_weight(gen, dev, D):
    return (1.0 + 0.1 * torch.randn((D,), generator=gen, device=dev)).to(torch.bfloat16)


def build_layer(gen: torch.Generator, dev, E: int = 256, D: int = D_MODEL, I: int = EXPERT_I) -> DecoderLayer:
    """One layer with seeded random weights: q/k/v/o 4-bit int6; routed experts of 1-3 bits (E2M1 at 1-2, int5 at
    3); a 4-bit int5 shared expert with a sigmoid gate; a bf16 router ~N(0, 0.02)."""
    qkv = Dn.Dense([WL.matrix(D, Q_OUT, 4, "int6", gen, dev), WL.matrix(D, KV_OUT, 4, "int6", gen, dev),
                    WL.matrix(D, KV_OUT, 4, "int6", gen, dev)])
    o = Dn.Dense([WL.matrix(Q_OUT, D, 4, "int6", gen, dev)])
    widths = torch.randint(1, 4, (E,), generator=gen, device=dev).tolist()
    grid = {1: "e2m1", 2: "e2m1", 3: "int5"}
    experts = [tuple(WL.matrix(k, n, b, grid[b], gen, dev) for k, n in ((D, I), (D, I), (I, D))) for b in widths]
    shared = tuple(WL.matrix(k, n, 4, "int5", gen, dev) for k, n in ((D, I), (D, I), (I, D)))
    gate_w = (torch.randn((D,), generator=gen, device=dev) * 0.05).to(torch.bfloat16)
    router = (torch.randn((E, D), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    moe = G.prepare(experts, shared, gate_w)
    # both launches at ATTN_W waves, so the chained launch keeps the bits of the launches apart
    for d in (qkv, o):
        d.plans = [(sk, ATTN_W, pf) for sk, _, pf in d.plans]
    attn = Dn.DenseMulti([qkv, o], after=[False, True], W=ATTN_W)
    return DecoderLayer(_norm_weight(gen, dev, D), qkv, o, attn, _norm_weight(gen, dev, D), router, moe, experts,
                        shared)


class Buffers:
    """Every activation of a T-row pass, allocated once (graph capture needs fixed addresses)."""

    def __init__(self, T: int, vocab: int, dev, D: int = D_MODEL):
        bf = torch.bfloat16
        self.T = T
        self.ids_in = torch.zeros((T,), dtype=torch.int32, device=dev)
        self.ids_out = torch.zeros((T,), dtype=torch.int32, device=dev)
        self.h = torch.zeros((T, D), dtype=bf, device=dev)
        self.h2 = torch.zeros((T, D), dtype=bf, device=dev)      # the residual between the qkv and routing launches
        self.a = torch.zeros((T, D), dtype=bf, device=dev)
        self.qkv = torch.zeros((T, Q_OUT + 2 * KV_OUT), dtype=bf, device=dev)
        self.o = torch.zeros((T, D), dtype=bf, device=dev)
        self.moe = torch.zeros((T, D), dtype=bf, device=dev)
        self.moe_shared = torch.zeros((T, D), dtype=bf, device=dev)
        self.logits = torch.zeros((T, vocab), dtype=bf, device=dev)
        self.argmax_part = torch.zeros((T * -(-vocab // 4096),), dtype=torch.int64, device=dev)   # a key a slice
        self.argmax_cnt = torch.zeros((T * 32,), dtype=torch.int32, device=dev)                   # zero between uses


class SyntheticDecoder:
    def __init__(self, n_layers: int = 40, seed: int = 5, device="cuda", E: int = 256, vocab: int = VOCAB,
                 head_bits: int = 6):
        dev = torch.device(device)
        gen = torch.Generator(device=dev).manual_seed(seed)
        self.dev, self.vocab, self.E = dev, vocab, E
        self.layers = [build_layer(gen, dev, E) for _ in range(n_layers)]
        self.embedding = torch.randn((vocab, D_MODEL), generator=gen, device=dev).to(torch.bfloat16)
        self.final_norm = _norm_weight(gen, dev, D_MODEL)
        self.head = Dn.Dense([WL.matrix(D_MODEL, vocab, head_bits, "mcg", gen, dev)])
        self.scratch = G.scratch(self.layers[0].moe, Dn.MAX_ROWS, TOPK + 1, dev)
        self._bufs: dict[int, Buffers] = {}

    def buffers(self, T: int) -> Buffers:
        if T not in self._bufs:
            if not 0 < T <= Dn.MAX_ROWS:
                raise ValueError(f"a pass takes 1..{Dn.MAX_ROWS} rows, got {T}")
            self._bufs[T] = Buffers(T, self.vocab, self.dev)
        return self._bufs[T]

    def fused_norms(self, T: int) -> bool:
        """Whether the layers' norms run inside the qkv and routing launches for T rows."""
        return FUSE_NORMS and T <= 4 and self.layers[0].qkv.norm_fusable(T)

    def fused_head_norm(self, T: int) -> bool:
        return FUSE_NORMS and self.head.norm_fusable(T)

    def layer_forward(self, L: DecoderLayer, b: Buffers, first: bool, picks: list | None = None):
        e = ext()
        q = b.qkv[:, :Q_OUT]
        d1, d2 = (None, None) if first else (b.moe, b.moe_shared)
        if self.fused_norms(b.T):
            if MULTI_ATTN:
                L.attn.forward([None, q], [b.qkv, b.o], norm=(b.h, d1, d2, L.norm1, EPS, b.h2))
            else:
                L.qkv.forward_rmsnorm(b.h, d1, d2, L.norm1, EPS, b.h2, out=b.qkv)
                L.o.forward(q, out=b.o)
            G.route_rmsnorm(b.h2, b.o, L.norm2, EPS, b.h, b.a, L.router, TOPK, L.moe, self.scratch)
        else:
            e.add_rmsnorm(b.h, d1, d2, L.norm1, b.a, EPS)
            if MULTI_ATTN:
                L.attn.forward([b.a, q], [b.qkv, b.o])
            else:
                L.qkv.forward(b.a, out=b.qkv)
                L.o.forward(q, out=b.o)
            e.add_rmsnorm(b.h, b.o, None, L.norm2, b.a, EPS)
            G.route(b.a, L.router, TOPK, L.moe, self.scratch)
        if picks is not None:                     # eager runs only: the distinct experts this layer reads
            n = int(self.scratch.count.item())
            picks.append(self.scratch.ids[:n].clone())
        G.routed2(b.a, None, None, L.moe, self.scratch, out=b.moe, out_shared=b.moe_shared, k=TOPK)

    def forward(self, T: int, head: bool = True, picks: list | None = None) -> Buffers:
        """One pass over the rows of buffers(T): ids_in -> every layer -> (head) logits and ids_out."""
        b = self.buffers(T)
        e = ext()
        e.embed(b.ids_in, self.embedding, b.h)
        for i, L in enumerate(self.layers):
            self.layer_forward(L, b, i == 0, picks)
        if head:
            if self.fused_head_norm(T):
                self.head.forward_rmsnorm(b.h, b.moe, b.moe_shared, self.final_norm, EPS, b.h2, out=b.logits)
            else:
                e.add_rmsnorm(b.h, b.moe, b.moe_shared, self.final_norm, b.a, EPS)
                self.head.forward(b.a, out=b.logits)
            e.argmax(b.logits, b.ids_out, b.argmax_part, b.argmax_cnt)
        return b

    def prefill_buffers(self, T: int) -> Buffers:
        key = ("prefill", T)
        if key not in self._bufs:
            self._bufs[key] = Buffers(T, self.vocab, self.dev)
        return self._bufs[key]

    def prefill_scratch(self, T: int) -> G.PrefillScratch:
        """The MoE prefill scratch for prompts of T tokens, with the dense layers' prompt scratch grown to match."""
        L0 = self.layers[0]
        L0.qkv.reserve_prompt(T)
        L0.o.reserve_prompt(T)
        return G.prefill_scratch(L0.moe, T, TOPK + 1, self.dev)

    def prefill_layer(self, L: DecoderLayer, b: Buffers, first: bool, ps: G.PrefillScratch):
        """One layer of prefill over the rows of b: the dense layers as prompt launches, the MoE over the whole prompt
        (its picks left in ps.pick, slots a row)."""
        e = ext()
        d1, d2 = (None, None) if first else (b.moe, b.moe_shared)
        e.add_rmsnorm(b.h, d1, d2, L.norm1, b.a, EPS)
        L.qkv.forward_tile(b.a, out=b.qkv)
        L.o.forward_tile(b.qkv[:, :Q_OUT], out=b.o)
        e.add_rmsnorm(b.h, b.o, None, L.norm2, b.a, EPS)
        G.prefill(b.a, None, None, L.moe, ps, TOPK, gate=L.router, out=b.moe, out_shared=b.moe_shared)

    def prefill(self, T: int, head_rows: int = 1) -> Buffers:
        """A whole prompt of T tokens (prefill_buffers(T).ids_in) in the tile mode: the dense layers as prompt launches
        (Dense.forward_tile: each weight decoded once for every 128 rows), every layer's MoE over the whole prompt
        (experts.prefill: routing in one launch, one grouping, each picked expert decoded once), then the head (a prompt
        launch too) and argmax on the last head_rows tokens. Rows still never interact, but a row's bits are those of the tile mode,
        not of decode."""
        b = self.prefill_buffers(T)
        e = ext()
        e.embed(b.ids_in, self.embedding, b.h)
        ps = self.prefill_scratch(T)
        self.head.reserve_prompt(head_rows)
        for i, L in enumerate(self.layers):
            self.prefill_layer(L, b, i == 0, ps)
        e.add_rmsnorm(b.h, b.moe, b.moe_shared, self.final_norm, b.a, EPS)
        tail = slice(T - head_rows, T)
        self.head.forward_tile(b.a[tail], out=b.logits[tail])
        e.argmax(b.logits[tail], b.ids_out[tail])
        return b

    def algorithmic_bytes(self, picks: list[torch.Tensor], tokens: int, head: bool = True) -> int:
        """Weight bytes a pass over `tokens` rows reads: trellis + suh + svh of q/k/v/o, of the shared expert and of
        every distinct routed expert picked (picks from an eager forward), the bf16 router, the RMSNorm weights, one
        embedding row a token, and the head."""
        total = tokens * D_MODEL * 2
        for L, ids in zip(self.layers, picks):
            total += WL.nbytes(L.qkv.mats) + WL.nbytes(L.o.mats) + WL.nbytes(L.shared)
            total += L.router.numel() * 2 + (L.norm1.numel() + L.norm2.numel()) * 2
            for u in ids.tolist():
                if u < len(L.experts):
                    total += WL.nbytes(L.experts[u])
        if head:
            total += WL.nbytes(self.head.mats) + self.final_norm.numel() * 2
        return total

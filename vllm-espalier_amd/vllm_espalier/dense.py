"""Dense trellis layers in one launch (csrc/dense.hip): every matrix of a vLLM layer, x in the model's dtype, output
written into each matrix's columns, no casts or cat. Up to 32 rows (decode); above that ops.py windows them.
(The surface of vllm_espalier/dense.py:1-103.)

Each matrix keeps its own suh/svh. All matrices of one launch share K and codebook; a layer that mixes them runs one
launch per group into the same output. The K split (`plan`) depends on the layer's shape alone, so a row's bits
never depend on the batch.
"""
from __future__ import annotations

import os

import torch

from .experts import KERNEL_CB, ext
from ._env import env

MAX_ROWS = 32
COUNTER_STRIDE = 32          # ints between two 128-column blocks' arrival counters (one 128-byte line each)
ROT_SMEM = int(os.environ.get("ESPALIER_DENSE_ROTATION_SMEM", 64 * 1024))   # fuse the input rotation up to this much LDS
_scratch: dict = {}
_outgrown: list = []         # scratch a growth replaced: kept alive, since graphs captured before it still use it


def plan(K: int, N: int, sms: int) -> tuple[int, int, int]:
    """(K splits SK, waves a workgroup W, tiles in flight) for a K -> N layer of 128-column blocks, from its shape
    alone so a row's bits never depend on the batch (the reference's sm89 heuristic is dense.py:22-39). A gfx950
    workgroup is 4 * KW waves on one block, KW of them on every 32-k step column; a split is a run of whole 32-k
    steps, SK need not divide them. The decode of a workgroup's share is bound by its CU's VALU, so the plan spreads
    the layer over the CUs, SK = CUs // blocks (one workgroup a CU), but keeps 4 steps a split: below that the
    fixed costs (rotation, hand-off) outweigh the shorter decode, and 32-row windows lose more to the extra partials
    than single rows gain (cold sweeps on MI355X). Then 16 waves when a split has 8 steps or more, 8 from 4, else 4,
    but at most 8 when the launch has more workgroups than CUs (the LM head: 97 us against 113 at 16 waves).
    ESPALIER_DENSE_TILE_PLAN="sk,w,pf" forces."""
    forced = env("ESPALIER_DENSE_TILE_PLAN")
    if forced:
        sk, w, pf = (int(v) for v in forced.split(","))
        return sk, w, pf
    nb = N // 128
    steps_all = K // 32
    sk = max(1, min(steps_all // 4, sms // nb))
    steps = -(-steps_all // sk)
    w = 16 if steps >= 8 else 8 if steps >= 4 else 4
    if nb * sk > sms:
        w = min(w, 8)            # more workgroups than CUs: two of 8 waves share a CU and hide each other's waits
    return sk, w, 2


def scratch(device, z_floats: int, xh_halves: int):
    """Shared scratch, grown while layers are prepared, never during a forward. A buffer that a growth replaces is
    never freed: a graph captured before the growth keeps writing to the buffer it was captured with."""
    s = _scratch.get(device)
    if s is None or s[0].numel() < z_floats or s[1].numel() < xh_halves:
        z = max(z_floats, s[0].numel() if s else 0, 1)
        h = max(xh_halves, s[1].numel() if s else 0, 1)
        if s is not None:
            _outgrown.append(s)
        s = (torch.empty(z, dtype=torch.float32, device=device), torch.empty(h, dtype=torch.half, device=device))
        _scratch[device] = s
    return s


def _sms(dev) -> int:
    if dev.type == "cuda" and torch.cuda.is_available():
        return torch.cuda.get_device_properties(dev).multi_processor_count
    return 256                                   # MI355X


class Dense:
    MAX_ROWS = MAX_ROWS

    def __init__(self, mats, n_out: int | None = None):
        self.mats = list(mats)
        m0 = self.mats[0]
        self.K = m0.in_features
        if any(m.in_features != self.K for m in self.mats):
            raise ValueError("every matrix of a dense layer must share its input width")
        self.groups = []                       # launches: (matrix indices, k2, kernel cb)
        for i, m in enumerate(self.mats):
            key = (2 * m.K, KERNEL_CB[m.cb])
            if self.groups and (self.groups[-1][1], self.groups[-1][2]) == key and len(self.groups[-1][0]) < 4:
                self.groups[-1][0].append(i)
            else:
                self.groups.append(([i], *key))
        self.col0 = []
        c = 0
        for m in self.mats:
            self.col0.append(c)
            c += m.out_features
        self.N = c
        self.n_out = n_out or c
        dev = m0.trellis.device
        sms = _sms(dev)
        self.plans, nbt_max, z = [], 0, 0
        for idx, _, _ in self.groups:
            n = sum(self.mats[i].out_features for i in idx)
            p = plan(self.K, n, sms)
            self.plans.append(p)
            nbt_max = max(nbt_max, n // 128)
            z = max(z, p[0] * MAX_ROWS * n)
        self.counters = torch.zeros(COUNTER_STRIDE * nbt_max, dtype=torch.int32, device=dev)
        scratch(dev, z, 4 * MAX_ROWS * self.K)

    def forward(self, x, trellis=None, suh=None, svh=None, out=None):
        """x [M, K] (M <= 32) -> [M, n_out] in x's dtype; trellis/suh/svh lists override the matrices' own tensors
        (module buffers under torch.compile)."""
        M = x.shape[0]
        trellis = trellis or [m.trellis for m in self.mats]
        suh = suh or [m.suh for m in self.mats]
        svh = svh or [m.svh for m in self.mats]
        y = out if out is not None else torch.empty((M, self.n_out), dtype=x.dtype, device=x.device)
        if self.n_out > self.N:
            y[:, self.N:].zero_()
        z, xh = scratch(x.device, 0, 0)
        if x.stride(-1) != 1:
            x = x.contiguous()
        for (idx, k2, cb), (sk, w, pf) in zip(self.groups, self.plans):
            ext().dense(x, [trellis[i] for i in idx], [suh[i] for i in idx], [svh[i] for i in idx],
                        [self.col0[i] for i in idx], y, xh, z, self.counters, k2, cb, sk, w, pf, ROT_SMEM)
        return y

    def norm_fusable(self, M: int) -> bool:
        """Whether forward_rmsnorm runs in one launch for M rows: one launch group, four waves a row, and the rotated
        rows in the fused rotation's shared memory."""
        if len(self.groups) != 1:
            return False
        sk, w, _ = self.plans[0]
        steps = -(-(self.K // 32) // sk)
        chunks = -(-(steps * 32 + 96) // 128)
        return M <= w // 4 and self.K <= 8192 and M * chunks * 128 * 2 <= ROT_SMEM

    def forward_rmsnorm(self, h, d1, d2, norm_w, eps: float, h_out, out):
        """forward(RMSNorm(h + d1 + d2) * norm_w) with the residual h + d1 + d2 stored to h_out, the norm made inside
        the launch (bit-identical to add_rmsnorm then forward). h, d1, d2: [M, K] contiguous, the model's dtype."""
        z, _ = scratch(h.device, 0, 0)
        (idx, k2, cb), (sk, w, pf) = self.groups[0], self.plans[0]
        ext().dense_rmsnorm(h, d1, d2, norm_w, eps, h_out, [self.mats[i].trellis for i in idx],
                            [self.mats[i].suh for i in idx], [self.mats[i].svh for i in idx],
                            [self.col0[i] for i in idx], out, z, self.counters, k2, cb, sk, w, ROT_SMEM)
        return out

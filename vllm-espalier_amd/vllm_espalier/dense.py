"""Dense trellis layers for decode: every matrix of one vLLM layer in as few esp_dense launches as the codes allow (the
interface of vllm_espalier/dense.py: Dense, plan, scratch, MAX_ROWS).

A vLLM layer fuses several checkpoint matrices (q/k/v, gate/up); each keeps its own suh/svh, so they are never
concatenated into one trellis. A launch takes up to four of them that share the input width, the bit width and the
codebook; it reads x once in the model's dtype and writes each matrix's columns of y in that dtype. Up to MAX_ROWS rows
a launch; ops.py windows longer inputs.

The K split of a launch (`plan`) is a function of the layer's shape alone, so the bits of a row never depend on the
other rows of the batch.
"""
from __future__ import annotations

import itertools
import os
from dataclasses import dataclass

import torch

from ._env import env
from .experts import KERNEL_CB, ext

MAX_ROWS = 32
COUNTER_STRIDE = 32          # ints between two 128-column blocks' arrival counters (one 128-byte line each)
MAX_MATRICES = 4             # matrices one esp_dense launch takes
ROT_SMEM = int(os.environ.get("ESPALIER_DENSE_ROTATION_SMEM", 64 * 1024))   # fuse the input rotation up to this much LDS


def plan(K: int, N: int, sms: int) -> tuple[int, int, int]:
    """(K splits SK, waves a workgroup W, tiles in flight) for a K -> N layer of 128-column blocks, from its shape
    alone so a row's bits never depend on the batch (the reference's sm89 heuristic is dense.py:22-39). A gfx950
    workgroup is 4 * KW waves on one block, KW of them on every 32-k step column; a split is a run of whole 32-k
    steps, SK need not divide them. The decode of a workgroup's share is bound by its CU's VALU, so the plan spreads
    the layer over the CUs, SK = CUs // blocks (one workgroup a CU), but keeps 4 steps a split: below that the
    fixed costs (rotation, hand-off) outweigh the shorter decode, and 32-row windows lose more to the extra partials
    than single rows gain. Then 16 waves when a split has 4 steps or more, else 4, but at most 8 when the launch has
    more workgroups than CUs (the LM head: 97 us against 113 at 16 waves). bench.py --sweep (cold, MI355X) confirms the
    K splits of config 2's four launches at 1 and 32 rows, and the 16 waves also for the 4-step splits of the shared
    gate/up and down (1 row 6.95 -> 6.91 and 6.49 -> 6.46 us, 32 rows 12.1 -> 10.2 and 8.7 -> 8.0 us against 8
    waves). ESPALIER_DENSE_TILE_PLAN="sk,w,pf" forces."""
    forced = env("ESPALIER_DENSE_TILE_PLAN")
    if forced:
        sk, w, pf = (int(v) for v in forced.split(","))
        return sk, w, pf
    nb = N // 128
    steps_all = K // 32
    sk = max(1, min(steps_all // 4, sms // nb))
    steps = -(-steps_all // sk)
    w = 16 if steps >= 4 else 4
    if nb * sk > sms:
        w = min(w, 8)            # more workgroups than CUs: two of 8 waves share a CU and hide each other's waits
    return sk, w, 2


def tile_plan(K: int, N: int) -> int:
    """K splits of a prompt launch (esp_dense_tile) of a K -> N layer, from its shape alone (so a row's bits never
    depend on the prompt's length): the most splits that keep a 512-row prompt (4 tiles of 128 rows) within two 8-wave
    workgroups a CU, 4 * blocks * SK <= 512, so the grid stays resident and the split-K finish is spread over the
    splits; at most 8 (the spread finish's batch of partial loads) and splits of at least 128 k. From a sweep of every
    launch's SK at 128 / 512 / 2048 rows with the spread finish (config 2: qkv 3, o 8, shared gate/up 8, shared down 4,
    the fastest at 512 and 128 rows: o 35.7 -> 31.8 us and shared down 20.9 -> 17.4 us at 512 rows against the earlier
    4 and 1). At 2048 rows, where the grid is not resident and one split finishes each tile, fewer splits would be
    faster (o 81 us at 2 against 109 at 8). ESPALIER_DENSE_PROMPT_SK forces."""
    forced = env("ESPALIER_DENSE_PROMPT_SK")
    if forced:
        return int(forced)
    blocks = N // 128
    return max(1, min(128 // blocks, 8, K // 128))


TILE_ROWS = 128              # rows a prompt-launch workgroup
# launches whose last K split can poll the others' partials run as esp_dense_own over an all-ones partials buffer (the
# same bits, no arrival count); ESPALIER_DENSE_OWN=0 runs every launch as esp_dense
OWN = env("ESPALIER_DENSE_OWN", "1") != "0"


class _SharedScratch:
    """The split-K partials Z (fp32) and the unfused rotation's rows xh (fp16), one pair a device, shared by every
    layer (layers run one after another). Sizes only grow. A pair that a growth replaces is kept for good only when a
    graph may write to it (it was handed out during a stream capture); otherwise it is dropped, and the caching
    allocator reuses its memory, so a series of growing prompts outside capture keeps only the current pair."""

    def __init__(self, ones: bool = False):
        self.ones = ones                     # Z every bit set (the all-ones partials of esp_dense_own)
        self.current: dict = {}
        self.captured: set = set()          # devices whose current pair was handed out during a capture
        self.retired: list = []

    def reserve(self, device, z_floats: int, xh_halves: int):
        have = self.current.get(device)
        capturing = device.type == "cuda" and torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
        if have is not None and have[0].numel() >= z_floats and have[1].numel() >= xh_halves:
            if capturing:
                self.captured.add(device)
            return have
        if have is not None:
            if device in self.captured:
                self.retired.append(have)
            z_floats, xh_halves = max(z_floats, have[0].numel()), max(xh_halves, have[1].numel())
        self.captured.discard(device)
        z = (torch.full((max(z_floats, 1),), -1, dtype=torch.int32, device=device).view(torch.float32) if self.ones
             else torch.empty(max(z_floats, 1), dtype=torch.float32, device=device))
        pair = (z,
                torch.empty(max(xh_halves, 1), dtype=torch.float16, device=device))
        self.current[device] = pair
        if capturing:
            self.captured.add(device)
        return pair


_SHARED = _SharedScratch()
_OWN = _SharedScratch(ones=True)


def scratch(device, z_floats: int, xh_halves: int):
    """(Z, xh) of the device, grown to at least the given sizes."""
    return _SHARED.reserve(device, z_floats, xh_halves)


def own_partials(device, z_floats: int):
    """The device's all-ones partials buffer of esp_dense_own (left all-ones by every launch), grown to at least
    z_floats."""
    return _OWN.reserve(device, z_floats, 0)[0]


def polls(M: int, sk: int, w: int) -> bool:
    """Whether a launch of M rows, sk K splits and w waves takes esp_dense_own's polled hand-off: its last split holds
    one (row, split) partial a 32-lane half."""
    return sk > 1 and M * (sk - 1) <= 2 * w


_PROMPT = _SharedScratch()
_PROMPT_COUNTERS: dict = {}


def prompt_scratch(device, z_floats: int, xh_halves: int, counters: int):
    """(Z, xh, counters) of the device for prompt launches, grown to at least the given sizes (the counters zero, and
    left zero by every launch)."""
    was_captured = device in _PROMPT.captured            # before reserve: a growth there resets the mark
    z, xh = _PROMPT.reserve(device, z_floats, xh_halves)
    cnt = _PROMPT_COUNTERS.get(device)
    if cnt is None or cnt.numel() < counters:
        if cnt is not None and (was_captured or device in _PROMPT.captured):
            _PROMPT.retired.append((cnt,))
        cnt = _PROMPT_COUNTERS[device] = torch.zeros(max(counters, 1), dtype=torch.int32, device=device)
    return z, xh, cnt


def _cu_count(device) -> int:
    if device.type == "cuda" and torch.cuda.is_available():
        return torch.cuda.get_device_properties(device).multi_processor_count
    return 256                                   # MI355X


@dataclass(frozen=True)
class Launch:
    """One esp_dense launch: the matrices (indices into Dense.mats), their common half-bits and kernel codebook, the
    columns they write, and the shape's plan."""
    members: tuple
    k2: int
    cb: int
    n: int
    sk: int
    w: int
    pf: int


class Dense:
    MAX_ROWS = MAX_ROWS

    def __init__(self, mats, n_out: int | None = None):
        self.mats = list(mats)
        widths = {m.in_features for m in self.mats}
        if len(widths) != 1:
            raise ValueError(f"the matrices of a dense layer must share their input width, got {sorted(widths)}")
        (self.K,) = widths
        offsets = list(itertools.accumulate((m.out_features for m in self.mats), initial=0))
        self.col0, self.N = offsets[:-1], offsets[-1]
        self.n_out = n_out or self.N
        device = self.mats[0].trellis.device
        cus = _cu_count(device)
        self.launches = []
        for code, run in itertools.groupby(range(len(self.mats)), key=self._code):
            run = list(run)
            for i in range(0, len(run), MAX_MATRICES):
                members = tuple(run[i:i + MAX_MATRICES])
                n = sum(self.mats[j].out_features for j in members)
                self.launches.append(Launch(members, *code, n, *plan(self.K, n, cus)))
        blocks = max(l.n // 128 for l in self.launches)
        self.counters = torch.zeros(COUNTER_STRIDE * blocks, dtype=torch.int32, device=device)
        scratch(device, max(l.sk * MAX_ROWS * l.n for l in self.launches), 4 * MAX_ROWS * self.K)
        own_partials(device, max(l.sk * 2 * l.w // max(l.sk - 1, 1) * l.n for l in self.launches))

    def _code(self, i: int) -> tuple[int, int]:
        m = self.mats[i]
        return 2 * m.K, KERNEL_CB[m.cb]

    @property
    def groups(self) -> list:
        """(matrix indices, k2, kernel codebook) of each launch."""
        return [(list(l.members), l.k2, l.cb) for l in self.launches]

    @property
    def plans(self) -> list:
        """(SK, W, PF) of each launch."""
        return [(l.sk, l.w, l.pf) for l in self.launches]

    @plans.setter
    def plans(self, plans) -> None:
        """Replace the launches' plans (the scratch must already be large enough for them)."""
        if len(plans) != len(self.launches):
            raise ValueError(f"{len(plans)} plans for {len(self.launches)} launches")
        self.launches = [Launch(l.members, l.k2, l.cb, l.n, *p) for l, p in zip(self.launches, plans)]

    def forward(self, x, trellis=None, suh=None, svh=None, out=None):
        """x [M, K] (M <= MAX_ROWS) -> [M, n_out] in x's dtype. trellis / suh / svh: lists that replace the matrices'
        own tensors (the module buffers a compiled graph passes in)."""
        codes = trellis or [m.trellis for m in self.mats]
        pre = suh or [m.suh for m in self.mats]
        post = svh or [m.svh for m in self.mats]
        y = torch.empty((x.shape[0], self.n_out), dtype=x.dtype, device=x.device) if out is None else out
        if self.n_out > self.N:
            y[:, self.N:].zero_()                     # padding columns (the LM head's vocabulary padding)
        if x.stride(-1) != 1:
            x = x.contiguous()
        z, xh = scratch(x.device, 0, 0)
        e = ext()
        M = x.shape[0]
        for l in self.launches:
            pick = l.members
            # a launch whose last split can poll the others' partials runs over the all-ones buffer (the same bits)
            if OWN and polls(M, l.sk, l.w):
                run, zl = e.dense_own, own_partials(x.device, l.sk * M * l.n)
            else:
                run, zl = e.dense, z
            run(x, [codes[i] for i in pick], [pre[i] for i in pick], [post[i] for i in pick],
                [self.col0[i] for i in pick], y, xh, zl, self.counters, l.k2, l.cb, l.sk, l.w, l.pf, ROT_SMEM)
        return y

    def reserve_prompt(self, T: int) -> None:
        """Grow the prompt scratch for forward_tile over T rows (done before a graph is captured)."""
        device = self.mats[0].trellis.device
        tiles = -(-T // TILE_ROWS)
        z = max(tiles * tile_plan(self.K, l.n) * TILE_ROWS * l.n for l in self.launches)
        xh = max(len(l.members) for l in self.launches) * -(-T // 16) * 16 * self.K
        cnt = max(tiles * (l.n // 128) * COUNTER_STRIDE for l in self.launches)
        prompt_scratch(device, z, xh, cnt)

    def forward_tile(self, x, trellis=None, suh=None, svh=None, out=None):
        """x [T, K], any T (a prompt) -> [T, n_out] in x's dtype, each weight decoded once for every 128 rows
        (esp_dense_tile). A row's bits are its own (the same at any T), not those of forward. trellis / suh / svh:
        lists that replace the matrices' own tensors, as in forward."""
        codes = trellis or [m.trellis for m in self.mats]
        pre = suh or [m.suh for m in self.mats]
        post = svh or [m.svh for m in self.mats]
        T = x.shape[0]
        y = torch.empty((T, self.n_out), dtype=x.dtype, device=x.device) if out is None else out
        if self.n_out > self.N:
            y[:, self.N:].zero_()
        if x.stride(-1) != 1:
            x = x.contiguous()
        self.reserve_prompt(T)
        z, xh, cnt = prompt_scratch(x.device, 0, 0, 0)
        e = ext()
        for l in self.launches:
            pick = l.members
            e.dense_tile(x, [codes[i] for i in pick], [pre[i] for i in pick], [post[i] for i in pick],
                         [self.col0[i] for i in pick], y, xh, z, cnt, l.k2, l.cb, tile_plan(self.K, l.n))
        return y

    def norm_fusable(self, M: int) -> bool:
        """Whether forward_rmsnorm runs in one launch for M rows: a single launch, four waves a row, and the rotated
        rows within the fused rotation's shared memory."""
        if len(self.launches) != 1:
            return False
        l = self.launches[0]
        steps = -(-(self.K // 32) // l.sk)
        blocks = -(-(steps * 32 + 96) // 128)
        return M <= l.w // 4 and self.K <= 8192 and M * blocks * 128 * 2 <= ROT_SMEM

    def forward_rmsnorm(self, h, d1, d2, norm_w, eps: float, h_out, out):
        """forward(RMSNorm(h + d1 + d2) * norm_w) with the residual h + d1 + d2 stored to h_out, the norm made inside
        the launch (bit-identical to add_rmsnorm then forward). h, d1, d2: [M, K] contiguous, the model's dtype."""
        z, _ = scratch(h.device, 0, 0)
        l = self.launches[0]
        ms = [self.mats[i] for i in l.members]
        ext().dense_rmsnorm(h, d1, d2, norm_w, eps, h_out, [m.trellis for m in ms], [m.suh for m in ms],
                            [m.svh for m in ms], [self.col0[i] for i in l.members], out, z, self.counters, l.k2, l.cb,
                            l.sk, l.w, ROT_SMEM)
        return out


class DenseMulti:
    """Several one-launch Dense layers as a single esp_dense_multi launch: independent layers side by side, or a chain
    in which layer i reads layer i-1's output (after[i]): one launch gap and one weight-landing latency for all of
    them. Every layer keeps its own plan's K splits; the waves a workgroup are the same for all (W), so a layer's bits
    equal its own launch at that W."""

    def __init__(self, layers, after=None, W: int = 16):
        self.layers = list(layers)
        self.after = list(after) if after is not None else [False] * len(self.layers)
        if not 1 <= len(self.layers) <= 4 or len(self.after) != len(self.layers) or self.after[0]:
            raise ValueError("1 to 4 layers; only a layer after the first may read the previous one's output")
        if any(len(d.launches) != 1 for d in self.layers):
            raise ValueError("every layer of a multi launch must be a single launch group")
        self.W = W
        # a chain's hand-off maps a consumer's ticket to a launch through its K splits, over counts that only grow: the
        # plans are fixed here, and forward refuses a layer whose plan has changed since
        self.plans = [d.launches[0] for d in self.layers]
        device = self.layers[0].mats[0].trellis.device
        blocks = sum(d.launches[0].n // 128 for d in self.layers)
        # the split-K arrival counters (left zero by every launch), then a chain's 64-bit running hand-off counts (a
        # column block's done count and its ticket count)
        self.split_counters = COUNTER_STRIDE * blocks
        self.counters = torch.zeros(3 * self.split_counters, dtype=torch.int32, device=device)
        z = sum(-(-(d.launches[0].sk * MAX_ROWS * d.launches[0].n) // 64) * 64 for d in self.layers)
        scratch(device, z, 0)

    def forward(self, xs, outs, norm=None):
        """xs[i] [M, K_i] rows of layer i (for a layer after its predecessor, a view of that layer's output); outs[i]
        [M, n_out_i] in the model's dtype. norm = (h, d1, d2, w, eps, h_out): layer 0's rows are RMSNorm(h + d1 + d2)
        * w, made in the launch, with the residual stored to h_out (xs[0] is then unused)."""
        z, _ = scratch(outs[0].device, 0, 0)
        launches = [d.launches[0] for d in self.layers]
        if launches != self.plans:
            raise ValueError("a layer's plan changed after its multi launch was built: build a new DenseMulti")
        h, d1, d2, w, eps, h_out = norm if norm is not None else (None, None, None, None, 0.0, None)
        x0 = h if norm is not None else xs[0]
        ext().dense_multi([x0] + list(xs[1:]), [[d.mats[i].trellis for i in l.members] for d, l in zip(self.layers, launches)],
                          [[d.mats[i].suh for i in l.members] for d, l in zip(self.layers, launches)],
                          [[d.mats[i].svh for i in l.members] for d, l in zip(self.layers, launches)],
                          [[d.col0[i] for i in l.members] for d, l in zip(self.layers, launches)], list(outs),
                          [l.k2 for l in launches], [l.cb for l in launches], [l.sk for l in launches],
                          [int(a) for a in self.after], z, self.counters, self.W, ROT_SMEM, h, d1, d2, w, h_out, eps)
        return outs

"""GPU checks of the drop-in boundary with the reference caller's own buffers, and of the device status word.

1. The reference's Dense (vllm_espalier/dense.py:53-103) sizes its scratch as counters = 2 per 128 columns, Z =
   SK * 32 * N floats, xh = 4 * 32 * K halves (dense.py:76-85), with its own plan (dense.py:22-39) for the device's CU
   count. espalier_ext.dense driven with exactly those buffers and that plan must equal this package's Dense forced to
   the same plan, bit for bit, and leave the counters zero.
2. The reference's Scratch (experts.py:141-166) sizes Z from its tile_config (experts.py:59-68): the reference's
   six-launch sequence (routed2, experts.py:231-261) through espalier_ext with those buffers equals this package's
   routed2 forced to the same K splits, bit for bit.
3. A grouped table naming a (codebook, K2) with no kernel, or a width outside the launch's [lo, hi], runs no GEMM for
   that expert: its partials are NaN and esp_status reports the bit (the reference traps instead,
   experts_grouped.cuh:288,293).
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from vllm_espalier import dense as Dn
from vllm_espalier import experts as G
from vllm_espalier import workloads as WL

pytestmark = pytest.mark.gpu
D, I = 2048, 512


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def reference_plan(K: int, N: int, sms: int):
    """The reference's (K splits, warps, tiles in flight), restated from dense.py:22-39 (its sm89 sweep)."""
    nb, kt = N // 128, K // 16
    if nb >= 8 * sms:
        return 1, 4, 1
    if 2 * nb >= 3 * sms and kt % (8 * 2) == 0:
        return 1, 8, 1
    w, sk = 4, 1
    while nb * sk < 2 * sms and kt % (2 * sk * w) == 0 and kt // (2 * sk * w) >= 2:
        sk *= 2
    return sk, w, 1


def reference_tile_config(K: int, N: int, gateup: bool):
    """The reference's grouped tile setting (experts.py:59-68): the first candidate that divides the shape."""
    cands = [(4, 4, 4, 2) if gateup else (4, 4, 1, 2), (8, 4, 4, 1) if gateup else (8, 4, 1, 1), (8, 4, 2, 1),
             (8, 4, 1, 1), (4, 4, 2, 2), (4, 4, 1, 2)]
    for nt, w, sk, pf in cands:
        if K % (16 * sk * w) == 0 and N % (16 * nt) == 0:
            return nt, w, sk, pf
    raise ValueError((K, N))


BLOCK = [("qkv", 2048, [(4096, "int6"), (512, "int6"), (512, "int6")]), ("o", 4096, [(2048, "int6")]),
         ("gate_up", 2048, [(512, "int5"), (512, "int5")]), ("down", 512, [(2048, "int5")])]


@pytest.mark.parametrize("M", [1, 8, 32])
@pytest.mark.parametrize("name,K,outs", BLOCK)
def test_dense_with_reference_buffers(dev, ext, monkeypatch, name, K, outs, M):
    print(f"dense reference buffers {name} M={M}", flush=True)
    gen = torch.Generator().manual_seed(sum(map(ord, name)) + M)
    mats = [WL.matrix(K, n, 4, g, gen, dev) for n, g in outs]
    N = sum(m.out_features for m in mats)
    sms = torch.cuda.get_device_properties(dev).multi_processor_count
    sk, w, pf = reference_plan(K, N, sms)
    # the reference Dense's buffers (dense.py:76-85): counters 2 a block, Z SK * 32 * N, xh 4 * 32 * K
    counters = torch.zeros(2 * (N // 128), dtype=torch.int32, device=dev)
    z = torch.empty(sk * 32 * N, dtype=torch.float32, device=dev)
    xh = torch.empty(4 * 32 * K, dtype=torch.half, device=dev)
    x = torch.randn((M, K), generator=gen).to(torch.bfloat16).to(dev)
    y_ref = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    k2, cb = 2 * mats[0].K, G.KERNEL_CB[mats[0].cb]
    col0 = [sum(m.out_features for m in mats[:i]) for i in range(len(mats))]
    for _ in range(2):                                   # twice: the counters must come back zero
        ext.dense(x, [m.trellis for m in mats], [m.suh for m in mats], [m.svh for m in mats], col0, y_ref, xh, z,
                  counters, k2, cb, sk, w, pf, 32 * 1024)
        torch.cuda.synchronize()
        assert int(counters.abs().sum()) == 0
    # this package's Dense forced to the same plan gives the same bits
    monkeypatch.setenv("ESPALIER_DENSE_TILE_PLAN", f"{sk},{w},{pf}")
    d = Dn.Dense(mats)
    assert d.plans == [(sk, w, pf)]
    y = d.forward(x)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    # and both meet the parity bar against the oracle
    m0 = mats[0]
    W = O.dequant_f32(m0.trellis.cpu().numpy(), 2 * m0.K, G.KERNEL_CB[m0.cb])
    ref = O.linear_ref(O.bf16_to_f32(bits(x)), W, bits(m0.suh), bits(m0.svh))
    assert O.rel_l2(y_ref[:, :m0.out_features].float().cpu().numpy(), ref) < 2e-2


def _layer(n_experts, seed, dev):
    gen = torch.Generator().manual_seed(seed)
    widths = [(1, "e2m1"), (2, "e2m1"), (3, "int5")]
    experts = [tuple(WL.matrix(k, n, *widths[e % 3], gen, dev) for k, n in ((D, I), (D, I), (I, D)))
               for e in range(n_experts)]
    sh = tuple(WL.matrix(k, n, 4, "int5", gen, dev) for k, n in ((D, I), (D, I), (I, D)))
    gw = (torch.randn((D,), generator=gen) * 0.05).to(torch.bfloat16).to(dev)
    return G.prepare(experts, sh, gw), experts, sh, gw


@pytest.mark.parametrize("R", [1, 8, 32])
def test_grouped_with_reference_scratch(dev, ext, monkeypatch, R):
    """The reference's routed2 launch sequence (experts.py:231-261) with its Scratch sizes and tile settings."""
    print(f"grouped reference scratch R={R}", flush=True)
    L, experts, sh, gw = _layer(24, 31, dev)
    k, slots, rows = 8, 9, 32
    P = rows * slots
    cfg_gu, cfg_d = reference_tile_config(D, I, True), reference_tile_config(I, D, False)
    # the reference Scratch (experts.py:144-162)
    xg = torch.zeros((P, D), dtype=torch.half, device=dev)
    xu = torch.zeros((P, D), dtype=torch.half, device=dev)
    xd = torch.zeros((P, I), dtype=torch.half, device=dev)
    z = torch.zeros((max(2 * cfg_gu[2] * I, cfg_d[2] * D) * P,), dtype=torch.float32, device=dev)
    y = torch.zeros((P, D), dtype=torch.float32, device=dev)
    maxu = min(P, L.E)
    pick_s = torch.zeros((P,), dtype=torch.int32, device=dev)
    wts_s = torch.zeros((P,), dtype=torch.float32, device=dev)
    ids_s = torch.zeros((maxu,), dtype=torch.int32, device=dev)
    count = torch.zeros((1,), dtype=torch.int32, device=dev)
    members_s = torch.full((maxu * rows,), -1, dtype=torch.int32, device=dev)
    gen = torch.Generator().manual_seed(100 + R)
    x = torch.randn((R, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = torch.stack([torch.randperm(24, generator=gen)[:k] for _ in range(R)]).to(torch.int32).to(dev)
    wts = torch.softmax(torch.randn((R, k), generator=gen), -1).to(dev)
    Pw = R * slots
    mu = min(R * slots, L.E)
    ids, members = ids_s[:mu], members_s[:mu * R].view(mu, R)
    pk, wt = pick_s[:Pw], wts_s[:Pw]
    out = torch.empty((R, D), dtype=torch.bfloat16, device=dev)
    osh = torch.empty((R, D), dtype=torch.bfloat16, device=dev)
    ext.group_shared(pick, wts, x, x.stride(0), L.gate_w, L.shared_id, pk, wt, ids, count, members, R, k, L.E)
    ext.rot_in(x, x.stride(0), pk, L.suh_g, L.suh_u, xg, xu, R, D, slots, L.E)
    nt, w, sk, pf = cfg_gu
    ext.grouped(xg, xu, L.ptr[0], L.ptr[1], L.k2[0], L.k2[1], L.cb[0], L.cb[1], ids, count, members, z, 2, D, I, Pw,
                sk, slots, nt, w, pf, L.k2_gu[0], L.k2_gu[1])
    ext.gateup_epilogue(z, pk, L.svh_g, L.svh_u, L.suh_d, xd, R, Pw, I, sk, slots, L.E, math.inf, 1)
    nt, w, sk, pf = cfg_d
    ext.grouped(xd, xd, L.ptr[2], L.ptr[2], L.k2[2], L.k2[2], L.cb[2], L.cb[2], ids, count, members, z, 1, I, D, Pw,
                sk, slots, nt, w, pf, L.k2_d[0], L.k2_d[1])
    ext.down_combine2(z, pk, L.svh_d, y, wt, out, osh, R, Pw, D, sk, slots, L.E, k)
    torch.cuda.synchronize()
    # this package's routed2 forced to the reference's splits and waves: the same bits
    monkeypatch.setenv("ESPALIER_GROUPED_TILE_PLAN", f"{cfg_gu[1]},{cfg_gu[2]};{cfg_d[1]},{cfg_d[2]}")
    monkeypatch.setattr(G, "FUSED", False)
    s = G.Scratch(L.E, D, I, rows, slots, dev)
    o2, s2 = G.routed2(x, pick, wts, L, s)
    torch.cuda.synchronize()
    assert torch.equal(o2.view(torch.int16), out.view(torch.int16))
    assert torch.equal(s2.view(torch.int16), osh.view(torch.int16))
    assert np.isfinite(out.float().cpu().numpy()).all()


def _status(ext):
    return int(ext.status(True))


def test_grouped_table_without_kernel_sets_status(dev, ext):
    """A table entry with no kernel (E2M1 at K2 8) and one wider than the launch's hi: NaN partials for exactly those
    experts' member rows, the status bits set, the other experts' partials unchanged; a clean launch leaves it 0."""
    L, experts, sh, gw = _layer(6, 41, dev)
    assert _status(ext) == 0
    R, k, slots = 2, 3, 4
    pick = torch.tensor([[0, 1, 2], [3, 4, 5]], dtype=torch.int32, device=dev)
    wts = torch.full((R, k), 1 / 3, dtype=torch.float32, device=dev)
    x = torch.randn((R, D), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(dev)
    s = G.Scratch(L.E, D, I, 32, slots, dev)
    Pw = R * slots
    ids, members = s.window(R)
    ext.group_shared(pick, wts, x, D, L.gate_w, L.shared_id, s.pick[:Pw], s.wts[:Pw], ids, s.count, members, R, k,
                     L.E)
    ext.rot_in(x, D, s.pick[:Pw], L.suh_g, L.suh_u, s.xg, s.xu, R, D, slots, L.E)
    nt, w, sk, pf = s.cfg_gu

    def gateup(k2_tab, cb_tab, lo, hi):
        s.z.zero_()
        ext.grouped(s.xg, s.xu, L.ptr[0], L.ptr[1], k2_tab, L.k2[1], cb_tab, L.cb[1], ids, s.count, members, s.z, 2,
                    D, I, Pw, sk, slots, nt, w, pf, lo, hi)
        torch.cuda.synchronize()
        return s.z[:2 * sk * Pw * I].view(2, sk, Pw, I).cpu().clone()

    clean = gateup(L.k2[0], L.cb[0], L.k2_gu[0], L.k2_gu[1])
    assert _status(ext) == 0 and np.isfinite(clean.numpy()).all()
    # expert 1 (a 2-bit E2M1 matrix) given E2M1 at K2 8: no kernel; expert 4 given mcg at K2 10, a pair with a
    # kernel but wider than the launch's hi (8, the shared expert's): the stage was not sized for it
    lo, hi = L.k2_gu
    assert (lo, hi) == (2, 8)
    k2_bad, cb_bad = L.k2[0].clone(), L.cb[0].clone()
    k2_bad[1] = 8
    k2_bad[4] = 10
    cb_bad[4] = 1
    bad = gateup(k2_bad, cb_bad, lo, hi)
    st = _status(ext)
    assert st == 3, st                                    # ESP_STATUS_NO_KERNEL | ESP_STATUS_WIDTH_RANGE
    assert _status(ext) == 0                              # cleared by the read before
    # gate partials: rows whose slot picked expert 1 or 4 are NaN across every split and column; the rest unchanged
    pk = s.pick[:Pw].cpu().numpy()
    for p in range(Pw):
        if pk[p] in (1, 4):
            assert np.isnan(bad[0, :, p].numpy()).all(), p
        else:
            assert torch.equal(bad[0, :, p], clean[0, :, p]), p
    assert torch.equal(bad[1], clean[1])                  # the up projection's table was valid


def test_moe_gateup_table_without_kernel_sets_status(dev, ext):
    """The fused gate/up launch with a table entry that has no kernel: the status bit, non-finite xd rows for that
    expert's members, finite rows elsewhere, counters left zero."""
    L, experts, sh, gw = _layer(6, 43, dev)
    assert _status(ext) == 0
    R, k, slots = 2, 3, 4
    pick = torch.tensor([[0, 1, 2], [3, 4, 5]], dtype=torch.int32, device=dev)
    wts = torch.full((R, k), 1 / 3, dtype=torch.float32, device=dev)
    x = torch.randn((R, D), generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(dev)
    s = G.Scratch(L.E, D, I, 32, slots, dev)
    Pw = R * slots
    ids, members = s.window(R)
    ext.group_shared(pick, wts, x, D, L.gate_w, L.shared_id, s.pick[:Pw], s.wts[:Pw], ids, s.count, members, R, k,
                     L.E)
    nt, w, sk, pf = s.cfg_gu
    cb_bad = L.cb[1].clone()
    cb_bad[2] = 7                                         # int6 at K2 2/4/6 (expert 2 is 3-bit int5: K2 6 has int6)
    k2_bad = L.k2[1].clone()
    k2_bad[2] = 4                                         # int6 at K2 4: no kernel
    s.xd.fill_(0)
    ext.moe_gateup(x, D, L.suh_g, L.suh_u, L.ptr[0], L.ptr[1], L.k2[0], k2_bad, L.cb[0], cb_bad, ids, s.count,
                   members, s.z, s.counters, L.svh_g, L.svh_u, L.suh_d, s.xd, D, I, Pw, sk, slots, w, L.k2_gu[0],
                   L.k2_gu[1], math.inf, 1)
    torch.cuda.synchronize()
    assert _status(ext) == 1
    assert int(s.counters.abs().sum()) == 0
    xd = s.xd[:Pw].float().cpu().numpy()
    pk = s.pick[:Pw].cpu().numpy()
    for p in range(Pw):
        if pk[p] == 2:
            assert not np.isfinite(xd[p]).any(), p
        else:
            assert np.isfinite(xd[p]).all(), p

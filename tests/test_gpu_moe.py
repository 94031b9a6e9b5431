"""GPU parity of the expert pipeline (csrc/moe.hip) against the CPU oracle.

Bars: grouping, routing ids and the router's bf16 logits bit-exact against exact routing (exactly rounded bf16 logits,
top-k by logit with the lowest id on ties); routing weights within 1e-6; rot_in and down_combine2 bit-exact (same
operation order as the reference); gateup_epilogue within 1 fp16 ulp (expf); the full MoE layer within 2e-2 relative
L2 of the fp64 reference and within the reference's own bf16 gate (5e-4 above the output-rounding floor,
tests/gpu_grouped_shared.py:149-152). Self-consistency (tests/gpu_grouped*.py, gpu_route.py): rows alone == rows in the
window, graph replay == eager, bf16 routed2 == fp32 routed rounded.
"""
import numpy as np
import pytest
import torch

import oracle as O
from vllm_espalier import experts as G
from vllm_espalier import workloads as WL

pytestmark = pytest.mark.gpu
D, I = 2048, 512


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def distinct_picks(R, E, k, gen):
    return torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(R)]).to(torch.int32)


# ---------------------------------------------------------------------------------------------------------------
# grouping
# ---------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("R,slots,dups", [(1, 9, False), (4, 9, False), (17, 9, False), (32, 9, False),
                                          (8, 8, True), (40, 8, False)])
def test_group_bit_exact(dev, ext, R, slots, dups):
    gen = torch.Generator().manual_seed(R * 100 + slots)
    E = 257
    if dups:
        pick = torch.randint(0, 20, (R, slots), generator=gen).to(torch.int32)     # repeated ids in a row
    else:
        pick = distinct_picks(R, E, slots, gen)
    maxu = min(R * slots, E)
    uids = torch.full((maxu,), -7, dtype=torch.int32, device=dev)
    members = torch.full((maxu, R), -7, dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    ext.group(pick.to(dev).reshape(-1), uids, count, members, R, slots, E)
    cnt, u, m = O.group(pick.numpy(), R, slots, E, R)
    assert int(count.item()) == cnt
    assert np.array_equal(uids[:cnt].cpu().numpy(), u)
    assert np.array_equal(members[:cnt].cpu().numpy(), m)


def test_group_limits_raise(dev, ext):
    pick = torch.zeros(40, dtype=torch.int32, device=dev)
    uids = torch.zeros(40, dtype=torch.int32, device=dev)
    members = torch.zeros((40, 1), dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="32 slots"):
        ext.group(pick, uids, count, members, 1, 40, 10)


# ---------------------------------------------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------------------------------------------
def router_inputs(R, seed, H=2048, E=256, near_ties=True):
    """gate ~ N(0, 0.02) bf16; rows ~ unit-RMS with ~1% channels x4 (gpu_route.py:79); then near-tie rows whose exact
    logits are single dyadic products: x = one-hot, so logit_e = gate[e][j] exactly."""
    gen = torch.Generator().manual_seed(seed)
    gate = (torch.randn((E, H), generator=gen) * 0.02).to(torch.bfloat16)
    big = 1 + 3 * (torch.rand(H, generator=gen) < 0.01).float()
    x = (torch.randn((R, H), generator=gen) * big).to(torch.bfloat16)
    sgate = (torch.randn((H,), generator=gen) * 0.02).to(torch.bfloat16)
    if near_ties and R >= 3:
        # row 0: experts 10 and 20 tie exactly at rank 8 / 9 (expert 10 must win); row 1: experts 30 and 31 one bf16
        # ulp apart at rank 8 / 9 (the larger wins); row 2: a tie between 40 and 7 at the top
        for r, j in ((0, 5), (1, 6), (2, 7)):
            x[r].zero_()
            x[r, j] = 1.0
            gate[:, j] = (torch.rand(E, generator=gen) * 0.0625).to(torch.bfloat16)   # below every planted value
        top = [0.5, 0.4375, 0.375, 0.34375, 0.3125, 0.28125, 0.265625]
        for i, v in enumerate(top):
            gate[50 + i, 5] = v
            gate[60 + i, 6] = v
        gate[10, 5] = gate[20, 5] = 0.25
        gate[30, 6] = 0.25
        gate[31, 6] = torch.tensor(0.25, dtype=torch.bfloat16).view(torch.int16).add(1).view(torch.bfloat16)
        gate[40, 7] = gate[7, 7] = 0.75
    return x, gate, sgate


def run_route(ext, dev, x, gate, sgate, k, shared_id):
    R, H = x.shape
    E = gate.shape[0]
    has = shared_id >= 0
    slots = k + has
    maxu = min(R * slots, E + has)
    logits = torch.zeros(R * (E + has), dtype=torch.float32, device=dev)
    counter = torch.zeros(1, dtype=torch.int32, device=dev)
    pick = torch.zeros(R * slots, dtype=torch.int32, device=dev)
    wts = torch.zeros(R * slots, dtype=torch.float32, device=dev)
    uids = torch.zeros(maxu, dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    members = torch.full((maxu, R), -7, dtype=torch.int32, device=dev)
    ext.route_group(x.to(dev), gate.to(dev), sgate.to(dev) if has else None, k, shared_id, logits, counter, pick,
                    wts, uids, count, members)
    torch.cuda.synchronize()
    assert int(counter.item()) == 0, "the arrival counter must be left zero"
    return logits, pick.view(R, slots), wts.view(R, slots), uids, count, members


@pytest.mark.parametrize("R", [1, 3, 8, 32])
@pytest.mark.parametrize("shared", [True, False])
def test_route_group_exact(dev, ext, R, shared):
    x, gate, sgate = router_inputs(R, 40 + R)
    k, E = 8, 256
    sid = E if shared else -1
    logits, pick, wts, uids, count, members = run_route(ext, dev, x, gate, sgate, k, sid)
    opick, owts, ologits, osl = O.route(bits(x), bits(gate), k, bits(sgate) if shared else None, sid)
    C = E + shared
    lg = logits.view(R, C)
    # the logits buffer holds the exactly rounded bf16 logits
    got_l = O.f32_to_bf16(lg[:, :E].cpu().numpy())
    assert np.array_equal(got_l, ologits), f"{int((got_l != ologits).sum())} logits differ"
    assert np.array_equal(pick.cpu().numpy(), opick)
    assert np.abs(wts.cpu().numpy().astype(np.float64) - owts).max() < 1e-6
    if R >= 3:
        p = pick.cpu().numpy()
        assert 10 in p[0, :k] and 20 not in p[0, :k]
        assert 31 in p[1, :k] and 30 not in p[1, :k]
        assert list(p[2, :2]) == [7, 40]
    cnt, u, m = O.group(opick, R, k + shared, E + shared, R)
    assert int(count.item()) == cnt
    assert np.array_equal(uids[:cnt].cpu().numpy(), u) and np.array_equal(members[:cnt].cpu().numpy(), m)


@pytest.mark.parametrize("R,shared", [(1, True), (33, True), (100, False), (517, True)])
def test_route_rows_equals_windows_and_oracle(dev, ext, R, shared):
    """route_rows over a whole prompt (fp64-MFMA logits, then a wave a row) against route_group window by window, bit
    for bit (logits, picks, weights), and against the oracle's exact routing."""
    print(f"route_rows R={R} shared={shared}", flush=True)
    x, gate, sgate = router_inputs(R, 500 + R)
    k, E = 8, 256
    sid = E if shared else -1
    slots = k + shared
    xd, gd, sd = x.to(dev), gate.to(dev), sgate.to(dev) if shared else None
    logits = torch.full((R * (E + shared),), float("nan"), dtype=torch.float32, device=dev)
    pick = torch.full((R * slots,), -7, dtype=torch.int32, device=dev)
    wts = torch.full((R * slots,), float("nan"), dtype=torch.float32, device=dev)
    ext.route_rows(xd, gd, sd, k, sid, logits, pick, wts)
    torch.cuda.synchronize()
    for r0 in range(0, R, 32):
        n = min(32, R - r0)
        lw, pw, ww, *_ = run_route(ext, dev, x[r0:r0 + n].contiguous(), gate, sgate, k, sid)
        assert torch.equal(lw, logits[r0 * (E + shared):(r0 + n) * (E + shared)]), r0
        assert torch.equal(pw.reshape(-1), pick[r0 * slots:(r0 + n) * slots]), r0
        assert torch.equal(ww.reshape(-1), wts[r0 * slots:(r0 + n) * slots]), r0
    opick, owts, _, _ = O.route(bits(x), bits(gate), k, bits(sgate) if shared else None, sid)
    assert np.array_equal(pick.view(R, slots).cpu().numpy(), opick)
    assert np.abs(wts.view(R, slots).cpu().numpy().astype(np.float64) - owts).max() < 1e-6


@pytest.mark.parametrize("R", [1, 45])
def test_route_rows_fp16_strided(dev, ext, R):
    """route_rows with fp16 rows and router weights, the rows a view into wider rows (row stride 2304): the same
    logits, picks and weights as route_group's fp16 path, window by window."""
    print(f"route_rows fp16 R={R}", flush=True)
    x, gate, sgate = router_inputs(R, 900 + R, near_ties=False)
    x, gate, sgate = x.half(), gate.half(), sgate.half()
    k, E, sid, slots = 8, 256, 256, 9
    wide = torch.zeros((R, 2048 + 256), dtype=torch.float16)
    wide[:, :2048] = x
    xd = wide.to(dev)[:, :2048]
    logits = torch.full((R * (E + 1),), float("nan"), dtype=torch.float32, device=dev)
    pick = torch.full((R * slots,), -7, dtype=torch.int32, device=dev)
    wts = torch.full((R * slots,), float("nan"), dtype=torch.float32, device=dev)
    ext.route_rows(xd, gate.to(dev), sgate.to(dev), k, sid, logits, pick, wts)
    torch.cuda.synchronize()
    for r0 in range(0, R, 32):
        n = min(32, R - r0)
        lw, pw, ww, *_ = run_route(ext, dev, x[r0:r0 + n].contiguous(), gate, sgate, k, sid)
        assert torch.equal(lw, logits[r0 * (E + 1):(r0 + n) * (E + 1)]), r0
        assert torch.equal(pw.reshape(-1), pick[r0 * slots:(r0 + n) * slots]), r0
        assert torch.equal(ww.reshape(-1), wts[r0 * slots:(r0 + n) * slots]), r0


def test_route_group_rows_alone_and_graph(dev, ext):
    x, gate, sgate = router_inputs(8, 77, near_ties=False)
    logits, pick, wts, *_ = run_route(ext, dev, x, gate, sgate, 8, 256)
    pick, wts = pick.clone(), wts.clone()
    for r in range(8):
        _, p1, w1, *_ = run_route(ext, dev, x[r:r + 1].contiguous(), gate, sgate, 8, 256)
        assert torch.equal(p1[0], pick[r]) and torch.equal(w1[0], wts[r])
    # graph replay == eager
    xd, gd, sd = x.to(dev), gate.to(dev), sgate.to(dev)
    R, k, E = 8, 8, 256
    bufs = [torch.zeros(R * (E + 1), dtype=torch.float32, device=dev), torch.zeros(1, dtype=torch.int32, device=dev),
            torch.zeros(R * 9, dtype=torch.int32, device=dev), torch.zeros(R * 9, dtype=torch.float32, device=dev),
            torch.zeros(min(R * 9, E + 1), dtype=torch.int32, device=dev), torch.zeros(1, dtype=torch.int32, device=dev),
            torch.full((min(R * 9, E + 1), R), -1, dtype=torch.int32, device=dev)]
    ext.route_group(xd, gd, sd, k, 256, *bufs)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ext.route_group(xd, gd, sd, k, 256, *bufs)
    for i in range(3):
        bufs[2].zero_()
        bufs[3].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(bufs[2].view(R, 9), pick) and torch.equal(bufs[3].view(R, 9), wts), f"replay {i}"


@pytest.mark.parametrize("R,E,shared,dtype,delta", [(1, 256, True, "bf16", True), (1, 256, False, "bf16", True),
                                                     (1, 100, True, "bf16", True), (2, 256, True, "bf16", True),
                                                     (4, 256, True, "bf16", True), (1, 256, True, "fp16", True),
                                                     (3, 256, True, "fp16", True), (1, 256, True, "bf16", False),
                                                     (2, 256, True, "fp16", False), (1, 256, True, "bf16", 4096),
                                                     (2, 100, True, "bf16", 1024)])
def test_route_group_rmsnorm_sentinel(dev, ext, R, E, shared, dtype, delta):
    """route_group_rmsnorm (the norm inside the routing launch; its logits an all-ones hand-off buffer, which at one
    row the last workgroup polls instead of counting arrivals) against add_rmsnorm then route_group: the normalised
    rows, the residual, picks, weights and grouping bit for bit; the logits left all-ones and the counter zero, over
    two launches in a row and graph replays (each reading the all-ones the previous one left). Without the delta, h
    holds planted -0 and +0 elements, which the residual must keep bit for bit."""
    # delta: True / False, or a width other than 2048 (with the delta: the launch's general norm path)
    H = 2048 if isinstance(delta, bool) else delta
    print(f"route_group_rmsnorm R={R} E={E} shared={shared} {dtype} delta={delta} H={H}", flush=True)
    k, eps = 8, 1e-6
    t = torch.bfloat16 if dtype == "bf16" else torch.float16
    x, gate, sgate = router_inputs(R, 700 + R + E, H=H, E=E, near_ties=R >= 3)
    x, gate, sgate = x.to(t), gate.to(t), sgate.to(t)
    gen = torch.Generator().manual_seed(710 + R + E)
    if not delta:
        x[:, 5::97] = -0.0
        x[:, 7::101] = 0.0
    h = x.to(dev)
    d1 = (torch.randn((R, H), generator=gen) * 0.5).to(t).to(dev) if delta else None
    w = (1 + 0.1 * torch.randn(H, generator=gen)).to(t).to(dev)
    sid = E if shared else -1
    h_ref, a_ref = h.clone(), torch.empty_like(h)
    ext.add_rmsnorm(h_ref, d1, None, w, a_ref, eps)
    _, pick_r, wts_r, uids_r, count_r, members_r = run_route(ext, dev, a_ref, gate, sgate, k, sid)
    cnt = int(count_r.item())
    slots = k + shared
    maxu = min(R * slots, E + shared)
    logits = torch.full((R * (E + shared),), -1, dtype=torch.int32, device=dev).view(torch.float32)
    counter = torch.zeros(1, dtype=torch.int32, device=dev)
    pick = torch.zeros(R * slots, dtype=torch.int32, device=dev)
    wts = torch.zeros(R * slots, dtype=torch.float32, device=dev)
    uids = torch.zeros(maxu, dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    members = torch.full((maxu, R), -7, dtype=torch.int32, device=dev)
    h_out, a_out = torch.empty_like(h), torch.empty_like(h)
    gd, sd = gate.to(dev), sgate.to(dev) if shared else None

    def launch():
        ext.route_group_rmsnorm(h, d1, w, eps, h_out, a_out, gd, sd, k, sid, logits, counter, pick, wts, uids, count,
                                members)

    def check(tag):
        torch.cuda.synchronize()
        assert torch.equal(a_out.view(torch.int16), a_ref.view(torch.int16)), tag
        assert torch.equal(h_out.view(torch.int16), h_ref.view(torch.int16)), tag
        assert torch.equal(pick.view(R, slots), pick_r) and torch.equal(wts.view(R, slots), wts_r), tag
        assert int(count.item()) == cnt, tag
        assert torch.equal(uids[:cnt], uids_r[:cnt]) and torch.equal(members[:cnt], members_r[:cnt]), tag
        assert bool((logits.view(torch.int32) == -1).all()), f"{tag}: the logits must be left all-ones"
        assert int(counter.item()) == 0, f"{tag}: the counter must be left zero"

    def clear():
        for t in (pick, wts, uids, count, h_out, a_out):
            t.zero_()
        members.fill_(-7)

    ext.status(clear=True)
    for i in range(2):
        clear()
        launch()
        check(f"launch {i}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    for i in range(3):
        clear()
        g.replay()
        check(f"replay {i}")
        torch.randn((64, 64), device=dev).sum()           # eager work between replays
    assert ext.status() == 0


@pytest.mark.parametrize("R,shared", [(1, True), (1, False), (3, True), (32, True)])
def test_route_group_own_equals_route_group(dev, ext, R, shared):
    """esp_route_group_own (route_group over its own all-ones logits buffer: polled by the last workgroup at one row,
    restored by the top-k waves at more) against esp_route_group: picks, weights and grouping bit for bit, near-ties
    included, over launches in a row and graph replays; the logits left all-ones and the counter zero."""
    print(f"route_group_own R={R} shared={shared}", flush=True)
    x, gate, sgate = router_inputs(R, 800 + R, near_ties=R >= 3)
    k, E = 8, 256
    sid = E if shared else -1
    _, pick_r, wts_r, uids_r, count_r, members_r = run_route(ext, dev, x, gate, sgate, k, sid)
    cnt = int(count_r.item())
    slots, C = k + shared, E + shared
    maxu = min(R * slots, C)
    logits = torch.full((R * C,), -1, dtype=torch.int32, device=dev).view(torch.float32)
    counter = torch.zeros(1, dtype=torch.int32, device=dev)
    pick = torch.zeros(R * slots, dtype=torch.int32, device=dev)
    wts = torch.zeros(R * slots, dtype=torch.float32, device=dev)
    uids = torch.zeros(maxu, dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    members = torch.full((maxu, R), -7, dtype=torch.int32, device=dev)
    xd, gd, sd = x.to(dev), gate.to(dev), sgate.to(dev) if shared else None

    def launch():
        ext.route_group_own(xd, gd, sd, k, sid, logits, counter, pick, wts, uids, count, members)

    def check(tag):
        torch.cuda.synchronize()
        assert torch.equal(pick.view(R, slots), pick_r) and torch.equal(wts.view(R, slots), wts_r), tag
        assert int(count.item()) == cnt, tag
        assert torch.equal(uids[:cnt], uids_r[:cnt]) and torch.equal(members[:cnt], members_r[:cnt]), tag
        assert bool((logits.view(torch.int32) == -1).all()), f"{tag}: the logits must be left all-ones"
        assert int(counter.item()) == 0, f"{tag}: the counter must be left zero"

    def clear():
        for t in (pick, wts, uids, count):
            t.zero_()
        members.fill_(-7)

    ext.status(clear=True)
    for i in range(2):
        clear()
        launch()
        check(f"launch {i}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    for i in range(3):
        clear()
        g.replay()
        check(f"replay {i}")
        torch.randn((64, 64), device=dev).sum()           # eager work between replays
    assert ext.status() == 0


def test_route_group_limits_raise(dev, ext):
    x, gate, sgate = router_inputs(2, 1, near_ties=False)
    with pytest.raises(RuntimeError, match="shape limits"):
        run_route(ext, dev, x, torch.cat([gate, gate]), sgate, 8, -1)       # E = 512 > 256


# ---------------------------------------------------------------------------------------------------------------
# group_shared, rot_in, epilogues
# ---------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("R", [1, 8, 32])
def test_group_shared(dev, ext, R):
    gen = torch.Generator().manual_seed(R)
    k, E = 8, 257
    pick = distinct_picks(R, 256, k, gen)
    wts = torch.softmax(torch.randn((R, k), generator=gen), -1)
    x = torch.randn((R, D), generator=gen).to(torch.bfloat16)
    gw = (torch.randn((D,), generator=gen) * 0.05).to(torch.bfloat16)
    slots = k + 1
    maxu = min(R * slots, E)
    po = torch.zeros(R * slots, dtype=torch.int32, device=dev)
    wo = torch.zeros(R * slots, dtype=torch.float32, device=dev)
    uids = torch.zeros(maxu, dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    members = torch.full((maxu, R), -7, dtype=torch.int32, device=dev)
    ext.group_shared(pick.to(dev).contiguous(), wts.to(dev).contiguous(), x.to(dev), D, gw.to(dev), 256, po, wo, uids,
                     count, members, R, k, E)
    torch.cuda.synchronize()
    want_pick = np.concatenate([pick.numpy(), np.full((R, 1), 256, np.int32)], 1)
    assert np.array_equal(po.view(R, slots).cpu().numpy(), want_pick)
    wv = wo.view(R, slots).cpu().numpy()
    assert np.array_equal(wv[:, :k], wts.numpy())
    xs = O.bf16_to_f32(bits(x)).astype(np.float64) @ O.bf16_to_f32(bits(gw)).astype(np.float64)
    assert np.abs(wv[:, k] - 1 / (1 + np.exp(-xs))).max() < 1e-6
    cnt, u, m = O.group(want_pick, R, slots, E, R)
    assert int(count.item()) == cnt
    assert np.array_equal(uids[:cnt].cpu().numpy(), u) and np.array_equal(members[:cnt].cpu().numpy(), m)


@pytest.mark.parametrize("R,slots,K", [(5, 3, 512), (70, 9, 1024), (64, 17, 384)])
def test_rot_in_bit_exact(dev, ext, R, slots, K):
    """rot_in against the oracle's rotation, invalid picks left untouched, from a decode window's few rows to a
    prompt's (more slots than 16, K of 3 and 8 blocks)."""
    gen = torch.Generator().manual_seed(3 + R)
    E = 6
    x = torch.randn((R, K), generator=gen).to(torch.bfloat16)
    pick = torch.randint(-1, E + 1, (R, slots), generator=gen).to(torch.int32)       # includes invalid picks
    suh0 = (torch.randint(0, 2, (E, K), generator=gen) * 2 - 1).half()
    suh1 = torch.randn((E, K), generator=gen).half()
    o0 = torch.full((R * slots, K), 7.0, dtype=torch.half, device=dev)
    o1 = torch.full((R * slots, K), 7.0, dtype=torch.half, device=dev)
    ext.rot_in(x.to(dev), K, pick.to(dev).reshape(-1), suh0.to(dev), suh1.to(dev), o0, o1, R, K, slots, E)
    g0, g1 = bits(o0), bits(o1)
    seven = np.float16(7.0).view(np.uint16)
    for p in range(R * slots):
        e = int(pick.view(-1)[p])
        if 0 <= e < E:
            row = bits(x[p // slots:p // slots + 1])
            assert np.array_equal(g0[p], O.rotate(row, "bf16", bits(suh0[e]))[0])
            assert np.array_equal(g1[p], O.rotate(row, "bf16", bits(suh1[e]))[0])
        else:
            assert (g0[p] == seven).all() and (g1[p] == seven).all()


def test_gateup_epilogue(dev, ext):
    gen = torch.Generator().manual_seed(4)
    R, slots, E, N, SK = 3, 3, 5, 512, 4
    P = R * slots
    Z = torch.randn((2, SK, P, N), generator=gen) * 3
    pick = torch.randint(-1, E, (P,), generator=gen).to(torch.int32)
    svh_g, svh_u, suh_d = (torch.randn((E, N), generator=gen).half() for _ in range(3))
    xd = torch.zeros((P, N), dtype=torch.half, device=dev)
    for mode in (1, 0):
        ext.gateup_epilogue(Z.to(dev), pick.to(dev), svh_g.to(dev), svh_u.to(dev), suh_d.to(dev), xd, R, P, N, SK,
                            slots, E, float("inf") if mode else 7.0, mode)
        want = O.gateup_epilogue(Z.numpy(), pick.numpy(), bits(svh_g), bits(svh_u), bits(suh_d), P, N, SK, E,
                                 float("inf") if mode else 7.0, mode)
        got = bits(xd).astype(np.int32)
        valid = ((pick >= 0) & (pick < E)).numpy()
        # expf may differ by an ulp between libraries: allow 1 fp16 ulp, and count exact matches
        diff = np.abs(got[valid] - want[valid].astype(np.int32))
        assert diff.max() <= 1, f"act_mode {mode}: max ulp difference {diff.max()}"
        assert (diff == 0).mean() > 0.99


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_down_combine2_bit_exact(dev, ext, out_dtype):
    gen = torch.Generator().manual_seed(5)
    R, slots, E, Dd, SK = 4, 9, 20, 512, 2
    P = R * slots
    Z = torch.randn((SK, P, Dd), generator=gen) * 2
    pick = torch.randint(-2, E, (P,), generator=gen).to(torch.int32)
    svh_d = torch.randn((E, Dd), generator=gen).half()
    y0 = torch.randn((P, Dd), generator=gen)                       # stale rows an invalid pick reuses
    wts = torch.rand((P,), generator=gen)
    y = y0.clone().to(dev)
    out = torch.zeros((R, Dd), dtype=out_dtype, device=dev)
    osh = torch.zeros((R, Dd), dtype=out_dtype, device=dev)
    ext.down_combine2(Z.to(dev), pick.to(dev), svh_d.to(dev), y, wts.to(dev), out, osh, R, P, Dd, SK, slots, E,
                      slots - 1)
    wo, ws, wy = O.down_combine2(Z.numpy(), pick.numpy(), bits(svh_d), y0.numpy(), wts.numpy(), R, P, Dd, SK, E,
                                 slots, slots - 1)
    assert np.array_equal(y.cpu().numpy(), wy)
    if out_dtype == torch.float32:
        assert np.array_equal(out.cpu().numpy(), wo) and np.array_equal(osh.cpu().numpy(), ws)
    else:
        cast = (lambda a: O.f32_to_bf16(a)) if out_dtype == torch.bfloat16 else (lambda a: a.astype(np.float16).view(np.uint16))
        assert np.array_equal(bits(out), cast(wo)) and np.array_equal(bits(osh), cast(ws))
    # down_combine (fp32, all slots) and combine follow the same chain
    out32 = torch.zeros((R, Dd), dtype=torch.float32, device=dev)
    ext.down_combine(Z.to(dev), pick.to(dev), svh_d.to(dev), y0.clone().to(dev), wts.to(dev), out32, R, P, Dd, SK,
                     slots, E)
    wo_all, _, _ = O.down_combine2(Z.numpy(), pick.numpy(), bits(svh_d), y0.numpy(), wts.numpy(), R, P, Dd, SK, E,
                                   slots, slots, shared=False)
    assert np.array_equal(out32.cpu().numpy(), wo_all)
    yd = y0.clone().to(dev)
    ext.down_epilogue(Z.to(dev), pick.to(dev), svh_d.to(dev), yd, R, P, Dd, SK, slots, E)
    assert np.array_equal(yd.cpu().numpy(), wy)
    oc = torch.zeros((R, Dd), dtype=torch.float32, device=dev)
    ext.combine(yd, wts.to(dev), oc, R, Dd, slots)
    assert np.array_equal(oc.cpu().numpy(), wo_all)


def test_down_combine2_without_y(dev, ext):
    """y = None (esp_down_combine2 with a null y, the whole-prompt path): no per-slot outputs stored, and an invalid
    pick adds zero, which is the oracle's sum over stale rows of zeros, bit for bit."""
    gen = torch.Generator().manual_seed(9)
    R, slots, E, Dd, SK = 5, 9, 20, 512, 1
    P = R * slots
    Z = torch.randn((SK, P, Dd), generator=gen)
    pick = torch.randint(-2, E, (P,), generator=gen).to(torch.int32)
    svh_d = torch.randn((E, Dd), generator=gen).half()
    wts = torch.rand((P,), generator=gen)
    out = torch.zeros((R, Dd), dtype=torch.bfloat16, device=dev)
    osh = torch.zeros((R, Dd), dtype=torch.bfloat16, device=dev)
    ext.down_combine2(Z.to(dev), pick.to(dev), svh_d.to(dev), None, wts.to(dev), out, osh, R, P, Dd, SK, slots, E,
                      slots - 1)
    wo, ws, _ = O.down_combine2(Z.numpy(), pick.numpy(), bits(svh_d), np.zeros((P, Dd), np.float32), wts.numpy(), R,
                                P, Dd, SK, E, slots, slots - 1)
    assert (pick < 0).any() and np.array_equal(bits(out), O.f32_to_bf16(wo))
    assert np.array_equal(bits(osh), O.f32_to_bf16(ws))


@pytest.mark.parametrize("R,Dd,SK,slots,out_dtype,with_y", [(70, 640, 2, 9, torch.bfloat16, True),
                                                          (64, 2048, 1, 9, torch.bfloat16, False),
                                                          (100, 512, 3, 32, torch.float32, True),
                                                          (65, 256, 1, 4, torch.float16, False)])
def test_down_combine2_many_rows(dev, ext, R, Dd, SK, slots, out_dtype, with_y):
    """From 64 rows down_combine2 runs a workgroup a row (blocks in groups of 4, the last one short when D / 128 is
    not a multiple of 4): bit-exact against the oracle, invalid picks included, with y stored or absent."""
    print(f"down_combine2 rows={R} D={Dd} SK={SK} slots={slots} {out_dtype} y={with_y}", flush=True)
    gen = torch.Generator().manual_seed(R + Dd + slots)
    E = 24
    P = R * slots + 3
    Z = torch.randn((SK, P, Dd), generator=gen)
    pick = torch.randint(-2, E, (P,), generator=gen).to(torch.int32)
    svh_d = torch.randn((E, Dd), generator=gen).half()
    y0 = torch.randn((P, Dd), generator=gen) if with_y else torch.zeros((P, Dd))
    wts = torch.rand((P,), generator=gen)
    y = y0.clone().to(dev) if with_y else None
    out = torch.zeros((R, Dd), dtype=out_dtype, device=dev)
    osh = torch.zeros((R, Dd), dtype=out_dtype, device=dev)
    ext.down_combine2(Z.to(dev), pick.to(dev), svh_d.to(dev), y, wts.to(dev), out, osh, R, P, Dd, SK, slots, E,
                      slots - 1)
    wo, ws, wy = O.down_combine2(Z.numpy(), pick.numpy(), bits(svh_d), y0.numpy(), wts.numpy(), R, P, Dd, SK, E,
                                 slots, slots - 1)
    if with_y:
        assert np.array_equal(y.cpu().numpy()[:R * slots], wy[:R * slots])
    if out_dtype == torch.float32:
        assert np.array_equal(out.cpu().numpy(), wo) and np.array_equal(osh.cpu().numpy(), ws)
    else:
        cast = (lambda a: O.f32_to_bf16(a)) if out_dtype == torch.bfloat16 else (lambda a: a.astype(np.float16).view(np.uint16))
        assert np.array_equal(bits(out), cast(wo)) and np.array_equal(bits(osh), cast(ws))


@pytest.mark.parametrize("slots", [4, 8, 13, 32])
def test_down_combine2_slot_counts(dev, ext, slots):
    """down_combine2 launches a 32-lane half a slot (at least 256 threads, up to 1024 at 32 slots): bit-exact against
    the oracle at every width, the routed sum over all but the last slot and the last one gated apart."""
    print(f"down_combine2 slots={slots}", flush=True)
    gen = torch.Generator().manual_seed(50 + slots)
    R, E, Dd, SK = 3, 40, 256, 3
    P = R * slots
    Z = torch.randn((SK, P, Dd), generator=gen)
    pick = torch.randint(-1, E, (P,), generator=gen).to(torch.int32)
    svh_d = torch.randn((E, Dd), generator=gen).half()
    y0 = torch.randn((P, Dd), generator=gen)
    wts = torch.rand((P,), generator=gen)
    y = y0.clone().to(dev)
    out = torch.zeros((R, Dd), dtype=torch.float32, device=dev)
    osh = torch.zeros((R, Dd), dtype=torch.float32, device=dev)
    ext.down_combine2(Z.to(dev), pick.to(dev), svh_d.to(dev), y, wts.to(dev), out, osh, R, P, Dd, SK, slots, E,
                      slots - 1)
    wo, ws, wy = O.down_combine2(Z.numpy(), pick.numpy(), bits(svh_d), y0.numpy(), wts.numpy(), R, P, Dd, SK, E,
                                 slots, slots - 1)
    assert np.array_equal(y.cpu().numpy(), wy)
    assert np.array_equal(out.cpu().numpy(), wo) and np.array_equal(osh.cpu().numpy(), ws)


# ---------------------------------------------------------------------------------------------------------------
# the whole layer
# ---------------------------------------------------------------------------------------------------------------
WIDTHS = [(1, "e2m1"), (2, "e2m1"), (3, "int5")]


def make_layer(n_experts, seed, dev, shared=True):
    gen = torch.Generator().manual_seed(seed)
    experts = []
    for e in range(n_experts):
        b, g = WIDTHS[e % 3]
        experts.append((WL.matrix(D, I, b, g, gen, dev), WL.matrix(D, I, b, g, gen, dev),
                        WL.matrix(I, D, b, g, gen, dev)))
    sh = gw = None
    if shared:
        sh = (WL.matrix(D, I, 4, "int5", gen, dev), WL.matrix(D, I, 4, "int5", gen, dev),
              WL.matrix(I, D, 4, "int5", gen, dev))
        gw = (torch.randn((D,), generator=gen) * 0.05).to(torch.bfloat16).to(dev)
    L = G.prepare(experts, sh, gw)
    return L, experts, sh, gw


_W = {}


def weight(m):
    key = m.trellis.data_ptr()
    if key not in _W:
        _W[key] = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, G.KERNEL_CB[m.cb]).astype(np.float64)
    return _W[key]


def mlp_ref(x, mats):
    g, u, d = mats

    def lin(v, m):
        return O.linear_ref(v, weight(m), bits(m.suh), bits(m.svh))
    a = lin(x, g)
    return lin(a / (1 + np.exp(-a)) * lin(x, u), d)


def moe_ref(x, pick, wts, experts, sh, gw):
    xf = O.bf16_to_f32(bits(x)).astype(np.float64)
    out = np.zeros_like(xf)
    for r in range(xf.shape[0]):
        for j in range(pick.shape[1]):
            out[r] += float(wts[r, j]) * mlp_ref(xf[r:r + 1], experts[int(pick[r, j])])[0]
    shr = None
    if sh is not None:
        gate = 1 / (1 + np.exp(-(xf @ O.bf16_to_f32(bits(gw)).astype(np.float64))))
        shr = gate[:, None] * mlp_ref(xf, sh)
    return out, shr


@pytest.fixture(scope="module")
def layer16(dev):
    return make_layer(16, 21, dev)


@pytest.mark.parametrize("R", [1, 4, 32])
def test_moe_layer_parity(dev, layer16, R):
    print(f"moe layer R={R}", flush=True)
    L, experts, sh, gw = layer16
    gen = torch.Generator().manual_seed(R)
    s = G.scratch(L, 32, 9, dev)
    x = torch.randn((R, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = distinct_picks(R, 16, 8, gen).to(dev)
    wts = torch.softmax(torch.randn((R, 8), generator=gen), -1).to(dev)
    out, osh = G.routed2(x, pick, wts, L, s)
    torch.cuda.synchronize()
    rref, sref = moe_ref(x, pick.cpu().numpy(), wts.cpu().numpy(), experts, sh, gw)
    for got, ref in ((out, rref), (osh, sref)):
        g = got.float().cpu().numpy()
        assert O.rel_l2(g, ref) < 2e-2
        gate = O.rel_max_above_floor(g, ref, "bf16")
        assert gate < 5e-4, f"max error above the bf16 floor {gate:.3e}"


def test_moe_fused_routing_layer(dev):
    """route_group then routed2(pick=None): the six-launch pipeline of apply_monolithic (moe.py:288-329)."""
    L, experts, sh, gw = make_layer(256 // 16, 22, dev)
    R = 8
    gen = torch.Generator().manual_seed(8)
    router = (torch.randn((16, D), generator=gen) * 0.02).to(torch.bfloat16).to(dev)
    x = torch.randn((R, D), generator=gen).to(torch.bfloat16).to(dev)
    s = G.scratch(L, 32, 9, dev)
    G.route(x, router, 8, L, s)
    out, osh = G.routed2(x, None, None, L, s, k=8)
    torch.cuda.synchronize()
    opick, owts, _, _ = O.route(bits(x), bits(router), 8, bits(gw), 16)
    rref, sref = moe_ref(x, opick[:, :8], owts[:, :8], experts, sh, gw)
    assert O.rel_l2(out.float().cpu().numpy(), rref) < 2e-2
    assert O.rel_l2(osh.float().cpu().numpy(), sref) < 2e-2


@pytest.mark.parametrize("R", [2, 8, 17, 32])
def test_moe_rows_alone_equal_window(dev, layer16, R):
    L, *_ = layer16
    gen = torch.Generator().manual_seed(50 + R)
    s = G.scratch(L, 32, 9, dev)
    x = torch.randn((R, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = distinct_picks(R, 16, 8, gen).to(dev)
    wts = torch.softmax(torch.randn((R, 8), generator=gen), -1).to(dev)
    o, sh = (t.clone() for t in G.routed2(x, pick, wts, L, s))
    for r in range(R):
        o1, s1 = G.routed2(x[r:r + 1], pick[r:r + 1], wts[r:r + 1], L, s)
        assert torch.equal(o1[0], o[r]) and torch.equal(s1[0], sh[r]), f"row {r}"


@pytest.mark.parametrize("R", [1, 8, 32])
def test_moe_graph_replay_equals_eager(dev, layer16, R):
    L, *_ = layer16
    gen = torch.Generator().manual_seed(60 + R)
    s = G.scratch(L, 32, 9, dev)
    x = torch.randn((R, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = distinct_picks(R, 16, 8, gen).to(dev)
    wts = torch.softmax(torch.randn((R, 8), generator=gen), -1).to(dev)
    out = torch.empty((R, D), dtype=torch.bfloat16, device=dev)
    osh = torch.empty_like(out)
    eo, es = (t.clone() for t in G.routed2(x, pick, wts, L, s))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        G.routed2(x, pick, wts, L, s, out, osh)
    for i in range(3):
        out.zero_()
        osh.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eo) and torch.equal(osh, es), f"replay {i}"
        G.routed2(x, pick, wts, L, s)
        torch.cuda.synchronize()


def test_routed2_bf16_equals_routed_fp32_rounded(dev):
    L, *_ = make_layer(12, 23, dev, shared=False)
    s0 = G.scratch(L, 32, 8, dev)
    for R in (1, 8, 32):
        gen = torch.Generator().manual_seed(70 + R)
        x = torch.randn((R, D), generator=gen).to(torch.bfloat16).to(dev)
        pick = distinct_picks(R, 12, 8, gen).to(dev)
        wts = torch.softmax(torch.randn((R, 8), generator=gen), -1).to(dev)
        ref32 = G.routed(x, pick, wts, L, s0).clone()
        out, sh = G.routed2(x, pick, wts, L, s0)
        assert sh is None and out.dtype == torch.bfloat16 and torch.equal(out, ref32.to(torch.bfloat16))


@pytest.mark.parametrize("R,invalid", [(1, False), (4, False), (32, False), (5, True)])
def test_moe_fused_launches_equal_unfused(dev, layer16, R, invalid, monkeypatch):
    """routed2 with rot_in, the gate/up GEMM and its epilogue in one launch (esp_moe_gateup) against the reference's
    launch sequence (rot_in, grouped, gateup_epilogue), bit for bit, at every window width (the production switch uses
    it for up to FUSED_ROWS rows), with out-of-range picks too."""
    print(f"moe fused R={R} invalid={invalid}", flush=True)
    L, *_ = layer16
    gen = torch.Generator().manual_seed(80 + R)
    s = G.scratch(L, 32, 9, dev)
    x = torch.randn((R, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = distinct_picks(R, 16, 8, gen)
    if invalid:
        pick[1, 3] = -1
        pick[R - 1, 0] = 17                                  # past every table entry (16 routed + shared)
    pick = pick.to(dev)
    wts = torch.softmax(torch.randn((R, 8), generator=gen), -1).to(dev)
    monkeypatch.setattr(G, "CHAIN", False)                  # esp_moe_gateup itself (the chain: test_gpu_moe_chain)
    monkeypatch.setattr(G, "FUSED", False)
    uo, us = (t.clone() for t in G.routed2(x, pick, wts, L, s))
    monkeypatch.setattr(G, "FUSED", True)
    monkeypatch.setattr(G, "FUSED_ROWS", 32)
    fo, fs = (t.clone() for t in G.routed2(x, pick, wts, L, s))
    torch.cuda.synchronize()
    assert torch.equal(fo.view(torch.int16), uo.view(torch.int16))
    assert torch.equal(fs.view(torch.int16), us.view(torch.int16))
    assert int(s.counters.abs().sum()) == 0                 # every arrival counter left at zero


def test_moe_fused_sixteen_splits(dev, layer16, monkeypatch):
    """esp_moe_gateup at 16 K splits (past eight, the epilogue loads the gate and the up partials as two sets of
    device-scope loads, not one) against the unfused launches at the same splits, bit for bit, counters left zero."""
    monkeypatch.setenv("ESPALIER_GROUPED_TILE_PLAN", "4,16;4,4")
    L, *_ = layer16
    s = G.Scratch(L.E, L.D, L.I, 32, 9, dev)
    assert s.cfg_gu[2] == 16
    gen = torch.Generator().manual_seed(99)
    R = 2
    x = torch.randn((R, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = distinct_picks(R, 16, 8, gen).to(dev)
    wts = torch.softmax(torch.randn((R, 8), generator=gen), -1).to(dev)
    monkeypatch.setattr(G, "CHAIN", False)
    monkeypatch.setattr(G, "FUSED", False)
    uo, us = (t.clone() for t in G.routed2(x, pick, wts, L, s))
    monkeypatch.setattr(G, "FUSED", True)
    fo, fs = (t.clone() for t in G.routed2(x, pick, wts, L, s))
    torch.cuda.synchronize()
    assert torch.equal(fo.view(torch.int16), uo.view(torch.int16))
    assert torch.equal(fs.view(torch.int16), us.view(torch.int16))
    assert int(s.counters.abs().sum()) == 0

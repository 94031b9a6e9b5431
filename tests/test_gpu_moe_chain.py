"""esp_moe_chain, the decode MoE layer after its routing as one launch (the fused gate/up programs, the down programs
that decode their weights before reading their xd slice, and the combine), against the separate launches it
replaces (esp_moe_gateup, esp_grouped, esp_down_combine2: the reference's launch chain, experts.py:231-261), bit for
bit: given picks (out-of-range ones too), fused routing, graph replays with eager work between them, and the BASELINE
config-4 layer (256 experts of 1-3 bits plus the 4-bit shared expert). Every reader count and arrival counter is left
zero, the launch's own xd and down partials are back to their all-ones sentinel, and no wait times out (status 0). A table entry without a kernel gives the NaN partials and status bit of the
separate launches.
"""
import math

import numpy as np
import pytest
import torch

from vllm_espalier import experts as G
from vllm_espalier import workloads as WL

pytestmark = pytest.mark.gpu
D, I = 2048, 512
WIDTHS = [(1, "e2m1"), (2, "e2m1"), (3, "int5")]


def make_layer(n_experts, seed, dev):
    gen = torch.Generator().manual_seed(seed)
    experts = [tuple(WL.matrix(k, n, b, g, gen, dev) for k, n in ((D, I), (D, I), (I, D)))
               for b, g in (WIDTHS[e % 3] for e in range(n_experts))]
    sh = tuple(WL.matrix(k, n, 4, "int5", gen, dev) for k, n in ((D, I), (D, I), (I, D)))
    gw = (torch.randn((D,), generator=gen) * 0.05).to(torch.bfloat16).to(dev)
    return G.prepare(experts, sh, gw)


def distinct_picks(R, E, k, gen):
    return torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(R)]).to(torch.int32)


def _sentinel(s):
    """The chained launch's own xd and down partials hold every bit set between launches."""
    return bool((s.xdc.view(torch.int16) == -1).all()) and bool((s.zd.view(torch.int32) == -1).all())


def _clean(ext, s):
    torch.cuda.synchronize()
    assert int(s.flags.abs().sum()) == 0, "reader counts left non-zero"
    assert int(s.counters.abs().sum()) == 0, "arrival counters left non-zero"
    assert _sentinel(s), "xd or the down partials not put back to the all-ones sentinel"
    assert int(ext.status(True)) == 0, "a wait timed out or a table entry had no kernel"


def _pass(L, s, x, pick, wts, chain, monkeypatch, k=8):
    monkeypatch.setattr(G, "CHAIN", chain)
    out, sh = G.routed2(x, pick, wts, L, s, k=k)
    P = x.shape[0] * s.slots
    return out.clone(), sh.clone(), s.y[:P].clone()


@pytest.fixture(scope="module")
def layer16(dev):
    return make_layer(16, 31, dev)


@pytest.mark.parametrize("R,invalid", [(1, False), (2, False), (4, False), (4, True)])
def test_chain_equals_separate(dev, ext, layer16, R, invalid, monkeypatch):
    print(f"moe chain R={R} invalid={invalid}", flush=True)
    L = layer16
    s = G.scratch(L, 32, 9, dev)
    gen = torch.Generator().manual_seed(10 + R)
    x = torch.randn((R, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = distinct_picks(R, 16, 8, gen)
    if invalid:
        pick[1, 3] = -1
        pick[R - 1, 0] = 17                                  # past every table entry (16 routed + shared)
    pick = pick.to(dev)
    wts = torch.softmax(torch.randn((R, 8), generator=gen), -1).to(dev)
    so, ss, sy = _pass(L, s, x, pick, wts, False, monkeypatch)
    co, cs, cy = _pass(L, s, x, pick, wts, True, monkeypatch)
    _clean(ext, s)
    assert torch.equal(co.view(torch.int16), so.view(torch.int16))
    assert torch.equal(cs.view(torch.int16), ss.view(torch.int16))
    valid = (s.pick[:R * 9] >= 0) & (s.pick[:R * 9] < L.E)
    assert torch.equal(cy[valid].view(torch.int32), sy[valid].view(torch.int32))      # every slot's down output


@pytest.mark.parametrize("R", [1, 3])
def test_chain_fused_routing(dev, ext, layer16, R, monkeypatch):
    """route_group, then the chained launch on its tables (the decoder's form) against the separate launches."""
    print(f"moe chain fused routing R={R}", flush=True)
    L = layer16
    s = G.scratch(L, 32, 9, dev)
    gen = torch.Generator().manual_seed(20 + R)
    router = (torch.randn((16, D), generator=gen) * 0.02).to(torch.bfloat16).to(dev)
    x = torch.randn((R, D), generator=gen).to(torch.bfloat16).to(dev)
    G.route(x, router, 8, L, s)
    so, ss, _ = _pass(L, s, x, None, None, False, monkeypatch)
    co, cs, _ = _pass(L, s, x, None, None, True, monkeypatch)
    _clean(ext, s)
    assert torch.equal(co.view(torch.int16), so.view(torch.int16))
    assert torch.equal(cs.view(torch.int16), ss.view(torch.int16))


def test_chain_graph_replay(dev, ext, layer16, monkeypatch):
    """Graph replays of the chained launch equal its eager result, with eager launches between the replays (the flags
    are reset inside each launch, so nothing carries over)."""
    L = layer16
    monkeypatch.setattr(G, "CHAIN", True)
    s = G.scratch(L, 32, 9, dev)
    gen = torch.Generator().manual_seed(33)
    x = torch.randn((2, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = distinct_picks(2, 16, 8, gen).to(dev)
    wts = torch.softmax(torch.randn((2, 8), generator=gen), -1).to(dev)
    out = torch.empty((2, D), dtype=torch.bfloat16, device=dev)
    osh = torch.empty_like(out)
    eo, es = (t.clone() for t in G.routed2(x, pick, wts, L, s))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        G.routed2(x, pick, wts, L, s, out, osh)
    for i in range(4):
        out.fill_(float("nan"))
        osh.fill_(float("nan"))
        g.replay()
        _clean(ext, s)
        assert torch.equal(out.view(torch.int16), eo.view(torch.int16)), f"replay {i}"
        assert torch.equal(osh.view(torch.int16), es.view(torch.int16)), f"replay {i}"
        G.routed2(x, pick, wts, L, s)


@pytest.mark.parametrize("R", [1, 4])
def test_chain_full_size(dev, ext, R, monkeypatch):
    """256 routed experts (widths 1-3 bits drawn per expert) plus the 4-bit shared expert, routed by
    a 256 x 2048 router in the routing launch, then the chained layer against the separate launches."""
    print(f"moe chain full size R={R}", flush=True)
    gen = torch.Generator().manual_seed(40 + R)
    widths = torch.randint(1, 4, (256,), generator=gen).tolist()
    grid = {1: "e2m1", 2: "e2m1", 3: "int5"}
    experts = [tuple(WL.matrix(k, n, b, grid[b], gen, dev) for k, n in ((D, I), (D, I), (I, D))) for b in widths]
    sh = tuple(WL.matrix(k, n, 4, "int5", gen, dev) for k, n in ((D, I), (D, I), (I, D)))
    gw = (torch.randn((D,), generator=gen) * 0.05).to(torch.bfloat16).to(dev)
    L = G.prepare(experts, sh, gw)
    s = G.scratch(L, 32, 9, dev)
    router = (torch.randn((256, D), generator=gen) * 0.02).to(torch.bfloat16).to(dev)
    x = torch.randn((R, D), generator=gen).to(torch.bfloat16).to(dev)
    G.route(x, router, 8, L, s)
    so, ss, _ = _pass(L, s, x, None, None, False, monkeypatch)
    co, cs, _ = _pass(L, s, x, None, None, True, monkeypatch)
    _clean(ext, s)
    assert torch.equal(co.view(torch.int16), so.view(torch.int16))
    assert torch.equal(cs.view(torch.int16), ss.view(torch.int16))
    assert torch.isfinite(co.float()).all() and torch.isfinite(cs.float()).all()


def test_chain_table_without_kernel_sets_status(dev, ext, layer16):
    """A down table entry with no kernel: that expert's partials are NaN (so are the combined rows that pick it),
    the status bit is set, the other rows stay finite, and the flags and counters are still left zero."""
    L = layer16
    s = G.scratch(L, 32, 9, dev)
    assert int(ext.status(True)) == 0
    R, k, slots = 2, 8, 9
    pick = torch.tensor([[0, 1, 2, 3, 4, 5, 6, 7], [8, 9, 10, 11, 12, 13, 14, 15]], dtype=torch.int32, device=dev)
    wts = torch.full((R, k), 1 / 8, dtype=torch.float32, device=dev)
    x = torch.randn((R, D), generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(dev)
    P = R * slots
    ids, members = s.window(R)
    ext.group_shared(pick, wts, x, D, L.gate_w, L.shared_id, s.pick[:P], s.wts[:P], ids, s.count, members, R, k, L.E)
    cb_bad, k2_bad = L.cb[2].clone(), L.k2[2].clone()
    cb_bad[2], k2_bad[2] = 7, 4                               # int6 at K2 4: no kernel
    out = torch.empty((R, D), dtype=torch.bfloat16, device=dev)
    osh = torch.empty_like(out)
    (tg, tu, td), (bg, bu, _), (cg, cu, _) = L.ptr, L.k2, L.cb
    ext.moe_chain(x, D, L.suh_g, L.suh_u, tg, tu, td, bg, bu, k2_bad, cg, cu, cb_bad, ids, s.count, members,
                  s.pick[:P], s.wts[:P], L.svh_g, L.svh_u, L.suh_d, L.svh_d, s.xdc, s.z, s.zd, s.y, out, osh,
                  s.counters, s.flags, D, I, s.cfg_gu[2], slots, L.E, k, *L.k2_gu, 2, 8, math.inf, 1)
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="status 0x1: .*has no kernel"):
        G.check_status()                                      # reads the word and clears it
    assert int(ext.status()) == 0
    assert int(s.flags.abs().sum()) == 0 and int(s.counters.abs().sum()) == 0 and _sentinel(s)
    o = out.float().cpu().numpy()
    assert not np.isfinite(o[0]).any()                        # row 0 picks expert 2
    assert np.isfinite(o[1]).all() and torch.isfinite(osh.float()).all()

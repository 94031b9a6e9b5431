"""The whole-prompt MoE path (experts.prefill, ESPALIER_PREFILL_MODE=tile) and the pieces it adds to the boundary:
grouping beyond one workgroup (esp_group / esp_group_shared over more than 1056 picks) and esp_grouped with more than
32 members an expert (member tiles).

Bars: the wide grouping bit-exact against the oracle's grouping (repeats, invalid ids, members past maxm dropped);
the wide group_shared's tables bit-equal to the one-workgroup path's; prefill outputs within 2e-2 relative L2 of the
fp64 reference; a token's prefill output independent of the other tokens of the prompt (rows alone == rows in the
prompt, bit for bit); fused routing over windows == the same picks given, bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle as O
from vllm_espalier import experts as G
from vllm_espalier import workloads as WL

pytestmark = pytest.mark.gpu
D, I = 2048, 512


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("R,slots,E,maxm,repeats", [(200, 9, 257, 200, False), (130, 9, 20, 130, True),
                                                    (300, 8, 64, 40, False)])
def test_group_wide_bit_exact(dev, ext, R, slots, E, maxm, repeats):
    print(f"wide grouping R={R} slots={slots} E={E} maxm={maxm}", flush=True)
    gen = torch.Generator().manual_seed(R + E)
    if repeats:
        pick = torch.randint(-2, E + 3, (R, slots), generator=gen).to(torch.int32)     # repeats and invalid ids
    else:
        pick = torch.stack([torch.randperm(E, generator=gen)[:slots] for _ in range(R)]).to(torch.int32)
    assert R * slots > 1056
    maxu = min(R * slots, E)
    uids = torch.full((maxu,), -7, dtype=torch.int32, device=dev)
    members = torch.full((maxu, maxm), -7, dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    ext.group(pick.to(dev).reshape(-1), uids, count, members, R, slots, E)
    cnt, u, m = O.group(pick.numpy(), R, slots, E, maxm)
    assert int(count.item()) == cnt
    assert np.array_equal(uids[:cnt].cpu().numpy(), u)
    assert np.array_equal(members[:cnt].cpu().numpy(), m)


def test_group_shared_wide_tables_equal_small(dev, ext):
    """130 rows (1170 picks: the wide path) against the same rows in windows of 100 (the one-workgroup path): the pick
    and weight tables bit for bit, the shared slot's sigmoid weight included; the grouping against the oracle."""
    gen = torch.Generator().manual_seed(5)
    R, k, E = 130, 8, 257
    pick = torch.stack([torch.randperm(256, generator=gen)[:k] for _ in range(R)]).to(torch.int32).to(dev)
    wts = torch.softmax(torch.randn((R, k), generator=gen), -1).to(dev)
    x = torch.randn((R, D), generator=gen).to(torch.bfloat16).to(dev)
    gw = (torch.randn((D,), generator=gen) * 0.05).to(torch.bfloat16).to(dev)
    slots = k + 1

    def tables(r0, r1):
        n = (r1 - r0) * slots
        po = torch.zeros(n, dtype=torch.int32, device=dev)
        wo = torch.zeros(n, dtype=torch.float32, device=dev)
        mu = min(n, E)
        uids = torch.zeros(mu, dtype=torch.int32, device=dev)
        members = torch.full((mu, r1 - r0), -7, dtype=torch.int32, device=dev)
        count = torch.zeros(1, dtype=torch.int32, device=dev)
        ext.group_shared(pick[r0:r1].contiguous(), wts[r0:r1].contiguous(), x[r0:r1], D, gw, 256, po, wo, uids,
                         count, members, r1 - r0, k, E)
        return po, wo, uids, count, members
    po, wo, uids, count, members = tables(0, R)
    a = tables(0, 100)
    b = tables(100, R)
    assert torch.equal(po, torch.cat([a[0], b[0]])) and torch.equal(wo, torch.cat([a[1], b[1]]))
    cnt, u, m = O.group(po.cpu().numpy(), R, slots, E, R)
    assert int(count.item()) == cnt
    assert np.array_equal(uids[:cnt].cpu().numpy(), u) and np.array_equal(members[:cnt].cpu().numpy(), m)


def _layer(n_experts, seed, dev):
    gen = torch.Generator().manual_seed(seed)
    widths = [(1, "e2m1"), (2, "e2m1"), (3, "int5")]
    experts = [tuple(WL.matrix(kk, n, *widths[e % 3], gen, dev) for kk, n in ((D, I), (D, I), (I, D)))
               for e in range(n_experts)]
    sh = tuple(WL.matrix(kk, n, 4, "int5", gen, dev) for kk, n in ((D, I), (D, I), (I, D)))
    gw = (torch.randn((D,), generator=gen) * 0.05).to(torch.bfloat16).to(dev)
    router = (torch.randn((n_experts, D), generator=gen) * 0.02).to(torch.bfloat16).to(dev)
    return G.prepare(experts, sh, gw), experts, sh, gw, router


@pytest.fixture(scope="module")
def layer16(dev):
    return _layer(16, 61, dev)


_W: dict = {}


def _weight(m):
    key = m.trellis.data_ptr()
    if key not in _W:
        _W[key] = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, G.KERNEL_CB[m.cb]).astype(np.float64)
    return _W[key]


def _mlp(x, mats):
    g, u, d = mats

    def lin(v, m):
        return O.linear_ref(v, _weight(m), bits(m.suh), bits(m.svh))
    a = lin(x, g)
    return lin(a / (1 + np.exp(-a)) * lin(x, u), d)


@pytest.mark.parametrize("T", [40, 100])
def test_prefill_matches_oracle(dev, layer16, T):
    """16 experts, top-8 of them a token: every expert has T / 2 members on average (up to 100: member tiles)."""
    print(f"prefill moe vs oracle T={T}", flush=True)
    L, experts, sh, gw, _ = layer16
    gen = torch.Generator().manual_seed(T)
    x = torch.randn((T, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = torch.stack([torch.randperm(16, generator=gen)[:8] for _ in range(T)]).to(torch.int32)
    wts = torch.softmax(torch.randn((T, 8), generator=gen), -1)
    s = G.prefill_scratch(L, 128, 9, dev)
    out, osh = G.prefill(x, pick.to(dev), wts.to(dev), L, s, 8)
    torch.cuda.synchronize()
    assert int(ext_status(G)) == 0
    xf = O.bf16_to_f32(bits(x)).astype(np.float64)
    rref = np.zeros_like(xf)
    for r in range(T):
        for j in range(8):
            rref[r] += float(wts[r, j]) * _mlp(xf[r:r + 1], experts[int(pick[r, j])])[0]
    gate = 1 / (1 + np.exp(-(xf @ O.bf16_to_f32(bits(gw)).astype(np.float64))))
    sref = gate[:, None] * _mlp(xf, sh)
    assert O.rel_l2(out.float().cpu().numpy(), rref) < 2e-2
    assert O.rel_l2(osh.float().cpu().numpy(), sref) < 2e-2


def ext_status(G):
    return G.ext().status(True)


@pytest.mark.parametrize("T", [33, 100])
def test_prefill_rows_alone_equal_prompt(dev, layer16, T):
    print(f"prefill rows alone T={T}", flush=True)
    L, *_ = layer16
    gen = torch.Generator().manual_seed(200 + T)
    x = torch.randn((T, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = torch.stack([torch.randperm(16, generator=gen)[:8] for _ in range(T)]).to(torch.int32).to(dev)
    wts = torch.softmax(torch.randn((T, 8), generator=gen), -1).to(dev)
    s = G.prefill_scratch(L, 128, 9, dev)
    out, osh = (t.clone() for t in G.prefill(x, pick, wts, L, s, 8))
    for r in range(T):
        o1, s1 = G.prefill(x[r:r + 1], pick[r:r + 1], wts[r:r + 1], L, s, 8)
        assert torch.equal(o1.view(torch.int16), out[r:r + 1].view(torch.int16)), r
        assert torch.equal(s1.view(torch.int16), osh[r:r + 1].view(torch.int16)), r


def test_prefill_fused_routing_equals_given_picks(dev, layer16):
    """route_group over 32-token windows inside prefill against the same windows' picks handed in."""
    L, experts, sh, gw, router = layer16
    T = 70
    x = torch.randn((T, D), generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).to(dev)
    s = G.prefill_scratch(L, 128, 9, dev)
    out, osh = (t.clone() for t in G.prefill(x, None, None, L, s, 8, gate=router))
    routed = s.pick[:T * 9].view(T, 9)[:, :8].contiguous()
    weights = s.wts[:T * 9].view(T, 9)[:, :8].contiguous()
    opick, _, _, _ = O.route(bits(x), bits(router), 8, bits(gw), 16)
    assert np.array_equal(s.pick[:T * 9].view(T, 9).cpu().numpy(), opick)      # exact routing
    o2, s2 = G.prefill(x, routed, weights, L, s, 8)
    assert torch.equal(o2.view(torch.int16), out.view(torch.int16))
    assert torch.equal(s2.view(torch.int16), osh.view(torch.int16))


def test_prefill_close_to_windows(dev, layer16):
    """The whole-prompt path against the 32-token windows of decode's pipeline (a different K split, so not the same
    bits): within 1e-2 relative L2 of each other."""
    L, *_ = layer16
    T = 96
    gen = torch.Generator().manual_seed(8)
    x = torch.randn((T, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = torch.stack([torch.randperm(16, generator=gen)[:8] for _ in range(T)]).to(torch.int32).to(dev)
    wts = torch.softmax(torch.randn((T, 8), generator=gen), -1).to(dev)
    s = G.prefill_scratch(L, 128, 9, dev)
    out, osh = (t.clone() for t in G.prefill(x, pick, wts, L, s, 8))
    wo, ws = G.windows(x, pick, wts, L, G.scratch(L, 32, 9, dev))
    assert O.rel_l2(out.float().cpu().numpy(), wo.float().cpu().numpy()) < 1e-2
    assert O.rel_l2(osh.float().cpu().numpy(), ws.float().cpu().numpy()) < 1e-2


@pytest.mark.parametrize("T,sk", [(40, 1), (100, 1), (100, 8), (517, 1)])
def test_tile_list_and_grouped_list(dev, ext, layer16, T, sk):
    """esp_tile_list: the non-empty (expert slot, member tile) pairs of a whole prompt's grouping, in order, against a
    count of each expert's members; esp_grouped_list over them: the partials of esp_grouped bit for bit (gate/up and
    down, staged and unstaged programs, one K split and eight)."""
    print(f"tile list T={T} sk={sk}", flush=True)
    L = layer16[0]
    E = 16
    gen = torch.Generator().manual_seed(700 + T)
    pick = torch.stack([torch.randperm(E, generator=gen)[:8] for _ in range(T)]).to(torch.int32).to(dev)
    slots, P = 8, T * 8
    maxu = min(P, E)
    uids = torch.zeros(maxu, dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    members = torch.full((maxu, T), -1, dtype=torch.int32, device=dev)
    ext.group(pick.reshape(-1), uids, count, members, T, slots, E)
    cap = G.tile_list_cap(maxu, T, P)
    tiles = torch.full((1 + cap,), -5, dtype=torch.int32, device=dev)
    ext.tile_list(count, members, maxu, P, tiles)
    torch.cuda.synchronize()
    cnt = int(count.item())
    m = members.cpu().numpy()
    want = [(u << 16) | t for u in range(cnt) for t in range(-(-int((m[u] >= 0).sum()) // 32))]
    got = tiles.cpu().numpy()
    assert got[0] == len(want) and list(got[1:1 + len(want)]) == want
    for mats, K, N, X, ptr, k2, cb, kk in ((2, D, I, None, L.ptr[:2], L.k2[:2], L.cb[:2], L.k2_gu),
                                           (1, I, D, None, L.ptr[2:] * 2, L.k2[2:] * 2, L.cb[2:] * 2, L.k2_d)):
        xs = torch.randn((P, K), generator=gen).half().to(dev)
        s_ = sk if mats == 2 else 1
        z0 = torch.zeros((mats * s_ * P * N,), dtype=torch.float32, device=dev)
        z1 = torch.zeros_like(z0)
        ext.grouped(xs, xs, ptr[0], ptr[1], k2[0], k2[1], cb[0], cb[1], uids, count, members, z0, mats, K, N, P, s_,
                    slots, 8, G.PREFILL_WAVES, 2, *kk)
        ext.grouped_list(xs, xs, ptr[0], ptr[1], k2[0], k2[1], cb[0], cb[1], uids, count, members, tiles, z1, mats,
                         K, N, P, s_, slots, G.PREFILL_WAVES, *kk)
        torch.cuda.synchronize()
        assert torch.equal(z0.view(torch.int32), z1.view(torch.int32)), (mats, s_)
    assert int(ext.status(True)) == 0


def test_tile_list_over_its_bound_raises_status(dev, ext):
    """A member table with more non-empty tiles than a grouping of P picks can have (P given as 1): the list keeps its
    bound's entries and the status word reports ESP_STATUS_TILE_LIST (8)."""
    ext.status(True)
    maxu, maxm = 16, 100
    members = torch.arange(maxu * maxm, dtype=torch.int32, device=dev).reshape(maxu, maxm)
    count = torch.tensor([maxu], dtype=torch.int32, device=dev)
    cap = G.tile_list_cap(maxu, maxm, 1)
    tiles = torch.zeros((1 + cap,), dtype=torch.int32, device=dev)
    ext.tile_list(count, members, maxu, 1, tiles)
    torch.cuda.synchronize()
    assert int(tiles[0].item()) == cap == 17
    assert int(ext.status(True)) & 8


def test_grouped_list_short_grid_raises_status(dev, ext, layer16):
    """esp_grouped_list launched for fewer picks than its tile list was built for (P given as 32 for a 517-token
    grouping): its grid, the bound for 32 picks, is shorter than the list, so listed tiles would be left undone; the
    status word reports ESP_STATUS_TILE_LIST (8). The down projection (one matrix, one split) keeps every access inside
    the full-size buffers."""
    L = layer16[0]
    E, T, slots = 16, 517, 8
    ext.status(True)
    gen = torch.Generator().manual_seed(711)
    pick = torch.stack([torch.randperm(E, generator=gen)[:8] for _ in range(T)]).to(torch.int32).to(dev)
    P = T * slots
    maxu = min(P, E)
    uids = torch.zeros(maxu, dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    members = torch.full((maxu, T), -1, dtype=torch.int32, device=dev)
    ext.group(pick.reshape(-1), uids, count, members, T, slots, E)
    tiles = torch.zeros((1 + G.tile_list_cap(maxu, T, P),), dtype=torch.int32, device=dev)
    ext.tile_list(count, members, maxu, P, tiles)
    torch.cuda.synchronize()
    assert int(tiles[0].item()) > G.tile_list_cap(maxu, T, 32)
    xs = torch.randn((P, I), generator=gen).half().to(dev)
    z = torch.zeros((P * D,), dtype=torch.float32, device=dev)
    t, b, c = L.ptr[2], L.k2[2], L.cb[2]
    ext.grouped_list(xs, xs, t, t, b, b, c, c, uids, count, members, tiles, z, 1, I, D, 32, 1, slots,
                     G.PREFILL_WAVES, *L.k2_d)
    torch.cuda.synchronize()
    assert int(ext.status(True)) & 8


def test_prefill_past_the_grouping_limit(dev, layer16):
    """A prompt of PREFILL_MAX_ROWS + 1 tokens (the shared expert alone then has more members than one whole-prompt
    grouping takes) runs as chunks: its first and last rows equal the same rows run alone, bit for bit."""
    L = layer16[0]
    T = G.PREFILL_MAX_ROWS + 1
    print(f"prefill moe past the grouping limit T={T}", flush=True)
    gen = torch.Generator().manual_seed(16385)
    x = torch.randn((T, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = torch.stack([torch.randperm(16, generator=gen)[:8] for _ in range(T)]).to(torch.int32).to(dev)
    wts = torch.softmax(torch.randn((T, 8), generator=gen), -1).to(dev)
    s = G.prefill_scratch(L, G.PREFILL_MAX_ROWS, 9, dev)
    out, osh = (t.clone() for t in G.prefill(x, pick, wts, L, s, 8))
    torch.cuda.synchronize()
    assert int(ext_status(G)) == 0
    for r in (0, T - 1):
        o1, s1 = G.prefill(x[r:r + 1], pick[r:r + 1], wts[r:r + 1], L, s, 8)
        assert torch.equal(o1[0].view(torch.int16), out[r].view(torch.int16)), r
        assert torch.equal(s1[0].view(torch.int16), osh[r].view(torch.int16)), r

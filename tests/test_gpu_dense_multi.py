"""esp_dense_multi (several dense launches in one grid) against the same launches run one by one, bit for bit:
independent groups side by side (BASELINE config 2's block: qkv, o, shared gate/up, shared down), and chains in which
a group reads the previous group's output (qkv then o on q, as the synthetic decoder runs them), with and without the
RMSNorm of the first group's input made in the launch. Counters are left zero and no wait times out (status 0); graph
replays equal eager launches. A chain's hand-off counts only grow, so a multi launch replayed many times (graph
replays, eager calls) keeps waiting for the right launch's producer.
"""
import numpy as np
import pytest
import torch

import oracle as O
from vllm_espalier import dense as Dn
from vllm_espalier import experts as G
from vllm_espalier import workloads as WL

pytestmark = pytest.mark.gpu
W = 16
BLOCK = [(2048, [(4096, "int6"), (512, "int6"), (512, "int6")]), (4096, [(2048, "int6")]),
         (2048, [(512, "int5"), (512, "int5")]), (512, [(2048, "int5")])]


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _layers(specs, seed, dev):
    gen = torch.Generator().manual_seed(seed)
    layers = [Dn.Dense([WL.matrix(K, n, 4, g, gen, dev) for n, g in outs]) for K, outs in specs]
    for d in layers:                                   # the multi launch's waves, so one-by-one gives the same bits
        d.plans = [(sk, W, pf) for sk, _, pf in d.plans]
    return layers


def _clean(ext, multi):
    torch.cuda.synchronize()
    assert int(multi.counters[:multi.split_counters].abs().sum()) == 0, "split-K counters left non-zero"
    assert int(ext.status(True)) == 0, "a wait timed out"


@pytest.mark.parametrize("M", [1, 8, 32])
def test_multi_independent_block_equals_separate(dev, ext, M):
    print(f"dense_multi independent block M={M}", flush=True)
    layers = _layers(BLOCK, 70 + M, dev)
    gen = torch.Generator().manual_seed(M)
    xs = [torch.randn((M, d.K), generator=gen).to(torch.bfloat16).to(dev) for d in layers]
    want = [d.forward(x).clone() for d, x in zip(layers, xs)]
    multi = Dn.DenseMulti(layers, W=W)
    for _ in range(2):
        outs = [torch.full_like(w, float("nan")) for w in want]
        multi.forward(xs, outs)
        _clean(ext, multi)
        for i, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o.view(torch.int16), w.view(torch.int16)), f"group {i}"


@pytest.mark.parametrize("off", [0, 1024])
@pytest.mark.parametrize("M", [1, 4, 32])
def test_multi_chain_qkv_then_o(dev, ext, M, off):
    """o reads 4096 columns of qkv's output from column `off` inside the launch, each workgroup waiting for the qkv
    column blocks that hold its x (at off 1024 those span all three of qkv's matrices)."""
    print(f"dense_multi chain qkv -> o M={M} off={off}", flush=True)
    qkv, o = _layers(BLOCK[:2], 80 + M, dev)
    x = torch.randn((M, 2048), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(dev)
    y1 = qkv.forward(x).clone()
    y2 = o.forward(y1[:, off:off + 4096]).clone()
    multi = Dn.DenseMulti([qkv, o], after=[False, True], W=W)
    for _ in range(3):
        a = torch.full((M, 5120), float("nan"), dtype=torch.bfloat16, device=dev)
        b = torch.full((M, 2048), float("nan"), dtype=torch.bfloat16, device=dev)
        multi.forward([x, a[:, off:off + 4096]], [a, b])
        _clean(ext, multi)
        assert torch.equal(a.view(torch.int16), y1.view(torch.int16))
        assert torch.equal(b.view(torch.int16), y2.view(torch.int16))
    # and the chain's o meets the parity bar against the oracle (fed the GPU's q)
    m = o.mats[0]
    Wt = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, G.KERNEL_CB[m.cb])
    ref = O.linear_ref(O.bf16_to_f32(bits(y1[:, off:off + 4096])), Wt, bits(m.suh), bits(m.svh))
    assert O.rel_l2(b.float().cpu().numpy(), ref) < 2e-2


@pytest.mark.parametrize("M", [1, 3])
def test_multi_chain_with_norm(dev, ext, M):
    """The first group normalises its input in the launch (dense_rmsnorm's arithmetic), the second reads its output."""
    print(f"dense_multi chain with norm M={M}", flush=True)
    qkv, o = _layers(BLOCK[:2], 90 + M, dev)
    gen = torch.Generator().manual_seed(9)
    h = (torch.randn((M, 2048), generator=gen) * 2).to(torch.bfloat16).to(dev)
    d1 = torch.randn((M, 2048), generator=gen).to(torch.bfloat16).to(dev)
    w = (1 + 0.1 * torch.randn((2048,), generator=gen)).to(torch.bfloat16).to(dev)
    h_ref = torch.empty_like(h)
    y1 = torch.empty((M, 5120), dtype=torch.bfloat16, device=dev)
    qkv.forward_rmsnorm(h, d1, None, w, 1e-6, h_ref, y1)
    y2 = o.forward(y1[:, :4096]).clone()
    multi = Dn.DenseMulti([qkv, o], after=[False, True], W=W)
    for _ in range(2):
        h_out = torch.empty_like(h)
        a = torch.full((M, 5120), float("nan"), dtype=torch.bfloat16, device=dev)
        b = torch.full((M, 2048), float("nan"), dtype=torch.bfloat16, device=dev)
        multi.forward([None, a[:, :4096]], [a, b], norm=(h, d1, None, w, 1e-6, h_out))
        _clean(ext, multi)
        assert torch.equal(h_out.view(torch.int16), h_ref.view(torch.int16))
        assert torch.equal(a.view(torch.int16), y1.view(torch.int16))
        assert torch.equal(b.view(torch.int16), y2.view(torch.int16))


def test_multi_chain_graph_replay(dev, ext):
    qkv, o = _layers(BLOCK[:2], 99, dev)
    x = torch.randn((1, 2048), generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(dev)
    multi = Dn.DenseMulti([qkv, o], after=[False, True], W=W)
    a = torch.empty((1, 5120), dtype=torch.bfloat16, device=dev)
    b = torch.empty((1, 2048), dtype=torch.bfloat16, device=dev)
    multi.forward([x, a[:, :4096]], [a, b])
    torch.cuda.synchronize()
    ea, eb = a.clone(), b.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        multi.forward([x, a[:, :4096]], [a, b])
    for i in range(4):
        a.fill_(float("nan"))
        b.fill_(float("nan"))
        g.replay()
        _clean(ext, multi)
        assert torch.equal(a.view(torch.int16), ea.view(torch.int16)), i
        assert torch.equal(b.view(torch.int16), eb.view(torch.int16)), i
        multi.forward([x, a[:, :4096]], [a, b])         # eager work between replays


def test_multi_rejects_bad_groups(dev, ext):
    qkv, o = _layers(BLOCK[:2], 3, dev)
    with pytest.raises(ValueError):
        Dn.DenseMulti([qkv, o], after=[True, False])
    multi = Dn.DenseMulti([qkv, o], W=W)
    x = torch.zeros((1, 2048), dtype=torch.bfloat16, device=dev)
    xo = torch.zeros((1, 4096), dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="counters"):        # too few counters: refused before any launch
        ext.dense_multi([x, xo], [[m.trellis for m in qkv.mats], [m.trellis for m in o.mats]],
                        [[m.suh for m in qkv.mats], [m.suh for m in o.mats]],
                        [[m.svh for m in qkv.mats], [m.svh for m in o.mats]], [qkv.col0, o.col0],
                        [torch.empty((1, 5120), dtype=torch.bfloat16, device=dev),
                         torch.empty((1, 2048), dtype=torch.bfloat16, device=dev)],
                        [8, 8], [7, 7], [qkv.plans[0][0], o.plans[0][0]], [0, 0], Dn.scratch(dev, 0, 0)[0],
                        multi.counters[:10], W, Dn.ROT_SMEM)
    a = torch.empty((1, 5120), dtype=torch.bfloat16, device=dev)
    b = torch.empty((1, 2048), dtype=torch.bfloat16, device=dev)
    chain = Dn.DenseMulti([qkv, o], after=[False, True], W=W)
    for xo_bad in (xo, a[:, 64:4160]):                         # not the producer's output; not on a block edge
        with pytest.raises(RuntimeError, match="previous group"):
            chain.forward([x, xo_bad], [a, b])
    _clean(ext, chain)


def test_multi_refuses_a_changed_plan(dev, ext):
    """A chain's hand-off maps a consumer's ticket to its launch through the consumer's K splits: a layer whose plan
    changes after the multi launch was built is refused before any launch, and a new DenseMulti over the changed plan
    keeps the bits of the launches apart."""
    qkv, o = _layers(BLOCK[:2], 5, dev)
    x = torch.randn((1, 2048), generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).to(dev)
    chain = Dn.DenseMulti([qkv, o], after=[False, True], W=W)
    a = torch.empty((1, 5120), dtype=torch.bfloat16, device=dev)
    b = torch.empty((1, 2048), dtype=torch.bfloat16, device=dev)
    sk, w, pf = o.plans[0]
    o.plans = [(sk // 2, w, pf)]
    with pytest.raises(ValueError, match="plan changed"):
        chain.forward([x, a[:, :4096]], [a, b])
    fresh = Dn.DenseMulti([qkv, o], after=[False, True], W=W)
    fresh.forward([x, a[:, :4096]], [a, b])
    _clean(ext, fresh)
    y1 = qkv.forward(x)
    assert torch.equal(a.view(torch.int16), y1.view(torch.int16))
    assert torch.equal(b.view(torch.int16), o.forward(y1[:, :4096]).view(torch.int16))

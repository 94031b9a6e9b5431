"""The vLLM methods' apply on the GPU, driven through stand-in layers (vLLM is not importable here): EspLinearMethod
(the reference's linear.py:100-117) against the library calls it stands for, bit for bit, in each prefill mode, and
against the oracle on the per-matrix path; EspMoEMethod.apply / apply_monolithic (moe.py:123-212) against
experts.routed2 / windows / prefill on the same tables, bit for bit, with the shared expert folded into the launch
(its output stored where vLLM's runner reads it) or left to the runner; apply_monolithic's first call (the runner's
gate still in place, real logits) through the router's select_experts, the later ones routed inside.
"""
import types

import numpy as np
import pytest
import torch

import oracle as O
from vllm_espalier import dense as Dn
from vllm_espalier import experts as G
from vllm_espalier import linear as Lin
from vllm_espalier import moe as Moe
from vllm_espalier import ops
from vllm_espalier import workloads as WL

pytestmark = pytest.mark.gpu
D, I = 2048, 512


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _linear_layer(dev, prefix, shards, K, seed):
    layer = torch.nn.Module()
    method = Lin.EspLinearMethod(prefix)
    with torch.device(dev):
        method.create_weights(layer, K, [n for _, n, _ in shards], K, sum(n for _, n, _ in shards), torch.bfloat16)
    gen = torch.Generator().manual_seed(seed)
    for shard, n, grid in shards:
        for suffix, t in WL.matrix_tensors(K, n, 4, grid, gen).items():
            p = getattr(layer, suffix)
            p.weight_loader(p, t, shard)
    method.process_weights_after_loading(layer)
    return method, layer


QKV = [("q", 4096, "int6"), ("k", 512, "int6"), ("v", 512, "int6")]


@pytest.mark.parametrize("mode", ["chunk", "tile"])
@pytest.mark.parametrize("T", [1, 32, 70])
def test_linear_apply_equals_dense(dev, monkeypatch, mode, T):
    print(f"linear apply {mode} T={T}", flush=True)
    monkeypatch.setattr(ops, "PREFILL", mode)
    method, layer = _linear_layer(dev, "model.layers.0.self_attn.qkv_proj", QKV, D, 31)
    d = ops.DENSE_LAYERS[layer.espalier.dense_key]
    x = torch.randn((1, T, D), generator=torch.Generator().manual_seed(T)).to(torch.bfloat16).to(dev)
    bias = torch.randn((5120,), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(dev)
    y = method.apply(layer, x)
    assert y.shape == (1, T, 5120)
    x2 = x.reshape(T, D)
    if T <= 32:
        want = d.forward(x2)
    elif mode == "tile":
        want = d.forward_tile(x2)
    else:
        want = torch.cat([d.forward(x2[r:r + 32]) for r in range(0, T, 32)])
    assert torch.equal(y.reshape(T, -1).view(torch.int16), want.view(torch.int16))
    yb = method.apply(layer, x, bias)
    assert torch.equal(yb.view(torch.int16), (y + bias).view(torch.int16))


def test_linear_apply_per_matrix_path(dev, monkeypatch):
    """ESPALIER_FUSED_DENSE=0: each matrix through espalier::matmul (fp16 rows), outputs in shard order, the padding
    of a head zero; within the parity bar of the oracle."""
    monkeypatch.setattr(Lin, "DENSE", False)
    method, layer = _linear_layer(dev, "lm_head", [(None, 1024, "mcg")], 1024, 32)
    x = torch.randn((3, 1024), generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(dev)
    y = method.apply(layer, x)
    m = layer.espalier.mats[0]
    W = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, G.KERNEL_CB[m.cb])
    ref = O.linear_ref(O.bf16_to_f32(bits(x)), W, bits(m.suh), bits(m.svh))
    assert O.rel_l2(y.float().cpu().numpy(), ref) < 2e-2


# ---- MoE
class _MLP(torch.nn.Module):
    """vLLM's shared-expert MLP as the method reads it: gate_up_proj / down_proj with their trellis matrices and a
    one-output sigmoid gate."""

    def __init__(self, gate, up, down, gate_w):
        super().__init__()
        self.gate_up_proj = torch.nn.Module()
        self.gate_up_proj.espalier = types.SimpleNamespace(mats=[gate, up])
        self.down_proj = torch.nn.Module()
        self.down_proj.espalier = types.SimpleNamespace(mats=[down])
        self.expert_gate = torch.nn.Linear(D, 1, bias=False)
        self.expert_gate.weight.data = gate_w.reshape(1, D)


class _Shared:
    """vLLM's SharedExperts as the method uses it."""

    def __init__(self, mlp, order):
        self._layer, self.order = mlp, order
        self._output, self._output_idx = [None, None], 1
        self.calls = []

    def _determine_shared_experts_order(self, x):
        return self.order

    def forward(self, x, order):
        self.calls.append(order)


class _Router:
    """vLLM's router as the method calls it: softmax top-k with renormalisation, in fp32."""
    top_k, renormalize, scoring_func = 8, True, "softmax"

    def select_experts(self, hidden_states, router_logits, topk_indices_dtype=None, input_ids=None):
        w, ids = torch.topk(torch.softmax(router_logits.float(), -1), self.top_k, dim=-1)
        return w / w.sum(-1, keepdim=True), ids.to(topk_indices_dtype)


class _Runner:
    routed_input_transform = None

    def __init__(self, gate_w, shared):
        self.router = _Router()
        self.gate = torch.nn.Linear(D, gate_w.shape[0], bias=False)
        self.gate.weight.data = gate_w
        self._shared_experts = shared


@pytest.fixture(scope="module")
def moe16(dev):
    gen = torch.Generator().manual_seed(71)
    E = 16
    widths = [(1, "e2m1"), (2, "e2m1"), (3, "int5")]
    named, experts = [], []
    for e in range(E):
        b, grid = widths[e % 3]
        trio = []
        for proj, (k, n) in (("gate_proj", (D, I)), ("up_proj", (D, I)), ("down_proj", (I, D))):
            t = WL.matrix_tensors(k, n, b, grid, gen)
            named += [(f"experts.{e}.{proj}.{s}", v) for s, v in t.items()]
            trio.append(t)
        experts.append(trio)
    shared = [WL.matrix(k, n, 4, "int5", gen, dev) for k, n in ((D, I), (D, I), (I, D))]
    gate_w = (torch.randn((D,), generator=gen) * 0.05).to(torch.bfloat16).to(dev)
    router = (torch.randn((E, D), generator=gen) * 0.02).to(torch.bfloat16).to(dev)
    return named, shared, gate_w, router


def _moe_layer(dev, moe16, order):
    named, shared, gate_w, router = moe16
    method = Moe.EspMoEMethod()
    layer = torch.nn.Module()
    layer.layer_name = "model.layers.0.mlp.experts"
    with torch.device(dev):
        method.create_weights(layer, 16, D, I, torch.bfloat16)
    list(layer.load_weights(iter(named)))
    method.process_weights_after_loading(layer)
    sh = _Shared(_MLP(*shared, gate_w), order)
    layer.espalier_runner = _Runner(router, sh)
    return method, layer, sh


def _direct(layer, x, pick, wts, shared, gate_w, mode, gate=None):
    """The same layer through experts.py directly: its own tables with the shared expert folded in."""
    L = G.prepare(layer.espalier.experts, tuple(shared), gate_w)
    T = x.shape[0]
    if T <= 32:
        s = G.scratch(L, 32, 9, x.device)
        if pick is None:
            G.route(x, gate, 8, L, s)
        return G.routed2(x, pick, wts, L, s, k=8)
    if mode == "tile":
        return G.prefill(x, pick, wts, L, G.prefill_scratch(L, T, 9, x.device), 8, gate=gate)
    return G.windows(x, pick, wts, L, G.scratch(L, 32, 9, x.device), k=8, gate=gate)


@pytest.mark.parametrize("mode", ["chunk", "tile"])
@pytest.mark.parametrize("T", [3, 70])
def test_moe_apply_folds_shared(dev, moe16, monkeypatch, mode, T):
    print(f"moe apply {mode} T={T}", flush=True)
    monkeypatch.setattr(ops, "PREFILL", mode)
    method, layer, sh = _moe_layer(dev, moe16, Moe.SharedExpertsOrder.MK_INTERNAL_OVERLAPPED)
    gen = torch.Generator().manual_seed(T)
    x = torch.randn((T, D), generator=gen).to(torch.bfloat16).to(dev)
    ids = torch.stack([torch.randperm(16, generator=gen)[:8] for _ in range(T)]).to(dev)          # int64, as vLLM
    wts = torch.softmax(torch.randn((T, 8), generator=gen), -1).to(dev)
    out = method.apply(layer, x, wts, ids, shared_experts=sh, shared_experts_input=x).clone()
    folded = sh._output[1].clone()
    assert sh.calls == []                                                # folded: the runner's MLP never ran
    wo, ws = _direct(layer, x, ids.to(torch.int32).contiguous(), wts.float().contiguous(), moe16[1], moe16[2], mode)
    assert torch.equal(out.view(torch.int16), wo.view(torch.int16))
    assert torch.equal(folded.view(torch.int16), ws.view(torch.int16))


def test_moe_apply_external_shared_and_expert_loop(dev, moe16, monkeypatch):
    """The shared expert left to the runner (its order not internal): no fold, the routed sum alone. Then the
    expert-by-expert path (ESPALIER_GROUPED_EXPERTS=0) against the grouped one: within 2e-2."""
    method, layer, sh = _moe_layer(dev, moe16, Moe.SharedExpertsOrder.EXTERNAL)
    gen = torch.Generator().manual_seed(5)
    # small rows: the expert loop hands its SwiGLU outputs to espalier::matmul in fp16, which random weights at unit
    # inputs overflow
    x = (torch.randn((4, D), generator=gen) * 0.02).to(torch.bfloat16).to(dev)
    ids = torch.stack([torch.randperm(16, generator=gen)[:8] for _ in range(4)]).to(dev)
    wts = torch.softmax(torch.randn((4, 8), generator=gen), -1).to(dev)
    out = method.apply(layer, x, wts, ids, shared_experts=sh, shared_experts_input=x).clone()
    assert sh._output == [None, None] and sh.calls == []
    L = G.prepare(layer.espalier.experts)                                # no shared slot
    wo, _ = G.routed2(x, ids.to(torch.int32).contiguous(), wts.float().contiguous(), L, G.scratch(L, 32, 8, dev),
                      k=8)
    assert torch.equal(out.view(torch.int16), wo.view(torch.int16))
    monkeypatch.setattr(Moe, "GROUPED", False)
    loop = method.apply(layer, x, wts, ids)
    assert O.rel_l2(loop.float().cpu().numpy(), out.float().cpu().numpy()) < 2e-2


@pytest.mark.parametrize("mode", ["chunk", "tile"])
@pytest.mark.parametrize("T", [2, 45])
def test_moe_apply_monolithic_routes_inside(dev, moe16, monkeypatch, mode, T):
    print(f"moe apply_monolithic {mode} T={T}", flush=True)
    monkeypatch.setattr(ops, "PREFILL", mode)
    method, layer, sh = _moe_layer(dev, moe16, Moe.SharedExpertsOrder.MK_INTERNAL_OVERLAPPED)
    runner = layer.espalier_runner
    x = torch.randn((T, D), generator=torch.Generator().manual_seed(40 + T)).to(torch.bfloat16).to(dev)
    logits = runner.gate(x)                                              # the first call: the runner's own gate
    first = method.apply_monolithic(layer, x, logits).clone()
    w, ids = runner.router.select_experts(x, logits, torch.int32)
    assert torch.equal(first.view(torch.int16), method.apply(layer, x, w, ids, sh, x).view(torch.int16))
    assert isinstance(runner.gate, Moe.HiddenStatesGate) and runner.gate(x)[0] is x
    out = method.apply_monolithic(layer, x, x).clone()                   # from now on the gate hands x on
    wo, ws = _direct(layer, x, None, None, moe16[1], moe16[2], mode, gate=moe16[3])
    assert torch.equal(out.view(torch.int16), wo.view(torch.int16))
    assert torch.equal(sh._output[1].view(torch.int16), ws.view(torch.int16))

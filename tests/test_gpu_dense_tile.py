"""GPU parity of the prompt launch (esp_dense_tile, Dense.forward_tile: each weight decoded once for every 128 rows)
against the CPU oracle, at BASELINE config 1 / 2 shapes and across codebooks and widths.

Bars: outputs within 2e-2 relative L2 of the dequantise-then-fp64-matmul reference (the parity bar) and within the
reference's max-error gate (< 5e-4 above the output-rounding floor, tests/gpu_dense.py:217-223); the fp32 output
within 1e-4 relative L2 of the same product taken from the fp16 rotated input (which pins the tile GEMM's arithmetic);
a row's bits independent of the prompt (rows alone == rows in a 300-row prompt, bit for bit); graph replay == eager;
counters left zero; every K split within the bar.
"""
import numpy as np
import pytest
import torch

import oracle as O
from vllm_espalier import dense as D
from vllm_espalier import experts, workloads as WL

pytestmark = pytest.mark.gpu

CONFIGS = {
    "cfg1": [(2048, 2048, 4, "int6")],
    "qkv": [(2048, 4096, 4, "int6"), (2048, 512, 4, "int6"), (2048, 512, 4, "int6")],
    "o": [(4096, 2048, 4, "int6")],
    "shared_gate_up": [(2048, 512, 4, "int5"), (2048, 512, 4, "int5")],
    "shared_down": [(512, 2048, 4, "int5")],
    "mcg6": [(1024, 1024, 6, "mcg")],
    "e2m1_2": [(1024, 768, 2, "e2m1")],
    "int5_3": [(1024, 512, 3, "int5")],
    "mcg1": [(512, 256, 1, "mcg")],
    "mcg8": [(512, 384, 8, "mcg")],
}


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _mats(shapes, seed, dev):
    gen = torch.Generator().manual_seed(seed)
    return [WL.matrix(K, N, b, g, gen, dev) for K, N, b, g in shapes]


def _tight_weight(m):
    kcb = experts.KERNEL_CB[m.cb]
    if kcb in (6, 7):
        q = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, kcb + 16).astype(np.float64)
        return q * float(O.GRID_C[kcb])
    return O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, kcb).astype(np.float64)


def _tile(d, x, y, sk=None):
    """forward_tile into y (any dtype), with the layer's prompt plan or K splits sk."""
    d.reserve_prompt(x.shape[0])
    z, xh, cnt = D.prompt_scratch(x.device, 0, 0, 0)
    for (idx, k2, cb), l in zip(d.groups, d.launches):
        experts.ext().dense_tile(x, [d.mats[i].trellis for i in idx], [d.mats[i].suh for i in idx],
                                 [d.mats[i].svh for i in idx], [d.col0[i] for i in idx], y, xh, z, cnt, k2, cb,
                                 D.tile_plan(d.K, l.n) if sk is None else sk)
    return y


def _check(d, mats, x, y, y32):
    xb = bits(x)
    for m, c0 in zip(mats, d.col0):
        W = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, experts.KERNEL_CB[m.cb])
        got = y[:, c0:c0 + m.out_features].float().cpu().numpy()
        ref = O.linear_ref(O.bf16_to_f32(xb), W, bits(m.suh), bits(m.svh))
        e = O.rel_l2(got, ref)
        assert e < 2e-2, f"rel L2 {e:.3e}"
        gate = O.rel_max_above_floor(got, ref, "bf16")
        assert gate < 5e-4, f"max error above the output floor {gate:.3e}"
        tight = O.dense_ref(O.rotate(xb, "bf16", bits(m.suh)), _tight_weight(m), bits(m.svh))
        et = O.rel_l2(y32[:, c0:c0 + m.out_features].cpu().numpy(), tight)
        assert et < 1e-4, f"rel L2 of the fp32 output vs the fp16-input product {et:.3e}"


@pytest.mark.parametrize("T", [1, 129, 300])
@pytest.mark.parametrize("name", list(CONFIGS))
def test_tile_parity(dev, name, T):
    print(f"dense_tile {name} T={T}", flush=True)
    mats = _mats(CONFIGS[name], 21, dev)
    d = D.Dense(mats)
    x = torch.randn((T, d.K), generator=torch.Generator().manual_seed(T)).to(torch.bfloat16).to(dev)
    y = d.forward_tile(x)
    y32 = _tile(d, x, torch.zeros((T, d.n_out), dtype=torch.float32, device=dev))
    torch.cuda.synchronize()
    _check(d, mats, x, y, y32)
    assert int(D.prompt_scratch(dev, 0, 0, 0)[2].abs().sum()) == 0, "counters left non-zero"


@pytest.mark.parametrize("name", ["qkv", "o", "mcg6"])
def test_tile_rows_alone_equal_prompt(dev, name):
    """A row's output alone (T = 1), in a 130-row prompt and in a 300-row prompt, bit for bit, at tile edges."""
    print(f"dense_tile rows alone {name}", flush=True)
    mats = _mats(CONFIGS[name], 22, dev)
    d = D.Dense(mats)
    x = torch.randn((300, d.K), generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(dev)
    y = d.forward_tile(x).clone()
    y130 = d.forward_tile(x[:130]).clone()
    assert torch.equal(y130.view(torch.int16), y[:130].view(torch.int16))
    for r in (0, 1, 15, 16, 127, 128, 255, 256, 299):
        y1 = d.forward_tile(x[r:r + 1])
        assert torch.equal(y1.view(torch.int16), y[r:r + 1].view(torch.int16)), r


@pytest.mark.parametrize("name", ["qkv", "o"])
def test_tile_long_prompt(dev, ext, name):
    """A 2049-row prompt (17 row tiles: a grid past what the device holds at once, so the splits of a tile finish it
    together while later tiles wait to be dispatched): rows alone equal their rows in the prompt, bit for bit, the
    counters are left zero and no wait timed out."""
    print(f"dense_tile long prompt {name}", flush=True)
    assert int(ext.status(True)) == 0
    mats = _mats(CONFIGS[name], 26, dev)
    d = D.Dense(mats)
    T = 2049
    x = torch.randn((T, d.K), generator=torch.Generator().manual_seed(11)).to(torch.bfloat16).to(dev)
    y = d.forward_tile(x).clone()
    torch.cuda.synchronize()
    assert int(ext.status(True)) == 0, "a split's wait timed out"
    assert int(D.prompt_scratch(dev, 0, 0, 0)[2].abs().sum()) == 0, "counters left non-zero"
    assert torch.isfinite(y.float()).all()
    for r in (0, 127, 128, 1024, 2047, 2048):
        y1 = d.forward_tile(x[r:r + 1])
        assert torch.equal(y1.view(torch.int16), y[r:r + 1].view(torch.int16)), r


@pytest.mark.parametrize("sk", [1, 2, 5, 16])
def test_tile_k_splits(dev, ext, sk):
    """Any K split meets the bar (o: K 4096, 128 steps); counters come back zero after each."""
    print(f"dense_tile o SK={sk}", flush=True)
    mats = _mats(CONFIGS["o"], 23, dev)
    d = D.Dense(mats)
    T = 200
    x = torch.randn((T, d.K), generator=torch.Generator().manual_seed(sk)).to(torch.bfloat16).to(dev)
    d.reserve_prompt(T)
    D.prompt_scratch(dev, -(-T // 128) * sk * 128 * d.N, 0, 0)
    y = _tile(d, x, torch.empty((T, d.n_out), dtype=torch.bfloat16, device=dev), sk)
    y32 = _tile(d, x, torch.zeros((T, d.n_out), dtype=torch.float32, device=dev), sk)
    torch.cuda.synchronize()
    _check(d, mats, x, y, y32)
    assert int(D.prompt_scratch(dev, 0, 0, 0)[2].abs().sum()) == 0


def test_tile_close_to_windows(dev):
    """The prompt launch against esp_dense over 32-row windows (another order of the fp32 sums): within 1e-3."""
    mats = _mats(CONFIGS["qkv"], 24, dev)
    d = D.Dense(mats)
    T = 100
    x = torch.randn((T, d.K), generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).to(dev)
    yt = d.forward_tile(x).clone()
    yw = torch.empty_like(yt)
    for r0 in range(0, T, 32):
        d.forward(x[r0:r0 + 32], out=yw[r0:r0 + 32])
    assert O.rel_l2(yt.float().cpu().numpy(), yw.float().cpu().numpy()) < 1e-3


def test_tile_graph_replay(dev):
    mats = _mats(CONFIGS["qkv"], 25, dev)
    d = D.Dense(mats)
    T = 150
    x = torch.randn((T, d.K), generator=torch.Generator().manual_seed(10)).to(torch.bfloat16).to(dev)
    y = torch.empty((T, d.n_out), dtype=torch.bfloat16, device=dev)
    d.forward_tile(x, out=y)
    torch.cuda.synchronize()
    want = y.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        d.forward_tile(x, out=y)
    for i in range(3):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16)), i
        torch.randn((64, 64), device=dev).sum()            # eager work between replays
    assert int(D.prompt_scratch(dev, 0, 0, 0)[2].abs().sum()) == 0


def test_tile_rejects_small_scratch(dev, ext):
    mats = _mats(CONFIGS["o"], 26, dev)
    d = D.Dense(mats)
    m = mats[0]
    x = torch.zeros((130, d.K), dtype=torch.bfloat16, device=dev)
    y = torch.empty((130, d.N), dtype=torch.bfloat16, device=dev)
    z = torch.zeros(2 * 2 * 128 * d.N, dtype=torch.float32, device=dev)
    cnt = torch.zeros(2 * (d.N // 128) * 32, dtype=torch.int32, device=dev)
    xh_small = torch.empty(130 * d.K, dtype=torch.float16, device=dev)           # 144 rows are needed
    with pytest.raises(RuntimeError, match="xh"):
        ext.dense_tile(x, [m.trellis], [m.suh], [m.svh], [0], y, xh_small, z, cnt, 2 * m.K, experts.KERNEL_CB[m.cb], 2)
    xh = torch.empty(144 * d.K, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="Z needs"):
        ext.dense_tile(x, [m.trellis], [m.suh], [m.svh], [0], y, xh, z, cnt, 2 * m.K, experts.KERNEL_CB[m.cb], 3)
    with pytest.raises(RuntimeError, match="SK at most"):
        ext.dense_tile(x, [m.trellis], [m.suh], [m.svh], [0], y, xh, z, cnt, 2 * m.K, experts.KERNEL_CB[m.cb], 129)

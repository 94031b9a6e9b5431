"""GPU parity of the dense path (csrc/dense.hip) against the CPU oracle.

Bars: dequant and had bit-exact; dense GEMM outputs within 2e-2 relative L2 of the dequantise-then-fp64-matmul
reference (the parity bar), within the reference's own gate (max error over max |ref| minus the output-rounding
floor < 5e-4, tests/gpu_dense.py:217-223) and within 1e-4 relative L2 of the same product taken from the kernel's
own fp16 rotated input (which pins the GEMM arithmetic). Self-consistency gates of tests/gpu_dense.py: merged launch ==
each matrix alone, rows alone == rows in the window, graph replay == eager, all bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle as O
from vllm_espalier import dense as D
from vllm_espalier import experts, ops, workloads as WL

pytestmark = pytest.mark.gpu


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("cb,k2", sorted(experts.COMPILED))
@pytest.mark.parametrize("K,N", [(256, 256), (48, 64), (1024, 1024)])
def test_dequant_bit_exact(dev, ext, cb, k2, K, N):
    print(f"dequant cb={cb} k2={k2} K={K} N={N}", flush=True)
    gen = torch.Generator().manual_seed(1000 + cb * 32 + k2)
    t = torch.randint(-32768, 32768, (K // 16, N // 16, 8 * k2), dtype=torch.int32, generator=gen).to(torch.int16)
    want = O.dequant(t.numpy(), k2, cb)
    out = torch.full((K, N), float("nan"), dtype=torch.float16, device=dev)
    ext.dequant(t.to(dev), out, k2, cb)
    got = bits(out)
    assert np.array_equal(got, want), f"{int((got != want).sum())} of {got.size} values differ"


@pytest.mark.parametrize("cb,k2", [(19, 2), (19, 4), (19, 6), (22, 4), (22, 6), (22, 8), (23, 6), (23, 8), (23, 10)])
def test_dequant_grid_index_bit_exact(dev, ext, cb, k2):
    """The GEMMs' decode forms (E2M1 / 0.75, the int5 / int6 grid index q; the sums are scaled after) against the
    oracle's, over a million random states (all 65536 but about 0.01 expected missing), the sign of a zero q aside."""
    print(f"dequant grid index cb={cb} k2={k2}", flush=True)
    gen = torch.Generator().manual_seed(2000 + cb * 32 + k2)
    t = torch.randint(-32768, 32768, (64, 64, 8 * k2), dtype=torch.int32, generator=gen).to(torch.int16)
    want = O.dequant(t.numpy(), k2, cb)
    out = torch.full((1024, 1024), float("nan"), dtype=torch.float16, device=dev)
    ext.dequant(t.to(dev), out, k2, cb)
    got = bits(out)
    if cb != 19:
        got[got == 0x8000] = 0               # q = -0 (rintf of a small negative product) only ever enters sums
    assert np.array_equal(got, want), f"{int((got != want).sum())} of {got.size} values differ"


def test_dequant_unsupported_raises(dev, ext):
    t = torch.zeros((2, 2, 8 * 3), dtype=torch.int16, device=dev)
    out = torch.empty((32, 32), dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="no instance"):
        ext.dequant(t, out, 3, 1)


@pytest.mark.parametrize("pre,post", [(True, False), (False, True), (True, True), (False, False)])
def test_had_bit_exact(dev, ext, pre, post):
    gen = torch.Generator().manual_seed(7)
    M, K = 5, 512
    x = torch.randn((M, K), generator=gen).to(torch.float16)
    p = torch.randn((K,), generator=gen).to(torch.float16) if pre else None
    q = torch.randn((K,), generator=gen).to(torch.float16) if post else None
    y = torch.empty_like(x, device=dev)
    ext.had(x.to(dev), None if p is None else p.to(dev), None if q is None else q.to(dev), y)
    want = O.had(bits(x), None if p is None else bits(p), None if q is None else bits(q))
    assert np.array_equal(bits(y), want)


def _mats(shapes, seed, dev):
    gen = torch.Generator().manual_seed(seed)
    return [WL.matrix(K, N, b, g, gen, dev) for K, N, b, g in shapes]


def _dense_call(d, x, y, rot_smem=None):
    """One Dense launch set into y (any dtype) through the extension, with the layer's plans."""
    z, xh = D.scratch(x.device, 0, 0)
    for (idx, k2, cb), (sk, w, pf) in zip(d.groups, d.plans):
        experts.ext().dense(x, [d.mats[i].trellis for i in idx], [d.mats[i].suh for i in idx],
                            [d.mats[i].svh for i in idx], [d.col0[i] for i in idx], y, xh, z, d.counters, k2, cb,
                            sk, w, pf, D.ROT_SMEM if rot_smem is None else rot_smem)
    return y


def _tight_weight(m):
    """The weight the GEMM multiplies: the decoded value, or for the int5 / int6 grids q * c without the fp16
    rounding of the reference's grouped decode (the dense reference path, dense.cu:123,292,312)."""
    kcb = experts.KERNEL_CB[m.cb]
    if kcb in (6, 7):
        q = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, kcb + 16).astype(np.float64)
        return q * float(O.GRID_C[kcb])
    return O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, kcb).astype(np.float64)


def _check_dense(d, mats, x, y):
    xb = bits(x)
    y32 = _dense_call(d, x, torch.zeros((x.shape[0], d.n_out), dtype=torch.float32, device=x.device))
    for m, c0 in zip(mats, d.col0):
        kcb = experts.KERNEL_CB[m.cb]
        W = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, kcb)
        got = y[:, c0:c0 + m.out_features].float().cpu().numpy()
        # 1. the parity bar: the dequantise-then-fp64-matmul reference from the bf16 input
        ref = O.linear_ref(O.bf16_to_f32(xb), W, bits(m.suh), bits(m.svh))
        e = O.rel_l2(got, ref)
        assert e < 2e-2, f"rel L2 {e:.3e}"
        gate = O.rel_max_above_floor(got, ref, "bf16" if y.dtype == torch.bfloat16 else np.float16)
        assert gate < 5e-4, f"max error above the output floor {gate:.3e}"
        # 2. the GEMM arithmetic, fp32 out: the same product from the kernel's fp16 rotated input
        xh = O.rotate(xb, "bf16", bits(m.suh))
        tight = O.dense_ref(xh, _tight_weight(m), bits(m.svh))
        et = O.rel_l2(y32[:, c0:c0 + m.out_features].cpu().numpy(), tight)
        assert et < 1e-4, f"rel L2 of the fp32 output vs the fp16-input product {et:.3e}"


CONFIGS = {
    # one 2048x2048 4-bit int6 matrix
    "cfg1": [(2048, 2048, 4, "int6")],
    # config 2's launches: qkv (q 4096, k 512, v 512), o, shared gate/up, shared down
    "qkv": [(2048, 4096, 4, "int6"), (2048, 512, 4, "int6"), (2048, 512, 4, "int6")],
    "o": [(4096, 2048, 4, "int6")],
    "shared_gate_up": [(2048, 512, 4, "int5"), (2048, 512, 4, "int5")],
    "shared_down": [(512, 2048, 4, "int5")],
    # other codebooks / widths
    "mcg6": [(1024, 1024, 6, "mcg")],
    "e2m1_2": [(1024, 768, 2, "e2m1")],
    "int5_3": [(1024, 512, 3, "int5")],
    "mcg1": [(512, 256, 1, "mcg")],
    "mcg8": [(512, 384, 8, "mcg")],
}


@pytest.mark.parametrize("name", list(CONFIGS))
@pytest.mark.parametrize("M", [1, 8, 32])
def test_dense_parity(dev, name, M):
    print(f"dense {name} M={M}", flush=True)
    mats = _mats(CONFIGS[name], 11, dev)
    d = D.Dense(mats)
    gen = torch.Generator().manual_seed(100 + M)
    x = torch.randn((M, d.K), generator=gen).to(torch.bfloat16).to(dev)
    y = d.forward(x)
    torch.cuda.synchronize()
    _check_dense(d, mats, x, y)


@pytest.mark.parametrize("name", ["qkv", "shared_gate_up"])
def test_dense_merged_equals_alone(dev, name):
    mats = _mats(CONFIGS[name], 12, dev)
    d = D.Dense(mats)
    x = torch.randn((8, d.K), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(dev)
    y = d.forward(x).clone()
    for m, c in zip(mats, d.col0):
        di = D.Dense([m])
        di.plans = [d.plans[0]]                 # the same K split as in the merged launch
        assert torch.equal(di.forward(x), y[:, c:c + m.out_features])


@pytest.mark.parametrize("name", ["qkv", "o", "mcg6"])
@pytest.mark.parametrize("M", [2, 8, 17, 32])
def test_dense_row_invariance(dev, name, M):
    mats = _mats(CONFIGS[name], 13, dev)
    d = D.Dense(mats)
    x = torch.randn((M, d.K), generator=torch.Generator().manual_seed(M)).to(torch.bfloat16).to(dev)
    y = d.forward(x).clone()
    ya = torch.cat([d.forward(x[r:r + 1]).clone() for r in range(M)])
    assert torch.equal(y, ya)


@pytest.mark.parametrize("name", ["qkv", "o", "shared_gate_up", "shared_down"])
@pytest.mark.parametrize("M", [4, 9, 32])
def test_dense_split_finish_rows(dev, ext, name, M):
    """config 2's four launches over 4-32 rows, all with K splits: each row equals its bits alone, every arrival
    counter is left zero and the status word stays 0. o and gate/up take 16 splits (two rounds of partial loads in
    the finisher)."""
    assert int(ext.status(True)) == 0
    mats = _mats(CONFIGS[name], 17, dev)
    d = D.Dense(mats)
    assert all(sk > 1 for sk, _, _ in d.plans)
    x = torch.randn((M, d.K), generator=torch.Generator().manual_seed(40 + M)).to(torch.bfloat16).to(dev)
    y = d.forward(x).clone()
    torch.cuda.synchronize()
    assert int(d.counters.abs().sum()) == 0
    assert int(ext.status(True)) == 0
    for r in (0, M // 2, M - 1):
        assert torch.equal(d.forward(x[r:r + 1]).view(torch.int16), y[r:r + 1].view(torch.int16)), r


@pytest.mark.parametrize("name", ["qkv", "o", "shared_gate_up", "shared_down"])
@pytest.mark.parametrize("M", [1, 2, 5, 8, 32])
def test_dense_own_equals_dense(dev, ext, name, M):
    """esp_dense_own (Z an all-ones buffer of the caller's: the last split polls the others' partials where it can
    hold one a 32-lane half, else arrivals are counted and the finisher restores the all-ones) against esp_dense:
    y bit for bit over launches in a row and graph replays; Z left all-ones, counters zero, no wait timed out."""
    print(f"dense_own {name} M={M}", flush=True)
    mats = _mats(CONFIGS[name], 31, dev)
    d = D.Dense(mats)
    x = torch.randn((M, d.K), generator=torch.Generator().manual_seed(40 + M)).to(torch.bfloat16).to(dev)
    want = _dense_call(d, x, torch.empty((M, d.n_out), dtype=torch.bfloat16, device=dev)).clone()
    _, xh = D.scratch(dev, 0, 0)
    zo = torch.full((max(sk * M * l.n for l, (sk, _, _) in zip(d.launches, d.plans)),), -1, dtype=torch.int32,
                    device=dev).view(torch.float32)
    y = torch.empty((M, d.n_out), dtype=torch.bfloat16, device=dev)

    def launch():
        for (idx, k2, cb), (sk, w, pf) in zip(d.groups, d.plans):
            ext.dense_own(x, [d.mats[i].trellis for i in idx], [d.mats[i].suh for i in idx],
                          [d.mats[i].svh for i in idx], [d.col0[i] for i in idx], y, xh, zo, d.counters, k2, cb, sk,
                          w, pf, D.ROT_SMEM)

    def check(tag):
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16)), tag
        assert bool((zo.view(torch.int32) == -1).all()), f"{tag}: Z must be left all-ones"
        assert int(d.counters.abs().sum()) == 0, f"{tag}: counters must be left zero"

    ext.status(True)
    assert D.polls(M, d.plans[0][0], d.plans[0][1]) == (M * (d.plans[0][0] - 1) <= 2 * d.plans[0][1])
    for i in range(2):
        y.zero_()
        launch()
        check(f"launch {i}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    for i in range(3):
        y.zero_()
        g.replay()
        check(f"replay {i}")
        torch.randn((64, 64), device=dev).sum()           # eager work between replays
    assert int(ext.status(True)) == 0, "a wait timed out"


@pytest.mark.parametrize("M", [1, 8, 32])
def test_dense_graph_replay_equals_eager(dev, M):
    mats = _mats(CONFIGS["qkv"], 14, dev)
    d = D.Dense(mats)
    x = torch.randn((M, d.K), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(dev)
    out = torch.empty((M, d.n_out), dtype=x.dtype, device=dev)
    eager = d.forward(x).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        d.forward(x, out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        d.forward(x, out=out)
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        d.forward(x)                             # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("name", ["cfg1", "qkv", "mcg1"])
@pytest.mark.parametrize("M", [1, 16, 32])
def test_dense_unfused_rotation_same_bits(dev, name, M):
    mats = _mats(CONFIGS[name], 17, dev)
    d = D.Dense(mats)
    x = torch.randn((M, d.K), generator=torch.Generator().manual_seed(M)).to(torch.bfloat16).to(dev)
    fused = _dense_call(d, x, torch.zeros((M, d.n_out), dtype=x.dtype, device=dev), rot_smem=1 << 30)
    unfused = _dense_call(d, x, torch.zeros((M, d.n_out), dtype=x.dtype, device=dev), rot_smem=0)
    assert torch.equal(fused, unfused)


def test_dense_fp32_and_fp16_io(dev):
    mats = _mats(CONFIGS["shared_down"], 15, dev)
    d = D.Dense(mats)
    x32 = torch.randn((4, d.K), generator=torch.Generator().manual_seed(9)).to(dev)
    y32 = d.forward(x32)
    xb = x32.to(torch.bfloat16)
    m = mats[0]
    W = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, experts.KERNEL_CB[m.cb])
    ref = O.linear_ref(x32.cpu().numpy(), W, bits(m.suh), bits(m.svh))
    assert y32.dtype == torch.float32 and O.rel_l2(y32.cpu().numpy(), ref) < 2e-3
    y16 = d.forward(x32.half())
    assert y16.dtype == torch.float16 and O.rel_l2(y16.float().cpu().numpy(), ref) < 2e-3
    del xb


@pytest.mark.parametrize("T", [1, 33, 70])
def test_matmul_op_windows(dev, T):
    m = _mats([(512, 256, 4, "int6")], 16, dev)[0]
    x = torch.randn((T, 512), generator=torch.Generator().manual_seed(T)).half().to(dev)
    y = torch.ops.espalier.matmul(x, m.trellis, m.suh, m.svh, m.K, m.cb)
    y1 = torch.cat([torch.ops.espalier.matmul(x[i:i + 1], m.trellis, m.suh, m.svh, m.K, m.cb) for i in range(T)])
    assert y.dtype == torch.float16 and torch.equal(y, y1)
    W = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, experts.KERNEL_CB[m.cb])
    ref = O.linear_ref(x.float().cpu().numpy(), W, bits(m.suh), bits(m.svh))
    assert O.rel_l2(y.float().cpu().numpy(), ref) < 2e-3


@pytest.mark.parametrize("T", [33, 70])
def test_prefill_gemm_mode(dev, monkeypatch, T):
    """ESPALIER_PREFILL_MODE=gemm (ops.py): above 32 rows every matrix is decoded by the dequant kernel, rotated by the
    had kernel on both sides and multiplied by torch's fp16 matmul. Within the 2e-2 bar of the dequantise-then-fp64
    reference, per matrix (espalier::matmul) and for a layer of three matrices with padded output (espalier::dense);
    not bit-identical to the windowed kernels (another summation order), so compared with the reference only."""
    monkeypatch.setattr(ops, "PREFILL", "gemm")
    mats = _mats([(512, 384, 4, "int6"), (512, 256, 3, "int5"), (512, 128, 2, "e2m1")], 18 + T, dev)
    x = torch.randn((T, 512), generator=torch.Generator().manual_seed(T)).to(torch.bfloat16).to(dev)
    refs = []
    for m in mats:
        W = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, experts.KERNEL_CB[m.cb])
        refs.append(O.linear_ref(x.float().cpu().numpy(), W, bits(m.suh), bits(m.svh)))
        y = torch.ops.espalier.matmul(x.half(), m.trellis, m.suh, m.svh, m.K, m.cb)
        assert y.dtype == torch.float16 and y.shape == (T, m.out_features)
        assert O.rel_l2(y.float().cpu().numpy(), refs[-1]) < 2e-2
    d = D.Dense(mats, n_out=896)
    key = next(ops.DENSE_KEYS)
    ops.DENSE_LAYERS[key] = d
    try:
        y = torch.ops.espalier.dense(x, [m.trellis for m in mats], [m.suh for m in mats], [m.svh for m in mats], key)
    finally:
        ops.DENSE_LAYERS.pop(key)
    assert y.dtype == x.dtype and y.shape == (T, 896)
    assert O.rel_l2(y[:, :768].float().cpu().numpy(), np.concatenate(refs, axis=1)) < 2e-2
    assert not y[:, 768:].any()

"""GPU checks of the decode-step glue (csrc/step.hip) and of the synthetic decoder built on the trellis layers
(vllm_espalier/step.py).

Bars: embed and argmax bit-exact against torch; add_rmsnorm's residual bit-exact and its output within one bf16 /
fp16 ulp of a CPU fp32 restatement (the only freedom is the order of the sum of squares); the decoder: rows alone ==
the same rows in one window, graph replay == eager, all bit for bit.
"""
import numpy as np
import pytest
import torch

from vllm_espalier import step as S

pytestmark = pytest.mark.gpu


def test_embed_rows_and_invalid_ids(dev, ext):
    gen = torch.Generator().manual_seed(7)
    table = torch.randn((1000, 2048), generator=gen).to(torch.bfloat16)
    ids = torch.tensor([3, 999, 0, -1, 1000, 512], dtype=torch.int32)
    h = torch.full((6, 2048), float("nan"), dtype=torch.bfloat16, device=dev)
    ext.embed(ids.to(dev), table.to(dev), h)
    want = torch.zeros((6, 2048), dtype=torch.bfloat16)
    for i, t in enumerate(ids.tolist()):
        if 0 <= t < 1000:
            want[i] = table[t]
    assert torch.equal(h.cpu().view(torch.int16), want.view(torch.int16))


def _ulps(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    x = a.view(torch.int16).numpy().astype(np.int32)
    y = b.view(torch.int16).numpy().astype(np.int32)
    # sign-magnitude bits to a monotone integer line
    x = np.where(x < 0, -(x & 0x7FFF), x)
    y = np.where(y < 0, -(y & 0x7FFF), y)
    return np.abs(x - y)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("deltas", [0, 1, 2])
def test_add_rmsnorm(dev, ext, dtype, deltas):
    print(f"add_rmsnorm {dtype} deltas={deltas}", flush=True)
    gen = torch.Generator().manual_seed(11 + deltas)
    T, D, eps = 5, 2048, 1e-6
    h = (torch.randn((T, D), generator=gen) * 3).to(dtype)
    d = [torch.randn((T, D), generator=gen).to(dtype) for _ in range(deltas)]
    w = (1 + 0.1 * torch.randn((D,), generator=gen)).to(dtype)
    hg = h.to(dev)
    out = torch.empty((T, D), dtype=dtype, device=dev)
    ext.add_rmsnorm(hg, d[0].to(dev) if deltas > 0 else None, d[1].to(dev) if deltas > 1 else None, w.to(dev), out,
                    eps)
    z = h.float()
    for t in d:
        z = z + t.float()
    hr = z.to(dtype)
    inv = 1.0 / torch.sqrt((hr.float() ** 2).sum(dim=1, keepdim=True) / D + eps)
    ref = ((hr.float() * inv) * w.float()).to(dtype)
    assert torch.equal(hg.cpu().view(torch.int16), hr.view(torch.int16))
    u = _ulps(out.cpu(), ref)
    assert u.max() <= 1 and (u == 0).mean() > 0.99, (u.max(), (u == 0).mean())


def _argmax_scratch(dev, T, N):
    """esp_argmax's split scratch: ceil(N / 4096) keys and one 32-int counter line a row."""
    return (torch.zeros((T * -(-N // 4096),), dtype=torch.int64, device=dev),
            torch.zeros((T * 32,), dtype=torch.int32, device=dev))


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_argmax_ties_nan_and_tail(dev, ext, dtype, split):
    gen = torch.Generator().manual_seed(3)
    N = 151936
    x = torch.randn((4, N), generator=gen).to(dtype)
    x[1, 70000] = 40.0
    x[1, 9] = 40.0                                   # a tie across slices: the lower index wins
    x[2, 123456] = float("nan")                       # NaN counts as the largest
    x[3, N - 1] = 50.0                                 # the last element
    ids = torch.empty((4,), dtype=torch.int32, device=dev)
    scratch = _argmax_scratch(dev, 4, N) if split else (None, None)
    for _ in range(2):                                # twice: the counters are left zero for the next call
        ids.fill_(-1)
        ext.argmax(x.to(dev), ids, *scratch)
        got = ids.cpu().tolist()
        assert got[0] == int(torch.argmax(x[0].float()))
        assert got[1:] == [9, 123456, N - 1]
    if split:
        assert int(scratch[1].abs().sum()) == 0
    # an odd width and a strided view (rows of a wider buffer)
    y = torch.randn((3, 1000), generator=gen).to(dtype)
    yg = torch.zeros((3, 1008), dtype=dtype, device=dev)
    yg[:, :1000] = y.to(dev)
    yg[:, 1000:] = 100.0                              # outside N: never read
    ids3 = torch.empty((3,), dtype=torch.int32, device=dev)
    ext.argmax(yg[:, :999], ids3, *(_argmax_scratch(dev, 3, 999) if split else (None, None)))
    assert ids3.cpu().tolist() == torch.argmax(y[:, :999].float(), dim=1).tolist()


@pytest.mark.parametrize("N", [4097, 8195, 12288, 40003])
def test_argmax_split_slices(dev, ext, N):
    """Slice edges: the maximum in the first, the last, a partial last group, and equal maxima in two slices."""
    gen = torch.Generator().manual_seed(N)
    W = (N + 7) // 8 * 8
    x = torch.randn((5, W), generator=gen).to(torch.bfloat16)
    x[0, 0] = 30.0
    x[1, N - 1] = 30.0
    x[2, 4096] = 30.0
    x[3, 4095] = 30.0
    x[3, N - 2] = 30.0
    x[4, :] = -1.0                                    # all equal: index 0
    xd = x.to(dev)
    ids = torch.empty((5,), dtype=torch.int32, device=dev)
    part, cnt = _argmax_scratch(dev, 5, N)
    ext.argmax(xd[:, :N], ids, part, cnt)
    want = torch.argmax(x[:, :N].float(), dim=1).to(torch.int32)
    assert torch.equal(ids.cpu(), want)
    assert ids.cpu().tolist()[:5] == [0, N - 1, 4096, 4095, 0]
    assert int(cnt.abs().sum()) == 0


@pytest.fixture(scope="module")
def small_decoder(dev):
    return S.SyntheticDecoder(n_layers=2, seed=9, device=dev, E=16, vocab=5120)   # two argmax slices


def _run(dec, ids):
    b = dec.buffers(len(ids))
    b.ids_in.copy_(torch.tensor(ids, dtype=torch.int32))
    dec.forward(len(ids))
    torch.cuda.synchronize()
    return b.a.cpu().clone(), b.logits.cpu().clone(), b.ids_out.cpu().clone()


def test_decoder_rows_alone_equal_window(small_decoder):
    ids = [5, 4095, 17, 300]
    a4, l4, o4 = _run(small_decoder, ids)
    assert torch.isfinite(l4.float()).all()
    assert torch.equal(o4, torch.argmax(l4.float(), dim=1).to(torch.int32))
    for r, t in enumerate(ids):
        a1, l1, o1 = _run(small_decoder, [t])
        assert torch.equal(a1.view(torch.int16), a4[r:r + 1].view(torch.int16)), r
        assert torch.equal(l1.view(torch.int16), l4[r:r + 1].view(torch.int16)), r
        assert int(o1[0]) == int(o4[r])


def test_decoder_graph_replay_equals_eager(small_decoder):
    """Three greedy steps: eager (ids fed back on the host) against a graph whose step ends by copying its argmax
    into its own input, replayed three times with eager work between the replays."""
    dec = small_decoder
    b = dec.buffers(1)
    eager = []
    b.ids_in.fill_(42)
    for _ in range(3):
        dec.forward(1)
        eager.append((b.logits.cpu().clone(), int(b.ids_out.item())))
        b.ids_in.copy_(b.ids_out)

    def step():
        dec.forward(1)
        b.ids_in.copy_(b.ids_out)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        b.ids_in.fill_(42)
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    b.ids_in.fill_(42)
    torch.cuda.synchronize()
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(b.logits.cpu().view(torch.int16), eager[i][0].view(torch.int16)), i
        assert int(b.ids_out.item()) == eager[i][1], i
        torch.randn((64, 64), device=b.h.device).sum()        # eager work between replays


@pytest.mark.parametrize("T", [1, 2])
def test_decoder_fused_norms_equal_separate(small_decoder, T, monkeypatch):
    """The norms inside the qkv, routing and head launches (dense_rmsnorm, route_group_rmsnorm) against add_rmsnorm
    launches of their own: logits and the residual stream bit for bit. The qkv launch normalises four waves a row, so
    at ATTN_W = 8 waves a workgroup the norms run inside the launches for up to 2 rows (beyond, apart)."""
    dec = small_decoder
    ids = [7, 1234, 4000][:T]
    assert not dec.fused_norms(S.ATTN_W // 4 + 1)
    res = {}
    for fused in (False, True):
        monkeypatch.setattr(S, "FUSE_NORMS", fused)
        assert dec.fused_norms(T) == fused and dec.fused_head_norm(T) == fused
        b = dec.buffers(T)
        b.ids_in.copy_(torch.tensor(ids, dtype=torch.int32))
        dec.forward(T)
        torch.cuda.synchronize()
        final_residual = b.h2 if fused else b.h               # the fused head stores it to the second buffer
        res[fused] = (b.logits.cpu().clone(), final_residual.cpu().clone(), b.ids_out.cpu().clone())
    for x, y in zip(res[False], res[True]):
        assert torch.equal(x.view(torch.int16) if x.dtype == torch.bfloat16 else x,
                           y.view(torch.int16) if y.dtype == torch.bfloat16 else y)


@pytest.mark.parametrize("T", [1, 3, 8])
def test_decoder_multi_attention_equals_apart(small_decoder, T, monkeypatch):
    """qkv and o as one chained launch (DenseMulti) against the two launches apart: logits and residuals bit for bit."""
    dec = small_decoder
    ids = [(7 + 613 * i) % 5120 for i in range(T)]
    res = {}
    for multi in (False, True):
        monkeypatch.setattr(S, "MULTI_ATTN", multi)
        b = dec.buffers(T)
        b.ids_in.copy_(torch.tensor(ids, dtype=torch.int32))
        dec.forward(T)
        torch.cuda.synchronize()
        res[multi] = (b.logits.cpu().clone(), b.h.cpu().clone(), b.h2.cpu().clone(), b.ids_out.cpu().clone())
    for x, y in zip(res[False], res[True]):
        assert torch.equal(x.view(torch.int16) if x.dtype == torch.bfloat16 else x,
                           y.view(torch.int16) if y.dtype == torch.bfloat16 else y)


def test_decoder_prefill_rows_alone_equal_prompt(small_decoder):
    """The tile prefill (prompt launches for the dense layers, routing and grouping over the whole prompt): every
    row's logits alone (a 1-token prompt) equal that row's logits in a 70-token prompt, bit for bit, and they stay
    close to decode's windows (another order of the sums)."""
    dec = small_decoder
    T = 70
    ids = [(11 + 977 * i) % 5120 for i in range(T)]
    b = dec.prefill_buffers(T)
    b.ids_in.copy_(torch.tensor(ids, dtype=torch.int32))
    dec.prefill(T, head_rows=T)
    torch.cuda.synchronize()
    logits, out = b.logits.cpu().clone(), b.ids_out.cpu().clone()
    assert torch.isfinite(logits.float()).all()
    assert torch.equal(out, torch.argmax(logits.float(), dim=1).to(torch.int32))
    for r in (0, 31, 32, 69):
        b1 = dec.prefill_buffers(1)
        b1.ids_in.fill_(ids[r])
        dec.prefill(1)
        torch.cuda.synchronize()
        assert torch.equal(b1.logits.cpu().view(torch.int16), logits[r:r + 1].view(torch.int16)), r
    _, lw, _ = _run(dec, ids[:32])
    err = (lw.float() - logits[:32].float()).norm() / lw.float().norm()
    assert err < 2e-2, float(err)

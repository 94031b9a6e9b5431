"""The BASELINE config-5 decoder itself (40 layers, 256 routed experts + the shared expert a layer, the 2048 x 151936
6-bit mcg head) under the property checks, all bit for bit: rows alone == the same rows in one window, graph replay ==
eager greedy steps, norms inside their consumers' launches == separate norm launches. (The oracle comparison at full
width, stage by stage, is test_gpu_fullsize.py's one-layer decoder.)
"""
import pytest
import torch

from vllm_espalier import step as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def decoder40(dev):
    print("building the 40-layer decoder", flush=True)
    dec = S.SyntheticDecoder(n_layers=40, seed=5, device=dev)
    assert dec.E == 256 and dec.vocab == 151936 and len(dec.layers) == 40
    return dec


def _run(dec, ids):
    b = dec.buffers(len(ids))
    b.ids_in.copy_(torch.tensor(ids, dtype=torch.int32))
    dec.forward(len(ids))
    torch.cuda.synchronize()
    return b.logits.cpu().clone(), b.ids_out.cpu().clone()


def test_decoder40_rows_alone_equal_window(decoder40):
    ids = [5, 151935, 17, 70000]
    l4, o4 = _run(decoder40, ids)
    assert torch.isfinite(l4.float()).all()
    assert torch.equal(o4, torch.argmax(l4.float(), dim=1).to(torch.int32))
    for r, t in enumerate(ids):
        l1, o1 = _run(decoder40, [t])
        assert torch.equal(l1.view(torch.int16), l4[r:r + 1].view(torch.int16)), r
        assert int(o1[0]) == int(o4[r])


def test_decoder40_window_of_32(decoder40):
    """A full 32-row window (the prefill width, separate norm launches) gives each row its single-row bits."""
    ids = [(i * 4751 + 3) % 151936 for i in range(32)]
    l32, o32 = _run(decoder40, ids)
    for r in (0, 13, 31):
        l1, o1 = _run(decoder40, [ids[r]])
        assert torch.equal(l1.view(torch.int16), l32[r:r + 1].view(torch.int16)), r
        assert int(o1[0]) == int(o32[r])


def test_decoder40_graph_replay_equals_eager(decoder40):
    dec = decoder40
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


@pytest.mark.parametrize("T", [1, 2, 3])
def test_decoder40_fused_norms_equal_separate(decoder40, T, monkeypatch):
    dec = decoder40
    ids = [7, 1234, 150000][:T]
    res = {}
    for fused in (False, True):
        monkeypatch.setattr(S, "FUSE_NORMS", fused)
        # qkv at ATTN_W = 8 waves a workgroup normalises four waves a row: inside the launch up to 2 rows
        assert dec.fused_norms(T) == (fused and T <= S.ATTN_W // 4)
        # the full-width head (8 waves a workgroup) fuses its norm up to 2 rows; the residual it keeps in h2
        assert dec.fused_head_norm(T) == (fused and T <= 2)
        b = dec.buffers(T)
        b.ids_in.copy_(torch.tensor(ids, dtype=torch.int32))
        dec.forward(T)
        torch.cuda.synchronize()
        final_residual = b.h2 if dec.fused_head_norm(T) else b.h
        res[fused] = (b.logits.cpu().clone(), final_residual.cpu().clone(), b.ids_out.cpu().clone())
    for x, y in zip(res[False], res[True]):
        assert torch.equal(x.view(torch.int16) if x.dtype == torch.bfloat16 else x,
                           y.view(torch.int16) if y.dtype == torch.bfloat16 else y)

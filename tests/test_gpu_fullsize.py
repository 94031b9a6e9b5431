"""GPU parity at BASELINE's full sizes (configs 4 and 5) against the CPU oracle.

- The 2048 x 151936 6-bit mcg LM head through Dense at 1 and 4 rows: within 2e-2 relative L2 of the dequantise-then-
  fp64-matmul reference (oracle dequantisation, fp64 Hadamards), and within the reference's own gate (5e-4 above the
  bf16 output floor, tests/gpu_dense.py:217-223).
- A 256-expert MoE layer with BASELINE's per-expert widths ({1, 2, 3} bits: E2M1 at 1-2, int5 at 3) plus the 4-bit
  shared expert, at 1, 4 and 32 tokens (at 32 the grouped grid is 257 experts wide), with given picks and with fused
  routing: routing ids bit-exact against exact routing; outputs within 2e-2 relative L2 of the plain fp64 reference,
  and within the 5e-4 max-error gate of a rounding-faithful one (the kernels' exact-grid int5 weights, fp16 rotated
  inputs and fp16 down input, the roundings the reference pipeline makes too).
- A one-layer decoder at full width (E = 256, vocab 151936), stage by stage against an fp64 composition of oracle
  pieces, each stage fed the GPU's own observed input: residual adds bit-exact, norms within one bf16 ulp, routing
  ids exact, GEMMs within the bars above, the next ids the argmax of the logits.
- Prefill windows (ESPALIER_PREFILL_MODE=chunk): at 33, 100 and 517 rows the espalier::dense op (every dense kind of
  config 2 and the head) and experts.windows (given picks and fused routing) equal the same rows run one at a time,
  bit for bit (the reference's gate P1, tests/gpu_prefill.py:3-5).
- The prompt paths (ESPALIER_PREFILL_MODE=tile) at full size: every dense kind of config 2 as prompt launches over
  517 rows within the GEMM bars against the oracle (the head on a sample of its rows), and the 256-expert layer over
  a whole prompt (one routing launch, one grouping, member tiles: the shared expert has every row) with exact
  routing and its outputs within the MoE bars on sampled rows; rows alone == rows in the prompt, bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle as O
from vllm_espalier import dense as Dn
from vllm_espalier import experts as G
from vllm_espalier import ops
from vllm_espalier import step as S
from vllm_espalier import workloads as WL

pytestmark = pytest.mark.gpu
D, I, VOCAB = 2048, 512, 151936


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def bf(t: torch.Tensor) -> np.ndarray:
    return O.bf16_to_f32(bits(t)).astype(np.float64)


_W: dict = {}


def weight(m) -> np.ndarray:
    """The oracle's decoded weight (fp64) of an EspMatrix, cached by trellis address."""
    key = m.trellis.data_ptr()
    if key not in _W:
        _W[key] = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, G.KERNEL_CB[m.cb]).astype(np.float64)
    return _W[key]


def lin(x: np.ndarray, m) -> np.ndarray:
    return O.linear_ref(x, weight(m), bits(m.suh), bits(m.svh))


def head_ref(x: np.ndarray, m, chunk: int = 8192) -> np.ndarray:
    """linear_ref over column chunks of a very wide matrix (the head), never holding its whole fp64 weight."""
    xr = O.had64(x.astype(np.float64) * O.f16(bits(m.suh)).astype(np.float64))
    t = m.trellis.cpu().numpy()
    svh = O.f16(bits(m.svh)).astype(np.float64)
    out = np.empty((x.shape[0], m.out_features))
    for c0 in range(0, m.out_features, chunk):
        nt0, nt1 = c0 // 16, min(m.out_features, c0 + chunk) // 16
        W = O.dequant_f32(np.ascontiguousarray(t[:, nt0:nt1]), 2 * m.K, G.KERNEL_CB[m.cb])
        out[:, c0:c0 + W.shape[1]] = O.had64(xr @ W.astype(np.float64)) * svh[c0:c0 + W.shape[1]]
    return out


def check_gemm(got: torch.Tensor, ref: np.ndarray, gate: bool = True):
    g = got.float().cpu().numpy()
    e = O.rel_l2(g, ref)
    assert e < 2e-2, f"rel L2 {e:.3e}"
    if gate:
        f = O.rel_max_above_floor(g, ref, "bf16" if got.dtype == torch.bfloat16 else np.float16)
        assert f < 5e-4, f"max error above the output floor {f:.3e}"


# ---------------------------------------------------------------------------------------------------------------
# config 5's LM head
# ---------------------------------------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def head(dev):
    gen = torch.Generator(device=dev).manual_seed(151)
    return Dn.Dense([WL.matrix(D, VOCAB, 6, "mcg", gen, dev)])


@pytest.mark.parametrize("M", [1, 4])
def test_lm_head_full_width(dev, head, M):
    print(f"LM head M={M}", flush=True)
    x = torch.randn((M, D), generator=torch.Generator().manual_seed(M)).to(torch.bfloat16).to(dev)
    y = head.forward(x)
    torch.cuda.synchronize()
    check_gemm(y, head_ref(bf(x), head.mats[0]))


# ---------------------------------------------------------------------------------------------------------------
# config 4 at 256 experts
# ---------------------------------------------------------------------------------------------------------------
def baseline_moe(dev, seed: int, E: int = 256):
    """BASELINE config 4's layer: per-expert width uniform in {1, 2, 3} bits, the shared expert 4-bit int5."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    widths = torch.randint(1, 4, (E,), generator=gen, device=dev).tolist()
    grid = {1: "e2m1", 2: "e2m1", 3: "int5"}
    experts = [tuple(WL.matrix(k, n, b, grid[b], gen, dev) for k, n in ((D, I), (D, I), (I, D))) for b in widths]
    shared = tuple(WL.matrix(k, n, 4, "int5", gen, dev) for k, n in ((D, I), (D, I), (I, D)))
    gate_w = (torch.randn((D,), generator=gen, device=dev) * 0.05).to(torch.bfloat16)
    router = (torch.randn((E, D), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    return G.prepare(experts, shared, gate_w), experts, shared, gate_w, router


@pytest.fixture(scope="module")
def moe256(dev):
    return baseline_moe(dev, 256)


def mlp_ref(x: np.ndarray, mats) -> np.ndarray:
    g, u, d = mats
    a = lin(x, g)
    return lin(a / (1 + np.exp(-a)) * lin(x, u), d)


_WT: dict = {}


def tight_weight(m) -> np.ndarray:
    """The weight the grouped GEMM multiplies: the decoded value, except the int5 / int6 grids, which it decodes as
    the index q and scales its fp32 sums by c afterwards, so q * c unrounded (the dense reference path does the same,
    dense.cu:123,292,312)."""
    key = m.trellis.data_ptr()
    if key not in _WT:
        kcb = G.KERNEL_CB[m.cb]
        if kcb in (6, 7):
            q = O.dequant_f32(m.trellis.cpu().numpy(), 2 * m.K, kcb + 16).astype(np.float64)
            _WT[key] = q * float(O.GRID_C[kcb])
        else:
            _WT[key] = weight(m)
    return _WT[key]


def mlp_faithful(x_bits: np.ndarray, mats) -> np.ndarray:
    """The expert MLP with the pipeline's own roundings (experts.cu:97-162): the rotated inputs H(x * suh) rounded
    to fp16 (rot_in, bit-exact from the oracle), the gate/up epilogue's output rounded to fp16 (the down input), fp64
    everywhere else."""
    g, u, d = mats
    xg = O.f16(O.rotate(x_bits, "bf16", bits(g.suh))).astype(np.float64)
    xu = O.f16(O.rotate(x_bits, "bf16", bits(u.suh))).astype(np.float64)
    gate = O.had64(xg @ tight_weight(g)) * O.f16(bits(g.svh)).astype(np.float64)
    up = O.had64(xu @ tight_weight(u)) * O.f16(bits(u.svh)).astype(np.float64)
    act = gate / (1 + np.exp(-gate)) * up
    xd = O.had64(act * O.f16(bits(d.suh)).astype(np.float64)).astype(np.float16).astype(np.float64)
    return O.had64(xd @ tight_weight(d)) * O.f16(bits(d.svh)).astype(np.float64)


def moe_ref(x: torch.Tensor, pick, wts, experts, shared, gate_w, faithful: bool = False):
    """(routed sum, gated shared output) in fp64 for bf16 rows x: plain (dequantised weights, no intermediate
    rounding) or faithful (mlp_faithful)."""
    xb = bits(x)
    xf = O.bf16_to_f32(xb).astype(np.float64)
    mlp = (lambda r, mats: mlp_faithful(xb[r], mats)) if faithful else (lambda r, mats: mlp_ref(xf[r], mats))
    out = np.zeros_like(xf)
    sh = np.zeros_like(xf)
    for r in range(xf.shape[0]):
        for j in range(pick.shape[1]):
            out[r] += float(wts[r, j]) * mlp(slice(r, r + 1), experts[int(pick[r, j])])[0]
        sh[r] = mlp(slice(r, r + 1), shared)[0]
    gate = 1 / (1 + np.exp(-(xf @ bf(gate_w))))
    return out, gate[:, None] * sh


def check_moe(out, osh, x, pick, wts, experts, shared, gate_w):
    """2e-2 relative L2 against the plain fp64 reference; the reference's 5e-4 max-error gate above the bf16 output
    floor (tests/gpu_grouped_shared.py:149-152) against the rounding-faithful one."""
    rref, sref = moe_ref(x, pick, wts, experts, shared, gate_w)
    check_gemm(out, rref, gate=False)
    check_gemm(osh, sref, gate=False)
    rf, sf = moe_ref(x, pick, wts, experts, shared, gate_w, faithful=True)
    for got, ref in ((out, rf), (osh, sf)):
        f = O.rel_max_above_floor(got.float().cpu().numpy(), ref, "bf16")
        assert f < 5e-4, f"max error above the bf16 floor {f:.3e}"


@pytest.mark.parametrize("T", [1, 4, 32])
def test_moe_256_experts_given_picks(dev, moe256, T):
    print(f"moe 256 experts, given picks, T={T}", flush=True)
    L, experts, shared, gate_w, _ = moe256
    gen = torch.Generator().manual_seed(400 + T)
    x = torch.randn((T, D), generator=gen).to(torch.bfloat16).to(dev)
    pick = torch.stack([torch.randperm(256, generator=gen)[:8] for _ in range(T)]).to(torch.int32)
    wts = torch.softmax(torch.randn((T, 8), generator=gen), -1)
    s = G.scratch(L, 32, 9, dev)
    out, osh = G.routed2(x, pick.to(dev), wts.to(dev), L, s)
    torch.cuda.synchronize()
    if T == 32:
        assert int(s.count.item()) == len(set(pick.view(-1).tolist())) + 1     # distinct routed + the shared slot
    check_moe(out, osh, x, pick.numpy(), wts.numpy(), experts, shared, gate_w)


@pytest.mark.parametrize("T", [1, 4, 32])
def test_moe_256_experts_fused_routing(dev, moe256, T):
    print(f"moe 256 experts, fused routing, T={T}", flush=True)
    L, experts, shared, gate_w, router = moe256
    x = torch.randn((T, D), generator=torch.Generator().manual_seed(500 + T)).to(torch.bfloat16).to(dev)
    s = G.scratch(L, 32, 9, dev)
    G.route(x, router, 8, L, s)
    out, osh = G.routed2(x, None, None, L, s, k=8)
    torch.cuda.synchronize()
    opick, owts, _, _ = O.route(bits(x), bits(router), 8, bits(gate_w), 256)
    assert np.array_equal(s.pick[:T * 9].view(T, 9).cpu().numpy(), opick)
    assert np.abs(s.wts[:T * 9].view(T, 9).cpu().numpy().astype(np.float64) - owts).max() < 1e-6
    check_moe(out, osh, x, opick[:, :8], owts[:, :8], experts, shared, gate_w)


# ---------------------------------------------------------------------------------------------------------------
# config 5: one full-width layer, stage by stage
# ---------------------------------------------------------------------------------------------------------------
def norm_ref(h: np.ndarray, w: torch.Tensor, eps: float = S.EPS) -> np.ndarray:
    """bf16 bits of (h * 1 / sqrt(mean(h^2) + eps)) * w in fp32 (the decode-step glue's RMSNorm)."""
    hf = torch.from_numpy(h.astype(np.float32))
    inv = 1.0 / torch.sqrt((hf ** 2).sum(dim=1, keepdim=True) / hf.shape[1] + eps)
    return bits(((hf * inv) * w.float().cpu()).to(torch.bfloat16))


def ulps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    x, y = a.astype(np.int16).astype(np.int32), b.astype(np.int16).astype(np.int32)
    x = np.where(x < 0, -(x & 0x7FFF), x)
    y = np.where(y < 0, -(y & 0x7FFF), y)
    return np.abs(x - y)


def add_bf16(*xs: np.ndarray) -> np.ndarray:
    """bf16 bits of the fp32 sum taken in argument order (the residual adds)."""
    z = xs[0].astype(np.float32)
    for v in xs[1:]:
        z = z + v.astype(np.float32)
    return O.f32_to_bf16(z)


@pytest.fixture(scope="module")
def decoder1(dev):
    return S.SyntheticDecoder(n_layers=1, seed=77, device=dev)


@pytest.mark.parametrize("T", [1, 2])
def test_decoder_layer_full_width_stages(dev, decoder1, T):
    print(f"one full-width decoder layer, T={T}", flush=True)
    dec = decoder1
    assert dec.fused_norms(T) and dec.fused_head_norm(T)      # (the full-width head fuses its norm up to 2 rows)
    L = dec.layers[0]
    ids = [5, 151935, 70000][:T]
    b = dec.buffers(T)
    b.ids_in.copy_(torch.tensor(ids, dtype=torch.int32))
    dec.forward(T)
    torch.cuda.synchronize()
    x0 = bf(dec.embedding[torch.tensor(ids, device=dev)])
    # qkv from the norm of the embeddings (the fused launch keeps its normalised rows to itself)
    a1 = O.bf16_to_f32(norm_ref(x0, L.norm1)).astype(np.float64)
    q_cols = [(0, 4096), (4096, 4608), (4608, 5120)]
    for m, (c0, c1) in zip(L.qkv.mats, q_cols):
        check_gemm(b.qkv[:, c0:c1], lin(a1, m), gate=False)
    # o reads q itself (the attention placeholder)
    check_gemm(b.o, lin(bf(b.qkv[:, :4096]), L.o.mats[0]))
    # the residual after o, and the router's normalised input
    h_mid = bits(b.h)
    assert np.array_equal(h_mid, add_bf16(x0, bf(b.o)))
    u = ulps(bits(b.a), norm_ref(O.bf16_to_f32(h_mid), L.norm2))
    assert u.max() <= 1 and (u == 0).mean() > 0.99
    # routing on the GPU's normalised rows: ids exact
    opick, owts, _, _ = O.route(bits(b.a), bits(L.router), 8, bits(L.moe.gate_w), 256)
    assert np.array_equal(dec.scratch.pick[:T * 9].view(T, 9).cpu().numpy(), opick)
    check_moe(b.moe, b.moe_shared, b.a, opick[:, :8], owts[:, :8], L.experts, L.shared, L.moe.gate_w)
    # the final residual (the fused head stores it to h2), the head and the argmax
    h2 = bits(b.h2)
    assert np.array_equal(h2, add_bf16(O.bf16_to_f32(h_mid), bf(b.moe), bf(b.moe_shared)))
    af = O.bf16_to_f32(norm_ref(O.bf16_to_f32(h2), dec.final_norm)).astype(np.float64)
    check_gemm(b.logits, head_ref(af, dec.head.mats[0]), gate=False)
    assert b.ids_out.cpu().tolist() == torch.argmax(b.logits.float(), dim=1).cpu().tolist()


# ---------------------------------------------------------------------------------------------------------------
# prefill windows: rows alone == window
# ---------------------------------------------------------------------------------------------------------------
def _dense_op(mats):
    key = next(ops.DENSE_KEYS)
    ops.DENSE_LAYERS[key] = Dn.Dense(mats)
    return key


@pytest.fixture(scope="module")
def dense_kinds(dev, head):
    gen = torch.Generator(device=dev).manual_seed(9)
    kinds = {
        "qkv": [WL.matrix(D, 4096, 4, "int6", gen, dev), WL.matrix(D, 512, 4, "int6", gen, dev),
                WL.matrix(D, 512, 4, "int6", gen, dev)],
        "o": [WL.matrix(4096, D, 4, "int6", gen, dev)],
        "shared_gate_up": [WL.matrix(D, I, 4, "int5", gen, dev), WL.matrix(D, I, 4, "int5", gen, dev)],
        "shared_down": [WL.matrix(I, D, 4, "int5", gen, dev)],
        "lm_head": head.mats,
    }
    return {k: (_dense_op(v), v) for k, v in kinds.items()}


@pytest.mark.parametrize("T", [33, 100, 517])
@pytest.mark.parametrize("kind", ["qkv", "o", "shared_gate_up", "shared_down", "lm_head"])
def test_prefill_dense_rows_alone_equal_window(dev, dense_kinds, kind, T):
    print(f"prefill dense {kind} T={T}", flush=True)
    assert ops.PREFILL == "chunk"
    key, mats = dense_kinds[kind]
    trellis, suh, svh = [m.trellis for m in mats], [m.suh for m in mats], [m.svh for m in mats]
    x = torch.randn((T, mats[0].in_features), generator=torch.Generator().manual_seed(T)).to(torch.bfloat16).to(dev)
    y = torch.ops.espalier.dense(x, trellis, suh, svh, key)
    assert y.shape == (T, sum(m.out_features for m in mats))
    rows = torch.empty_like(y)
    for r in range(T):
        rows[r:r + 1] = torch.ops.espalier.dense(x[r:r + 1], trellis, suh, svh, key)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), rows.view(torch.int16))


@pytest.mark.parametrize("T", [33, 100, 517])
@pytest.mark.parametrize("routing", ["given", "fused"])
def test_prefill_moe_rows_alone_equal_window(dev, moe256, T, routing):
    print(f"prefill moe {routing} T={T}", flush=True)
    L, experts, shared, gate_w, router = moe256
    gen = torch.Generator().manual_seed(600 + T)
    x = torch.randn((T, D), generator=gen).to(torch.bfloat16).to(dev)
    s = G.scratch(L, 32, 9, dev)
    if routing == "given":
        pick = torch.stack([torch.randperm(256, generator=gen)[:8] for _ in range(T)]).to(torch.int32).to(dev)
        wts = torch.softmax(torch.randn((T, 8), generator=gen), -1).to(dev)
        out, sh = G.windows(x, pick, wts, L, s)
    else:
        pick = wts = None
        out, sh = G.windows(x, None, None, L, s, k=8, gate=router)
    out, sh = out.clone(), sh.clone()
    for r in range(T):
        if routing == "given":
            o1, s1 = G.routed2(x[r:r + 1], pick[r:r + 1], wts[r:r + 1], L, s)
        else:
            G.route(x[r:r + 1], router, 8, L, s)
            o1, s1 = G.routed2(x[r:r + 1], None, None, L, s, k=8)
        assert torch.equal(o1.view(torch.int16), out[r:r + 1].view(torch.int16)), r
        assert torch.equal(s1.view(torch.int16), sh[r:r + 1].view(torch.int16)), r


# ---------------------------------------------------------------------------------------------------------------
# the prompt paths (tile mode) at full size
# ---------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("kind", ["qkv", "o", "shared_gate_up", "shared_down", "lm_head"])
def test_prompt_dense_full_size(dev, dense_kinds, kind):
    """Dense.forward_tile over 517 rows (four full 128-row tiles and a 5-row one) against the oracle; rows at tile
    edges alone equal the same rows in the prompt, bit for bit."""
    print(f"prompt dense {kind} T=517", flush=True)
    key, mats = dense_kinds[kind]
    d = ops.DENSE_LAYERS[key]
    T = 517
    x = torch.randn((T, mats[0].in_features), generator=torch.Generator().manual_seed(700)).to(torch.bfloat16).to(dev)
    y = d.forward_tile(x).clone()
    torch.cuda.synchronize()
    xf = bf(x)
    if kind == "lm_head":
        rows = [0, 127, 128, 516]                            # the head's fp64 reference on a sample of rows
        check_gemm(y[rows], head_ref(xf[rows], mats[0]))
    else:
        for m, c0 in zip(mats, d.col0):
            check_gemm(y[:, c0:c0 + m.out_features], lin(xf, m))
    for r in (0, 127, 128, 512, 516):
        y1 = d.forward_tile(x[r:r + 1])
        assert torch.equal(y1.view(torch.int16), y[r:r + 1].view(torch.int16)), r


@pytest.mark.parametrize("T", [200, 517])
def test_prompt_moe_256_experts(dev, moe256, T):
    """experts.prefill over a whole prompt with fused routing (route_rows): picks bit-exact against exact routing,
    outputs within the MoE bars on sampled rows, rows alone == rows in the prompt."""
    print(f"prompt moe 256 experts T={T}", flush=True)
    L, experts, shared, gate_w, router = moe256
    x = torch.randn((T, D), generator=torch.Generator().manual_seed(800 + T)).to(torch.bfloat16).to(dev)
    ps = G.prefill_scratch(L, T, 9, dev)
    out, osh = (t.clone() for t in G.prefill(x, None, None, L, ps, 8, gate=router))
    torch.cuda.synchronize()
    assert int(G.ext().status(True)) == 0
    opick, owts, _, _ = O.route(bits(x), bits(router), 8, bits(gate_w), 256)
    assert np.array_equal(ps.pick[:T * 9].view(T, 9).cpu().numpy(), opick)
    rows = [0, 1, 31, 32, 100, T - 2, T - 1]
    check_moe(out[rows], osh[rows], x[rows], opick[rows, :8], owts[rows, :8], experts, shared, gate_w)
    for r in (0, 33, T - 1):
        o1, s1 = G.prefill(x[r:r + 1], None, None, L, ps, 8, gate=router)
        assert torch.equal(o1.view(torch.int16), out[r:r + 1].view(torch.int16)), r
        assert torch.equal(s1.view(torch.int16), osh[r:r + 1].view(torch.int16)), r

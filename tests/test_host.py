"""Host-side logic of the package on the CPU: launch plans, tile settings, launch grouping, checkpoint parsing and
the expert tables. Nothing here calls a kernel."""
import numpy as np
import pytest
import torch

import oracle as O
from vllm_espalier import dense as D
from vllm_espalier import experts as X
from vllm_espalier import workloads as WL
from vllm_espalier.matrix import EspMatrix

# BASELINE shapes (K, N): config 1, the config-2 launches, the config-5 head
SHAPES = [(2048, 2048), (2048, 5120), (4096, 2048), (2048, 1024), (512, 2048), (2048, 151936)]


def test_tables_match_the_oracle():
    assert X.KERNEL_CB == O.KERNEL_CB
    assert X.COMPILED == O.COMPILED


@pytest.mark.parametrize("K,N", SHAPES)
def test_dense_plan_is_valid(K, N):
    sk, w, pf = D.plan(K, N, 256)
    assert w in (4, 8, 16) and 1 <= sk <= K // 32         # splits of whole 32-k steps
    steps = -(-(K // 32) // sk)                           # the longest split
    assert steps >= w // 4                                # every k slot of the workgroup has a step
    assert (N // 128) * sk <= max(N // 128, 256)          # the splits keep to a workgroup a CU


def _chunks_max(K, SK):
    """esp_dense's bound on the 128-blocks one split's rotated rows touch (its shared-memory sizing)."""
    sq, sr = divmod(K // 32, SK)
    steps_max = sq + (sr > 0)
    aligned = sr == 0 and sq % 4 == 0
    return steps_max // 4 if aligned else (steps_max * 32 + 96 + 127) // 128


@pytest.mark.parametrize("K", [128, 256, 384, 512, 1024, 2048, 4096, 6144])
def test_dense_splits_cover_k_and_fit_the_rotation_buffer(K):
    """The kernel's split s of S = K/32 = SQ*SK + SR steps starts at s*SQ + min(s, SR) and has SQ + (s < SR): the
    splits tile the steps in order, and no split's rotated rows (the 128-blocks its range touches) exceed the shared
    memory esp_dense sizes for them."""
    S = K // 32
    for SK in range(1, S + 1):
        sq, sr = divmod(S, SK)
        bounds = [(s * sq + min(s, sr), s * sq + min(s, sr) + sq + (s < sr)) for s in range(SK)]
        assert bounds[0][0] == 0 and bounds[-1][1] == S
        assert all(b[1] == c[0] for b, c in zip(bounds, bounds[1:]))
        assert all(b[1] > b[0] for b in bounds)
        cmax = _chunks_max(K, SK)
        for s0, s1 in bounds:
            k0, kr = 32 * s0, 32 * (s1 - s0)
            chunks = ((k0 + kr + 127) >> 7) - (k0 >> 7)
            assert chunks <= cmax, (K, SK, s0, s1)
            assert 32 * (s1 - s0) <= 32 * ((S + SK - 1) // SK)          # the stage buffer's size


@pytest.mark.parametrize("K,N", SHAPES + [(2048, 512), (1024, 1024), (8192, 4096)])
def test_prompt_plan_is_valid(K, N):
    """The prompt launches' K splits: 1 to 8, splits of at least 128 k (one 4-step stage), and at 512 rows (four
    128-row tiles) a grid within two workgroups a CU that one more split would pass (unless capped)."""
    sk = D.tile_plan(K, N)
    assert 1 <= sk <= min(8, max(1, K // 128))
    per_split = 4 * (N // 128)
    assert per_split * sk <= 512 or sk == 1
    assert per_split * (sk + 1) > 512 or sk in (8, K // 128)


def test_prompt_plan_config2():
    """config 2's launches: qkv 3 splits (480 workgroups at 512 rows), o 8 (512), shared gate/up 8 (256), shared
    down 4 (256, its K of 512 in splits of 128)."""
    assert [D.tile_plan(K, N) for K, N in ((2048, 5120), (4096, 2048), (2048, 1024), (512, 2048))] == [3, 8, 8, 4]


def test_dense_plan_depends_on_shape_only(monkeypatch):
    assert D.plan(2048, 5120, 256) == D.plan(2048, 5120, 256)
    monkeypatch.setenv("ESPALIER_DENSE_TILE_PLAN", "2,8,1")
    assert D.plan(2048, 5120, 256) == (2, 8, 1)


@pytest.mark.parametrize("K,N", [(2048, 512), (512, 2048), (2048, 1024), (4096, 4096)])
def test_tile_config_is_valid(K, N):
    nt, w, sk, pf = X.tile_config(K, N, True)
    assert nt == 8 and w in (4, 8, 16) and sk >= 1
    assert K % (32 * sk) == 0 and (K // sk) // 32 >= (w // 4)


def test_tile_config_rejects_ragged():
    with pytest.raises(ValueError):
        X.tile_config(2048, 500, True)


def _mat(K, N, bits, grid, seed=0):
    return WL.matrix(K, N, bits, grid, torch.Generator().manual_seed(seed), "cpu")


def test_dense_groups_launches_by_codebook_and_width():
    mats = [_mat(256, 128, 4, "int6"), _mat(256, 256, 4, "int6"), _mat(256, 128, 4, "int5"),
            _mat(256, 128, 3, "int5"), _mat(256, 128, 3, "int5")]
    d = D.Dense(mats)
    assert [(g[0], g[1], g[2]) for g in d.groups] == [([0, 1], 8, 7), ([2], 8, 6), ([3, 4], 6, 6)]
    assert d.col0 == [0, 128, 384, 512, 640] and d.N == 768
    six = D.Dense([_mat(256, 128, 4, "int6", s) for s in range(6)])
    assert [len(g[0]) for g in six.groups] == [4, 2]      # at most 4 matrices a launch
    with pytest.raises(ValueError):
        D.Dense([_mat(256, 128, 4, "int6"), _mat(512, 128, 4, "int6")])


def test_espmatrix_codebook_markers():
    t = WL.matrix_tensors(32, 32, 2, "mcg", torch.Generator().manual_seed(1))
    assert EspMatrix(t).cb == 0
    assert EspMatrix({**t, "mul1": torch.zeros(1)}).cb == 1
    assert EspMatrix({**t, "esp_grid": torch.tensor([4], dtype=torch.int32)}).cb == 4
    with pytest.raises(ValueError):
        EspMatrix({k: v for k, v in t.items() if k != "mcg"})
    with pytest.raises(ValueError):
        EspMatrix({**t, "esp_grid": torch.tensor([7], dtype=torch.int32)})
    bad = dict(t)
    bad["esp_trellis"] = t["esp_trellis"][:1]
    with pytest.raises(ValueError):
        EspMatrix(bad)


def test_workload_bytes_and_determinism():
    a = WL.matrix_tensors(2048, 2048, 4, "int6", torch.Generator().manual_seed(3))
    b = WL.matrix_tensors(2048, 2048, 4, "int6", torch.Generator().manual_seed(3))
    assert all(torch.equal(a[k], b[k]) for k in a)
    m = EspMatrix(a)
    assert WL.nbytes([m]) == 2105344                      # config 1's algorithmic bytes
    s = a["suh"].float()
    assert torch.all(s.abs() == 1)


def test_prepare_tables():
    E, Dm, I = 3, 256, 128
    exps = [tuple(_mat(k, n, b, g, 10 * e + j) for j, (k, n) in enumerate([(Dm, I), (Dm, I), (I, Dm)]))
            for e, (b, g) in enumerate([(1, "e2m1"), (2, "e2m1"), (3, "int5")])]
    shared = tuple(_mat(k, n, 4, "int6", 99 + j) for j, (k, n) in enumerate([(Dm, I), (Dm, I), (I, Dm)]))
    L = X.prepare(exps, shared, gate_w=torch.zeros(Dm, dtype=torch.bfloat16))
    assert L.E == 4 and L.shared_id == 3 and (L.D, L.I) == (Dm, I)
    assert L.k2[0].tolist() == [2, 4, 6, 8] and L.cb[0].tolist() == [3, 3, 6, 7]
    assert L.k2_gu == (2, 8)
    assert L.ptr[2][1].item() == exps[1][2].trellis.data_ptr()
    # suh/svh rebound as rows of the stacks
    assert exps[2][0].suh.data_ptr() == L.suh_g[2].data_ptr()
    bad = [tuple(_mat(k, n, 4, "e2m1", j) for j, (k, n) in enumerate([(Dm, I), (Dm, I), (I, Dm)]))]
    with pytest.raises(NotImplementedError):
        X.prepare(bad)                                    # E2M1 has no 4-bit instance


def test_int6_index_through_magic_sum():
    """The dense kernels' int6 grid index (csrc/trellis.hpp, codebook 23): fp16(v * k' + 1536) - 1536 with
    k' = 0x1.f6628p+2 equals the reference's rintf(f32(v) * k) on every mcg value, whether the mixed fma rounds its
    exact sum straight to fp16 or first to fp32; every v * k' stays more than 2^-13 from a half-integer. Exact rational
    arithmetic over the 10,746 distinct values."""
    from fractions import Fraction as F
    mcg = np.unique(O.codebook_table(1))
    v = O.f16(mcg).astype(np.float64)
    q_ref = np.rint((v.astype(np.float32) * np.float32(float.fromhex("0x1.f660bap+2"))).astype(np.float32))
    kp = F(float.fromhex("0x1.f6628p+2"))
    for a, q in zip(v.tolist(), q_ref.tolist()):
        e = F(a) * kp
        fl = e.numerator // e.denominator
        assert abs(e - fl - F(1, 2)) > F(1, 8192)
        direct = fl + 1 if e - fl > F(1, 2) else fl                     # no ties: the distance check above
        via_f32 = int(np.float16(np.float32(float(e + 1536)))) - 1536
        assert direct == q and via_f32 == q, (a, q, direct, via_f32)


@pytest.mark.parametrize("E,k,T", [(16, 8, 517), (256, 8, 512), (256, 9, 2048), (64, 2, 33)])
def test_tile_list_cap_bounds_every_grouping(E, k, T):
    """tile_list_cap(maxu, T, P) bounds the non-empty 32-row member tiles of any grouping of P = T * k picks: the sum
    over experts of ceil(members / 32) is at most ceil(P / 32) + the experts used, and at most maxu * ceil(T / 32).
    Checked on random picks, on picks piled onto a few experts, and on every expert given one member more than a
    multiple of 32 (the worst case of the first bound)."""
    rng = np.random.default_rng(E * 1000 + T)
    P = T * k
    maxu = min(P, E)
    cap = X.tile_list_cap(maxu, T, P)
    cases = [rng.integers(0, E, size=P), rng.integers(0, min(E, 3), size=P)]
    skew = np.concatenate([np.full(33, e) for e in range(E)] * (P // (33 * E) + 1))[:P]
    cases.append(skew)
    for picks in cases:
        counts = np.bincount(picks, minlength=E)
        counts = np.minimum(counts, T)               # a token picks an expert once: at most T members an expert
        tiles = int(sum(-(-int(c) // 32) for c in counts if c > 0))
        assert tiles <= cap, (tiles, cap)
    assert cap <= maxu * -(-T // 32)


def test_shared_scratch_keeps_outgrown_buffers_only_when_captured():
    """dense._SharedScratch: a pair outgrown outside any capture is dropped (the allocator reuses it); one handed out
    during a capture is kept, since a graph may still write to it."""
    from vllm_espalier import dense as Dn
    s = Dn._SharedScratch()
    dev = torch.device("cpu")
    a = s.reserve(dev, 10, 10)
    b = s.reserve(dev, 20, 10)
    assert s.retired == [] and s.reserve(dev, 5, 5) is b and b[0].numel() == 20 and b[1].numel() == 10
    s.captured.add(dev)                          # as if b had been handed out inside a stream capture
    c = s.reserve(dev, 40, 10)
    assert len(s.retired) == 1 and s.retired[0] is b and c[0].numel() == 40
    assert dev not in s.captured                 # the new pair has not been captured yet
    del a


def test_status_bits_match_the_header():
    """experts.check_status names every ESP_STATUS_* bit of include/espalier.h, with the header's values."""
    import re
    from pathlib import Path
    text = (Path(__file__).resolve().parent.parent / "include" / "espalier.h").read_text()
    bits = {int(v) for v in re.findall(r"^#define ESP_STATUS_\w+ (\d+)", text, re.M)}
    assert bits == {b for b, _ in X.STATUS_BITS}

"""CPU pins of the oracle (oracle/): every C restatement is checked against something it does not share code or
algorithm with -- numpy / torch conversions, exact rational arithmetic, closed forms and invariants, and the
codebook facts read from the reference (experts_grouped.cuh:21-80). No GPU, no HIP library."""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle as O

RNG = np.random.default_rng(20261201)


# ---------------------------------------------------------------------------------------------------------------
# number formats
# ---------------------------------------------------------------------------------------------------------------

def test_f16_to_f32_all_patterns():
    L = O.lib()
    bits = np.arange(65536, dtype=np.uint32)
    got = np.array([L.eo_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_against_numpy():
    L = O.lib()
    x = np.concatenate([
        RNG.standard_normal(20000).astype(np.float32) * np.float32(3.0),
        (RNG.standard_normal(5000) * 1e-6).astype(np.float32),           # subnormal range of fp16
        (RNG.standard_normal(2000) * 7e4).astype(np.float32),            # overflow to inf
        # exact ties between adjacent fp16 values: midpoints of random fp16 pairs
        ((RNG.integers(0x0400, 0x7B00, 5000).astype(np.uint16).view(np.float16).astype(np.float32)
          + np.nextafter(RNG.integers(0x0400, 0x7B00, 5000).astype(np.uint16).view(np.float16),
                         np.float16(np.inf)).astype(np.float32)) * np.float32(0.5)),
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.996, 6.0e-8, 2.98e-8, np.inf, -np.inf], dtype=np.float32),
    ])
    got = np.array([L.eo_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_bf16_rne_against_torch():
    L = O.lib()
    x = np.concatenate([RNG.standard_normal(20000).astype(np.float32),
                        (RNG.standard_normal(2000) * 1e-39).astype(np.float32),
                        np.array([3.4e38, -3.4e38, 0.0, -0.0], dtype=np.float32)])
    got = np.array([L.eo_f32_to_bf16(float(v)) for v in x], dtype=np.uint16)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    assert np.array_equal(O.f32_to_bf16(x), ref)


def _bf16_exact(v: Fraction) -> int:
    """RNE of an exact rational to bf16 bits (8 significant bits), by integer arithmetic."""
    if v == 0:
        return 0
    sign = 0x8000 if v < 0 else 0
    a = abs(v)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                                     # subnormals share the exponent of the smallest normal
    scaled = a / Fraction(2) ** (e - 7)                  # 8 significant bits above the point
    q, r = divmod(scaled.numerator, scaled.denominator)
    if 2 * r > scaled.denominator or (2 * r == scaled.denominator and q & 1):
        q += 1
    f = np.float32(float(Fraction(q) * Fraction(2) ** (e - 7)))
    return sign | int(f.view(np.uint32) >> 16)


def test_f64_to_bf16_single_rounding():
    """eo_f64_to_bf16 rounds the double once (route.cu rounds the fp64-exact logit once to bf16); torch converts via
    float32 (double rounding), so the check is exact rational rounding, including doubles that sit just off a bf16
    tie, where a double rounding would go the wrong way."""
    L = O.lib()
    vals = list(RNG.standard_normal(3000) * 4.0)
    for _ in range(500):                                   # bf16 ties nudged by one double ulp either way
        b = float(np.float32(RNG.standard_normal()).astype(np.float32))
        hi16 = (np.float32(b).view(np.uint32) >> 16) << 16
        tie = float(np.uint32(hi16 | 0x8000).view(np.float32))
        vals += [tie, np.nextafter(tie, np.inf), np.nextafter(tie, -np.inf)]
    for v in vals:
        assert L.eo_f64_to_bf16(float(v)) == _bf16_exact(Fraction(float(v))), v


# ---------------------------------------------------------------------------------------------------------------
# codebooks (experts_grouped.cuh:21-80): facts read off the reference, and second algorithms
# ---------------------------------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def mcg():
    return O.codebook_table(1)


def test_mcg_codebook_facts(mcg):
    v = O.f16(mcg)
    assert len(np.unique(v)) == 10746
    assert float(np.abs(v).max()) == 3.94921875            # c * top, experts_grouped.cuh:43
    assert not np.isnan(v.astype(np.float32)).any()


def test_mcg_against_uint64_arithmetic(mcg):
    """The hash in 64-bit integer arithmetic reduced mod 2^32, and the pair add in float64 rounded once to fp16 (an
    fp16 + fp16 sum is exact in float64)."""
    s = np.arange(65536, dtype=np.uint64)
    x = (s * np.uint64(0xCBAC1FED)) % np.uint64(1 << 32)
    x = (x & np.uint64(0x8FFF8FFF)) ^ np.uint64(0x3B603B60)
    lo = (x & np.uint64(0xFFFF)).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (x >> np.uint64(16)).astype(np.uint16).view(np.float16).astype(np.float64)
    ref = (lo + hi).astype(np.float16)
    assert np.array_equal(O.f16(mcg).view(np.uint16), ref.view(np.uint16))


def test_e2m1_nearest_grid_point(mcg):
    """E2M1 (cb 3) snaps |v| to the nearest of 0.75 * {0, .5, 1, 1.5, 2, 3, 4, 6}, a tie going to the smaller value,
    and keeps v's sign (so -0 exists): here by argmin of distances in float64, not by thresholds."""
    t = O.codebook_table(3)
    v = O.f16(mcg).astype(np.float64)
    grid = 0.75 * np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6])
    d = np.abs(np.abs(v)[:, None] - grid[None, :])
    idx = np.argmin(d, axis=1)                              # argmin returns the first (smaller) on ties
    ref = np.where(np.signbit(v), -grid[idx], grid[idx]).astype(np.float16)
    assert np.array_equal(t, ref.view(np.uint16))
    assert len(np.unique(O.f16(t).astype(np.float64))) == 15
    assert int(np.sum(t == 0x8000)) == 4331


def test_e2m1_gemm_form_times_three_quarters(mcg):
    """The GEMMs' E2M1 form (19) is the fp4 grid itself, {0, .5, 1, 1.5, 2, 3, 4, 6} with the sign (and -0), and 0.75
    times it is the reference value exactly (the GEMM scales its fp32 sums by 0.75)."""
    t3 = O.f16(O.codebook_table(3)).astype(np.float64)
    t19 = O.f16(O.codebook_table(19)).astype(np.float64)
    assert set(np.abs(t19).tolist()) <= {0, 0.5, 1, 1.5, 2, 3, 4, 6}
    assert np.array_equal(t19 * 0.75, t3)
    assert np.array_equal(np.signbit(t19), np.signbit(t3))


@pytest.mark.parametrize("cb,top", [(6, 15), (7, 31)])
def test_int_grid_by_division(mcg, cb, top):
    """q = rint(v * k) of the kernels equals rint(v / c) on every mcg value (the definition, experts_grouped.cuh:40-43)
    and the value is fp16(q * c)."""
    q = O.grid_q_table(cb)
    v = O.f16(mcg).astype(np.float32)
    c = O.GRID_C[cb]
    assert np.array_equal(q, np.rint(v / c).astype(np.int32))
    assert q.min() == -top and q.max() == top and len(np.unique(q)) == 2 * top + 1
    vals = O.codebook_table(cb)
    assert np.array_equal(vals, (q.astype(np.float32) * c).astype(np.float16).view(np.uint16))
    assert np.array_equal(O.codebook_table(cb + 16), q.astype(np.float16).view(np.uint16))   # cb 22/23: q itself


# ---------------------------------------------------------------------------------------------------------------
# trellis unpack (experts_grouped.cuh:83-154) and the dequantisation (:321-340)
# ---------------------------------------------------------------------------------------------------------------

def _words(tile16: np.ndarray) -> list[int]:
    u = np.ascontiguousarray(tile16, dtype=np.int16).view(np.uint16).astype(np.uint32)
    return [int(u[2 * i]) | (int(u[2 * i + 1]) << 16) for i in range(len(u) // 2)]


def _state_bigint(words: list[int], b: int, p: int) -> int:
    """The 16 stream bits ending at (p+1)*b of the circular big-endian stream, from one big integer."""
    L = 32 * len(words)
    S = 0
    for w in words:
        S = (S << 32) | w
    T = (S << L) | S                                          # two laps: windows that wrap are contiguous
    a = (p + 1) * b - 16 + L                                  # first stream bit of the window in the doubled stream
    return (T >> (2 * L - a - 16)) & 0xFFFF


def _place(p: int) -> tuple[int, int]:
    lane, j = p // 8, p % 8
    q, t, g = j // 2, lane % 4, lane // 4
    return 2 * t + 8 * (q & 1) + (j & 1), g + 8 * (q >> 1)


@pytest.mark.parametrize("k2", [2, 4, 6, 8, 10, 12, 14, 16])
def test_state_unpack_bigint(k2):
    b = k2 // 2
    for _ in range(4):
        tile = RNG.integers(-32768, 32768, 16 * b).astype(np.int16)
        words = np.array(_words(tile), dtype=np.uint32)
        for p in range(256):
            assert O.state(words, k2, p) == _state_bigint(list(map(int, words)), b, p)


def test_position_is_the_tile_bijection():
    seen = set()
    for p in range(256):
        kn = O.position(p)
        assert kn == _place(p)
        seen.add(kn)
    assert len(seen) == 256


@pytest.mark.parametrize("cb,k2", sorted(O.COMPILED))
def test_dequant_composition(cb, k2):
    """eo_dequant (tiled, threaded C) equals the composition bigint state -> codebook table -> placement."""
    b = k2 // 2
    K, N = 32, 48
    tr = RNG.integers(-32768, 32768, (K // 16, N // 16, 16 * b)).astype(np.int16)
    table = O.codebook_table(cb)
    ref = np.empty((K, N), dtype=np.uint16)
    for kt in range(K // 16):
        for nt in range(N // 16):
            words = _words(tr[kt, nt])
            for p in range(256):
                kk, nn = _place(p)
                ref[16 * kt + kk, 16 * nt + nn] = table[_state_bigint(words, b, p)]
    assert np.array_equal(O.dequant(tr, k2, cb), ref)
    f32 = O.dequant_f32(tr, k2, cb)
    assert np.array_equal(f32, O.f16(ref).astype(np.float32))


# The reference's own unpack, emulated lane by lane: Fmt / LaneMap / fetch / decode_tile (experts_grouped.cuh:83-154)
# and dequant_kernel's placement (:321-340). A 32-lane warp holds tile word l in lane l (and word 32 + l in its
# second register, load_words :168-177); fetch(idx) is a shuffle from lane idx & 31. This is the warp's algorithm,
# not the closed form, so it pins the oracle's reading of the format independently of test_state_unpack_bigint.
def _ref_fmt(k2: int):
    TW = 4 * k2
    GV = 2 if k2 >= 13 else (4 if (k2 == 7 or 9 <= k2 <= 12 or k2 == 16) else 8)

    def end(p):
        return (p >> 1) * k2 + (k2 if p & 1 else k2 >> 1)
    return TW, GV, 8 // GV, end


def _ref_decode_tile_states(words: list[int], k2: int, lane: int) -> list[int]:
    TW, GV, NG, end = _ref_fmt(k2)
    M32 = 0xFFFFFFFF
    if k2 == 8:
        w0, p = words[lane], words[(lane + 31) & 31]
        s = ((((p & M32) << 32) | w0) >> 20) & M32             # __funnelshift_r(w0, p, 20)
        return [(s >> 8) & 0xFFFF, (s >> 4) & 0xFFFF, s & 0xFFFF, w0 >> 16, (w0 >> 12) & 0xFFFF,
                (w0 >> 8) & 0xFFFF, (w0 >> 4) & 0xFFFF, w0 & 0xFFFF]
    st = [0] * 8
    for g in range(NG):
        last_end = end(8 * lane + g * GV + GV - 1) + 128 * k2
        hr = (last_end - 1) >> 5
        hi, lo, sh = hr % TW, (hr + TW - 1) % TW, (hr + 1) * 32 - last_end
        mm = ((words[lo] << 32) | words[hi]) >> sh
        for j in range(GV):
            st[g * GV + j] = (mm >> (end(GV - 1) - end(j))) & 0xFFFF
    return st


@pytest.mark.parametrize("k2", [2, 4, 6, 8, 10, 12, 14, 16])
def test_state_unpack_matches_reference_lane_map(k2):
    """Every lane's eight states from the emulated reference decode equal the oracle's eo_state, and the reference
    dequant_kernel's placement of them equals eo_position, over random tiles."""
    b = k2 // 2
    for _ in range(20):
        tile = RNG.integers(-32768, 32768, 16 * b).astype(np.int16)
        words = _words(tile)
        wa = np.array(words, dtype=np.uint32)
        for lane in range(32):
            st = _ref_decode_tile_states(words, k2, lane)
            g, t = lane >> 2, lane & 3
            for j in range(8):
                p = 8 * lane + j
                assert O.state(wa, k2, p) == st[j], (k2, lane, j)
                q = j >> 1                                     # half2 v[q] = (st[2q], st[2q+1]), rows row, row + 1
                assert O.position(p) == (2 * t + 8 * (q & 1) + (j & 1), g + 8 * (q >> 1)), (lane, j)


@pytest.mark.parametrize("cb,k2", sorted(O.COMPILED))
def test_dequant_matches_reference_kernel_emulation(cb, k2):
    """O.dequant on a 2 x 3 tile matrix equals the emulated reference dequant_kernel: lane decode, codebook pairs,
    out[row][col] / out[row + 1][col] stores."""
    b = k2 // 2
    tr = RNG.integers(-32768, 32768, (2, 3, 16 * b)).astype(np.int16)
    table = O.codebook_table(cb)
    ref = np.full((32, 48), 0xDEAD, dtype=np.uint16)
    for kt in range(2):
        for nt in range(3):
            words = _words(tr[kt, nt])
            for lane in range(32):
                st = _ref_decode_tile_states(words, k2, lane)
                g, t = lane >> 2, lane & 3
                for q in range(4):
                    col, row = nt * 16 + g + 8 * (q >> 1), kt * 16 + 2 * t + 8 * (q & 1)
                    ref[row, col] = table[st[2 * q]]
                    ref[row + 1, col] = table[st[2 * q + 1]]
    assert np.array_equal(O.dequant(tr, k2, cb), ref)


def test_dequant_rejects_unsupported():
    tr = np.zeros((1, 1, 16 * 5), dtype=np.int16)
    with pytest.raises(ValueError):
        O.dequant(tr, 10, 3)                                   # E2M1 only at K2 2/4/6


# ---------------------------------------------------------------------------------------------------------------
# Hadamard (experts.cu:79-90, dense.cu:92-128)
# ---------------------------------------------------------------------------------------------------------------

def test_fwht_integers_exact_sylvester():
    """On small integers every partial sum is exact, so the transform must equal the Sylvester product exactly."""
    H = O.sylvester().astype(np.int64)
    for _ in range(20):
        v = RNG.integers(-1000, 1000, 128)
        assert np.array_equal(O.fwht128_f32(v.astype(np.float32)).astype(np.int64), H @ v)


def test_fwht_involution_and_float():
    H = O.sylvester()
    v = RNG.standard_normal(128).astype(np.float32)
    y = O.fwht128_f32(v).astype(np.float64)
    assert np.allclose(y, H @ v.astype(np.float64), rtol=0, atol=1e-4)
    z = O.fwht128_f32(O.fwht128_f32(v)) / np.float32(128.0)
    assert np.allclose(z, v, rtol=0, atol=1e-5)


def test_rotate_within_one_ulp_of_fp64():
    M, K = 4, 512
    x = RNG.standard_normal((M, K)).astype(np.float32)
    suh = np.where(RNG.integers(0, 2, K) == 1, 1.0, -1.0).astype(np.float16)
    xb = O.f32_to_bf16(x)
    got = O.f16(O.rotate(xb, "bf16", suh.view(np.uint16))).astype(np.float64)
    ref = O.had64(O.bf16_to_f32(xb).astype(np.float64) * suh.astype(np.float64))
    ulp = np.abs(np.spacing(ref.astype(np.float16)).astype(np.float64))
    assert np.all(np.abs(got - ref) <= ulp)
    # f32 input path and fp16 input path agree with the bf16 path on the same values
    assert np.array_equal(O.rotate(O.bf16_to_f32(xb), "f32", suh.view(np.uint16)), O.rotate(xb, "bf16", suh.view(np.uint16)))


def test_had_pre_post_against_fp64():
    M, K = 3, 256
    x = RNG.standard_normal((M, K)).astype(np.float16)
    pre = RNG.standard_normal(K).astype(np.float16)
    post = RNG.standard_normal(K).astype(np.float16)
    got = O.f16(O.had(x.view(np.uint16), pre.view(np.uint16), post.view(np.uint16))).astype(np.float64)
    ref = O.had64(x.astype(np.float64) * pre.astype(np.float64)) * post.astype(np.float64)
    assert np.allclose(got, ref, rtol=2e-3, atol=2e-3)
    plain = O.f16(O.had(x.view(np.uint16))).astype(np.float64)
    assert np.allclose(plain, O.had64(x.astype(np.float64)), rtol=2e-3, atol=2e-3)


# ---------------------------------------------------------------------------------------------------------------
# routing (route.cu:35-181) and grouping (experts.cu:19-76)
# ---------------------------------------------------------------------------------------------------------------

def _route_fraction(xb, gb, k, sgb):
    """Exact rational logits -> bf16 -> softmax over the picks in float64 (the reference's softmax is fp32; weights
    are compared with a tolerance) -> lowest id on ties."""
    R, H = xb.shape
    E = gb.shape[0]
    xf = O.bf16_to_f32(xb).astype(np.float64)
    gf = O.bf16_to_f32(gb).astype(np.float64)
    picks, wts, bits = [], [], []
    for r in range(R):
        lb = [_bf16_exact(sum((Fraction(float(a)) * Fraction(float(c)) for a, c in zip(xf[r], gf[e])), Fraction(0)))
              for e in range(E)]
        l = O.bf16_to_f32(np.array(lb, dtype=np.uint16)).astype(np.float64)
        order = sorted(range(E), key=lambda e: (-l[e], e))[:k]
        p = np.exp(l[order] - l.max())
        picks.append(order)
        wts.append(p / p.sum())
        bits.append(lb)
    shared = None
    if sgb is not None:
        sf = O.bf16_to_f32(sgb).astype(np.float64)
        shared = [float(sum((Fraction(float(a)) * Fraction(float(c)) for a, c in zip(xf[r], sf)), Fraction(0)))
                  for r in range(R)]
    return np.array(picks), np.array(wts), np.array(bits, dtype=np.uint16), shared


def test_route_exact_with_ties():
    R, H, E, k = 5, 128, 48, 8
    x = O.f32_to_bf16(RNG.standard_normal((R, H)).astype(np.float32))
    g = O.f32_to_bf16((RNG.standard_normal((E, H)) * 0.02).astype(np.float32))
    g[7] = g[3]                                              # two experts with identical logits in every row
    g[20] = g[11]
    sg = O.f32_to_bf16((RNG.standard_normal(H) * 0.02).astype(np.float32))
    pick, wts, logits, sl = O.route(x, g, k, sg, shared_id=E)
    rp, rw, rb, rs = _route_fraction(x, g, k, sg)
    assert np.array_equal(logits, rb)
    assert np.array_equal(pick[:, :k], rp)
    assert np.allclose(wts[:, :k], rw, rtol=1e-12, atol=0)
    assert np.all(pick[:, k] == E)
    assert np.allclose(sl, rs, rtol=1e-15, atol=0)
    assert np.allclose(wts[:, k], 1.0 / (1.0 + np.exp(-np.array(rs))), rtol=1e-12)
    for r in range(R):                                       # ties keep the lower id first
        row = list(pick[r, :k])
        for a, b in ((3, 7), (11, 20)):
            if a in row and b in row:
                assert row.index(a) < row.index(b)


def _group_closed_form(pick, R, slots, E):
    members = {}
    for r in range(R):
        for s in range(slots):
            e = int(pick[r * slots + s])
            if 0 <= e < E:
                members.setdefault(e, []).append(r * 32 + s)
    uids = sorted(members)
    return uids, [members[u] for u in uids]


@pytest.mark.parametrize("R,slots,E", [(1, 9, 257), (4, 9, 257), (32, 9, 257), (7, 3, 5)])
def test_group_closed_form(R, slots, E):
    pick = RNG.integers(-1, E + 2, R * slots).astype(np.int32)     # includes invalid ids on both sides
    maxm = R * slots
    cnt, uids, members = O.group(pick, R, slots, E, maxm)
    ru, rm = _group_closed_form(pick, R, slots, E)
    assert cnt == len(ru) and list(uids) == ru
    for i, m in enumerate(rm):
        assert list(members[i, :len(m)]) == m
        assert np.all(members[i, len(m):] == -1)


# ---------------------------------------------------------------------------------------------------------------
# epilogues (experts.cu:117-162, 340-393): float64 recomputation within fp32 rounding
# ---------------------------------------------------------------------------------------------------------------

def test_gateup_epilogue_fp64():
    P, N, SK, E = 6, 256, 2, 4
    Z = RNG.standard_normal((2, SK, P, N)).astype(np.float32)
    pick = np.array([0, 3, -1, 2, 1, 3], dtype=np.int32)
    svh_g, svh_u = (RNG.standard_normal((E, N)).astype(np.float16) for _ in range(2))
    suh_d = np.where(RNG.integers(0, 2, (E, N)) == 1, 1.0, -1.0).astype(np.float16)
    xd = O.gateup_epilogue(Z, pick, svh_g.view(np.uint16), svh_u.view(np.uint16), suh_d.view(np.uint16), P, N, SK, E)
    for p in range(P):
        e = pick[p]
        if e < 0:
            assert np.all(xd[p] == 0)
            continue
        g = O.had64(Z[0, :, p].astype(np.float64).sum(0)) * svh_g[e]
        u = O.had64(Z[1, :, p].astype(np.float64).sum(0)) * svh_u[e]
        act = g / (1.0 + np.exp(-g)) * u
        ref = O.had64(act * suh_d[e])
        got = O.f16(xd[p]).astype(np.float64)
        assert np.allclose(got, ref, rtol=2e-3, atol=2e-3 * np.abs(ref).max())


def test_down_combine2_fp64():
    rows, D, SK, E, k = 3, 256, 2, 5, 2
    slots = k + 1
    P = rows * slots
    Z = RNG.standard_normal((SK, P, D)).astype(np.float32)
    pick = np.array([[0, 2, 4], [1, 3, 4], [2, 0, 4]], dtype=np.int32).reshape(-1)
    svh_d = RNG.standard_normal((E, D)).astype(np.float16)
    wts = RNG.random((rows, slots)).astype(np.float32)
    y0 = np.zeros((P, D), dtype=np.float32)
    out, osh, y = O.down_combine2(Z, pick, svh_d.view(np.uint16), y0, wts, rows, P, D, SK, E, slots, k)
    for r in range(rows):
        ys = [O.had64(Z[:, r * slots + s].astype(np.float64).sum(0)) * svh_d[pick[r * slots + s]] for s in range(slots)]
        ref = sum(wts[r, s] * ys[s] for s in range(k))
        assert np.allclose(out[r], ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
        assert np.allclose(osh[r], wts[r, k] * ys[k], rtol=1e-4, atol=1e-4 * np.abs(ys[k]).max())

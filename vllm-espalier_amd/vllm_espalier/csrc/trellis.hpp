// EXL3 16-bit-state trellis decode for gfx950, laid out for the 16x16x32 f16 MFMA B operand.
//
// Format (experts_grouped.cuh:83-154): a 16x16 tile of a b-bit matrix is TW = 8b uint32 words, read as one circular
// big-endian bit stream of L = 256b bits (stream bit j = bit 31 - j%32 of word j/32). State p (0..255) is the 16
// stream bits ending at (p + 1) * b, earliest bit most significant; it holds W[2t + 8(q&1) + (j&1)][g + 8(q>>1)] for
// lane = p/8, j = p%8, q = j/2, t = lane%4, g = lane/4 (dequant_kernel's placement, :330-338).
//
// MFMA mapping. v_mfma_f32_16x16x32_f16 takes, from lane l, 8 k values of B column l%16 in k group G = l/16. One
// B operand here covers two k tiles (32 k) of one n tile: lane (c = l%16, G) decodes column c of k tile G/2, the
// 8 states with t in {2(G&1), 2(G&1)+1}: two runs of 4 consecutive states,
//   run A: p = 32(c&7) + 4(c>>3) + 16(G&1) + {0,1,2,3}   (k = 4(G&1) + {0, 1, 8, 9})
//   run B: run A + 8                                       (k = 4(G&1) + {2, 3, 10, 11}).
// The B slots are put in natural k order, [4(G&1) + 0..3, 8 + 4(G&1) + 0..3] of the lane's k tile, so the A operand
// (lane l: row l%16, same k group) reads x at those k: two 8-byte loads, no permutation.
//
// Each run's 4 windows lie inside 3b + 16 <= 40 stream bits: three words are loaded, a funnel shift by the lane's
// bit offset lines the run up at bit 63 of (R0:R1), and window j is 16 bits at offset j*b of that 64-bit value.
#pragma once

#include "common.hpp"

namespace esp {

constexpr uint32_t MCG_MUL = 0xCBAC1FEDu;   // experts_grouped.cuh:67
constexpr uint32_t MCG_MASK = 0x8FFF8FFFu;  // :73
constexpr uint32_t MCG_XOR = 0x3B603B60u;
constexpr float E2M1_K = (4.0f / 3.0f) * (1.0f - 0x1p-16f);   // E2M1 snap scale, exact midpoints nudged below

// int5 / int6 grids: k reproduces rintf(v / c) (experts_grouped.cuh:40-42)
constexpr float GRID_K5 = 0x1.e62c10p+1f;
constexpr float GRID_K6 = 0x1.f660bap+2f;
// int6 grid index through one mixed fma a value: fp16(v * GRID_K6M + 1536) = 1536 + q. With this k every mcg value's
// v * k lies at least 1.5e-4 from a half-integer (so no rounding of the sum, to fp32 and then fp16 or straight to fp16,
// can move it across one) and rounds to the same q as rintf(v * GRID_K6) does; with GRID_K6 itself two values differ.
constexpr float GRID_K6M = 0x1.f6628p+2f;
constexpr float GRID_MAGIC = 1536.0f;                    // fp16 ulp 1 on [1024, 2048): the fraction is rounded off
__host__ __device__ constexpr float grid_c(int cb) { return cb == 6 ? 3.94921875f / 15.0f : 3.94921875f / 31.0f; }

// The form a GEMM decodes codebook cb in, and the factor its fp32 sums take afterwards: the int5 / int6 grids as their
// index q (22 / 23, sums * c), E2M1 on its unscaled grid {0, .5, 1, 1.5, 2, 3, 4, 6} (19, sums * 0.75); mcg as it is.
// Every product is exact either way (fp16 x fp16 in fp32); only the order of the roundings in the sums moves.
__host__ __device__ constexpr int gemm_cb(int cb) { return cb == 6 || cb == 7 ? cb + 16 : cb == 3 ? 19 : cb; }
__host__ __device__ constexpr float gemm_scale(int cb) {
    return cb == 6 || cb == 7 ? grid_c(cb) : cb == 3 ? 0.75f : 1.0f;
}

// Per-lane constants of the MFMA B-operand decode for b = K2/2 bits: word indices (mod TW) and funnel shifts of the
// two runs. The same for every tile of a matrix.
template <int K2>
struct LanePlan {
    static constexpr int B = K2 / 2, TW = 4 * K2;
    int wa, wb;      // first word of run A / B
    int sha, shb;    // funnel shifts (32 - bit offset of the run in its first word)
    __device__ __forceinline__ explicit LanePlan(int lane) {
        const int c = lane & 15, G = lane >> 4;
        const int pa = 32 * (c & 7) + 4 * (c >> 3) + 16 * (G & 1);
        const int sa = (pa + 1) * B - 16, sb = (pa + 9) * B - 16;   // first stream bit of each run's first window
        const int qa = (sa - 1) >> 5, qb = (sb - 1) >> 5;          // floor division (sa may be negative)
        sha = 32 - (sa - 32 * qa);
        shb = 32 - (sb - 32 * qb);
        wa = (qa + TW) % TW;
        wb = (qb + TW) % TW;
    }
};

// The 6 words of one tile a lane needs: w[0..2] for run A, w[3..5] for run B.
template <int K2>
__device__ __forceinline__ void load_words(const uint32_t* __restrict__ tile, const LanePlan<K2>& lp, uint32_t (&w)[6]) {
    constexpr int TW = 4 * K2;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        int ia = lp.wa + i, ib = lp.wb + i;
        ia = ia >= TW ? ia - TW : ia;
        ib = ib >= TW ? ib - TW : ib;
        w[i] = __builtin_nontemporal_load(tile + ia);
        w[3 + i] = __builtin_nontemporal_load(tile + ib);
    }
}

// window j (0..3) of a run lined up in (r0:r1)
template <int B, int J>
__device__ __forceinline__ uint32_t window(uint32_t r0, uint32_t r1) {
    constexpr int off = J * B;
    if constexpr (off <= 16)
        return __builtin_amdgcn_ubfe(r0, 16 - off, 16);
    else
        return __builtin_amdgcn_alignbit(r0, r1, 48 - off) & 0xFFFFu;
}

// the 4 states of a run starting in words (w0, w1, w2) at funnel shift sh
template <int B>
__device__ __forceinline__ void run_states(uint32_t w0, uint32_t w1, uint32_t w2, int sh, uint32_t (&s)[4]) {
    const uint32_t r0 = __builtin_amdgcn_alignbit(w0, w1, sh);
    const uint32_t r1 = __builtin_amdgcn_alignbit(w1, w2, sh);
    s[0] = window<B, 0>(r0, r1);
    s[1] = window<B, 1>(r0, r1);
    s[2] = window<B, 2>(r0, r1);
    s[3] = window<B, 3>(r0, r1);
}

__device__ __forceinline__ uint32_t mcg_hash(uint32_t s) { return (s * MCG_MUL & MCG_MASK) ^ MCG_XOR; }

// mcg values of two states as packed fp16 (lo = s0): the two halves of each hash added in one RNE fp16 add
// (experts_grouped.cuh:64-79). Two v_add_f16 reading the halves through SDWA, the second writing the high half of the
// result and keeping its low half: two instructions a pair, where gathering the halves for one packed add takes three.
__device__ __forceinline__ uint32_t mcg_pair(uint32_t s0, uint32_t s1) {
    const uint32_t x0 = mcg_hash(s0), x1 = mcg_hash(s1);
    uint32_t d;
    asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
        : "=v"(d) : "v"(x0));
    asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
        : "+v"(d) : "v"(x1));
    return d;
}

// mcg value of one state: the two halves of its hash added in one RNE fp16 add (a v_add_f16 reading the high half
// through SDWA), in the low half of the register
__device__ __forceinline__ _Float16 mcg_one(uint32_t s) {
    const f16x2 h = __builtin_bit_cast(f16x2, mcg_hash(s));
    return h[0] + h[1];
}

// f32(v) * k with one rounding, v read as fp16 by v_fma_mix_f32 (no separate conversion); the +0 addend leaves every
// product unchanged (v is never -0: the sum of two opposite halves is +0)
__device__ __forceinline__ float mul_mix(_Float16 v, float k) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(v), "v"(k));
    return r;
}

// Codebook value pair. CB: 1 mcg; 3 E2M1 snap; 6 / 7 fp16(q * c) on the int5 / int6 grid; the GEMM forms (gemm_cb):
// 19 the E2M1 snap / 0.75 and 22 / 23 the grid index q itself (fp16, exact), whose sums the caller scales.
template <int CB>
__device__ __forceinline__ uint32_t decode_pair(uint32_t s0, uint32_t s1) {
    if constexpr (CB == 1) {
        return mcg_pair(s0, s1);
    } else if constexpr (CB == 3 || CB == 19) {
        // E2M1 (experts_grouped.cuh:25-38): |v| snapped to 0.75 * {0, .5, 1, 1.5, 2, 3, 4, 6}, a tie going to the
        // smaller value, with v's sign (so -0 exists). gfx950's FP4 conversion rounds to that grid (x 4/3) to nearest
        // even, saturating, keeping the sign; scaling by k = 4/3 (1 - 2^-16) in fp32 first puts every exact midpoint
        // just below (ties then go down) and moves nothing else across one (fp16 values near a midpoint are 2^-11 or
        // more apart, relative). Back to fp16 through the same instruction pair, then * 0.75 (exact).
        const float k = E2M1_K;
        const float y0 = mul_mix(mcg_one(s0), k), y1 = mul_mix(mcg_one(s1), k);   // no packing of the two values
        // the conversion writes byte 0 of code and keeps the other three, which nothing reads: an output operand
        uint32_t code, h;
        asm("v_cvt_scalef32_pk_fp4_f32 %0, %1, %2, %3" : "=v"(code) : "v"(y0), "v"(y1), "v"(1.0f));
        asm("v_cvt_scalef32_pk_f16_fp4 %0, %1, %2" : "=v"(h) : "v"(code), "v"(1.0f));
        if constexpr (CB == 19) return h;                  // the unscaled grid: the GEMM scales its sums by 0.75
        const f16x2 q = __builtin_bit_cast(f16x2, h) * f16x2{(_Float16)0.75f, (_Float16)0.75f};
        return __builtin_bit_cast(uint32_t, q);
    } else if constexpr (CB == 23) {
        uint32_t d;                                      // the high half is written next, by v_fma_mixhi_f16
        const float k = GRID_K6M, m = GRID_MAGIC;
        asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(mcg_one(s0)), "v"(k), "v"(m));
        asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "+v"(d) : "v"(mcg_one(s1)), "v"(k), "v"(m));
        const f16x2 q = __builtin_bit_cast(f16x2, d) - f16x2{(_Float16)GRID_MAGIC, (_Float16)GRID_MAGIC};   // exact
        return __builtin_bit_cast(uint32_t, q);
    } else {
        static_assert(CB == 6 || CB == 7 || CB == 22, "codebook");
        constexpr float k = (CB == 6 || CB == 22) ? GRID_K5 : GRID_K6;
        const float q0 = __builtin_rintf(mul_mix(mcg_one(s0), k)), q1 = __builtin_rintf(mul_mix(mcg_one(s1), k));
        if constexpr (CB == 22 || CB == 23) {
            const f16x2 r = {(_Float16)q0, (_Float16)q1};           // |q| <= 31: exact
            return __builtin_bit_cast(uint32_t, r);
        } else {
            constexpr float c = grid_c(CB);
            const f16x2 r = {(_Float16)(q0 * c), (_Float16)(q1 * c)};   // one RNE rounding each
            return __builtin_bit_cast(uint32_t, r);
        }
    }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A lane's MFMA B operand for one tile from its 6 words, as 4 packed fp16 pairs: slots in natural k order,
// [A0 A1 | B0 B1 | A2 A3 | B2 B3] (k = 4(G&1) + {0,1 | 2,3 | 8,9 | 10,11}).
template <int CB, int K2>
__device__ __forceinline__ u32x4 decode_words(const uint32_t (&w)[6], const LanePlan<K2>& lp) {
    constexpr int B = K2 / 2;
    uint32_t sa[4], sb[4];
    run_states<B>(w[0], w[1], w[2], lp.sha, sa);
    run_states<B>(w[3], w[4], w[5], lp.shb, sb);
    uint32_t r[4];
    r[0] = decode_pair<CB>(sa[0], sa[1]);
    r[1] = decode_pair<CB>(sb[0], sb[1]);
    r[2] = decode_pair<CB>(sa[2], sa[3]);
    r[3] = decode_pair<CB>(sb[2], sb[3]);
    const u32x4 v = {r[0], r[1], r[2], r[3]};
    return v;
}

template <int CB, int K2>
__device__ __forceinline__ f16x8 decode_b(const uint32_t (&w)[6], const LanePlan<K2>& lp) {
    return __builtin_bit_cast(f16x8, decode_words<CB, K2>(w, lp));
}

// fp16 bits of B slot i (0..7) of a decoded operand
__device__ __forceinline__ uint16_t slot_bits(const u32x4& v, int i) {
    const uint32_t word = v[i >> 1];
    return (uint16_t)((i & 1) ? (word >> 16) : (word & 0xFFFFu));
}

// k offset (inside its 16-k tile) of B slot i for k group G
__host__ __device__ constexpr int slot_k(int G, int i) { return 4 * (G & 1) + (i & 3) + 8 * (i >> 2); }

// The (codebook, K2) pairs with kernels (experts_grouped.cuh:227-229).
#define ESP_CASES(X) \
    X(1, 2) X(1, 4) X(1, 6) X(1, 8) X(1, 10) X(1, 12) X(1, 14) X(1, 16) \
    X(3, 2) X(3, 4) X(3, 6) X(6, 4) X(6, 6) X(6, 8) X(7, 6) X(7, 8) X(7, 10)
// The GEMMs' forms of the E2M1 / int5 / int6 pairs (gemm_cb; dequantised only to test them)
#define ESP_GRID_CASES(X) X(19, 2) X(19, 4) X(19, 6) X(22, 4) X(22, 6) X(22, 8) X(23, 6) X(23, 8) X(23, 10)

__host__ __device__ constexpr bool supported(int cb, int k2) {
    return (cb == 1 && k2 >= 2 && k2 <= 16 && k2 % 2 == 0) || (cb == 3 && (k2 == 2 || k2 == 4 || k2 == 6)) ||
           (cb == 6 && (k2 == 4 || k2 == 6 || k2 == 8)) || (cb == 7 && (k2 == 6 || k2 == 8 || k2 == 10));
}

}  // namespace esp

// The K loop shared by the dense and the grouped trellis GEMMs on gfx950.
//
// A workgroup is 4 * KW waves on one 128-column block (8 n tiles); wave (p, kw) owns n tiles 2p, 2p+1 and every
// KW-th 32-k step of the workgroup's K range. The compressed tiles of the block reach LDS through
// global_load_lds_dwordx4 (16 bytes a lane, no VGPRs): the whole K range in one stage when it fits, else in stages of
// at most STAGE_BYTES, double-buffered (the next stage is issued right after the current one has landed, so it
// streams while the current one is decoded). Every load of a stage is issued before any of it is waited on, so a CU
// keeps its whole share of a small matrix in flight at once.
//
// Per 32-k step a lane reads its 6 words of each of its two tiles from LDS, decodes them into an MFMA B operand
// (trellis.hpp), and issues one v_mfma_f32_16x16x32_f16 per 16-row group.
#pragma once

#include "common.hpp"
#include "trellis.hpp"

namespace esp {

constexpr int STAGE_BYTES = 32 * 1024;

typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef __attribute__((address_space(1))) const void* global_void_ptr;

// 32-k steps a stage holds: a step is 2 k tiles x 8 n tiles x 4 * K2 words (>= 8 for K2 <= 16)
__host__ __device__ constexpr int stage_max_steps(int k2) { return STAGE_BYTES / (2 * 8 * 4 * k2 * 4); }

// LDS layout of a stage: [k tile][8 n tiles][TW words]
template <int K2>
struct StagePlan {
    static constexpr int TW = 4 * K2;
    static constexpr int ROW_WORDS = 8 * TW;                                   // one k tile of the block
    static constexpr int MAX_STEPS = stage_max_steps(K2);
};

// Cache policy of the trellis copies: non-temporal (the nt bit of gfx950's global_load_lds). A decode step streams
// ~1 GB of trellis words, each read once, through the 256 MB MALL; marked non-temporal they do not push out what the
// step reads again soon and waits on (activations, routing tables, scales, norm weights, router weights).
constexpr int CPOL_NT = 2;

// Copy k tiles [kt0, kt0 + rows) of the block (n tiles nt0..nt0+7) into lds: 16-byte units, 64 a wave instruction,
// issued by waves w0 .. w0 + nw - 1 of the workgroup (the others issue nothing).
template <int K2>
__device__ __forceinline__ void issue_stage_waves(const uint32_t* __restrict__ T, int NTILES, int kt0, int rows,
                                                  int nt0, uint32_t* lds, int w0, int nw) {
    constexpr int TW = 4 * K2, UPR = 2 * TW;                                   // 16-byte units a k tile row
    const int units = rows * UPR;
    const int wave = (int)(threadIdx.x >> 6) - w0, lane = threadIdx.x & 63;
    if (wave < 0 || wave >= nw) return;
    for (int u0 = wave * 64; u0 < units; u0 += nw * 64) {
        const int u = u0 + lane;
        if (u < units) {
            const int r = u / UPR, w = (u - r * UPR) * 4;
            const uint32_t* src = T + ((size_t)(kt0 + r) * NTILES + nt0) * TW + w;
            __builtin_amdgcn_global_load_lds((global_void_ptr)src, (lds_void_ptr)(lds + u0 * 4), 16, 0, CPOL_NT);
        }
    }
}

// issue_stage_waves by every wave of the workgroup
template <int K2>
__device__ __forceinline__ void issue_stage(const uint32_t* __restrict__ T, int NTILES, int kt0, int rows, int nt0,
                                            uint32_t* lds) {
    constexpr int TW = 4 * K2, UPR = 2 * TW;                                   // 16-byte units a k tile row
    const int units = rows * UPR;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int u0 = wave * 64; u0 < units; u0 += (int)blockDim.x) {
        const int u = u0 + lane;
        if (u < units) {
            const int r = u / UPR, w = (u - r * UPR) * 4;
            const uint32_t* src = T + ((size_t)(kt0 + r) * NTILES + nt0) * TW + w;
            __builtin_amdgcn_global_load_lds((global_void_ptr)src, (lds_void_ptr)(lds + u0 * 4), 16, 0, CPOL_NT);
        }
    }
}

// issue_stage for a K2 known only at run time (a launch whose experts differ in width): the same units in the same
// LDS places as issue_stage<K2>, issued by waves w0 .. of the workgroup (the ones below issue nothing)
__device__ __forceinline__ void issue_stage_rt(const uint32_t* __restrict__ T, int k2, int NTILES, int kt0, int rows,
                                               int nt0, uint32_t* lds, int w0 = 0) {
    const int TW = 4 * k2, UPR = 2 * TW;
    const int units = rows * UPR;
    const int wave = (int)(threadIdx.x >> 6) - w0, lane = threadIdx.x & 63;
    if (wave < 0) return;
    for (int u0 = wave * 64; u0 < units; u0 += (int)blockDim.x - 64 * w0) {
        const int u = u0 + lane;
        if (u < units) {
            const int r = u / UPR, w = (u - r * UPR) * 4;
            const uint32_t* src = T + ((size_t)(kt0 + r) * NTILES + nt0) * TW + w;
            __builtin_amdgcn_global_load_lds((global_void_ptr)src, (lds_void_ptr)(lds + u0 * 4), 16, 0, CPOL_NT);
        }
    }
}

// 32-k steps of the first stage block_gemm expects issued (prologue_issued) for a range of `steps`
__host__ __device__ constexpr int first_stage_steps(int k2, int steps) {
    return steps < stage_max_steps(k2) ? steps : stage_max_steps(k2);
}

__device__ __forceinline__ void wait_stage() {
    __builtin_amdgcn_s_waitcnt(0);        // vmcnt, expcnt, lgkmcnt all zero: this wave's copies have landed
    __syncthreads();
}

// Per-lane LDS word offsets (inside one tile) of the 6 words decode_words reads.
template <int K2>
struct LdsWords {
    int off[6];
    __device__ __forceinline__ explicit LdsWords(const LanePlan<K2>& lp) {
        constexpr int TW = 4 * K2;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int ia = lp.wa + i, ib = lp.wb + i;
            off[i] = ia >= TW ? ia - TW : ia;
            off[3 + i] = ib >= TW ? ib - TW : ib;
        }
    }
};

// The K loop. The workgroup's waves are (pair p = wave % 4, k slot kw = wave / 4): n tiles 2p, 2p+1 of the block and
// every KW-th 32-k step of the workgroup's range, starting at step kw, in increasing order. AL(g, k, av) fills the A
// operand of row group g for the step starting at absolute k. All threads of the workgroup take part in the copies.
template <int CB, int K2, int MG, typename AL>
__device__ __forceinline__ void block_gemm(const uint32_t* __restrict__ T, int NTILES, int nt0, int k0, int kr,
                                           int KW, uint32_t* stage_lds, const AL& aload, f32x4 (&acc)[2][MG],
                                           bool prologue_issued) {
    constexpr int TW = 4 * K2;
    constexpr int ROW_WORDS = StagePlan<K2>::ROW_WORDS;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;   // scalar k loop
    const int pair = wave & 3, kw = wave >> 2;
    const int G = lane >> 4;
    const int steps = kr >> 5;
    const int sst = steps < StagePlan<K2>::MAX_STEPS ? steps : StagePlan<K2>::MAX_STEPS;   // steps a stage
    const int nst = (steps + sst - 1) / sst;
    const int buf_words = 2 * sst * ROW_WORDS;
    const LanePlan<K2> lp(lane);
    const LdsWords<K2> lw(lp);
    // this lane's tiles inside a step: k tile (G >> 1), n tiles 2p + j
    const int lane_base = ((G >> 1) * 8 + 2 * pair) * TW;

#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < MG; ++g) acc[j][g] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (!prologue_issued) issue_stage<K2>(T, NTILES, k0 >> 4, 2 * sst, nt0, stage_lds);
    for (int s = 0; s < nst; ++s) {
        wait_stage();
        if (s + 1 < nst) {
            const int first = (s + 1) * sst, n = (steps - first) < sst ? (steps - first) : sst;
            issue_stage<K2>(T, NTILES, (k0 >> 4) + 2 * first, 2 * n, nt0, stage_lds + ((s + 1) & 1) * buf_words);
        }
        const uint32_t* buf = stage_lds + (s & 1) * buf_words + lane_base;
        const int first = s * sst, n = (steps - first) < sst ? (steps - first) : sst;
        const int st0 = ((kw - first) % KW + KW) % KW;      // first local step of this wave's k slot
        for (int st = st0; st < n; st += KW) {
            const uint32_t* tl = buf + st * 2 * ROW_WORDS;
            uint32_t w[2][6];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 6; ++i) w[j][i] = tl[j * TW + lw.off[i]];
            f16x8 av[MG];
#pragma unroll
            for (int g = 0; g < MG; ++g) aload(g, k0 + 32 * (first + st), av[g]);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const f16x8 b = __builtin_bit_cast(f16x8, decode_words<CB, K2>(w[j], lp));
#pragma unroll
                for (int g = 0; g < MG; ++g)
                    acc[j][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[g], b, acc[j][g], 0, 0, 0);
            }
        }
    }
}

// Decode ahead of the A rows: for a K range held whole in one landed stage, the B operands of this wave's steps (those
// block_gemm gives it: steps kw, kw + KW, ... of the range), decoded into registers before the rows exist. A consumer
// of a chained launch does this while its producer is still running, then mfma_ahead runs the MFMAs in block_gemm's
// order, so the sums are bit-identical. MAXS bounds the wave's steps (the caller checks it).
template <int MAXS>
struct AheadB {
    u32x4 b[MAXS][2];
};

template <int CB, int K2, int MAXS>
__device__ __forceinline__ void decode_ahead(const uint32_t* stage_lds, int kr, int KW, AheadB<MAXS>& pb) {
    constexpr int TW = 4 * K2;
    constexpr int ROW_WORDS = StagePlan<K2>::ROW_WORDS;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int pair = wave & 3, kw = wave >> 2;
    const int G = lane >> 4;
    const int steps = kr >> 5;
    const LanePlan<K2> lp(lane);
    const LdsWords<K2> lw(lp);
    const uint32_t* buf = stage_lds + ((G >> 1) * 8 + 2 * pair) * TW;
#pragma unroll
    for (int i = 0; i < MAXS; ++i) {
        const int st = kw + i * KW;
        if (st < steps) {
            const uint32_t* tl = buf + st * 2 * ROW_WORDS;
            uint32_t w[2][6];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 6; ++q) w[j][q] = tl[j * TW + lw.off[q]];
#pragma unroll
            for (int j = 0; j < 2; ++j) pb.b[i][j] = decode_words<CB, K2>(w[j], lp);
        }
    }
}

template <int MG, int MAXS, typename AL>
__device__ __forceinline__ void mfma_ahead(const AheadB<MAXS>& pb, int k0, int kr, int KW, const AL& aload,
                                           f32x4 (&acc)[2][MG]) {
    const int kw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) >> 2;
    const int steps = kr >> 5;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < MG; ++g) acc[j][g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < MAXS; ++i) {
        const int st = kw + i * KW;
        if (st < steps) {
            f16x8 av[MG];
#pragma unroll
            for (int g = 0; g < MG; ++g) aload(g, k0 + 32 * st, av[g]);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const f16x8 b = __builtin_bit_cast(f16x8, pb.b[i][j]);
#pragma unroll
                for (int g = 0; g < MG; ++g)
                    acc[j][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[g], b, acc[j][g], 0, 0, 0);
            }
        }
    }
}

// The [M][128] sums of the block in red (fp32, [KW][M][128]) from every wave's accumulators; the caller adds the KW
// slices in order after a barrier.
template <int MG>
__device__ __forceinline__ void store_partials(float* red, int M, const f32x4 (&acc)[2][MG]) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int pair = wave & 3, kw = wave >> 2;
    const int c = lane & 15, G = lane >> 4;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < MG; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = g * 16 + 4 * G + i;
                if (row < M) red[((size_t)kw * M + row) * 128 + 32 * pair + 16 * j + c] = acc[j][g][i];
            }
}

// LDS words a block_gemm call needs for its stages
template <int K2>
__host__ __device__ constexpr int stage_words(int kr) {
    const int steps = kr / 32;
    const int sst = steps < StagePlan<K2>::MAX_STEPS ? steps : StagePlan<K2>::MAX_STEPS;
    const int nst = (steps + sst - 1) / sst;
    return (nst > 1 ? 2 : 1) * 2 * sst * StagePlan<K2>::ROW_WORDS;
}

// host mirror of stage_words for a runtime K2
inline int host_stage_words(int k2, int kr) {
    const int row_words = 32 * k2;
    const int max_steps = stage_max_steps(k2);
    const int steps = kr / 32;
    const int sst = steps < max_steps ? steps : max_steps;
    const int nst = (steps + sst - 1) / sst;
    return (nst > 1 ? 2 : 1) * 2 * sst * row_words;
}

// A operand from fp16 rows in shared memory (LDS = true) or global memory: row group g's lane row, slots
// [4(G&1) + 0..3, 8 + 4(G&1) + 0..3] of the lane's k tile (G >> 1), as trellis.hpp's B slots. Every lane loads, with
// no branch: a lane of a missing row (past the rows or members) is given a present row's address by its caller, and
// since row i of an MFMA result depends on row i of A alone, those rows' sums are simply never stored. Shared-memory
// rows carry their address space, so their loads are ds_read and never flat: a flat load counts against vmcnt, which
// returns in order, so each step's A load would also wait for the trellis copies still in flight.
template <int MG, bool LDS>
struct RowsA;

template <int MG>
struct RowsA<MG, true> {
    typedef __attribute__((address_space(3))) const uint16_t* ptr_t;
    typedef __attribute__((address_space(3))) const uint64_t* u64_t;
    ptr_t row[MG];
    int kbase;          // absolute k of row[g][0]
    __device__ __forceinline__ void set(int g, const uint16_t* p) { row[g] = (ptr_t)p; }
    __device__ __forceinline__ void operator()(int g, int k, f16x8& av) const {
        typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
        const ptr_t p = row[g] + (k - kbase);
        const uint64_t lo = *(u64_t)(p), hi = *(u64_t)(p + 8);
        const u32x4_t t = {(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
        av = __builtin_bit_cast(f16x8, t);
    }
};

// rows in global memory (generic pointers: this form measured faster than address-space-1 loads with a flag)
template <int MG>
struct RowsA<MG, false> {
    const uint16_t* row[MG];
    int kbase;          // absolute k of row[g][0]
    __device__ __forceinline__ void set(int g, const uint16_t* p) { row[g] = p; }
    __device__ __forceinline__ void operator()(int g, int k, f16x8& av) const {
        typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
        const uint16_t* p = row[g] + (k - kbase);
        const uint2 lo = *reinterpret_cast<const uint2*>(p), hi = *reinterpret_cast<const uint2*>(p + 8);
        const u32x4_t t = {lo.x, lo.y, hi.x, hi.y};
        av = __builtin_bit_cast(f16x8, t);
    }
};

}  // namespace esp

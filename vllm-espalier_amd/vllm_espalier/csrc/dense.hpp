// The dense trellis GEMM's per-workgroup program, shared by esp_dense's kernel (dense.hip) and the multi-group launch
// (dense_multi.hip): its arguments, the finishing transform, and dense_program itself, with the host-side argument
// builder both launches use.
#pragma once

#include "common.hpp"
#include "trellis.hpp"
#include "gemm.hpp"
#include "norm.hpp"
#include "../../../include/espalier.h"

namespace esp {

constexpr int MAX_SHARDS = 4;

#ifdef ESP_PHASE_TRACE
// Timing build only (build.py --phase-trace; bench.py --phase-trace reads it): thread 0 of each workgroup records the
// 100 MHz real-time counter at the phases of dense_program into g_phase[workgroup][8]: 0 start, 1 the first stage's
// copies issued, 2 input rows ready, 3 its own wave's K loop done, 4 partials stored, 5 last to arrive (the finisher),
// 6 the finisher's stores drained; slot 7 holds the XCD (bits 0-3) and 1 << 8 for a finisher. The arithmetic is the
// product build's; only the finisher's final drain is added.
constexpr int PHASE_WGS = 8192;
static __device__ unsigned long long g_phase[PHASE_WGS * 8];
__device__ __forceinline__ int phase_wg() { return (int)(blockIdx.x + blockIdx.y * gridDim.x); }
__device__ __forceinline__ void phase_mark(int slot) {
    if (threadIdx.x == 0 && phase_wg() < PHASE_WGS) g_phase[phase_wg() * 8 + slot] = __builtin_amdgcn_s_memrealtime();
}
__device__ __forceinline__ void phase_xcd(int finisher) {
    if (threadIdx.x == 0 && phase_wg() < PHASE_WGS) {
        unsigned xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        g_phase[phase_wg() * 8 + 7] = (unsigned long long)(xcc & 0xFu) | ((unsigned long long)finisher << 8);
    }
}
#define ESP_PHASE(slot) esp::phase_mark(slot)
#define ESP_PHASE_XCD(finisher) esp::phase_xcd(finisher)
#define ESP_PHASE_DRAIN()               \
    do {                                \
        __builtin_amdgcn_s_waitcnt(0);  \
        __syncthreads();                \
    } while (0)
#else
#define ESP_PHASE(slot) ((void)0)
#define ESP_PHASE_XCD(finisher) ((void)0)
#define ESP_PHASE_DRAIN() ((void)0)
#endif

struct Shard {
    const uint32_t* T;       // trellis words [K/16][N/16][4*K2]
    const uint16_t* suh;     // [K]
    const uint16_t* svh;     // [N]
    int nb0, nb, col0;       // first 128-column block in the launch, blocks, first output column
    float scale;             // factor of the sums of the decoded form (gemm_scale: c, 0.75 or 1)
};

struct DenseArgs {
    Shard s[MAX_SHARDS];
    int n;
    const void* x;
    int x_dtype, x_stride;
    const uint16_t* xh;      // unfused input rotation: fp16 [n][M][K]
    void* y;
    int y_dtype, y_stride;
    float* Z;
    int* counters;
    int M, K, SK, NBT, fused, xs_stride, stage_bytes;
    int SQ, SR;              // K / 32 steps = SQ * SK + SR: split s has SQ + (s < SR) steps
    int cnt_stride;          // ints between two column blocks' arrival counters (32: a 128-byte line each)
    int gather;              // the last workgroup loads the M * SK partials one a 32-lane half (shared memory holds them)
    // esp_dense_own: Z holds all-ones between launches. 2: split SK - 1 (dispatched after the others) polls the other
    // splits' partials, no arrival count; 1: arrivals counted, and the finisher puts the all-ones back
    int own;
    // esp_dense_rmsnorm: the input rows are RMSNorm(h + d1 + d2) * nw (norm.hpp), made in the launch; workgroup (0, 0)
    // stores the residual h + d1 + d2 to nh_out. Rows of h, d1, d2 and nh_out are x_stride apart.
    const uint16_t* nh;
    const uint16_t* nd1;
    const uint16_t* nd2;
    const uint16_t* nw;
    uint16_t* nh_out;
    float neps;
    int norm;
    // a group of a multi launch (esp_dense_multi); all null / zero in a plain launch. Counters are 64-bit, one a
    // column block, DONE_STRIDE apart, and only grow: in the n-th launch (from 0) a producer block's finisher takes its
    // done count to n + 1, and a consumer workgroup's ticket (its block's pass count, taken when it starts) / SK is n.
    unsigned long long* done;              // producer: done counts of its column blocks, or null
    const unsigned long long* wait_done;   // consumer: the producer's done counts (x is the producer's y)
    unsigned long long* pass;              // consumer: its column blocks' ticket counts
    int wait_off;                          // consumer: x's first column in the producer's y, in 128-column blocks
    int wp_n;                              // consumer: the producer's shards, as y column blocks [wp_c0, + wp_nb)
    int wp_c0[4], wp_nb0[4], wp_nb[4];     //   holding the producer's column blocks wp_nb0 ...
    int ahead;                             // consumer: decode its B operands before the wait (dense_program)
    int case_id;             // cb * 32 + k2 of the group (the multi kernel's instance)
};

// A consumer's waves hold at most this many steps' B operands decoded ahead (8 VGPRs a step)
constexpr int AHEAD_STEPS = 4;

// y rows of one lane (4 values at i) in y's dtype: device-coherent stores when another workgroup of the same launch
// reads them (a consumer group of a multi launch)
__device__ __forceinline__ void store4_y(void* p, int dtype, size_t i, const float (&v)[4], bool coherent) {
    if (!coherent) {
        store4(p, dtype, i, v);
        return;
    }
    if (dtype == F32) {
        float* q = static_cast<float*>(p) + i;
        store_dev(reinterpret_cast<unsigned long long*>(q),
                  (unsigned long long)__float_as_uint(v[0]) | ((unsigned long long)__float_as_uint(v[1]) << 32));
        store_dev(reinterpret_cast<unsigned long long*>(q + 2),
                  (unsigned long long)__float_as_uint(v[2]) | ((unsigned long long)__float_as_uint(v[3]) << 32));
    } else {
        uint16_t h[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = dtype == BF16 ? f2bf(v[j]) : f2h(v[j]);
        const unsigned long long u = (unsigned long long)h[0] | ((unsigned long long)h[1] << 16) |
                                     ((unsigned long long)h[2] << 32) | ((unsigned long long)h[3] << 48);
        store_dev(reinterpret_cast<unsigned long long*>(static_cast<uint16_t*>(p) + i), u);
    }
}

// rot128_load with device-coherent loads of x (x written earlier in the same launch by another workgroup)
__device__ __forceinline__ RotIn rot128_load_dev(const void* x, int x_dtype, size_t xi, const uint16_t* suh,
                                                 int lane32) {
    RotIn r;
    if (x_dtype == F32) {
        const unsigned long long* q =
            reinterpret_cast<const unsigned long long*>(static_cast<const float*>(x) + xi + 4 * lane32);
        const unsigned long long a = load_dev(q), b = load_dev(q + 1);
        r.raw = make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
    } else {
        const unsigned long long a = load_dev(
            reinterpret_cast<const unsigned long long*>(static_cast<const uint16_t*>(x) + xi + 4 * lane32));
        r.raw = make_uint4((uint32_t)a, (uint32_t)(a >> 32), 0u, 0u);
    }
    r.su = *reinterpret_cast<const uint2*>(suh + 4 * lane32);
    return r;
}

// A consumer workgroup of a multi launch waits for its producer group: nothing outside a multi launch; the multi
// launch's wait is defined in dense_multi.hip, before its kernel
constexpr int DONE_STRIDE = 16;            // 64-bit counters between two column blocks' (one 128-byte line each)

template <bool MULTI>
__device__ __forceinline__ void dense_wait_producer(const DenseArgs& a, unsigned long long ticket, int c0, int chunks);
template <>
__device__ __forceinline__ void dense_wait_producer<false>(const DenseArgs&, unsigned long long, int, int) {}

// After a finisher's y stores: drain them, then count column block nbg done for the consumer group
__device__ __forceinline__ void signal_done(const DenseArgs& a, int nbg) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(a.done + (size_t)nbg * DONE_STRIDE, 1ull, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
}
// the finished outputs of one row's 128 columns from their fp32 sums, 4 a lane: H / sqrt(128), * c, * svh
// (dense.cu:120-128); sv holds the lane's 4 svh values (fp16 bits), loaded when the workgroup starts
__device__ __forceinline__ void finish(float (&v)[4], int l32, uint2 sv, float scale) {
    fwht128(v, l32);
    const float s[4] = {h2f((uint16_t)(sv.x & 0xFFFFu)), h2f((uint16_t)(sv.x >> 16)), h2f((uint16_t)(sv.y & 0xFFFFu)),
                        h2f((uint16_t)(sv.y >> 16))};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[j] *= scale;
        v[j] *= HAD_SCALE * s[j];
    }
}

// ORs bits into esp_dense_own's status word (dense.hip; only its launches call it)
__device__ void dense_raise_status(int bits);

// The work of one workgroup: column block nbg of the launch, K split `split`. smem: the dynamic shared memory;
// last, npart, ninv: small shared scratch of the calling kernel.
template <int CB, int K2, int MG, bool MULTI>
__device__ __forceinline__ void dense_program(const DenseArgs& a, const int nbg, const int split, unsigned char* smem,
                                              int& last, float* npart, float* ninv) {
    // a consumer group's ticket, taken first so its round trip overlaps the producer's work
    ESP_PHASE(0);
    ESP_PHASE_XCD(0);
    unsigned long long ticket = 0;
    if (MULTI && a.wait_done && threadIdx.x == 0)
        ticket = __hip_atomic_fetch_add(a.pass + (size_t)nbg * DONE_STRIDE, 1ull, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    // What the first copy and the input rows need -- every shard's trellis and sign pointers, first block and width,
    // the split and the launch shape -- in one round of kernel-argument loads, consumed together by one empty asm: an
    // indexed load of the workgroup's shard would wait for the shard's selection, and each later first use for its
    // own round trip.
    const Shard* sa = a.s;
    const uint32_t* T4[MAX_SHARDS];
    const uint16_t *suh4[MAX_SHARDS], *svh4[MAX_SHARDS];
    int nb04[MAX_SHARDS], nb4[MAX_SHARDS];
#pragma unroll
    for (int i = 0; i < MAX_SHARDS; ++i) {
        T4[i] = sa[i].T;
        suh4[i] = sa[i].suh;
        svh4[i] = sa[i].svh;
        nb04[i] = sa[i].nb0;
        nb4[i] = sa[i].nb;
    }
    const int an = a.n, aM = a.M, aSQ = a.SQ, aSR = a.SR, anorm = a.norm, afused = a.fused;
    const int nthreads = (int)blockDim.x;
    asm volatile("" ::"s"(T4[0]), "s"(T4[1]), "s"(T4[2]), "s"(T4[3]), "s"(nb04[0]), "s"(nb04[1]), "s"(nb04[2]),
                 "s"(nb04[3]), "s"(nb4[0]), "s"(nb4[1]), "s"(nb4[2]), "s"(nb4[3]), "s"(an), "s"(aM), "s"(aSQ),
                 "s"(aSR), "s"(anorm), "s"(afused), "s"(nthreads));
    asm volatile("" ::"s"(suh4[0]), "s"(suh4[1]), "s"(suh4[2]), "s"(suh4[3]), "s"(svh4[0]), "s"(svh4[1]),
                 "s"(svh4[2]), "s"(svh4[3]));
    int si = 0;
#pragma unroll
    for (int i = 1; i < MAX_SHARDS; ++i)
        if (i < an && nbg >= nb04[i]) si = i;
    // the shard's fields picked among the loaded ones; its output column and factor read by index (first used at the
    // end, so their round trip is hidden)
    struct {
        const uint32_t* T;
        int nb0, nb;
        const uint16_t *suh, *svh;
        int col0;
        float scale;
    } S{T4[0], nb04[0], nb4[0], suh4[0], svh4[0], 0, 0.f};
#pragma unroll
    for (int i = 1; i < MAX_SHARDS; ++i)
        if (si == i) {
            S.T = T4[i];
            S.nb0 = nb04[i];
            S.nb = nb4[i];
            S.suh = suh4[i];
            S.svh = svh4[i];
        }
    S.col0 = a.s[si].col0;
    S.scale = a.s[si].scale;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l32 = lane & 31, half = lane >> 5;
    const int c = lane & 15, G = lane >> 4;
    const int NTILES = S.nb * 8;
    const int cb_local = nbg - S.nb0;                       // column block inside the matrix
    // of the K / 32 steps = SQ * SK + SR, split s takes SQ + (s < SR) in order: SK need not divide the steps
    const int s0 = split * a.SQ + (split < a.SR ? split : a.SR);
    const int k0 = s0 * 32, kr = (a.SQ + (split < a.SR)) * 32;
    const int M = a.M;
    const int NW = (int)(blockDim.x >> 6), KW = NW >> 2;
    uint32_t* stage = reinterpret_cast<uint32_t*>(smem);

    // 0. the first stage of trellis copies, in flight while the input rows are rotated; the block's output scales.
    // With the norm in the launch and waves to spare, the copies come from the waves that do not normalise (4 a row
    // do), so the norm's loads are not queued behind them (vmcnt returns in order) and its barriers can leave them
    // in flight. The scales are loaded after the copies are issued: they need the shard's other fields, a later
    // round of argument loads.
    const bool norm_apart = a.norm && 4 * M < NW;
    // Without the norm, the waves that rotate the input rows (a (row, 128-block) a 32-lane half) issue no copies when
    // the others suffice, so their row loads are not queued behind the stage (vmcnt returns in order): the rows are
    // rotated while the stage lands, not after it
    bool rows_apart = false;
    int rot_waves = 0;
    if constexpr (MG == 1) {
        rot_waves = (M * (((k0 + kr + 127) >> 7) - (k0 >> 7)) + 1) >> 1;
        rows_apart = a.fused && !a.norm && !(MULTI && a.wait_done) && rot_waves + 4 <= NW;
    }
    {
        const int steps = kr >> 5;
        const int sst = steps < StagePlan<K2>::MAX_STEPS ? steps : StagePlan<K2>::MAX_STEPS;
        if (norm_apart)
            issue_stage_waves<K2>(S.T, NTILES, k0 >> 4, 2 * sst, cb_local * 8, stage, 4 * M, NW - 4 * M);
        else if (rows_apart)
            issue_stage_waves<K2>(S.T, NTILES, k0 >> 4, 2 * sst, cb_local * 8, stage, rot_waves, NW - rot_waves);
        else
            issue_stage<K2>(S.T, NTILES, k0 >> 4, 2 * sst, cb_local * 8, stage);
    }
    const uint2 sv = *reinterpret_cast<const uint2*>(S.svh + cb_local * 128 + 4 * l32);
    ESP_PHASE(1);

    // 1. input rows, rotated, for this K range: shared memory (fused) or the rot launch's xh
    AheadB<AHEAD_STEPS> pb;   // a consumer's B operands decoded ahead (MULTI, a.ahead)
    RowsA<MG, true> al;       // fused: the rotated rows in shared memory
    RowsA<MG, false> ag;      // else the rot launch's xh
    if (a.fused) {
        // the 128-blocks the K range touches (a split may start or end inside one)
        uint16_t* xs = reinterpret_cast<uint16_t*>(smem + a.stage_bytes);
        const int c0 = k0 >> 7, chunks = ((k0 + kr + 127) >> 7) - c0;
        if (a.norm) {
            // every workgroup normalises the rows itself: the whole row's sum of squares, with the z of its K range
            // kept in xs (the rotation then turns it into its rotated input in place, one half-wave a 128-block);
            // the norm and sign weights of a half-wave's first block are in flight with the rows
            const bool bf = a.x_dtype == BF16;
            int idx = wave * 2 + half;
            uint2 wq = make_uint2(0u, 0u), su = make_uint2(0u, 0u);
            auto weights = [&](int i) __attribute__((always_inline)) {
                const int kb = (c0 + i % chunks) * 128 + 4 * l32;
                wq = *reinterpret_cast<const uint2*>(a.nw + kb);
                su = *reinterpret_cast<const uint2*>(S.suh + kb);
            };
            if (idx < M * chunks) weights(idx);
            uint4 zq[NORM_CHUNKS];
            if (norm_apart)
                norm_rows_inv<true>(a.nh, a.nd1, a.nd2, a.x_stride, M, a.K, a.neps, bf, npart, ninv, zq, xs,
                                    a.xs_stride, c0 * 128, (c0 + chunks) * 128);
            else
                norm_rows_inv(a.nh, a.nd1, a.nd2, a.x_stride, M, a.K, a.neps, bf, npart, ninv, zq, xs, a.xs_stride,
                              c0 * 128, (c0 + chunks) * 128);
            if (nbg == 0 && split == 0) norm_rows_store(zq, M, a.K, a.x_stride, a.nh_out);
            while (idx < M * chunks) {
                const int r = idx / chunks, ch = idx % chunks;
                uint16_t* xp = xs + (size_t)r * a.xs_stride + ch * 128 + 4 * l32;
                const RotIn in = norm_rot_in(*reinterpret_cast<const uint2*>(xp), wq, su, ninv[r], bf);
                *reinterpret_cast<uint2*>(xp) = rot128_apply(in, a.x_dtype, l32);
                idx += 2 * NW;
                if (idx < M * chunks) weights(idx);
            }
        } else if (MULTI && a.wait_done) {
            // x is the output of the producer group of this launch. With `ahead` the K range is one stage: it is
            // landed and decoded into registers first, so the wait overlaps the producer with this decode. Then wait
            // for x and read it device-coherently.
            if constexpr (MULTI) {
                if (a.ahead) {
                    wait_stage();
                    decode_ahead<CB, K2, AHEAD_STEPS>(stage, kr, KW, pb);
                }
            }
            dense_wait_producer<MULTI>(a, ticket, c0, chunks);
            for (int idx = wave * 2 + half; idx < M * chunks; idx += 2 * NW) {
                const int r = idx / chunks, ch = idx % chunks;
                const int kb = (c0 + ch) * 128;
                const RotIn in = rot128_load_dev(a.x, a.x_dtype, (size_t)r * a.x_stride + kb, S.suh + kb, l32);
                *reinterpret_cast<uint2*>(xs + (size_t)r * a.xs_stride + ch * 128 + 4 * l32) =
                    rot128_apply(in, a.x_dtype, l32);
            }
        } else {
            for (int idx = wave * 2 + half; idx < M * chunks; idx += 2 * NW) {
                const int r = idx / chunks, ch = idx % chunks;
                const int kb = (c0 + ch) * 128;
                const uint2 u = rot128(a.x, a.x_dtype, (size_t)r * a.x_stride + kb, S.suh + kb, l32);
                *reinterpret_cast<uint2*>(xs + (size_t)r * a.xs_stride + ch * 128 + 4 * l32) = u;
            }
        }
#pragma unroll
        for (int g = 0; g < MG; ++g) {
            const int row = g * 16 + c;                     // a row past M reads row 0: its sums are never stored
            al.set(g, xs + (size_t)(row < M ? row : 0) * a.xs_stride + 16 * (G >> 1) + 4 * (G & 1));
        }
        al.kbase = c0 * 128;
    } else {
        const uint16_t* X = a.xh + (size_t)si * M * a.K;
#pragma unroll
        for (int g = 0; g < MG; ++g) {
            const int row = g * 16 + c;
            ag.set(g, X + (size_t)(row < M ? row : 0) * a.K + 16 * (G >> 1) + 4 * (G & 1));
        }
        ag.kbase = 0;
    }

    // 2. the K loop (its first wait is a workgroup barrier, after which the rotated rows are visible); a consumer
    // that decoded ahead only runs the MFMAs, after a barrier for the rows
    ESP_PHASE(2);
    f32x4 acc[2][MG];
    bool decoded = false;
    if constexpr (MULTI) decoded = a.ahead && a.wait_done;
    if (decoded) {
        if constexpr (MULTI) {
            __syncthreads();
            mfma_ahead<MG, AHEAD_STEPS>(pb, k0, kr, KW, al, acc);
        }
    } else if (a.fused) {
        block_gemm<CB, K2, MG>(S.T, NTILES, cb_local * 8, k0, kr, KW, stage, al, acc, true);
    } else {
        block_gemm<CB, K2, MG>(S.T, NTILES, cb_local * 8, k0, kr, KW, stage, ag, acc, true);
    }

    ESP_PHASE(3);
    // 3. the block's [M][128] sums: every wave's partials in shared memory (the stages are no longer read), the KW
    // k slots added in order
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);
    store_partials<MG>(red, M, acc);
    __syncthreads();
    auto row_sum = [&](int r) {
        float4 s4 = *reinterpret_cast<const float4*>(red + (size_t)r * 128 + 4 * l32);
        for (int q = 1; q < KW; ++q) {
            const float4 u = *reinterpret_cast<const float4*>(red + ((size_t)q * M + r) * 128 + 4 * l32);
            s4.x += u.x; s4.y += u.y; s4.z += u.z; s4.w += u.w;
        }
        return s4;
    };

    const int ycol = S.col0 + cb_local * 128 + 4 * l32;
    const bool coherent = MULTI && a.done != nullptr;
    if (a.SK == 1) {
        for (int r = wave * 2 + half; r < M; r += 2 * NW) {
            const float4 s4 = row_sum(r);
            float v[4] = {s4.x, s4.y, s4.z, s4.w};
            finish(v, l32, sv, S.scale);
            store4_y(a.y, a.y_dtype, (size_t)r * a.y_stride + ycol, v, coherent);
        }
        ESP_PHASE(4);
        ESP_PHASE(5);
        ESP_PHASE_XCD(1);
        ESP_PHASE_DRAIN();
        ESP_PHASE(6);
        if (coherent) signal_done(a, nbg);
        return;
    }
    // 4. K splits: partials to Z, the last split of the block to arrive adds them in split order and finishes
    const size_t zrow = (size_t)a.NBT * 128;
    const DevBuf zb(a.Z);
    constexpr uint32_t empty = 0xFFFFFFFFu;
    const float4 e4 = make_float4(__uint_as_float(empty), __uint_as_float(empty), __uint_as_float(empty),
                                  __uint_as_float(empty));
    if constexpr (!MULTI) {
        if (a.own == 2) {
            // the splits below SK - 1 store their partials and leave; split SK - 1 loads each of theirs, one (row,
            // split) a 32-lane half, until no word is all-ones (bounded: ~20 ms, then ESP_STATUS_WAIT_TIMEOUT), puts
            // the all-ones back, and adds each row's splits in split order, its own (from shared memory) last
            if (split != a.SK - 1) {
                for (int r = wave * 2 + half; r < M; r += 2 * NW)
                    zb.store4(a.Z + ((size_t)split * M + r) * zrow + nbg * 128 + 4 * l32, row_sum(r));
                ESP_PHASE(4);
                return;
            }
            ESP_PHASE(4);
            const int others = a.SK - 1, idx = wave * 2 + half;
            float4* zs = reinterpret_cast<float4*>(smem + (size_t)KW * M * 128 * 4);   // past the block's sums
            if (idx < M * others) {
                const int r = idx / others, q = idx - r * others;
                float* zp = a.Z + ((size_t)q * M + r) * zrow + nbg * 128 + 4 * l32;
                float4 u = zb.load4(zp);
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                while (__float_as_uint(u.x) == empty || __float_as_uint(u.y) == empty ||
                       __float_as_uint(u.z) == empty || __float_as_uint(u.w) == empty) {
                    __builtin_amdgcn_s_sleep(1);
                    if (__builtin_amdgcn_s_memrealtime() - t0 > 2000000ull) {
                        if (l32 == 0) dense_raise_status(ESP_STATUS_WAIT_TIMEOUT);
                        break;
                    }
                    u = zb.load4(zp);
                }
                zs[idx * 32 + l32] = u;
                zb.store4(zp, e4);
            }
            __syncthreads();
            ESP_PHASE(5);
            ESP_PHASE_XCD(1);
            for (int r = idx; r < M; r += 2 * NW) {
                float4 s = zs[(r * others) * 32 + l32];
                for (int q = 1; q < others; ++q) {
                    const float4 u = zs[(r * others + q) * 32 + l32];
                    s.x += u.x; s.y += u.y; s.z += u.z; s.w += u.w;
                }
                const float4 own = row_sum(r);
                s.x += own.x; s.y += own.y; s.z += own.z; s.w += own.w;
                float v[4] = {s.x, s.y, s.z, s.w};
                finish(v, l32, sv, S.scale);
                store4_y(a.y, a.y_dtype, (size_t)r * a.y_stride + ycol, v, coherent);
            }
            ESP_PHASE_DRAIN();
            ESP_PHASE(6);
            return;
        }
    }
    for (int r = wave * 2 + half; r < M; r += 2 * NW)
        zb.store4(a.Z + ((size_t)split * M + r) * zrow + nbg * 128 + 4 * l32, row_sum(r));
    int* const cnt_p = a.counters + (size_t)nbg * a.cnt_stride;
    ESP_PHASE(4);
    if (!arrive_last(cnt_p, a.SK, &last)) return;
    ESP_PHASE(5);
    ESP_PHASE_XCD(1);
    const size_t zsplit = (size_t)M * zrow;
    if (a.gather) {
        // every (row, split) partial in flight at once, one a 32-lane half, through shared memory (the k slots'
        // partials there are no longer read); then each row's splits added in split order
        float4* zs = reinterpret_cast<float4*>(smem);
        const int idx = wave * 2 + half;
        if (idx < M * a.SK) {
            const int r = idx / a.SK, q = idx - r * a.SK;
            zs[idx * 32 + l32] = zb.load4(a.Z + (size_t)q * zsplit + (size_t)r * zrow + nbg * 128 + 4 * l32);
        }
        __syncthreads();
        if (a.own && idx < M * a.SK) {                      // the partials are read: the all-ones back
            const int r = idx / a.SK, q = idx - r * a.SK;
            zb.store4(a.Z + (size_t)q * zsplit + (size_t)r * zrow + nbg * 128 + 4 * l32, e4);
        }
        for (int r = wave * 2 + half; r < M; r += 2 * NW) {
            float4 s = zs[(r * a.SK) * 32 + l32];
            for (int q = 1; q < a.SK; ++q) {
                const float4 u = zs[(r * a.SK + q) * 32 + l32];
                s.x += u.x; s.y += u.y; s.z += u.z; s.w += u.w;
            }
            float v[4] = {s.x, s.y, s.z, s.w};
            finish(v, l32, sv, S.scale);
            store4_y(a.y, a.y_dtype, (size_t)r * a.y_stride + ycol, v, coherent);
        }
        if (threadIdx.x == 0) store_dev(cnt_p, 0);
        ESP_PHASE_DRAIN();
        ESP_PHASE(6);
        if (coherent) signal_done(a, nbg);
        return;
    }
    for (int r = wave * 2 + half; r < M; r += 2 * NW) {
        const float* zp = a.Z + (size_t)r * zrow + nbg * 128 + 4 * l32;
        float4 s;
        for (int q0 = 0; q0 < a.SK; q0 += 8) {             // up to eight splits' loads in flight at once
            float4 u[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (q0 + i < a.SK) u[i] = zb.load4(zp + (q0 + i) * zsplit);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (q0 + i == 0) {
                    s = u[0];                                  // split 0 starts the sum (dense.cu:223-233)
                } else if (q0 + i < a.SK) {
                    s.x += u[i].x; s.y += u[i].y; s.z += u[i].z; s.w += u[i].w;
                }
            }
            if (a.own) {                                        // the partials are read: the all-ones back
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (q0 + i < a.SK) zb.store4(const_cast<float*>(zp) + (q0 + i) * zsplit, e4);
            }
        }
        float v[4] = {s.x, s.y, s.z, s.w};
        finish(v, l32, sv, S.scale);
        store4_y(a.y, a.y_dtype, (size_t)r * a.y_stride + ycol, v, coherent);
    }
    if (threadIdx.x == 0) store_dev(cnt_p, 0);  // every split of the block arrived
    ESP_PHASE_DRAIN();
    ESP_PHASE(6);
    if (coherent) signal_done(a, nbg);
}

}  // namespace esp

struct DenseNorm {
    const void* h;
    const void* d1;
    const void* d2;
    const void* w;
    void* h_out;
    double eps;
};

// A validated launch: its arguments, grid, waves, shared memory and row groups
struct DenseLaunch {
    esp::DenseArgs a;
    dim3 grid;
    int W;
    size_t smem;
    int mg;
};

// esp_dense's checks and arguments without the launch (dense.hip)
int prepare_dense(const void* x, int x_dtype, int64_t x_stride, int64_t M, int64_t K, int64_t n_shards,
                  const void* const* trellis, const void* const* suh, const void* const* svh, const int64_t* n_cols,
                  const int64_t* col0, void* y, int y_dtype, int64_t y_stride, int64_t y_cols, void* xh,
                  int64_t xh_numel, float* Z, int64_t z_numel, int32_t* counters, int64_t counters_numel, int64_t k2,
                  int64_t cb, int64_t SK, int64_t W, int64_t rot_smem, const DenseNorm* nrm, DenseLaunch& L);

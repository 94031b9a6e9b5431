// Routed + shared expert pipeline on gfx950: fused routing (router GEMV + top-k + grouping), grouping, input rotation,
// the grouped trellis GEMM over the distinct experts, and the epilogues (experts.cu, route.cu, experts_grouped.cuh
// define the contract).
//
// Grouping: distinct picks in id order, each with its member rows (code row * 32 + slot) in pick order, -1 padded.
// When every expert appears at most once a row (top-k picks are distinct) and R <= 32, a row bitmask per expert gives
// each member's rank as a popcount; otherwise each expert scans the picks in order.
#include "common.hpp"
#include "trellis.hpp"
#include "gemm.hpp"
#include "norm.hpp"
#include "route.hpp"
#include "../../../include/espalier.h"

namespace esp {

constexpr int GT = 256;                 // threads of the grouping / routing tail blocks
constexpr int MAX_PICKS = 32 * 33;      // R * slots limit of the routing window (route.cu:191)
constexpr int MAX_GROUP_IDS = 4096;     // ids the grouping covers (experts.cu:437)

// ------------------------------------------------------------------------------------------------------------------
// block-level grouping of sh_pick[0..n) (shared memory) over ids [0, nid)
// ------------------------------------------------------------------------------------------------------------------
template <int NID>
struct GroupSmemT {
    int cnt[NID];
    unsigned mask[NID];
    int place[NID];
    int wave_tot[16];
    int dup;
};
typedef GroupSmemT<MAX_GROUP_IDS> GroupSmem;

template <typename GS>
__device__ void group_block(const int* sh_pick, int n, int R, int slots, int nid, int maxm, int* __restrict__ uids,
                            int* __restrict__ ucount, int* __restrict__ members, GS& g) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int GT = (int)blockDim.x;                     // the workgroup's threads (up to 1024)
    for (int e = tid; e < nid; e += GT) {
        g.cnt[e] = 0;
        g.mask[e] = 0u;
    }
    if (tid == 0) g.dup = R > 32;
    __syncthreads();
    for (int i = tid; i < n; i += GT) {
        const int e = sh_pick[i];
        if (e >= 0 && e < nid) {
            atomicAdd(&g.cnt[e], 1);
            if (R <= 32) atomicOr(&g.mask[e], 1u << (i / slots));
        }
    }
    __syncthreads();
    // exclusive scan of used[e] in id order: each thread a contiguous id range
    const int per = (nid + GT - 1) / GT;
    const int e0 = tid * per;
    int used = 0;
    for (int e = e0; e < e0 + per && e < nid; ++e) {
        used += g.cnt[e] > 0;
        if (R <= 32 && g.cnt[e] != __builtin_popcount(g.mask[e])) g.dup = 1;   // an id twice in a row
    }
    int inc = used;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(inc, o, 64);
        if (lane >= o) inc += v;
    }
    if (lane == 63) g.wave_tot[wave] = inc;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; ++w) base += g.wave_tot[w];
    int place = base + inc - used;
    for (int e = e0; e < e0 + per && e < nid; ++e) {
        if (g.cnt[e] > 0) {
            g.place[e] = place;
            uids[place] = e;
            ++place;
        } else {
            g.place[e] = -1;
        }
    }
    if (tid == GT - 1) *ucount = place;
    __syncthreads();
    if (!g.dup) {
        // at most once a row: a member's rank is the number of earlier rows holding the same id
        for (int i = tid; i < n; i += GT) {
            const int e = sh_pick[i];
            if (e < 0 || e >= nid) continue;
            const int r = i / slots;
            const int rank = __builtin_popcount(g.mask[e] & ((1u << r) - 1u));
            if (rank < maxm) members[g.place[e] * maxm + rank] = r * 32 + (i % slots);
        }
        for (int e = tid; e < nid; e += GT) {
            if (g.place[e] < 0) continue;
            for (int m = g.cnt[e]; m < maxm; ++m) members[g.place[e] * maxm + m] = -1;
        }
    } else {
        for (int e = tid; e < nid; e += GT) {
            if (g.place[e] < 0) continue;
            int j = 0;
            for (int i = 0; i < n && j < maxm; ++i)
                if (sh_pick[i] == e) members[g.place[e] * maxm + j++] = (i / slots) * 32 + (i % slots);
            for (; j < maxm; ++j) members[g.place[e] * maxm + j] = -1;
        }
    }
}

// group_block's tables for n <= 64 picks, by one wave (lane i holds pick i) with no barriers: a pick's member rank is
// the number of earlier picks (pick order) with its id -- what group_block gives whether or not an id repeats inside a
// row -- and an id's place the number of smaller distinct ids. Every lane of the wave calls it. Its two passes are
// serial in n (about 12 dependent instructions a pick each), so it beats group_block's four barriers only for a few
// picks (one token's 9 on MI355X: 0.65 us less a routing launch; 36 picks take 1.6 us more).
constexpr int GROUP_WAVE_MAX = 16;
__device__ void group_wave(const int* sh_pick, int n, int slots, int nid, int maxm, int* __restrict__ uids,
                           int* __restrict__ ucount, int* __restrict__ members) {
    const int lane = threadIdx.x & 63;
    const int e = lane < n ? sh_pick[lane] : -1;
    const bool valid = e >= 0 && e < nid;
    int rank = 0, cnt = 0;
    for (int j = 0; j < n; ++j) {
        const int ej = __builtin_amdgcn_readlane(e, j);
        const bool same = valid && ej == e;
        rank += same && j < lane;
        cnt += same;
    }
    const uint64_t first = __ballot(valid && rank == 0);
    int place = 0;
    for (int j = 0; j < n; ++j) {
        const int ej = __builtin_amdgcn_readlane(e, j);
        place += ((first >> j) & 1u) && ej < e;
    }
    if (lane == 0) *ucount = __builtin_popcountll(first);
    if (!valid) return;
    if (rank == 0) {
        uids[place] = e;
        for (int m = cnt; m < maxm; ++m) members[place * maxm + m] = -1;
    }
    if (rank < maxm) members[place * maxm + rank] = (lane / slots) * 32 + (lane % slots);
}

__global__ __launch_bounds__(GT) void group_kernel(const int* __restrict__ pick, int* __restrict__ uids,
                                                   int* __restrict__ ucount, int* __restrict__ members, int R,
                                                   int slots, int E, int maxm) {
    __shared__ int sh_pick[MAX_PICKS];
    __shared__ GroupSmem g;
    const int n = R * slots;
    for (int i = threadIdx.x; i < n; i += GT) sh_pick[i] = pick[i];
    __syncthreads();
    group_block(sh_pick, n, R, slots, E, maxm, uids, ucount, members, g);
}

// ------------------------------------------------------------------------------------------------------------------
// fp64 dot products of bf16 / fp16 rows: a bf16 x bf16 product is exact in fp64 and the accumulation order is fixed
// (lane-strided chunks of 4, then a fixed butterfly), so a row's value never depends on the other rows.
// ------------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ void load4_16(const uint16_t* p, int bf16, double (&v)[4]) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    const uint16_t h[4] = {(uint16_t)(u.x & 0xFFFFu), (uint16_t)(u.x >> 16), (uint16_t)(u.y & 0xFFFFu),
                           (uint16_t)(u.y >> 16)};
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (double)(bf16 ? bf2f(h[j]) : h2f(h[j]));
}


// ------------------------------------------------------------------------------------------------------------------
// route_group (route.cu:35-181). Workgroups of 16 waves; wave w of workgroup b computes router column
// c = 4b + (w & 3) (an expert, or the shared gate) for rows r = w >> 2, + 4, ...: each lane takes 8 consecutive h a
// 512-wide chunk, exact fp64 products and sums (bf16 x bf16 products are exact in fp64; the sums are exact for
// ordinary data), a DPP reduction across the wave, one rounding to bf16. The last workgroup to arrive (relaxed
// device-scope counter) ranks each row's experts with one 32-bit key (the logit's bf16 bits made order-preserving,
// then 0xFFFF - id, so the wave maximum is the largest logit with the lowest id on ties), takes k maxima, the
// softmax over the picks and the shared gate's sigmoid, and groups the picks.
// ------------------------------------------------------------------------------------------------------------------
// Device status word of the library (one per GPU): bits the kernels set when a device-resident table names something
// they cannot run, which the host cannot check without reading the tables back. Read and cleared by esp_status.
__device__ int g_status;

__device__ __forceinline__ void raise_status(int bits) {
    __hip_atomic_fetch_or(&g_status, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// NORM: the launch normalises its input rows (esp_route_group_rmsnorm; a.norm set), an instance of its own so that the
// plain routing's code does not carry the norm's
template <int BF16, bool NORM>
__global__ __launch_bounds__(RT) void route_group_kernel(RouteArgs a) {
    extern __shared__ __align__(16) unsigned char rsmem[];     // norm: the normalised rows [R][H]
    __shared__ int last;
    __shared__ int sh_pick[MAX_PICKS];
    __shared__ GroupSmemT<RT_MAX_IDS> g;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int has = a.shared_id >= 0, C = a.E + has, slots = a.k + has;
    // window blockIdx.y of a.win rows (one window, all R rows, for esp_route_group): its rows, logits, counter line
    // and pick / weight tables
    const int r0 = (int)blockIdx.y * a.win, R = a.R - r0 < a.win ? a.R - r0 : a.win;
    float* const logits = a.logits + (size_t)r0 * C;
    int* const counter = a.counter + blockIdx.y * 32;
    int* const pick_out = a.pick_out + (size_t)r0 * slots;
    float* const wts_out = a.wts_out + (size_t)r0 * slots;
    const uint16_t* xrows = a.x + (size_t)r0 * a.x_stride;
    int xstride = a.x_stride;
    // this wave's router column c, rows rg, rg + 4, ...; h in groups of 2048 (4 chunks of 8 a lane)
    const int c = blockIdx.x * RT_COLS + (wave & 3), rg = wave >> 2;
    const bool active = c < C && rg < R;
    const uint16_t* w = c < a.E ? a.gate + (size_t)c * a.H : a.sgate;
    auto load8 = [&](const uint16_t* p, int h, uint2 (&v)[2]) __attribute__((always_inline)) {
        route_load8(p, h, a.H, v);
    };
    uint2 gv[4][2];
    auto gate_loads = [&]() __attribute__((always_inline)) {
        if (active && a.H <= 2048) {
#pragma unroll
            for (int q = 0; q < 4; ++q) load8(w, 512 * q + 8 * lane, gv[q]);
        }
    };
    if constexpr (!NORM) gate_loads();
    if constexpr (NORM) {
        // every workgroup normalises the rows itself (four waves a row); workgroup 0 also stores them. The rows'
        // loads go first, then the norm weights and the gate's chunks, which stay in flight while the rows are
        // normalised (vector loads return in order; the norm's barriers wait only for shared memory).
        __shared__ float npart[16], ninv[4];
        const int r = tid >> 8, t = tid & 255;
        uint4 wq[NORM_CHUNKS];
        auto after_rows = [&]() __attribute__((always_inline)) {
#pragma unroll
            for (int c = 0; c < NORM_CHUNKS; ++c) {
                const int i = (c * 256 + t) * 8;
                wq[c] = make_uint4(0u, 0u, 0u, 0u);
                if (r < R && i < a.H) wq[c] = *reinterpret_cast<const uint4*>(a.nw + i);
            }
            gate_loads();
        };
        uint4 zq[NORM_CHUNKS];
        if (a.H == 2048) {
            // the same loads without conditions inside the rows' waves (the only active ones: rg = r < R), so that
            // the rows' use waits for the rows alone; a column past the router's loads row 0 of the gate, unused
            auto after_rows_2048 = [&]() __attribute__((always_inline)) {
                wq[0] = *reinterpret_cast<const uint4*>(a.nw + t * 8);
#pragma unroll
                for (int k = 1; k < NORM_CHUNKS; ++k) wq[k] = make_uint4(0u, 0u, 0u, 0u);
                const uint16_t* wl = c < C ? w : a.gate;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    gv[q][0] = *reinterpret_cast<const uint2*>(wl + 512 * q + 8 * lane);
                    gv[q][1] = *reinterpret_cast<const uint2*>(wl + 512 * q + 8 * lane + 4);
                }
            };
            norm_rows_inv_2048(a.nh, a.nd1, a.x_stride, R, a.neps, BF16, npart, ninv, zq, after_rows_2048);
        } else {
            norm_rows_inv_then(a.nh, a.nd1, nullptr, a.x_stride, R, a.H, a.neps, BF16, npart, ninv, zq, after_rows);
        }
        uint16_t* xs = reinterpret_cast<uint16_t*>(rsmem);
        if (r < R) {
            const size_t o = (size_t)r * a.x_stride;
#pragma unroll
            for (int c = 0; c < NORM_CHUNKS; ++c) {
                const int i = (c * 256 + t) * 8;
                if (i < a.H) {
                    const uint4 q = norm_scale8(zq[c], wq[c], ninv[r], BF16);
                    *reinterpret_cast<uint4*>(xs + (size_t)r * a.H + i) = q;
                    if (blockIdx.x == 0) {
                        *reinterpret_cast<uint4*>(a.na_out + o + i) = q;
                        *reinterpret_cast<uint4*>(a.nh_out + o + i) = zq[c];
                    }
                }
            }
        }
        __syncthreads();
        xrows = xs;
        xstride = a.H;
    }

    // 1. logits. The gate's chunks stay in registers across the rows and the next row's x is in flight while the
    // current row is summed.
    {
        if (active) {
            auto dot = [&](const uint2 (&xv)[4][2], const uint2 (&gv)[4][2], double acc) __attribute__((always_inline)) {
                return route_dot<BF16>(xv, gv, acc);
            };
            uint2 xv[4][2], xn[4][2];
            if (a.H <= 2048) {
#pragma unroll
                for (int q = 0; q < 4; ++q) load8(xrows + (size_t)rg * xstride, 512 * q + 8 * lane, xv[q]);
                for (int r = rg; r < R; r += 4) {
                    if (r + 4 < R) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) load8(xrows + (size_t)(r + 4) * xstride, 512 * q + 8 * lane, xn[q]);
                    }
                    const double s = wave_sum_f64_dpp(dot(xv, gv, 0.0));
                    if (lane == 0) store_dev(logits + (size_t)r * C + c, c < a.E ? bf2f(f64_to_bf16(s)) : (float)s);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        xv[q][0] = xn[q][0];
                        xv[q][1] = xn[q][1];
                    }
                }
            } else {
                for (int r = rg; r < R; r += 4) {
                    double acc = 0.0;
                    for (int h0 = 0; h0 < a.H; h0 += 2048) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            load8(w, h0 + 512 * q + 8 * lane, gv[q]);
                            load8(xrows + (size_t)r * xstride, h0 + 512 * q + 8 * lane, xv[q]);
                        }
                        acc = dot(xv, gv, acc);
                    }
                    const double s = wave_sum_f64_dpp(acc);
                    if (lane == 0) store_dev(logits + (size_t)r * C + c, c < a.E ? bf2f(f64_to_bf16(s)) : (float)s);
                }
            }
        }
    }
    // one row (a decode step): wave 0 takes the top-k and groups its picks itself (route_one_row)
    const bool one_row = R == 1 && a.uids != nullptr && slots <= 64;
    if (a.sentinel && one_row) {
        // no arrival count: the last workgroup, dispatched after every other, polls the logits themselves
        if (blockIdx.x == gridDim.x - 1 && wave == 0) {
            const bool late = route_one_row<true>(a, logits, pick_out, wts_out, lane);
            if (__ballot(late) != 0 && lane == 0) raise_status(ESP_STATUS_WAIT_TIMEOUT);
        }
        return;
    }
    if (!arrive_last(counter, (int)gridDim.x, &last)) return;
    if (one_row) {
        if (wave == 0) route_one_row<false>(a, logits, pick_out, wts_out, lane);
        if (tid == 0) store_dev(counter, 0);
        return;
    }

    // 2. per row (one wave a row): k maxima of the keys, softmax weights over the picks, the shared gate's sigmoid
    const int NW = RT / 64;
    for (int r = wave; r < R; r += NW) {
        int e_mine;
        float w_mine, w_shared;
        bool late = false;
        topk_row<1>(logits + (size_t)r * C, a.E, a.k, has, lane, e_mine, w_mine, w_shared, late);
        if (a.sentinel)                                  // the row's logits read: the sentinel back
            for (int e = lane; e < C; e += 64) store_dev(logits + (size_t)r * C + e, __uint_as_float(ROUTE_EMPTY));
        if (lane < a.k) {
            pick_out[r * slots + lane] = e_mine;
            wts_out[r * slots + lane] = w_mine;
            sh_pick[r * slots + lane] = e_mine;
        }
        if (has && lane == 0) {
            pick_out[r * slots + a.k] = a.shared_id;
            wts_out[r * slots + a.k] = w_shared;
            sh_pick[r * slots + a.k] = a.shared_id;
        }
    }
    __syncthreads();

    // 3. grouping of the picks (ids < E + has): one wave for a few; none for esp_route_rows (its caller groups)
    if (a.uids == nullptr) {
        if (tid == 0) store_dev(counter, 0);
        return;
    }
    if (R * slots <= GROUP_WAVE_MAX) {
        if (wave == 0) group_wave(sh_pick, R * slots, slots, C, a.maxm, a.uids, a.ucount, a.members);
    } else {
        group_block(sh_pick, R * slots, R, slots, C, a.maxm, a.uids, a.ucount, a.members, g);
    }
    if (tid == 0) store_dev(counter, 0);
}

// ------------------------------------------------------------------------------------------------------------------
// group_shared (experts.cu:247-330): extended pick / weight tables with the shared slot, then the grouping
// ------------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(GT) void group_shared_kernel(const int* __restrict__ pick_in, const float* __restrict__ wts_in,
                                                          const uint16_t* __restrict__ x, int x_stride, int bf16,
                                                          const uint16_t* __restrict__ gate_w, int H, int shared_id,
                                                          int* __restrict__ pick_out, float* __restrict__ wts_out,
                                                          int* __restrict__ uids, int* __restrict__ ucount,
                                                          int* __restrict__ members, int R, int slots_in, int E,
                                                          int maxm) {
    __shared__ int sh_pick[MAX_PICKS];
    __shared__ GroupSmem g;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int has = shared_id >= 0, slots = slots_in + has, n = R * slots;
    for (int i = tid; i < n; i += GT) {
        const int r = i / slots, k = i % slots;
        const int e = k < slots_in ? pick_in[r * slots_in + k] : shared_id;
        sh_pick[i] = e;
        pick_out[i] = e;
        if (k < slots_in) wts_out[i] = wts_in[r * slots_in + k];
    }
    if (has) {
        for (int r = wave; r < R; r += GT / 64) {
            double acc = 0.0;
            for (int h = 4 * lane; h < H; h += 256) {
                double xv[4], wv[4];
                load4_16(x + (size_t)r * x_stride + h, bf16, xv);
                load4_16(gate_w + h, bf16, wv);
#pragma unroll
                for (int q = 0; q < 4; ++q) acc = __builtin_fma(xv[q], wv[q], acc);
            }
            const double s = wave_sum_f64_dpp(acc);
            if (lane == 0) wts_out[r * slots + slots_in] = 1.f / (1.f + expf(-(float)s));
        }
    }
    __syncthreads();
    group_block(sh_pick, n, R, slots, E, maxm, uids, ucount, members, g);
}

// ------------------------------------------------------------------------------------------------------------------
// Grouping of windows larger than one workgroup's shared memory holds (more than MAX_PICKS picks: prefill over a
// whole prompt): one workgroup per expert id. Every workgroup scans all the picks, chunk by chunk in pick order,
// setting the ids it sees in a bitmask (an expert's place is then the number of used ids below it) and ranking its own
// id's picks by ballots and a scan over its waves; the tables are group_block's, entry for entry.
// ------------------------------------------------------------------------------------------------------------------
constexpr int GW = 256;
constexpr int GW_MAX_M = 16384;           // members an expert (its list is kept in shared memory)

__global__ __launch_bounds__(GW) void group_wide_kernel(const int* __restrict__ pick, int n, int slots, int nid,
                                                        int maxm, int* __restrict__ uids, int* __restrict__ ucount,
                                                        int* __restrict__ members) {
    extern __shared__ int mem_sh[];                      // this id's member codes, in pick order
    __shared__ unsigned used[MAX_GROUP_IDS / 32];
    __shared__ int wave_cnt[GW / 64];
    __shared__ int place_sh;
    const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int words = (nid + 31) >> 5;
    for (int w = tid; w < words; w += GW) used[w] = 0u;
    __syncthreads();
    int count = 0;                                       // this id's picks so far (the same in every thread)
    for (int base = 0; base < n; base += GW) {
        const int i = base + tid;
        const int v = i < n ? pick[i] : -1;
        const bool valid = v >= 0 && v < nid;
        if (valid) atomicOr(&used[v >> 5], 1u << (v & 31));
        const bool mine = valid && v == e;
        const uint64_t bal = __ballot(mine);
        if (lane == 0) wave_cnt[wave] = __builtin_popcountll(bal);
        __syncthreads();
        int before = 0, total = 0;
#pragma unroll
        for (int w = 0; w < GW / 64; ++w) {
            const int c = wave_cnt[w];
            before += w < wave ? c : 0;
            total += c;
        }
        if (mine) {
            const int rank = count + before + __builtin_popcountll(bal & ((1ull << lane) - 1ull));
            if (rank < maxm) mem_sh[rank] = (i / slots) * 32 + (i % slots);
        }
        count += total;
        __syncthreads();                                 // wave_cnt is rewritten by the next chunk
    }
    if (e == 0 && tid == 0) {
        int u = 0;
        for (int w = 0; w < words; ++w) u += __builtin_popcount(used[w]);
        *ucount = u;
    }
    if (count == 0) return;                              // the same in every thread
    if (tid == 0) {
        int p = __builtin_popcount(used[e >> 5] & ((1u << (e & 31)) - 1u));
        for (int w = 0; w < (e >> 5); ++w) p += __builtin_popcount(used[w]);
        place_sh = p;
        uids[p] = e;
    }
    __syncthreads();
    const size_t at = (size_t)place_sh * maxm;
    for (int m = tid; m < maxm; m += GW) members[at + m] = m < count ? mem_sh[m] : -1;
}

// group_shared's pick / weight tables for any number of rows, a wave a row: the routed slots copied, the shared slot
// added with weight sigmoid(x . gate_w) computed exactly as group_shared_kernel does (the same bits)
__global__ __launch_bounds__(256) void shared_slots_kernel(const int* __restrict__ pick_in, const float* __restrict__ wts_in,
                                                           const uint16_t* __restrict__ x, int x_stride, int bf16,
                                                           const uint16_t* __restrict__ gate_w, int H, int shared_id,
                                                           int* __restrict__ pick_out, float* __restrict__ wts_out,
                                                           int R, int slots_in) {
    const int lane = threadIdx.x & 63, r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= R) return;
    const int has = shared_id >= 0, slots = slots_in + has;
    for (int k = lane; k < slots_in; k += 64) {
        pick_out[r * slots + k] = pick_in[r * slots_in + k];
        wts_out[r * slots + k] = wts_in[r * slots_in + k];
    }
    if (!has) return;
    if (lane == 0) pick_out[r * slots + slots_in] = shared_id;
    double acc = 0.0;
    for (int h = 4 * lane; h < H; h += 256) {
        double xv[4], wv[4];
        load4_16(x + (size_t)r * x_stride + h, bf16, xv);
        load4_16(gate_w + h, bf16, wv);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc = __builtin_fma(xv[q], wv[q], acc);
    }
    const double sum = wave_sum_f64_dpp(acc);
    if (lane == 0) wts_out[r * slots + slots_in] = 1.f / (1.f + expf(-(float)sum));
}

// ------------------------------------------------------------------------------------------------------------------
// rot_in (experts.cu:97-115): one workgroup a slot row p. Its pick is read once (workgroup-uniform, so the expert's
// sign rows are scalar addresses); the row's 2 * K / 128 (matrix, 128-block) chunks go 4 a 32-lane half, every chunk's
// row and sign loads in flight before the first rotation. A chunk's arithmetic is rot128's, so the bits are too.
// ------------------------------------------------------------------------------------------------------------------
constexpr int RI_CHUNKS = 4;                 // chunks a 32-lane half holds in flight

__global__ __launch_bounds__(256) void rot_in_kernel(const uint16_t* __restrict__ x, int x_dtype, int x_stride,
                                                     const int* __restrict__ pick, const uint16_t* __restrict__ suh0,
                                                     const uint16_t* __restrict__ suh1, uint16_t* __restrict__ out0,
                                                     uint16_t* __restrict__ out1, int K, int slots, int E) {
    const int p = blockIdx.x;
    const int e = pick[p];
    if (e < 0 || e >= E) return;                         // workgroup-uniform: an invalid pick's rows stay as they are
    const int l32 = threadIdx.x & 31, hw = threadIdx.x >> 5;
    const int nb = K >> 7, jobs = 2 * nb;                // chunk j: matrix j / nb, 128-block j % nb
    const size_t xrow = (size_t)(p / slots) * x_stride, orow = (size_t)p * K;
    const uint16_t* s0 = suh0 + (size_t)e * K;
    const uint16_t* s1 = suh1 + (size_t)e * K;
    for (int j0 = hw; j0 < jobs; j0 += 8 * RI_CHUNKS) {
        RotIn in[RI_CHUNKS];
#pragma unroll
        for (int c = 0; c < RI_CHUNKS; ++c) {
            const int j = j0 + 8 * c;
            if (j < jobs) {
                const int mat = j >= nb, blk = j - mat * nb;
                in[c] = rot128_load(x, x_dtype, xrow + blk * 128, (mat ? s1 : s0) + blk * 128, l32);
            }
        }
#pragma unroll
        for (int c = 0; c < RI_CHUNKS; ++c) {
            const int j = j0 + 8 * c;
            if (j < jobs) {
                const int mat = j >= nb, blk = j - mat * nb;
                *reinterpret_cast<uint2*>((mat ? out1 : out0) + orow + blk * 128 + 4 * l32) =
                    rot128_apply(in[c], x_dtype, l32);
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------------------------
// grouped (experts_grouped.cuh:237-318): program (distinct expert u, 128-column block, split * mats). 4 waves, wave w
// owns n tiles 2w, 2w+1 of the block over the split's K range; up to 32 member rows in two 16-row MFMA groups, so an
// expert's weights stream once whatever its member count. The int5 / int6 grids are decoded as their index q and the
// sums scaled by c before they are stored.
// ------------------------------------------------------------------------------------------------------------------
struct GroupedArgs {
    const uint16_t* X0;
    const uint16_t* X1;
    const int64_t* TP0;
    const int64_t* TP1;
    const int* B0;
    const int* B1;
    const int* C0;
    const int* C1;
    const int* uids;
    const int* ucount;
    const int* members;
    float* Z;
    int K, N, P, SK, maxm, slots;
    // the fused gate/up launch only (esp_moe_gateup: rot_in before, gateup_epilogue after)
    const void* x;                 // the model's rows, rotated in the launch (gate/up)
    int x_dtype, x_stride;
    const uint16_t* suh0;          // [E][K] input signs of gate / up
    const uint16_t* suh1;
    const uint16_t* svh0;          // [E][N] output scales of gate / up
    const uint16_t* svh1;
    const uint16_t* suh_d;         // [E][N] down input signs (gate/up epilogue)
    uint16_t* xd;                  // [P][N] fp16 down input
    float limit;
    int act_mode;
    int* counters;                 // arrival counters CNT_STRIDE apart: zero on entry, left zero
    int stage_bytes, xs_stride;    // rotated rows in shared memory after the stages
    int lo, hi;                    // the K2 range the launch's stages are sized for
    int mt;                        // member tiles of 32 an expert (MODE 0: ceil(maxm / 32); MODE 1: 1)
    const int* tiles;              // esp_grouped_list: the non-empty (expert slot, member tile) pairs (tile_list_kernel);
                                   // null: grid x is the expert slot and grid z holds the member tile
    int staged;                    // MODE 0: the member rows staged through shared memory (grouped_body_staged)
    int chain;                     // MODE 1 in the chained MoE launch: xd is stored device-coherently, 8 bytes a lane,
                                   // over the launch's all-ones sentinel, and read by the down programs of the launch
};

// The GEMM of one program. A rows: member m's row is abase + (by_member ? m : its slot row) * astride, holding k from
// kbase, in shared memory (LDS) or global memory. dev: the partials go to Z with device-scope stores (another
// workgroup of the launch reads them).
template <int CB, int K2, int MG, bool LDS>
__device__ __forceinline__ void grouped_body(const GroupedArgs& a, const uint32_t* __restrict__ T,
                                             const uint16_t* abase, int astride, int kbase, bool by_member,
                                             const int* rows_sh, int nrows, int mat, int split, float scale,
                                             uint32_t* stage, bool issued, bool dev, int yb) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l32 = lane & 31, half = lane >> 5;
    const int c = lane & 15, G = lane >> 4;
    const int NW = (int)(blockDim.x >> 6), KW = NW >> 2;
    const int NTILES = a.N >> 4;
    const int nt0 = yb * 8;
    const int kr = a.K / a.SK, k0 = split * kr;
    RowsA<MG, LDS> al;
#pragma unroll
    for (int g = 0; g < MG; ++g) {
        const int m = g * 16 + c;
        const int p = rows_sh[m];
        // a missing member (p < 0) reads row 0: its sums are never stored
        al.set(g, abase + (size_t)(p >= 0 ? (by_member ? m : p) : 0) * astride + 16 * (G >> 1) + 4 * (G & 1));
    }
    al.kbase = kbase;
    f32x4 acc[2][MG];
    block_gemm<CB, K2, MG>(T, NTILES, nt0, k0, kr, KW, stage, al, acc, issued);
    // the k slots' partials added in order, then one member row a 32-lane half
    __syncthreads();
    float* red = reinterpret_cast<float*>(stage);
    store_partials<MG>(red, nrows, acc);
    __syncthreads();
    float* Zm = a.Z + ((size_t)mat * a.SK + split) * a.P * a.N;
    for (int m = wave * 2 + half; m < nrows; m += 2 * NW) {
        float4 s4 = *reinterpret_cast<const float4*>(red + (size_t)m * 128 + 4 * l32);
        for (int q = 1; q < KW; ++q) {
            const float4 u = *reinterpret_cast<const float4*>(red + ((size_t)q * nrows + m) * 128 + 4 * l32);
            s4.x += u.x; s4.y += u.y; s4.z += u.z; s4.w += u.w;
        }
        s4.x *= scale; s4.y *= scale; s4.z *= scale; s4.w *= scale;
        float* zp = Zm + (size_t)rows_sh[m] * a.N + nt0 * 16 + 4 * l32;
        if (dev)
            DevBuf(a.Z).store4(zp, s4);
        else
            *reinterpret_cast<float4*>(zp) = s4;
    }
}

// The unfused launch's K loop for K ranges of several stages (a whole prompt's gate/up: 64 steps a program): the member
// rows' K slices reach shared memory by DMA in the same stages as the trellis tiles. Read from global memory at each
// step instead, a row load is queued behind the next stage's copies (vector-memory loads return in order), so with two
// waves a SIMD nothing hides it. Stage s holds AST_STEPS steps: the block's tiles, then one slice of AST_STEPS * 32
// halves a member row, AST_ROW halves apart (16 bytes of padding keep the 16 rows an MFMA reads on different banks).
// Each wave takes the same steps in the same order as block_gemm, so the sums are bit-identical to grouped_body's.
constexpr int AST_STEPS = 4;
constexpr int AST_MIN_STEPS = 9;         // K ranges of at least this many steps take the staged path
constexpr int AST_ROW = AST_STEPS * 32 + 8;
__host__ __device__ constexpr int staged_buf_bytes(int k2) { return AST_STEPS * 2 * 32 * k2 * 4 + 32 * AST_ROW * 2; }

template <int CB, int K2, int MG>
__device__ __forceinline__ void grouped_body_staged(const GroupedArgs& a, const uint32_t* __restrict__ T,
                                                    const uint16_t* abase, const int* rows_sh, int nrows, int mat,
                                                    int split, float scale, uint32_t* stage, int yb) {
    constexpr int TW = 4 * K2;
    constexpr int ROW_WORDS = StagePlan<K2>::ROW_WORDS;
    constexpr int B_WORDS = AST_STEPS * 2 * ROW_WORDS;
    constexpr int BUF_BYTES = staged_buf_bytes(K2);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int l32 = lane & 31, half = lane >> 5, c = lane & 15, G = lane >> 4;
    const int NW = (int)(blockDim.x >> 6), KW = NW >> 2, pair = wave & 3, kw = wave >> 2;
    const int NTILES = a.N >> 4, nt0 = yb * 8;
    const int kr = a.K / a.SK, k0 = split * kr, steps = kr >> 5;
    const int nst = (steps + AST_STEPS - 1) / AST_STEPS;
    unsigned char* const sbase = reinterpret_cast<unsigned char*>(stage);
    // The copies' addresses, worked out once: a stage moves every trellis unit by whole k-tile rows and every member
    // row's slice by whole steps, so a wave keeps its units' offsets inside a stage (issue_stage's units u = u0 +
    // lane, u0 = wave * 64 + i * threads, 16-byte units of k-tile row u / UPR) and its member rows' offsets
    // (rows wave, wave + NW, ...: at most 32 / 4).
    constexpr int UPR = 2 * TW, TU = 2 * AST_STEPS * UPR, TU_IT = (TU + 255) / 256;
    const int nthr = (int)blockDim.x;
    int t_off[TU_IT];
#pragma unroll
    for (int i = 0; i < TU_IT; ++i) {
        const int u = wave * 64 + i * nthr + lane, r = u / UPR;
        t_off[i] = (r * NTILES + nt0) * TW + (u - r * UPR) * 4;
    }
    int a_row[8];                                           // wave-uniform: kept in scalar registers
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int m = wave + j * NW;
        a_row[j] = __builtin_amdgcn_readfirstlane(m < nrows ? rows_sh[m] * a.K + k0 : 0);
    }
    const int lane8 = lane * 8;
    const uint32_t* Tk = T + (size_t)(k0 >> 4) * NTILES * TW;      // the split's first k-tile row
    // stage st into buffer st & 1: the tiles (every thread, as issue_stage), then a member row a wave instruction (4
    // 16-byte units a step, lanes past them idle), rows past nrows never copied (their A slots are read, their sums
    // never stored)
    auto issue = [&](int st) __attribute__((always_inline)) {
        const int first = st * AST_STEPS, n = steps - first < AST_STEPS ? steps - first : AST_STEPS;
        unsigned char* buf = sbase + (st & 1) * BUF_BYTES;
        uint32_t* tb = reinterpret_cast<uint32_t*>(buf);
        const uint32_t* Ts = Tk + (size_t)(2 * first) * NTILES * TW;
#pragma unroll
        for (int i = 0; i < TU_IT; ++i) {
            const int u0 = wave * 64 + i * nthr;
            if (u0 < 2 * n * UPR && u0 + lane < 2 * n * UPR)
                __builtin_amdgcn_global_load_lds((global_void_ptr)(Ts + t_off[i]), (lds_void_ptr)(tb + u0 * 4), 16, 0,
                                                 CPOL_NT);
        }
        uint16_t* abuf = reinterpret_cast<uint16_t*>(buf + B_WORDS * 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int m = wave + j * NW;
            if (m < nrows && lane < 4 * n)
                __builtin_amdgcn_global_load_lds((global_void_ptr)(abase + a_row[j] + first * 32 + lane8),
                                                 (lds_void_ptr)(abuf + m * AST_ROW), 16, 0, 0);
        }
    };
    f32x4 acc[2][MG];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < MG; ++g) acc[j][g] = f32x4{0.f, 0.f, 0.f, 0.f};
    const LanePlan<K2> lp(lane);
    const LdsWords<K2> lw(lp);
    const int lane_base = ((G >> 1) * 8 + 2 * pair) * TW;
    issue(0);
    for (int st = 0; st < nst; ++st) {
        wait_stage();
        if (st + 1 < nst) issue(st + 1);
        const int first = st * AST_STEPS, n = steps - first < AST_STEPS ? steps - first : AST_STEPS;
        const unsigned char* buf = sbase + (st & 1) * BUF_BYTES;
        const uint32_t* bb = reinterpret_cast<const uint32_t*>(buf) + lane_base;
        const uint16_t* ab = reinterpret_cast<const uint16_t*>(buf + B_WORDS * 4);
        RowsA<MG, true> al;
#pragma unroll
        for (int g = 0; g < MG; ++g) {
            const int m = g * 16 + c;
            al.set(g, ab + (m < nrows ? m : 0) * AST_ROW + 16 * (G >> 1) + 4 * (G & 1));
        }
        al.kbase = 0;
        const int st0 = ((kw - first) % KW + KW) % KW;          // this wave's first step of the stage
        for (int ls = st0; ls < n; ls += KW) {
            const uint32_t* tl = bb + ls * 2 * ROW_WORDS;
            uint32_t w[2][6];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 6; ++i) w[j][i] = tl[j * TW + lw.off[i]];
            f16x8 av[MG];
#pragma unroll
            for (int g = 0; g < MG; ++g) al(g, 32 * ls, av[g]);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const f16x8 b = __builtin_bit_cast(f16x8, decode_words<CB, K2>(w[j], lp));
#pragma unroll
                for (int g = 0; g < MG; ++g)
                    acc[j][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[g], b, acc[j][g], 0, 0, 0);
            }
        }
    }
    // the k slots' partials added in order, then one member row a 32-lane half (as grouped_body)
    __syncthreads();
    float* red = reinterpret_cast<float*>(stage);
    store_partials<MG>(red, nrows, acc);
    __syncthreads();
    float* Zm = a.Z + ((size_t)mat * a.SK + split) * a.P * a.N;
    for (int m = wave * 2 + half; m < nrows; m += 2 * NW) {
        float4 s4 = *reinterpret_cast<const float4*>(red + (size_t)m * 128 + 4 * l32);
        for (int q = 1; q < KW; ++q) {
            const float4 u = *reinterpret_cast<const float4*>(red + ((size_t)q * nrows + m) * 128 + 4 * l32);
            s4.x += u.x; s4.y += u.y; s4.z += u.z; s4.w += u.w;
        }
        s4.x *= scale; s4.y *= scale; s4.z *= scale; s4.w *= scale;
        *reinterpret_cast<float4*>(Zm + (size_t)rows_sh[m] * a.N + nt0 * 16 + 4 * l32) = s4;
    }
}

// ------------------------------------------------------------------------------------------------------------------
// epilogues (experts.cu:117-241, 332-393); one 32-lane half per (row, 128-block) unit
// ------------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16r(float x) { return bf2f(f2bf(x)); }

// sum over SK splits (stride apart) of the 4 floats at p, in split order, with up to 8 splits' loads in flight;
// DEV: device-scope loads (partials another workgroup of the same launch stored)
template <bool DEV = false>
__device__ __forceinline__ void sum_splits4(const float* __restrict__ p, size_t stride, int SK, float (&v)[4],
                                            const float* zbase = nullptr) {
    const DevBuf zb(zbase);                              // DEV: the partials lie within 4 GiB above zbase
    for (int q0 = 0; q0 < SK; q0 += 8) {
        float4 u[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (q0 + i < SK)
                u[i] = DEV ? zb.load4(p + (size_t)(q0 + i) * stride)
                           : *reinterpret_cast<const float4*>(p + (size_t)(q0 + i) * stride);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (q0 + i == 0) {
                v[0] = u[0].x; v[1] = u[0].y; v[2] = u[0].z; v[3] = u[0].w;
            } else if (q0 + i < SK) {
                v[0] += u[i].x; v[1] += u[i].y; v[2] += u[i].z; v[3] += u[i].w;
            }
        }
    }
}

// sum_splits4 of two partial sets (gate at pg, up at pu) with all 2 * SK loads in flight at once (SK <= 8), each summed
// in split order as sum_splits4 does
template <bool DEV>
__device__ __forceinline__ void sum_splits4x2(const float* __restrict__ pg, const float* __restrict__ pu, size_t stride,
                                              int SK, float (&g)[4], float (&u)[4], const float* zbase = nullptr) {
    const DevBuf zb(zbase);                              // DEV: the partials lie within 4 GiB above zbase
    float4 a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (i < SK) {
            a[i] = DEV ? zb.load4(pg + (size_t)i * stride) : *reinterpret_cast<const float4*>(pg + (size_t)i * stride);
            b[i] = DEV ? zb.load4(pu + (size_t)i * stride) : *reinterpret_cast<const float4*>(pu + (size_t)i * stride);
        }
    g[0] = a[0].x; g[1] = a[0].y; g[2] = a[0].z; g[3] = a[0].w;
    u[0] = b[0].x; u[1] = b[0].y; u[2] = b[0].z; u[3] = b[0].w;
#pragma unroll
    for (int i = 1; i < 8; ++i)
        if (i < SK) {
            g[0] += a[i].x; g[1] += a[i].y; g[2] += a[i].z; g[3] += a[i].w;
            u[0] += b[i].x; u[1] += b[i].y; u[2] += b[i].z; u[3] += b[i].w;
        }
}

// 4 values as fp16 (f2h, as store4) in one device-scope 8-byte store: a workgroup of the same launch reads them
__device__ __forceinline__ void store4_dev16(uint16_t* p, size_t i, const float (&v)[4]) {
    const unsigned long long u = (unsigned long long)f2h(v[0]) | ((unsigned long long)f2h(v[1]) << 16) |
                                 ((unsigned long long)f2h(v[2]) << 32) | ((unsigned long long)f2h(v[3]) << 48);
    store_dev(reinterpret_cast<unsigned long long*>(p + i), u);
}

__device__ __forceinline__ void load4_f16(const uint16_t* p, float (&v)[4]) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    v[0] = h2f((uint16_t)(u.x & 0xFFFFu)); v[1] = h2f((uint16_t)(u.x >> 16));
    v[2] = h2f((uint16_t)(u.y & 0xFFFFu)); v[3] = h2f((uint16_t)(u.y >> 16));
}

// gate/up epilogue of one (slot row, 4 columns a lane) unit from its summed splits: H, * svh / sqrt(128), SwiGLU
// (act_mode 1: fp32; 0: with the reference's bf16 roundings; clamped to limit), * suh_d, H / sqrt(128)
// (experts.cu:120-162). at = e * N + the lane's first column.
// the three fp16 scale vectors gateup_unit reads, 4 columns a lane (raw bits)
struct GateupScales {
    uint2 g, u, d;
};
__device__ __forceinline__ GateupScales gateup_scales(const uint16_t* __restrict__ svh_g, const uint16_t* __restrict__ svh_u,
                                                      const uint16_t* __restrict__ suh_d, size_t at) {
    return GateupScales{*reinterpret_cast<const uint2*>(svh_g + at), *reinterpret_cast<const uint2*>(svh_u + at),
                        *reinterpret_cast<const uint2*>(suh_d + at)};
}

__device__ __forceinline__ void unpack4_f16(uint2 u, float (&v)[4]) {
    v[0] = h2f((uint16_t)(u.x & 0xFFFFu)); v[1] = h2f((uint16_t)(u.x >> 16));
    v[2] = h2f((uint16_t)(u.y & 0xFFFFu)); v[3] = h2f((uint16_t)(u.y >> 16));
}

__device__ __forceinline__ void gateup_unit(float (&gv)[4], float (&uv)[4], const GateupScales& sc, float limit,
                                            int act_mode, int l32, float (&v)[4]) {
    fwht128(gv, l32);
    fwht128(uv, l32);
    float sg[4], su[4], sd[4];
    unpack4_f16(sc.g, sg);
    unpack4_f16(sc.u, su);
    unpack4_f16(sc.d, sd);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float act;
        if (act_mode == 0) {
            const float gg = fminf(bf16r(gv[j] * HAD_SCALE * sg[j]), limit);
            const float uu = fminf(fmaxf(bf16r(uv[j] * HAD_SCALE * su[j]), -limit), limit);
            act = bf16r(bf16r(gg / (1.f + expf(-gg))) * uu);
        } else {
            const float gg = fminf(gv[j] * HAD_SCALE * sg[j], limit);
            const float uu = fminf(fmaxf(uv[j] * HAD_SCALE * su[j], -limit), limit);
            act = gg / (1.f + expf(-gg)) * uu;
        }
        v[j] = __fmul_rn(act, sd[j]);
    }
    fwht128(v, l32);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] *= HAD_SCALE;
}

__global__ __launch_bounds__(256) void gateup_epilogue_kernel(const float* __restrict__ Z, const int* __restrict__ pick,
                                                              const uint16_t* __restrict__ svh_g,
                                                              const uint16_t* __restrict__ svh_u,
                                                              const uint16_t* __restrict__ suh_d,
                                                              uint16_t* __restrict__ xd, int P, int N, int SK, int E,
                                                              float limit, int act_mode) {
    const int l32 = threadIdx.x & 31;
    const long unit = (long)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int nb = N >> 7;
    if (unit >= (long)P * nb) return;
    const int p = (int)(unit / nb), blk = (int)(unit % nb);
    const int n = blk * 128 + 4 * l32;
    // the splits' loads go out with the pick's (they do not depend on it)
    float gv[4], uv[4];
    sum_splits4(Z + (size_t)p * N + n, (size_t)P * N, SK, gv);
    sum_splits4(Z + ((size_t)SK * P + p) * N + n, (size_t)P * N, SK, uv);
    const int e = pick[p];
    if (e < 0 || e >= E) return;
    float v[4];
    gateup_unit(gv, uv, gateup_scales(svh_g, svh_u, suh_d, (size_t)e * N + n), limit, act_mode, l32, v);
    store4(xd, F16, (size_t)p * N + n, v);
}

__global__ __launch_bounds__(256) void down_epilogue_kernel(const float* __restrict__ Z, const int* __restrict__ pick,
                                                            const uint16_t* __restrict__ svh_d, float* __restrict__ y,
                                                            int P, int D, int SK, int E) {
    const int l32 = threadIdx.x & 31;
    const long unit = (long)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int nb = D >> 7;
    if (unit >= (long)P * nb) return;
    const int p = (int)(unit / nb), blk = (int)(unit % nb);
    const int n = blk * 128 + 4 * l32;
    float v[4];
    sum_splits4(Z + (size_t)p * D + n, (size_t)P * D, SK, v);
    const int e = pick[p];
    if (e < 0 || e >= E) return;
    float sv[4];
    load4_f16(svh_d + (size_t)e * D + n, sv);
    fwht128(v, l32);
#pragma unroll
    for (int j = 0; j < 4; ++j) y[(size_t)p * D + n + j] = v[j] * HAD_SCALE * sv[j];
}

__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ y, const float* __restrict__ wts,
                                                      float* __restrict__ out, int rows, int D, int slots) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)rows * D) return;
    const int r = (int)(i / D), d = (int)(i % D);
    float acc = 0.f;
    for (int k = 0; k < slots; ++k) acc = fmaf(wts[r * slots + k], y[((size_t)r * slots + k) * D + d], acc);
    out[(size_t)r * D + d] = acc;
}

// down epilogue of every slot of one (row r, 128-block) into part, then the routed fma chain in slot order and the
// shared slot's gated output (experts.cu:340-393); n_routed == slots and out_shared == nullptr give down_combine. At
// least 256 threads; every thread calls it. y == nullptr: no slot's output is stored, and an invalid pick adds zero
// (where it would reuse y's stored row).
template <int OUT_DTYPE, bool DEV = false>
__device__ __forceinline__ void down_combine_unit(const float* __restrict__ Z, const int* __restrict__ pick,
                                                  const uint16_t* __restrict__ svh_d, float* __restrict__ y,
                                                  const float* __restrict__ wts, void* __restrict__ out,
                                                  void* __restrict__ out_shared, int P, int D, int SK, int E,
                                                  int slots, int n_routed, int r, int blk, float (*part)[128]) {
    const int l32 = threadIdx.x & 31, hw = threadIdx.x >> 5, nhw = (int)(blockDim.x >> 5);
    const int n0 = blk * 128;
    __shared__ float wts_sh[32];
    if ((int)threadIdx.x < slots) wts_sh[threadIdx.x] = wts[r * slots + threadIdx.x];   // in flight with the splits
    for (int k = hw; k < slots; k += nhw) {
        const int p = r * slots + k;
        const int n = n0 + 4 * l32;
        float v[4];
        sum_splits4<DEV>(Z + (size_t)p * D + n, (size_t)P * D, SK, v, Z);   // in flight with the pick
        const int e = pick[p];
        float o[4];
        if (e >= 0 && e < E) {
            float sv[4];
            load4_f16(svh_d + (size_t)e * D + n, sv);
            fwht128(v, l32);
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = v[j] * HAD_SCALE * sv[j];
            if (y != nullptr) *reinterpret_cast<float4*>(y + (size_t)p * D + n) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = y != nullptr ? y[(size_t)p * D + n + j] : 0.f;   // reuses y's row
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) part[k][4 * l32 + j] = o[j];
    }
    __syncthreads();
    const int col = threadIdx.x & 127;
    const size_t at = (size_t)r * D + n0 + col;
    if (threadIdx.x < 128) {
        float acc = 0.f;
        for (int q = 0; q < n_routed; ++q) acc = fmaf(wts_sh[q], part[q][col], acc);
        if constexpr (OUT_DTYPE == F32) static_cast<float*>(out)[at] = acc;
        else if constexpr (OUT_DTYPE == BF16) static_cast<uint16_t*>(out)[at] = f2bf(acc);
        else static_cast<uint16_t*>(out)[at] = f2h(acc);
    } else if (threadIdx.x < 256 && out_shared != nullptr && n_routed < slots) {
        const float v = wts_sh[n_routed] * part[n_routed][col];
        if constexpr (OUT_DTYPE == F32) static_cast<float*>(out_shared)[at] = v;
        else if constexpr (OUT_DTYPE == BF16) static_cast<uint16_t*>(out_shared)[at] = f2bf(v);
        else static_cast<uint16_t*>(out_shared)[at] = f2h(v);
    }
}

template <int OUT_DTYPE>
__global__ __launch_bounds__(1024) void down_combine_kernel(const float* __restrict__ Z, const int* __restrict__ pick,
                                                           const uint16_t* __restrict__ svh_d, float* __restrict__ y,
                                                           const float* __restrict__ wts, void* __restrict__ out,
                                                           void* __restrict__ out_shared, int P, int D, int SK, int E,
                                                           int slots, int n_routed) {
    __shared__ float part[32][128];
    down_combine_unit<OUT_DTYPE>(Z, pick, svh_d, y, wts, out, out_shared, P, D, SK, E, slots, n_routed, blockIdx.x,
                                 blockIdx.y, part);
}

// down_combine for many rows (a prompt): one workgroup (8 32-lane halves) a (row, group of DCR_BLOCKS 128-blocks), the
// row's picks and weights read once into shared memory for the group; a half-wave takes up to DCR_U (slot, block)
// units of the group with all their loads in flight, then the fma chain in slot order over the group's columns.
// Element for element the arithmetic of down_combine_unit (a workgroup a (row, 128-block)), which the few-row launches
// keep.
constexpr int DCR_BLOCKS = 4, DCR_U = 5, DCR_ROWS = 64;   // DCR_ROWS: rows from which esp_down_combine* use this form

template <int OUT_DTYPE>
__global__ __launch_bounds__(256) void down_combine_rows_kernel(const float* __restrict__ Z,
                                                                const int* __restrict__ pick,
                                                                const uint16_t* __restrict__ svh_d,
                                                                float* __restrict__ y, const float* __restrict__ wts,
                                                                void* __restrict__ out, void* __restrict__ out_shared,
                                                                int P, int D, int SK, int E, int slots, int n_routed) {
    extern __shared__ float dcr_part[];                      // [slots][DCR_BLOCKS * 128]
    __shared__ float wts_sh[32];
    __shared__ int e_sh[32];
    constexpr int GW = DCR_BLOCKS * 128;
    const int r = blockIdx.x, l32 = threadIdx.x & 31, hw = threadIdx.x >> 5;
    if ((int)threadIdx.x < slots) {
        wts_sh[threadIdx.x] = wts[r * slots + threadIdx.x];
        e_sh[threadIdx.x] = pick[r * slots + threadIdx.x];
    }
    __syncthreads();
    const int nbt = D >> 7;
    {
        const int b0 = blockIdx.y * DCR_BLOCKS;
        const int nbk = nbt - b0 < DCR_BLOCKS ? nbt - b0 : DCR_BLOCKS, units = slots * nbk;
        for (int u0 = hw; u0 < units; u0 += 8 * DCR_U) {
            float v[DCR_U][4], sv[DCR_U][4];
#pragma unroll
            for (int i = 0; i < DCR_U; ++i) {               // every unit's loads first
                const int u = u0 + 8 * i;
                if (u < units) {
                    const int k = u / nbk, n = (b0 + u - k * nbk) * 128 + 4 * l32, e = e_sh[k];
                    sum_splits4(Z + (size_t)(r * slots + k) * D + n, (size_t)P * D, SK, v[i]);
                    if (e >= 0 && e < E) load4_f16(svh_d + (size_t)e * D + n, sv[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < DCR_U; ++i) {
                const int u = u0 + 8 * i;
                if (u < units) {                            // uniform over the half-wave
                    const int k = u / nbk, bl = u - k * nbk, n = (b0 + bl) * 128 + 4 * l32, e = e_sh[k];
                    const size_t pi = (size_t)(r * slots + k) * D + n;
                    float o[4];
                    if (e >= 0 && e < E) {
                        fwht128(v[i], l32);
#pragma unroll
                        for (int j = 0; j < 4; ++j) o[j] = v[i][j] * HAD_SCALE * sv[i][j];
                        if (y != nullptr) *reinterpret_cast<float4*>(y + pi) = make_float4(o[0], o[1], o[2], o[3]);
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j) o[j] = y != nullptr ? y[pi + j] : 0.f;   // reuses y's row
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) dcr_part[k * GW + bl * 128 + 4 * l32 + j] = o[j];
                }
            }
        }
        __syncthreads();
        for (int c = threadIdx.x; c < nbk * 128; c += 256) {
            const size_t at = (size_t)r * D + b0 * 128 + c;
            float acc = 0.f;
            for (int q = 0; q < n_routed; ++q) acc = fmaf(wts_sh[q], dcr_part[q * GW + c], acc);
            if constexpr (OUT_DTYPE == F32) static_cast<float*>(out)[at] = acc;
            else if constexpr (OUT_DTYPE == BF16) static_cast<uint16_t*>(out)[at] = f2bf(acc);
            else static_cast<uint16_t*>(out)[at] = f2h(acc);
            if (out_shared != nullptr && n_routed < slots) {
                const float sv1 = wts_sh[n_routed] * dcr_part[n_routed * GW + c];
                if constexpr (OUT_DTYPE == F32) static_cast<float*>(out_shared)[at] = sv1;
                else if constexpr (OUT_DTYPE == BF16) static_cast<uint16_t*>(out_shared)[at] = f2bf(sv1);
                else static_cast<uint16_t*>(out_shared)[at] = f2h(sv1);
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------------------------
// esp_tile_list: the non-empty (expert slot u, member tile t) pairs of a grouping, in (u, t) order, for
// esp_grouped_list: tiles[0] = their number, tiles[1 + i] = u << 16 | t. A tile is non-empty iff its first member is
// (members come first in a row, -1 padded). One workgroup: each thread tests its run of consecutive pairs with every
// load in flight, then a block-wide prefix of the counts places the entries. At most cap entries are written; a
// grouping with more raises ESP_STATUS_TILE_LIST (its grouped launches would miss tiles).
// ------------------------------------------------------------------------------------------------------------------
constexpr int TL_THREADS = 1024, TL_PER = 32;           // pairs a thread at most (maxu * mt <= 32768)

__global__ __launch_bounds__(TL_THREADS) void tile_list_kernel(const int* __restrict__ ucount,
                                                              const int* __restrict__ members, int maxu, int maxm,
                                                              int mt, int* __restrict__ tiles, int cap) {
    __shared__ int wave_tot[TL_THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // the count and the first eight pairs' first members in flight together: every slot of the member table lies
    // inside it, and slots past the count are masked once it has arrived
    const int cnt_raw = ucount[0];
    const int per = (maxu * mt + TL_THREADS - 1) / TL_THREADS, q0 = tid * per;
    unsigned flags = 0u;
    int pairs = -1;
    for (int i0 = 0; i0 < per; i0 += 8) {                  // eight pairs' first members in flight at a time
        int v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = q0 + i0 + i;
            v[i] = -1;
            if (i0 + i < per && q < maxu * mt) {
                const int u = q / mt, t = q - u * mt;
                v[i] = members[(size_t)u * maxm + t * 32];
            }
        }
        if (pairs < 0) {
            const int cnt = cnt_raw < maxu ? cnt_raw : maxu;
            pairs = cnt * mt;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (v[i] >= 0 && q0 + i0 + i < pairs) flags |= 1u << (i0 + i);
    }
    const int n = __builtin_popcount(flags);
    int incl = n;                                          // inclusive prefix of n over the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    if (lane == 63) wave_tot[wave] = incl;
    __syncthreads();
    int before = incl - n, total = 0;
#pragma unroll
    for (int w = 0; w < TL_THREADS / 64; ++w) {
        const int c = wave_tot[w];
        before += w < wave ? c : 0;
        total += c;
    }
    for (int i = 0; i < per; ++i)
        if ((flags >> i) & 1u) {
            const int q = q0 + i, u = q / mt;
            if (before < cap) tiles[1 + before] = (u << 16) | (q - u * mt);
            ++before;
        }
    if (tid == 0) {
        tiles[0] = total < cap ? total : cap;
        if (total > cap) raise_status(ESP_STATUS_TILE_LIST);
    }
}

// ------------------------------------------------------------------------------------------------------------------
// The grouped kernel. MODE 0: esp_grouped, its member rows read from global memory at each step. MODE 2: esp_grouped
// with the member rows staged through shared memory (grouped_body_staged), an instance of its own so that its copy
// plan's registers do not lower the occupancy of MODE 0. MODE 1 (esp_moe_gateup): the member rows' K range rotated
// into shared memory in the launch (rot_in's arithmetic), and the last of the 2 * SK programs of an (expert,
// 128-column block) to arrive runs gateup_epilogue for its member rows.
// ------------------------------------------------------------------------------------------------------------------
// The program of workgroup (bx, by, bz) of a grid whose y extent is ny (by is the 128-column block): the kernel's
// whole body, a function of its indices so that the chained MoE launch (moe_chain_kernel) runs the same gate/up
// program under indices of its own.
template <int MODE>
__device__ __forceinline__ void grouped_program(const GroupedArgs& a, int bx, int by, int bz, int ny,
                                                unsigned char* smem) {
    uint32_t* stage = reinterpret_cast<uint32_t*>(smem);
    // program: expert slot u, member tile (32 members of the expert's list), K split, matrix; with a work list, the
    // slot and tile are the list's entry bx (workgroups past the list's length exit: workgroup-uniform)
    int u, mtile, zz;
    if (MODE != 1 && a.tiles != nullptr) {
        // a grid smaller than the list (a caller that sized the launch for fewer picks or members than esp_tile_list
        // was given) would leave listed tiles' partials stale: say so in the status word
        if (bx == 0 && threadIdx.x == 0 && a.tiles[0] > (int)gridDim.x) raise_status(ESP_STATUS_TILE_LIST);
        if (bx >= a.tiles[0]) return;
        const int ent = a.tiles[1 + bx];
        u = ent >> 16;
        mtile = ent & 0xFFFF;
        zz = bz;
    } else {
        u = bx;
        mtile = bz % a.mt;
        zz = bz / a.mt;
    }
    const int split = zz % a.SK, mat = zz / a.SK;
    const int wave = threadIdx.x >> 6, l32 = threadIdx.x & 31, half = (threadIdx.x >> 5) & 1;
    const int NW = (int)(blockDim.x >> 6);
    __shared__ int rows_sh[32];
    __shared__ int nrows;
    // the count, the expert id and the member rows depend on u alone: all three loads in flight at once
    // (u < gridDim.x <= the tables' length, or u < the count for a list entry, so the loads stay in bounds)
    const int cnt = a.ucount[0];
    const int e = a.uids[u];
    if (threadIdx.x < 64) {
        const int m = threadIdx.x, mm = mtile * 32 + m;
        const int code = m < 32 && mm < a.maxm ? a.members[(size_t)u * a.maxm + mm] : -1;
        const int rp = code >= 0 ? (code >> 5) * a.slots + (code & 31) : -1;
        if (m < 32) rows_sh[m] = rp;
        const uint64_t valid = __ballot(rp >= 0);          // members come first, -1 padded
        if (m == 0) nrows = __builtin_popcountll(valid);
    }
    if (u >= cnt) return;                                   // workgroup-uniform
    const uint32_t* T = reinterpret_cast<const uint32_t*>(mat ? a.TP1[e] : a.TP0[e]);
    const int k2 = mat ? a.B1[e] : a.B0[e];
    const int cb = mat ? a.C1[e] : a.C0[e];
    __syncthreads();
    if (nrows == 0) return;
    const int kr = a.K / a.SK, k0 = split * kr;
    // An expert whose table entry has no kernel, or whose width lies outside the [lo, hi] the stages were sized for:
    // no copy is issued (a wider expert would overrun the stage) and no GEMM runs; the program's partials become NaN,
    // so every output that reads them is NaN, and the status word records why.
    if (!supported(cb, k2) || k2 < a.lo || k2 > a.hi) {
        if (threadIdx.x == 0) raise_status(supported(cb, k2) ? ESP_STATUS_WIDTH_RANGE : ESP_STATUS_NO_KERNEL);
        float* Zm = a.Z + ((size_t)mat * a.SK + split) * a.P * a.N;
        const float qn = __builtin_nanf("");
        const float4 nan4 = make_float4(qn, qn, qn, qn);
        for (int m = wave * 2 + half; m < nrows; m += 2 * NW) {
            float* zp = Zm + (size_t)rows_sh[m] * a.N + by * 128 + 4 * l32;
            if (MODE == 1)
                DevBuf(a.Z).store4(zp, nan4);
            else
                *reinterpret_cast<float4*>(zp) = nan4;
        }
        if constexpr (MODE != 1) return;
    }
    const bool runs = supported(cb, k2) && k2 >= a.lo && k2 <= a.hi;
    const uint16_t* abase = mat ? a.X1 : a.X0;
    int astride = a.K, kbase = 0;
    GateupScales sc{};
    if (MODE == 1 && runs) {
        // the first stage's copies in flight, then the member rows' K range, rotated, into shared memory; the
        // epilogue's scales (the expert's, for this lane's 4 columns) ride along, for the workgroup that runs it.
        // The waves that rotate (a (row, 128-block) a 32-lane half) issue no copies when others are left for them:
        // vector loads return in order, so rows loaded after the copies would wait for the whole stage.
        const int chunks = kr >> 7;
        const int rot_waves = (nrows * chunks + 1) >> 1;
        issue_stage_rt(T, k2, a.N >> 4, k0 >> 4, 2 * first_stage_steps(k2, kr >> 5), by * 8, stage,
                       rot_waves < NW ? rot_waves : 0);
        sc = gateup_scales(a.svh0, a.svh1, a.suh_d, (size_t)e * a.N + by * 128 + 4 * l32);
        uint16_t* xs = reinterpret_cast<uint16_t*>(smem + a.stage_bytes);
        const uint16_t* suh = (mat ? a.suh1 : a.suh0) + (size_t)e * a.K;
        for (int idx = wave * 2 + half; idx < nrows * chunks; idx += 2 * NW) {
            const int m = idx / chunks, ch = idx - m * chunks;
            const int row = rows_sh[m] / a.slots;
            const int kb = k0 + ch * 128;
            const uint2 v = rot128(a.x, a.x_dtype, (size_t)row * a.x_stride + kb, suh + kb, l32);
            *reinterpret_cast<uint2*>(xs + (size_t)m * a.xs_stride + ch * 128 + 4 * l32) = v;
        }
        abase = xs;
        astride = a.xs_stride;
        kbase = k0;
    } else if (MODE == 1) {                                 // not run, but it may still be the last to arrive
        sc = gateup_scales(a.svh0, a.svh1, a.suh_d, (size_t)e * a.N + by * 128 + 4 * l32);
    }
    const bool two = nrows > 16;
    switch (runs ? cb * 32 + k2 : -1) {
#define ESP_GROUPED_CASE(CB_, K2_)                                                                            \
    case CB_ * 32 + K2_: {                                                                                    \
        constexpr int KCB = gemm_cb(CB_);                                                                     \
        const float scale = gemm_scale(CB_);                                                                  \
        if constexpr (MODE == 2) {                                                                            \
            if (two)                                                                                          \
                grouped_body_staged<KCB, K2_, 2>(a, T, abase, rows_sh, nrows, mat, split, scale, stage, by);      \
            else                                                                                              \
                grouped_body_staged<KCB, K2_, 1>(a, T, abase, rows_sh, nrows, mat, split, scale, stage, by);      \
        } else if (two) {                                                                                     \
            grouped_body<KCB, K2_, 2, MODE == 1>(a, T, abase, astride, kbase, MODE == 1, rows_sh, nrows, mat, split,     \
                                      scale, stage, MODE == 1, MODE == 1, by);                                    \
        } else {                                                                                              \
            grouped_body<KCB, K2_, 1, MODE == 1>(a, T, abase, astride, kbase, MODE == 1, rows_sh, nrows, mat, split,     \
                                      scale, stage, MODE == 1, MODE == 1, by);                                    \
        }                                                                                                     \
        break;                                                                                                \
    }
        ESP_CASES(ESP_GROUPED_CASE)
#undef ESP_GROUPED_CASE
        default:
            break;                                          // not run: the partials were set to NaN above
    }
    if constexpr (MODE == 1) {
        __shared__ int last;
        int* cnt_p = a.counters + ((size_t)u * ny + by) * CNT_STRIDE;
        if (!arrive_last(cnt_p, 2 * a.SK, &last)) return;
        const int n = by * 128 + 4 * l32;
        for (int m = wave * 2 + half; m < nrows; m += 2 * NW) {
            const int p = rows_sh[m];
            float gv[4], uv[4], v[4];
            if (a.SK <= 8) {
                sum_splits4x2<true>(a.Z + (size_t)p * a.N + n, a.Z + ((size_t)a.SK * a.P + p) * a.N + n,
                                    (size_t)a.P * a.N, a.SK, gv, uv, a.Z);
            } else {
                sum_splits4<true>(a.Z + (size_t)p * a.N + n, (size_t)a.P * a.N, a.SK, gv, a.Z);
                sum_splits4<true>(a.Z + ((size_t)a.SK * a.P + p) * a.N + n, (size_t)a.P * a.N, a.SK, uv, a.Z);
            }
            gateup_unit(gv, uv, sc, a.limit, a.act_mode, l32, v);
            if (a.chain)                                    // read in the same launch: device-coherent stores
                store4_dev16(a.xd, (size_t)p * a.N + n, v);
            else
                store4(a.xd, F16, (size_t)p * a.N + n, v);
        }
        if (threadIdx.x == 0) store_dev(cnt_p, 0);          // every program of the block arrived
    }
}

template <int MODE>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(5))) void grouped_kernel_t(GroupedArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    grouped_program<MODE>(a, blockIdx.x, blockIdx.y, blockIdx.z, gridDim.y, smem);
}

// ------------------------------------------------------------------------------------------------------------------
// esp_moe_chain: the decode MoE layer after its routing as ONE launch of three program groups (no counterpart in the
// reference, whose experts.py:231-261 runs them as separate launches). Workgroups of 4 waves, ids in dependency order:
//   [0, n_gu)           the fused gate/up programs (esp_moe_gateup's grouped_program<1>); the epilogue of each
//                       (expert slot, 128-column block) stores its rows of xd device-coherently, 8 bytes a lane;
//   [n_gu, + n_dn)      the down programs (expert slot u, output block yb, K split s = gate/up column block s): the
//                       split's trellis tiles land and are decoded into registers (decode_ahead); then the program
//                       reads its member rows' xd slice as soon as the epilogue has stored it, runs the MFMAs in
//                       block_gemm's order and stores its partials device-coherently;
//   [.., + R * D/128)   the combine programs (row r, block yb): down_combine_unit's arithmetic on each valid slot's
//                       partials, read as soon as the down programs have stored them.
// The hand-offs carry no flags: xd and the down partials are buffers of this launch alone that hold an all-ones
// sentinel (no fp16 quad and no fp32 value the kernels store has that bit pattern: their NaNs are the canonical quiet
// ones), and a reader loads each 8- or 16-byte piece device-coherently until no word of it is all-ones. A piece is
// read, then put back to all-ones in the same launch: xd of (u, s) by the last of its 16 down programs (a count
// reset with it), a partial by the one combine program that reads it. So both buffers hold the sentinel between
// launches. Waits are bounded (~20 ms of s_memrealtime, then ESP_STATUS_WAIT_TIMEOUT) and end: producers have lower
// ids and never wait, so an XCD dispatches every producer before any consumer. Each program's arithmetic is that of
// the separate launches, in the same order, so the results are bit-identical.
// ------------------------------------------------------------------------------------------------------------------
struct ChainArgs {
    GroupedArgs gu;                // the fused gate/up group (chain set)
    GroupedArgs dn;                // the down group: X0 = xd, Z = the down partials, K = I, N = D, SK = I / 128
    const int* pick;
    const float* wts;
    const uint16_t* svh_d;
    float* y;
    void* out;
    void* out_shared;
    int R, E, n_routed;
    int* xd_seen;                  // per (expert slot, gate/up column block): down programs that read its xd
    int nexp, n_gu, n_dn;
};

constexpr int CHAIN_ROWS = 4;      // rows the chained launch takes (its member rows: one 16-row MFMA group)
constexpr int CHAIN_AHEAD = 4;     // steps of a down program (128 k) a wave decodes ahead: 32 VGPRs
constexpr int CHAIN_MAX_SPLITS = 8;                  // down K splits (I / 128) the combine polls at once
constexpr unsigned long long CHAIN_EMPTY = ~0ull;    // the sentinel of the launch's xd and down partials

__device__ __forceinline__ bool chain_late(uint64_t t0) {
    return __builtin_amdgcn_s_memrealtime() - t0 > 2000000ull;       // ~20 ms at 100 MHz
}

// The member rows' xd slice of (expert slot u, column block s): 128 halves a row, a 32-lane half a row, each lane's
// 8 bytes loaded device-coherently until the epilogue has stored them, into shared memory (xs, rows xs_stride
// halves apart) when xs is given. The last of the n_seen readers of the slice puts the sentinel back, and its count.
__device__ __forceinline__ void chain_take_xd(uint16_t* xd, int K, int k0, const int* rows_sh, int nrows, uint16_t* xs,
                                              int xs_stride, int* seen, int n_seen) {
    const int wave = threadIdx.x >> 6, l32 = threadIdx.x & 31, half = (threadIdx.x >> 5) & 1;
    const int NW = (int)(blockDim.x >> 6);
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (int m = wave * 2 + half; m < nrows; m += 2 * NW) {
        const unsigned long long* q =
            reinterpret_cast<const unsigned long long*>(xd + (size_t)rows_sh[m] * K + k0 + 4 * l32);
        unsigned long long v = load_dev(q);
        while (v == CHAIN_EMPTY) {
            __builtin_amdgcn_s_sleep(1);
            if (chain_late(t0)) {
                raise_status(ESP_STATUS_WAIT_TIMEOUT);
                break;
            }
            v = load_dev(q);
        }
        if (xs != nullptr) *reinterpret_cast<unsigned long long*>(xs + m * xs_stride + 4 * l32) = v;
    }
    __shared__ int last_reader;
    __syncthreads();
    if (threadIdx.x == 0) {
        last_reader = __hip_atomic_fetch_add(seen, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n_seen - 1;
        if (last_reader) store_dev(seen, 0);
    }
    __syncthreads();
    if (last_reader)                                 // every reader has its copy: the slice back to the sentinel
        for (int m = wave * 2 + half; m < nrows; m += 2 * NW)
            store_dev(reinterpret_cast<unsigned long long*>(xd + (size_t)rows_sh[m] * K + k0 + 4 * l32), CHAIN_EMPTY);
}

// One down program's GEMM after its prologue: the split's stage (4 steps of 32 k: kr = 128) decoded ahead, its
// member rows' xd slice, the MFMAs, the scaled partials to Z
template <int KCB, int K2>
__device__ __forceinline__ void chain_down_body(const ChainArgs& c, const uint32_t* __restrict__ T, const int* rows_sh,
                                                int nrows, int yb, int s, float scale, int* seen,
                                                unsigned char* smem) {
    const GroupedArgs& a = c.dn;
    uint32_t* stage = reinterpret_cast<uint32_t*>(smem);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l32 = lane & 31, half = lane >> 5;
    const int cl = lane & 15, G = lane >> 4;
    const int NW = (int)(blockDim.x >> 6), KW = NW >> 2;
    const int kr = a.K / a.SK, k0 = s * kr;
    issue_stage<K2>(T, a.N >> 4, k0 >> 4, kr >> 4, yb * 8, stage);
    wait_stage();
    AheadB<CHAIN_AHEAD> pb;
    decode_ahead<KCB, K2, CHAIN_AHEAD>(stage, kr, KW, pb);
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem + a.stage_bytes);
    chain_take_xd(const_cast<uint16_t*>(a.X0), a.K, k0, rows_sh, nrows, xs, a.xs_stride, seen, a.N >> 7);
    RowsA<1, true> al;
    al.set(0, xs + (cl < nrows ? cl : 0) * a.xs_stride + 16 * (G >> 1) + 4 * (G & 1));   // absent rows read row 0
    al.kbase = k0;
    f32x4 acc[2][1];
    mfma_ahead<1, CHAIN_AHEAD>(pb, k0, kr, KW, al, acc);
    // the k slots' partials added in order, scaled, one member row a 32-lane half (grouped_body's)
    __syncthreads();
    float* red = reinterpret_cast<float*>(stage);
    store_partials<1>(red, nrows, acc);
    __syncthreads();
    float* Zm = a.Z + (size_t)s * a.P * a.N;
    const DevBuf zb(a.Z);
    for (int m = wave * 2 + half; m < nrows; m += 2 * NW) {
        float4 s4 = *reinterpret_cast<const float4*>(red + (size_t)m * 128 + 4 * l32);
        for (int q = 1; q < KW; ++q) {
            const float4 u = *reinterpret_cast<const float4*>(red + ((size_t)q * nrows + m) * 128 + 4 * l32);
            s4.x += u.x; s4.y += u.y; s4.z += u.z; s4.w += u.w;
        }
        s4.x *= scale; s4.y *= scale; s4.z *= scale; s4.w *= scale;
        zb.store4(Zm + (size_t)rows_sh[m] * a.N + yb * 128 + 4 * l32, s4);
    }
}

__device__ __forceinline__ void chain_down(const ChainArgs& c, int local, unsigned char* smem) {
    const GroupedArgs& a = c.dn;
    const int nyd = a.N >> 7, nb_gu = c.gu.N >> 7;
    const int u = local % c.nexp, yb = (local / c.nexp) % nyd, s = local / (c.nexp * nyd);
    __shared__ int rows_sh[32];
    __shared__ int nrows;
    const int cnt = a.ucount[0];
    const int e = a.uids[u];
    if (threadIdx.x < 64) {
        const int m = threadIdx.x;
        const int code = m < a.maxm ? a.members[(size_t)u * a.maxm + m] : -1;
        const int rp = code >= 0 ? (code >> 5) * a.slots + (code & 31) : -1;
        if (m < 32) rows_sh[m] = rp;
        const uint64_t valid = __ballot(rp >= 0);          // members come first, -1 padded
        if (m == 0) nrows = __builtin_popcountll(valid);
    }
    if (u >= cnt) return;                                   // no gate/up unit of this slot: nothing to read
    const uint32_t* T = reinterpret_cast<const uint32_t*>(a.TP0[e]);
    const int k2 = a.B0[e], cb = a.C0[e];
    __syncthreads();
    int* seen = c.xd_seen + ((size_t)u * nb_gu + s) * CNT_STRIDE;
    const bool runs = supported(cb, k2) && k2 >= a.lo && k2 <= a.hi;
    switch (runs ? cb * 32 + k2 : -1) {
#define ESP_CHAIN_CASE(CB_, K2_)                                                                              \
    case CB_ * 32 + K2_:                                                                                      \
        chain_down_body<gemm_cb(CB_), K2_>(c, T, rows_sh, nrows, yb, s, gemm_scale(CB_), seen, smem);         \
        break;
        ESP_CASES(ESP_CHAIN_CASE)
#undef ESP_CHAIN_CASE
        default: {                          // no kernel for the expert's table entry: NaN partials, as grouped's
            chain_take_xd(const_cast<uint16_t*>(a.X0), a.K, s * 128, rows_sh, nrows, nullptr, 0, seen, nyd);
            if (threadIdx.x == 0) raise_status(supported(cb, k2) ? ESP_STATUS_WIDTH_RANGE : ESP_STATUS_NO_KERNEL);
            const int wave = threadIdx.x >> 6, l32 = threadIdx.x & 31, half = (threadIdx.x >> 5) & 1;
            const float qn = __builtin_nanf("");
            for (int m = wave * 2 + half; m < nrows; m += 2 * (int)(blockDim.x >> 6))
                DevBuf(a.Z).store4(a.Z + (size_t)s * a.P * a.N + (size_t)rows_sh[m] * a.N + yb * 128 + 4 * l32,
                                   make_float4(qn, qn, qn, qn));
            break;
        }
    }
}

// down_combine_unit's arithmetic for (row r, block yb) with every valid slot's SK partials loaded device-coherently
// until the down programs have stored them (no word all-ones), then put back to the sentinel
template <int OUT_DTYPE>
__device__ __forceinline__ void chain_combine(const ChainArgs& c, int local, unsigned char* smem) {
    const GroupedArgs& a = c.dn;
    const int D = a.N, P = a.P, SK = a.SK, slots = a.slots;
    const int nyd = D >> 7;
    const int r = local / nyd, blk = local % nyd;
    float (*part)[128] = reinterpret_cast<float (*)[128]>(smem);
    const int l32 = threadIdx.x & 31, hw = threadIdx.x >> 5, nhw = (int)(blockDim.x >> 5);
    const int n0 = blk * 128;
    __shared__ float wts_sh[32];
    if ((int)threadIdx.x < slots) wts_sh[threadIdx.x] = c.wts[r * slots + threadIdx.x];
    const DevBuf zb(a.Z);
    const uint32_t empty = 0xFFFFFFFFu;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (int k = hw; k < slots; k += nhw) {
        const int p = r * slots + k;
        const int n = n0 + 4 * l32;
        const int e = c.pick[p];
        float o[4];
        if (e >= 0 && e < c.E) {
            float* zp = a.Z + (size_t)p * D + n;
            float4 u[CHAIN_MAX_SPLITS];
#pragma unroll
            for (int q = 0; q < CHAIN_MAX_SPLITS; ++q)
                if (q < SK) u[q] = zb.load4(zp + (size_t)q * P * D);
            float v[4];
#pragma unroll
            for (int q = 0; q < CHAIN_MAX_SPLITS; ++q)
                if (q < SK) {
                    auto pending = [&](const float4& t) {
                        return __float_as_uint(t.x) == empty || __float_as_uint(t.y) == empty ||
                               __float_as_uint(t.z) == empty || __float_as_uint(t.w) == empty;
                    };
                    while (pending(u[q])) {
                        __builtin_amdgcn_s_sleep(1);
                        if (chain_late(t0)) {
                            raise_status(ESP_STATUS_WAIT_TIMEOUT);
                            break;
                        }
                        u[q] = zb.load4(zp + (size_t)q * P * D);
                    }
                    if (q == 0) {                            // split 0 starts the sum, the others follow in order
                        v[0] = u[0].x; v[1] = u[0].y; v[2] = u[0].z; v[3] = u[0].w;
                    } else {
                        v[0] += u[q].x; v[1] += u[q].y; v[2] += u[q].z; v[3] += u[q].w;
                    }
                }
            const float4 e4 = make_float4(__uint_as_float(empty), __uint_as_float(empty), __uint_as_float(empty),
                                          __uint_as_float(empty));
#pragma unroll
            for (int q = 0; q < CHAIN_MAX_SPLITS; ++q)
                if (q < SK) zb.store4(zp + (size_t)q * P * D, e4);
            float sv[4];
            load4_f16(c.svh_d + (size_t)e * D + n, sv);
            fwht128(v, l32);
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = v[j] * HAD_SCALE * sv[j];
            if (c.y != nullptr) *reinterpret_cast<float4*>(c.y + (size_t)p * D + n) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = c.y != nullptr ? c.y[(size_t)p * D + n + j] : 0.f;   // reuses y's row
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) part[k][4 * l32 + j] = o[j];
    }
    __syncthreads();
    const int col = threadIdx.x & 127;
    const size_t at = (size_t)r * D + n0 + col;
    if (threadIdx.x < 128) {
        float acc = 0.f;
        for (int q = 0; q < c.n_routed; ++q) acc = fmaf(wts_sh[q], part[q][col], acc);
        if constexpr (OUT_DTYPE == F32) static_cast<float*>(c.out)[at] = acc;
        else if constexpr (OUT_DTYPE == BF16) static_cast<uint16_t*>(c.out)[at] = f2bf(acc);
        else static_cast<uint16_t*>(c.out)[at] = f2h(acc);
    } else if (threadIdx.x < 256 && c.out_shared != nullptr && c.n_routed < slots) {
        const float v = wts_sh[c.n_routed] * part[c.n_routed][col];
        if constexpr (OUT_DTYPE == F32) static_cast<float*>(c.out_shared)[at] = v;
        else if constexpr (OUT_DTYPE == BF16) static_cast<uint16_t*>(c.out_shared)[at] = f2bf(v);
        else static_cast<uint16_t*>(c.out_shared)[at] = f2h(v);
    }
}

template <int OUT_DTYPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5))) void moe_chain_kernel(ChainArgs c) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int id = blockIdx.x;
    if (id < c.n_gu) {
        const int ny = c.gu.N >> 7;
        const int rest = id / c.nexp;
        grouped_program<1>(c.gu, id % c.nexp, rest % ny, rest / ny, ny, smem);
    } else if (id < c.n_gu + c.n_dn) {
        chain_down(c, id - c.n_gu, smem);
    } else {
        chain_combine<OUT_DTYPE>(c, id - c.n_gu - c.n_dn, smem);
    }
}



// ------------------------------------------------------------------------------------------------------------------
// esp_route_rows: a whole prompt's routing in two launches. The router logits on the fp64 matrix cores: a workgroup is
// RL_WAVES waves on one tile of 16 rows x 16 expert columns, wave w summing the products of K range w with
// v_mfma_f64_16x16x4f64 (the shared gate's column is the top-k launch's: as a 17th column tile of E = 256 it would take
// 32 more workgroups than the 512 two a CU hold at 512 rows, a second round for one column). Lane (i, q) of a wave feeds row i's and column i's elements at the same k;
// a step of 32 k gives lane group q the 8 from 8 q (one 16-byte load a lane, 64 contiguous bytes a row), so each MFMA
// adds 4 products and the steps cover every k once.
// bf16 x bf16 products are exact in fp64 and so are their sums for ordinary data, so after the one rounding (bf16 for
// the experts, fp32 for the shared gate) the logits equal route_group's, whose sums run in another order. The waves'
// partials are added in wave order. Then route_topk_kernel: one wave a row, the shared gate's fp64 dot (as
// shared_slots_kernel's: the same exact sum) and topk_row.
// ------------------------------------------------------------------------------------------------------------------
constexpr int RL_WAVES = 8;
constexpr int RL_BATCH = 4;
typedef double f64x4 __attribute__((ext_vector_type(4)));

// 8 consecutive k of one row (xv) and one router column (gv): 8 MFMAs, in k order
template <int BF16>
__device__ __forceinline__ f64x4 route_mfma8(uint4 xv, uint4 gv, f64x4 acc) {
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const uint32_t xh = (t & 1) ? xw[t >> 1] >> 16 : xw[t >> 1] & 0xFFFFu;
        const uint32_t gh = (t & 1) ? gw[t >> 1] >> 16 : gw[t >> 1] & 0xFFFFu;
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64(bits16_to_f64(xh, BF16), bits16_to_f64(gh, BF16), acc, 0, 0, 0);
    }
    return acc;
}

template <int BF16>
__global__ __launch_bounds__(RL_WAVES * 64) void route_logits_kernel(const uint16_t* __restrict__ x, int x_stride,
                                                                     const uint16_t* __restrict__ gate, int R, int H,
                                                                     int E, int C, float* __restrict__ logits) {
    __shared__ double part[RL_WAVES - 1][4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane & 15, q = lane >> 4;
    const int r0 = blockIdx.y * 16, c0 = blockIdx.x * 16;
    const int r = r0 + i < R ? r0 + i : R - 1;                 // rows and columns past the ends: their sums unused
    const int c = c0 + i < E ? c0 + i : E - 1;
    const uint16_t* xr = x + (size_t)r * x_stride;
    const uint16_t* gr = gate + (size_t)c * H;
    const int kw = H / RL_WAVES;                                // elements of a wave, a multiple of 64
    const int kb = wave * kw + 8 * q;                           // a row's 4 lane groups read 64 contiguous bytes
    f64x4 acc = {0.0, 0.0, 0.0, 0.0};
    int k = 0;
    for (; k + 32 * RL_BATCH <= kw; k += 32 * RL_BATCH) {       // RL_BATCH loads in flight before the first MFMA
        uint4 xv[RL_BATCH], gv[RL_BATCH];
#pragma unroll
        for (int j = 0; j < RL_BATCH; ++j) {
            xv[j] = *reinterpret_cast<const uint4*>(xr + kb + k + 32 * j);
            gv[j] = *reinterpret_cast<const uint4*>(gr + kb + k + 32 * j);
        }
#pragma unroll
        for (int j = 0; j < RL_BATCH; ++j) acc = route_mfma8<BF16>(xv[j], gv[j], acc);
    }
    for (; k < kw; k += 32)
        acc = route_mfma8<BF16>(*reinterpret_cast<const uint4*>(xr + kb + k),
                                *reinterpret_cast<const uint4*>(gr + kb + k), acc);
    // lane l holds D[l / 16 + 4 v][l % 16], v = 0..3 (the f64 instruction's layout, unlike the f32 ones' 4 (l / 16) + v)
    if (wave > 0) {
#pragma unroll
        for (int v = 0; v < 4; ++v) part[wave - 1][v][lane] = acc[v];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        double sum = acc[v];
        for (int w = 1; w < RL_WAVES; ++w) sum += part[w - 1][v][lane];
        const int row = r0 + q + 4 * v, col = c0 + i;
        if (row < R && col < E) logits[(size_t)row * C + col] = bf2f(f64_to_bf16(sum));
    }
}

__global__ __launch_bounds__(256) void route_topk_kernel(float* __restrict__ logits, int R, int E, int k,
                                                         int shared_id, const uint16_t* __restrict__ x, int x_stride,
                                                         int bf16, const uint16_t* __restrict__ sgate, int H,
                                                         int* __restrict__ pick_out, float* __restrict__ wts_out) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= R) return;                                        // wave-uniform
    const bool has = shared_id >= 0;
    const int C = E + has, slots = k + has;
    float ls = 0.f;
    if (has) {                                                 // the shared gate's logit: x . sgate, one rounding
        double acc = 0.0;                                      // 2048 k at a time, all their loads in flight
        for (int h0 = 0; h0 < H; h0 += 2048) {
            uint2 xu[8], wu[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int h = h0 + 4 * lane + 256 * j;
                if (h < H) {
                    xu[j] = *reinterpret_cast<const uint2*>(x + (size_t)r * x_stride + h);
                    wu[j] = *reinterpret_cast<const uint2*>(sgate + h);
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (h0 + 4 * lane + 256 * j >= H) break;
                const uint16_t xh[4] = {(uint16_t)(xu[j].x & 0xFFFFu), (uint16_t)(xu[j].x >> 16),
                                        (uint16_t)(xu[j].y & 0xFFFFu), (uint16_t)(xu[j].y >> 16)};
                const uint16_t wh[4] = {(uint16_t)(wu[j].x & 0xFFFFu), (uint16_t)(wu[j].x >> 16),
                                        (uint16_t)(wu[j].y & 0xFFFFu), (uint16_t)(wu[j].y >> 16)};
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    acc = __builtin_fma((double)(bf16 ? bf2f(xh[q]) : h2f(xh[q])),
                                        (double)(bf16 ? bf2f(wh[q]) : h2f(wh[q])), acc);
            }
        }
        ls = (float)wave_sum_f64_dpp(acc);
        if (lane == 0) logits[(size_t)r * C + E] = ls;
    }
    int e_mine;
    float w_mine, w_shared;
    bool late = false;
    topk_row<0>(logits + (size_t)r * C, E, k, false, lane, e_mine, w_mine, w_shared, late);
    if (has) w_shared = 1.f / (1.f + expf(-ls));             // topk_row's sigmoid of the shared logit
    if (lane < k) {
        pick_out[(size_t)r * slots + lane] = e_mine;
        wts_out[(size_t)r * slots + lane] = w_mine;
    }
    if (has && lane == 0) {
        pick_out[(size_t)r * slots + k] = shared_id;
        wts_out[(size_t)r * slots + k] = w_shared;
    }
}

}  // namespace esp

// ======================================================================================================================
// C ABI
// ======================================================================================================================
using namespace esp;

static unsigned units_grid(long units, int per_block) { return (unsigned)((units + per_block - 1) / per_block); }

extern "C" int esp_group(const int32_t* pick, int32_t* uids, int64_t maxu, int32_t* ucount, int32_t* members,
                         int64_t maxm, int64_t R, int64_t slots, int64_t E, void* stream) {
    ESP_REQUIRE(pick && uids && ucount && members, "group: null pointer");
    ESP_REQUIRE(E >= 1 && E <= MAX_GROUP_IDS, "too many experts for the grouping kernel");
    ESP_REQUIRE(slots >= 1 && slots <= 32, "at most 32 slots a row");
    ESP_REQUIRE(R >= 1 && R * slots <= (int64_t(1) << 24), "grouping window too large");
    ESP_REQUIRE(maxu >= (R * slots < E ? R * slots : E), "uids too small");
    ESP_REQUIRE(maxm >= 1, "members too small");
    if (R * slots > MAX_PICKS) {                     // past one workgroup's shared memory: a workgroup an id
        ESP_REQUIRE(maxm <= GW_MAX_M, "group: at most 16384 members an expert");
        group_wide_kernel<<<(unsigned)E, GW, (size_t)maxm * 4, (hipStream_t)stream>>>(
            pick, (int)(R * slots), (int)slots, (int)E, (int)maxm, uids, ucount, members);
        return esp_host::launch_check("group (wide)");
    }
    group_kernel<<<1, GT, 0, (hipStream_t)stream>>>(pick, uids, ucount, members, (int)R, (int)slots, (int)E,
                                                     (int)maxm);
    return esp_host::launch_check("group");
}

struct RouteNorm {
    const void* h;
    const void* d1;
    const void* w;
    void* h_out;
    void* a_out;
    double eps;
};

static int route_impl(const void* x, int x_dtype, int64_t x_stride, int64_t R, int64_t H, const void* gate, int64_t E,
                      const void* sgate, int64_t k, int64_t shared_id, float* logits, int64_t logits_numel,
                      int32_t* counter, int32_t* pick_out, float* wts_out, int32_t* uids, int64_t maxu,
                      int32_t* ucount, int32_t* members, int64_t maxm, const RouteNorm* nrm, void* stream,
                      int sentinel = 0) {
    const int has = shared_id >= 0;
    ESP_REQUIRE(x && gate && logits && counter && pick_out && wts_out && uids && ucount && members,
                "route_group: null pointer");
    ESP_REQUIRE(x_dtype == ESP_BF16 || x_dtype == ESP_F16, "x: bf16/fp16");
    ESP_REQUIRE(E >= 1 && E <= 256 && k >= 1 && k <= 16 && k <= E && H % 256 == 0 && H > 0,
                "route_group: shape limits");
    ESP_REQUIRE(E + has <= RT_MAX_IDS, "route_group: too many router columns");
    ESP_REQUIRE(R >= 1 && R * (k + has) <= MAX_PICKS && k + has <= 32, "route_group: window too large");
    ESP_REQUIRE(!has || sgate, "the shared gate weight is needed with a shared slot");
    ESP_REQUIRE(logits_numel >= R * (E + has), "logits scratch too small");
    ESP_REQUIRE(x_stride >= H && x_stride % 4 == 0, "x row stride");
    ESP_REQUIRE(((uintptr_t)x & 7) == 0 && ((uintptr_t)gate & 7) == 0 && (!sgate || ((uintptr_t)sgate & 7) == 0),
                "route_group: x / gate must be 8-byte aligned");
    ESP_REQUIRE(maxu >= (R * (k + has) < E + has ? R * (k + has) : E + has), "uids too small");
    ESP_REQUIRE(maxm >= 1, "members too small");
    RouteArgs a{};
    a.x = static_cast<const uint16_t*>(x);
    a.gate = static_cast<const uint16_t*>(gate);
    a.sgate = static_cast<const uint16_t*>(sgate);
    a.logits = logits;
    a.counter = counter;
    a.pick_out = pick_out;
    a.wts_out = wts_out;
    a.uids = uids;
    a.ucount = ucount;
    a.members = members;
    a.x_stride = (int)x_stride;
    a.bf16 = x_dtype == ESP_BF16;
    a.R = (int)R;
    a.H = (int)H;
    a.E = (int)E;
    a.k = (int)k;
    a.shared_id = (int)shared_id;
    a.maxm = (int)maxm;
    a.win = (int)R;
    a.sentinel = sentinel;
    size_t smem = 0;
    if (nrm) {
        ESP_REQUIRE(nrm->h && nrm->w && nrm->h_out && nrm->a_out, "route_group_rmsnorm: null pointer");
        ESP_REQUIRE(R <= RT / 256, "route_group_rmsnorm: at most 4 rows (four waves normalise a row)");
        ESP_REQUIRE(H <= NORM_MAX_D && x_stride % 8 == 0 &&
                        ((uintptr_t)nrm->h | (uintptr_t)nrm->d1 | (uintptr_t)nrm->w | (uintptr_t)nrm->h_out |
                         (uintptr_t)nrm->a_out) % 16 == 0,
                    "route_group_rmsnorm: H at most 8192, rows 16-byte aligned");
        a.nh = static_cast<const uint16_t*>(nrm->h);
        a.nd1 = static_cast<const uint16_t*>(nrm->d1);
        a.nw = static_cast<const uint16_t*>(nrm->w);
        a.nh_out = static_cast<uint16_t*>(nrm->h_out);
        a.na_out = static_cast<uint16_t*>(nrm->a_out);
        a.neps = (float)nrm->eps;
        a.norm = 1;
        smem = (size_t)R * H * 2;
    }
    const unsigned grid = (unsigned)((E + has + RT_COLS - 1) / RT_COLS);
    const void* fn = a.norm ? (a.bf16 ? (const void*)route_group_kernel<1, true> : (const void*)route_group_kernel<0, true>)
                            : (a.bf16 ? (const void*)route_group_kernel<1, false> : (const void*)route_group_kernel<0, false>);
    if (smem > 64 * 1024 && hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
        return esp_host::fail(ESP_ERR_HIP, "route_group: cannot raise the shared memory limit to %zu bytes", smem);
    if (a.norm && a.bf16)
        route_group_kernel<1, true><<<grid, RT, smem, (hipStream_t)stream>>>(a);
    else if (a.norm)
        route_group_kernel<0, true><<<grid, RT, smem, (hipStream_t)stream>>>(a);
    else if (a.bf16)
        route_group_kernel<1, false><<<grid, RT, smem, (hipStream_t)stream>>>(a);
    else
        route_group_kernel<0, false><<<grid, RT, smem, (hipStream_t)stream>>>(a);
    return esp_host::launch_check("route_group");
}

extern "C" int esp_route_rows(const void* x, int x_dtype, int64_t x_stride, int64_t R, int64_t H, const void* gate,
                              int64_t E, const void* sgate, int64_t k, int64_t shared_id, float* logits,
                              int64_t logits_numel, int32_t* pick_out, float* wts_out, void* stream) {
    const int has = shared_id >= 0;
    ESP_REQUIRE(x && gate && logits && pick_out && wts_out, "route_rows: null pointer");
    ESP_REQUIRE(x_dtype == ESP_BF16 || x_dtype == ESP_F16, "x: bf16/fp16");
    ESP_REQUIRE(E >= 1 && E <= 256 && k >= 1 && k <= 16 && k <= E && H % 256 == 0 && H > 0,
                "route_rows: shape limits");
    ESP_REQUIRE(k + has <= 32, "route_rows: at most 32 slots a row");
    ESP_REQUIRE(!has || sgate, "the shared gate weight is needed with a shared slot");
    ESP_REQUIRE(R >= 1 && (R + 15) / 16 <= 65535, "route_rows: 1 to 1048560 rows");
    ESP_REQUIRE(logits_numel >= R * (E + has), "logits scratch too small");
    ESP_REQUIRE(x_stride >= H && x_stride % 8 == 0, "route_rows: x row stride a multiple of 8 elements");
    ESP_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)gate & 15) == 0 && (!sgate || ((uintptr_t)sgate & 15) == 0),
                "route_rows: x / gate must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    const int C = (int)(E + has);
    const dim3 grid((unsigned)((E + 15) / 16), (unsigned)((R + 15) / 16));
    const uint16_t *xp = static_cast<const uint16_t*>(x), *gp = static_cast<const uint16_t*>(gate),
                   *sp = static_cast<const uint16_t*>(sgate);
    if (x_dtype == ESP_BF16)
        route_logits_kernel<1><<<grid, RL_WAVES * 64, 0, st>>>(xp, (int)x_stride, gp, (int)R, (int)H, (int)E, C,
                                                               logits);
    else
        route_logits_kernel<0><<<grid, RL_WAVES * 64, 0, st>>>(xp, (int)x_stride, gp, (int)R, (int)H, (int)E, C,
                                                               logits);
    int rc = esp_host::launch_check("route_rows logits");
    if (rc) return rc;
    route_topk_kernel<<<(unsigned)((R + 3) / 4), 256, 0, st>>>(logits, (int)R, (int)E, (int)k, (int)shared_id, xp,
                                                               (int)x_stride, x_dtype == ESP_BF16 ? 1 : 0, sp, (int)H,
                                                               pick_out, wts_out);
    return esp_host::launch_check("route_rows");
}

extern "C" int esp_route_group(const void* x, int x_dtype, int64_t x_stride, int64_t R, int64_t H, const void* gate,
                               int64_t E, const void* sgate, int64_t k, int64_t shared_id, float* logits,
                               int64_t logits_numel, int32_t* counter, int32_t* pick_out, float* wts_out,
                               int32_t* uids, int64_t maxu, int32_t* ucount, int32_t* members, int64_t maxm,
                               void* stream) {
    return route_impl(x, x_dtype, x_stride, R, H, gate, E, sgate, k, shared_id, logits, logits_numel, counter,
                      pick_out, wts_out, uids, maxu, ucount, members, maxm, nullptr, stream);
}

extern "C" int esp_route_group_own(const void* x, int x_dtype, int64_t x_stride, int64_t R, int64_t H,
                                   const void* gate, int64_t E, const void* sgate, int64_t k, int64_t shared_id,
                                   float* logits, int64_t logits_numel, int32_t* counter, int32_t* pick_out,
                                   float* wts_out, int32_t* uids, int64_t maxu, int32_t* ucount, int32_t* members,
                                   int64_t maxm, void* stream) {
    return route_impl(x, x_dtype, x_stride, R, H, gate, E, sgate, k, shared_id, logits, logits_numel, counter,
                      pick_out, wts_out, uids, maxu, ucount, members, maxm, nullptr, stream, 1);
}

extern "C" int esp_route_group_rmsnorm(const void* h, const void* d1, const void* norm_w, double eps, void* h_out,
                                       void* a_out, int x_dtype, int64_t x_stride, int64_t R, int64_t H,
                                       const void* gate, int64_t E, const void* sgate, int64_t k, int64_t shared_id,
                                       float* logits, int64_t logits_numel, int32_t* counter, int32_t* pick_out,
                                       float* wts_out, int32_t* uids, int64_t maxu, int32_t* ucount,
                                       int32_t* members, int64_t maxm, void* stream) {
    const RouteNorm nrm{h, d1, norm_w, h_out, a_out, eps};
    return route_impl(h, x_dtype, x_stride, R, H, gate, E, sgate, k, shared_id, logits, logits_numel, counter,
                      pick_out, wts_out, uids, maxu, ucount, members, maxm, &nrm, stream, 1);
}

extern "C" int esp_group_shared(const int32_t* pick_in, const float* wts_in, const void* x, int x_dtype,
                                int64_t x_stride, int64_t H, const void* gate_w, int64_t shared_id, int32_t* pick_out,
                                float* wts_out, int32_t* uids, int64_t maxu, int32_t* ucount, int32_t* members,
                                int64_t maxm, int64_t R, int64_t slots_in, int64_t E, void* stream) {
    const int has = shared_id >= 0;
    const int64_t slots = slots_in + has;
    ESP_REQUIRE(pick_in && wts_in && pick_out && wts_out && uids && ucount && members, "group_shared: null pointer");
    ESP_REQUIRE(E >= 1 && E <= MAX_GROUP_IDS, "too many experts for the grouping kernel");
    ESP_REQUIRE(slots >= 1 && slots <= 32, "at most 32 slots a row");
    ESP_REQUIRE(R >= 1 && R * slots <= (int64_t(1) << 24), "grouping window too large");
    ESP_REQUIRE(!has || (gate_w && x), "a shared slot needs its gate weight");
    ESP_REQUIRE(!has || (x_dtype == ESP_BF16 || x_dtype == ESP_F16), "x: bf16/fp16");
    ESP_REQUIRE(!has || (H % 256 == 0 && x_stride % 4 == 0), "group_shared: H must be a multiple of 256");
    ESP_REQUIRE(maxu >= (R * slots < E ? R * slots : E), "uids too small");
    ESP_REQUIRE(maxm >= 1, "members too small");
    if (R * slots > MAX_PICKS) {                     // past one workgroup's shared memory: the tables, then the grouping
        ESP_REQUIRE(maxm <= GW_MAX_M, "group_shared: at most 16384 members an expert");
        hipStream_t st = (hipStream_t)stream;
        shared_slots_kernel<<<(unsigned)((R + 3) / 4), 256, 0, st>>>(
            pick_in, wts_in, static_cast<const uint16_t*>(x), (int)x_stride, x_dtype == ESP_BF16,
            static_cast<const uint16_t*>(gate_w), (int)H, (int)shared_id, pick_out, wts_out, (int)R, (int)slots_in);
        const int rc = esp_host::launch_check("group_shared (slots)");
        if (rc) return rc;
        group_wide_kernel<<<(unsigned)E, GW, (size_t)maxm * 4, st>>>(pick_out, (int)(R * slots), (int)slots, (int)E,
                                                                      (int)maxm, uids, ucount, members);
        return esp_host::launch_check("group_shared (wide)");
    }
    group_shared_kernel<<<1, GT, 0, (hipStream_t)stream>>>(
        pick_in, wts_in, static_cast<const uint16_t*>(x), (int)x_stride, x_dtype == ESP_BF16,
        static_cast<const uint16_t*>(gate_w), (int)H, (int)shared_id, pick_out, wts_out, uids, ucount, members,
        (int)R, (int)slots_in, (int)E, (int)maxm);
    return esp_host::launch_check("group_shared");
}

extern "C" int esp_rot_in(const void* x, int x_dtype, int64_t x_stride, const int32_t* pick, const void* suh0,
                          const void* suh1, void* out0, void* out1, int64_t rows, int64_t K, int64_t slots, int64_t E,
                          void* stream) {
    ESP_REQUIRE(x && pick && suh0 && suh1 && out0 && out1, "rot_in: null pointer");
    ESP_REQUIRE(x_dtype == ESP_BF16 || x_dtype == ESP_F16, "x: bf16/fp16");
    ESP_REQUIRE(K % 128 == 0 && K > 0, "K must be a multiple of 128");
    ESP_REQUIRE(x_stride >= K && x_stride % 4 == 0, "x row stride");
    ESP_REQUIRE((((uintptr_t)x | (uintptr_t)suh0 | (uintptr_t)suh1 | (uintptr_t)out0 | (uintptr_t)out1) & 7) == 0,
                "rot_in: x, suh and the outputs must be 8-byte aligned");
    ESP_REQUIRE(rows * slots < (int64_t(1) << 31), "rot_in: at most 2^31 - 1 slot rows");
    if (rows * slots <= 0) return esp_host::ok();
    rot_in_kernel<<<(unsigned)(rows * slots), 256, 0, (hipStream_t)stream>>>(
        static_cast<const uint16_t*>(x), x_dtype, (int)x_stride, pick, static_cast<const uint16_t*>(suh0),
        static_cast<const uint16_t*>(suh1), static_cast<uint16_t*>(out0), static_cast<uint16_t*>(out1), (int)K,
        (int)slots, (int)E);
    return esp_host::launch_check("rot_in");
}

// the largest number of non-empty member tiles a grouping of P picks over nexp_max expert slots can have: the sum
// over experts of ceil(members / 32) is at most P / 32 + the experts used
static int64_t tile_list_cap(int64_t nexp_max, int64_t maxm, int64_t P) {
    const int64_t mt = (maxm + 31) / 32, bound = (P + 31) / 32 + nexp_max;
    return nexp_max * mt < bound ? nexp_max * mt : bound;
}

// esp_grouped, or esp_grouped_list when tiles is given (then grid x runs over the list's entries)
static int grouped_impl(const void* X0, const void* X1, const int64_t* TP0, const int64_t* TP1, const int32_t* B0,
                        const int32_t* B1, const int32_t* C0, const int32_t* C1, const int32_t* uids, int64_t nexp_max,
                        const int32_t* ucount, const int32_t* members, int64_t maxm, float* Z, int64_t z_numel,
                        int64_t mats, int64_t K, int64_t N, int64_t P, int64_t SK, int64_t slots, int64_t warps,
                        int64_t lo, int64_t hi, const int32_t* tiles, void* stream) {
    ESP_REQUIRE(X0 && X1 && TP0 && TP1 && B0 && B1 && C0 && C1 && uids && ucount && members && Z,
                "grouped: null pointer");
    ESP_REQUIRE(mats == 1 || mats == 2, "mats must be 1 or 2");
    ESP_REQUIRE(SK >= 1 && K > 0 && N > 0 && K % (32 * SK) == 0 && N % 128 == 0, "K and N must split evenly");
    ESP_REQUIRE(z_numel >= mats * SK * P * N, "Z too small");
    ESP_REQUIRE(maxm >= 1 && maxm <= 65536, "members a row of the table: 1 to 65536");
    ESP_REQUIRE(slots >= 1 && slots <= 32, "at most 32 slots a row");
    ESP_REQUIRE(lo >= 2 && hi <= 16 && lo <= hi, "K2 range must lie in [2, 16]");
    ESP_REQUIRE(warps == 4 || warps == 8 || warps == 16, "warps (waves a workgroup) must be 4, 8 or 16");
    ESP_REQUIRE((((uintptr_t)X0 | (uintptr_t)X1 | (uintptr_t)Z) & 15) == 0,
                "grouped: X0 / X1 and Z must be 16-byte aligned (rows and partials move 16 bytes at a time)");
    const int64_t mt = (maxm + 31) / 32;                 // an expert's members in tiles of 32 (experts_grouped.cuh:244)
    ESP_REQUIRE(mats * SK * mt <= 65535, "grouped: too many member tiles, splits and matrices for one launch");
    if (nexp_max <= 0) return esp_host::ok();
    GroupedArgs a{};
    a.mt = (int)mt;
    a.X0 = static_cast<const uint16_t*>(X0);
    a.X1 = static_cast<const uint16_t*>(X1);
    a.TP0 = TP0;
    a.TP1 = TP1;
    a.B0 = B0;
    a.B1 = B1;
    a.C0 = C0;
    a.C1 = C1;
    a.uids = uids;
    a.ucount = ucount;
    a.members = members;
    a.Z = Z;
    a.K = (int)K;
    a.N = (int)N;
    a.P = (int)P;
    a.SK = (int)SK;
    a.maxm = (int)maxm;
    a.slots = (int)slots;
    a.lo = (int)lo;
    a.hi = (int)hi;
    a.tiles = tiles;
    dim3 grid((unsigned)nexp_max, (unsigned)(N / 128), (unsigned)(mats * SK * mt));
    if (tiles != nullptr) grid = dim3((unsigned)tile_list_cap(nexp_max, maxm, P), (unsigned)(N / 128), (unsigned)(mats * SK));
    // K ranges of AST_MIN_STEPS steps or more stage the member rows with the tiles (grouped_body_staged), whose
    // member-row offsets are 32-bit and whose waves hold at most 8 member rows each
    a.staged = (K / SK) / 32 >= AST_MIN_STEPS;
    ESP_REQUIRE(!a.staged || (P * K < (int64_t(1) << 31) && warps >= 4),
                "grouped: a staged launch needs P * K below 2^31 and at least 4 waves");
    const size_t stage = a.staged ? 2 * (size_t)staged_buf_bytes((int)hi)
                                  : (size_t)host_stage_words((int)hi, (int)(K / SK)) * 4;   // the widest expert's
    const size_t red = (size_t)(warps / 4) * 32 * 128 * 4;                         // the k slots' partials
    const size_t smem = stage > red ? stage : red;
    if (smem > 64 * 1024 &&
        hipFuncSetAttribute(a.staged ? (const void*)grouped_kernel_t<2> : (const void*)grouped_kernel_t<0>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) !=
            hipSuccess)
        return esp_host::fail(ESP_ERR_HIP, "grouped: cannot raise the shared memory limit to %zu bytes", smem);
    if (a.staged)
        grouped_kernel_t<2><<<grid, (unsigned)(64 * warps), smem, (hipStream_t)stream>>>(a);
    else
        grouped_kernel_t<0><<<grid, (unsigned)(64 * warps), smem, (hipStream_t)stream>>>(a);
    return esp_host::launch_check("grouped");
}

extern "C" int esp_grouped(const void* X0, const void* X1, const int64_t* TP0, const int64_t* TP1, const int32_t* B0,
                           const int32_t* B1, const int32_t* C0, const int32_t* C1, const int32_t* uids,
                           int64_t nexp_max, const int32_t* ucount, const int32_t* members, int64_t maxm, float* Z,
                           int64_t z_numel, int64_t mats, int64_t K, int64_t N, int64_t P, int64_t SK, int64_t slots,
                           int64_t nt, int64_t warps, int64_t pf, int64_t lo, int64_t hi, void* stream) {
    (void)nt;
    (void)pf;
    return grouped_impl(X0, X1, TP0, TP1, B0, B1, C0, C1, uids, nexp_max, ucount, members, maxm, Z, z_numel, mats, K,
                        N, P, SK, slots, warps, lo, hi, nullptr, stream);
}

extern "C" int esp_tile_list(const int32_t* ucount, const int32_t* members, int64_t nexp_max, int64_t maxm, int64_t P,
                             int32_t* tiles, int64_t tiles_numel, void* stream) {
    ESP_REQUIRE(ucount && members && tiles, "tile_list: null pointer");
    ESP_REQUIRE(nexp_max >= 1 && nexp_max < 65536 && maxm >= 1 && maxm <= 65536 && P >= 1,
                "tile_list: 1 to 65535 expert slots, 1 to 65536 members a row, P >= 1");
    const int64_t mt = (maxm + 31) / 32, cap = tile_list_cap(nexp_max, maxm, P);
    ESP_REQUIRE(nexp_max * mt <= (int64_t)TL_THREADS * TL_PER, "tile_list: at most 32768 (expert, member tile) pairs");
    ESP_REQUIRE(tiles_numel >= 1 + cap, "tile_list: tiles needs 1 + min(E * ceil(maxm / 32), ceil(P / 32) + E) ints");
    tile_list_kernel<<<1, TL_THREADS, 0, (hipStream_t)stream>>>(ucount, members, (int)nexp_max, (int)maxm, (int)mt,
                                                                tiles, (int)cap);
    return esp_host::launch_check("tile_list");
}

extern "C" int esp_grouped_list(const void* X0, const void* X1, const int64_t* TP0, const int64_t* TP1,
                                const int32_t* B0, const int32_t* B1, const int32_t* C0, const int32_t* C1,
                                const int32_t* uids, int64_t nexp_max, const int32_t* ucount, const int32_t* members,
                                int64_t maxm, const int32_t* tiles, float* Z, int64_t z_numel, int64_t mats, int64_t K,
                                int64_t N, int64_t P, int64_t SK, int64_t slots, int64_t warps, int64_t lo, int64_t hi,
                                void* stream) {
    ESP_REQUIRE(tiles, "grouped_list: null tile list");
    ESP_REQUIRE(nexp_max < 65536, "grouped_list: at most 65535 expert slots");
    return grouped_impl(X0, X1, TP0, TP1, B0, B1, C0, C1, uids, nexp_max, ucount, members, maxm, Z, z_numel, mats, K,
                        N, P, SK, slots, warps, lo, hi, tiles, stream);
}

static int grouped_launch_gateup(const GroupedArgs& a, int64_t nexp_max, int64_t warps, size_t smem, hipStream_t st) {
    if (smem > 64 * 1024 && hipFuncSetAttribute((const void*)grouped_kernel_t<1>,
                                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
        return esp_host::fail(ESP_ERR_HIP, "moe_gateup: cannot raise the shared memory limit to %zu bytes", smem);
    dim3 grid((unsigned)nexp_max, (unsigned)(a.N / 128), (unsigned)(2 * a.SK));
    grouped_kernel_t<1><<<grid, (unsigned)(64 * warps), smem, st>>>(a);
    return esp_host::launch_check("moe_gateup");
}

// esp_moe_gateup's checks and arguments without the launch (also the chained launch's gate/up group)
static int gateup_args(const void* x, int x_dtype, int64_t x_stride, const void* suh_g, const void* suh_u,
                       const int64_t* TP0, const int64_t* TP1, const int32_t* B0, const int32_t* B1, const int32_t* C0,
                       const int32_t* C1, const int32_t* uids, int64_t nexp_max, const int32_t* ucount,
                       const int32_t* members, int64_t maxm, float* Z, int64_t z_numel, int32_t* counters,
                       int64_t counters_numel, const void* svh_g, const void* svh_u, const void* suh_d, void* xd,
                       int64_t K, int64_t N, int64_t P, int64_t SK, int64_t slots, int64_t warps, int64_t lo,
                       int64_t hi, double limit, int64_t act_mode, GroupedArgs& a, size_t& smem_out) {
    ESP_REQUIRE(x && suh_g && suh_u && TP0 && TP1 && B0 && B1 && C0 && C1 && uids && ucount && members && Z &&
                    counters && svh_g && svh_u && suh_d && xd,
                "moe_gateup: null pointer");
    ESP_REQUIRE(x_dtype == ESP_BF16 || x_dtype == ESP_F16, "x: bf16/fp16");
    ESP_REQUIRE(SK >= 1 && K > 0 && N > 0 && K % (128 * SK) == 0 && N % 128 == 0,
                "moe_gateup: K must split into whole 128-blocks, N a multiple of 128");
    ESP_REQUIRE(x_stride >= K && x_stride % 4 == 0, "x row stride");
    ESP_REQUIRE(((uintptr_t)Z & 15) == 0 && (((uintptr_t)x | (uintptr_t)suh_g | (uintptr_t)suh_u | (uintptr_t)svh_g |
                                               (uintptr_t)svh_u | (uintptr_t)suh_d | (uintptr_t)xd) & 7) == 0,
                "moe_gateup: Z 16-byte aligned, x, the scales and xd 8-byte aligned");
    ESP_REQUIRE(z_numel >= 2 * SK * P * N, "Z too small");
    ESP_REQUIRE(2 * SK * P * N <= (int64_t(1) << 30), "moe_gateup: the partials must fit in 4 GiB");
    ESP_REQUIRE(maxm >= 1 && maxm <= 32, "at most 32 member rows an expert");
    ESP_REQUIRE(slots >= 1 && slots <= 32, "at most 32 slots a row");
    ESP_REQUIRE(lo >= 2 && hi <= 16 && lo <= hi, "K2 range must lie in [2, 16]");
    ESP_REQUIRE(warps == 4 || warps == 8 || warps == 16, "warps (waves a workgroup) must be 4, 8 or 16");
    ESP_REQUIRE(counters_numel >= nexp_max * (N / 128) * CNT_STRIDE, "counters: 32 ints per (expert, 128 columns)");
    a = GroupedArgs{};
    a.mt = 1;
    a.X0 = a.X1 = nullptr;
    a.TP0 = TP0;
    a.TP1 = TP1;
    a.B0 = B0;
    a.B1 = B1;
    a.C0 = C0;
    a.C1 = C1;
    a.uids = uids;
    a.ucount = ucount;
    a.members = members;
    a.Z = Z;
    a.K = (int)K;
    a.N = (int)N;
    a.P = (int)P;
    a.SK = (int)SK;
    a.maxm = (int)maxm;
    a.slots = (int)slots;
    a.x = x;
    a.x_dtype = x_dtype;
    a.x_stride = (int)x_stride;
    a.suh0 = static_cast<const uint16_t*>(suh_g);
    a.suh1 = static_cast<const uint16_t*>(suh_u);
    a.svh0 = static_cast<const uint16_t*>(svh_g);
    a.svh1 = static_cast<const uint16_t*>(svh_u);
    a.suh_d = static_cast<const uint16_t*>(suh_d);
    a.xd = static_cast<uint16_t*>(xd);
    a.limit = (float)limit;
    a.act_mode = (int)act_mode;
    a.counters = counters;
    a.lo = (int)lo;
    a.hi = (int)hi;
    const int64_t kr = K / SK;
    const size_t stage = (size_t)host_stage_words((int)hi, (int)kr) * 4;   // the widest expert's stages
    a.stage_bytes = (int)stage;
    a.xs_stride = (int)kr + 8;                                             // pad rows across the LDS banks
    // the rotated rows and the k slots' partials of at most maxm member rows (a program's members are <= maxm)
    const size_t xs = (size_t)maxm * a.xs_stride * 2;
    const size_t red = (size_t)(warps / 4) * maxm * 128 * 4;
    smem_out = stage + xs > red ? stage + xs : red;
    ESP_REQUIRE(smem_out <= 160 * 1024, "moe_gateup: shared memory exceeds 160 KiB");
    return ESP_OK;
}

extern "C" int esp_moe_gateup(const void* x, int x_dtype, int64_t x_stride, const void* suh_g, const void* suh_u,
                              const int64_t* TP0, const int64_t* TP1, const int32_t* B0, const int32_t* B1,
                              const int32_t* C0, const int32_t* C1, const int32_t* uids, int64_t nexp_max,
                              const int32_t* ucount, const int32_t* members, int64_t maxm, float* Z, int64_t z_numel,
                              int32_t* counters, int64_t counters_numel, const void* svh_g, const void* svh_u,
                              const void* suh_d, void* xd, int64_t K, int64_t N, int64_t P, int64_t SK, int64_t slots,
                              int64_t warps, int64_t lo, int64_t hi, double limit, int64_t act_mode, void* stream) {
    GroupedArgs a{};
    size_t smem = 0;
    const int rc = gateup_args(x, x_dtype, x_stride, suh_g, suh_u, TP0, TP1, B0, B1, C0, C1, uids, nexp_max, ucount,
                               members, maxm, Z, z_numel, counters, counters_numel, svh_g, svh_u, suh_d, xd, K, N, P,
                               SK, slots, warps, lo, hi, limit, act_mode, a, smem);
    if (rc) return rc;
    if (nexp_max <= 0) return esp_host::ok();
    return grouped_launch_gateup(a, nexp_max, warps, smem, (hipStream_t)stream);
}

extern "C" int esp_moe_chain(const void* x, int x_dtype, int64_t x_stride, const void* suh_g, const void* suh_u,
                             const int64_t* TP0, const int64_t* TP1, const int64_t* TP2, const int32_t* B0,
                             const int32_t* B1, const int32_t* B2, const int32_t* C0, const int32_t* C1,
                             const int32_t* C2, const int32_t* uids, int64_t nexp_max, const int32_t* ucount,
                             const int32_t* members, int64_t rows, const int32_t* pick, const float* wts,
                             const void* svh_g, const void* svh_u, const void* suh_d, const void* svh_d, void* xd,
                             float* Z, int64_t z_numel, float* Zd, int64_t zd_numel, float* y, void* out,
                             int out_dtype, void* out_shared, int32_t* counters, int64_t counters_numel,
                             int32_t* flags, int64_t flags_numel, int64_t D, int64_t I, int64_t SK, int64_t slots,
                             int64_t E, int64_t n_routed, int64_t lo, int64_t hi, int64_t lo_d, int64_t hi_d,
                             double limit, int64_t act_mode, void* stream) {
    ESP_REQUIRE(rows >= 1 && rows <= CHAIN_ROWS, "moe_chain: 1 to 4 rows");
    const int64_t P = rows * slots;
    GroupedArgs gu{};
    size_t smem_gu = 0;
    int rc = gateup_args(x, x_dtype, x_stride, suh_g, suh_u, TP0, TP1, B0, B1, C0, C1, uids, nexp_max, ucount, members,
                         rows, Z, z_numel, counters, counters_numel, svh_g, svh_u, suh_d, xd, D, I, P, SK, slots, 4,
                         lo, hi, limit, act_mode, gu, smem_gu);
    if (rc) return rc;
    ESP_REQUIRE(TP2 && B2 && C2 && pick && wts && svh_d && Zd && y && out && flags, "moe_chain: null pointer");
    ESP_REQUIRE(out_dtype >= 0 && out_dtype <= 2, "moe_chain: out dtype");
    ESP_REQUIRE(n_routed >= 0 && n_routed <= slots && E >= 1, "moe_chain: n_routed <= slots");
    ESP_REQUIRE(I % 128 == 0 && I / 128 <= 64 && D % 128 == 0, "moe_chain: I and D multiples of 128");
    ESP_REQUIRE(lo_d >= 2 && hi_d <= 16 && lo_d <= hi_d, "moe_chain: down K2 range must lie in [2, 16]");
    ESP_REQUIRE((((uintptr_t)Zd | (uintptr_t)y) & 15) == 0 && ((uintptr_t)xd & 7) == 0 && ((uintptr_t)svh_d & 7) == 0,
                "moe_chain: Zd and y 16-byte aligned, xd and svh_d 8-byte aligned");
    const int64_t SKd = I / 128;                         // a down split a gate/up column block
    ESP_REQUIRE(SKd <= CHAIN_MAX_SPLITS, "moe_chain: I at most 1024 (8 down splits of 128)");
    ESP_REQUIRE(zd_numel >= SKd * P * D, "moe_chain: Zd needs I / 128 * P * D floats");
    ESP_REQUIRE(SKd * P * D <= (int64_t(1) << 30), "moe_chain: the down partials must fit in 4 GiB");
    const int64_t nb_gu = I / 128, nyd = D / 128;
    const int64_t lines = 2 * nexp_max * nb_gu + 2 * nyd;
    ESP_REQUIRE(flags_numel >= lines * CNT_STRIDE, "moe_chain: flags need 32 ints a line, 2 * (nexp * I + D) / 128 lines");
    ESP_REQUIRE(((uintptr_t)flags & 3) == 0, "moe_chain: flags 4-byte aligned");
    if (nexp_max <= 0) return esp_host::ok();
    ChainArgs c{};
    c.gu = gu;
    c.gu.chain = 1;
    c.xd_seen = flags;                                   // the first nexp_max * I / 128 lines: xd's reader counts
    GroupedArgs& dn = c.dn;
    dn.mt = 1;
    dn.X0 = dn.X1 = static_cast<const uint16_t*>(xd);
    dn.TP0 = dn.TP1 = TP2;
    dn.B0 = dn.B1 = B2;
    dn.C0 = dn.C1 = C2;
    dn.uids = uids;
    dn.ucount = ucount;
    dn.members = members;
    dn.Z = Zd;
    dn.K = (int)I;
    dn.N = (int)D;
    dn.P = (int)P;
    dn.SK = (int)SKd;
    dn.maxm = (int)rows;
    dn.slots = (int)slots;
    dn.lo = (int)lo_d;
    dn.hi = (int)hi_d;
    dn.stage_bytes = host_stage_words((int)hi_d, 128) * 4;
    dn.xs_stride = 128 + 8;
    c.pick = pick;
    c.wts = wts;
    c.svh_d = static_cast<const uint16_t*>(svh_d);
    c.y = y;
    c.out = out;
    c.out_shared = out_shared;
    c.R = (int)rows;
    c.E = (int)E;
    c.n_routed = (int)n_routed;
    c.nexp = (int)nexp_max;
    c.n_gu = (int)(nexp_max * nb_gu * 2 * SK);
    c.n_dn = (int)(nexp_max * nyd * SKd);
    const int n_cb = (int)(rows * nyd);
    const size_t smem_dn = (size_t)dn.stage_bytes + (size_t)16 * dn.xs_stride * 2;
    const size_t smem_cb = (size_t)slots * 128 * 4;
    size_t smem = smem_gu > smem_dn ? smem_gu : smem_dn;
    smem = smem > smem_cb ? smem : smem_cb;
    hipStream_t st = (hipStream_t)stream;
    const void* kern = out_dtype == ESP_BF16 ? (const void*)moe_chain_kernel<BF16>
                       : out_dtype == ESP_F16 ? (const void*)moe_chain_kernel<F16>
                                              : (const void*)moe_chain_kernel<F32>;
    if (smem > 64 * 1024 &&
        hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
        return esp_host::fail(ESP_ERR_HIP, "moe_chain: cannot raise the shared memory limit to %zu bytes", smem);
    const unsigned grid = (unsigned)(c.n_gu + c.n_dn + n_cb);
    if (out_dtype == ESP_BF16)
        moe_chain_kernel<BF16><<<grid, 256, smem, st>>>(c);
    else if (out_dtype == ESP_F16)
        moe_chain_kernel<F16><<<grid, 256, smem, st>>>(c);
    else
        moe_chain_kernel<F32><<<grid, 256, smem, st>>>(c);
    return esp_host::launch_check("moe_chain");
}

extern "C" int esp_gateup_epilogue(const float* Z, const int32_t* pick, const void* svh_g, const void* svh_u,
                                   const void* suh_d, void* xd, int64_t rows, int64_t P, int64_t N, int64_t SK,
                                   int64_t slots, int64_t E, double limit, int64_t act_mode, void* stream) {
    ESP_REQUIRE(Z && pick && svh_g && svh_u && suh_d && xd, "gateup_epilogue: null pointer");
    ESP_REQUIRE(N % 128 == 0 && N > 0, "N must be a multiple of 128");
    ESP_REQUIRE(SK >= 1, "SK must be positive");
    ESP_REQUIRE(rows * slots <= P, "rows * slots must not exceed P");
    ESP_REQUIRE(((uintptr_t)Z & 15) == 0 && (((uintptr_t)svh_g | (uintptr_t)svh_u | (uintptr_t)suh_d |
                                               (uintptr_t)xd) & 7) == 0,
                "gateup_epilogue: Z 16-byte aligned, the scales and xd 8-byte aligned");
    const long units = rows * slots * (N / 128);
    if (units <= 0) return esp_host::ok();
    gateup_epilogue_kernel<<<units_grid(units, 8), 256, 0, (hipStream_t)stream>>>(
        Z, pick, static_cast<const uint16_t*>(svh_g), static_cast<const uint16_t*>(svh_u),
        static_cast<const uint16_t*>(suh_d), static_cast<uint16_t*>(xd), (int)P, (int)N, (int)SK, (int)E,
        (float)limit, (int)act_mode);
    return esp_host::launch_check("gateup_epilogue");
}

extern "C" int esp_down_epilogue(const float* Z, const int32_t* pick, const void* svh_d, float* y, int64_t rows,
                                 int64_t P, int64_t D, int64_t SK, int64_t slots, int64_t E, void* stream) {
    ESP_REQUIRE(Z && pick && svh_d && y, "down_epilogue: null pointer");
    ESP_REQUIRE(D % 128 == 0 && D > 0, "D must be a multiple of 128");
    ESP_REQUIRE(rows * slots <= P, "rows * slots must not exceed P");
    const long units = rows * slots * (D / 128);
    if (units <= 0) return esp_host::ok();
    down_epilogue_kernel<<<units_grid(units, 8), 256, 0, (hipStream_t)stream>>>(
        Z, pick, static_cast<const uint16_t*>(svh_d), y, (int)P, (int)D, (int)SK, (int)E);
    return esp_host::launch_check("down_epilogue");
}

extern "C" int esp_combine(const float* y, const float* wts, float* out, int64_t rows, int64_t D, int64_t slots,
                           void* stream) {
    ESP_REQUIRE(y && wts && out, "combine: null pointer");
    const long n = rows * D;
    if (n <= 0) return esp_host::ok();
    combine_kernel<<<units_grid(n, 256), 256, 0, (hipStream_t)stream>>>(y, wts, out, (int)rows, (int)D, (int)slots);
    return esp_host::launch_check("combine");
}

static int down_combine_any(const float* Z, const int32_t* pick, const void* svh_d, float* y, const float* wts,
                            void* out, int out_dtype, void* out_shared, int64_t rows, int64_t P, int64_t D, int64_t SK,
                            int64_t slots, int64_t E, int64_t n_routed, void* stream) {
    ESP_REQUIRE(Z && pick && svh_d && wts && out, "down_combine: null pointer");
    ESP_REQUIRE(slots >= 1 && slots <= 32, "at most 32 slots a row");
    ESP_REQUIRE(D % 128 == 0 && D > 0, "D must be a multiple of 128");
    ESP_REQUIRE(n_routed >= 0 && n_routed <= slots, "n_routed <= slots");
    ESP_REQUIRE(rows * slots <= P, "rows * slots must not exceed P");
    if (rows <= 0) return esp_host::ok();
    hipStream_t s = (hipStream_t)stream;
    auto svh = static_cast<const uint16_t*>(svh_d);
    if (rows >= DCR_ROWS) {                                 // a workgroup a (row, 4 128-blocks)
        ESP_REQUIRE(rows < (int64_t(1) << 31), "down_combine: at most 2^31 - 1 rows");
        const size_t smem = (size_t)slots * DCR_BLOCKS * 128 * 4;
        const dim3 g((unsigned)rows, (unsigned)((D / 128 + DCR_BLOCKS - 1) / DCR_BLOCKS));
        if (out_dtype == ESP_BF16)
            down_combine_rows_kernel<BF16><<<g, 256, smem, s>>>(Z, pick, svh, y, wts, out, out_shared, (int)P, (int)D,
                                                                (int)SK, (int)E, (int)slots, (int)n_routed);
        else if (out_dtype == ESP_F16)
            down_combine_rows_kernel<F16><<<g, 256, smem, s>>>(Z, pick, svh, y, wts, out, out_shared, (int)P, (int)D,
                                                               (int)SK, (int)E, (int)slots, (int)n_routed);
        else
            down_combine_rows_kernel<F32><<<g, 256, smem, s>>>(Z, pick, svh, y, wts, out, out_shared, (int)P, (int)D,
                                                               (int)SK, (int)E, (int)slots, (int)n_routed);
        return esp_host::launch_check("down_combine");
    }
    dim3 grid((unsigned)rows, (unsigned)(D / 128));
    // a 32-lane half a slot, so every slot's partials are loaded in one round (9 slots: 320 threads, not 256)
    const unsigned nt = slots * 32 <= 256 ? 256u : (unsigned)((slots * 32 + 63) / 64 * 64);
    if (out_dtype == ESP_BF16)
        down_combine_kernel<BF16><<<grid, nt, 0, s>>>(Z, pick, svh, y, wts, out, out_shared, (int)P, (int)D, (int)SK,
                                                      (int)E, (int)slots, (int)n_routed);
    else if (out_dtype == ESP_F16)
        down_combine_kernel<F16><<<grid, nt, 0, s>>>(Z, pick, svh, y, wts, out, out_shared, (int)P, (int)D, (int)SK,
                                                     (int)E, (int)slots, (int)n_routed);
    else
        down_combine_kernel<F32><<<grid, nt, 0, s>>>(Z, pick, svh, y, wts, out, out_shared, (int)P, (int)D, (int)SK,
                                                     (int)E, (int)slots, (int)n_routed);
    return esp_host::launch_check("down_combine");
}

extern "C" int esp_down_combine(const float* Z, const int32_t* pick, const void* svh_d, float* y, const float* wts,
                                float* out, int64_t rows, int64_t P, int64_t D, int64_t SK, int64_t slots, int64_t E,
                                void* stream) {
    return down_combine_any(Z, pick, svh_d, y, wts, out, ESP_F32, nullptr, rows, P, D, SK, slots, E, slots, stream);
}

extern "C" int esp_down_combine2(const float* Z, const int32_t* pick, const void* svh_d, float* y, const float* wts,
                                 void* out, int out_dtype, void* out_shared, int64_t rows, int64_t P, int64_t D,
                                 int64_t SK, int64_t slots, int64_t E, int64_t n_routed, void* stream) {
    return down_combine_any(Z, pick, svh_d, y, wts, out, out_dtype, out_shared, rows, P, D, SK, slots, E, n_routed,
                            stream);
}

extern "C" int esp_status(int32_t* status, int clear, void* stream) {
    ESP_REQUIRE(status, "status: null pointer");
    hipStream_t st = (hipStream_t)stream;
    int v = 0;
    *status = 0;
    if (hipMemcpyFromSymbolAsync(&v, HIP_SYMBOL(g_status), sizeof(int), 0, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return esp_host::fail(ESP_ERR_HIP, "status: cannot read the device status word");
    if (esp_host::dense_status(clear, st, status)) return ESP_ERR_HIP;
    if (esp_host::tile_status(clear, st, status)) return ESP_ERR_HIP;
    if (esp_host::dense_own_status(clear, st, status)) return ESP_ERR_HIP;
    *status |= v;
    if (clear && v) {
        const int zero = 0;
        if (hipMemcpyToSymbolAsync(HIP_SYMBOL(g_status), &zero, sizeof(int), 0, hipMemcpyHostToDevice, st) !=
                hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            return esp_host::fail(ESP_ERR_HIP, "status: cannot clear the device status word");
    }
    return esp_host::ok();
}

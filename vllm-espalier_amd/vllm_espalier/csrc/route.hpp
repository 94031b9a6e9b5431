// Pieces of the routing launches (route_group_kernel, route_topk_kernel): the launch arguments, exact fp64 logits
// rounded once to bf16, and one row's top-k / softmax / grouping by one wave.
#pragma once

#include "common.hpp"

namespace esp {

// bf16 bits of a double, one rounding (to nearest, ties to even)
__device__ __forceinline__ uint16_t f64_to_bf16(double d) {
    const uint64_t x = __builtin_bit_cast(uint64_t, d);
    const uint32_t sign = (uint32_t)(x >> 48) & 0x8000u;
    const uint64_t ax = x & 0x7FFFFFFFFFFFFFFFull;
    if (ax > 0x7FF0000000000000ull) return (uint16_t)(sign | 0x7FC0u);
    const int e = (int)(ax >> 52);
    if (e == 0) return (uint16_t)sign;
    int E = e - 1023 + 127;
    if (E >= 255) return (uint16_t)(sign | 0x7F80u);
    const uint64_t m = (ax & ((1ull << 52) - 1)) | (1ull << 52);
    const int shift = E >= 1 ? 45 : 45 + (1 - E);
    if (shift > 54) return (uint16_t)sign;
    uint64_t q = m >> shift;
    const uint64_t rem = m & ((1ull << shift) - 1), half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1;
    uint32_t bits;
    if (E >= 1) {
        if (q == 256) {
            q = 128;
            E += 1;
            if (E >= 255) return (uint16_t)(sign | 0x7F80u);
        }
        bits = ((uint32_t)E << 7) | (uint32_t)(q & 0x7Fu);
    } else {
        bits = (uint32_t)q;
    }
    return (uint16_t)(sign | bits);
}

struct RouteArgs {
    const uint16_t* x;
    const uint16_t* gate;
    const uint16_t* sgate;
    float* logits;
    int* counter;
    int* pick_out;
    float* wts_out;
    int* uids;
    int* ucount;
    int* members;
    int x_stride, bf16, R, H, E, k, shared_id, maxm;
    int win;                         // rows a window (blockIdx.y): R for esp_route_group, 32 for esp_route_rows
    // esp_route_group_rmsnorm: x = RMSNorm(h + d1) * nw (norm.hpp), made in the launch into shared memory; workgroup 0
    // stores it to na_out and the residual h + d1 to nh_out. Rows of h, d1, nh_out and na_out are x_stride apart.
    const uint16_t* nh;
    const uint16_t* nd1;
    const uint16_t* nw;
    uint16_t* nh_out;
    uint16_t* na_out;
    float neps;
    int norm;
    // logits hold all-ones between launches (esp_route_group_rmsnorm): at one row the last workgroup (dispatched after
    // the others) polls them until no logit is all-ones, with no arrival count; every launch puts the all-ones back
    int sentinel;
};

constexpr int RT = 1024;             // threads of a route workgroup
constexpr int RT_COLS = 4;           // router columns a workgroup
constexpr int RT_MAX_IDS = 512;      // ids the routing's grouping covers (E + 1 <= 257)

__device__ __forceinline__ double bits16_to_f64(uint32_t h, int bf16) {
    return bf16 ? (double)bf2f((uint16_t)h) : (double)h2f((uint16_t)h);
}

// order-preserving unsigned key of a bf16 value (held as the high half of an fp32): larger value, larger key
__device__ __forceinline__ uint32_t bf16_order(float v) {
    const uint32_t h = __builtin_bit_cast(uint32_t, v) >> 16;
    return (h & 0x8000u) ? (~h & 0xFFFFu) : (h | 0x8000u);
}
__device__ __forceinline__ float bf16_unorder(uint32_t k) {
    const uint32_t h = (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu);
    return __builtin_bit_cast(float, h << 16);
}

// One row's routing from its logits, by one wave: lr holds the E bf16-rounded router logits, then the shared gate's
// logit. The k largest (one order-preserving 32-bit key an expert: the logit's bf16 bits, then 0xFFFF - id, so ties go
// to the lowest id), their softmax weights (exponentials of the k maxima at once, the sum in pick order), and the
// shared slot's sigmoid weight. Lane t < k returns pick t; every lane returns the shared weight (when has). LOAD 0:
// plain loads; 1: device-coherent loads (the logits were stored by other workgroups of the same launch), a lane
// holding experts lane + 64 q; 2: as 1, with one 16-byte load a lane of experts 4 lane + q (E == 256, lr 16-byte
// aligned). Every load, the shared logit's too, is issued before any is used (one round trip). POLL: the logits
// were stored over the all-ones sentinel; each is reloaded (bounded, ~20 ms) until it is not all-ones, and `late` is
// set where a wait gave up (the caller raises its status bit).
constexpr uint32_t ROUTE_EMPTY = 0xFFFFFFFFu;     // the all-ones sentinel of esp_route_group_rmsnorm's logits

__device__ __forceinline__ bool route_late(uint64_t t0) {
    return __builtin_amdgcn_s_memrealtime() - t0 > 2000000ull;       // ~20 ms at 100 MHz
}

template <int LOAD, bool POLL = false>
__device__ __forceinline__ void topk_row(const float* lr, int E, int k, bool has, int lane, int& e_out, float& w_out,
                                         float& w_shared, bool& late) {
    auto expert = [lane](int q) __attribute__((always_inline)) { return LOAD == 2 ? 4 * lane + q : lane + 64 * q; };
    float l4[4];
    if constexpr (LOAD == 2) {
        const DevBuf lb(lr);
        float4 v = lb.load4(lr + 4 * lane);
        if constexpr (POLL) {
            // until the other workgroups' logits have landed: no word all-ones (bounded)
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            while (__float_as_uint(v.x) == ROUTE_EMPTY || __float_as_uint(v.y) == ROUTE_EMPTY ||
                   __float_as_uint(v.z) == ROUTE_EMPTY || __float_as_uint(v.w) == ROUTE_EMPTY) {
                __builtin_amdgcn_s_sleep(1);
                if (route_late(t0)) {
                    late = true;
                    break;
                }
                v = lb.load4(lr + 4 * lane);
            }
        }
        l4[0] = v.x; l4[1] = v.y; l4[2] = v.z; l4[3] = v.w;
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = expert(q);
            l4[q] = e < E ? (LOAD ? load_dev(lr + e) : lr[e]) : 0.f;
        }
        if constexpr (POLL) {
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
#pragma unroll
            for (int q = 0; q < 4; ++q)
                while (expert(q) < E && __float_as_uint(l4[q]) == ROUTE_EMPTY) {
                    __builtin_amdgcn_s_sleep(1);
                    if (route_late(t0)) {
                        late = true;
                        break;
                    }
                    l4[q] = load_dev(lr + expert(q));
                }
        }
    }
    float ls = has ? (LOAD ? load_dev(lr + E) : lr[E]) : 0.f;
    if constexpr (POLL) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (has && __float_as_uint(ls) == ROUTE_EMPTY) {
            __builtin_amdgcn_s_sleep(1);
            if (route_late(t0)) {
                late = true;
                break;
            }
            ls = load_dev(lr + E);
        }
    }
    uint32_t key[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = expert(q);
        key[q] = e < E ? (bf16_order(l4[q]) << 16) | (0xFFFFu - (uint32_t)e) : 0u;
    }
    float l_mine = 0.f;
    int e_mine = -1;
    for (int t = 0; t < k; ++t) {
        uint32_t m = key[0] > key[1] ? key[0] : key[1];
        const uint32_t m2 = key[2] > key[3] ? key[2] : key[3];
        m = m > m2 ? m : m2;
        m = wave_max_u32(m);
        const int e = (int)(0xFFFFu - (m & 0xFFFFu));
        if (lane == t) {
            e_mine = e;
            l_mine = bf16_unorder(m >> 16);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (expert(q) == e) key[q] = 0u;
    }
    const float mx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l_mine), 0));   // pick 0's
    const float p_mine = expf(l_mine - mx);
    float psum = 0.f;
    for (int t = 0; t < k; ++t)
        psum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p_mine), t));
    e_out = e_mine;
    w_out = p_mine / psum;
    w_shared = has ? 1.f / (1.f + expf(-ls)) : 0.f;
}


// A row's picks and tables by one wave (one row, a decode step), from its logits at `logits`: the top-k (topk_row), then
// the grouping in registers -- the ids of one row are distinct (top-k picks and the shared id), so a pick's place is
// the number of smaller ids and its member rank 0 -- with no shared-memory round trip or barrier (group_wave's
// tables). POLL: the logits were stored by other workgroups of the launch over the all-ones sentinel; wait (bounded)
// until none is all-ones, then put the all-ones back. Returns whether a wait gave up.
template <bool POLL>
__device__ __forceinline__ bool route_one_row(const RouteArgs& a, float* logits, int* pick_out, float* wts_out,
                                              int lane) {
    const int has = a.shared_id >= 0, C = a.E + has, slots = a.k + has;
    int e_mine;
    float w_mine, w_shared;
    bool late = false;
    const bool wide = a.E == 256 && ((uintptr_t)logits & 15) == 0;
    if (wide)
        topk_row<2, POLL>(logits, a.E, a.k, has, lane, e_mine, w_mine, w_shared, late);
    else
        topk_row<1, POLL>(logits, a.E, a.k, has, lane, e_mine, w_mine, w_shared, late);
    if constexpr (POLL) {
        // the logits are read: the sentinel back for the next launch
        const float e1 = __uint_as_float(ROUTE_EMPTY);
        if (wide) {
            DevBuf(logits).store4(logits + 4 * lane, make_float4(e1, e1, e1, e1));
        } else {
            for (int e = lane; e < a.E; e += 64) store_dev(logits + e, e1);
        }
        if (has && lane == 0) store_dev(logits + a.E, e1);
    }
    int id = -1;
    if (lane < a.k) {
        pick_out[lane] = e_mine;
        wts_out[lane] = w_mine;
        id = e_mine;
    }
    if (has && lane == a.k) {
        pick_out[a.k] = a.shared_id;
        wts_out[a.k] = w_shared;
        id = a.shared_id;
    }
    const bool valid = lane < slots && id >= 0 && id < C;
    int place = 0;
    for (int j = 0; j < slots; ++j) {
        const int ej = __builtin_amdgcn_readlane(id, j);
        place += ej >= 0 && ej < C && ej < id;
    }
    const uint64_t vm = __ballot(valid);
    if (lane == 0) *a.ucount = __builtin_popcountll(vm);
    if (valid) {
        a.uids[place] = id;
        a.members[(size_t)place * a.maxm] = lane;                            // row 0, slot lane
        for (int m = 1; m < a.maxm; ++m) a.members[(size_t)place * a.maxm + m] = -1;
    }
    return late;
}

// 8 consecutive 16-bit values of p from h (two 8-byte loads), zeros past H
__device__ __forceinline__ void route_load8(const uint16_t* p, int h, int H, uint2 (&v)[2]) {
    if (h < H) {
        v[0] = *reinterpret_cast<const uint2*>(p + h);
        v[1] = *reinterpret_cast<const uint2*>(p + h + 4);
    } else {
        v[0] = v[1] = make_uint2(0u, 0u);
    }
}

// a lane's share of a logit: its 4 chunks of 8 (x, gate) pairs, exact fp64 products added to acc in order
template <int BF16>
__device__ __forceinline__ double route_dot(const uint2 (&xv)[4][2], const uint2 (&gv)[4][2], double acc) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t gw[4] = {gv[q][0].x, gv[q][0].y, gv[q][1].x, gv[q][1].y};
        const uint32_t xw[4] = {xv[q][0].x, xv[q][0].y, xv[q][1].x, xv[q][1].y};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc = __builtin_fma(bits16_to_f64(xw[j] & 0xFFFFu, BF16), bits16_to_f64(gw[j] & 0xFFFFu, BF16), acc);
            acc = __builtin_fma(bits16_to_f64(xw[j] >> 16, BF16), bits16_to_f64(gw[j] >> 16, BF16), acc);
        }
    }
    return acc;
}

}  // namespace esp

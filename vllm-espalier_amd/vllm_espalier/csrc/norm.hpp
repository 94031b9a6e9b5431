// Residual add + RMSNorm of one row, in one fixed order shared by every kernel that computes it (add_rmsnorm, and the
// dense and routing launches that normalise their own input rows), so they all produce the same bits.
//
// A row is spread over 256 threads (t = 0..255, four waves): thread t holds elements (c * 256 + t) * 8 .. + 8 of the
// chunks c < NORM_CHUNKS. z = h + d1 + d2 in fp32 (each delta optional), rounded to the model dtype when a delta was
// added (the stored residual); the sum of squares runs over c, then the 8 elements, in each thread, then a DPP sum
// inside each wave, then ((w0 + w1) + w2) + w3; inv = 1 / sqrt(sum / D + eps); out = (z * inv) * w.
#pragma once

#include "common.hpp"

namespace esp {

constexpr int NORM_CHUNKS = 4;                  // D <= 8 * 256 * NORM_CHUNKS = 8192
constexpr int NORM_MAX_D = 8 * 256 * NORM_CHUNKS;

// fp32 sum across a wave through DPP, in every lane (the fixed order of wave_sum_f64_dpp, no LDS)
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, dpp_u32<CTRL, ROW_MASK>(__builtin_bit_cast(uint32_t, v), 0u));
}
__device__ __forceinline__ float wave_sum_f32(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    v += dpp_f32<0x142, 0xA>(v);
    v += dpp_f32<0x143, 0xC>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(uint32_t, v), 63));
}

__device__ __forceinline__ uint16_t to16(float v, bool bf) { return bf ? f2bf(v) : f2h(v); }
__device__ __forceinline__ float from16(uint16_t b, bool bf) { return bf ? bf2f(b) : h2f(b); }

__device__ __forceinline__ uint4 pack8_16(const float (&v)[8], bool bf) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (uint32_t)to16(v[2 * i], bf) | ((uint32_t)to16(v[2 * i + 1], bf) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// z of 8 elements from their raw h, d1, d2 (16-bit, 8 a uint4; a delta only when has1 / has2): h + d1 + d2 in fp32,
// rounded to the model dtype when a delta was added (the stored residual, exact). Returns z packed.
__device__ __forceinline__ uint4 norm_z8_of(uint4 uh, uint4 u1, uint4 u2, bool has1, bool has2, bool bf,
                                            float (&z)[8]) {
    auto unpack = [bf](uint4 u, float (&v)[8]) __attribute__((always_inline)) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[2 * k] = from16((uint16_t)(w[k] & 0xFFFFu), bf);
            v[2 * k + 1] = from16((uint16_t)(w[k] >> 16), bf);
        }
    };
    unpack(uh, z);
    if (has1) {
        float a[8];
        unpack(u1, a);
#pragma unroll
        for (int j = 0; j < 8; ++j) z[j] += a[j];
    }
    if (has2) {
        float b[8];
        unpack(u2, b);
#pragma unroll
        for (int j = 0; j < 8; ++j) z[j] += b[j];
    }
    if (has1 || has2) {
#pragma unroll
        for (int j = 0; j < 8; ++j) z[j] = from16(to16(z[j], bf), bf);     // the stored (rounded) residual
        return pack8_16(z, bf);
    }
    return uh;
}

// Thread t's chunks of row (h, d1, d2) (elements (c * 256 + t) * 8 .. + 8, c < NORM_CHUNKS, those below D): z packed
// in the model dtype (the stored residual, exact; h itself when no delta is added) and its share of the sum of squares.
// Every load is issued before any is used, so the three operands cost one memory round trip. `after` runs between the
// loads and their first use: loads it issues are queued behind the rows' (vector loads return in order).
struct NoLoads {
    __device__ __forceinline__ void operator()() const {}
};
template <typename F = NoLoads>
__device__ __forceinline__ float norm_z_rows(const uint16_t* h, const uint16_t* d1, const uint16_t* d2, int D, bool bf,
                                             int t, uint4 (&zq)[NORM_CHUNKS], const F& after = F{}) {
    const uint16_t* p1 = d1 ? d1 : h;             // a stand-in row keeps the loads free of the delta branches
    const uint16_t* p2 = d2 ? d2 : h;
    uint4 uh[NORM_CHUNKS], u1[NORM_CHUNKS], u2[NORM_CHUNKS];
#pragma unroll
    for (int c = 0; c < NORM_CHUNKS; ++c) {
        const int i = (c * 256 + t) * 8;
        uh[c] = u1[c] = u2[c] = make_uint4(0u, 0u, 0u, 0u);
        if (i < D) {
            uh[c] = *reinterpret_cast<const uint4*>(h + i);
            u1[c] = *reinterpret_cast<const uint4*>(p1 + i);
            u2[c] = *reinterpret_cast<const uint4*>(p2 + i);
        }
    }
    after();
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NORM_CHUNKS; ++c) {
        zq[c] = uh[c];
        if ((c * 256 + t) * 8 < D) {
            float z[8];
            zq[c] = norm_z8_of(uh[c], u1[c], u2[c], d1 != nullptr, d2 != nullptr, bf, z);
#pragma unroll
            for (int j = 0; j < 8; ++j) ss += z[j] * z[j];
        }
    }
    return ss;
}

// 1 / sqrt(mean + eps) from the four waves' sums
__device__ __forceinline__ float norm_inv(const float* part4, int D, float eps) {
    const float total = ((part4[0] + part4[1]) + part4[2]) + part4[3];
    return 1.0f / sqrtf(total / (float)D + eps);
}

// Rows r < R of a workgroup of at least 256 * R threads: waves 4r..4r+3 take row r (thread t = tid & 255). Every
// thread calls it (LDS_ONLY: its barriers wait only for shared-memory work, see lds_barrier); on return inv_sh[r] holds row r's scale and zq thread t's chunks of row r's z (norm_z_rows). With
// zs (shared memory), the z elements i in [lo, hi) of row r are also stored at zs[r * zs_stride + i - lo], visible to
// the whole workgroup on return (lo and hi multiples of 8). Two workgroup barriers inside. Row r of h / d1 / d2
// starts at r * stride.
// A workgroup barrier that waits only for this wave's shared-memory work (not for its global loads or LDS copies in
// flight, as __syncthreads' fence does): for exchanges through shared memory while trellis copies stream in.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <bool LDS_ONLY = false>
__device__ __forceinline__ void norm_rows_inv(const uint16_t* h, const uint16_t* d1, const uint16_t* d2, int stride,
                                              int R, int D, float eps, bool bf, float* part_sh, float* inv_sh,
                                              uint4 (&zq)[NORM_CHUNKS], uint16_t* zs = nullptr, int zs_stride = 0,
                                              int lo = 0, int hi = 0) {
    const int wave = threadIdx.x >> 6, r = wave >> 2, t = threadIdx.x & 255;
    if (r < R) {
        const size_t o = (size_t)r * stride;
        const float ss = wave_sum_f32(norm_z_rows(h + o, d1 ? d1 + o : nullptr, d2 ? d2 + o : nullptr, D, bf, t, zq));
        if ((threadIdx.x & 63) == 0) part_sh[wave] = ss;
        if (zs) {
#pragma unroll
            for (int c = 0; c < NORM_CHUNKS; ++c) {
                const int i = (c * 256 + t) * 8;
                if (i < D && i >= lo && i < hi) *reinterpret_cast<uint4*>(zs + (size_t)r * zs_stride + (i - lo)) = zq[c];
            }
        }
    }
    if constexpr (LDS_ONLY) lds_barrier(); else __syncthreads();
    if ((int)threadIdx.x < R) inv_sh[threadIdx.x] = norm_inv(part_sh + 4 * threadIdx.x, D, eps);
    if constexpr (LDS_ONLY) lds_barrier(); else __syncthreads();
}

// norm_rows_inv's scales for D = 2048 (one chunk a thread) and no second delta, with the caller's own loads issued
// behind the rows' (after, run by the rows' waves once). Inside the rows' waves every load is unconditional, so the
// compiler can wait for the rows alone (vmcnt counts what after issued): after's loads stay in flight while the rows
// are summed, and the two barriers wait only for shared-memory work. Same sums in the same order as norm_rows_inv.
template <typename F>
__device__ __forceinline__ void norm_rows_inv_2048(const uint16_t* h, const uint16_t* d1, int stride, int R, float eps,
                                                   bool bf, float* part_sh, float* inv_sh, uint4 (&zq)[NORM_CHUNKS],
                                                   const F& after) {
    const int wave = threadIdx.x >> 6, r = wave >> 2, t = threadIdx.x & 255;
#pragma unroll
    for (int c = 1; c < NORM_CHUNKS; ++c) zq[c] = make_uint4(0u, 0u, 0u, 0u);
    if (r < R) {
        const size_t o = (size_t)r * stride + (size_t)t * 8;
        // A missing delta is -0 in every element (h + -0 = h exactly, -0 included), so the sum is always formed and
        // the delta's load always issued before `after`'s (h stands in for its address); a load used only under
        // the delta's condition would be sunk behind them
        const uint16_t* p1 = d1 ? d1 : h;
        const uint4 uh = *reinterpret_cast<const uint4*>(h + o);
        const uint4 l1 = *reinterpret_cast<const uint4*>(p1 + o);
        const uint4 u1 = d1 ? l1 : make_uint4(0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u);
        after();
        float z[8];
        zq[0] = norm_z8_of(uh, u1, u1, true, false, bf, z);
        if (!d1) zq[0] = uh;                                  // the residual is h itself, bit for bit (NaNs too)
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += z[j] * z[j];
        ss = wave_sum_f32(ss);
        if ((threadIdx.x & 63) == 0) part_sh[wave] = ss;
    }
    lds_barrier();
    if ((int)threadIdx.x < R) inv_sh[threadIdx.x] = norm_inv(part_sh + 4 * threadIdx.x, 2048, eps);
    lds_barrier();
}

// norm_rows_inv's scales (no zs) with the caller's own loads issued behind the rows' (after, run by every thread once):
// they stay in flight through the two barriers, which wait only for shared-memory work
template <typename F>
__device__ __forceinline__ void norm_rows_inv_then(const uint16_t* h, const uint16_t* d1, const uint16_t* d2,
                                                   int stride, int R, int D, float eps, bool bf, float* part_sh,
                                                   float* inv_sh, uint4 (&zq)[NORM_CHUNKS], const F& after) {
    const int wave = threadIdx.x >> 6, r = wave >> 2, t = threadIdx.x & 255;
    if (r < R) {
        const size_t o = (size_t)r * stride;
        const float ss =
            wave_sum_f32(norm_z_rows(h + o, d1 ? d1 + o : nullptr, d2 ? d2 + o : nullptr, D, bf, t, zq, after));
        if ((threadIdx.x & 63) == 0) part_sh[wave] = ss;
    } else {
        after();
    }
    lds_barrier();
    if ((int)threadIdx.x < R) inv_sh[threadIdx.x] = norm_inv(part_sh + 4 * threadIdx.x, D, eps);
    lds_barrier();
}

// thread t's chunks of its row (norm_rows_inv's zq) stored at row (o = r * stride) of out
__device__ __forceinline__ void norm_rows_store(const uint4 (&zq)[NORM_CHUNKS], int R, int D, size_t stride,
                                                uint16_t* out) {
    const int r = (int)(threadIdx.x >> 8), t = threadIdx.x & 255;
    if (r >= R) return;
#pragma unroll
    for (int c = 0; c < NORM_CHUNKS; ++c) {
        const int i = (c * 256 + t) * 8;
        if (i < D) *reinterpret_cast<uint4*>(out + (size_t)r * stride + i) = zq[c];
    }
}

// (z * inv) * w of 8 packed elements, packed in the model dtype
__device__ __forceinline__ uint4 norm_scale8(uint4 zq, uint4 wq, float inv, bool bf) {
    const uint32_t zw[4] = {zq.x, zq.y, zq.z, zq.w}, ww[4] = {wq.x, wq.y, wq.z, wq.w};
    float o8[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        o8[2 * k] = (from16((uint16_t)(zw[k] & 0xFFFFu), bf) * inv) * from16((uint16_t)(ww[k] & 0xFFFFu), bf);
        o8[2 * k + 1] = (from16((uint16_t)(zw[k] >> 16), bf) * inv) * from16((uint16_t)(ww[k] >> 16), bf);
    }
    return pack8_16(o8, bf);
}

// the rotation's input (RotIn, 16-bit raw) of 4 elements from their z (packed), norm weights w and signs su:
// (z * inv) * w in the model dtype
__device__ __forceinline__ RotIn norm_rot_in(uint2 zq, uint2 wq, uint2 su, float inv, bool bf) {
    const uint32_t zw[2] = {zq.x, zq.y}, ww[2] = {wq.x, wq.y};
    uint32_t q[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const uint16_t lo = to16((from16((uint16_t)(zw[k] & 0xFFFFu), bf) * inv) * from16((uint16_t)(ww[k] & 0xFFFFu), bf), bf);
        const uint16_t hi = to16((from16((uint16_t)(zw[k] >> 16), bf) * inv) * from16((uint16_t)(ww[k] >> 16), bf), bf);
        q[k] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    RotIn r;
    r.raw = make_uint4(q[0], q[1], 0u, 0u);
    r.su = su;
    return r;
}

}  // namespace esp

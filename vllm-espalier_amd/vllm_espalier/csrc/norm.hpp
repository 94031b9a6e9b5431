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

// 8 consecutive 16-bit elements (bf16 or fp16) as fp32
__device__ __forceinline__ void load8_16(const uint16_t* p, bool bf, float (&v)[8]) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint16_t lo = (uint16_t)(w[i] & 0xFFFFu), hi = (uint16_t)(w[i] >> 16);
        v[2 * i] = bf ? bf2f(lo) : h2f(lo);
        v[2 * i + 1] = bf ? bf2f(hi) : h2f(hi);
    }
}

__device__ __forceinline__ uint16_t to16(float v, bool bf) { return bf ? f2bf(v) : f2h(v); }
__device__ __forceinline__ float from16(uint16_t b, bool bf) { return bf ? bf2f(b) : h2f(b); }

__device__ __forceinline__ uint4 pack8_16(const float (&v)[8], bool bf) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (uint32_t)to16(v[2 * i], bf) | ((uint32_t)to16(v[2 * i + 1], bf) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// z of the 8 elements at offset o (a multiple of 8) of a row
__device__ __forceinline__ void norm_z8(const uint16_t* h, const uint16_t* d1, const uint16_t* d2, size_t o, bool bf,
                                        float (&z)[8]) {
    load8_16(h + o, bf, z);
    if (d1) {
        float a[8];
        load8_16(d1 + o, bf, a);
#pragma unroll
        for (int j = 0; j < 8; ++j) z[j] += a[j];
    }
    if (d2) {
        float b[8];
        load8_16(d2 + o, bf, b);
#pragma unroll
        for (int j = 0; j < 8; ++j) z[j] += b[j];
    }
    if (d1 || d2) {
#pragma unroll
        for (int j = 0; j < 8; ++j) z[j] = from16(to16(z[j], bf), bf);     // the stored (rounded) residual
    }
}

// z of the 4 elements at offset o (a multiple of 4) of a row: the same arithmetic as norm_z8
__device__ __forceinline__ void norm_z4(const uint16_t* h, const uint16_t* d1, const uint16_t* d2, size_t o, bool bf,
                                        float (&z)[4]) {
    auto load4 = [&](const uint16_t* p, float (&v)[4]) {
        const uint2 u = *reinterpret_cast<const uint2*>(p + o);
        v[0] = from16((uint16_t)(u.x & 0xFFFFu), bf); v[1] = from16((uint16_t)(u.x >> 16), bf);
        v[2] = from16((uint16_t)(u.y & 0xFFFFu), bf); v[3] = from16((uint16_t)(u.y >> 16), bf);
    };
    load4(h, z);
    if (d1) {
        float a[4];
        load4(d1, a);
#pragma unroll
        for (int j = 0; j < 4; ++j) z[j] += a[j];
    }
    if (d2) {
        float b[4];
        load4(d2, b);
#pragma unroll
        for (int j = 0; j < 4; ++j) z[j] += b[j];
    }
    if (d1 || d2) {
#pragma unroll
        for (int j = 0; j < 4; ++j) z[j] = from16(to16(z[j], bf), bf);
    }
}

// the rotation's input (RotIn, 16-bit raw) of lane32's 4 elements at row offset o + 4 * lane32, normalised:
// (z * inv) * w in the model dtype; w holds the norm weights from the same column, suh the sign vector's
__device__ __forceinline__ RotIn norm_rot_load(const uint16_t* h, const uint16_t* d1, const uint16_t* d2,
                                               const uint16_t* w, size_t o, float inv, bool bf, const uint16_t* suh,
                                               int lane32) {
    float z[4];
    norm_z4(h, d1, d2, o + 4 * lane32, bf, z);
    const uint2 wu = *reinterpret_cast<const uint2*>(w + 4 * lane32);
    const float wv[4] = {from16((uint16_t)(wu.x & 0xFFFFu), bf), from16((uint16_t)(wu.x >> 16), bf),
                         from16((uint16_t)(wu.y & 0xFFFFu), bf), from16((uint16_t)(wu.y >> 16), bf)};
    uint16_t q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = to16((z[j] * inv) * wv[j], bf);
    RotIn r;
    r.raw = make_uint4((uint32_t)q[0] | ((uint32_t)q[1] << 16), (uint32_t)q[2] | ((uint32_t)q[3] << 16), 0u, 0u);
    r.su = *reinterpret_cast<const uint2*>(suh + 4 * lane32);
    return r;
}

// thread t's share of the sum of squares of row (h, d1, d2)
__device__ __forceinline__ float norm_partial(const uint16_t* h, const uint16_t* d1, const uint16_t* d2, int D,
                                              bool bf, int t) {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NORM_CHUNKS; ++c) {
        const int i = (c * 256 + t) * 8;
        if (i < D) {
            float z[8];
            norm_z8(h, d1, d2, i, bf, z);
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

// The residual rows of a workgroup's norm_rows_inv (waves 4r..4r+3 on row r < R) stored to out (the same stride)
__device__ __forceinline__ void norm_rows_store(const uint16_t* h, const uint16_t* d1, const uint16_t* d2, int stride,
                                                int R, int D, bool bf, uint16_t* out) {
    const int r = (int)(threadIdx.x >> 8), t = threadIdx.x & 255;
    if (r >= R) return;
    const size_t o = (size_t)r * stride;
#pragma unroll
    for (int c = 0; c < NORM_CHUNKS; ++c) {
        const int i = (c * 256 + t) * 8;
        if (i < D) {
            float z[8];
            norm_z8(h + o, d1 ? d1 + o : nullptr, d2 ? d2 + o : nullptr, i, bf, z);
            *reinterpret_cast<uint4*>(out + o + i) = pack8_16(z, bf);
        }
    }
}

// Rows r < R of a workgroup of at least 256 * R threads: waves 4r..4r+3 take row r. Every thread calls it; on return
// inv_sh[r] holds row r's scale (two workgroup barriers inside). Row r of h / d1 / d2 starts at r * stride.
__device__ __forceinline__ void norm_rows_inv(const uint16_t* h, const uint16_t* d1, const uint16_t* d2, int stride,
                                              int R, int D, float eps, bool bf, float* part_sh, float* inv_sh) {
    const int wave = threadIdx.x >> 6, r = wave >> 2, t = threadIdx.x & 255;
    if (r < R) {
        const size_t o = (size_t)r * stride;
        const float ss = wave_sum_f32(norm_partial(h + o, d1 ? d1 + o : nullptr, d2 ? d2 + o : nullptr, D, bf, t));
        if ((threadIdx.x & 63) == 0) part_sh[wave] = ss;
    }
    __syncthreads();
    if ((int)threadIdx.x < R) inv_sh[threadIdx.x] = norm_inv(part_sh + 4 * threadIdx.x, D, eps);
    __syncthreads();
}

}  // namespace esp

// Shared device helpers of the gfx950 kernel layer: fp16/bf16 conversions, wave64 lane exchanges, the 128-point
// Walsh-Hadamard transform, and the C-ABI error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

namespace esp {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 1 / sqrt(128), the reference's constant (dense.cu:23, experts.cu:17)
constexpr float HAD_SCALE = 0.08838834764831845f;

enum DType : int { F16 = 0, BF16 = 1, F32 = 2 };

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// fp32 -> fp16, RNE, of f as an fp32 value: the empty asm keeps the compiler from folding the operation that made f
// into the conversion (a product would become one v_fma_mixlo_f16, rounded once to fp16, where the reference rounds
// to fp32 first and then to fp16)
__device__ __forceinline__ uint16_t f2h(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float bf2f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {                                                      // RNE
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// one element of a 16-bit (f16 / bf16) or f32 array as f32
__device__ __forceinline__ float load_elem(const void* p, int dtype, size_t i) {
    if (dtype == F32) return static_cast<const float*>(p)[i];
    const uint16_t h = static_cast<const uint16_t*>(p)[i];
    return dtype == BF16 ? bf2f(h) : h2f(h);
}

// four consecutive elements starting at i (i a multiple of 4)
__device__ __forceinline__ void load4(const void* p, int dtype, size_t i, float (&v)[4]) {
    if (dtype == F32) {
        const float4 u = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
        v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
    } else {
        const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
        const uint16_t h[4] = {(uint16_t)(u.x & 0xFFFFu), (uint16_t)(u.x >> 16), (uint16_t)(u.y & 0xFFFFu),
                               (uint16_t)(u.y >> 16)};
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = dtype == BF16 ? bf2f(h[j]) : h2f(h[j]);
    }
}

__device__ __forceinline__ void store4(void* p, int dtype, size_t i, const float (&v)[4]) {
    if (dtype == F32) {
        *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
        uint16_t h[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = dtype == BF16 ? f2bf(v[j]) : f2h(v[j]);
        uint2 u;
        u.x = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
        u.y = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i) = u;
    }
}

// lane ^ M inside each 32-lane half of the wave: quad DPP for 1 and 2, ds_swizzle's bitmask mode above. (An all-VALU
// form -- quad_perm + row_half_mirror for 4, row_ror:8, v_permlane16_swap for 16 -- was measured on MI355X: no faster
// where a rotation is latency-bound, 1.3 % slower on 32-row dense blocks, where the extra VALU work competes.)
template <int M>
__device__ __forceinline__ float xor_lane32(float v) {
    int i = __builtin_bit_cast(int, v);
    if constexpr (M == 1)
        i = __builtin_amdgcn_update_dpp(0, i, 0xB1, 0xF, 0xF, false);     // quad_perm [1,0,3,2]
    else if constexpr (M == 2)
        i = __builtin_amdgcn_update_dpp(0, i, 0x4E, 0xF, 0xF, false);     // quad_perm [2,3,0,1]
    else
        i = __builtin_amdgcn_ds_swizzle(i, (M << 10) | 0x1F);             // and 0x1F, or 0, xor M
    return __builtin_bit_cast(float, i);
}

template <int M>
__device__ __forceinline__ void fwht_stage(float (&v)[4], int lane32) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float o = xor_lane32<M>(v[j]);
        v[j] = (lane32 & M) ? o - v[j] : v[j] + o;
    }
}

// Walsh-Hadamard transform of 128 fp32 values held 4 a lane by 32 lanes (lane l: elements 4l..4l+3). Strides 1 and 2
// in registers, then 4..64 across lanes; the lower element of each pair takes a + b, the upper a - b. The stage order
// is the reference's (experts.cu:79-90), so the fp32 results are the same bits.
__device__ __forceinline__ void fwht128(float (&v)[4], int lane32) {
    const float a = v[0] + v[1], b = v[0] - v[1], c = v[2] + v[3], d = v[2] - v[3];
    v[0] = a + c; v[1] = b + d; v[2] = a - c; v[3] = b - d;
    fwht_stage<1>(v, lane32);
    fwht_stage<2>(v, lane32);
    fwht_stage<4>(v, lane32);
    fwht_stage<8>(v, lane32);
    fwht_stage<16>(v, lane32);
}

// ---- wave64 reductions through DPP (no LDS round trips) ----
// The total lands in lane 63: pairs and quads (quad_perm), 8-lane halves (row_half_mirror), 16-lane rows
// (row_mirror), then rows 1 and 3 take row 0 and 2's totals (row_bcast:15) and row 3 takes rows 0-1's
// (row_bcast:31). Lanes outside a step's row mask add the identity (the `old` operand).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v, uint32_t identity) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)v, CTRL, ROW_MASK, 0xF, false);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = dpp_u32<CTRL, ROW_MASK>((uint32_t)u, 0u), hi = dpp_u32<CTRL, ROW_MASK>((uint32_t)(u >> 32), 0u);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);    // +0.0 where the row mask excludes the lane
}

// the wave's sum, in every lane (fp64: exact whenever the partial sums are, whatever the order)
__device__ __forceinline__ double wave_sum_f64_dpp(double v) {
    v += dpp_f64<0xB1>(v);            // quad_perm [1,0,3,2]
    v += dpp_f64<0x4E>(v);            // quad_perm [2,3,0,1]
    v += dpp_f64<0x141>(v);           // row_half_mirror
    v += dpp_f64<0x140>(v);           // row_mirror
    v += dpp_f64<0x142, 0xA>(v);      // row_bcast:15 into rows 1, 3
    v += dpp_f64<0x143, 0xC>(v);      // row_bcast:31 into rows 2, 3
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)u, 63), hi = __builtin_amdgcn_readlane((uint32_t)(u >> 32), 63);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// the wave's maximum (unsigned), in every lane
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    uint32_t o;
    o = dpp_u32<0xB1>(v, 0u);       v = v > o ? v : o;
    o = dpp_u32<0x4E>(v, 0u);       v = v > o ? v : o;
    o = dpp_u32<0x141>(v, 0u);      v = v > o ? v : o;
    o = dpp_u32<0x140>(v, 0u);      v = v > o ? v : o;
    o = dpp_u32<0x142, 0xA>(v, 0u); v = v > o ? v : o;
    o = dpp_u32<0x143, 0xC>(v, 0u); v = v > o ? v : o;
    return __builtin_amdgcn_readlane(v, 63);
}

// fp16 H(x * suh) / sqrt(128) of the 128 values of x starting at xi (dtype), 4 a lane of a 32-lane half; the multiply
// is never contracted into the butterfly (dense.cu:92-108). Split into the loads (RotIn) and the arithmetic, so a
// caller can put the loads in flight before other memory work.
struct RotIn {
    uint4 raw;       // the 4 elements' bits: 4 floats, or 4 halves in raw.x, raw.y
    uint2 su;
};

__device__ __forceinline__ RotIn rot128_load(const void* x, int x_dtype, size_t xi, const uint16_t* suh, int lane32) {
    RotIn r;
    if (x_dtype == F32) {
        r.raw = *reinterpret_cast<const uint4*>(static_cast<const float*>(x) + xi + 4 * lane32);
    } else {
        const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(x) + xi + 4 * lane32);
        r.raw = make_uint4(u.x, u.y, 0u, 0u);
    }
    r.su = *reinterpret_cast<const uint2*>(suh + 4 * lane32);
    return r;
}

__device__ __forceinline__ uint2 rot128_apply(RotIn r, int x_dtype, int lane32) {
    float v[4];
    if (x_dtype == F32) {
        v[0] = __builtin_bit_cast(float, r.raw.x); v[1] = __builtin_bit_cast(float, r.raw.y);
        v[2] = __builtin_bit_cast(float, r.raw.z); v[3] = __builtin_bit_cast(float, r.raw.w);
    } else {
        const uint16_t h[4] = {(uint16_t)(r.raw.x & 0xFFFFu), (uint16_t)(r.raw.x >> 16), (uint16_t)(r.raw.y & 0xFFFFu),
                               (uint16_t)(r.raw.y >> 16)};
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = x_dtype == BF16 ? bf2f(h[j]) : h2f(h[j]);
    }
    v[0] = __fmul_rn(v[0], h2f((uint16_t)(r.su.x & 0xFFFFu)));
    v[1] = __fmul_rn(v[1], h2f((uint16_t)(r.su.x >> 16)));
    v[2] = __fmul_rn(v[2], h2f((uint16_t)(r.su.y & 0xFFFFu)));
    v[3] = __fmul_rn(v[3], h2f((uint16_t)(r.su.y >> 16)));
    fwht128(v, lane32);
    uint2 u;
    u.x = (uint32_t)f2h(v[0] * HAD_SCALE) | ((uint32_t)f2h(v[1] * HAD_SCALE) << 16);
    u.y = (uint32_t)f2h(v[2] * HAD_SCALE) | ((uint32_t)f2h(v[3] * HAD_SCALE) << 16);
    return u;
}

__device__ __forceinline__ uint2 rot128(const void* x, int x_dtype, size_t xi, const uint16_t* suh, int lane32) {
    return rot128_apply(rot128_load(x, x_dtype, xi, suh, lane32), x_dtype, lane32);
}

// ---- hand-off of partial results between workgroups ----
// MI355X's eight XCDs each have their own L2, so an agent-scope release fence writes back the whole L2 (buffer_wbl2):
// ~100 ns a fence, serialised per XCD, which at thousands of waves a launch costs more than the GEMM. Partials
// instead travel with device-scope (sc1) stores and loads, which are coherent across XCDs by themselves: a workgroup
// stores its partials with store_dev, arrive_last drains its stores (s_waitcnt) before one relaxed device-scope count,
// and the last workgroup to arrive reads every partial back with load_dev.
__device__ __forceinline__ void store_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int load_dev(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long load_dev(const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Device-scope 16-byte accesses: one buffer_load / buffer_store_dwordx4 with cache policy sc1 (coherent across the
// XCDs' L2s, as the agent-scope atomics above are), so a 32-lane half moves whole 128-byte lines. The buffer resource
// covers 4 GiB from base, which every lane shares; each lane's address goes in as its byte offset from base.
constexpr int CPOL_SC1 = 16;                    // the cache-policy operand's sc1 bit (gfx94x / gfx950)
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
struct DevBuf {
    __amdgpu_buffer_rsrc_t r;
    const char* b;
    __device__ __forceinline__ explicit DevBuf(const void* base)
        : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, 0x00020000)),
          b(static_cast<const char*>(base)) {}
    __device__ __forceinline__ uint32_t off(const float* p) const {
        return (uint32_t)(reinterpret_cast<const char*>(p) - b);
    }
    __device__ __forceinline__ float4 load4(const float* p) const {
        const u32x4v v = __builtin_amdgcn_raw_buffer_load_b128(r, off(p), 0, CPOL_SC1);
        return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
    }
    __device__ __forceinline__ void store4(float* p, const float4& v) const {
        const u32x4v u = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
        __builtin_amdgcn_raw_buffer_store_b128(u, r, off(p), 0, CPOL_SC1);
    }
};

constexpr int CNT_STRIDE = 32;   // ints between two arrival counters: one 128-byte line each, so workgroups arriving
                                 // on different counters never queue on one line's atomics

// True in every thread of the last of `total` workgroups to call it on `counter` (the count is left at total; the
// last workgroup resets it with store_dev once it has read the partials). Every thread of the workgroup calls it.
__device__ __forceinline__ bool arrive_last(int* counter, int total, int* sh_flag) {
    __builtin_amdgcn_s_waitcnt(0);          // this wave's device-scope stores have completed
    __syncthreads();
    if (threadIdx.x == 0)
        *sh_flag = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1;
    __syncthreads();
    return *sh_flag != 0;
}

}  // namespace esp

// ---- C-ABI error plumbing (host) ----
namespace esp_host {
const char* last_error();
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int ok();
int launch_check(const char* what);
int dense_status(int clear, hipStream_t st, int* out);     // dense_multi.hip: the dense launches' status word
int tile_status(int clear, hipStream_t st, int* out);      // dense_tile.hip: the prompt launches' status word
int dense_own_status(int clear, hipStream_t st, int* out); // dense.hip: esp_dense_own's status word
}  // namespace esp_host

#define ESP_REQUIRE(cond, ...)                                                                  \
    do {                                                                                        \
        if (!(cond)) return esp_host::fail(ESP_ERR_ARG, __VA_ARGS__);                           \
    } while (0)

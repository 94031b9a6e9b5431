// Decode-step glue for the synthetic decoder step around the trellis layers, on gfx950: the token embedding gather,
// the residual add fused with RMSNorm, and the greedy argmax over the logits. In a served model vLLM provides these
// (VocabParallelEmbedding, fused_add_rms_norm, the sampler); the step that measures whole-model decode tok/s on
// synthetic weights needs them on the device so one HIP graph holds the step and the next token never leaves HBM.
//
// Every reduction runs in a fixed order (lane slices, then DPP inside a wave, then the waves in index order), so a
// row's result depends on that row alone.
#include "../../../include/espalier.h"
#include "common.hpp"
#include "norm.hpp"

namespace esp {

// ------------------------------------------------------------------------------------------------------------------
// embed: h[t] = table[ids[t]] (ids outside [0, vocab) give a zero row). One workgroup a row, 16 bytes a lane.
// ------------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* __restrict__ ids, const uint16_t* __restrict__ table,
                                                    int64_t vocab, uint16_t* __restrict__ h, int D) {
    const int t = blockIdx.x;
    const int64_t id = ids[t];
    const bool valid = id >= 0 && id < vocab;
    for (int i = threadIdx.x * 8; i < D; i += blockDim.x * 8) {
        uint4 u = make_uint4(0u, 0u, 0u, 0u);
        if (valid) u = *reinterpret_cast<const uint4*>(table + id * D + i);
        *reinterpret_cast<uint4*>(h + (size_t)t * D + i) = u;
    }
}

// ------------------------------------------------------------------------------------------------------------------
// add_rmsnorm: h = z (the residual, rounded), out = (z * inv) * w, in norm.hpp's order. One workgroup of 256 a row.
// ------------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(uint16_t* __restrict__ h, const uint16_t* __restrict__ d1,
                                                          const uint16_t* __restrict__ d2,
                                                          const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
                                                          int D, float eps, int bf) {
    __shared__ float part[4], inv_sh[1];
    const int t = threadIdx.x;
    const size_t o = (size_t)blockIdx.x * D;
    uint4 wq[NORM_CHUNKS];
#pragma unroll
    for (int c = 0; c < NORM_CHUNKS; ++c) {                 // the weights first: in flight with the rows
        const int i = (c * 256 + t) * 8;
        wq[c] = make_uint4(0u, 0u, 0u, 0u);
        if (i < D) wq[c] = *reinterpret_cast<const uint4*>(w + i);
    }
    uint4 zq[NORM_CHUNKS];
    // every read of h is done before h is written
    norm_rows_inv(h + o, d1 ? d1 + o : nullptr, d2 ? d2 + o : nullptr, D, 1, D, eps, bf, part, inv_sh, zq);
    const float inv = inv_sh[0];
#pragma unroll
    for (int c = 0; c < NORM_CHUNKS; ++c) {
        const int i = (c * 256 + t) * 8;
        if (i < D) {
            if (d1 || d2) *reinterpret_cast<uint4*>(h + o + i) = zq[c];
            *reinterpret_cast<uint4*>(out + o + i) = norm_scale8(zq[c], wq[c], inv, bf);
        }
    }
}

// ------------------------------------------------------------------------------------------------------------------
// argmax: ids[t] = the index of the largest logit of row t, the lowest index among equal ones (torch.argmax);
// a NaN counts as the largest. Keys: the value's bits made order-preserving, above the complemented index.
// ------------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t order16(uint16_t b) { return (b & 0x8000u) ? (uint32_t)(~b & 0xFFFFu) : (b | 0x8000u); }

__device__ __forceinline__ uint64_t key_of(uint16_t b, bool bf, int idx) {
    uint32_t k;
    if (bf) {
        const bool nan = (b & 0x7FFFu) > 0x7F80u;
        k = nan ? 0xFFFFu : order16(b);
    } else {
        const bool nan = (b & 0x7FFFu) > 0x7C00u;
        k = nan ? 0xFFFFu : order16(b);
    }
    return ((uint64_t)k << 32) | (uint32_t)(~(uint32_t)idx);
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

constexpr int ARGMAX_BATCH = 8;

__global__ __launch_bounds__(1024) void argmax_kernel(const uint16_t* __restrict__ logits, int64_t stride, int N,
                                                      int bf, int32_t* __restrict__ ids) {
    __shared__ uint64_t part[16];
    const int t = blockIdx.x;
    const uint16_t* row = logits + (size_t)t * stride;
    uint64_t best = 0;
    const int nv = N & ~7;
    const int step = (int)blockDim.x * 8;
    for (int i0 = threadIdx.x * 8; i0 < nv; i0 += ARGMAX_BATCH * step) {
        uint4 u[ARGMAX_BATCH];                                 // a batch of 16-byte loads in flight at once
#pragma unroll
        for (int b = 0; b < ARGMAX_BATCH; ++b)
            if (i0 + b * step < nv) u[b] = *reinterpret_cast<const uint4*>(row + i0 + b * step);
#pragma unroll
        for (int b = 0; b < ARGMAX_BATCH; ++b) {
            const int i = i0 + b * step;
            if (i >= nv) break;
            const uint32_t w[4] = {u[b].x, u[b].y, u[b].z, u[b].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                best = umax64(best, key_of((uint16_t)(w[j] & 0xFFFFu), bf, i + 2 * j));
                best = umax64(best, key_of((uint16_t)(w[j] >> 16), bf, i + 2 * j + 1));
            }
        }
    }
    for (int i = nv + (int)threadIdx.x; i < N; i += blockDim.x) best = umax64(best, key_of(row[i], bf, i));
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)best, m), hi = (uint32_t)__shfl_xor((int)(best >> 32), m);
        best = umax64(best, ((uint64_t)hi << 32) | lo);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) part[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = part[0];
        for (int q = 1; q < (int)(blockDim.x >> 6); ++q) b = umax64(b, part[q]);
        ids[t] = (int32_t)~(uint32_t)b;
    }
}

}  // namespace esp

// ======================================================================================================================
// C ABI
// ======================================================================================================================
using namespace esp;

extern "C" int esp_embed(const int32_t* ids, const void* table, int64_t vocab, void* h, int64_t T, int64_t D,
                         void* stream) {
    ESP_REQUIRE(ids && table && h, "embed: null pointer");
    ESP_REQUIRE(D > 0 && D % 8 == 0 && vocab > 0, "embed: D must be a positive multiple of 8");
    ESP_REQUIRE(((uintptr_t)table | (uintptr_t)h) % 16 == 0, "embed: table and h must be 16-byte aligned");
    if (T <= 0) return esp_host::ok();
    embed_kernel<<<(unsigned)T, 256, 0, (hipStream_t)stream>>>(ids, static_cast<const uint16_t*>(table), vocab,
                                                                static_cast<uint16_t*>(h), (int)D);
    return esp_host::launch_check("embed");
}

extern "C" int esp_add_rmsnorm(void* h, const void* d1, const void* d2, const void* w, void* out, int64_t T,
                               int64_t D, double eps, int dtype, void* stream) {
    ESP_REQUIRE(h && w && out, "add_rmsnorm: null pointer");
    ESP_REQUIRE(dtype == ESP_BF16 || dtype == ESP_F16, "add_rmsnorm: dtype must be bf16 or fp16");
    ESP_REQUIRE(D > 0 && D % 8 == 0 && D <= NORM_MAX_D, "add_rmsnorm: D must be a positive multiple of 8, at most %d",
                NORM_MAX_D);
    ESP_REQUIRE(((uintptr_t)h | (uintptr_t)d1 | (uintptr_t)d2 | (uintptr_t)w | (uintptr_t)out) % 16 == 0,
                "add_rmsnorm: every tensor must be 16-byte aligned");
    if (T <= 0) return esp_host::ok();
    add_rmsnorm_kernel<<<(unsigned)T, 256, 0, (hipStream_t)stream>>>(
        static_cast<uint16_t*>(h), static_cast<const uint16_t*>(d1), static_cast<const uint16_t*>(d2),
        static_cast<const uint16_t*>(w), static_cast<uint16_t*>(out), (int)D, (float)eps, dtype == ESP_BF16);
    return esp_host::launch_check("add_rmsnorm");
}

extern "C" int esp_argmax(const void* logits, int64_t stride, int64_t T, int64_t N, int dtype, int32_t* ids,
                          void* stream) {
    ESP_REQUIRE(logits && ids, "argmax: null pointer");
    ESP_REQUIRE(dtype == ESP_BF16 || dtype == ESP_F16, "argmax: dtype must be bf16 or fp16");
    ESP_REQUIRE(N > 0 && N < (1ll << 31) && stride >= N, "argmax: need 0 < N < 2^31 and stride >= N");
    ESP_REQUIRE((uintptr_t)logits % 16 == 0 && stride % 8 == 0, "argmax: rows must be 16-byte aligned");
    if (T <= 0) return esp_host::ok();
    argmax_kernel<<<(unsigned)T, 1024, 0, (hipStream_t)stream>>>(static_cast<const uint16_t*>(logits), stride,
                                                                  (int)N, dtype == ESP_BF16, ids);
    return esp_host::launch_check("argmax");
}

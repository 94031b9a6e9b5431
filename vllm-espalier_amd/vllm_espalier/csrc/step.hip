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

// The maximum key of a workgroup of 256 threads (4 waves), in thread 0
__device__ __forceinline__ uint64_t block_max_key256(uint64_t best, uint64_t* sh) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)best, m), hi = (uint32_t)__shfl_xor((int)(best >> 32), m);
        best = umax64(best, ((uint64_t)hi << 32) | lo);
    }
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = best;
    __syncthreads();
    return umax64(umax64(sh[0], sh[1]), umax64(sh[2], sh[3]));
}

// argmax over many workgroups: workgroup (b, t) takes slice b of row t (SL elements, a multiple of 8, at most 4096:
// two 16-byte loads a thread, both in flight), its largest key goes to part[t * NB + b], and the last of the NB to
// arrive on counter t takes the largest of the NB keys. The keys are argmax_kernel's, so the result is the same.
constexpr int ARGMAX_SLICE = 4096;
constexpr int ARGMAX_MAX_SLICES = 1024;

__global__ __launch_bounds__(256) void argmax_split_kernel(const uint16_t* __restrict__ logits, int64_t stride, int N,
                                                           int SL, int bf, unsigned long long* __restrict__ part,
                                                           int* __restrict__ counters, int32_t* __restrict__ ids) {
    __shared__ uint64_t sh[4];
    __shared__ int last;
    const int b = blockIdx.x, t = blockIdx.y, NB = gridDim.x, tid = threadIdx.x;
    const uint16_t* row = logits + (size_t)t * stride;
    const int s0 = b * SL, s1 = max(s0, min(N, s0 + SL));  // a slice past N is empty
    const int nv = s0 + ((s1 - s0) & ~7);                  // the slice's whole 8-element groups end here
    uint64_t best = 0;
    uint4 u[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = s0 + 8 * (tid + 256 * j);
        if (i < nv) u[j] = *reinterpret_cast<const uint4*>(row + i);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = s0 + 8 * (tid + 256 * j);
        if (i < nv) {
            const uint32_t w[4] = {u[j].x, u[j].y, u[j].z, u[j].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                best = umax64(best, key_of((uint16_t)(w[q] & 0xFFFFu), bf, i + 2 * q));
                best = umax64(best, key_of((uint16_t)(w[q] >> 16), bf, i + 2 * q + 1));
            }
        }
    }
    for (int i = nv + tid; i < s1; i += 256) best = umax64(best, key_of(row[i], bf, i));
    best = block_max_key256(best, sh);
    if (tid == 0) store_dev(part + (size_t)t * NB + b, (unsigned long long)best);
    int* cnt = counters + (size_t)t * CNT_STRIDE;
    if (!arrive_last(cnt, NB, &last)) return;
    __syncthreads();                                        // sh is reused below
    uint64_t k = 0;
    for (int q = tid; q < NB; q += 256) k = umax64(k, load_dev(part + (size_t)t * NB + q));
    k = block_max_key256(k, sh);
    if (tid == 0) {
        ids[t] = (int32_t)~(uint32_t)k;
        store_dev(cnt, 0);                                  // every slice of the row arrived
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
                          int64_t* part, int64_t part_numel, int32_t* counters, int64_t counters_numel, void* stream) {
    ESP_REQUIRE(logits && ids, "argmax: null pointer");
    ESP_REQUIRE(dtype == ESP_BF16 || dtype == ESP_F16, "argmax: dtype must be bf16 or fp16");
    ESP_REQUIRE(N > 0 && N < (1ll << 31) && stride >= N, "argmax: need 0 < N < 2^31 and stride >= N");
    ESP_REQUIRE((uintptr_t)logits % 16 == 0 && stride % 8 == 0, "argmax: rows must be 16-byte aligned");
    ESP_REQUIRE((part == nullptr) == (counters == nullptr), "argmax: part and counters go together");
    if (T <= 0) return esp_host::ok();
    const int64_t nb = (N + ARGMAX_SLICE - 1) / ARGMAX_SLICE;
    if (part && nb > 1 && nb <= ARGMAX_MAX_SLICES && T <= 65535) {
        ESP_REQUIRE(part_numel >= T * nb, "argmax: part needs ceil(N / %d) keys a row", ARGMAX_SLICE);
        ESP_REQUIRE(counters_numel >= T * CNT_STRIDE, "argmax: counters need %d ints a row", CNT_STRIDE);
        const int64_t sl = ((N + nb - 1) / nb + 7) / 8 * 8;   // <= ARGMAX_SLICE, a multiple of 8
        argmax_split_kernel<<<dim3((unsigned)nb, (unsigned)T), 256, 0, (hipStream_t)stream>>>(
            static_cast<const uint16_t*>(logits), stride, (int)N, (int)sl, dtype == ESP_BF16,
            reinterpret_cast<unsigned long long*>(part), counters, ids);
        return esp_host::launch_check("argmax");
    }
    argmax_kernel<<<(unsigned)T, 1024, 0, (hipStream_t)stream>>>(static_cast<const uint16_t*>(logits), stride,
                                                                  (int)N, dtype == ESP_BF16, ids);
    return esp_host::launch_check("argmax");
}

// Measurement probes for bench.py --probes (libespalier_probe.so; not part of the kernel layer's ABI): the ceilings
// the decode kernels are held to on the device they run on.
//   esp_probe_empty   an empty kernel, for the launch floor of a graph of launches
//   esp_probe_read    a streaming read of a buffer (16-byte nontemporal loads), for the attainable HBM read rate
//   esp_probe_valu    8 independent chains of one VALU instruction a lane, for its issue rate
//   esp_probe_lds     random byte / half lookups into a 64 KiB / 128 KiB shared-memory table, for the rate a table
//                     decode of the codebooks could reach
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ void empty_kernel() {}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void read_kernel(const u32x4* __restrict__ src, int64_t n16, uint32_t* __restrict__ sink) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    uint32_t acc = 0u;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const u32x4 v = __builtin_nontemporal_load(src + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;          // keeps the loads; practically never stores
}

template <int OP>
__device__ __forceinline__ void step(uint32_t& a, uint32_t b) {
    if constexpr (OP == 0) asm volatile("v_add_u32 %0, %0, %1" : "+v"(a) : "v"(b));
    else if constexpr (OP == 1) asm volatile("v_mul_lo_u32 %0, %0, %1" : "+v"(a) : "v"(b));
    else if constexpr (OP == 2) asm volatile("v_bfe_u32 %0, %0, 3, 16" : "+v"(a));
    else if constexpr (OP == 3) asm volatile("v_perm_b32 %0, %0, %1, %2" : "+v"(a) : "v"(b), "v"(0x05040100u));
    else if constexpr (OP == 4) asm volatile("v_fma_mix_f32 %0, %0, %1, 0 op_sel_hi:[1,0,0]" : "+v"(a) : "v"(b));
    else if constexpr (OP == 5) asm volatile("v_pk_add_f16 %0, %0, %1" : "+v"(a) : "v"(b));
    else asm volatile("v_add_f16_sdwa %0, %0, %0 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
                      : "+v"(a));
}

template <int OP>
__global__ __launch_bounds__(1024) void valu_kernel(int iters, uint32_t* __restrict__ out) {
    uint32_t c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = threadIdx.x + 0x3C003C00u * (j + 1);
    const uint32_t b = 0x3C003C01u ^ blockIdx.x;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j) step<OP>(c[j], b);
    }
    uint32_t r = 0u;
#pragma unroll
    for (int j = 0; j < 8; ++j) r ^= c[j];
    if (r == 0x9E3779B9u) out[0] = r;
}

// Every lane looks up 8 entries an iteration at byte offsets base + 4096 j (the immediate offset field), base a
// lane's own pseudo-random position, stepped by an odd lane-dependent stride an iteration and kept inside the table:
// 8 lookups for about 3 VALU instructions. WIDE: 16-bit entries of a 128 KiB table, else bytes of a 64 KiB one.
template <bool WIDE>
__global__ __launch_bounds__(1024) void lds_kernel(int iters, uint32_t* __restrict__ out) {
    extern __shared__ __align__(16) uint32_t tab[];
    constexpr uint32_t BYTES = WIDE ? 131072u : 65536u;
    for (uint32_t i = threadIdx.x; i < BYTES / 4; i += blockDim.x) tab[i] = i * 0x9E3779B1u;
    __syncthreads();
    typedef __attribute__((address_space(3))) const unsigned char* lds_u8;
    typedef __attribute__((address_space(3))) const uint16_t* lds_u16;
    const uint32_t span = BYTES - 8 * 4096;                     // base + 4096 * 7 + 1 stays inside the table
    uint32_t base = (threadIdx.x * 2654435761u + blockIdx.x * 40503u) % span;
    const uint32_t stride = ((threadIdx.x * 7919u) | 1u) % span;
    uint32_t acc = 0u;
    for (int it = 0; it < iters; ++it) {
        uint32_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if constexpr (WIDE) v[j] = ((lds_u16)tab)[(base & ~1u) / 2 + 2048 * j];
            else v[j] = ((lds_u8)tab)[base + 4096 * j];
        }
        acc = acc + v[0] + v[1];
        acc = acc + v[2] + v[3];
        acc = acc + v[4] + v[5];
        acc = acc + v[6] + v[7];
        base += stride;
        base = base >= span ? base - span : base;
    }
    if (acc == 0x9E3779B9u) out[0] = acc;
}

}  // namespace

extern "C" int esp_probe_clock_khz(void) {
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&khz, hipDeviceAttributeClockRate, dev) != hipSuccess)
        return -1;
    return khz;
}

extern "C" int esp_probe_empty(int64_t grid, void* stream) {
    if (grid < 1 || grid > (1 << 20)) return 1;
    empty_kernel<<<(unsigned)grid, 64, 0, (hipStream_t)stream>>>();
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

extern "C" int esp_probe_read(const void* src, int64_t bytes, void* sink, int64_t grid, void* stream) {
    if (!src || !sink || bytes < 16 || bytes % 16 || grid < 1) return 1;
    read_kernel<<<(unsigned)grid, 256, 0, (hipStream_t)stream>>>(static_cast<const u32x4*>(src), bytes / 16,
                                                                 static_cast<uint32_t*>(sink));
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

// op: 0 v_add_u32, 1 v_mul_lo_u32, 2 v_bfe_u32, 3 v_perm_b32, 4 v_fma_mix_f32, 5 v_pk_add_f16, 6 v_add_f16 (SDWA)
extern "C" int esp_probe_valu(int op, int iters, int64_t grid, int waves, void* out, void* stream) {
    if (!out || iters < 1 || grid < 1 || waves < 1 || waves > 16) return 1;
    hipStream_t s = (hipStream_t)stream;
    const unsigned threads = 64u * (unsigned)waves;
    uint32_t* o = static_cast<uint32_t*>(out);
    switch (op) {
        case 0: valu_kernel<0><<<(unsigned)grid, threads, 0, s>>>(iters, o); break;
        case 1: valu_kernel<1><<<(unsigned)grid, threads, 0, s>>>(iters, o); break;
        case 2: valu_kernel<2><<<(unsigned)grid, threads, 0, s>>>(iters, o); break;
        case 3: valu_kernel<3><<<(unsigned)grid, threads, 0, s>>>(iters, o); break;
        case 4: valu_kernel<4><<<(unsigned)grid, threads, 0, s>>>(iters, o); break;
        case 5: valu_kernel<5><<<(unsigned)grid, threads, 0, s>>>(iters, o); break;
        case 6: valu_kernel<6><<<(unsigned)grid, threads, 0, s>>>(iters, o); break;
        default: return 1;
    }
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

// wide 0: byte lookups in a 64 KiB table; 1: 16-bit lookups in a 128 KiB table. One workgroup of `waves` waves a CU.
extern "C" int esp_probe_lds(int wide, int iters, int64_t grid, int waves, void* out, void* stream) {
    if (!out || iters < 1 || grid < 1 || waves < 1 || waves > 16) return 1;
    hipStream_t s = (hipStream_t)stream;
    const unsigned threads = 64u * (unsigned)waves;
    uint32_t* o = static_cast<uint32_t*>(out);
    if (wide) {
        if (hipFuncSetAttribute((const void*)lds_kernel<true>, hipFuncAttributeMaxDynamicSharedMemorySize, 131072) !=
            hipSuccess)
            return 2;
        lds_kernel<true><<<(unsigned)grid, threads, 131072, s>>>(iters, o);
    } else {
        if (hipFuncSetAttribute((const void*)lds_kernel<false>, hipFuncAttributeMaxDynamicSharedMemorySize, 65536) !=
            hipSuccess)
            return 2;
        lds_kernel<false><<<(unsigned)grid, threads, 65536, s>>>(iters, o);
    }
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

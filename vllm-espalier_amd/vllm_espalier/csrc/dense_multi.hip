// esp_dense_multi: up to four dense launches in one grid (the groups side by side, or a chain in which a group reads
// the previous group's output), the per-workgroup program of dense.hpp under each group's arguments.
#include "dense.hpp"

namespace esp {

// Device status of the dense launches (read and cleared by esp_status through dense_status)
__device__ int g_dense_status;

// Thread 0 waits until the producer's done count reaches this launch's target, (n + 1) * blocks with n = ticket /
// the group's workgroups, for at most ~20 ms of device time: past that it records ESP_STATUS_WAIT_TIMEOUT and goes on,
// so a launch can never hang. Nothing is reset (the counters are 64-bit).
template <>
__device__ __forceinline__ void dense_wait_producer<true>(const DenseArgs& a, unsigned long long ticket) {
    if (threadIdx.x == 0) {
        const unsigned long long target = (ticket / (unsigned)a.pass_total + 1ull) * (unsigned)a.wait_total;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();        // 100 MHz
        while (load_dev(a.wait_done) < target) {
            __builtin_amdgcn_s_sleep(4);
            if (__builtin_amdgcn_s_memrealtime() - t0 > 2000000ull) {
                __hip_atomic_fetch_or(&g_dense_status, ESP_STATUS_WAIT_TIMEOUT, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------------------------------------------------------------
// esp_dense_multi: up to MAX_GROUPS dense launches in one grid. Group g's workgroups are [start[g], start[g + 1]),
// column block = local id % blocks, split = local id / blocks; a group whose x is the previous group's y waits for it
// (dense_wait_producer) after issuing its first trellis copies. Workgroups are dispatched in id order on each XCD, so every
// producer workgroup is resident or done before a consumer workgroup can occupy its place: the waits always end.
// ------------------------------------------------------------------------------------------------------------------
constexpr int MAX_GROUPS = 4;

struct MultiArgs {
    DenseArgs g[MAX_GROUPS];
    int ng;
    int start[MAX_GROUPS + 1];
    int nbt[MAX_GROUPS];
};

// The arguments are read where the launch put them, in the kernel-argument segment (constant address space), never
// through the by-value parameter: indexing that with the run-time group would copy the whole block (~1.4 KiB) into
// every lane's private memory.
typedef __attribute__((address_space(4))) const MultiArgs* MultiArgsPtr;

template <int MG>
__global__ __launch_bounds__(1024) void dense_multi_kernel(MultiArgs) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int last;
    __shared__ float npart[16], ninv[4];
    const MultiArgsPtr m = (MultiArgsPtr)__builtin_amdgcn_kernarg_segment_ptr();
    const int id = blockIdx.x;
    int gi = 0;
#pragma unroll
    for (int i = 1; i < MAX_GROUPS; ++i)
        if (i < m->ng && id >= m->start[i]) gi = i;
    const DenseArgs& a = *(const DenseArgs*)&m->g[gi];
    const int local = id - m->start[gi], nb = m->nbt[gi];
    const int nbg = local % nb, split = local / nb;
    switch (a.case_id) {
#define ESP_MULTI_CASE(CB_, K2_)                                                                      \
    case CB_ * 32 + K2_:                                                                              \
        dense_program<gemm_cb(CB_), K2_, MG, true>(a, nbg, split, smem, last, npart, ninv);                 \
        break;
        ESP_CASES(ESP_MULTI_CASE)
#undef ESP_MULTI_CASE
    }
}

}  // namespace esp

using namespace esp;

template <int MG>
static int launch_multi(const MultiArgs& m, int W, size_t smem, hipStream_t st) {
    auto kern = dense_multi_kernel<MG>;
    if (smem > 64 * 1024 &&
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
        return esp_host::fail(ESP_ERR_HIP, "dense_multi: cannot raise the shared memory limit to %zu bytes", smem);
    kern<<<dim3((unsigned)m.start[m.ng]), 64 * W, smem, st>>>(m);
    return ESP_OK;
}

extern "C" int esp_dense_multi(int64_t n_groups, const esp_dense_group* groups, int64_t M, int64_t W, float* Z,
                               int64_t z_numel, int32_t* counters, int64_t counters_numel, int64_t rot_smem,
                               void* stream) {
    ESP_REQUIRE(groups && n_groups >= 1 && n_groups <= MAX_GROUPS, "dense_multi: 1 to 4 groups");
    ESP_REQUIRE(Z && counters, "dense_multi: null scratch");
    ESP_REQUIRE(((uintptr_t)counters & 7) == 0, "dense_multi: counters must be 8-byte aligned");
    MultiArgs m{};
    m.ng = (int)n_groups;
    int64_t z_off = 0, c_off = 0;
    size_t smem = 0;
    int mg = 1;
    // the group's own counters first (split-K arrivals, 32 ints a column block), then two lines a group: its done
    // count and its pass count
    int64_t lines = 0;
    for (int g = 0; g < n_groups; ++g) {
        int64_t nb = 0;
        for (int s = 0; s < groups[g].n_shards && s < MAX_SHARDS; ++s) nb += groups[g].n_cols[s] / 128;
        lines += nb;
    }
    const int64_t link_base = lines * CNT_STRIDE;
    ESP_REQUIRE(counters_numel >= link_base + 2 * n_groups * CNT_STRIDE,
                "dense_multi: counters need 32 ints a column block of every group, and 64 a group");
    for (int g = 0; g < n_groups; ++g) {
        const esp_dense_group& G = groups[g];
        ESP_REQUIRE(G.n_shards >= 1 && G.n_shards <= MAX_SHARDS, "dense_multi: 1 to 4 matrices a group");
        ESP_REQUIRE(!G.after_previous || (g > 0 && G.norm_h == nullptr),
                    "dense_multi: only a group after the first may read the previous group's output, and not through "
                    "an in-launch norm");
        int64_t nb = 0;
        for (int s = 0; s < G.n_shards; ++s) nb += G.n_cols[s] / 128;
        const int64_t zg = G.SK > 1 ? (G.SK * M * nb * 128 + 63) / 64 * 64 : 0;
        ESP_REQUIRE(z_off + zg <= z_numel, "dense_multi: Z needs the sum over groups of SK * M * N floats");
        DenseNorm nrm{G.norm_h, G.norm_d1, G.norm_d2, G.norm_w, G.norm_h_out, G.norm_eps};
        DenseLaunch L{};
        const int rc = prepare_dense(G.x, G.x_dtype, G.x_stride, M, G.K, G.n_shards, G.trellis, G.suh, G.svh,
                                     G.n_cols, G.col0, G.y, G.y_dtype, G.y_stride, G.y_cols, nullptr, 0, Z + z_off, zg,
                                     counters + c_off, nb * CNT_STRIDE, G.k2, G.cb, G.SK, W, rot_smem,
                                     G.norm_h ? &nrm : nullptr, L);
        if (rc) return rc;
        ESP_REQUIRE(L.a.fused, "dense_multi: every group's input rotation must fit the fused rotation's shared memory");
        m.g[g] = L.a;
        m.nbt[g] = L.a.NBT;
        m.start[g + 1] = m.start[g] + L.a.NBT * (int)G.SK;
        smem = L.smem > smem ? L.smem : smem;
        mg = L.mg;
        z_off += zg;
        c_off += nb * CNT_STRIDE;
    }
    for (int g = 1; g < n_groups; ++g) {
        if (!groups[g].after_previous) continue;
        unsigned long long* link = reinterpret_cast<unsigned long long*>(counters + link_base);
        m.g[g - 1].done = link + (2 * (g - 1)) * (CNT_STRIDE / 2);
        m.g[g].wait_done = m.g[g - 1].done;
        m.g[g].wait_total = m.nbt[g - 1];
        m.g[g].pass = link + (2 * g + 1) * (CNT_STRIDE / 2);
        m.g[g].pass_total = m.start[g + 1] - m.start[g];
    }
    hipStream_t st = (hipStream_t)stream;
    const int rc = mg == 1 ? launch_multi<1>(m, (int)W, smem, st) : launch_multi<2>(m, (int)W, smem, st);
    if (rc) return rc;
    return esp_host::launch_check("dense_multi");
}

namespace esp_host {
// the dense launches' device status word into *out (ORed), cleared if asked (esp_status)
int dense_status(int clear, hipStream_t st, int* out) {
    int v = 0;
    if (hipMemcpyFromSymbolAsync(&v, HIP_SYMBOL(g_dense_status), sizeof(int), 0, hipMemcpyDeviceToHost, st) !=
            hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return fail(ESP_ERR_HIP, "status: cannot read the dense status word");
    *out |= v;
    if (clear && v) {
        const int zero = 0;
        if (hipMemcpyToSymbolAsync(HIP_SYMBOL(g_dense_status), &zero, sizeof(int), 0, hipMemcpyHostToDevice, st) !=
                hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            return fail(ESP_ERR_HIP, "status: cannot clear the dense status word");
    }
    return ESP_OK;
}
}  // namespace esp_host

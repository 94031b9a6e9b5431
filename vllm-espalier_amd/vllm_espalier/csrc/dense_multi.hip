// esp_dense_multi: up to four dense launches in one grid (the groups side by side, or a chain in which a group reads
// the previous group's output), the per-workgroup program of dense.hpp under each group's arguments.
#include "dense.hpp"

namespace esp {

// Device status of the dense launches (read and cleared by esp_status through dense_status)
__device__ int g_dense_status;

// Wave 0 waits for the producer's column blocks that hold the workgroup's x chunks [c0, c0 + chunks), a lane a block:
// in the n-th launch (n = ticket / SK) each must be counted done n + 1 times. A wait runs for at most ~20 ms of device
// time: past that it records ESP_STATUS_WAIT_TIMEOUT and goes on, so a launch can never hang. Nothing is reset (the
// counts are 64-bit).
template <>
__device__ __forceinline__ void dense_wait_producer<true>(const DenseArgs& a, unsigned long long ticket, int c0,
                                                          int chunks) {
    if (threadIdx.x < 64) {
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)ticket);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(ticket >> 32));
        const unsigned long long target = (((unsigned long long)hi << 32) | lo) / (unsigned)a.SK + 1ull;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();        // 100 MHz
        bool late = false;
        for (int i = (int)threadIdx.x; i < chunks && !late; i += 64) {
            const int yb = a.wait_off + c0 + i;                       // the x chunk's column block in the producer's y
            int pb = 0;
#pragma unroll
            for (int s = 0; s < MAX_SHARDS; ++s)
                if (s < a.wp_n && yb >= a.wp_c0[s] && yb < a.wp_c0[s] + a.wp_nb[s]) pb = a.wp_nb0[s] + yb - a.wp_c0[s];
            const unsigned long long* p = a.wait_done + (size_t)pb * DONE_STRIDE;
            while (load_dev(p) < target) {
                __builtin_amdgcn_s_sleep(2);
                if (__builtin_amdgcn_s_memrealtime() - t0 > 2000000ull) {
                    late = true;
                    break;
                }
            }
        }
        if (late)
            __hip_atomic_fetch_or(&g_dense_status, ESP_STATUS_WAIT_TIMEOUT, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
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
    // the groups' split-K arrival counters first (32 ints a column block), then two 128-byte lines a column block of
    // every group: its done count (a producer's) and its ticket count (a consumer's)
    int64_t blocks = 0;
    int64_t nbs[MAX_GROUPS] = {};
    for (int g = 0; g < n_groups; ++g) {
        for (int s = 0; s < groups[g].n_shards && s < MAX_SHARDS; ++s) nbs[g] += groups[g].n_cols[s] / 128;
        blocks += nbs[g];
    }
    const int64_t link_base = blocks * CNT_STRIDE;
    ESP_REQUIRE(counters_numel >= 3 * link_base,
                "dense_multi: counters need 96 ints a column block of every group");
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
    unsigned long long* link = reinterpret_cast<unsigned long long*>(counters + link_base);
    for (int g = 0, lb = 0; g < n_groups; lb += 2 * (int)nbs[g], ++g) {
        if (g + 1 < n_groups && groups[g + 1].after_previous) m.g[g].done = link + (size_t)lb * DONE_STRIDE;
        if (!groups[g].after_previous) continue;
        // x must be a slice of whole 128-column blocks of the producer's y, every one of them an output of the producer
        const esp_dense_group &P = groups[g - 1], &C = groups[g];
        ESP_REQUIRE(C.x_dtype == P.y_dtype && C.x_stride == P.y_stride,
                    "dense_multi: a group after the previous group reads its output (same dtype and row stride)");
        const int64_t esz = P.y_dtype == ESP_F32 ? 4 : 2;
        const intptr_t d = (const char*)C.x - (const char*)P.y;
        ESP_REQUIRE(d >= 0 && d % (128 * esz) == 0 && d / esz + C.K <= P.y_cols,
                    "dense_multi: x of a group after the previous one starts at a multiple of 128 columns of the "
                    "previous group's y, inside its rows");
        DenseArgs& A = m.g[g];
        A.wait_off = (int)(d / esz / 128);
        A.wp_n = m.g[g - 1].n;
        for (int s = 0; s < A.wp_n; ++s) {
            const Shard& S = m.g[g - 1].s[s];
            ESP_REQUIRE(S.col0 % 128 == 0, "dense_multi: a producer's output columns start at a multiple of 128");
            A.wp_c0[s] = S.col0 / 128;
            A.wp_nb0[s] = S.nb0;
            A.wp_nb[s] = S.nb;
        }
        for (int64_t yb = A.wait_off; yb < A.wait_off + C.K / 128; ++yb) {
            bool covered = false;
            for (int s = 0; s < A.wp_n; ++s) covered |= yb >= A.wp_c0[s] && yb < A.wp_c0[s] + A.wp_nb[s];
            ESP_REQUIRE(covered, "dense_multi: every column of x must be an output of the previous group");
        }
        A.wait_done = m.g[g - 1].done;
        A.pass = link + (size_t)(lb + nbs[g]) * DONE_STRIDE;
        // decode ahead of the wait when the longest split is one stage and a wave's steps fit the registers
        const int steps_max = A.SQ + (A.SR > 0), kw = (int)W / 4;
        A.ahead = steps_max <= stage_max_steps((int)C.k2) && (steps_max + kw - 1) / kw <= AHEAD_STEPS;
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

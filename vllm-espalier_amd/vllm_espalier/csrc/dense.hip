// Dense trellis layers for decode (1-32 rows) on gfx950, plus the trellis dequantisation and the standalone Hadamard.
//
// esp_dense: every matrix of one layer (<= 4 sharing the input and the codebook) in one launch, y_s = H(H(x * suh_s)
// @ W_s) * svh_s written into each matrix's columns of y (dense.cu:1-9, 273-340 define the contract).
//
// Work split. A workgroup is 4 * KW waves on one 128-column block (the output Hadamard's width) and one K range: of
// the S = K / 32 steps of 32 k, = SQ * SK + SR, split s takes the next SQ + (s < SR), so SK need not divide S and a
// launch can match the CU count. Wave (p, kw) owns n tiles 2p, 2p+1 of the block and every KW-th step of the range
// (gemm.hpp); the KW partial sums are added in order through shared memory. Per 32-k step a wave decodes 2 B operands
// (trellis -> fp16 in registers, trellis.hpp) and issues one v_mfma_f32_16x16x32_f16 per B operand and 16-row group
// (rows 0-15, 16-31): weights stream from HBM once for all rows. Split K (SK > 1) goes through Z, and the last workgroup of a column block to arrive (atomic counter) adds the
// splits in order and finishes; counters are left zero.
//
// Row invariance: a row's sums depend only on that row (MFMA keeps rows apart), the K split and per-wave ranges
// depend on the shape alone, and splits are added in a fixed order.
#include "dense.hpp"

#include <mutex>

namespace esp {

// Device status of esp_dense_own's bounded waits (read and cleared by esp_status through dense_own_status)
__device__ int g_dense_own_status;

__device__ void dense_raise_status(int bits) {
    __hip_atomic_fetch_or(&g_dense_own_status, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------------------------------------------------------
// dequant: out fp16 [K][N]. A wave decodes one 32k x 16n block (two k tiles of one n tile) with the MFMA lane decode
// (the same code the GEMMs run) and scatters its 8 values a lane.
// ------------------------------------------------------------------------------------------------------------------
template <int CB, int K2>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ T, uint16_t* __restrict__ out,
                                                      int K, int N) {
    constexpr int TW = 4 * K2;
    const int lane = threadIdx.x & 63;
    const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);   // (k pair, n tile)
    const int NT = N >> 4, KP = (K >> 5);
    const int kp = blk / NT, nt = blk % NT;
    if (kp >= KP) return;
    const int c = lane & 15, G = lane >> 4;
    const int kt = 2 * kp + (G >> 1);
    const LanePlan<K2> lp(lane);
    uint32_t w[6];
    load_words<K2>(T + ((size_t)kt * NT + nt) * TW, lp, w);
    const u32x4 b = decode_words<CB, K2>(w, lp);
    const int col = nt * 16 + c;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int row = kt * 16 + slot_k(G, i);
        out[(size_t)row * N + col] = slot_bits(b, i);
    }
}

// K a multiple of 16 but not of 32: the last k tile pairs with nothing, handled by this single-tile variant
template <int CB, int K2>
__global__ __launch_bounds__(256) void dequant_tail_kernel(const uint32_t* __restrict__ T, uint16_t* __restrict__ out,
                                                           int K, int N) {
    constexpr int TW = 4 * K2;
    const int lane = threadIdx.x & 63;
    const int nt = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int NT = N >> 4;
    if (nt >= NT) return;
    const int c = lane & 15, G = lane >> 4;
    if (G >= 2) return;                                      // only the lanes of the first k tile
    const int kt = (K >> 4) - 1;
    const LanePlan<K2> lp(lane);
    uint32_t w[6];
    load_words<K2>(T + ((size_t)kt * NT + nt) * TW, lp, w);
    const u32x4 b = decode_words<CB, K2>(w, lp);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[(size_t)(kt * 16 + slot_k(G, i)) * N + nt * 16 + c] = slot_bits(b, i);
}

// ------------------------------------------------------------------------------------------------------------------
// had: y = fp16(H(x * pre) / sqrt(128) * post) (dense.cu:242-265). A wave takes two 128-blocks, one per 32-lane half.
// ------------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void had_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ pre,
                                                  const uint16_t* __restrict__ post, uint16_t* __restrict__ y, int M,
                                                  int K) {
    const int l32 = threadIdx.x & 31;
    const long unit = (long)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int nb = K >> 7;
    if (unit >= (long)M * nb) return;
    const int row = (int)(unit / nb), blk = (int)(unit % nb);
    const size_t i = (size_t)row * K + blk * 128 + 4 * l32;
    float v[4];
    load4(x, F16, i, v);
    if (pre) {
        float s[4];
        load4(pre, F16, blk * 128 + 4 * l32, s);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = __fmul_rn(v[j], s[j]);
    }
    fwht128(v, l32);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] *= HAD_SCALE;
    if (post) {
        float s[4];
        load4(post, F16, blk * 128 + 4 * l32, s);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] *= s[j];
    }
    store4(y, F16, i, v);
}

// ------------------------------------------------------------------------------------------------------------------
// dense: unfused input rotation xh[s][row][k] = fp16(H(x * suh_s) / sqrt(128)) (dense.cu:110-117)
// ------------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dense_rot_kernel(DenseArgs a, uint16_t* __restrict__ xh) {
    const int l32 = threadIdx.x & 31;
    const int nb = a.K >> 7;
    const long unit = (long)blockIdx.x * 8 + (threadIdx.x >> 5);   // (shard, row, block)
    if (unit >= (long)a.n * a.M * nb) return;
    const int blk = (int)(unit % nb);
    const int row = (int)((unit / nb) % a.M);
    const int s = (int)(unit / ((long)nb * a.M));
    const uint2 u = rot128(a.x, a.x_dtype, (size_t)row * a.x_stride + blk * 128, a.s[s].suh + blk * 128, l32);
    *reinterpret_cast<uint2*>(xh + ((size_t)s * a.M + row) * a.K + blk * 128 + 4 * l32) = u;
}

template <int CB, int K2, int MG>
__global__ __launch_bounds__(1024) void dense_kernel(DenseArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int last;
    __shared__ float npart[16], ninv[4];
    dense_program<CB, K2, MG, false>(a, blockIdx.x, blockIdx.y, smem, last, npart, ninv);
}

template <int KCB, int K2, int MG>
static int launch_dense(const DenseArgs& a, dim3 grid, int W, size_t smem, hipStream_t st) {
    auto kern = dense_kernel<KCB, K2, MG>;
    if (smem > 64 * 1024 &&
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
        return esp_host::fail(ESP_ERR_HIP, "dense: cannot raise the shared memory limit to %zu bytes", smem);
    kern<<<grid, 64 * W, smem, st>>>(a);
    return ESP_OK;
}

}  // namespace esp

// ======================================================================================================================
// C ABI
// ======================================================================================================================
using namespace esp;

extern "C" int esp_dequant(const void* trellis, void* out, int64_t K, int64_t N, int64_t k2, int64_t cb,
                           void* stream) {
    ESP_REQUIRE(trellis && out, "dequant: null pointer");
    ESP_REQUIRE(K > 0 && N > 0 && K % 16 == 0 && N % 16 == 0, "dequant: K and N must be positive multiples of 16");
    if (!(supported((int)cb, (int)k2) || ((cb == 22 || cb == 23) && supported((int)cb - 16, (int)k2)) ||
          (cb == 19 && supported(3, (int)k2))))
        return esp_host::fail(ESP_ERR_UNSUPPORTED, "no instance for codebook %lld K2 %lld", (long long)cb,
                              (long long)k2);
    hipStream_t s = (hipStream_t)stream;
    const long blocks = (K / 32) * (N / 16);
    const unsigned grid = (unsigned)((blocks + 3) / 4);
    const bool tail = (K % 32) != 0;
    const unsigned tgrid = (unsigned)((N / 16 + 3) / 4);
    auto T = static_cast<const uint32_t*>(trellis);
    auto o = static_cast<uint16_t*>(out);
    switch (cb * 32 + k2) {
#define ESP_DQ(CB_, K2_)                                                                                   \
    case CB_ * 32 + K2_:                                                                                   \
        if (grid) dequant_kernel<CB_, K2_><<<grid, 256, 0, s>>>(T, o, (int)K, (int)N);                     \
        if (tail) dequant_tail_kernel<CB_, K2_><<<tgrid, 256, 0, s>>>(T, o, (int)K, (int)N);               \
        break;
        ESP_CASES(ESP_DQ)
        ESP_GRID_CASES(ESP_DQ)
#undef ESP_DQ
    }
    return esp_host::launch_check("dequant");
}

extern "C" int esp_had(const void* x, const void* pre, const void* post, void* y, int64_t M, int64_t K,
                       void* stream) {
    ESP_REQUIRE(x && y, "had: null pointer");
    ESP_REQUIRE(K % 128 == 0, "had: K must be a multiple of 128");
    if (M <= 0 || K <= 0) return esp_host::ok();
    const long units = M * (K / 128);
    had_kernel<<<(unsigned)((units + 7) / 8), 256, 0, (hipStream_t)stream>>>(
        static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(pre), static_cast<const uint16_t*>(post),
        static_cast<uint16_t*>(y), (int)M, (int)K);
    return esp_host::launch_check("had");
}

// esp_dense's checks and arguments (dense.cu:276-340 define the contract), without the launch. xh must be given when
// the rotation is not fused (need_xh reports it before xh is checked, for callers that place xh afterwards).
int prepare_dense(const void* x, int x_dtype, int64_t x_stride, int64_t M, int64_t K, int64_t n_shards,
                         const void* const* trellis, const void* const* suh, const void* const* svh,
                         const int64_t* n_cols, const int64_t* col0, void* y, int y_dtype, int64_t y_stride,
                         int64_t y_cols, void* xh, int64_t xh_numel, float* Z, int64_t z_numel, int32_t* counters,
                         int64_t counters_numel, int64_t k2, int64_t cb, int64_t SK, int64_t W, int64_t rot_smem,
                         const DenseNorm* nrm, DenseLaunch& L) {
    ESP_REQUIRE(n_shards >= 1 && n_shards <= MAX_SHARDS, "1 to 4 matrices a launch");
    ESP_REQUIRE(M >= 1 && M <= 32, "1 to 32 rows");
    ESP_REQUIRE(K > 0 && K % 128 == 0 && SK >= 1 && SK <= K / 32,
                "K must be a multiple of 128 and SK at most K / 32 (splits of whole 32-k steps)");
    ESP_REQUIRE(x_dtype >= 0 && x_dtype <= 2 && y_dtype >= 0 && y_dtype <= 2, "x / y dtype");
    ESP_REQUIRE(W == 4 || W == 8 || W == 16, "W (waves a workgroup) must be 4, 8 or 16");
    ESP_REQUIRE(x_stride >= K && y_stride >= y_cols, "x / y row stride");
    // the kernels move 4 elements of a row at once (8 bytes, 16 for fp32) and trellis tiles 16 bytes at a time
    ESP_REQUIRE(((uintptr_t)x % (x_dtype == ESP_F32 ? 16 : 8)) == 0 && x_stride % 4 == 0 &&
                    ((uintptr_t)y % (y_dtype == ESP_F32 ? 16 : 8)) == 0 && y_stride % 4 == 0,
                "x / y must be 8-byte aligned (16 for fp32) with row strides a multiple of 4 elements");
    if (!supported((int)cb, (int)k2))
        return esp_host::fail(ESP_ERR_UNSUPPORTED, "unsupported codebook/width: cb=%lld k2=%lld", (long long)cb,
                              (long long)k2);
    DenseArgs a{};
    int nbt = 0;
    const float c = gemm_scale((int)cb);
    for (int s = 0; s < n_shards; ++s) {
        const int64_t N = n_cols[s];
        ESP_REQUIRE(N > 0 && N % 128 == 0, "matrix shape");
        ESP_REQUIRE(col0[s] >= 0 && col0[s] + N <= y_cols, "matrix columns past y");
        ESP_REQUIRE(trellis[s] && suh[s] && svh[s], "dense: null matrix pointer");
        ESP_REQUIRE(((uintptr_t)trellis[s] & 15) == 0 && ((uintptr_t)suh[s] & 7) == 0 && ((uintptr_t)svh[s] & 7) == 0 &&
                        col0[s] % 4 == 0,
                    "dense: trellis 16-byte aligned, suh / svh 8-byte aligned, col0 a multiple of 4");
        a.s[s] = Shard{static_cast<const uint32_t*>(trellis[s]), static_cast<const uint16_t*>(suh[s]),
                       static_cast<const uint16_t*>(svh[s]), nbt, (int)(N / 128), (int)col0[s], c};
        nbt += (int)(N / 128);
    }
    a.n = (int)n_shards;
    // the reference's contract (dense.cu:296): Z holds SK * M * N floats, counters at least 2 per 128 columns. The
    // counters are spread as far apart as the buffer allows, up to one 128-byte line each (a caller sizing them
    // 32 per 128 columns keeps arrivals on different counters off each other's line).
    ESP_REQUIRE(SK == 1 || (Z && z_numel >= SK * M * nbt * 128 && counters && counters_numel >= 2 * (int64_t)nbt),
                "scratch too small: Z needs SK*M*N floats, counters 2 per 128 columns");
    ESP_REQUIRE(SK * M * nbt * 128 <= (int64_t(1) << 30), "dense: the partials must fit in 4 GiB");
    ESP_REQUIRE(SK == 1 || (((uintptr_t)Z & 15) == 0 && ((uintptr_t)counters & 3) == 0),
                "dense: Z must be 16-byte aligned");
    const int64_t sq = (K / 32) / SK, sr = (K / 32) % SK;
    const int64_t steps_max = sq + (sr > 0);                  // the longest split
    const int64_t kr = steps_max * 32;
    // 128-blocks a split's rotated rows touch: exact when every split starts and ends on one, else the bound for a
    // range starting up to 96 past a block's start
    const bool aligned = sr == 0 && sq % 4 == 0;
    const int64_t chunks_max = aligned ? steps_max / 4 : (steps_max * 32 + 96 + 127) / 128;
    const int xs_stride = (int)(chunks_max * 128) + 8;        // pad rows across the LDS banks
    const bool fused = M * chunks_max * 128 * 2 <= rot_smem;
    if (nrm) {
        ESP_REQUIRE(nrm->h && nrm->w && nrm->h_out, "dense_rmsnorm: null pointer");
        ESP_REQUIRE(x_dtype == ESP_BF16 || x_dtype == ESP_F16, "dense_rmsnorm: rows must be bf16 or fp16");
        ESP_REQUIRE(M <= W / 4, "dense_rmsnorm: at most W / 4 rows (four waves normalise a row)");
        ESP_REQUIRE(K % 8 == 0 && K <= NORM_MAX_D && x_stride % 8 == 0 &&
                        ((uintptr_t)nrm->h | (uintptr_t)nrm->d1 | (uintptr_t)nrm->d2 | (uintptr_t)nrm->w |
                         (uintptr_t)nrm->h_out) % 16 == 0,
                    "dense_rmsnorm: K at most 8192, rows 16-byte aligned");
        ESP_REQUIRE(fused, "dense_rmsnorm: the rows must fit the fused rotation's shared memory");
        a.nh = static_cast<const uint16_t*>(nrm->h);
        a.nd1 = static_cast<const uint16_t*>(nrm->d1);
        a.nd2 = static_cast<const uint16_t*>(nrm->d2);
        a.nw = static_cast<const uint16_t*>(nrm->w);
        a.nh_out = static_cast<uint16_t*>(nrm->h_out);
        a.neps = (float)nrm->eps;
        a.norm = 1;
    }
    if (!fused) ESP_REQUIRE(xh && xh_numel >= n_shards * M * K && ((uintptr_t)xh & 7) == 0, "xh too small or unaligned");
    a.x = x;
    a.x_dtype = x_dtype;
    a.x_stride = (int)x_stride;
    a.xh = static_cast<const uint16_t*>(xh);
    a.y = y;
    a.y_dtype = y_dtype;
    a.y_stride = (int)y_stride;
    a.Z = Z;
    a.counters = counters;
    a.M = (int)M;
    a.K = (int)K;
    a.SK = (int)SK;
    a.SQ = (int)sq;
    a.SR = (int)sr;
    a.NBT = nbt;
    a.cnt_stride = SK == 1 ? 0 : (int)(counters_numel / nbt < CNT_STRIDE ? counters_numel / nbt : CNT_STRIDE);
    a.fused = fused;
    a.xs_stride = xs_stride;
    a.case_id = (int)(cb * 32 + k2);
    const size_t stage_bytes = (size_t)host_stage_words((int)k2, (int)kr) * 4;
    a.stage_bytes = (int)stage_bytes;
    const size_t smem_x = stage_bytes + (fused ? (size_t)M * xs_stride * 2 : 0);
    const size_t smem_red = (size_t)(W / 4) * M * 128 * 4;
    const size_t smem = smem_x > smem_red ? smem_x : smem_red;
    ESP_REQUIRE(smem <= 160 * 1024, "dense: shared memory for the fused rotation exceeds 160 KiB");
    // more splits than one batch of loads: spread them over the last workgroup's 32-lane halves when they all fit
    a.gather = SK > 8 && M * SK <= 2 * W && (size_t)M * SK * 32 * 16 <= smem;
    L.a = a;
    L.grid = dim3((unsigned)nbt, (unsigned)SK);
    L.W = (int)W;
    L.smem = smem;
    L.mg = M > 16 ? 2 : 1;
    return ESP_OK;
}

static int launch_prepared(const DenseLaunch& L, hipStream_t st) {
    const DenseArgs& a = L.a;
    if (!a.fused) {
        const long units = (long)a.n * a.M * (a.K / 128);
        dense_rot_kernel<<<(unsigned)((units + 7) / 8), 256, 0, st>>>(a, const_cast<uint16_t*>(a.xh));
        int rc = esp_host::launch_check("dense rotation");
        if (rc) return rc;
    }
    int rc = ESP_OK;
    switch (a.case_id) {
#define ESP_DENSE_CASE(CB_, K2_)                                                                           \
    case CB_ * 32 + K2_: {                                                                                 \
        constexpr int KCB = gemm_cb(CB_);                                                                  \
        rc = L.mg == 1 ? launch_dense<KCB, K2_, 1>(a, L.grid, L.W, L.smem, st)                              \
                       : launch_dense<KCB, K2_, 2>(a, L.grid, L.W, L.smem, st);                             \
        break;                                                                                             \
    }
        ESP_CASES(ESP_DENSE_CASE)
#undef ESP_DENSE_CASE
    }
    if (rc) return rc;
    return esp_host::launch_check("dense");
}

static int dense_impl(const void* x, int x_dtype, int64_t x_stride, int64_t M, int64_t K, int64_t n_shards,
                      const void* const* trellis, const void* const* suh, const void* const* svh, const int64_t* n_cols,
                      const int64_t* col0, void* y, int y_dtype, int64_t y_stride, int64_t y_cols, void* xh,
                      int64_t xh_numel, float* Z, int64_t z_numel, int32_t* counters, int64_t counters_numel,
                      int64_t k2, int64_t cb, int64_t SK, int64_t W, int64_t rot_smem, const DenseNorm* nrm,
                      void* stream, bool own = false) {
    DenseLaunch L{};
    const int rc = prepare_dense(x, x_dtype, x_stride, M, K, n_shards, trellis, suh, svh, n_cols, col0, y, y_dtype,
                                 y_stride, y_cols, xh, xh_numel, Z, z_numel, counters, counters_numel, k2, cb, SK, W,
                                 rot_smem, nrm, L);
    if (rc) return rc;
    if (own && SK > 1) {
        // the polled hand-off when the finisher holds one (row, split) partial a 32-lane half and they fit its shared
        // memory past the block's sums; else the arrivals are counted and the finisher restores the all-ones
        const bool poll = M * (SK - 1) <= 2 * L.W && (size_t)(L.W / 4 + SK - 1) * M * 512 <= L.smem;
        L.a.own = poll ? 2 : 1;
    }
    return launch_prepared(L, (hipStream_t)stream);
}

extern "C" int esp_dense(const void* x, int x_dtype, int64_t x_stride, int64_t M, int64_t K, int64_t n_shards,
                         const void* const* trellis, const void* const* suh, const void* const* svh,
                         const int64_t* n_cols, const int64_t* col0, void* y, int y_dtype, int64_t y_stride,
                         int64_t y_cols, void* xh, int64_t xh_numel, float* Z, int64_t z_numel, int32_t* counters,
                         int64_t counters_numel, int64_t k2, int64_t cb, int64_t SK, int64_t W, int64_t PF,
                         int64_t rot_smem, void* stream) {
    (void)PF;
    ESP_REQUIRE(x, "dense: null x");
    return dense_impl(x, x_dtype, x_stride, M, K, n_shards, trellis, suh, svh, n_cols, col0, y, y_dtype, y_stride,
                      y_cols, xh, xh_numel, Z, z_numel, counters, counters_numel, k2, cb, SK, W, rot_smem, nullptr,
                      stream);
}

extern "C" int esp_dense_own(const void* x, int x_dtype, int64_t x_stride, int64_t M, int64_t K, int64_t n_shards,
                             const void* const* trellis, const void* const* suh, const void* const* svh,
                             const int64_t* n_cols, const int64_t* col0, void* y, int y_dtype, int64_t y_stride,
                             int64_t y_cols, void* xh, int64_t xh_numel, float* Z, int64_t z_numel, int32_t* counters,
                             int64_t counters_numel, int64_t k2, int64_t cb, int64_t SK, int64_t W, int64_t PF,
                             int64_t rot_smem, void* stream) {
    (void)PF;
    ESP_REQUIRE(x, "dense_own: null x");
    return dense_impl(x, x_dtype, x_stride, M, K, n_shards, trellis, suh, svh, n_cols, col0, y, y_dtype, y_stride,
                      y_cols, xh, xh_numel, Z, z_numel, counters, counters_numel, k2, cb, SK, W, rot_smem, nullptr,
                      stream, true);
}

extern "C" int esp_dense_rmsnorm(const void* h, const void* d1, const void* d2, const void* norm_w, double eps,
                                 void* h_out, int x_dtype, int64_t x_stride, int64_t M, int64_t K, int64_t n_shards,
                                 const void* const* trellis, const void* const* suh, const void* const* svh,
                                 const int64_t* n_cols, const int64_t* col0, void* y, int y_dtype, int64_t y_stride,
                                 int64_t y_cols, float* Z, int64_t z_numel, int32_t* counters, int64_t counters_numel,
                                 int64_t k2, int64_t cb, int64_t SK, int64_t W, int64_t rot_smem, void* stream) {
    const DenseNorm nrm{h, d1, d2, norm_w, h_out, eps};
    return dense_impl(h, x_dtype, x_stride, M, K, n_shards, trellis, suh, svh, n_cols, col0, y, y_dtype, y_stride,
                      y_cols, nullptr, 0, Z, z_numel, counters, counters_numel, k2, cb, SK, W, rot_smem, &nrm, stream);
}

// ======================================================================================================================
// esp_dense_noalloc: esp_dense with its scratch (arrival counters, split-K partials, unfused rotation rows) in a
// file-scope device array instead of caller buffers, for callers that cannot allocate. Layout of the array:
//   [0, NOALLOC_COUNTER_BYTES)       arrival counters, one a 128-column block, as far apart as fit (up to 32 ints)
//   [NOALLOC_COUNTER_BYTES, ...)     Z, SK * M * sum(n_cols) floats, then xh (n_shards * M * K halves) if unfused
// The counters start zero: the array has no initializer, so it lives in the code object's zero-filled segment, which
// the loader allocates zeroed on each device it loads the library's code onto; every launch leaves the counters it used
// zero, so no call clears them, and nothing is launched besides the GEMM (a first call inside stream capture records
// only the GEMM). Calls overlapping on one GPU share the array and race.
// ======================================================================================================================
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(16) << 20;
constexpr size_t NOALLOC_COUNTER_BYTES = size_t(64) << 10;

static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[NOALLOC_MAX_DEVICES];     // the array's device address, per device

// The array's address on the current device, looked up the first time the device uses it (no device work).
int noalloc_scratch(unsigned char** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES)
        return esp_host::fail(ESP_ERR_HIP, "dense_noalloc: no current device");
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (g_noalloc_ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return esp_host::fail(ESP_ERR_HIP, "dense_noalloc: cannot resolve the scratch array: %s",
                                  hipGetErrorString(e));
        g_noalloc_ptr[dev] = p;
    }
    *out = static_cast<unsigned char*>(g_noalloc_ptr[dev]);
    return ESP_OK;
}
}  // namespace

extern "C" int esp_dense_noalloc(const void* x, int x_dtype, int64_t x_stride, int64_t M, int64_t K,
                                 int64_t n_shards, const void* const* trellis, const void* const* suh,
                                 const void* const* svh, const int64_t* n_cols, const int64_t* col0, void* y,
                                 int y_dtype, int64_t y_stride, int64_t y_cols, int64_t k2, int64_t cb, int64_t SK,
                                 int64_t W, int64_t PF, int64_t rot_smem, void* stream) {
    (void)PF;
    ESP_REQUIRE(x && n_cols, "dense_noalloc: null x / n_cols");
    ESP_REQUIRE(n_shards >= 1 && n_shards <= MAX_SHARDS, "1 to 4 matrices a launch");
    ESP_REQUIRE(M >= 1 && M <= 32 && K > 0 && K % 128 == 0 && SK >= 1 && SK <= K / 32, "dense_noalloc: shape");
    int64_t nbt = 0;
    for (int64_t s = 0; s < n_shards; ++s) {
        ESP_REQUIRE(n_cols[s] > 0 && n_cols[s] % 128 == 0, "matrix shape");
        nbt += n_cols[s] / 128;
    }
    // what the launch needs of the array: the counters (at least 2 ints a block, the esp_dense minimum), Z, and xh
    // for the unfused rotation (esp_dense's fusion test, repeated here to size it)
    const int64_t counters_numel = (int64_t)(NOALLOC_COUNTER_BYTES / 4);
    ESP_REQUIRE(SK == 1 || 2 * nbt <= counters_numel,
                "dense_noalloc: %lld column blocks need more arrival counters than the scratch array holds (%lld)",
                (long long)nbt, (long long)counters_numel);
    const int64_t z_numel = SK > 1 ? SK * M * nbt * 128 : 0;
    const int64_t sq = (K / 32) / SK, sr = (K / 32) % SK;
    const int64_t steps_max = sq + (sr > 0);
    const bool aligned = sr == 0 && sq % 4 == 0;
    const int64_t chunks_max = aligned ? steps_max / 4 : (steps_max * 32 + 96 + 127) / 128;
    const bool fused = M * chunks_max * 128 * 2 <= rot_smem;
    const int64_t xh_numel = fused ? 0 : n_shards * M * K;
    const size_t z_bytes = ((size_t)z_numel * 4 + 255) / 256 * 256;
    const size_t need = NOALLOC_COUNTER_BYTES + z_bytes + (size_t)xh_numel * 2;
    if (need > NOALLOC_SCRATCH_BYTES)
        return esp_host::fail(ESP_ERR_ARG,
                              "dense_noalloc: this launch needs %zu bytes of scratch, the array holds %zu "
                              "(use esp_dense with caller buffers)",
                              need, NOALLOC_SCRATCH_BYTES);
    unsigned char* base = nullptr;
    const int rc = noalloc_scratch(&base);
    if (rc) return rc;
    int32_t* counters = reinterpret_cast<int32_t*>(base);
    float* Z = reinterpret_cast<float*>(base + NOALLOC_COUNTER_BYTES);
    void* xh = base + NOALLOC_COUNTER_BYTES + z_bytes;
    return dense_impl(x, x_dtype, x_stride, M, K, n_shards, trellis, suh, svh, n_cols, col0, y, y_dtype, y_stride,
                      y_cols, fused ? nullptr : xh, xh_numel, SK > 1 ? Z : nullptr, z_numel, counters,
                      counters_numel, k2, cb, SK, W, rot_smem, nullptr, stream);
}

#ifdef ESP_PHASE_TRACE
// The timing build's phase records of esp_dense's workgroups (dense.hpp): copy n words out, or clear them all
extern "C" int esp_phase_read(unsigned long long* host, int64_t n) {
    ESP_REQUIRE(host && n >= 0 && n <= (int64_t)esp::PHASE_WGS * 8, "phase_read: 0 to %d words", esp::PHASE_WGS * 8);
    if (hipMemcpyFromSymbol(host, HIP_SYMBOL(esp::g_phase), (size_t)n * 8, 0, hipMemcpyDeviceToHost) != hipSuccess)
        return esp_host::fail(ESP_ERR_HIP, "phase_read: copy failed");
    return esp_host::ok();
}
extern "C" int esp_phase_clear(void) {
    static unsigned long long zero[esp::PHASE_WGS * 8];
    if (hipMemcpyToSymbol(HIP_SYMBOL(esp::g_phase), zero, sizeof(zero), 0, hipMemcpyHostToDevice) != hipSuccess)
        return esp_host::fail(ESP_ERR_HIP, "phase_clear: copy failed");
    return esp_host::ok();
}
#endif

namespace esp_host {
// esp_dense_own's device status word into *out (ORed), cleared if asked (esp_status)
int dense_own_status(int clear, hipStream_t st, int* out) {
    int v = 0;
    if (hipMemcpyFromSymbolAsync(&v, HIP_SYMBOL(esp::g_dense_own_status), sizeof(int), 0, hipMemcpyDeviceToHost, st) !=
            hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return fail(ESP_ERR_HIP, "status: cannot read the dense launches' status word");
    *out |= v;
    if (clear && v) {
        const int zero = 0;
        if (hipMemcpyToSymbolAsync(HIP_SYMBOL(esp::g_dense_own_status), &zero, sizeof(int), 0, hipMemcpyHostToDevice,
                                   st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            return fail(ESP_ERR_HIP, "status: cannot clear the dense launches' status word");
    }
    return ESP_OK;
}
}  // namespace esp_host

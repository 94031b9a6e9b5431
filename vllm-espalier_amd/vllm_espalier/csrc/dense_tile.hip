// esp_dense_tile: a dense layer over a whole prompt (any number of rows) on gfx950, each weight decoded once for every
// 128 rows instead of once a 32-row window.
//
// Two launches. (1) tile_rot_kernel rotates every row once a matrix, xh_s = fp16(H(x * suh_s) / sqrt(128)), and stores
// it in MFMA A-fragment order: [matrix][row group of 16][32-k step][64 lanes][8 halves], one 1 KiB block a (row
// group, step) holding exactly what v_mfma_f32_16x16x32_f16 reads from each lane (lane c + 16 G: row c, the k slots
// of trellis.hpp's B operand). (2) dense_tile_kernel: a workgroup is 8 waves on one 128-column block, one K split and
// one tile of up to 128 rows (8 row groups). The tile's A blocks and the block's trellis tiles reach LDS through
// global_load_lds (no VGPRs, no VALU), double-buffered in stages of 4 steps; a wave (pair p = n tiles 2p, 2p+1; k slot
// kw of 2) decodes its two B operands of a step once and issues 16 MFMAs with them (8 row groups x 2 tiles). The two
// k slots' sums are added in shared memory (slot 0, then slot 1), and split K goes through Z with the last split to
// arrive adding the splits in order and finishing, as esp_dense does.
//
// Row invariance: a row's sums depend only on its own A rows, the K split (a function of the caller's plan) and the
// fixed step order, never on the other rows of the prompt or its place in a tile.
#include <type_traits>

#include "dense.hpp"

namespace esp {

constexpr int TILE_ROWS = 128;                  // rows a workgroup
constexpr int TILE_RG = TILE_ROWS / 16;         // row groups a workgroup
constexpr int TILE_WAVES = 8;                   // 4 pairs x 2 k slots
constexpr int TILE_KW = TILE_WAVES / 4;
constexpr int TILE_STEPS = 4;                   // 32-k steps a stage
constexpr int TILE_FRAG = 512;                  // halves a (row group, step) block: 64 lanes x 8
constexpr int RED_STRIDE = 132;                 // floats between two rows of the block's sums (banks apart)
constexpr int RED_BYTES = TILE_ROWS * RED_STRIDE * 4;

#ifdef ESP_PHASE_TRACE
// Timing build only (build.py --phase-trace): thread 0 of each workgroup records the 100 MHz real-time counter into
// g_tile_phase[workgroup][8]: 0 start, 1 the first stage landed, 2 the ticks spent in the later stage waits (a sum),
// 3 its own wave's K loop done, 4 the block's sums in shared memory, 5 partials stored and arrived (or y stored at one
// split), 6 the finisher done; slot 7 holds the XCD (bits 0-3), 1 << 8 for a finisher and the stage count << 16.
constexpr int TILE_PHASE_WGS = 8192;
static __device__ unsigned long long g_tile_phase[TILE_PHASE_WGS * 8];
__device__ __forceinline__ int tile_phase_wg() {
    return (int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
}
__device__ __forceinline__ void tile_phase_set(int slot, unsigned long long v) {
    if (threadIdx.x == 0 && tile_phase_wg() < TILE_PHASE_WGS) g_tile_phase[tile_phase_wg() * 8 + slot] = v;
}
__device__ __forceinline__ void tile_phase_info(int finisher, int nst) {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    tile_phase_set(7, (unsigned long long)(xcc & 0xFu) | ((unsigned long long)finisher << 8) |
                          ((unsigned long long)nst << 16));
}
#define TILE_PHASE(slot) tile_phase_set(slot, __builtin_amdgcn_s_memrealtime())
#define TILE_PHASE_SET(slot, v) tile_phase_set(slot, v)
#define TILE_PHASE_INFO(finisher, nst) tile_phase_info(finisher, nst)
#define TILE_PHASE_DRAIN()              \
    do {                                \
        __builtin_amdgcn_s_waitcnt(0);  \
        __syncthreads();                \
    } while (0)
#define TILE_NOW() __builtin_amdgcn_s_memrealtime()
#else
#define TILE_PHASE(slot) ((void)0)
#define TILE_PHASE_SET(slot, v) ((void)0)
#define TILE_PHASE_INFO(finisher, nst) ((void)0)
#define TILE_PHASE_DRAIN() ((void)0)
#define TILE_NOW() 0ull
#endif

// Device status of the prompt launches: ESP_STATUS_WAIT_TIMEOUT when a spread finish gave up waiting (read and cleared
// by esp_status through tile_status)
__device__ int g_tile_status;

struct TileArgs {
    Shard s[MAX_SHARDS];
    int n;
    const uint16_t* xh;      // fragment-ordered rotated rows [n][RG][K / 32][64][8]
    void* y;
    int y_dtype, y_stride;
    float* Z;                // [row tiles][SK][128][NBT * 128]
    int* counters;           // [row tiles][NBT][CNT_STRIDE]
    int T, K, SK, NBT, SQ, SR, RG;
    int spread;              // every workgroup of the launch resident at once: each split finishes a share of the rows
};

// Every split of a (row tile, column block) waits here until all `total` have stored their partials: thread 0 counts
// its arrival, spins on the count (bounded: ~20 ms of s_memrealtime, then ESP_STATUS_WAIT_TIMEOUT and on), then counts
// itself past on *seen; the last one past resets both to zero.
__device__ __forceinline__ void tile_all_arrived(int* counter, int* seen, int total) {
    __builtin_amdgcn_s_waitcnt(0);          // this wave's device-scope partial stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();          // 100 MHz
        while (load_dev(counter) < total) {
            __builtin_amdgcn_s_sleep(1);
            if (__builtin_amdgcn_s_memrealtime() - t0 > 2000000ull) {
                __hip_atomic_fetch_or(&g_tile_status, ESP_STATUS_WAIT_TIMEOUT, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
        if (__hip_atomic_fetch_add(seen, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1) {
            store_dev(counter, 0);
            store_dev(seen, 0);
        }
    }
    __syncthreads();
}

// xh of tile_rot_kernel: a workgroup takes one matrix, one row group of 16 rows and one 128-chunk of K, which fill
// exactly the 4 (row group, step) A blocks of that chunk: a 32-lane half rotates 2 rows (rows past T are zero) into
// their fragment places in shared memory, then the 4 KiB go out as one 16-byte store a thread, contiguous in xh
__global__ __launch_bounds__(256) void tile_rot_kernel(const void* __restrict__ x, int x_dtype, int x_stride, int T,
                                                       int K, int n, const uint16_t* suh0, const uint16_t* suh1,
                                                       const uint16_t* suh2, const uint16_t* suh3,
                                                       uint16_t* __restrict__ xh, int RG) {
    __shared__ __align__(16) uint16_t frag[4 * TILE_FRAG];
    const int l32 = threadIdx.x & 31, hw = threadIdx.x >> 5;
    const int nb = K >> 7;
    const int ch = (int)(blockIdx.x % nb), rg = (int)((blockIdx.x / nb) % RG), s = (int)(blockIdx.x / (nb * RG));
    const uint16_t* suh = s == 0 ? suh0 : s == 1 ? suh1 : s == 2 ? suh2 : suh3;
    // the lane's 4 consecutive k (ch * 128 + 4 l32 ...) are 4 consecutive halves of one A fragment lane
    const int kk = (4 * l32) & 31, kt = kk & 15;
    const int sl = l32 >> 3;                                  // the step inside the chunk
    const int G = 2 * (kk >> 4) + ((kt >> 2) & 1), hi = kt >> 3;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int rr = 2 * hw + i, r = rg * 16 + rr;
        uint2 u = make_uint2(0u, 0u);
        if (r < T) u = rot128(x, x_dtype, (size_t)r * x_stride + ch * 128, suh + ch * 128, l32);
        *reinterpret_cast<uint2*>(frag + (sl * 64 + rr + 16 * G) * 8 + 4 * hi) = u;
    }
    __syncthreads();
    uint16_t* dst = xh + (((size_t)s * RG + rg) * (K >> 5) + ch * 4) * TILE_FRAG;
    reinterpret_cast<uint4*>(dst)[threadIdx.x] = reinterpret_cast<const uint4*>(frag)[threadIdx.x];
}

typedef __attribute__((address_space(3))) const f16x8* lds_f16x8_ptr;

// The finisher's rows of one half-wave (rows rbase, rbase + 16, ...): RPB rows at a time with the other splits'
// partials of those rows in flight together (RPB * OM loads, OM >= SK - 1), its own split's sums read from shared
// memory (own: the block's [128][RED_STRIDE] sums), each row's splits added in split order, then the output transform
// and y. zp0 is the half-wave's column slice of split 0's row 0 in Z. The loads take no branch (a load under a
// lane-dependent branch is waited on before the next one): a row past Mt still lies in Z's 128 rows of the tile and is
// read but not used, and a slot past SK - 1 reads split 0 again.
template <int RPB, int OM>
__device__ __forceinline__ void tile_finish_rows(const DevBuf& zb, const float* zp0, size_t zrow, size_t zsplit,
                                                 const float* own, int wave, int rbase, int Mt, int SK, int split,
                                                 int l32, uint2 sv, float scale, void* y, int y_dtype, size_t ybase,
                                                 int y_stride) {
    constexpr int RSTEP = 2 * TILE_WAVES, ITERS = TILE_ROWS / RSTEP;
    for (int i0 = 0; i0 < ITERS && 2 * wave + i0 * RSTEP < Mt; i0 += RPB) {
        float4 u[RPB][OM];
#pragma unroll
        for (int i = 0; i < RPB; ++i) {
            const int r = rbase + (i0 + i) * RSTEP;
#pragma unroll
            for (int o = 0; o < OM; ++o) {
                const int q = o >= SK - 1 ? 0 : o < split ? o : o + 1;    // the o-th split other than its own
                u[i][o] = zb.load4(zp0 + r * zrow + q * zsplit);
            }
        }
#pragma unroll
        for (int i = 0; i < RPB; ++i) {
            const int r = rbase + (i0 + i) * RSTEP;
            if (r < Mt) {
                const float4 mine = *reinterpret_cast<const float4*>(own + r * RED_STRIDE + 4 * l32);
                float4 s = split == 0 ? mine : u[i][0];
#pragma unroll
                for (int q = 1; q <= OM; ++q)
                    if (q < SK) {
                        const float4 t = q == split ? mine : q < split ? u[i][q < OM ? q : OM - 1] : u[i][q - 1];
                        s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
                    }
                float v[4] = {s.x, s.y, s.z, s.w};
                finish(v, l32, sv, scale);
                store4(y, y_dtype, ybase + (size_t)r * y_stride, v);
            }
        }
    }
}

// A split's share [lo, hi) of the tile's rows after every split arrived: each row's partials added in split order, its
// own split's from shared memory (own: the block's [128][RED_STRIDE] sums), RPB rows of a half-wave with all their
// other splits' loads (OM >= SK - 1) in flight; a row past hi reads a row of Z's 128 (not used), so no load branches
template <int RPB, int OM>
__device__ __forceinline__ void tile_finish_share(const DevBuf& zb, const float* zp0, size_t zrow, size_t zsplit,
                                                  const float* own, int lo, int hi, int SK, int split, int rbase,
                                                  int l32, uint2 sv, float scale, void* y, int y_dtype, size_t ybase,
                                                  int y_stride) {
    constexpr int RSTEP = 2 * TILE_WAVES;
    for (int r0 = lo + rbase; r0 < hi; r0 += RPB * RSTEP) {
        float4 u[RPB][OM];
#pragma unroll
        for (int i = 0; i < RPB; ++i) {
            const int r = r0 + i * RSTEP < TILE_ROWS ? r0 + i * RSTEP : TILE_ROWS - 1;
#pragma unroll
            for (int o = 0; o < OM; ++o) {
                const int q = o >= SK - 1 ? 0 : o < split ? o : o + 1;    // the o-th split other than its own
                u[i][o] = zb.load4(zp0 + r * zrow + q * zsplit);
            }
        }
#pragma unroll
        for (int i = 0; i < RPB; ++i) {
            const int r = r0 + i * RSTEP;
            if (r < hi) {
                const float4 mine = *reinterpret_cast<const float4*>(own + r * RED_STRIDE + 4 * l32);
                float4 s = split == 0 ? mine : u[i][0];
#pragma unroll
                for (int q = 1; q <= OM; ++q)
                    if (q < SK) {
                        const float4 t = q == split ? mine : q < split ? u[i][q < OM ? q : OM - 1] : u[i][q - 1];
                        s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
                    }
                float v[4] = {s.x, s.y, s.z, s.w};
                finish(v, l32, sv, scale);
                store4(y, y_dtype, ybase + (size_t)r * y_stride, v);
            }
        }
    }
}

template <int CB, int K2>
__global__ __launch_bounds__(TILE_WAVES * 64) void dense_tile_kernel(TileArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    // the arrival flag sits past the block's sums (no static shared memory: at 4-bit widths two workgroups of 80 KiB
    // then share a CU, each hiding the other's stage waits)
    int* const last = reinterpret_cast<int*>(smem + RED_BYTES);
    constexpr int TW = 4 * K2;
    constexpr int ROW_WORDS = StagePlan<K2>::ROW_WORDS;            // one k tile of the block
    constexpr int B_BUF = TILE_STEPS * 2 * ROW_WORDS;              // words a B stage
    constexpr int A_BUF = TILE_RG * TILE_STEPS * TILE_FRAG;        // halves an A stage
    const int nbg = blockIdx.x, split = blockIdx.y, mt = blockIdx.z;
    TILE_PHASE(0);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int l32 = lane & 31, half = lane >> 5, pair = wave & 3, kw = wave >> 2, G = lane >> 4;

    // the column block's matrix: its fields picked by unrolled compares (an indexed read of the argument block would
    // copy it to private memory)
    int si = 0;
#pragma unroll
    for (int i = 1; i < MAX_SHARDS; ++i)
        if (i < a.n && nbg >= a.s[i].nb0) si = i;
    const uint32_t* Tw = a.s[0].T;
    const uint16_t* svh = a.s[0].svh;
    int nb0 = a.s[0].nb0, nbs = a.s[0].nb, col0 = a.s[0].col0;
    float scale = a.s[0].scale;
#pragma unroll
    for (int i = 1; i < MAX_SHARDS; ++i)
        if (si == i) {
            Tw = a.s[i].T;
            svh = a.s[i].svh;
            nb0 = a.s[i].nb0;
            nbs = a.s[i].nb;
            col0 = a.s[i].col0;
            scale = a.s[i].scale;
        }
    const int cb_local = nbg - nb0, NTILES = nbs * 8;
    const int s0 = split * a.SQ + (split < a.SR ? split : a.SR), steps = a.SQ + (split < a.SR);
    const int m0 = mt * TILE_ROWS, Mt = a.T - m0 < TILE_ROWS ? a.T - m0 : TILE_ROWS, rgt = (Mt + 15) >> 4;
    const int ksteps = a.K >> 5;
    const uint16_t* X = a.xh + (((size_t)si * a.RG + mt * TILE_RG) * ksteps + s0) * TILE_FRAG;
    // the trellis stages first: their words are read at per-lane addresses plus constants, which fit the LDS reads'
    // 16-bit immediate offsets only below 64 KiB (past it every read needs an address add)
    uint32_t* sb = reinterpret_cast<uint32_t*>(smem);
    uint16_t* sa = reinterpret_cast<uint16_t*>(smem + 2 * B_BUF * 4);

    // stage st of the split into buffer buf: the block's trellis tiles, then the tile's A blocks (rgt row groups x n
    // steps of 64 16-byte units; a wave's 64 units are one block, so its LDS destination is one contiguous KiB)
    auto issue = [&](int st, int buf) __attribute__((always_inline)) {
        const int first = st * TILE_STEPS, n = steps - first < TILE_STEPS ? steps - first : TILE_STEPS;
        issue_stage<K2>(Tw, NTILES, (s0 + first) * 2, 2 * n, cb_local * 8, sb + buf * B_BUF);
        const int units = rgt * n * 64;
        for (int u0 = wave * 64; u0 < units; u0 += TILE_WAVES * 64) {
            const int g = u0 / (n * 64), r0 = u0 - g * n * 64;
            const uint16_t* src = X + ((size_t)g * ksteps + first) * TILE_FRAG + (r0 + lane) * 8;
            uint16_t* dst = sa + buf * A_BUF + (g * TILE_STEPS * 64 + r0) * 8;
            __builtin_amdgcn_global_load_lds((global_void_ptr)src, (lds_void_ptr)dst, 16, 0, 0);
        }
    };

    f32x4 acc[2][TILE_RG];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < TILE_RG; ++g) acc[j][g] = f32x4{0.f, 0.f, 0.f, 0.f};
    const LanePlan<K2> lp(lane);
    const LdsWords<K2> lw(lp);
    const int lane_base = ((G >> 1) * 8 + 2 * pair) * TW;
    const int nst = (steps + TILE_STEPS - 1) / TILE_STEPS;
    const uint2 sv = *reinterpret_cast<const uint2*>(svh + cb_local * 128 + 4 * l32);

    // a tile of fewer than 128 rows (the prompt's last, or a short prompt) reads and multiplies only its row groups;
    // a full tile keeps the loop free of those tests
    auto run = [&](auto full) __attribute__((always_inline)) {
        constexpr bool FULL = decltype(full)::value;
        issue(0, 0);
        unsigned long long waited = 0;
        (void)waited;
        for (int st = 0; st < nst; ++st) {
            const unsigned long long t0 = TILE_NOW();
            (void)t0;
            wait_stage();                           // stage st landed; every wave is done with buffer (st + 1) & 1
#ifdef ESP_PHASE_TRACE
            if (st == 0)
                TILE_PHASE(1);
            else
                waited += TILE_NOW() - t0;
#endif
            if (st + 1 < nst) issue(st + 1, (st + 1) & 1);
            const int first = st * TILE_STEPS, n = steps - first < TILE_STEPS ? steps - first : TILE_STEPS;
            const uint32_t* bb = sb + (st & 1) * B_BUF + lane_base;
            const uint16_t* ab = sa + (st & 1) * A_BUF + lane * 8;
            for (int ls = kw; ls < n; ls += TILE_KW) {
                // the trellis words, then every row group's A fragment, all in flight while the words are decoded (LDS
                // reads return in order). Rows of the tile's last row group past T are zeros of xh, and their sums
                // are never stored.
                uint32_t w[2][6];
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int i = 0; i < 6; ++i) w[j][i] = bb[ls * 2 * ROW_WORDS + j * TW + lw.off[i]];
                f16x8 av[TILE_RG];
                if (FULL) {
#pragma unroll
                    for (int g = 0; g < TILE_RG; ++g) av[g] = *(lds_f16x8_ptr)(ab + (g * TILE_STEPS + ls) * TILE_FRAG);
                }
                f16x8 b[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) b[j] = decode_b<CB, K2>(w[j], lp);
#pragma unroll
                for (int g = 0; g < TILE_RG; ++g)
                    if (FULL || g < rgt) {
                        // a partial tile reads each row group's fragment where it uses it (fewer live registers)
                        if (!FULL) av[g] = *(lds_f16x8_ptr)(ab + (g * TILE_STEPS + ls) * TILE_FRAG);
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            acc[j][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[g], b[j], acc[j][g], 0, 0, 0);
                    }
            }
        }
        TILE_PHASE_SET(2, waited);
        TILE_PHASE(3);
    };
    if (rgt == TILE_RG)
        run(std::true_type{});
    else
        run(std::false_type{});

    // the block's [Mt][128] sums: k slot 0's accumulators into shared memory, then slot 1's added to them
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);
    const int c = lane & 15;
#pragma unroll
    for (int q = 0; q < TILE_KW; ++q) {
        if (kw == q) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int g = 0; g < TILE_RG; ++g)
                    if (g < rgt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            float* p = red + (g * 16 + 4 * G + i) * RED_STRIDE + 32 * pair + 16 * j + c;
                            *p = q == 0 ? acc[j][g][i] : *p + acc[j][g][i];
                        }
        }
        __syncthreads();
    }
    TILE_PHASE(4);
    const int ycol = col0 + cb_local * 128 + 4 * l32;
    const size_t yrow0 = (size_t)m0 * a.y_stride;
    if (a.SK == 1) {
        for (int r = wave * 2 + half; r < Mt; r += 2 * TILE_WAVES) {
            const float4 s4 = *reinterpret_cast<const float4*>(red + r * RED_STRIDE + 4 * l32);
            float v[4] = {s4.x, s4.y, s4.z, s4.w};
            finish(v, l32, sv, scale);
            store4(a.y, a.y_dtype, yrow0 + (size_t)r * a.y_stride + ycol, v);
        }
        TILE_PHASE_DRAIN();
        TILE_PHASE(5);
        TILE_PHASE_INFO(0, nst);
        return;
    }
    // K splits: partials to Z, the last split of the (row tile, column block) to arrive adds them in split order
    const size_t zrow = (size_t)a.NBT * 128, zsplit = (size_t)TILE_ROWS * zrow;
    float* Zt = a.Z + (size_t)mt * a.SK * zsplit;
    const DevBuf zb(a.Z);
    for (int r = wave * 2 + half; r < Mt; r += 2 * TILE_WAVES)
        zb.store4(Zt + split * zsplit + r * zrow + nbg * 128 + 4 * l32,
                  *reinterpret_cast<const float4*>(red + r * RED_STRIDE + 4 * l32));
    int* const cnt_p = a.counters + ((size_t)mt * a.NBT + nbg) * CNT_STRIDE;
    if (a.spread) {
        // every split finishes a share of the rows once all have arrived (the sums and order of one finisher)
        tile_all_arrived(cnt_p, cnt_p + 1, a.SK);
        TILE_PHASE(5);
        const int per = (Mt + a.SK - 1) / a.SK, lo = split * per, hi = lo + per < Mt ? lo + per : Mt;
        const float* zp0 = Zt + nbg * 128 + 4 * l32;
        if (a.SK <= 3)
            tile_finish_share<4, 2>(zb, zp0, zrow, zsplit, red, lo, hi, a.SK, split, wave * 2 + half, l32, sv, scale,
                                    a.y, a.y_dtype, yrow0 + ycol, a.y_stride);
        else if (a.SK <= 5)
            tile_finish_share<2, 4>(zb, zp0, zrow, zsplit, red, lo, hi, a.SK, split, wave * 2 + half, l32, sv, scale,
                                    a.y, a.y_dtype, yrow0 + ycol, a.y_stride);
        else if (a.SK <= 9)
            tile_finish_share<1, 8>(zb, zp0, zrow, zsplit, red, lo, hi, a.SK, split, wave * 2 + half, l32, sv, scale,
                                    a.y, a.y_dtype, yrow0 + ycol, a.y_stride);
        TILE_PHASE_DRAIN();
        TILE_PHASE(6);
        TILE_PHASE_INFO(1, nst);                          // every split finishes its share
        return;
    }
    const bool finisher = arrive_last(cnt_p, a.SK, last);
    TILE_PHASE(5);
    TILE_PHASE_INFO(finisher ? 1 : 0, nst);
    if (!finisher) return;
    // the other splits' partials, up to 16 loads in flight a lane (the rows' device-scope round trips overlap instead
    // of following one another, eight rows a half-wave); its own split's sums are still in shared memory
    const float* zp0 = Zt + nbg * 128 + 4 * l32;
    if (a.SK <= 3) {
        tile_finish_rows<8, 2>(zb, zp0, zrow, zsplit, red, wave, wave * 2 + half, Mt, a.SK, split, l32, sv,
                               scale, a.y, a.y_dtype, yrow0 + ycol, a.y_stride);
    } else if (a.SK <= 4) {
        tile_finish_rows<4, 3>(zb, zp0, zrow, zsplit, red, wave, wave * 2 + half, Mt, a.SK, split, l32, sv,
                               scale, a.y, a.y_dtype, yrow0 + ycol, a.y_stride);
    } else if (a.SK <= 8) {
        tile_finish_rows<2, 7>(zb, zp0, zrow, zsplit, red, wave, wave * 2 + half, Mt, a.SK, split, l32, sv,
                               scale, a.y, a.y_dtype, yrow0 + ycol, a.y_stride);
    } else for (int r = wave * 2 + half; r < Mt; r += 2 * TILE_WAVES) {
        const float* zp = Zt + r * zrow + nbg * 128 + 4 * l32;
        float4 s;
        for (int q0 = 0; q0 < a.SK; q0 += 8) {              // up to eight splits' loads in flight at once
            float4 u[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (q0 + i < a.SK) u[i] = zb.load4(zp + (q0 + i) * zsplit);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (q0 + i == 0) {
                    s = u[0];
                } else if (q0 + i < a.SK) {
                    s.x += u[i].x; s.y += u[i].y; s.z += u[i].z; s.w += u[i].w;
                }
            }
        }
        float v[4] = {s.x, s.y, s.z, s.w};
        finish(v, l32, sv, scale);
        store4(a.y, a.y_dtype, yrow0 + (size_t)r * a.y_stride + ycol, v);
    }
    if (threadIdx.x == 0) store_dev(cnt_p, 0);          // every split of the block arrived
    TILE_PHASE_DRAIN();
    TILE_PHASE(6);
}

template <int KCB, int K2>
static int launch_tile(const TileArgs& a0, dim3 grid, size_t smem, hipStream_t st) {
    auto kern = dense_tile_kernel<KCB, K2>;
    if (smem > 64 * 1024 &&
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
        return esp_host::fail(ESP_ERR_HIP, "dense_tile: cannot raise the shared memory limit to %zu bytes", smem);
    TileArgs a = a0;
    // The finish spread over the splits: a split waits only for the other splits of its own (row tile, column block),
    // and a row tile's workgroups are consecutive ids (grid.x * grid.y of them). Workgroups are dispatched in id order,
    // so the lowest unfinished tile always has every workgroup dispatched (all lower ones are done) and finishes: it
    // is enough that a tile's workgroups fit on the device with room to spare (half the resident workgroups, the CUs
    // times what a CU holds of this kernel at this shared memory). The waits are bounded either way.
    if (a.SK > 1 && a.SK <= 9) {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)kern, TILE_WAVES * 64, smem) ==
                hipSuccess &&
            2L * grid.x * grid.y <= (long)cus * per_cu)
            a.spread = 1;
    }
    kern<<<grid, TILE_WAVES * 64, smem, st>>>(a);
    return ESP_OK;
}

}  // namespace esp

using namespace esp;

#ifdef ESP_PHASE_TRACE
// The timing build's phase records of esp_dense_tile's workgroups: copy n words out, or clear them all
extern "C" int esp_tile_phase_read(unsigned long long* host, int64_t n) {
    ESP_REQUIRE(host && n >= 0 && n <= (int64_t)esp::TILE_PHASE_WGS * 8, "tile_phase_read: 0 to %d words",
                esp::TILE_PHASE_WGS * 8);
    if (hipMemcpyFromSymbol(host, HIP_SYMBOL(esp::g_tile_phase), (size_t)n * 8, 0, hipMemcpyDeviceToHost) != hipSuccess)
        return esp_host::fail(ESP_ERR_HIP, "tile_phase_read: copy failed");
    return esp_host::ok();
}
extern "C" int esp_tile_phase_clear(void) {
    static unsigned long long zero[esp::TILE_PHASE_WGS * 8];
    if (hipMemcpyToSymbol(HIP_SYMBOL(esp::g_tile_phase), zero, sizeof(zero), 0, hipMemcpyHostToDevice) != hipSuccess)
        return esp_host::fail(ESP_ERR_HIP, "tile_phase_clear: copy failed");
    return esp_host::ok();
}
#endif

namespace esp_host {
// the prompt launches' device status word into *out (ORed), cleared if asked (esp_status)
int tile_status(int clear, hipStream_t st, int* out) {
    int v = 0;
    if (hipMemcpyFromSymbolAsync(&v, HIP_SYMBOL(g_tile_status), sizeof(int), 0, hipMemcpyDeviceToHost, st) !=
            hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return fail(ESP_ERR_HIP, "status: cannot read the prompt launches' status word");
    *out |= v;
    if (clear && v) {
        const int zero = 0;
        if (hipMemcpyToSymbolAsync(HIP_SYMBOL(g_tile_status), &zero, sizeof(int), 0, hipMemcpyHostToDevice, st) !=
                hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            return fail(ESP_ERR_HIP, "status: cannot clear the prompt launches' status word");
    }
    return ESP_OK;
}
}  // namespace esp_host

extern "C" int esp_dense_tile(const void* x, int x_dtype, int64_t x_stride, int64_t T, int64_t K, int64_t n_shards,
                              const void* const* trellis, const void* const* suh, const void* const* svh,
                              const int64_t* n_cols, const int64_t* col0, void* y, int y_dtype, int64_t y_stride,
                              int64_t y_cols, void* xh, int64_t xh_numel, float* Z, int64_t z_numel,
                              int32_t* counters, int64_t counters_numel, int64_t k2, int64_t cb, int64_t SK,
                              void* stream) {
    ESP_REQUIRE(x && y && xh && trellis && suh && svh && n_cols && col0, "dense_tile: null pointer");
    ESP_REQUIRE(n_shards >= 1 && n_shards <= MAX_SHARDS, "dense_tile: 1 to 4 matrices a launch");
    ESP_REQUIRE(T >= 1, "dense_tile: at least one row");
    ESP_REQUIRE(K > 0 && K % 128 == 0 && SK >= 1 && SK <= K / 32,
                "dense_tile: K must be a multiple of 128 and SK at most K / 32");
    ESP_REQUIRE(x_dtype >= 0 && x_dtype <= 2 && y_dtype >= 0 && y_dtype <= 2, "dense_tile: x / y dtype");
    ESP_REQUIRE(x_stride >= K && y_stride >= y_cols, "dense_tile: x / y row stride");
    ESP_REQUIRE(((uintptr_t)x % (x_dtype == ESP_F32 ? 16 : 8)) == 0 && x_stride % 4 == 0 &&
                    ((uintptr_t)y % (y_dtype == ESP_F32 ? 16 : 8)) == 0 && y_stride % 4 == 0 &&
                    ((uintptr_t)xh & 15) == 0 && ((uintptr_t)Z & 15) == 0,
                "dense_tile: x / y 8-byte aligned (16 for fp32) with row strides a multiple of 4 elements, xh and Z "
                "16-byte aligned");
    if (!supported((int)cb, (int)k2))
        return esp_host::fail(ESP_ERR_UNSUPPORTED, "unsupported codebook/width: cb=%lld k2=%lld", (long long)cb,
                              (long long)k2);
    TileArgs a{};
    int nbt = 0;
    const float c = gemm_scale((int)cb);
    const uint16_t* su[MAX_SHARDS] = {};
    for (int s = 0; s < n_shards; ++s) {
        const int64_t N = n_cols[s];
        ESP_REQUIRE(N > 0 && N % 128 == 0, "dense_tile: matrix shape");
        ESP_REQUIRE(col0[s] >= 0 && col0[s] + N <= y_cols, "dense_tile: matrix columns past y");
        ESP_REQUIRE(trellis[s] && suh[s] && svh[s], "dense_tile: null matrix pointer");
        ESP_REQUIRE(((uintptr_t)trellis[s] & 15) == 0 && ((uintptr_t)suh[s] & 7) == 0 && ((uintptr_t)svh[s] & 7) == 0 &&
                        col0[s] % 4 == 0,
                    "dense_tile: trellis 16-byte aligned, suh / svh 8-byte aligned, col0 a multiple of 4");
        a.s[s] = Shard{static_cast<const uint32_t*>(trellis[s]), static_cast<const uint16_t*>(suh[s]),
                       static_cast<const uint16_t*>(svh[s]), nbt, (int)(N / 128), (int)col0[s], c};
        su[s] = static_cast<const uint16_t*>(suh[s]);
        nbt += (int)(N / 128);
    }
    const int64_t RG = (T + 15) / 16, tiles = (T + TILE_ROWS - 1) / TILE_ROWS;
    ESP_REQUIRE(tiles <= 65535, "dense_tile: at most 65535 tiles of 128 rows");
    ESP_REQUIRE(xh_numel >= n_shards * RG * 16 * K, "dense_tile: xh needs n_shards * ceil(T / 16) * 16 * K halves");
    ESP_REQUIRE(SK == 1 || (Z && counters && z_numel >= tiles * SK * TILE_ROWS * nbt * 128 &&
                            counters_numel >= tiles * nbt * CNT_STRIDE),
                "dense_tile: with SK > 1, Z needs ceil(T / 128) * SK * 128 * N floats and counters 32 ints a "
                "(128-row tile, 128-column block)");
    ESP_REQUIRE(tiles * SK * TILE_ROWS * nbt * 128 <= (int64_t(1) << 30), "dense_tile: the partials must fit in 4 GiB");
    a.n = (int)n_shards;
    a.xh = static_cast<const uint16_t*>(xh);
    a.y = y;
    a.y_dtype = y_dtype;
    a.y_stride = (int)y_stride;
    a.Z = Z;
    a.counters = counters;
    a.T = (int)T;
    a.K = (int)K;
    a.SK = (int)SK;
    a.NBT = nbt;
    a.SQ = (int)((K / 32) / SK);
    a.SR = (int)((K / 32) % SK);
    a.RG = (int)RG;
    const size_t stage = 2 * (size_t)TILE_RG * TILE_STEPS * TILE_FRAG * 2 + 2 * (size_t)TILE_STEPS * 2 * 32 * k2 * 4;
    const size_t red = (size_t)RED_BYTES + 16;                   // the sums, then the arrival flag
    const size_t smem = stage > red ? stage : red;
    hipStream_t st = (hipStream_t)stream;
    const long units = (long)n_shards * RG * (K / 128);          // (matrix, row group, 128-chunk)
    tile_rot_kernel<<<(unsigned)units, 256, 0, st>>>(x, x_dtype, (int)x_stride, (int)T, (int)K,
                                                                 (int)n_shards, su[0], su[1], su[2], su[3],
                                                                 static_cast<uint16_t*>(xh), (int)RG);
    int rc = esp_host::launch_check("dense_tile rotation");
    if (rc) return rc;
    const dim3 grid((unsigned)nbt, (unsigned)SK, (unsigned)tiles);
    switch (cb * 32 + k2) {
#define ESP_TILE_CASE(CB_, K2_)                                          \
    case CB_ * 32 + K2_:                                                 \
        rc = launch_tile<gemm_cb(CB_), K2_>(a, grid, smem, st);          \
        break;
        ESP_CASES(ESP_TILE_CASE)
#undef ESP_TILE_CASE
    }
    if (rc) return rc;
    return esp_host::launch_check("dense_tile");
}

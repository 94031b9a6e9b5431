/* espalier.h -- C ABI of the MI355X (gfx950) trellis kernel layer, libespalier_hip.so.
 *
 * One entry point per function of the reference's extension module `espalier_ext`
 * (vllm_espalier/csrc/experts.cpp:234-248), with the same argument order and meaning, as plain pointers and sizes:
 *   - tensors become device pointers plus the sizes the reference reads from them;
 *   - the stream is the caller's hipStream_t (the reference launches on the current stream);
 *   - every launch is asynchronous and nothing here allocates or synchronises, so calls are legal under graph
 *     capture. The caller owns every buffer.
 * Errors: a call returns ESP_OK (0) or an ESP_ERR_* code, and esp_last_error() holds a message. The reference
 * raises these as TORCH_CHECK failures (RuntimeError in Python); the torch binding raises the same.
 * dtype codes: ESP_F16 0, ESP_BF16 1, ESP_F32 2.
 * Codebook ids are the kernels' (1 mcg, 3 E2M1, 6 int5, 7 int6), K2 = 2 * bits; the supported (cb, K2) pairs are
 * mcg at K2 2..16 (even), E2M1 at 2, 4, 6, int5 at 4, 6, 8, int6 at 6, 8, 10 (experts_grouped.cuh:227-229).
 */
#ifndef ESPALIER_H
#define ESPALIER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ESP_OK 0
#define ESP_ERR_ARG 1          /* a shape, size, limit or layout check failed */
#define ESP_ERR_UNSUPPORTED 2  /* no kernel for this codebook / width / tile setting */
#define ESP_ERR_HIP 3          /* the HIP runtime reported an error */

#define ESP_F16 0
#define ESP_BF16 1
#define ESP_F32 2

/* Bits of the device status word (esp_status). */
#define ESP_STATUS_NO_KERNEL 1    /* a grouped launch met an expert whose (codebook, K2) has no kernel */
#define ESP_STATUS_WIDTH_RANGE 2  /* a grouped launch met an expert whose K2 lies outside the launch's [lo, hi] */
#define ESP_STATUS_WAIT_TIMEOUT 4 /* a launch gave up waiting (~20 ms): a chained launch (dense_multi, moe_chain) for a
                                     producer, a prompt launch (dense_tile) for the other K splits of a tile, or
                                     route_group_own / route_group_rmsnorm at one row for the other workgroups'
                                     logits, or dense_own for the other K splits' partials */
#define ESP_STATUS_TILE_LIST 8    /* esp_tile_list met more non-empty member tiles than its bound (a malformed table),
                                   * or esp_grouped_list's grid (sized from its P and maxm) is shorter than the list */

/* Message of the last failed call on this host thread ("" if none). */
const char* esp_last_error(void);

/* The device status word of the current GPU into *status, cleared afterwards when clear != 0. The grouped launches
 * (esp_grouped, esp_moe_gateup) read each expert's width and codebook from device tables the host does not see;
 * where an entry has no kernel (the reference traps: experts_grouped.cuh:288,293) or a width outside [lo, hi], the
 * launch issues no copy for that expert, sets its K-split partials to NaN (so every output built from them is
 * non-finite) and ORs ESP_STATUS_* bits into this word. No counterpart in the reference extension. Synchronises
 * `stream` (a diagnostic call, not for the decode loop). */
int esp_status(int32_t* status, int clear, void* stream);

/* ABI version (incremented on any signature change). */
int esp_abi_version(void);

/* Replaces `had` (experts.cpp:226-232, dense.cu:242-265, 342-351): y = fp16(H(x * pre) / sqrt(128) * post) along rows
 * of 128. x, y fp16 [M][K] (y may alias x); pre / post fp16 [K] or NULL. K % 128 == 0. */
int esp_had(const void* x, const void* pre, const void* post, void* y, int64_t M, int64_t K, void* stream);

/* Replaces `dequant` (experts.cpp:68-77, experts_grouped.cuh:321-340, 379-387): out fp16 [K][N] = the decoded
 * weight of a trellis int16 [K/16][N/16][8 * k2]. cb 1 / 3 / 6 / 7 as the reference; cb 22 / 23 (this library's
 * addition) give the int5 / int6 grid index q as fp16 (the dense kernels decode it and scale the sums by c). */
int esp_dequant(const void* trellis, void* out, int64_t K, int64_t N, int64_t k2, int64_t cb, void* stream);

/* Replaces `dense` (experts.cpp:193-211, dense.cu:273-340): for each of n_shards (1..4) matrices sharing x,
 * y[:, col0[s] : col0[s] + n_cols[s]] = H(H(x * suh_s) @ W_s) * svh_s, M <= 32 rows.
 * x [M][x_stride] (x_dtype), trellis[s] int16 [K/16][n_cols[s]/16][8*k2], suh[s] fp16 [K], svh[s] fp16 [n_cols[s]],
 * y [M][y_stride] (y_dtype) with y_cols columns. Scratch: xh fp16 (xh_numel halves; n_shards*M*K used when the input
 * rotation is not fused), Z fp32 (z_numel; SK*M*sum(n_cols) used when SK > 1, at most 2^30 floats: the partials
 * are addressed by 32-bit byte offsets), counters int32 (counters_numel >= 2 * sum(n_cols)/128 when SK > 1, the
 * reference's size; one counter a 128-column block, min(32, counters_numel / (sum(n_cols)/128)) ints apart, so 32 a
 * block keeps each on a 128-byte line of its own; zero on entry and left zero). SK K splits; W, PF tile hints; the
 * input rotation is fused when M * (K / SK) * 2 <= rot_smem bytes. Alignment (torch's allocations meet it): x and y
 * 8-byte aligned (16 for fp32) with row strides a multiple of 4 elements, col0 a multiple of 4, trellis 16-byte
 * aligned, suh / svh and xh 8-byte aligned, Z 16-byte aligned; else ESP_ERR_ARG. */
int esp_dense(const void* x, int x_dtype, int64_t x_stride, int64_t M, int64_t K, int64_t n_shards,
              const void* const* trellis, const void* const* suh, const void* const* svh, const int64_t* n_cols,
              const int64_t* col0, void* y, int y_dtype, int64_t y_stride, int64_t y_cols, void* xh, int64_t xh_numel,
              float* Z, int64_t z_numel, int32_t* counters, int64_t counters_numel, int64_t k2, int64_t cb, int64_t SK,
              int64_t W, int64_t PF, int64_t rot_smem, void* stream);

/* esp_dense with Z as the launch's own hand-off buffer: every bit of Z set (0xFF bytes) on entry, and left so. Where the
 * last K split's workgroup can hold one (row, split) partial a 32-lane half (M * (SK - 1) <= 2 W, in its shared
 * memory), it reads the other splits' partials once none is all-ones, with no arrival count (a bounded wait: ~20 ms,
 * then ESP_STATUS_WAIT_TIMEOUT); otherwise the arrivals are counted as in esp_dense and the finisher puts the all-ones
 * back. Bit-identical to esp_dense; counters zero on entry and left zero. No counterpart in the reference (whose Z is
 * plain scratch): for callers that keep a partials buffer across calls. */
int esp_dense_own(const void* x, int x_dtype, int64_t x_stride, int64_t M, int64_t K, int64_t n_shards,
                  const void* const* trellis, const void* const* suh, const void* const* svh, const int64_t* n_cols,
                  const int64_t* col0, void* y, int y_dtype, int64_t y_stride, int64_t y_cols, void* xh,
                  int64_t xh_numel, float* Z, int64_t z_numel, int32_t* counters, int64_t counters_numel, int64_t k2,
                  int64_t cb, int64_t SK, int64_t W, int64_t PF, int64_t rot_smem, void* stream);

/* esp_dense over any number of rows (a whole prompt), for prefill: the same layer, with each weight decoded once for
 * every 128 rows instead of once a 32-row window. No counterpart in the reference (its prefill re-decodes the weights
 * every window, README.md:115-117, and names a dedicated prefill GEMM as planned). Arguments as esp_dense, with
 * T >= 1 rows. Scratch: xh fp16 (xh_numel >= n_shards * ceil(T / 16) * 16 * K halves: the rows rotated once a
 * matrix, in MFMA fragment order), and with SK > 1, Z fp32 (z_numel >= ceil(T / 128) * SK * 128 * sum(n_cols), at most
 * 2^30 floats) and counters int32 (counters_numel >= 32 * ceil(T / 128) * sum(n_cols) / 128; zero on entry and left
 * zero). A row's bits depend on its own input and SK only: the same for any T and any place in the prompt, but not
 * those of esp_dense (another order of the sums). When every workgroup of the launch fits on the device at once, each
 * K split finishes a share of its tile's rows after all splits have arrived (the same sums in the same order; a wait
 * past ~20 ms sets ESP_STATUS_WAIT_TIMEOUT). Alignment as esp_dense, xh and Z 16-byte aligned. */
int esp_dense_tile(const void* x, int x_dtype, int64_t x_stride, int64_t T, int64_t K, int64_t n_shards,
                   const void* const* trellis, const void* const* suh, const void* const* svh, const int64_t* n_cols,
                   const int64_t* col0, void* y, int y_dtype, int64_t y_stride, int64_t y_cols, void* xh,
                   int64_t xh_numel, float* Z, int64_t z_numel, int32_t* counters, int64_t counters_numel, int64_t k2,
                   int64_t cb, int64_t SK, void* stream);

/* Replaces `route_group` (experts.cpp:214-223, route.cu:35-207): router logits x @ gate^T (+ the shared gate), top-k
 * by the exactly rounded bf16 logits (lowest id on ties), weights renormalised over the picks, the shared slot's
 * weight sigmoid(x . sgate), then the grouping of the picks. x [R][x_stride] and gate [E][H] in one dtype (bf16 or
 * fp16); sgate [H] or NULL (needed when shared_id >= 0). logits fp32 scratch (logits_numel >= R * (E + has));
 * counter int32 [1] zero on entry and left zero; pick_out int32 / wts_out fp32 [R * (k + has)]; uids int32 [maxu];
 * ucount int32 [1]; members int32 [maxu][maxm]. Limits: E <= 256, k <= 16, H % 256 == 0, R * (k + has) <= 1056. */
int esp_route_group(const void* x, int x_dtype, int64_t x_stride, int64_t R, int64_t H, const void* gate, int64_t E,
                    const void* sgate, int64_t k, int64_t shared_id, float* logits, int64_t logits_numel,
                    int32_t* counter, int32_t* pick_out, float* wts_out, int32_t* uids, int64_t maxu, int32_t* ucount,
                    int32_t* members, int64_t maxm, void* stream);

/* esp_route_group with its logits as the launch's own hand-off buffer, as esp_route_group_rmsnorm's: every bit of
 * logits set (0xFF bytes) on entry, and left so; at one row the last workgroup reads the others' logits once none is
 * all-ones instead of counting arrivals (the counter stays zero), with a bounded wait (~20 ms, then
 * ESP_STATUS_WAIT_TIMEOUT). Bit-identical to esp_route_group. No counterpart in the reference (whose logits are plain
 * scratch): for callers that own a logits buffer across calls. */
int esp_route_group_own(const void* x, int x_dtype, int64_t x_stride, int64_t R, int64_t H, const void* gate,
                        int64_t E, const void* sgate, int64_t k, int64_t shared_id, float* logits,
                        int64_t logits_numel, int32_t* counter, int32_t* pick_out, float* wts_out, int32_t* uids,
                        int64_t maxu, int32_t* ucount, int32_t* members, int64_t maxm, void* stream);

/* esp_route_group's routing for any number of rows, without the grouping: the same logits, picks and weights (a row's
 * routing depends on that row alone; bf16 x bf16 products and their sums are exact in fp64 for ordinary data, so the
 * order of the sums does not show after the rounding), for a whole prompt in two launches: the logits on the fp64
 * matrix cores (16-row x 16-column tiles), then one wave a row for the top-k. No counterpart in the reference, which
 * routes a prompt one 32-token window a launch; for prompts grouped afterwards in one piece (esp_group /
 * esp_group_shared over all rows). pick_out / wts_out [R][k + has]; logits >= R * (E + has) floats. H a multiple of
 * 256, x rows and gate 16-byte aligned, x_stride a multiple of 8. */
int esp_route_rows(const void* x, int x_dtype, int64_t x_stride, int64_t R, int64_t H, const void* gate, int64_t E,
                   const void* sgate, int64_t k, int64_t shared_id, float* logits, int64_t logits_numel,
                   int32_t* pick_out, float* wts_out, void* stream);

/* Replaces `group_shared` (experts.cpp:154-172, experts.cu:247-330, 518-539): pick/weight tables with the shared
 * expert as slot slots_in (weight sigmoid(x . gate_w), fp32), then the grouping. pick_in int32 / wts_in fp32
 * [R][slots_in]; x [R][x_stride] with H columns; gate_w [H] (x's dtype) or NULL; pick_out / wts_out [R * slots].
 * Windows of more than 1056 picks (a whole prompt) are grouped by a workgroup an expert id, with the same tables
 * (maxm <= 16384). */
int esp_group_shared(const int32_t* pick_in, const float* wts_in, const void* x, int x_dtype, int64_t x_stride,
                     int64_t H, const void* gate_w, int64_t shared_id, int32_t* pick_out, float* wts_out,
                     int32_t* uids, int64_t maxu, int32_t* ucount, int32_t* members, int64_t maxm, int64_t R,
                     int64_t slots_in, int64_t E, void* stream);

/* Replaces `group` (experts.cpp:79-90, experts.cu:23-76, 435-455): distinct picks in [0, E) in id order (uids,
 * ucount) and their members row * 32 + slot in pick order, -1 padded to maxm (any window: beyond 1056 picks a
 * workgroup an expert id, maxm <= 16384). */
int esp_group(const int32_t* pick, int32_t* uids, int64_t maxu, int32_t* ucount, int32_t* members, int64_t maxm,
              int64_t R, int64_t slots, int64_t E, void* stream);

/* Replaces `rot_in` (experts.cpp:92-104, experts.cu:97-115, 457-475): out0/out1 fp16 [rows*slots][K] =
 * fp16(H(x[row] * suh0/1[pick]) / sqrt(128)) for every valid pick (0 <= pick < E); x bf16/fp16 [rows][x_stride];
 * suh0/1 fp16 [E][K]. */
int esp_rot_in(const void* x, int x_dtype, int64_t x_stride, const int32_t* pick, const void* suh0, const void* suh1,
               void* out0, void* out1, int64_t rows, int64_t K, int64_t slots, int64_t E, void* stream);

/* Replaces `grouped` (experts.cpp:44-66, experts_grouped.cuh:237-318, 360-377): Z fp32 [mats][SK][P][N] = the K-split
 * partial sums of X_mat[row] @ W_mat[e] for every member row of every distinct expert u < ucount. X0/X1 fp16 [P][K];
 * TP0/TP1 int64 [E] trellis device pointers; B0/B1 int32 [E] K2; C0/C1 int32 [E] codebook ids; uids [nexp_max];
 * members [nexp_max][maxm], maxm any size: an expert's members run in tiles of 32 (the reference's are 16,
 * experts_grouped.cuh:244), each tile decoding the expert's weights once. nt, warps, pf are tile hints; lo/hi bound
 * the K2 of the launch's experts (an expert outside them, or with no kernel, gets NaN partials and a status bit:
 * esp_status). */
int esp_grouped(const void* X0, const void* X1, const int64_t* TP0, const int64_t* TP1, const int32_t* B0,
                const int32_t* B1, const int32_t* C0, const int32_t* C1, const int32_t* uids, int64_t nexp_max,
                const int32_t* ucount, const int32_t* members, int64_t maxm, float* Z, int64_t z_numel, int64_t mats,
                int64_t K, int64_t N, int64_t P, int64_t SK, int64_t slots, int64_t nt, int64_t warps, int64_t pf,
                int64_t lo, int64_t hi, void* stream);

/* esp_grouped over a work list, for groupings of a whole prompt. No counterpart in the reference, which groups a
 * 32-token window at a time: there an expert has at most 32 * slots members, here up to the prompt's length, and a
 * grid of every expert slot times every possible member tile is mostly empty workgroups (at 512 tokens 4112 of which
 * ~400 have members). esp_tile_list writes the non-empty (expert slot u, member tile t) pairs of a grouping (uids,
 * ucount, members as esp_group writes them) into tiles: tiles[0] = their number, tiles[1 + i] = u << 16 | t in (u, t)
 * order; tiles needs 1 + min(nexp_max * ceil(maxm / 32), ceil(P / 32) + nexp_max) ints, and nexp_max *
 * ceil(maxm / 32) <= 32768. Every slot of members [nexp_max][maxm] is read (slots past *ucount are masked). esp_grouped_list then runs esp_grouped's programs for the listed pairs only, with the same
 * arguments (less the tile hints) and the same bits. One list serves every launch over the same grouping. */
int esp_tile_list(const int32_t* ucount, const int32_t* members, int64_t nexp_max, int64_t maxm, int64_t P,
                  int32_t* tiles, int64_t tiles_numel, void* stream);
int esp_grouped_list(const void* X0, const void* X1, const int64_t* TP0, const int64_t* TP1, const int32_t* B0,
                     const int32_t* B1, const int32_t* C0, const int32_t* C1, const int32_t* uids, int64_t nexp_max,
                     const int32_t* ucount, const int32_t* members, int64_t maxm, const int32_t* tiles, float* Z,
                     int64_t z_numel, int64_t mats, int64_t K, int64_t N, int64_t P, int64_t SK, int64_t slots,
                     int64_t warps, int64_t lo, int64_t hi, void* stream);

/* Replaces `gateup_epilogue` (experts.cpp:106-118, experts.cu:120-162, 477-487): per valid pick p, the gate / up
 * splits of Z [2][SK][P][N] summed in order, H, * svh, SwiGLU (act_mode 1: fp32; 0: bf16 roundings; clamped to
 * limit), * suh_d, H -> xd fp16 [P][N]. svh_g/svh_u/suh_d fp16 [E][N]. */
int esp_gateup_epilogue(const float* Z, const int32_t* pick, const void* svh_g, const void* svh_u, const void* suh_d,
                        void* xd, int64_t rows, int64_t P, int64_t N, int64_t SK, int64_t slots, int64_t E,
                        double limit, int64_t act_mode, void* stream);

/* Replaces `down_epilogue` (experts.cpp:120-129, experts.cu:165-184): y fp32 [P][D] = H(sum of Z [SK][P][D]) *
 * svh_d[pick] / sqrt(128) for every valid pick. */
int esp_down_epilogue(const float* Z, const int32_t* pick, const void* svh_d, float* y, int64_t rows, int64_t P,
                      int64_t D, int64_t SK, int64_t slots, int64_t E, void* stream);

/* Replaces `combine` (experts.cpp:131-137, experts.cu:187-195): out fp32 [rows][D] = sum over slots in order of
 * wts * y (fp32 fma chain from 0). */
int esp_combine(const float* y, const float* wts, float* out, int64_t rows, int64_t D, int64_t slots, void* stream);

/* Replaces `down_combine` (experts.cpp:139-151, experts.cu:198-241): down_epilogue then combine over all slots,
 * fp32 out [rows][D]; an invalid pick reuses y's stored row. */
int esp_down_combine(const float* Z, const int32_t* pick, const void* svh_d, float* y, const float* wts, float* out,
                     int64_t rows, int64_t P, int64_t D, int64_t SK, int64_t slots, int64_t E, void* stream);

/* Replaces `down_combine2` (experts.cpp:175-190, experts.cu:340-393, 541-559): as down_combine, the routed sum over
 * the first n_routed slots into out, and w * y of slot n_routed into out_shared (may be NULL), both in out_dtype.
 * y may be NULL here and in esp_down_combine (no counterpart in the reference, whose y is always given): then no
 * slot's output is stored and an invalid pick adds zero instead of y's stored row. */
int esp_down_combine2(const float* Z, const int32_t* pick, const void* svh_d, float* y, const float* wts, void* out,
                      int out_dtype, void* out_shared, int64_t rows, int64_t P, int64_t D, int64_t SK, int64_t slots,
                      int64_t E, int64_t n_routed, void* stream);

/* ---- Fused MoE launch (csrc/moe.hip). No counterpart in the reference extension: a composition of the reference
 * functions above, with the same arithmetic in the same order (bit-identical results), in one launch instead of three.
 * counters: int32 zero on entry and left zero, 32 apart (one 128-byte line each). ---- */

/* rot_in + grouped (mats = 2) + gateup_epilogue in one launch: the member rows of each distinct expert are rotated
 * (x * suh, H) inside the launch, and the last of the 2 * SK programs of an (expert, 128-column block) to arrive runs the
 * gate/up epilogue of its rows into xd fp16 [P][N]. Arguments as esp_rot_in, esp_grouped and esp_gateup_epilogue;
 * (K / SK) % 128 == 0; counters >= nexp_max * (N / 128) * 32; the 2 * SK * P * N partials at most 2^30 floats. */
int esp_moe_gateup(const void* x, int x_dtype, int64_t x_stride, const void* suh_g, const void* suh_u,
                   const int64_t* TP0, const int64_t* TP1, const int32_t* B0, const int32_t* B1, const int32_t* C0,
                   const int32_t* C1, const int32_t* uids, int64_t nexp_max, const int32_t* ucount,
                   const int32_t* members, int64_t maxm, float* Z, int64_t z_numel, int32_t* counters,
                   int64_t counters_numel, const void* svh_g, const void* svh_u, const void* suh_d, void* xd, int64_t K,
                   int64_t N, int64_t P, int64_t SK, int64_t slots, int64_t warps, int64_t lo, int64_t hi,
                   double limit, int64_t act_mode, void* stream);

/* The decode MoE layer after its routing as ONE launch: esp_moe_gateup's fused gate/up programs, the down programs
 * (esp_grouped's, K split into the I / 128 gate/up column blocks) and esp_down_combine2's combine, as three program
 * groups of one grid, each consumer reading inside the launch the pieces it needs as soon as they are stored
 * (bounded waits: past ~20 ms a wait sets ESP_STATUS_WAIT_TIMEOUT instead of hanging). A down program lands and
 * decodes its weights before it reads its xd slice. Bit-identical to esp_moe_gateup + esp_grouped (mats 1, SK =
 * I / 128) + esp_down_combine2. No counterpart in the reference, which launches them apart (experts.py:231-261). The
 * tables as esp_moe_gateup's (TP0, B0, C0 gate; TP1, B1, C1 up) and esp_grouped's down launch (TP2, B2, C2, K2 range
 * [lo_d, hi_d]); members [nexp_max][rows]; 1 <= rows <= 4; I <= 1024; Z >= 2 * SK * P * I floats (gate/up partials),
 * Zd >= (I / 128) * P * D floats (down partials, apart from Z), P = rows * slots; xd fp16 [P][I]; y fp32 [P][D]
 * per-slot outputs; out / out_shared [rows][D] in out_dtype; counters >= nexp_max * (I / 128) * 32 ints and flags >=
 * 32 * 2 * (nexp_max * I / 128 + D / 128) ints, both zero on entry and left zero. xd and Zd are this launch's own
 * hand-off buffers (no other launch may write them): every bit set (0xFF bytes) on entry, and left so. */
int esp_moe_chain(const void* x, int x_dtype, int64_t x_stride, const void* suh_g, const void* suh_u,
                  const int64_t* TP0, const int64_t* TP1, const int64_t* TP2, const int32_t* B0, const int32_t* B1,
                  const int32_t* B2, const int32_t* C0, const int32_t* C1, const int32_t* C2, const int32_t* uids,
                  int64_t nexp_max, const int32_t* ucount, const int32_t* members, int64_t rows, const int32_t* pick,
                  const float* wts, const void* svh_g, const void* svh_u, const void* suh_d, const void* svh_d,
                  void* xd, float* Z, int64_t z_numel, float* Zd, int64_t zd_numel, float* y, void* out,
                  int out_dtype, void* out_shared, int32_t* counters, int64_t counters_numel, int32_t* flags,
                  int64_t flags_numel, int64_t D, int64_t I, int64_t SK, int64_t slots, int64_t E, int64_t n_routed,
                  int64_t lo, int64_t hi, int64_t lo_d, int64_t hi_d, double limit, int64_t act_mode, void* stream);

/* esp_dense with the input rows normalised in the launch: x = RMSNorm(h + d1 + d2) * norm_w (d1, d2 may be NULL),
 * bit-identical to esp_add_rmsnorm followed by esp_dense; the residual h + d1 + d2 is stored to h_out (not h: other
 * workgroups still read h). No counterpart in the reference (vLLM runs the norm as its own launch). M <= W / 4,
 * K <= 8192, bf16/fp16 rows x_stride apart, the fused rotation (M * K / SK * 2 <= rot_smem); no xh. */
int esp_dense_rmsnorm(const void* h, const void* d1, const void* d2, const void* norm_w, double eps, void* h_out,
                      int x_dtype, int64_t x_stride, int64_t M, int64_t K, int64_t n_shards, const void* const* trellis,
                      const void* const* suh, const void* const* svh, const int64_t* n_cols, const int64_t* col0,
                      void* y, int y_dtype, int64_t y_stride, int64_t y_cols, float* Z, int64_t z_numel,
                      int32_t* counters, int64_t counters_numel, int64_t k2, int64_t cb, int64_t SK, int64_t W,
                      int64_t rot_smem, void* stream);

/* esp_route_group with the router input normalised in the launch: x = RMSNorm(h + d1) * norm_w, bit-identical to
 * esp_add_rmsnorm followed by esp_route_group; x is stored to a_out and the residual h + d1 to h_out. No counterpart in
 * the reference. R <= 4, H <= 8192, rows x_stride apart, 16-byte aligned. Unlike esp_route_group's, logits is this
 * launch's own hand-off buffer (no other launch may write it): every bit set (0xFF bytes) on entry, and left so. At one
 * row the last workgroup reads the others' logits once none is all-ones (no arrival count; counter stays zero), with
 * a bounded wait (~20 ms, then ESP_STATUS_WAIT_TIMEOUT). */
int esp_route_group_rmsnorm(const void* h, const void* d1, const void* norm_w, double eps, void* h_out, void* a_out,
                            int x_dtype, int64_t x_stride, int64_t R, int64_t H, const void* gate, int64_t E,
                            const void* sgate, int64_t k, int64_t shared_id, float* logits, int64_t logits_numel,
                            int32_t* counter, int32_t* pick_out, float* wts_out, int32_t* uids, int64_t maxu,
                            int32_t* ucount, int32_t* members, int64_t maxm, void* stream);

/* One group of esp_dense_multi: the arguments of one esp_dense launch (x, the matrices, y, k2 / cb / SK), plus
 * after_previous: x is (a view of) the previous group's y, read once every column block of that group is finished;
 * and an optional RMSNorm of the input as esp_dense_rmsnorm has it (norm_h non-NULL; not with after_previous). */
typedef struct esp_dense_group {
    const void* x;
    int x_dtype;
    int64_t x_stride, K, n_shards;
    const void* trellis[4];
    const void* suh[4];
    const void* svh[4];
    int64_t n_cols[4], col0[4];
    void* y;
    int y_dtype;
    int64_t y_stride, y_cols, k2, cb, SK;
    int after_previous;
    const void* norm_h;
    const void* norm_d1;
    const void* norm_d2;
    const void* norm_w;
    void* norm_h_out;
    double norm_eps;
} esp_dense_group;

/* Up to 4 dense launches (esp_dense's arithmetic and bits, group by group) in one launch, with M <= 32 rows and W waves
 * a workgroup for every group. No counterpart in the reference, which launches each vLLM layer on its own: this runs a
 * layer's dense launches -- independent ones side by side, or a chain such as qkv then o (after_previous) -- as one
 * grid, so one launch gap and one weight-landing latency serve them all. A consumer group's x must be whole 128-column
 * blocks of the producer's y (same dtype and row stride, x - y a multiple of 128 elements, every column an output of
 * the producer). Its workgroups issue their first trellis copies, then wait for just the producer column blocks that
 * hold their K range (the producer's finishers store y device-coherently and count their block done); workgroups are
 * dispatched in id order and producers come first, so the waits end, and a wait past ~20 ms sets
 * ESP_STATUS_WAIT_TIMEOUT (esp_status) instead of hanging. Every group's input rotation must be the fused one
 * (M * (K / SK) * 2 <= rot_smem). Scratch: Z (z_numel >= sum over groups of SK * M * sum(n_cols), each rounded up to
 * 64 floats; at most 2^30 floats a group), counters (8-byte aligned, counters_numel >= 96 * B with B = sum over groups
 * of sum(n_cols)/128; zero before a buffer's first launch. The first 32 * B ints, split-K arrivals, are left zero; the
 * rest hold 64-bit running counts of the chain's hand-offs, two a column block, which only grow, so one buffer serves
 * one chain of groups for the life of the process). */
int esp_dense_multi(int64_t n_groups, const esp_dense_group* groups, int64_t M, int64_t W, float* Z, int64_t z_numel,
                    int32_t* counters, int64_t counters_numel, int64_t rot_smem, void* stream);

/* esp_dense without caller scratch, for callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference. Arguments and results as esp_dense (the
 * same kernels, the same bits); the arrival counters, the split-K partials Z and the unfused rotation's rows live in a
 * 16 MiB device array of the library, one per GPU, held until the process ends. A launch needing more than that
 * (64 KiB of counters, then SK * M * sum(n_cols) * 4 bytes of partials rounded to 256, then n_shards * M * K * 2 bytes
 * when the rotation is not fused) fails with ESP_ERR_ARG. Nothing is allocated and nothing but the GEMM is launched:
 * the array's address is looked up on a device's first call; its counters start zero (the array has no initializer, so
 * it is zero-filled where the library's code is loaded) and every launch leaves them zero. Calls on one GPU share the
 * array, so calls that overlap in time (on different streams, or from different threads) race. */
int esp_dense_noalloc(const void* x, int x_dtype, int64_t x_stride, int64_t M, int64_t K, int64_t n_shards,
                      const void* const* trellis, const void* const* suh, const void* const* svh,
                      const int64_t* n_cols, const int64_t* col0, void* y, int y_dtype, int64_t y_stride,
                      int64_t y_cols, int64_t k2, int64_t cb, int64_t SK, int64_t W, int64_t PF, int64_t rot_smem,
                      void* stream);

/* ---- Decode-step glue (csrc/step.hip). No counterpart in the reference extension: in a served model vLLM does
 * these (VocabParallelEmbedding, fused_add_rms_norm, the greedy sampler). They let the synthetic decoder step run as
 * one HIP graph whose next token stays on the device. ---- */

/* h [T][D] = table [vocab][D] rows ids[t] (int32 on the device); an id outside [0, vocab) gives a zero row. bf16 or
 * fp16 (16-bit copy). D % 8 == 0; table and h 16-byte aligned. */
int esp_embed(const int32_t* ids, const void* table, int64_t vocab, void* h, int64_t T, int64_t D, void* stream);

/* Residual add and RMSNorm: z = h + d1 + d2 in fp32 (d1, d2 may be NULL), h = z in dtype (left as is without
 * deltas), out = (h * (1 / sqrt(mean(h^2) + eps))) * w in dtype, h as stored. dtype ESP_BF16 or ESP_F16; [T][D]
 * row-major, D % 8 == 0, D <= 8192, 16-byte aligned. */
int esp_add_rmsnorm(void* h, const void* d1, const void* d2, const void* w, void* out, int64_t T, int64_t D,
                    double eps, int dtype, void* stream);

/* ids[t] = argmax of logits row t (rows of `stride` elements, N used), the lowest index among equal maxima, a NaN
 * counting as the largest (torch.argmax). dtype ESP_BF16 or ESP_F16; rows 16-byte aligned. With scratch (part: at
 * least T * ceil(N / 4096) int64 keys; counters: T * 32 int32, zero on entry and left zero) a row is split over
 * workgroups of 4096 elements and the last to arrive reduces their keys; without (both NULL), one workgroup a row.
 * The same ids either way. */
int esp_argmax(const void* logits, int64_t stride, int64_t T, int64_t N, int dtype, int32_t* ids, int64_t* part,
               int64_t part_numel, int32_t* counters, int64_t counters_numel, void* stream);

#ifdef __cplusplus
}
#endif
#endif

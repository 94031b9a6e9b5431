/* CPU oracle for the vllm-espalier trellis kernel layer -- TEST INFRASTRUCTURE ONLY.
 *
 * This library restates, in plain C, the arithmetic of the reference's hot path so that the HIP kernels can be
 * checked against it. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only as
 * the checker (or the timed CPU baseline); the product path never calls it.
 *
 * Every function cites the reference file:line it follows (paths relative to the reference repository root).
 * fp16 / bf16 values travel as their uint16 bit patterns.
 */
#ifndef ESPALIER_ORACLE_H
#define ESPALIER_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- IEEE conversions (round to nearest even, subnormals kept) ---- */
uint16_t eo_f32_to_f16(float f);
float eo_f16_to_f32(uint16_t h);
uint16_t eo_f32_to_bf16(float f);
uint16_t eo_f64_to_bf16(double d);
float eo_bf16_to_f32(uint16_t b);

/* ---- codebooks: vllm_espalier/csrc/experts_grouped.cuh:23-80 ---- */
uint16_t eo_mcg(uint32_t state);                 /* cb 1 */
uint16_t eo_e2m1(uint32_t state);                /* cb 3 */
int eo_grid_q(uint32_t state, int cb);           /* int5 (6 / 22) or int6 (7 / 23) grid index q */
uint16_t eo_decode(uint32_t state, int cb);      /* cb 1, 3, 6, 7, 22, 23; 0xFFFF-free: returns the value bits */
int eo_supported(int cb, int k2);                /* the compiled (cb, K2) set, experts_grouped.cuh:227-229 */

/* ---- trellis state unpack: experts_grouped.cuh:83-154 ---- */
uint32_t eo_state(const uint32_t* tile_words, int k2, int p);   /* state p (0..255) of one 16x16 tile */
void eo_position(int p, int* k, int* n);                         /* placement of state p inside the tile */

/* ---- dequant: experts_grouped.cuh:321-340. trellis int16 [K/16][N/16][8*k2]; out fp16 bits [K][N].
 *      Returns 0, or -1 for an unsupported (cb, k2). threads <= 0 uses every core. */
int eo_dequant(const int16_t* trellis, int K, int N, int k2, int cb, uint16_t* out, int threads);
/* dequant into fp32 (the decoded fp16 values widened), same contract. */
int eo_dequant_f32(const int16_t* trellis, int K, int N, int k2, int cb, float* out, int threads);

/* ---- Walsh-Hadamard over 128 fp32 values in the reference's butterfly order: experts.cu:79-90, dense.cu:43-54 ---- */
void eo_fwht128(float* v);

/* ---- had: dense.cu:242-265. x, y fp16 [M][K]; pre / post fp16 [K] or NULL. */
void eo_had(const uint16_t* x, const uint16_t* pre, const uint16_t* post, uint16_t* y, int M, int K);

/* ---- input rotation: dense.cu:92-108 / experts.cu:97-115. x in dtype (0 f16, 1 bf16, 2 f32) [M][x_stride];
 *      out fp16 [M][K] = fp16(H(x * suh) / sqrt(128)). */
void eo_rotate(const void* x, int x_dtype, int x_stride, const uint16_t* suh, uint16_t* out, int M, int K);

/* ---- grouping: experts.cu:23-76 (group_kernel) and route.cu:132-180.
 *      pick [n] (n = R * slots); ids counted in [0, E). Writes uids[0..count), members[count][maxm]
 *      (code row*32+slot, -1 pad). Returns count. */
int eo_group(const int* pick, int R, int slots, int E, int maxm, int* uids, int* members);

/* ---- routing (route.cu:35-181, as exact routing): x [R][H] bf16, gate [E][H] bf16, sgate [H] bf16 or NULL.
 *      logits: exactly rounded bf16 of the exact dot products (ties to even); top-k by logit (lowest id on ties);
 *      weights p/sum renormalised over the picks in fp64; shared slot sigmoid of the exact shared-gate dot.
 *      pick/wts [R][k + has]. logit_bits [R][E] (bf16 bits) and shared_logit [R] (fp64) are outputs for tests. */
void eo_route(const uint16_t* x, const uint16_t* gate, const uint16_t* sgate, int R, int H, int E, int k,
              int shared_id, int* pick, double* wts, uint16_t* logit_bits, double* shared_logit);
/* the exact dot product of two bf16 vectors, correctly rounded to fp64 (Shewchuk expansion). */
double eo_dot_bf16_exact(const uint16_t* a, const uint16_t* b, int n, int* sign_of_residual);

/* ---- epilogues of the grouped expert pipeline (fp32, the reference's operation order) ---- */
/* experts.cu:120-162. Z [2][SK][P][N] fp32; pick [P]; svh_g, svh_u [E][N] fp16; suh_d [E][N] fp16; xd fp16 [P][N]. */
void eo_gateup_epilogue(const float* Z, const int* pick, const uint16_t* svh_g, const uint16_t* svh_u,
                        const uint16_t* suh_d, uint16_t* xd, int P, int N, int SK, int E, float limit, int act_mode);
/* experts.cu:340-393. Z [SK][P][D]; y [P][D] fp32 (read for invalid picks, written for valid ones); wts [R*slots];
 *      out / out_shared [R][D] as fp32 values (the caller rounds to its dtype). */
void eo_down_combine2(const float* Z, const int* pick, const uint16_t* svh_d, float* y, const float* wts,
                      float* out, float* out_shared, int rows, int P, int D, int SK, int E, int slots, int n_routed);

#ifdef __cplusplus
}
#endif
#endif

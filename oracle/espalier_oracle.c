/* CPU oracle for the vllm-espalier trellis kernel layer -- TEST INFRASTRUCTURE ONLY (see espalier_oracle.h).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp). The floating-point restatements rely on
 * FLT_EVAL_METHOD == 0 (x86-64 SSE): every float expression is evaluated in single precision, as on the GPU.
 */
#include "espalier_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#if defined(_OPENMP)
#include <omp.h>
#endif

#if !defined(__FLT_EVAL_METHOD__) || __FLT_EVAL_METHOD__ != 0
#error "the oracle needs single-precision float evaluation (FLT_EVAL_METHOD 0)"
#endif

/* 1 / sqrt(128) as the reference writes it: dense.cu:23, experts.cu:17 */
static const float HAD_SCALE = 0.08838834764831845f;

/* ------------------------------------------------------------------------------------------------------------ */
/* IEEE conversions                                                                                             */
/* ------------------------------------------------------------------------------------------------------------ */

uint16_t eo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return sign | 0x7E00u;          /* NaN */
    if (ax >= 0x477FF000u) return sign | 0x7C00u;         /* >= 65520 rounds to infinity */
    if (ax >= 0x38800000u) {                              /* normal fp16: >= 2^-14 */
        const uint32_t e = (ax >> 23) - 112u;
        const uint32_t m = ax & 0x7FFFFFu;
        uint32_t h = (e << 10) | (m >> 13);
        const uint32_t r = m & 0x1FFFu;
        if (r > 0x1000u || (r == 0x1000u && (h & 1u))) h += 1u;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return sign;                    /* below 2^-25 (2^-25 itself ties to 0) */
    const uint32_t e = ax >> 23;                          /* 102..112 */
    const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - e;                      /* to units of 2^-24 */
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float eo_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {                                          /* subnormal: m * 2^-24, exact in fp32 */
            float f = (float)m * 5.9604644775390625e-08f;
            memcpy(&x, &f, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t eo_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float eo_bf16_to_f32(uint16_t b) {
    const uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* double -> bf16 with a single rounding (no pass through fp32). dir is the sign of (exact - d) when d stands for
 * a more precise value: it only matters when d lies exactly halfway between two bf16 values. */
static uint16_t f64_to_bf16_dir(double d, int dir) {
    uint64_t x;
    memcpy(&x, &d, 8);
    const uint16_t sign = (uint16_t)((x >> 48) & 0x8000u);
    const uint64_t ax = x & 0x7FFFFFFFFFFFFFFFull;
    if (ax > 0x7FF0000000000000ull) return sign | 0x7FC0u;
    if (ax == 0x7FF0000000000000ull) return sign | 0x7F80u;
    const int e = (int)(ax >> 52);
    if (e == 0) return sign;                              /* fp64 subnormals are far below the bf16 range */
    int E = e - 1023 + 127;                               /* bf16 biased exponent */
    if (E >= 255) return sign | 0x7F80u;
    const uint64_t m = (ax & ((1ull << 52) - 1)) | (1ull << 52);
    const int shift = E >= 1 ? 45 : 45 + (1 - E);
    if (shift > 54) return sign;
    uint64_t q = m >> shift;
    const uint64_t rem = m & ((1ull << shift) - 1), half = 1ull << (shift - 1);
    int up;
    if (rem != half) {
        up = rem > half;
    } else if (dir == 0) {
        up = (int)(q & 1u);                               /* a true tie: to even */
    } else {
        up = (dir > 0) == (sign == 0);                    /* the exact value is beyond the midpoint in magnitude */
    }
    q += (uint64_t)up;
    uint32_t bits;
    if (E >= 1) {
        if (q == 256) {
            q = 128;
            E += 1;
            if (E >= 255) return sign | 0x7F80u;
        }
        bits = ((uint32_t)E << 7) | (uint32_t)(q & 0x7Fu);
    } else {
        bits = (uint32_t)q;                               /* q == 128 is the smallest normal, bits 0x0080 */
    }
    return (uint16_t)(sign | bits);
}

uint16_t eo_f64_to_bf16(double d) { return f64_to_bf16_dir(d, 0); }

/* ------------------------------------------------------------------------------------------------------------ */
/* codebooks: experts_grouped.cuh:21-80                                                                         */
/* ------------------------------------------------------------------------------------------------------------ */

/* fp16 + fp16 with one RNE rounding. Both operands of the mcg sum have exponents in [-3, 0], so the float sum is
 * exact and the only rounding is the final one to fp16, as in __hadd2. */
static uint16_t h_add(uint16_t a, uint16_t b) {
    return eo_f32_to_f16(eo_f16_to_f32(a) + eo_f16_to_f32(b));
}

/* cb 1 (mcg): experts_grouped.cuh:64-79 -- x = s * 0xCBAC1FED; (x & 0x8FFF8FFF) ^ 0x3B603B60; lo half + hi half */
uint16_t eo_mcg(uint32_t s) {
    uint32_t x = s * 0xCBAC1FEDu;
    x = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
    return h_add((uint16_t)(x & 0xFFFFu), (uint16_t)(x >> 16));
}

/* cb 3 (E2M1 snap of mcg): experts_grouped.cuh:25-38 with ESP_E2M1_C = 0.75 (:21). Every partial sum of the
 * step chain is exact in fp16, so the float sums below carry the same values; the sign of the mcg value is OR-ed in
 * (so -0.0 occurs). */
uint16_t eo_e2m1(uint32_t s) {
    const uint16_t m = eo_mcg(s);
    const float a = eo_f16_to_f32((uint16_t)(m & 0x7FFFu));
    const float C = 0.75f;
    float acc = (a > 0.25f * C) ? 0.5f * C : 0.0f;
    acc += (a > 0.75f * C) ? 0.5f * C : 0.0f;
    acc += (a > 1.25f * C) ? 0.5f * C : 0.0f;
    acc += (a > 1.75f * C) ? 0.5f * C : 0.0f;
    acc += (a > 2.5f * C) ? 1.0f * C : 0.0f;
    acc += (a > 3.5f * C) ? 1.0f * C : 0.0f;
    acc += (a > 5.0f * C) ? 2.0f * C : 0.0f;
    return (uint16_t)(eo_f32_to_f16(acc) | (m & 0x8000u));
}

/* int5 / int6 grid index: experts_grouped.cuh:39-55 -- q = rintf(f32(mcg) * k) */
int eo_grid_q(uint32_t s, int cb) {
    const float k = (cb == 6 || cb == 22) ? 0x1.e62c10p+1f : 0x1.f660bap+2f;
    const float v = eo_f16_to_f32(eo_mcg(s));
    return (int)rintf(v * k);
}

uint16_t eo_decode(uint32_t s, int cb) {
    switch (cb) {
        case 1: return eo_mcg(s);
        case 3: return eo_e2m1(s);
        case 6:
        case 7: {
            /* fp16(q * c), c = 3.94921875f / top: experts_grouped.cuh:41,47 */
            const float c = 3.94921875f / (cb == 6 ? 15.0f : 31.0f);
            return eo_f32_to_f16((float)eo_grid_q(s, cb) * c);
        }
        case 22:
        case 23: return eo_f32_to_f16((float)eo_grid_q(s, cb));   /* :49-55 */
        /* 19: not a reference codebook; the GEMMs' unscaled E2M1 form (the value / 0.75, exact), checked against it */
        case 19: return eo_f32_to_f16(eo_f16_to_f32(eo_e2m1(s)) / 0.75f);
        default: return 0x7E00u;
    }
}

/* ESP_CASES, experts_grouped.cuh:227-229 */
int eo_supported(int cb, int k2) {
    if (cb == 1) return k2 >= 2 && k2 <= 16 && (k2 % 2) == 0;
    if (cb == 3) return k2 == 2 || k2 == 4 || k2 == 6;
    if (cb == 6) return k2 == 4 || k2 == 6 || k2 == 8;
    if (cb == 7) return k2 == 6 || k2 == 8 || k2 == 10;
    return 0;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* trellis unpack: experts_grouped.cuh:83-154                                                                   */
/* ------------------------------------------------------------------------------------------------------------ */

/* Fmt<K2>::end (:90): the stream bit at which window p ends */
static int fmt_end(int k2, int p) { return (p >> 1) * k2 + ((p & 1) ? k2 : (k2 >> 1)); }

/* The tile's TW = 4*K2 words are one circular big-endian bit stream of L = 128*K2 bits: stream bit j is bit
 * 31 - (j mod 32) of word j / 32 (the word order of LaneMap's hi/lo merge, :102-107). State p is the 16 stream bits
 * ending at fmt_end(p), the earliest bit most significant (decode_tile's shift-and-mask, :145-147). */
uint32_t eo_state(const uint32_t* w, int k2, int p) {
    const int L = 128 * k2, e = fmt_end(k2, p);
    uint32_t s = 0;
    for (int i = 16; i >= 1; --i) {
        const int j = ((e - i) % L + L) % L;
        s = (s << 1) | ((w[j >> 5] >> (31 - (j & 31))) & 1u);
    }
    return s;
}

/* dequant_kernel's placement (:330-338): lane = p / 8, j = p % 8, q = j / 2, t = lane % 4, g = lane / 4;
 * row 2t + 8(q & 1) + (j & 1), column g + 8(q >> 1). */
void eo_position(int p, int* k, int* n) {
    const int lane = p >> 3, j = p & 7, q = j >> 1, t = lane & 3, g = lane >> 2;
    *k = 2 * t + 8 * (q & 1) + (j & 1);
    *n = g + 8 * (q >> 1);
}

static int dequant_any(const int16_t* trellis, int K, int N, int k2, int cb, uint16_t* out16, float* out32,
                       int threads) {
    /* 22 / 23 decode the int5 / int6 index q at the widths of 6 / 7 */
    if (!eo_supported(cb >= 22 ? cb - 16 : cb == 19 ? 3 : cb, k2) || K % 16 || N % 16) return -1;
    const int KT = K / 16, NT = N / 16, TW = 4 * k2;
    int pos_k[256], pos_n[256];
    for (int p = 0; p < 256; ++p) eo_position(p, &pos_k[p], &pos_n[p]);
#if defined(_OPENMP)
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
    for (int kt = 0; kt < KT; ++kt) {
        uint32_t w[64];
        for (int nt = 0; nt < NT; ++nt) {
            memcpy(w, trellis + ((size_t)kt * NT + nt) * (size_t)(2 * TW), (size_t)TW * 4);
            for (int p = 0; p < 256; ++p) {
                const uint16_t v = eo_decode(eo_state(w, k2, p), cb);
                const size_t at = (size_t)(kt * 16 + pos_k[p]) * N + (size_t)(nt * 16 + pos_n[p]);
                if (out16) out16[at] = v;
                if (out32) out32[at] = eo_f16_to_f32(v);
            }
        }
    }
    return 0;
}

int eo_dequant(const int16_t* trellis, int K, int N, int k2, int cb, uint16_t* out, int threads) {
    return dequant_any(trellis, K, N, k2, cb, out, NULL, threads);
}

int eo_dequant_f32(const int16_t* trellis, int K, int N, int k2, int cb, float* out, int threads) {
    return dequant_any(trellis, K, N, k2, cb, NULL, out, threads);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Hadamard: experts.cu:79-90 (the same butterfly as dense.cu:43-54)                                            */
/* ------------------------------------------------------------------------------------------------------------ */

/* Natural-order FWHT with the strides in increasing order (1, 2 inside a lane, then 4..64 across lanes in the
 * reference); the lower element of each pair takes a + b, the upper a - b. */
void eo_fwht128(float* v) {
    for (int h = 1; h < 128; h <<= 1)
        for (int i = 0; i < 128; i += 2 * h)
            for (int j = i; j < i + h; ++j) {
                const float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
}

/* had_kernel, dense.cu:242-265: y = fp16(H(x * pre) * HAD_SCALE * post) */
void eo_had(const uint16_t* x, const uint16_t* pre, const uint16_t* post, uint16_t* y, int M, int K) {
    float v[128];
    for (int r = 0; r < M; ++r)
        for (int b = 0; b < K; b += 128) {
            for (int j = 0; j < 128; ++j) {
                v[j] = eo_f16_to_f32(x[(size_t)r * K + b + j]);
                if (pre) v[j] = v[j] * eo_f16_to_f32(pre[b + j]);
            }
            eo_fwht128(v);
            for (int j = 0; j < 128; ++j) {
                float o = v[j] * HAD_SCALE;
                if (post) o = o * eo_f16_to_f32(post[b + j]);
                y[(size_t)r * K + b + j] = eo_f32_to_f16(o);
            }
        }
}

static float load_any(const void* p, int dtype, size_t i) {
    if (dtype == 2) return ((const float*)p)[i];
    if (dtype == 1) return eo_bf16_to_f32(((const uint16_t*)p)[i]);
    return eo_f16_to_f32(((const uint16_t*)p)[i]);
}

/* rot128, dense.cu:92-108 / rot_in_kernel, experts.cu:97-115: fp16(H(x * suh) * HAD_SCALE) */
void eo_rotate(const void* x, int x_dtype, int x_stride, const uint16_t* suh, uint16_t* out, int M, int K) {
    float v[128];
    for (int r = 0; r < M; ++r)
        for (int b = 0; b < K; b += 128) {
            for (int j = 0; j < 128; ++j)
                v[j] = load_any(x, x_dtype, (size_t)r * x_stride + b + j) * eo_f16_to_f32(suh[b + j]);
            eo_fwht128(v);
            for (int j = 0; j < 128; ++j) out[(size_t)r * K + b + j] = eo_f32_to_f16(v[j] * HAD_SCALE);
        }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* grouping: experts.cu:19-76, route.cu:132-180                                                                 */
/* ------------------------------------------------------------------------------------------------------------ */

int eo_group(const int* pick, int R, int slots, int E, int maxm, int* uids, int* members) {
    const int n = R * slots;
    int count = 0;
    for (int e = 0; e < E; ++e) {
        int j = 0, hit = 0;
        for (int i = 0; i < n; ++i)
            if (pick[i] == e) {
                hit = 1;
                if (j < maxm) members[count * maxm + j++] = (i / slots) * 32 + (i % slots);
            }
        if (!hit) continue;
        for (; j < maxm; ++j) members[count * maxm + j] = -1;
        uids[count++] = e;
    }
    return count;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* exact routing                                                                                                */
/* ------------------------------------------------------------------------------------------------------------ */

/* Shewchuk's non-overlapping expansion (the algorithm of Python's math.fsum). */
typedef struct {
    double p[64];
    int n;
} expansion;

static void exp_add(expansion* s, double x) {
    int i = 0;
    for (int j = 0; j < s->n; ++j) {
        double y = s->p[j];
        if (fabs(x) < fabs(y)) {
            const double t = x;
            x = y;
            y = t;
        }
        const double hi = x + y, lo = y - (hi - x);
        if (lo != 0.0) s->p[i++] = lo;
        x = hi;
    }
    s->p[i++] = x;
    s->n = i;
}

/* correctly rounded fp64 value of the expansion (math.fsum's final step) */
static double exp_round(const expansion* s) {
    int n = s->n;
    double hi = 0.0, lo = 0.0;
    if (n > 0) {
        hi = s->p[--n];
        while (n > 0) {
            const double x = hi, y = s->p[--n];
            hi = x + y;
            const double yr = hi - x;
            lo = y - yr;
            if (lo != 0.0) break;
        }
        if (n > 0 && ((lo < 0.0 && s->p[n - 1] < 0.0) || (lo > 0.0 && s->p[n - 1] > 0.0))) {
            const double y = lo * 2.0, x = hi + y, yr = x - hi;
            if (y == yr) hi = x;
        }
    }
    return hi;
}

/* sign of (exact - d) */
static int exp_residual_sign(const expansion* s, double d) {
    expansion t = *s;
    exp_add(&t, -d);
    for (int i = t.n - 1; i >= 0; --i)
        if (t.p[i] != 0.0) return t.p[i] > 0.0 ? 1 : -1;
    return 0;
}

double eo_dot_bf16_exact(const uint16_t* a, const uint16_t* b, int n, int* sign_of_residual) {
    expansion s;
    s.n = 0;
    for (int i = 0; i < n; ++i) {
        /* a bf16 x bf16 product has at most 16 significant bits: exact in fp64 */
        const double pr = (double)eo_bf16_to_f32(a[i]) * (double)eo_bf16_to_f32(b[i]);
        if (pr != 0.0) exp_add(&s, pr);
        if (s.n > 60) {                                   /* keep the expansion short: renormalise */
            expansion t;
            t.n = 0;
            for (int j = 0; j < s.n; ++j) exp_add(&t, s.p[j]);
            s = t;
        }
    }
    const double d = exp_round(&s);
    if (sign_of_residual) *sign_of_residual = exp_residual_sign(&s, d);
    return d;
}

/* bf16 of the exact value given its correctly rounded fp64 d and the sign of (exact - d): the exact value and d
 * round alike except when d is itself a bf16 midpoint, where the residual decides. */
static uint16_t bf16_of_exact(double d, int residual_sign) { return f64_to_bf16_dir(d, residual_sign); }

void eo_route(const uint16_t* x, const uint16_t* gate, const uint16_t* sgate, int R, int H, int E, int k,
              int shared_id, int* pick, double* wts, uint16_t* logit_bits, double* shared_logit) {
    const int has = shared_id >= 0, slots = k + has;
    float* l = (float*)malloc(sizeof(float) * (size_t)E);
    unsigned char* used = (unsigned char*)malloc((size_t)E);
    for (int r = 0; r < R; ++r) {
        for (int e = 0; e < E; ++e) {
            int sg = 0;
            const double d = eo_dot_bf16_exact(x + (size_t)r * H, gate + (size_t)e * H, H, &sg);
            const uint16_t b = bf16_of_exact(d, sg);
            if (logit_bits) logit_bits[(size_t)r * E + e] = b;
            l[e] = eo_bf16_to_f32(b);
            used[e] = 0;
        }
        /* top-k by logit, lowest id on ties: the order of softmax probabilities of the bf16 logits (route.cu:97-117,
         * which takes argmax over p = expf(l - max) with the lowest id on ties) */
        double mx = -INFINITY;
        for (int e = 0; e < E; ++e) mx = l[e] > mx ? l[e] : mx;
        double psum = 0.0;
        double ps[32];
        for (int t = 0; t < k; ++t) {
            int be = -1;
            for (int e = 0; e < E; ++e)
                if (!used[e] && (be < 0 || l[e] > l[be])) be = e;
            used[be] = 1;
            pick[r * slots + t] = be;
            ps[t] = exp((double)l[be] - mx);
            psum += ps[t];
        }
        for (int t = 0; t < k; ++t) wts[r * slots + t] = ps[t] / psum;
        if (has) {
            const double sd = eo_dot_bf16_exact(x + (size_t)r * H, sgate, H, NULL);
            if (shared_logit) shared_logit[r] = sd;
            pick[r * slots + k] = shared_id;
            wts[r * slots + k] = 1.0 / (1.0 + exp(-sd));
        }
    }
    free(l);
    free(used);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* grouped-pipeline epilogues (fp32, the reference's operation order)                                          */
/* ------------------------------------------------------------------------------------------------------------ */

static float bf16r(float x) { return eo_bf16_to_f32(eo_f32_to_bf16(x)); }

/* gateup_epilogue_kernel, experts.cu:120-162 */
void eo_gateup_epilogue(const float* Z, const int* pick, const uint16_t* svh_g, const uint16_t* svh_u,
                        const uint16_t* suh_d, uint16_t* xd, int P, int N, int SK, int E, float limit, int act_mode) {
    float gv[128], uv[128], v[128];
    for (int p = 0; p < P; ++p) {
        const int e = pick[p];
        if (e < 0 || e >= E) continue;
        for (int b = 0; b < N; b += 128) {
            for (int j = 0; j < 128; ++j) {
                float sg = 0.f, su = 0.f;
                for (int s = 0; s < SK; ++s) {
                    sg += Z[((size_t)(0 * SK + s) * P + p) * N + b + j];
                    su += Z[((size_t)(1 * SK + s) * P + p) * N + b + j];
                }
                gv[j] = sg;
                uv[j] = su;
            }
            eo_fwht128(gv);
            eo_fwht128(uv);
            for (int j = 0; j < 128; ++j) {
                const size_t at = (size_t)e * N + b + j;
                float act;
                if (act_mode == 0) {
                    const float gg = fminf(bf16r(gv[j] * HAD_SCALE * eo_f16_to_f32(svh_g[at])), limit);
                    const float uu = fminf(fmaxf(bf16r(uv[j] * HAD_SCALE * eo_f16_to_f32(svh_u[at])), -limit), limit);
                    act = bf16r(bf16r(gg / (1.f + expf(-gg))) * uu);
                } else {
                    const float gg = fminf(gv[j] * HAD_SCALE * eo_f16_to_f32(svh_g[at]), limit);
                    const float uu = fminf(fmaxf(uv[j] * HAD_SCALE * eo_f16_to_f32(svh_u[at]), -limit), limit);
                    act = gg / (1.f + expf(-gg)) * uu;
                }
                v[j] = act * eo_f16_to_f32(suh_d[at]);
            }
            eo_fwht128(v);
            for (int j = 0; j < 128; ++j) xd[(size_t)p * N + b + j] = eo_f32_to_f16(v[j] * HAD_SCALE);
        }
    }
}

/* down_combine2_kernel, experts.cu:340-393 */
void eo_down_combine2(const float* Z, const int* pick, const uint16_t* svh_d, float* y, const float* wts,
                      float* out, float* out_shared, int rows, int P, int D, int SK, int E, int slots, int n_routed) {
    float v[128];
    float* part = (float*)malloc(sizeof(float) * 128 * (size_t)slots);
    for (int r = 0; r < rows; ++r)
        for (int b = 0; b < D; b += 128) {
            for (int k = 0; k < slots; ++k) {
                const int p = r * slots + k, e = pick[p];
                if (e >= 0 && e < E) {
                    for (int j = 0; j < 128; ++j) {
                        float s = 0.f;
                        for (int q = 0; q < SK; ++q) s += Z[((size_t)q * P + p) * D + b + j];
                        v[j] = s;
                    }
                    eo_fwht128(v);
                    for (int j = 0; j < 128; ++j) {
                        const float o = v[j] * HAD_SCALE * eo_f16_to_f32(svh_d[(size_t)e * D + b + j]);
                        y[(size_t)p * D + b + j] = o;
                        part[k * 128 + j] = o;
                    }
                } else {
                    for (int j = 0; j < 128; ++j) part[k * 128 + j] = y[(size_t)p * D + b + j];
                }
            }
            for (int j = 0; j < 128; ++j) {
                float acc = 0.f;
                for (int q = 0; q < n_routed; ++q) acc = fmaf(wts[r * slots + q], part[q * 128 + j], acc);
                out[(size_t)r * D + b + j] = acc;
                if (out_shared && n_routed < slots)
                    out_shared[(size_t)r * D + b + j] = wts[r * slots + n_routed] * part[n_routed * 128 + j];
            }
        }
    free(part);
}

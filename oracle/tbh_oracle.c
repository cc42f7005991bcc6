/*
 * tbh_oracle.c -- CPU restatement of TinyBrain's INT8/INT4 quantized-matmul
 * path (vivekptnk/tinybrain, Swift).  TEST INFRASTRUCTURE: the checker for the
 * HIP backend, never part of the product.  Built with -ffp-contract=off so
 * that every fp32 expression rounds exactly as the Swift source does (Swift
 * does not contract a*b+c into an FMA).
 *
 * Parity pins for each function are listed in tests/test_oracle.py.
 */
#include "tbh_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Float.leastNonzeroMagnitude (the smallest positive subnormal). */
#define SWIFT_LEAST_NONZERO FLT_TRUE_MIN

static double now_seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* ------------------------------------------------------------------------ */
/* Synthetic inputs.  Not a reference function: the reference's generator    */
/* (SeededGenerator LCG, ModelWeights.swift:18-29, fed through Box-Muller,    */
/* Tensor.swift:1623-1644) needs Swift's Float.random to reproduce.           */
/* ------------------------------------------------------------------------ */
uint64_t orc_splitmix64(uint64_t *state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void orc_fill_normal(uint64_t seed, double mean, double std, float *out, int64_t n) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = ((double)(orc_splitmix64(&s) >> 11) + 0.5) * 0x1p-53;
        double u2 = (double)(orc_splitmix64(&s) >> 11) * 0x1p-53;
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + std * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(mean + std * r * sin(two_pi * u2));
    }
}

/* ------------------------------------------------------------------------ */
/* INT4 nibbles                                                               */
/* ------------------------------------------------------------------------ */

/* packInt4, QuantizedTensor.swift:314-319: clamp to [-7, 7], keep 4 bits,
 * value1 in the high nibble.  Swift's Int8 `<<` drops the bits shifted out. */
int8_t orc_pack_int4(int8_t v1, int8_t v2) {
    int a = v1 < -7 ? -7 : (v1 > 7 ? 7 : v1);
    int b = v2 < -7 ? -7 : (v2 > 7 ? 7 : v2);
    unsigned hi = ((unsigned)a & 0x0Fu) << 4;
    unsigned lo = (unsigned)b & 0x0Fu;
    return (int8_t)(uint8_t)((hi | lo) & 0xFFu);
}

/* Sign extension of one nibble, QuantizedTensor.swift:207-212 / :327-328:
 * raw in 0..15, raw > 7 => raw - 16.  Note nibble 0x8 decodes to -8. */
static inline int32_t nibble_to_int(unsigned raw) {
    return raw > 7u ? (int32_t)raw - 16 : (int32_t)raw;
}

/* unpackInt4, QuantizedTensor.swift:322-331.  Swift's `packed >> 4` on Int8
 * is an arithmetic shift; `& 0x0F` then keeps the nibble either way. */
void orc_unpack_int4(int8_t packed, int8_t *v1, int8_t *v2) {
    unsigned b = (uint8_t)packed;
    *v1 = (int8_t)nibble_to_int((b >> 4) & 0x0Fu);
    *v2 = (int8_t)nibble_to_int(b & 0x0Fu);
}

/* Flat INT4 decode of element i, QuantizedTensor.swift:201-213: byte i/2,
 * high nibble for even i, low nibble for odd i. */
int32_t orc_int4_at(const int8_t *data, int64_t i) {
    unsigned b = (uint8_t)data[i >> 1];
    unsigned raw = (i & 1) == 0 ? ((b >> 4) & 0x0Fu) : (b & 0x0Fu);
    return nibble_to_int(raw);
}

/* ------------------------------------------------------------------------ */
/* Quantizers                                                                 */
/* ------------------------------------------------------------------------ */

static inline float round_mode(float v, int32_t rounding) {
    /* Swift round(): half away from zero.  np.round: half to even. */
    return rounding == ORC_ROUND_NUMPY ? rintf(v) : roundf(v);
}

static inline float clampf(float v, float lo, float hi) {
    /* Swift max(lo, min(hi, v)) */
    float m = v < hi ? v : hi;
    return m > lo ? m : lo;
}

/* quantizePerChannel, QuantizedTensor.swift:379-424. */
void orc_quantize_per_channel(const float *w, int64_t rows, int64_t cols,
                              int8_t *q, float *scales, int32_t rounding) {
    for (int64_t c = 0; c < cols; ++c) {                       /* :389-404 */
        float abs_max = 0.0f;
        for (int64_t r = 0; r < rows; ++r) {
            float v = fabsf(w[r * cols + c]);
            if (v > abs_max) abs_max = v;
        }
        scales[c] = abs_max < SWIFT_LEAST_NONZERO ? 1.0f : abs_max / 127.0f;
    }
    for (int64_t r = 0; r < rows; ++r) {                       /* :407-415 */
        for (int64_t c = 0; c < cols; ++c) {
            int64_t i = r * cols + c;
            float qv = round_mode(w[i] / scales[c], rounding);
            q[i] = (int8_t)clampf(qv, -127.0f, 127.0f);
        }
    }
}

static void min_max(const float *w, int64_t n, float *mn, float *mx) {
    /* Array.min() ?? 0 / Array.max() ?? 0 */
    float a = 0.0f, b = 0.0f;
    if (n > 0) {
        a = b = w[0];
        for (int64_t i = 1; i < n; ++i) {
            if (w[i] < a) a = w[i];
            if (w[i] > b) b = w[i];
        }
    }
    *mn = a;
    *mx = b;
}

/* quantizeSymmetric, QuantizedTensor.swift:427-449. */
void orc_quantize_symmetric(const float *w, int64_t n, int8_t *q, float *scale,
                            int32_t rounding) {
    float mn, mx;
    min_max(w, n, &mn, &mx);
    float abs_max = fmaxf(fabsf(mn), fabsf(mx));
    float s = abs_max > SWIFT_LEAST_NONZERO ? abs_max / 127.0f : 1.0f;
    for (int64_t i = 0; i < n; ++i)
        q[i] = (int8_t)clampf(round_mode(w[i] / s, rounding), -127.0f, 127.0f);
    *scale = s;
}

/* quantizeAsymmetric, QuantizedTensor.swift:452-476.  Returns ORC_E_TRAP when
 * Int8(round(-min/scale - 128)) is out of range (Swift traps there, e.g. for
 * all-positive data). */
int32_t orc_quantize_asymmetric(const float *w, int64_t n, int8_t *q, float *scale,
                                int8_t *zero_point, int32_t rounding) {
    float mn, mx;
    min_max(w, n, &mn, &mx);
    float range = mx - mn;
    float s = range > SWIFT_LEAST_NONZERO ? range / 255.0f : 1.0f;
    float zf = round_mode(-mn / s - 128.0f, rounding);
    if (!(zf >= -128.0f && zf <= 127.0f)) return ORC_E_TRAP;
    int8_t zp = (int8_t)zf;
    for (int64_t i = 0; i < n; ++i) {
        float qv = round_mode(w[i] / s, rounding) + (float)zp;
        q[i] = (int8_t)clampf(qv, -128.0f, 127.0f);
    }
    *scale = s;
    *zero_point = zp;
    return ORC_OK;
}

/* quantizeINT4, QuantizedTensor.swift:502-560; with ORC_ROUND_NUMPY it is
 * quantize_int4_per_group, Scripts/convert_model.py:398-459 (same flat
 * grouping, np.clip then astype(int8), pack even -> high nibble). */
void orc_quantize_int4(const float *w, int64_t n, int64_t group_size,
                       int8_t *packed, float *scales, int8_t *zero_points,
                       int32_t rounding) {
    int64_t gs = group_size;
    int64_t groups = (n + gs - 1) / gs;
    uint8_t *out = (uint8_t *)packed;
    memset(out, 0, (size_t)((n + 1) / 2));
    for (int64_t g = 0; g < groups; ++g) {
        int64_t start = g * gs;
        int64_t end = start + gs < n ? start + gs : n;
        float mn, mx;
        min_max(w + start, end - start, &mn, &mx);            /* :518-519 */
        float abs_max = fmaxf(fabsf(mn), fabsf(mx));          /* :522 */
        float s = abs_max < SWIFT_LEAST_NONZERO ? 1.0f : abs_max / 7.0f;
        scales[g] = s;
        if (zero_points) zero_points[g] = 0;
        for (int64_t i = start; i < end; ++i) {               /* :533-548 */
            int v = (int)clampf(round_mode(w[i] / s, rounding), -7.0f, 7.0f);
            unsigned nib = (unsigned)v & 0x0Fu;
            if ((i & 1) == 0) out[i >> 1] = (uint8_t)(nib << 4);
            else out[i >> 1] |= (uint8_t)nib;
        }
    }
}

/* quantizeINT4PerChannel, QuantizedTensor.swift:563-606. */
void orc_quantize_int4_per_channel(const float *w, int64_t rows, int64_t cols,
                                   int8_t *packed, float *scales, int32_t rounding) {
    uint8_t *out = (uint8_t *)packed;
    memset(out, 0, (size_t)((rows * cols + 1) / 2));
    for (int64_t c = 0; c < cols; ++c) {
        float abs_max = 0.0f;
        for (int64_t r = 0; r < rows; ++r) {
            float v = fabsf(w[r * cols + c]);
            if (v > abs_max) abs_max = v;
        }
        scales[c] = abs_max < SWIFT_LEAST_NONZERO ? 1.0f : abs_max / 7.0f;
    }
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < cols; ++c) {
            int64_t i = r * cols + c;
            int v = (int)clampf(round_mode(w[i] / scales[c], rounding), -7.0f, 7.0f);
            unsigned nib = (unsigned)v & 0x0Fu;
            if ((i & 1) == 0) out[i >> 1] = (uint8_t)(nib << 4);
            else out[i >> 1] |= (uint8_t)nib;
        }
    }
}

/* quantize_int8_per_channel, 2-D branch, Scripts/convert_model.py:383-395:
 * scale = max|row| / 127 (1.0 for a zero row), q = np.round(row / scale)
 * cast to int8 without a clip (|row/scale| <= 127 by construction). */
void orc_convert_int8_per_channel(const float *w_nk, int64_t n_rows, int64_t k_cols,
                                  int8_t *q_nk, float *scales) {
    for (int64_t r = 0; r < n_rows; ++r) {
        const float *row = w_nk + r * k_cols;
        float abs_max = 0.0f;
        for (int64_t k = 0; k < k_cols; ++k) {
            float v = fabsf(row[k]);
            if (v > abs_max) abs_max = v;
        }
        float s = abs_max > 0.0f ? abs_max / 127.0f : 1.0f;
        scales[r] = s;
        for (int64_t k = 0; k < k_cols; ++k)
            q_nk[r * k_cols + k] = (int8_t)rintf(row[k] / s);
    }
}

/* ------------------------------------------------------------------------ */
/* QuantizedTensor.init preconditions, QuantizedTensor.swift:124-155          */
/* ------------------------------------------------------------------------ */
static int64_t shape_count(const orc_qtensor *qt) {
    return qt->rank >= 2 ? qt->dims[0] * qt->dims[1] : qt->dims[0];
}

int32_t orc_validate(const orc_qtensor *qt) {
    if (!qt || qt->rank < 1 || qt->rank > 2) return ORC_E_INVALID;
    int64_t count = shape_count(qt);
    if (qt->precision == ORC_PREC_INT8) {
        if (qt->data_count != count) return ORC_E_INVALID;
    } else if (qt->precision == ORC_PREC_INT4) {
        if (qt->data_count != (count + 1) / 2) return ORC_E_INVALID;
    } else {
        return ORC_E_INVALID;
    }
    switch (qt->mode) {
    case ORC_MODE_PER_CHANNEL:
    case ORC_MODE_INT4_PER_CHANNEL: {
        int64_t ch = qt->rank >= 2 ? qt->dims[1] : qt->dims[0];
        if (qt->n_scales != ch) return ORC_E_INVALID;
        break;
    }
    case ORC_MODE_SYMMETRIC:
    case ORC_MODE_ASYMMETRIC:
        if (qt->n_scales != 1) return ORC_E_INVALID;
        break;
    case ORC_MODE_INT4:
        if (qt->group_size > 0) {
            if (qt->n_scales != (count + qt->group_size - 1) / qt->group_size)
                return ORC_E_INVALID;
        } else if (qt->n_scales != 1) {
            return ORC_E_INVALID;
        }
        break;
    default:
        return ORC_E_INVALID;
    }
    if (qt->zero_points && qt->n_zero_points != qt->n_scales) return ORC_E_INVALID;
    return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* dequantize(), QuantizedTensor.swift:182-286                                */
/* value = (Float(q) - Float(zp)) * scale: one fp32 rounding, no FMA.        */
/* ------------------------------------------------------------------------ */
static inline int32_t zp_at(const orc_qtensor *qt, int64_t idx) {
    return qt->zero_points ? (int32_t)qt->zero_points[idx] : 0;
}

int32_t orc_dequantize(const orc_qtensor *qt, float *out) {
    if (orc_validate(qt) != ORC_OK) return ORC_E_INVALID;
    int64_t count = shape_count(qt);
    memset(out, 0, (size_t)count * sizeof(float));            /* :183 */
    switch (qt->mode) {
    case ORC_MODE_INT4: {                                       /* :186-216 */
        int64_t gs = qt->group_size > 0 ? qt->group_size : count;
        for (int64_t i = 0; i < count; ++i) {
            int64_t g = i / gs;
            float s = qt->scales[g];
            float zp = (float)zp_at(qt, g);
            out[i] = ((float)orc_int4_at(qt->data, i) - zp) * s;
        }
        break;
    }
    case ORC_MODE_INT4_PER_CHANNEL: {                           /* :218-238 */
        /* One scale per *row* here, although the quantizer writes one per
         * column: scales[ch] traps when rows > cols. */
        int64_t nch = qt->dims[0];
        int64_t csize = count / nch;
        for (int64_t ch = 0; ch < nch; ++ch) {
            if (ch >= qt->n_scales) return ORC_E_TRAP;
            float s = qt->scales[ch];
            float zp = (float)zp_at(qt, ch);
            for (int64_t j = 0; j < csize; ++j) {
                int64_t i = ch * csize + j;
                out[i] = ((float)orc_int4_at(qt->data, i) - zp) * s;
            }
        }
        break;
    }
    case ORC_MODE_PER_CHANNEL: {                                /* :241-271 */
        if (qt->rank == 2) {
            int64_t rows = qt->dims[0], cols = qt->dims[1];
            for (int64_t r = 0; r < rows; ++r)
                for (int64_t c = 0; c < cols; ++c) {
                    int64_t i = r * cols + c;
                    out[i] = ((float)qt->data[i] - (float)zp_at(qt, c)) * qt->scales[c];
                }
        } else {
            int64_t nch = qt->dims[0];
            int64_t csize = qt->data_count / nch;
            for (int64_t ch = 0; ch < nch; ++ch)
                for (int64_t i = ch * csize; i < (ch + 1) * csize; ++i)
                    out[i] = ((float)qt->data[i] - (float)zp_at(qt, ch)) * qt->scales[ch];
        }
        break;
    }
    case ORC_MODE_SYMMETRIC:
    case ORC_MODE_ASYMMETRIC: {                                 /* :273-281 */
        float s = qt->scales[0];
        float zp = (float)zp_at(qt, 0);
        if (qt->data_count > count) return ORC_E_TRAP;
        for (int64_t i = 0; i < qt->data_count; ++i)
            out[i] = ((float)qt->data[i] - zp) * s;
        break;
    }
    default:
        return ORC_E_INVALID;
    }
    return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* matmulCPU, Tensor.swift:839-861 (row-major NoTrans sgemm, alpha 1 beta 0)  */
/* ------------------------------------------------------------------------ */
#define ORC_NB 2048  /* output columns per task: the accumulators stay in L1/L2 */

void orc_sgemm(int64_t M, int64_t N, int64_t K, const float *A, const float *B,
               float *C, int32_t threads) {
    int64_t nblocks = (N + ORC_NB - 1) / ORC_NB;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
    for (int64_t nb = 0; nb < nblocks; ++nb) {
        int64_t n0 = nb * ORC_NB;
        int64_t n1 = n0 + ORC_NB < N ? n0 + ORC_NB : N;
        int64_t w = n1 - n0;
        for (int64_t m0 = 0; m0 < M; m0 += 8) {
            int64_t mc = M - m0 < 8 ? M - m0 : 8;
            float acc[8][ORC_NB];
            for (int64_t m = 0; m < mc; ++m)
                for (int64_t j = 0; j < w; ++j) acc[m][j] = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                const float *brow = B + k * N + n0;
                for (int64_t m = 0; m < mc; ++m) {
                    float a = A[(m0 + m) * K + k];
                    float *am = acc[m];
                    for (int64_t j = 0; j < w; ++j) am[j] += a * brow[j];
                }
            }
            for (int64_t m = 0; m < mc; ++m)
                memcpy(C + (m0 + m) * N + n0, acc[m], (size_t)w * sizeof(float));
        }
    }
}

void orc_gemm_f64(int64_t M, int64_t N, int64_t K, const float *A, const float *B,
                  double *C, int32_t threads) {
    int64_t nblocks = (N + ORC_NB - 1) / ORC_NB;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
    for (int64_t nb = 0; nb < nblocks; ++nb) {
        int64_t n0 = nb * ORC_NB;
        int64_t n1 = n0 + ORC_NB < N ? n0 + ORC_NB : N;
        int64_t w = n1 - n0;
        double *acc = (double *)malloc((size_t)w * sizeof(double));
        for (int64_t m = 0; m < M; ++m) {
            for (int64_t j = 0; j < w; ++j) acc[j] = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                double a = (double)A[m * K + k];
                const float *brow = B + k * N + n0;
                for (int64_t j = 0; j < w; ++j) acc[j] += a * (double)brow[j];
            }
            memcpy(C + m * N + n0, acc, (size_t)w * sizeof(double));
        }
        free(acc);
    }
}

/* Tensor.matmul(QuantizedTensor) fallback, QuantizedTensor.swift:640-642. */
int32_t orc_matmul_quantized_cpu(const float *x, int64_t M, const orc_qtensor *qt,
                                 float *y, int32_t threads,
                                 double *dequant_seconds, double *gemm_seconds) {
    if (orc_validate(qt) != ORC_OK || qt->rank != 2) return ORC_E_INVALID;
    int64_t K = qt->dims[0], N = qt->dims[1];
    double t0 = now_seconds();
    float *w = (float *)malloc((size_t)(K * N) * sizeof(float));  /* fresh buffer */
    if (!w) return ORC_E_INVALID;
    int32_t st = orc_dequantize(qt, w);
    double t1 = now_seconds();
    if (st == ORC_OK) orc_sgemm(M, N, K, x, w, y, threads);
    double t2 = now_seconds();
    free(w);
    if (dequant_seconds) *dequant_seconds = t1 - t0;
    if (gemm_seconds) *gemm_seconds = t2 - t1;
    return st;
}

/* ------------------------------------------------------------------------ */
/* Best-effort CPU (not a reference function): the fused dequant-GEMV that   */
/* the baseline plan reports beside the reference path as an upper bound     */
/* for the host.  y = x . dequant(W) for M rows without writing the          */
/* dequantized matrix: every quantized element is read once per 8 rows of x  */
/* and dequantized in registers, on all threads.  The dequantized values are  */
/* orc_dequantize's and the sum over k runs in orc_sgemm's order, so y       */
/* equals the reference path's bit for bit.                                   */
/*   nk = 0: element (k, n) at flat index k*N + n (the reference's indexing); */
/*   nk = 1: element (k, n) at n*K + k (the converter's INT4 storage), with   */
/*           groups of group_size along k.                                   */
/* ------------------------------------------------------------------------ */
int32_t orc_matmul_quantized_fused(const float *x, int64_t M, const orc_qtensor *qt, float *y,
                                   int32_t threads, int32_t nk) {
    if (orc_validate(qt) != ORC_OK || qt->rank != 2) return ORC_E_INVALID;
    if (!(qt->mode == ORC_MODE_PER_CHANNEL || qt->mode == ORC_MODE_INT4)) return ORC_E_INVALID;
    if (nk && qt->mode != ORC_MODE_INT4) return ORC_E_INVALID;
    const int64_t K = qt->dims[0], N = qt->dims[1];
    const int64_t gs = qt->group_size > 0 ? qt->group_size : K * N;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#endif
    if (nk) {
        /* one output column n at a time: its K elements are contiguous */
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 64) num_threads(nt)
#endif
        for (int64_t n = 0; n < N; ++n) {
            for (int64_t m0 = 0; m0 < M; m0 += 8) {
                int64_t mc = M - m0 < 8 ? M - m0 : 8;
                float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
                int64_t i = n * K, g = i / gs, r = i % gs;
                for (int64_t k = 0; k < K; ++k, ++i) {
                    float wv = ((float)orc_int4_at(qt->data, i) - (float)zp_at(qt, g)) * qt->scales[g];
                    if (++r == gs) { r = 0; ++g; }
                    for (int64_t m = 0; m < mc; ++m) acc[m] += x[(m0 + m) * K + k] * wv;
                }
                for (int64_t m = 0; m < mc; ++m) y[(m0 + m) * N + n] = acc[m];
            }
        }
        return ORC_OK;
    }
    int64_t nblocks = (N + ORC_NB - 1) / ORC_NB;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
    for (int64_t nb = 0; nb < nblocks; ++nb) {
        int64_t n0 = nb * ORC_NB;
        int64_t n1 = n0 + ORC_NB < N ? n0 + ORC_NB : N;
        int64_t w = n1 - n0;
        float wrow[ORC_NB];
        for (int64_t m0 = 0; m0 < M; m0 += 8) {
            int64_t mc = M - m0 < 8 ? M - m0 : 8;
            float acc[8][ORC_NB];
            for (int64_t m = 0; m < mc; ++m)
                for (int64_t j = 0; j < w; ++j) acc[m][j] = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                if (qt->mode == ORC_MODE_PER_CHANNEL) {
                    const int8_t *d = qt->data + k * N + n0;
                    for (int64_t j = 0; j < w; ++j)
                        wrow[j] = ((float)d[j] - (float)zp_at(qt, n0 + j)) * qt->scales[n0 + j];
                } else {
                    int64_t i = k * N + n0, g = i / gs, r = i % gs;   /* group stepped, not divided */
                    for (int64_t j = 0; j < w; ++j, ++i) {
                        wrow[j] = ((float)orc_int4_at(qt->data, i) - (float)zp_at(qt, g)) * qt->scales[g];
                        if (++r == gs) { r = 0; ++g; }
                    }
                }
                for (int64_t m = 0; m < mc; ++m) {
                    float a = x[(m0 + m) * K + k];
                    float *am = acc[m];
                    for (int64_t j = 0; j < w; ++j) am[j] += a * wrow[j];
                }
            }
            for (int64_t m = 0; m < mc; ++m)
                memcpy(y + (m0 + m) * N + n0, acc[m], (size_t)w * sizeof(float));
        }
    }
    return ORC_OK;
}


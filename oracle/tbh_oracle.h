/*
 * tbh_oracle.h -- CPU restatement of TinyBrain's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * backend: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product (tinybrain_amd, libtinybrain_hip.so) never
 * links or calls it.
 *
 * Each function restates one reference function; the citation (path:line,
 * relative to the vivekptnk/tinybrain tree) is given beside it.  Shapes follow
 * the reference: a 2-D quantized weight has shape [K, N] = [in, out] and its
 * elements sit in a flat array (runtime layout: flat index i = k*N + n).
 */
#ifndef TBH_ORACLE_H
#define TBH_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* QuantizationMode, Sources/TinyBrainRuntime/QuantizedTensor.swift:31-37 */
enum {
    ORC_MODE_SYMMETRIC = 0,
    ORC_MODE_ASYMMETRIC = 1,
    ORC_MODE_PER_CHANNEL = 2,
    ORC_MODE_INT4 = 3,
    ORC_MODE_INT4_PER_CHANNEL = 4
};

/* QuantizationPrecision, QuantizedTensor.swift:40-57 (codes are the TBF
 * precision byte, ModelWeights.swift:395 / :679) */
enum { ORC_PREC_INT8 = 1, ORC_PREC_INT4 = 2 };

/* Rounding used by a quantizer.  Swift's Float.round() rounds half away from
 * zero (C roundf); numpy's np.round rounds half to even (C rintf in the
 * default rounding mode). */
enum { ORC_ROUND_SWIFT = 0, ORC_ROUND_NUMPY = 1 };

/* Status codes. */
enum { ORC_OK = 0, ORC_E_INVALID = 1, ORC_E_TRAP = 2 };

/* struct QuantizedTensor, QuantizedTensor.swift:62-166.  rank is 1 or 2;
 * dims[1] is ignored for rank 1.  zero_points may be NULL (Swift nil). */
typedef struct orc_qtensor {
    int32_t rank;
    int64_t dims[2];
    const int8_t *data;
    int64_t data_count;
    const float *scales;
    int64_t n_scales;
    const int8_t *zero_points;
    int64_t n_zero_points;
    int32_t mode;
    int32_t precision;
    int64_t group_size;
} orc_qtensor;

/* --- deterministic synthetic inputs (not a reference function) ---------- */
uint64_t orc_splitmix64(uint64_t *state);
/* n samples of N(mean, std) as fp32: splitmix64 -> Box-Muller in double. */
void orc_fill_normal(uint64_t seed, double mean, double std, float *out, int64_t n);

/* --- INT4 nibble helpers ------------------------------------------------ */
/* QuantizedTensor.packInt4, QuantizedTensor.swift:314-319 */
int8_t orc_pack_int4(int8_t v1, int8_t v2);
/* QuantizedTensor.unpackInt4, QuantizedTensor.swift:322-331 */
void orc_unpack_int4(int8_t packed, int8_t *v1, int8_t *v2);
/* One element of the flat INT4 decode, QuantizedTensor.swift:201-213. */
int32_t orc_int4_at(const int8_t *data, int64_t i);

/* --- quantizers ---------------------------------------------------------- */
/* quantizePerChannel, QuantizedTensor.swift:379-424.  w is [rows, cols]
 * row-major; one scale per column (output channel). */
void orc_quantize_per_channel(const float *w, int64_t rows, int64_t cols,
                              int8_t *q, float *scales, int32_t rounding);
/* quantizeSymmetric, QuantizedTensor.swift:427-449. */
void orc_quantize_symmetric(const float *w, int64_t n, int8_t *q, float *scale,
                            int32_t rounding);
/* quantizeAsymmetric, QuantizedTensor.swift:452-476. */
int32_t orc_quantize_asymmetric(const float *w, int64_t n, int8_t *q, float *scale,
                                int8_t *zero_point, int32_t rounding);
/* quantizeINT4, QuantizedTensor.swift:502-560 (ORC_ROUND_SWIFT), and
 * quantize_int4_per_group, Scripts/convert_model.py:398-459 (ORC_ROUND_NUMPY;
 * the converter flattens the PyTorch [N, K] tensor, so its groups run along
 * K).  Writes ceil(n/2) packed bytes, ceil(n/gs) scales and as many zero
 * points (all 0). */
void orc_quantize_int4(const float *w, int64_t n, int64_t group_size,
                       int8_t *packed, float *scales, int8_t *zero_points,
                       int32_t rounding);
/* quantizeINT4PerChannel, QuantizedTensor.swift:563-606. */
void orc_quantize_int4_per_channel(const float *w, int64_t rows, int64_t cols,
                                   int8_t *packed, float *scales, int32_t rounding);
/* quantize_int8_per_channel (2-D branch), Scripts/convert_model.py:383-395:
 * per row of the PyTorch [N, K] tensor, np.round, no clip. */
void orc_convert_int8_per_channel(const float *w_nk, int64_t n_rows, int64_t k_cols,
                                  int8_t *q_nk, float *scales);

/* --- QuantizedTensor.init preconditions, QuantizedTensor.swift:124-155 --- */
int32_t orc_validate(const orc_qtensor *qt);

/* --- dequantize(), QuantizedTensor.swift:182-286 ------------------------- */
/* Writes shape.count floats.  Returns ORC_E_TRAP where the Swift code would
 * trap (out-of-range index), ORC_E_INVALID for a bad descriptor. */
int32_t orc_dequantize(const orc_qtensor *qt, float *out);

/* --- matmul -------------------------------------------------------------- */
/* Tensor.matmulCPU, Tensor.swift:839-861: cblas_sgemm(RowMajor, NoTrans,
 * NoTrans, M, N, K, 1, A, K, B, N, 0, C, N).  fp32 accumulation in k order,
 * OpenMP over output columns with `threads` threads (<= 0: all). */
void orc_sgemm(int64_t M, int64_t N, int64_t K, const float *A, const float *B,
               float *C, int32_t threads);
/* float64 oracle of the same product: C = sum_k (double)A[m,k]*(double)B[k,n]. */
void orc_gemm_f64(int64_t M, int64_t N, int64_t K, const float *A, const float *B,
                  double *C, int32_t threads);
/* Tensor.matmul(QuantizedTensor) CPU fallback, QuantizedTensor.swift:640-642:
 * dequantize() (single-threaded, fresh [K,N] buffer) then matmulCPU.
 * dequant_seconds / gemm_seconds (nullable) receive the two phase times. */
int32_t orc_matmul_quantized_cpu(const float *x, int64_t M, const orc_qtensor *qt,
                                 float *y, int32_t threads,
                                 double *dequant_seconds, double *gemm_seconds);

/* Best-effort CPU fused dequant-GEMV (not a reference function; an upper
 * bound for the host reported beside the reference path).  nk = 0: element
 * (k, n) at flat index k*N + n; nk = 1: at n*K + k (converter INT4 storage).
 * PER_CHANNEL (nk = 0 only) and INT4 modes.  Same y as
 * orc_matmul_quantized_cpu over the same dequantized values. */
int32_t orc_matmul_quantized_fused(const float *x, int64_t M, const orc_qtensor *qt, float *y,
                                   int32_t threads, int32_t nk);

#ifdef __cplusplus
}
#endif
#endif /* TBH_ORACLE_H */

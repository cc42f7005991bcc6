/*
 * tinybrain_hip.h -- C ABI of TinyBrainHIP, the MI355X (gfx950) backend for
 * TinyBrain's INT8/INT4 weight-only quantized matmul.
 *
 * The ABI is what a Swift `HIPBackend: QuantizedMatMulBackend` binds through
 * a module map (`module CTinyBrainHIP { header "tinybrain_hip.h";
 * link "tinybrain_hip"; export * }`).  Signatures carry plain pointers and
 * sizes only.  All references are to vivekptnk/tinybrain paths.
 *
 * Conventions
 *   - A weight has the reference shape [K, N] = [in_features, out_features]
 *     (QuantizedTensor.shape, Sources/TinyBrainRuntime/QuantizedTensor.swift:73);
 *     x is [M, K] row-major fp32, y is [M, N] row-major fp32.
 *   - Every call returns a tbh_status; on failure tbh_last_error() returns a
 *     message for the calling thread.  A Swift wrapper maps every non-zero
 *     status to `throw`, which keeps the reference's fallback to its CPU path
 *     (QuantizedTensor.swift:630-642).
 */
#ifndef TINYBRAIN_HIP_H
#define TINYBRAIN_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TBH_ABI_VERSION 1

/* ---- status ------------------------------------------------------------ */
typedef int32_t tbh_status;
enum {
    TBH_OK = 0,
    TBH_E_INVALID = 1,      /* bad descriptor, shape mismatch, null pointer */
    TBH_E_UNSUPPORTED = 2,  /* a valid reference input this backend does not take */
    TBH_E_NODEVICE = 3,     /* no usable gfx950 device */
    TBH_E_OOM = 4,          /* device or host allocation failed */
    TBH_E_HIP = 5           /* any other HIP runtime error */
};

/* ---- descriptor codes -------------------------------------------------- */
/* QuantizationPrecision; the values are the TBF precision byte
 * (ModelWeights.swift:395 writes them, :679 reads them). */
enum { TBH_PREC_INT8 = 1, TBH_PREC_INT4 = 2 };

/* QuantizationMode, QuantizedTensor.swift:31-37. */
enum {
    TBH_MODE_SYMMETRIC = 0,        /* INT8, one scale                      */
    TBH_MODE_ASYMMETRIC = 1,       /* INT8, one scale + one zero point     */
    TBH_MODE_PER_CHANNEL = 2,      /* INT8, one scale per output column n  */
    TBH_MODE_INT4 = 3,             /* INT4, one scale per flat group       */
    TBH_MODE_INT4_PER_CHANNEL = 4  /* rejected with TBH_E_UNSUPPORTED: the
                                      reference's dequantize() reads its
                                      scales along dim 0 while its quantizer
                                      writes them along dim 1
                                      (QuantizedTensor.swift:218-238 vs
                                      :563-606), so the caller's CPU
                                      fallback is the only defined result  */
};

/* Order of the flat element array.
 *   KN_FLAT: element (k, n) is flat index k*N + n -- the runtime layout that
 *            Tensor.quantize() writes (QuantizedTensor.swift:379-424,
 *            :502-560) and dequantize() reads (:182-286).
 *   NK_FLAT: element (k, n) is flat index n*K + k -- what
 *            Scripts/convert_model.py:398-459 writes for INT4 (it quantizes
 *            the PyTorch [N, K] tensor flattened and only reverses the
 *            recorded shape, :489-502), i.e. groups run along K.
 * For INT4 the group of flat index i is i / group_size in both layouts. */
enum { TBH_LAYOUT_KN_FLAT = 0, TBH_LAYOUT_NK_FLAT = 1 };

/* struct QuantizedTensor (QuantizedTensor.swift:62-166) as plain data.
 * Counts are checked exactly as QuantizedTensor.init checks them
 * (QuantizedTensor.swift:124-155):
 *   data_bytes    == K*N (INT8) or ceil(K*N/2) (INT4, even flat index in the
 *                    high nibble, QuantizedTensor.swift:201-213)
 *   n_scales      == N (PER_CHANNEL), 1 (SYMMETRIC/ASYMMETRIC),
 *                    ceil(K*N/group_size) (INT4, group_size > 0),
 *                    1 (INT4, group_size == 0: one group of K*N)
 *   n_zero_points == n_scales when zero_points != NULL. */
typedef struct tbh_qtensor_desc {
    int64_t K;
    int64_t N;
    int32_t precision;          /* TBH_PREC_*   */
    int32_t mode;               /* TBH_MODE_*   */
    int32_t layout;             /* TBH_LAYOUT_* */
    int32_t group_size;         /* INT4 only; 0 = single group */
    const int8_t *data;
    int64_t data_bytes;
    const float *scales;
    int64_t n_scales;
    const int8_t *zero_points;  /* nullable (Swift nil) */
    int64_t n_zero_points;
} tbh_qtensor_desc;

/* Which kernel family serves a weight (see tbh_weight_info.path). */
enum {
    TBH_PATH_INT8_ROW = 0,      /* INT8, one scale (and zero point) per row  */
    TBH_PATH_INT4_KGROUP = 1,   /* INT4, scales per (row, K-segment)         */
    TBH_PATH_INT4_NGROUP = 2,   /* INT4 runtime layout, scales per (K, N-block) */
    TBH_PATH_GENERIC = 3        /* any other INT4 grouping: slow, exact decode */
};

typedef struct tbh_weight_info {
    int64_t K;
    int64_t N;
    int32_t precision;
    int32_t mode;
    int32_t layout;
    int32_t group_size;
    int32_t path;               /* TBH_PATH_* */
    int32_t has_zero_points;    /* non-zero zero points were kept */
    int64_t device_bytes;       /* bytes this weight holds in HBM */
    int64_t stream_bytes;       /* bytes one matmul reads from it:
                                   packed weights + scales + zero points */
} tbh_weight_info;

typedef struct tbh_device tbh_device;
typedef struct tbh_weight tbh_weight;

/* ---- library ----------------------------------------------------------- */
int32_t tbh_abi_version(void);
/* Message of the last failure on the calling thread ("" if none). */
const char *tbh_last_error(void);
const char *tbh_status_string(tbh_status status);

/* ---- device ------------------------------------------------------------ */
/* Replaces MetalBackend.init (Sources/TinyBrainMetal/MetalBackend.swift:38-56)
 * and MetalBackend.isAvailable: opens HIP device `ordinal` (must be gfx950)
 * with one internal stream.  TBH_E_NODEVICE when absent. */
tbh_status tbh_device_open(int32_t ordinal, tbh_device **out);
/* Waits for the device's work and frees what the library allocated on it.
 * Destroy the device's weights and decoders first: their destroy calls read
 * the device handle. */
tbh_status tbh_device_close(tbh_device *dev);
/* HIP device ordinal and compute-unit count of an open device. */
tbh_status tbh_device_get_info(const tbh_device *dev, int32_t *ordinal, int32_t *cu_count);

/* Launch-rule overrides of an open device, for measurement and tests.  No
 * reference counterpart (MetalBackend's launch shapes are fixed,
 * MetalBackend.swift:949-956).  Every accepted value keeps results within
 * the matmul tolerance; TBH_E_INVALID for unknown options or values.
 *   TBH_OPT_SGEMV_MIN_ROWS: fewest rows of x (2..9, 9 = never) that go to the
 *     matrix-core small-M GEMV for every weight; 0 restores the per-weight
 *     rule.  The environment variable TBH_SGEMV_MIN_ROWS, read when the
 *     device opens, sets the initial value.
 *   TBH_OPT_NOALLOC_SCRATCH_BYTES: the most scratch bytes
 *     tbh_matmul_device_noalloc may use on this device, 1 .. 16 MiB; 0 (the
 *     default) is the whole 16 MiB array.  A call needing more is rejected.
 *   TBH_OPT_MFMA_MIN_ROWS: fewest rows of fp32 x that tbh_matmul* send to the
 *     MFMA GEMM (x split exactly into bf16 pieces) for every weight; 0
 *     restores the per-weight rule.
 *   TBH_OPT_HOST_ENTRY: how tbh_matmul moves x and y for up to 8 rows of x:
 *     0 = DMA copies through device staging; 1 = a copy launch brings x from
 *     page-locked staging and the kernels write y into it; 2 (default) = as
 *     1, with one row of x read by the kernels in place.  Initially the
 *     environment variable TBH_HOST_ENTRY when set.
 *   TBH_OPT_HOST_WAIT: how tbh_matmul waits in modes 1 and 2: 1 (default) =
 *     poll a completion word in page-locked memory for up to 200 us, then
 *     block; 0 = block on the stream.  Initially TBH_HOST_WAIT when set. */
enum {
    TBH_OPT_SGEMV_MIN_ROWS = 1,
    TBH_OPT_NOALLOC_SCRATCH_BYTES = 2,
    TBH_OPT_MFMA_MIN_ROWS = 3,
    TBH_OPT_HOST_ENTRY = 4,
    TBH_OPT_HOST_WAIT = 5
};
tbh_status tbh_device_set_option(tbh_device *dev, int32_t option, int64_t value);

/* ---- weights ----------------------------------------------------------- */
/* Replaces the weight upload of MetalBackend.cachedQuantizedBuffers
 * (MetalBackend.swift:1282-1308) and cachedINT4Buffers (:1322-1359): copies
 * the descriptor's arrays and repacks them ONCE into the gfx950 layout; the
 * caller may free its arrays on return.  Thread-safe.  K or N above 2^30
 * returns TBH_E_UNSUPPORTED (the caller's CPU fallback takes it). */
tbh_status tbh_weight_create(tbh_device *dev, const tbh_qtensor_desc *desc,
                             tbh_weight **out);
/* One weight that computes the outputs of n weights reading the same input,
 * side by side: y[M, N_0 + ... + N_{n-1}] = x . [dequantize(W_0) | ... ],
 * repacked once, so that the projections of a layer that read one x (q, k
 * and v; gate and up: ModelRunner.swift:418-452, where each is its own
 * apply(toRow:) call, ModelWeights.swift:47-68) run as one launch.  No
 * single reference counterpart: it is a one-time repack of
 * TransformerLayerWeights' quantized projections.  The parts must share K
 * and precision and be concatenable without re-quantizing: INT8 in the
 * [K][N] layout (per-channel, or a per-tensor scale repeated per column),
 * INT4 in the converter layout (groups along K), or runtime-layout INT4 whose
 * groups tile every part's N; zero points on all parts or none.  Otherwise
 * TBH_E_UNSUPPORTED (or TBH_E_INVALID for inconsistent descriptors).
 * Results are within the matmul tolerance of the parts' products (the
 * kernels chosen for the wider weight may sum in another order). */
tbh_status tbh_weight_create_concat(tbh_device *dev, int32_t n,
                                    const tbh_qtensor_desc *const *parts,
                                    tbh_weight **out);
tbh_status tbh_weight_destroy(tbh_weight *w);
tbh_status tbh_weight_get_info(const tbh_weight *w, tbh_weight_info *info);

/* ---- matmul ------------------------------------------------------------ */
/* Replaces QuantizedMatMulBackend.matmulQuantized
 * (Sources/TinyBrainRuntime/Backend.swift:173-175), implemented by
 * MetalBackend.matmulQuantized / matmulINT4 (MetalBackend.swift:894-1048):
 * y[M,N] = x[M,K] . dequantize(w)[K,N] with fp32 accumulation.
 * Host pointers; synchronous (the reference commits and waits, :959-960).
 * Up to 8 rows of x, the kernels read x from and write y to page-locked
 * host staging, and the calling thread polls a completion word there for up
 * to 200 us before it blocks on the stream; more rows move by DMA.
 * Calls on one device are serialised.  Like the Metal kernels, one call
 * covers any M (MetalBackend.swift:949-956): a few rows run on the GEMV
 * kernels; from a per-weight row count (8..64, TBH_OPT_MFMA_MIN_ROWS) INT8
 * rows, INT4 K-group weights and runtime-layout INT4 whose N-blocks tile 64
 * outputs (16, 32 or a multiple of 64 rows, or one block) run on the bf16
 * MFMA GEMM with every fp32 x row split exactly into three bf16 pieces (for
 * the runtime layout, x times the N-block's per-k scale, one fp32 rounding,
 * then split); past 64 rows INT8 rows and INT4 K-groups take x as two f16
 * pieces, scaled by a power of two per row, holding it to 2^-22 of the row's
 * largest element, on the f16 MFMA.  The GEMV kernels stage a row of
 * x in LDS, so a K past about 13 K (INT8) or 14.5 K (INT4) elements runs on
 * the MFMA GEMM at every M (runtime-layout INT4 of such a K keeps the
 * reference's flat array and runs on the generic kernel); a long K that is
 * not a multiple of 8, or an x that is not 16-byte aligned, returns
 * TBH_E_UNSUPPORTED. */
tbh_status tbh_matmul(tbh_device *dev, const float *x, int64_t M, int64_t K,
                      const tbh_weight *w, float *y);

/* Same product on device pointers, enqueued on `stream` (a hipStream_t of the
 * weight's device; NULL = the null stream).  Returns after the launch.
 * Launches that split K (matrix-core GEMV, MFMA GEMM) keep their partial sums,
 * and the MFMA GEMM past 64 rows its per-row exponents of x (an int32 per
 * row), in a workspace the library allocates per (device, stream) on first use and
 * keeps, with every buffer it outgrew, until tbh_device_close (a graph
 * captured on the stream may still hold them): a caller that creates many
 * short-lived streams should reuse a few, or call
 * tbh_matmul_device_noalloc.  A graph captured on a stream holds that
 * stream's current workspace, which later eager calls on the same stream
 * reuse: such a graph must not be replayed (on any stream) while eager
 * calls on its capture stream are in flight, or both write the same partial
 * sums. */
tbh_status tbh_matmul_device(const tbh_weight *w, const float *x, int64_t M,
                             int64_t K, float *y, void *stream);

/* No reference counterpart.  tbh_matmul_device for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  Same product, same kernels, same
 * arguments; the split-K partial sums (matrix-core small-M GEMV, MFMA GEMM)
 * and the GEMM's per-row exponents of x
 * go to a fixed 16 MiB scratch array per GPU (held until the process ends)
 * instead of a per-stream workspace, and the call makes no allocation.  A
 * call one of whose launches would need more than the scratch holds (16 MiB,
 * or TBH_OPT_NOALLOC_SCRATCH_BYTES) returns TBH_E_INVALID before that launch
 * is enqueued; rows of x that an earlier launch of the same call took on a
 * route without scratch (x runs in pieces of up to 8 rows, and pieces can
 * take different routes) may already have been written, so y is then
 * unspecified (decode shapes need at most a few MiB).  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (different
 * streams, or graphs replayed concurrently) race and must be serialised by
 * the caller. */
tbh_status tbh_matmul_device_noalloc(const tbh_weight *w, const float *x, int64_t M,
                                     int64_t K, float *y, void *stream);

/* Replaces LinearLayerWeights.apply(toRow:)
 * (Sources/TinyBrainRuntime/ModelWeights.swift:47-68): y = x . dequantize(w)
 * as tbh_matmul_device computes it, then y[m][n] += bias[n] (one fp32 add,
 * after the product, as the reference's host loop does).  bias: device
 * pointer to N floats, or NULL for no bias.  Device pointers, enqueued on
 * `stream`. */
tbh_status tbh_linear_device(const tbh_weight *w, const float *x, int64_t M,
                             int64_t K, const float *bias, float *y, void *stream);

/* Prefill: the same product for M >= 64 rows of bf16 activations, on bf16
 * MFMA.  The reference has no bf16 path; it multiplies
 * fp32 activations by dequantize(w) with cblas_sgemm
 * (QuantizedTensor.swift:640-642, Tensor.swift:839-861), which is the
 * product computed here for x = the bf16 values widened to fp32: weight
 * operands are exact integers (INT8: q - zp, the row scale applied after
 * accumulation; INT4 K-groups: 16 (q - zp), each 32-deep MFMA's partial
 * product times its group scale; INT4 runtime layout up to 64 rows: 16 q
 * against x times the N-block's per-k scale, rounded once in fp32 and split
 * exactly into three bf16 pieces), accumulation is fp32.  INT4 runtime
 * layout past 64 rows runs on f16 MFMA: the dequantized weight fl(q * s),
 * scaled by a power of two per N-block, as two f16 pieces holding it to
 * 2^-21 of itself, against x scaled by a power of two per row (exact), with
 * a pass over x for the row exponents in the stream's workspace.  x is [M, K] row-major bf16 bits
 * (16-byte aligned, K % 8 == 0), y is [M, N] fp32, both device pointers;
 * enqueued on `stream`.  TBH_E_UNSUPPORTED for weights outside the INT8
 * row / INT4 K-group / INT4 runtime-layout paths (tbh_weight_info.path), for
 * runtime-layout N-blocks that do not tile 64 outputs, or for the MFMA tile
 * layout. */
tbh_status tbh_matmul_bf16_device(const tbh_weight *w, const uint16_t *x, int64_t M,
                                  int64_t K, float *y, void *stream);

/* ---- decode step (LLaMA-style models, one sequence) -------------------- */
/* Replaces ModelRunner.step (Sources/TinyBrainRuntime/ModelRunner.swift:168-208)
 * for the pre-norm LLaMA architecture (applyLayer :418-459, attention
 * :496-592): RMSNorm, Q/K/V, RoPE, grouped-query attention over a KV cache,
 * output projection and residual, RMSNorm, SwiGLU FFN and residual, final
 * RMSNorm and the LM head, every projection on the quantized GEMV.  Gemma /
 * Phi variants, biases and X-Ray observers are not covered.  The position is
 * kept on the device and advanced by each step, so a step captured in a HIP
 * graph replays as the next one. */
typedef struct tbh_decoder tbh_decoder;
typedef struct tbh_decoder_config {
    int32_t num_layers;
    int32_t hidden;          /* ModelConfig.hiddenDim */
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t intermediate;    /* ModelConfig.intermediateDim */
    int32_t vocab;
    int32_t max_seq;         /* KV cache length, <= 16384 */
    float rms_eps;           /* 1e-5 (Tensor.swift:1512) */
    float rope_base;         /* 10000 (ModelRunner.swift:478) */
} tbh_decoder_config;

/* embeddings: [vocab][hidden] fp32 (ModelWeights.tokenEmbeddings);
 * final_norm: [hidden]; lm_head: [hidden, vocab] (ModelWeights.output).
 * Host pointers, copied. */
tbh_status tbh_decoder_create(tbh_device *dev, const tbh_decoder_config *cfg,
                              const float *embeddings, const float *final_norm,
                              const tbh_qtensor_desc *lm_head, tbh_decoder **out);
/* One TransformerLayerWeights (ModelWeights.swift): norms [hidden] and the
 * seven projections as [K, N] quantized tensors (q [hidden, hidden], k and v
 * [hidden, kv_dim], o [hidden, hidden], gate and up [hidden, intermediate],
 * down [intermediate, hidden]).  Q|K|V and gate|up are concatenated along N
 * into one repacked weight each.  Needs weights without zero points: INT8
 * in the runtime layout, INT4 in the converter layout (groups along K) or
 * INT4 in the runtime layout (Tensor.quantize(.int4), groups along N) whose
 * groups tile every projection's N. */
tbh_status tbh_decoder_set_layer(tbh_decoder *d, int32_t layer, const float *input_norm,
                                 const float *post_attention_norm,
                                 const tbh_qtensor_desc *q, const tbh_qtensor_desc *k,
                                 const tbh_qtensor_desc *v, const tbh_qtensor_desc *o,
                                 const tbh_qtensor_desc *gate, const tbh_qtensor_desc *up,
                                 const tbh_qtensor_desc *down);
tbh_status tbh_decoder_destroy(tbh_decoder *d);
/* ModelRunner.reset (:213-216) is set_position(d, 0). */
tbh_status tbh_decoder_set_position(tbh_decoder *d, int32_t position);
tbh_status tbh_decoder_get_position(const tbh_decoder *d, int32_t *position);
/* Enqueue one step for `token` on `stream`; logits: device [vocab] (NULL:
 * internal buffer). */
tbh_status tbh_decoder_step_device(tbh_decoder *d, int32_t token, float *logits, void *stream);
/* Synchronous step; logits: host [vocab]. */
tbh_status tbh_decoder_step(tbh_decoder *d, int32_t token, float *logits);

/* ---- TBF v1 model files ------------------------------------------------ */
/* Reader of the .tbf files ModelWeights.save writes and ModelWeights.load
 * reads (Sources/TinyBrainRuntime/ModelWeights.swift:376-488, :496-798), and
 * Scripts/convert_model.py:462-706 writes.  The file is memory-mapped and
 * every field bounds-checked (malformed: TBH_E_INVALID).  Descriptors and
 * fp32 pointers point into the mapping and stay valid until tbh_tbf_close. */
typedef struct tbh_tbf tbh_tbf;
typedef struct tbh_tbf_config {    /* ModelConfig (ModelRunner.swift:26-120) */
    int32_t num_layers;
    int32_t hidden;
    int32_t num_heads;
    int32_t num_kv_heads;          /* default num_heads */
    int32_t vocab;
    int32_t max_seq;
    int32_t intermediate;          /* default 4 * hidden */
    float partial_rotary_factor;   /* default 1.0 */
    char architecture[16];         /* default "llama" */
} tbh_tbf_config;
typedef struct tbh_tbf_tensor_info {
    const char *name;              /* owned by the file handle */
    int32_t ndim;
    int32_t quantized;             /* has a quantization metadata entry */
    int64_t dims[4];
    int64_t offset;                /* absolute file offset of the blob */
    int64_t bytes;
} tbh_tbf_tensor_info;

tbh_status tbh_tbf_open(const char *path, tbh_tbf **out);
tbh_status tbh_tbf_close(tbh_tbf *f);
tbh_status tbh_tbf_get_config(const tbh_tbf *f, tbh_tbf_config *cfg);
int32_t tbh_tbf_tensor_count(const tbh_tbf *f);
tbh_status tbh_tbf_tensor(const tbh_tbf *f, int32_t index, tbh_tbf_tensor_info *t);
tbh_status tbh_tbf_find(const tbh_tbf *f, const char *name, int32_t *index);
/* The quantized tensor as ModelWeights.load builds it (:676-685): precision
 * 2 is INT4 (layout NK_FLAT when the converter wrote it, mode byte 3;
 * KN_FLAT when ModelWeights.save did, mode byte 2); INT8 mode 2 is
 * per-channel, other INT8 modes symmetric. */
tbh_status tbh_tbf_qtensor(const tbh_tbf *f, int32_t index, tbh_qtensor_desc *desc);
tbh_status tbh_tbf_floats(const tbh_tbf *f, int32_t index, const float **data, int64_t *count);
/* A decoder for a LLaMA-architecture file (ModelWeights.load followed by
 * ModelRunner): every quantized projection repacked once; max_seq 0 = the
 * file's maxSeqLen.  TBH_E_UNSUPPORTED for other architectures, biases or an
 * ungated FFN. */
tbh_status tbh_tbf_load_decoder(tbh_device *dev, const tbh_tbf *f, int32_t max_seq,
                                tbh_decoder **out);

/* ---- dequantize (verification) ----------------------------------------- */
/* Replaces QuantizedTensor.dequantize() (QuantizedTensor.swift:182-286) for
 * the uploaded weight: writes the [K, N] row-major fp32 matrix that the
 * matmul multiplies by, bit-identical to (float)(q - zp) * scale.  For
 * KN_FLAT weights this is exactly the reference's dequantize() output; for
 * NK_FLAT INT4 it is that output read in the converter's [N, K] order and
 * transposed.  Host pointer, synchronous. */
tbh_status tbh_dequantize(tbh_device *dev, const tbh_weight *w, float *out);
tbh_status tbh_dequantize_device(const tbh_weight *w, float *out, void *stream);

/* ---- the other backend protocols (Backend.swift:177-228) --------------- */
/* Each op has a host-pointer call (synchronous, serialised per device, like
 * tbh_matmul) and a _device call (device pointers, enqueued on a hipStream_t
 * and returning after the launch).  Sizes of 0 are no-ops.  Results are fp32
 * computed in fp32. */

/* SoftmaxBackend.softmax (Backend.swift:180-186; MetalBackend.swift:1073-1134,
 * Shaders/Softmax.metal): each of `rows` rows of `cols` elements becomes
 * exp(x - max) / (sum + 1e-7), the epsilon of Tensor.softmaxCPU
 * (Tensor.swift:1271-1330). */
tbh_status tbh_softmax(tbh_device *dev, const float *x, int64_t rows, int64_t cols, float *y);
tbh_status tbh_softmax_device(tbh_device *dev, const float *x, int64_t rows, int64_t cols, float *y,
                              void *stream);

/* RMSNormBackend.rmsnorm (Backend.swift:188-199; MetalBackend.swift:1146-1207):
 * per row of `hidden` elements, y = x * (1 / sqrt(sum(x^2) / hidden + eps)) *
 * weight, as Tensor.rmsNormCPU (Tensor.swift:1538-1556). */
tbh_status tbh_rmsnorm(tbh_device *dev, const float *x, int64_t rows, int64_t hidden, const float *weight,
                       float eps, float *y);
tbh_status tbh_rmsnorm_device(tbh_device *dev, const float *x, int64_t rows, int64_t hidden,
                              const float *weight, float eps, float *y, void *stream);

/* ActivationBackend (Backend.swift:222-228): silu y = x / (1 + exp(-x))
 * (Tensor.swift:1135-1141); gelu, tanh form, y = 0.5 x (1 + tanh(sqrt(2/pi)
 * (x + 0.044715 x^3))) (Tensor.swift:1107-1121). */
tbh_status tbh_silu(tbh_device *dev, const float *x, int64_t n, float *y);
tbh_status tbh_silu_device(tbh_device *dev, const float *x, int64_t n, float *y, void *stream);
tbh_status tbh_gelu(tbh_device *dev, const float *x, int64_t n, float *y);
tbh_status tbh_gelu_device(tbh_device *dev, const float *x, int64_t n, float *y, void *stream);

/* AttentionBackend.attention (Backend.swift:201-220; MetalBackend.swift:1381-1525,
 * Shaders/FlashAttention.metal).  q [batch][seq_len][num_heads * head_dim],
 * k and v [batch][kv_len][num_kv_heads * head_dim], optional additive mask
 * [kv_len] shared by every query (0 attends, -inf ignores), out shaped like
 * q.  Query head h reads key/value head h / (num_heads / num_kv_heads);
 * scores are q.k / sqrt(head_dim) + mask; out = sum(p v) / (sum(p) + 1e-7)
 * with p = exp(score - max) over all kv_len positions.  A row whose
 * positions are all masked gives NaN, as the reference's CPU attention does;
 * kv_len 0 gives zeros. 
 * num_heads must be a multiple of num_kv_heads; head_dim <= 256. */
typedef struct tbh_attention_shape {
    int64_t batch;
    int64_t seq_len;
    int64_t kv_len;
    int32_t head_dim;
    int32_t num_heads;
    int32_t num_kv_heads;
} tbh_attention_shape;

tbh_status tbh_attention(tbh_device *dev, const tbh_attention_shape *shape, const float *q, const float *k,
                         const float *v, const float *mask, float *out);
tbh_status tbh_attention_device(tbh_device *dev, const tbh_attention_shape *shape, const float *q,
                                const float *k, const float *v, const float *mask, float *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* TINYBRAIN_HIP_H */

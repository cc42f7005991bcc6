// tbh_internal.h -- shared definitions of libtinybrain_hip (not installed).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "tinybrain_hip.h"

namespace tbh {

// Repacked HBM layouts.  A "chunk" is 16 bytes of one row: 16 INT8 or 32
// INT4 elements along K, loaded by one lane with one 128-bit load.
constexpr int kChunkBytes = 16;
constexpr int kInt8ChunkElems = 16;
constexpr int kInt4ChunkElems = 32;

// INT4 K-group scales and zero points of the row layout, [Np / 4][G][4]:
// the four rows of a row quad sit side by side for each group, so a wave
// that owns four rows reads the scales of one chunk with one 16-byte load.
// Np is a multiple of 8.
__host__ __device__ __forceinline__ int64_t kgroup_index(int64_t n, int64_t g, int64_t G) {
    return ((n >> 2) * G + g) * 4 + (n & 3);
}

// Largest K or N of a weight: the kernels hold row and column indices (and
// their padded forms) in 32-bit integers.
constexpr int64_t kMaxDim = (int64_t)1 << 30;

// Largest x plus y (bytes) that tbh_matmul passes through its page-locked
// host staging; larger calls copy straight from the caller's arrays.
constexpr size_t kPinnedStageBytes = (size_t)64 << 20;

// Largest x tile (M * Kp fp32) the VALU GEMV keeps in LDS.
constexpr int64_t kMaxLdsBytes = 64 * 1024;

// MFMA GEMV tiles: 16 rows x 128 K (INT4) or x 64 K (INT8) per 1 KiB, and
// the LDS budget of one stage of x fragments.
constexpr int kMfmaInt4TileK = 128;
constexpr int kMfmaInt8TileK = 64;
constexpr int64_t kMgemvLdsBytes = 32 * 1024;
constexpr int kMgemvDepth = 4;  // weight tiles in flight per wave

enum class Path : int32_t {
    Int8Row = TBH_PATH_INT8_ROW,
    Int4KGroup = TBH_PATH_INT4_KGROUP,
    Int4NGroup = TBH_PATH_INT4_NGROUP,
    Generic = TBH_PATH_GENERIC,
};

}  // namespace tbh

struct tbh_device {
    int32_t ordinal = 0;
    int32_t cu_count = 0;
    hipStream_t stream = nullptr;
    std::mutex mu;               // serialises tbh_matmul / tbh_dequantize
    std::atomic<int> sgemv_min_rows{0};   // TBH_OPT_SGEMV_MIN_ROWS; 0 = per-weight rule
    std::atomic<int> mfma_min_rows{0};    // TBH_OPT_MFMA_MIN_ROWS; 0 = per-weight rule
    void *stage = nullptr;       // device staging for the host-pointer calls
    size_t stage_bytes = 0;
    void *pin = nullptr;         // page-locked host staging for the host-pointer calls
    void *pin_dev = nullptr;     // the device's view of it
    size_t pin_bytes = 0;
    uint32_t *done_flag = nullptr;   // coherent host word a host-pointer call's last launch writes
    uint32_t *done_flag_dev = nullptr;   // the device's view of it
    uint32_t done_seq = 0;           // value the next call waits for (under mu)
    std::atomic<int> host_entry{2};  // TBH_OPT_HOST_ENTRY: how tbh_matmul moves x and y
    std::atomic<int> host_wait{1};   // TBH_OPT_HOST_WAIT: how tbh_matmul waits
    void *noalloc_scratch = nullptr;   // this GPU's scratch array (tbh_matmul_device_noalloc)
    std::atomic<int64_t> noalloc_limit{0};   // TBH_OPT_NOALLOC_SCRATCH_BYTES; 0 = the whole array

    // Per-stream device workspaces (split-K partial sums): calls on different
    // streams never share one.  A workspace that has to grow is replaced, not
    // freed: the old buffer moves to `retired`, because a HIP graph captured
    // earlier on that stream still holds its address.  Both lists are freed
    // by tbh_device_close after one device-wide synchronisation.
    struct Workspace {
        hipStream_t stream;
        void *ptr;
        size_t bytes;
    };
    std::mutex ws_mu;
    std::vector<Workspace> workspaces;
    std::vector<void *> retired;
};

struct tbh_weight {
    tbh_device *dev = nullptr;
    int64_t K = 0, N = 0;
    int32_t precision = 0, mode = 0, layout = 0, group_size = 0;
    tbh::Path path = tbh::Path::Generic;

    // fast paths: data [Np][row_bytes], offset-binary values
    int64_t Kp = 0, Np = 0, row_bytes = 0;
    uint8_t *data = nullptr;
    float *scales = nullptr;     // Int8Row [Np]; Int4KGroup [Np/4][G][4] (row quads); Int4NGroup [NB][Kp]
    int8_t *zp = nullptr;        // Int8Row [Np]; Int4KGroup as scales; null when all zero
    int64_t groups_per_row = 1;  // G (Int4KGroup)
    int32_t chunks_per_group = 1;
    int32_t rows_per_nblock = 1; // Int4NGroup
    // Int4NGroup built by the decoder from two weights of equal shape whose
    // rows are interleaved (row 2j: first weight's j, row 2j + 1: second's):
    // scales are both weights' tables stacked, nb_half N-blocks each.
    bool ng_pairs = false;
    int32_t nb_half = 0;
    // Int4NGroup (not pairs): per N-block e with |scale| < 2^e for its finite
    // scales (0 when all are zero), for the prefill GEMM's f16 scaling
    int32_t *ng_sexp = nullptr;
    int64_t n_ng_sexp = 0;
    // some N-block holds a nonzero finite scale below 2^(e - 36), so that a
    // weight 16 q s 2^(8 - e) can fall under the f16 range: the prefill GEMM
    // takes a variant that floors such scales (gemm_ngw with FLOOR)
    bool ng_wide = false;
    bool mfma_tiles = false;     // data in 1 KiB MFMA tiles (else K-contiguous rows)

    // generic path: the reference arrays as given
    int8_t *raw = nullptr;
    int64_t raw_bytes = 0;
    float *raw_scales = nullptr;
    int64_t n_scales = 0;
    int8_t *raw_zp = nullptr;

    // element counts of the device arrays above, as uploaded
    int64_t n_data = 0, n_scales_dev = 0, n_zp_dev = 0;
    int64_t n_raw = 0, n_raw_scales = 0, n_raw_zp = 0;

    int64_t device_bytes = 0;
    int64_t stream_bytes = 0;
};

namespace tbh {

// Thread-local error reporting (tbh_api.hip).
tbh_status set_error(tbh_status st, const std::string &msg);
tbh_status hip_error(hipError_t e, const char *what);
// Makes `ordinal` the calling thread's current HIP device (tbh_api.hip).
tbh_status use_device(int32_t ordinal);

// Two INT4 runtime-layout weights (groups along N) of one shape as one
// Int4NGroup weight with their rows interleaved (row 2j: a's j, row 2j + 1:
// b's j) for the decode step's gate|up pair epilogue (tbh_api.hip).
tbh_status create_ngroup_pair(tbh_device *dev, const tbh_qtensor_desc *a, const tbh_qtensor_desc *b,
                              tbh_weight **out);

// Host-side check, before any launch, that the device arrays a weight's
// kernels index exist and have the sizes those kernels assume.
bool weight_arrays_ok(const tbh_weight &w);

// Kernel launchers.  The API layer checks shapes and weight_arrays_ok first.
struct GemvArgs {
    const float *x;
    int64_t ldx;
    float *y;
    int64_t ldy;
    int64_t M;
};

// Fast VALU dequant-GEMV for M <= 4 rows of x (tbh_gemv.hip).  Returns
// hipErrorInvalidValue when the x tile does not fit in LDS.
hipError_t launch_gemv(const tbh_weight &w, const GemvArgs &a, hipStream_t s);
// Largest number of x rows one launch_gemv call handles for this weight
// (0 when the fast path cannot take it).
int64_t gemv_max_rows(const tbh_weight &w);
// Whether launch_gemv takes eight rows of this x in one launch (the burst
// kernel; K up to 2048 INT8 or INT4, no zero points, 16-byte aligned x).
bool gemv8_supported(const tbh_weight &w, const float *x, int64_t ldx);

// Fused decode GEMV (M = 1, tbh_gemv.hip): y = W . pro(x) (+ y).
enum {
    PRO_NONE = 0,     // x as given
    PRO_RMSNORM = 1,  // rmsnorm(x) * g with epsilon eps (Tensor.swift:1543-1556)
};
enum {
    EPI_STORE = 0,       // y = result
    EPI_ACCUMULATE = 1,  // y += result (the residual adds, ModelRunner.swift:434, :457)
    EPI_SILU_PAIR = 2,   // rows 2j, 2j + 1 are a gate and an up row:
                         // y[j] = silu(r[2j]) * r[2j + 1] (:449-451)
};
struct FusedGemvArgs {
    const float *x;
    const float *g;
    float eps;
    float *y;
    int prologue;
    int epilogue;
    float *x_copy = nullptr;     // also store x as given here ([K], not aliasing x or y)
    int32_t *advance = nullptr;  // also add 1 to advance[0] (read by no other work of the launch)
};
bool gemv_fused_supported(const tbh_weight &w);
hipError_t launch_gemv_fused(const tbh_weight &w, const FusedGemvArgs &f, hipStream_t s);

// MFMA dequant-GEMV for 2 <= M <= 8 rows of x on row-layout INT4 K-group
// weights without zero points (tbh_sgemv.hip).  launch_sgemv returns
// hipErrorInvalidValue for shapes it does not take (odd alignment of x,
// M out of range, no workspace while capturing a long row).
bool sgemv_supported(const tbh_weight &w);
struct Scratch;
hipError_t launch_sgemv(const tbh_weight &w, const GemvArgs &a, hipStream_t s, const Scratch &scr);

// MFMA dequant-GEMV for M <= 8 rows of x on MFMA-tiled weights (tbh_mgemv.hip).
hipError_t launch_mgemv(const tbh_weight &w, const GemvArgs &a, hipStream_t s);

// Generic INT4 kernel over the reference flat layout (tbh_ref_kernels.hip).
hipError_t launch_generic(const tbh_weight &w, const GemvArgs &a, hipStream_t s);

// Prefill dequant-GEMM on bf16 MFMA (tbh_prefill.hip): x [M][ldx] bf16
// bits, y [M][ldy] fp32.  Needs prefill_supported(w) (INT8 rows, INT4
// K-groups, runtime-layout INT4 whose N-blocks tile 64 outputs), K % 8 == 0,
// ldx % 8 == 0 and a 16-byte aligned x.
bool prefill_supported(const tbh_weight &w);
hipError_t launch_prefill(const tbh_weight &w, const uint16_t *x, int64_t ldx, int64_t M, float *y,
                          int64_t ldy, hipStream_t s, const Scratch &scr);

// The same GEMM for fp32 x [M][ldx] (16-byte aligned rows, K % 8 == 0):
// each x row is split exactly into three bf16 pieces and a zero
// row, the four rows go through the bf16 MFMAs, and the epilogue adds each
// row's four results; past 64 rows of INT8-row or INT4 K-group weights, two
// f16 pieces of x scaled per row on the f16 MFMA (tbh_prefill.hip).
// hipErrorInvalidValue for weights or shapes it does not take.
hipError_t launch_prefill_f32(const tbh_weight &w, const float *x, int64_t ldx, int64_t M, float *y,
                              int64_t ldy, hipStream_t s, const Scratch &scr);

// Device workspace of at least `bytes` owned by (dev, stream), grown on
// demand (tbh_api.hip).  Growing allocates a new buffer and keeps the old one
// until the device closes.  Returns nullptr when it would have to grow while
// the stream is being captured into a graph, or when the allocation fails.
void *stream_workspace(tbh_device *dev, hipStream_t s, size_t bytes);

// Where a launch takes its scratch memory (split-K partial sums) from: the
// per-stream workspace of `dev`, grown on demand, or a fixed buffer that is
// never grown (the no-allocation entry point).
struct Scratch {
    tbh_device *dev = nullptr;
    void *fixed = nullptr;
    size_t fixed_bytes = 0;
    mutable size_t shortfall = 0;   // bytes a fixed buffer could not provide
    // bytes at the start of the buffer that a caller keeps for itself (a
    // multiple of 256): get() hands out memory after them
    size_t offset = 0;

    bool is_fixed() const { return fixed != nullptr; }
    // nullptr when the bytes are not available: a fixed buffer too small
    // (shortfall set; the launcher then returns hipErrorOutOfMemory before
    // launching anything), or a workspace that cannot grow (capture, OOM;
    // the launcher then takes a path without scratch).
    void *get(hipStream_t s, size_t bytes) const {
        if (fixed) {
            if (offset + bytes <= fixed_bytes) return (char *)fixed + offset;
            shortfall = offset + bytes;
            return nullptr;
        }
        void *b = stream_workspace(dev, s, offset + bytes);
        return b ? (char *)b + offset : nullptr;
    }
};

// Bit-exact dequantization to [K, N] row-major (tbh_ref_kernels.hip).
hipError_t launch_dequant(const tbh_weight &w, float *out, hipStream_t s);

}  // namespace tbh

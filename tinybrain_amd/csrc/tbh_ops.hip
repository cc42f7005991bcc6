// tbh_ops.hip -- the backend protocols on either side of the quantized
// matmul (Sources/TinyBrainRuntime/Backend.swift:177-228): softmax, RMSNorm,
// SiLU / GELU and attention, replacing MetalBackend's implementations
// (Sources/TinyBrainMetal/MetalBackend.swift:1062-1260, 1362-1525).
//
// Row ops (softmax, RMSNorm) give each row one wave (short rows, four rows
// per 256-thread block) or one block (rows longer than kWaveRowMax); a
// thread walks its strided elements with 16-byte loads when the row allows,
// and the partial results meet through cross-lane reductions.  Softmax keeps
// a running (max, sum) pair per thread, so x is read twice (once for the
// pair, once for the output) instead of the reference kernel's three reads
// and two writes.  Attention gives each (batch, query, head) row one wave:
// a lane scores one key position of a 64-position tile, the wave keeps an
// online softmax across tiles, and each lane accumulates head_dim / 64
// output elements from coalesced value rows.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "tbh_internal.h"

namespace tbh {
namespace {

constexpr float kSoftmaxEps = 1e-7f;   // Tensor.softmaxCPU default; Softmax.metal
constexpr float kAttnEps = 1e-7f;      // FlashAttention.metal final division
constexpr int64_t kWaveRowMax = 1024;  // longest row one wave handles
constexpr int kAttnMaxHeadDim = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// (max, sum of exp(x - max)) pairs: merge b into a.  An empty pair is
// (-inf, 0).
__device__ __forceinline__ void ms_merge(float &m, float &s, float m2, float s2) {
    const float mm = fmaxf(m, m2);
    if (mm == -INFINITY) return;
    s = s * expf(m - mm) + s2 * expf(m2 - mm);
    m = mm;
}

__device__ __forceinline__ void ms_add(float &m, float &s, float x) {
    if (x == -INFINITY) return;  // contributes exp(-inf) = 0
    if (x > m) {
        s = s * expf(m - x) + 1.0f;
        m = x;
    } else {
        s += expf(x - m);
    }
}

// Reduction of one value per thread over a row's threads: a wave (W == 1)
// or the whole 256-thread block (W == 4).
template <int W>
__device__ __forceinline__ float row_sum(float v, float *red) {
    v = wave_sum(v);
    if (W == 1) return v;
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

template <int W>
__device__ __forceinline__ void row_ms(float &m, float &s, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
        ms_merge(m, s, m2, s2);
    }
    if (W == 1) return;
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        red[2 * wave] = m;
        red[2 * wave + 1] = s;
    }
    __syncthreads();
    m = red[0];
    s = red[1];
#pragma unroll
    for (int i = 1; i < 4; ++i) ms_merge(m, s, red[2 * i], red[2 * i + 1]);
}

// Softmax over rows.  W = waves per row (1: four rows per block; 4: one row
// per block).  VEC: 16-byte loads and stores (cols % 4 == 0, aligned rows).
template <int W, bool VEC>
__global__ __launch_bounds__(256) void softmax_rows(const float *__restrict__ x, float *__restrict__ y,
                                                    int64_t rows, int64_t cols) {
    __shared__ float red[8];
    constexpr int T = 64 * W;
    const int64_t row = (int64_t)blockIdx.x * (4 / W) + (threadIdx.x / T);
    const int t = threadIdx.x % T;
    // Rows past the end compute on the last row and store nothing, so every
    // thread reaches the block barriers.
    const int64_t r = row < rows ? row : rows - 1;
    const float *xr = x + r * cols;
    float m = -INFINITY, s = 0.0f;
    if (VEC) {
        for (int64_t i = t; i < cols / 4; i += T) {
            const float4 v = ((const float4 *)xr)[i];
            ms_add(m, s, v.x);
            ms_add(m, s, v.y);
            ms_add(m, s, v.z);
            ms_add(m, s, v.w);
        }
    } else {
        for (int64_t i = t; i < cols; i += T) ms_add(m, s, xr[i]);
    }
    row_ms<W>(m, s, red);
    if (row >= rows) return;
    // Tensor.softmaxCPU: exp(x - max) / (sum + epsilon); an all -inf row
    // gives NaN there (x - max = NaN) and here.
    const float den = s + kSoftmaxEps;
    float *yr = y + r * cols;
    if (VEC) {
        for (int64_t i = t; i < cols / 4; i += T) {
            const float4 v = ((const float4 *)xr)[i];
            float4 o;
            o.x = expf(v.x - m) / den;
            o.y = expf(v.y - m) / den;
            o.z = expf(v.z - m) / den;
            o.w = expf(v.w - m) / den;
            ((float4 *)yr)[i] = o;
        }
    } else {
        for (int64_t i = t; i < cols; i += T) yr[i] = expf(xr[i] - m) / den;
    }
}

template <int W, bool VEC>
__global__ __launch_bounds__(256) void rmsnorm_rows(const float *__restrict__ x, const float *__restrict__ g,
                                                    float eps, float *__restrict__ y, int64_t rows,
                                                    int64_t hidden) {
    __shared__ float red[8];
    constexpr int T = 64 * W;
    const int64_t row = (int64_t)blockIdx.x * (4 / W) + (threadIdx.x / T);
    const int t = threadIdx.x % T;
    const int64_t r = row < rows ? row : rows - 1;
    const float *xr = x + r * hidden;
    float ss = 0.0f;
    if (VEC) {
        for (int64_t i = t; i < hidden / 4; i += T) {
            const float4 v = ((const float4 *)xr)[i];
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    } else {
        for (int64_t i = t; i < hidden; i += T) ss += xr[i] * xr[i];
    }
    ss = row_sum<W>(ss, red);
    if (row >= rows) return;
    // Tensor.rmsNormCPU: invRMS = 1 / sqrt(ss / hidden + eps); x * invRMS * w
    const float inv = 1.0f / sqrtf(ss / (float)hidden + eps);
    float *yr = y + r * hidden;
    if (VEC) {
        for (int64_t i = t; i < hidden / 4; i += T) {
            const float4 v = ((const float4 *)xr)[i], w = ((const float4 *)g)[i];
            ((float4 *)yr)[i] = float4{v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w};
        }
    } else {
        for (int64_t i = t; i < hidden; i += T) yr[i] = xr[i] * inv * g[i];
    }
}

enum Act { ACT_SILU = 0, ACT_GELU = 1 };

template <int A>
__device__ __forceinline__ float act(float x, float s2p) {
    if (A == ACT_SILU) return x / (1.0f + expf(-x));
    const float x3 = x * x * x;
    const float inner = s2p * (x + 0.044715f * x3);
    return 0.5f * x * (1.0f + tanhf(inner));
}

template <int A, bool VEC>
__global__ __launch_bounds__(256) void activation(const float *__restrict__ x, float *__restrict__ y, int64_t n,
                                                  float s2p) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (VEC) {
        for (int64_t i = i0; i < n / 4; i += stride) {
            const float4 v = ((const float4 *)x)[i];
            ((float4 *)y)[i] = float4{act<A>(v.x, s2p), act<A>(v.y, s2p), act<A>(v.z, s2p), act<A>(v.w, s2p)};
        }
        for (int64_t i = (n / 4) * 4 + i0; i < n; i += stride) y[i] = act<A>(x[i], s2p);
    } else {
        for (int64_t i = i0; i < n; i += stride) y[i] = act<A>(x[i], s2p);
    }
}

struct AttnArgs {
    const float *q, *k, *v, *mask;
    float *out;
    int64_t rows;  // batch * seq_len * num_heads
    int64_t seq_len, kv_len;
    int32_t hd, nh, nkv;
    float scale;
};

// One wave per (batch, query, head) row; ND = output elements per lane.
template <int ND, bool VEC>
__global__ __launch_bounds__(256) void attention_rows(const AttnArgs a) {
    __shared__ __attribute__((aligned(16))) float qs[4][kAttnMaxHeadDim];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    const int64_t r = row < a.rows ? row : a.rows - 1;
    const int h = (int)(r % a.nh);
    const int64_t bq = r / a.nh;               // batch * seq_len + query
    const int64_t b = bq / a.seq_len;
    const int kvh = h / (a.nh / a.nkv);
    const int64_t kvd = (int64_t)a.nkv * a.hd;
    const float *qrow = a.q + bq * a.nh * a.hd + (int64_t)h * a.hd;
    const float *kb = a.k + b * a.kv_len * kvd + (int64_t)kvh * a.hd;
    const float *vb = a.v + b * a.kv_len * kvd + (int64_t)kvh * a.hd;
    for (int d = lane; d < a.hd; d += 64) qs[wave][d] = qrow[d];
    __syncthreads();

    float m = -INFINITY, l = 0.0f, o[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) o[i] = 0.0f;
    for (int64_t t0 = 0; t0 < a.kv_len; t0 += 64) {
        const int64_t t = t0 + lane;
        float s = -INFINITY;
        if (t < a.kv_len) {
            const float *kr = kb + t * kvd;
            float dot = 0.0f;
            if (VEC) {
                for (int d = 0; d < a.hd; d += 4) {
                    const float4 kv = *(const float4 *)(kr + d), qv = *(const float4 *)&qs[wave][d];
                    dot += qv.x * kv.x + qv.y * kv.y + qv.z * kv.z + qv.w * kv.w;
                }
            } else {
                for (int d = 0; d < a.hd; ++d) dot += qs[wave][d] * kr[d];
            }
            s = dot * a.scale;
            if (a.mask) s += a.mask[t];
        }
        const float nm = fmaxf(m, wave_max(s));
        if (nm == -INFINITY) continue;  // every position so far is masked
        const float corr = expf(m - nm);
        const float p = expf(s - nm);
        l = l * corr + wave_sum(p);
#pragma unroll
        for (int i = 0; i < ND; ++i) o[i] *= corr;
        const int nt = (int)std::min<int64_t>(64, a.kv_len - t0);
        for (int j = 0; j < nt; ++j) {
            const float pj = __shfl(p, j);
            const float *vr = vb + (t0 + j) * kvd;
#pragma unroll
            for (int i = 0; i < ND; ++i) {
                const int d = lane + 64 * i;
                if (d < a.hd) o[i] += pj * vr[d];
            }
        }
        m = nm;
    }
    if (row >= a.rows) return;
    float *orow = a.out + bq * a.nh * a.hd + (int64_t)h * a.hd;
    const float den = l + kAttnEps;
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        const int d = lane + 64 * i;
        // No positions (kv_len 0) leaves zeros, as both reference kernels do;
        // positions that are all masked give NaN, as the reference's CPU
        // attention does (exp(-inf - -inf)).
        if (d < a.hd) orow[d] = (m == -INFINITY && a.kv_len > 0) ? NAN : o[i] / den;
    }
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

unsigned grid_for(int64_t blocks, const tbh_device *dev) {
    const int64_t cap = 8 * (int64_t)std::max(1, dev->cu_count);
    return (unsigned)std::max<int64_t>(1, std::min(blocks, cap));
}

hipError_t launch_softmax(const float *x, int64_t rows, int64_t cols, float *y, hipStream_t s) {
    const bool vec = cols % 4 == 0 && aligned16(x) && aligned16(y);
    if (cols <= kWaveRowMax) {
        const dim3 grid((unsigned)((rows + 3) / 4));
        if (vec) hipLaunchKernelGGL((softmax_rows<1, true>), grid, dim3(256), 0, s, x, y, rows, cols);
        else hipLaunchKernelGGL((softmax_rows<1, false>), grid, dim3(256), 0, s, x, y, rows, cols);
    } else {
        const dim3 grid((unsigned)rows);
        if (vec) hipLaunchKernelGGL((softmax_rows<4, true>), grid, dim3(256), 0, s, x, y, rows, cols);
        else hipLaunchKernelGGL((softmax_rows<4, false>), grid, dim3(256), 0, s, x, y, rows, cols);
    }
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, int64_t rows, int64_t hidden, const float *g, float eps, float *y,
                          hipStream_t s) {
    const bool vec = hidden % 4 == 0 && aligned16(x) && aligned16(y) && aligned16(g);
    if (hidden <= kWaveRowMax) {
        const dim3 grid((unsigned)((rows + 3) / 4));
        if (vec) hipLaunchKernelGGL((rmsnorm_rows<1, true>), grid, dim3(256), 0, s, x, g, eps, y, rows, hidden);
        else hipLaunchKernelGGL((rmsnorm_rows<1, false>), grid, dim3(256), 0, s, x, g, eps, y, rows, hidden);
    } else {
        const dim3 grid((unsigned)rows);
        if (vec) hipLaunchKernelGGL((rmsnorm_rows<4, true>), grid, dim3(256), 0, s, x, g, eps, y, rows, hidden);
        else hipLaunchKernelGGL((rmsnorm_rows<4, false>), grid, dim3(256), 0, s, x, g, eps, y, rows, hidden);
    }
    return hipGetLastError();
}

// sqrt(2 / pi) formed in fp32 as Tensor.geluCPU does (Tensor.swift:1110)
float gelu_s2p() { return std::sqrt(2.0f / 3.14159265358979f); }

template <int A>
hipError_t launch_act(const tbh_device *dev, const float *x, int64_t n, float *y, hipStream_t s) {
    const bool vec = aligned16(x) && aligned16(y);
    const unsigned grid = grid_for(((vec ? n / 4 : n) + 255) / 256, dev);
    if (vec) hipLaunchKernelGGL((activation<A, true>), dim3(grid), dim3(256), 0, s, x, y, n, gelu_s2p());
    else hipLaunchKernelGGL((activation<A, false>), dim3(grid), dim3(256), 0, s, x, y, n, gelu_s2p());
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t s) {
    const bool vec = a.hd % 4 == 0 && aligned16(a.q) && aligned16(a.k);
    const dim3 grid((unsigned)((a.rows + 3) / 4));
    const int nd = (a.hd + 63) / 64;
#define TBH_ATTN(ND)                                                                                     \
    do {                                                                                                 \
        if (vec) hipLaunchKernelGGL((attention_rows<ND, true>), grid, dim3(256), 0, s, a);              \
        else hipLaunchKernelGGL((attention_rows<ND, false>), grid, dim3(256), 0, s, a);                 \
    } while (0)
    switch (nd) {
    case 1: TBH_ATTN(1); break;
    case 2: TBH_ATTN(2); break;
    case 3: TBH_ATTN(3); break;
    default: TBH_ATTN(4); break;
    }
#undef TBH_ATTN
    return hipGetLastError();
}

// Grows the device's staging buffer (callers hold dev->mu).
tbh_status ensure_stage(tbh_device *dev, size_t need) {
    if (dev->stage_bytes >= need) return TBH_OK;
    hipFree(dev->stage);
    dev->stage = nullptr;
    dev->stage_bytes = 0;
    hipError_t e = hipMalloc(&dev->stage, need);
    if (e != hipSuccess) return hip_error(e, "staging buffer");
    dev->stage_bytes = need;
    return TBH_OK;
}

size_t pad256(size_t b) { return (b + 255) & ~size_t(255); }

// Host-pointer call: copy the inputs in, run `enqueue` on the device's
// stream, copy the output back, wait.
template <class F>
tbh_status host_call(tbh_device *dev, const char *what, std::initializer_list<std::pair<const void *, size_t>> ins,
                     void *out, size_t out_bytes, F enqueue) {
    std::lock_guard<std::mutex> lock(dev->mu);
    tbh_status st = use_device(dev->ordinal);
    if (st != TBH_OK) return st;
    size_t need = pad256(out_bytes);
    for (auto &in : ins) need += pad256(in.second);
    st = ensure_stage(dev, need);
    if (st != TBH_OK) return st;
    char *p = (char *)dev->stage;
    std::vector<const void *> dptr;
    for (auto &in : ins) {
        if (in.first && in.second) {
            hipError_t e = hipMemcpyAsync(p, in.first, in.second, hipMemcpyHostToDevice, dev->stream);
            if (e != hipSuccess) return hip_error(e, what);
            dptr.push_back(p);
        } else {
            dptr.push_back(nullptr);
        }
        p += pad256(in.second);
    }
    hipError_t e = enqueue(dptr, (void *)p, dev->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(out, p, out_bytes, hipMemcpyDeviceToHost, dev->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
    if (e != hipSuccess) return hip_error(e, what);
    return TBH_OK;
}

tbh_status check_rows(const char *what, tbh_device *dev, const void *x, int64_t rows, int64_t cols,
                      const void *y) {
    if (!dev) return set_error(TBH_E_INVALID, std::string(what) + ": dev is NULL");
    if (rows < 0 || cols < 0) return set_error(TBH_E_INVALID, std::string(what) + ": negative size");
    if (rows > 0 && cols > 0 && (!x || !y)) return set_error(TBH_E_INVALID, std::string(what) + ": NULL pointer");
    if (rows > INT32_MAX) return set_error(TBH_E_UNSUPPORTED, std::string(what) + ": more than 2^31 rows");
    return TBH_OK;
}

tbh_status check_attention(tbh_device *dev, const tbh_attention_shape *sh, const float *q, const float *k,
                           const float *v, const float *out, AttnArgs &a) {
    if (!dev || !sh) return set_error(TBH_E_INVALID, "attention: NULL device or shape");
    if (sh->batch < 0 || sh->seq_len < 0 || sh->kv_len < 0 || sh->head_dim <= 0 || sh->num_heads <= 0 ||
        sh->num_kv_heads <= 0)
        return set_error(TBH_E_INVALID, "attention: invalid shape");
    if (sh->num_heads < sh->num_kv_heads || sh->num_heads % sh->num_kv_heads != 0)
        return set_error(TBH_E_INVALID, "numHeads must be a multiple of numKVHeads");
    if (sh->head_dim > kAttnMaxHeadDim)
        return set_error(TBH_E_UNSUPPORTED, "attention: head_dim > 256");
    a.rows = sh->batch * sh->seq_len * sh->num_heads;
    if (a.rows > 0 && (!q || !out || (sh->kv_len > 0 && (!k || !v))))
        return set_error(TBH_E_INVALID, "attention: NULL pointer");
    if ((a.rows + 3) / 4 > INT32_MAX) return set_error(TBH_E_UNSUPPORTED, "attention: too many rows");
    a.seq_len = sh->seq_len;
    a.kv_len = sh->kv_len;
    a.hd = sh->head_dim;
    a.nh = sh->num_heads;
    a.nkv = sh->num_kv_heads;
    a.scale = 1.0f / std::sqrt((float)sh->head_dim);  // MetalBackend.swift:1458
    return TBH_OK;
}

}  // namespace
}  // namespace tbh

using namespace tbh;

extern "C" {

tbh_status tbh_softmax_device(tbh_device *dev, const float *x, int64_t rows, int64_t cols, float *y,
                              void *stream) {
    tbh_status st = check_rows("tbh_softmax", dev, x, rows, cols, y);
    if (st != TBH_OK || rows == 0 || cols == 0) return st;
    if ((st = use_device(dev->ordinal)) != TBH_OK) return st;
    hipError_t e = launch_softmax(x, rows, cols, y, (hipStream_t)stream);
    return e == hipSuccess ? TBH_OK : hip_error(e, "softmax launch");
}

tbh_status tbh_softmax(tbh_device *dev, const float *x, int64_t rows, int64_t cols, float *y) {
    tbh_status st = check_rows("tbh_softmax", dev, x, rows, cols, y);
    if (st != TBH_OK || rows == 0 || cols == 0) return st;
    const size_t b = (size_t)(rows * cols) * sizeof(float);
    return host_call(dev, "tbh_softmax", {{x, b}}, y, b, [&](const std::vector<const void *> &d, void *o, hipStream_t s) {
        return launch_softmax((const float *)d[0], rows, cols, (float *)o, s);
    });
}

tbh_status tbh_rmsnorm_device(tbh_device *dev, const float *x, int64_t rows, int64_t hidden, const float *weight,
                              float eps, float *y, void *stream) {
    tbh_status st = check_rows("tbh_rmsnorm", dev, x, rows, hidden, y);
    if (st != TBH_OK || rows == 0 || hidden == 0) return st;
    if (!weight) return set_error(TBH_E_INVALID, "tbh_rmsnorm: weight is NULL");
    if ((st = use_device(dev->ordinal)) != TBH_OK) return st;
    hipError_t e = launch_rmsnorm(x, rows, hidden, weight, eps, y, (hipStream_t)stream);
    return e == hipSuccess ? TBH_OK : hip_error(e, "rmsnorm launch");
}

tbh_status tbh_rmsnorm(tbh_device *dev, const float *x, int64_t rows, int64_t hidden, const float *weight,
                       float eps, float *y) {
    tbh_status st = check_rows("tbh_rmsnorm", dev, x, rows, hidden, y);
    if (st != TBH_OK || rows == 0 || hidden == 0) return st;
    if (!weight) return set_error(TBH_E_INVALID, "tbh_rmsnorm: weight is NULL");
    const size_t b = (size_t)(rows * hidden) * sizeof(float);
    return host_call(dev, "tbh_rmsnorm", {{x, b}, {weight, (size_t)hidden * sizeof(float)}}, y, b,
                     [&](const std::vector<const void *> &d, void *o, hipStream_t s) {
                         return launch_rmsnorm((const float *)d[0], rows, hidden, (const float *)d[1], eps,
                                               (float *)o, s);
                     });
}

#define TBH_ACTIVATION(NAME, A)                                                                            \
    tbh_status tbh_##NAME##_device(tbh_device *dev, const float *x, int64_t n, float *y, void *stream) {   \
        tbh_status st = check_rows("tbh_" #NAME, dev, x, 1, n, y);                                         \
        if (st != TBH_OK || n == 0) return st;                                                             \
        if ((st = use_device(dev->ordinal)) != TBH_OK) return st;                                          \
        hipError_t e = launch_act<A>(dev, x, n, y, (hipStream_t)stream);                                  \
        return e == hipSuccess ? TBH_OK : hip_error(e, #NAME " launch");                                  \
    }                                                                                                      \
    tbh_status tbh_##NAME(tbh_device *dev, const float *x, int64_t n, float *y) {                         \
        tbh_status st = check_rows("tbh_" #NAME, dev, x, 1, n, y);                                         \
        if (st != TBH_OK || n == 0) return st;                                                             \
        const size_t b = (size_t)n * sizeof(float);                                                        \
        return host_call(dev, "tbh_" #NAME, {{x, b}}, y, b,                                                \
                         [&](const std::vector<const void *> &d, void *o, hipStream_t s) {                \
                             return launch_act<A>(dev, (const float *)d[0], n, (float *)o, s);            \
                         });                                                                               \
    }

TBH_ACTIVATION(silu, ACT_SILU)
TBH_ACTIVATION(gelu, ACT_GELU)
#undef TBH_ACTIVATION

tbh_status tbh_attention_device(tbh_device *dev, const tbh_attention_shape *shape, const float *q, const float *k,
                                const float *v, const float *mask, float *out, void *stream) {
    AttnArgs a{};
    tbh_status st = check_attention(dev, shape, q, k, v, out, a);
    if (st != TBH_OK || a.rows == 0) return st;
    if ((st = use_device(dev->ordinal)) != TBH_OK) return st;
    a.q = q;
    a.k = k;
    a.v = v;
    a.mask = mask;
    a.out = out;
    hipError_t e = launch_attention(a, (hipStream_t)stream);
    return e == hipSuccess ? TBH_OK : hip_error(e, "attention launch");
}

tbh_status tbh_attention(tbh_device *dev, const tbh_attention_shape *shape, const float *q, const float *k,
                         const float *v, const float *mask, float *out) {
    AttnArgs a{};
    tbh_status st = check_attention(dev, shape, q, k, v, out, a);
    if (st != TBH_OK || a.rows == 0) return st;
    const size_t qb = (size_t)(a.rows * a.hd) * sizeof(float);
    const size_t kb = (size_t)(shape->batch * a.kv_len * a.nkv * a.hd) * sizeof(float);
    const size_t mb = mask ? (size_t)a.kv_len * sizeof(float) : 0;
    return host_call(dev, "tbh_attention", {{q, qb}, {k, kb}, {v, kb}, {mask, mb}}, out, qb,
                     [&](const std::vector<const void *> &d, void *o, hipStream_t s) {
                         a.q = (const float *)d[0];
                         a.k = (const float *)d[1];
                         a.v = (const float *)d[2];
                         a.mask = (const float *)d[3];
                         a.out = (float *)o;
                         return launch_attention(a, s);
                     });
}

}  // extern "C"

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
// and two writes.
//
// Attention: when there are too few (query, key/value head) pairs to fill
// the chip, the key positions are split over several blocks, each writing a
// partial (max, sum, output) per head to a workspace, and a second kernel
// merges them (split-KV decoding).  Head dimensions 16/32/64/128 take one
// wave per (query, query head, range): the four waves of a block are query
// heads of one key/value head and share its rows through L1.  Other head
// dimensions that are multiples of 4 take a block per (query, key/value
// head) serving up to 8 query heads (256 positions per pass, one per
// thread); the rest a one-wave-per-row kernel.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "tbh_internal.h"
#include "tbh_wave.h"

namespace tbh {
namespace {

constexpr float kSoftmaxEps = 1e-7f;   // Tensor.softmaxCPU default; Softmax.metal
constexpr float kAttnEps = 1e-7f;      // FlashAttention.metal final division
constexpr int64_t kWaveRowMax = 1024;  // longest row one wave handles
constexpr int kAttnMaxHeadDim = 256;

__device__ __forceinline__ float wave_sum(float v) { return wave::sum(v); }
__device__ __forceinline__ float wave_max(float v) { return wave::max(v); }

// (max, sum of exp(x - max)) pairs: merge b into a.  An empty pair is
// (-inf, 0).
__device__ __forceinline__ void ms_merge(float &m, float &s, float m2, float s2) {
    const float mm = fmaxf(m, m2);
    if (mm == -INFINITY) return;
    s = s * expf(m - mm) + s2 * expf(m2 - mm);
    m = mm;
}

// Four values at once: one rescale per float4 instead of one per element.
__device__ __forceinline__ void ms_add4(float &m, float &s, float4 v) {
    const float mx = fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
    if (mx == -INFINITY) return;
    if (mx > m) {
        s *= expf(m - mx);
        m = mx;
    }
    s += (expf(v.x - m) + expf(v.y - m)) + (expf(v.z - m) + expf(v.w - m));
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
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < W; ++i) t += red[i];
    return t;
}

template <int W>
__device__ __forceinline__ void row_ms(float &m, float &s, float *red) {
    // pairs of partner lanes merged with DPP inside each 16-lane row, then
    // the four rows through readlane
    {
        float m2 = wave::dpp<wave::kXor1>(m), s2 = wave::dpp<wave::kXor1>(s);
        ms_merge(m, s, m2, s2);
        m2 = wave::dpp<wave::kXor2>(m), s2 = wave::dpp<wave::kXor2>(s);
        ms_merge(m, s, m2, s2);
        m2 = wave::dpp<wave::kHalfMirror>(m), s2 = wave::dpp<wave::kHalfMirror>(s);
        ms_merge(m, s, m2, s2);
        m2 = wave::dpp<wave::kRowMirror>(m), s2 = wave::dpp<wave::kRowMirror>(s);
        ms_merge(m, s, m2, s2);
        float mm = wave::lane_value(m, 0), ss = wave::lane_value(s, 0);
#pragma unroll
        for (int r = 16; r < 64; r += 16) ms_merge(mm, ss, wave::lane_value(m, r), wave::lane_value(s, r));
        m = mm;
        s = ss;
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
    for (int i = 1; i < W; ++i) ms_merge(m, s, red[2 * i], red[2 * i + 1]);
}

// Softmax over rows.  W = waves per row (1: four rows per 256-thread block;
// 16: one row per 1024-thread block).  VEC: 16-byte loads and stores
// (cols % 4 == 0, aligned rows).
template <int W, bool VEC>
__global__ __launch_bounds__(W == 1 ? 256 : 64 * W) void softmax_rows(const float *__restrict__ x,
                                                                     float *__restrict__ y, int64_t rows,
                                                                     int64_t cols) {
    __shared__ float red[2 * W];
    constexpr int T = 64 * W;
    const int64_t row = W == 1 ? (int64_t)blockIdx.x * 4 + (threadIdx.x / T) : (int64_t)blockIdx.x;
    const int t = threadIdx.x % T;
    // Rows past the end compute on the last row and store nothing, so every
    // thread reaches the block barriers.
    const int64_t r = row < rows ? row : rows - 1;
    const float *xr = x + r * cols;
    float m = -INFINITY, s = 0.0f;
    if (VEC) {
        for (int64_t i = t; i < cols / 4; i += T) ms_add4(m, s, ((const float4 *)xr)[i]);
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

// Register-resident rows (16-byte aligned rows, cols % 4 == 0, at most
// 8 * 64 * W float4 per row): thread t of a row's 64 * W threads holds float4
// elements t, t + 64 W, ... in registers, so x is read from memory once and y
// written once.  W = 1: four rows per 256-thread block; W = 4 or 16: one row
// per block.
template <int W>
__device__ __forceinline__ float block_max(float v, float *red) {
    v = wave_max(v);
    if (W == 1) return v;
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < W; ++i) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}

template <int W>
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    if (W == 1) return v;
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float r = 0.0f;
#pragma unroll
    for (int i = 0; i < W; ++i) r += red[i];
    __syncthreads();
    return r;
}

template <int W, int R>
__global__ __launch_bounds__(W == 1 ? 256 : 64 * W) void softmax_reg(const float *__restrict__ x,
                                                                    float *__restrict__ y, int64_t rows,
                                                                    int64_t cols) {
    __shared__ float red[W];
    constexpr int T = 64 * W;
    const int64_t row = W == 1 ? (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6) : (int64_t)blockIdx.x;
    const int t = threadIdx.x % T;
    const int64_t r = row < rows ? row : rows - 1;   // every thread reaches the barriers
    const float4 *xr = (const float4 *)(x + r * cols);
    const int n4 = (int)(cols / 4);
    float4 v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int j = t + T * i;
        v[i] = j < n4 ? xr[min(j, n4 - 1)] : float4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
    // Each thread exponentiates its own elements against its own maximum as
    // soon as its loads land (overlapping the exponentials with the rest of
    // the block's loads); the block maximum M then rescales by e^(m_t - M):
    // e^(x - m_t) e^(m_t - M) = e^(x - M).  Tensor.softmaxCPU computes
    // exp(x - max) / (sum + epsilon); an all -inf row gives NaN there
    // (x - max = NaN) and here (m_t - M = NaN).
    float mt = -INFINITY;
#pragma unroll
    for (int i = 0; i < R; ++i) mt = fmaxf(mt, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
    const bool none = mt == -INFINITY;  // this thread's elements are all -inf (or padding)
    float st = 0.0f;
#pragma unroll
    for (int i = 0; i < R; ++i) {
        v[i] = none ? float4{0.f, 0.f, 0.f, 0.f}
                    : float4{expf(v[i].x - mt), expf(v[i].y - mt), expf(v[i].z - mt), expf(v[i].w - mt)};
        const int j = t + T * i;
        if (j < n4) st += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
    const float m = block_max<W>(mt, red);
    const float f = expf(mt - m);
    const float sm = block_sum<W>(none ? 0.0f : st * f, red);
    if (row >= rows) return;
    const float k = f / (sm + kSoftmaxEps);
    float4 *yr = (float4 *)(y + r * cols);
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int j = t + T * i;
        if (j < n4) yr[j] = float4{v[i].x * k, v[i].y * k, v[i].z * k, v[i].w * k};
    }
}

template <int W, int R>
__global__ __launch_bounds__(W == 1 ? 256 : 64 * W) void rmsnorm_reg(const float *__restrict__ x,
                                                                    const float *__restrict__ g, float eps,
                                                                    float *__restrict__ y, int64_t rows,
                                                                    int64_t hidden) {
    __shared__ float red[W];
    constexpr int T = 64 * W;
    const int64_t row = W == 1 ? (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6) : (int64_t)blockIdx.x;
    const int t = threadIdx.x % T;
    const int64_t r = row < rows ? row : rows - 1;
    const float4 *xr = (const float4 *)(x + r * hidden);
    const float4 *g4 = (const float4 *)g;
    const int n4 = (int)(hidden / 4);
    float4 v[R], w[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int j = min(t + T * i, n4 - 1);
        v[i] = xr[j];
        w[i] = g4[j];
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < R; ++i)
        if (t + T * i < n4) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    ss = block_sum<W>(ss, red);
    if (row >= rows) return;
    // Tensor.rmsNormCPU: invRMS = 1 / sqrt(ss / hidden + eps); x * invRMS * w
    const float inv = 1.0f / sqrtf(ss / (float)hidden + eps);
    float4 *yr = (float4 *)(y + r * hidden);
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int j = t + T * i;
        if (j < n4)
            yr[j] = float4{v[i].x * inv * w[i].x, v[i].y * inv * w[i].y, v[i].z * inv * w[i].z, v[i].w * inv * w[i].w};
    }
}

// Launches the register-resident form when the row fits (returns false
// otherwise): W from {1, 4, 16} threads-per-row waves, R float4 per thread.
template <class K1, class K4, class K16>
bool launch_reg_rows(int64_t rows, int64_t cols, hipStream_t s, K1 k1, K4 k4, K16 k16) {
    const int64_t n4 = cols / 4;
    auto rpt = [](int64_t n, int t) { const int64_t r = (n + t - 1) / t; return r <= 1 ? 1 : r <= 2 ? 2 : r <= 4 ? 4 : 8; };
    if (n4 <= 64 * 4) k1(rpt(n4, 64), dim3((unsigned)((rows + 3) / 4)), dim3(256), s);
    else if (n4 <= 256 * 8) k4(rpt(n4, 256), dim3((unsigned)rows), dim3(256), s);
    else if (n4 <= 1024 * 8) k16(rpt(n4, 1024), dim3((unsigned)rows), dim3(1024), s);
    else return false;
    return true;
}

#define TBH_REG_LAUNCHER(NAME, KERNEL, W, ...)                                                     \
    auto NAME = [&](int R, dim3 grid, dim3 block, hipStream_t st) {                                \
        switch (R) {                                                                               \
        case 1: hipLaunchKernelGGL((KERNEL<W, 1>), grid, block, 0, st, __VA_ARGS__); break;        \
        case 2: hipLaunchKernelGGL((KERNEL<W, 2>), grid, block, 0, st, __VA_ARGS__); break;        \
        case 4: hipLaunchKernelGGL((KERNEL<W, 4>), grid, block, 0, st, __VA_ARGS__); break;        \
        default: hipLaunchKernelGGL((KERNEL<W, 8>), grid, block, 0, st, __VA_ARGS__); break;       \
        }                                                                                          \
    }

enum Act { ACT_SILU = 0, ACT_GELU = 1 };

template <int A>
__device__ __forceinline__ float act(float x, float s2p) {
    if (A == ACT_SILU) return x / (1.0f + expf(-x));
    const float x3 = x * x * x;
    const float inner = s2p * (x + 0.044715f * x3);
    return 0.5f * x * (1.0f + tanhf(inner));
}

// Elementwise.  Vector form: each thread takes UN 16-byte pieces per pass,
// their loads issued before any compute (us per call on 2048 x 5632, UN / grid
// cap in blocks per CU: SiLU 1 / 8 19.1, 2 / 16 18.6, 4 / 8 20.0; GELU 19.6,
// 18.6, 19.9).
template <int A, bool VEC, int UN>
__global__ __launch_bounds__(256) void activation(const float *__restrict__ x, float *__restrict__ y, int64_t n,
                                                  float s2p) {
    if (VEC) {
        const int64_t n4 = n / 4;
        const int64_t stride = (int64_t)gridDim.x * 256 * UN;
        for (int64_t i = (int64_t)blockIdx.x * 256 * UN + threadIdx.x; i < n4; i += stride) {
            float4 v[UN];
#pragma unroll
            for (int j = 0; j < UN; ++j) {
                const int64_t e = i + 256 * j;
                v[j] = ((const float4 *)x)[e < n4 ? e : i];   // past the end: re-read a valid piece
            }
#pragma unroll
            for (int j = 0; j < UN; ++j) {
                const int64_t e = i + 256 * j;
                if (e < n4)
                    ((float4 *)y)[e] = float4{act<A>(v[j].x, s2p), act<A>(v[j].y, s2p), act<A>(v[j].z, s2p),
                                              act<A>(v[j].w, s2p)};
            }
        }
        const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
        if (t < n - n4 * 4) y[n4 * 4 + t] = act<A>(x[n4 * 4 + t], s2p);
    } else {
        const int64_t stride = (int64_t)gridDim.x * 256;
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) y[i] = act<A>(x[i], s2p);
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
            const float pj = wave::lane_value(p, j);
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

constexpr int kGrpHeads = 8;   // query heads one block serves
constexpr int kPass = 256;     // positions scored per pass, one per thread
constexpr int kRedPad = 4 * kGrpHeads + 1;

struct GrpArgs {
    AttnArgs a;
    int32_t rep;       // query heads per key/value head
    int32_t hchunks;   // ceil(rep / kGrpHeads)
    int32_t splits;    // blocks per group along the key positions
    int64_t chunk;     // positions per split
    int64_t units;     // batch * seq_len * nkv * hchunks
    float *part;       // splits > 1: [units * splits][2 * kGrpHeads + kGrpHeads * hd]
};

__global__ __launch_bounds__(256) void attention_group(const GrpArgs g) {
    const AttnArgs &a = g.a;
    __shared__ __attribute__((aligned(16))) float qs[kGrpHeads][kAttnMaxHeadDim];
    __shared__ float ps[kGrpHeads][kPass];
    __shared__ float redm[4][kGrpHeads], reds[4][kGrpHeads];
    __shared__ float red_o[256 * kRedPad];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t unit = blockIdx.x / g.splits;
    const int split = (int)(blockIdx.x % g.splits);
    const int hc = (int)(unit % g.hchunks);
    const int64_t grp = unit / g.hchunks;                 // (batch * seq_len + query) * nkv + kvh
    const int kvh = (int)(grp % a.nkv);
    const int64_t bq = grp / a.nkv;
    const int64_t b = bq / a.seq_len;
    const int nhb = min(kGrpHeads, g.rep - hc * kGrpHeads);
    const int head0 = kvh * g.rep + hc * kGrpHeads;
    const int hd = a.hd, hd4 = hd / 4;
    const int64_t kvd = (int64_t)a.nkv * hd;
    const float *kb = a.k + b * a.kv_len * kvd + (int64_t)kvh * hd;
    const float *vb = a.v + b * a.kv_len * kvd + (int64_t)kvh * hd;
    const float *qb = a.q + bq * a.nh * hd + (int64_t)head0 * hd;
    for (int o = tid; o < kGrpHeads * hd; o += 256) {
        const int h = o / hd;
        qs[h][o % hd] = h < nhb ? qb[o] : 0.0f;
    }
    const int64_t c0 = split * g.chunk, c1 = min(a.kv_len, c0 + g.chunk);
    // value phase mapping: lane = pp * lpr + d4
    const int lpr = hd4, ppi = 64 / lpr;
    const int pp = lane / lpr, d4 = lane % lpr;
    const bool vlane = pp < ppi;

    float m[kGrpHeads], l[kGrpHeads];
    float4 acc[kGrpHeads];
#pragma unroll
    for (int h = 0; h < kGrpHeads; ++h) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
        acc[h] = float4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    for (int64_t p0 = c0; p0 < c1; p0 += kPass) {
        // ---- scores of position p0 + tid for every head of the group
        const int64_t t = p0 + tid;
        const bool valid = t < c1;
        float sc[kGrpHeads];
#pragma unroll
        for (int h = 0; h < kGrpHeads; ++h) sc[h] = 0.0f;
        if (valid) {
            const float4 *kr = (const float4 *)(kb + t * kvd);
#pragma unroll 4
            for (int i = 0; i < hd4; ++i) {
                const float4 kv = kr[i];
#pragma unroll
                for (int h = 0; h < kGrpHeads; ++h) {
                    const float4 qv = *(const float4 *)&qs[h][4 * i];
                    sc[h] += qv.x * kv.x + qv.y * kv.y + qv.z * kv.z + qv.w * kv.w;
                }
            }
        }
        const float mk = (valid && a.mask) ? a.mask[t] : 0.0f;
#pragma unroll
        for (int h = 0; h < kGrpHeads; ++h) {
            sc[h] = valid ? sc[h] * a.scale + mk : -INFINITY;
            const float wm = wave_max(sc[h]);
            if (lane == 0) redm[wave][h] = wm;
        }
        __syncthreads();
        float corr[kGrpHeads];
#pragma unroll
        for (int h = 0; h < kGrpHeads; ++h) {
            const float pm = fmaxf(fmaxf(redm[0][h], redm[1][h]), fmaxf(redm[2][h], redm[3][h]));
            const float nm = fmaxf(m[h], pm);
            corr[h] = nm == -INFINITY ? 1.0f : expf(m[h] - nm);
            const float pv = nm == -INFINITY ? 0.0f : expf(sc[h] - nm);
            ps[h][tid] = pv;
            const float ws = wave_sum(pv);
            if (lane == 0) reds[wave][h] = ws;
            m[h] = nm;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < kGrpHeads; ++h) {
            l[h] = l[h] * corr[h] + ((reds[0][h] + reds[1][h]) + (reds[2][h] + reds[3][h]));
            acc[h].x *= corr[h];
            acc[h].y *= corr[h];
            acc[h].z *= corr[h];
            acc[h].w *= corr[h];
        }
        // ---- p * v over this wave's 64 positions of the pass
        if (vlane) {
#pragma unroll 4
            for (int r = pp; r < 64; r += ppi) {
                const int tp = wave * 64 + r;
                if (p0 + tp >= c1) break;
                const float4 v = *(const float4 *)(vb + (p0 + tp) * kvd + 4 * d4);
#pragma unroll
                for (int h = 0; h < kGrpHeads; ++h) {
                    const float pr = ps[h][tp];
                    acc[h].x += pr * v.x;
                    acc[h].y += pr * v.y;
                    acc[h].z += pr * v.z;
                    acc[h].w += pr * v.w;
                }
            }
        }
        __syncthreads();   // ps and redm are rewritten by the next pass
    }

    // ---- sum the value accumulators over lanes and waves
#pragma unroll
    for (int h = 0; h < kGrpHeads; ++h) {
        red_o[tid * kRedPad + 4 * h + 0] = vlane ? acc[h].x : 0.0f;
        red_o[tid * kRedPad + 4 * h + 1] = vlane ? acc[h].y : 0.0f;
        red_o[tid * kRedPad + 4 * h + 2] = vlane ? acc[h].z : 0.0f;
        red_o[tid * kRedPad + 4 * h + 3] = vlane ? acc[h].w : 0.0f;
    }
    __syncthreads();
    float *part = g.splits > 1 ? g.part + (unit * g.splits + split) * (2 * kGrpHeads + kGrpHeads * hd) : nullptr;
    if (part && tid < kGrpHeads) {
        // m and l are uniform over the block; thread h stores head h's pair
#pragma unroll
        for (int h = 0; h < kGrpHeads; ++h)
            if (h == tid) {
                part[h] = m[h];
                part[kGrpHeads + h] = l[h];
            }
    }
    for (int o = tid; o < nhb * hd; o += 256) {
        const int h = o / hd, d = o % hd;
        float v = 0.0f;
        for (int w = 0; w < 4; ++w)
            for (int q = 0; q < ppi; ++q) v += red_o[(w * 64 + q * lpr + d / 4) * kRedPad + 4 * h + d % 4];
        float mh = 0.0f, lh = 0.0f;
#pragma unroll
        for (int hh = 0; hh < kGrpHeads; ++hh)
            if (hh == h) {
                mh = m[hh];
                lh = l[hh];
            }
        if (part) {
            part[2 * kGrpHeads + h * hd + d] = v;
        } else {
            float *orow = a.out + bq * a.nh * hd + (int64_t)(head0 + h) * hd;
            orow[d] = (mh == -INFINITY && a.kv_len > 0) ? NAN : v / (lh + kAttnEps);
        }
    }
}

// Orders a wave's LDS writes before later LDS reads by other lanes of the
// same wave (the waves of attention_wave never wait for each other).
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Attention for head_dim HD in {16, 32, 64, 128}: one wave per (query row,
// query head, range of key positions); a block's four waves are four query
// heads of one key/value head, so they share the range's key and value rows
// through L1, and no wave waits for another.  A pass covers 64 positions.
// Lane (pg, d4) loads 16-byte piece d4 of key and value rows pg, pg + PPI,
// ... (PPI = 64 / (HD / 4) rows per load instruction, so every load reads
// whole row segments); its partial dot products with q piece d4 are summed
// over the row's HD / 4 lanes by a DPP transpose-sum, after which the lane
// holds the score of position pg + PPI * d4.  Max and sum by DPP, p * v
// over the value pieces.  The wave keeps an online softmax across passes;
// with one split it writes the output, else its range's (max, sum, p.v)
// partial for attention_combine.
template <int HD>
__global__ __launch_bounds__(256) void attention_wave(const GrpArgs g) {
    constexpr int HD4 = HD / 4, PPI = 64 / HD4, NV = HD4;
    const AttnArgs &a = g.a;
    __shared__ float ps[4][64];
    __shared__ float4 red[4][64];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nquad = (g.rep + 3) / 4;
    int64_t bi = blockIdx.x;
    const int split = (int)(bi % g.splits);
    bi /= g.splits;
    const int quad = (int)(bi % nquad);
    bi /= nquad;
    const int kvh = (int)(bi % a.nkv);
    const int64_t bq = bi / a.nkv;                // batch * seq_len + query
    const int hg = quad * 4 + w;
    if (hg >= g.rep) return;
    const int head = kvh * g.rep + hg;
    const int64_t batch = bq / a.seq_len;
    const int64_t kvd = (int64_t)a.nkv * HD;
    const float *kb = a.k + batch * a.kv_len * kvd + (int64_t)kvh * HD;
    const float *vb = a.v + batch * a.kv_len * kvd + (int64_t)kvh * HD;
    const int64_t c0 = split * g.chunk, c1 = min(a.kv_len, c0 + g.chunk);
    const int pg = lane / HD4, d4 = lane % HD4;
    const float *qrow = a.q + (bq * a.nh + head) * HD + 4 * d4;
    const float4 q4 = float4{qrow[0], qrow[1], qrow[2], qrow[3]};   // q rows need not be 16-byte aligned

    float m = -INFINITY, l = 0.0f;
    float4 acc = float4{0.f, 0.f, 0.f, 0.f};
    for (int64_t p0 = c0; p0 < c1; p0 += 64) {
        const int64_t last = c1 - 1;
        float4 kreg[HD4], vreg[NV];
#pragma unroll
        for (int j = 0; j < HD4; ++j)
            kreg[j] = *(const float4 *)(kb + min(p0 + pg + j * PPI, last) * kvd + 4 * d4);
#pragma unroll
        for (int j = 0; j < NV; ++j)
            vreg[j] = *(const float4 *)(vb + min(p0 + pg + j * PPI, last) * kvd + 4 * d4);
        const int64_t t = p0 + pg + PPI * d4;     // this lane's position after the transpose-sum
        const bool tv = t < c1;
        const float mk = a.mask ? a.mask[min(t, last)] : 0.0f;
        float part[HD4];
#pragma unroll
        for (int j = 0; j < HD4; ++j)
            part[j] = q4.x * kreg[j].x + q4.y * kreg[j].y + q4.z * kreg[j].z + q4.w * kreg[j].w;
        const float d = wave::transpose_sum<HD4>(part, lane);
        const float sc = tv ? d * a.scale + mk : -INFINITY;
        const float nm = fmaxf(m, wave_max(sc));
        if (nm == -INFINITY) continue;            // every position so far masked (uniform)
        const float corr = expf(m - nm);
        const float p = expf(sc - nm);
        l = l * corr + wave_sum(p);
        ps[w][pg + PPI * d4] = p;
        wave_lds_fence();
        acc.x *= corr;
        acc.y *= corr;
        acc.z *= corr;
        acc.w *= corr;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const float pr = ps[w][pg + j * PPI];   // 0 past the range
            acc.x += pr * vreg[j].x;
            acc.y += pr * vreg[j].y;
            acc.z += pr * vreg[j].z;
            acc.w += pr * vreg[j].w;
        }
        m = nm;
        wave_lds_fence();                         // ps is rewritten by the next pass
    }
    red[w][lane] = acc;
    wave_lds_fence();
    if (lane < HD4) {
        float4 o = red[w][lane];
#pragma unroll
        for (int q = 1; q < PPI; ++q) {
            const float4 v = red[w][q * HD4 + lane];
            o.x += v.x;
            o.y += v.y;
            o.z += v.z;
            o.w += v.w;
        }
        if (g.splits == 1) {
            // no positions (kv_len 0) leaves zeros; all masked gives NaN
            const bool dead = m == -INFINITY && a.kv_len > 0;
            const float den = l + kAttnEps;
            float *orow = a.out + (bq * a.nh + head) * HD + 4 * lane;
            *(float4 *)orow = dead ? float4{NAN, NAN, NAN, NAN} : float4{o.x / den, o.y / den, o.z / den, o.w / den};
        } else {
            const int64_t unit = (bq * a.nkv + kvh) * g.hchunks + hg / kGrpHeads;
            const int hs = hg % kGrpHeads;
            float *part = g.part + (unit * g.splits + split) * (2 * kGrpHeads + kGrpHeads * HD);
            if (lane == 0) {
                part[hs] = m;
                part[kGrpHeads + hs] = l;
            }
            *(float4 *)&part[2 * kGrpHeads + hs * HD + 4 * lane] = o;
        }
    }
}

// Merges the split partials of attention_group / attention_wave: per head,
// M = max m_s, out = sum(o_s e^(m_s - M)) / (sum(l_s e^(m_s - M)) + eps).
// One block per (unit, head); thread (sg, d4) loads the partials of splits
// sg, sg + 256 / (hd / 4), ... (kCombineLoads of them) in one memory trip
// (more splits than that take further trips).
constexpr int kCombineLoads = 4;

__global__ __launch_bounds__(256) void attention_combine(const GrpArgs g) {
    const AttnArgs &a = g.a;
    __shared__ float4 red[256];
    __shared__ float rs[8];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, hd = a.hd, hd4 = hd / 4;
    const int64_t unit = blockIdx.x / kGrpHeads;
    const int h = (int)(blockIdx.x % kGrpHeads);
    const int hc = (int)(unit % g.hchunks);
    if (h >= g.rep - hc * kGrpHeads) return;   // uniform over the block
    const int64_t grp = unit / g.hchunks;
    const int kvh = (int)(grp % a.nkv);
    const int64_t bq = grp / a.nkv;
    const int64_t stride = 2 * kGrpHeads + (int64_t)kGrpHeads * hd;
    const float *pb = g.part + unit * g.splits * stride;
    const int sg = tid / hd4, d4 = tid % hd4, nsg = 256 / hd4;
    const bool slane = sg < nsg;
    float mv[kCombineLoads], lv[kCombineLoads];
    float4 ov[kCombineLoads];
#pragma unroll
    for (int j = 0; j < kCombineLoads; ++j) {
        const int sp = min(sg + nsg * j, g.splits - 1);
        mv[j] = pb[sp * stride + h];
        lv[j] = pb[sp * stride + kGrpHeads + h];
        ov[j] = *(const float4 *)(pb + sp * stride + 2 * kGrpHeads + h * hd + 4 * d4);
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int j = 0; j < kCombineLoads; ++j)
        if (slane && sg + nsg * j < g.splits) mloc = fmaxf(mloc, mv[j]);
    for (int sp = sg + nsg * kCombineLoads; slane && sp < g.splits; sp += nsg) mloc = fmaxf(mloc, pb[sp * stride + h]);
    mloc = wave_max(mloc);
    if (lane == 0) rs[wv] = mloc;
    __syncthreads();
    const float M = fmaxf(fmaxf(rs[0], rs[1]), fmaxf(rs[2], rs[3]));
    float L = 0.0f;
    float4 o = float4{0.f, 0.f, 0.f, 0.f};
    if (M != -INFINITY) {
        auto add = [&](float m, float l, float4 v) {
            const float e = expf(m - M);
            if (d4 == 0) L += e * l;   // one thread per split counts its sum
            o.x += e * v.x;
            o.y += e * v.y;
            o.z += e * v.z;
            o.w += e * v.w;
        };
#pragma unroll
        for (int j = 0; j < kCombineLoads; ++j)
            if (slane && sg + nsg * j < g.splits) add(mv[j], lv[j], ov[j]);
        for (int sp = sg + nsg * kCombineLoads; slane && sp < g.splits; sp += nsg)
            add(pb[sp * stride + h], pb[sp * stride + kGrpHeads + h],
                *(const float4 *)(pb + sp * stride + 2 * kGrpHeads + h * hd + 4 * d4));
    }
    L = wave_sum(L);
    if (lane == 0) rs[4 + wv] = L;
    red[tid] = o;
    __syncthreads();
    if (tid < hd4) {
        float4 r = float4{0.f, 0.f, 0.f, 0.f};
        for (int q = 0; q < nsg; ++q) {
            const float4 v = red[q * hd4 + tid];
            r.x += v.x;
            r.y += v.y;
            r.z += v.z;
            r.w += v.w;
        }
        const float den = ((rs[4] + rs[5]) + (rs[6] + rs[7])) + kAttnEps;
        const int head = kvh * g.rep + hc * kGrpHeads + h;
        float4 *orow = (float4 *)(a.out + (bq * a.nh + head) * hd) + tid;
        *orow = M == -INFINITY ? float4{NAN, NAN, NAN, NAN} : float4{r.x / den, r.y / den, r.z / den, r.w / den};
    }
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

unsigned grid_for(int64_t blocks, const tbh_device *dev) {
    const int64_t cap = 8 * (int64_t)std::max(1, dev->cu_count);
    return (unsigned)std::max<int64_t>(1, std::min(blocks, cap));
}

hipError_t launch_softmax(const float *x, int64_t rows, int64_t cols, float *y, hipStream_t s) {
    const bool vec = cols % 4 == 0 && aligned16(x) && aligned16(y);
    if (vec) {
        TBH_REG_LAUNCHER(k1, softmax_reg, 1, x, y, rows, cols);
        TBH_REG_LAUNCHER(k4, softmax_reg, 4, x, y, rows, cols);
        TBH_REG_LAUNCHER(k16, softmax_reg, 16, x, y, rows, cols);
        if (launch_reg_rows(rows, cols, s, k1, k4, k16)) return hipGetLastError();
    }
    if (cols <= kWaveRowMax) {
        const dim3 grid((unsigned)((rows + 3) / 4));
        if (vec) hipLaunchKernelGGL((softmax_rows<1, true>), grid, dim3(256), 0, s, x, y, rows, cols);
        else hipLaunchKernelGGL((softmax_rows<1, false>), grid, dim3(256), 0, s, x, y, rows, cols);
    } else {
        const dim3 grid((unsigned)rows);
        if (vec) hipLaunchKernelGGL((softmax_rows<16, true>), grid, dim3(1024), 0, s, x, y, rows, cols);
        else hipLaunchKernelGGL((softmax_rows<16, false>), grid, dim3(1024), 0, s, x, y, rows, cols);
    }
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, int64_t rows, int64_t hidden, const float *g, float eps, float *y,
                          hipStream_t s) {
    const bool vec = hidden % 4 == 0 && aligned16(x) && aligned16(y) && aligned16(g);
    if (vec) {
        TBH_REG_LAUNCHER(k1, rmsnorm_reg, 1, x, g, eps, y, rows, hidden);
        TBH_REG_LAUNCHER(k4, rmsnorm_reg, 4, x, g, eps, y, rows, hidden);
        TBH_REG_LAUNCHER(k16, rmsnorm_reg, 16, x, g, eps, y, rows, hidden);
        if (launch_reg_rows(rows, hidden, s, k1, k4, k16)) return hipGetLastError();
    }
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
    constexpr int UN = 2;
    const int64_t cus = std::max(1, dev->cu_count);
    const unsigned grid = vec ? (unsigned)std::max<int64_t>(1, std::min((n / 4 + 256 * UN - 1) / (256 * UN), 16 * cus))
                              : grid_for((n + 255) / 256, dev);
    if (vec) {
        hipLaunchKernelGGL((activation<A, true, UN>), dim3(grid), dim3(256), 0, s, x, y, n, gelu_s2p());
    } else {
        hipLaunchKernelGGL((activation<A, false, 1>), dim3(grid), dim3(256), 0, s, x, y, n, gelu_s2p());
    }
    return hipGetLastError();
}

hipError_t launch_attention_rows(const AttnArgs &a, hipStream_t s);

hipError_t launch_attention(tbh_device *dev, const AttnArgs &a, hipStream_t s) {
    if (a.hd % 4 != 0 || !aligned16(a.k) || !aligned16(a.v) || !aligned16(a.out)) return launch_attention_rows(a, s);
    GrpArgs g{};
    g.a = a;
    g.rep = a.nh / a.nkv;
    g.hchunks = (g.rep + kGrpHeads - 1) / kGrpHeads;
    g.units = (a.rows / a.nh) * a.nkv * g.hchunks;
    g.splits = 1;
    g.chunk = std::max<int64_t>(a.kv_len, 1);
    const bool wave = a.hd == 16 || a.hd == 32 || a.hd == 64 || a.hd == 128;
    // blocks per split: (query row, KV head, 4 query heads) for attention_wave,
    // (query row, KV head, 8 query heads) for attention_group
    const int64_t per_split = wave ? (a.rows / a.nh) * a.nkv * ((g.rep + 3) / 4) : g.units;
    const int64_t target = 2 * (int64_t)std::max(1, dev->cu_count);
    if (per_split < target && a.kv_len > 64) {
        const int64_t want =
            std::min<int64_t>(std::min((target + per_split - 1) / per_split, (a.kv_len + 63) / 64), 1024);
        g.chunk = ((a.kv_len + want - 1) / want + 63) / 64 * 64;
        g.splits = (int32_t)((a.kv_len + g.chunk - 1) / g.chunk);
    }
    if (g.splits > 1) {
        const size_t bytes = (size_t)(g.units * g.splits * (2 * kGrpHeads + kGrpHeads * a.hd)) * sizeof(float);
        g.part = (float *)stream_workspace(dev, s, bytes);
        if (!g.part) {   // no workspace (graph capture before any eager call): one split
            g.splits = 1;
            g.chunk = std::max<int64_t>(a.kv_len, 1);
        }
    }
    if (per_split * g.splits > INT32_MAX) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(per_split * g.splits));
    switch (a.hd) {
    case 16: hipLaunchKernelGGL(attention_wave<16>, grid, dim3(256), 0, s, g); break;
    case 32: hipLaunchKernelGGL(attention_wave<32>, grid, dim3(256), 0, s, g); break;
    case 64: hipLaunchKernelGGL(attention_wave<64>, grid, dim3(256), 0, s, g); break;
    case 128: hipLaunchKernelGGL(attention_wave<128>, grid, dim3(256), 0, s, g); break;
    default: hipLaunchKernelGGL(attention_group, grid, dim3(256), 0, s, g); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || g.splits == 1) return e;
    hipLaunchKernelGGL(attention_combine, dim3((unsigned)(g.units * kGrpHeads)), dim3(256), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_attention_rows(const AttnArgs &a, hipStream_t s) {
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
    (void)hipFree(dev->stage);   // replaced below; a failed free leaves nothing to undo
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
    hipError_t e = launch_attention(dev, a, (hipStream_t)stream);
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
                         return launch_attention(dev, a, s);
                     });
}

}  // extern "C"

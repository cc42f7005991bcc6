// tbh_ref_kernels.hip -- exact-decode kernels:
//   * generic_int4: matmul straight from the reference's flat INT4 array for
//     groupings no repacked layout describes (slow path, any shape);
//   * dequant_*: writes dequantize() of an uploaded weight in [K, N] order,
//     one fp32 rounding per element, for bit-exact verification.
// The element rule is QuantizedTensor.dequantize()
// (Sources/TinyBrainRuntime/QuantizedTensor.swift:186-216, :241-255):
//   value = (Float(q) - Float(zp)) * scale.
#include "tbh_internal.h"

namespace tbh {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Flat INT4 decode of element i: byte i/2, even i in the high nibble,
// raw > 7 => raw - 16 (QuantizedTensor.swift:201-213).
__device__ __forceinline__ int int4_at(const int8_t *raw, int64_t i) {
    unsigned b = (uint8_t)raw[i >> 1];
    unsigned nib = (i & 1) == 0 ? (b >> 4) & 0xFu : b & 0xFu;
    return nib > 7u ? (int)nib - 16 : (int)nib;
}

struct GenericParams {
    const float *x;
    int64_t ldx;
    float *y;
    int64_t ldy;
    int64_t M, K, N, gs;
    int32_t layout;
    const int8_t *raw;
    const float *scales;
    const int8_t *zp;
};

// One wave per output column n; lanes stride over K.
__global__ __launch_bounds__(256) void generic_int4(const GenericParams p) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t n = (int64_t)blockIdx.x * 4 + wave;
    if (n >= p.N) return;
    for (int64_t m = 0; m < p.M; ++m) {
        float acc = 0.0f;
        for (int64_t k = lane; k < p.K; k += 64) {
            const int64_t i = p.layout == TBH_LAYOUT_KN_FLAT ? k * p.N + n : n * p.K + k;
            const int64_t g = i / p.gs;
            const float z = p.zp ? (float)p.zp[g] : 0.0f;
            const float v = __fmul_rn((float)int4_at(p.raw, i) - z, p.scales[g]);
            acc = __builtin_fmaf(p.x[m * p.ldx + k], v, acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) p.y[m * p.ldy + n] = acc;
    }
}

struct DequantParams {
    float *out;
    int64_t K, N;
    int64_t Kp, row_bytes;
    const uint8_t *data;
    const float *scales;
    const int8_t *zp;
    int64_t G;
    int32_t cpg, rpn;
    // generic
    int64_t gs;
    int32_t layout;
    const int8_t *raw;
};

// INT8 repacked row: element k at byte (k & ~3) + {0, 2, 1, 3}[k & 3],
// value q + 128.
__global__ void dequant_int8_row(const DequantParams p) {
    const int64_t total = p.K * p.N;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t k = idx / p.N, n = idx - k * p.N;
        const int j = (int)(k & 3);
        const int bp = j == 1 ? 2 : (j == 2 ? 1 : j);
        const int q = (int)p.data[n * p.row_bytes + (k & ~int64_t(3)) + bp] - 128;
        const int z = p.zp ? (int)p.zp[n] : 0;
        p.out[idx] = __fmul_rn((float)q - (float)z, p.scales[n]);
    }
}

// INT4 repacked row: element k in 32-bit word k/8 at bit offset
// {0, 16, 4, 20, 8, 24, 12, 28}[k % 8], value q + 8.
__device__ __forceinline__ int int4_repacked(const uint8_t *row, int64_t k) {
    const uint32_t word = ((const uint32_t *)row)[k >> 3];
    const int j = (int)(k & 7);
    const int shift = ((j & 1) << 4) | ((j >> 1) << 2);
    return (int)((word >> shift) & 0xFu) - 8;
}

__global__ void dequant_int4_kgroup(const DequantParams p) {
    const int64_t total = p.K * p.N;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t k = idx / p.N, n = idx - k * p.N;
        const int q = int4_repacked(p.data + n * p.row_bytes, k);
        const int64_t gi = kgroup_index(n, (k / kInt4ChunkElems) / p.cpg, p.G);
        const int z = p.zp ? (int)p.zp[gi] : 0;
        p.out[idx] = __fmul_rn((float)q - (float)z, p.scales[gi]);
    }
}

__global__ void dequant_int4_ngroup(const DequantParams p) {
    const int64_t total = p.K * p.N;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t k = idx / p.N, n = idx - k * p.N;
        const int q = int4_repacked(p.data + n * p.row_bytes, k);
        p.out[idx] = __fmul_rn((float)q, p.scales[(n / p.rpn) * p.Kp + k]);
    }
}

// INT8 MFMA tiles: element (k, n) is in tile (n / 16, k / 64), lane
// n % 16 + 16 * ((k % 32) / 8), word 2 * ((k % 64) / 32) + (k % 8) / 4, byte
// position {0, 2, 1, 3}[k % 4]; value q + 128.
__global__ void dequant_int8_tiles(const DequantParams p) {
    const int64_t total = p.K * p.N;
    const int64_t SC = p.Kp / kMfmaInt8TileK;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t k = idx / p.N, n = idx - k * p.N;
        const int l = (int)(n % 16) + 16 * (int)((k % 32) / 8);
        const int word = 2 * (int)((k % 64) / 32) + (int)((k % 8) / 4);
        const int j = (int)(k & 3);
        const int bp = j == 1 ? 2 : (j == 2 ? 1 : j);
        const int64_t off = ((n / 16) * SC + k / 64) * 1024 + 16 * l + 4 * word + bp;
        const int q = (int)p.data[off] - 128;
        const int z = p.zp ? (int)p.zp[n] : 0;
        p.out[idx] = __fmul_rn((float)q - (float)z, p.scales[n]);
    }
}

// INT4 MFMA tiles: element (k, n) is in tile (n / 16, k / 128), lane
// n % 16 + 16 * ((k % 32) / 8), word (k % 128) / 32, nibble at bit offset
// {0, 16, 4, 20, 8, 24, 12, 28}[k % 8]; value q + 8.  Scales are per row
// (G == 1) or per (row, 32-element chunk) in tile order.
__global__ void dequant_int4_tiles(const DequantParams p) {
    const int64_t total = p.K * p.N;
    const int64_t SC = p.Kp / kMfmaInt4TileK;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t k = idx / p.N, n = idx - k * p.N;
        const int l = (int)(n % 16) + 16 * (int)((k % 32) / 8);
        const int word = (int)((k % 128) / 32);
        const int64_t tile = (n / 16) * SC + k / 128;
        const uint32_t w = ((const uint32_t *)(p.data + tile * 1024))[4 * l + word];
        const int e = (int)(k & 7);
        const int shift = ((e & 1) << 4) | ((e >> 1) << 2);
        const int q = (int)((w >> shift) & 0xFu) - 8;
        const int64_t si = p.G == 1 ? n : (tile * 16 + n % 16) * 4 + word;
        const int z = p.zp ? (int)p.zp[si] : 0;
        p.out[idx] = __fmul_rn((float)q - (float)z, p.scales[si]);
    }
}

__global__ void dequant_int4_generic(const DequantParams p) {
    const int64_t total = p.K * p.N;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t k = idx / p.N, n = idx - k * p.N;
        const int64_t i = p.layout == TBH_LAYOUT_KN_FLAT ? idx : n * p.K + k;
        const int64_t g = i / p.gs;
        const float z = p.zp ? (float)p.zp[g] : 0.0f;
        p.out[idx] = __fmul_rn((float)int4_at(p.raw, i) - z, p.scales[g]);
    }
}

}  // namespace

hipError_t launch_generic(const tbh_weight &w, const GemvArgs &a, hipStream_t s) {
    if (w.path != Path::Generic) return hipErrorInvalidValue;
    GenericParams p{};
    p.x = a.x;
    p.ldx = a.ldx;
    p.y = a.y;
    p.ldy = a.ldy;
    p.M = a.M;
    p.K = w.K;
    p.N = w.N;
    p.gs = w.group_size > 0 ? w.group_size : w.K * w.N;
    p.layout = w.layout;
    p.raw = w.raw;
    p.scales = w.raw_scales;
    p.zp = w.raw_zp;
    const int64_t blocks = (w.N + 3) / 4;
    hipLaunchKernelGGL(generic_int4, dim3((unsigned)blocks), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_dequant(const tbh_weight &w, float *out, hipStream_t s) {
    if (w.ng_pairs) return hipErrorInvalidValue;   // decoder-internal interleaved weights
    DequantParams p{};
    p.out = out;
    p.K = w.K;
    p.N = w.N;
    p.Kp = w.Kp;
    p.row_bytes = w.row_bytes;
    p.data = w.data;
    p.scales = w.path == Path::Generic ? w.raw_scales : w.scales;
    p.zp = w.path == Path::Generic ? w.raw_zp : w.zp;
    p.G = w.groups_per_row;
    p.cpg = w.chunks_per_group;
    p.rpn = w.rows_per_nblock;
    p.gs = w.group_size > 0 ? w.group_size : w.K * w.N;
    p.layout = w.layout;
    p.raw = w.raw;
    const int64_t total = w.K * w.N;
    const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
    if (w.mfma_tiles) {
        if (w.precision == TBH_PREC_INT8)
            hipLaunchKernelGGL(dequant_int8_tiles, dim3(blocks), dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL(dequant_int4_tiles, dim3(blocks), dim3(256), 0, s, p);
        return hipGetLastError();
    }
    switch (w.path) {
    case Path::Int8Row: hipLaunchKernelGGL(dequant_int8_row, dim3(blocks), dim3(256), 0, s, p); break;
    case Path::Int4KGroup: hipLaunchKernelGGL(dequant_int4_kgroup, dim3(blocks), dim3(256), 0, s, p); break;
    case Path::Int4NGroup: hipLaunchKernelGGL(dequant_int4_ngroup, dim3(blocks), dim3(256), 0, s, p); break;
    case Path::Generic: hipLaunchKernelGGL(dequant_int4_generic, dim3(blocks), dim3(256), 0, s, p); break;
    }
    return hipGetLastError();
}

}  // namespace tbh

// tbh_gemv.hip -- VALU dequant-GEMV for decode (M = 1..4 rows of x).
//
// Replaces the MSL kernels matmul_int8_dequant / matmul_int4_dequant
// (Sources/TinyBrainMetal/Shaders/Dequant.metal:49-79,
// DequantINT4.metal:95-137), which give each output one thread and walk K
// with a stride-N load.  Here one wave64 owns R output rows; each lane streams
// 16-byte chunks of those rows (K-contiguous after the one-time repack) with
// non-temporal 128-bit loads, so every load instruction moves 1 KiB of
// contiguous HBM.
//
// Unpack (per 32-bit word of packed weights, values stored offset-binary):
//   INT8: (w & 0x00FF00FF) | 0x64006400 is the f16 pair 1024 + (q+128);
//         the same on w >> 8 gives the other two bytes.
//   INT4: (w & 0x000F000F) | 0x64006400 is 1024 + (q+8) and
//         (w & 0x00F000F0) | 0x64006400 is 1024 + 16*(q+8); again on w >> 8.
// One v_pk_add_f16 per pair subtracts the offset (and the zero point), which
// leaves q - zp (or 16*(q - zp)) exactly in f16; v_fma_mix_f32 then multiplies
// that f16 by the fp32 x element and accumulates in fp32.  The x elements
// paired with the 16x nibbles are stored in LDS pre-divided by 16, so every
// product is exactly (q - zp) * x rounded once, as in an fp32 FMA.  Scales
// are applied once per row (INT8, per-channel), once per 32-element chunk
// (INT4 K-groups), or folded into x per K element (INT4 runtime layout).
#include "tbh_internal.h"

namespace tbh {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

enum { S_ROW = 0, S_KGROUP = 1, S_NGROUP = 2 };

struct KParams {
    const float *x;
    int64_t ldx;
    float *y;
    int64_t ldy;
    const uint8_t *data;
    int64_t row_bytes;
    const float *scales;
    const int8_t *zp;
    int32_t K, Kp, N, Np;
    int32_t chunks;  // chunks per row
    int32_t G;       // INT4 K-groups per row
    int32_t cpg;     // chunks per K-group
    int32_t rpn;     // rows per N-block (INT4 runtime layout)
};

__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t d;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(m), "v"(o));
    return d;
}

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }

__device__ __forceinline__ h2 splat(float v) {
    h2 r;
    r.x = (_Float16)v;
    r.y = (_Float16)v;
    return r;
}

__device__ __forceinline__ float fmix(_Float16 h, float x, float acc) {
    return __builtin_fmaf((float)h, x, acc);  // v_fma_mix_f32
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// LDS slot of x element k: chunks are padded by 4 floats so that the
// 128-bit reads of 8 consecutive lanes (one chunk each) cover all 32 banks.
template <int CE>
__device__ __forceinline__ int lds_index(int k) {
    return (k / CE) * (CE + 4) + (k % CE);
}

template <int PREC, int SM, int M, int R, bool ZP>
__global__ __launch_bounds__(256) void gemv_valu(const KParams p) {
    constexpr int CE = PREC == 8 ? 16 : 32;  // elements per 16-byte chunk
    constexpr int CS = CE + 4;               // padded LDS floats per chunk
    extern __shared__ float4 xs4[];  // float4-typed so that x reads are ds_read_b128
    float *xs = reinterpret_cast<float *>(xs4);
    const int tid = threadIdx.x;
    const int lds_row = p.chunks * CS;

    // stage x [M][Kp] into LDS (zero beyond K; INT4 16x slots pre-divided)
    for (int m = 0; m < M; ++m) {
        const float *xr = p.x + (int64_t)m * p.ldx;
        for (int k = tid; k < p.Kp; k += 256) {
            float v = k < p.K ? xr[k] : 0.0f;
            if (PREC == 4 && (k & 2)) v *= 0.0625f;
            xs[m * lds_row + lds_index<CE>(k)] = v;
        }
    }
    __syncthreads();

    const int wave = tid >> 6, lane = tid & 63;
    const int nrg = p.Np / R;
    const uint32_t kMagic = 0x64006400u;
    const uint32_t kLo = PREC == 8 ? 0x00FF00FFu : 0x000F000Fu;
    const uint32_t kHi = 0x00F000F0u;

    for (int rg = blockIdx.x * 4 + wave; rg < nrg; rg += gridDim.x * 4) {
        const int n0 = rg * R;
        float acc[M][R];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

        // per-row offset constants (INT8 row zero points)
        h2 c8[R];
        if (PREC == 8) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                c8[r] = splat(-(1152.0f + (ZP ? (float)p.zp[n0 + r] : 0.0f)));
        }
        const float *tcol = nullptr;  // INT4 runtime layout: per-k scales of this N-block
        if (SM == S_NGROUP) tcol = p.scales + (int64_t)(n0 / p.rpn) * p.Kp;

        for (int c = lane; c < p.chunks; c += 64) {
            u32x4 w[R];
#pragma unroll
            for (int r = 0; r < R; ++r)
                w[r] = __builtin_nontemporal_load(
                    (const u32x4 *)(p.data + (int64_t)(n0 + r) * p.row_bytes + (int64_t)c * 16));

            if (PREC == 8) {
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    float4 xv[M];
#pragma unroll
                    for (int m = 0; m < M; ++m)
                        xv[m] = xs4[(m * lds_row + c * CS + 4 * d) >> 2];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const uint32_t wv = w[r][d];
                        h2 p0 = as_h2(and_or(wv, kLo, kMagic)) + c8[r];
                        h2 p1 = as_h2(and_or(wv >> 8, kLo, kMagic)) + c8[r];
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            float t = acc[m][r];
                            t = fmix(p0.x, xv[m].x, t);
                            t = fmix(p0.y, xv[m].y, t);
                            t = fmix(p1.x, xv[m].z, t);
                            t = fmix(p1.y, xv[m].w, t);
                            acc[m][r] = t;
                        }
                    }
                }
            } else {
                h2 c1[R], c16[R];
                float s[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float z = 0.0f;
                    if (SM == S_KGROUP) {
                        const int64_t gi = (int64_t)(n0 + r) * p.G + c / p.cpg;
                        s[r] = p.scales[gi];
                        if (ZP) z = (float)p.zp[gi];
                    }
                    c1[r] = splat(-(1032.0f + z));
                    c16[r] = splat(-(1152.0f + 16.0f * z));
                }
                float part[M][R];
#pragma unroll
                for (int m = 0; m < M; ++m)
#pragma unroll
                    for (int r = 0; r < R; ++r) part[m][r] = 0.0f;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    float4 xa[M], xb[M];
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        xa[m] = xs4[(m * lds_row + c * CS + 8 * d) >> 2];
                        xb[m] = xs4[(m * lds_row + c * CS + 8 * d + 4) >> 2];
                    }
                    if (SM == S_NGROUP) {
                        const float4 ta = *(const float4 *)&tcol[c * 32 + 8 * d];
                        const float4 tb = *(const float4 *)&tcol[c * 32 + 8 * d + 4];
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            xa[m].x *= ta.x; xa[m].y *= ta.y; xa[m].z *= ta.z; xa[m].w *= ta.w;
                            xb[m].x *= tb.x; xb[m].y *= tb.y; xb[m].z *= tb.z; xb[m].w *= tb.w;
                        }
                    }
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const uint32_t wv = w[r][d];
                        const uint32_t w8 = wv >> 8;
                        h2 p0 = as_h2(and_or(wv, kLo, kMagic)) + c1[r];
                        h2 p1 = as_h2(and_or(wv, kHi, kMagic)) + c16[r];
                        h2 p2 = as_h2(and_or(w8, kLo, kMagic)) + c1[r];
                        h2 p3 = as_h2(and_or(w8, kHi, kMagic)) + c16[r];
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            float t = (SM == S_KGROUP) ? part[m][r] : acc[m][r];
                            t = fmix(p0.x, xa[m].x, t);
                            t = fmix(p0.y, xa[m].y, t);
                            t = fmix(p1.x, xa[m].z, t);
                            t = fmix(p1.y, xa[m].w, t);
                            t = fmix(p2.x, xb[m].x, t);
                            t = fmix(p2.y, xb[m].y, t);
                            t = fmix(p3.x, xb[m].z, t);
                            t = fmix(p3.y, xb[m].w, t);
                            if (SM == S_KGROUP) part[m][r] = t;
                            else acc[m][r] = t;
                        }
                    }
                }
                if (SM == S_KGROUP) {
#pragma unroll
                    for (int m = 0; m < M; ++m)
#pragma unroll
                        for (int r = 0; r < R; ++r) acc[m][r] = __builtin_fmaf(s[r], part[m][r], acc[m][r]);
                }
            }
        }

        // reduce across the wave and write
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float v = wave_sum(acc[m][r]);
                const int n = n0 + r;
                if (lane == 0 && n < p.N) {
                    if (SM == S_ROW) v *= p.scales[n];
                    p.y[(int64_t)m * p.ldy + n] = v;
                }
            }
    }
}

template <int PREC>
constexpr int chunk_elems() { return PREC == 8 ? kInt8ChunkElems : kInt4ChunkElems; }

int64_t lds_bytes_for(const tbh_weight &w, int64_t M) {
    const int ce = w.precision == TBH_PREC_INT8 ? kInt8ChunkElems : kInt4ChunkElems;
    return M * (w.Kp / ce) * (ce + 4) * (int64_t)sizeof(float);
}

template <int PREC, int SM, int M, int R, bool ZP>
hipError_t launch_one(const KParams &p, int blocks, size_t lds, hipStream_t s) {
    hipLaunchKernelGGL((gemv_valu<PREC, SM, M, R, ZP>), dim3(blocks), dim3(256), lds, s, p);
    return hipGetLastError();
}

template <int PREC, int SM, int M, bool ZP>
hipError_t dispatch_r(int R, const KParams &p, int blocks, size_t lds, hipStream_t s) {
    switch (R) {
    case 1: return launch_one<PREC, SM, M, 1, ZP>(p, blocks, lds, s);
    case 2: return launch_one<PREC, SM, M, 2, ZP>(p, blocks, lds, s);
    case 4: return launch_one<PREC, SM, M, 4, ZP>(p, blocks, lds, s);
    case 8:
        if constexpr (M <= 2) return launch_one<PREC, SM, M, 8, ZP>(p, blocks, lds, s);
        return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

template <int PREC, int SM, bool ZP>
hipError_t dispatch_m(int M, int R, const KParams &p, int blocks, size_t lds, hipStream_t s) {
    switch (M) {
    case 1: return dispatch_r<PREC, SM, 1, ZP>(R, p, blocks, lds, s);
    case 2: return dispatch_r<PREC, SM, 2, ZP>(R, p, blocks, lds, s);
    case 3: return dispatch_r<PREC, SM, 3, ZP>(R, p, blocks, lds, s);
    case 4: return dispatch_r<PREC, SM, 4, ZP>(R, p, blocks, lds, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

int64_t gemv_max_rows(const tbh_weight &w) {
    if (w.path == Path::Generic) return 0;
    for (int64_t m = 4; m >= 1; --m)
        if (lds_bytes_for(w, m) <= kMaxLdsBytes) return m;
    return 0;
}

hipError_t launch_gemv(const tbh_weight &w, const GemvArgs &a, hipStream_t s) {
    const int M = (int)a.M;
    if (M < 1 || M > 4) return hipErrorInvalidValue;
    const int64_t lds = lds_bytes_for(w, M);
    if (lds > kMaxLdsBytes) return hipErrorInvalidValue;

    KParams p{};
    p.x = a.x;
    p.ldx = a.ldx;
    p.y = a.y;
    p.ldy = a.ldy;
    p.data = w.data;
    p.row_bytes = w.row_bytes;
    p.scales = w.scales;
    p.zp = w.zp;
    p.K = (int32_t)w.K;
    p.Kp = (int32_t)w.Kp;
    p.N = (int32_t)w.N;
    p.Np = (int32_t)w.Np;
    const bool int8 = w.precision == TBH_PREC_INT8;
    p.chunks = (int32_t)(w.Kp / (int8 ? kInt8ChunkElems : kInt4ChunkElems));
    p.G = (int32_t)w.groups_per_row;
    p.cpg = w.chunks_per_group;
    p.rpn = w.rows_per_nblock;

    // Rows per wave: as many as keep >= 8 waves per CU busy, within the
    // register budget (M*R <= 16) and dividing the N-block height.
    const int64_t target_waves = 8LL * std::max(1, w.dev->cu_count);
    int R = 8;
    while (R > 1 && (w.Np / R < target_waves || M * R > 16 ||
                     (w.path == Path::Int4NGroup && p.rpn % R != 0) || (M > 2 && R > 4)))
        R /= 2;
    const int64_t waves = w.Np / R;
    const int64_t max_blocks = 8LL * std::max(1, w.dev->cu_count);
    const int blocks = (int)std::max<int64_t>(1, std::min((waves + 3) / 4, max_blocks));
    const bool zp = w.zp != nullptr;

    switch (w.path) {
    case Path::Int8Row:
        return zp ? dispatch_m<8, S_ROW, true>(M, R, p, blocks, (size_t)lds, s)
                  : dispatch_m<8, S_ROW, false>(M, R, p, blocks, (size_t)lds, s);
    case Path::Int4KGroup:
        return zp ? dispatch_m<4, S_KGROUP, true>(M, R, p, blocks, (size_t)lds, s)
                  : dispatch_m<4, S_KGROUP, false>(M, R, p, blocks, (size_t)lds, s);
    case Path::Int4NGroup:
        return dispatch_m<4, S_NGROUP, false>(M, R, p, blocks, (size_t)lds, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace tbh

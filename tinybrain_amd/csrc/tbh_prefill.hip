// tbh_prefill.hip -- prefill dequant-GEMM on bf16 MFMA (M >= 64 rows of x).
//
// y[M, N] = x[M, K] (bf16) . dequantize(W)[K, N], fp32 accumulation, for the
// repacked K-contiguous row layout.  This is the one dense contraction of the
// path: the reference runs it as dequantize() + cblas_sgemm on the CPU
// (Sources/TinyBrainRuntime/QuantizedTensor.swift:640-642,
// Tensor.swift:839-861) or as the MSL dequant kernels one output per thread
// (Shaders/Dequant.metal:49-79, DequantINT4.metal:95-137).
//
// A 256-thread block owns a BM x BN output tile; its four waves own
// (BM/2) x (BN/2) each, as TM x TN tiles of v_mfma_f32_16x16x32_bf16.  Per
// K step of 64 the block stages x (bf16, as given) and the dequantized weight
// tile in LDS; global loads of step t+1 are in flight while step t's MFMAs
// run.  Weight operands are exact:
//   * INT8 (one scale per row): q - zp is an integer of magnitude <= 255,
//     exact in bf16; the row scale multiplies the fp32 result once.
//   * INT4 K-groups: v = (q - zp) * scale is formed in fp32 with the
//     reference's single rounding, then split into three bf16 pieces
//     v = hi + mid + lo by truncation (24 significant bits), and each piece
//     is one MFMA.  The products x * piece are exact in fp32.
// Accumulation is fp32 in the MFMA.
#include "tbh_internal.h"

namespace tbh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;           // K per staged step (two MFMA K-steps of 32)
constexpr int kRowPad = 8;        // bf16 of padding per LDS row (16 bytes)
constexpr int kLdsRow = kBK + kRowPad;
constexpr int kDepth = 2;         // K steps whose global loads are in flight at once

struct PParams {
    const uint16_t *x;   // bf16 bits, [M][ldx]
    int64_t ldx;
    float *y;
    int64_t ldy;
    const uint8_t *data;
    int64_t row_bytes;
    const float *scales;
    const int8_t *zp;
    int32_t M, K, N, Np;
    int32_t chunks;  // 16-byte chunks per row
    int32_t G;       // INT4 K-groups per row
    int32_t cpg;     // chunks per K-group
};

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Two fp32 values -> one dword of two bf16 (upper halves; exact when the low
// halves are zero, else truncation).
__device__ __forceinline__ uint32_t pack_hi16(float lo_elem, float hi_elem) {
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hi_elem),
                                 __builtin_bit_cast(uint32_t, lo_elem), 0x07060302u);
}

// Byte J of w as fp32 (v_cvt_f32_ubyteJ).
template <int J>
__device__ __forceinline__ float ubyte(uint32_t w) {
    return (float)((w >> (8 * J)) & 0xFFu);
}

__device__ __forceinline__ float trunc_bf16(float v) {
    return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) & 0xFFFF0000u);
}

template <int PREC, int BM, int BN, bool ZP>
__global__ __launch_bounds__(256) void gemm_bf16(const PParams p) {
    constexpr int CE = PREC == 8 ? 16 : 32;       // elements per chunk
    constexpr int NS = PREC == 8 ? 1 : 3;         // bf16 pieces per weight
    constexpr int CPR = kBK / CE;                 // chunks per row per step
    constexpr int WCH = BN * CPR;                 // weight chunks per step
    constexpr int WPT = (WCH + 255) / 256;        // per thread (last may idle)
    constexpr int XSEG = BM * (kBK / 8);          // 16-byte x segments per step
    constexpr int XPT = XSEG / 256;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 16, TN = WN / 16;
    static_assert(XSEG % 256 == 0, "BM must be a multiple of 32");

    __shared__ __attribute__((aligned(16))) uint16_t xs[BM * kLdsRow];
    __shared__ __attribute__((aligned(16))) uint16_t ws[NS * BN * kLdsRow];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int nsteps = (p.chunks * CE + kBK - 1) / kBK;

    // ---- global -> registers for one step, into register stage d of kDepth:
    // the loads of steps t+1 .. t+kDepth-1 are in flight while step t runs
    u32x4 xr[kDepth][XPT];
    bool xin[kDepth][XPT];   // segment within K, applied at the LDS store
    u32x4 wr[kDepth][WPT];
    float sr[kDepth][WPT];
    int8_t zq[kDepth][WPT];
    // Only addresses are computed here; everything that uses a loaded value
    // (masks, conversions) happens in store_step, kDepth - 1 steps later.
    auto load_step = [&](int t, int d) {
        const int k0 = t * kBK;
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int s = tid + 256 * j;
            const int row = s / (kBK / 8), kq = s % (kBK / 8);
            const int m = min(m0 + row, p.M - 1), k = k0 + 8 * kq;
            // K % 8 == 0: a segment is all in or out.  Rows past M read row
            // M-1 (finite values; their outputs are never stored).
            xin[d][j] = k < p.K;
            xr[d][j] = *(const u32x4 *)(p.x + (int64_t)m * p.ldx + (k < p.K ? k : 0));
        }
#pragma unroll
        for (int j = 0; j < WPT; ++j) {
            const int s = tid + 256 * j;
            const int row = s / CPR, c = t * CPR + s % CPR;
            const int n = n0 + row;
            const bool in = s < WCH && n < p.Np && c < p.chunks;
            // Out-of-range chunks read a valid chunk: rows past N are never
            // stored and K padding meets x = 0, so the values do not matter.
            const int64_t nn = in ? n : 0, cc = in ? c : 0;
            wr[d][j] = __builtin_nontemporal_load((const u32x4 *)(p.data + nn * p.row_bytes + cc * 16));
            if (PREC == 4) {
                const int64_t gi = nn * p.G + cc / p.cpg;
                sr[d][j] = p.scales[gi];
                if (ZP) zq[d][j] = p.zp[gi];
            } else if (ZP) {
                zq[d][j] = p.zp[nn];
            }
        }
    };

    // ---- registers -> LDS (x as is; weights dequantized to bf16 pieces)
    auto store_step = [&](int d) {
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int s = tid + 256 * j;
            const int row = s / (kBK / 8), kq = s % (kBK / 8);
            *(u32x4 *)&xs[row * kLdsRow + 8 * kq] = xin[d][j] ? xr[d][j] : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < WPT; ++j) {
            const int s = tid + 256 * j;
            if (s < WCH) {
                const int row = s / CPR, cl = s % CPR;
                uint16_t *dst = &ws[row * kLdsRow + cl * CE];
                if (PREC == 8) {
                    // bytes {0,2,1,3} of each word are k+{0,1,2,3}; value u - 128 - zp
                    const float off = 128.0f + (ZP ? (float)zq[d][j] : 0.0f);
                    uint32_t o[8];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t w = wr[d][j][q];
                        const float f0 = ubyte<0>(w) - off;
                        const float f1 = ubyte<2>(w) - off;
                        const float f2 = ubyte<1>(w) - off;
                        const float f3 = ubyte<3>(w) - off;
                        o[2 * q] = pack_hi16(f0, f1);
                        o[2 * q + 1] = pack_hi16(f2, f3);
                    }
                    *(u32x4 *)dst = u32x4{o[0], o[1], o[2], o[3]};
                    *(u32x4 *)(dst + 8) = u32x4{o[4], o[5], o[6], o[7]};
                } else {
                    // nibble of k % 8 at bit {0,16,4,20,8,24,12,28}; value
                    // (u - 8 - zp) * scale, one fp32 rounding
                    const float off = 8.0f + (ZP ? (float)zq[d][j] : 0.0f);
                    const float sc = sr[d][j];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t w = wr[d][j][q];
                        uint32_t oh[4], om[4], ol[4];
#pragma unroll
                        for (int e = 0; e < 8; e += 2) {
                            const int sh0 = ((e >> 1) << 2), sh1 = 16 + ((e >> 1) << 2);
                            const float v0 = __fmul_rn((float)((w >> sh0) & 15u) - off, sc);
                            const float v1 = __fmul_rn((float)((w >> sh1) & 15u) - off, sc);
                            const float h0 = trunc_bf16(v0), h1 = trunc_bf16(v1);
                            const float r0 = v0 - h0, r1 = v1 - h1;
                            const float g0 = trunc_bf16(r0), g1 = trunc_bf16(r1);
                            oh[e >> 1] = pack_hi16(h0, h1);
                            om[e >> 1] = pack_hi16(g0, g1);
                            ol[e >> 1] = pack_hi16(r0 - g0, r1 - g1);
                        }
                        *(u32x4 *)(dst + 8 * q) = u32x4{oh[0], oh[1], oh[2], oh[3]};
                        *(u32x4 *)(dst + BN * kLdsRow + 8 * q) = u32x4{om[0], om[1], om[2], om[3]};
                        *(u32x4 *)(dst + 2 * BN * kLdsRow + 8 * q) = u32x4{ol[0], ol[1], ol[2], ol[3]};
                    }
                }
            }
        }
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Steps are padded to a multiple of kDepth and every iteration loads and
    // computes unconditionally: steps past K read clamped addresses and meet
    // x = 0, so they add nothing, and the loop body has no branches at which
    // the compiler would have to wait for every load in flight.
    const int nsteps_pad = ((nsteps + kDepth - 1) / kDepth) * kDepth;
#pragma unroll
    for (int d = 0; d < kDepth; ++d) load_step(d, d);
    for (int t0 = 0; t0 < nsteps_pad; t0 += kDepth) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            store_step(d);
            lds_barrier();
            load_step(t0 + d + kDepth, d);
#pragma unroll
            for (int ks = 0; ks < kBK / 32; ++ks) {
                const int kofs = ks * 32 + 8 * (lane >> 4);
                bf16x8 af[TM];
#pragma unroll
                for (int a = 0; a < TM; ++a)
                    af[a] = *(const bf16x8 *)&xs[(wm * WM + a * 16 + (lane & 15)) * kLdsRow + kofs];
#pragma unroll
                for (int ps = 0; ps < NS; ++ps) {
#pragma unroll
                    for (int b = 0; b < TN; ++b) {
                        const bf16x8 bfr = *(const bf16x8 *)&ws[ps * BN * kLdsRow +
                                                                (wn * WN + b * 16 + (lane & 15)) * kLdsRow + kofs];
#pragma unroll
                        for (int a = 0; a < TM; ++a)
                            acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[a], bfr, acc[a][b], 0, 0, 0);
                    }
                }
            }
            lds_barrier();
        }
    }

    // ---- epilogue: lane holds C[4 (lane / 16) + e][lane % 16] of each tile
#pragma unroll
    for (int b = 0; b < TN; ++b) {
        const int n = n0 + wn * WN + b * 16 + (lane & 15);
        if (n >= p.N) continue;
        const float sc = PREC == 8 ? p.scales[n] : 1.0f;
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = m0 + wm * WM + a * 16 + 4 * (lane >> 4) + e;
                if (m < p.M) p.y[(int64_t)m * p.ldy + n] = PREC == 8 ? acc[a][b][e] * sc : acc[a][b][e];
            }
    }
}

template <int PREC, int BM, int BN>
hipError_t launch_tile(const PParams &p, hipStream_t s) {
    const dim3 grid((unsigned)((p.Np + BN - 1) / BN), (unsigned)((p.M + BM - 1) / BM));
    if (p.zp)
        hipLaunchKernelGGL((gemm_bf16<PREC, BM, BN, true>), grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((gemm_bf16<PREC, BM, BN, false>), grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

template <int PREC>
hipError_t launch_prec(const PParams &p, int64_t cus, hipStream_t s) {
    // Largest tile that still gives every CU a block.
    const int64_t t128 = ((p.Np + 127) / 128) * ((p.M + 127) / 128);
    const int64_t t64x128 = ((p.Np + 127) / 128) * ((p.M + 63) / 64);
    if (t128 >= cus) return launch_tile<PREC, 128, 128>(p, s);
    if (t64x128 >= cus) return launch_tile<PREC, 64, 128>(p, s);
    return launch_tile<PREC, 64, 64>(p, s);
}

}  // namespace

bool prefill_supported(const tbh_weight &w) {
    return !w.mfma_tiles && (w.path == Path::Int8Row || w.path == Path::Int4KGroup);
}

hipError_t launch_prefill(const tbh_weight &w, const uint16_t *x, int64_t ldx, int64_t M, float *y,
                          int64_t ldy, hipStream_t s) {
    if (!prefill_supported(w) || M < 1 || w.K % 8 != 0 || ldx % 8 != 0 ||
        ((uintptr_t)x & 15) != 0)
        return hipErrorInvalidValue;
    PParams p{};
    p.x = x;
    p.ldx = ldx;
    p.y = y;
    p.ldy = ldy;
    p.data = w.data;
    p.row_bytes = w.row_bytes;
    p.scales = w.scales;
    p.zp = w.zp;
    p.M = (int32_t)M;
    p.K = (int32_t)w.K;
    p.N = (int32_t)w.N;
    p.Np = (int32_t)w.Np;
    const bool int8 = w.precision == TBH_PREC_INT8;
    p.chunks = (int32_t)(w.Kp / (int8 ? kInt8ChunkElems : kInt4ChunkElems));
    p.G = (int32_t)w.groups_per_row;
    p.cpg = w.chunks_per_group;
    const int64_t cus = std::max(1, w.dev->cu_count);
    return int8 ? launch_prec<8>(p, cus, s) : launch_prec<4>(p, cus, s);
}

}  // namespace tbh

// tbh_mgemv.hip -- MFMA dequant-GEMV for decode (M = 1..8 rows of x).
//
// Replaces the MSL kernels matmul_int8_dequant / matmul_int4_dequant
// (Sources/TinyBrainMetal/Shaders/Dequant.metal:49-79,
// DequantINT4.metal:95-137) for INT8 (any per-row scale) and INT4 with
// K-grouped scales.  The multiply-accumulate runs on the matrix cores with
// v_mfma_f32_16x16x32_f16; the vector ALUs only unpack weights.
//
// Operands of one MFMA (16 output rows n x 32 K elements):
//   B (weights): lane l holds the 8 K elements 8*(l/16)..+7 of row l%16 as
//     f16 values q - zp, exact: the repacked word's nibbles/bytes are OR-ed
//     into the f16 magic 0x6400 (1024 + u) and one v_pk_add_f16 subtracts
//     the offset, as in the VALU kernel.  INT4 slots 2, 3, 6, 7 hold 16*(q-zp).
//   A (x): rows 2m and 2m+1 carry x[m] split into f16 pieces hi + lo
//     (22 significant bits), after scaling the row by a power of two 2^-e_m
//     so that max|x[m]| lands in [2^14, 2^15) (no overflow, no subnormal
//     loss); INT4 slots 2, 3, 6, 7 are pre-divided by 16.  Rows >= 2M are 0.
//   C: lane l holds rows 4*(l/16)..+3 of column l%16, i.e. (m = 2g, hi),
//     (2g, lo), (2g+1, hi), (2g+1, lo) for g = l/16.
// Every product q * x_piece is exact in fp32 and accumulates in fp32; the
// result is y = 2^e_m * s * (C_hi + C_lo).  Per-row scales (INT8, INT4 with
// one group per row) are applied once at the end; INT4 K-group scales are
// applied per 32-element chunk to a fresh C tile.
//
// HBM layout (one-time repack): 1 KiB tiles of 16 rows x 128 K (INT4) or
// 16 rows x 64 K (INT8); lane l's 16 bytes are its B words for the 4 (INT4)
// or 2 (INT8) MFMAs of the tile, so each wave load is 1 KiB contiguous.
//
// Schedule: block = 4 waves = RT row tiles x KP K-parts.  Waves stream their
// tiles with a 4-deep register prefetch; x fragments for one K tile live in
// LDS (restaged at uniform barrier points); K-part partials are summed in LDS
// in a fixed order (deterministic).
#include <cmath>
#include <cstdlib>

#include "tbh_internal.h"

namespace tbh {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

struct MParams {
    const float *x;
    int64_t ldx;
    float *y;
    int64_t ldy;
    const uint8_t *data;      // [ntiles][SC] 1 KiB tiles
    const float *scales;      // ROW: [Np]; KGROUP: [ntiles][SC][16][4]
    const int8_t *zp;         // same shapes as scales (int8)
    int32_t K, N;
    int32_t ntiles;           // Np / 16
    int32_t SC;               // K tiles per row tile (Kp / SCK)
    int32_t SCT;              // K tiles per LDS stage (multiple of D * KP)
    int32_t IPG;              // work items per row-tile group (ceil(SC / KP) rounded to D)
    int32_t x_vec4;           // x rows 16-byte aligned and K % 4 == 0
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

// Waits for this thread's LDS writes, then a workgroup barrier that does not
// wait for outstanding global loads (so the weight prefetch stays in flight).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// B fragment of one INT4 word (8 nibbles at bit offsets 0,16,4,20,8,24,12,28).
__device__ __forceinline__ half8 unpack_int4(uint32_t w, h2 c1, h2 c16) {
    const uint32_t kMagic = 0x64006400u, kLo = 0x000F000Fu, kHi = 0x00F000F0u;
    const uint32_t w8 = w >> 8;
    const h2 p0 = as_h2(and_or(w, kLo, kMagic)) + c1;
    const h2 p1 = as_h2(and_or(w, kHi, kMagic)) + c16;
    const h2 p2 = as_h2(and_or(w8, kLo, kMagic)) + c1;
    const h2 p3 = as_h2(and_or(w8, kHi, kMagic)) + c16;
    half8 r;
    r[0] = p0.x; r[1] = p0.y; r[2] = p1.x; r[3] = p1.y;
    r[4] = p2.x; r[5] = p2.y; r[6] = p3.x; r[7] = p3.y;
    return r;
}

// B fragment of two INT8 words (bytes at positions 0,2,1,3 in each word).
__device__ __forceinline__ half8 unpack_int8(uint32_t w0, uint32_t w1, h2 c8) {
    const uint32_t kMagic = 0x64006400u, kLo = 0x00FF00FFu;
    const h2 a0 = as_h2(and_or(w0, kLo, kMagic)) + c8;
    const h2 a1 = as_h2(and_or(w0 >> 8, kLo, kMagic)) + c8;
    const h2 b0 = as_h2(and_or(w1, kLo, kMagic)) + c8;
    const h2 b1 = as_h2(and_or(w1 >> 8, kLo, kMagic)) + c8;
    half8 r;
    r[0] = a0.x; r[1] = a0.y; r[2] = a1.x; r[3] = a1.y;
    r[4] = b0.x; r[5] = b0.y; r[6] = b1.x; r[7] = b1.y;
    return r;
}

enum { SM_ROW = 0, SM_KGROUP = 1 };

template <int PREC, int SM, int M, int RT, bool ZP>
__global__ __launch_bounds__(256) void mgemv(const MParams p) {
    constexpr int KP = 4 / RT;                 // waves splitting K per row tile
    constexpr int CPT = PREC == 4 ? 4 : 2;     // 32-element chunks (= MFMAs) per tile
    constexpr int FR = 2 * M;                  // A rows in use
    constexpr int D = kMgemvDepth;             // prefetch depth (tiles)
    constexpr int FCHUNK = 4 * FR;             // 16-byte fragments per chunk

    extern __shared__ u32x4 lds[];             // A fragments of one stage
    __shared__ float red[KP > 1 ? (KP - 1) * RT * 64 * 2 : 1];
    __shared__ float xmax[4][M];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int slot = wave % RT, kp = wave / RT;
    const int g = lane >> 4, r16 = lane & 15;

    // ---- work items of this wave: (row-tile group, K tile), group-major.
    // Groups are strided over the (persistent) grid; every group has IPG
    // items (a multiple of D, uniform for all waves), the tail ones empty.
    const int ngt = (p.ntiles + RT - 1) / RT;
    const int my_groups = (int)blockIdx.x < ngt ? (ngt - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;
    const int total = my_groups * p.IPG;
    auto item_rt = [&](int t) { return ((int)blockIdx.x + (t / p.IPG) * (int)gridDim.x) * RT + slot; };
    auto item_sc = [&](int t) { return kp + (t % p.IPG) * KP; };

    auto tile_base = [&](int t, int &sc) -> int64_t {
        t = min(t, max(total - 1, 0));
        const int rtc = min(item_rt(t), p.ntiles - 1);
        sc = min(item_sc(t), p.SC - 1);
        return (int64_t)rtc * p.SC + sc;  // tile index
    };
    u32x4 b[D];
    f32x4 sk[D];
    uint32_t zk[D];
    auto load_item = [&](int t, int i) {
        int sc;
        const int64_t tb = tile_base(t, sc);
        b[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p.data) + tb * 64 + lane);
        if (SM == SM_KGROUP) sk[i] = *reinterpret_cast<const f32x4 *>(p.scales + (tb * 16 + r16) * 4);
        if (SM == SM_KGROUP && ZP) zk[i] = *reinterpret_cast<const uint32_t *>(p.zp + (tb * 16 + r16) * 4);
    };

    // ---- x: per-row power-of-two exponent (block-wide max |x[m]|), then the
    // A fragments of the first LDS stage.  When the stage covers all of K and
    // x has at most 256 units of 8 values, x is read from L2 once.
    const int chunks_total = p.SC * CPT;
    const int first_nch = min(p.SCT * CPT, chunks_total);

    auto load_unit = [&](int u, int nch, int c0, float (&v)[8], int &m) {
        // unit u = (m, local chunk, kb): 8 consecutive x values, zero beyond K
        const int per_m = nch * 4;
        m = u / per_m;
        const int rest = u - m * per_m;
        const int k = 32 * (c0 + (rest >> 2)) + 8 * (rest & 3);
        const float *xr = p.x + (int64_t)min(m, M - 1) * p.ldx;
        if (p.x_vec4) {
            const float4 a4 = *(const float4 *)(xr + min(k, p.K - 4));
            const float4 b4 = *(const float4 *)(xr + min(k + 4, p.K - 4));
            v[0] = a4.x; v[1] = a4.y; v[2] = a4.z; v[3] = a4.w;
            v[4] = b4.x; v[5] = b4.y; v[6] = b4.z; v[7] = b4.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = xr[min(k + e, p.K - 1)];
        }
        const bool in = m < M;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (in && k + e < p.K) ? v[e] : 0.0f;
    };
    int ex[M];
    auto write_unit = [&](int u, int nch, const float (&v)[8], int m) {
        const int per_m = nch * 4;
        if (m >= M) return;
        const int rest = u - m * per_m;
        const int cl = rest >> 2, kb = rest & 3;
        int e_m = 0;
#pragma unroll
        for (int mm = 0; mm < M; ++mm) e_m = mm == m ? ex[mm] : e_m;
        const float f = ldexpf(1.0f, -e_m), f16th = f * 0.0625f;
        half8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float t = v[e] * ((PREC == 4 && (e & 2)) ? f16th : f);
            const _Float16 h = (_Float16)t;
            hi[e] = h;
            lo[e] = (_Float16)(t - (float)h);
        }
        const int fb = cl * FCHUNK + kb * FR + 2 * m;
        lds[fb] = __builtin_bit_cast(u32x4, hi);
        lds[fb + 1] = __builtin_bit_cast(u32x4, lo);
    };
    auto block_exponents = [&](float (&mx)[M]) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float v = mx[m];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
            if (lane == 0) xmax[wave][m] = v;
        }
        lds_barrier();
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float v = fmaxf(fmaxf(xmax[0][m], xmax[1][m]), fmaxf(xmax[2][m], xmax[3][m]));
            // brings max|x| into [2^14, 2^15); 0 for zero or non-finite rows
            ex[m] = (v > 0.0f && v <= 3.4e38f) ? ilogbf(v) - 14 : 0;
        }
    };
    auto stage = [&](int c0, int nch) {
        for (int u0 = 0; u0 < M * nch * 4; u0 += 256) {
            float v[8];
            int m;
            load_unit(u0 + tid, nch, c0, v, m);
            write_unit(u0 + tid, nch, v, m);
        }
    };
    {
        // x loads go out before the weight prefetch: vmcnt retires loads in
        // order, so x can then be waited for while the weights stay in flight
        constexpr int XU = 3;  // x units (8 values) per thread in the one-pass case
        float mx[M];
#pragma unroll
        for (int m = 0; m < M; ++m) mx[m] = 0.0f;
        const int units = M * chunks_total * 4;
        if (p.SCT >= p.SC && units <= 256 * XU) {
            float v[XU][8];
            int um[XU];
#pragma unroll
            for (int t = 0; t < XU; ++t) load_unit(tid + 256 * t, first_nch, 0, v[t], um[t]);
            __builtin_amdgcn_sched_barrier(0);  // keep the x loads ahead of the weight loads
#pragma unroll
            for (int i = 0; i < D; ++i) load_item(i, i);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < XU; ++t) {
                float lm = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) lm = fmaxf(lm, fabsf(v[t][e]));
#pragma unroll
                for (int mm = 0; mm < M; ++mm) mx[mm] = um[t] == mm ? fmaxf(mx[mm], lm) : mx[mm];
            }
            block_exponents(mx);
#pragma unroll
            for (int t = 0; t < XU; ++t) write_unit(tid + 256 * t, first_nch, v[t], um[t]);
        } else {
#pragma unroll
            for (int i = 0; i < D; ++i) load_item(i, i);
            for (int u0 = 0; u0 < units; u0 += 256) {
                float v[8];
                int m;
                load_unit(u0 + tid, chunks_total, 0, v, m);
                float lm = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) lm = fmaxf(lm, fabsf(v[e]));
#pragma unroll
                for (int mm = 0; mm < M; ++mm) mx[mm] = m == mm ? fmaxf(mx[mm], lm) : mx[mm];
            }
            block_exponents(mx);
            stage(0, first_nch);
        }
    }
    lds_barrier();

    // A fragment of this lane (row r16 of block g).  Rows >= 2M feed only C
    // rows that are never read, so those lanes may read any fragment.
    const int a_lane = g * FR + (r16 < FR ? r16 : FR - 1);

    f32x4 cacc = {0.f, 0.f, 0.f, 0.f};  // SM_ROW: running C
    float acc0 = 0.0f, acc1 = 0.0f;     // SM_KGROUP: scaled sums of (m=2g) and (m=2g+1)
    auto compute = [&](const u32x4 &bw, const f32x4 &sv, uint32_t z, int sc, h2 c8, h2 c1d, h2 c16d) {
        const u32x4 *ap = lds + (sc % p.SCT) * CPT * FCHUNK + a_lane;
        if (PREC == 4) {
            half8 bf[4], af[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                h2 c1 = c1d, c16 = c16d;
                if (SM == SM_KGROUP && ZP) {
                    const float zf = (float)(int8_t)((z >> (8 * j)) & 0xFF);
                    c1 = splat(-(1032.0f + zf));
                    c16 = splat(-(1152.0f + 16.0f * zf));
                }
                bf[j] = unpack_int4(bw[j], c1, c16);
                af[j] = __builtin_bit_cast(half8, ap[j * FCHUNK]);
            }
            if (SM == SM_KGROUP) {
                f32x4 c[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[j], bf[j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc0 = __builtin_fmaf(sv[j], c[j][0] + c[j][1], acc0);
                    if (M > 1) acc1 = __builtin_fmaf(sv[j], c[j][2] + c[j][3], acc1);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) cacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[j], bf[j], cacc, 0, 0, 0);
            }
        } else {
            half8 bf[2], af[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                bf[j] = unpack_int8(bw[2 * j], bw[2 * j + 1], c8);
                af[j] = __builtin_bit_cast(half8, ap[j * FCHUNK]);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) cacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[j], bf[j], cacc, 0, 0, 0);
        }
    };

    // ---- main loop over items in blocks of D (uniform trip count in the block)
    int stage_idx = 0;
    for (int t0 = 0; t0 < total; t0 += D) {
        const int rt = item_rt(t0);
        const int rtc = min(rt, p.ntiles - 1);
        // offset constants of this row tile (per lane for a per-row zero point)
        const float zrow = (SM == SM_ROW && ZP) ? (float)p.zp[(int64_t)rtc * 16 + r16] : 0.0f;
        const h2 c8 = splat(-(1152.0f + zrow));
        const h2 c1d = splat(-(1032.0f + zrow)), c16d = splat(-(1152.0f + 16.0f * zrow));
        const int st = ((t0 % p.IPG) * KP) / p.SCT;  // LDS stage (multi-stage grids only)
        if (st != stage_idx) {
            lds_barrier();
            stage(st * p.SCT * CPT, min(p.SCT * CPT, chunks_total - st * p.SCT * CPT));
            lds_barrier();
            stage_idx = st;
        }
#pragma unroll
        for (int i = 0; i < D; ++i) {
            const int sc = item_sc(t0 + i);
            if (sc < p.SC) compute(b[i], sk[i], zk[i], sc, c8, c1d, c16d);
            load_item(t0 + i + D, i);
        }
        if ((t0 + D) % p.IPG == 0) {
            // row tile done: per-lane results for (m = 2g) and (m = 2g + 1)
            float v0, v1;
            if (SM == SM_KGROUP) {
                v0 = acc0;
                v1 = acc1;
            } else {
                v0 = cacc[0] + cacc[1];
                v1 = cacc[2] + cacc[3];
            }
            if (KP > 1) {
                // K-part partials: parts 1..KP-1 park in LDS, part 0 adds them in order
                if (kp > 0) {
                    float *dst = red + (((kp - 1) * RT + slot) * 64 + lane) * 2;
                    dst[0] = v0;
                    dst[1] = v1;
                }
                lds_barrier();
                if (kp == 0) {
#pragma unroll
                    for (int q = 1; q < KP; ++q) {
                        const float *src = red + (((q - 1) * RT + slot) * 64 + lane) * 2;
                        v0 += src[0];
                        v1 += src[1];
                    }
                }
                lds_barrier();  // red is reused by the next row tile
            }
            if (kp == 0 && rt < p.ntiles) {
                const int n = rt * 16 + r16;
                if (n < p.N) {
                    const float srow = SM == SM_ROW ? p.scales[n] : 1.0f;
                    int e0 = 0, e1 = 0;
#pragma unroll
                    for (int mm = 0; mm < M; ++mm) {
                        e0 = mm == 2 * g ? ex[mm] : e0;
                        e1 = mm == 2 * g + 1 ? ex[mm] : e1;
                    }
                    if (2 * g < M) p.y[(int64_t)(2 * g) * p.ldy + n] = ldexpf(v0 * srow, e0);
                    if (2 * g + 1 < M) p.y[(int64_t)(2 * g + 1) * p.ldy + n] = ldexpf(v1 * srow, e1);
                }
            }
            cacc = f32x4{0.f, 0.f, 0.f, 0.f};
            acc0 = 0.0f;
            acc1 = 0.0f;
        }
    }
}

int env_int(const char *name, int dflt) {
    const char *v = std::getenv(name);
    return v && *v ? std::atoi(v) : dflt;
}

template <int PREC, int SM, int M, int RT, bool ZP>
hipError_t launch_one(const MParams &p, int blocks, size_t lds, hipStream_t s) {
    hipLaunchKernelGGL((mgemv<PREC, SM, M, RT, ZP>), dim3(blocks), dim3(256), lds, s, p);
    return hipGetLastError();
}

template <int PREC, int SM, int M, bool ZP>
hipError_t dispatch_rt(int RT, const MParams &p, int blocks, size_t lds, hipStream_t s) {
    switch (RT) {
    case 1: return launch_one<PREC, SM, M, 1, ZP>(p, blocks, lds, s);
    case 2: return launch_one<PREC, SM, M, 2, ZP>(p, blocks, lds, s);
    case 4: return launch_one<PREC, SM, M, 4, ZP>(p, blocks, lds, s);
    default: return hipErrorInvalidValue;
    }
}

template <int PREC, int SM, bool ZP>
hipError_t dispatch_m(int M, int RT, const MParams &p, int blocks, size_t lds, hipStream_t s) {
    switch (M) {
    case 1: return dispatch_rt<PREC, SM, 1, ZP>(RT, p, blocks, lds, s);
    case 2: return dispatch_rt<PREC, SM, 2, ZP>(RT, p, blocks, lds, s);
    case 3: return dispatch_rt<PREC, SM, 3, ZP>(RT, p, blocks, lds, s);
    case 4: return dispatch_rt<PREC, SM, 4, ZP>(RT, p, blocks, lds, s);
    case 5: return dispatch_rt<PREC, SM, 5, ZP>(RT, p, blocks, lds, s);
    case 6: return dispatch_rt<PREC, SM, 6, ZP>(RT, p, blocks, lds, s);
    case 7: return dispatch_rt<PREC, SM, 7, ZP>(RT, p, blocks, lds, s);
    case 8: return dispatch_rt<PREC, SM, 8, ZP>(RT, p, blocks, lds, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_mgemv(const tbh_weight &w, const GemvArgs &a, hipStream_t s) {
    const int M = (int)a.M;
    if (M < 1 || M > 8 || !w.mfma_tiles) return hipErrorInvalidValue;
    const bool int4 = w.precision == TBH_PREC_INT4;
    const int sck = int4 ? kMfmaInt4TileK : kMfmaInt8TileK;
    const int cpt = int4 ? 4 : 2;

    MParams p{};
    p.x = a.x;
    p.ldx = a.ldx;
    p.y = a.y;
    p.ldy = a.ldy;
    p.data = w.data;
    p.scales = w.scales;
    p.zp = w.zp;
    p.K = (int32_t)w.K;
    p.N = (int32_t)w.N;
    p.ntiles = (int32_t)(w.Np / 16);
    p.SC = (int32_t)(w.Kp / sck);
    p.x_vec4 = (w.K % 4 == 0 && a.ldx % 4 == 0 && ((uintptr_t)a.x & 15) == 0) ? 1 : 0;

    // Row tiles per block (RT) x K-parts (KP = 4 / RT): split K inside the
    // block when there are few row tiles, so small N still fills the GPU.
    static const int rt_force = env_int("TBH_MGEMV_RT", 0);
    const int64_t cus = std::max(1, w.dev->cu_count);
    int RT = p.ntiles >= 8 * cus ? 4 : (p.ntiles >= 4 * cus ? 2 : 1);
    if (rt_force == 1 || rt_force == 2 || rt_force == 4) RT = rt_force;
    // LDS stage: K tiles per stage, a multiple of 4 * KP, within the budget
    const int64_t frag_bytes_per_tile = (int64_t)cpt * 4 * 2 * M * 16;
    while (RT < 4 && kMgemvDepth * (4 / RT) * frag_bytes_per_tile > kMgemvLdsBytes) RT *= 2;
    const int KP = 4 / RT;
    int64_t sct = kMgemvLdsBytes / frag_bytes_per_tile;
    const int64_t step = kMgemvDepth * KP;
    sct = std::max<int64_t>(step, sct / step * step);
    if (sct >= p.SC) sct = (p.SC + step - 1) / step * step;
    p.SCT = (int32_t)sct;
    const size_t lds = (size_t)(sct * frag_bytes_per_tile);
    if (lds > (size_t)kMgemvLdsBytes) return hipErrorInvalidValue;

    p.IPG = (int32_t)(((p.SC + KP - 1) / KP + kMgemvDepth - 1) / kMgemvDepth * kMgemvDepth);
    // persistent grid when one LDS stage covers K (x staged once per block)
    static const int bpc = env_int("TBH_MGEMV_BLOCKS_PER_CU", 3);
    const int64_t ngt = (p.ntiles + RT - 1) / RT;
    const int blocks = (int)(p.SCT >= p.SC ? std::min<int64_t>(ngt, bpc * cus) : ngt);
    const bool zp = w.zp != nullptr;
    const bool kgroup = w.path == Path::Int4KGroup && w.groups_per_row > 1;
    if (int4) {
        if (kgroup)
            return zp ? dispatch_m<4, SM_KGROUP, true>(M, RT, p, blocks, lds, s)
                      : dispatch_m<4, SM_KGROUP, false>(M, RT, p, blocks, lds, s);
        return zp ? dispatch_m<4, SM_ROW, true>(M, RT, p, blocks, lds, s)
                  : dispatch_m<4, SM_ROW, false>(M, RT, p, blocks, lds, s);
    }
    return zp ? dispatch_m<8, SM_ROW, true>(M, RT, p, blocks, lds, s)
              : dispatch_m<8, SM_ROW, false>(M, RT, p, blocks, lds, s);
}

}  // namespace tbh

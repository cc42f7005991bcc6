// tbh_gemv.hip -- VALU dequant-GEMV for decode (M = 1..4 rows of x per launch).
//
// Replaces the MSL kernels matmul_int8_dequant / matmul_int4_dequant
// (Sources/TinyBrainMetal/Shaders/Dequant.metal:49-79,
// DequantINT4.metal:95-137), which give each output one thread and walk K
// with a stride-N load.  Here one wave64 owns R output rows at a time; each
// lane streams 16-byte chunks of those rows (K-contiguous after the one-time
// repack) with non-temporal 128-bit loads, so every load instruction moves
// 1 KiB of contiguous HBM.
//
// Two schedules:
//   * gemv_burst (M in {1, 2, 4, 8}, no zero points, rows up to 64 * 6 chunks):
//     one wave per U rows (long rows at M = 1: two waves per U rows, each
//     taking half of every row's chunks), every load of the wave issued at
//     kernel start, so a launch
//     puts the whole matrix's reads in flight at once and pays HBM latency
//     about once -- the decode shapes are only 2-70 MB, a few microseconds
//     of HBM time, so latency and ramp dominate otherwise;
//   * gemv_valu (everything else): a persistent grid (a few blocks per CU)
//     where a wave walks (row group, chunk iteration) items and issues the
//     loads of item t+1 before it computes item t.
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
#include <cstdlib>

#include "tbh_internal.h"
#include "tbh_wave.h"

namespace tbh {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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
    int32_t cpg_shift;  // log2(cpg) when cpg is a power of two, else -1
    int32_t rpn;     // rows per N-block (INT4 runtime layout)
    int32_t nb_half; // INT4 runtime layout, gate|up rows interleaved: N-blocks of the first part
    int32_t x_vec4;  // x rows are 16-byte aligned and K % 4 == 0
    int32_t m_act;   // x rows present (the burst kernel's M may round it up: rows
                     // from m_act on re-read row m_act - 1 and are not stored)
    // fused decode prologue / epilogue (gemv_burst with M = 1 only)
    const float *g;    // PRO_RMSNORM: norm weight [K]
    float eps;         // PRO_RMSNORM: epsilon
    float *xcopy;      // non-null: block 0 also stores x as given here ([K])
    int32_t *advance;  // non-null: block 0 adds 1 to advance[0]
};


__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    return (a & m) | o;  // v_and_or_b32 when m and o are registers (see opaque)
}

// A constant the compiler may not fold: kept in a register, it lets
// (a & m) | o select one v_and_or_b32 (VOP3 takes no literal on gfx9)
// instead of v_and_b32 + v_or_b32 with literals.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
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

constexpr int pow2_ceil(int v) { return v <= 1 ? 1 : 2 * pow2_ceil((v + 1) / 2); }

// DPP lane permutations (gfx9 dpp_ctrl codes).
enum : int {
    kDppXor1 = 0xB1,         // quad_perm [1,0,3,2]
    kDppXor2 = 0x4E,         // quad_perm [2,3,0,1]
    kDppRor8 = 0x128,        // row_ror:8 (= lane ^ 8 inside a 16-lane row)
    kDppRowMirror = 0x140,   // lane l <- 15 - l within the row
    kDppHalfMirror = 0x141,  // lane l <- 7 - l within each 8-lane half row
};

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 0xF, 0xF, false));
}

// Partner value of lane ^ O.  Across rows by v_permlane16_swap /
// v_permlane32_swap of v with itself (a VALU exchange: v_permlane16_swap
// trades odd rows of its first operand with even rows of its second, so
// result [1] holds row r ^ 1 in even rows and [0] in odd rows; likewise for
// 32-lane halves), inside a row by DPP; __shfl_xor would be an LDS round trip.
template <int O>
__device__ __forceinline__ float xchg(float v) {
    if constexpr (O == 8) {
        return dpp<kDppRor8>(v);
    } else if constexpr (O == 16 || O == 32) {
        const uint32_t u = __builtin_bit_cast(uint32_t, v);
        const auto r = O == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                               : __builtin_amdgcn_permlane32_swap(u, u, false, false);
        const bool upper = (__lane_id() & O) != 0;
        return __builtin_bit_cast(float, upper ? r[0] : r[1]);
    } else {
        return __shfl_xor(v, O);
    }
}

// One transpose-reduce stage over the first CNT values: lanes with bit O set
// keep the upper half of the values, the others the lower half; each kept
// value absorbs the partner lane's copy.
template <int CNT, int O, int V>
__device__ __forceinline__ void transpose_stages(float (&v)[V], int lane) {
    if constexpr (CNT > 1) {
        const bool upper = (lane & O) != 0;
#pragma unroll
        for (int i = 0; i < CNT / 2; ++i) {
            const float send = upper ? v[i] : v[i + CNT / 2];
            const float keep = upper ? v[i + CNT / 2] : v[i];
            v[i] = keep + xchg<O>(send);
        }
        transpose_stages<CNT / 2, O / 2, V>(v, lane);
    }
}

// Plain sum over aligned groups of G lanes (G a power of two), low bits first.
template <int G>
__device__ __forceinline__ float group_sum(float r) {
    if constexpr (G >= 2) r += dpp<kDppXor1>(r);
    if constexpr (G >= 4) r += dpp<kDppXor2>(r);
    if constexpr (G >= 8) r += dpp<kDppHalfMirror>(r);   // quads already reduced
    if constexpr (G >= 16) r += dpp<kDppRowMirror>(r);   // halves already reduced
    if constexpr (G >= 32) r += xchg<16>(r);
    if constexpr (G >= 64) r += xchg<32>(r);
    return r;
}

// Sums V (a power of two <= 32) per-lane values over the 64 lanes of a wave
// with a transpose-reduce: each exchange stage halves the number of values a
// lane carries, so the cost is about V exchanges instead of 6 V.  Afterwards
// every lane holds the total of value index
// sum_s bit(lane, 5 - s) * (V >> (s + 1)), s = 0 .. log2(V) - 1.
template <int V>
__device__ __forceinline__ float reduce_multi(float (&v)[V], int lane) {
    transpose_stages<V, 32, V>(v, lane);
    return group_sum<64 / V>(v[0]);
}

template <int V>
__device__ __forceinline__ int reduce_index(int lane) {
    int idx = 0;
#pragma unroll
    for (int s = 0, cnt = V; cnt > 1; ++s, cnt >>= 1) idx += ((lane >> (5 - s)) & 1) * (cnt / 2);
    return idx;
}

// LDS slot of x element k: chunks are padded by 4 floats so that the
// 128-bit reads of 8 consecutive lanes (one chunk each) cover all 32 banks.
template <int CE>
__device__ __forceinline__ int lds_index(int k) {
    return (k / CE) * (CE + 4) + (k % CE);
}

template <int PREC, int M, bool VEC4>
__device__ __forceinline__ void stage_x_round(const KParams &p, float4 *xs4, int lds_row, int tid,
                                              int base) {
    constexpr int CE = PREC == 8 ? 16 : 32;
    constexpr int XU = 4;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float *xr = p.x + (int64_t)m * p.ldx;
        float4 v[XU];
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            const int k = 4 * (base + u * 256 + tid);
            if constexpr (VEC4) {
                const float4 t = *(const float4 *)(xr + min(k, p.K - 4));
                const bool in = k < p.K;
                v[u] = float4{in ? t.x : 0.f, in ? t.y : 0.f, in ? t.z : 0.f, in ? t.w : 0.f};
            } else {
                const float a0 = xr[min(k, p.K - 1)], a1 = xr[min(k + 1, p.K - 1)];
                const float a2 = xr[min(k + 2, p.K - 1)], a3 = xr[min(k + 3, p.K - 1)];
                v[u] = float4{k < p.K ? a0 : 0.f, k + 1 < p.K ? a1 : 0.f,
                              k + 2 < p.K ? a2 : 0.f, k + 3 < p.K ? a3 : 0.f};
            }
        }
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            const int k = 4 * (base + u * 256 + tid);
            if (k < p.Kp) {
                float4 t = v[u];
                if (PREC == 4) { t.z *= 0.0625f; t.w *= 0.0625f; }
                xs4[(m * lds_row + lds_index<CE>(k)) >> 2] = t;
            }
        }
    }
}

// Stages x [M][Kp] into LDS: zero beyond K, INT4 slots k % 4 in {2, 3}
// pre-divided by 16.  Each thread issues its loads of a round (4 float4 per
// row, on clamped always-in-bounds addresses, zeroed afterwards by selects)
// before it waits, so staging costs one L2 round trip for Kp <= 4096.  The
// first round is peeled out of the loop so the compiler does not wait for
// the weight loads already in flight.
template <int PREC, int M, bool VEC4>
__device__ __forceinline__ void stage_x(const KParams &p, float4 *xs4, int lds_row, int tid) {
    const int k4n = p.Kp >> 2;  // float4 slots per x row
    stage_x_round<PREC, M, VEC4>(p, xs4, lds_row, tid, 0);
    if (k4n > 1024) {
        for (int base = 1024; base < k4n; base += 1024)
            stage_x_round<PREC, M, VEC4>(p, xs4, lds_row, tid, base);
    }
}

template <int PREC, int SM, int M, int R, bool ZP>
__global__ __launch_bounds__(256) void gemv_valu(const KParams p) {
    constexpr int CE = PREC == 8 ? 16 : 32;  // elements per 16-byte chunk
    constexpr int CS = CE + 4;               // padded LDS floats per chunk
    constexpr int V = pow2_ceil(M * R);      // values per lane to reduce
    extern __shared__ float4 xs4[];          // float4-typed: x reads are ds_read_b128

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int GW = gridDim.x * 4;
    const int gw = blockIdx.x * 4 + wave;
    const int nrg = p.Np / R;
    const int iters = (p.chunks + 63) >> 6;  // chunk iterations per row group
    const int items = gw < nrg ? ((nrg - gw + GW - 1) / GW) * iters : 0;
    const int lds_row = p.chunks * CS;

    // ---- weight (and K-group scale) loads of one work item
    u32x4 wc[R], wn[R];
    float sc[R], sn[R], zc[R], zn[R];
    auto load_item = [&](int t, u32x4 (&w)[R], float (&s)[R], float (&z)[R]) {
        const int rg = gw + (t / iters) * GW;
        int c = lane + 64 * (t % iters);
        c = c < p.chunks ? c : p.chunks - 1;  // idle lanes re-read a valid chunk
        const uint8_t *base = p.data + (int64_t)rg * R * p.row_bytes + (int64_t)c * 16;
#pragma unroll
        for (int r = 0; r < R; ++r)
            w[r] = __builtin_nontemporal_load((const u32x4 *)(base + (int64_t)r * p.row_bytes));
        if (SM == S_KGROUP) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int64_t gi = kgroup_index((int64_t)rg * R + r, c / p.cpg, p.G);
                s[r] = p.scales[gi];
                z[r] = ZP ? (float)p.zp[gi] : 0.0f;
            }
        }
    };
    if (items > 0) load_item(0, wc, sc, zc);

    // ---- stage x [M][Kp] into LDS (zero beyond K; INT4 16x slots pre-divided).
    if (p.x_vec4) stage_x<PREC, M, true>(p, xs4, lds_row, tid);
    else stage_x<PREC, M, false>(p, xs4, lds_row, tid);
    __syncthreads();

    const uint32_t kMagic = opaque(0x64006400u);
    const uint32_t kLo = opaque(PREC == 8 ? 0x00FF00FFu : 0x000F000Fu);
    const uint32_t kHi = opaque(0x00F000F0u);

    float acc[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

    for (int t = 0; t < items; ++t) {
        if (t + 1 < items) load_item(t + 1, wn, sn, zn);
        const int rg = gw + (t / iters) * GW;
        const int n0 = rg * R;
        const int c = lane + 64 * (t % iters);

        if (c < p.chunks) {
            if (PREC == 8) {
                h2 c8[R];
#pragma unroll
                for (int r = 0; r < R; ++r)
                    c8[r] = splat(-(1152.0f + (ZP ? (float)p.zp[n0 + r] : 0.0f)));
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    float4 xv[M];
#pragma unroll
                    for (int m = 0; m < M; ++m) xv[m] = xs4[(m * lds_row + c * CS + 4 * d) >> 2];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const uint32_t wv = wc[r][d];
                        const h2 p0 = as_h2(and_or(wv, kLo, kMagic)) + c8[r];
                        const h2 p1 = as_h2(and_or(wv >> 8, kLo, kMagic)) + c8[r];
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            float a = acc[m][r];
                            a = fmix(p0.x, xv[m].x, a);
                            a = fmix(p0.y, xv[m].y, a);
                            a = fmix(p1.x, xv[m].z, a);
                            a = fmix(p1.y, xv[m].w, a);
                            acc[m][r] = a;
                        }
                    }
                }
            } else {
                h2 c1[R], c16[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float z = (SM == S_KGROUP && ZP) ? zc[r] : 0.0f;
                    c1[r] = splat(-(1032.0f + z));
                    c16[r] = splat(-(1152.0f + 16.0f * z));
                }
                const float *tcol = nullptr;  // runtime layout: per-k scales of this N-block
                if (SM == S_NGROUP) tcol = p.scales + (int64_t)(n0 / p.rpn) * p.Kp + c * 32;
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
                        const float4 ta = *(const float4 *)&tcol[8 * d];
                        const float4 tb = *(const float4 *)&tcol[8 * d + 4];
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            xa[m].x *= ta.x; xa[m].y *= ta.y; xa[m].z *= ta.z; xa[m].w *= ta.w;
                            xb[m].x *= tb.x; xb[m].y *= tb.y; xb[m].z *= tb.z; xb[m].w *= tb.w;
                        }
                    }
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const uint32_t wv = wc[r][d];
                        const uint32_t w8 = wv >> 8;
                        const h2 p0 = as_h2(and_or(wv, kLo, kMagic)) + c1[r];
                        const h2 p1 = as_h2(and_or(wv, kHi, kMagic)) + c16[r];
                        const h2 p2 = as_h2(and_or(w8, kLo, kMagic)) + c1[r];
                        const h2 p3 = as_h2(and_or(w8, kHi, kMagic)) + c16[r];
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            float a = part[m][r];
                            a = fmix(p0.x, xa[m].x, a);
                            a = fmix(p0.y, xa[m].y, a);
                            a = fmix(p1.x, xa[m].z, a);
                            a = fmix(p1.y, xa[m].w, a);
                            a = fmix(p2.x, xb[m].x, a);
                            a = fmix(p2.y, xb[m].y, a);
                            a = fmix(p3.x, xb[m].z, a);
                            a = fmix(p3.y, xb[m].w, a);
                            part[m][r] = a;
                        }
                    }
                }
#pragma unroll
                for (int m = 0; m < M; ++m)
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        acc[m][r] = SM == S_KGROUP ? __builtin_fmaf(sc[r], part[m][r], acc[m][r])
                                                   : acc[m][r] + part[m][r];
            }
        }

        if (t % iters == iters - 1) {
            // row group done: reduce across the wave and write
            float v[V];
#pragma unroll
            for (int i = 0; i < V; ++i) v[i] = i < M * R ? acc[i / R][i % R] : 0.0f;
            const float tot = reduce_multi<V>(v, lane);
            const int idx = reduce_index<V>(lane);
            if ((lane & (64 / V - 1)) == 0 && idx < M * R) {
                const int m = idx / R, n = n0 + idx % R;
                if (n < p.N) p.y[(int64_t)m * p.ldy + n] = SM == S_ROW ? tot * p.scales[n] : tot;
            }
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            wc[r] = wn[r];
            sc[r] = sn[r];
            zc[r] = zn[r];
        }
    }
}

// A wave-uniform element offset pinned in scalar registers: loads then take
// the form base (SGPR pair) + 32-bit lane offset, instead of the compiler
// folding the row offset into per-lane 64-bit multiply-adds.
__device__ __forceinline__ int64_t uniform_offset(int64_t v) {
    asm volatile("" : "+s"(v));
    return v;
}

// Workgroup barrier that orders LDS only: it does not wait for the global
// loads still in flight, which a full __syncthreads() fence would.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---- burst kernel: every load of a wave in flight at once -----------------
//
// A wave owns U consecutive rows and reads all of them -- I 16-byte chunks
// per row and lane, chunk c = lane + 64 i -- with loads issued back to back
// at kernel start, ahead of any compute (U * I <= 16, so at most 64 VGPRs of
// weights per lane).  The x loads go out first; x is written to LDS while
// the weight loads are still in flight, behind a barrier that waits for LDS
// only.  Compute then consumes the chunks in issue order, so each wait is
// for the oldest outstanding load.  The grid is not persistent: one wave
// per U rows, so a launch issues the whole matrix's reads in its first
// microsecond when it fits the GPU, and HBM latency is paid about once.
// INT8 rows (one scale per row) and INT4 K-groups without zero points; and
// INT4 with groups along N (the runtime layout, NG > 0): rows of one N-block
// share a scale per k, so the block stages x times that scale row in LDS and
// the rows need no scale of their own.  NG = 1: the block's rows lie in one
// N-block; NG = 2 (M = 1): rows alternate between two interleaved weights
// (gate and up rows), the block stages one scaled copy of x for each, and
// row u reads copy u & 1.
//
// WV waves per block; KS = 2 splits every row's chunks between two waves of
// the block (wave w takes row group w % (WV / 2) and chunk iterations
// I (w / (WV / 2)) .. I (w / (WV / 2)) + I - 1), and the upper part's wave
// totals are added to the lower part's through LDS, lower + upper, in the
// same launch.  A long row then takes half its chunk iterations in each of
// two waves of four rows, instead of all of them in one wave of two rows:
// every x chunk a wave reads from LDS serves four rows, and an INT4 row
// quad's four scales come in one load.  A block stages all of x once
// whatever its K split.
template <int PREC, int M, int U, int I, int PRO, int EPI, int NG, int WV = 4, int KS = 1>
__global__ __launch_bounds__(64 * WV) void gemv_burst(const KParams p) {
    constexpr int CE = PREC == 8 ? 16 : 32;
    constexpr int CS = CE + 4;
    constexpr int V = M * U;           // M and U are powers of two
    constexpr int NT = 64 * WV;        // threads per block
    constexpr int RG = WV / KS;        // row groups per block
    constexpr int XR = 16 * I * KS * CE / NT;  // float4 x loads per thread and x row
    constexpr int XC = NG == 2 ? 2 : M;   // x copies in LDS
    static_assert(PRO == PRO_NONE || M == 1, "fused prologues take one x row");
    static_assert(NG == 0 || PREC == 4, "groups along N are INT4 only");
    static_assert(NG != 2 || (M == 1 && U % 2 == 0), "interleaved pairs: one x row, whole pairs per wave");
    static_assert((WV == 4 || WV == 8) && (KS == 1 || KS == 2), "four or eight waves, one or two K parts");
    static_assert(XR * NT == 16 * I * KS * CE, "whole float4 x loads per thread");
    extern __shared__ float4 xs4[];
    __shared__ float red[WV];
    __shared__ float upper_tot[KS > 1 ? RG * 64 : 1];

    constexpr int lds_row = 64 * I * KS * CS;  // LDS floats per x row: every slot the loads cover
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps r0 scalar
    const int part = KS == 1 ? 0 : wave / RG;   // K part of this wave
    const int grp = KS == 1 ? wave : wave % RG;  // row group of this wave
    const int r0 = (blockIdx.x * RG + grp) * U;

    // ---- 1. x loads (16-byte aligned rows, K % 4 == 0; clamped addresses,
    // zeroed beyond K).  No branches before the weight loads: a branch merge
    // makes the compiler wait for every load issued before it.
    float4 xv[M][XR];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float *xr = p.x + (int64_t)(M == 1 ? 0 : min(m, p.m_act - 1)) * p.ldx;
#pragma unroll
        for (int r = 0; r < XR; ++r) {
            const int k = 4 * (tid + NT * r);
            const float4 t = *(const float4 *)(xr + min(k, p.K - 4));  // x_vec4 holds
            const bool in = k < p.K;
            xv[m][r] = float4{in ? t.x : 0.f, in ? t.y : 0.f, in ? t.z : 0.f, in ? t.w : 0.f};
        }
    }
    // NG: this block's per-k scale row(s), [Kp] each, read like x
    float4 tv[NG == 2 ? 2 : 1][XR];
    if constexpr (NG > 0) {
        const int rb = blockIdx.x * RG * U;   // the block's first row
#pragma unroll
        for (int c = 0; c < (NG == 2 ? 2 : 1); ++c) {
            const int nb = NG == 2 ? c * p.nb_half + min((rb >> 1) / p.rpn, p.nb_half - 1) : rb / p.rpn;
            const float *tr = p.scales + (int64_t)nb * p.Kp;
#pragma unroll
            for (int r = 0; r < XR; ++r) {
                const int k = 4 * (tid + NT * r);
                tv[c][r] = *(const float4 *)(tr + min(k, p.Kp - 4));   // beyond Kp: x is zero
            }
        }
    }
    float4 av[XR];  // PRO_RMSNORM: g
    if constexpr (PRO == PRO_RMSNORM) {
#pragma unroll
        for (int r = 0; r < XR; ++r) {
            const int k = 4 * (tid + NT * r);
            const float4 t = *(const float4 *)(p.g + min(k, p.K - 4));
            const bool in = k < p.K;
            av[r] = float4{in ? t.x : 0.f, in ? t.y : 0.f, in ? t.z : 0.f, in ? t.w : 0.f};
        }
    }

    // ---- 2. all weight (and scale) loads of the wave, in consumption order.
    // Row and quad base addresses are wave-uniform (scalar registers); a lane
    // adds only its chunk offset, so no 64-bit address math lands on the VALU.
    u32x4 w[I][U];
    float s[I][U];
#pragma unroll
    for (int i = 0; i < I; ++i) {
        const int c = min(lane + 64 * (part * I + i), p.chunks - 1);  // idle lanes re-read a valid chunk
        // a shift, not a division: a per-lane integer division here delays
        // every wave's first loads (measured 9.7 -> 9.0 us on 32000x2048)
        const int g = c >> p.cpg_shift;
        if constexpr (PREC == 4 && NG == 0 && U >= 4) {
            // a row quad's four scales of group g in one 16-byte load, issued
            // ahead of the quad's weights so the first row need not wait for
            // the last load of the wave
#pragma unroll
            for (int q = 0; q < U / 4; ++q) {
                const int quad = min(r0 + 4 * q, p.Np - 4);  // r0 is a multiple of 4
                const float *sq = p.scales + uniform_offset((int64_t)(quad >> 2) * p.G * 4);
                const f32x4 sv = __builtin_nontemporal_load((const f32x4 *)(sq + (uint32_t)(4 * g)));
                s[i][4 * q] = sv.x;
                s[i][4 * q + 1] = sv.y;
                s[i][4 * q + 2] = sv.z;
                s[i][4 * q + 3] = sv.w;
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the scale loads first
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int row = min(r0 + u, p.Np - 1);
            const uint8_t *rp = p.data + uniform_offset((int64_t)row * p.row_bytes);
            w[i][u] = __builtin_nontemporal_load((const u32x4 *)(rp + (uint32_t)(16 * c)));
            if (PREC == 4 && NG == 0 && U < 4)
                s[i][u] = p.scales[(int64_t)(row >> 2) * p.G * 4 + (row & 3) + 4 * g];  // kgroup_index
        }
    }
    const int ridx = reduce_index<V>(lane);  // value this lane holds after the reduce
    const float rs = PREC == 8 ? p.scales[min(r0 + ridx % U, p.Np - 1)] : 0.0f;
    const float yin = EPI == EPI_ACCUMULATE ? p.y[min(r0 + ridx % U, p.N - 1)] : 0.0f;
    // Nothing that consumes a load may be scheduled above this point.
    __builtin_amdgcn_sched_barrier(0);

    // ---- decode-step duties of block 0: keep x as given (the step's
    // residual stream when x is an embedding row) and advance the position
    // (no other launch of the step is running)
    if constexpr (M == 1) {
        if (p.xcopy != nullptr && blockIdx.x == 0) {
#pragma unroll
            for (int r = 0; r < XR; ++r) {
                const int k = 4 * (tid + NT * r);
                if (k < p.K) *(float4 *)(p.xcopy + k) = xv[0][r];
            }
        }
    }
    if (p.advance != nullptr && blockIdx.x == 0 && tid == 0) p.advance[0] += 1;

    // ---- fused prologue: x <- rmsnorm(x) * g (reference order of
    // operations: Tensor.swift:1543-1556)
    if constexpr (PRO == PRO_RMSNORM) {
        float ss = 0.0f;
#pragma unroll
        for (int r = 0; r < XR; ++r)
            ss += xv[0][r].x * xv[0][r].x + xv[0][r].y * xv[0][r].y + xv[0][r].z * xv[0][r].z +
                  xv[0][r].w * xv[0][r].w;
        ss = wave::sum(ss);   // DPP and readlane: no LDS round trip per step
        if (lane == 0) red[wave] = ss;
        lds_barrier();
        ss = (red[0] + red[1]) + (red[2] + red[3]);
        if constexpr (WV == 8) ss += (red[4] + red[5]) + (red[6] + red[7]);
        const float inv = 1.0f / __builtin_sqrtf(ss / (float)p.K + p.eps);
#pragma unroll
        for (int r = 0; r < XR; ++r) {
            xv[0][r].x = xv[0][r].x * inv * av[r].x;
            xv[0][r].y = xv[0][r].y * inv * av[r].y;
            xv[0][r].z = xv[0][r].z * inv * av[r].z;
            xv[0][r].w = xv[0][r].w * inv * av[r].w;
        }
    }

    // ---- 3. x -> LDS (INT4 slots k % 4 in {2, 3} pre-divided by 16).  The
    // stores are unconditional (zeros beyond K): a conditional store would let
    // the compiler sink its x load behind the weight loads.
#pragma unroll
    for (int m = 0; m < XC; ++m)
#pragma unroll
        for (int r = 0; r < XR; ++r) {
            const int k = 4 * (tid + NT * r);
            float4 t = xv[NG == 2 ? 0 : m][r];
            if constexpr (NG > 0) {
                const float4 sc = tv[NG == 2 ? m : 0][r];
                t = float4{t.x * sc.x, t.y * sc.y, t.z * sc.z, t.w * sc.w};
            }
            if (PREC == 4) { t.z *= 0.0625f; t.w *= 0.0625f; }
            xs4[(m * lds_row + lds_index<CE>(k)) >> 2] = t;
        }
    lds_barrier();
    // idle wave of the last block (after the barrier); with a K split every
    // wave reaches the second barrier below (an idle one computes on clamped,
    // valid rows and stores nothing)
    if (KS == 1 && r0 >= p.Np) return;

    // ---- 4. unpack and accumulate, chunk by chunk in issue order: the x
    // elements of chunk c are read from LDS once, then every row's chunk is
    // finished as soon as its load has landed.
    const uint32_t kMagic = opaque(0x64006400u);
    const uint32_t kLo = opaque(PREC == 8 ? 0x00FF00FFu : 0x000F000Fu);
    const uint32_t kHi = opaque(0x00F000F0u);
    float acc[M][U];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int u = 0; u < U; ++u) acc[m][u] = 0.0f;

#pragma unroll
    for (int i = 0; i < I; ++i) {
        const int c = lane + 64 * (part * I + i);
        const bool has = (KS == 1 && i < I - 1) || c < p.chunks;
        if constexpr (M >= 8) {
            // eight x rows: each row's chunk is unpacked once into f16
            // pairs, then the x rows are taken one at a time (all eight
            // rows' x chunks at once would not fit the registers)
            if (has) {
                constexpr int XQ = CE / 4;
                constexpr int NPAIR = CE / 2;   // f16 pairs per chunk
                h2 ph[U][NPAIR];
#pragma unroll
                for (int u = 0; u < U; ++u)
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t wv = w[i][u][d];
                        if (PREC == 8) {
                            const h2 c8 = splat(-1152.0f);
                            ph[u][2 * d] = as_h2(and_or(wv, kLo, kMagic)) + c8;
                            ph[u][2 * d + 1] = as_h2(and_or(wv >> 8, kLo, kMagic)) + c8;
                        } else {
                            const h2 c1 = splat(-1032.0f), c16 = splat(-1152.0f);
                            const uint32_t w8 = wv >> 8;
                            ph[u][4 * d] = as_h2(and_or(wv, kLo, kMagic)) + c1;
                            ph[u][4 * d + 1] = as_h2(and_or(wv, kHi, kMagic)) + c16;
                            ph[u][4 * d + 2] = as_h2(and_or(w8, kLo, kMagic)) + c1;
                            ph[u][4 * d + 3] = as_h2(and_or(w8, kHi, kMagic)) + c16;
                        }
                    }
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    float4 xq[XQ];
#pragma unroll
                    for (int q = 0; q < XQ; ++q) xq[q] = xs4[(m * lds_row + c * CS + 4 * q) >> 2];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        float a0 = PREC == 8 ? acc[m][u] : 0.0f, a1 = 0.0f;
#pragma unroll
                        for (int d = 0; d < 4; ++d) {
                            if (PREC == 8) {
                                const h2 p0 = ph[u][2 * d], p1 = ph[u][2 * d + 1];
                                a0 = fmix(p0.x, xq[d].x, a0);
                                a1 = fmix(p1.x, xq[d].z, a1);
                                a0 = fmix(p0.y, xq[d].y, a0);
                                a1 = fmix(p1.y, xq[d].w, a1);
                            } else {
                                const h2 p0 = ph[u][4 * d], p1 = ph[u][4 * d + 1];
                                const h2 p2 = ph[u][4 * d + 2], p3 = ph[u][4 * d + 3];
                                const float4 xa = xq[2 * d], xb = xq[2 * d + 1];
                                a0 = fmix(p0.x, xa.x, a0);
                                a1 = fmix(p2.x, xb.x, a1);
                                a0 = fmix(p0.y, xa.y, a0);
                                a1 = fmix(p2.y, xb.y, a1);
                                a0 = fmix(p1.x, xa.z, a0);
                                a1 = fmix(p3.x, xb.z, a1);
                                a0 = fmix(p1.y, xa.w, a0);
                                a1 = fmix(p3.y, xb.w, a1);
                            }
                        }
                        if (PREC == 8) acc[m][u] = a0 + a1;
                        else acc[m][u] = NG > 0 ? acc[m][u] + (a0 + a1)
                                                : __builtin_fmaf(s[i][u], a0 + a1, acc[m][u]);
                    }
                }
            }
        } else if (has) {
            constexpr int XQ = CE / 4;  // float4 of x per chunk and x row
            float4 xq[XC][XQ];
#pragma unroll
            for (int m = 0; m < XC; ++m)
#pragma unroll
                for (int q = 0; q < XQ; ++q) xq[m][q] = xs4[(m * lds_row + c * CS + 4 * q) >> 2];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (PREC == 8) {
                    const h2 c8 = splat(-1152.0f);
                    // two interleaved FMA chains per row: back-to-back dependent
                    // v_fma_mix_f32 would need a wait state each
                    float a0[M], a1[M];
#pragma unroll
                    for (int m = 0; m < M; ++m) { a0[m] = acc[m][u]; a1[m] = 0.0f; }
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t wv = w[i][u][d];
                        const h2 p0 = as_h2(and_or(wv, kLo, kMagic)) + c8;
                        const h2 p1 = as_h2(and_or(wv >> 8, kLo, kMagic)) + c8;
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            a0[m] = fmix(p0.x, xq[m][d].x, a0[m]);
                            a1[m] = fmix(p1.x, xq[m][d].z, a1[m]);
                            a0[m] = fmix(p0.y, xq[m][d].y, a0[m]);
                            a1[m] = fmix(p1.y, xq[m][d].w, a1[m]);
                        }
                    }
#pragma unroll
                    for (int m = 0; m < M; ++m) acc[m][u] = a0[m] + a1[m];
                } else {
                    const h2 c1 = splat(-1032.0f), c16 = splat(-1152.0f);
                    // two interleaved FMA chains per row (see INT8)
                    float a0[M], a1[M];
#pragma unroll
                    for (int m = 0; m < M; ++m) { a0[m] = 0.0f; a1[m] = 0.0f; }
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t wv = w[i][u][d];
                        const uint32_t w8 = wv >> 8;
                        const h2 p0 = as_h2(and_or(wv, kLo, kMagic)) + c1;
                        const h2 p1 = as_h2(and_or(wv, kHi, kMagic)) + c16;
                        const h2 p2 = as_h2(and_or(w8, kLo, kMagic)) + c1;
                        const h2 p3 = as_h2(and_or(w8, kHi, kMagic)) + c16;
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            const int xc = NG == 2 ? (u & 1) : m;   // r0 is even: row r0 + u is a gate row when u is
                            const float4 xa = xq[xc][2 * d], xb = xq[xc][2 * d + 1];
                            a0[m] = fmix(p0.x, xa.x, a0[m]);
                            a1[m] = fmix(p2.x, xb.x, a1[m]);
                            a0[m] = fmix(p0.y, xa.y, a0[m]);
                            a1[m] = fmix(p2.y, xb.y, a1[m]);
                            a0[m] = fmix(p1.x, xa.z, a0[m]);
                            a1[m] = fmix(p3.x, xb.z, a1[m]);
                            a0[m] = fmix(p1.y, xa.w, a0[m]);
                            a1[m] = fmix(p3.y, xb.w, a1[m]);
                        }
                    }
#pragma unroll
                    for (int m = 0; m < M; ++m)
                        acc[m][u] = NG > 0 ? acc[m][u] + (a0[m] + a1[m])
                                           : __builtin_fmaf(s[i][u], a0[m] + a1[m], acc[m][u]);
                }
            }
        }
    }

    // ---- 5. reduce across the wave and write
    float v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = acc[j / U][j % U];
    float tot = reduce_multi<V>(v, lane);
    if constexpr (KS > 1) {
        // lower K part + upper K part, in that order
        if (part == 1) upper_tot[grp * 64 + lane] = tot;
        lds_barrier();
        if (part == 1) return;
        tot += upper_tot[grp * 64 + lane];
    }
    if constexpr (EPI == EPI_SILU_PAIR) {
        // value ridx ^ 1 (the pair's other row) sits at lane ^ (64 / V)
        static_assert(M == 1 && U >= 2, "pairs of rows within one wave");
        const float r = PREC == 8 ? tot * rs : tot;
        const float other = xchg<64 / V>(r);
        if ((lane & (64 / V - 1)) == 0 && (ridx & 1) == 0) {
            const int n = r0 + ridx;
            if (n < p.N) p.y[n / 2] = (r / (1.0f + expf(-r))) * other;
        }
    } else if ((lane & (64 / V - 1)) == 0) {
        const int m = ridx / U, n = r0 + ridx % U;
        const float v = PREC == 8 ? tot * rs : tot;
        if (n < p.N && (M == 1 || m < p.m_act)) p.y[(int64_t)m * p.ldy + n] = EPI == EPI_ACCUMULATE ? yin + v : v;
    }
}

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

int env_int(const char *name, int dflt) {
    const char *v = std::getenv(name);
    return v && *v ? std::atoi(v) : dflt;
}

// Burst-kernel shapes: chunk iterations per row I <= kBurstMaxI, rows per
// wave U a power of two with U * I <= 16.  Eight x rows take rows of at most
// 2 x 64 chunks and up to 80 KB of LDS (two blocks per CU): eight staged x
// copies of 64 x I x (32 + 4) floats fit that for INT8 at I <= 2 (K <= 2048)
// but INT4 only at I = 1 (K <= 2048; I = 2 would need 144 KB).
constexpr int kBurstMaxI = 6;
constexpr int64_t kBurst8LdsBytes = 80 * 1024;

// Block layouts of the burst kernel: waves per block and K parts per row.
enum BurstLayout : int { kW4K1 = 0, kW4K2 = 1, kW8K2 = 2 };

template <int PREC, int M, int U, int I, int PRO, int EPI, int NG, int WV, int KS>
hipError_t launch_burst_one(const KParams &p, size_t lds, hipStream_t s) {
    if constexpr (U * I > 16 || M * U > 32 || (EPI == EPI_SILU_PAIR && (U < 2 || M != 1)) ||
                  (NG > 0 && PREC != 4) || (NG == 2 && (M != 1 || U % 2 != 0)) || (M == 8 && I > 2)) {
        return hipErrorInvalidValue;
    } else {
        constexpr int RG = WV / KS;   // row groups per block
        const int64_t waves = (p.Np + U - 1) / U;
        const unsigned blocks = (unsigned)((waves + RG - 1) / RG);
        hipLaunchKernelGGL((gemv_burst<PREC, M, U, I, PRO, EPI, NG, WV, KS>), dim3(blocks), dim3(64 * WV), lds, s,
                           p);
        return hipGetLastError();
    }
}

// K-split layouts are built for one x row and up to 3 chunk iterations per part
template <int PREC, int M, int U, int I, int PRO, int EPI, int NG>
hipError_t burst_layout(int kw, const KParams &p, size_t lds, hipStream_t s) {
    if (kw == kW4K1) return launch_burst_one<PREC, M, U, I, PRO, EPI, NG, 4, 1>(p, lds, s);
    if constexpr (M == 1 && I <= 3) {
        if (kw == kW4K2) return launch_burst_one<PREC, M, U, I, PRO, EPI, NG, 4, 2>(p, lds, s);
        if (kw == kW8K2) return launch_burst_one<PREC, M, U, I, PRO, EPI, NG, 8, 2>(p, lds, s);
    }
    return hipErrorInvalidValue;
}

template <int PREC, int M, int I, int PRO, int EPI, int NG>
hipError_t burst_u(int U, int kw, const KParams &p, size_t lds, hipStream_t s) {
    switch (U) {
    case 1: return burst_layout<PREC, M, 1, I, PRO, EPI, NG>(kw, p, lds, s);
    case 2: return burst_layout<PREC, M, 2, I, PRO, EPI, NG>(kw, p, lds, s);
    case 4: return burst_layout<PREC, M, 4, I, PRO, EPI, NG>(kw, p, lds, s);
    case 8: return burst_layout<PREC, M, 8, I, PRO, EPI, NG>(kw, p, lds, s);
    case 16: return burst_layout<PREC, M, 16, I, PRO, EPI, NG>(kw, p, lds, s);
    default: return hipErrorInvalidValue;
    }
}

template <int PREC, int M, int PRO, int EPI, int NG = 0>
hipError_t burst_i(int I, int U, int kw, const KParams &p, size_t lds, hipStream_t s) {
    switch (I) {
    case 1: return burst_u<PREC, M, 1, PRO, EPI, NG>(U, kw, p, lds, s);
    case 2: return burst_u<PREC, M, 2, PRO, EPI, NG>(U, kw, p, lds, s);
    case 3: return burst_u<PREC, M, 3, PRO, EPI, NG>(U, kw, p, lds, s);
    case 4: return burst_u<PREC, M, 4, PRO, EPI, NG>(U, kw, p, lds, s);
    case 5: return burst_u<PREC, M, 5, PRO, EPI, NG>(U, kw, p, lds, s);
    case 6: return burst_u<PREC, M, 6, PRO, EPI, NG>(U, kw, p, lds, s);
    default: return hipErrorInvalidValue;
    }
}

template <int PREC, int NG = 0>
hipError_t burst_m(int M, int I, int U, int kw, const KParams &p, size_t lds, hipStream_t s) {
    switch (M) {
    case 1: return burst_i<PREC, 1, PRO_NONE, EPI_STORE, NG>(I, U, kw, p, lds, s);
    case 2: return burst_i<PREC, 2, PRO_NONE, EPI_STORE, NG>(I, U, kw, p, lds, s);
    case 4: return burst_i<PREC, 4, PRO_NONE, EPI_STORE, NG>(I, U, kw, p, lds, s);
    case 8: return burst_i<PREC, 8, PRO_NONE, EPI_STORE, NG>(I, U, kw, p, lds, s);
    default: return hipErrorInvalidValue;
    }
}

// The fused decode variants (M = 1): the prologue / epilogue pairs a decode
// step uses.  Interleaved gate|up weights with groups along N take the
// two-copy form (NG = 2) of the pair epilogue.
template <int PREC, int NG = 0>
hipError_t burst_fused(int pro, int epi, int I, int U, int kw, const KParams &p, size_t lds, hipStream_t s) {
    if (NG < 2 && pro == PRO_RMSNORM && epi == EPI_STORE)
        return burst_i<PREC, 1, PRO_RMSNORM, EPI_STORE, NG>(I, U, kw, p, lds, s);
    if (NG < 2 && pro == PRO_NONE && epi == EPI_ACCUMULATE)
        return burst_i<PREC, 1, PRO_NONE, EPI_ACCUMULATE, NG>(I, U, kw, p, lds, s);
    if (NG != 1 && pro == PRO_RMSNORM && epi == EPI_SILU_PAIR)
        return burst_i<PREC, 1, PRO_RMSNORM, EPI_SILU_PAIR, NG>(I, U, kw, p, lds, s);
    return hipErrorInvalidValue;
}

}  // namespace

int64_t gemv_max_rows(const tbh_weight &w) {
    if (w.path == Path::Generic) return 0;
    for (int64_t m = 4; m >= 1; --m)
        if (lds_bytes_for(w, m) <= kMaxLdsBytes) return m;
    return 0;
}

namespace {

KParams make_params(const tbh_weight &w, const GemvArgs &a) {
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
    p.cpg_shift = -1;
    for (int sh = 0; sh < 31; ++sh)
        if (p.cpg > 0 && p.cpg == (1 << sh)) p.cpg_shift = sh;
    p.rpn = w.rows_per_nblock;
    p.nb_half = w.nb_half;
    p.x_vec4 = (w.K % 4 == 0 && a.ldx % 4 == 0 && ((uintptr_t)a.x & 15) == 0) ? 1 : 0;
    p.m_act = (int32_t)a.M;
    p.g = a.x;
    p.eps = 0.0f;
    return p;
}

// Burst kernel eligibility: M in {1, 2, 4}, no zero points, rows of at most
// 64 * kBurstMaxI chunks, INT4 K-groups of a power-of-two number of chunks,
// 16-byte aligned x rows with K % 4 == 0, x tile in LDS.  U: the largest power of two (U * I <= 16) that still leaves
// `waves_per_cu` waves per CU, so small matrices spread over the whole GPU
// and large ones keep up to 16 chunk loads in flight per lane.
bool burst_shape(const tbh_weight &w, const KParams &p, int M, int *I_out, int *U_out,
                 int64_t *lds_out, int *kw_out) {
    static const int kernel_sel = env_int("TBH_GEMV_PERSISTENT", 0);
    static const int burst_wpc = env_int("TBH_GEMV_WAVES_PER_CU", 16);
    static const int u_force = env_int("TBH_GEMV_U", 0);
    static const int ks_force = env_int("TBH_GEMV_KS", 0);
    static const int wv_force = env_int("TBH_GEMV_WV", 0);
    const int It = (p.chunks + 63) / 64;   // chunk iterations per row
    const int64_t cus = std::max(1, w.dev->cu_count);
    // K parts per row.  One x row with rows of five or six chunk iterations
    // (INT4 K > 8192, INT8 K > 4096), or of four with at least 32 rows per CU:
    // two waves per row, four rows per wave, when that still leaves 8 waves
    // per CU.  A wave then reads each staged x chunk for four rows, and the
    // waves of a long matrix hold 8-12 chunks each instead of 12-16 (us per
    // launch, one part / two: INT4 4096x11008 9.07-9.29 / 8.41-8.54, INT8
    // 11008x4096 10.0-10.8 / 9.50-9.77, INT4 8192x8192 11.07 / 10.26; INT8
    // 4096x4096, already two rows of 8 chunks per wave, 4.86 / 4.94; INT8
    // 2048x5632, too few rows, 3.97 / 4.01; rows of two or three iterations
    // no faster).
    int ks = 1, wv = 4;
    const bool split = ks_force == 2 || (ks_force == 0 && M == 1 && It >= 4 && w.Np / 4 >= 4 * cus &&
                                         (It >= 5 || w.Np / 4 >= 8 * cus));
    if (M == 1 && split && It >= 2 && (It + 1) / 2 <= 3) {
        ks = 2;
        wv = wv_force == 8 ? 8 : 4;
    }
    const int I = (It + ks - 1) / ks;     // chunk iterations per wave
    const int ce = w.precision == TBH_PREC_INT8 ? kInt8ChunkElems : kInt4ChunkElems;
    const bool ng = w.path == Path::Int4NGroup;
    const int copies = w.ng_pairs ? 2 : M;   // x copies the block stages in LDS
    const int64_t blds = (int64_t)copies * 64 * I * ks * (ce + 4) * (int64_t)sizeof(float);
    if (kernel_sel || !(M == 1 || M == 2 || M == 4 || M == 8) || w.zp != nullptr || It > kBurstMaxI ||
        !p.x_vec4 || blds > (M == 8 ? kBurst8LdsBytes : kMaxLdsBytes) || (M == 8 && It > 2) || !(w.path == Path::Int8Row || w.path == Path::Int4KGroup || ng) ||
        (w.path == Path::Int4KGroup && p.cpg_shift < 0) || w.mfma_tiles || (w.ng_pairs && M != 1) ||
        (ng && (p.rpn <= 0 || p.Kp % 4 != 0)))
        return false;
    // U * I <= 16 weight chunks per lane; M * U <= 32 values in the reduce
    int U = 1;
    if (M == 1 && ks == 2 && ks_force == 0) {
        U = 4;
    } else if (M == 1) {
        // one x row: four rows per wave once that still leaves >= 8 waves
        // per CU, else two (measured on every decode shape of the 1.1B and
        // 7B models and the four INT4 shapes: one row per wave is slower
        // even on 2048-row matrices, eight or more rows per wave slower
        // everywhere)
        if (4 * I <= 16 && w.Np / 4 >= 8 * cus) U = 4;
        else if (2 * I <= 16) U = 2;
        // ... and four (at most 8 chunks per lane) where that brings the
        // launch to at most one four-wave block per CU: one round of blocks
        // beat two or a partial second (us per launch, U = 2 / 4, graphs of
        // one shape: INT4 4096x2048 3.36 / 3.05, INT8 2560x2048 3.07 / 2.96
        // -- the 1.1B decode step's Q|K|V, 1828 -> 1850 tokens/s on one box).
        // Eight rows per wave also reached one round on INT4 5632x2048 and
        // 8192x2048 and read faster alone (3.80 -> 3.66, 4.17 -> 4.00 us), but
        // in the four-shape step 5632x2048 went 3.65-3.67 -> 3.76-3.79 us, so
        // the rule stops at four.
        if (!ng) {
            for (int u = U; u <= 4 && u * I <= 8; u *= 2) {
                if ((w.Np + 4 * u - 1) / (4 * u) <= cus) {
                    U = u;
                    break;
                }
            }
        }
    } else {
        // two or four x rows: at least two rows per wave (the block stages its
        // x rows once for 4 U weight rows; us per launch, U = 1 / 2, M = 2
        // and 4: INT4 5632x2048 4.49 / 4.35, 6.69 / 5.61; INT8 5632x2048
        // 4.69 / 4.42, 6.80 / 5.67; INT4 2048x2048 3.16 / 3.11, 4.08 / 3.78),
        // more while that still leaves burst_wpc waves per CU (INT4
        // 32000x2048 at M = 4: U = 4 16.8 us, U = 2 19.5)
        if (2 * I <= 16) U = 2;
        while (2 * U * I <= 16 && 2 * U * M <= 32 && w.Np / (2 * U) >= burst_wpc * cus) U *= 2;
    }
    if (u_force > 0 && u_force * I <= 16 && u_force * M <= 32 && (u_force & (u_force - 1)) == 0) U = u_force;
    if (ng) {
        // a block's 4 U rows (2 U rows of each weight when interleaved) lie
        // in one N-block of the scale table.  Eight rows per wave make a
        // block cover a 32-row N-block, so each scale row is read by one
        // block instead of two (runtime layout, us per launch U = 4 / 8:
        // 32000x2048 10.30 / 9.25, 5632x2048 4.19 / 4.00; 2048x2048 3.13 /
        // 3.52 with too few waves)
        if (u_force == 0 && M == 1 && !w.ng_pairs && 8 * I <= 16 && p.rpn % 32 == 0 && w.Np >= 4096) U = 8;
        if (w.ng_pairs) U = std::max(U, 2);
        const int rg = wv / ks;   // row groups per block
        const int per_block = w.ng_pairs ? rg / 2 : rg;
        while (U > 1 && p.rpn % (per_block * U) != 0) U /= 2;
        if (p.rpn % (per_block * U) != 0 || (w.ng_pairs && U < 2) || U * I > 16) return false;
    }
    *I_out = I;
    *U_out = U;
    *lds_out = blds;
    *kw_out = ks == 1 ? kW4K1 : wv == 4 ? kW4K2 : kW8K2;
    return true;
}

}  // namespace

bool gemv8_supported(const tbh_weight &w, const float *x, int64_t ldx) {
    if (w.ng_pairs) return false;
    GemvArgs a{x, ldx, nullptr, w.N, 8};
    KParams p = make_params(w, a);
    int I, U, kw;
    int64_t lds;
    return burst_shape(w, p, 8, &I, &U, &lds, &kw);
}

bool gemv_fused_supported(const tbh_weight &w) {
    GemvArgs a{nullptr, w.K, nullptr, w.N, 1};
    KParams p = make_params(w, a);
    p.x_vec4 = w.K % 4 == 0;  // the caller's buffers are 16-byte aligned
    int I, U, kw;
    int64_t lds;
    return burst_shape(w, p, 1, &I, &U, &lds, &kw);
}

hipError_t launch_gemv_fused(const tbh_weight &w, const FusedGemvArgs &f, hipStream_t s) {
    GemvArgs a{f.x, w.K, f.y, w.N, 1};
    KParams p = make_params(w, a);
    p.g = f.g ? f.g : f.x;
    p.eps = f.eps;
    p.xcopy = f.x_copy;
    p.advance = f.advance;
    if (f.g && ((uintptr_t)f.g & 15)) return hipErrorInvalidValue;
    int I, U, kw;
    int64_t lds;
    if (!burst_shape(w, p, 1, &I, &U, &lds, &kw)) return hipErrorInvalidValue;
    if (f.epilogue == EPI_SILU_PAIR) {
        if (w.N % 2 != 0 || 2 * I > 16) return hipErrorInvalidValue;
        U = std::max(U, 2);   // both rows of a pair in one wave
    }
    if (w.ng_pairs != (f.epilogue == EPI_SILU_PAIR && w.path == Path::Int4NGroup)) return hipErrorInvalidValue;
    if (w.precision == TBH_PREC_INT8) return burst_fused<8>(f.prologue, f.epilogue, I, U, kw, p, (size_t)lds, s);
    if (w.path == Path::Int4NGroup)
        return w.ng_pairs ? burst_fused<4, 2>(f.prologue, f.epilogue, I, U, kw, p, (size_t)lds, s)
                          : burst_fused<4, 1>(f.prologue, f.epilogue, I, U, kw, p, (size_t)lds, s);
    return burst_fused<4>(f.prologue, f.epilogue, I, U, kw, p, (size_t)lds, s);
}

hipError_t launch_gemv(const tbh_weight &w, const GemvArgs &a, hipStream_t s) {
    const int M = (int)a.M;
    if (M >= 5 && M <= 8 && !w.ng_pairs) {   // the eight-row burst kernel only (rows past M masked)
        KParams p = make_params(w, a);
        int I, U, kw;
        int64_t blds;
        if (!burst_shape(w, p, 8, &I, &U, &blds, &kw)) return hipErrorInvalidValue;
        if (w.path == Path::Int8Row) return burst_m<8>(8, I, U, kw, p, (size_t)blds, s);
        return w.path == Path::Int4NGroup ? burst_m<4, 1>(8, I, U, kw, p, (size_t)blds, s)
                                          : burst_m<4>(8, I, U, kw, p, (size_t)blds, s);
    }
    if (M < 1 || M > 4 || w.ng_pairs) return hipErrorInvalidValue;
    const int64_t lds = lds_bytes_for(w, M);
    if (lds > kMaxLdsBytes) return hipErrorInvalidValue;
    KParams p = make_params(w, a);
    const int64_t cus = std::max(1, w.dev->cu_count);
    {
        // three rows on the four-row burst kernel, the fourth masked
        // (us per launch, VALU kernel at M = 3 / burst at M = 4: INT4
        // 2048x2048 4.48 / 3.61-3.78, 5632x2048 6.16 / 5.59)
        const int Mb = M == 3 ? 4 : M;
        int I, U, kw;
        int64_t blds;
        if (burst_shape(w, p, Mb, &I, &U, &blds, &kw)) {
            if (w.path == Path::Int8Row) return burst_m<8>(Mb, I, U, kw, p, (size_t)blds, s);
            return w.path == Path::Int4NGroup ? burst_m<4, 1>(Mb, I, U, kw, p, (size_t)blds, s)
                                              : burst_m<4>(Mb, I, U, kw, p, (size_t)blds, s);
        }
    }

    // Persistent grid: a few 4-wave blocks per CU.  Rows per wave (R): as
    // many as still give every wave work, within the register budget
    // (M*R <= 16) and dividing the N-block height of the runtime layout.
    static const int bpc = env_int("TBH_GEMV_BLOCKS_PER_CU", 2);
    static const int r_force = env_int("TBH_GEMV_ROWS", 0);
    const int64_t max_blocks = bpc * cus;
    int R = 8;
    while (R > 1 && (w.Np / R < 4 * max_blocks || M * R > 16 ||
                     (w.path == Path::Int4NGroup && p.rpn % R != 0) || (M > 2 && R > 4)))
        R /= 2;
    if (r_force > 0 && M * r_force <= 16 && !(M > 2 && r_force > 4) && w.Np % r_force == 0 &&
        !(w.path == Path::Int4NGroup && p.rpn % r_force != 0))
        R = r_force;
    const int64_t groups = w.Np / R;
    const int blocks = (int)std::max<int64_t>(1, std::min((groups + 3) / 4, max_blocks));
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

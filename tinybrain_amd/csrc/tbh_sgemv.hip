// tbh_sgemv.hip -- dequant-GEMV for 2..8 rows of x on the matrix cores,
// reading the K-contiguous row layout of INT4 K-group weights.
//
// Replaces the MSL kernel matmul_int4_dequant (Sources/TinyBrainMetal/
// Shaders/DequantINT4.metal:95-137) for M > 1, where the VALU kernel's
// multiply-adds grow with M and dominate: here the vector ALUs only unpack
// weights and apply group scales, and one v_mfma_f32_16x16x32_f16 serves all
// M rows of x at once.
//
// Operands of one MFMA (16 weight rows n x one 32-element K chunk = one
// K-group slice, so one group scale per row and MFMA):
//   A (x): row 2m + h carries piece h of x[m] (h = 0: hi, 1: lo), split in
//     f16 after scaling by 2^-e_m, where 2^-e_m brings the block's max
//     |x[m]| into [2^14, 2^15) (rows whose max is below 2^-113 into
//     [2, 2^14)): hi + lo hold 22 significant bits relative to that max, no
//     overflow.  INT4 slots k % 8 in {2, 3, 6, 7} are pre-divided by
//     16 (the unpack leaves 16 * q there).  Rows >= 2M are never read back.
//     M is 2..8; an odd M leaves the last lane pair's second row unused.
//   B (weights): lane (n, kb) holds K sub-block kb of the chunk for row n as
//     f16 q (exact): the nibbles are OR-ed into the f16 magic 0x6400 and one
//     v_pk_add_f16 subtracts the offset, as in the VALU kernel.
//   C: lane (n, g) holds rows 4g..4g+3 of column n: x rows 2g and 2g + 1,
//     hi and lo.  y[m][n] = 2^e_m * sum over chunks of s[n][chunk] * (C_hi + C_lo).
// Every product q * x_piece is exact in fp32 and accumulates in fp32.
//
// Data movement: lane (n, r) of a wave loads chunk c + r of its row n (16
// bytes, 32 K elements; a load instruction covers 64 contiguous bytes of 16
// rows) together with that chunk's scale; a 4 x 4 transpose of 32-bit words
// across the wave's four 16-lane rows (v_permlane32_swap, v_permlane16_swap)
// then gives lane (n, kb) word kb of chunks c .. c + 3 -- one B operand per
// MFMA -- and all four scales.  The x fragments of the block's K range are
// built in LDS and shared by the block's eight waves; the weight loads run
// two steps ahead of the MFMAs, the first two issued right behind the x
// loads so that they land while x is staged (a wave that issues all of its
// loads at once sits at the issue until most of them are accepted, then
// computes every step after the data has arrived).  Small N is split along K over blocks; a
// second kernel adds the splits in split order (deterministic).
#include <cmath>
#include <cstdlib>

#include "tbh_internal.h"
#include "tbh_wave.h"

namespace tbh {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 128;      // weight rows per block: 8 waves x 16
constexpr int kWaves = 8;
constexpr int kStepChunks = 4;  // chunks per step: one per 16-lane row of a wave
constexpr int kXUnits = 8;      // x float4 units per thread (M * kchunks * 8 <= 512 * kXUnits)
// f16 per LDS fragment row: 32 + 8 of padding.  These 80-byte rows leave
// the A fragment reads (lane l: row l % 16, 16-byte column l / 16) 2-way
// bank-conflicted on gfx950; 96-byte rows measured conflict-free but no
// faster (M = 4, 8 and the 7B projection set within noise: the kernel waits
// on its weight stream), so the smaller LDS footprint stays.
constexpr int kFragRow = 40;

struct SParams {
    const float *x;
    int64_t ldx;
    float *y;
    int64_t ldy;
    float *part;              // splits > 1: [splits][M][N]
    const uint8_t *data;
    int64_t row_bytes;
    const float *scales;      // row quads [Np / 4][G][4]
    int32_t K, N, Np, G;
    int32_t cpg_shift;        // log2(chunks per group)
    int32_t chunks;           // 32-element chunks per row
    int32_t kchunks;          // chunks per block: 4 NS, a multiple of 16, at most 64
    int32_t splits;
};

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

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// B operand of one INT4 word (8 nibbles at bit offsets 0,16,4,20,8,24,12,28):
// f16 q for k % 8 in {0, 1, 4, 5}, 16 q for {2, 3, 6, 7}.
__device__ __forceinline__ half8 unpack_int4(uint32_t w, uint32_t magic, uint32_t lo, uint32_t hi, h2 c1,
                                             h2 c16) {
    const uint32_t w8 = w >> 8;
    const h2 p0 = as_h2((w & lo) | magic) + c1;
    const h2 p1 = as_h2((w & hi) | magic) + c16;
    const h2 p2 = as_h2((w8 & lo) | magic) + c1;
    const h2 p3 = as_h2((w8 & hi) | magic) + c16;
    half8 r;
    r[0] = p0.x; r[1] = p0.y; r[2] = p1.x; r[3] = p1.y;
    r[4] = p2.x; r[5] = p2.y; r[6] = p3.x; r[7] = p3.y;
    return r;
}

// 4 x 4 transpose of 32-bit words across the four 16-lane rows of a wave:
// row r of v[w] holds X[r][w] before and X[w][r] after (two
// v_permlane32_swap, two v_permlane16_swap).
__device__ __forceinline__ void transpose4(uint32_t (&v)[4]) {
    auto a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);  // rows 2,3 of v0 <-> rows 0,1 of v2
    auto b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
    auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);  // odd rows of v0 <-> even rows of v1
    auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    v[0] = c[0];
    v[1] = c[1];
    v[2] = d[0];
    v[3] = d[1];
}

template <int M, int NS, int D>
__global__ __launch_bounds__(512) void sgemv_int4(const SParams p) {
    constexpr int R2 = 2 * M;                 // A rows in use
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    // [kchunks][R2][kFragRow] f16 x fragments | [M] fp32 2^e | [8][M] row maxima
    _Float16 *frag = (_Float16 *)smem;
    float *pe = (float *)(smem + (size_t)kStepChunks * NS * R2 * kFragRow * 2);
    float *red = pe + M;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int split = blockIdx.x % p.splits, nb = blockIdx.x / p.splits;
    const int cb = split * kStepChunks * NS;  // first chunk of this block
    const int n = lane & 15, g = lane >> 4;
    const int row0 = nb * kRows + wave * 16;
    const int row = min(row0 + n, p.Np - 1);  // rows past Np re-read the last row (never stored)

    // ---- 1. x loads (unit u = (m, chunk, float4 q), zero beyond K)
    constexpr int KC = kStepChunks * NS;     // chunks of this block (= p.kchunks)
    constexpr int units = M * KC * 8;
    float4 xv[kXUnits];
#pragma unroll
    for (int i = 0; i < kXUnits; ++i) {
        const int u = min(tid + 512 * i, units - 1);
        const int m = u / (KC * 8), rest = u % (KC * 8);
        const int k = 32 * cb + 4 * rest;   // rest = local chunk * 8 + q
        const float4 t = *(const float4 *)(p.x + (int64_t)m * p.ldx + min(k, p.K - 4));
        const bool in = k < p.K;
        xv[i] = float4{in ? t.x : 0.f, in ? t.y : 0.f, in ? t.z : 0.f, in ? t.w : 0.f};
    }

    // ---- 2. weight and scale loads, D steps ahead of their use: lane (n, r)
    // takes chunk cb + 4 t + r of row n for step t.  Chunks past the row
    // re-read its last chunk and meet x = 0.  The first D steps go out right
    // behind the x loads, so they land while x is staged; the rest follow
    // one step at a time (a wave that issues every load of its range at once
    // stalls at the issue -- each load touches 16 rows' cache lines -- and
    // cannot compute meanwhile).
    const uint8_t *wrow = p.data + (int64_t)row * p.row_bytes;
    const float *srow = p.scales + (int64_t)(row >> 2) * p.G * 4 + (row & 3);
    u32x4 wr[D];
    float sr[D];
    auto load_step = [&](int t) {
        const int c = min(cb + kStepChunks * t + g, p.chunks - 1);
        wr[t % D] = __builtin_nontemporal_load((const u32x4 *)(wrow + 16 * c));
        sr[t % D] = srow[4 * (c >> p.cpg_shift)];
    };
#pragma unroll
    for (int t = 0; t < D && t < NS; ++t) load_step(t);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 3. x fragments: per-row exponent from the block's max |x[m]|
    // (each thread's units, then its wave by DPP, then the eight waves)
    float mx[M];
#pragma unroll
    for (int m = 0; m < M; ++m) mx[m] = 0.0f;
#pragma unroll
    for (int i = 0; i < kXUnits; ++i) {
        const int u = tid + 512 * i;
        if (512 * i < units && u < units) {
            const int m = u / (KC * 8);
            const float a = fmaxf(fmaxf(fabsf(xv[i].x), fabsf(xv[i].y)), fmaxf(fabsf(xv[i].z), fabsf(xv[i].w)));
#pragma unroll
            for (int mm = 0; mm < M; ++mm) mx[mm] = mm == m ? fmaxf(mx[mm], a) : mx[mm];
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float v = wave::max(mx[m]);
        if (lane == 0) red[wave * M + m] = v;
    }
    lds_barrier();
    float fm[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float a = red[m];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) a = fmaxf(a, red[w * M + m]);
        // 2^-e brings the row max a into [2^14, 2^15) from its exponent
        // field; e >= -127 keeps 2^-e finite (a below 2^-113, subnormal a
        // included, lands in [2, 2^14) instead); zero or non-finite rows: e = 0
        const int eb = (int)((__builtin_bit_cast(uint32_t, a) >> 23) & 0xFF);
        const int e = eb == 255 || a == 0.0f ? 0 : max(eb - 141, -127);
        fm[m] = __builtin_bit_cast(float, (uint32_t)(127 - e) << 23);
        if (tid == 0)   // 2^e: a normal float for e >= -126, the subnormal 2^-127 below
            pe[m] = __builtin_bit_cast(float, e >= -126 ? (uint32_t)(e + 127) << 23 : 0x00400000u);
    }
#pragma unroll
    for (int i = 0; i < kXUnits; ++i) {
        const int u = tid + 512 * i;
        if (512 * i < units && u < units) {
            const int m = u / (KC * 8), rest = u % (KC * 8);
            const int cl = rest >> 3, q = rest & 7;
            float f = fm[0];
#pragma unroll
            for (int mm = 1; mm < M; ++mm) f = mm == m ? fm[mm] : f;
            const float f16th = f * 0.0625f;
            const float v[4] = {xv[i].x * f, xv[i].y * f, xv[i].z * f16th, xv[i].w * f16th};
            half4 hi, lo;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const _Float16 h = (_Float16)v[j];
                hi[j] = h;
                lo[j] = (_Float16)(v[j] - (float)h);
            }
            _Float16 *fb = frag + ((size_t)cl * R2 + 2 * m) * kFragRow + 4 * q;
            *(half4 *)fb = hi;
            *(half4 *)(fb + kFragRow) = lo;
        }
    }
    lds_barrier();


    // ---- 4. per step: transpose, then per chunk j unpack, MFMA, scale
    const uint32_t kMagic = opaque(0x64006400u), kLo = opaque(0x000F000Fu), kHi = opaque(0x00F000F0u);
    const h2 c1 = splat(-1032.0f), c16 = splat(-1152.0f);
    const int arow = min(n, R2 - 1);          // A row of this lane (rows >= 2M: any row)
    const int m0 = 2 * g;                     // x rows of this lane's C values: m0, m0 + 1
    float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
    for (int t = 0; t < NS; ++t) {
        // lane (n, g) <- word g of chunks c .. c + 3, and their 4 scales
        uint32_t bw[4] = {wr[t % D][0], wr[t % D][1], wr[t % D][2], wr[t % D][3]};
        transpose4(bw);
        const uint32_t su = __builtin_bit_cast(uint32_t, sr[t % D]);
        if (t + D < NS) load_step(t + D);   // refill the slot just read
        uint32_t sv[4] = {su, su, su, su};
        transpose4(sv);
        const int cl0 = kStepChunks * t;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const half8 bf = unpack_int4(bw[j], kMagic, kLo, kHi, c1, c16);
            const half8 af = *(const half8 *)(frag + ((size_t)(cl0 + j) * R2 + arow) * kFragRow + 8 * g);
            const f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            const float sj = __builtin_bit_cast(float, sv[j]);
            acc0 = __builtin_fmaf(sj, c[0] + c[1], acc0);
            acc1 = __builtin_fmaf(sj, c[2] + c[3], acc1);
        }
        // finish each step's accumulation within the step: left to the IR
        // passes, the adds sink to the end and every MFMA result of every
        // step stays live in registers
        asm volatile("" : "+v"(acc0), "+v"(acc1));
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- 5. store (or this split's partial), times 2^e of each row
    const int rn = row0 + n;
    if (m0 < M && rn < p.N) {
        acc0 *= pe[m0];
        acc1 *= pe[min(m0 + 1, M - 1)];
        float *out = p.splits == 1 ? p.y : p.part + (int64_t)split * M * p.N;
        const int64_t ld = p.splits == 1 ? p.ldy : p.N;
        out[(int64_t)m0 * ld + rn] = acc0;
        if (m0 + 1 < M) out[(int64_t)(m0 + 1) * ld + rn] = acc1;
    }
}

// y[m][n] = sum over splits s = 0, 1, ... of part[s][m][n], in that order;
// up to kSumBatch partials are loaded together before they are added, so a
// sum costs one memory round trip per kSumBatch splits.
constexpr int kSumBatch = 8;

__global__ __launch_bounds__(256) void sgemv_split_sum(const float *part, int32_t splits, int32_t M, int32_t N,
                                                       float *y, int64_t ldy) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)M * N) return;
    const int64_t m = i / N, n = i % N, mn = (int64_t)M * N;
    float s = 0.0f;
    for (int k0 = 0; k0 < splits; k0 += kSumBatch) {
        float u[kSumBatch];
#pragma unroll
        for (int j = 0; j < kSumBatch; ++j) u[j] = part[(int64_t)min(k0 + j, splits - 1) * mn + i];
#pragma unroll
        for (int j = 0; j < kSumBatch; ++j)
            if (k0 + j < splits) s += u[j];
    }
    y[m * ldy + n] = s;
}

template <int M, int NS>
hipError_t launch_mn(const SParams &p, unsigned blocks, size_t lds, hipStream_t s) {
    static const int depth = [] {
        const char *v = std::getenv("TBH_SGEMV_DEPTH");
        return v && *v ? std::atoi(v) : 2;   // measured best of 2, 4, 8
    }();
    if (depth >= 8) hipLaunchKernelGGL((sgemv_int4<M, NS, 8>), dim3(blocks), dim3(512), lds, s, p);
    else if (depth <= 2) hipLaunchKernelGGL((sgemv_int4<M, NS, 2>), dim3(blocks), dim3(512), lds, s, p);
    else hipLaunchKernelGGL((sgemv_int4<M, NS, 4>), dim3(blocks), dim3(512), lds, s, p);
    return hipGetLastError();
}

template <int M>
hipError_t launch_m(int ns, const SParams &p, unsigned blocks, size_t lds, hipStream_t s) {
    switch (ns) {
    case 4: return launch_mn<M, 4>(p, blocks, lds, s);
    case 8: return launch_mn<M, 8>(p, blocks, lds, s);
    case 12: return launch_mn<M, 12>(p, blocks, lds, s);
    default: return launch_mn<M, 16>(p, blocks, lds, s);
    }
}

}  // namespace

bool sgemv_supported(const tbh_weight &w) {
    if (w.path != Path::Int4KGroup || w.mfma_tiles || w.zp || w.Kp < 128) return false;
    const int cpg = w.chunks_per_group;
    return cpg > 0 && (cpg & (cpg - 1)) == 0 && w.Np % 8 == 0;
}

hipError_t launch_sgemv(const tbh_weight &w, const GemvArgs &a, hipStream_t s, const Scratch &scr) {
    const int M = (int)a.M;
    if (!sgemv_supported(w) || M < 2 || M > 8) return hipErrorInvalidValue;
    if (w.K % 4 != 0 || a.ldx % 4 != 0 || ((uintptr_t)a.x & 15) != 0) return hipErrorInvalidValue;
    SParams p{};
    p.x = a.x;
    p.ldx = a.ldx;
    p.y = a.y;
    p.ldy = a.ldy;
    p.data = w.data;
    p.row_bytes = w.row_bytes;
    p.scales = w.scales;
    p.K = (int32_t)w.K;
    p.N = (int32_t)w.N;
    p.Np = (int32_t)w.Np;
    p.G = (int32_t)w.groups_per_row;
    p.cpg_shift = 0;
    while ((1 << p.cpg_shift) < w.chunks_per_group) ++p.cpg_shift;
    p.chunks = (int32_t)(w.Kp / kInt4ChunkElems);

    // K split: none when the row blocks alone give 3/4 of the CUs a block;
    // otherwise enough splits for about three blocks per CU (a wave keeps
    // only two steps of loads in flight, so a small grid is latency-bound:
    // the 7B projection set at M = 8 ran 10 % faster with three blocks per
    // CU than with 3/4 of a block).  Each block covers a multiple of 16
    // chunks and at most 64 (its loads all in flight: NS <= 16 steps; its x
    // fragments within LDS; its x units within kXUnits per thread).
    constexpr int kGrain = 16, kMaxChunks = 64;
    static_assert(kMaxChunks * 8 * 8 <= 512 * kXUnits, "x units of M = 8 rows per thread");
    const int64_t nblk = (w.Np + kRows - 1) / kRows;
    const int64_t cus = std::max(1, w.dev->cu_count);
    static const int split_pct = [] {
        const char *v = std::getenv("TBH_SGEMV_SPLIT_PCT");   // percent of the CUs to fill by K splits
        return v && *v ? std::atoi(v) : 300;
    }();
    // At most kMaxSplits splits unless fewer would leave CUs without a block:
    // past that, more splits add partial sums faster than they add blocks
    // (us per call at M = 8 / 4, 22 / 8 splits: 4096x11008 16.4 / 15.0,
    // 14.0 / 12.8; 2048x5632, whose 16 row blocks need 11 splits for a block
    // per CU, 9.7 against 10.5 with 6).  TBH_SGEMV_MAX_SPLITS overrides it.
    static const int max_splits = [] {
        const char *v = std::getenv("TBH_SGEMV_MAX_SPLITS");
        return v && *v ? std::atoi(v) : 0;
    }();
    constexpr int64_t kMaxSplits = 8;
    int64_t want =
        4 * nblk >= 3 * cus ? 1 : std::max<int64_t>(1, (split_pct * cus / 100 + nblk - 1) / nblk);
    want = std::min<int64_t>(want, max_splits > 0 ? max_splits : std::max(kMaxSplits, (cus + nblk - 1) / nblk));
    int64_t kchunks = ((p.chunks + want - 1) / want + kGrain - 1) / kGrain * kGrain;
    kchunks = std::min<int64_t>(kchunks, kMaxChunks);
    int64_t splits = (p.chunks + kchunks - 1) / kchunks;
    if (splits > 1) {
        p.part = (float *)scr.get(s, (size_t)(splits * M * w.N) * sizeof(float));
        if (!p.part && scr.is_fixed()) return hipErrorOutOfMemory;
        if (!p.part) {
            // no workspace (a graph being captured before any eager call): one
            // split when the whole row fits in one block, else the caller
            // falls back to the VALU kernel
            const int64_t whole = (p.chunks + kGrain - 1) / kGrain * kGrain;
            if (whole > kMaxChunks) return hipErrorInvalidValue;
            splits = 1;
            kchunks = whole;
        }
    }
    p.kchunks = (int32_t)kchunks;
    p.splits = (int32_t)splits;
    const size_t lds = (size_t)kchunks * 2 * M * kFragRow * 2 + (size_t)(M + kWaves * M) * 4;
    const unsigned blocks = (unsigned)(nblk * splits);
    const int ns = (int)(kchunks / kStepChunks);
    hipError_t e;
    switch (M) {
    case 2: e = launch_m<2>(ns, p, blocks, lds, s); break;
    case 3: e = launch_m<3>(ns, p, blocks, lds, s); break;
    case 4: e = launch_m<4>(ns, p, blocks, lds, s); break;
    case 5: e = launch_m<5>(ns, p, blocks, lds, s); break;
    case 6: e = launch_m<6>(ns, p, blocks, lds, s); break;
    case 7: e = launch_m<7>(ns, p, blocks, lds, s); break;
    default: e = launch_m<8>(ns, p, blocks, lds, s); break;
    }
    if (e != hipSuccess || splits == 1) return e;
    const int64_t total = (int64_t)M * w.N;
    hipLaunchKernelGGL(sgemv_split_sum, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, p.part,
                       (int32_t)splits, (int32_t)M, (int32_t)w.N, a.y, a.ldy);
    return hipGetLastError();
}

}  // namespace tbh

// tbh_prefill.hip -- prefill dequant-GEMM on bf16 MFMA (M >= 64 rows of x).
//
// y[M, N] = x[M, K] (bf16) . dequantize(W)[K, N], fp32 accumulation, for the
// repacked K-contiguous row layout.  This is the one dense contraction of the
// path: the reference runs it as dequantize() + cblas_sgemm on the CPU
// (Sources/TinyBrainRuntime/QuantizedTensor.swift:640-642,
// Tensor.swift:839-861) or as the MSL dequant kernels one output per thread
// (Shaders/Dequant.metal:49-79, DequantINT4.metal:95-137).
//
// A block of four or eight waves owns a BM x BN output tile; its waves, as
// 2 x (waves / 2), own (BM/2) x (BN/(waves/2)) each, as TM x TN tiles of
// v_mfma_f32_16x16x32_bf16 (eight waves: two per SIMD from one block).  Per
// K step of 64 (128 for unsplit INT4 128 x 128 tiles) the block stages x
// (bf16, as given) and the dequantized weight tile in LDS; global loads of
// step t+1 are in flight while step t's MFMAs run.  Weight operands are exact:
//   * INT8 (one scale per row): q - zp is an integer of magnitude <= 255,
//     exact in bf16; the row scale multiplies the fp32 result once.
//   * INT4 K-groups: groups are whole multiples of 32 along K, so each
//     32-deep MFMA K-slice lies in one group.  The slice's MFMA takes the
//     integer 16 (q - zp) (exact in bf16) into a zeroed accumulator, and the
//     group scale multiplies that partial product once before it is added
//     to the tile's accumulator; the epilogue multiplies by 1/16.  Scaling
//     every operand of a sum by a power of two commutes with fp32 rounding,
//     so the outputs are those of the unscaled products.
// Accumulation is fp32.
#include "tbh_internal.h"

#include <algorithm>
#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>

namespace tbh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kBK = 64;           // K per staged step (two MFMA K-steps of 32) unless a launch takes 128
// bf16 of padding per LDS row (32 bytes): rows of 160 (K steps of 64) or 288
// (of 128) bytes.  The MFMA fragment reads (lane l: row l % 16, 16-byte
// column l / 16) measured conflict-free with these strides on gfx950 and
// 2-way conflicted with 144 / 272-byte rows (16 bytes of padding), which
// cost 1-6 % per launch (rocprofv3 SQ_LDS_BANK_CONFLICT per LDS
// instruction 2.98 -> 1.02 on INT8 M = 2048).
constexpr int kRowPad = 16;
constexpr int kDepth = 2;         // K steps whose global loads are in flight at once

struct PParams {
    const uint16_t *x;   // bf16 bits, [M][ldx]
    const float *xf;     // fp32 mode: x as fp32 [Mout][ldx], row r of the product = piece r % 4 of row r / 4
    int64_t ldx;
    float *y;            // [M][ldy]; with split-K, split z writes y + z * split_stride
    int64_t ldy;
    int64_t split_stride;
    int32_t split_steps; // K steps per split (a multiple of kDepth)
    const uint8_t *data;
    int64_t row_bytes;
    const float *scales;
    const int8_t *zp;
    int32_t M, K, N, Np;
    int32_t Mout;    // output rows: M, or M / 4 in fp32 mode
    int32_t chunks;  // 16-byte chunks per row
    int32_t G;       // INT4 K-groups per row
    int32_t cpg;     // chunks per K-group
    int32_t rpn;     // runtime-layout INT4: rows per N-block (scales: [nbk][chunks * 32])
    int32_t nbk;     // runtime-layout INT4: N-blocks
    // Split tail (bf16 x, K-group weights; tail_first >= 0): a one-dimensional
    // grid whose blocks [0, tail_first) take tile b over the whole K, and
    // whose remaining blocks take tile tail_first + q / tail_parts over K
    // steps [r tail_steps, (r + 1) tail_steps), r = q % tail_parts, writing
    // that part's tile to tail_part[r][q / tail_parts][BM][BN].  Tiles are
    // numbered N-tile first (tiles_n per row of tiles), as the 3-D grid
    // dispatches them.
    int32_t tail_first, tail_parts, tail_steps, tail_n, tiles_n;
    float *tail_part;
    // gemm_ngw: per x row e with |x| < 2^e over its finite values, and the
    // weight's per N-block e with |s| < 2^e over its finite scales
    const int32_t *row_exp;
    const int32_t *nb_exp;
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

// Two fp32 values -> one dword of two f16 (round to nearest even).
__device__ __forceinline__ uint32_t pack_f16(float lo_elem, float hi_elem) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo_elem, hi_elem}, f16x2));
}

// One 16x16x32 MFMA of eight 16-bit operands per lane: f16 or bf16.
template <bool F16>
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                     0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// A 32-bit word as fp32.  By value: __builtin_bit_cast applied directly to
// an element of an ext_vector_type value (v[1]) reads element 0.
__device__ __forceinline__ float as_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// An fp32 value split exactly into three bf16 values, x = p[0] + p[1] + p[2]:
// p[0] keeps the upper 16 bits of x, p[1] the upper 16 bits of the exact
// remainder x - p[0] (at most 16 significant bits), p[2] the rest (at most 8
// significant bits, so exact in bf16).  Non-finite x stays in p[0].
__device__ __forceinline__ void split3(float x, float (&p)[3]) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    p[0] = __builtin_bit_cast(float, b & 0xFFFF0000u);
    const float r1 = (b & 0x7F800000u) != 0x7F800000u ? x - p[0] : 0.0f;
    p[1] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, r1) & 0xFFFF0000u);
    p[2] = r1 - p[1];
}

// Byte J of w, read as a signed byte, as fp32 (one sign-extending byte
// select of v_cvt_f32_i32).
template <int J>
__device__ __forceinline__ float sbyte(uint32_t w) {
    return (float)(int8_t)(uint8_t)(w >> (8 * J));
}

// XF = 1 (fp32 x): product row r is piece r % 4 of x row r / 4 (split3;
// piece 3 is zero), so the four rows a lane holds in each 16 x 16
// accumulator tile are the pieces of one x row, and the epilogue adds them
// into that row's output.  XF = 2: the same from bf16 x (widened exactly).
// XF = 3 (fp32 x, INT8 rows or INT4 K-groups): two product rows per x row,
// on the f16 MFMA: x is scaled exactly by 2^(15 - e) (e: the row's bound,
// |x| < 2^e over its finite values, from row_exponents) and split into
// hi = f16(x') and lo = f16(x' - hi) (the difference exact in fp32; 0 for a
// non-finite x', which hi holds), row r = piece r % 2 of x row r / 2; the
// weights' integers (q - zp, 16 (q - zp)) are exact in f16, and the
// epilogue adds the two rows and scales back by 2^(e - 15).  The pieces hold
// x' to 2^-22 of itself (2^-25 absolute below the f16 normal range); half
// the MFMAs and staged rows of XF = 1.
//
// NC > 0: INT4 in the runtime layout (groups along N: one scale per
// (N-block of rpn rows, k)).  The scale varies along K inside an MFMA, so it
// goes on the x side: the tile's NC N-blocks each get their own LDS copy of
// x, copy c holding split3(fl(x[k] * s[nb0 + c][k])) (fp32 product, split
// exactly into three bf16 pieces), and an MFMA of output columns in N-block
// c reads copy c against the exact integers 16 q.  Each term differs from the
// reference's x * fl(q * s) only in which fp32 product is rounded.
//
// Eight-wave blocks with K steps of 64 are held to four waves per SIMD
// (two blocks per CU) where that fits: not the INT4 128 x 128 tiles (about
// 180 VGPRs) nor runtime-layout tiles holding two or more x copies (their
// LDS allows one block per CU).
template <int PREC, int BM, int BN, int WV, int BK, int NC>
constexpr bool kFourWavesPerSimd = WV == 8 && BK == 64 && NC <= 1 && !(PREC == 4 && BM == 128 && BN == 128);

template <int PREC, int BM, int BN, bool ZP, int WV, int BK, int XF, int NC>
__global__ __launch_bounds__(64 * WV) __attribute__((amdgpu_waves_per_eu(kFourWavesPerSimd<PREC, BM, BN, WV, BK, NC> ? 4 : 1)))
void gemm_bf16(const PParams p) {
    static_assert(NC == 0 || (PREC == 4 && XF != 0 && !ZP), "runtime-layout INT4 stages split x, no zero points");
    static_assert(XF != 2 || NC > 0, "bf16 x is split only for runtime-layout scales");
    static_assert(XF != 3 || NC == 0, "two f16 pieces of fp32 x take weights with exact integers");
    constexpr int XP = XF == 3 ? 2 : 4;                     // product rows per x row (split x)
    constexpr bool F16 = XF == 3;                           // f16 operands and MFMA
    constexpr int NCC = NC > 0 ? NC : 1;                    // copies of x in LDS
    // Steps wholly inside K and the N tile run an unmasked loop form, except
    // in INT4 blocks with K steps of 128 (256 VGPRs), which run every step
    // masked: with the second form their spilled registers went from 2 to 14-17.
    constexpr bool kTwoForm = !(PREC == 4 && BK == 128);
    constexpr int kLdsRow = BK + kRowPad;
    constexpr int NT = 64 * WV;                   // threads; waves as 2 x (WV / 2)
    constexpr int WC = WV / 2;
    constexpr int CE = PREC == 8 ? 16 : 32;       // elements per chunk
    constexpr int CPR = BK / CE;                 // chunks per row per step
    constexpr int WCH = BN * CPR;                 // weight chunks per step
    constexpr int WPT = (WCH + NT - 1) / NT;      // per thread (last may idle)
    constexpr int XSEG = BM * (BK / 8);          // 16-byte x segments per step
    constexpr int XPT = XSEG / NT;
    constexpr int WM = BM / 2, WN = BN / WC;
    constexpr int TM = WM / 16, TN = WN / 16;
    static_assert(XSEG % NT == 0 && TN >= 1, "tile too small for the waves");

    // two LDS buffers: step t + 1 is staged while step t's MFMAs read
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][NCC][BM * kLdsRow];
    __shared__ __attribute__((aligned(16))) uint16_t ws[2][BN * kLdsRow];
    __shared__ float ssc[2][PREC == 4 && NC == 0 ? BN * CPR : 1];   // INT4 K-groups: scale of each (row, K-slice)

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WC, wn = wave % WC;
    int tn = blockIdx.x, tm = blockIdx.y, kpart = blockIdx.z, tr = -1;   // tr: tail tile
    if constexpr (XF == 0) {
        if (p.tail_first >= 0) {
            const int bid = blockIdx.x;
            int tile = bid;
            kpart = 0;
            if (bid >= p.tail_first) {
                const int q = bid - p.tail_first;
                tr = q / p.tail_parts;
                kpart = q % p.tail_parts;
                tile = p.tail_first + tr;
            }
            tn = tile % p.tiles_n;
            tm = tile / p.tiles_n;
        }
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const int nsteps = (p.chunks * CE + BK - 1) / BK;
    // This block's K steps [t_begin, t_end); x past kend reads as zero, so
    // the padded steps at a split's end add nothing.
    const int sps = tr >= 0 ? p.tail_steps : p.split_steps;
    const int t_begin = kpart * sps;
    const int t_end = min(nsteps, t_begin + sps);
    const int kend = min(p.K, t_end * BK);

    // INT8 row scales of this lane's output columns, loaded before the K loop;
    // INT4 weights are staged as 16 (q - zp)
    float scn[TN];
#pragma unroll
    for (int b = 0; b < TN; ++b)
        scn[b] = PREC == 8 ? p.scales[min(n0 + wn * WN + b * 16 + (lane & 15), p.Np - 1)] : 0.0625f;

    // ---- global -> registers for one step, into register stage d of kDepth:
    // the loads of steps t+1 .. t+kDepth-1 are in flight while step t runs
    // split x: a segment is 8 elements of one x row (two 16-byte loads of
    // fp32, one of bf16), staged as the four product rows of its pieces; with
    // runtime-layout scales an item is a (segment, copy) pair and also loads
    // the copy's 8 scales
    constexpr int XSEGF = (BM / XP) * (BK / 8);
    constexpr int XPTF = XF ? (XSEGF * NCC + NT - 1) / NT : 1;
    constexpr int XPTL = XF ? XPTF : XPT;
    u32x4 xr[kDepth][XPTL][XF == 1 || XF == 3 ? 2 : 1];
    u32x4 xsc[kDepth][NC > 0 ? XPTL : 1][2];
    bool xin[kDepth][XPTL];   // segment within K, applied at the LDS store
    // XF = 3: each item's x row, so its scaling exponent, is the same in every step
    int xsh[XF == 3 ? XPTL : 1];
    if constexpr (XF == 3) {
#pragma unroll
        for (int j = 0; j < XPTF; ++j)
            xsh[j] = 15 - p.row_exp[min(m0 / XP + min(tid + NT * j, XSEGF - 1) / (BK / 8), p.Mout - 1)];
    }
    u32x4 wr[kDepth][WPT];
    float sr[kDepth][WPT];
    int8_t zq[kDepth][WPT];
    // Only addresses are computed here; everything that uses a loaded value
    // (masks, conversions) happens in store_step, kDepth - 1 steps later.
    // full (std::true_type): step t lies wholly inside this block's K range
    // and the block's N tile inside the weight, so no address is clamped and
    // no segment masked (the K loop takes this form for all but its last
    // iterations).
    auto load_step = [&](int t, int d, auto full) {
        constexpr bool FULL = decltype(full)::value && !XF && kTwoForm;
        const int k0 = t * BK;
        if constexpr (XF) {
#pragma unroll
            for (int j = 0; j < XPTF; ++j) {
                const int i = min(tid + NT * j, XSEGF * NCC - 1);   // threads past the last item repeat it
                const int s = NCC == 1 ? i : i % XSEGF;
                const int qrow = s / (BK / 8), kq = s % (BK / 8);
                const int m = min(m0 / XP + qrow, p.Mout - 1), k = k0 + 8 * kq;
                const int kk = k < p.K ? k : 0;
                xin[d][j] = k < kend;
                if constexpr (XF == 1 || XF == 3) {
                    const float *src = p.xf + (int64_t)m * p.ldx + kk;
                    xr[d][j][0] = *(const u32x4 *)src;
                    xr[d][j][1] = *(const u32x4 *)(src + 4);
                } else {
                    xr[d][j][0] = *(const u32x4 *)(p.x + (int64_t)m * p.ldx + kk);
                }
                if constexpr (NC > 0) {
                    // copy i / XSEGF: N-block n0 / rpn + copy (clamped; tiles
                    // past the last N-block store nothing)
                    const int nb = min(n0 / p.rpn + i / XSEGF, p.nbk - 1);
                    const float *sp = p.scales + (int64_t)nb * (p.chunks * CE) + kk;
                    xsc[d][j][0] = *(const u32x4 *)sp;
                    xsc[d][j][1] = *(const u32x4 *)(sp + 4);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < XPT; ++j) {
                const int s = tid + NT * j;
                const int row = s / (BK / 8), kq = s % (BK / 8);
                const int m = min(m0 + row, p.M - 1), k = k0 + 8 * kq;
                // K % 8 == 0: a segment is all in or out.  Rows past M read row
                // M-1 (finite values; their outputs are never stored).
                xin[d][j] = FULL || k < kend;
                xr[d][j][0] = *(const u32x4 *)(p.x + (int64_t)m * p.ldx + (FULL || k < p.K ? k : 0));
            }
        }
#pragma unroll
        for (int j = 0; j < WPT; ++j) {
            const int s = tid + NT * j;
            const int row = s / CPR, c = t * CPR + s % CPR;
            const int n = n0 + row;
            // (the INT4 128-deep kernel keeps the run-time s < WCH test here and in
            // store_step: with it folded, that kernel's register allocation
            // spilled 6-11 more registers)
            const bool in = ((kTwoForm && WCH % NT == 0) || s < WCH) && (FULL || (n < p.Np && c < p.chunks));
            // Out-of-range chunks read a valid chunk: rows past N are never
            // stored and K padding meets x = 0, so the values do not matter.
            const int64_t nn = in ? n : 0, cc = in ? c : 0;
            wr[d][j] = __builtin_nontemporal_load((const u32x4 *)(p.data + nn * p.row_bytes + cc * 16));
            if constexpr (PREC == 4 && NC == 0) {
                const int64_t gi = kgroup_index(nn, cc / p.cpg, p.G);
                sr[d][j] = p.scales[gi];
                if (ZP) zq[d][j] = p.zp[gi];
            } else if constexpr (ZP) {
                zq[d][j] = p.zp[nn];
            }
        }
    };

    // ---- registers -> LDS (x as is; weights dequantized to bf16 pieces)
    auto store_step = [&](int d, int bb, auto full) {
        constexpr bool FULL = decltype(full)::value && !XF && kTwoForm;
        if constexpr (XF) {
            // segment (quad row qrow, kq) of copy i / XSEGF -> product rows
            // 4 qrow + piece
#pragma unroll
            for (int j = 0; j < XPTF; ++j) {
                const int i = tid + NT * j;
                if (i < XSEGF * NCC) {
                    const int s = NCC == 1 ? i : i % XSEGF;
                    const int qrow = s / (BK / 8), kq = s % (BK / 8);
                    if constexpr (XF == 3) {
                        uint32_t hi[4], lo[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            float a = as_f32(xr[d][j][(2 * q) / 4][(2 * q) % 4]);
                            float b = as_f32(xr[d][j][(2 * q + 1) / 4][(2 * q + 1) % 4]);
                            if (!xin[d][j]) a = b = 0.0f;
                            a = __builtin_ldexpf(a, xsh[j]);
                            b = __builtin_ldexpf(b, xsh[j]);
                            const f16x2 h = __builtin_convertvector(f32x2{a, b}, f16x2);
                            const f32x2 hb = __builtin_convertvector(h, f32x2);
                            const float ra = a - hb[0], rb = b - hb[1];
                            hi[q] = __builtin_bit_cast(uint32_t, h);
                            lo[q] = pack_f16(__builtin_isnan(ra) ? 0.0f : ra, __builtin_isnan(rb) ? 0.0f : rb);
                        }
                        uint16_t *dst = &xs[bb][0][(2 * qrow) * kLdsRow + 8 * kq];
                        *(u32x4 *)dst = u32x4{hi[0], hi[1], hi[2], hi[3]};
                        *(u32x4 *)(dst + kLdsRow) = u32x4{lo[0], lo[1], lo[2], lo[3]};
                        continue;
                    }
                    float pc[8][3];
#pragma unroll
                    for (int h = 0; h < 8; ++h) {
                        const int e = 4 * (h % 2) + h / 2;   // 0, 4, 1, 5, ...: the two loads' elements alternate
                        float v;
                        if constexpr (XF == 1) {
                            v = as_f32(xr[d][j][e / 4][e % 4]);
                        } else {   // bf16 element e: low half of word e / 2 when e is even
                            const uint32_t wv = xr[d][j][0][e / 2];
                            v = as_f32(e % 2 ? wv & 0xFFFF0000u : wv << 16);
                        }
                        if constexpr (NC > 0) v *= as_f32(xsc[d][j][e / 4][e % 4]);
                        split3(xin[d][j] ? v : 0.0f, pc[e]);
                    }
                    uint16_t *dst = &xs[bb][NCC == 1 ? 0 : i / XSEGF][(4 * qrow) * kLdsRow + 8 * kq];
#pragma unroll
                    for (int piece = 0; piece < 3; ++piece) {
                        uint32_t o[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) o[e] = pack_hi16(pc[2 * e][piece], pc[2 * e + 1][piece]);
                        *(u32x4 *)(dst + piece * kLdsRow) = u32x4{o[0], o[1], o[2], o[3]};
                    }
                    *(u32x4 *)(dst + 3 * kLdsRow) = u32x4{0, 0, 0, 0};
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < XPT; ++j) {
                const int s = tid + NT * j;
                const int row = s / (BK / 8), kq = s % (BK / 8);
                *(u32x4 *)&xs[bb][0][row * kLdsRow + 8 * kq] = FULL || xin[d][j] ? xr[d][j][0] : u32x4{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int j = 0; j < WPT; ++j) {
            const int s = tid + NT * j;
            if ((kTwoForm && WCH % NT == 0) || s < WCH) {
                const int row = s / CPR, cl = s % CPR;
                uint16_t *dst = &ws[bb][row * kLdsRow + cl * CE];
                if (PREC == 8) {
                    // bytes {0,2,1,3} of each word are k+{0,1,2,3}, each stored as
                    // u = q + 128: flipping the top bit of every byte leaves q as a
                    // signed byte.  Value q - zp.
                    const float zf = ZP ? (float)zq[d][j] : 0.0f;
                    uint32_t o[8];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t w = wr[d][j][q] ^ 0x80808080u;
                        const float f0 = sbyte<0>(w) - zf;
                        const float f1 = sbyte<2>(w) - zf;
                        const float f2 = sbyte<1>(w) - zf;
                        const float f3 = sbyte<3>(w) - zf;
                        o[2 * q] = F16 ? pack_f16(f0, f1) : pack_hi16(f0, f1);
                        o[2 * q + 1] = F16 ? pack_f16(f2, f3) : pack_hi16(f2, f3);
                    }
                    *(u32x4 *)dst = u32x4{o[0], o[1], o[2], o[3]};
                    *(u32x4 *)(dst + 8) = u32x4{o[4], o[5], o[6], o[7]};
                } else {
                    // nibble of k % 8 at bit {0,16,4,20,8,24,12,28}, stored as
                    // u = q + 8: flipping the top bit of every nibble leaves q as a
                    // 4-bit two's complement value.  Moved into the upper half of
                    // its byte (high nibbles masked in place, low nibbles shifted
                    // up), a nibble reads as the signed byte 16 q.  Value 16 (q - zp).
                    const float zf = ZP ? 16.0f * (float)zq[d][j] : 0.0f;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t w = wr[d][j][q] ^ 0x88888888u;
                        const uint32_t hi = w & 0xF0F0F0F0u;          // bytes: k + {2, 6, 3, 7}
                        const uint32_t lo = (w << 4) & 0xF0F0F0F0u;   // bytes: k + {0, 4, 1, 5}
                        uint32_t o[4];
                        if constexpr (F16) {
                            o[0] = pack_f16(sbyte<0>(lo) - zf, sbyte<2>(lo) - zf);
                            o[1] = pack_f16(sbyte<0>(hi) - zf, sbyte<2>(hi) - zf);
                            o[2] = pack_f16(sbyte<1>(lo) - zf, sbyte<3>(lo) - zf);
                            o[3] = pack_f16(sbyte<1>(hi) - zf, sbyte<3>(hi) - zf);
                        } else {
                            o[0] = pack_hi16(sbyte<0>(lo) - zf, sbyte<2>(lo) - zf);
                            o[1] = pack_hi16(sbyte<0>(hi) - zf, sbyte<2>(hi) - zf);
                            o[2] = pack_hi16(sbyte<1>(lo) - zf, sbyte<3>(lo) - zf);
                            o[3] = pack_hi16(sbyte<1>(hi) - zf, sbyte<3>(hi) - zf);
                        }
                        *(u32x4 *)(dst + 8 * q) = u32x4{o[0], o[1], o[2], o[3]};
                    }
                    if constexpr (NC == 0) ssc[bb][s] = sr[d][j];
                }
            }
        }
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    // runtime-layout scales: copy c serves the tile's columns [c, c + 1) * BN / NC
    constexpr int kColsPerCopy = BN / NCC;
    constexpr bool kWaveOneCopy = kColsPerCopy >= WN;   // all of a wave's columns in one copy
    static_assert(kColsPerCopy % 16 == 0, "an MFMA's 16 columns lie in one N-block");
    auto compute = [&](int bb) {
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            const int kofs = ks * 32 + 8 * (lane >> 4);
            bf16x8 af[TM];
            if constexpr (kWaveOneCopy) {
                const int cw = NCC == 1 ? 0 : (wn * WN) / kColsPerCopy;
#pragma unroll
                for (int a = 0; a < TM; ++a)
                    af[a] = *(const bf16x8 *)&xs[bb][cw][(wm * WM + a * 16 + (lane & 15)) * kLdsRow + kofs];
            }
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int wrow = wn * WN + b * 16 + (lane & 15);
                const bf16x8 bfr = *(const bf16x8 *)&ws[bb][wrow * kLdsRow + kofs];
                if constexpr (!kWaveOneCopy) {
                    const int cb = (wn * WN + b * 16) / kColsPerCopy;
#pragma unroll
                    for (int a = 0; a < TM; ++a)
                        af[a] = *(const bf16x8 *)&xs[bb][cb][(wm * WM + a * 16 + (lane & 15)) * kLdsRow + kofs];
                }
                if (PREC == 8 || NC > 0) {
#pragma unroll
                    for (int a = 0; a < TM; ++a)
                        acc[a][b] = mfma16<F16>(af[a], bfr, acc[a][b]);
                } else {
                    const float sc = ssc[bb][wrow * CPR + ks];
#pragma unroll
                    for (int a = 0; a < TM; ++a) {
                        const f32x4 part = mfma16<F16>(af[a], bfr, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[a][b][e] = __builtin_fmaf(part[e], sc, acc[a][b][e]);
                    }
                }
            }
        }
    };

    // Register ring slot s holds a step's global loads; LDS buffer t % 2 holds
    // step t.  Each iteration stages step t + 1 from its slot into the other
    // buffer, refills that slot with step t + 3, computes step t, and ends with
    // the one barrier of the step (step t + 1 visible, step t's reads done).
    // Steps are padded to a multiple of kDepth and every iteration loads and
    // computes unconditionally: steps past K read clamped addresses and meet
    // x = 0, so they add nothing, and the loop body has no branches at which
    // the compiler would have to wait for every load in flight.  (Rings of
    // four steps measured slower: INT8 5632x2048 at M = 2048 76.2 -> 84.7 us,
    // M = 512 31.6 -> 32.4 us; six steps for split launches, INT8 M = 64
    // 14.7 -> 18.6 us.)
    // The iterations whose four steps t0 + 1 .. t0 + 4 all lie below t_full
    // (inside K, in a full N tile) run without clamps or masks.
    static_assert(kDepth == 2, "two register slots, two LDS buffers");
    const int t_stop = t_begin + ((t_end - t_begin + kDepth - 1) / kDepth) * kDepth;
    const std::false_type part;
    load_step(t_begin, 0, part);
    load_step(t_begin + 1, 1, part);
    store_step(0, 0, part);
    lds_barrier();
    load_step(t_begin + 2, 0, part);
    // INT8 with bf16 x issues a step's MFMAs before it stages the next step,
    // so the dequantization and LDS stores run while the matrix cores work
    // (same results bit for bit; INT8 5632x2048 M = 2048 74.4 -> 71.9 us,
    // M = 512 30.6 -> 29.8 us).  The INT4 kernels keep staging first: in
    // that order their register allocation spills (M = 128 17.9 -> 27.3
    // us); so does the fp32-x form, which lost 2-3 % (M = 128 x rows 31.2 ->
    // 32.2 us).
    auto iteration = [&](int t0, auto full) {
        if constexpr (PREC == 8 && XF == 0) {
            compute(0);                    // step t0
            store_step(1, 1, full);        // step t0 + 1
            load_step(t0 + 3, 1, full);
            lds_barrier();
            compute(1);                    // step t0 + 1
            store_step(0, 0, full);        // step t0 + 2
            load_step(t0 + 4, 0, full);
            lds_barrier();
        } else {
            store_step(1, 1, full);        // step t0 + 1
            load_step(t0 + 3, 1, full);
            compute(0);                    // step t0
            lds_barrier();
            store_step(0, 0, full);        // step t0 + 2
            load_step(t0 + 4, 0, full);
            compute(1);                    // step t0 + 1
            lds_barrier();
        }
    };
    if constexpr (kTwoForm) {
        const int t_full = n0 + BN <= p.Np ? kend / BK : 0;
        int t0 = t_begin;
        for (; t0 < t_stop && t0 + 4 < t_full; t0 += 2) iteration(t0, std::true_type{});
        for (; t0 < t_stop; t0 += 2) iteration(t0, part);
    } else {
        // the same iteration written out (measured 1-2 % faster than the
        // lambda call in this kernel: INT4 2048x5632 at M = 2048 84.8 against
        // 86.6 us)
        for (int t0 = t_begin; t0 < t_stop; t0 += 2) {
            store_step(1, 1, part);
            load_step(t0 + 3, 1, part);
            compute(0);
            lds_barrier();
            store_step(0, 0, part);
            load_step(t0 + 4, 0, part);
            compute(1);
            lds_barrier();
        }
    }

    // ---- epilogue: lane holds C[4 (lane / 16) + e][lane % 16] of each tile
    float *out = p.y + (int64_t)blockIdx.z * p.split_stride;
    const int mrow = m0 + wm * WM + 4 * (lane >> 4), ncol = n0 + wn * WN + (lane & 15);
    if constexpr (XF == 3) {
        // the lane's four rows are the two pieces of x rows (mrow + 16 a) / 2
        // and the next
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int n = ncol + b * 16;
            if (n >= p.N) continue;
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                const int m = (mrow + a * 16) >> 1;
                if (m < p.Mout)
                    out[(int64_t)m * p.ldy + n] =
                        __builtin_ldexpf(acc[a][b][0] + acc[a][b][1], p.row_exp[m] - 15) * scn[b];
                if (m + 1 < p.Mout)
                    out[(int64_t)(m + 1) * p.ldy + n] =
                        __builtin_ldexpf(acc[a][b][2] + acc[a][b][3], p.row_exp[m + 1] - 15) * scn[b];
            }
        }
        return;
    }
    if constexpr (XF) {
        // the lane's four rows are the pieces of x row (mrow + 16 a) / 4
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int n = ncol + b * 16;
            if (n >= p.N) continue;
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                const int m = (mrow + a * 16) >> 2;
                const float v = ((acc[a][b][0] + acc[a][b][1]) + acc[a][b][2]) + acc[a][b][3];
                if (m < p.Mout) out[(int64_t)m * p.ldy + n] = v * scn[b];
            }
        }
        return;
    }
    if (tr >= 0) {
        // a split-tail part: the whole tile into its slot of tail_part (the
        // sum reads the elements inside the output)
        float *tp = p.tail_part + (int64_t)(kpart * p.tail_n + tr) * (BM * BN);
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    tp[(mrow - m0 + a * 16 + e) * BN + ncol - n0 + b * 16] = acc[a][b][e] * scn[b];
        return;
    }
    if (m0 + BM <= p.M && n0 + BN <= p.N) {
        // whole tile in range: no per-element branches
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    out[(int64_t)(mrow + a * 16 + e) * p.ldy + ncol + b * 16] = acc[a][b][e] * scn[b];
    } else {
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int n = ncol + b * 16;
            if (n >= p.N) continue;
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = mrow + a * 16 + e;
                    if (m < p.M) out[(int64_t)m * p.ldy + n] = acc[a][b][e] * scn[b];
                }
        }
    }
}

// The low f16 piece of a weight w' whose high piece was rounded toward zero
// (r = w' - hi, exact; NaN for a non-finite w', which hi holds): r, but at
// least 2^-24 in magnitude and with w's sign unless w' = 0, so that an
// infinite x meets two pieces of one sign (inf * w' as one product: +-inf,
// or NaN for w' = 0) and never inf * 0 = NaN from an empty low piece.  A
// nonzero |w'| below 2^-24 would also empty the high piece; the FLOOR
// variant of gemm_ngw keeps every nonzero scale at 2^-28 or more after
// scaling, so that |w'| >= 16 * 2^-28 for q != 0 (at most 2^-21 added on
// a 2^15 scale), for weights whose scales span that far (tbh_weight.ng_wide).
__device__ __forceinline__ float lo_piece(float w, float r) {
    return w == 0.0f ? 0.0f : __builtin_copysignf(__builtin_fmaxf(__builtin_fabsf(r), 0x1p-24f), w);
}

// Runtime-layout INT4 (one scale per (N-block, k)) with bf16 x, scaled on
// the weight side: each weight's fl(q * s), the reference's dequantized
// value, is scaled exactly by 2^(12 - eb) (|s| < 2^eb over the N-block's
// finite scales, so |w'| < 2^15) and staged as two f16 pieces, hi = w'
// rounded toward zero and lo = lo_piece(w', w' - hi), in two LDS row blocks;
// x is staged once as f16 scaled by 2^(15 - er) (bf16 values are exact in
// f16 there), every A fragment meets both pieces, and y = 2^(er + eb - 27) *
// sum(x' hi + x' lo).  The pieces hold w' to 2^-21 of itself, and to 2^-24
// absolute below the f16 normal range.  Each weight element and each x
// element is staged once per tile.  (Scaling and splitting x instead, once
// per N-block of a tile, as gemm_bf16 does up to 64 rows, stages N / rpn
// times the x elements: at 2048x5632, N-blocks of 32, two f16 pieces of x
// took 99 / 373 us at M = 512 / 2048 against 56 / 155 us here.)
//
// fp32 x (F32, p.xf): two product rows per x row, the f16 pieces hi =
// f16(x') and lo = f16(x' - hi) of x' = x 2^(15 - er) (to 2^-22 of the
// row's largest element; 0 in lo for a non-finite x', which hi holds), so
// four MFMAs per x fragment and weight; the epilogue adds the two rows.
//
// Tiles BM product rows by BN outputs, WV waves as 2 x (WV / 2), K steps of
// 64 in two LDS buffers with a two-step register ring (the gemm_bf16 loop);
// K split z of p.split_steps steps writes p.y + z * p.split_stride.
template <int BM, int BN, int WV, bool F32, bool FLOOR>
__global__ __launch_bounds__(64 * WV) __attribute__((amdgpu_waves_per_eu(WV == 8 ? 4 : 1)))
void gemm_ngw(const PParams p) {
    constexpr int BK = 64, kLdsRow = BK + kRowPad;
    constexpr int NT = 64 * WV, WC = WV / 2;
    constexpr int WM = BM / 2, WN = BN / WC, TM = WM / 16, TN = WN / 16;
    constexpr int XP = F32 ? 2 : 1;                          // product rows per x row
    constexpr int XSEG = (BM / XP) * (BK / 8), XPT = XSEG / NT;   // x: 8-element segments per step
    constexpr int WIT = BN * (BK / 8), WPT = WIT / NT;     // weights: 8-k words per step
    static_assert(XSEG % NT == 0 && WIT % NT == 0 && TM >= 1 && TN >= 1, "tile too small for the waves");

    __shared__ __attribute__((aligned(16))) uint16_t xs[2][BM * kLdsRow];
    __shared__ __attribute__((aligned(16))) uint16_t ws[2][2 * BN * kLdsRow];   // hi rows, then lo rows

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WC, wn = wave % WC;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN, kpart = blockIdx.z;
    const int kp = p.chunks * 32;   // padded row length (the scale table's too)
    const int nsteps = (kp + BK - 1) / BK;
    const int t_begin = kpart * p.split_steps;
    const int t_end = min(nsteps, t_begin + p.split_steps);
    const int kend = min(p.K, t_end * BK);

    // each item's row is the same in every step, so its scaling exponent is too
    int xsh[XPT], wsh[WPT];
#pragma unroll
    for (int j = 0; j < XPT; ++j) xsh[j] = 15 - p.row_exp[min(m0 / XP + (tid + NT * j) / (BK / 8), p.Mout - 1)];
#pragma unroll
    for (int j = 0; j < WPT; ++j) wsh[j] = 8 - p.nb_exp[min(n0 + (tid + NT * j) / (BK / 8), p.Np - 1) / p.rpn];

    u32x4 xr[kDepth][XPT][XP];
    bool xin[kDepth][XPT];
    uint32_t wr[kDepth][WPT];
    u32x4 sr[kDepth][WPT][2];
    auto load_step = [&](int t, int d) {
        const int k0 = t * BK;
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int s = tid + NT * j, row = s / (BK / 8), k = k0 + 8 * (s % (BK / 8));
            const int m = min(m0 / XP + row, p.Mout - 1);   // rows past M read row M - 1 (never stored)
            const int kk = k < p.K ? k : 0;
            xin[d][j] = k < kend;
            if constexpr (F32) {
                const float *src = p.xf + (int64_t)m * p.ldx + kk;
                xr[d][j][0] = *(const u32x4 *)src;
                xr[d][j][1] = *(const u32x4 *)(src + 4);
            } else {
                xr[d][j][0] = *(const u32x4 *)(p.x + (int64_t)m * p.ldx + kk);
            }
        }
#pragma unroll
        for (int j = 0; j < WPT; ++j) {
            const int s = tid + NT * j, row = s / (BK / 8), k = k0 + 8 * (s % (BK / 8));
            const int n = min(n0 + row, p.Np - 1);
            const int kk = k < kp ? k : 0;   // past the padded row: any valid word (x is 0 there)
            // word kk / 8 of the row: nibbles of k + {0, 2, 4, 6} at bits 0, 4, 8, 12, of
            // k + {1, 3, 5, 7} at bits 16, 20, 24, 28
            wr[d][j] = __builtin_nontemporal_load((const uint32_t *)(p.data + (int64_t)n * p.row_bytes + kk / 2));
            const float *sp = p.scales + (int64_t)(n / p.rpn) * kp + kk;
            sr[d][j][0] = *(const u32x4 *)sp;
            sr[d][j][1] = *(const u32x4 *)(sp + 4);
        }
    };
    auto store_step = [&](int d, int bb) {
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int s = tid + NT * j, row = s / (BK / 8), kq = s % (BK / 8);
            if constexpr (F32) {
                uint32_t hi[4], lo[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float a = as_f32(xr[d][j][q / 2][(2 * q) % 4]), b = as_f32(xr[d][j][q / 2][(2 * q + 1) % 4]);
                    if (!xin[d][j]) a = b = 0.0f;
                    a = __builtin_ldexpf(a, xsh[j]);
                    b = __builtin_ldexpf(b, xsh[j]);
                    const f16x2 h = __builtin_convertvector(f32x2{a, b}, f16x2);
                    const f32x2 hb = __builtin_convertvector(h, f32x2);
                    const float ra = a - hb[0], rb = b - hb[1];
                    hi[q] = __builtin_bit_cast(uint32_t, h);
                    lo[q] = pack_f16(__builtin_isnan(ra) ? 0.0f : ra, __builtin_isnan(rb) ? 0.0f : rb);
                }
                uint16_t *dst = &xs[bb][(2 * row) * kLdsRow + 8 * kq];
                *(u32x4 *)dst = u32x4{hi[0], hi[1], hi[2], hi[3]};
                *(u32x4 *)(dst + kLdsRow) = u32x4{lo[0], lo[1], lo[2], lo[3]};
            } else {
                uint32_t o[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t wv = xin[d][j] ? xr[d][j][0][q] : 0u;   // bf16 elements 2q (low half), 2q + 1
                    const float a = as_f32(wv << 16), b = as_f32(wv & 0xFFFF0000u);
                    o[q] = pack_f16(__builtin_ldexpf(a, xsh[j]), __builtin_ldexpf(b, xsh[j]));
                }
                *(u32x4 *)&xs[bb][row * kLdsRow + 8 * kq] = u32x4{o[0], o[1], o[2], o[3]};
            }
        }
#pragma unroll
        for (int j = 0; j < WPT; ++j) {
            const int s = tid + NT * j, row = s / (BK / 8), kw = s % (BK / 8);
            // u = q + 8 per nibble: flipping each nibble's top bit leaves q as
            // a 4-bit two's complement value, read as the signed byte 16 q once
            // moved into the upper half of its byte
            const uint32_t w = wr[d][j] ^ 0x88888888u;
            const uint32_t hi = w & 0xF0F0F0F0u;          // bytes: k + {2, 6, 3, 7}
            const uint32_t lo = (w << 4) & 0xF0F0F0F0u;   // bytes: k + {0, 4, 1, 5}
            const float q16[8] = {sbyte<0>(lo), sbyte<2>(lo), sbyte<0>(hi), sbyte<2>(hi),
                                  sbyte<1>(lo), sbyte<3>(lo), sbyte<1>(hi), sbyte<3>(hi)};
            uint32_t ph[4], pl[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // 16 q * (s 2^(8 - eb)) = fl(q s) 2^(12 - eb), exactly
                float sa = __builtin_ldexpf(as_f32(sr[d][j][q / 2][(2 * q) % 4]), wsh[j]);
                float sb = __builtin_ldexpf(as_f32(sr[d][j][q / 2][(2 * q + 1) % 4]), wsh[j]);
                if constexpr (FLOOR) {
                    sa = sa == 0.0f ? sa : __builtin_copysignf(__builtin_fmaxf(__builtin_fabsf(sa), 0x1p-28f), sa);
                    sb = sb == 0.0f ? sb : __builtin_copysignf(__builtin_fmaxf(__builtin_fabsf(sb), 0x1p-28f), sb);
                }
                const float a = q16[2 * q] * sa;
                const float b = q16[2 * q + 1] * sb;
                const f16x2 h = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(a, b));   // toward zero
                const f32x2 hb = __builtin_convertvector(h, f32x2);
                ph[q] = __builtin_bit_cast(uint32_t, h);
                pl[q] = pack_f16(lo_piece(a, a - hb[0]), lo_piece(b, b - hb[1]));
            }
            uint16_t *dst = &ws[bb][row * kLdsRow + 8 * kw];
            *(u32x4 *)dst = u32x4{ph[0], ph[1], ph[2], ph[3]};
            *(u32x4 *)(dst + BN * kLdsRow) = u32x4{pl[0], pl[1], pl[2], pl[3]};
        }
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int bb) {
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            const int kofs = ks * 32 + 8 * (lane >> 4);
            f16x8 af[TM];
#pragma unroll
            for (int a = 0; a < TM; ++a)
                af[a] = *(const f16x8 *)&xs[bb][(wm * WM + a * 16 + (lane & 15)) * kLdsRow + kofs];
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int wrow = wn * WN + b * 16 + (lane & 15);
                const f16x8 bh = *(const f16x8 *)&ws[bb][wrow * kLdsRow + kofs];
                const f16x8 bl = *(const f16x8 *)&ws[bb][(BN + wrow) * kLdsRow + kofs];
#pragma unroll
                for (int a = 0; a < TM; ++a) {
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bh, acc[a][b], 0, 0, 0);
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bl, acc[a][b], 0, 0, 0);
                }
            }
        }
    };

    // the register ring and LDS buffers of gemm_bf16: each iteration stages
    // step t + 1, refills its slot with step t + 3, computes step t, and ends
    // with the step's one barrier; steps past this split's K meet x = 0
    const int t_stop = t_begin + ((t_end - t_begin + kDepth - 1) / kDepth) * kDepth;
    load_step(t_begin, 0);
    load_step(t_begin + 1, 1);
    store_step(0, 0);
    lds_barrier();
    load_step(t_begin + 2, 0);
    for (int t0 = t_begin; t0 < t_stop; t0 += 2) {
        store_step(1, 1);
        load_step(t0 + 3, 1);
        compute(0);
        lds_barrier();
        store_step(0, 0);
        load_step(t0 + 4, 0);
        compute(1);
        lds_barrier();
    }

    // lane holds C[4 (lane / 16) + e][lane % 16] of each 16 x 16 tile
    float *out = p.y + (int64_t)kpart * p.split_stride;
    const int mrow = m0 + wm * WM + 4 * (lane >> 4), ncol = n0 + wn * WN + (lane & 15);
#pragma unroll
    for (int b = 0; b < TN; ++b) {
        const int n = ncol + b * 16;
        if (n >= p.N) continue;
        const int eb = p.nb_exp[n / p.rpn] - 27;
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            if constexpr (F32) {   // rows e = 0, 1: the pieces of x row (mrow + 16 a) / 2; e = 2, 3: the next
                const int m = (mrow + a * 16) >> 1;
                if (m < p.Mout)
                    out[(int64_t)m * p.ldy + n] = __builtin_ldexpf(acc[a][b][0] + acc[a][b][1], eb + p.row_exp[m]);
                if (m + 1 < p.Mout)
                    out[(int64_t)(m + 1) * p.ldy + n] =
                        __builtin_ldexpf(acc[a][b][2] + acc[a][b][3], eb + p.row_exp[m + 1]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = mrow + a * 16 + e;
                    if (m < p.Mout) out[(int64_t)m * p.ldy + n] = __builtin_ldexpf(acc[a][b][e], eb + p.row_exp[m]);
                }
            }
        }
    }
}

// e[r] = the least e with |x[r][k]| < 2^e for every finite element of each
// row of x, bf16 bits (F32 = false) or fp32 (0 for a row with none but
// zeros; -126 when the largest is subnormal): one block of 256 threads per
// row.  Non-finite elements stay non-finite through the scaling.  Rows
// 16-byte aligned, K a multiple of the 16-byte segment.
template <bool F32>
__global__ __launch_bounds__(256) void row_exponents(const void *__restrict__ xv, int64_t ldx, int32_t K,
                                                     int32_t rows, int32_t *__restrict__ e) {
    constexpr int EPS = F32 ? 4 : 8;   // elements per 16-byte segment
    __shared__ uint32_t wmax[4];
    const int r = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const char *xr = (const char *)xv + (int64_t)r * ldx * (F32 ? 4 : 2);
    uint32_t mx = 0;   // largest finite |x| as bits (magnitudes order as their bits)
#pragma unroll 4
    for (int k = threadIdx.x * EPS; k < K; k += 256 * EPS) {
        const u32x4 v = *(const u32x4 *)(xr + (int64_t)k * (F32 ? 4 : 2));
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if constexpr (F32) {
                const uint32_t a = v[c] & 0x7FFFFFFFu;
                mx = max(mx, a < 0x7F800000u ? a : 0u);
            } else {
                const uint32_t lo = v[c] & 0x7FFFu, hi = (v[c] >> 16) & 0x7FFFu;
                mx = max(mx, max(lo < 0x7F80u ? lo : 0u, hi < 0x7F80u ? hi : 0u));
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, o));
    if (lane == 0) wmax[wave] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
        mx = max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));
        const int E = (int)(mx >> (F32 ? 23 : 7));   // exponent field
        e[r] = mx == 0 ? 0 : (E == 0 ? -126 : E - 126);
    }
}

// y = sum over splits of the partial tiles, in split order (deterministic).
// The partials of up to kSumBatch splits are loaded together before they are
// added (clamped addresses, selected afterwards), so a sum costs one memory
// round trip per kSumBatch splits instead of one per split.
constexpr int kSumBatch = 8;

__global__ __launch_bounds__(256) void split_sum4(const float4 *__restrict__ part, int64_t stride4, int splits,
                                                  float4 *__restrict__ y, int64_t n4) {
    for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        float4 v = part[i];
        for (int z0 = 1; z0 < splits; z0 += kSumBatch) {
            float4 u[kSumBatch];
#pragma unroll
            for (int j = 0; j < kSumBatch; ++j) u[j] = part[min(z0 + j, splits - 1) * stride4 + i];
#pragma unroll
            for (int j = 0; j < kSumBatch; ++j) {
                if (z0 + j < splits) {
                    v.x += u[j].x;
                    v.y += u[j].y;
                    v.z += u[j].z;
                    v.w += u[j].w;
                }
            }
        }
        y[i] = v;
    }
}

__global__ __launch_bounds__(256) void split_sum(const float *__restrict__ part, int64_t stride, int splits,
                                                 float *__restrict__ y, int64_t n) {
    for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        float v = part[i];
        for (int z0 = 1; z0 < splits; z0 += kSumBatch) {
            float u[kSumBatch];
#pragma unroll
            for (int j = 0; j < kSumBatch; ++j) u[j] = part[min(z0 + j, splits - 1) * stride + i];
#pragma unroll
            for (int j = 0; j < kSumBatch; ++j)
                if (z0 + j < splits) v += u[j];
        }
        y[i] = v;
    }
}

// The split tail's sums: element e of tail tile r (four at a time) =
// tail_part[0][r][e] + tail_part[1][r][e] + ..., in part order, written to
// y where the tile lies inside the output.
template <int BM, int BN>
__global__ __launch_bounds__(256) void tail_sum(const PParams p, float *y, int64_t ldy, int vec) {
    constexpr int Q = BM * BN / 4;   // float4 per tile
    const int64_t total = (int64_t)p.tail_n * Q;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int r = (int)(i / Q), e = 4 * (int)(i % Q);
        const int tile = p.tail_first + r;
        const int m = (tile / p.tiles_n) * BM + e / BN, n = (tile % p.tiles_n) * BN + e % BN;
        if (m >= p.M || n >= p.N) continue;
        float4 acc = float4{0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < p.tail_parts; ++j) {
            const float4 v = *(const float4 *)(p.tail_part + (int64_t)(j * p.tail_n + r) * (BM * BN) + e);
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
        }
        float *o = y + (int64_t)m * ldy + n;
        if (vec && n + 3 < p.N) {
            *(float4 *)o = acc;
        } else {
            const float a[4] = {acc.x, acc.y, acc.z, acc.w};
            for (int q = 0; q < 4 && n + q < p.N; ++q) o[q] = a[q];
        }
    }
}

// Blocks of `kern` (launched with `threads` threads) one CU holds at once on
// the current device, from the runtime's occupancy calculation, asked once
// per kernel, block size and device (0 when the query fails).
static int blocks_per_cu_of(const void *kern, hipError_t (*query)(int *, const void *, int), int threads) {
    static std::mutex mu;
    static std::map<std::tuple<const void *, int, int>, int> seen;
    int dev = 0;
    (void)hipGetDevice(&dev);
    const auto key = std::make_tuple(kern, threads, dev);
    std::lock_guard<std::mutex> lock(mu);
    const auto it = seen.find(key);
    if (it != seen.end()) return it->second;
    int occ = 0;
    if (query(&occ, kern, threads) != hipSuccess) occ = 0;
    seen.emplace(key, occ);
    return occ;
}

// What a launch without a K split needs to split its tail: the K steps, the
// CU count and the workspace.
struct TailReq {
    int nsteps;
    int64_t cus;
    const Scratch *scr;
};

// Launches kern over `grid` (no K split).  With a TailReq: when the tiles
// fill r >= 1 whole rounds of the blocks the GPU holds at once (the
// occupancy of kern) and leave at most one tile per CU for a last round,
// the leftover tiles are split along K into parts (2..8, as below), so the
// last round takes a fraction of a tile's time instead of a whole one;
// tail_sum then adds the parts.  Bits differ from the unsplit launch only in
// those tiles' summation order, and a given shape always takes the same
// form.
template <int BM, int BN, typename Kern>
hipError_t launch_tail(Kern kern, int threads, dim3 grid, PParams p, const TailReq *tq, hipStream_t s) {
    p.tail_first = -1;
    if (tq != nullptr && grid.z == 1) {
        static const bool off = [] {   // TBH_PREFILL_TAIL=0: no split tail
            const char *v = std::getenv("TBH_PREFILL_TAIL");
            return v && *v == '0';
        }();
        const int occ = off ? 0 : blocks_per_cu_of((const void *)kern, [](int *n, const void *k, int t) {
            return hipOccupancyMaxActiveBlocksPerMultiprocessor(n, k, t, 0);
        }, threads);
        if (occ > 0) {
            const int64_t S = (int64_t)occ * tq->cus, T = (int64_t)grid.x * grid.y, R = T % S;
            // The last round's R tiles take one tile's time on their own CUs;
            // split P ways they take ceil(R P / CUs) / P of it (blocks sharing
            // a CU run side by side).  Take the best P of 2..8 when that is at
            // most half a tile's time.
            int parts = 0, steps = 0;
            if (T > S && R > 0 && R <= tq->cus) {
                double best = 0.5;
                for (int P = 2; P <= 8; ++P) {
                    int st = (tq->nsteps + P - 1) / P;
                    st = (st + kDepth - 1) / kDepth * kDepth;
                    const int Pr = (tq->nsteps + st - 1) / st;   // parts after rounding the steps
                    if (Pr < 2) continue;
                    const double t = (double)((R * Pr + tq->cus - 1) / tq->cus) / Pr;
                    if (t <= best && (parts == 0 || t < best)) {
                        best = t;
                        parts = Pr;
                        steps = st;
                    }
                }
            }
            if (parts >= 2) {
                const size_t bytes = (size_t)parts * (size_t)R * BM * BN * sizeof(float);
                const bool room = !tq->scr->is_fixed() || tq->scr->offset + bytes <= tq->scr->fixed_bytes;
                float *tp = room ? (float *)tq->scr->get(s, bytes) : nullptr;
                if (tp != nullptr) {
                    p.tail_first = (int32_t)(T - R);
                    p.tail_parts = parts;
                    p.tail_steps = steps;
                    p.tail_n = (int32_t)R;
                    p.tiles_n = (int32_t)grid.x;
                    p.tail_part = tp;
                    p.split_steps = tq->nsteps;
                    void *args[] = {&p};
                    hipError_t e = hipLaunchKernel((const void *)kern, dim3((unsigned)(T - R + R * parts)),
                                                   dim3(threads), args, 0, s);
                    if (e != hipSuccess) return e;
                    const int64_t n4 = R * (BM * BN / 4);
                    const int vec = p.ldy % 4 == 0 && ((uintptr_t)p.y & 15) == 0;
                    hipLaunchKernelGGL((tail_sum<BM, BN>), dim3((unsigned)std::min<int64_t>(4 * tq->cus, (n4 + 255) / 256)),
                                       dim3(256), 0, s, p, p.y, p.ldy, vec);
                    return hipGetLastError();
                }
            }
        }
    }
    void *args[] = {&p};
    return hipLaunchKernel((const void *)kern, grid, dim3(threads), args, 0, s);
}

// Product rows per fp32 x row for INT8-row and INT4 K-group weights: 2 (f16
// pieces, XF = 3) unless TBH_PREFILL_F32_PIECES=4 asks for three bf16 pieces
// and a zero row (XF = 1).
int f32_x_pieces() {
    static const int v = [] {
        const char *e = std::getenv("TBH_PREFILL_F32_PIECES");
        return e && std::atoi(e) == 4 ? 4 : 2;
    }();
    return v;
}

// Fewest x rows that take the f16 forms, which need a pass over x for the
// row exponents (TBH_PREFILL_F16_MIN): bf16 x on runtime-layout INT4
// (gemm_ngw) and fp32 x on INT8 rows or INT4 K-groups (gemm_bf16, XF = 3).
// Fewer rows go to the three-bf16-piece forms, whose time the extra launch
// would exceed (2048x5632 at M = 64, us: runtime layout 24.1 / 26.6, fp32 x
// INT4 K-groups 20.2 / 21.8, INT8 20.3 / 20.7).
int64_t f16_min_rows() {
    static const int64_t v = [] {
        const char *e = std::getenv("TBH_PREFILL_F16_MIN");
        return e && *e ? std::max<int64_t>(1, std::atoll(e)) : (int64_t)65;
    }();
    return v;
}

template <int PREC, int BM, int BN, int BK, int NC>
hipError_t launch_tile(const PParams &p, int splits, hipStream_t s, const TailReq *tq = nullptr) {
    static const int waves = [] {   // 4 or 8 forces the waves per block
        const char *v = std::getenv("TBH_PREFILL_WAVES");
        return v && *v ? std::atoi(v) : 0;
    }();
    const dim3 grid((unsigned)((p.Np + BN - 1) / BN), (unsigned)((p.M + BM - 1) / BM), (unsigned)splits);
    if constexpr (NC > 0) {   // runtime-layout INT4: split x (fp32, or bf16 widened)
        constexpr int WVN = BM == 128 ? 8 : 4;
        if (p.xf) hipLaunchKernelGGL((gemm_bf16<4, BM, BN, false, WVN, BK, 1, NC>), grid, dim3(64 * WVN), 0, s, p);
        else hipLaunchKernelGGL((gemm_bf16<4, BM, BN, false, WVN, BK, 2, NC>), grid, dim3(64 * WVN), 0, s, p);
    } else {
        const bool w8 = waves == 8 || (waves != 4 && BN == 128 && (p.M >= 256 || PREC == 4));
        if (p.xf && p.row_exp) {   // fp32 x as two f16 pieces
            if (p.zp) {
                if (w8) hipLaunchKernelGGL((gemm_bf16<PREC, BM, BN, true, 8, BK, 3, 0>), grid, dim3(512), 0, s, p);
                else hipLaunchKernelGGL((gemm_bf16<PREC, BM, BN, true, 4, BK, 3, 0>), grid, dim3(256), 0, s, p);
            } else {
                if (w8) hipLaunchKernelGGL((gemm_bf16<PREC, BM, BN, false, 8, BK, 3, 0>), grid, dim3(512), 0, s, p);
                else hipLaunchKernelGGL((gemm_bf16<PREC, BM, BN, false, 4, BK, 3, 0>), grid, dim3(256), 0, s, p);
            }
        } else if (p.xf) {   // fp32 x as three bf16 pieces and a zero row
            if (p.zp) {
                if (w8) hipLaunchKernelGGL((gemm_bf16<PREC, BM, BN, true, 8, BK, 1, 0>), grid, dim3(512), 0, s, p);
                else hipLaunchKernelGGL((gemm_bf16<PREC, BM, BN, true, 4, BK, 1, 0>), grid, dim3(256), 0, s, p);
            } else {
                if (w8) hipLaunchKernelGGL((gemm_bf16<PREC, BM, BN, false, 8, BK, 1, 0>), grid, dim3(512), 0, s, p);
                else hipLaunchKernelGGL((gemm_bf16<PREC, BM, BN, false, 4, BK, 1, 0>), grid, dim3(256), 0, s, p);
            }
        } else if (p.zp) {
            if (w8) return launch_tail<BM, BN>(gemm_bf16<PREC, BM, BN, true, 8, BK, 0, 0>, 512, grid, p, tq, s);
            return launch_tail<BM, BN>(gemm_bf16<PREC, BM, BN, true, 4, BK, 0, 0>, 256, grid, p, tq, s);
        } else {
            if (w8) return launch_tail<BM, BN>(gemm_bf16<PREC, BM, BN, false, 8, BK, 0, 0>, 512, grid, p, tq, s);
            return launch_tail<BM, BN>(gemm_bf16<PREC, BM, BN, false, 4, BK, 0, 0>, 256, grid, p, tq, s);
        }
    }
    return hipGetLastError();
}

// Blocks a split-K launch aims for, per CU: `dflt` unless
// TBH_PREFILL_BLOCKS_PER_CU is set (0 disables split-K).
int blocks_per_cu(int dflt) {
    static const int v = [] {
        const char *e = std::getenv("TBH_PREFILL_BLOCKS_PER_CU");
        return e ? std::max(0, std::atoi(e)) : -1;
    }();
    return v >= 0 ? v : dflt;
}

constexpr int kMinSplitK = 256;  // K a split keeps at least

// y[0, n) = the sum of `splits` partial arrays part + z n, in split order.
hipError_t launch_split_sum(const float *part, int splits, float *y, int64_t n, int64_t cus, hipStream_t s) {
    const int64_t grid_cap = 4 * cus;
    if (n % 4 == 0 && ((uintptr_t)y & 15) == 0) {
        const int64_t n4 = n / 4;
        hipLaunchKernelGGL(split_sum4, dim3((unsigned)std::min(grid_cap, (n4 + 255) / 256)), dim3(256), 0, s,
                           (const float4 *)part, n4, splits, (float4 *)y, n4);
    } else {
        hipLaunchKernelGGL(split_sum, dim3((unsigned)std::min(grid_cap, (n + 255) / 256)), dim3(256), 0, s,
                           part, n, splits, y, n);
    }
    return hipGetLastError();
}

// Runtime-layout INT4 on the weight-side kernel (p.row_exp set; bf16 x with
// p.M = x rows, or fp32 x with p.M = 2 x rows): 128 x 64 tiles as 8-wave
// blocks past 64 product rows, else 64 x 64 as 4-wave blocks, split along K
// to a block per CU.
hipError_t launch_ngw(const tbh_weight &w, PParams p, hipStream_t s, const Scratch &scr) {
    p.rpn = w.rows_per_nblock;
    p.nbk = (int32_t)((w.Np + w.rows_per_nblock - 1) / w.rows_per_nblock);
    constexpr int BK = 64;
    const int nsteps = (int)((p.chunks * kInt4ChunkElems + BK - 1) / BK);
    const int64_t cus = std::max(1, w.dev->cu_count);
    static const int force = [] {   // 64 or 128: the tile's product rows (lab override)
        const char *v = std::getenv("TBH_PREFILL_NGW_ROWS");
        return v && *v ? std::atoi(v) : 0;
    }();
    const bool big = force ? force == 128 : p.M > 64;
    const int64_t bm = big ? 128 : 64;
    const int64_t tiles = ((p.Np + 63) / 64) * ((p.M + bm - 1) / bm);
    const int bpc = blocks_per_cu(1);
    int splits = 1, sps = nsteps;
    if (tiles < bpc * cus && p.ldy == p.N) {
        const int64_t want = (bpc * cus + tiles - 1) / tiles;
        sps = (int)std::max<int64_t>(kMinSplitK / BK, (nsteps + want - 1) / want);
        sps = (sps + kDepth - 1) / kDepth * kDepth;
        splits = (nsteps + sps - 1) / sps;
    }
    float *const y = p.y;
    const int64_t n = (int64_t)p.Mout * p.N;
    float *part = nullptr;
    if (splits > 1) {
        part = (float *)scr.get(s, (size_t)(splits * n) * sizeof(float));
        if (!part && scr.is_fixed()) return hipErrorOutOfMemory;
        if (!part) {          // no workspace (graph capture before any eager call): one pass
            splits = 1;
            sps = nsteps;
        }
    }
    p.split_steps = sps;
    if (splits > 1) {
        p.y = part;
        p.split_stride = n;
    }
    const dim3 grid((unsigned)((p.Np + 63) / 64), (unsigned)((p.M + bm - 1) / bm), (unsigned)splits);
    if (w.ng_wide) {
        if (p.xf) {
            if (big) hipLaunchKernelGGL((gemm_ngw<128, 64, 8, true, true>), grid, dim3(512), 0, s, p);
            else hipLaunchKernelGGL((gemm_ngw<64, 64, 4, true, true>), grid, dim3(256), 0, s, p);
        } else {
            if (big) hipLaunchKernelGGL((gemm_ngw<128, 64, 8, false, true>), grid, dim3(512), 0, s, p);
            else hipLaunchKernelGGL((gemm_ngw<64, 64, 4, false, true>), grid, dim3(256), 0, s, p);
        }
    } else if (p.xf) {
        if (big) hipLaunchKernelGGL((gemm_ngw<128, 64, 8, true, false>), grid, dim3(512), 0, s, p);
        else hipLaunchKernelGGL((gemm_ngw<64, 64, 4, true, false>), grid, dim3(256), 0, s, p);
    } else {
        if (big) hipLaunchKernelGGL((gemm_ngw<128, 64, 8, false, false>), grid, dim3(512), 0, s, p);
        else hipLaunchKernelGGL((gemm_ngw<64, 64, 4, false, false>), grid, dim3(256), 0, s, p);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    return launch_split_sum(part, splits, y, n, cus, s);
}

// K is split over blocks when there are fewer than bpc blocks per CU.  BK:
// K per staged step (64 or 128).
template <int PREC, int BM, int BN, int BK = kBK, int NC = 0>
hipError_t launch_split(const tbh_weight &w, PParams p, int64_t tiles, int bpc, hipStream_t s,
                        const Scratch &scr) {
    const int nsteps = (int)((p.chunks * (PREC == 8 ? kInt8ChunkElems : kInt4ChunkElems) + BK - 1) / BK);
    const int64_t cus = std::max(1, w.dev->cu_count);
    int splits = 1, sps = nsteps;
    bpc = blocks_per_cu(bpc);
    if (tiles < bpc * cus && p.ldy == p.N) {
        const int64_t want = (bpc * cus + tiles - 1) / tiles;
        sps = (int)std::max<int64_t>(kMinSplitK / BK, (nsteps + want - 1) / want);
        sps = (sps + kDepth - 1) / kDepth * kDepth;
        splits = (nsteps + sps - 1) / sps;
    }
    float *const y = p.y;
    const int64_t n = (int64_t)p.Mout * p.N;
    float *part = nullptr;
    if (splits > 1) {
        part = (float *)scr.get(s, (size_t)(splits * n) * sizeof(float));
        if (!part && scr.is_fixed()) return hipErrorOutOfMemory;
        if (!part) {          // no workspace (graph capture before any eager call): one pass
            splits = 1;
            sps = nsteps;
        }
    }
    p.split_steps = sps;
    if (splits > 1) {
        p.y = part;
        p.split_stride = n;
    }
    const TailReq tq{nsteps, cus, &scr};
    hipError_t e = launch_tile<PREC, BM, BN, BK, NC>(p, splits, s, splits == 1 ? &tq : nullptr);
    if (e != hipSuccess || splits == 1) return e;
    return launch_split_sum(part, splits, y, n, cus, s);
}

template <int PREC>
hipError_t launch_prec(const tbh_weight &w, const PParams &p, hipStream_t s, const Scratch &scr) {
    const int64_t cus = std::max(1, w.dev->cu_count);
    const int64_t t128 = ((p.Np + 127) / 128) * ((p.M + 127) / 128);
    const int64_t t64x128 = ((p.Np + 127) / 128) * ((p.M + 63) / 64);
    const int64_t t64 = ((p.Np + 63) / 64) * ((p.M + 63) / 64);
    static const int force = [] {   // 1: 64 x 64, 2: 64 x 128, 3: 128 x 128 tiles
        const char *v = std::getenv("TBH_PREFILL_TILE");
        return v && *v ? std::atoi(v) : 0;
    }();
    if (force == 1) return launch_split<PREC, 64, 64>(w, p, t64, 2, s, scr);
    if (force == 2) return launch_split<PREC, 64, 128>(w, p, t64x128, 1, s, scr);
    if (force == 3) return launch_split<PREC, 128, 128>(w, p, t128, 1, s, scr);
    if (p.M >= 256) {
        // Timestamps inside the kernel showed a block with one wave per SIMD
        // spending three quarters of each K step on global-load waits,
        // dequantization, LDS traffic and barriers that nothing overlaps;
        // two blocks on a CU took 1.2x the time of one.  So: 128 x 128 tiles
        // as 8-wave blocks (two waves per SIMD) when they give every CU a
        // block; else 64 x 64 tiles when they give two blocks per CU without
        // a K split (64 x 128 tiles never do here: there are at most twice as
        // many as 128 x 128 tiles, which are fewer than the CUs); else 128 x
        // 128 split along K to a block per CU.  Measured
        // against 4-wave blocks chosen to give every CU a block: INT8
        // 5632x2048 M = 512 35.1 -> 31 us (64 x 64), INT4 2048x5632 M = 512
        // 52.2 -> 32.5 us (128 x 128, 4 splits), M = 2048 136 -> 89 us; INT8
        // M = 2048 unchanged at 77 us.
        // INT4 128 x 128 tiles without a K split stage K steps of 128 (half
        // the barriers and loop trips per flop; its group scale per MFMA
        // makes each step's VALU work larger): 2048x5632 M = 2048 90.4 ->
        // 84.1 us.  INT8 launches measured slower with 128 (M = 512 on 64 x 64
        // tiles 31.7 -> 33.6 us, M = 2048 79.0 -> 79.9 us), and the split INT4
        // launch at M = 512 no faster (32.4 -> 32.8 us).
        // INT4 takes 64 x 64 tiles only with bf16 x and short rows, else the
        // split 128 x 128 tiles (us, 64 x 64 / 128 x 128 split: bf16 x,
        // 5632x2048 (32 K steps) M = 512 36.0 / 41.8, 2048x5632 (88 steps) at
        // 1024 rows 74.1 / 47.6; fp32 x in two f16 pieces, 5632x2048 M = 512
        // 90.9 / 74.6, 2048x5632 M = 512 101.8 / 58.2).
        if (t128 >= cus)
            return PREC == 4 ? launch_split<PREC, 128, 128, 128>(w, p, t128, 1, s, scr)
                             : launch_split<PREC, 128, 128>(w, p, t128, 1, s, scr);
        const int64_t steps64 = (p.chunks * (int64_t)(PREC == 8 ? kInt8ChunkElems : kInt4ChunkElems) + 63) / 64;
        if (t64 >= 2 * cus && (PREC == 8 || (!p.xf && steps64 <= 48)))
            return launch_split<PREC, 64, 64>(w, p, t64, 2, s, scr);
        return launch_split<PREC, 128, 128>(w, p, t128, 1, s, scr);
    }
    // Fewer rows (HBM-bound).  INT4, whose K steps carry a group scale per
    // MFMA: 64 x 128 tiles as 8-wave blocks, split along K to a block per CU
    // (2048x5632: M = 64 16.9 -> 14.9 us, M = 128 22.2 -> 18.5 us).  INT8:
    // the largest tile that still gives every CU a block; below that, 64 x 64
    // tiles split along K until there are two blocks per CU (a 64 x 64 block
    // does little work per K step, so one per CU leaves its latency exposed;
    // 8-wave 64 x 128 tiles measured the same at M = 64 and 4 % slower at
    // M = 128).
    // fp32 x at 32..63 rows (128..252 product rows): 128 x 128 tiles split
    // along K (2048x5632 at 32 rows 16.6 -> 14.8 us; bf16 x at M = 128 is
    // slower that way, 18.1 -> 20.4 us)
    if (PREC == 4 && p.xf && p.M >= 128) return launch_split<PREC, 128, 128>(w, p, t128, 1, s, scr);
    if (PREC == 4) return launch_split<PREC, 64, 128>(w, p, t64x128, 1, s, scr);
    if (t128 >= cus) return launch_split<PREC, 128, 128>(w, p, t128, 1, s, scr);
    if (t64x128 >= cus) return launch_split<PREC, 64, 128>(w, p, t64x128, 1, s, scr);
    return launch_split<PREC, 64, 64>(w, p, t64, 2, s, scr);
}

// Copies of x a 64-column tile of a runtime-layout INT4 weight needs (its
// N-blocks), or 0 when the N-blocks do not tile the 64 columns evenly.
int ng_copies(const tbh_weight &w) {
    const int64_t rpn = w.rows_per_nblock;
    if (rpn >= w.Np || rpn % 64 == 0) return 1;
    if (rpn == 32) return 2;
    if (rpn == 16) return 4;
    return 0;
}

// Runtime-layout INT4 (one scale per (N-block, k)) with x given as p.x (bf16)
// or p.xf (fp32), p.M = 4 * x rows: 64 x 64 tiles (16 x rows by 64 outputs,
// four waves) or 128 x 64 tiles (32 x rows, eight waves), split along K when
// the tiles are fewer than the CUs.
hipError_t launch_ngroup(const tbh_weight &w, PParams p, hipStream_t s, const Scratch &scr) {
    p.rpn = w.rows_per_nblock;
    p.nbk = (int32_t)((w.Np + w.rows_per_nblock - 1) / w.rows_per_nblock);
    const int64_t tiles = ((p.Np + 63) / 64) * ((p.M + 63) / 64);
    // past 16 x rows (64 product rows): 128 x 64 tiles as 8-wave blocks,
    // which re-read the weights half as often (2048x5632, N-blocks of 32, us
    // per call 64 / 128 product rows: M = 64 28.1 / 24.6, M = 128 49.2 /
    // 41.0, M = 512 160.1 / 133.9, M = 2048 598 / 508); with four copies of
    // x the 128-row tile does not fit the LDS
    if (p.M > 64) {
        const int64_t t128 = ((p.Np + 63) / 64) * ((p.M + 127) / 128);
        switch (ng_copies(w)) {
        case 1: return launch_split<4, 128, 64, kBK, 1>(w, p, t128, 1, s, scr);
        case 2: return launch_split<4, 128, 64, kBK, 2>(w, p, t128, 1, s, scr);
        default: break;
        }
    }
    switch (ng_copies(w)) {
    case 1: return launch_split<4, 64, 64, kBK, 1>(w, p, tiles, 2, s, scr);
    case 2: return launch_split<4, 64, 64, kBK, 2>(w, p, tiles, 2, s, scr);
    case 4: return launch_split<4, 64, 64, kBK, 4>(w, p, tiles, 2, s, scr);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool prefill_supported(const tbh_weight &w) {
    if (w.mfma_tiles) return false;
    if (w.path == Path::Int4NGroup) return !w.ng_pairs && !w.zp && ng_copies(w) > 0;
    return w.path == Path::Int8Row || w.path == Path::Int4KGroup;
}

static PParams prefill_params(const tbh_weight &w, int64_t ldx, float *y, int64_t ldy) {
    PParams p{};
    p.tail_first = -1;   // the three-dimensional grid unless launch_tail splits a tail
    p.ldx = ldx;
    p.y = y;
    p.ldy = ldy;
    p.data = w.data;
    p.row_bytes = w.row_bytes;
    p.scales = w.scales;
    p.zp = w.zp;
    p.K = (int32_t)w.K;
    p.N = (int32_t)w.N;
    p.Np = (int32_t)w.Np;
    const bool int8 = w.precision == TBH_PREC_INT8;
    p.chunks = (int32_t)(w.Kp / (int8 ? kInt8ChunkElems : kInt4ChunkElems));
    p.G = (int32_t)w.groups_per_row;
    p.cpg = w.chunks_per_group;
    return p;
}

// Rows of x per GEMM launch.  The grid's second dimension counts row tiles,
// and the fp32 and runtime-layout forms run up to four product rows per x
// row in 32-bit row indices; longer x is taken in chunks of this many rows, one
// launch (and split sum) after the other on the caller's stream.
constexpr int64_t kGemmRowsPerLaunch = (int64_t)1 << 18;

static hipError_t launch_rows(const tbh_weight &w, PParams &p, hipStream_t s, const Scratch &scr) {
    if (w.path == Path::Int4NGroup) return launch_ngroup(w, p, s, scr);
    return w.precision == TBH_PREC_INT8 ? launch_prec<8>(w, p, s, scr) : launch_prec<4>(w, p, s, scr);
}

hipError_t launch_prefill_f32(const tbh_weight &w, const float *x, int64_t ldx, int64_t M, float *y,
                              int64_t ldy, hipStream_t s, const Scratch &scr) {
    if (!prefill_supported(w) || M < 1 || w.K % 8 != 0 || ldx % 4 != 0 || ((uintptr_t)x & 15) != 0)
        return hipErrorInvalidValue;
    // Past 64 rows every x row becomes two f16 pieces scaled by a power of two
    // per row, after a pass that finds each row's exponent bound (an int32 per
    // row, ahead of the split-K scratch), for gemm_bf16 (INT8 rows, INT4
    // K-groups) or the weight-side gemm_ngw (runtime-layout INT4); fewer rows,
    // or a workspace that cannot grow (graph capture before any eager call),
    // take three bf16 pieces and a zero row.
    // us per call, four / two pieces: INT8 5632x2048 M = 512 70.8 / 52.5,
    // 2048 253 / 166; INT4 2048x5632 M = 128 29.3 / 25.8, 512 79.9 / 58.7,
    // 2048 315 / 189.
    const bool ng = w.path == Path::Int4NGroup;
    const bool two = f32_x_pieces() == 2 && (!ng || w.ng_sexp != nullptr);
    for (int64_t m0 = 0; m0 < M; m0 += kGemmRowsPerLaunch) {
        const int64_t mc = std::min(kGemmRowsPerLaunch, M - m0);
        PParams p = prefill_params(w, ldx, y + m0 * ldy, ldy);
        p.xf = x + m0 * ldx;
        Scratch sub = scr;
        int64_t pieces = 4;
        if (two && mc >= f16_min_rows()) {
            const size_t off = ((size_t)mc * sizeof(int32_t) + 255) / 256 * 256;
            int32_t *re = (int32_t *)scr.get(s, off);
            if (re == nullptr && scr.is_fixed()) return hipErrorOutOfMemory;
            if (re != nullptr) {
                hipLaunchKernelGGL(row_exponents<true>, dim3((unsigned)mc), dim3(256), 0, s, (const void *)p.xf, ldx,
                                   (int32_t)w.K, (int32_t)mc, re);
                p.row_exp = re;
                sub.offset = scr.offset + off;
                pieces = 2;
            }
        }
        p.M = (int32_t)(pieces * mc);
        p.Mout = (int32_t)mc;
        hipError_t e;
        if (ng && pieces == 2) {   // runtime layout: the weight-side kernel, x in two f16 pieces
            p.nb_exp = w.ng_sexp;
            e = launch_ngw(w, p, s, sub);
        } else {
            e = launch_rows(w, p, s, sub);
        }
        if (e != hipSuccess) {
            scr.shortfall = sub.shortfall;
            return e;
        }
    }
    return hipSuccess;
}

hipError_t launch_prefill(const tbh_weight &w, const uint16_t *x, int64_t ldx, int64_t M, float *y,
                          int64_t ldy, hipStream_t s, const Scratch &scr) {
    if (!prefill_supported(w) || M < 1 || w.K % 8 != 0 || ldx % 8 != 0 || ((uintptr_t)x & 15) != 0)
        return hipErrorInvalidValue;
    // runtime-layout INT4: past 64 rows the weight-side kernel, after a pass
    // that finds each x row's exponent bound (an int32 per row, ahead of the
    // split-K scratch); up to 64 rows, or when that scratch is not to be had,
    // gemm_bf16 with every x row as three bf16 pieces of fl(x * s) and a zero
    // row.  2048x5632, us per call, pieces / weight side: M = 64 24.1 / 26.6
    // (the extra pass), 128 40.2 / 26.0, 512 131.6 / 53.2, 2048 516 / 157.
    const bool ng = w.path == Path::Int4NGroup;
    const bool wside = ng && w.ng_sexp != nullptr;
    for (int64_t m0 = 0; m0 < M; m0 += kGemmRowsPerLaunch) {
        const int64_t mc = std::min(kGemmRowsPerLaunch, M - m0);
        PParams p = prefill_params(w, ldx, y + m0 * ldy, ldy);
        p.x = x + m0 * ldx;
        Scratch sub = scr;
        if (wside && mc >= f16_min_rows()) {
            const size_t off = ((size_t)mc * sizeof(int32_t) + 255) / 256 * 256;
            int32_t *re = (int32_t *)scr.get(s, off);
            if (re != nullptr) {
                hipLaunchKernelGGL(row_exponents<false>, dim3((unsigned)mc), dim3(256), 0, s, (const void *)p.x, ldx,
                                   (int32_t)w.K, (int32_t)mc, re);
                p.row_exp = re;
                p.nb_exp = w.ng_sexp;
                p.M = (int32_t)mc;
                p.Mout = (int32_t)mc;
                sub.offset = scr.offset + off;
                const hipError_t e = launch_ngw(w, p, s, sub);
                if (e != hipSuccess) {
                    scr.shortfall = sub.shortfall;
                    return e;
                }
                continue;
            }
        }
        p.M = (int32_t)((ng ? 4 : 1) * mc);
        p.Mout = (int32_t)mc;
        const hipError_t e = launch_rows(w, p, s, sub);
        if (e != hipSuccess) {
            scr.shortfall = sub.shortfall;
            return e;
        }
    }
    return hipSuccess;
}

}  // namespace tbh

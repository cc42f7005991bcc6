// tbh_decode.hip -- GPU decode step for LLaMA-style models.
//
// Restates ModelRunner.step / applyLayer / attention
// (Sources/TinyBrainRuntime/ModelRunner.swift:168-208, :392-459, :470-592)
// with every projection on the quantized GEMV, for one sequence (M = 1):
//
//   h = embedding[token]                                      (:170)
//   per layer:
//     qkv = W_qkv . rmsnorm(h) * g_in                          (:420-425, :497-499)
//     q, k <- RoPE(pos); append k, v to the cache; ctx = softmax(q K^T / sqrt(d)) V
//                                                              (:470-592)
//     h += W_o . ctx                                           (:434)
//     act = silu(W_gate . x) * (W_up . x), x = rmsnorm(h) * g_post
//                                                              (:436-451)
//     h += W_down . act                                        (:452-457)
//   logits = W_lm . rmsnorm(h) * g_final                       (:186-199)
//
// Six launches per layer: Q|K|V and gate|up are each one weight
// (concatenated along N at set-up; gate and up rows interleaved so one wave
// holds both rows of a pair and its epilogue writes silu(gate) * up),
// RMSNorm runs in the GEMV's x staging, the residual adds in its epilogue,
// and attention is two kernels:
// one block per (KV head, range of 32 cache positions at head_dim 64 and 128,
// else 64) does RoPE, the cache append
// and that range's softmax partials for the KV head's query heads, and a
// merge kernel assembles the context.  The token position lives
// in device memory and the step ends with a one-thread kernel that advances
// it, so a captured step replays as the next one.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <vector>

#include "tbh_internal.h"
#include "tbh_wave.h"

struct tbh_decoder {
    tbh_device *dev = nullptr;
    tbh_decoder_config cfg{};
    int32_t head_dim = 0, kv_dim = 0, qkv_dim = 0;
    struct Layer {
        tbh_weight *qkv = nullptr, *o = nullptr, *gu = nullptr, *down = nullptr;
    };
    std::vector<Layer> layers;
    tbh_weight *lm_head = nullptr;
    // device memory
    float *emb = nullptr;        // [vocab][hidden]
    float *norms = nullptr;      // [layers][2][hidden] then [hidden] (final)
    float *kcache = nullptr;     // [layers][max_seq][kv_dim]
    float *vcache = nullptr;
    float *h = nullptr, *qkv = nullptr, *ctx = nullptr, *gu = nullptr, *logits = nullptr;
    float *attn_o = nullptr;     // attention range partials (one layer at a time):
    float2 *attn_ml = nullptr;   //   context sums [splits][hidden], (m, l) [splits][heads]
    float *rope_theta = nullptr; // [head_dim / 2] RoPE frequencies
    int32_t attn_splits = 1;
    int32_t *pos = nullptr;      // [0] position, [1] overflow flag
    std::vector<void *> allocs;
};

namespace tbh {
namespace {

struct AttnParams {
    const float *qkv;
    float *kcache, *vcache;  // this layer
    float *ctx;
    float *part_o;           // [splits][hidden]: range context sums, heads in ctx order
    float2 *part_ml;         // [splits][nh]: range max score m and sum l of exp(score - m)
    const float *theta;      // [hd / 2]: base^(-2i / hd), fp32
    int32_t *pos;            // [0] position, [1] overflow flag
    int32_t nh, nkv, hd, kvd, hidden, max_seq;
    int32_t rep, splits;
    int32_t wpb;             // attention_split waves per block: min(4, rep)
    float rope_base, scale;
};

constexpr int kMaxHd = 128;
// Cache positions one attention wave covers: 32 at head_dim 64 and 128, else
// 64.  At head_dim 128, 64 positions' key and value rows took every register
// of the wave (256 VGPRs and 79 AGPRs, one wave per SIMD; 166 VGPRs with
// 32).  Tokens per second at context 512, ranges of 64 / 32 / 16 positions:
// 7B shape 650 / 669 / 650, 1.1B shape 1751 / 1788 / 1776.
constexpr int attn_range(int hd) { return hd == 128 || hd == 64 ? 32 : 64; }

// sin and cos of a RoPE angle formed in fp32 as the reference forms it
// (Float(pos) * theta, ModelRunner.swift:480-486).  The angle is reduced by
// 2 pi in double precision first, so sincosf only sees |r| <= pi and never
// takes its large-argument path (a table walk in memory on the critical
// path of the kernel).
__device__ __forceinline__ void rope_sincos(float ang, float *sn, float *cs) {
    const double a = (double)ang;
    const double k = rint(a * 0.15915494309189535);  // 1 / (2 pi)
    sincosf((float)fma(-k, 6.283185307179586, a), sn, cs);
}

// Orders a wave's LDS writes before its later LDS reads by other lanes of
// the same wave (no block barrier: the waves of a block are independent).
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Attention of one decode step, split over the cache.  One wave per (query
// head, range of attn_range(HD) positions <= pos): it writes the range's softmax
// partial -- max m, sum l of exp(score - m), and sum of exp(score - m) * v --
// and attention_merge combines the ranges.  A block's waves are up to four
// query heads of one KV head (ModelRunner.swift:524-536, kvHead = head /
// repeats), so they share the range's key and value rows through L1; a KV
// head with fewer than four query heads gets blocks of that many waves (no
// idle waves to dispatch).  The grid covers max_seq and waves past pos
// return at once.
//
// Every global load is issued before the position is read: the position,
// this step's q, k, v and RoPE frequencies, and the range's cache rows (the
// cache is zero-filled at creation and only ever holds finite values, so
// rows past pos are harmless -- they get p = 0 -- and row pos is replaced by
// the new k and v).  The wave applies RoPE (interleaved pairs, fp32;
// :470-494) to its query head and the new k, scores one position per lane,
// reduces max and sum with DPP, and sums p * v with 16-byte value pieces
// (lane (pg, d4) covers rows pg, pg + 64 / (hd / 4), ...).  The wave of the
// group's first head appends the new k and v to the cache (:503-516).
template <int HD>
__global__ __launch_bounds__(256) void attention_split(const AttnParams a) {
    constexpr int kSplit = attn_range(HD);
    constexpr int HD4 = HD / 4, PPI = 64 / HD4, NV = (kSplit + PPI - 1) / PPI, NP = HD / 2;
    constexpr int NPL = (NP + 63) / 64;  // RoPE pairs per lane
    static_assert(kSplit == 64 || (HD4 & (HD4 - 1)) == 0, "short ranges take the cooperative key loads");
    __shared__ __attribute__((aligned(16))) float qs[4][HD];
    __shared__ __attribute__((aligned(16))) float kn[4][HD];
    __shared__ __attribute__((aligned(16))) float vn[4][HD];
    __shared__ float ps[4][kSplit];
    __shared__ float4 red[4][64];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nquad = (a.rep + a.wpb - 1) / a.wpb;
    const int split = blockIdx.x % a.splits;
    const int quad = (blockIdx.x / a.splits) % nquad;
    const int kvh = blockIdx.x / (a.splits * nquad);
    const int hg = quad * a.wpb + w;            // head within the KV group
    if (hg >= a.rep) return;
    const int head = kvh * a.rep + hg;
    const int c0 = split * kSplit;
    const int64_t kvo = (int64_t)kvh * HD;
    const int last = a.max_seq - 1;

    const int pos = a.pos[0];
    float qx0[NPL], qx1[NPL], kx0[NPL], kx1[NPL], th[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int pr = min(lane + 64 * i, NP - 1);
        qx0[i] = a.qkv[head * HD + 2 * pr];
        qx1[i] = a.qkv[head * HD + 2 * pr + 1];
        kx0[i] = a.qkv[a.hidden + kvo + 2 * pr];
        kx1[i] = a.qkv[a.hidden + kvo + 2 * pr + 1];
        th[i] = a.theta[pr];
    }
    float vx[NPL * 2];
#pragma unroll
    for (int i = 0; i < 2 * NPL; ++i) vx[i] = a.qkv[a.hidden + a.kvd + kvo + min(lane + 64 * i, HD - 1)];
    // key rows: with HD / 4 a power of two, lane (pg, d4) reads piece d4 of
    // rows pg, pg + PPI, ... (whole row segments per load instruction) and a
    // DPP transpose-sum assembles the scores; otherwise one row per lane
    constexpr bool kCoop = (HD4 & (HD4 - 1)) == 0;
    constexpr int NK = kCoop ? kSplit / PPI : HD4;   // key loads per lane
    // values a lane carries into the transpose-sum: one per lane of its HD4
    // group (key loads past NK are zero)
    constexpr int NT = kCoop ? HD4 : 1;
    static_assert(!kCoop || NK <= NT, "a lane's key loads fit its transpose group");
    const int pg = lane / HD4, d4 = lane % HD4;
    float4 kreg[NK];
    if constexpr (kCoop) {
#pragma unroll
        for (int j = 0; j < NK; ++j)
            kreg[j] = *(const float4 *)(a.kcache + (int64_t)min(c0 + pg + j * PPI, last) * a.kvd + kvo + 4 * d4);
    } else {
        const float *kr = a.kcache + (int64_t)min(c0 + lane, last) * a.kvd + kvo;
#pragma unroll
        for (int i = 0; i < HD4; ++i) kreg[i] = *(const float4 *)(kr + 4 * i);
    }
    float4 vreg[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int r = min(pg + j * PPI, kSplit - 1);
        vreg[j] = *(const float4 *)(a.vcache + (int64_t)min(c0 + r, last) * a.kvd + kvo + 4 * d4);
    }
    if (pos < 0 || pos >= a.max_seq) {  // cache full: flag it, write nothing
        if (blockIdx.x == 0 && threadIdx.x == 0) a.pos[1] = 1;
        return;
    }
    if (c0 > pos) return;

    // RoPE at pos for this head's q and the new k; the new v
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int pr = lane + 64 * i;
        if (pr < NP) {
            float c, sn;
            rope_sincos((float)pos * th[i], &sn, &c);
            qs[w][2 * pr] = qx0[i] * c - qx1[i] * sn;
            qs[w][2 * pr + 1] = qx0[i] * sn + qx1[i] * c;
            kn[w][2 * pr] = kx0[i] * c - kx1[i] * sn;
            kn[w][2 * pr + 1] = kx0[i] * sn + kx1[i] * c;
        }
    }
#pragma unroll
    for (int i = 0; i < 2 * NPL; ++i)
        if (lane + 64 * i < HD) vn[w][lane + 64 * i] = vx[i];
    wave_lds_fence();

    // one position per lane: lane (pg, d4) scores position pg + PPI * d4
    // (cooperative form; lanes past the range score nothing) or position lane
    const int tl = kCoop ? pg + PPI * d4 : lane;
    const int t = c0 + tl;
    const bool tvalid = t <= pos && tl < kSplit;
    float d = 0.0f;
    if constexpr (kCoop) {
        const float4 q4 = *(const float4 *)&qs[w][4 * d4];
        const float4 n4 = *(const float4 *)&kn[w][4 * d4];
        const float dn = q4.x * n4.x + q4.y * n4.y + q4.z * n4.z + q4.w * n4.w;
        float part[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            if (j < NK) {
                const float dj = q4.x * kreg[j].x + q4.y * kreg[j].y + q4.z * kreg[j].z + q4.w * kreg[j].w;
                part[j] = c0 + pg + j * PPI == pos ? dn : dj;   // row pos: the new k
            } else {
                part[j] = 0.0f;
            }
        }
        d = wave::transpose_sum<NT>(part, lane);
    } else {
        const bool tnew = t == pos;
#pragma unroll
        for (int i = 0; i < HD4; ++i) {
            const float4 k4 = tnew ? *(const float4 *)&kn[w][4 * i] : kreg[i];
            const float4 q4 = *(const float4 *)&qs[w][4 * i];
            d += q4.x * k4.x + q4.y * k4.y + q4.z * k4.z + q4.w * k4.w;
        }
    }
    const float sc = tvalid ? d * a.scale : -INFINITY;
    const float m = wave::max(sc);                    // finite: position c0 <= pos
    const float p = tvalid ? expf(sc - m) : 0.0f;
    const float l = wave::sum(p);
    if (tl < kSplit) ps[w][tl] = p;
    wave_lds_fence();

    float4 acc = float4{0.f, 0.f, 0.f, 0.f};
    if (pg < PPI) {
        const float4 vn4 = *(const float4 *)&vn[w][4 * d4];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int r = pg + j * PPI;
            if (r < kSplit) {
                const float4 v4 = c0 + r == pos ? vn4 : vreg[j];
                const float pr = ps[w][r];
                acc.x += pr * v4.x;
                acc.y += pr * v4.y;
                acc.z += pr * v4.z;
                acc.w += pr * v4.w;
            }
        }
    }
    red[w][lane] = acc;
    wave_lds_fence();

    if (lane == 0) a.part_ml[split * a.nh + head] = float2{m, l};
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
        *(float4 *)&a.part_o[(int64_t)split * a.hidden + head * HD + 4 * lane] = o;
        // append the new k and v (the group's first head, range holding pos);
        // the row-pos values this launch loaded are never used
        if (hg == 0 && pos < c0 + kSplit) {
            *(float4 *)&a.kcache[(int64_t)pos * a.kvd + kvo + 4 * lane] = *(const float4 *)&kn[w][4 * lane];
            *(float4 *)&a.vcache[(int64_t)pos * a.kvd + kvo + 4 * lane] = *(const float4 *)&vn[w][4 * lane];
        }
    }
}

// ctx of head h = sum over splits of e^(m_s - M) o_s / sum of e^(m_s - M) l_s
// with M = max m_s (the softmax of :545-551 assembled from the ranges).  One
// wave per head, no block barriers: lane (sg, d4) loads the partials
// of splits sg, sg + 64 / (hd / 4), ... (up to kMergeLoads of them) together
// with the position, so up to 32 ranges (1024 positions at head_dim 64 and
// 128, 2048 at 48 or 80..112) cost one memory round trip; splits past pos are
// masked out afterwards.  Max and sum by DPP; the value pieces of the split
// groups meet in LDS.
template <int HD>
__global__ __launch_bounds__(64) void attention_merge(const AttnParams a) {
    constexpr int HD4 = HD / 4, NSG = 64 / HD4;
    constexpr int kSplit = attn_range(HD);
    constexpr int kMergeLoads = HD == 128 ? 16 : 8;
    __shared__ float4 red[64];
    const int lane = threadIdx.x;
    const int head = blockIdx.x;
    const int sg = lane / HD4, d4 = lane % HD4;
    const bool slane = sg < NSG;
    const float *po = a.part_o + head * HD + 4 * min(d4, HD4 - 1);
    const float2 *pml = a.part_ml + head;
    const int pos = a.pos[0];
    float2 mlv[kMergeLoads];
    float4 ov[kMergeLoads];
#pragma unroll
    for (int j = 0; j < kMergeLoads; ++j) {
        const int sp = min(sg + NSG * j, a.splits - 1);
        mlv[j] = pml[sp * a.nh];
        ov[j] = *(const float4 *)(po + (int64_t)sp * a.hidden);
    }
    if (pos < 0 || pos >= a.max_seq) return;
    const int ns = pos / kSplit + 1;
    float mloc = -INFINITY;
#pragma unroll
    for (int j = 0; j < kMergeLoads; ++j)
        if (slane && sg + NSG * j < ns) mloc = fmaxf(mloc, mlv[j].x);
    for (int sp = sg + NSG * kMergeLoads; slane && sp < ns; sp += NSG) mloc = fmaxf(mloc, pml[sp * a.nh].x);
    const float M = wave::max(mloc);
    float L = 0.0f;
    float4 o = float4{0.f, 0.f, 0.f, 0.f};
    auto add = [&](float2 ml, float4 v) {
        const float e = expf(ml.x - M);
        if (d4 == 0) L += e * ml.y;   // one lane per split counts its sum
        o.x += e * v.x;
        o.y += e * v.y;
        o.z += e * v.z;
        o.w += e * v.w;
    };
#pragma unroll
    for (int j = 0; j < kMergeLoads; ++j)
        if (slane && sg + NSG * j < ns) add(mlv[j], ov[j]);
    for (int sp = sg + NSG * kMergeLoads; slane && sp < ns; sp += NSG)
        add(pml[sp * a.nh], *(const float4 *)(po + (int64_t)sp * a.hidden));
    L = wave::sum(L);
    red[lane] = o;
    wave_lds_fence();
    if (lane < HD4) {
        float4 r = red[lane];
#pragma unroll
        for (int q = 1; q < NSG; ++q) {
            const float4 v = red[q * HD4 + lane];
            r.x += v.x;
            r.y += v.y;
            r.z += v.z;
            r.w += v.w;
        }
        const float inv = 1.0f / L;
        *(float4 *)&a.ctx[(int64_t)head * HD + 4 * lane] = float4{r.x * inv, r.y * inv, r.z * inv, r.w * inv};
    }
}

template <int HD>
hipError_t launch_attention_hd(const AttnParams &ap, hipStream_t s) {
    const int nquad = (ap.rep + ap.wpb - 1) / ap.wpb;
    hipLaunchKernelGGL(attention_split<HD>, dim3((unsigned)(ap.nkv * nquad * ap.splits)),
                       dim3((unsigned)(64 * ap.wpb)), 0, s, ap);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attention_merge<HD>, dim3((unsigned)ap.nh), dim3(64), 0, s, ap);
    return hipGetLastError();
}

hipError_t launch_attention(const AttnParams &ap, hipStream_t s) {
    switch (ap.hd) {
    case 16: return launch_attention_hd<16>(ap, s);
    case 32: return launch_attention_hd<32>(ap, s);
    case 48: return launch_attention_hd<48>(ap, s);
    case 64: return launch_attention_hd<64>(ap, s);
    case 80: return launch_attention_hd<80>(ap, s);
    case 96: return launch_attention_hd<96>(ap, s);
    case 112: return launch_attention_hd<112>(ap, s);
    default: return launch_attention_hd<128>(ap, s);
    }
}

// ---- host: concatenation of projection weights along N ---------------------

struct OwnedDesc {
    tbh_qtensor_desc d{};
    std::vector<int8_t> data, zp;
    std::vector<float> scales;
};

int64_t expected_scales(const tbh_qtensor_desc &d) {
    if (d.precision == TBH_PREC_INT8) return d.mode == TBH_MODE_PER_CHANNEL ? d.N : 1;
    const int64_t count = d.K * d.N;
    return d.group_size > 0 ? (count + d.group_size - 1) / d.group_size : 1;
}

// Concatenates [K, N_i] weights along N into one weight that computes every
// part's outputs in order.  INT8: the runtime [K][N] layout with one scale
// per column or per tensor (a per-tensor scale is repeated per column).
// INT4: the converter layout (groups of group_size along K, K % group_size ==
// 0, even K * N_i), where concatenation is of the flat arrays; or the runtime
// [K][N] layout with groups along N (N_i % group_size == 0), where each k
// row of the result is the parts' k rows (and their scales) side by side.
tbh_status concat_n(const tbh_qtensor_desc *const *parts, int n, OwnedDesc &out) {
    for (int i = 0; i < n; ++i) {
        const tbh_qtensor_desc *d = parts[i];
        if (!d || !d->data || !d->scales) return set_error(TBH_E_INVALID, "concatenated weights: NULL weight");
        if (d->K != parts[0]->K || d->precision != parts[0]->precision)
            return set_error(TBH_E_INVALID, "concatenated weights differ in K or precision");
        if (d->n_scales != expected_scales(*d))
            return set_error(TBH_E_INVALID, "concatenated weights: scale count does not match mode/shape");
        if ((d->zero_points != nullptr) != (parts[0]->zero_points != nullptr))
            return set_error(TBH_E_UNSUPPORTED, "concatenated weights: zero points on some parts only");
    }
    const int64_t K = parts[0]->K;
    int64_t N = 0;
    for (int i = 0; i < n; ++i) N += parts[i]->N;
    out.d = *parts[0];
    out.d.N = N;
    const bool has_zp = parts[0]->zero_points != nullptr;
    if (parts[0]->precision == TBH_PREC_INT8) {
        for (int i = 0; i < n; ++i)
            if (parts[i]->layout != TBH_LAYOUT_KN_FLAT || parts[i]->data_bytes != K * parts[i]->N ||
                !(parts[i]->mode == TBH_MODE_PER_CHANNEL || parts[i]->mode == TBH_MODE_SYMMETRIC ||
                  parts[i]->mode == TBH_MODE_ASYMMETRIC))
                return set_error(TBH_E_UNSUPPORTED, "concatenated weights: INT8 parts must be the [K][N] runtime layout");
        out.data.resize((size_t)(K * N));
        out.scales.resize((size_t)N);
        if (has_zp) out.zp.resize((size_t)N);
        int64_t off = 0;
        for (int i = 0; i < n; ++i) {
            const tbh_qtensor_desc &d = *parts[i];
            for (int64_t k = 0; k < K; ++k)
                std::memcpy(&out.data[(size_t)(k * N + off)], d.data + k * d.N, (size_t)d.N);
            for (int64_t c = 0; c < d.N; ++c) {
                const int64_t si = d.mode == TBH_MODE_PER_CHANNEL ? c : 0;
                out.scales[(size_t)(off + c)] = d.scales[si];
                if (has_zp) out.zp[(size_t)(off + c)] = d.zero_points[si];
            }
            off += d.N;
        }
        out.d.mode = TBH_MODE_PER_CHANNEL;
        out.d.data_bytes = K * N;
        out.d.n_scales = N;
    } else if (parts[0]->layout == TBH_LAYOUT_KN_FLAT) {
        const int32_t gs = parts[0]->group_size;
        for (int i = 0; i < n; ++i)
            if (parts[i]->layout != TBH_LAYOUT_KN_FLAT || parts[i]->mode != TBH_MODE_INT4 ||
                parts[i]->group_size != gs || gs <= 0 || parts[i]->N % gs != 0 || gs % 2 != 0 ||
                parts[i]->data_bytes != K * parts[i]->N / 2)
                return set_error(TBH_E_UNSUPPORTED,
                                 "concatenated weights: runtime-layout INT4 parts need groups that tile N");
        out.data.resize((size_t)(K * N / 2));
        out.scales.resize((size_t)(K * N / gs));
        if (has_zp) out.zp.resize(out.scales.size());
        int64_t off = 0;   // in outputs
        for (int i = 0; i < n; ++i) {
            const tbh_qtensor_desc &d = *parts[i];
            const int64_t ng = d.N / gs;
            for (int64_t k = 0; k < K; ++k) {
                std::memcpy(&out.data[(size_t)((k * N + off) / 2)], d.data + k * d.N / 2, (size_t)(d.N / 2));
                std::memcpy(&out.scales[(size_t)((k * N + off) / gs)], d.scales + k * ng, (size_t)ng * sizeof(float));
                if (has_zp) std::memcpy(&out.zp[(size_t)((k * N + off) / gs)], d.zero_points + k * ng, (size_t)ng);
            }
            off += d.N;
        }
        out.d.data_bytes = (int64_t)out.data.size();
        out.d.n_scales = (int64_t)out.scales.size();
    } else {
        const int32_t gs = parts[0]->group_size;
        for (int i = 0; i < n; ++i)
            if (parts[i]->layout != TBH_LAYOUT_NK_FLAT || parts[i]->mode != TBH_MODE_INT4 ||
                parts[i]->group_size != gs || gs <= 0 || K % gs != 0 || (K * parts[i]->N) % 2 != 0 ||
                parts[i]->data_bytes != K * parts[i]->N / 2)
                return set_error(TBH_E_UNSUPPORTED,
                                 "concatenated weights: INT4 parts must be the converter layout with K-groups");
        for (int i = 0; i < n; ++i) {
            const tbh_qtensor_desc &d = *parts[i];
            out.data.insert(out.data.end(), d.data, d.data + d.data_bytes);
            out.scales.insert(out.scales.end(), d.scales, d.scales + d.n_scales);
            if (has_zp) out.zp.insert(out.zp.end(), d.zero_points, d.zero_points + d.n_scales);
        }
        out.d.data_bytes = (int64_t)out.data.size();
        out.d.n_scales = (int64_t)out.scales.size();
    }
    out.d.data = out.data.data();
    out.d.scales = out.scales.data();
    out.d.zero_points = has_zp ? out.zp.data() : nullptr;
    out.d.n_zero_points = has_zp ? out.d.n_scales : 0;
    return TBH_OK;
}

// Reorders a two-part concatenation [A | B] (N = 2 * half outputs) so that
// output 2j is A's j and output 2j + 1 is B's j.
void interleave_halves(OwnedDesc &od) {
    const int64_t K = od.d.K, N = od.d.N, half = N / 2;
    const bool has_zp = !od.zp.empty();
    if (od.d.precision == TBH_PREC_INT8) {   // [K][N] bytes, one scale per column
        std::vector<int8_t> data(od.data.size());
        for (int64_t k = 0; k < K; ++k)
            for (int64_t j = 0; j < half; ++j) {
                data[(size_t)(k * N + 2 * j)] = od.data[(size_t)(k * N + j)];
                data[(size_t)(k * N + 2 * j + 1)] = od.data[(size_t)(k * N + half + j)];
            }
        od.data.swap(data);
        std::vector<float> sc(od.scales.size());
        std::vector<int8_t> zp(od.zp.size());
        for (int64_t j = 0; j < half; ++j) {
            sc[(size_t)(2 * j)] = od.scales[(size_t)j];
            sc[(size_t)(2 * j + 1)] = od.scales[(size_t)(half + j)];
            if (has_zp) {
                zp[(size_t)(2 * j)] = od.zp[(size_t)j];
                zp[(size_t)(2 * j + 1)] = od.zp[(size_t)(half + j)];
            }
        }
        od.scales.swap(sc);
        od.zp.swap(zp);
    } else {   // converter layout: N rows of K / 2 bytes, G = K / gs scales per row
        const int64_t rb = K / 2, G = K / od.d.group_size;
        std::vector<int8_t> data(od.data.size());
        std::vector<float> sc(od.scales.size());
        std::vector<int8_t> zp(od.zp.size());
        for (int64_t j = 0; j < half; ++j)
            for (int p = 0; p < 2; ++p) {
                const int64_t src = p * half + j, dst = 2 * j + p;
                std::memcpy(&data[(size_t)(dst * rb)], &od.data[(size_t)(src * rb)], (size_t)rb);
                std::memcpy(&sc[(size_t)(dst * G)], &od.scales[(size_t)(src * G)], (size_t)G * sizeof(float));
                if (has_zp) std::memcpy(&zp[(size_t)(dst * G)], &od.zp[(size_t)(src * G)], (size_t)G);
            }
        od.data.swap(data);
        od.scales.swap(sc);
        od.zp.swap(zp);
    }
    od.d.data = od.data.data();
    od.d.scales = od.scales.data();
    od.d.zero_points = has_zp ? od.zp.data() : nullptr;
}

// interleave: two parts of equal N whose outputs alternate (gate|up rows).
tbh_status make_weight(tbh_decoder *dec, const tbh_qtensor_desc *const *parts, int n, int64_t K,
                       int64_t N, tbh_weight **out, bool interleave = false) {
    if (interleave && n == 2 && parts[0] && parts[1] && parts[0]->precision == TBH_PREC_INT4 &&
        parts[0]->layout == TBH_LAYOUT_KN_FLAT) {
        // runtime-layout INT4: a block's rows must share their N-block's
        // scale per k, so the pair is built with one scale table per part
        if (parts[0]->K != K || parts[1]->K != K || parts[0]->N + parts[1]->N != N)
            return set_error(TBH_E_INVALID, "decoder: projection shape mismatch");
        tbh_status st = create_ngroup_pair(dec->dev, parts[0], parts[1], out);
        if (st != TBH_OK) return st;
        if (!gemv_fused_supported(**out))
            return set_error(TBH_E_UNSUPPORTED, "decoder: gate|up projection needs the burst GEMV path");
        return TBH_OK;
    }
    OwnedDesc od;
    tbh_status st = n == 1 ? TBH_OK : concat_n(parts, n, od);
    if (st != TBH_OK) return st;
    if (interleave) {
        if (n != 2 || parts[0]->N != parts[1]->N)
            return set_error(TBH_E_INVALID, "decoder: gate and up projections differ in shape");
        interleave_halves(od);
    }
    const tbh_qtensor_desc *d = n == 1 ? parts[0] : &od.d;
    if (!d) return set_error(TBH_E_INVALID, "decoder: NULL weight");
    if (d->K != K || d->N != N) return set_error(TBH_E_INVALID, "decoder: projection shape mismatch");
    st = tbh_weight_create(dec->dev, d, out);
    if (st != TBH_OK) return st;
    if (!gemv_fused_supported(**out))
        return set_error(TBH_E_UNSUPPORTED,
                         "decoder: projection needs the burst GEMV path (INT8 rows or INT4 K-groups, "
                         "no zero points, K <= 64*6 chunks)");
    return TBH_OK;
}

template <class T>
tbh_status dmalloc(tbh_decoder *d, T **p, size_t count) {
    void *m = nullptr;
    hipError_t e = hipMalloc(&m, count * sizeof(T));
    if (e != hipSuccess) return set_error(TBH_E_OOM, "decoder: device allocation failed");
    d->allocs.push_back(m);
    *p = (T *)m;
    return TBH_OK;
}

}  // namespace
}  // namespace tbh

using namespace tbh;

extern "C" {

tbh_status tbh_weight_create_concat(tbh_device *dev, int32_t n, const tbh_qtensor_desc *const *parts,
                                    tbh_weight **out) {
    if (!dev || !parts || !out) return set_error(TBH_E_INVALID, "tbh_weight_create_concat: NULL argument");
    if (n < 1) return set_error(TBH_E_INVALID, "tbh_weight_create_concat: n < 1");
    *out = nullptr;
    if (n == 1) return tbh_weight_create(dev, parts[0], out);
    OwnedDesc od;
    const tbh_status st = concat_n(parts, n, od);
    if (st != TBH_OK) return st;
    return tbh_weight_create(dev, &od.d, out);
}

tbh_status tbh_decoder_destroy(tbh_decoder *d) {
    if (!d) return TBH_OK;
    (void)hipSetDevice(d->dev->ordinal);
    for (auto &l : d->layers) {
        tbh_weight_destroy(l.qkv);
        tbh_weight_destroy(l.o);
        tbh_weight_destroy(l.gu);
        tbh_weight_destroy(l.down);
    }
    tbh_weight_destroy(d->lm_head);
    for (void *p : d->allocs) (void)hipFree(p);
    delete d;
    return TBH_OK;
}

tbh_status tbh_decoder_create(tbh_device *dev, const tbh_decoder_config *cfg, const float *embeddings,
                              const float *final_norm, const tbh_qtensor_desc *lm_head,
                              tbh_decoder **out) {
    if (!out) return set_error(TBH_E_INVALID, "tbh_decoder_create: out is NULL");
    *out = nullptr;
    if (!dev || !cfg || !embeddings || !final_norm || !lm_head)
        return set_error(TBH_E_INVALID, "tbh_decoder_create: NULL argument");
    const tbh_decoder_config &c = *cfg;
    if (c.num_layers < 1 || c.hidden < 1 || c.num_heads < 1 || c.num_kv_heads < 1 || c.vocab < 1 ||
        c.intermediate < 1 || c.max_seq < 1)
        return set_error(TBH_E_INVALID, "tbh_decoder_create: non-positive dimension");
    if (c.hidden % c.num_heads != 0 || c.num_heads % c.num_kv_heads != 0)
        return set_error(TBH_E_INVALID, "tbh_decoder_create: heads must divide hidden and each other");
    const int32_t hd = c.hidden / c.num_heads;
    if (hd % 4 != 0 || hd > 256 || c.hidden % 4 != 0 || c.intermediate % 4 != 0 ||
        (c.num_heads / c.num_kv_heads) * hd > 1024)
        return set_error(TBH_E_UNSUPPORTED,
                         "tbh_decoder_create: needs head_dim % 4 == 0, head_dim <= 256, hidden and "
                         "intermediate multiples of 4, (heads per KV head) * head_dim <= 1024");
    if (hd > kMaxHd || hd % 16 != 0)
        return set_error(TBH_E_UNSUPPORTED,
                         "tbh_decoder_create: attention needs head_dim a multiple of 16, <= 128");
    std::unique_ptr<tbh_decoder> d(new tbh_decoder);
    d->dev = dev;
    d->cfg = c;
    d->head_dim = hd;
    d->kv_dim = hd * c.num_kv_heads;
    d->qkv_dim = c.hidden + 2 * d->kv_dim;
    d->layers.resize((size_t)c.num_layers);
    if (hipSetDevice(dev->ordinal) != hipSuccess) return set_error(TBH_E_HIP, "hipSetDevice");

    tbh_status st;
    const size_t H = (size_t)c.hidden, L = (size_t)c.num_layers;
    if ((st = dmalloc(d.get(), &d->emb, (size_t)c.vocab * H)) != TBH_OK) return st;
    if ((st = dmalloc(d.get(), &d->norms, (2 * L + 1) * H)) != TBH_OK) return st;
    const size_t cache = L * (size_t)c.max_seq * (size_t)d->kv_dim;
    if ((st = dmalloc(d.get(), &d->kcache, cache)) != TBH_OK) return st;
    if ((st = dmalloc(d.get(), &d->vcache, cache)) != TBH_OK) return st;
    if ((st = dmalloc(d.get(), &d->h, H)) != TBH_OK) return st;
    if ((st = dmalloc(d.get(), &d->qkv, (size_t)d->qkv_dim)) != TBH_OK) return st;
    if ((st = dmalloc(d.get(), &d->ctx, H)) != TBH_OK) return st;
    if ((st = dmalloc(d.get(), &d->gu, 2 * (size_t)c.intermediate)) != TBH_OK) return st;
    if ((st = dmalloc(d.get(), &d->logits, (size_t)c.vocab)) != TBH_OK) return st;
    if ((st = dmalloc(d.get(), &d->pos, 2)) != TBH_OK) return st;
    d->attn_splits = (c.max_seq + attn_range(d->head_dim) - 1) / attn_range(d->head_dim);
    if ((st = dmalloc(d.get(), &d->attn_o, (size_t)d->attn_splits * H)) != TBH_OK) return st;
    if ((st = dmalloc(d.get(), &d->attn_ml, (size_t)d->attn_splits * c.num_heads)) != TBH_OK) return st;
    // RoPE frequencies theta_i = base^(-2i / hd) in fp32 (ModelRunner.swift:476-479)
    std::vector<float> theta((size_t)hd / 2);
    for (int32_t i = 0; i < hd / 2; ++i) theta[(size_t)i] = std::pow(c.rope_base, -((float)(2 * i) / (float)hd));
    if ((st = dmalloc(d.get(), &d->rope_theta, theta.size())) != TBH_OK) return st;
    if (hipMemcpy(d->rope_theta, theta.data(), theta.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
        return set_error(TBH_E_HIP, "tbh_decoder_create: upload RoPE frequencies");
    if (hipMemcpy(d->emb, embeddings, (size_t)c.vocab * H * sizeof(float), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d->norms + 2 * L * H, final_norm, H * sizeof(float), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(d->pos, 0, 2 * sizeof(int32_t)) != hipSuccess ||
        hipMemset(d->kcache, 0, cache * sizeof(float)) != hipSuccess ||
        hipMemset(d->vcache, 0, cache * sizeof(float)) != hipSuccess)
        return set_error(TBH_E_HIP, "tbh_decoder_create: upload");
    const tbh_qtensor_desc *lm[1] = {lm_head};
    if ((st = make_weight(d.get(), lm, 1, c.hidden, c.vocab, &d->lm_head)) != TBH_OK) {
        tbh_decoder_destroy(d.release());
        return st;
    }
    *out = d.release();
    return TBH_OK;
}

tbh_status tbh_decoder_set_layer(tbh_decoder *d, int32_t layer, const float *input_norm,
                                 const float *post_attention_norm, const tbh_qtensor_desc *q,
                                 const tbh_qtensor_desc *k, const tbh_qtensor_desc *v,
                                 const tbh_qtensor_desc *o, const tbh_qtensor_desc *gate,
                                 const tbh_qtensor_desc *up, const tbh_qtensor_desc *down) {
    if (!d) return set_error(TBH_E_INVALID, "tbh_decoder_set_layer: decoder is NULL");
    const tbh_decoder_config &c = d->cfg;
    if (layer < 0 || layer >= c.num_layers) return set_error(TBH_E_INVALID, "tbh_decoder_set_layer: layer");
    if (!input_norm || !post_attention_norm)
        return set_error(TBH_E_INVALID, "tbh_decoder_set_layer: NULL norm weight");
    if (hipSetDevice(d->dev->ordinal) != hipSuccess) return set_error(TBH_E_HIP, "hipSetDevice");
    auto &L = d->layers[(size_t)layer];
    tbh_weight *nw[4] = {nullptr, nullptr, nullptr, nullptr};
    const tbh_qtensor_desc *qkv[3] = {q, k, v};
    const tbh_qtensor_desc *od[1] = {o};
    const tbh_qtensor_desc *gu[2] = {gate, up};
    const tbh_qtensor_desc *dd[1] = {down};
    tbh_status st = make_weight(d, qkv, 3, c.hidden, d->qkv_dim, &nw[0]);
    if (st == TBH_OK) st = make_weight(d, od, 1, c.hidden, c.hidden, &nw[1]);
    if (st == TBH_OK) st = make_weight(d, gu, 2, c.hidden, 2 * (int64_t)c.intermediate, &nw[2], true);
    if (st == TBH_OK) st = make_weight(d, dd, 1, c.intermediate, c.hidden, &nw[3]);
    const size_t H = (size_t)c.hidden;
    if (st == TBH_OK &&
        (hipMemcpy(d->norms + (2 * (size_t)layer) * H, input_norm, H * sizeof(float), hipMemcpyHostToDevice) !=
             hipSuccess ||
         hipMemcpy(d->norms + (2 * (size_t)layer + 1) * H, post_attention_norm, H * sizeof(float),
                   hipMemcpyHostToDevice) != hipSuccess))
        st = set_error(TBH_E_HIP, "tbh_decoder_set_layer: upload norms");
    if (st != TBH_OK) {
        for (auto *w : nw) tbh_weight_destroy(w);
        return st;
    }
    tbh_weight_destroy(L.qkv);
    tbh_weight_destroy(L.o);
    tbh_weight_destroy(L.gu);
    tbh_weight_destroy(L.down);
    L.qkv = nw[0];
    L.o = nw[1];
    L.gu = nw[2];
    L.down = nw[3];
    return TBH_OK;
}

tbh_status tbh_decoder_set_position(tbh_decoder *d, int32_t position) {
    if (!d) return set_error(TBH_E_INVALID, "tbh_decoder_set_position: decoder is NULL");
    if (position < 0 || position > d->cfg.max_seq)
        return set_error(TBH_E_INVALID, "tbh_decoder_set_position: position out of range");
    if (hipSetDevice(d->dev->ordinal) != hipSuccess) return set_error(TBH_E_HIP, "hipSetDevice");
    const int32_t v[2] = {position, 0};
    if (hipMemcpy(d->pos, v, sizeof(v), hipMemcpyHostToDevice) != hipSuccess)
        return set_error(TBH_E_HIP, "tbh_decoder_set_position");
    return TBH_OK;
}

tbh_status tbh_decoder_get_position(const tbh_decoder *d, int32_t *position) {
    if (!d || !position) return set_error(TBH_E_INVALID, "tbh_decoder_get_position: NULL argument");
    if (hipSetDevice(d->dev->ordinal) != hipSuccess) return set_error(TBH_E_HIP, "hipSetDevice");
    int32_t v[2];
    if (hipMemcpy(v, d->pos, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess)
        return set_error(TBH_E_HIP, "tbh_decoder_get_position");
    if (v[1]) return set_error(TBH_E_INVALID, "decoder: a step ran with a full KV cache (position >= max_seq)");
    *position = v[0];
    return TBH_OK;
}

tbh_status tbh_decoder_step_device(tbh_decoder *d, int32_t token, float *logits, void *stream) {
    if (!d) return set_error(TBH_E_INVALID, "tbh_decoder_step_device: decoder is NULL");
    const tbh_decoder_config &c = d->cfg;
    if (token < 0 || token >= c.vocab)
        return set_error(TBH_E_INVALID, "Token id out of bounds (ModelWeights.swift:165)");
    for (const auto &l : d->layers)
        if (!l.qkv || !l.o || !l.gu || !l.down)
            return set_error(TBH_E_INVALID, "tbh_decoder_step_device: a layer has no weights");
    if (hipSetDevice(d->dev->ordinal) != hipSuccess) return set_error(TBH_E_HIP, "hipSetDevice");
    hipStream_t s = (hipStream_t)stream;
    const size_t H = (size_t)c.hidden;
    float *out = logits ? logits : d->logits;
    AttnParams ap{};
    ap.qkv = d->qkv;
    ap.ctx = d->ctx;
    ap.pos = d->pos;
    ap.nh = c.num_heads;
    ap.nkv = c.num_kv_heads;
    ap.hd = d->head_dim;
    ap.kvd = d->kv_dim;
    ap.hidden = c.hidden;
    ap.max_seq = c.max_seq;
    ap.rope_base = c.rope_base;
    ap.part_o = d->attn_o;
    ap.part_ml = d->attn_ml;
    ap.theta = d->rope_theta;
    ap.rep = c.num_heads / c.num_kv_heads;
    {
        static const int wpb_force = [] {
            const char *v = std::getenv("TBH_ATTN_WPB");
            return v && *v ? std::atoi(v) : 0;
        }();
        ap.wpb = wpb_force == 4 ? 4 : std::min(4, ap.rep);
    }
    ap.splits = d->attn_splits;
    ap.scale = 1.0f / std::sqrt((float)d->head_dim);
    hipError_t e = hipSuccess;
    for (int32_t l = 0; l < c.num_layers && e == hipSuccess; ++l) {
        const auto &L = d->layers[(size_t)l];
        const float *g_in = d->norms + (2 * (size_t)l) * H, *g_post = g_in + H;
        // layer 0 reads the token's embedding row and stores it as the
        // residual stream h (ModelRunner.swift:170); later layers read h
        FusedGemvArgs qa{d->h, g_in, c.rms_eps, d->qkv, PRO_RMSNORM, EPI_STORE};
        if (l == 0) {
            qa.x = d->emb + (size_t)token * H;
            qa.x_copy = d->h;
        }
        e = launch_gemv_fused(*L.qkv, qa, s);
        if (e != hipSuccess) break;
        ap.kcache = d->kcache + (size_t)l * c.max_seq * d->kv_dim;
        ap.vcache = d->vcache + (size_t)l * c.max_seq * d->kv_dim;
        e = launch_attention(ap, s);
        if (e != hipSuccess) break;
        e = launch_gemv_fused(*L.o, FusedGemvArgs{d->ctx, nullptr, 0.0f, d->h, PRO_NONE, EPI_ACCUMULATE}, s);
        if (e != hipSuccess) break;
        // gate and up rows interleaved: the epilogue writes silu(gate) * up
        e = launch_gemv_fused(*L.gu, FusedGemvArgs{d->h, g_post, c.rms_eps, d->gu, PRO_RMSNORM, EPI_SILU_PAIR}, s);
        if (e != hipSuccess) break;
        e = launch_gemv_fused(*L.down, FusedGemvArgs{d->gu, nullptr, 0.0f, d->h, PRO_NONE, EPI_ACCUMULATE}, s);
    }
    if (e == hipSuccess) {
        // the LM head also advances the position: every launch that reads it
        // (the layers' attention) precedes it on the stream
        FusedGemvArgs la{d->h, d->norms + 2 * (size_t)c.num_layers * H, c.rms_eps, out, PRO_RMSNORM, EPI_STORE};
        la.advance = d->pos;
        e = launch_gemv_fused(*d->lm_head, la, s);
    }
    if (e != hipSuccess) return hip_error(e, "decoder step launch");
    return TBH_OK;
}

tbh_status tbh_decoder_step(tbh_decoder *d, int32_t token, float *logits) {
    if (!d || !logits) return set_error(TBH_E_INVALID, "tbh_decoder_step: NULL argument");
    std::lock_guard<std::mutex> lock(d->dev->mu);
    tbh_status st = tbh_decoder_step_device(d, token, nullptr, d->dev->stream);
    if (st != TBH_OK) return st;
    if (hipMemcpyAsync(logits, d->logits, (size_t)d->cfg.vocab * sizeof(float), hipMemcpyDeviceToHost,
                       d->dev->stream) != hipSuccess ||
        hipStreamSynchronize(d->dev->stream) != hipSuccess)
        return set_error(TBH_E_HIP, "tbh_decoder_step: copy logits");
    int32_t pos;
    return tbh_decoder_get_position(d, &pos);
}

}  // extern "C"

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
//     gu  = W_gate|up . rmsnorm(h) * g_post                    (:436-451)
//     h += W_down . (silu(gate) * up)                          (:449-457)
//   logits = W_lm . rmsnorm(h) * g_final                       (:186-199)
//
// Six launches per layer: Q|K|V and gate|up are each one weight
// (concatenated along N at set-up), RMSNorm and SiLU*up run in the GEMV's x
// staging, the residual adds in its epilogue, and two attention kernels do
// RoPE, the cache append, softmax over position slices and their combination.  The token position lives
// in device memory and the step ends with a one-thread kernel that advances
// it, so a captured step replays as the next one.
#include <cmath>
#include <cstring>
#include <memory>
#include <vector>

#include "tbh_internal.h"

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
    int32_t *pos = nullptr;      // [0] position, [1] overflow flag
    float *attn_part = nullptr;  // attention slice partials
    int32_t attn_splits = 1;
    std::vector<void *> allocs;
};

namespace tbh {
namespace {

struct AttnParams {
    const float *qkv;
    float *kcache, *vcache;  // this layer
    float *ctx;
    int32_t *pos;            // [0] position, [1] overflow flag
    float *part;             // [num_heads][S][head_dim + 2] partial (max, sum, context)
    int32_t nh, nkv, hd, kvd, hidden, max_seq, S;
    float rope_base, scale;
};

constexpr int kMaxSplits = 16;

// LDS floats of one attention block: q [rep][hd+4], K tile [tc][hd+4],
// V tile [tc][hd], scores [rep][tc], new k and v [hd] each, per-head running
// max / sum / rescale [rep] each.  Rows of q and K are padded by four floats
// (16 bytes, so rows stay float4-aligned) to spread the (head, position) dot
// products over the banks.
__host__ __device__ inline int attn_tile(int hd) { return hd <= 64 ? 64 : 4096 / hd; }
__host__ __device__ inline int attn_lds_floats(int rep, int hd) {
    const int tc = attn_tile(hd);
    return rep * (hd + 4) + tc * (hd + 4) + tc * hd + rep * tc + 2 * hd + 3 * rep;
}

// Grid (num_kv_heads, S): block (g, s) serves every query head of KV group g
// (ModelRunner.swift:524-536: kvHead = head / repeats) over the s-th slice of
// positions 0..pos, with a running max / sum / context per head (the
// softmax of :545-551 taken over the slice), K and V tiles staged in LDS once
// for all heads of the group, and writes its (max, sum, context) partials;
// attention_combine merges them.  The block whose slice holds `pos` appends
// the RoPE'd k and the v of position pos (:470-494, :503-516) to the cache;
// every block computes its own copy of them, so none waits for another.
__global__ __launch_bounds__(256) void attention_step(const AttnParams a) {
    extern __shared__ float lds[];
    const int g = blockIdx.x, sl = blockIdx.y, tid = threadIdx.x;
    const int rep = a.nh / a.nkv, hd = a.hd, hp = hd + 4, tc = attn_tile(hd);
    float *qs = lds;                    // [rep][hp]
    float *kb = qs + rep * hp;          // [tc][hp]
    float *vb = kb + tc * hp;           // [tc][hd]
    float *sc = vb + tc * hd;           // [rep][tc]
    float *kn = sc + rep * tc;          // [hd] new k (RoPE'd)
    float *vn = kn + hd;                // [hd] new v
    float *mrun = vn + hd;              // [rep] running max
    float *lrun = mrun + rep;           // [rep] running sum
    float *alpha = lrun + rep;          // [rep] rescale of this tile

    const int pos = a.pos[0];
    if (pos < 0 || pos >= a.max_seq) {  // cache full: flag it, write nothing
        if (g == 0 && sl == 0 && tid == 0) a.pos[1] = 1;
        return;
    }
    const int n = pos + 1;
    const int chunk = (n + a.S - 1) / a.S;
    const int t0 = min(n, sl * chunk), t1 = min(n, t0 + chunk);

    // RoPE (interleaved pairs, theta = base^(-i/hd), fp32) on the group's q
    // heads and on the new k; copy the new v
    const float *qin = a.qkv + (int64_t)g * rep * hd;
    const float *kin = a.qkv + a.hidden + g * hd;
    const float *vin = a.qkv + a.hidden + a.kvd + g * hd;
    for (int j = tid; j < (rep + 1) * (hd / 2); j += 256) {
        const int r = j / (hd / 2), i = 2 * (j % (hd / 2));
        const float theta = powf(a.rope_base, -((float)i / (float)hd));
        const float ang = (float)pos * theta;
        const float c = cosf(ang), s = sinf(ang);
        const float *src = r < rep ? qin + r * hd : kin;
        float *dst = r < rep ? qs + r * hp : kn;
        const float x0 = src[i], x1 = src[i + 1];
        dst[i] = x0 * c - x1 * s;
        dst[i + 1] = x0 * s + x1 * c;
    }
    for (int d = tid; d < hd; d += 256) vn[d] = vin[d];
    for (int r = tid; r < rep; r += 256) {
        mrun[r] = -INFINITY;
        lrun[r] = 0.0f;
    }
    __syncthreads();
    if (pos >= t0 && pos < t1)
        for (int d = tid; d < hd; d += 256) {
            a.kcache[(int64_t)pos * a.kvd + g * hd + d] = kn[d];
            a.vcache[(int64_t)pos * a.kvd + g * hd + d] = vn[d];
        }

    // this thread's context accumulator: head r4 = tid / (hd/4), dims 4*(tid % (hd/4))..+3
    // (rep * hd <= 1024: one float4 per thread)
    const int pairs4 = rep * hd / 4;
    float4 acc = float4{0.f, 0.f, 0.f, 0.f};
    const int lane32 = tid & 31;

    for (int c0 = t0; c0 < t1; c0 += tc) {
        const int cl = min(tc, t1 - c0);
        // K, V rows of the tile -> LDS.  All of a thread's global loads go out
        // first (tc * hd <= 4096: at most four float4 of each per thread, on
        // clamped in-range rows); row pos is then taken from this block's copy.
        const int hd4 = hd / 4, nld = cl * hd4;
        float4 kv[4], vv[4];
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int j = min(tid + 256 * it, nld - 1);
            const int64_t row = (int64_t)(c0 + j / hd4) * a.kvd + g * hd + 4 * (j % hd4);
            kv[it] = *(const float4 *)&a.kcache[row];
            vv[it] = *(const float4 *)&a.vcache[row];
        }
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int j = tid + 256 * it;
            if (j < nld) {
                const int t = j / hd4, d4 = j % hd4;
                const bool cur = c0 + t == pos;
                const float4 kl = *(const float4 *)&kn[4 * d4], vl = *(const float4 *)&vn[4 * d4];
                *(float4 *)&kb[t * hp + 4 * d4] = cur ? kl : kv[it];
                *(float4 *)&vb[t * hd + 4 * d4] = cur ? vl : vv[it];
            }
        }
        __syncthreads();
        // scores of the tile, one (head, position) per thread, d in order
        for (int j = tid; j < rep * cl; j += 256) {
            const int r = j / cl, t = j % cl;
            const float4 *qr = (const float4 *)&qs[r * hp], *kr = (const float4 *)&kb[t * hp];
            float dot = 0.0f;
#pragma unroll 4
            for (int d4 = 0; d4 < hd / 4; ++d4) {
                const float4 q = qr[d4], k = kr[d4];
                dot = __builtin_fmaf(q.x, k.x, dot);
                dot = __builtin_fmaf(q.y, k.y, dot);
                dot = __builtin_fmaf(q.z, k.z, dot);
                dot = __builtin_fmaf(q.w, k.w, dot);
            }
            sc[r * tc + t] = dot * a.scale;
        }
        __syncthreads();
        // running max and sum per head, 32 lanes per head; sc <- exp(score - max)
        for (int r0 = 0; r0 < rep; r0 += 8) {
            const int r = r0 + (tid >> 5);
            float mx = -INFINITY;
            if (r < rep)
                for (int t = lane32; t < cl; t += 32) mx = fmaxf(mx, sc[r * tc + t]);
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 32));
            float l = 0.0f;
            if (r < rep) {
                mx = fmaxf(mx, mrun[r]);
                for (int t = lane32; t < cl; t += 32) {
                    const float e = expf(sc[r * tc + t] - mx);
                    sc[r * tc + t] = e;
                    l += e;
                }
            }
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) l += __shfl_xor(l, o, 32);
            __syncthreads();  // every lane has read mrun[r] before it changes
            if (r < rep && lane32 == 0) {
                const float f = expf(mrun[r] - mx);
                alpha[r] = f;
                lrun[r] = lrun[r] * f + l;
                mrun[r] = mx;
            }
        }
        __syncthreads();
        if (tid < pairs4) {
            const int r = tid / (hd / 4), d = 4 * (tid % (hd / 4));
            const float f = alpha[r];
            float4 v = float4{acc.x * f, acc.y * f, acc.z * f, acc.w * f};
#pragma unroll 4
            for (int t = 0; t < cl; ++t) {
                const float p = sc[r * tc + t];
                const float4 x = *(const float4 *)&vb[t * hd + d];
                v.x = __builtin_fmaf(p, x.x, v.x);
                v.y = __builtin_fmaf(p, x.y, v.y);
                v.z = __builtin_fmaf(p, x.z, v.z);
                v.w = __builtin_fmaf(p, x.w, v.w);
            }
            acc = v;
        }
        __syncthreads();
    }

    // partials of this slice
    const int W = hd + 2;
    if (tid < pairs4) {
        const int r = tid / (hd / 4), d = 4 * (tid % (hd / 4));
        float *pp = a.part + ((int64_t)(g * rep + r) * a.S + sl) * W;
        pp[2 + d] = acc.x;
        pp[3 + d] = acc.y;
        pp[4 + d] = acc.z;
        pp[5 + d] = acc.w;
        if (d == 0) {
            pp[0] = mrun[r];
            pp[1] = lrun[r];
        }
    }
}

// Combines the S slices of attention_step into the context of one query head
// per block: context = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s.  A
// kernel of its own, so the slices' writes are visible without device-scope
// fences in the slice kernel.
__global__ __launch_bounds__(256) void attention_combine(const AttnParams a) {
    const int h = blockIdx.x, W = a.hd + 2;
    if (a.pos[1]) return;  // the slice kernel saw a full cache and wrote nothing
    const float *pp = a.part + (int64_t)h * a.S * W;
    for (int d = threadIdx.x; d < a.hd; d += 256) {
        float m[kMaxSplits], l[kMaxSplits], c[kMaxSplits];
#pragma unroll
        for (int j = 0; j < kMaxSplits; ++j) {
            const bool in = j < a.S;
            const int jj = in ? j : 0;
            const float mj = pp[jj * W], lj = pp[jj * W + 1], cj = pp[jj * W + 2 + d];
            m[j] = in ? mj : -INFINITY;
            l[j] = in ? lj : 0.0f;
            c[j] = in ? cj : 0.0f;
        }
        float M = -INFINITY;
#pragma unroll
        for (int j = 0; j < kMaxSplits; ++j) M = fmaxf(M, m[j]);
        float L = 0.0f, C = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxSplits; ++j) {
            const float f = m[j] == -INFINITY ? 0.0f : expf(m[j] - M);
            L = __builtin_fmaf(f, l[j], L);
            C = __builtin_fmaf(f, c[j], C);
        }
        a.ctx[h * a.hd + d] = C / L;
    }
}

__global__ void embed_row(const float *emb, int32_t token, int32_t hidden, float *h) {
    const int64_t base = (int64_t)token * hidden;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
        h[i] = emb[base + i];
}

__global__ void advance_position(int32_t *pos) {
    if (threadIdx.x == 0 && blockIdx.x == 0) pos[0] += 1;
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
// 0, even K * N_i), where concatenation is of the flat arrays.
tbh_status concat_n(const tbh_qtensor_desc *const *parts, int n, OwnedDesc &out) {
    for (int i = 0; i < n; ++i) {
        const tbh_qtensor_desc *d = parts[i];
        if (!d || !d->data || !d->scales) return set_error(TBH_E_INVALID, "decoder: NULL weight");
        if (d->K != parts[0]->K || d->precision != parts[0]->precision)
            return set_error(TBH_E_INVALID, "decoder: concatenated weights differ in K or precision");
        if (d->n_scales != expected_scales(*d))
            return set_error(TBH_E_INVALID, "decoder: scale count does not match mode/shape");
        if ((d->zero_points != nullptr) != (parts[0]->zero_points != nullptr))
            return set_error(TBH_E_UNSUPPORTED, "decoder: zero points on some parts only");
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
                return set_error(TBH_E_UNSUPPORTED, "decoder: INT8 weights must be [K][N] runtime layout");
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
    } else {
        const int32_t gs = parts[0]->group_size;
        for (int i = 0; i < n; ++i)
            if (parts[i]->layout != TBH_LAYOUT_NK_FLAT || parts[i]->mode != TBH_MODE_INT4 ||
                parts[i]->group_size != gs || gs <= 0 || K % gs != 0 || (K * parts[i]->N) % 2 != 0 ||
                parts[i]->data_bytes != K * parts[i]->N / 2)
                return set_error(TBH_E_UNSUPPORTED,
                                 "decoder: INT4 weights must be the converter layout with K-groups");
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

tbh_status make_weight(tbh_decoder *dec, const tbh_qtensor_desc *const *parts, int n, int64_t K,
                       int64_t N, tbh_weight **out) {
    OwnedDesc od;
    tbh_status st = n == 1 ? TBH_OK : concat_n(parts, n, od);
    if (st != TBH_OK) return st;
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
    {
        const int64_t lds = (int64_t)attn_lds_floats(c.num_heads / c.num_kv_heads, hd) * (int64_t)sizeof(float);
        if (lds > 64 * 1024)
            return set_error(TBH_E_UNSUPPORTED, "tbh_decoder_create: attention tile exceeds 64 KiB of LDS");
    }
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
    // attention slices: up to 256 blocks per launch, at least 8 positions each
    d->attn_splits =
        std::max(1, std::min({kMaxSplits, 256 / c.num_kv_heads, std::max(1, c.max_seq / 8)}));
    const size_t part = (size_t)c.num_heads * d->attn_splits * (hd + 2);
    if ((st = dmalloc(d.get(), &d->attn_part, part)) != TBH_OK) return st;
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
    if (st == TBH_OK) st = make_weight(d, gu, 2, c.hidden, 2 * (int64_t)c.intermediate, &nw[2]);
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
    hipLaunchKernelGGL(embed_row, dim3((unsigned)((H + 255) / 256)), dim3(256), 0, s, d->emb, token,
                       c.hidden, d->h);
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
    ap.scale = 1.0f / std::sqrt((float)d->head_dim);
    ap.part = d->attn_part;
    ap.S = d->attn_splits;
    const size_t attn_lds =
        (size_t)attn_lds_floats(c.num_heads / c.num_kv_heads, d->head_dim) * sizeof(float);
    hipError_t e = hipSuccess;
    for (int32_t l = 0; l < c.num_layers && e == hipSuccess; ++l) {
        const auto &L = d->layers[(size_t)l];
        const float *g_in = d->norms + (2 * (size_t)l) * H, *g_post = g_in + H;
        e = launch_gemv_fused(*L.qkv, FusedGemvArgs{d->h, nullptr, g_in, c.rms_eps, d->qkv, 1, 0}, s);
        if (e != hipSuccess) break;
        ap.kcache = d->kcache + (size_t)l * c.max_seq * d->kv_dim;
        ap.vcache = d->vcache + (size_t)l * c.max_seq * d->kv_dim;
        hipLaunchKernelGGL(attention_step, dim3((unsigned)c.num_kv_heads, (unsigned)d->attn_splits),
                           dim3(256), attn_lds, s, ap);
        hipLaunchKernelGGL(attention_combine, dim3((unsigned)c.num_heads), dim3(256), 0, s, ap);
        e = launch_gemv_fused(*L.o, FusedGemvArgs{d->ctx, nullptr, nullptr, 0.0f, d->h, 0, 1}, s);
        if (e != hipSuccess) break;
        e = launch_gemv_fused(*L.gu, FusedGemvArgs{d->h, nullptr, g_post, c.rms_eps, d->gu, 1, 0}, s);
        if (e != hipSuccess) break;
        e = launch_gemv_fused(*L.down, FusedGemvArgs{d->gu, d->gu + c.intermediate, nullptr, 0.0f, d->h, 2, 1},
                              s);
    }
    if (e == hipSuccess)
        e = launch_gemv_fused(*d->lm_head,
                              FusedGemvArgs{d->h, nullptr, d->norms + 2 * (size_t)c.num_layers * H, c.rms_eps,
                                            out, 1, 0},
                              s);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(advance_position, dim3(1), dim3(64), 0, s, d->pos);
        e = hipGetLastError();
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

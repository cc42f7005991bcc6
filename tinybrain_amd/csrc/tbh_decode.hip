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
// Five launches per layer: Q|K|V and gate|up are each one weight
// (concatenated along N at set-up), RMSNorm and SiLU*up run in the GEMV's x
// staging, the residual adds in its epilogue, and one attention kernel does
// RoPE, the cache append, softmax and the context.  The token position lives
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
    std::vector<void *> allocs;
};

namespace tbh {
namespace {

struct AttnParams {
    const float *qkv;
    float *kcache, *vcache;  // this layer
    float *ctx;
    int32_t *pos;            // [0] position, [1] overflow flag
    int32_t nh, nkv, hd, kvd, hidden, max_seq;
    float rope_base, scale;
};

constexpr int kAttnThreads = 512;
constexpr int kAttnUnits = 20;  // K and V float4 loads per thread per batch
constexpr int kMaxHd = 128;

// Positions one batch covers: every thread loads kAttnUnits float4 of K and
// of V, so a batch is kAttnUnits * kAttnThreads / (hd / 4) positions.
__host__ __device__ inline int attn_batch(int hd) { return kAttnUnits * kAttnThreads / (hd / 4); }
// LDS floats: q, new k, new v [hd] each; wave partials [8]; per-thread
// context partials [kAttnThreads][4].
__host__ __device__ inline int attn_lds_floats(int hd) { return 3 * hd + 8 + 4 * kAttnThreads; }

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One block per query head h, KV group h / (num_heads / num_kv_heads)
// (ModelRunner.swift:524-536).  RoPE (interleaved pairs, theta =
// base^(-i/hd), fp32; :470-494) on q and the new k; the first head of each
// group appends the new k and v to the cache at pos (:503-516) and every
// block uses its own copy for position pos.  Positions go in batches: each
// thread issues all its K and V loads of a batch together (thread <-> one
// float4 column of hd/4 and positions tid/(hd/4) + i * 512/(hd/4)), scores
// them against q with the hd/4 lanes of a row summed by shuffles, and the
// block keeps a running max / sum / context (the softmax of :545-551) over
// the batches.  One launch produces the context; HBM latency is paid about
// once per batch.
__global__ __launch_bounds__(kAttnThreads) void attention_head(const AttnParams a) {
    extern __shared__ float lds[];
    const int h = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int rep = a.nh / a.nkv, kvh = h / rep, hd = a.hd, H4 = hd / 4;
    float *qs = lds;              // [hd]
    float *kn = qs + hd;          // [hd]
    float *vn = kn + hd;          // [hd]
    float *red = vn + hd;         // [8]
    float4 *cs = (float4 *)(red + 8);  // [kAttnThreads]

    // Everything that does not depend on the position is loaded before it:
    // this thread's RoPE pair and v element, and the first batch's K / V rows
    // 0..NB-1 (in bounds whatever the position; rows past it are masked).
    const int NB = attn_batch(hd);
    const int d4 = tid % H4, j0 = tid / H4, jstep = kAttnThreads / H4;
    const int64_t col = (int64_t)kvh * hd + 4 * d4;
    float4 kv[kAttnUnits], vv[kAttnUnits];
    auto load_batch = [&](int b0, int nb) {
#pragma unroll
        for (int i = 0; i < kAttnUnits; ++i) {
            const int64_t row = (int64_t)(b0 + min(j0 + i * jstep, nb - 1)) * a.kvd + col;
            kv[i] = *(const float4 *)&a.kcache[row];
            vv[i] = *(const float4 *)&a.vcache[row];
        }
    };
    load_batch(0, min(NB, a.max_seq));
    const float *qin = a.qkv + (int64_t)h * hd;
    const float *kin = a.qkv + a.hidden + kvh * hd;
    const float *vin = a.qkv + a.hidden + a.kvd + kvh * hd;
    const int jr = tid < hd ? tid : 0, ir = 2 * (jr % (hd / 2));
    const float *src = jr < hd / 2 ? qin : kin;
    const float x0 = src[ir], x1 = src[ir + 1];
    const float vx = vin[jr];

    const int pos = a.pos[0];
    if (pos < 0 || pos >= a.max_seq) {  // cache full: flag it, write nothing
        if (h == 0 && tid == 0) a.pos[1] = 1;
        return;
    }
    const int n = pos + 1;
    if (tid < hd) {
        const float theta = powf(a.rope_base, -((float)ir / (float)hd));
        const float ang = (float)pos * theta;
        const float c = cosf(ang), sn = sinf(ang);
        float *dst = jr < hd / 2 ? qs : kn;
        dst[ir] = x0 * c - x1 * sn;
        dst[ir + 1] = x0 * sn + x1 * c;
        vn[tid] = vx;
    }
    lds_barrier();
    if (h % rep == 0)
        for (int d = tid; d < hd; d += kAttnThreads) {
            a.kcache[(int64_t)pos * a.kvd + kvh * hd + d] = kn[d];
            a.vcache[(int64_t)pos * a.kvd + kvh * hd + d] = vn[d];
        }
    const float4 q4 = *(const float4 *)&qs[4 * d4];
    const float4 kn4 = *(const float4 *)&kn[4 * d4], vn4 = *(const float4 *)&vn[4 * d4];

    float M = -INFINITY, L = 0.0f;
    float4 C = float4{0.f, 0.f, 0.f, 0.f};
    for (int b0 = 0; b0 < n; b0 += NB) {
        const int nb = min(NB, n - b0);
        if (b0 > 0) load_batch(b0, nb);
        // scores of this thread's positions (the hd/4 lanes of a row summed)
        float sc[kAttnUnits];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < kAttnUnits; ++i) {
            const int j = j0 + i * jstep;
            const float4 k4 = b0 + j == pos ? kn4 : kv[i];
            float dot = q4.x * k4.x;
            dot = __builtin_fmaf(q4.y, k4.y, dot);
            dot = __builtin_fmaf(q4.z, k4.z, dot);
            dot = __builtin_fmaf(q4.w, k4.w, dot);
            for (int o = 1; o < H4; o <<= 1) dot += __shfl_xor(dot, o);
            sc[i] = j < nb ? dot * a.scale : -INFINITY;
            mx = fmaxf(mx, sc[i]);
        }
        // block max of the batch
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        if (lane == 0) red[wave] = mx;
        lds_barrier();
        mx = red[0];
        for (int w = 1; w < kAttnThreads / 64; ++w) mx = fmaxf(mx, red[w]);
        const float mnew = fmaxf(M, mx);
        const float f = expf(M - mnew);
        float ps = 0.0f;
        float4 cb = float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < kAttnUnits; ++i) {
            const int j = j0 + i * jstep;
            const float p = j < nb ? expf(sc[i] - mnew) : 0.0f;
            const float4 v4 = b0 + j == pos ? vn4 : vv[i];
            ps += d4 == 0 ? p : 0.0f;  // one copy per position
            cb.x = __builtin_fmaf(p, v4.x, cb.x);
            cb.y = __builtin_fmaf(p, v4.y, cb.y);
            cb.z = __builtin_fmaf(p, v4.z, cb.z);
            cb.w = __builtin_fmaf(p, v4.w, cb.w);
        }
        // block sum of the batch
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o);
        lds_barrier();  // every wave has read red[] (the max)
        if (lane == 0) red[wave] = ps;
        lds_barrier();
        ps = 0.0f;
        for (int w = 0; w < kAttnThreads / 64; ++w) ps += red[w];
        L = L * f + ps;
        M = mnew;
        C = float4{__builtin_fmaf(C.x, f, cb.x), __builtin_fmaf(C.y, f, cb.y),
                   __builtin_fmaf(C.z, f, cb.z), __builtin_fmaf(C.w, f, cb.w)};
        lds_barrier();  // red[] free for the next batch
    }
    // context: sum the partials of the threads that share a float4 column
    cs[tid] = C;
    lds_barrier();
    if (tid < H4) {
        float4 r = float4{0.f, 0.f, 0.f, 0.f};
        for (int k = 0; k < jstep; ++k) {
            const float4 c = cs[tid + k * H4];
            r.x += c.x;
            r.y += c.y;
            r.z += c.z;
            r.w += c.w;
        }
        const float inv = 1.0f / L;
        *(float4 *)&a.ctx[h * hd + 4 * tid] = float4{r.x * inv, r.y * inv, r.z * inv, r.w * inv};
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
    const size_t attn_lds = (size_t)attn_lds_floats(d->head_dim) * sizeof(float);
    hipError_t e = hipSuccess;
    for (int32_t l = 0; l < c.num_layers && e == hipSuccess; ++l) {
        const auto &L = d->layers[(size_t)l];
        const float *g_in = d->norms + (2 * (size_t)l) * H, *g_post = g_in + H;
        e = launch_gemv_fused(*L.qkv, FusedGemvArgs{d->h, nullptr, g_in, c.rms_eps, d->qkv, 1, 0}, s);
        if (e != hipSuccess) break;
        ap.kcache = d->kcache + (size_t)l * c.max_seq * d->kv_dim;
        ap.vcache = d->vcache + (size_t)l * c.max_seq * d->kv_dim;
        hipLaunchKernelGGL(attention_head, dim3((unsigned)c.num_heads), dim3(kAttnThreads), attn_lds, s, ap);
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

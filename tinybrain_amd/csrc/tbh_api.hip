// tbh_api.hip -- C ABI of libtinybrain_hip: devices, weight upload + repack,
// matmul dispatch.  Kernels live in tbh_gemv.hip and tbh_ref_kernels.hip.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <thread>
#include <vector>

#include "tbh_internal.h"

// Device memory of tbh_matmul_device_noalloc: its split-K partial sums live
// here instead of in a per-stream workspace, so the call never allocates.
// Each GPU the library runs on holds its own copy of the array (its own
// address, looked up once per device in tbh_device_open) until the process
// ends.  Host code only ever uses that looked-up address: the array's name
// in host code is a host-side stand-in, not device memory.
static constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace tbh {

namespace {
thread_local std::string g_last_error;

int host_threads() {
    unsigned n = std::thread::hardware_concurrency();
    return (int)std::max(1u, std::min(n, 16u));
}

// Runs fn(lo, hi) over [0, n) split into contiguous pieces on host threads.
template <class F>
void parallel_for(int64_t n, F fn) {
    int t = host_threads();
    if (n < 4096 || t == 1) {
        fn(int64_t(0), n);
        return;
    }
    std::vector<std::thread> pool;
    int64_t step = (n + t - 1) / t;
    for (int i = 0; i < t; ++i) {
        int64_t lo = i * step, hi = std::min(n, lo + step);
        if (lo >= hi) break;
        pool.emplace_back([=] { fn(lo, hi); });
    }
    for (auto &th : pool) th.join();
}

int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }
}  // namespace

tbh_status set_error(tbh_status st, const std::string &msg) {
    g_last_error = msg;
    return st;
}

tbh_status hip_error(hipError_t e, const char *what) {
    std::string m = std::string(what) + ": " + hipGetErrorString(e);
    return set_error(e == hipErrorOutOfMemory ? TBH_E_OOM : TBH_E_HIP, m);
}

}  // namespace tbh

using namespace tbh;

#define TBH_HIP(call, what)                          \
    do {                                             \
        hipError_t e_ = (call);                      \
        if (e_ != hipSuccess) return hip_error(e_, what); \
    } while (0)

// Makes the weight's device current on the calling thread.
tbh_status tbh::use_device(int32_t ordinal) {
    int cur = -1;
    TBH_HIP(hipGetDevice(&cur), "hipGetDevice");
    if (cur != ordinal) TBH_HIP(hipSetDevice(ordinal), "hipSetDevice");
    return TBH_OK;
}

extern "C" {

int32_t tbh_abi_version(void) { return TBH_ABI_VERSION; }

const char *tbh_last_error(void) { return g_last_error.c_str(); }

const char *tbh_status_string(tbh_status st) {
    switch (st) {
    case TBH_OK: return "TBH_OK";
    case TBH_E_INVALID: return "TBH_E_INVALID";
    case TBH_E_UNSUPPORTED: return "TBH_E_UNSUPPORTED";
    case TBH_E_NODEVICE: return "TBH_E_NODEVICE";
    case TBH_E_OOM: return "TBH_E_OOM";
    case TBH_E_HIP: return "TBH_E_HIP";
    default: return "TBH_E_UNKNOWN";
    }
}

// ---------------------------------------------------------------------------
// device
// ---------------------------------------------------------------------------
tbh_status tbh_device_open(int32_t ordinal, tbh_device **out) {
    if (!out) return set_error(TBH_E_INVALID, "tbh_device_open: out is NULL");
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
        return set_error(TBH_E_NODEVICE, "tbh_device_open: no HIP device");
    if (ordinal < 0 || ordinal >= count)
        return set_error(TBH_E_NODEVICE, "tbh_device_open: ordinal out of range");
    hipDeviceProp_t prop;
    TBH_HIP(hipGetDeviceProperties(&prop, ordinal), "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return set_error(TBH_E_NODEVICE, std::string("tbh_device_open: device is ") +
                                             prop.gcnArchName + ", this library is built for gfx950");
    TBH_HIP(hipSetDevice(ordinal), "hipSetDevice");
    auto dev = std::make_unique<tbh_device>();
    dev->ordinal = ordinal;
    // this device's copy of the no-allocation scratch array (device `ordinal`
    // is current here)
    TBH_HIP(hipGetSymbolAddress(&dev->noalloc_scratch, HIP_SYMBOL(scratch)),
            "tbh_device_open: scratch address");
    if (!dev->noalloc_scratch) return set_error(TBH_E_HIP, "tbh_device_open: scratch address is NULL");
    dev->cu_count = prop.multiProcessorCount;
    if (const char *v = std::getenv("TBH_SGEMV_MIN_ROWS"); v && *v) {   // read once, at open; 0: the rule
        const int r = std::atoi(v);
        dev->sgemv_min_rows.store(r == 0 ? 0 : std::min(9, std::max(2, r)), std::memory_order_relaxed);
    }
    if (const char *v = std::getenv("TBH_HOST_ENTRY"); v && *v) {   // initial TBH_OPT_HOST_ENTRY
        const int m = std::atoi(v);
        if (m >= 0 && m <= 2) dev->host_entry.store(m, std::memory_order_relaxed);
    }
    if (const char *v = std::getenv("TBH_HOST_WAIT"); v && *v) {    // initial TBH_OPT_HOST_WAIT
        const int m = std::atoi(v);
        if (m == 0 || m == 1) dev->host_wait.store(m, std::memory_order_relaxed);
    }
    TBH_HIP(hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking), "hipStreamCreate");
    *out = dev.release();
    return TBH_OK;
}

tbh_status tbh_device_close(tbh_device *dev) {
    if (!dev) return TBH_OK;
    // teardown: statuses are not actionable here, the handle goes away regardless
    (void)use_device(dev->ordinal);
    // One device-wide wait covers every stream that used a workspace; those
    // streams belong to the caller and may already be destroyed.
    (void)hipDeviceSynchronize();
    if (dev->stage) (void)hipFree(dev->stage);
    if (dev->pin) (void)hipHostFree(dev->pin);
    if (dev->done_flag) (void)hipHostFree(dev->done_flag);
    for (auto &ws : dev->workspaces) (void)hipFree(ws.ptr);
    for (void *p : dev->retired) (void)hipFree(p);
    if (dev->stream) (void)hipStreamDestroy(dev->stream);
    delete dev;
    return TBH_OK;
}

tbh_status tbh_device_set_option(tbh_device *dev, int32_t option, int64_t value) {
    if (!dev) return set_error(TBH_E_INVALID, "tbh_device_set_option: dev is NULL");
    switch (option) {
    case TBH_OPT_SGEMV_MIN_ROWS:
        if (value != 0 && (value < 2 || value > 9))
            return set_error(TBH_E_INVALID, "TBH_OPT_SGEMV_MIN_ROWS takes 0 (per-weight rule) or 2..9");
        dev->sgemv_min_rows.store((int)value, std::memory_order_relaxed);
        return TBH_OK;
    case TBH_OPT_HOST_ENTRY:
        if (value < 0 || value > 2)
            return set_error(TBH_E_INVALID, "TBH_OPT_HOST_ENTRY takes 0 (DMA copies), 1 (copy launch, y to host "
                                            "memory) or 2 (one row of x read in place)");
        dev->host_entry.store((int)value, std::memory_order_relaxed);
        return TBH_OK;
    case TBH_OPT_HOST_WAIT:
        if (value != 0 && value != 1)
            return set_error(TBH_E_INVALID, "TBH_OPT_HOST_WAIT takes 0 (stream synchronise) or 1 (polled word)");
        dev->host_wait.store((int)value, std::memory_order_relaxed);
        return TBH_OK;
    case TBH_OPT_MFMA_MIN_ROWS:
        if (value < 0 || value > INT32_MAX)
            return set_error(TBH_E_INVALID, "TBH_OPT_MFMA_MIN_ROWS takes 0 (per-weight rule) or a row count");
        dev->mfma_min_rows.store((int)value, std::memory_order_relaxed);
        return TBH_OK;
    case TBH_OPT_NOALLOC_SCRATCH_BYTES:
        if (value < 0 || value > (int64_t)kNoAllocScratchBytes)
            return set_error(TBH_E_INVALID, "TBH_OPT_NOALLOC_SCRATCH_BYTES takes 0 (all of it) or 1 .. " +
                                                std::to_string(kNoAllocScratchBytes));
        dev->noalloc_limit.store(value, std::memory_order_relaxed);
        return TBH_OK;
    default: return set_error(TBH_E_INVALID, "tbh_device_set_option: unknown option");
    }
}

tbh_status tbh_device_get_info(const tbh_device *dev, int32_t *ordinal, int32_t *cu_count) {
    if (!dev) return set_error(TBH_E_INVALID, "tbh_device_get_info: dev is NULL");
    if (ordinal) *ordinal = dev->ordinal;
    if (cu_count) *cu_count = dev->cu_count;
    return TBH_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// descriptor validation: QuantizedTensor.init preconditions
// (QuantizedTensor.swift:124-155) plus the combinations this backend takes
// ---------------------------------------------------------------------------
static tbh_status validate_desc(const tbh_qtensor_desc *d) {
    if (!d) return set_error(TBH_E_INVALID, "descriptor is NULL");
    if (d->K <= 0 || d->N <= 0)
        return set_error(TBH_E_INVALID, "weight shape must be [K>0, N>0]");
    if (d->layout != TBH_LAYOUT_KN_FLAT && d->layout != TBH_LAYOUT_NK_FLAT)
        return set_error(TBH_E_INVALID, "unknown layout");
    if (d->group_size < 0) return set_error(TBH_E_INVALID, "group_size < 0");
    if (d->K > kMaxDim || d->N > kMaxDim)
        return set_error(TBH_E_UNSUPPORTED, "K and N must each be at most 2^30 (the kernels index rows and "
                                            "columns of a weight with 32-bit integers)");
    const int64_t count = d->K * d->N;
    if (d->precision == TBH_PREC_INT8) {
        if (d->data_bytes != count)
            return set_error(TBH_E_INVALID, "INT8: data count must match shape");
    } else if (d->precision == TBH_PREC_INT4) {
        if (d->data_bytes != (count + 1) / 2)
            return set_error(TBH_E_INVALID, "INT4: data count should be ceil(shape.count / 2)");
    } else {
        return set_error(TBH_E_INVALID, "unknown precision");
    }
    int64_t want_scales = 0;
    switch (d->mode) {
    case TBH_MODE_PER_CHANNEL:
    case TBH_MODE_INT4_PER_CHANNEL: want_scales = d->N; break;
    case TBH_MODE_SYMMETRIC:
    case TBH_MODE_ASYMMETRIC: want_scales = 1; break;
    case TBH_MODE_INT4:
        want_scales = d->group_size > 0 ? (count + d->group_size - 1) / d->group_size : 1;
        break;
    default: return set_error(TBH_E_INVALID, "unknown mode");
    }
    if (d->n_scales != want_scales)
        return set_error(TBH_E_INVALID, "scale count does not match mode/shape (need " +
                                            std::to_string(want_scales) + ", got " +
                                            std::to_string(d->n_scales) + ")");
    if (!d->data || !d->scales) return set_error(TBH_E_INVALID, "data or scales is NULL");
    if (d->zero_points && d->n_zero_points != d->n_scales)
        return set_error(TBH_E_INVALID, "Zero points must match scales");
    if (d->precision == TBH_PREC_INT8 &&
        !(d->mode == TBH_MODE_SYMMETRIC || d->mode == TBH_MODE_ASYMMETRIC ||
          d->mode == TBH_MODE_PER_CHANNEL))
        return set_error(TBH_E_UNSUPPORTED, "INT8 precision with an INT4 mode");
    if (d->precision == TBH_PREC_INT4 && d->mode == TBH_MODE_INT4_PER_CHANNEL)
        return set_error(TBH_E_UNSUPPORTED,
                         "int4PerChannel: the reference's dequantize() and quantizer disagree "
                         "on the channel axis; use the caller's CPU fallback");
    if (d->precision == TBH_PREC_INT4 && d->mode != TBH_MODE_INT4)
        return set_error(TBH_E_UNSUPPORTED, "INT4 precision with an INT8 mode");
    return TBH_OK;
}

// ---------------------------------------------------------------------------
// host repack
// ---------------------------------------------------------------------------
namespace {

// q-matrix [N][K] (int8 values, K contiguous) from the flat reference array.
std::vector<int8_t> expand_nk(const tbh_qtensor_desc &d) {
    const int64_t K = d.K, N = d.N;
    std::vector<int8_t> q((size_t)(K * N));
    const uint8_t *src = reinterpret_cast<const uint8_t *>(d.data);
    const bool int4 = d.precision == TBH_PREC_INT4;
    auto at = [&](int64_t i) -> int8_t {
        if (!int4) return (int8_t)src[i];
        unsigned b = src[i >> 1];
        unsigned raw = (i & 1) == 0 ? (b >> 4) & 0xFu : b & 0xFu;
        return (int8_t)(raw > 7 ? (int)raw - 16 : (int)raw);
    };
    if (d.layout == TBH_LAYOUT_NK_FLAT) {
        parallel_for(N, [&](int64_t lo, int64_t hi) {
            for (int64_t n = lo; n < hi; ++n)
                for (int64_t k = 0; k < K; ++k) q[n * K + k] = at(n * K + k);
        });
    } else {
        // transpose in 64 x 64 tiles
        const int64_t T = 64;
        int64_t tiles_n = (N + T - 1) / T;
        parallel_for(tiles_n, [&](int64_t lo, int64_t hi) {
            for (int64_t tn = lo; tn < hi; ++tn) {
                int64_t n0 = tn * T, n1 = std::min(N, n0 + T);
                for (int64_t k0 = 0; k0 < K; k0 += T) {
                    int64_t k1 = std::min(K, k0 + T);
                    for (int64_t k = k0; k < k1; ++k)
                        for (int64_t n = n0; n < n1; ++n) q[n * K + k] = at(k * N + n);
                }
            }
        });
    }
    return q;
}

// INT8 row [Kp] bytes: within each 4-byte word, elements k..k+3 sit at byte
// positions {0, 2, 1, 3} so that (w & 0x00FF00FF) and ((w >> 8) & 0x00FF00FF)
// hold the pairs (k, k+1) and (k+2, k+3).  Values are offset binary (q+128).
void pack_int8_rows(const std::vector<int8_t> &q, int64_t K, int64_t N, int64_t Kp, int64_t Np,
                    std::vector<uint8_t> &out) {
    static const int bp[4] = {0, 2, 1, 3};
    out.assign((size_t)(Np * Kp), 0x80);
    parallel_for(N, [&](int64_t lo, int64_t hi) {
        for (int64_t n = lo; n < hi; ++n) {
            uint8_t *row = out.data() + n * Kp;
            const int8_t *qr = q.data() + n * K;
            for (int64_t k = 0; k < K; ++k)
                row[(k & ~int64_t(3)) + bp[k & 3]] = (uint8_t)((int)qr[k] + 128);
        }
    });
}

// INT4 row [Kp/2] bytes: each 32-bit word holds 8 consecutive elements
// k..k+7 as offset-binary nibbles (q+8) at bit offsets
// {0, 16, 4, 20, 8, 24, 12, 28}, which the kernel turns into f16 pairs with
// two AND-ORs per shift.
void pack_int4_rows(const std::vector<int8_t> &q, int64_t K, int64_t N, int64_t Kp, int64_t Np,
                    std::vector<uint8_t> &out) {
    static const int nb[8] = {0, 16, 4, 20, 8, 24, 12, 28};
    const int64_t row_words = Kp / 8;
    out.assign((size_t)(Np * Kp / 2), 0x88);
    parallel_for(N, [&](int64_t lo, int64_t hi) {
        for (int64_t n = lo; n < hi; ++n) {
            uint32_t *row = reinterpret_cast<uint32_t *>(out.data() + n * (Kp / 2));
            const int8_t *qr = q.data() + n * K;
            for (int64_t wi = 0; wi < row_words; ++wi) {
                uint32_t word = 0;
                for (int j = 0; j < 8; ++j) {
                    int64_t k = wi * 8 + j;
                    int v = k < K ? qr[k] : 0;
                    word |= (uint32_t)((v + 8) & 0xF) << nb[j];
                }
                row[wi] = word;
            }
        }
    });
}

// MFMA tiles (INT8): 1 KiB per (16-row tile rt, 64-element K tile sc).  Lane
// l's 16 bytes are 4 words; words 2j and 2j+1 hold the 8 elements
// k = 64 sc + 32 j + 8 (l / 16) + e of row 16 rt + l % 16, 4 per word at byte
// positions {0, 2, 1, 3}, value q + 128.
void pack_int8_tiles(const std::vector<int8_t> &q, int64_t K, int64_t N, int64_t Kp, int64_t Np,
                     std::vector<uint8_t> &out) {
    static const int bp[4] = {0, 2, 1, 3};
    const int64_t SC = Kp / kMfmaInt8TileK, ntiles = Np / 16;
    out.assign((size_t)(ntiles * SC * 1024), 0x80);
    parallel_for(ntiles, [&](int64_t lo, int64_t hi) {
        for (int64_t rt = lo; rt < hi; ++rt)
            for (int64_t sc = 0; sc < SC; ++sc) {
                uint8_t *tile = out.data() + (rt * SC + sc) * 1024;
                for (int l = 0; l < 64; ++l) {
                    const int64_t n = rt * 16 + (l & 15);
                    if (n >= N) continue;
                    const int8_t *qr = q.data() + n * K;
                    for (int d = 0; d < 4; ++d)
                        for (int e4 = 0; e4 < 4; ++e4) {
                            const int64_t k = sc * 64 + 32 * (d >> 1) + 8 * (l >> 4) + 4 * (d & 1) + e4;
                            if (k < K) tile[16 * l + 4 * d + bp[e4]] = (uint8_t)((int)qr[k] + 128);
                        }
                }
            }
    });
}

// MFMA tiles (INT4): 1 KiB per (16-row tile rt, 128-element K tile sc).  Lane
// l's word j holds the 8 elements k = 128 sc + 32 j + 8 (l / 16) + e of row
// 16 rt + l % 16 as nibbles q + 8 at bit offsets {0, 16, 4, 20, 8, 24, 12, 28}.
void pack_int4_tiles(const std::vector<int8_t> &q, int64_t K, int64_t N, int64_t Kp, int64_t Np,
                     std::vector<uint8_t> &out) {
    static const int nb[8] = {0, 16, 4, 20, 8, 24, 12, 28};
    const int64_t SC = Kp / kMfmaInt4TileK, ntiles = Np / 16;
    out.assign((size_t)(ntiles * SC * 1024), 0x88);
    parallel_for(ntiles, [&](int64_t lo, int64_t hi) {
        for (int64_t rt = lo; rt < hi; ++rt)
            for (int64_t sc = 0; sc < SC; ++sc) {
                uint32_t *tile = reinterpret_cast<uint32_t *>(out.data() + (rt * SC + sc) * 1024);
                for (int l = 0; l < 64; ++l) {
                    const int64_t n = rt * 16 + (l & 15);
                    if (n >= N) continue;
                    const int8_t *qr = q.data() + n * K;
                    for (int j = 0; j < 4; ++j) {
                        uint32_t word = 0;
                        for (int e = 0; e < 8; ++e) {
                            const int64_t k = sc * 128 + 32 * j + 8 * (l >> 4) + e;
                            const int v = k < K ? qr[k] : 0;
                            word |= (uint32_t)((v + 8) & 0xF) << nb[e];
                        }
                        tile[4 * l + j] = word;
                    }
                }
            }
    });
}

// HBM layout of new weights: K-contiguous rows for the VALU GEMV (default,
// fastest measured for decode, M = 1) or, with TBH_LAYOUT=tiles, 1 KiB MFMA
// tiles for the MFMA GEMV.
bool use_row_layout() {
    const char *v = std::getenv("TBH_LAYOUT");
    return !(v && std::strcmp(v, "tiles") == 0);
}

bool any_nonzero(const int8_t *p, int64_t n) {
    if (!p) return false;
    for (int64_t i = 0; i < n; ++i)
        if (p[i] != 0) return true;
    return false;
}

template <class T>
hipError_t upload(T **dst, const T *src, size_t count, int64_t &bytes, int64_t &n_out) {
    size_t nbytes = std::max<size_t>(count * sizeof(T), 1);
    hipError_t e = hipMalloc((void **)dst, nbytes);
    if (e != hipSuccess) return e;
    bytes += (int64_t)(count * sizeof(T));
    n_out = (int64_t)count;
    return hipMemcpy(*dst, src, count * sizeof(T), hipMemcpyHostToDevice);
}

// Statuses of the frees are not actionable: the weight goes away regardless.
void free_weight(tbh_weight *w) {
    if (!w) return;
    for (void *p : {(void *)w->data, (void *)w->scales, (void *)w->zp, (void *)w->raw, (void *)w->raw_scales,
                    (void *)w->raw_zp, (void *)w->ng_sexp})
        (void)hipFree(p);
    delete w;
}

}  // namespace

extern "C" {

tbh_status tbh_weight_create(tbh_device *dev, const tbh_qtensor_desc *desc, tbh_weight **out) {
    if (!out) return set_error(TBH_E_INVALID, "tbh_weight_create: out is NULL");
    *out = nullptr;
    if (!dev) return set_error(TBH_E_INVALID, "tbh_weight_create: dev is NULL");
    tbh_status st = validate_desc(desc);
    if (st != TBH_OK) return st;
    st = use_device(dev->ordinal);
    if (st != TBH_OK) return st;

    const tbh_qtensor_desc &d = *desc;
    std::unique_ptr<tbh_weight, void (*)(tbh_weight *)> w(new tbh_weight, free_weight);
    w->dev = dev;
    w->K = d.K;
    w->N = d.N;
    w->precision = d.precision;
    w->mode = d.mode;
    w->layout = d.layout;
    w->group_size = d.group_size;
    const int64_t K = d.K, N = d.N, count = K * N;
    const bool has_zp = any_nonzero(d.zero_points, d.n_zero_points);
    hipError_t e = hipSuccess;

    if (d.precision == TBH_PREC_INT8) {
        w->path = Path::Int8Row;
        w->mfma_tiles = !use_row_layout();
        std::vector<int8_t> q = expand_nk(d);
        std::vector<uint8_t> packed;
        if (w->mfma_tiles) {
            w->Kp = round_up(K, kMfmaInt8TileK);
            w->Np = round_up(N, 16);
            pack_int8_tiles(q, K, N, w->Kp, w->Np, packed);
        } else {
            w->Kp = round_up(K, kInt8ChunkElems);
            w->Np = round_up(N, 8);
            w->row_bytes = w->Kp;
            pack_int8_rows(q, K, N, w->Kp, w->Np, packed);
        }
        std::vector<float> s((size_t)w->Np, 0.0f);
        std::vector<int8_t> z((size_t)w->Np, 0);
        const bool per_ch = d.mode == TBH_MODE_PER_CHANNEL;
        for (int64_t n = 0; n < N; ++n) {
            s[n] = d.scales[per_ch ? n : 0];
            if (d.zero_points) z[n] = d.zero_points[per_ch ? n : 0];
        }
        e = upload(&w->data, packed.data(), packed.size(), w->device_bytes, w->n_data);
        if (e == hipSuccess) e = upload(&w->scales, s.data(), s.size(), w->device_bytes, w->n_scales_dev);
        if (e == hipSuccess && has_zp) e = upload(&w->zp, z.data(), z.size(), w->device_bytes, w->n_zp_dev);
        w->stream_bytes = K * N + 4 * N + (has_zp ? N : 0);
    } else {
        const int64_t gs = d.group_size > 0 ? d.group_size : count;
        auto group_of = [&](int64_t k, int64_t n) -> int64_t {
            int64_t i = d.layout == TBH_LAYOUT_KN_FLAT ? k * N + n : n * K + k;
            return i / gs;
        };
        // Which tables describe the grouping exactly?
        bool kgroup = false, ngroup = false;
        int64_t seg = 0;       // Int4KGroup: K-segment length sharing one scale (0 = whole row)
        int64_t rpn = 0;       // Int4NGroup: rows sharing one per-k scale column
        if (gs >= count) {
            kgroup = true;
            seg = 0;
        } else if (d.layout == TBH_LAYOUT_NK_FLAT) {
            if (K % gs == 0 && gs % kInt4ChunkElems == 0) { kgroup = true; seg = gs; }
            else if (gs % K == 0) { kgroup = true; seg = 0; }
        } else {
            // The N-group kernels stage a row of x in LDS; with a longer K
            // the weight keeps the reference's flat array (generic kernel).
            const int64_t x_lds = round_up(K, kInt4ChunkElems) / kInt4ChunkElems * (kInt4ChunkElems + 4) * 4;
            if (!has_zp && x_lds <= kMaxLdsBytes) {
                if (N % gs == 0) { ngroup = true; rpn = gs; }
                else if (gs % N == 0) { ngroup = true; rpn = 0; }
            }
        }
        if (kgroup && !use_row_layout()) {
            // MFMA tiles; per-row scale when one group spans the row, else one
            // scale (and zero point) per (row, 32-element chunk) in tile order
            w->path = Path::Int4KGroup;
            w->mfma_tiles = true;
            w->Kp = round_up(K, kMfmaInt4TileK);
            w->Np = round_up(N, 16);
            const int64_t G = seg ? K / seg : 1;
            w->groups_per_row = G;
            w->chunks_per_group = (int32_t)(seg ? seg / kInt4ChunkElems : w->Kp / kInt4ChunkElems);
            std::vector<int8_t> q = expand_nk(d);
            std::vector<uint8_t> packed;
            pack_int4_tiles(q, K, N, w->Kp, w->Np, packed);
            e = upload(&w->data, packed.data(), packed.size(), w->device_bytes, w->n_data);
            std::vector<float> s;
            std::vector<int8_t> z;
            if (G == 1) {
                s.assign((size_t)w->Np, 0.0f);
                z.assign((size_t)w->Np, 0);
                for (int64_t n = 0; n < N; ++n) {
                    const int64_t gi = group_of(0, n);
                    s[n] = d.scales[gi];
                    if (d.zero_points) z[n] = d.zero_points[gi];
                }
            } else {
                const int64_t SC = w->Kp / kMfmaInt4TileK, ntiles = w->Np / 16;
                s.assign((size_t)(ntiles * SC * 64), 0.0f);
                z.assign((size_t)(ntiles * SC * 64), 0);
                for (int64_t n = 0; n < N; ++n)
                    for (int64_t c = 0; c < K / kInt4ChunkElems; ++c) {
                        const int64_t gi = group_of(c * kInt4ChunkElems, n);
                        const int64_t at = (((n / 16) * SC + c / 4) * 16 + n % 16) * 4 + c % 4;
                        s[at] = d.scales[gi];
                        if (d.zero_points) z[at] = d.zero_points[gi];
                    }
            }
            if (e == hipSuccess) e = upload(&w->scales, s.data(), s.size(), w->device_bytes, w->n_scales_dev);
            if (e == hipSuccess && has_zp) e = upload(&w->zp, z.data(), z.size(), w->device_bytes, w->n_zp_dev);
            w->stream_bytes = (count + 1) / 2 + 4 * N * G + (has_zp ? N * G : 0);
        } else if (kgroup || ngroup) {
            w->Kp = round_up(K, kInt4ChunkElems);
            w->Np = round_up(N, 8);
            w->row_bytes = w->Kp / 2;
            std::vector<int8_t> q = expand_nk(d);
            std::vector<uint8_t> packed;
            pack_int4_rows(q, K, N, w->Kp, w->Np, packed);
            e = upload(&w->data, packed.data(), packed.size(), w->device_bytes, w->n_data);
            if (kgroup) {
                w->path = Path::Int4KGroup;
                const int64_t G = seg ? K / seg : 1;
                w->groups_per_row = G;
                w->chunks_per_group = (int32_t)(seg ? seg / kInt4ChunkElems : w->Kp / kInt4ChunkElems);
                std::vector<float> s((size_t)(w->Np * G), 0.0f);
                std::vector<int8_t> z((size_t)(w->Np * G), 0);
                for (int64_t n = 0; n < N; ++n)
                    for (int64_t g = 0; g < G; ++g) {
                        const int64_t gi = group_of(seg ? g * seg : 0, n);
                        s[kgroup_index(n, g, G)] = d.scales[gi];
                        if (d.zero_points) z[kgroup_index(n, g, G)] = d.zero_points[gi];
                    }
                if (e == hipSuccess) e = upload(&w->scales, s.data(), s.size(), w->device_bytes, w->n_scales_dev);
                if (e == hipSuccess && has_zp) e = upload(&w->zp, z.data(), z.size(), w->device_bytes, w->n_zp_dev);
                w->stream_bytes = (count + 1) / 2 + 4 * N * G + (has_zp ? N * G : 0);
            } else {
                w->path = Path::Int4NGroup;
                w->rows_per_nblock = (int32_t)(rpn ? rpn : w->Np);
                const int64_t NB = (w->Np + w->rows_per_nblock - 1) / w->rows_per_nblock;
                std::vector<float> t((size_t)(NB * w->Kp), 0.0f);
                for (int64_t nb = 0; nb < NB; ++nb) {
                    int64_t n = std::min(N - 1, nb * w->rows_per_nblock);
                    if (nb * w->rows_per_nblock >= N) continue;
                    for (int64_t k = 0; k < K; ++k) t[nb * w->Kp + k] = d.scales[group_of(k, n)];
                }
                if (e == hipSuccess) e = upload(&w->scales, t.data(), t.size(), w->device_bytes, w->n_scales_dev);
                // per N-block e with |s| < 2^e for its finite scales, for the
                // prefill GEMM's f16 scaling of x * s
                std::vector<int32_t> ex((size_t)NB, 0);
                for (int64_t nb = 0; nb < NB; ++nb) {
                    float mx = 0.0f;
                    for (int64_t k = 0; k < K; ++k) {
                        const float a = std::fabs(t[nb * w->Kp + k]);
                        if (std::isfinite(a)) mx = std::max(mx, a);
                    }
                    int e2 = 0;
                    if (mx > 0.0f) (void)std::frexp(mx, &e2);
                    ex[(size_t)nb] = e2;
                    const float lo_ok = std::ldexp(1.0f, e2 - 36);
                    for (int64_t k = 0; k < K && !w->ng_wide; ++k) {
                        const float a = std::fabs(t[nb * w->Kp + k]);
                        w->ng_wide = a > 0.0f && a < lo_ok;
                    }
                }
                if (e == hipSuccess) e = upload(&w->ng_sexp, ex.data(), ex.size(), w->device_bytes, w->n_ng_sexp);
                w->stream_bytes = (count + 1) / 2 + 4 * d.n_scales;
            }
        } else {
            w->path = Path::Generic;
            w->raw_bytes = d.data_bytes;
            w->n_scales = d.n_scales;
            e = upload(&w->raw, d.data, (size_t)d.data_bytes, w->device_bytes, w->n_raw);
            if (e == hipSuccess) e = upload(&w->raw_scales, d.scales, (size_t)d.n_scales, w->device_bytes, w->n_raw_scales);
            if (e == hipSuccess && has_zp)
                e = upload(&w->raw_zp, d.zero_points, (size_t)d.n_scales, w->device_bytes, w->n_raw_zp);
            w->stream_bytes = d.data_bytes + 4 * d.n_scales + (has_zp ? d.n_scales : 0);
        }
    }
    if (e != hipSuccess) return hip_error(e, "tbh_weight_create: upload");
    if (!weight_arrays_ok(*w))
        return set_error(TBH_E_INVALID, "tbh_weight_create: internal layout inconsistency");
    *out = w.release();
    return TBH_OK;
}

}  // extern "C"

// Two INT4 runtime-layout weights (groups along N) of one shape as one weight
// whose row 2j is a's output j and row 2j + 1 is b's: the decoder's gate|up
// projection, whose GEMV epilogue pairs the two rows.  Scales: a's per-k
// table then b's, nb_half N-blocks each.
tbh_status tbh::create_ngroup_pair(tbh_device *dev, const tbh_qtensor_desc *a, const tbh_qtensor_desc *b,
                                   tbh_weight **out) {
    *out = nullptr;
    for (const tbh_qtensor_desc *d : {a, b}) {
        tbh_status st = validate_desc(d);
        if (st != TBH_OK) return st;
        if (d->precision != TBH_PREC_INT4 || d->layout != TBH_LAYOUT_KN_FLAT || d->group_size <= 0 ||
            any_nonzero(d->zero_points, d->n_zero_points))
            return set_error(TBH_E_UNSUPPORTED, "pair weight: needs INT4 runtime-layout weights without zero points");
    }
    if (a->K != b->K || a->N != b->N || a->group_size != b->group_size)
        return set_error(TBH_E_INVALID, "pair weight: the two weights differ in shape or group size");
    const int64_t K = a->K, Nh = a->N, gs = a->group_size;
    int64_t rpn;
    if (Nh % gs == 0) rpn = gs;            // groups of gs outputs share a scale per k
    else if (gs % Nh == 0) rpn = 0;        // every output of a k-block shares one scale
    else return set_error(TBH_E_UNSUPPORTED, "pair weight: groups must tile N");
    tbh_status st = use_device(dev->ordinal);
    if (st != TBH_OK) return st;
    std::unique_ptr<tbh_weight, void (*)(tbh_weight *)> w(new tbh_weight, free_weight);
    w->dev = dev;
    w->K = K;
    w->N = 2 * Nh;
    w->precision = TBH_PREC_INT4;
    w->mode = TBH_MODE_INT4;
    w->layout = TBH_LAYOUT_KN_FLAT;
    w->group_size = (int32_t)gs;
    w->path = Path::Int4NGroup;
    w->ng_pairs = true;
    w->Kp = round_up(K, kInt4ChunkElems);
    w->Np = round_up(2 * Nh, 8);
    w->row_bytes = w->Kp / 2;
    w->rows_per_nblock = (int32_t)(rpn ? rpn : w->Np);
    const int64_t NBh = rpn ? (Nh + rpn - 1) / rpn : 1;
    w->nb_half = (int32_t)NBh;
    const std::vector<int8_t> qa = expand_nk(*a), qb = expand_nk(*b);
    std::vector<int8_t> q((size_t)(2 * Nh * K));
    for (int64_t j = 0; j < Nh; ++j) {
        std::memcpy(&q[(size_t)(2 * j * K)], &qa[(size_t)(j * K)], (size_t)K);
        std::memcpy(&q[(size_t)((2 * j + 1) * K)], &qb[(size_t)(j * K)], (size_t)K);
    }
    std::vector<uint8_t> packed;
    pack_int4_rows(q, K, 2 * Nh, w->Kp, w->Np, packed);
    std::vector<float> t((size_t)(2 * NBh * w->Kp), 0.0f);
    for (int c = 0; c < 2; ++c) {
        const tbh_qtensor_desc &d = c == 0 ? *a : *b;
        for (int64_t nb = 0; nb < NBh; ++nb) {
            const int64_t n = rpn ? nb * rpn : 0;
            for (int64_t k = 0; k < K; ++k) t[(size_t)((c * NBh + nb) * w->Kp + k)] = d.scales[(k * Nh + n) / gs];
        }
    }
    hipError_t e = upload(&w->data, packed.data(), packed.size(), w->device_bytes, w->n_data);
    if (e == hipSuccess) e = upload(&w->scales, t.data(), t.size(), w->device_bytes, w->n_scales_dev);
    if (e != hipSuccess) return hip_error(e, "pair weight: upload");
    w->stream_bytes = 2 * ((K * Nh + 1) / 2 + 4 * a->n_scales);
    if (!weight_arrays_ok(*w)) return set_error(TBH_E_INVALID, "pair weight: internal layout inconsistency");
    *out = w.release();
    return TBH_OK;
}

extern "C" {

tbh_status tbh_weight_destroy(tbh_weight *w) {
    if (!w) return TBH_OK;
    use_device(w->dev->ordinal);
    free_weight(w);
    return TBH_OK;
}

tbh_status tbh_weight_get_info(const tbh_weight *w, tbh_weight_info *info) {
    if (!w || !info) return set_error(TBH_E_INVALID, "tbh_weight_get_info: NULL argument");
    info->K = w->K;
    info->N = w->N;
    info->precision = w->precision;
    info->mode = w->mode;
    info->layout = w->layout;
    info->group_size = w->group_size;
    info->path = (int32_t)w->path;
    info->has_zero_points = (w->zp || w->raw_zp) ? 1 : 0;
    info->device_bytes = w->device_bytes;
    info->stream_bytes = w->stream_bytes;
    return TBH_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// device-array consistency (checked before every launch)
// ---------------------------------------------------------------------------
namespace tbh {
bool weight_arrays_ok(const tbh_weight &w) {
    if (w.K <= 0 || w.N <= 0) return false;
    const bool int4 = w.precision == TBH_PREC_INT4;
    auto zp_ok = [&](int64_t want) { return w.zp == nullptr ? w.n_zp_dev == 0 : w.n_zp_dev == want; };
    if (w.path == Path::Generic) {
        const int64_t cnt = w.K * w.N;
        const int64_t gs = w.group_size > 0 ? w.group_size : cnt;
        const int64_t groups = (cnt + gs - 1) / gs;
        return int4 && w.raw && w.raw_scales && w.n_raw == (cnt + 1) / 2 && w.n_raw_scales == groups &&
               (w.raw_zp == nullptr || w.n_raw_zp == groups);
    }
    if (!w.data || !w.scales || w.Kp < w.K || w.Np < w.N) return false;
    if (w.mfma_tiles) {
        const int64_t tk = int4 ? kMfmaInt4TileK : kMfmaInt8TileK;
        if (w.Kp % tk || w.Np % 16) return false;
        const int64_t tiles = (w.Np / 16) * (w.Kp / tk);
        if (w.n_data != tiles * 1024) return false;
        const int64_t ns = (int4 && w.groups_per_row > 1) ? tiles * 64 : w.Np;
        if (int4 && w.groups_per_row > 1 && w.Kp / kInt4ChunkElems < w.groups_per_row) return false;
        return w.n_scales_dev == ns && zp_ok(ns);
    }
    if (!int4) return w.n_data == w.Np * w.Kp && w.row_bytes == w.Kp && w.n_scales_dev == w.Np && zp_ok(w.Np);
    if (w.n_data != w.Np * w.Kp / 2 || w.row_bytes != w.Kp / 2 || w.Kp % kInt4ChunkElems) return false;
    if (w.path == Path::Int4KGroup) {
        const int64_t chunks = w.Kp / kInt4ChunkElems;
        return w.groups_per_row >= 1 && (int64_t)w.chunks_per_group * w.groups_per_row == chunks &&
               w.n_scales_dev == w.Np * w.groups_per_row && zp_ok(w.Np * w.groups_per_row);
    }
    if (w.path == Path::Int4NGroup) {
        if (w.rows_per_nblock <= 0 || w.zp) return false;
        if (w.ng_pairs) return w.nb_half > 0 && w.n_scales_dev == 2 * (int64_t)w.nb_half * w.Kp;
        const int64_t nb = (w.Np + w.rows_per_nblock - 1) / w.rows_per_nblock;
        return w.n_scales_dev == nb * w.Kp && w.ng_sexp && w.n_ng_sexp == nb;
    }
    return false;
}

void *stream_workspace(tbh_device *dev, hipStream_t s, size_t bytes) {
    std::lock_guard<std::mutex> lock(dev->ws_mu);
    tbh_device::Workspace *ws = nullptr;
    for (auto &e : dev->workspaces)
        if (e.stream == s) ws = &e;
    if (ws && ws->bytes >= bytes) return ws->ptr;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return nullptr;
    // Grow by replacement: work queued on this stream, and any graph captured
    // on it, may still use the old buffer, so it stays allocated (retired)
    // until tbh_device_close.  Growth doubles, so the retired bytes stay below
    // the live buffer's.
    const size_t mib = size_t(1) << 20;
    size_t grown = (bytes + mib - 1) & ~(mib - 1);
    if (ws) grown = std::max(grown, 2 * ws->bytes);
    void *p = nullptr;
    if (hipMalloc(&p, grown) != hipSuccess) return nullptr;
    if (!ws) {
        dev->workspaces.push_back({s, nullptr, 0});
        ws = &dev->workspaces.back();
    }
    if (ws->ptr) dev->retired.push_back(ws->ptr);
    ws->ptr = p;
    ws->bytes = grown;
    return ws->ptr;
}
}  // namespace tbh

extern "C" {

// ---------------------------------------------------------------------------
// matmul
// ---------------------------------------------------------------------------

// Fewest rows of x sent to the matrix-core GEMV (9: never).  The VALU
// kernels' time grows with M * N * K (their multiply-adds are the bound from
// 4 rows on), the matrix-core kernel's hardly with M, so the crossover falls
// with the weight's size and K.  Measured crossovers (INT4 g32, us per launch
// VALU / matrix cores): 4096 x 11008 at M = 2 16.5 / 12.4; 11008 x 4096 at
// M = 3 12.2 / 11.5; 32000 x 4096 at M = 3 28.7 / 22.1; 4096 x 4096 at M = 4
// 10.7 / 7.8 (M = 3: 7.2 / 7.8); 2048 x 5632 at M = 4 9.3 / 8.0; 5632 x 2048
// at M = 5 9.9 / 8.0 (M = 4: 6.5 / 7.6); 2048 x 2048 never (M = 8: 7.5 / 8.5,
// the matrix-core launch needs a K split and its split sum).
static int64_t sgemv_min_rows(const tbh_weight &w) {
    const int64_t nk = w.N * w.K;
    if (w.K >= 8192) return 2;
    if (nk >= (int64_t)40 << 20) return 3;
    if (w.K >= 4096) return 4;
    if (nk >= (int64_t)8 << 20) return 5;
    return 9;
}

// Fewest rows of fp32 x that go to the MFMA GEMM (each row split exactly into
// three bf16 pieces; launch_prefill_f32) instead of the GEMV kernels, which
// stream the whole weight once per 2..8 rows.  Measured crossovers, us per
// call GEMV / GEMM: INT8 5632x2048 M = 8 13.5 / 10.9; INT8 2048x2048 M = 8
// 7.5 / 7.9, M = 12 10.7 / 8.0; INT4 2048x2048 M = 12 11.4 / 10.1 (M = 8
// 7.8 / 9.7); INT4 4096x11008 M = 32 61.0 / 44.6; INT4 11008x4096 M = 32
// 56.5 / 49.9 (M = 24 42.2 / 49.1); INT4 32000x2048 M = 64 101.7 / 67.5
// (M = 48 76.5 / 78.4).
// Runtime-layout INT4 has no matrix-core GEMV, so its GEMV route is the VALU
// kernel four rows per launch: GEMM from 8 rows (2048x5632 M = 8 21.9 /
// 13.8, 11008x4096 42.4 / 38.5) or 12 on weights under 8 Mi elements and on
// N >= 16384 (2048x2048 M = 8 8.5 / 9.3, M = 12 12.5 / 9.4; 32000x2048 M = 8
// 35.0 / 40.0, M = 12 49.6 / 39.2).
//
// burst8: the weight takes eight rows of this x in one burst GEMV launch
// (gemv8_supported).  Below 16384 outputs that launch beats the GEMM at
// exactly 8 rows (us per call, GEMM / one 8-row launch: INT8 5632x2048 11.2
// / 9.2, 11264x2048 15.4 / 15.7; runtime-layout INT4 5632x2048 13.1 / 9.9;
// INT8 32000x2048 27.4 / 32.4), so those weights start the GEMM at 9.
static int64_t mfma_min_rows(const tbh_weight &w, bool burst8) {
    const int64_t nk = w.N * w.K;
    const bool big = nk >= ((int64_t)8 << 20);
    if (w.path == Path::Int4NGroup) return big && w.N < 16384 ? (burst8 ? 9 : 8) : 12;
    if (w.precision == TBH_PREC_INT8) return big ? (burst8 && w.N < 16384 ? 9 : 8) : 12;
    if (nk <= ((int64_t)24 << 20)) return 12;
    return w.N >= 16384 ? 64 : 32;
}

static tbh_status matmul_enqueue(const tbh_weight *w, const float *x, int64_t M, float *y,
                                 hipStream_t s, const Scratch &scr) {
    if (!weight_arrays_ok(*w))
        return set_error(TBH_E_INVALID, "weight device arrays are inconsistent with its layout");
    const int mfma_forced = w->dev->mfma_min_rows.load(std::memory_order_relaxed);
    const bool burst8 = !w->mfma_tiles && gemv8_supported(*w, x, w->K);
    const int64_t mfma_min = mfma_forced > 0 ? mfma_forced : mfma_min_rows(*w, burst8);
    // The GEMV kernels stage a whole row of x in LDS; past about 13 K (INT8)
    // or 14.5 K (INT4) elements it does not fit, and every row count goes to
    // the MFMA GEMM, which streams K through LDS in steps.
    const bool gemv_fits = w->mfma_tiles || w->path == Path::Generic || gemv_max_rows(*w) > 0;
    const bool mfma_ok = prefill_supported(*w) && w->K % 8 == 0 && ((uintptr_t)x & 15) == 0;
    if (!gemv_fits && !mfma_ok)
        return set_error(TBH_E_UNSUPPORTED,
                         "K = " + std::to_string(w->K) + " is too long for the GEMV kernels' staged x, and the "
                         "MFMA GEMM needs K % 8 == 0 and a 16-byte aligned x");
    if ((M >= mfma_min || !gemv_fits) && mfma_ok) {
        const hipError_t e = launch_prefill_f32(*w, x, w->K, M, y, w->N, s, scr);
        if (e == hipSuccess) return TBH_OK;
        if (e == hipErrorOutOfMemory && scr.is_fixed())
            return set_error(TBH_E_INVALID, "this call needs " + std::to_string(scr.shortfall) +
                                                " bytes of scratch; the no-allocation entry point holds " +
                                                std::to_string(scr.fixed_bytes));
        if (e != hipErrorInvalidValue) return hip_error(e, "matmul kernel launch");
        if (!gemv_fits) return set_error(TBH_E_UNSUPPORTED, "K too long for the GEMV kernels, shape refused by the MFMA GEMM");
        // shapes the GEMM does not take run on the GEMV kernels below
    }
    // 2..8 rows of x per launch on the matrix cores when the weight allows
    // it and M reaches sgemv_min_rows; below that the VALU kernels are as
    // fast or faster.  The device option TBH_OPT_SGEMV_MIN_ROWS sets one
    // threshold for every shape (2..9; 9 turns the MFMA path off).
    const int forced = w->dev->sgemv_min_rows.load(std::memory_order_relaxed);
    const int64_t sg_min = forced > 0 ? std::max(2, forced) : sgemv_min_rows(*w);
    const bool sg = M >= sg_min && sgemv_supported(*w);
    // Eight rows at a time on the burst GEMV when the weight and x allow it
    // and the matrix-core GEMV does not take them (INT4 2048x2048 at M = 8:
    // 6.9 us as two 4-row launches, 4.8 us as one), or takes them on a weight
    // of at most 12 Mi elements (INT4 5632x2048: 9.0 us there, 8.6-8.9 us as
    // one burst launch; 8192x2048: 9.2-9.4 against 10.5-11.0).  Five to seven
    // rows take the same launch with the rows past M masked (INT4 2048x2048
    // at M = 5 / 7: 6.3 / 8.2 us as 4 + 1 / 4 + 3 rows, 5.0 / 5.0 us as one
    // launch).
    const bool b8 = burst8 && M >= 5;
    const bool b8_over_sg = w->N * w->K <= ((int64_t)12 << 20);
    const int64_t rows = w->mfma_tiles || sg || b8 ? 8 : gemv_max_rows(*w);
    for (int64_t m0 = 0; m0 < M;) {
        int64_t mc = rows > 0 ? std::min(rows, M - m0) : M - m0;
        GemvArgs a{x + m0 * w->K, w->K, y + m0 * w->N, w->N, mc};
        hipError_t e = hipErrorInvalidValue;
        if (w->mfma_tiles) e = launch_mgemv(*w, a, s);
        else if (b8 && mc >= 5 && (!(sg && mc >= sg_min) || (mc == 8 && b8_over_sg))) e = launch_gemv(*w, a, s);
        if (e == hipErrorInvalidValue && !w->mfma_tiles && sg && mc >= sg_min) e = launch_sgemv(*w, a, s, scr);
        if (e == hipErrorOutOfMemory && scr.is_fixed())
            return set_error(TBH_E_INVALID, "this call needs " + std::to_string(scr.shortfall) +
                                                " bytes of scratch; the no-allocation entry point holds " +
                                                std::to_string(scr.fixed_bytes));
        if (e == hipErrorInvalidValue && !w->mfma_tiles) {
            // the VALU kernels (at most gemv_max_rows rows per launch)
            const int64_t vr = gemv_max_rows(*w);
            mc = vr > 0 ? std::min(vr, mc) : mc;
            a.M = mc;
            e = vr > 0 ? launch_gemv(*w, a, s) : launch_generic(*w, a, s);
        }
        if (e != hipSuccess) return hip_error(e, "matmul kernel launch");
        m0 += mc;
    }
    return TBH_OK;
}

tbh_status tbh_matmul_device(const tbh_weight *w, const float *x, int64_t M, int64_t K, float *y,
                             void *stream) {
    if (!w) return set_error(TBH_E_INVALID, "tbh_matmul_device: weight is NULL");
    if (M < 0) return set_error(TBH_E_INVALID, "tbh_matmul_device: M < 0");
    if (K != w->K) return set_error(TBH_E_INVALID, "Dimensions must match (x K != weight K)");
    if (M == 0) return TBH_OK;
    if (!x || !y) return set_error(TBH_E_INVALID, "tbh_matmul_device: x or y is NULL");
    tbh_status st = use_device(w->dev->ordinal);
    if (st != TBH_OK) return st;
    Scratch scr;
    scr.dev = w->dev;
    return matmul_enqueue(w, x, M, y, (hipStream_t)stream, scr);
}

tbh_status tbh_matmul_device_noalloc(const tbh_weight *w, const float *x, int64_t M, int64_t K, float *y,
                                     void *stream) {
    if (!w) return set_error(TBH_E_INVALID, "tbh_matmul_device_noalloc: weight is NULL");
    if (M < 0) return set_error(TBH_E_INVALID, "tbh_matmul_device_noalloc: M < 0");
    if (K != w->K) return set_error(TBH_E_INVALID, "Dimensions must match (x K != weight K)");
    if (M == 0) return TBH_OK;
    if (!x || !y) return set_error(TBH_E_INVALID, "tbh_matmul_device_noalloc: x or y is NULL");
    if (!w->dev->noalloc_scratch)
        return set_error(TBH_E_INVALID, "tbh_matmul_device_noalloc: device has no scratch address");
    tbh_status st = use_device(w->dev->ordinal);
    if (st != TBH_OK) return st;
    const int64_t limit = w->dev->noalloc_limit.load(std::memory_order_relaxed);
    Scratch scr;
    scr.fixed = w->dev->noalloc_scratch;
    scr.fixed_bytes = limit > 0 ? (size_t)limit : kNoAllocScratchBytes;
    return matmul_enqueue(w, x, M, y, (hipStream_t)stream, scr);
}

// y[m][n] += bias[n] over [M][N] (the bias add of ModelWeights.swift:51-63).
static __global__ __launch_bounds__(256) void add_bias_rows(float *y, const float *bias, int64_t M, int64_t N) {
    const int64_t total = M * N;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256)
        y[i] += bias[i % N];
}

tbh_status tbh_linear_device(const tbh_weight *w, const float *x, int64_t M, int64_t K, const float *bias,
                             float *y, void *stream) {
    tbh_status st = tbh_matmul_device(w, x, M, K, y, stream);
    if (st != TBH_OK || M == 0 || !bias) return st;
    const int64_t total = M * w->N;
    const int64_t blocks = std::min<int64_t>((total + 255) / 256, 4 * std::max(1, w->dev->cu_count));
    hipLaunchKernelGGL(add_bias_rows, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, y, bias, M,
                       w->N);
    TBH_HIP(hipGetLastError(), "tbh_linear_device: bias launch");
    return TBH_OK;
}

// x from page-locked host memory into the device staging buffer: one
// 16-byte load and store per thread (src and dst 16-byte aligned).
static __global__ __launch_bounds__(256) void stage_x(const float *__restrict__ src, float *__restrict__ dst,
                                                       int64_t n) {
    const int64_t n4 = n / 4, stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride)
        reinterpret_cast<float4 *>(dst)[i] = reinterpret_cast<const float4 *>(src)[i];
    for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

// Completion word for the host-pointer calls: one thread stores the call's
// sequence number into coherent host memory once every earlier launch on the
// stream has finished (stream order), so the host sees completion by reading
// its own memory instead of waiting for the stream's completion signal.
static __global__ __launch_bounds__(64) void mark_done(uint32_t *flag, uint32_t seq) {
    if (threadIdx.x == 0) __hip_atomic_store(flag, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// How tbh_matmul waits when the kernels write y into locked host memory
// (TBH_OPT_HOST_WAIT, initially TBH_HOST_WAIT): 1 (default) = a mark_done
// launch after the call's kernels, the host polling the word for up to
// kHostSpinUs before falling back to hipStreamSynchronize; 0 =
// hipStreamSynchronize.  INT4 g32 at M = 1, us per call, synchronize /
// poll: 2048x2048 18.2 / 14.8, 32000x2048 28.6 / 26.2; at M = 8 2048x2048
// 24.5 / 20.7.  With the DMA copies (TBH_OPT_HOST_ENTRY = 0) polling did not
// pay (M = 8 step 205 / 259 us) and the stream is synchronised.
constexpr double kHostSpinUs = 200.0;

// Waits for the work enqueued so far on dev->stream.  With TBH_HOST_WAIT = 1
// and a completion word, enqueues mark_done and polls the word (bounded),
// then falls back to (or finishes with) hipStreamSynchronize's status.
static hipError_t host_wait(tbh_device *dev) {
    if (dev->host_wait.load(std::memory_order_relaxed) == 1) {
        if (!dev->done_flag) {
            void *p = nullptr, *pd = nullptr;
            if (hipHostMalloc(&p, 64, hipHostMallocMapped | hipHostMallocCoherent) == hipSuccess) {
                if (hipHostGetDevicePointer(&pd, p, 0) == hipSuccess) {
                    dev->done_flag = (uint32_t *)p;
                    dev->done_flag_dev = (uint32_t *)pd;
                    __atomic_store_n(dev->done_flag, 0u, __ATOMIC_RELEASE);
                } else {
                    (void)hipHostFree(p);
                }
            }
        }
        if (dev->done_flag) {
            const uint32_t seq = ++dev->done_seq;
            hipLaunchKernelGGL(mark_done, dim3(1), dim3(64), 0, dev->stream, dev->done_flag_dev, seq);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            const auto t0 = std::chrono::steady_clock::now();
            while (__atomic_load_n(dev->done_flag, __ATOMIC_ACQUIRE) != seq) {
                const double us =
                    std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
                if (us > kHostSpinUs) return hipStreamSynchronize(dev->stream);
            }
            return hipSuccess;
        }
    }
    return hipStreamSynchronize(dev->stream);
}

// How tbh_matmul moves x and y when they fit the page-locked staging buffer
// (TBH_OPT_HOST_ENTRY, initially TBH_HOST_ENTRY): 0 = DMA copies to and from
// device staging; 1 = a copy kernel reads x from the locked buffer into
// device staging and the matmul kernels write y straight into the locked
// buffer; 2 (default) = as 1, except that one row of x is read by the matmul
// kernels straight from the locked buffer (no copy launch).  INT4 g32, us per
// call with the polled wait, modes 1 / 2: M = 1 2048x2048 14.8 / 12.9,
// 5632x2048 16.9 / 14.0, 32000x2048 26.2 / 23.1 (DMA copies: 19.7, 28.6,
// 38.0); at M = 8, where every block reading eight rows over the bus lost
// (2048x2048 20.7 against 24.7), the copy launch stays.

tbh_status tbh_matmul(tbh_device *dev, const float *x, int64_t M, int64_t K, const tbh_weight *w,
                      float *y) {
    if (!dev || !w) return set_error(TBH_E_INVALID, "tbh_matmul: NULL device or weight");
    if (w->dev != dev) return set_error(TBH_E_INVALID, "tbh_matmul: weight belongs to another device");
    if (M < 0) return set_error(TBH_E_INVALID, "tbh_matmul: M < 0");
    if (K != w->K) return set_error(TBH_E_INVALID, "Dimensions must match (x K != weight K)");
    if (M == 0) return TBH_OK;
    if (!x || !y) return set_error(TBH_E_INVALID, "tbh_matmul: x or y is NULL");
    std::lock_guard<std::mutex> lock(dev->mu);
    tbh_status st = use_device(dev->ordinal);
    if (st != TBH_OK) return st;
    const size_t xb = (size_t)(M * K) * sizeof(float), yb = (size_t)(M * w->N) * sizeof(float);
    const size_t need = ((xb + 255) & ~size_t(255)) + yb;
    if (dev->stage_bytes < need) {
        (void)hipFree(dev->stage);   // replaced below; a failed free leaves nothing to undo
        dev->stage = nullptr;
        dev->stage_bytes = 0;
        TBH_HIP(hipMalloc(&dev->stage, need), "tbh_matmul: staging buffer");
        dev->stage_bytes = need;
    }
    float *dx = (float *)dev->stage;
    float *dy = (float *)((char *)dev->stage + ((xb + 255) & ~size_t(255)));
    // Page-locked host staging: the CPU copies x into it and y out of it.  Up
    // to 8 rows of x the kernels read x from it and write y into it
    // themselves (TBH_OPT_HOST_ENTRY); more rows move by DMA from and to device
    // staging, which already beat the runtime's staging of pageable memory
    // (INT4 g32 at M = 1, us per call: 2048x2048 33.9 -> 19.7, 2048x5632
    // 33.7 -> 27.1).  Calls above kPinnedStageBytes, or when no locked memory
    // can be had, copy from the caller's arrays.
    bool pinned = need <= kPinnedStageBytes;
    if (pinned && dev->pin_bytes < need) {
        if (dev->pin) (void)hipHostFree(dev->pin);   // every earlier call has synchronised
        dev->pin = nullptr;
        dev->pin_dev = nullptr;
        dev->pin_bytes = 0;
        size_t grown = (size_t)1 << 20;
        while (grown < need) grown *= 2;
        // coherent: kernels that read x from it or write y into it (TBH_HOST_ENTRY
        // 1, 2) see the host's latest bytes, and the host sees theirs once the
        // stream has synchronised, whatever the caches held from earlier calls
        if (hipHostMalloc(&dev->pin, grown, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) {
            dev->pin = nullptr;
            pinned = false;
        } else if (hipHostGetDevicePointer(&dev->pin_dev, dev->pin, 0) != hipSuccess) {
            (void)hipHostFree(dev->pin);
            dev->pin = nullptr;
            dev->pin_dev = nullptr;
            pinned = false;
        } else {
            dev->pin_bytes = grown;
        }
    }
    float *px = pinned ? (float *)dev->pin : nullptr;
    float *py = pinned ? (float *)((char *)dev->pin + ((xb + 255) & ~size_t(255))) : nullptr;
    Scratch scr;
    scr.dev = dev;
    const int mode = pinned && M <= 8 ? dev->host_entry.load(std::memory_order_relaxed) : 0;
    if (mode > 0) {
        // the kernels address the locked buffer directly (device view of it)
        float *dpx = (float *)dev->pin_dev;
        float *dpy = (float *)((char *)dpx + ((xb + 255) & ~size_t(255)));
        std::memcpy(px, x, xb);
        const float *xin = dpx;
        if (mode == 1 || M > 1) {
            const int64_t n = M * K;
            const unsigned blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>(256, (n / 4 + 255) / 256));
            hipLaunchKernelGGL(stage_x, dim3(blocks), dim3(256), 0, dev->stream, (const float *)dpx, dx, n);
            TBH_HIP(hipGetLastError(), "tbh_matmul: stage x");
            xin = dx;
        }
        st = matmul_enqueue(w, xin, M, dpy, dev->stream, scr);
        if (st != TBH_OK) {
            (void)hipStreamSynchronize(dev->stream);
            return st;
        }
        TBH_HIP(host_wait(dev), "tbh_matmul: synchronize");
        std::memcpy(y, py, yb);
        return TBH_OK;
    }
    if (pinned) std::memcpy(px, x, xb);
    TBH_HIP(hipMemcpyAsync(dx, pinned ? px : x, xb, hipMemcpyHostToDevice, dev->stream), "tbh_matmul: copy x");
    st = matmul_enqueue(w, dx, M, dy, dev->stream, scr);
    if (st != TBH_OK) {
        // the copy of the caller's x may still be queued: wait for it before
        // the caller can release x (the status returned is the launch error)
        (void)hipStreamSynchronize(dev->stream);
        return st;
    }
    TBH_HIP(hipMemcpyAsync(pinned ? py : y, dy, yb, hipMemcpyDeviceToHost, dev->stream), "tbh_matmul: copy y");
    TBH_HIP(hipStreamSynchronize(dev->stream), "tbh_matmul: synchronize");
    if (pinned) std::memcpy(y, py, yb);
    return TBH_OK;
}

tbh_status tbh_matmul_bf16_device(const tbh_weight *w, const uint16_t *x, int64_t M, int64_t K,
                                  float *y, void *stream) {
    if (!w) return set_error(TBH_E_INVALID, "tbh_matmul_bf16_device: weight is NULL");
    if (M < 0) return set_error(TBH_E_INVALID, "tbh_matmul_bf16_device: M < 0");
    if (K != w->K) return set_error(TBH_E_INVALID, "Dimensions must match (x K != weight K)");
    if (M == 0) return TBH_OK;
    if (!x || !y) return set_error(TBH_E_INVALID, "tbh_matmul_bf16_device: x or y is NULL");
    if (!prefill_supported(*w))
        return set_error(TBH_E_UNSUPPORTED,
                         "tbh_matmul_bf16_device: needs an INT8 row, INT4 K-group or runtime-layout INT4 "
                         "weight (N-blocks of 16, 32 or a multiple of 64 rows) in the row layout");
    if (K % 8 != 0 || ((uintptr_t)x & 15) != 0)
        return set_error(TBH_E_UNSUPPORTED,
                         "tbh_matmul_bf16_device: needs K % 8 == 0 and a 16-byte aligned x");
    if (!weight_arrays_ok(*w))
        return set_error(TBH_E_INVALID, "weight device arrays are inconsistent with its layout");
    tbh_status st = use_device(w->dev->ordinal);
    if (st != TBH_OK) return st;
    Scratch scr;
    scr.dev = w->dev;
    hipError_t e = launch_prefill(*w, x, K, M, y, w->N, (hipStream_t)stream, scr);
    if (e != hipSuccess) return hip_error(e, "prefill kernel launch");
    return TBH_OK;
}

// ---------------------------------------------------------------------------
// dequantize
// ---------------------------------------------------------------------------
tbh_status tbh_dequantize_device(const tbh_weight *w, float *out, void *stream) {
    if (!w || !out) return set_error(TBH_E_INVALID, "tbh_dequantize_device: NULL argument");
    if (!weight_arrays_ok(*w))
        return set_error(TBH_E_INVALID, "weight device arrays are inconsistent with its layout");
    tbh_status st = use_device(w->dev->ordinal);
    if (st != TBH_OK) return st;
    hipError_t e = launch_dequant(*w, out, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "dequantize kernel launch");
    return TBH_OK;
}

tbh_status tbh_dequantize(tbh_device *dev, const tbh_weight *w, float *out) {
    if (!dev || !w || !out) return set_error(TBH_E_INVALID, "tbh_dequantize: NULL argument");
    if (w->dev != dev) return set_error(TBH_E_INVALID, "tbh_dequantize: weight belongs to another device");
    if (!weight_arrays_ok(*w))
        return set_error(TBH_E_INVALID, "weight device arrays are inconsistent with its layout");
    std::lock_guard<std::mutex> lock(dev->mu);
    tbh_status st = use_device(dev->ordinal);
    if (st != TBH_OK) return st;
    const size_t bytes = (size_t)(w->K * w->N) * sizeof(float);
    float *d = nullptr;
    TBH_HIP(hipMalloc(&d, bytes), "tbh_dequantize: output buffer");
    hipError_t e = launch_dequant(*w, d, dev->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(out, d, bytes, hipMemcpyDeviceToHost, dev->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
    const hipError_t ef = hipFree(d);
    if (e == hipSuccess) e = ef;
    if (e != hipSuccess) return hip_error(e, "tbh_dequantize");
    return TBH_OK;
}

}  // extern "C"

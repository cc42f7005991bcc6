// tbh_tbf.hip -- reader of TinyBrain Binary Format (.tbf) v1 files (host code).
//
// The format is what ModelWeights.save writes and ModelWeights.load reads
// (Sources/TinyBrainRuntime/ModelWeights.swift:376-488, :496-798), and what
// Scripts/convert_model.py:48-70, :462-706 writes:
//
//   "TBFM", u32 version = 1, u32 n, n bytes of config JSON        pad to 4 KiB
//   u32 count; per quantized tensor: u32 n, name, u8 precision (1 INT8,
//     2 INT4), u8 mode, u32 group size, u32 n, f32 scales[n], u32 n,
//     i8 zero points[n]                                            pad to 4 KiB
//   u32 count; per tensor: u32 n, name, u32 ndim, i32 dims[ndim],
//     u64 absolute offset, u64 byte size                           pad to 4 KiB
//   blobs, each 4 KiB aligned (fp32 or the quantized data bytes)
//
// The file is memory-mapped (the reference reads it whole,
// ModelWeights.swift:505) and every field is bounds-checked: a malformed file
// is TBH_E_INVALID, never a read past the mapping.  Quantized tensors map to
// descriptors as ModelWeights.load does (:676-685): precision 2 is INT4;
// INT8 mode 2 is per-channel, any other INT8 mode symmetric.  INT4 data from
// the converter (mode byte 3) is the PyTorch [N, K] array flattened with the
// shape stored reversed (convert_model.py:489-502), i.e. TBH_LAYOUT_NK_FLAT;
// INT4 from ModelWeights.save (mode byte 2) is the runtime [K, N] layout.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "tbh_internal.h"

struct tbh_tbf {
    int fd = -1;
    const uint8_t *base = nullptr;
    size_t size = 0;
    std::string config_json;
    tbh_tbf_config config{};
    struct Meta {
        uint8_t precision = 0, mode = 0;
        uint32_t group_size = 0;
        std::vector<float> scales_copy;  // copied: the mapping may be unaligned here
        std::vector<int8_t> zp;
    };
    struct Tensor {
        std::string name;
        std::vector<int64_t> dims;
        uint64_t offset = 0, bytes = 0;
        int meta = -1;  // index into metas, -1 when fp32
    };
    std::vector<Meta> metas;
    std::vector<Tensor> tensors;
    std::map<std::string, int> by_name;
    std::map<std::string, int> meta_by_name;
};

namespace tbh {
namespace {

struct Cursor {
    const uint8_t *p;
    size_t n, off = 0;
    bool ok = true;
    bool need(size_t k) {
        if (!ok || k > n || off > n - k) ok = false;
        return ok;
    }
    template <class T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, p + off, sizeof(T));
            off += sizeof(T);
        }
        return v;
    }
    std::string str(size_t len) {
        if (!need(len)) return {};
        std::string s(reinterpret_cast<const char *>(p + off), len);
        off += len;
        return s;
    }
    void align4k() { off = ((off + 4095) / 4096) * 4096; }
};

// Minimal reader of the flat JSON object the two writers produce:
// {"key": number | "string", ...}.  Returns false on anything else.
bool parse_config(const std::string &js, tbh_tbf_config &c) {
    std::map<std::string, std::string> kv;
    size_t i = 0;
    auto ws = [&] { while (i < js.size() && isspace((unsigned char)js[i])) ++i; };
    ws();
    if (i >= js.size() || js[i] != '{') return false;
    ++i;
    for (;;) {
        ws();
        if (i < js.size() && js[i] == '}') break;
        if (i >= js.size() || js[i] != '"') return false;
        size_t e = js.find('"', i + 1);
        if (e == std::string::npos) return false;
        std::string key = js.substr(i + 1, e - i - 1);
        i = e + 1;
        ws();
        if (i >= js.size() || js[i] != ':') return false;
        ++i;
        ws();
        std::string val;
        if (i < js.size() && js[i] == '"') {
            e = js.find('"', i + 1);
            if (e == std::string::npos) return false;
            val = js.substr(i + 1, e - i - 1);
            i = e + 1;
        } else {
            size_t s = i;
            while (i < js.size() && js[i] != ',' && js[i] != '}' && !isspace((unsigned char)js[i])) ++i;
            val = js.substr(s, i - s);
        }
        kv[key] = val;
        ws();
        if (i < js.size() && js[i] == ',') {
            ++i;
            continue;
        }
        if (i < js.size() && js[i] == '}') break;
        return false;
    }
    auto num = [&](const char *k, double dflt, bool required, bool *ok) -> double {
        auto it = kv.find(k);
        if (it == kv.end()) {
            if (required) *ok = false;
            return dflt;
        }
        char *end = nullptr;
        double v = strtod(it->second.c_str(), &end);
        if (end == it->second.c_str()) *ok = false;
        return v;
    };
    bool ok = true;
    // required and defaulted keys as ModelConfig.init(from:) (ModelRunner.swift:109-120)
    c.num_layers = (int32_t)num("numLayers", 0, true, &ok);
    c.hidden = (int32_t)num("hiddenDim", 0, true, &ok);
    c.num_heads = (int32_t)num("numHeads", 0, true, &ok);
    c.vocab = (int32_t)num("vocabSize", 0, true, &ok);
    c.max_seq = (int32_t)num("maxSeqLen", 0, true, &ok);
    c.num_kv_heads = (int32_t)num("numKVHeads", c.num_heads, false, &ok);
    c.intermediate = (int32_t)num("intermediateDim", 4.0 * c.hidden, false, &ok);
    c.partial_rotary_factor = (float)num("partialRotaryFactor", 1.0, false, &ok);
    auto a = kv.find("architecture");
    const std::string arch = a == kv.end() ? "llama" : a->second;
    std::memset(c.architecture, 0, sizeof(c.architecture));
    std::strncpy(c.architecture, arch.c_str(), sizeof(c.architecture) - 1);
    return ok && c.num_layers > 0 && c.hidden > 0 && c.num_heads > 0 && c.vocab > 0 && c.num_kv_heads > 0 &&
           c.intermediate > 0;
}

tbh_status parse(tbh_tbf &f) {
    Cursor c{f.base, f.size};
    if (c.str(4) != "TBFM") return set_error(TBH_E_INVALID, "tbf: bad magic (not a TBF file)");
    const uint32_t version = c.get<uint32_t>();
    if (!c.ok) return set_error(TBH_E_INVALID, "tbf: file too small");
    if (version != 1) return set_error(TBH_E_UNSUPPORTED, "tbf: unsupported version " + std::to_string(version));
    const uint32_t clen = c.get<uint32_t>();
    f.config_json = c.str(clen);
    if (!c.ok) return set_error(TBH_E_INVALID, "tbf: truncated config");
    if (!parse_config(f.config_json, f.config)) return set_error(TBH_E_INVALID, "tbf: unreadable config JSON");

    c.align4k();
    const uint32_t nmeta = c.get<uint32_t>();
    if (!c.ok || nmeta > f.size / 14) return set_error(TBH_E_INVALID, "tbf: bad metadata count");
    for (uint32_t i = 0; i < nmeta; ++i) {
        const uint32_t nl = c.get<uint32_t>();
        if (!c.ok || nl > 4096) return set_error(TBH_E_INVALID, "tbf: bad tensor name length");
        std::string name = c.str(nl);
        tbh_tbf::Meta m;
        m.precision = c.get<uint8_t>();
        m.mode = c.get<uint8_t>();
        m.group_size = c.get<uint32_t>();
        const uint32_t ns = c.get<uint32_t>();
        if (!c.ok || !c.need((size_t)ns * 4)) return set_error(TBH_E_INVALID, "tbf: truncated scales");
        m.scales_copy.resize(ns);
        std::memcpy(m.scales_copy.data(), f.base + c.off, (size_t)ns * 4);
        c.off += (size_t)ns * 4;
        const uint32_t nz = c.get<uint32_t>();
        if (!c.ok || !c.need(nz)) return set_error(TBH_E_INVALID, "tbf: truncated zero points");
        m.zp.resize(nz);
        std::memcpy(m.zp.data(), f.base + c.off, nz);
        c.off += nz;
        if (m.precision != 1 && m.precision != 2)
            return set_error(TBH_E_UNSUPPORTED, "tbf: precision code " + std::to_string(m.precision) + " of " + name);
        f.meta_by_name[name] = (int)f.metas.size();
        f.metas.push_back(std::move(m));
    }

    c.align4k();
    const uint32_t nt = c.get<uint32_t>();
    if (!c.ok || nt > f.size / 24) return set_error(TBH_E_INVALID, "tbf: bad tensor count");
    for (uint32_t i = 0; i < nt; ++i) {
        tbh_tbf::Tensor t;
        const uint32_t nl = c.get<uint32_t>();
        if (!c.ok || nl > 4096) return set_error(TBH_E_INVALID, "tbf: bad tensor name length");
        t.name = c.str(nl);
        const uint32_t nd = c.get<uint32_t>();
        if (!c.ok || nd < 1 || nd > 4) return set_error(TBH_E_INVALID, "tbf: bad rank of " + t.name);
        int64_t count = 1;
        for (uint32_t d = 0; d < nd; ++d) {
            const int32_t v = c.get<int32_t>();
            if (v <= 0) return set_error(TBH_E_INVALID, "tbf: bad dimension of " + t.name);
            t.dims.push_back(v);
            count *= v;
            if (count > (int64_t)1 << 40) return set_error(TBH_E_INVALID, "tbf: tensor too large: " + t.name);
        }
        t.offset = c.get<uint64_t>();
        t.bytes = c.get<uint64_t>();
        if (!c.ok) return set_error(TBH_E_INVALID, "tbf: truncated index");
        if (t.offset > f.size || t.bytes > f.size - t.offset)
            return set_error(TBH_E_INVALID, "tbf: blob of " + t.name + " lies outside the file");
        auto mi = f.meta_by_name.find(t.name);
        if (mi != f.meta_by_name.end()) {
            t.meta = mi->second;
            const tbh_tbf::Meta &m = f.metas[(size_t)t.meta];
            const int64_t want = m.precision == 2 ? (count + 1) / 2 : count;
            if ((int64_t)t.bytes != want)
                return set_error(TBH_E_INVALID, "tbf: data size of " + t.name + " does not match its shape");
        } else if ((int64_t)t.bytes != 4 * count || t.offset % 4 != 0) {
            return set_error(TBH_E_INVALID, "tbf: fp32 blob of " + t.name + " does not match its shape");
        }
        if (f.by_name.count(t.name)) return set_error(TBH_E_INVALID, "tbf: duplicate tensor " + t.name);
        f.by_name[t.name] = (int)f.tensors.size();
        f.tensors.push_back(std::move(t));
    }
    return TBH_OK;
}

}  // namespace
}  // namespace tbh

using namespace tbh;

extern "C" {

tbh_status tbh_tbf_close(tbh_tbf *f) {
    if (!f) return TBH_OK;
    if (f->base) munmap(const_cast<uint8_t *>(f->base), f->size);
    if (f->fd >= 0) close(f->fd);
    delete f;
    return TBH_OK;
}

tbh_status tbh_tbf_open(const char *path, tbh_tbf **out) {
    if (!out) return set_error(TBH_E_INVALID, "tbh_tbf_open: out is NULL");
    *out = nullptr;
    if (!path) return set_error(TBH_E_INVALID, "tbh_tbf_open: path is NULL");
    std::unique_ptr<tbh_tbf> f(new tbh_tbf);
    f->fd = open(path, O_RDONLY);
    if (f->fd < 0) return set_error(TBH_E_INVALID, std::string("tbf: cannot open ") + path);
    struct stat st;
    if (fstat(f->fd, &st) != 0 || st.st_size < 12) {
        tbh_tbf_close(f.release());
        return set_error(TBH_E_INVALID, "tbf: file too small");
    }
    f->size = (size_t)st.st_size;
    void *m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (m == MAP_FAILED) {
        tbh_tbf_close(f.release());
        return set_error(TBH_E_OOM, "tbf: mmap failed");
    }
    f->base = (const uint8_t *)m;
    tbh_status st2 = parse(*f);
    if (st2 != TBH_OK) {
        tbh_tbf_close(f.release());
        return st2;
    }
    *out = f.release();
    return TBH_OK;
}

tbh_status tbh_tbf_get_config(const tbh_tbf *f, tbh_tbf_config *cfg) {
    if (!f || !cfg) return set_error(TBH_E_INVALID, "tbh_tbf_get_config: NULL argument");
    *cfg = f->config;
    return TBH_OK;
}

int32_t tbh_tbf_tensor_count(const tbh_tbf *f) { return f ? (int32_t)f->tensors.size() : 0; }

tbh_status tbh_tbf_tensor(const tbh_tbf *f, int32_t i, tbh_tbf_tensor_info *t) {
    if (!f || !t) return set_error(TBH_E_INVALID, "tbh_tbf_tensor: NULL argument");
    if (i < 0 || i >= (int32_t)f->tensors.size()) return set_error(TBH_E_INVALID, "tbh_tbf_tensor: index");
    const auto &x = f->tensors[(size_t)i];
    std::memset(t, 0, sizeof(*t));
    t->name = x.name.c_str();
    t->ndim = (int32_t)x.dims.size();
    for (size_t d = 0; d < x.dims.size(); ++d) t->dims[d] = x.dims[d];
    t->offset = (int64_t)x.offset;
    t->bytes = (int64_t)x.bytes;
    t->quantized = x.meta >= 0;
    return TBH_OK;
}

tbh_status tbh_tbf_find(const tbh_tbf *f, const char *name, int32_t *index) {
    if (!f || !name || !index) return set_error(TBH_E_INVALID, "tbh_tbf_find: NULL argument");
    auto it = f->by_name.find(name);
    if (it == f->by_name.end()) return set_error(TBH_E_INVALID, std::string("tbf: missing tensor ") + name);
    *index = it->second;
    return TBH_OK;
}

tbh_status tbh_tbf_qtensor(const tbh_tbf *f, int32_t i, tbh_qtensor_desc *d) {
    if (!f || !d) return set_error(TBH_E_INVALID, "tbh_tbf_qtensor: NULL argument");
    if (i < 0 || i >= (int32_t)f->tensors.size()) return set_error(TBH_E_INVALID, "tbh_tbf_qtensor: index");
    const auto &t = f->tensors[(size_t)i];
    if (t.meta < 0) return set_error(TBH_E_INVALID, "tbf: " + t.name + " is not quantized");
    if (t.dims.size() != 2) return set_error(TBH_E_INVALID, "tbf: " + t.name + " is not 2-D");
    const auto &m = f->metas[(size_t)t.meta];
    std::memset(d, 0, sizeof(*d));
    d->K = t.dims[0];
    d->N = t.dims[1];
    if (m.precision == 2) {
        d->precision = TBH_PREC_INT4;
        d->mode = TBH_MODE_INT4;
        d->layout = m.mode == 3 ? TBH_LAYOUT_NK_FLAT : TBH_LAYOUT_KN_FLAT;
    } else {
        d->precision = TBH_PREC_INT8;
        d->mode = m.mode == 2 ? TBH_MODE_PER_CHANNEL : TBH_MODE_SYMMETRIC;
        d->layout = TBH_LAYOUT_KN_FLAT;
    }
    d->group_size = (int32_t)m.group_size;
    d->data = reinterpret_cast<const int8_t *>(f->base + t.offset);
    d->data_bytes = (int64_t)t.bytes;
    d->scales = m.scales_copy.data();
    d->n_scales = (int64_t)m.scales_copy.size();
    d->zero_points = m.zp.empty() ? nullptr : m.zp.data();
    d->n_zero_points = (int64_t)m.zp.size();
    return TBH_OK;
}

tbh_status tbh_tbf_floats(const tbh_tbf *f, int32_t i, const float **data, int64_t *count) {
    if (!f || !data || !count) return set_error(TBH_E_INVALID, "tbh_tbf_floats: NULL argument");
    if (i < 0 || i >= (int32_t)f->tensors.size()) return set_error(TBH_E_INVALID, "tbh_tbf_floats: index");
    const auto &t = f->tensors[(size_t)i];
    if (t.meta >= 0) return set_error(TBH_E_INVALID, "tbf: " + t.name + " is quantized, not fp32");
    *data = reinterpret_cast<const float *>(f->base + t.offset);
    *count = (int64_t)(t.bytes / 4);
    return TBH_OK;
}

tbh_status tbh_tbf_load_decoder(tbh_device *dev, const tbh_tbf *f, int32_t max_seq, tbh_decoder **out) {
    if (!out) return set_error(TBH_E_INVALID, "tbh_tbf_load_decoder: out is NULL");
    *out = nullptr;
    if (!dev || !f) return set_error(TBH_E_INVALID, "tbh_tbf_load_decoder: NULL argument");
    const tbh_tbf_config &c = f->config;
    if (std::string(c.architecture) != "llama" || c.partial_rotary_factor != 1.0f)
        return set_error(TBH_E_UNSUPPORTED,
                         "tbf: the GPU decoder covers the LLaMA architecture (full RoPE) only");
    auto idx = [&](const std::string &name, int32_t *i) { return tbh_tbf_find(f, name.c_str(), i); };
    auto floats = [&](const std::string &name, int64_t want, const float **p) -> tbh_status {
        int32_t i;
        tbh_status st = idx(name, &i);
        int64_t n = 0;
        if (st == TBH_OK) st = tbh_tbf_floats(f, i, p, &n);
        if (st == TBH_OK && n != want) st = set_error(TBH_E_INVALID, "tbf: " + name + " has the wrong size");
        return st;
    };
    auto qt = [&](const std::string &name, tbh_qtensor_desc *d) -> tbh_status {
        int32_t i;
        tbh_status st = idx(name, &i);
        if (st == TBH_OK) st = tbh_tbf_qtensor(f, i, d);
        return st;
    };
    for (const char *b : {"output_bias", "final_norm_bias"})
        if (f->by_name.count(b)) return set_error(TBH_E_UNSUPPORTED, "tbf: biases are not supported by the decoder");
    tbh_decoder_config dc{};
    dc.num_layers = c.num_layers;
    dc.hidden = c.hidden;
    dc.num_heads = c.num_heads;
    dc.num_kv_heads = c.num_kv_heads;
    dc.intermediate = c.intermediate;
    dc.vocab = c.vocab;
    dc.max_seq = max_seq > 0 ? max_seq : c.max_seq;
    dc.rms_eps = 1e-5f;
    dc.rope_base = 10000.0f;
    const float *emb, *fnorm;
    tbh_qtensor_desc lm;
    tbh_status st = floats("embeddings", (int64_t)c.vocab * c.hidden, &emb);
    if (st == TBH_OK) st = floats("final_norm", c.hidden, &fnorm);
    if (st == TBH_OK) st = qt("output", &lm);
    tbh_decoder *dec = nullptr;
    if (st == TBH_OK) st = tbh_decoder_create(dev, &dc, emb, fnorm, &lm, &dec);
    for (int32_t l = 0; st == TBH_OK && l < c.num_layers; ++l) {
        const std::string p = "layer_" + std::to_string(l) + "_";
        for (const char *b : {"attn_q_bias", "attn_k_bias", "attn_v_bias", "attn_o_bias", "ffn_up_bias",
                              "ffn_down_bias", "ln_input_bias"})
            if (f->by_name.count(p + b)) st = set_error(TBH_E_UNSUPPORTED, "tbf: biases are not supported by the decoder");
        if (st == TBH_OK && !f->by_name.count(p + "ffn_gate"))
            st = set_error(TBH_E_UNSUPPORTED, "tbf: the decoder needs a gated (SwiGLU) FFN");
        tbh_qtensor_desc q{}, k{}, v{}, o{}, g{}, u{}, dn{};
        const float *gin = nullptr, *gpost = nullptr;
        if (st == TBH_OK) st = qt(p + "attn_q", &q);
        if (st == TBH_OK) st = qt(p + "attn_k", &k);
        if (st == TBH_OK) st = qt(p + "attn_v", &v);
        if (st == TBH_OK) st = qt(p + "attn_o", &o);
        if (st == TBH_OK) st = qt(p + "ffn_gate", &g);
        if (st == TBH_OK) st = qt(p + "ffn_up", &u);
        if (st == TBH_OK) st = qt(p + "ffn_down", &dn);
        if (st == TBH_OK) st = floats(p + "ln_input", c.hidden, &gin);
        if (st == TBH_OK) st = floats(p + "ln_post", c.hidden, &gpost);
        if (st == TBH_OK) st = tbh_decoder_set_layer(dec, l, gin, gpost, &q, &k, &v, &o, &g, &u, &dn);
    }
    if (st != TBH_OK) {
        tbh_decoder_destroy(dec);
        return st;
    }
    *out = dec;
    return TBH_OK;
}

}  // extern "C"

// safetensors reader, NeMo tensor-name map and weight loaders (include/ud_safetensors.h).
// Host-only C++.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/ud_safetensors.h"

int ud_set_error(int code, const char* msg);   // encoder.hip

namespace {

int sfail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return ud_set_error(code, buf);
}

// ------------------------------------------------------------------ a JSON subset parser
// Enough JSON for a safetensors header: objects, arrays, strings (with escapes), numbers,
// true/false/null.  Values are kept as a small tree.
struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0;
    int64_t inum = 0;
    bool is_int = false;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
};

struct JParser {
    const char* p;
    const char* e;
    int depth = 0;
    bool ok = true;

    void ws() { while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++; }
    bool lit(const char* s) {
        const size_t n = strlen(s);
        if ((size_t)(e - p) < n || strncmp(p, s, n) != 0) return false;
        p += n;
        return true;
    }
    bool string(std::string& out) {
        if (p >= e || *p != '"') return false;
        p++;
        while (p < e && *p != '"') {
            if (*p == '\\') {
                if (++p >= e) return false;
                switch (*p) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        if (e - p < 5) return false;
                        unsigned cp = 0;
                        for (int i = 1; i <= 4; i++) {
                            const char c = p[i];
                            cp <<= 4;
                            if (c >= '0' && c <= '9') cp |= c - '0';
                            else if (c >= 'a' && c <= 'f') cp |= c - 'a' + 10;
                            else if (c >= 'A' && c <= 'F') cp |= c - 'A' + 10;
                            else return false;
                        }
                        p += 4;
                        if (cp < 0x80) out += (char)cp;                       // names here are ASCII
                        else if (cp < 0x800) { out += (char)(0xC0 | (cp >> 6)); out += (char)(0x80 | (cp & 63)); }
                        else { out += (char)(0xE0 | (cp >> 12)); out += (char)(0x80 | ((cp >> 6) & 63)); out += (char)(0x80 | (cp & 63)); }
                        break;
                    }
                    default: return false;
                }
                p++;
            } else {
                out += *p++;
            }
        }
        if (p >= e) return false;
        p++;
        return true;
    }
    bool value(JVal& v) {
        if (++depth > 64) return false;
        ws();
        if (p >= e) return false;
        bool r = true;
        if (*p == '{') {
            v.kind = JVal::OBJ;
            p++;
            ws();
            if (p < e && *p == '}') { p++; depth--; return true; }
            while (r) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p >= e || *p != ':') return false;
                p++;
                JVal x;
                if (!value(x)) return false;
                v.obj.emplace_back(std::move(k), std::move(x));
                ws();
                if (p < e && *p == ',') { p++; continue; }
                if (p < e && *p == '}') { p++; break; }
                return false;
            }
        } else if (*p == '[') {
            v.kind = JVal::ARR;
            p++;
            ws();
            if (p < e && *p == ']') { p++; depth--; return true; }
            while (true) {
                JVal x;
                if (!value(x)) return false;
                v.arr.push_back(std::move(x));
                ws();
                if (p < e && *p == ',') { p++; continue; }
                if (p < e && *p == ']') { p++; break; }
                return false;
            }
        } else if (*p == '"') {
            v.kind = JVal::STR;
            r = string(v.str);
        } else if (lit("true")) {
            v.kind = JVal::BOOL; v.num = 1;
        } else if (lit("false")) {
            v.kind = JVal::BOOL;
        } else if (lit("null")) {
            v.kind = JVal::NUL;
        } else {
            const char* s = p;
            if (p < e && (*p == '-' || *p == '+')) p++;
            bool frac = false;
            while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '-' || *p == '+')) {
                if (*p == '.' || *p == 'e' || *p == 'E') frac = true;
                p++;
            }
            if (p == s) return false;
            std::string t(s, p);
            char* end = nullptr;
            v.kind = JVal::NUM;
            v.num = strtod(t.c_str(), &end);
            if (end != t.c_str() + t.size()) return false;
            if (!frac) {
                v.inum = strtoll(t.c_str(), &end, 10);
                v.is_int = end == t.c_str() + t.size();
            }
        }
        depth--;
        return r;
    }
};

// ------------------------------------------------------------------ name map
// HF model.safetensors name -> NeMo state_dict name (docs/specs/nemotron.md:246-287).  Prefix rewrites
// first (whole-name prefixes), then per-layer attention / conv-norm suffixes.
struct Rewrite { const char* from; const char* to; };
const Rewrite kPrefix[] = {
    {"encoder.subsampling.conv_in.", "encoder.pre_encode.conv.0."},
    {"encoder.subsampling.layers.0.depthwise_conv.", "encoder.pre_encode.conv.2."},
    {"encoder.subsampling.layers.0.pointwise_conv.", "encoder.pre_encode.conv.3."},
    {"encoder.subsampling.layers.1.depthwise_conv.", "encoder.pre_encode.conv.5."},
    {"encoder.subsampling.layers.1.pointwise_conv.", "encoder.pre_encode.conv.6."},
    {"encoder.subsampling.linear.", "encoder.pre_encode.out."},
    {"decoder.embedding.", "decoder.prediction.embed."},
    {"decoder.lstm.", "decoder.prediction.dec_rnn.lstm."},
    {"decoder.decoder_projector.", "joint.pred."},
    {"encoder_projector.", "joint.enc."},
    {"joint.head.", "joint.joint_net.2."},
};
const Rewrite kLayerSuffix[] = {
    {"self_attn.q_proj.weight", "self_attn.linear_q.weight"},
    {"self_attn.k_proj.weight", "self_attn.linear_k.weight"},
    {"self_attn.v_proj.weight", "self_attn.linear_v.weight"},
    {"self_attn.o_proj.weight", "self_attn.linear_out.weight"},
    {"self_attn.relative_k_proj.weight", "self_attn.linear_pos.weight"},
    {"self_attn.bias_u", "self_attn.pos_bias_u"},
    {"self_attn.bias_v", "self_attn.pos_bias_v"},
    {"conv.norm.weight", "conv.batch_norm.weight"},
    {"conv.norm.bias", "conv.batch_norm.bias"},
};

std::string nemo_name(const std::string& n) {
    for (const Rewrite& r : kPrefix) {
        const size_t k = strlen(r.from);
        if (n.compare(0, k, r.from) == 0) return std::string(r.to) + n.substr(k);
    }
    const char* lp = "encoder.layers.";
    if (n.compare(0, strlen(lp), lp) == 0) {
        const size_t dot = n.find('.', strlen(lp));
        if (dot != std::string::npos) {
            const std::string suffix = n.substr(dot + 1);
            for (const Rewrite& r : kLayerSuffix)
                if (suffix == r.from) return n.substr(0, dot + 1) + r.to;
        }
    }
    return n;
}

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const int exp = (h >> 10) & 0x1F;
    const uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {                                   // subnormal: man * 2^-24
            float v = (float)man * (1.0f / 16777216.0f);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((uint32_t)(exp + 112) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

}  // namespace

struct ud_safetensors {
    struct Entry {
        std::string name;
        int dtype;
        size_t elem;
        std::vector<int64_t> shape;
        int64_t count;
        size_t begin, end;                         // absolute file offsets
    };
    void* base = nullptr;
    size_t size = 0;
    std::vector<Entry> entries;                    // sorted by name
    std::map<std::string, size_t> index;
};

extern "C" UD_API int ud_safetensors_open(const char* path, ud_safetensors** out) {
    if (!path || !out) return sfail(UD_ERR_INVALID, "ud_safetensors_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return sfail(UD_ERR_WEIGHT, "ud_safetensors_open: cannot open %s", path);
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 8) {
        close(fd);
        return sfail(UD_ERR_WEIGHT, "ud_safetensors_open: %s is not a safetensors file (too short)", path);
    }
    const size_t size = (size_t)sb.st_size;
    void* base = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (base == MAP_FAILED) return sfail(UD_ERR_WEIGHT, "ud_safetensors_open: mmap of %s failed", path);
    ud_safetensors* st = new ud_safetensors();
    st->base = base;
    st->size = size;
    auto bad = [&](const char* why) {
        ud_safetensors_close(st);
        return sfail(UD_ERR_WEIGHT, "ud_safetensors_open: %s: %s", path, why);
    };
    uint64_t hn = 0;
    memcpy(&hn, base, 8);                          // little-endian (the only byte order targeted)
    if (hn > size - 8) return bad("header length beyond the end of the file");
    const char* hp = static_cast<const char*>(base) + 8;
    JParser jp{hp, hp + hn};
    JVal root;
    if (!jp.value(root) || root.kind != JVal::OBJ) return bad("header is not a JSON object");
    const size_t data0 = 8 + (size_t)hn;
    for (auto& kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const JVal& v = kv.second;
        if (v.kind != JVal::OBJ) return bad("tensor entry is not an object");
        const JVal *dt = nullptr, *sh = nullptr, *off = nullptr;
        for (auto& f : v.obj) {
            if (f.first == "dtype") dt = &f.second;
            else if (f.first == "shape") sh = &f.second;
            else if (f.first == "data_offsets") off = &f.second;
        }
        if (!dt || dt->kind != JVal::STR || !sh || sh->kind != JVal::ARR || !off || off->kind != JVal::ARR ||
            off->arr.size() != 2)
            return bad("tensor entry lacks dtype / shape / data_offsets");
        ud_safetensors::Entry en;
        en.name = kv.first;
        static const struct { const char* n; int d; size_t s; } kinds[] = {
            {"F32", UD_ST_F32, 4}, {"BF16", UD_ST_BF16, 2}, {"F16", UD_ST_F16, 2}, {"F64", UD_ST_OTHER, 8},
            {"I64", UD_ST_OTHER, 8}, {"I32", UD_ST_OTHER, 4}, {"I16", UD_ST_OTHER, 2}, {"I8", UD_ST_OTHER, 1},
            {"U8", UD_ST_OTHER, 1}, {"BOOL", UD_ST_OTHER, 1}};
        en.dtype = -1;
        for (auto& k : kinds)
            if (dt->str == k.n) { en.dtype = k.d; en.elem = k.s; }
        if (en.dtype < 0) return bad("unknown dtype");
        en.count = 1;
        for (const JVal& d : sh->arr) {
            if (d.kind != JVal::NUM || !d.is_int || d.inum < 0) return bad("bad shape");
            en.shape.push_back(d.inum);
            en.count *= d.inum;
        }
        if (en.shape.size() > 8) return bad("rank above 8");
        for (const JVal& o : off->arr)
            if (o.kind != JVal::NUM || !o.is_int || o.inum < 0) return bad("bad data_offsets");
        en.begin = data0 + (size_t)off->arr[0].inum;
        en.end = data0 + (size_t)off->arr[1].inum;
        if (en.begin > en.end || en.end > size) return bad("data_offsets outside the file");
        if (en.end - en.begin != (size_t)en.count * en.elem) return bad("byte range does not match dtype x shape");
        st->entries.push_back(std::move(en));
    }
    std::sort(st->entries.begin(), st->entries.end(),
              [](const ud_safetensors::Entry& a, const ud_safetensors::Entry& b) { return a.name < b.name; });
    for (size_t i = 0; i < st->entries.size(); i++) {
        if (!st->index.emplace(st->entries[i].name, i).second) return bad("duplicate tensor name");
    }
    *out = st;
    return UD_OK;
}

extern "C" UD_API void ud_safetensors_close(ud_safetensors* st) {
    if (!st) return;
    if (st->base) munmap(st->base, st->size);
    delete st;
}

extern "C" UD_API int32_t ud_safetensors_count(const ud_safetensors* st) { return st ? (int32_t)st->entries.size() : 0; }

extern "C" UD_API const char* ud_safetensors_name(const ud_safetensors* st, int32_t i) {
    if (!st || i < 0 || i >= (int32_t)st->entries.size()) return nullptr;
    return st->entries[i].name.c_str();
}

static const ud_safetensors::Entry* find(const ud_safetensors* st, const char* name) {
    auto it = st->index.find(name);
    return it == st->index.end() ? nullptr : &st->entries[it->second];
}

extern "C" UD_API int ud_safetensors_info(const ud_safetensors* st, const char* name, int32_t* dtype, int64_t* shape,
                                          int32_t* ndim) {
    if (!st || !name) return sfail(UD_ERR_INVALID, "ud_safetensors_info: null argument");
    const ud_safetensors::Entry* e = find(st, name);
    if (!e) return sfail(UD_ERR_WEIGHT, "ud_safetensors_info: no tensor '%s'", name);
    if (dtype) *dtype = e->dtype;
    if (ndim) *ndim = (int32_t)e->shape.size();
    if (shape)
        for (size_t i = 0; i < e->shape.size(); i++) shape[i] = e->shape[i];
    return UD_OK;
}

extern "C" UD_API int ud_safetensors_read_f32(const ud_safetensors* st, const char* name, float* out, int64_t count) {
    if (!st || !name || (!out && count > 0)) return sfail(UD_ERR_INVALID, "ud_safetensors_read_f32: null argument");
    const ud_safetensors::Entry* e = find(st, name);
    if (!e) return sfail(UD_ERR_WEIGHT, "ud_safetensors_read_f32: no tensor '%s'", name);
    if (count != e->count)
        return sfail(UD_ERR_WEIGHT, "ud_safetensors_read_f32: '%s' has %lld values, %lld requested", name,
                     (long long)e->count, (long long)count);
    const uint8_t* p = static_cast<const uint8_t*>(st->base) + e->begin;
    switch (e->dtype) {
        case UD_ST_F32: memcpy(out, p, (size_t)count * 4); break;
        case UD_ST_BF16:
            for (int64_t i = 0; i < count; i++) {
                uint16_t b;
                memcpy(&b, p + 2 * i, 2);
                const uint32_t u = (uint32_t)b << 16;
                memcpy(&out[i], &u, 4);
            }
            break;
        case UD_ST_F16:
            for (int64_t i = 0; i < count; i++) {
                uint16_t h;
                memcpy(&h, p + 2 * i, 2);
                out[i] = half_to_float(h);
            }
            break;
        default: return sfail(UD_ERR_WEIGHT, "ud_safetensors_read_f32: '%s' is not F32, F16 or BF16", name);
    }
    return UD_OK;
}

extern "C" UD_API int ud_nemo_name(const char* name, char* out, int32_t cap) {
    if (!name || !out || cap < 1) return sfail(UD_ERR_INVALID, "ud_nemo_name: bad argument");
    const std::string n = nemo_name(name);
    if ((int32_t)n.size() + 1 > cap) return sfail(UD_ERR_SHAPE, "ud_nemo_name: buffer too small");
    memcpy(out, n.c_str(), n.size() + 1);
    return UD_OK;
}

// Loads the tensors whose NeMo name `want` accepts into `set`.
template <typename Want, typename Set>
static int load_matching(const ud_safetensors* st, Want want, Set set, int32_t* n_loaded) {
    int32_t n = 0;
    std::vector<float> buf;
    for (const ud_safetensors::Entry& e : st->entries) {
        const std::string nn = nemo_name(e.name);
        if (!want(nn)) continue;
        buf.resize((size_t)e.count);
        int rc = ud_safetensors_read_f32(st, e.name.c_str(), buf.data(), e.count);
        if (rc != UD_OK) return rc;
        if ((rc = set(nn.c_str(), buf.data(), e.count)) != UD_OK) return rc;
        n++;
    }
    if (n_loaded) *n_loaded = n;
    return UD_OK;
}

extern "C" UD_API int ud_encoder_load_safetensors(ud_encoder* enc, const ud_safetensors* st, int32_t* n_loaded) {
    if (!enc || !st) return sfail(UD_ERR_INVALID, "ud_encoder_load_safetensors: null argument");
    ud_encoder_config cfg;
    int rc = ud_encoder_get_config(enc, &cfg);
    if (rc != UD_OK) return rc;
    const int layers = cfg.layers;
    return load_matching(
        st,
        [layers](const std::string& nn) {
            if (nn.compare(0, 19, "encoder.pre_encode.") == 0) return true;
            if (nn.compare(0, 15, "encoder.layers.") != 0) return false;
            const long li = strtol(nn.c_str() + 15, nullptr, 10);
            return li >= 0 && li < layers;          // layers beyond this encoder's depth are skipped
        },
        [enc](const char* nn, const float* v, int64_t c) { return ud_encoder_set_weight(enc, nn, v, c); }, n_loaded);
}

extern "C" UD_API int ud_rnnt_load_safetensors(ud_rnnt* r, const ud_safetensors* st, int32_t* n_loaded) {
    if (!r || !st) return sfail(UD_ERR_INVALID, "ud_rnnt_load_safetensors: null argument");
    return load_matching(
        st, [](const std::string& nn) { return nn.compare(0, 19, "decoder.prediction.") == 0 || nn.compare(0, 6, "joint.") == 0; },
        [r](const char* nn, const float* v, int64_t c) { return ud_rnnt_set_weight(r, nn, v, c); }, n_loaded);
}

extern "C" UD_API int ud_mel_load_safetensors(const ud_safetensors* st, ud_mel** out) {
    if (!st || !out) return sfail(UD_ERR_INVALID, "ud_mel_load_safetensors: null argument");
    *out = nullptr;
    int32_t dt, nd;
    int64_t shape[8];
    int rc = ud_safetensors_info(st, "preprocessor.featurizer.fb", &dt, shape, &nd);
    if (rc != UD_OK) return rc;
    int64_t count = 1;
    for (int i = 0; i < nd; i++) count *= shape[i];
    if (nd < 1 || shape[nd - 1] != 257 || count % 257 != 0 || count / 257 < 1 || count / 257 > 256)
        return sfail(UD_ERR_WEIGHT, "preprocessor.featurizer.fb: expected [.., n_mels, 257]");
    std::vector<float> fb((size_t)count), win(400);
    if ((rc = ud_safetensors_read_f32(st, "preprocessor.featurizer.fb", fb.data(), count)) != UD_OK) return rc;
    if ((rc = ud_safetensors_read_f32(st, "preprocessor.featurizer.window", win.data(), 400)) != UD_OK) return rc;
    return ud_mel_create(fb.data(), (int32_t)(count / 257), win.data(), out);
}

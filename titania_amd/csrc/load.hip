// Loading a model from a Hugging Face directory (model/model.rs:40-77): the
// architecture from config.json (model/config.rs:9-36) and bf16 tensors from
// model.safetensors (model/weights.rs:19-81), uploaded to the device.
//
// safetensors: an 8-byte little-endian header length, a JSON header mapping
// each tensor name to {dtype, shape, data_offsets} (plus "__metadata__"),
// then the tensor bytes, offsets relative to the end of the header.
#include <cstdint>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.h"

namespace {

using th::fail;

// ---- a small strict JSON reader (RFC 8259 values) ----

struct Json {
    enum Kind { kNull, kBool, kInt, kFloat, kString, kArray, kObject } kind = kNull;
    bool b = false;
    long long i = 0;  // kInt (integer literals that fit)
    double f = 0;     // kFloat, and kInt as a double
    std::string s;
    std::vector<Json> a;
    std::vector<std::pair<std::string, Json>> o;

    const Json *get(const char *key) const {
        for (const auto &kv : o)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonReader {
  public:
    JsonReader(const char *p, size_t n) : p_(p), end_(p + n) {}

    bool parse(Json &out, std::string &err) {
        if (!value(out, 0) || (ws(), p_ != end_)) {
            if (err_.empty()) err_ = "trailing characters";
            err = err_ + " at byte " + std::to_string(consumed());
            return false;
        }
        return true;
    }

  private:
    const char *p_, *end_, *start_ = p_;
    std::string err_;

    size_t consumed() const { return (size_t)(p_ - start_); }
    bool fail(const char *what) {
        if (err_.empty()) err_ = what;
        return false;
    }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char *w) {
        size_t n = strlen(w);
        if ((size_t)(end_ - p_) < n || memcmp(p_, w, n) != 0) return fail("invalid literal");
        p_ += n;
        return true;
    }
    static void utf8(std::string &s, unsigned cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(unsigned &v) {
        if (end_ - p_ < 4) return fail("short \\u escape");
        v = 0;
        for (int k = 0; k < 4; ++k) {
            char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool string(std::string &s) {
        ++p_;  // opening quote
        while (p_ < end_ && *p_ != '"') {
            unsigned char c = (unsigned char)*p_++;
            if (c < 0x20) return fail("control character in string");
            if (c != '\\') {
                s += (char)c;
                continue;
            }
            if (p_ == end_) return fail("unterminated escape");
            char e = *p_++;
            switch (e) {
            case '"': s += '"'; break;
            case '\\': s += '\\'; break;
            case '/': s += '/'; break;
            case 'b': s += '\b'; break;
            case 'f': s += '\f'; break;
            case 'n': s += '\n'; break;
            case 'r': s += '\r'; break;
            case 't': s += '\t'; break;
            case 'u': {
                unsigned cp;
                if (!hex4(cp)) return false;
                if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                    unsigned lo;
                    if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
                    p_ += 2;
                    if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                } else if (cp >= 0xDC00 && cp < 0xE000) {
                    return fail("lone surrogate");
                }
                utf8(s, cp);
                break;
            }
            default: return fail("bad escape");
            }
        }
        if (p_ == end_) return fail("unterminated string");
        ++p_;
        return true;
    }
    bool number(Json &v) {
        const char *b = p_;
        bool integral = true;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ == end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad number");
        if (*p_ == '0') ++p_;
        else
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ < end_ && *p_ == '.') {
            integral = false;
            ++p_;
            if (p_ == end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad fraction");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integral = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ == end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad exponent");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        std::string tok(b, p_);
        v.f = strtod(tok.c_str(), nullptr);
        v.kind = Json::kFloat;
        if (integral) {
            errno = 0;
            long long x = strtoll(tok.c_str(), nullptr, 10);
            if (errno == 0) {
                v.kind = Json::kInt;
                v.i = x;
            }
        }
        return true;
    }
    bool value(Json &v, int depth) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p_ == end_) return fail("unexpected end");
        switch (*p_) {
        case 'n': v.kind = Json::kNull; return lit("null");
        case 't': v.kind = Json::kBool; v.b = true; return lit("true");
        case 'f': v.kind = Json::kBool; v.b = false; return lit("false");
        case '"': v.kind = Json::kString; return string(v.s);
        case '[': {
            ++p_;
            v.kind = Json::kArray;
            ws();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            for (;;) {
                v.a.emplace_back();
                if (!value(v.a.back(), depth + 1)) return false;
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return fail("expected , or ]");
            }
        }
        case '{': {
            ++p_;
            v.kind = Json::kObject;
            ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            for (;;) {
                ws();
                if (p_ == end_ || *p_ != '"') return fail("expected a key");
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p_ == end_ || *p_ != ':') return fail("expected :");
                ++p_;
                v.o.emplace_back(std::move(key), Json());
                if (!value(v.o.back().second, depth + 1)) return false;
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return fail("expected , or }");
            }
        }
        default:
            if (*p_ == '-' || (*p_ >= '0' && *p_ <= '9')) return number(v);
            return fail("unexpected character");
        }
    }
};

int read_file(const std::string &path, std::string &out) {
    int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(TH_ERR_INVALID, "%s: %s", path.c_str(), strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return fail(TH_ERR_INVALID, "%s: %s", path.c_str(), strerror(errno));
    }
    out.resize((size_t)st.st_size);
    size_t got = 0;
    while (got < out.size()) {
        ssize_t r = pread(fd, &out[got], out.size() - got, (off_t)got);
        if (r <= 0) {
            close(fd);
            return fail(TH_ERR_INVALID, "%s: read failed", path.c_str());
        }
        got += (size_t)r;
    }
    close(fd);
    return TH_OK;
}

// serde_json's handling of the Config fields: usize from integer literals
// only; f32 from any number (parsed as f64, then rounded to f32).
int need_size(const Json &root, const char *key, int64_t &out, const char *path) {
    const Json *v = root.get(key);
    if (!v) return fail(TH_ERR_INVALID, "%s: missing field `%s`", path, key);
    if (v->kind != Json::kInt || v->i < 0) return fail(TH_ERR_INVALID, "%s: `%s` is not an unsigned integer", path, key);
    out = v->i;
    return TH_OK;
}

int need_f32(const Json &root, const char *key, float &out, const char *path) {
    const Json *v = root.get(key);
    if (!v) return fail(TH_ERR_INVALID, "%s: missing field `%s`", path, key);
    if (v->kind != Json::kInt && v->kind != Json::kFloat) return fail(TH_ERR_INVALID, "%s: `%s` is not a number", path, key);
    out = (float)(v->kind == Json::kInt ? (double)v->i : v->f);
    return TH_OK;
}

int parse_config(const std::string &path, th_config &c) {
    std::string text;
    TRY(read_file(path, text));
    Json root;
    std::string err;
    if (!JsonReader(text.data(), text.size()).parse(root, err))
        return fail(TH_ERR_INVALID, "%s: %s", path.c_str(), err.c_str());
    if (root.kind != Json::kObject) return fail(TH_ERR_INVALID, "%s: not a JSON object", path.c_str());
    const char *p = path.c_str();
    c = th_config{};
    TRY(need_size(root, "hidden_size", c.hidden_size, p));
    TRY(need_size(root, "intermediate_size", c.intermediate_size, p));
    TRY(need_size(root, "num_hidden_layers", c.num_hidden_layers, p));
    TRY(need_size(root, "num_attention_heads", c.num_attention_heads, p));
    TRY(need_size(root, "num_key_value_heads", c.num_key_value_heads, p));
    TRY(need_f32(root, "rms_norm_eps", c.rms_norm_eps, p));
    TRY(need_f32(root, "rope_theta", c.rope_theta, p));
    TRY(need_size(root, "vocab_size", c.vocab_size, p));
    // head_dim: Option<usize>, else hidden_size / num_attention_heads (config.rs:32-35).
    const Json *hd = root.get("head_dim");
    if (hd && hd->kind != Json::kNull) {
        TRY(need_size(root, "head_dim", c.head_dim, p));
    } else {
        TH_REQUIRE(c.num_attention_heads > 0, "%s: num_attention_heads must be positive", p);
        c.head_dim = c.hidden_size / c.num_attention_heads;
    }
    // tie_word_embeddings: bool, false when absent (config.rs:22-24).
    const Json *tie = root.get("tie_word_embeddings");
    if (tie) {
        if (tie->kind != Json::kBool) return fail(TH_ERR_INVALID, "%s: `tie_word_embeddings` is not a bool", p);
        c.tie_word_embeddings = tie->b ? 1 : 0;
    }
    return TH_OK;
}

struct Entry {
    std::string dtype;
    std::vector<size_t> shape;
    uint64_t begin = 0, end = 0;
};

// An open safetensors file (model/weights.rs:19-58).
struct SafeTensors {
    std::string path;
    int fd = -1;
    uint64_t data_start = 0, data_len = 0;
    std::map<std::string, Entry> entries;

    ~SafeTensors() {
        if (fd >= 0) close(fd);
    }

    int open_file(const std::string &p) {
        path = p;
        fd = open(p.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) return fail(TH_ERR_INVALID, "%s: %s", p.c_str(), strerror(errno));
        struct stat st;
        if (fstat(fd, &st) != 0) return fail(TH_ERR_INVALID, "%s: %s", p.c_str(), strerror(errno));
        const uint64_t size = (uint64_t)st.st_size;
        unsigned char len8[8];
        if (size < 8 || pread(fd, len8, 8, 0) != 8) return fail(TH_ERR_INVALID, "%s: no header length", p.c_str());
        uint64_t hlen = 0;
        for (int k = 7; k >= 0; --k) hlen = (hlen << 8) | len8[k];
        if (hlen > size - 8) return fail(TH_ERR_INVALID, "%s: header length %llu past the end of the file", p.c_str(),
                                         (unsigned long long)hlen);
        std::string header((size_t)hlen, '\0');
        if (hlen && pread(fd, &header[0], (size_t)hlen, 8) != (ssize_t)hlen)
            return fail(TH_ERR_INVALID, "%s: short header", p.c_str());
        data_start = 8 + hlen;
        data_len = size - data_start;
        Json root;
        std::string err;
        if (!JsonReader(header.data(), header.size()).parse(root, err))
            return fail(TH_ERR_INVALID, "%s: header: %s", p.c_str(), err.c_str());
        if (root.kind != Json::kObject) return fail(TH_ERR_INVALID, "%s: header is not a JSON object", p.c_str());
        for (const auto &kv : root.o) {
            if (kv.first == "__metadata__") continue;
            const Json &e = kv.second;
            const Json *dt = e.get("dtype"), *sh = e.get("shape"), *off = e.get("data_offsets");
            if (e.kind != Json::kObject || !dt || dt->kind != Json::kString || !sh || sh->kind != Json::kArray ||
                !off || off->kind != Json::kArray || off->a.size() != 2)
                return fail(TH_ERR_INVALID, "%s: malformed entry '%s'", p.c_str(), kv.first.c_str());
            Entry en;
            en.dtype = dt->s;
            for (const Json &d : sh->a) {
                if (d.kind != Json::kInt || d.i < 0)
                    return fail(TH_ERR_INVALID, "%s: bad shape of '%s'", p.c_str(), kv.first.c_str());
                en.shape.push_back((size_t)d.i);
            }
            if (off->a[0].kind != Json::kInt || off->a[1].kind != Json::kInt || off->a[0].i < 0 ||
                off->a[1].i < off->a[0].i || (uint64_t)off->a[1].i > data_len)
                return fail(TH_ERR_INVALID, "%s: data_offsets of '%s' out of range", p.c_str(), kv.first.c_str());
            en.begin = (uint64_t)off->a[0].i;
            en.end = (uint64_t)off->a[1].i;
            entries[kv.first] = std::move(en);
        }
        return TH_OK;
    }

    bool contains(const std::string &name) const { return entries.count(name) != 0; }

    // model/weights.rs:63-80: a BF16 tensor, uploaded.
    int upload(th_device *dev, const std::string &name, th_weight **out) {
        auto it = entries.find(name);
        if (it == entries.end()) return fail(TH_ERR_INVALID, "missing tensor '%s'", name.c_str());
        const Entry &e = it->second;
        if (e.dtype != "BF16")
            return fail(TH_ERR_INVALID, "tensor '%s' is %s, expected BF16", name.c_str(), e.dtype.c_str());
        // The element count and its byte size, refused when either overflows
        // (a crafted shape could otherwise wrap to the size of its data).
        size_t n = 1;
        for (size_t d : e.shape)
            if (__builtin_mul_overflow(n, d, &n) || n > SIZE_MAX / 2)
                return fail(TH_ERR_INVALID, "tensor '%s': the element count of its shape overflows", name.c_str());
        if (e.end - e.begin != 2 * (uint64_t)n)
            return fail(TH_ERR_INVALID, "tensor '%s': %llu bytes for %zu bf16 values", name.c_str(),
                        (unsigned long long)(e.end - e.begin), n);
        std::vector<uint16_t> data(n);
        size_t got = 0;
        const size_t bytes = 2 * n;
        char *dst = reinterpret_cast<char *>(data.data());
        while (got < bytes) {
            ssize_t r = pread(fd, dst + got, bytes - got, (off_t)(data_start + e.begin + got));
            if (r <= 0) return fail(TH_ERR_INVALID, "%s: reading '%s' failed", path.c_str(), name.c_str());
            got += (size_t)r;
        }
        return th_upload(dev, data.data(), e.shape.data(), e.shape.size(), out);
    }
};

}  // namespace

extern "C" {

int th_config_load(const char *path, th_config *out) {
    TH_REQUIRE(path && out, "th_config_load: null argument");
    return parse_config(path, *out);
}

int th_model_load(th_device *dev, const char *dir, th_model **out) {
    TH_REQUIRE(dev && dir && out, "th_model_load: null argument");
    TH_NOT_CAPTURING(dev, "th_model_load");
    const std::string d(dir);
    th_config c;
    TRY(parse_config(d + "/config.json", c));
    TH_REQUIRE(c.num_hidden_layers > 0 && c.num_hidden_layers < 4096, "config.json: %lld layers",
               (long long)c.num_hidden_layers);
    SafeTensors st;
    TRY(st.open_file(d + "/model.safetensors"));
    // Uploaded in the order model.rs:49-74 loads them; the model owns them.
    std::vector<th_weight *> w;
    auto release = [&]() {
        for (th_weight *x : w)
            if (x) th_weight_free(dev, x);
    };
    auto load = [&](const std::string &name, bool optional) -> int {
        th_weight *h = nullptr;
        if (optional && !st.contains(name)) {
            w.push_back(nullptr);
            return TH_OK;
        }
        int rc = st.upload(dev, name, &h);
        if (rc == TH_OK) w.push_back(h);
        return rc;
    };
    static const char *const kLayer[] = {"input_layernorm.weight",          "self_attn.q_proj.weight",
                                         "self_attn.k_proj.weight",         "self_attn.v_proj.weight",
                                         "self_attn.o_proj.weight",         "self_attn.q_norm.weight",
                                         "self_attn.k_norm.weight",         "post_attention_layernorm.weight",
                                         "mlp.gate_proj.weight",            "mlp.up_proj.weight",
                                         "mlp.down_proj.weight"};
    int rc = TH_OK;
    for (int64_t l = 0; l < c.num_hidden_layers && rc == TH_OK; ++l)
        for (int k = 0; k < 11 && rc == TH_OK; ++k)
            rc = load("model.layers." + std::to_string(l) + "." + kLayer[k], k == 5 || k == 6);
    if (rc == TH_OK) rc = load("model.embed_tokens.weight", false);
    if (rc == TH_OK) rc = load("model.norm.weight", false);
    if (rc == TH_OK) {
        if (c.tie_word_embeddings) w.push_back(nullptr);
        else rc = load("lm_head.weight", false);
    }
    if (rc != TH_OK) {
        std::string msg = th_last_error();
        release();
        return th::fail(rc, "%s", msg.c_str());
    }
    th_model *m = nullptr;
    rc = th_model_create(dev, &c, w.data(), w.size(), &m);
    if (rc != TH_OK) {
        std::string msg = th_last_error();
        release();
        return th::fail(rc, "%s", msg.c_str());
    }
    th_model_own_weights(m, w.data(), w.size());
    *out = m;
    return TH_OK;
}

}  // extern "C"

// safetensors.cpp -- the safetensors reader and writer behind KV snapshots (host code).
#include "es/safetensors.h"

#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace es {
namespace st {
namespace {

// The subset of JSON a safetensors header uses: objects, arrays, strings, integers (and,
// for robustness, other numbers, true / false / null).
struct Json {
    enum Kind { Null, Bool, Int, Num, Str, Arr, Obj } kind = Null;
    int64_t i = 0;
    std::string s;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json *get(const std::string &key) const {
        for (const auto &kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonReader {
public:
    JsonReader(const char *b, const char *e) : p_(b), e_(e) {}
    bool parse(Json &out) {
        if (!value(out, 0)) return false;
        ws();
        return p_ == e_;
    }

private:
    const char *p_, *e_;
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char *w) {
        const size_t n = std::strlen(w);
        if ((size_t) (e_ - p_) < n || std::strncmp(p_, w, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void utf8(std::string &o, unsigned c) {
        if (c < 0x80) {
            o += (char) c;
        } else if (c < 0x800) {
            o += (char) (0xC0 | (c >> 6));
            o += (char) (0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            o += (char) (0xE0 | (c >> 12));
            o += (char) (0x80 | ((c >> 6) & 0x3F));
            o += (char) (0x80 | (c & 0x3F));
        } else {
            o += (char) (0xF0 | (c >> 18));
            o += (char) (0x80 | ((c >> 12) & 0x3F));
            o += (char) (0x80 | ((c >> 6) & 0x3F));
            o += (char) (0x80 | (c & 0x3F));
        }
    }
    bool hex4(unsigned &c) {
        if (e_ - p_ < 4) return false;
        c = 0;
        for (int k = 0; k < 4; ++k) {
            const char h = *p_++;
            c <<= 4;
            if (h >= '0' && h <= '9') c |= (unsigned) (h - '0');
            else if (h >= 'a' && h <= 'f') c |= (unsigned) (h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') c |= (unsigned) (h - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool str(std::string &o) {
        if (p_ >= e_ || *p_ != '"') return false;
        ++p_;
        while (p_ < e_ && *p_ != '"') {
            const char c = *p_++;
            if ((unsigned char) c < 0x20) return false;
            if (c != '\\') {
                o += c;
                continue;
            }
            if (p_ >= e_) return false;
            const char x = *p_++;
            switch (x) {
                case '"': o += '"'; break;
                case '\\': o += '\\'; break;
                case '/': o += '/'; break;
                case 'b': o += '\b'; break;
                case 'f': o += '\f'; break;
                case 'n': o += '\n'; break;
                case 'r': o += '\r'; break;
                case 't': o += '\t'; break;
                case 'u': {
                    unsigned c1;
                    if (!hex4(c1)) return false;
                    if (c1 >= 0xD800 && c1 < 0xDC00) {  // surrogate pair
                        unsigned c2;
                        if (!lit("\\u") || !hex4(c2) || c2 < 0xDC00 || c2 >= 0xE000) return false;
                        c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
                    }
                    utf8(o, c1);
                    break;
                }
                default: return false;
            }
        }
        if (p_ >= e_) return false;
        ++p_;
        return true;
    }
    bool value(Json &v, int depth) {
        if (depth > 16) return false;
        ws();
        if (p_ >= e_) return false;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = Json::Obj;
            ws();
            if (p_ < e_ && *p_ == '}') { ++p_; return true; }
            for (;;) {
                ws();
                std::string k;
                if (!str(k)) return false;
                ws();
                if (p_ >= e_ || *p_ != ':') return false;
                ++p_;
                Json x;
                if (!value(x, depth + 1)) return false;
                v.obj.emplace_back(std::move(k), std::move(x));
                ws();
                if (p_ < e_ && *p_ == ',') { ++p_; continue; }
                if (p_ < e_ && *p_ == '}') { ++p_; return true; }
                return false;
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = Json::Arr;
            ws();
            if (p_ < e_ && *p_ == ']') { ++p_; return true; }
            for (;;) {
                Json x;
                if (!value(x, depth + 1)) return false;
                v.arr.push_back(std::move(x));
                ws();
                if (p_ < e_ && *p_ == ',') { ++p_; continue; }
                if (p_ < e_ && *p_ == ']') { ++p_; return true; }
                return false;
            }
        }
        if (c == '"') {
            v.kind = Json::Str;
            return str(v.s);
        }
        if (lit("true")) { v.kind = Json::Bool; v.i = 1; return true; }
        if (lit("false")) { v.kind = Json::Bool; v.i = 0; return true; }
        if (lit("null")) { v.kind = Json::Null; return true; }
        // number: integers exactly, anything else only recognised
        const char *b = p_;
        if (p_ < e_ && *p_ == '-') ++p_;
        bool integral = true, digits = false;
        while (p_ < e_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                           *p_ == '+' || *p_ == '-')) {
            if (*p_ >= '0' && *p_ <= '9') digits = true;
            else integral = false;
            ++p_;
        }
        if (!digits) return false;
        if (integral) {
            const std::string t(b, p_);
            errno = 0;
            char *end = nullptr;
            const long long x = std::strtoll(t.c_str(), &end, 10);
            if (errno || !end || *end) return false;
            v.kind = Json::Int;
            v.i = x;
        } else {
            v.kind = Json::Num;
        }
        return true;
    }
};

std::string jsonEscape(const std::string &s) {
    std::string o = "\"";
    for (unsigned char c : s) {
        if (c == '"') o += "\\\"";
        else if (c == '\\') o += "\\\\";
        else if (c < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\u%04x", c);
            o += buf;
        } else {
            o += (char) c;
        }
    }
    return o + "\"";
}

}  // namespace

size_t stDtypeSize(const std::string &d) {
    if (d == "BF16" || d == "F16" || d == "I16" || d == "U16") return 2;
    if (d == "F32" || d == "I32" || d == "U32") return 4;
    if (d == "F64" || d == "I64" || d == "U64") return 8;
    if (d == "U8" || d == "I8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
    return 0;
}

bool writeSafetensors(const std::string &path, const std::vector<std::pair<std::string, StTensor>> &ts,
                      const std::map<std::string, std::string> &meta) {
    std::string h = "{\"__metadata__\":{";
    bool first = true;
    for (const auto &kv : meta) {
        h += (first ? "" : ",") + jsonEscape(kv.first) + ":" + jsonEscape(kv.second);
        first = false;
    }
    h += "}";
    uint64_t off = 0;
    for (const auto &t : ts) {
        h += "," + jsonEscape(t.first) + ":{\"dtype\":" + jsonEscape(t.second.dtype) + ",\"shape\":[";
        for (size_t i = 0; i < t.second.shape.size(); ++i)
            h += (i ? "," : "") + std::to_string(t.second.shape[i]);
        h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + t.second.bytes.size()) + "]}";
        off += t.second.bytes.size();
    }
    h += "}";
    while (h.size() % 8) h += ' ';  // the data section starts 8-byte aligned
    const std::string tmp = path + ".tmp";
    std::FILE *f = std::fopen(tmp.c_str(), "wb");
    if (!f) return false;
    uint8_t len[8];
    const uint64_t n = h.size();
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t) (n >> (8 * i));
    bool ok = std::fwrite(len, 1, 8, f) == 8 && std::fwrite(h.data(), 1, h.size(), f) == h.size();
    for (const auto &t : ts)
        ok = ok && (t.second.bytes.empty() ||
                    std::fwrite(t.second.bytes.data(), 1, t.second.bytes.size(), f) == t.second.bytes.size());
    ok = (std::fclose(f) == 0) && ok;
    if (!ok || std::rename(tmp.c_str(), path.c_str()) != 0) {
        std::remove(tmp.c_str());
        return false;
    }
    return true;
}

bool readSafetensors(const std::string &path, std::map<std::string, StTensor> &out,
                     std::map<std::string, std::string> &meta) {
    std::FILE *f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    struct Closer {
        std::FILE *f;
        ~Closer() { std::fclose(f); }
    } closer{f};
    if (std::fseek(f, 0, SEEK_END) != 0) return false;
    const long long fileSize = std::ftell(f);
    if (fileSize < 8 || std::fseek(f, 0, SEEK_SET) != 0) return false;
    uint8_t len[8];
    if (std::fread(len, 1, 8, f) != 8) return false;
    uint64_t n = 0;
    for (int i = 0; i < 8; ++i) n |= (uint64_t) len[i] << (8 * i);
    if (n == 0 || n > (uint64_t) (fileSize - 8) || n > (100u << 20)) return false;
    std::string h(n, '\0');
    if (std::fread(&h[0], 1, n, f) != n) return false;
    Json root;
    if (!JsonReader(h.data(), h.data() + h.size()).parse(root) || root.kind != Json::Obj) return false;
    const uint64_t dataSize = (uint64_t) fileSize - 8 - n;
    for (const auto &kv : root.obj) {
        if (kv.first == "__metadata__") {
            if (kv.second.kind != Json::Obj) return false;
            for (const auto &m : kv.second.obj) {
                if (m.second.kind != Json::Str) return false;
                meta[m.first] = m.second.s;
            }
            continue;
        }
        const Json &t = kv.second;
        const Json *dt = t.get("dtype"), *sh = t.get("shape"), *of = t.get("data_offsets");
        if (t.kind != Json::Obj || !dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr || !of ||
            of->kind != Json::Arr || of->arr.size() != 2)
            return false;
        StTensor st;
        st.dtype = dt->s;
        const size_t es = stDtypeSize(st.dtype);
        if (!es) return false;
        uint64_t numel = 1;
        for (const Json &d : sh->arr) {
            if (d.kind != Json::Int || d.i < 0 || d.i > (1LL << 40)) return false;
            st.shape.push_back(d.i);
            // at most 2^42 elements, checked before the product could wrap
            if (d.i != 0 && numel > (1ULL << 42) / (uint64_t) d.i) return false;
            numel *= (uint64_t) d.i;
        }
        if (of->arr[0].kind != Json::Int || of->arr[1].kind != Json::Int) return false;
        const long long b = of->arr[0].i, e = of->arr[1].i;
        if (b < 0 || e < b || (uint64_t) e > dataSize || (uint64_t) (e - b) != numel * es) return false;
        st.bytes.resize((size_t) (e - b));
        if (e > b) {
            if (std::fseek(f, (long) (8 + n + (uint64_t) b), SEEK_SET) != 0) return false;
            if (std::fread(st.bytes.data(), 1, st.bytes.size(), f) != st.bytes.size()) return false;
        }
        if (!out.emplace(kv.first, std::move(st)).second) return false;  // duplicate name
    }
    return true;
}

}  // namespace st
}  // namespace es

// safetensors_check.cpp -- drives the KV-snapshot container reader
// (apertura_amd/csrc/es/safetensors.cpp) over valid, malformed and mutated files.  Built
// by tests/test_sanitizers.py with AddressSanitizer and UndefinedBehaviorSanitizer, so
// any out-of-bounds access, overflow or use of freed memory aborts the run.
//
// Checked: a written file reads back byte for byte; each hand-made malformed file
// (truncated length or header, header length past the end, non-JSON, wrong kinds, bad
// offsets, unknown dtype, negative or huge shapes, duplicate names, deep nesting, broken
// escapes) is refused; thousands of random mutations of a valid file either are refused
// or read back tensors whose byte counts match their shapes.
#include "es/safetensors.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

using namespace es::st;

static int g_fail = 0;
#define CHECK(c, ...)                                \
    do {                                             \
        if (!(c)) {                                  \
            std::printf("FAIL %s: ", #c);            \
            std::printf(__VA_ARGS__);                \
            std::printf("\n");                       \
            ++g_fail;                                \
        }                                            \
    } while (0)

static std::string g_dir;

static std::string put(const std::string &name, const std::string &bytes) {
    const std::string p = g_dir + "/" + name;
    std::FILE *f = std::fopen(p.c_str(), "wb");
    if (!f) { std::printf("cannot write %s\n", p.c_str()); std::exit(2); }
    std::fwrite(bytes.data(), 1, bytes.size(), f);
    std::fclose(f);
    return p;
}

static std::string slurp(const std::string &p) {
    std::string s;
    std::FILE *f = std::fopen(p.c_str(), "rb");
    if (!f) return s;
    char buf[4096];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) s.append(buf, n);
    std::fclose(f);
    return s;
}

// A file with header `json` (length field = its size unless `len` is given) and `data`.
static std::string file_of(const std::string &json, const std::string &data, long long len = -1) {
    const unsigned long long n = len < 0 ? json.size() : (unsigned long long) len;
    std::string s(8, '\0');
    for (int i = 0; i < 8; ++i) s[i] = (char) ((n >> (8 * i)) & 255);
    return s + json + data;
}

static bool reads(const std::string &path) {
    std::map<std::string, StTensor> t;
    std::map<std::string, std::string> m;
    const bool ok = readSafetensors(path, t, m);
    if (ok)
        for (const auto &kv : t) {
            size_t numel = 1;
            for (int64_t d : kv.second.shape) numel *= (size_t) d;
            CHECK(kv.second.bytes.size() == numel * stDtypeSize(kv.second.dtype), "%s: %zu bytes for its shape",
                  kv.first.c_str(), kv.second.bytes.size());
        }
    return ok;
}

int main(int argc, char **argv) {
    if (argc < 2) { std::printf("usage: safetensors_check DIR [mutations]\n"); return 2; }
    g_dir = argv[1];
    const int mutations = argc > 2 ? std::atoi(argv[2]) : 3000;

    // 1. round trip
    std::vector<std::pair<std::string, StTensor>> ts;
    StTensor a{"BF16", {2, 3, 4}, {}}, b{"F32", {2, 5, 1}, {}}, c{"U8", {0, 7}, {}};
    for (int i = 0; i < 2 * 3 * 4 * 2; ++i) a.bytes.push_back((uint8_t) (i * 7));
    for (int i = 0; i < 2 * 5 * 4; ++i) b.bytes.push_back((uint8_t) (255 - i));
    ts.push_back({"k_0", a});
    ts.push_back({"rs_1", b});
    ts.push_back({"empty", c});
    std::map<std::string, std::string> meta{{"fingerprint", "fp \"quoted\" \\ \x01"}, {"pos", "24"}};
    const std::string good = g_dir + "/good.safetensors";
    CHECK(writeSafetensors(good, ts, meta), "write");
    {
        std::map<std::string, StTensor> t;
        std::map<std::string, std::string> m;
        CHECK(readSafetensors(good, t, m), "read back");
        CHECK(m == meta, "metadata differs");
        CHECK(t.size() == 3 && t["k_0"].bytes == a.bytes && t["rs_1"].bytes == b.bytes && t["empty"].bytes.empty() &&
                  t["rs_1"].shape == b.shape && t["k_0"].dtype == "BF16",
              "tensors differ");
    }
    const std::string valid = slurp(good);

    // 2. malformed files, each refused
    const std::string T = "{\"t\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[0,8]}}";
    const std::string D8(8, 'x');
    struct Case { const char *name; std::string bytes; };
    std::vector<Case> bad = {
        {"empty", ""},
        {"short_length", std::string(5, '\0')},
        {"zero_length", file_of("", D8)},
        {"length_past_end", file_of(T, D8, (long long) T.size() + 100)},
        {"length_huge", file_of(T, D8, 1LL << 62)},
        {"truncated_header", file_of(T, "", (long long) T.size()).substr(0, 8 + T.size() / 2)},
        {"not_json", file_of("hello", D8)},
        {"json_array", file_of("[1,2]", D8)},
        {"trailing_garbage", file_of(T + "x", D8)},
        {"metadata_not_object", file_of("{\"__metadata__\":3}", "")},
        {"metadata_value_not_string", file_of("{\"__metadata__\":{\"a\":1}}", "")},
        {"tensor_not_object", file_of("{\"t\":5}", D8)},
        {"missing_offsets", file_of("{\"t\":{\"dtype\":\"F32\",\"shape\":[2]}}", D8)},
        {"offsets_one", file_of("{\"t\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[0]}}", D8)},
        {"offsets_reversed", file_of("{\"t\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[8,0]}}", D8)},
        {"offsets_negative", file_of("{\"t\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[-8,0]}}", D8)},
        {"offsets_past_data", file_of("{\"t\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[4,12]}}", D8)},
        {"offsets_size_mismatch", file_of("{\"t\":{\"dtype\":\"F32\",\"shape\":[3],\"data_offsets\":[0,8]}}", D8)},
        {"offsets_not_int", file_of("{\"t\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[0,8.5]}}", D8)},
        {"unknown_dtype", file_of("{\"t\":{\"dtype\":\"Q4\",\"shape\":[2],\"data_offsets\":[0,8]}}", D8)},
        {"dtype_not_string", file_of("{\"t\":{\"dtype\":4,\"shape\":[2],\"data_offsets\":[0,8]}}", D8)},
        {"shape_negative", file_of("{\"t\":{\"dtype\":\"F32\",\"shape\":[-2],\"data_offsets\":[0,8]}}", D8)},
        {"shape_huge_product", file_of("{\"t\":{\"dtype\":\"F32\",\"shape\":[1099511627776,1099511627776],\"data_offsets\":[0,8]}}", D8)},
        {"shape_product_wraps_to_zero",
         file_of("{\"t\":{\"dtype\":\"U8\",\"shape\":[4294967296,4294967296],\"data_offsets\":[0,0]}}", "")},
        {"shape_not_array", file_of("{\"t\":{\"dtype\":\"F32\",\"shape\":2,\"data_offsets\":[0,8]}}", D8)},
        {"integer_overflow", file_of("{\"t\":{\"dtype\":\"F32\",\"shape\":[99999999999999999999999],\"data_offsets\":[0,8]}}", D8)},
        {"duplicate_name", file_of("{\"t\":{\"dtype\":\"U8\",\"shape\":[4],\"data_offsets\":[0,4]},"
                                   "\"t\":{\"dtype\":\"U8\",\"shape\":[4],\"data_offsets\":[4,8]}}", D8)},
        {"deep_nesting", file_of(std::string(40, '[') + std::string(40, ']'), "")},
        {"unterminated_string", file_of("{\"t", "")},
        {"bad_escape", file_of("{\"\\q\":1}", "")},
        {"short_unicode_escape", file_of("{\"\\u12", "")},
        {"lone_surrogate", file_of("{\"__metadata__\":{\"a\":\"\\ud800x\"}}", "")},
        {"control_char_in_string", file_of(std::string("{\"a\x01\":1}"), "")},
        {"number_without_digits", file_of("{\"t\":-}", "")},
    };
    for (auto &cs : bad) CHECK(!reads(put(std::string("bad_") + cs.name, cs.bytes)), "%s was accepted", cs.name);

    // 3. random mutations of the valid file: refused or consistent, never a memory error
    std::mt19937_64 rng(12345);
    int accepted = 0;
    for (int it = 0; it < mutations; ++it) {
        std::string s = valid;
        const int kind = (int) (rng() % 5);
        const int edits = 1 + (int) (rng() % 4);
        for (int e = 0; e < edits && !s.empty(); ++e) {
            const size_t at = rng() % s.size();
            if (kind == 0) s[at] = (char) (rng() & 255);                          // byte flip
            else if (kind == 1) s.resize(at);                                   // truncation
            else if (kind == 2) s.insert(at, 1, "{}[]\",:0-9e"[rng() % 11]);    // JSON punctuation
            else if (kind == 3 && s.size() >= 8) s[rng() % 8] = (char) (rng() & 255);  // header length
            else s.erase(at, 1 + rng() % 8);                                    // deletion
        }
        accepted += reads(put("mut.safetensors", s)) ? 1 : 0;
    }
    std::printf("%s: %zu malformed files refused, %d mutations (%d accepted), %d failures\n",
                g_fail ? "FAIL" : "OK", bad.size(), mutations, accepted, g_fail);
    return g_fail ? 1 : 0;
}

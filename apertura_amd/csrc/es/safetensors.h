// safetensors.h -- the safetensors container, host code only (no HIP): what
// ESSnapshot.cpp reads and writes for KV snapshots (Apertura ESKVCache.mm:215-456 writes
// and reads it through mx::save_safetensors / mx::load_safetensors).
//
// Layout: an 8-byte little-endian header length N, N bytes of JSON ({"__metadata__":
// {string: string}, "<name>": {"dtype", "shape", "data_offsets": [begin, end]}}), then the
// bytes the offsets index (row-major).  The reader trusts nothing in the file: it is built
// and run under AddressSanitizer and UndefinedBehaviorSanitizer over malformed and
// mutated files by tests/test_sanitizers.py.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <utility>
#include <vector>

namespace es {
namespace st {

struct StTensor {
    std::string dtype;             // "BF16", "F32", "U8", ...
    std::vector<int64_t> shape;
    std::vector<uint8_t> bytes;    // row-major payload
};

// Bytes per element of a safetensors dtype name; 0 for an unknown name.
size_t stDtypeSize(const std::string &d);

// Writes `path` (through path + ".tmp", renamed on success).  Tensor names must be unique.
bool writeSafetensors(const std::string &path, const std::vector<std::pair<std::string, StTensor>> &ts,
                      const std::map<std::string, std::string> &meta);

// Reads and validates a whole file: a header length inside the file (and at most 100 MiB),
// a header that is one JSON object, string metadata, every tensor's dtype known, its
// shape of non-negative integers, its offsets inside the data section spanning exactly
// numel * dtype size, names unique.  false on any defect (out and meta are then partial).
bool readSafetensors(const std::string &path, std::map<std::string, StTensor> &out,
                     std::map<std::string, std::string> &meta);

}  // namespace st
}  // namespace es

#pragma once
// es_fill.h -- zero-filling device memory of the ES layer with the library's fill kernel
// (esda_fill_i32) rather than hipMemsetAsync: a step a caller captures into a HIP graph then
// records kernel nodes only.
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "esda.h"

namespace es {

// Zero the first `bytes` of `p` rounded up to whole 4-byte words: `p` is the start of a
// Tensor::empty allocation, whose size is a whole number of words.
inline void zeroFill(void *p, size_t bytes, hipStream_t st) {
    const size_t words = (bytes + 3) / 4;
    constexpr size_t kChunk = size_t(1) << 30;  // words per fill launch (the count is int32)
    for (size_t w0 = 0; w0 < words; w0 += kChunk) {
        const size_t n = words - w0 < kChunk ? words - w0 : kChunk;
        const int rc = esda_fill_i32(static_cast<int32_t *>(p) + w0, 0, (int32_t) n, st);
        if (rc != ESDA_OK) throw std::runtime_error(std::string("ES zero fill: ") + esda_last_error());
    }
}

}  // namespace es

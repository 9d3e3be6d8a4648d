// stream_scratch.h -- a bounded per-thread map from (device, stream) to a scratch set, used by
// the free functions of the ES* layer that keep buffers between calls (esDecodeAttnGlobal and
// the prefill functions).  Calls on different streams never share a scratch set, so they may
// overlap.  At most kMaxStreamScratch sets live per thread: using one more stream releases the
// set used least recently.  Its buffers are freed by hipFree, which waits for the device's
// queued work first, so no kernel still in flight reads them; a graph captured earlier over an
// evicted set's buffers must not be replayed (capture on at most kMaxStreamScratch streams).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <list>
#include <stdexcept>
#include <string>
#include <utility>

namespace es {

constexpr std::size_t kMaxStreamScratch = 8;

template <class S>
S &streamScratch(hipStream_t st) {
    thread_local std::list<std::pair<std::pair<int, hipStream_t>, S>> sets;  // most recent first
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) throw std::runtime_error(std::string("hipGetDevice: ") + hipGetErrorString(e));
    const std::pair<int, hipStream_t> key{dev, st};
    for (auto it = sets.begin(); it != sets.end(); ++it) {
        if (it->first == key) {
            if (it != sets.begin()) sets.splice(sets.begin(), sets, it);
            return sets.front().second;
        }
    }
    if (sets.size() >= kMaxStreamScratch) sets.pop_back();
    sets.emplace_front(key, S{});
    return sets.front().second;
}

}  // namespace es

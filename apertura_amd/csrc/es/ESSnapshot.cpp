// ESSnapshot.cpp -- KV snapshot persistence, prefix markers and in-memory turn rewind for
// es::ESKVCache (Apertura ESKVCache.mm:121-456, ESKVCache.h:102-174).
//
// File format: safetensors, the layout the reference writes through mx::save_safetensors:
// an 8-byte little-endian header length N, N bytes of JSON ({"__metadata__": {string:
// string}, "<name>": {"dtype", "shape", "data_offsets": [begin, end]}}), then the bytes the
// offsets index (row-major).  Tensors: k_<i> / v_<i> ([kvHeads, live rows, headDim] bf16;
// raw-K layers k_<i> only); q8 raw layers rq_<i> (u8) + rs_<i> / rb_<i> (f32 [kvHeads, rows,
// 1]); marker windows m<j>_k_<i> / m<j>_v_<i>.  Metadata: fingerprint, pos, layers,
// marker_count, marker_<j>_pos, marker_<j>_fp; this library adds shared_<i> = "1" for a
// layer whose V is its K buffer (attention_k_eq_v decode), written as two equal tensors so
// that the reference's reader sees an ordinary k/v layer.
//
// Device work runs on the stream of the cache's last update / decode / prefill call
// (lastStream_): each member first waits for that stream, so the appends queued there have
// landed, and waits again for its own copies before it returns (snapshots and marks are rare).
// Nothing here synchronises the whole device.
#include "es/ESKVCache.h"

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "es/safetensors.h"
#include "esda.h"

namespace es {
namespace {

using st::StTensor;
using st::readSafetensors;
using st::stDtypeSize;
using st::writeSafetensors;

void hipOk(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

int chunkUp(int n) {
    return (n + ESKVCache::kGrowChunk - 1) / ESKVCache::kGrowChunk * ESKVCache::kGrowChunk;
}

// ------------------------------------------------------------------ device <-> host

// Rows [r0, r0 + n) of every head of a [kvHeads, cap, headDim] buffer -> host [kvHeads, n, headDim].
StTensor download(const Tensor &buf, int r0, int n, hipStream_t st) {
    StTensor t;
    t.dtype = buf.dtype == Dtype::bf16 ? "BF16" : buf.dtype == Dtype::f32 ? "F32" : "U8";
    t.shape = {buf.shape[0], n, buf.shape[2]};
    const size_t es = dtypeSize(buf.dtype);
    const size_t rowBytes = (size_t) buf.shape[2] * es;
    t.bytes.resize((size_t) buf.shape[0] * n * rowBytes);
    if (n > 0)
    {
        hipOk(hipMemcpy2DAsync(t.bytes.data(), (size_t) n * rowBytes,
                               static_cast<const char *>(buf.data) + (size_t) r0 * buf.strides[1] * es,
                               (size_t) buf.strides[0] * es, (size_t) n * rowBytes, (size_t) buf.shape[0],
                               hipMemcpyDeviceToHost, st),
              "ESKVCache snapshot download");
        hipOk(hipStreamSynchronize(st), "ESKVCache snapshot download");
    }
    return t;
}

// A fresh zeroed [kvHeads, cap, w] buffer of `dt` holding `rows` rows of host data
// [kvHeads, rowsStored, w] (rows <= rowsStored; the rest of the buffer is zero).
// The copy has finished when it returns (the host bytes may be released).
Tensor upload(const std::vector<uint8_t> &src, int64_t kvH, int64_t rowsStored, int64_t hd, int rows, int cap,
              hipStream_t st, Dtype dt = Dtype::bf16) {
    Tensor t = Tensor::empty({kvH, cap, hd}, dt);
    hipOk(hipMemsetAsync(t.data, 0, t.nbytes(), st), "ESKVCache snapshot clear");
    const size_t rowBytes = (size_t) hd * dtypeSize(dt);
    if (rows > 0)
        hipOk(hipMemcpy2DAsync(t.data, (size_t) cap * rowBytes, src.data(), (size_t) rowsStored * rowBytes,
                               (size_t) rows * rowBytes, (size_t) kvH, hipMemcpyHostToDevice, st),
              "ESKVCache snapshot upload");
    hipOk(hipStreamSynchronize(st), "ESKVCache snapshot upload");
    return t;
}

// A device copy of rows [r0, r0 + n) of every head (the marker / rewind window copies).
// Queued on st; the caller waits for st before the copy is used or its source changes.
Tensor copyWindow(const Tensor &buf, int r0, int n, hipStream_t st) {
    Tensor t = Tensor::empty({buf.shape[0], n, buf.shape[2]}, Dtype::bf16);
    const size_t rowBytes = (size_t) buf.shape[2] * 2;
    if (n > 0)
        hipOk(hipMemcpy2DAsync(t.data, (size_t) n * rowBytes,
                               static_cast<const char *>(buf.data) + (size_t) r0 * buf.strides[1] * 2,
                               (size_t) buf.strides[0] * 2, (size_t) n * rowBytes, (size_t) buf.shape[0],
                               hipMemcpyDeviceToDevice, st),
              "ESKVCache window copy");
    return t;
}

// A fresh chunk-aligned buffer with `src`'s rows at the front (the compaction layout).
// Queued on st, as copyWindow.
Tensor rehomeDevice(const Tensor &src, int cap, hipStream_t st) {
    const int64_t kvH = src.shape[0], n = src.shape[1], hd = src.shape[2];
    Tensor t = Tensor::empty({kvH, cap, hd}, Dtype::bf16);
    hipOk(hipMemsetAsync(t.data, 0, t.nbytes(), st), "ESKVCache rewind clear");
    if (n > 0)
        hipOk(hipMemcpy2DAsync(t.data, (size_t) cap * hd * 2, src.data, (size_t) src.strides[0] * 2,
                               (size_t) n * hd * 2, (size_t) kvH, hipMemcpyDeviceToDevice, st),
              "ESKVCache rewind install");
    return t;
}

uint16_t bf16Rne(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t) ((u >> 16) | 0x40);  // NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t) (u >> 16);
}

bool isKvTensor(const StTensor &t) {
    return t.dtype == "BF16" && t.shape.size() == 3 && t.shape[0] > 0 && t.shape[2] > 0 && t.shape[2] % 8 == 0 &&
           t.shape[1] < (1LL << 30);
}

int parseInt(const std::map<std::string, std::string> &meta, const std::string &key, bool &ok) {
    auto it = meta.find(key);
    if (it == meta.end()) {
        ok = false;
        return 0;
    }
    try {
        size_t used = 0;
        const long long v = std::stoll(it->second, &used);
        if (used != it->second.size() || v < INT32_MIN || v > INT32_MAX) ok = false;
        return (int) v;
    } catch (const std::exception &) {
        ok = false;
        return 0;
    }
}

}  // namespace

// ------------------------------------------------------------------ markers and rewind

ESKVCache::Marker ESKVCache::takeMarker(int pos, bool copyLost, hipStream_t st) const {
    hipOk(hipStreamSynchronize(st), "ESKVCache mark");
    Marker m;
    m.pos = pos;
    for (size_t i = 0; i < slots_.size(); ++i) {
        const Slot &s = slots_[i];
        if (!s.k || !s.v) continue;  // raw layers never evict: prefix-sliceable
        const int live = s.len - s.start;
        if (live >= pos && !(copyLost && s.lost)) continue;  // the full prefix is still there
        // Deep copy now: later appends overwrite these rows in place.
        Tensor k = copyWindow(*s.k, s.start, live, st);
        Tensor v = s.shared ? k : copyWindow(*s.v, s.start, live, st);
        m.slidingKV.push_back({(int) i, {k, v}});
    }
    hipOk(hipStreamSynchronize(st), "ESKVCache mark");  // later appends overwrite the source rows
    return m;
}

void ESKVCache::markPrefix(int pos, const std::string &fingerprint) {
    // Below the sliding window plus a prefill chunk an evicting layer cannot be told from
    // a never-evicting one (ESKVCache.mm:121-146).
    if (pos < 4096)
        throw std::invalid_argument("ESKVCache::markPrefix: marker positions below 4096 unsupported");
    Marker m = takeMarker(pos, /*copyLost=*/false, lastStream_);
    m.fp = fingerprint;
    markers_.push_back(std::move(m));
}

bool ESKVCache::markRewindPoint(int pos) {
    // ESKVCache.mm:148-179: layers whose buffer still holds the whole prefix are rewound by
    // truncation later (guarded by `lost`); evicting or already-compacted layers are copied.
    if (pos <= 0) return false;
    for (const auto &a : k_)
        if (a) return false;  // legacy storage: no rewind
    bool prealloc = false;
    for (const Slot &s : slots_) prealloc = prealloc || s.k.has_value();
    for (const RQ8Slot &s : rq8slots_) prealloc = prealloc || s.q.has_value();
    if (!prealloc) return false;
    rewindMark_ = takeMarker(pos, /*copyLost=*/true, lastStream_);
    return true;
}

int ESKVCache::rewindToMark() {
    // ESKVCache.mm:181-222: validate every layer before mutating any.
    if (!rewindMark_) return -1;
    const int P = rewindMark_->pos;
    std::vector<const std::pair<Tensor, Tensor> *> copyFor(slots_.size(), nullptr);
    for (const auto &lkv : rewindMark_->slidingKV) copyFor[lkv.first] = &lkv.second;
    for (size_t i = 0; i < slots_.size(); ++i) {
        const Slot &s = slots_[i];
        if ((s.k && !copyFor[i] && (s.lost || s.len < P)) || (rq8slots_[i].q && rq8slots_[i].len < P)) {
            rewindMark_.reset();
            return -1;
        }
    }
    // Build the new slots first (allocation may throw), then commit.
    std::vector<Slot> next = slots_;
    for (size_t i = 0; i < slots_.size(); ++i) {
        Slot &s = next[i];
        if (copyFor[i]) {
            // the mark's window, content at the front (eviction re-applies on the next append)
            const Tensor &k = copyFor[i]->first;
            const int content = (int) k.shape[1];
            const int cap = chunkUp(content + kGrowChunk);
            s.k = rehomeDevice(k, cap, lastStream_);
            s.v = s.shared ? *s.k : rehomeDevice(copyFor[i]->second, cap, lastStream_);
            s.len = content;
            s.start = 0;
            s.lost = content < P;
        } else if (s.k) {
            s.len = P;  // full-prefix buffer: cursor truncation
            s.start = 0;
        }
    }
    hipOk(hipStreamSynchronize(lastStream_), "ESKVCache rewind");
    slots_ = std::move(next);
    for (RQ8Slot &s : rq8slots_)
        if (s.q) s.len = P;  // q8 rows never evict: cursor truncation
    rewindMark_.reset();
    return P;
}

// ------------------------------------------------------------------ save / restore

bool ESKVCache::saveSnapshot(const std::string &path, const std::string &fingerprint, int pos) const {
    try {
        hipOk(hipStreamSynchronize(lastStream_), "ESKVCache snapshot");
        std::vector<std::pair<std::string, StTensor>> ts;
        std::map<std::string, std::string> meta;
        for (size_t i = 0; i < slots_.size(); ++i) {
            const Slot &s = slots_[i];
            const std::string id = std::to_string(i);
            if (const RQ8Slot &r = rq8slots_[i]; r.q) {
                // q8 raw layer: packed rows and the per-row scale / bias, live [0, len)
                ts.emplace_back("rq_" + id, download(*r.q, 0, r.len, lastStream_));
                ts.emplace_back("rs_" + id, download(*r.sc, 0, r.len, lastStream_));
                ts.emplace_back("rb_" + id, download(*r.bs, 0, r.len, lastStream_));
                continue;
            }
            if (!s.k) return false;  // a snapshot needs every layer primed
            StTensor k = download(*s.k, s.start, s.len - s.start, lastStream_);
            if (s.v) {
                StTensor v = s.shared ? k : download(*s.v, s.start, s.len - s.start, lastStream_);
                if (s.shared) meta["shared_" + id] = "1";
                ts.emplace_back("k_" + id, std::move(k));
                ts.emplace_back("v_" + id, std::move(v));
            } else {
                ts.emplace_back("k_" + id, std::move(k));  // raw-K: one pre-norm stream
            }
        }
        meta["fingerprint"] = fingerprint;
        meta["pos"] = std::to_string(pos);
        meta["layers"] = std::to_string(slots_.size());
        meta["marker_count"] = std::to_string(markers_.size());
        for (size_t mi = 0; mi < markers_.size(); ++mi) {
            const Marker &m = markers_[mi];
            const std::string tag = "marker_" + std::to_string(mi);
            meta[tag + "_pos"] = std::to_string(m.pos);
            meta[tag + "_fp"] = m.fp;
            for (const auto &lkv : m.slidingKV) {
                const std::string sfx = "_" + std::to_string(lkv.first);
                const Tensor &k = lkv.second.first;
                ts.emplace_back("m" + std::to_string(mi) + "_k" + sfx, download(k, 0, (int) k.shape[1], lastStream_));
                ts.emplace_back("m" + std::to_string(mi) + "_v" + sfx,
                                download(lkv.second.second, 0, (int) k.shape[1], lastStream_));
            }
        }
        return writeSafetensors(path, ts, meta);
    } catch (const std::exception &) {
        return false;
    }
}

int ESKVCache::restoreSnapshot(const std::string &path, const std::string &fingerprint, RawMode mode,
                               const std::function<std::string(int)> &prefixFp) {
    try {
        std::map<std::string, StTensor> T;
        std::map<std::string, std::string> meta;
        if (!readSafetensors(path, T, meta)) return -1;
        bool ok = true;
        const int fullPos = parseInt(meta, "pos", ok);
        const int layers = parseInt(meta, "layers", ok);
        if (!ok || !meta.count("fingerprint") || layers != (int) slots_.size() || fullPos < 0) return -1;
        auto has = [&](const std::string &n) { return T.count(n) != 0; };

        // A full-fingerprint match restores everything; otherwise the longest marker whose
        // fingerprint the caller reproduces (ESKVCache.mm:287-310).
        int targetPos = fullPos, markerIdx = -1;
        if (meta.at("fingerprint") != fingerprint) {
            bool okc = true;
            const int nMark = meta.count("marker_count") ? parseInt(meta, "marker_count", okc) : 0;
            if (!okc || !prefixFp || nMark <= 0) return -1;
            int bestPos = -1;
            for (int mi = 0; mi < nMark; ++mi) {
                const std::string tag = "marker_" + std::to_string(mi);
                if (!meta.count(tag + "_pos") || !meta.count(tag + "_fp")) continue;
                bool okp = true;
                const int mpos = parseInt(meta, tag + "_pos", okp);
                if (!okp || mpos <= bestPos) continue;
                const std::string cand = prefixFp(mpos);
                if (!cand.empty() && cand == meta.at(tag + "_fp")) {
                    bestPos = mpos;
                    markerIdx = mi;
                }
            }
            if (markerIdx < 0) return -1;
            targetPos = bestPos;
        }

        // Classify and validate every layer before touching the cache.
        enum Kind { Composite, RawK, RawQ8 };
        std::vector<Kind> kind(slots_.size());
        bool anyRaw = false;
        for (size_t i = 0; i < slots_.size(); ++i) {
            const std::string id = std::to_string(i);
            const std::string mk = "m" + std::to_string(markerIdx) + "_k_" + id;
            const std::string mv = "m" + std::to_string(markerIdx) + "_v_" + id;
            if (markerIdx >= 0 && has(mk)) {
                if (!has(mv) || !isKvTensor(T.at(mk)) || T.at(mv).shape != T.at(mk).shape ||
                    T.at(mv).dtype != "BF16")
                    return -1;
            }
            if (has("k_" + id) && has("v_" + id)) {
                const StTensor &k = T.at("k_" + id), &v = T.at("v_" + id);
                if (!isKvTensor(k) || v.dtype != "BF16" || v.shape != k.shape) return -1;
                kind[i] = Composite;
            } else if (has("k_" + id)) {
                if (!isKvTensor(T.at("k_" + id))) return -1;
                kind[i] = RawK;
                anyRaw = true;
            } else if (has("rq_" + id)) {
                if (!has("rs_" + id) || !has("rb_" + id)) return -1;
                const StTensor &q = T.at("rq_" + id), &sc = T.at("rs_" + id), &bs = T.at("rb_" + id);
                if (q.dtype != "U8" || q.shape.size() != 3 || q.shape[0] <= 0 || q.shape[2] <= 0 ||
                    q.shape[2] % 8 != 0 || sc.dtype != "F32" || bs.dtype != "F32" ||
                    sc.shape != std::vector<int64_t>{q.shape[0], q.shape[1], 1} || bs.shape != sc.shape)
                    return -1;
                kind[i] = RawQ8;
                anyRaw = true;
            } else {
                return -1;  // unprimed layer, or quantized-KV tensors (no quantized storage here)
            }
        }
        // Storage-mode gate (ESKVCache.mm:333-343): composite <-> raw is not derivable; the
        // two raw forms convert (q8 -> bf16 dequantizes, bf16 -> q8 quantizes).
        if (mode != RawMode::asStored) {
            if (anyRaw && mode == RawMode::composite) return -1;
            if (!anyRaw && mode != RawMode::composite) return -1;
        }
        // Layers that end as q8 rows: stored q8 kept (asStored / rawQ8) and bf16 raw
        // quantized (rawQ8).  The q8 format is defined for 512-wide rows only.
        std::vector<bool> toQ8(slots_.size(), false);
        for (size_t i = 0; i < slots_.size(); ++i) {
            const std::string id = std::to_string(i);
            if (kind[i] == RawQ8 && mode != RawMode::raw) toQ8[i] = true;
            if (kind[i] == RawK && mode == RawMode::rawQ8) toQ8[i] = true;
            if (toQ8[i] && T.at(kind[i] == RawQ8 ? "rq_" + id : "k_" + id).shape[2] != 512) return -1;
        }

        // Build every layer's new slot (allocations may throw: nothing is committed yet).
        std::vector<Slot> next(slots_.size());
        std::vector<RQ8Slot> nextQ8(slots_.size());
        for (size_t i = 0; i < slots_.size(); ++i) {
            const std::string id = std::to_string(i);
            Slot &s = next[i];
            const std::string mk = "m" + std::to_string(markerIdx) + "_k_" + id;
            if (markerIdx >= 0 && T.count(mk)) {
                // an evicting layer takes the marker's window verbatim
                const StTensor &k = T.at(mk), &v = T.at("m" + std::to_string(markerIdx) + "_v_" + id);
                const int content = (int) k.shape[1];
                const int cap = chunkUp(content + kGrowChunk);
                s.k = upload(k.bytes, k.shape[0], content, k.shape[2], content, cap, lastStream_);
                const bool shared = meta.count("shared_" + id) && meta.at("shared_" + id) == "1" &&
                                    v.bytes == k.bytes;
                s.v = shared ? *s.k : upload(v.bytes, v.shape[0], content, v.shape[2], content, cap, lastStream_);
                s.shared = shared;
                s.len = content;
                s.lost = content < targetPos;
                continue;
            }
            if (kind[i] == RawQ8 && toQ8[i]) {
                // q8 rows kept as stored (ESKVCache.mm:384-392), cut at the target position
                const StTensor &q = T.at("rq_" + id), &sc = T.at("rs_" + id), &bs = T.at("rb_" + id);
                const int64_t kvH = q.shape[0], rows = q.shape[1];
                const int content = (int) std::min<int64_t>(rows, targetPos);
                const int cap = chunkUp(content + kGrowChunk);
                RQ8Slot &r = nextQ8[i];
                r.q = upload(q.bytes, kvH, rows, 512, content, cap, lastStream_, Dtype::u8);
                r.sc = upload(sc.bytes, kvH, rows, 1, content, cap, lastStream_, Dtype::f32);
                r.bs = upload(bs.bytes, kvH, rows, 1, content, cap, lastStream_, Dtype::f32);
                r.len = content;
                continue;
            }
            if (kind[i] == RawK && toQ8[i]) {
                // bf16 raw rows quantized during restore (ESKVCache.mm:394-408)
                const StTensor &k = T.at("k_" + id);
                const int64_t kvH = k.shape[0], rows = k.shape[1];
                const int content = (int) std::min<int64_t>(rows, targetPos);
                const int cap = chunkUp(content + kGrowChunk);
                RQ8Slot &r = nextQ8[i];
                r.q = upload({}, kvH, 0, 512, 0, cap, lastStream_, Dtype::u8);
                r.sc = upload({}, kvH, 0, 1, 0, cap, lastStream_, Dtype::f32);
                r.bs = upload({}, kvH, 0, 1, 0, cap, lastStream_, Dtype::f32);
                r.len = content;
                if (content > 0) {
                    const Tensor rowsDev = upload(k.bytes, kvH, rows, 512, content, content, lastStream_);
                    const int rc = esda_quantize_raw_rows(rowsDev.data, (int32_t) kvH, content, r.q->data,
                                                          (int64_t) cap * 512, static_cast<float *>(r.sc->data),
                                                          static_cast<float *>(r.bs->data), cap, 0, lastStream_);
                    if (rc != 0) throw std::runtime_error("ESKVCache restore: row quantization failed");
                    hipOk(hipStreamSynchronize(lastStream_), "ESKVCache restore quantize");
                }
                continue;
            }
            if (kind[i] == RawQ8) {
                // Rehydration (ESKVCache.mm:366-383): bf16(float(q) * scale + bias), the values
                // the q8 decode path computes on.
                const StTensor &q = T.at("rq_" + id), &sc = T.at("rs_" + id), &bs = T.at("rb_" + id);
                const int64_t kvH = q.shape[0], rows = q.shape[1], hd = q.shape[2];
                const int content = (int) std::min<int64_t>(rows, targetPos);
                std::vector<uint8_t> dq((size_t) kvH * rows * hd * 2);
                for (int64_t h = 0; h < kvH; ++h)
                    for (int64_t r = 0; r < rows; ++r) {
                        float scale, bias;
                        std::memcpy(&scale, &sc.bytes[(size_t) (h * rows + r) * 4], 4);
                        std::memcpy(&bias, &bs.bytes[(size_t) (h * rows + r) * 4], 4);
                        for (int64_t d = 0; d < hd; ++d) {
                            const size_t e = (size_t) ((h * rows + r) * hd + d);
                            const float prod = (float) q.bytes[e] * scale;
                            const uint16_t b = bf16Rne(prod + bias);
                            std::memcpy(&dq[e * 2], &b, 2);
                        }
                    }
                s.k = upload(dq, kvH, rows, hd, content, chunkUp(content + kGrowChunk), lastStream_);
                s.len = content;
                s.lost = content < targetPos;
                continue;
            }
            const StTensor &k = T.at("k_" + id);
            const int content = (int) std::min<int64_t>(k.shape[1], targetPos);
            const int cap = chunkUp(content + kGrowChunk);
            s.k = upload(k.bytes, k.shape[0], k.shape[1], k.shape[2], content, cap, lastStream_);
            if (kind[i] == Composite) {
                const StTensor &v = T.at("v_" + id);
                const bool shared = meta.count("shared_" + id) && meta.at("shared_" + id) == "1" &&
                                    v.bytes == k.bytes;
                s.v = shared ? *s.k : upload(v.bytes, v.shape[0], v.shape[1], v.shape[2], content, cap, lastStream_);
                s.shared = shared;
            }
            s.len = content;
            s.lost = content < targetPos;  // a stored sliding window is not a full prefix
        }
        hipOk(hipStreamSynchronize(lastStream_), "ESKVCache restore");
        slots_ = std::move(next);
        rq8slots_ = std::move(nextQ8);
        return targetPos;
    } catch (const std::exception &) {
        return -1;
    }
}

}  // namespace es

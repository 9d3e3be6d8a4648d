// reference_callers.cpp -- every ES* call that the reference's callers make, with their
// argument order and types, compiled against include/es (tests/test_boundary_compile.py
// runs g++ -fsyntax-only on it; nothing here is linked or run).  mx::array is spelled as
// es::Tensor, the library's stand-in for it; every other name is the reference's.
// Each call cites the reference line whose call it stands for.
#include "es/ESDecodeAttn.h"
#include "es/ESKVCache.h"
#include "es/ESPrefillAttn.h"

#include <array>
#include <string>
#include <utility>
#include <vector>

namespace mx {
using array = es::Tensor;
}

namespace es {

// ESAttention::keyValue (ESAttention.mm:77-108) and the elastic shared-KV scratch the
// model builds per forward (ESGemma4TextModel.mm:104, ESDecoderLayer.h:42).
std::pair<mx::array, mx::array> keyValueCalls(ESKVCache *cache, ESSharedKV *sharedKV, int layerIdx,
                                              const mx::array &k, const mx::array &v, int maxKeep,
                                              bool prealloc, bool sliding) {
    ESSharedKV shared;                                          // ESGemma4TextModel.mm:104
    (void) shared;
    if (sharedKV && maxKeep < 0) return sharedKV->get(sliding);  // ESAttention.mm:81
    auto kv = cache->update(layerIdx, k, v, maxKeep, prealloc);  // ESAttention.mm:105
    sharedKV->store(sliding, kv.first, kv.second);             // ESAttention.mm:106
    return kv;
}

// ESAttention::forwardRawKV (ESAttention.mm:253-302): bf16 and q8 raw streams.
mx::array rawCalls(ESKVCache *cache, int layerIdx, const mx::array &q, const mx::array &kRaw,
                   const mx::array &kw, float eps, const std::vector<float> &invFreq, bool prealloc) {
    ESKVCache::RawQ8 r = cache->updateRawQ8(layerIdx, kRaw);                       // ESAttention.mm:272
    mx::array o8 = esDecodeAttnGlobalQ8(q, r.qbuf, r.scbuf, r.bsbuf, r.len, r.pitch,  // ESAttention.mm:274-276
                                        kw, eps, invFreq);
    mx::array qv = r.qview, sc = r.sc, bs = r.bs;
    (void) o8, (void) qv, (void) sc, (void) bs;
    std::array<mx::array, 3> qsb = ESKVCache::quantizeRawRows(kRaw);               // ESAttention.mm:285
    (void) qsb;
    ESKVCache::Raw raw = cache->updateRaw(layerIdx, kRaw, prealloc);               // ESAttention.mm:290-292
    ESKVCache::Raw none{kRaw, kRaw, 1, 1};                                         // ESAttention.mm:292
    (void) none;
    mx::array view = raw.view;
    (void) view;
    return esDecodeAttnGlobal(q, raw.buffer, raw.len, raw.pitch, kw, eps, invFreq);  // ESAttention.mm:298-300
}

// ESAttention::forwardQuantKV (ESAttention.mm:335-360).
void quantCalls(ESKVCache *cache, int layerIdx, const mx::array &k, const mx::array &v, int gs, int bits,
                bool prealloc) {
    ESKVCache::QKV qkv = cache->updateQuant(layerIdx, k, v, gs, bits, prealloc);  // ESAttention.mm:354
    ESKVCache::QKV lit{qkv.kq, qkv.ks, qkv.kb, qkv.vq, qkv.vs, qkv.vb};           // ESAttention.mm:356
    (void) lit;
}

// The q8 row quantizer (ESKVCache.mm:513 calls the free function).
std::array<mx::array, 3> quantizerCall(const mx::array &kNew) { return esQuantizeRawRows(kNew); }

// ESCompiledStep (ESGenerationLoop.mm:104-238): slot adoption, the recorded step body and
// the eager maintenance between steps.
void compiledStepCalls(ESKVCache *cache, int i, bool cachePrealloc, const mx::array &pos,
                       const mx::array &slidingIdx, mx::array bk, mx::array bv) {
    auto kv = cache->current(i, cachePrealloc);          // ESGenerationLoop.mm:106
    (void) kv;
    cache->setSlot(i, std::move(bk), std::move(bv));     // ESGenerationLoop.mm:122
    cache->beginStep(/*globalIdx=*/pos, /*slidingIdx=*/slidingIdx);  // ESGenerationLoop.mm:134
    std::vector<mx::array> outs;
    outs.push_back(cache->slotK(i));                     // ESGenerationLoop.mm:175
    outs.push_back(cache->slotV(i));                     // ESGenerationLoop.mm:176
    cache->endStep();                                    // ESGenerationLoop.mm:178
    const mx::array &k = cache->slotK(i);                // ESGenerationLoop.mm:194
    (void) k;
    std::vector<mx::array> ins;
    ins.push_back(cache->takeSlotK(i));                  // ESGenerationLoop.mm:233
    ins.push_back(cache->takeSlotV(i));                  // ESGenerationLoop.mm:234
    cache->setSlot(i, outs[0], outs[1]);                 // ESGenerationLoop.mm:238
}

// Session-level calls (APLocalSession.mm, AperturaResearch/main.mm) and the step counter.
void sessionCalls(ESKVCache &cache, const std::string &path, const std::string &fp, int P,
                  const std::function<std::string(int)> &pf) {
    ESKVCache c(60);                                                        // ESKVCache.h:46
    (void) c;
    int pos = cache.restoreSnapshot(path, fp);                              // APLocalSession.mm:331
    pos = cache.restoreSnapshot(path, fp, ESKVCache::RawMode::raw);         // main.mm:1022
    pos = cache.restoreSnapshot(path, fp, ESKVCache::RawMode::rawQ8, pf);   // main.mm:893
    bool ok = cache.saveSnapshot(path, fp, P);                              // main.mm:552
    cache.markPrefix(P, fp);                                                // main.mm:886
    ok = ok && cache.markRewindPoint(pos);                                  // APLocalSession.mm:469
    const int mark = cache.rewindToMark();                                  // APLocalSession.mm:630
    (void) mark;
    cache.clearRewindMark();                                                // APLocalSession.mm:639
    cache.reset();                                                          // APLocalSession.mm:233
    cache.markStep(1);                                                      // ESKVCache.h:177
    const int n = cache.seqLen();                                           // ESKVCache.h:176
    (void) n;
    constexpr int chunk = ESKVCache::kGrowChunk;                            // ESKVCache.h:50
    static_assert(chunk == 256, "growth chunk");
}

}  // namespace es

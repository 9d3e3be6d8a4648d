#pragma once
//  ESKVCache -- per-layer key/value storage on the GPU with the reference's interface
//  (Apertura ESKVCache.h:44-224).  Buffers are [kvHeads, capacity, headDim] bf16 per
//  layer; update() appends along the sequence axis and returns the cached K/V as views.
//  Two storage modes, selected per call as in the reference (ESKVCache.h:7-21):
//    - legacy (prealloc=false): concat-grow, slice eviction (the bit-exact reference);
//    - prealloc (prealloc=true): in-place appends into a buffer grown in kGrowChunk-row
//      steps, a logical `start` cursor for sliding-window eviction, and compaction of the
//      live range into a fresh buffer when the write cursor reaches capacity.
//  decode() is the fused decode step of this library: the prealloc append and the
//  attention of the new token in one GPU pass (esda_decode), replacing update()
//  followed by SDPA at ESAttention.mm:105 and :188; prefill() / prefillRaw() append a
//  chunk and attend it (ESAttention.mm:168-193, 253-332 at seq > 1).
//  q8 raw-K storage (rawKVQ8: per-row affine u8 rows with an f32 scale and bias,
//  ESKVCache.mm:506-566), KV snapshots (the reference's safetensors layout), prefix
//  markers and turn rewind follow the reference (ESKVCache.mm:121-456), and so does the
//  compiled-step mode (ESKVCache.h:93-112: scatter appends at a device position into
//  full-capacity slots).  Quantized-KV storage (quantized_matmul groups, updateQuant) is
//  declared with the reference's signature and throws std::runtime_error; quantized-KV
//  snapshots are refused (-1).
//
//  Every call takes a HIP stream (nullptr = the default stream).  Buffer growth and
//  compaction synchronise that stream before the old buffer is released.  An instance
//  is used from one thread at a time (the reference runs its engine on one thread).
#include "ESTensor.h"

#include <array>
#include <functional>
#include <optional>
#include <string>
#include <utility>
#include <vector>

namespace es {

// Per-forward shared-KV scratch of elastic models (ESKVCache.h:31-42): the last layer of
// each attention type that stores its full K/V leaves them here for the shared layers of
// that type.  Type index 0 = sliding (local), 1 = full (global).  get() of a type nothing
// stored throws std::bad_optional_access.
struct ESSharedKV {
    std::optional<Tensor> k_[2], v_[2];
    void store(bool sliding, const Tensor &k, const Tensor &v) {
        const int t = sliding ? 0 : 1;
        k_[t] = k;
        v_[t] = v;
    }
    std::pair<Tensor, Tensor> get(bool sliding) const {
        const int t = sliding ? 0 : 1;
        return {k_[t].value(), v_[t].value()};
    }
};

class ESKVCache {
public:
    explicit ESKVCache(int numLayers);
    ~ESKVCache() = default;
    ESKVCache(const ESKVCache &) = delete;
    ESKVCache &operator=(const ESKVCache &) = delete;

    static constexpr int kGrowChunk = 256;

    // Append kNew/vNew ([kvHeads, nNew, headDim] bf16, rows contiguous) for `layer`;
    // returns the cached {K, V} as views [kvHeads, live, headDim].  maxKeep > 0 keeps
    // only the last maxKeep keys (sliding-window eviction).  (ESKVCache.mm:19-110)
    // Throws std::runtime_error when the slot holds raw-K content (ESKVCache.mm:59-62).
    // In prealloc mode a slot first filled with vNew aliasing kNew keeps one shared K=V
    // buffer (attention_k_eq_v); later appends to it must alias too.
    // In compiled-step mode (beginStep .. endStep) the mode arguments are ignored: the
    // single new row is written at the row the step's position tensor holds (slidingIdx
    // when maxKeep > 0, else globalIdx) and the full-capacity slot buffers are returned.
    std::pair<Tensor, Tensor> update(int layer, const Tensor &kNew, const Tensor &vNew, int maxKeep = 0,
                                     bool prealloc = false, hipStream_t stream = nullptr);

    // Quantized KV (ESKVCache.h:60-70): {packed, scales, biases} for K and V.  Not built
    // by this library (a quantized_matmul storage path, not the decode-attention kernels):
    // always throws std::runtime_error.
    struct QKV {
        Tensor kq, ks, kb, vq, vs, vb;
    };
    QKV updateQuant(int layer, const Tensor &kNew, const Tensor &vNew, int groupSize, int bits,
                    bool prealloc = false);

    // Compiled-step mode (ESKVCache.h:93-112).  beginStep takes device int32 [1] tensors
    // holding the cache ROW of this token for global and for sliding layers; until
    // endStep, update() scatters there (esda_kv_append with a device row index, so a
    // captured graph replays for any position).  The step driver owns slot layout and
    // compaction through slotK / slotV / setSlot / takeSlotK / takeSlotV.  Slot accessors
    // throw std::runtime_error for an empty slot.
    void beginStep(const Tensor &globalIdx, const Tensor &slidingIdx);
    void endStep();
    const Tensor &slotK(int layer) const;
    const Tensor &slotV(int layer) const;
    void setSlot(int layer, Tensor k, Tensor v);
    Tensor takeSlotK(int layer);
    Tensor takeSlotV(int layer);

    // Raw-K storage: only the pre-norm k_proj rows, one stream (ESKVCache.mm:458-504).
    // {live view [kvHeads, len, headDim], whole buffer, len, pitch (= buffer rows)}.
    struct Raw {
        Tensor view, buffer;
        int len, pitch;
    };
    Raw updateRaw(int layer, const Tensor &kNew, bool prealloc, hipStream_t stream = nullptr);
    // The Raw record of a prealloc raw-K slot without appending (the reference hands it out
    // only from updateRaw).  Throws std::runtime_error for a non-raw slot.
    Raw currentRaw(int layer) const;

    // q8 raw-K storage (ESKVCache.h:81-91): kNew [kvHeads, nNew, 512] bf16 raw rows are
    // quantized per row (u8 q, f32 scale and bias: x = q * scale + bias) and appended; the
    // three buffers share one cursor.  A slot holding bf16 raw rows (a restored snapshot)
    // is migrated on the first call: its live rows are quantized once and the bf16
    // buffer retired.  Throws std::runtime_error for a composite slot.  Views: q
    // [kvHeads, len, 512] u8, sc / bs [kvHeads, len, 1] f32; buffers of `pitch` rows.
    struct RawQ8 {
        Tensor qview, sc, bs, qbuf, scbuf, bsbuf;
        int len, pitch;
    };
    RawQ8 updateRawQ8(int layer, const Tensor &kNew, hipStream_t stream = nullptr);
    // The row quantizer behind updateRawQ8: {q u8 [kvH, n, 512], scale f32 [kvH, n, 1],
    // bias f32 [kvH, n, 1]} (ESKVCache.mm:506-511, esQuantizeRawRows).
    static std::array<Tensor, 3> quantizeRawRows(const Tensor &kNew, hipStream_t stream = nullptr);
    // Fused q8 decode step: updateRawQ8(layer, kNew) and esDecodeAttnGlobalQ8 over the slot
    // in one GPU pass (the kernel quantizes the new row itself).  kNew: [kvHeads, 1, 512].
    Tensor decodeRawQ8(int layer, const Tensor &q, const Tensor &kNew, const Tensor &kw, float eps,
                       const std::vector<float> &invFreq, hipStream_t stream = nullptr, Tensor *out = nullptr);
    // The RawQ8 record of a q8 slot without appending (throws std::runtime_error otherwise).
    RawQ8 currentRawQ8(int layer) const;

    // Fused decode step for `layer` (prealloc storage): appends the single new row of
    // kNew/vNew ([kvHeads, 1, headDim]) and returns softmax(scale q K^T) V over the rows
    // the reference would attend after update(maxKeep) under its mask: [numQHeads,
    // headDim] bf16 in `out` (allocated when null).  window > 0 is the sliding layer's
    // mask (ESGemma4TextModel.mm:68-83: the last `window` positions), applied whatever
    // maxKeep evicts -- the reference passes maxKeep = 0 with a window when the sliding
    // cache is off or the layer stores its full K/V (ESAttention.mm:99-103).  q:
    // numQHeads*headDim bf16, query heads kv-major.  vNew aliasing kNew (same data
    // pointer) is attention_k_eq_v: a slot created that way keeps one shared K=V buffer,
    // written and read once.
    Tensor decode(int layer, const Tensor &q, const Tensor &kNew, const Tensor &vNew, int maxKeep, int window,
                  float scale, hipStream_t stream = nullptr, Tensor *out = nullptr);

    // Fused raw-K decode step: updateRaw(layer, kNew, true) and esDecodeAttnGlobal over
    // the slot in one GPU pass.  kNew: [kvHeads, 1, 512] raw k_proj rows.
    Tensor decodeRaw(int layer, const Tensor &q, const Tensor &kNew, const Tensor &kw, float eps,
                     const std::vector<float> &invFreq, hipStream_t stream = nullptr, Tensor *out = nullptr);

    // Prefill chunk (ESAttention::keyValue then SDPA at seq > 1, ESAttention.mm:77-108,
    // 168-193): append kNew / vNew (seq rows; maxKeep as update, e.g. window + seq for a
    // chunked sliding layer), then attend q [numQ, seq, hd] over the live rows with the
    // reference's mask (pastLen = positions cached before the chunk; window 0 on global
    // layers).  Returns O [seq, numQ * hd] bf16 (esPrefillAttention).
    Tensor prefill(int layer, const Tensor &q, const Tensor &kNew, const Tensor &vNew, int maxKeep, int window,
                   float scale, int pastLen, bool prealloc = true, hipStream_t stream = nullptr, Tensor *out = nullptr);
    // Raw-K (q8 = false: updateRaw, prealloc) or q8 raw-K (updateRawQ8) prefill chunk,
    // ESAttention.mm:253-332: append the chunk's raw rows, then esPrefillAttnRaw(Q8) over
    // the whole stream.
    Tensor prefillRaw(int layer, const Tensor &q, const Tensor &kNew, const Tensor &kw, float eps,
                      const std::vector<float> &invFreq, int pastLen, float scale, bool q8 = false,
                      hipStream_t stream = nullptr, Tensor *out = nullptr);

    // The cached {K, V} without appending (ESKVCache.mm:112-119).
    std::pair<Tensor, Tensor> current(int layer, bool prealloc) const;

    // Persistence and rewind (ESKVCache.h:102-174, ESKVCache.mm:121-456).
    // markPrefix: remember position `pos` (>= 4096, else std::invalid_argument) with the
    // prompt-prefix fingerprint; layers whose live window no longer starts at row 0 of the
    // prefix (they evicted) have that window copied now.
    void markPrefix(int pos, const std::string &fingerprint);
    // saveSnapshot: safetensors file of every layer's live rows (k_<i>/v_<i>; raw layers
    // k_<i> only; q8 raw layers rq_<i> u8 + rs_<i> / rb_<i> f32 scale and bias), metadata {fingerprint, pos, layers, marker_*} and the markers' windows
    // (m<j>_k_<i>/m<j>_v_<i>).  false if a layer is unprimed or the file cannot be written.
    bool saveSnapshot(const std::string &path, const std::string &fingerprint, int pos) const;
    enum class RawMode { composite, raw, rawQ8, asStored };
    // restoreSnapshot: -1 (cache untouched) on a missing or malformed file, a layer-count
    // or fingerprint mismatch with no usable marker, or a storage-mode mismatch; otherwise
    // re-homes every layer into fresh chunk-aligned buffers and returns the restored
    // position (the snapshot's, or the longest marker whose fingerprint prefixFp(pos)
    // reproduces).  Raw streams convert to the requested mode: RawMode::raw dequantizes
    // stored q8 rows to bf16 (bf16(float(q) * scale + bias)), RawMode::rawQ8 quantizes
    // stored bf16 raw rows; asStored keeps each layer's stored form.  Composite <-> raw is
    // a mismatch.  Every layer's storage is replaced.
    int restoreSnapshot(const std::string &path, const std::string &fingerprint,
                        RawMode mode = RawMode::asStored,
                        const std::function<std::string(int)> &prefixFp = nullptr);
    // One in-memory rewind mark: markRewindPoint(pos) (false for legacy storage, pos <= 0
    // or an unprimed cache), rewindToMark() -> pos, or -1 when a layer can no longer be
    // rebuilt at pos (the mark is consumed either way).
    bool markRewindPoint(int pos);
    int rewindToMark();
    void clearRewindMark() { rewindMark_.reset(); }

    int seqLen() const { return seqLen_; }
    void markStep(int nNew) { seqLen_ += nNew; }
    void reset();

    int numLayers() const { return (int) slots_.size(); }
    // Prealloc slot bookkeeping (read-only).
    int slotLen(int layer) const { return slotQ8(layer) ? rq8slots_[layer].len : slotAt(layer).len; }
    int slotStart(int layer) const { return slotAt(layer).start; }
    int slotCapacity(int layer) const;
    bool slotLost(int layer) const { return slotAt(layer).lost; }
    bool slotShared(int layer) const { return slotAt(layer).shared; }
    bool slotRaw(int layer) const { return slotAt(layer).k.has_value() && !slotAt(layer).v.has_value(); }
    bool slotQ8(int layer) const { slotAt(layer); return rq8slots_[layer].q.has_value(); }

private:
    struct Slot {
        std::optional<Tensor> k, v;  // v empty: raw-K content
        int len = 0, start = 0;
        bool lost = false;    // rows before `start` were discarded by a compaction
        bool shared = false;  // v is the same buffer as k (attention_k_eq_v decode)
    };
    std::vector<std::optional<Tensor>> k_, v_;  // legacy storage
    std::vector<Slot> slots_;                   // prealloc storage
    // A position, its prefix fingerprint, and copies of the evicting layers' live windows
    // taken at that moment (layer index, {k, v}; v is k for a shared slot).
    struct Marker {
        int pos = 0;
        std::string fp;
        std::vector<std::pair<int, std::pair<Tensor, Tensor>>> slidingKV;
    };
    std::vector<Marker> markers_;
    std::optional<Marker> rewindMark_;
    // q8 raw storage: u8 rows [kvH, cap, 512] and scale / bias [kvH, cap, 1], live [0, len).
    struct RQ8Slot {
        std::optional<Tensor> q, sc, bs;
        int len = 0;
    };
    std::vector<RQ8Slot> rq8slots_;
    void growQ8(RQ8Slot &s, int nNew, hipStream_t stream);
    void migrateToQ8(int layer, hipStream_t stream);
    Marker takeMarker(int pos, bool copyLost, hipStream_t stream) const;
    int seqLen_ = 0;
    // The stream of the last update / decode / prefill call.  The persistence and rewind
    // members (which take no stream in the reference's signatures) wait for it and run their
    // copies on it, so appends queued there have landed; a caller that writes the cache's
    // buffers from several streams orders them before that stream, as its own calls need.
    hipStream_t lastStream_ = nullptr;
    // Compiled-step mode state (beginStep): the row index tensors of this token.
    bool stepMode_ = false;
    std::optional<Tensor> stepGlobalIdx_, stepSlidingIdx_;
    std::optional<Tensor> posDev_;     // per-layer position words for decode()
    std::optional<Tensor> workspace_;  // esda_decode / esda_decode_raw workspace
    std::optional<Tensor> invFreqDev_; // rotary table of the last decodeRaw()
    std::vector<float> invFreqHost_;
    std::optional<Tensor> ropeTab_;    // cos/sin rows of invFreqDev_ (esda_rope_table)
    int ropeRows_ = 0;

    const Slot &slotAt(int layer) const;
    void checkLayer(int layer) const;
    void growSlot(Slot &s, int nNew, hipStream_t stream, bool compactStart);
    void *workspace(size_t bytes, hipStream_t stream);
    // esda_rope_table of invFreqDev_ covering at least `rows` cache rows (grown in 4096-row
    // steps; the stream is synchronised before an old table is released).
    const void *ropeTable(int rows, hipStream_t stream);
    int *positionWord(int layer, int value, hipStream_t stream);
};

}  // namespace es

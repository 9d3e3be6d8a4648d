#pragma once
//  ESPrefillAttn -- attention of a prefill chunk (seq > 1 new tokens) over the cache, with
//  the reference's mask, backed by esda_prefill (include/esda_prefill.h).
//
//  The reference's prefill branch (Apertura ESAttention.mm:168-193 at seq > 1, and the
//  raw-K prefill ESAttention.mm:253-332) appends the chunk's K/V through ESKVCache and
//  calls mx::fast::scaled_dot_product_attention(Q, K, V, scale, "", M), M the additive
//  mask of ESGemma4TextModel.mm:68-83 (buildMask: key kj visible to query qi iff
//  kj <= pastLen + qi and, on sliding layers, kj > pastLen + qi - window) aligned to the
//  retained keys by alignMask (ESAttention.mm:17-22: the last seqK columns).  Here the mask
//  is index math inside the kernel.
#include "ESTensor.h"

#include <vector>

namespace es {

// q:      [numQ, seq, hd] bf16 (kv-major heads, post q-norm + RoPE), any head / row
//         strides with dense head dims -- the reference's transposed q.
// K, V:   [numKV, seqK, hd] bf16 views of the cache after the chunk's update (rows dense,
//         one head stride for both); key j sits at absolute position pastLen + seq - seqK + j.
// pastLen: positions cached before the chunk; window: 0 (global) or the sliding window.
// Returns O [seq, numQ * hd] bf16 (the reference's layout before o_proj).
// Throws std::invalid_argument on shape contracts.
Tensor esPrefillAttention(const Tensor &q, const Tensor &K, const Tensor &V, int pastLen, int window, float scale,
                          hipStream_t stream = nullptr, Tensor *out = nullptr);

// Raw-K prefill (ESAttention.mm:306-332): rawView [numKV, seqK, 512] bf16 pre-norm k_proj
// rows of positions 0 .. seqK-1 (seqK == pastLen + seq); K = kNorm(raw) roped by ops, V =
// vNorm(raw), both rebuilt into library scratch, then attention as above (no window).
// invFreq: the rotary table (hd/2 entries; a shorter table is zero-extended).
Tensor esPrefillAttnRaw(const Tensor &q, const Tensor &rawView, const Tensor &kw, float eps,
                        const std::vector<float> &invFreq, int pastLen, float scale, hipStream_t stream = nullptr,
                        Tensor *out = nullptr);

// The same over a q8 raw view (ESAttention.mm:270-282): qView [numKV, seqK, 512] u8 with
// scView / bsView [numKV, seqK, 1] f32 (ESKVCache::RawQ8's qview / sc / bs); rows are
// dequantised to bf16(float(q) * scale + bias) first.
Tensor esPrefillAttnRawQ8(const Tensor &q, const Tensor &qView, const Tensor &scView, const Tensor &bsView,
                          const Tensor &kw, float eps, const std::vector<float> &invFreq, int pastLen, float scale,
                          hipStream_t stream = nullptr, Tensor *out = nullptr);

}  // namespace es

#pragma once
//  ESDecodeAttn -- raw-K decode attention for the GLOBAL layers (head_dim 512) with the
//  reference's signature (Apertura ESDecodeAttn.h:22-28), backed by esda_decode_raw.
//  The kernel streams each cached raw k_proj row once and rebuilds in registers:
//      rinv = rsqrt(mean(kraw^2) + eps)
//      K    = bf16(rope(kraw * rinv * kw))   (rotary pairs (d, d + 256) for d < 64,
//                                             cos / sin of the fp32 angle rounded to bf16)
//      V    = kraw * rinv                    (folded into the softmax weight)
//  then attends the query heads of each kv head, split-K, merged in fp32.
#include "ESTensor.h"

#include <array>
#include <vector>

namespace es {

// q:      [numQ, 512] bf16, query heads kv-major, post q-norm + RoPE.
// rawBuf: the UNSLICED cache buffer [numKV, pitch, 512] bf16 of raw k_proj rows.
// len:    live rows (attended: rows 0 .. len-1; row t has rotary position t).
// kw:     k-norm weights [512] bf16.  invFreq: rotary table (>= 64 entries; the first
//         64 are used, a zero tail is the identity).  Returns O [numQ, 512] bf16.
// Throws std::invalid_argument on shape contracts (ESDecodeAttn.mm:419-422).
Tensor esDecodeAttnGlobal(const Tensor &q, const Tensor &rawBuf, int len, int pitch, const Tensor &kw,
                          float eps, const std::vector<float> &invFreq, hipStream_t stream = nullptr,
                          Tensor *out = nullptr);

// The same over a q8 raw stream (esDecodeAttnGlobalQ8, ESDecodeAttn.h:30-35,
// ESDecodeAttn.mm:455-489): qBuf [numKV, pitch, 512] u8 and scBuf / bsBuf [numKV, pitch, 1]
// f32, the unsliced buffers of ESKVCache::updateRawQ8; rows x = q * scale + bias.
Tensor esDecodeAttnGlobalQ8(const Tensor &q, const Tensor &qBuf, const Tensor &scBuf, const Tensor &bsBuf,
                            int len, int pitch, const Tensor &kw, float eps, const std::vector<float> &invFreq,
                            hipStream_t stream = nullptr, Tensor *out = nullptr);

// Per-row affine u8 quantizer (esQuantizeRawRows, ESDecodeAttn.h:39-43, ESDecodeAttn.mm:491-539):
// kNew [kvH, n, 512] bf16 -> {q u8 [kvH, n, 512], scale f32 [kvH, n, 1], bias f32 [kvH, n, 1]}
// with x ~ q * scale + bias.  One launch of quantize_rows_kernel (esda_quantize_raw_rows).
std::array<Tensor, 3> esQuantizeRawRows(const Tensor &kNew, hipStream_t stream = nullptr);

}  // namespace es

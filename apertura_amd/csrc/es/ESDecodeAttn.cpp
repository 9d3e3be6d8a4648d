// ESDecodeAttn.cpp -- esDecodeAttnGlobal (Apertura ESDecodeAttn.mm:415-453) over the
// esda_decode_raw kernels: the caller's cache rows are already appended (updateRaw), so
// the call attends rows 0 .. len-1 with no append.
#include "es/ESDecodeAttn.h"

#include <algorithm>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>

#include "es/ESKVCache.h"
#include "es/stream_scratch.h"
#include "es/es_fill.h"
#include "esda.h"

namespace es {
namespace {

void hipCheck(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void esdaCheck(int rc) {
    if (rc == ESDA_OK) return;
    if (rc == ESDA_ERR_INVALID_ARGUMENT) throw std::invalid_argument(esda_last_error());
    throw std::runtime_error(esda_last_error());
}

// Per-thread, per-device, per-stream scratch: the split workspace, the position word, the last
// rotary frequencies uploaded (the reference passes them by value on every call) and
// their cos/sin table (esda_rope_table, grown in 4096-row steps).
struct Scratch {
    std::optional<Tensor> workspace, pos, invFreq, ropeTab;
    std::vector<float> invFreqHost;
    int ropeRows = 0;
};

// The cos/sin table of s.invFreq covering `rows` cache rows.
const void *ropeTable(Scratch &s, int rows, hipStream_t st) {
    if (!s.ropeTab || s.ropeRows < rows) {
        if (s.ropeTab) hipCheck(hipStreamSynchronize(st), "rope table growth");
        const int n = (rows + 4095) / 4096 * 4096;
        s.ropeTab = Tensor::empty({(int64_t) n * 256}, Dtype::u8);
        esdaCheck(esda_rope_table(static_cast<const float *>(s.invFreq->data), n, s.ropeTab->data, st));
        s.ropeRows = n;
    }
    return s.ropeTab->data;
}

// One scratch set per (device, stream) of the calling thread (at most kMaxStreamScratch of
// them; stream_scratch.h): calls on different streams never share a position word,
// workspace or rebuilt rows, so they may overlap.
Scratch &scratch(hipStream_t st) { return streamScratch<Scratch>(st); }

}  // namespace

Tensor esDecodeAttnGlobal(const Tensor &q, const Tensor &rawBuf, int len, int pitch, const Tensor &kw,
                          float eps, const std::vector<float> &invFreq, hipStream_t st, Tensor *out) {
    // Shape contracts of ESDecodeAttn.mm:419-422.
    if (!rawBuf.defined() || rawBuf.dim() != 3 || rawBuf.dtype != Dtype::bf16 || rawBuf.shape[2] != 512)
        throw std::invalid_argument("esDecodeAttnGlobal: expects headDim 512");
    if (!q.defined() || q.dtype != Dtype::bf16 || !q.contiguous() || q.numel() % 512)
        throw std::invalid_argument("esDecodeAttnGlobal: q must be contiguous bf16 [numQ, 512]");
    const int numKV = (int) rawBuf.shape[0];
    const int numQ = (int) (q.numel() / 512);
    if (numQ != numKV * 8) throw std::invalid_argument("esDecodeAttnGlobal: expects 8 query heads per KV head");
    if (!rawBuf.contiguous() || pitch != rawBuf.shape[1])
        throw std::invalid_argument("esDecodeAttnGlobal: rawBuf must be the unsliced [numKV, pitch, 512] buffer");
    if (len <= 0 || len > pitch) throw std::invalid_argument("esDecodeAttnGlobal: need 0 < len <= pitch");
    if (!kw.defined() || kw.dtype != Dtype::bf16 || kw.numel() != 512 || !kw.contiguous())
        throw std::invalid_argument("esDecodeAttnGlobal: kw must be contiguous bf16 [512]");
    if (invFreq.size() < 64) throw std::invalid_argument("esDecodeAttnGlobal: invFreq needs >= 64 entries");

    Scratch &s = scratch(st);
    if (!s.invFreq || s.invFreqHost.size() != 64 || !std::equal(s.invFreqHost.begin(), s.invFreqHost.end(), invFreq.begin())) {
        if (s.invFreq) hipCheck(hipStreamSynchronize(st), "esDecodeAttnGlobal rotary table");
        s.invFreqHost.assign(invFreq.begin(), invFreq.begin() + 64);
        s.invFreq = Tensor::empty({64}, Dtype::f32);
        s.ropeTab.reset();
        s.ropeRows = 0;
        hipCheck(hipMemcpyAsync(s.invFreq->data, s.invFreqHost.data(), 64 * sizeof(float), hipMemcpyHostToDevice, st),
                 "esDecodeAttnGlobal rotary table upload");
        hipCheck(hipStreamSynchronize(st), "esDecodeAttnGlobal rotary table upload");
    }
    if (!s.pos) s.pos = Tensor::empty({1}, Dtype::i32);
    esdaCheck(esda_fill_i32(static_cast<int32_t *>(s.pos->data), len - 1, 1, st));

    esda_raw_desc d{};
    d.batch = 1;
    d.num_q_heads = numQ;
    d.num_kv_heads = numKV;
    d.head_dim = 512;
    d.cap = pitch;
    d.head_stride = (int64_t) pitch * 512;
    d.seq_stride = (int64_t) numKV * pitch * 512;
    d.max_visible = len;
    d.split_rows = 0;
    d.scale = 1.0f;
    d.eps = eps;
    size_t bytes = 0;
    esdaCheck(esda_decode_raw_workspace_size(&d, &bytes));
    if (!s.workspace || s.workspace->nbytes() < bytes) {
        if (s.workspace) hipCheck(hipStreamSynchronize(st), "esDecodeAttnGlobal workspace growth");
        s.workspace = Tensor::empty({(int64_t) std::max<size_t>(bytes, 1 << 20)}, Dtype::u8);
        zeroFill(s.workspace->data, 256, st);
    }
    Tensor o;
    if (out) {
        if (out->dtype != Dtype::bf16 || !out->contiguous() || out->numel() != (int64_t) numQ * 512)
            throw std::invalid_argument("esDecodeAttnGlobal: out must be contiguous bf16 [numQ, 512]");
        o = *out;
    } else {
        o = Tensor::empty({numQ, 512}, Dtype::bf16);
    }
    esda_raw_args a{};
    a.q = q.data;
    a.k_new = nullptr;
    a.raw_cache = rawBuf.data;
    a.pos = static_cast<const int32_t *>(s.pos->data);
    a.kw = kw.data;
    a.inv_freq = static_cast<const float *>(s.invFreq->data);
    a.rope_table = ropeTable(s, pitch, st);
    a.rope_table_rows = s.ropeRows;
    a.out = o.data;
    a.workspace = s.workspace->data;
    a.workspace_bytes = s.workspace->nbytes();
    esdaCheck(esda_decode_raw(&d, &a, st));
    return o;
}

Tensor esDecodeAttnGlobalQ8(const Tensor &q, const Tensor &qBuf, const Tensor &scBuf, const Tensor &bsBuf,
                            int len, int pitch, const Tensor &kw, float eps, const std::vector<float> &invFreq,
                            hipStream_t st, Tensor *out) {
    // Shape contracts of ESDecodeAttn.mm:459-465.
    if (!qBuf.defined() || qBuf.dim() != 3 || qBuf.shape[2] != 512)
        throw std::invalid_argument("esDecodeAttnGlobalQ8: expects headDim 512 with 8 query heads per KV head");
    if (qBuf.dtype != Dtype::u8) throw std::invalid_argument("esDecodeAttnGlobalQ8: qBuf must be uint8");
    if (!q.defined() || q.dtype != Dtype::bf16 || !q.contiguous() || q.numel() % 512)
        throw std::invalid_argument("esDecodeAttnGlobalQ8: q must be contiguous bf16 [numQ, 512]");
    const int numKV = (int) qBuf.shape[0];
    const int numQ = (int) (q.numel() / 512);
    if (numQ != numKV * 8)
        throw std::invalid_argument("esDecodeAttnGlobalQ8: expects headDim 512 with 8 query heads per KV head");
    if (invFreq.size() < 64) throw std::invalid_argument("esDecodeAttnGlobalQ8: invFreq table too short");
    if (!qBuf.contiguous() || pitch != qBuf.shape[1])
        throw std::invalid_argument("esDecodeAttnGlobalQ8: qBuf must be the unsliced [numKV, pitch, 512] buffer");
    for (const Tensor *t : {&scBuf, &bsBuf})
        if (!t->defined() || t->dtype != Dtype::f32 || !t->contiguous() || t->numel() != (int64_t) numKV * pitch)
            throw std::invalid_argument("esDecodeAttnGlobalQ8: scBuf / bsBuf must be f32 [numKV, pitch, 1]");
    if (len <= 0 || len > pitch) throw std::invalid_argument("esDecodeAttnGlobalQ8: need 0 < len <= pitch");
    if (!kw.defined() || kw.dtype != Dtype::bf16 || kw.numel() != 512 || !kw.contiguous())
        throw std::invalid_argument("esDecodeAttnGlobalQ8: kw must be contiguous bf16 [512]");

    Scratch &s = scratch(st);
    if (!s.invFreq || s.invFreqHost.size() != 64 || !std::equal(s.invFreqHost.begin(), s.invFreqHost.end(), invFreq.begin())) {
        if (s.invFreq) hipCheck(hipStreamSynchronize(st), "esDecodeAttnGlobalQ8 rotary table");
        s.invFreqHost.assign(invFreq.begin(), invFreq.begin() + 64);
        s.invFreq = Tensor::empty({64}, Dtype::f32);
        s.ropeTab.reset();
        s.ropeRows = 0;
        hipCheck(hipMemcpyAsync(s.invFreq->data, s.invFreqHost.data(), 64 * sizeof(float), hipMemcpyHostToDevice, st),
                 "esDecodeAttnGlobalQ8 rotary table upload");
        hipCheck(hipStreamSynchronize(st), "esDecodeAttnGlobalQ8 rotary table upload");
    }
    if (!s.pos) s.pos = Tensor::empty({1}, Dtype::i32);
    esdaCheck(esda_fill_i32(static_cast<int32_t *>(s.pos->data), len - 1, 1, st));

    esda_raw_desc d{};
    d.batch = 1;
    d.num_q_heads = numQ;
    d.num_kv_heads = numKV;
    d.head_dim = 512;
    d.cap = pitch;
    d.head_stride = (int64_t) pitch * 512;
    d.seq_stride = (int64_t) numKV * pitch * 512;
    d.max_visible = len;
    d.split_rows = 0;
    d.scale = 1.0f;
    d.eps = eps;
    size_t bytes = 0;
    esdaCheck(esda_decode_raw_workspace_size(&d, &bytes));
    if (!s.workspace || s.workspace->nbytes() < bytes) {
        if (s.workspace) hipCheck(hipStreamSynchronize(st), "esDecodeAttnGlobalQ8 workspace growth");
        s.workspace = Tensor::empty({(int64_t) std::max<size_t>(bytes, 1 << 20)}, Dtype::u8);
        zeroFill(s.workspace->data, 256, st);
    }
    Tensor o;
    if (out) {
        if (out->dtype != Dtype::bf16 || !out->contiguous() || out->numel() != (int64_t) numQ * 512)
            throw std::invalid_argument("esDecodeAttnGlobalQ8: out must be contiguous bf16 [numQ, 512]");
        o = *out;
    } else {
        o = Tensor::empty({numQ, 512}, Dtype::bf16);
    }
    esda_raw_q8_args a{};
    a.q = q.data;
    a.k_new = nullptr;
    a.q8_cache = qBuf.data;
    a.scale = static_cast<float *>(scBuf.data);
    a.bias = static_cast<float *>(bsBuf.data);
    a.sb_head_stride = pitch;
    a.sb_seq_stride = (int64_t) numKV * pitch;
    a.pos = static_cast<const int32_t *>(s.pos->data);
    a.kw = kw.data;
    a.inv_freq = static_cast<const float *>(s.invFreq->data);
    a.rope_table = ropeTable(s, pitch, st);
    a.rope_table_rows = s.ropeRows;
    a.out = o.data;
    a.workspace = s.workspace->data;
    a.workspace_bytes = s.workspace->nbytes();
    esdaCheck(esda_decode_raw_q8(&d, &a, st));
    return o;
}

std::array<Tensor, 3> esQuantizeRawRows(const Tensor &kNew, hipStream_t stream) {
    return ESKVCache::quantizeRawRows(kNew, stream);
}

}  // namespace es

// esda_decode.hip -- Gemma-4 decode attention for MI355X (gfx950, CDNA4).
//
// One decode step = fused KV append + split-K single-query attention + fp32 merge.
// Reference behaviour (Apertura tree): ESKVCache::update prealloc append
// (ESKVCache.mm:64-109) followed by mx::fast::scaled_dot_product_attention at
// ESAttention.mm:188, with the visibility rule of ESGemma4TextModel.mm:68-83 and the
// split merge of ESDecodeAttn.mm:253-273.
//
// Work decomposition
//   grid (splits, kv heads, sequences), 256 threads = 4 waves per workgroup.  A
//   workgroup owns `chunk` consecutive visible rows of one (sequence, kv head); its
//   waves take 16-row tiles round-robin, each with its own online-softmax state, and
//   merge in LDS at the end.  The whole GQA group (G <= 16 query heads) is one MFMA
//   N dimension, so every K/V byte is read from HBM once per group.
//
// Per 16-row tile (one wave):
//   S^T[16 keys x 16 heads] = K[16 x D] . Q^T[D x 16]   v_mfma_f32_16x16x32_bf16, D/32 steps
//       K comes straight from the 128-bit global loads (A operand: lane l holds row
//       l%16, dims 32k+8(l/16)..+8); Q^T sits in VGPRs for the whole kernel.
//   online softmax in the C layout (lane l: head l%16, keys 4(l/16)+r): the tile max
//       needs two cross-lane exchanges; the rescale of O runs only when a max grows.
//   O^T[D x 16] += V^T[D x 16 keys] . P^T[16 keys x 16]   v_mfma_f32_16x16x16_bf16, D/16
//       P^T is already in B-operand layout (same lane, same keys); V^T is gathered from
//       an LDS copy of the tile whose rows are padded by 16 bytes (conflict-free for the
//       128-bit row writes and the 16-bit column gathers; every address is a per-lane
//       base plus an immediate offset, so no address registers stay live).
//   With attention_k_eq_v the V tile *is* the K registers: one HBM read per row.
//
// The new token's row is read from k_new/v_new by the lane that owns it and stored
// into the cache by the same lane (bit-exact copy); no other workgroup reads that row.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>

#include "esda.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTile = 16;
constexpr int kMaxGroup = 16;
constexpr int kTargetGroups = 512;  // workgroups per launch the split heuristic aims for
constexpr float kLog2e = 1.4426950408889634f;

// ------------------------------------------------------------------ per-sequence view

struct SeqView {
    int nvis;    // visible rows
    int first;   // cache row of the oldest visible position
    int newrow;  // cache row receiving the new token
    int ok;
};

// Visible absolute positions are [lo, pos] with lo = max(0, pos - window + 1) for a
// sliding layer (ESGemma4TextModel.mm:68-83); rows hold p - row_base (linear) or
// p mod cap (ring).  Logical row j (0 = oldest) lives at cache row first + j (mod cap).
__device__ __forceinline__ SeqView seq_view(int pos, int base, int cap, int window, int ring) {
    SeqView v{0, 0, 0, 0};
    if (pos < 0) return v;
    int lo = window > 0 ? max(pos - window + 1, 0) : 0;
    if (ring) {
        v.newrow = pos % cap;
        v.first = lo % cap;
    } else {
        if (lo < base) lo = base;
        v.newrow = pos - base;
        if (v.newrow < 0 || v.newrow >= cap) return v;
        v.first = lo - base;
    }
    v.nvis = pos - lo + 1;
    v.ok = 1;
    return v;
}

struct AttendParams {
    const uint16_t *q, *k_new, *v_new;
    uint16_t *k_cache, *v_cache;
    const int *pos, *row_base;
    float *part_acc, *part_ml;
    int *status;
    long long seq_stride, head_stride;
    int B, Hq, Hkv, G, cap, window, ring, S, chunk;
    float scale_log2e;
};

// LDS row stride of a staged tile: 16 bytes of padding shift consecutive rows by 4
// banks, so 16 rows x 16-byte writes cover all banks and the 4 rows a column gather
// touches at once (rows 4g+e) fall into disjoint 8-dword windows.
template <int D>
constexpr int lds_row_bytes() { return D * 2 + 16; }

__device__ __forceinline__ float wave_max_across_groups(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

__device__ __forceinline__ void lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int D, bool SHARED>
struct TileRegs {
    uint4 k[D / 32];
    uint4 v[SHARED ? 1 : D / 32];
};

template <int D, bool SHARED>
__device__ __forceinline__ void load_tile(TileRegs<D, SHARED> &t, const uint16_t *ksrc,
                                          const uint16_t *vsrc, int lg) {
#pragma unroll
    for (int kk = 0; kk < D / 32; ++kk)
        t.k[kk] = *reinterpret_cast<const uint4 *>(ksrc + kk * 32 + lg * 8);
    if constexpr (!SHARED) {
#pragma unroll
        for (int kk = 0; kk < D / 32; ++kk)
            t.v[kk] = *reinterpret_cast<const uint4 *>(vsrc + kk * 32 + lg * 8);
    }
}

template <int D, bool SHARED>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(1, 1)))
void attend_kernel(AttendParams p) {
    constexpr int KK = D / 32;
    constexpr int DT = D / 16;
    constexpr int RS = lds_row_bytes<D>();
    // Per-wave V tile (16 padded rows); reused at the end for the cross-wave merge,
    // which needs 2 * G * D floats <= 128 * D bytes < 4 * 16 * RS bytes.
    __shared__ __attribute__((aligned(16))) unsigned char lds[kWaves * kTile * RS];
    __shared__ float lds_m[kWaves][kMaxGroup];
    __shared__ float lds_l[kWaves][kMaxGroup];

    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lg = lane >> 4;

    const int pos = p.pos[b];
    const int base = p.row_base ? p.row_base[b] : 0;
    const SeqView sv = seq_view(pos, base, p.cap, p.window, p.ring);
    if (!sv.ok) {
        if (split == 0 && kvh == 0 && tid == 0) atomicAdd(p.status, 1);
        return;
    }
    const int j0 = split * p.chunk;
    if (j0 >= sv.nvis) return;
    const int j1 = min(j0 + p.chunk, sv.nvis);
    if (split == p.S - 1 && j1 < sv.nvis && kvh == 0 && tid == 0) atomicAdd(p.status, 1);

    // Q^T operand: lane l carries head l%16 of the group (zero when l%16 >= G).
    bf16x8 qv[KK];
    {
        const bool qok = li < p.G;
        const uint16_t *qrow = p.q + ((size_t) b * p.Hq + (size_t) kvh * p.G + (qok ? li : 0)) * D + lg * 8;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            uint4 t = qok ? *reinterpret_cast<const uint4 *>(qrow + kk * 32) : make_uint4(0, 0, 0, 0);
            qv[kk] = __builtin_bit_cast(bf16x8, t);
        }
    }

    const size_t head_off = (size_t) b * p.seq_stride + (size_t) kvh * p.head_stride;
    uint16_t *kbase = p.k_cache + head_off;
    uint16_t *vbase = p.v_cache + head_off;
    const uint16_t *knew = p.k_new + ((size_t) b * p.Hkv + kvh) * D;
    const uint16_t *vnew = SHARED ? knew : p.v_new + ((size_t) b * p.Hkv + kvh) * D;
    unsigned char *wl = lds + wave * kTile * RS;
    unsigned char *wr_base = wl + li * RS + lg * 16;       // + 64*kk
    const unsigned char *gb[4];                              // + 32*dt
#pragma unroll
    for (int e = 0; e < 4; ++e) gb[e] = wl + (4 * lg + e) * RS + 2 * li;

    float m = -INFINITY, l = 0.0f;
    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int ntile = (j1 - j0 + kTile - 1) / kTile;

    // Row addressing for the tile starting at logical row jt: this lane loads row li.
    auto row_src = [&](int jt, const uint16_t *&ks, const uint16_t *&vs, int &is_new) {
        const int j = jt + li;
        const int jj = j < j1 ? j : j1 - 1;  // clamp: masked rows read a visible row
        int r = sv.first + jj;
        if (r >= p.cap) r -= p.cap;
        is_new = (j == sv.nvis - 1);
        const bool from_new = (jj == sv.nvis - 1);
        ks = from_new ? knew : kbase + (size_t) r * D;
        vs = from_new ? vnew : vbase + (size_t) r * D;
    };

    // One register buffer per wave: a tile's registers are dead once its QK MFMAs have
    // read them and its V rows sit in LDS, so the next tile's loads go into the same
    // registers and stay in flight through this tile's softmax and PV.
    TileRegs<D, SHARED> tr;
    int t = wave;
    int is_new = 0;
    if (t < ntile) {
        const uint16_t *ks, *vs;
        row_src(j0 + t * kTile, ks, vs, is_new);
        load_tile<D, SHARED>(tr, ks, vs, lg);
    }
    for (; t < ntile; t += kWaves) {
        const int jt = j0 + t * kTile;
        // Fused append: the owner of the new row copies it into the cache.
        if (is_new) {
            uint16_t *kd = kbase + (size_t) sv.newrow * D + lg * 8;
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) *reinterpret_cast<uint4 *>(kd + kk * 32) = tr.k[kk];
            if constexpr (!SHARED) {
                uint16_t *vd = vbase + (size_t) sv.newrow * D + lg * 8;
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) *reinterpret_cast<uint4 *>(vd + kk * 32) = tr.v[kk];
            }
        }
        // Scores S^T (keys x heads).
        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, tr.k[kk]), qv[kk], s, 0, 0, 0);
        // V tile -> LDS (row li, dims 32kk+8lg..+8).
        const uint4 *vsrc = SHARED ? tr.k : tr.v;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
            *reinterpret_cast<uint4 *>(wr_base + 64 * kk) = vsrc[kk];
        // Next tile of this wave into the same registers.
        if (t + kWaves < ntile) {
            const uint16_t *ks, *vs;
            row_src(jt + kWaves * kTile, ks, vs, is_new);
            load_tile<D, SHARED>(tr, ks, vs, lg);
        }
        // Online softmax (log2 domain); rows past the split end are masked.
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int jk = jt + 4 * lg + r;
            sc[r] = jk < j1 ? s[r] * p.scale_log2e : -INFINITY;
        }
        const float tmax = wave_max_across_groups(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
        const float mnew = fmaxf(m, tmax);
        if (__any(mnew > m)) {
            const float corr = __builtin_amdgcn_exp2f(m - mnew);
            l *= corr;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) acc[dt] *= corr;
        }
        m = mnew;
        bf16x4 pb;
#pragma unroll
        for (int r = 0; r < 4; ++r) pb[r] = (__bf16) __builtin_amdgcn_exp2f(sc[r] - m);
        l += ((float) pb[0] + (float) pb[1]) + ((float) pb[2] + (float) pb[3]);
        const short4v pbs = __builtin_bit_cast(short4v, pb);
        lds_fence();
        // O^T += V^T . P^T: lane (li, lg) gathers dim 16dt+li of rows 4lg+e.
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            short4v a;
#pragma unroll
            for (int e = 0; e < 4; ++e) a[e] = *reinterpret_cast<const short *>(gb[e] + 32 * dt);
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, pbs, acc[dt], 0, 0, 0);
        }
        lds_fence();
    }

    // ---- merge the 4 waves of this workgroup (log2-domain max, fp32 sums)
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (lg == 0) lds_m[wave][li] = m;
    __syncthreads();
    float mall = lds_m[0][li];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mall = fmaxf(mall, lds_m[w][li]);
    const float f = (m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - mall);
    l *= f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] *= f;
    if (lg == 0) lds_l[wave][li] = l;

    float *slot = reinterpret_cast<float *>(lds);  // [2][G][D]
    const bool hv = li < p.G;
    auto put = [&](int s) {
        if (hv) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                *reinterpret_cast<f32x4 *>(slot + ((size_t) s * p.G + li) * D + 16 * dt + 4 * lg) = acc[dt];
        }
    };
    auto take = [&](int s) {
        if (hv) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                acc[dt] += *reinterpret_cast<const f32x4 *>(slot + ((size_t) s * p.G + li) * D + 16 * dt + 4 * lg);
        }
    };
    if (wave >= 2) put(wave - 2);
    __syncthreads();
    if (wave < 2) take(wave);
    __syncthreads();
    if (wave == 1) put(0);
    __syncthreads();
    if (wave == 0) {
        take(0);
        const size_t pidx = (((size_t) b * p.Hkv + kvh) * p.S + split) * p.G;
        if (hv) {
            float *dst = p.part_acc + (pidx + li) * D;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                *reinterpret_cast<f32x4 *>(dst + 16 * dt + 4 * lg) = acc[dt];
            if (lg == 0) {
                float lt = 0.0f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) lt += lds_l[w][li];
                p.part_ml[(pidx + li) * 2 + 0] = mall;
                p.part_ml[(pidx + li) * 2 + 1] = lt;
            }
        }
    }
}

struct MergeParams {
    const float *part_acc, *part_ml;
    const int *pos, *row_base;
    uint16_t *out;
    int B, Hq, Hkv, G, D, cap, window, ring, S, chunk;
};

// Cross-split merge (ESDecodeAttn.mm:253-273 restated in the log2 domain):
// M = max_s m_s; O = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).  One thread per
// output element; splits past the sequence's visible rows were never written.
__global__ __launch_bounds__(64) void merge_kernel(MergeParams p) {
    const int h = blockIdx.y, b = blockIdx.z;
    const int d = blockIdx.x * 64 + threadIdx.x;
    const int kvh = h / p.G, g = h % p.G;
    const int pos = p.pos[b];
    const int base = p.row_base ? p.row_base[b] : 0;
    const SeqView sv = seq_view(pos, base, p.cap, p.window, p.ring);
    if (!sv.ok || d >= p.D) return;
    int ns = (sv.nvis + p.chunk - 1) / p.chunk;
    if (ns > p.S) ns = p.S;
    const size_t pbase = ((size_t) b * p.Hkv + kvh) * p.S;
    float mx = -INFINITY;
    for (int s = 0; s < ns; ++s) mx = fmaxf(mx, p.part_ml[((pbase + s) * p.G + g) * 2]);
    float o = 0.0f, lt = 0.0f;
    for (int s = 0; s < ns; ++s) {
        const size_t ix = (pbase + s) * p.G + g;
        const float w = __builtin_amdgcn_exp2f(p.part_ml[ix * 2] - mx);
        lt += p.part_ml[ix * 2 + 1] * w;
        o += p.part_acc[ix * p.D + d] * w;
    }
    const __bf16 r = (__bf16) (o / lt);
    p.out[((size_t) b * p.Hq + h) * p.D + d] = __builtin_bit_cast(uint16_t, r);
}

// Plain row copy for multi-row appends (slice_update at rows row0 .. row0 + n - 1).
__global__ __launch_bounds__(256) void append_kernel(uint16_t *cache, long long seq_stride,
                                                      long long head_stride, int Hkv, int D,
                                                      int cap, const uint16_t *src, int n_new,
                                                      const int *row0, int *status) {
    const int b = blockIdx.z, h = blockIdx.y;
    const int r0 = row0[b];
    if (r0 < 0 || r0 + n_new > cap) {
        if (h == 0 && blockIdx.x == 0 && threadIdx.x == 0 && status) atomicAdd(status, 1);
        return;
    }
    const int chunks = D / 8;
    const size_t total = (size_t) n_new * chunks;
    for (size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t) gridDim.x * blockDim.x) {
        const int r = (int) (i / chunks), c = (int) (i % chunks);
        const uint4 v = *reinterpret_cast<const uint4 *>(src + (((size_t) b * Hkv + h) * n_new + r) * D + c * 8);
        *reinterpret_cast<uint4 *>(cache + (size_t) b * seq_stride + (size_t) h * head_stride +
                                   (size_t) (r0 + r) * D + c * 8) = v;
    }
}

// ------------------------------------------------------------------------ host side

thread_local std::string g_err;

int fail(int code, const std::string &msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(ESDA_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// The library is built for gfx950 only: refuse other devices loudly.
int check_device() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    static std::mutex mu;
    static int checked[64] = {0};
    std::lock_guard<std::mutex> lk(mu);
    if (dev < 0 || dev >= 64) return fail(ESDA_ERR_DEVICE, "device index out of range");
    if (checked[dev] == 0) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
        checked[dev] = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
    }
    if (checked[dev] < 0) return fail(ESDA_ERR_DEVICE, "libesda.so is built for gfx950 only");
    return ESDA_OK;
}

bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

struct Plan {
    int G, maxvis, chunk, S;
    size_t off_ml, off_acc, bytes;
};

int make_plan(const esda_decode_desc *d, Plan *pl) {
    if (!d) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: null description");
    if (d->batch <= 0 || d->num_q_heads <= 0 || d->num_kv_heads <= 0)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: batch and head counts must be positive");
    if (d->head_dim != 128 && d->head_dim != 256 && d->head_dim != 512)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: head_dim must be 128, 256 or 512");
    if (d->num_q_heads % d->num_kv_heads)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: num_q_heads must be a multiple of num_kv_heads");
    const int G = d->num_q_heads / d->num_kv_heads;
    if (G > kMaxGroup)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: at most 16 query heads per kv head");
    if (d->cap <= 0) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: cap must be positive");
    if (d->window < 0) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: window must be >= 0");
    if (d->ring && (d->window <= 0 || d->window > d->cap))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: ring mode needs 0 < window <= cap");
    if (d->head_stride < (int64_t) d->cap * d->head_dim || (d->head_stride % 8) != 0)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: head_stride must be >= cap*head_dim and a multiple of 8");
    if (d->seq_stride < (int64_t) d->num_kv_heads * d->head_stride || (d->seq_stride % 8) != 0)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: seq_stride must be >= num_kv_heads*head_stride and a multiple of 8");
    if (d->split_rows < 0 || (d->split_rows % kTile) != 0)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: split_rows must be a multiple of 16");
    int bound = d->ring ? d->window : (d->window > 0 ? std::min(d->window, d->cap) : d->cap);
    int maxvis = d->max_visible > 0 ? std::min(d->max_visible, bound) : bound;
    int chunk = d->split_rows;
    if (chunk == 0) {
        const double rows = (double) maxvis * d->batch * d->num_kv_heads;
        long long c = (long long) std::ceil(rows / kTargetGroups);
        c = (c + 63) / 64 * 64;
        if (c < 64) c = 64;
        if (c > 8192) c = 8192;
        chunk = (int) c;
    }
    const int S = (maxvis + chunk - 1) / chunk;
    pl->G = G;
    pl->maxvis = maxvis;
    pl->chunk = chunk;
    pl->S = S;
    const size_t parts = (size_t) d->batch * d->num_kv_heads * S * G;
    pl->off_ml = 256;
    pl->off_acc = pl->off_ml + ((parts * 2 * sizeof(float) + 255) / 256) * 256;
    pl->bytes = pl->off_acc + parts * d->head_dim * sizeof(float);
    return ESDA_OK;
}

template <int D, bool SHARED>
hipError_t launch_attend(const AttendParams &ap, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((attend_kernel<D, SHARED>), grid, dim3(kThreads), 0, st, ap);
    return hipGetLastError();
}

hipError_t dispatch_attend(int D, bool shared, const AttendParams &ap, dim3 grid, hipStream_t st) {
    switch (D) {
        case 128: return shared ? launch_attend<128, true>(ap, grid, st) : launch_attend<128, false>(ap, grid, st);
        case 256: return shared ? launch_attend<256, true>(ap, grid, st) : launch_attend<256, false>(ap, grid, st);
        default:  return shared ? launch_attend<512, true>(ap, grid, st) : launch_attend<512, false>(ap, grid, st);
    }
}

}  // namespace

extern "C" {

const char *esda_last_error(void) { return g_err.c_str(); }

int esda_version(void) { return 100; }

int esda_decode_workspace_size(const esda_decode_desc *desc, size_t *bytes) {
    Plan pl;
    int rc = make_plan(desc, &pl);
    if (rc) return rc;
    if (!bytes) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_workspace_size: null output");
    *bytes = pl.bytes;
    return ESDA_OK;
}

int esda_decode_stages(const esda_decode_desc *d, const esda_decode_args *a, int stages,
                       void *stream) {
    Plan pl;
    int rc = make_plan(d, &pl);
    if (rc) return rc;
    if (!a) return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: null arguments");
    if (!a->q || !a->k_new || !a->k_cache || !a->v_cache || !a->pos || !a->out)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: null device pointer");
    if (!d->kv_shared && !a->v_new)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: v_new is required unless kv_shared");
    if (d->kv_shared && a->v_cache != a->k_cache)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: kv_shared needs v_cache == k_cache");
    if (!d->kv_shared && a->v_cache == a->k_cache)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: separate K/V need distinct caches");
    if (!aligned16(a->q) || !aligned16(a->k_new) || (a->v_new && !aligned16(a->v_new)) ||
        !aligned16(a->k_cache) || !aligned16(a->v_cache) || !aligned16(a->out))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode: tensors must be 16-byte aligned");
    if (!a->workspace || a->workspace_bytes < pl.bytes || !aligned16(a->workspace))
        return fail(ESDA_ERR_WORKSPACE, "esda_decode: workspace missing or smaller than esda_decode_workspace_size");
    if ((stages & (ESDA_STAGE_ATTEND | ESDA_STAGE_MERGE)) == 0 || (stages & ~3))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_stages: bad stage mask");
    rc = check_device();
    if (rc) return rc;

    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    unsigned char *ws = static_cast<unsigned char *>(a->workspace);
    float *part_ml = reinterpret_cast<float *>(ws + pl.off_ml);
    float *part_acc = reinterpret_cast<float *>(ws + pl.off_acc);
    if (stages & ESDA_STAGE_ATTEND) {
        AttendParams ap;
        ap.q = static_cast<const uint16_t *>(a->q);
        ap.k_new = static_cast<const uint16_t *>(a->k_new);
        ap.v_new = static_cast<const uint16_t *>(d->kv_shared ? a->k_new : a->v_new);
        ap.k_cache = static_cast<uint16_t *>(a->k_cache);
        ap.v_cache = static_cast<uint16_t *>(a->v_cache);
        ap.pos = a->pos;
        ap.row_base = a->row_base;
        ap.part_acc = part_acc;
        ap.part_ml = part_ml;
        ap.status = reinterpret_cast<int *>(ws);
        ap.seq_stride = d->seq_stride;
        ap.head_stride = d->head_stride;
        ap.B = d->batch;
        ap.Hq = d->num_q_heads;
        ap.Hkv = d->num_kv_heads;
        ap.G = pl.G;
        ap.cap = d->cap;
        ap.window = d->window;
        ap.ring = d->ring;
        ap.S = pl.S;
        ap.chunk = pl.chunk;
        ap.scale_log2e = d->scale * kLog2e;
        dim3 grid(pl.S, d->num_kv_heads, d->batch);
        hipError_t e = dispatch_attend(d->head_dim, d->kv_shared != 0, ap, grid, st);
        if (e != hipSuccess) return hip_fail(e, "attend_kernel launch");
    }
    if (stages & ESDA_STAGE_MERGE) {
        MergeParams mp;
        mp.part_acc = part_acc;
        mp.part_ml = part_ml;
        mp.pos = a->pos;
        mp.row_base = a->row_base;
        mp.out = static_cast<uint16_t *>(a->out);
        mp.B = d->batch;
        mp.Hq = d->num_q_heads;
        mp.Hkv = d->num_kv_heads;
        mp.G = pl.G;
        mp.D = d->head_dim;
        mp.cap = d->cap;
        mp.window = d->window;
        mp.ring = d->ring;
        mp.S = pl.S;
        mp.chunk = pl.chunk;
        dim3 grid(d->head_dim / 64, d->num_q_heads, d->batch);
        hipLaunchKernelGGL(merge_kernel, grid, dim3(64), 0, st, mp);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(e, "merge_kernel launch");
    }
    return ESDA_OK;
}

int esda_decode(const esda_decode_desc *desc, const esda_decode_args *args, void *stream) {
    return esda_decode_stages(desc, args, ESDA_STAGE_ATTEND | ESDA_STAGE_MERGE, stream);
}

int esda_decode_status(const esda_decode_desc *desc, void *workspace, int32_t *bad_sequences,
                       void *stream) {
    if (!workspace || !bad_sequences)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_decode_status: null pointer");
    (void) desc;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    int32_t v = 0;
    hipError_t e = hipMemcpyAsync(&v, workspace, sizeof(v), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "esda_decode_status read");
    const int32_t zero = 0;
    e = hipMemcpyAsync(workspace, &zero, sizeof(zero), hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "esda_decode_status clear");
    *bad_sequences = v;
    return ESDA_OK;
}

int esda_kv_append(void *cache, int64_t seq_stride, int64_t head_stride, int32_t batch,
                   int32_t num_kv_heads, int32_t head_dim, int32_t cap, const void *src,
                   int32_t n_new, const int32_t *row0, void *stream) {
    if (!cache || !src || !row0)
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_kv_append: null pointer");
    if (batch <= 0 || num_kv_heads <= 0 || n_new <= 0 || cap <= 0 || head_dim <= 0 || (head_dim % 8))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_kv_append: bad sizes");
    if (head_stride < (int64_t) cap * head_dim || seq_stride < (int64_t) num_kv_heads * head_stride ||
        (head_stride % 8) || (seq_stride % 8))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_kv_append: bad strides");
    if (!aligned16(cache) || !aligned16(src))
        return fail(ESDA_ERR_INVALID_ARGUMENT, "esda_kv_append: tensors must be 16-byte aligned");
    int rc = check_device();
    if (rc) return rc;
    const size_t total = (size_t) n_new * (head_dim / 8);
    int gx = (int) std::min<size_t>((total + 255) / 256, 1024);
    dim3 grid(gx, num_kv_heads, batch);
    hipLaunchKernelGGL(append_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<uint16_t *>(cache), (long long) seq_stride, (long long) head_stride,
                       num_kv_heads, head_dim, cap, static_cast<const uint16_t *>(src), n_new, row0,
                       nullptr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "append_kernel launch");
    return ESDA_OK;
}

}  // extern "C"

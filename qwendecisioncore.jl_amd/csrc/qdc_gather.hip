// qdc_gather.hip -- embedding gather (token id -> row copy) for gfx950, plus
// the host-side id check and the library's version/status strings.
//
// Fast paths move 16-byte chunks with nontemporal loads and stores.  A copy of
// the bits (bf16->bf16, f32->f32) takes one thread per chunk (row = thread /
// chunks per row), the plain-copy shape that measured fastest on gfx950.  The
// widening gather (bf16 table -> fp32 rows, each value shifted left by 16 bits)
// turns every 16-byte input chunk into 32 output bytes; there lane 2m of a
// wavefront loads chunk m and lane 2m+1 chunk 32+m of the wavefront's 64, and
// one neighbour swap (DPP) of half a chunk lets each of the two store
// instructions write one contiguous 1 KB span (each lane storing its own two
// halves would write 16-byte pieces 32 bytes apart, which left partly written
// lines and ~5% more bytes written than the output holds).  A wavefront-per-row
// kernel covers launches too large for 32-bit thread indices.  Results are
// bit-exact.  An id outside [0, vocab) yields a zero row and sets *error_flag
// (when given).
#include "qdc_common.hpp"

namespace qdc {
namespace {

constexpr int kUnroll = 4;

// widened copy of one bf16 chunk (8 values) as two fp32 chunks, or the bits as they are
template <typename TI, typename TO> __device__ __forceinline__ void put_chunk(TO *dst, u32x4 r) {
    if constexpr (sizeof(TI) == sizeof(TO)) {
        store_raw(dst, r);
    } else {
        u32x4 lo, hi;
        lo[0] = r[0] << 16; lo[1] = r[0] & 0xffff0000u;
        lo[2] = r[1] << 16; lo[3] = r[1] & 0xffff0000u;
        hi[0] = r[2] << 16; hi[1] = r[2] & 0xffff0000u;
        hi[2] = r[3] << 16; hi[3] = r[3] & 0xffff0000u;
        store_raw(dst, lo);
        store_raw(dst + 4, hi);
    }
}

template <typename TI, typename TO>
__global__ __launch_bounds__(kBlock) void gather_flat(TO *__restrict__ out,
                                                      const TI *__restrict__ table,
                                                      const int32_t *__restrict__ ids,
                                                      uint32_t total, FastDiv chunks, int64_t vocab,
                                                      int32_t *error_flag) {
    constexpr int V = Elem<TI>::kVec;
    const uint32_t g = blockIdx.x * kBlock + threadIdx.x;
    if (g >= total) return;
    const uint32_t row = fastdiv(g, chunks);
    const uint32_t c = g - row * chunks.d;
    const int64_t hidden = (int64_t)chunks.d * V;
    const int64_t id = ids[row];
    TO *dst = out + (int64_t)row * hidden + (int64_t)c * V;
    if (id < 0 || id >= vocab) {
        put_chunk<TI, TO>(dst, u32x4{0u, 0u, 0u, 0u});
        if (c == 0 && error_flag) atomicOr(error_flag, 1);
        return;
    }
    put_chunk<TI, TO>(dst, load_stream(table + id * hidden + (int64_t)c * V));
}

// bf16 table -> fp32 rows, 16-byte input chunks g of the flat [n_ids, chunks]
// grid; wavefront w covers chunks [64w, 64w + 64) and output chunks (4 fp32)
// [128w, 128w + 128).  No lane returns early: every lane takes part in the swap.
__device__ __forceinline__ u32x4 widen_pair(uint32_t a, uint32_t b) {
    return u32x4{a << 16, a & 0xffff0000u, b << 16, b & 0xffff0000u};
}

__global__ __launch_bounds__(kBlock) void gather_widen(float *__restrict__ out,
                                                       const bf16_t *__restrict__ table,
                                                       const int32_t *__restrict__ ids,
                                                       uint32_t total, FastDiv chunks,
                                                       int64_t vocab, int32_t *error_flag) {
    constexpr int V = Elem<bf16_t>::kVec;
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t base = blockIdx.x * kBlock + (threadIdx.x - lane);
    const uint32_t half = lane >> 1;
    const bool odd = lane & 1u;
    const uint32_t g = base + half + (odd ? kWave / 2 : 0u);
    u32x4 r = {0u, 0u, 0u, 0u};
    if (g < total) {
        const uint32_t row = fastdiv(g, chunks);
        const uint32_t c = g - row * chunks.d;
        const int64_t id = ids[row];
        if (id >= 0 && id < vocab)
            r = load_stream(table + id * ((int64_t)chunks.d * V) + (int64_t)c * V);
        else if (c == 0 && error_flag)
            atomicOr(error_flag, 1);
    }
    // Even lanes keep the low half (r[0], r[1]) of chunk `half` and send its high
    // half; odd lanes keep the high half (r[2], r[3]) of chunk 32 + half and send
    // its low half.  quad_perm [1,0,3,2] exchanges lane pairs (l, l ^ 1).
    const uint32_t send0 = odd ? r[0] : r[2], send1 = odd ? r[1] : r[3];
    const uint32_t got0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)send0, 0xB1, 0xf, 0xf, true);
    const uint32_t got1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)send1, 0xB1, 0xf, 0xf, true);
    // store 0: output chunk 2*base + lane = half (lane & 1) of input chunk base + lane/2
    // store 1: output chunk 2*base + 64 + lane, from input chunk base + 32 + lane/2
    const u32x4 first = odd ? widen_pair(got0, got1) : widen_pair(r[0], r[1]);
    const u32x4 second = odd ? widen_pair(r[2], r[3]) : widen_pair(got0, got1);
    float *dst = out + ((int64_t)base * 2 + lane) * 4;
    if (base + half < total) store_raw(dst, first);
    if (base + kWave / 2 + half < total) store_raw(dst + kWave * 4, second);
}

template <typename TI, typename TO>
__global__ __launch_bounds__(kBlock) void gather_rows(TO *__restrict__ out,
                                                      const TI *__restrict__ table,
                                                      const int32_t *__restrict__ ids,
                                                      int64_t n_ids, int64_t vocab,
                                                      int64_t hidden, int32_t *error_flag) {
    constexpr int V = Elem<TI>::kVec;  // input elements per 16-byte chunk
    const int lane = threadIdx.x % kWave;
    const int64_t row = (int64_t)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (row >= n_ids) return;  // uniform per wavefront
    const int64_t id = ids[row];
    TO *dst = out + row * hidden;
    const int64_t chunks = hidden / V;
    if (id < 0 || id >= vocab) {
        for (int64_t c = lane; c < chunks; c += kWave) put_chunk<TI, TO>(dst + c * V, u32x4{0u, 0u, 0u, 0u});
        if (lane == 0 && error_flag) atomicOr(error_flag, 1);
        return;
    }
    const u32x4 *src = reinterpret_cast<const u32x4 *>(table + id * hidden);
    for (int64_t base = 0; base < chunks; base += kWave * kUnroll) {
        u32x4 r[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t c = base + u * kWave + lane;
            if (c < chunks) r[u] = load_stream(src + c);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t c = base + u * kWave + lane;
            if (c >= chunks) continue;
            put_chunk<TI, TO>(dst + c * V, r[u]);
        }
    }
}

// One wavefront per row, element by element; any alignment and width.
template <typename TI, typename TO>
__global__ __launch_bounds__(kBlock) void gather_general(TO *__restrict__ out,
                                                         const TI *__restrict__ table,
                                                         const int32_t *__restrict__ ids,
                                                         int64_t n_ids, int64_t vocab,
                                                         int64_t hidden, int32_t *error_flag) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = (int64_t)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (row >= n_ids) return;
    const int64_t id = ids[row];
    TO *dst = out + row * hidden;
    const bool ok = id >= 0 && id < vocab;
    const TI *src = table + (ok ? id : 0) * hidden;
    for (int64_t i = lane; i < hidden; i += kWave) {
        if constexpr (sizeof(TI) == sizeof(TO)) {
            dst[i] = ok ? src[i] : TO(0);
        } else {
            dst[i] = ok ? to_f32(src[i]) : 0.0f;
        }
    }
    if (!ok && lane == 0 && error_flag) atomicOr(error_flag, 1);
}

// ------------------------------------------- gather + first input norm ---
// hidden[t] = table[ids[t]] (fp32 residual stream, bit-exact widening) and
// normed[t] = zero-centred RMSNorm(hidden[t]) * keep[t] in one pass over the
// table rows.  gather_rms_fast, groups of 4 elements (an 8-byte bf16 or 16-byte fp32 table
// piece, a 16-byte hidden chunk, an 8-byte bf16 or 16-byte fp32 normed piece):
// an LPR-lane set owns a row, lane l holds groups l, l+LPR, ... (CPL groups),
// so every load and store instruction of the set covers one contiguous span.
template <typename TT, typename TN, int LPR, int CPL>
__global__ __launch_bounds__(kBlock) void gather_rms_fast(
    float *__restrict__ hidden, TN *__restrict__ normed, const TT *__restrict__ table,
    const int32_t *__restrict__ ids, const Aux<TN> *__restrict__ w,
    const int32_t *__restrict__ keep, int64_t n, int64_t vocab, float eps, int32_t *error_flag) {
    constexpr int V = 4;
    constexpr int W = LPR * CPL * V;  // row width
    constexpr int RPB = kBlock / LPR;
    const int lane = threadIdx.x % LPR;
    const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
    const bool active = row < n;
    const int64_t id = active ? (int64_t)ids[row] : 0;
    const bool valid = active && id >= 0 && id < vocab;
    if (active && !valid && lane == 0 && error_flag) atomicOr(error_flag, 1);
    Frag<TT, V> xr[CPL];
    Frag<Aux<TN>, V> wr[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        if (valid) {
            xr[c] = stream_frag<TT, V>(table + id * W + (c * LPR + lane) * V);
        } else {
#pragma unroll
            for (int i = 0; i < Frag<TT, V>::kN; ++i) xr[c].r[i] = u32x4{0u, 0u, 0u, 0u};
        }
    }
#pragma unroll
    for (int c = 0; c < CPL; ++c) wr[c] = load_frag<Aux<TN>, V>(w + (c * LPR + lane) * V);
    const float keep_row = (active && keep) ? (float)keep[row] : 1.0f;
    float v[CPL][V];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        unpack(xr[c], v[c]);
        if (active) store_frag(hidden + row * W + (c * LPR + lane) * V, v[c]);
#pragma unroll
        for (int j = 0; j < V; ++j) ss += v[c][j] * v[c][j];
    }
    ss = group_sum<LPR>(ss);
    if (!active) return;
    const float s = rms_scale(ss, (float)W, eps);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        float wv[V], o[V];
        unpack(wr[c], wv);
#pragma unroll
        for (int j = 0; j < V; ++j) o[j] = (v[c][j] * s) * (1.0f + wv[j]);
        if (keep) {
#pragma unroll
            for (int j = 0; j < V; ++j) o[j] = o[j] * keep_row;
        }
        store_frag(normed + row * W + (c * LPR + lane) * V, o);
    }
}

// bf16 table and bf16 normed rows of a multiple of 512 elements: one
// wavefront per row, 16-byte table chunks.  Slot c covers chunks
// [64c, 64c + 64) of the row; lane 2m holds chunk 64c + m and lane 2m+1 chunk
// 64c + 32 + m, and the lane-pair exchange of gather_widen lets each fp32
// hidden store instruction write one contiguous 1 KB span; each normed store
// instruction writes the slot's 1 KB whole (lanes in chunk order m, 32 + m).
template <int CPL>
__global__ __launch_bounds__(kBlock) void gather_rms_bf16(
    float *__restrict__ hidden, bf16_t *__restrict__ normed, const bf16_t *__restrict__ table,
    const int32_t *__restrict__ ids, const bf16_t *__restrict__ w,
    const int32_t *__restrict__ keep, int64_t n, int64_t vocab, float eps,
    int32_t *error_flag) {
    constexpr int V = 8;
    constexpr int W = CPL * kWave * V;
    const uint32_t lane = threadIdx.x % kWave;
    const int64_t row = (int64_t)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (row >= n) return;  // uniform per wavefront
    const int64_t id = ids[row];
    const bool valid = id >= 0 && id < vocab;
    if (!valid && lane == 0 && error_flag) atomicOr(error_flag, 1);
    const bool odd = lane & 1u;
    const int mine = (int)(lane >> 1) + (odd ? kWave / 2 : 0);  // chunk within a slot
    u32x4 r[CPL], wr[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        r[c] = valid ? load_stream(table + id * W + (c * kWave + mine) * V)
                     : u32x4{0u, 0u, 0u, 0u};
        wr[c] = load_raw(w + (c * kWave + mine) * V);
    }
    const float keep_row = keep ? (float)keep[row] : 1.0f;
    float ss = 0.0f;
    float *hrow = hidden + row * W;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        float v[V];
        unpack(r[c], v);
#pragma unroll
        for (int j = 0; j < V; ++j) ss += v[j] * v[j];
        // even lanes keep the low half of chunk m, odd lanes the high half of
        // chunk 32 + m; store 0 is output chunk 2*(64c) + lane, store 1 the next 64
        const uint32_t send0 = odd ? r[c][0] : r[c][2], send1 = odd ? r[c][1] : r[c][3];
        const uint32_t got0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)send0, 0xB1, 0xf, 0xf, true);
        const uint32_t got1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)send1, 0xB1, 0xf, 0xf, true);
        const u32x4 first = odd ? widen_pair(got0, got1) : widen_pair(r[c][0], r[c][1]);
        const u32x4 second = odd ? widen_pair(r[c][2], r[c][3]) : widen_pair(got0, got1);
        float *dst = hrow + ((int64_t)c * kWave * 2 + lane) * 4;
        store_raw(dst, first);
        store_raw(dst + kWave * 4, second);
    }
    ss = group_sum<kWave>(ss);
    const float s = rms_scale(ss, (float)W, eps);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        float v[V], wv[V], o[V];
        unpack(r[c], v);
        unpack(wr[c], wv);
#pragma unroll
        for (int j = 0; j < V; ++j) o[j] = (v[j] * s) * (1.0f + wv[j]);
        if (keep) {
#pragma unroll
            for (int j = 0; j < V; ++j) o[j] = o[j] * keep_row;
        }
        store_raw(normed + row * W + (c * kWave + mine) * V, pack(o));
    }
}

// One wavefront per row, any width or alignment: the first pass widens the
// row into hidden and sums its squares, the second normalises it from hidden
// (written by the same lane, read back from cache).
template <typename TT, typename TN>
__global__ __launch_bounds__(kBlock) void gather_rms_general(
    float *__restrict__ hidden, TN *__restrict__ normed, const TT *__restrict__ table,
    const int32_t *__restrict__ ids, const Aux<TN> *__restrict__ w,
    const int32_t *__restrict__ keep, int64_t n, int64_t vocab, int64_t width, float eps,
    int32_t *error_flag) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = (int64_t)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (row >= n) return;  // uniform per wavefront
    const int64_t id = ids[row];
    const bool valid = id >= 0 && id < vocab;
    if (!valid && lane == 0 && error_flag) atomicOr(error_flag, 1);
    const TT *src = table + (valid ? id : 0) * width;
    float *h = hidden + row * width;
    float ss = 0.0f;
    for (int64_t i = lane; i < width; i += kWave) {
        const float v = valid ? to_f32(src[i]) : 0.0f;
        h[i] = v;
        ss += v * v;
    }
    ss = group_sum<kWave>(ss);
    const float s = rms_scale(ss, (float)width, eps);
    const float keep_row = keep ? (float)keep[row] : 1.0f;
    for (int64_t i = lane; i < width; i += kWave) {
        float o = (h[i] * s) * (1.0f + to_f32(w[i]));
        if (keep) o = o * keep_row;
        put_elem(normed, row * width + i, o);
    }
}

template <typename TT, typename TN, int LPR, int CPL>
int32_t launch_gather_rms_fast(float *hidden, TN *normed, const TT *table, const int32_t *ids,
                               const Aux<TN> *w, const int32_t *keep, int64_t n, int64_t vocab,
                               float eps, int32_t *error_flag, hipStream_t stream) {
    hipLaunchKernelGGL((gather_rms_fast<TT, TN, LPR, CPL>),
                       dim3((uint32_t)ceil_div(n, kBlock / LPR)), dim3(kBlock), 0, stream, hidden,
                       normed, table, ids, w, keep, n, vocab, eps, error_flag);
    return launch_status();
}

// Fast shapes by G = width / 4 groups: LPR = G/2 lanes of 2 groups for rows of
// up to 64 groups (a power of two), else 64 lanes of G/64 groups.
template <typename TT, typename TN>
int32_t launch_gather_rms(float *hidden, TN *normed, const TT *table, const int32_t *ids,
                          const Aux<TN> *w, const int32_t *keep, int64_t n, int64_t vocab,
                          int64_t width, float eps, bool fast, int32_t *error_flag,
                          hipStream_t stream) {
    if constexpr (sizeof(TT) == 2 && sizeof(TN) == 2) {
        const dim3 grid((uint32_t)ceil_div(n, kBlock / kWave));
        if (fast && width == 512)
            hipLaunchKernelGGL(gather_rms_bf16<1>, grid, dim3(kBlock), 0, stream, hidden, normed,
                               table, ids, w, keep, n, vocab, eps, error_flag);
        if (fast && width == 1024)
            hipLaunchKernelGGL(gather_rms_bf16<2>, grid, dim3(kBlock), 0, stream, hidden, normed,
                               table, ids, w, keep, n, vocab, eps, error_flag);
        if (fast && width == 2048)
            hipLaunchKernelGGL(gather_rms_bf16<4>, grid, dim3(kBlock), 0, stream, hidden, normed,
                               table, ids, w, keep, n, vocab, eps, error_flag);
        if (fast && (width == 512 || width == 1024 || width == 2048)) return launch_status();
    }
    if (fast && width % 4 == 0) {
#define QDC_GR(LPR, CPL)                                                                     \
    case LPR * CPL:                                                                          \
        return launch_gather_rms_fast<TT, TN, LPR, CPL>(hidden, normed, table, ids, w, keep, \
                                                        n, vocab, eps, error_flag, stream);
        switch (width / 4) {
            QDC_GR(1, 2)
            QDC_GR(2, 2)
            QDC_GR(4, 2)
            QDC_GR(8, 2)
            QDC_GR(16, 2)
            QDC_GR(32, 2)
            QDC_GR(64, 2)
            QDC_GR(64, 4)
            QDC_GR(64, 5)
            QDC_GR(64, 6)
            QDC_GR(64, 8)
            QDC_GR(64, 10)
            QDC_GR(64, 12)
            QDC_GR(64, 16)
            default:
                break;
        }
#undef QDC_GR
    }
    hipLaunchKernelGGL((gather_rms_general<TT, TN>), dim3((uint32_t)ceil_div(n, kBlock / kWave)),
                       dim3(kBlock), 0, stream, hidden, normed, table, ids, w, keep, n, vocab,
                       width, eps, error_flag);
    return launch_status();
}

template <typename TI, typename TO>
int32_t launch(void *out, const void *table, const int32_t *ids, int64_t n_ids, int64_t vocab,
               int64_t hidden, int32_t *error_flag, bool fast, hipStream_t stream) {
    const int64_t blocks = ceil_div(n_ids, kBlock / kWave);
    const int64_t chunks = hidden / Elem<TI>::kVec;
    if (fast && hidden % Elem<TI>::kVec == 0 && n_ids * chunks < ((int64_t)1 << 31)) {
        const uint32_t total = (uint32_t)(n_ids * chunks);
        if constexpr (sizeof(TI) != sizeof(TO))
            hipLaunchKernelGGL(gather_widen, dim3((uint32_t)ceil_div(total, kBlock)),
                               dim3(kBlock), 0, stream, (float *)out, (const bf16_t *)table, ids,
                               total, make_fastdiv((uint32_t)chunks), vocab, error_flag);
        else
            hipLaunchKernelGGL((gather_flat<TI, TO>), dim3((uint32_t)ceil_div(total, kBlock)),
                               dim3(kBlock), 0, stream, (TO *)out, (const TI *)table, ids, total,
                               make_fastdiv((uint32_t)chunks), vocab, error_flag);
    } else if (fast && hidden % Elem<TI>::kVec == 0)
        hipLaunchKernelGGL((gather_rows<TI, TO>), dim3((uint32_t)blocks), dim3(kBlock), 0, stream,
                           (TO *)out, (const TI *)table, ids, n_ids, vocab, hidden, error_flag);
    else
        hipLaunchKernelGGL((gather_general<TI, TO>), dim3((uint32_t)blocks), dim3(kBlock), 0,
                           stream, (TO *)out, (const TI *)table, ids, n_ids, vocab, hidden,
                           error_flag);
    return launch_status();
}

}  // namespace
}  // namespace qdc

using namespace qdc;

extern "C" const char *qdc_version(void) { return QDC_HIP_VERSION; }

extern "C" const char *qdc_status_string(int32_t status) {
    switch (status) {
        case QDC_OK: return "ok";
        case QDC_ERR_NULL: return "a required pointer is NULL";
        case QDC_ERR_SHAPE: return "invalid or inconsistent dimensions";
        case QDC_ERR_DTYPE: return "unsupported dtype";
        case QDC_ERR_RANGE: return "token id or position outside its table";
        case QDC_ERR_ALIAS: return "an output overlaps an input it may not alias";
        default: break;
    }
    return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
}

extern "C" int32_t qdc_check_ids(const int64_t *ids, int64_t n_ids, int64_t vocab) {
    if (n_ids < 0 || vocab < 0) return QDC_ERR_SHAPE;
    if (n_ids > 0 && !ids) return QDC_ERR_NULL;
    for (int64_t t = 0; t < n_ids; ++t)
        if (ids[t] < 0 || ids[t] >= vocab) return QDC_ERR_RANGE;
    return QDC_OK;
}

extern "C" int32_t qdc_embedding_gather(void *out, int32_t out_dtype, const void *table,
                                        int32_t table_dtype, const int32_t *ids, int64_t n_ids,
                                        int64_t vocab, int64_t hidden, int32_t *error_flag,
                                        hipStream_t stream) {
    if (!valid_dtype(out_dtype) || !valid_dtype(table_dtype)) return QDC_ERR_DTYPE;
    if (table_dtype == QDC_F32 && out_dtype == QDC_BF16) return QDC_ERR_DTYPE;  // not a copy
    if (n_ids < 0 || vocab < 0 || hidden < 0) return QDC_ERR_SHAPE;
    if (n_ids == 0 || hidden == 0) return QDC_OK;
    if (vocab == 0) return QDC_ERR_RANGE;
    if (n_ids >= ((int64_t)1 << 26)) return QDC_ERR_SHAPE;  // wavefront-per-row grid limit
    if (!out || !table || !ids) return QDC_ERR_NULL;
    const int64_t ti = elem_size(table_dtype), to = elem_size(out_dtype);
    if (overlaps(out, n_ids * hidden * to, table, vocab * hidden * ti) ||
        overlaps(out, n_ids * hidden * to, ids, n_ids * 4))
        return QDC_ERR_ALIAS;
    const bool fast = aligned16(out) && aligned16(table) && (hidden * ti) % 16 == 0;
    if (table_dtype == QDC_F32)
        return launch<float, float>(out, table, ids, n_ids, vocab, hidden, error_flag, fast, stream);
    if (out_dtype == QDC_BF16)
        return launch<bf16_t, bf16_t>(out, table, ids, n_ids, vocab, hidden, error_flag, fast,
                                      stream);
    return launch<bf16_t, float>(out, table, ids, n_ids, vocab, hidden, error_flag, fast, stream);
}

extern "C" int32_t qdc_embedding_gather_rmsnorm(void *hidden, void *normed, const void *table,
                                                int32_t table_dtype, const int32_t *ids,
                                                const void *weight, int32_t normed_dtype,
                                                const int32_t *token_mask, int64_t n_ids,
                                                int64_t vocab, int64_t width, float eps,
                                                int32_t *error_flag, hipStream_t stream) {
    const bool split = normed_dtype == QDC_BF16X2;  // with a bf16 weight
    if (!valid_dtype(table_dtype) || !(valid_dtype(normed_dtype) || split)) return QDC_ERR_DTYPE;
    if (n_ids < 0 || vocab < 0 || width < 0) return QDC_ERR_SHAPE;
    if (n_ids == 0 || width == 0) return QDC_OK;
    if (vocab == 0) return QDC_ERR_RANGE;
    if (n_ids >= ((int64_t)1 << 26)) return QDC_ERR_SHAPE;  // wavefront-per-row grid limit
    if (!hidden || !normed || !table || !ids || !weight) return QDC_ERR_NULL;
    if (split && !split_rows_ok(width, width)) return QDC_ERR_SHAPE;
    const int64_t ti = elem_size(table_dtype), tn = elem_size(normed_dtype);
    const int64_t tw = split ? 2 : tn;  // weight element bytes
    const int64_t hb = n_ids * width * 4, nb = n_ids * width * tn;
    const void *ins[4] = {table, ids, weight, token_mask};
    const int64_t in_bytes[4] = {vocab * width * ti, n_ids * 4, width * tw,
                                 token_mask ? n_ids * 4 : 0};
    for (int i = 0; i < 4; ++i)
        if (overlaps(hidden, hb, ins[i], in_bytes[i]) || overlaps(normed, nb, ins[i], in_bytes[i]))
            return QDC_ERR_ALIAS;
    if (overlaps(hidden, hb, normed, nb)) return QDC_ERR_ALIAS;
    if (error_flag && (overlaps(error_flag, 4, hidden, hb) || overlaps(error_flag, 4, normed, nb)))
        return QDC_ERR_ALIAS;
    const bool fast = aligned16(hidden) && aligned16(table) && aligned16(normed) &&
                      aligned16(weight) && (width * ti) % 16 == 0 && (width * tn) % 16 == 0;
    float *h = static_cast<float *>(hidden);
    if (split && table_dtype == QDC_BF16)
        return launch_gather_rms(h, (split_t *)normed, (const bf16_t *)table, ids,
                                 (const bf16_t *)weight, token_mask, n_ids, vocab, width, eps,
                                 fast, error_flag, stream);
    if (split)
        return launch_gather_rms(h, (split_t *)normed, (const float *)table, ids,
                                 (const bf16_t *)weight, token_mask, n_ids, vocab, width, eps,
                                 fast, error_flag, stream);
    if (table_dtype == QDC_BF16 && normed_dtype == QDC_BF16)
        return launch_gather_rms(h, (bf16_t *)normed, (const bf16_t *)table, ids,
                                 (const bf16_t *)weight, token_mask, n_ids, vocab, width, eps,
                                 fast, error_flag, stream);
    if (table_dtype == QDC_BF16)
        return launch_gather_rms(h, (float *)normed, (const bf16_t *)table, ids,
                                 (const float *)weight, token_mask, n_ids, vocab, width, eps,
                                 fast, error_flag, stream);
    if (normed_dtype == QDC_BF16)
        return launch_gather_rms(h, (bf16_t *)normed, (const float *)table, ids,
                                 (const bf16_t *)weight, token_mask, n_ids, vocab, width, eps,
                                 fast, error_flag, stream);
    return launch_gather_rms(h, (float *)normed, (const float *)table, ids,
                             (const float *)weight, token_mask, n_ids, vocab, width, eps, fast,
                             error_flag, stream);
}

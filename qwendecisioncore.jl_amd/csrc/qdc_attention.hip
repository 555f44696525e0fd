// qdc_attention.hip -- the bandwidth-bound row work around full attention's two
// batched GEMMs: the masked, scaled softmax over each query's score row, and the
// sigmoid output-gate merge that feeds the output projection.
//
// Softmax (attention_softmax_kernel!, ext/amdgpu_attention.jl:61-88; generic
// src/backbone.jl:237-259): for query j (position j = query index + q_offset)
// and key i, value = scores*scale when i <= j and mask[b, i] != 0, else
// -floatmax(Float32); probs = exp(value - max) / sum(exp(value - max)).  A query
// with no visible unmasked key therefore spreads 1/keys over every key, as the
// reference does.  exp runs on the hardware exp2 unit and the row sum is
// inverted once (the accurate library exp and a division per element made the
// kernel vector-ALU bound).
//
// Fast path: one wavefront per score row held in registers (keys <= 2048, 16-byte
// chunks dealt round-robin over the 64 lanes so every load instruction covers a
// contiguous 1 KB); keys after the query are never read (they are -floatmax),
// which halves the read traffic of a causal row on average.  The general path
// streams the row three times (max, sum, write).
//
// Gate merge (merge_gate_kernel!, ext/amdgpu_attention.jl:90-106; generic
// src/backbone.jl:258-259): out[t, h*dim + r] = values[b, h, s, r] *
// sigmoid(gate[t, h, r]) with t = b*seq + s, reading the PV GEMM output in its
// head-major layout and the gate straight out of the q||gate projection.
#include <cfloat>

#include "qdc_common.hpp"

namespace qdc {
namespace {

constexpr int kMaxRowChunks = 8;  // chunks of 4 keys per lane of one wavefront (2048 keys)
constexpr int kMaxRowWaves = 16;  // wavefronts per row in one workgroup (32768 keys)

template <int CTRL> __device__ __forceinline__ float dpp_max_step(float v) {
    return fmaxf(v, dpp<CTRL>(v));
}
// Maximum over the 64 lanes of a wavefront (every lane ends with it).
__device__ __forceinline__ float wave_max(float v) {
    v = dpp_max_step<0xB1>(v);
    v = dpp_max_step<0x4E>(v);
    v = dpp_max_step<0x141>(v);
    v = dpp_max_step<0x140>(v);
    // across rows with the lane swaps (see group_sum): the halves hold lanes l
    // and l ^ 16, then l and l ^ 32
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}

// exp(v - peak) for v <= peak on the hardware exp2 unit: exp2((v - peak) log2 e).
// The product's rounding perturbs the exponent by |v - peak| * 2^-24, i.e. a
// relative error of ~6e-8 |v - peak| on a value exp(v - peak): below 1e-6 for
// every term that is not already negligible next to the row maximum's 1.
__device__ __forceinline__ float exp_shifted(float v, float peak) {
    return __builtin_amdgcn_exp2f((v - peak) * 1.4426950408889634f);
}

struct Softmax {
    const float *scores;
    void *probs;
    const int32_t *mask;  // [batch, keys] or null (all keys unmasked)
    int64_t rows;         // batch * heads * queries
    int64_t keys;
    FastDiv queries;      // row -> query index
    FastDiv per_batch;    // row -> batch index (heads * queries rows per batch)
    int64_t q_offset;
    float scale;
};

template <typename TO> __device__ __forceinline__ void store4(TO *p, const float (&v)[4]);
template <> __device__ __forceinline__ void store4<float>(float *p, const float (&v)[4]) {
    store_chunk(p, v);
}
template <> __device__ __forceinline__ void store4<bf16_t>(bf16_t *p, const float (&v)[4]) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 r = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    __builtin_nontemporal_store(r, reinterpret_cast<u32x2 *>(p));
}

template <typename TO, int CPL>
__global__ __launch_bounds__(kBlock) void softmax_rows_fast(Softmax a) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = (int64_t)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (row >= a.rows) return;  // uniform per wavefront
    const uint32_t qi = (uint32_t)row - fastdiv((uint32_t)row, a.queries) * a.queries.d;
    const uint32_t b = fastdiv((uint32_t)row, a.per_batch);
    // keys [0, visible) are causally visible to this query
    const int64_t visible = min(a.keys, a.q_offset + (int64_t)qi + 1);
    const float *src = a.scores + row * a.keys;
    const int32_t *mrow = a.mask ? a.mask + (int64_t)b * a.keys : nullptr;

    float v[CPL][4];
    u32x4 raw[CPL];
    int4 mk[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int64_t k0 = ((int64_t)c * kWave + lane) * 4;
        raw[c] = u32x4{0u, 0u, 0u, 0u};
        mk[c] = int4{1, 1, 1, 1};
        if (k0 < visible) {
            raw[c] = load_stream(src + k0);
            if (mrow) mk[c] = *reinterpret_cast<const int4 *>(mrow + k0);
        }
    }
    float peak = -FLT_MAX;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int64_t k0 = ((int64_t)c * kWave + lane) * 4;
        const int mm[4] = {mk[c].x, mk[c].y, mk[c].z, mk[c].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool on = k0 + e < visible && mm[e] != 0;
            v[c][e] = on ? __uint_as_float(raw[c][e]) * a.scale : -FLT_MAX;
            peak = fmaxf(peak, v[c][e]);
        }
    }
    peak = wave_max(peak);
    const bool none = peak == -FLT_MAX;  // no visible unmasked key: every key gets 1/keys
    float total = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int64_t k0 = ((int64_t)c * kWave + lane) * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // chunks past the query hold -floatmax only: exp is 0
            v[c][e] = k0 < visible ? exp_shifted(v[c][e], peak) : 0.0f;
            total += v[c][e];
        }
    }
    total = group_sum<kWave>(total);
    const float inv_total = 1.0f / total;
    TO *dst = reinterpret_cast<TO *>(a.probs) + row * a.keys;
    const float uniform = 1.0f / (float)a.keys;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int64_t k0 = ((int64_t)c * kWave + lane) * 4;
        if (k0 >= a.keys) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = none ? uniform : (k0 + e < visible ? v[c][e] * inv_total : 0.0f);
        store4<TO>(dst + k0, o);
    }
}

// Rows longer than one wavefront's registers (more than 2048 keys): WPR
// wavefronts per row, the row's 16-byte chunks dealt round-robin over them (so
// the causally visible keys spread evenly), each wavefront reducing its share
// with DPP and lane swaps and the WPR partial maxima and sums meeting in LDS.
// Every score is read once and every probability written once, as in
// softmax_rows_fast; workgroups of max(4, WPR) wavefronts.  Wavefronts of rows
// past the end skip their loads and stores but reach both barriers.
template <typename TO, int CPL, int WPR>
__global__ __launch_bounds__(WPR > 4 ? WPR * kWave : kBlock) void softmax_rows_waves(Softmax a) {
    constexpr int NW = WPR > 4 ? WPR : kBlock / kWave;  // wavefronts per workgroup
    constexpr int RPB = NW / WPR;                       // rows per workgroup
    __shared__ float part_max[NW], part_sum[NW];
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int part = wave % WPR, first = wave - part;   // this row's wavefronts: [first, first+WPR)
    const int64_t row = (int64_t)blockIdx.x * RPB + wave / WPR;
    const bool valid = row < a.rows;
    const int64_t r = valid ? row : 0;
    const uint32_t qi = (uint32_t)r - fastdiv((uint32_t)r, a.queries) * a.queries.d;
    const uint32_t b = fastdiv((uint32_t)r, a.per_batch);
    const int64_t visible = valid ? min(a.keys, a.q_offset + (int64_t)qi + 1) : 0;
    const float *src = a.scores + r * a.keys;
    const int32_t *mrow = a.mask ? a.mask + (int64_t)b * a.keys : nullptr;

    float v[CPL][4];
    u32x4 raw[CPL];
    int4 mk[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int64_t k0 = ((int64_t)(c * WPR + part) * kWave + lane) * 4;
        raw[c] = u32x4{0u, 0u, 0u, 0u};
        mk[c] = int4{1, 1, 1, 1};
        if (k0 < visible) {
            raw[c] = load_stream(src + k0);
            if (mrow) mk[c] = *reinterpret_cast<const int4 *>(mrow + k0);
        }
    }
    float peak = -FLT_MAX;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int64_t k0 = ((int64_t)(c * WPR + part) * kWave + lane) * 4;
        const int mm[4] = {mk[c].x, mk[c].y, mk[c].z, mk[c].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool on = k0 + e < visible && mm[e] != 0;
            v[c][e] = on ? __uint_as_float(raw[c][e]) * a.scale : -FLT_MAX;
            peak = fmaxf(peak, v[c][e]);
        }
    }
    peak = wave_max(peak);
    if (lane == 0) part_max[wave] = peak;
    __syncthreads();
    peak = part_max[first];
#pragma unroll
    for (int j = 1; j < WPR; ++j) peak = fmaxf(peak, part_max[first + j]);
    const bool none = peak == -FLT_MAX;  // no visible unmasked key: every key gets 1/keys
    float total = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int64_t k0 = ((int64_t)(c * WPR + part) * kWave + lane) * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[c][e] = k0 < visible ? exp_shifted(v[c][e], peak) : 0.0f;
            total += v[c][e];
        }
    }
    total = group_sum<kWave>(total);
    if (lane == 0) part_sum[wave] = total;
    __syncthreads();
    total = part_sum[first];
#pragma unroll
    for (int j = 1; j < WPR; ++j) total += part_sum[first + j];
    if (!valid) return;
    const float inv_total = 1.0f / total;
    TO *dst = reinterpret_cast<TO *>(a.probs) + r * a.keys;
    const float uniform = 1.0f / (float)a.keys;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int64_t k0 = ((int64_t)(c * WPR + part) * kWave + lane) * 4;
        if (k0 >= a.keys) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = none ? uniform : (k0 + e < visible ? v[c][e] * inv_total : 0.0f);
        store4<TO>(dst + k0, o);
    }
}

template <typename TO>
__global__ __launch_bounds__(kBlock) void softmax_rows_general(Softmax a) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = (int64_t)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (row >= a.rows) return;
    const uint32_t qi = (uint32_t)row - fastdiv((uint32_t)row, a.queries) * a.queries.d;
    const uint32_t b = fastdiv((uint32_t)row, a.per_batch);
    const int64_t visible = min(a.keys, a.q_offset + (int64_t)qi + 1);
    const float *src = a.scores + row * a.keys;
    const int32_t *mrow = a.mask ? a.mask + (int64_t)b * a.keys : nullptr;
    auto value = [&](int64_t k) {
        return (k < visible && (!mrow || mrow[k] != 0)) ? src[k] * a.scale : -FLT_MAX;
    };
    float peak = -FLT_MAX;
    for (int64_t k = lane; k < visible; k += kWave) peak = fmaxf(peak, value(k));
    peak = wave_max(peak);
    const bool none = peak == -FLT_MAX;
    float total = 0.0f;
    for (int64_t k = lane; k < visible; k += kWave) total += exp_shifted(value(k), peak);
    total = group_sum<kWave>(total);
    const float inv_total = 1.0f / total;
    TO *dst = reinterpret_cast<TO *>(a.probs) + row * a.keys;
    const float uniform = 1.0f / (float)a.keys;
    for (int64_t k = lane; k < a.keys; k += kWave) {
        const float o = none ? uniform : (k < visible ? exp_shifted(value(k), peak) * inv_total : 0.0f);
        dst[k] = from_f32<TO>(o);
    }
}

struct Gate {
    const float *values;  // [batch, heads, seq, dim]
    const void *gate;     // element (t, h, r) at t*gate_tok + h*gate_head + r
    void *out;            // element (t, h*dim + r) at t*out_tok + h*dim + r
    int64_t gate_tok, gate_head, out_tok;
    int64_t total;        // tokens * heads * dim / 8 (fast) or elements (general)
    FastDiv chunks;       // dim / 8 (fast) or dim (general)
    FastDiv heads;
    FastDiv seq;
};

__device__ __forceinline__ float sigmoid_ref(float x) {
    // native_sigmoid(x) = 1/(1 + exp(-x)) (src/backbone.jl:196)
    return 1.0f / (1.0f + expf(-x));
}

// One thread per 8 elements of one (token, head) row: 4 in each half of the row.
template <typename TG, typename TO>
__global__ __launch_bounds__(kBlock) void gate_merge_fast(Gate a) {
    const int64_t g = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (g >= a.total) return;
    const uint32_t th = fastdiv((uint32_t)g, a.chunks);
    const uint32_t c = (uint32_t)g - th * a.chunks.d;
    const uint32_t t = fastdiv(th, a.heads);
    const uint32_t h = th - t * a.heads.d;
    const uint32_t b = fastdiv(t, a.seq);
    const uint32_t s = t - b * a.seq.d;
    const int64_t dim = (int64_t)a.chunks.d * 8, half = dim / 2;
    // elements [4c, 4c+4) and [dim/2 + 4c, dim/2 + 4c + 4): every load and store
    // instruction of a wavefront then covers contiguous spans
    const float *vp = a.values + (((int64_t)b * a.heads.d + h) * a.seq.d + s) * dim + c * 4;
    const TG *gp = reinterpret_cast<const TG *>(a.gate) + (int64_t)t * a.gate_tok +
                   (int64_t)h * a.gate_head + c * 4;
    const Frag<float, 4> vf0 = stream_frag<float, 4>(vp), vf1 = stream_frag<float, 4>(vp + half);
    const Frag<TG, 4> gf0 = stream_frag<TG, 4>(gp), gf1 = stream_frag<TG, 4>(gp + half);
    TO *op = reinterpret_cast<TO *>(a.out) + (int64_t)t * a.out_tok + (int64_t)h * dim + c * 4;
    float v0[4], v1[4], g0[4], g1[4];
    unpack(vf0, v0);
    unpack(vf1, v1);
    unpack(gf0, g0);
    unpack(gf1, g1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v0[j] = v0[j] * sigmoid_ref(g0[j]);
        v1[j] = v1[j] * sigmoid_ref(g1[j]);
    }
    store_frag<4>(op, v0);
    store_frag<4>(op + half, v1);
}

template <typename TG, typename TO>
__global__ __launch_bounds__(kBlock) void gate_merge_general(Gate a) {
    const int64_t g = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (g >= a.total) return;
    const uint32_t th = fastdiv((uint32_t)g, a.chunks);
    const uint32_t r = (uint32_t)g - th * a.chunks.d;
    const uint32_t t = fastdiv(th, a.heads);
    const uint32_t h = th - t * a.heads.d;
    const uint32_t b = fastdiv(t, a.seq);
    const uint32_t s = t - b * a.seq.d;
    const int64_t dim = a.chunks.d;
    const float v = a.values[(((int64_t)b * a.heads.d + h) * a.seq.d + s) * dim + r];
    const float gv = to_f32(reinterpret_cast<const TG *>(
        a.gate)[(int64_t)t * a.gate_tok + (int64_t)h * a.gate_head + r]);
    put_elem(reinterpret_cast<TO *>(a.out), (int64_t)t * a.out_tok + (int64_t)h * dim + r,
             v * sigmoid_ref(gv));
}

}  // namespace
}  // namespace qdc

using namespace qdc;

extern "C" int32_t qdc_attention_softmax(void *probs, int32_t probs_dtype, const float *scores,
                                         const int32_t *mask, int64_t batch, int64_t heads,
                                         int64_t queries, int64_t keys, int64_t q_offset,
                                         float scale, hipStream_t stream) {
    if (!valid_dtype(probs_dtype)) return QDC_ERR_DTYPE;
    if (batch < 0 || heads < 0 || queries < 0 || keys < 0 || q_offset < 0) return QDC_ERR_SHAPE;
    const int64_t rows = batch * heads * queries;
    if (rows == 0 || keys == 0) return QDC_OK;
    // one wavefront per row: rows * 64 work-items must stay below 2^32
    if (rows >= ((int64_t)1 << 26) || keys >= ((int64_t)1 << 31)) return QDC_ERR_SHAPE;
    if (!probs || !scores) return QDC_ERR_NULL;
    const int64_t out_bytes = rows * keys * elem_size(probs_dtype);
    const int64_t in_bytes = rows * keys * 4;
    // in place only as the same fp32 buffer; a mask must not be written either
    if (!(probs == (const void *)scores && probs_dtype == QDC_F32) &&
        overlaps(probs, out_bytes, scores, in_bytes))
        return QDC_ERR_ALIAS;
    if (mask && overlaps(probs, out_bytes, mask, batch * keys * 4)) return QDC_ERR_ALIAS;
    Softmax a{};
    a.scores = scores;
    a.probs = probs;
    a.mask = mask;
    a.rows = rows;
    a.keys = keys;
    a.queries = make_fastdiv((uint32_t)queries);
    a.per_batch = make_fastdiv((uint32_t)(heads * queries));
    a.q_offset = q_offset;
    a.scale = scale;
    const dim3 grid((uint32_t)ceil_div(rows, kBlock / kWave));
    const int64_t chunks = ceil_div(keys, 4 * kWave);  // chunks of 4 keys per lane
    // wavefronts per row beyond one: each keeps at most kMaxRowChunks chunks per lane;
    // the grid's work-items (rows * wpr * 64) stay below 2^32
    int64_t wpr = 1;
    while (wpr < kMaxRowWaves && chunks > wpr * kMaxRowChunks) wpr *= 2;
    const bool fast = keys % 4 == 0 && aligned16(scores) && aligned16(probs) &&
                      (!mask || aligned16(mask)) && chunks <= wpr * kMaxRowChunks &&
                      rows * wpr < ((int64_t)1 << 26);
#define QDC_SM(TO, CPL)                                                                      \
    hipLaunchKernelGGL((softmax_rows_fast<TO, CPL>), grid, dim3(kBlock), 0, stream, a);     \
    return launch_status();
#define QDC_SMW(TO, W)                                                                       \
    if (wpr == W) {                                                                          \
        constexpr int64_t nw = W > 4 ? W : kBlock / kWave;                                   \
        hipLaunchKernelGGL((softmax_rows_waves<TO, kMaxRowChunks, W>),                      \
                           dim3((uint32_t)ceil_div(rows, nw / W)), dim3(nw * kWave), 0,      \
                           stream, a);                                                       \
        return launch_status();                                                              \
    }
#define QDC_SM_ALL(TO)                                                                       \
    if (fast) {                                                                              \
        if (chunks <= 1) { QDC_SM(TO, 1) }                                                   \
        if (chunks <= 2) { QDC_SM(TO, 2) }                                                   \
        if (chunks <= 4) { QDC_SM(TO, 4) }                                                   \
        if (chunks <= 8) { QDC_SM(TO, 8) }                                                   \
        QDC_SMW(TO, 2)                                                                       \
        QDC_SMW(TO, 4)                                                                       \
        QDC_SMW(TO, 8)                                                                       \
        QDC_SMW(TO, 16)                                                                      \
    }                                                                                        \
    hipLaunchKernelGGL((softmax_rows_general<TO>), grid, dim3(kBlock), 0, stream, a);       \
    return launch_status();
    if (probs_dtype == QDC_BF16) { QDC_SM_ALL(bf16_t) }
    QDC_SM_ALL(float)
#undef QDC_SM_ALL
#undef QDC_SMW
#undef QDC_SM
}

extern "C" int32_t qdc_attention_gate(void *out, int32_t out_dtype, const float *values,
                                      const void *gate, int32_t gate_dtype, int64_t batch,
                                      int64_t seq, int64_t heads, int64_t head_dim,
                                      int64_t gate_tok, int64_t gate_head, int64_t out_tok,
                                      hipStream_t stream) {
    const bool split = out_dtype == QDC_BF16X2;
    if (!(valid_dtype(out_dtype) || split) || !valid_dtype(gate_dtype)) return QDC_ERR_DTYPE;
    if (batch < 0 || seq < 0 || heads <= 0 || head_dim <= 0) return QDC_ERR_SHAPE;
    if (split && !split_rows_ok(head_dim, out_tok)) return QDC_ERR_SHAPE;
    const int64_t tokens = batch * seq;
    if (tokens == 0) return QDC_OK;
    if (gate_head < head_dim || gate_tok < (heads - 1) * gate_head + head_dim ||
        out_tok < heads * head_dim)
        return QDC_ERR_SHAPE;
    const int64_t elems = tokens * heads * head_dim;
    if (elems >= ((int64_t)1 << 31)) return QDC_ERR_SHAPE;
    if (!out || !values || !gate) return QDC_ERR_NULL;
    const int64_t out_bytes = ((tokens - 1) * out_tok + heads * head_dim) * elem_size(out_dtype);
    const int64_t gate_bytes =
        ((tokens - 1) * gate_tok + (heads - 1) * gate_head + head_dim) * elem_size(gate_dtype);
    if (overlaps(out, out_bytes, values, elems * 4) || overlaps(out, out_bytes, gate, gate_bytes))
        return QDC_ERR_ALIAS;
    const int64_t eg = elem_size(gate_dtype), eo = elem_size(out_dtype);
    const bool fast = head_dim % 8 == 0 && aligned16(out) && aligned16(values) && aligned16(gate) &&
                      (gate_tok * eg) % 16 == 0 && (gate_head * eg) % 16 == 0 &&
                      (out_tok * eo) % 16 == 0;
    Gate a{};
    a.values = values;
    a.gate = gate;
    a.out = out;
    a.gate_tok = gate_tok;
    a.gate_head = gate_head;
    a.out_tok = out_tok;
    a.heads = make_fastdiv((uint32_t)heads);
    a.seq = make_fastdiv((uint32_t)seq);
    a.total = fast ? elems / 8 : elems;
    a.chunks = make_fastdiv((uint32_t)(fast ? head_dim / 8 : head_dim));
    const dim3 grid((uint32_t)ceil_div(a.total, kBlock));
#define QDC_GATE(TG, TO)                                                                      \
    if (fast)                                                                                 \
        hipLaunchKernelGGL((gate_merge_fast<TG, TO>), grid, dim3(kBlock), 0, stream, a);     \
    else                                                                                      \
        hipLaunchKernelGGL((gate_merge_general<TG, TO>), grid, dim3(kBlock), 0, stream, a);  \
    return launch_status();
    if (gate_dtype == QDC_BF16) {
        if (split) { QDC_GATE(bf16_t, split_t) }
        if (out_dtype == QDC_BF16) { QDC_GATE(bf16_t, bf16_t) }
        QDC_GATE(bf16_t, float)
    }
    if (split) { QDC_GATE(float, split_t) }
    if (out_dtype == QDC_BF16) { QDC_GATE(float, bf16_t) }
    QDC_GATE(float, float)
#undef QDC_GATE
}

// qdc_attention_prepare.hip -- the attention prologue of a full-attention
// layer in one launch: q and k normalised per head (zero-centred RMSNorm) and
// rotated (half-split partial RoPE), written straight into the layouts the two
// attention products read, and v moved into its head-major layout.
//
//   q_out [batch, heads, seq, dim]     rows of the Q.K^T product's left operand
//   k_out [batch, kv_heads, dim, seq]  K transposed: the product's right operand
//   v_out [batch, kv_heads, seq, dim]  the P.V product's right operand
//
// so both products run as plain batched GEMMs over (sequence, KV head) with
// the heads / kv_heads query heads of a KV head as one [group*seq, dim] block,
// without expanding K or V per query head and without layout copies.
//
// Fast path (16-byte aligned rows, dim/chunk = 2*LPR chunks with LPR a power of
// two in [4, 32], the rotary block inside the first chunk of each lane, seq a
// multiple of a chunk).  Workgroups take one of three roles:
//   Q rows:  the row groups of qdc_rope_rows.hpp (consecutive heads of a token).
//   K tiles: 64 tokens of one sequence and one KV head.  Each LPR-lane group
//            normalises and rotates 64 / (256 / LPR) token rows (per-row
//            positions), the tile is staged in LDS token-major with a row pitch
//            of dim*es + 4 bytes, and read back a column at a time: lane (d, k)
//            gathers tokens k*V .. k*V+V-1 of dimension d and stores them as one
//            16-byte piece, so every 8 (bf16) or 16 (fp32) lanes write one whole
//            128-byte line of a transposed row.  The 4-byte pad puts the 16-lane
//            row writes and the column reads on distinct banks.
//   V tiles: 16 tokens of one sequence and one KV head, copied into one
//            contiguous span of 16 * dim elements of the head-major output.
//            Small tiles: copying the V rows inside the K tiles (one workgroup per
//            64 tokens) measured 5.5% slower for the whole launch at 8 x 2048
//            tokens; 8-token tiles were 7% slower and 32-token tiles 1.5%.
// The three roles are dealt through the grid in proportion.
//
// General path (any alignment or shape): one wavefront per (token, head) row;
// the normalised rotary block is staged in LDS; K elements are written with the
// transposed stride, V copied element by element.
#include <algorithm>
#include <type_traits>

#include "qdc_common.hpp"
#include "qdc_rope_rows.hpp"

namespace qdc {
namespace {

constexpr int kTileTokens = 64;

template <typename T> struct PrepArgs {
    QKArgs<T> qk;  // qk.q: Q rows in, head-major rows out; rope tables, eps, dims
    const T *k_in, *v_in, *k_w;
    T *k_out, *v_out;
    int64_t k_in_tok, v_in_tok;
    int64_t batch, seq, kv_heads;
    int64_t tiles;                     // tiles of kTileTokens per sequence
    int64_t q_blocks, k_blocks, v_blocks;
    // role dealing (attention_prepare_fast): Q blocks over the first nq blocks
    // at the rate rq / 2^32 per block, K tiles over the first mk non-Q blocks
    // at rk / 2^32, both ceil(count * 2^32 / span) so that exactly q_blocks
    // and k_blocks are dealt
    int64_t nq, mk;
    uint64_t rq, rk;
    FastDiv kv_div, tiles_div, vtiles_div;  // kv_heads, tiles, V tiles per sequence
};

// One K tile: tokens [s0, s0 + 64) of sequence b, KV head g.
template <typename T, int LPR>
__device__ __forceinline__ void k_tile(const PrepArgs<T> &a, int64_t index) {
    constexpr int V = Elem<T>::kVec;
    constexpr int ES = (int)sizeof(T);
    constexpr int DIM = 2 * LPR * V;
    constexpr int GPB = kBlock / LPR;                 // lane groups per workgroup
    constexpr int ROWS = kTileTokens / GPB;           // token rows per lane group
    constexpr int PITCH = DIM * ES + 4;               // bytes per token row in LDS
    static_assert(ROWS >= 1 && ROWS * GPB == kTileTokens, "tile rows");
    __shared__ __align__(16) unsigned char tile[kTileTokens * PITCH];

    const QKArgs<T> &qa = a.qk;
    const int lane = threadIdx.x % LPR, grp = threadIdx.x / LPR;
    const uint32_t bt = fastdiv((uint32_t)index, a.kv_div);
    const int64_t g = (uint32_t)index - bt * a.kv_div.d;
    const uint32_t b32 = fastdiv(bt, a.tiles_div);
    const int64_t b = b32, s0 = (int64_t)(bt - b32 * a.tiles_div.d) * kTileTokens;
    const int hc = qa.half / V;
    const bool rotary = lane < 2 * hc;
    const bool first = lane < hc;
    const int c0 = lane, c1 = lane + LPR;
    const int pc = lane ^ hc;

    // the K rows first (HBM); each row's cos/sin (L2-resident tables) just
    // before its rotation
    u32x4 x0[ROWS], x1[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        x0[r] = x1[r] = u32x4{0u, 0u, 0u, 0u};
        const int64_t s = s0 + grp + GPB * r;
        if (s < a.seq) {
            const T *src = a.k_in + (b * a.seq + s) * a.k_in_tok + g * DIM;
            x0[r] = load_stream(src + c0 * V);
            x1[r] = load_stream(src + c1 * V);
        }
    }
    const u32x4 w0 = load_raw(a.k_w + c0 * V), w1 = load_raw(a.k_w + c1 * V);
    const u32x4 wp = load_raw(a.k_w + (rotary ? pc : c0) * V);
    u32x4 xp[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) xp[r][e] = (uint32_t)__shfl_xor((int)x0[r][e], hc, kWave);

    float ss[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        float v0[V], v1[V];
        unpack(x0[r], v0);
        unpack(x1[r], v1);
        ss[r] = 0.0f;
#pragma unroll
        for (int j = 0; j < V; ++j) ss[r] += v0[j] * v0[j];
#pragma unroll
        for (int j = 0; j < V; ++j) ss[r] += v1[j] * v1[j];
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) ss[r] = group_sum<LPR>(ss[r]);
    float wv0[V], wv1[V], wvp[V];
    unpack(w0, wv0);
    unpack(w1, wv1);
    unpack(wp, wvp);
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        float v0[V], v1[V];
        unpack(x0[r], v0);
        unpack(x1[r], v1);
        const float s = rms_scale(ss[r], (float)qa.dim, qa.eps);
#pragma unroll
        for (int j = 0; j < V; ++j) {
            v0[j] = (v0[j] * s) * (1.0f + wv0[j]);
            v1[j] = (v1[j] * s) * (1.0f + wv1[j]);
        }
        const int64_t tok = s0 + grp + GPB * r;
        if (rotary && tok < a.seq) {
            const int64_t i0 = (qa.pos_offset + tok) * qa.half + (lane & (hc - 1)) * V;
            u32x4 cr[V / 4], sr[V / 4];
#pragma unroll
            for (int q = 0; q < V / 4; ++q) {
                cr[q] = load_raw(qa.cos + i0 + 4 * q);
                sr[q] = load_raw(qa.sin + i0 + 4 * q);
            }
            float p[V];
            unpack(xp[r], p);
#pragma unroll
            for (int j = 0; j < V; ++j) p[j] = (p[j] * s) * (1.0f + wvp[j]);
#pragma unroll
            for (int q = 0; q < V / 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int j = 4 * q + e;
                    const float c = __uint_as_float(cr[q][e]), sn = __uint_as_float(sr[q][e]);
                    v0[j] = first ? v0[j] * c - p[j] * sn : v0[j] * c + p[j] * sn;
                }
        }
        // token row grp + GPB*r of the tile, token-major, 4-byte writes (the
        // pitch is 4-byte aligned only)
        unsigned char *row = tile + (grp + GPB * r) * PITCH;
        const u32x4 o0 = pack(v0), o1 = pack(v1);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            *reinterpret_cast<uint32_t *>(row + c0 * 16 + 4 * e) = o0[e];
            *reinterpret_cast<uint32_t *>(row + c1 * 16 + 4 * e) = o1[e];
        }
    }
    __syncthreads();
    // Transposed write: piece p = (dimension d, token block k) holds tokens
    // s0 + k*V .. s0 + k*V + V-1 of dimension d.  seq is a multiple of V, so a
    // piece is either wholly inside the sequence or wholly past its end.
    constexpr int KB = kTileTokens / V;  // token blocks per dimension
    T *out = a.k_out + (b * a.kv_heads + g) * (int64_t)DIM * a.seq + s0;
    for (int p = threadIdx.x; p < DIM * KB; p += kBlock) {
        const int d = p / KB, k = p - d * KB;
        if (s0 + k * V >= a.seq) continue;
        T vals[V];
#pragma unroll
        for (int j = 0; j < V; ++j)
            vals[j] = *reinterpret_cast<const T *>(tile + (k * V + j) * PITCH + d * ES);
        u32x4 piece;
        if constexpr (ES == 2) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                piece[e] = (uint32_t)vals[2 * e] | ((uint32_t)vals[2 * e + 1] << 16);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) piece[e] = __float_as_uint(vals[e]);
        }
        store_raw(out + (int64_t)d * a.seq + k * V, piece);
    }
}

// One V tile: kVTokens tokens of sequence b, KV head g; 16-byte chunks copied into the
// head-major rows (one contiguous span), kVTokens * CH / kBlock chunks per thread.
// A whole tile takes the unguarded form: with a guard per chunk the compiler put
// each load in a branch of its own and waited for it before the next store
// (the launch 2% slower at 8 x 2048 tokens; 32-token tiles unguarded measured the
// same as 16, 8-token tiles 4% slower).
constexpr int kVTokens = 16;
template <typename T, int LPR>
__device__ __forceinline__ void v_tile(const PrepArgs<T> &a, int64_t index) {
    constexpr int V = Elem<T>::kVec;
    constexpr int CH = 2 * LPR;
    constexpr int DIM = CH * V;
    constexpr int PER = (kVTokens * CH + kBlock - 1) / kBlock;
    const uint32_t bt = fastdiv((uint32_t)index, a.kv_div);
    const int64_t g = (uint32_t)index - bt * a.kv_div.d;
    const uint32_t b32 = fastdiv(bt, a.vtiles_div);
    const int64_t b = b32, s0 = (int64_t)(bt - b32 * a.vtiles_div.d) * kVTokens;
    const int64_t rows = std::min<int64_t>(kVTokens, a.seq - s0);
    T *out = a.v_out + ((b * a.kv_heads + g) * a.seq + s0) * DIM;
    const T *in = a.v_in + (b * a.seq + s0) * a.v_in_tok + g * DIM;
    u32x4 r[PER];
    if (rows == kVTokens && (kVTokens * CH) % kBlock == 0) {  // a whole tile: no guards
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int p = threadIdx.x + u * kBlock;
            r[u] = load_stream(in + (int64_t)(p / CH) * a.v_in_tok + (p % CH) * V);
        }
#pragma unroll
        for (int u = 0; u < PER; ++u) store_raw(out + (int64_t)(threadIdx.x + u * kBlock) * V, r[u]);
        return;
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int p = threadIdx.x + u * kBlock;
        if (p < rows * CH) r[u] = load_stream(in + (int64_t)(p / CH) * a.v_in_tok + (p % CH) * V);
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int p = threadIdx.x + u * kBlock;
        if (p < rows * CH) store_raw(out + (int64_t)p * V, r[u]);
    }
}

// Q, K and V workgroups are dealt through the grid in proportion: the count of
// Q blocks among blocks [0, i] is f(i) = floor((i+1) * rq / 2^32) over the
// first nq = 9n/10 blocks, and block i is a Q block when f(i) > f(i-1); the
// other blocks split between K and V the same way, the K tiles over the first
// 3/4 of them.  So every role streams from the first wave of workgroups, the
// long K tiles finish early and the short V tiles fill the launch's tail.  The
// rates are fixed-point multipliers computed on the host, and the K/V tile
// indices split with multiply-high divisions: the 64-bit divisions they replace
// (about a hundred scalar instructions each before a workgroup's first load)
// cost 1-2% of the launch at 8 x 2048 tokens.
template <typename T, int LPR, int RPGQ>
__global__ __launch_bounds__(kBlock) void attention_prepare_fast(PrepArgs<T> a) {
    // Q blocks over the first 9/10 of the grid, so the last stretch holds
    // only V tiles, the shortest workgroups (2-3% faster at 8 x 2048 tokens
    // than over the whole grid; 8/10 no better)
    const uint64_t i = blockIdx.x;
    const bool in_q = i < (uint64_t)a.nq;
    const int64_t q_upto = in_q ? (int64_t)(((i + 1) * a.rq) >> 32) : a.q_blocks;  // Q among [0, i]
    if (in_q && q_upto > (int64_t)((i * a.rq) >> 32)) {
        qk_side_contig<T, LPR, RPGQ>(a.qk, a.qk.q, q_upto - 1);
        return;
    }
    // K tiles, the longest workgroups, are dealt over the first 3/4 of the
    // non-Q blocks only, so none starts in the launch's last stretch (2-3%
    // faster at 8 x 2048 tokens than dealing them over all, 1/4-5/8 in between)
    const uint64_t j = i - (uint64_t)q_upto;
    const bool in_k = j < (uint64_t)a.mk;
    const int64_t k_upto = in_k ? (int64_t)(((j + 1) * a.rk) >> 32) : a.k_blocks;  // K among [0, j]
    if (in_k && k_upto > (int64_t)((j * a.rk) >> 32))
        k_tile<T, LPR>(a, k_upto - 1);
    else
        v_tile<T, LPR>(a, (int64_t)j - k_upto);
}

// General path: one wavefront per row; rows [0, tokens*heads) are Q, then
// tokens*kv_heads K rows, then tokens*kv_heads V rows.
constexpr int kMaxPrepareRotary = 1024;

template <typename T> struct GeneralPrep {
    const T *q_in, *k_in, *v_in, *q_w, *k_w;
    T *q_out, *k_out, *v_out;
    const float *cos, *sin;
    int64_t q_in_tok, q_in_head, k_in_tok, v_in_tok;
    int64_t seq, heads, kv_heads, dim, half, pos_offset, tokens;
    float eps;
};

template <typename T>
__global__ __launch_bounds__(kBlock) void attention_prepare_general(GeneralPrep<T> a) {
    __shared__ float staged[kBlock / kWave][kMaxPrepareRotary];
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int64_t row = (int64_t)blockIdx.x * (kBlock / kWave) + wave;
    const int64_t nq = a.tokens * a.heads, nk = a.tokens * a.kv_heads;
    float *st = staged[wave];
    const int64_t dim = a.dim, half = a.half;
    // role of this wavefront's row (uniform per wavefront): Q or K rows are
    // normalised and rotated, V rows copied; every wavefront reaches the barrier
    const bool is_v = row >= nq + nk && row < nq + 2 * nk;
    const bool is_qk = row < nq + nk;
    const bool is_k = is_qk && row >= nq;
    if (is_v) {  // copy into [b, g, s, :]
        const int64_t r = row - nq - nk, t = r / a.kv_heads, g = r - t * a.kv_heads;
        const int64_t b = t / a.seq, s = t - b * a.seq;
        const T *in = a.v_in + t * a.v_in_tok + g * dim;
        T *out = a.v_out + ((b * a.kv_heads + g) * a.seq + s) * dim;
        for (int64_t i = lane; i < dim; i += kWave) out[i] = in[i];
    }
    const T *in = nullptr, *w = nullptr;
    T *out = nullptr;
    int64_t es = 1, pos = 0;
    float sc = 0.0f;
    if (is_qk) {
        const int64_t r = is_k ? row - nq : row;
        const int64_t nh = is_k ? a.kv_heads : a.heads;
        const int64_t t = r / nh, h = r - t * nh;
        const int64_t b = t / a.seq, s = t - b * a.seq;
        in = is_k ? a.k_in + t * a.k_in_tok + h * dim : a.q_in + t * a.q_in_tok + h * a.q_in_head;
        w = is_k ? a.k_w : a.q_w;
        // q: [b, h, s, :] with unit element stride; k: [b, h, :, s] with stride seq
        out = is_k ? a.k_out + (b * a.kv_heads + h) * dim * a.seq + s
                   : a.q_out + ((b * a.heads + h) * a.seq + s) * dim;
        es = is_k ? a.seq : 1;
        pos = a.pos_offset + s;
        float ss = 0.0f;
        for (int64_t i = lane; i < dim; i += kWave) {
            const float v = to_f32(in[i]);
            ss += v * v;
        }
        ss = group_sum<kWave>(ss);
        sc = rms_scale(ss, (float)dim, a.eps);
        for (int64_t i = lane; i < 2 * half; i += kWave)
            st[i] = (to_f32(in[i]) * sc) * (1.0f + to_f32(w[i]));
    }
    __syncthreads();
    if (!is_qk) return;
    for (int64_t i = lane; i < dim; i += kWave) {
        float o;
        if (i < half) {
            const float c = a.cos[pos * half + i], sn = a.sin[pos * half + i];
            o = st[i] * c - st[i + half] * sn;
        } else if (i < 2 * half) {
            const float c = a.cos[pos * half + i - half], sn = a.sin[pos * half + i - half];
            o = st[i] * c + st[i - half] * sn;
        } else {
            o = (to_f32(in[i]) * sc) * (1.0f + to_f32(w[i]));
        }
        out[i * es] = from_f32<T>(o);
    }
}

template <typename T, int LPR, int RPGQ>
int32_t launch_fast(PrepArgs<T> a, hipStream_t stream) {
    constexpr int64_t gpb = kBlock / LPR;
    a.q_blocks = ceil_div(a.qk.q.rows / RPGQ, gpb);
    a.k_blocks = a.batch * a.tiles * a.kv_heads;
    const int64_t vtiles = (a.seq + kVTokens - 1) / kVTokens;
    a.v_blocks = a.batch * vtiles * a.kv_heads;
    const int64_t blocks = a.q_blocks + a.k_blocks + a.v_blocks;
    // fixed-point dealing rates: ceil(count * 2^32 / span) <= 2^32, so the
    // count of a role among the first `span` blocks is exactly `count`
    // (span < 2^32) and it grows by at most one per block
    auto rate = [](int64_t count, int64_t span) {
        return span > 0 ? (((uint64_t)count << 32) + (uint64_t)span - 1) / (uint64_t)span : 0;
    };
    a.nq = std::max<int64_t>(a.q_blocks, blocks * 9 / 10);
    a.rq = rate(a.q_blocks, a.nq);
    const int64_t m = a.k_blocks + a.v_blocks;
    a.mk = std::max<int64_t>(a.k_blocks, m * 3 / 4);
    a.rk = rate(a.k_blocks, a.mk);
    a.kv_div = make_fastdiv((uint32_t)a.kv_heads);
    a.tiles_div = make_fastdiv((uint32_t)std::max<int64_t>(a.tiles, 1));
    a.vtiles_div = make_fastdiv((uint32_t)std::max<int64_t>(vtiles, 1));
    hipLaunchKernelGGL((attention_prepare_fast<T, LPR, RPGQ>), dim3((uint32_t)blocks),
                       dim3(kBlock), 0, stream, a);
    return launch_status();
}

template <typename T, int LPR>
int32_t launch_lpr(const PrepArgs<T> &a, int64_t heads, hipStream_t stream) {
    if (heads % 4 == 0) return launch_fast<T, LPR, 4>(a, stream);
    if (heads % 2 == 0) return launch_fast<T, LPR, 2>(a, stream);
    return launch_fast<T, LPR, 1>(a, stream);
}

int32_t prepare(void *q_out, void *k_out, void *v_out, const void *q_in, const void *k_in,
                const void *v_in, const void *q_norm, const void *k_norm, const float *cos_table,
                const float *sin_table, int64_t batch, int64_t seq, int64_t heads,
                int64_t kv_heads, int64_t dim, int64_t rotary_dim, int64_t pos_offset,
                int64_t table_len, int64_t q_in_tok, int64_t q_in_head, int64_t k_in_tok,
                int64_t v_in_tok, float eps, int32_t dtype, hipStream_t stream) {
    if (!valid_dtype(dtype)) return QDC_ERR_DTYPE;
    if (batch < 0 || seq < 0 || heads < 0 || kv_heads <= 0 || heads % kv_heads || dim <= 0 ||
        rotary_dim < 0 || rotary_dim % 2 || rotary_dim > dim || pos_offset < 0 || table_len < 0)
        return QDC_ERR_SHAPE;
    const int64_t tokens = batch * seq;
    // a wavefront per row in the general grid, below 2^32 work-items
    if (dim > INT32_MAX || tokens * (heads + 2 * kv_heads) >= ((int64_t)1 << 26))
        return QDC_ERR_SHAPE;
    if (tokens == 0) return QDC_OK;
    // heads == 0: K and V only (the q pointers are not used and may be NULL)
    if (!k_out || !v_out || !k_in || !v_in || !k_norm) return QDC_ERR_NULL;
    if (heads > 0 && (!q_out || !q_in || !q_norm)) return QDC_ERR_NULL;
    if (rotary_dim > 0) {
        if (!cos_table || !sin_table) return QDC_ERR_NULL;
        if (pos_offset + seq > table_len) return QDC_ERR_RANGE;
    }
    // input rows must not overlap (tokens and heads), strides non-negative
    if (q_in_tok < 0 || q_in_head < 0 || k_in_tok < 0 || v_in_tok < 0) return QDC_ERR_SHAPE;
    if ((heads > 1 && q_in_head < dim) ||
        (heads > 0 && tokens > 1 && q_in_tok < (heads - 1) * q_in_head + dim) ||
        (tokens > 1 && (k_in_tok < kv_heads * dim || v_in_tok < kv_heads * dim)))
        return QDC_ERR_SHAPE;
    const int64_t es = elem_size(dtype);
    const int64_t q_bytes = tokens * heads * dim * es, kv_bytes = tokens * kv_heads * dim * es;
    const int64_t qi_bytes =
        heads > 0 ? ((tokens - 1) * q_in_tok + (heads - 1) * q_in_head + dim) * es : 0;
    const int64_t ki_bytes = ((tokens - 1) * k_in_tok + kv_heads * dim) * es;
    const int64_t vi_bytes = ((tokens - 1) * v_in_tok + kv_heads * dim) * es;
    const struct { const void *p; int64_t n; } outs[3] = {{q_out, q_bytes}, {k_out, kv_bytes},
                                                         {v_out, kv_bytes}},
                                              ins[3] = {{q_in, qi_bytes}, {k_in, ki_bytes},
                                                        {v_in, vi_bytes}};
    for (int i = 0; i < 3; ++i) {
        for (int j = 0; j < 3; ++j)
            if (overlaps(outs[i].p, outs[i].n, ins[j].p, ins[j].n)) return QDC_ERR_ALIAS;
        for (int j = i + 1; j < 3; ++j)
            if (overlaps(outs[i].p, outs[i].n, outs[j].p, outs[j].n)) return QDC_ERR_ALIAS;
    }

    auto fill = [&](auto *tag) -> int32_t {
        using T = std::remove_pointer_t<decltype(tag)>;
        constexpr int V = Elem<T>::kVec;
        const int64_t half = rotary_dim / 2;
        const int64_t chunks = dim / V, lpr = chunks / 2, hc = half / V;
        const bool fast =
            dim % V == 0 && chunks % 2 == 0 && lpr >= 4 && lpr <= 32 && (lpr & (lpr - 1)) == 0 &&
            half % V == 0 && 2 * hc <= lpr && (hc & (hc - 1)) == 0 && seq % V == 0 &&
            aligned16(q_out) && aligned16(k_out) && aligned16(v_out) && aligned16(q_in) &&
            aligned16(k_in) && aligned16(v_in) && aligned16(q_norm) && aligned16(k_norm) &&
            (rotary_dim == 0 || (aligned16(cos_table) && aligned16(sin_table))) &&
            ((q_in_tok | q_in_head | k_in_tok | v_in_tok) * es) % 16 == 0;
        if (fast) {
            PrepArgs<T> a{};
            a.qk.q = Side<T>{(const T *)q_in, (T *)q_out, (const T *)q_norm, q_in_tok, q_in_head,
                             dim, seq * dim, heads * seq * dim, tokens * heads,
                             make_fastdiv((uint32_t)std::max<int64_t>(heads, 1))};
            a.qk.cos = cos_table;
            a.qk.sin = sin_table;
            a.qk.seq_len = make_fastdiv((uint32_t)seq);
            a.qk.pos_offset = pos_offset;
            a.qk.half = (int32_t)half;
            a.qk.dim = (int32_t)dim;
            a.qk.eps = eps;
            a.k_in = (const T *)k_in;
            a.v_in = (const T *)v_in;
            a.k_w = (const T *)k_norm;
            a.k_out = (T *)k_out;
            a.v_out = (T *)v_out;
            a.k_in_tok = k_in_tok;
            a.v_in_tok = v_in_tok;
            a.batch = batch;
            a.seq = seq;
            a.kv_heads = kv_heads;
            a.tiles = ceil_div(seq, kTileTokens);
            switch (lpr) {
                case 4: return launch_lpr<T, 4>(a, heads, stream);
                case 8: return launch_lpr<T, 8>(a, heads, stream);
                case 16: return launch_lpr<T, 16>(a, heads, stream);
                case 32: return launch_lpr<T, 32>(a, heads, stream);
                default: break;
            }
        }
        if (rotary_dim > kMaxPrepareRotary) return QDC_ERR_SHAPE;
        GeneralPrep<T> gp{(const T *)q_in, (const T *)k_in, (const T *)v_in, (const T *)q_norm,
                          (const T *)k_norm, (T *)q_out, (T *)k_out, (T *)v_out, cos_table,
                          sin_table, q_in_tok, q_in_head, k_in_tok, v_in_tok, seq, heads,
                          kv_heads, dim, half, pos_offset, tokens, eps};
        const int64_t rows = tokens * (heads + 2 * kv_heads);
        hipLaunchKernelGGL((attention_prepare_general<T>),
                           dim3((uint32_t)ceil_div(rows, kBlock / kWave)), dim3(kBlock), 0,
                           stream, gp);
        return launch_status();
    };
    if (dtype == QDC_BF16) return fill((bf16_t *)nullptr);
    return fill((float *)nullptr);
}

}  // namespace
}  // namespace qdc

using namespace qdc;

extern "C" int32_t qdc_attention_prepare(void *q_out, void *k_out, void *v_out, const void *q_in,
                                         const void *k_in, const void *v_in, const void *q_norm,
                                         const void *k_norm, const float *cos_table,
                                         const float *sin_table, int64_t batch, int64_t seq_len,
                                         int64_t heads, int64_t kv_heads, int64_t head_dim,
                                         int64_t rotary_dim, int64_t pos_offset, int64_t table_len,
                                         int64_t q_in_tok, int64_t q_in_head, int64_t k_in_tok,
                                         int64_t v_in_tok, float eps, int32_t dtype,
                                         hipStream_t stream) {
    return prepare(q_out, k_out, v_out, q_in, k_in, v_in, q_norm, k_norm, cos_table, sin_table,
                   batch, seq_len, heads, kv_heads, head_dim, rotary_dim, pos_offset, table_len,
                   q_in_tok, q_in_head, k_in_tok, v_in_tok, eps, dtype, stream);
}

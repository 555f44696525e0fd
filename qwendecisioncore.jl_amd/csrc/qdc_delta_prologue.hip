// qdc_delta_prologue.hip -- the DeltaNet prologue row work in one pass over the
// packed projection [qkv | z | a | b] (one row per token; the launch grid keeps
// blocks x work-items per dimension below 2^32, so tokens < 2^26):
//   mixed  = silu(causal depthwise conv of the qkv block, K taps, per sequence)
//   q      = mixed_q / (sqrt(sum(mixed_q^2) + 1e-6) * sqrt(key_dim))   per key head
//   k      = mixed_k /  sqrt(sum(mixed_k^2) + 1e-6)                     per key head
//   v      = mixed_v
//   beta   = sigmoid(b);  decay = a_decay * softplus(a + dt_bias)       per value head
// Reference: causal_depthwise src/backbone.jl:264-276 (CPU four-tap form
// src/backbone_cpu.jl:787-809, same tap order), cpu_normalize_delta_heads!
// src/backbone_cpu.jl:411-427, cpu_delta_prepare src/backbone_cpu.jl:501-533,
// gates src/backbone.jl:293-296; AMDGPU causal_depthwise_kernel! /
// qk_normalize_kernel! and the beta/decay broadcasts, ext/amdgpu_delta.jl:1-33, 83-113, 154-159.
//
// Fast path: a thread owns 4 consecutive channels for a tile of 12 (bf16) or 8
// (fp32) consecutive tokens (4 in short launches), loads the tile's rows and the K-1 halo rows before
// it in one go (branch-free, so each token waits only for its own rows), then
// slides a K-tap window down the tile, so each projection row is read once
// from HBM (the halo rows again from a cache: tiles are dealt to the XCDs in
// runs of two) and each output chunk is one whole 16-byte store.  The kd/4 lanes of a key head are an aligned lane group,
// so the L2 norm reduces inside the group.  Outputs are fp32
// (the recurrence reads fp32).  Blocks of 32 tokens after the channel blocks
// compute the gates.
#include <cmath>
#include <type_traits>

#include "qdc_common.hpp"

namespace qdc {
namespace {

constexpr int kTaps = 4;    // fast-path convolution width (the Qwen3.5 default)

struct Prologue {
    const void *proj;
    int64_t ld;             // elements between token rows of proj
    int64_t a_off, b_off;   // columns of the a and b blocks
    const float *conv;      // [channels, taps]
    const float *a_decay, *dt_bias;
    float *q, *k, *v, *beta, *decay;
    int64_t ld_qk, ld_v;    // elements between the token rows of q and k, and of v
    int64_t tokens;
    FastDiv seq;            // sequence length (positions reset per sequence)
    int kh, kd, vh, vd, taps;
    int chunks;             // qkv channels / 4
    int qk_chunks;          // 2*kh*kd / 4
    uint32_t blocks_per_tile;  // fast path: channel blocks per tile
    uint32_t chan_blocks;      // fast path: channel workgroups (tiles padded to whole XCD runs)
                               // x blocks_per_tile; the gates blocks follow
    uint32_t tiles;            // fast path: tiles of the launch
    float sqrt_kd, inv_sqrt_kd;
};

__device__ __forceinline__ float sigmoid_f(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}
__device__ __forceinline__ float softplus_f(float x) {
    return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
}

// A thread owns 4 channels: 8 bytes of a bf16 (16 of an fp32) projection row
// and exactly one 16-byte fp32 output chunk, so every load and store
// instruction of a wavefront covers whole cache lines.  Tokens per thread: the
// tile's rows plus the kTaps-1 halo rows are all loaded before the first is used.
// bf16 tiles of 12 tokens (84 VGPRs, 5 waves per SIMD) measured fastest at the
// 0.8B shapes once the row loads were branch-free: 108.3 us against 108.4-109.9
// for 8-14 tokens, 110.6-111.3 for 16-20, 113.7 for 24 and 119.2 for 40 (and,
// with the XCD runs below, 4 and 6 tokens 123.5 and 111.0 against 106.9; 40 was
// the best of 8-64 while each row load sat in a branch of its own and the first
// token waited for the whole tile); fp32 tiles of 8 tokens: 143.4 us against
// 145.4 for 12 and 149.4 for 16 at 16384 tokens, 22.8 against 23.6 and 23.9 at
// 2048.  The halo rows (3 per tile) come from L2 or the last-level cache.
template <typename T> constexpr int tile_for() { return sizeof(T) == 2 ? 12 : 8; }
// Short launches (a single sequence of a few hundred tokens) take tiles of 4
// tokens: more workgroups on the chip and a 4-step chain per thread instead of
// 40 (the 3 halo rows per tile come from L2).  Each token's arithmetic is the
// same in either tile, so the outputs are bit-identical.
constexpr int kSmallTile = 4;
// Tokens per gates block.  The gates (beta, decay: 2 heads-wide columns in,
// 2 out per token) take their own blocks at the end of the grid instead of one
// block beside each tile's channel blocks: 3-4% faster at 2048 tokens and
// 0.5-1% at 16384 (0.8B dims), 20% at 2048 tokens of the 2-key-head synthetic
// dims, where the per-tile gates block was every other workgroup; 16-64 tokens
// measured alike, 128 slower (longer tail).
constexpr int kGateTokens = 32;
// Consecutive tiles per XCD run.  Runs of 2 halve the halo rows fetched into
// L2 from outside (read traffic 1.13x instead of 1.26x the algorithmic reads
// at 16384 tokens, 0.8B dims) at the same time in bf16 (2% faster in fp32);
// runs of 4 and 8 measured 1.5% and 3.5% slower in bf16.  Leaving the halo rows
// out altogether (a probe: zeros instead of loads) changed the time by under
// 0.3%: those L2 fills hit the last-level cache, they cost counted traffic,
// not time.
constexpr uint32_t kXcdRun = 2;

template <typename T> struct Raw4;  // 4 channels of one projection row
template <> struct Raw4<bf16_t> {
    typedef uint32_t type __attribute__((ext_vector_type(2)));
    static __device__ __forceinline__ void unpack(type r, float (&v)[4]) {
        v[0] = __uint_as_float(r[0] << 16); v[1] = __uint_as_float(r[0] & 0xffff0000u);
        v[2] = __uint_as_float(r[1] << 16); v[3] = __uint_as_float(r[1] & 0xffff0000u);
    }
};
template <> struct Raw4<float> {
    typedef u32x4 type;
    static __device__ __forceinline__ void unpack(type r, float (&v)[4]) {
        v[0] = __uint_as_float(r[0]); v[1] = __uint_as_float(r[1]);
        v[2] = __uint_as_float(r[2]); v[3] = __uint_as_float(r[3]);
    }
};

template <typename T, int LPH, int kTileT>
__global__ __launch_bounds__(kBlock) void delta_prologue_fast(Prologue a) {
    using Raw = typename Raw4<T>::type;
    constexpr int kRows = kTileT + kTaps - 1;  // rows t0-3 .. t0+tile-1
    // One-dimensional grid: the channel workgroups, then the gates blocks,
    // kGateTokens tokens each.
    if (blockIdx.x >= a.chan_blocks) {
        const int64_t g0 = (int64_t)(blockIdx.x - a.chan_blocks) * kGateTokens;
        for (int i = threadIdx.x; i < kGateTokens * a.vh; i += kBlock) {
            const int64_t t = g0 + i / a.vh;
            const int h = i % a.vh;
            if (t >= a.tokens) continue;
            const T *row = reinterpret_cast<const T *>(a.proj) + t * a.ld;
            const float bv = to_f32(row[a.b_off + h]);
            const float av = to_f32(row[a.a_off + h]);
            a.beta[t * a.vh + h] = sigmoid_f(bv);
            a.decay[t * a.vh + h] = a.a_decay[h] * softplus_f(av + a.dt_bias[h]);
        }
        return;
    }
    // Workgroup i runs on XCD i % 8 (the hardware deals workgroups round-robin
    // over the 8 XCDs).  XCD x takes runs of kXcdRun consecutive tiles, each
    // tile's channel blocks in a row, so the later tiles of a run find their
    // halo rows in this XCD's L2, loaded there by the tile before.
    const uint32_t nblk = a.blocks_per_tile;
    const uint32_t x = blockIdx.x & 7u, slot = blockIdx.x >> 3;
    const uint32_t per_run = kXcdRun * nblk;
    const uint32_t run = slot / per_run, r = slot - run * per_run;
    const uint32_t tile = (run * 8u + x) * kXcdRun + r / nblk, cblk = r % nblk;
    if (tile >= a.tiles) return;  // padding of the last runs
    const int64_t t0 = (int64_t)tile * kTileT;
    const int ci = cblk * kBlock + threadIdx.x;  // quad of 4 channels
    const bool live = ci < a.chunks;
    const int c0 = (live ? ci : 0) * 4;
    const bool is_q = ci < a.qk_chunks / 2, is_k = !is_q && ci < a.qk_chunks;
    // q and k heads are whole aligned lane groups and 2*kh*kd is a multiple of
    // 64 channels in practice, so is_qk is normally uniform per wavefront
    const bool is_qk = is_q || is_k;

    // position of t0 in its sequence; rows before that sequence's start are zero
    // for every token of the tile
    const uint32_t s0 = (uint32_t)t0 - fastdiv((uint32_t)t0, a.seq) * a.seq.d;
    const int64_t seq_start = t0 - s0;
    // The conv weights first (the first token needs them), then the rows, every
    // load unconditional so that none sits in a branch of its own and each
    // token waits only for its own rows.  Row addresses are clamped into the
    // launch (rows past the last token feed only tokens that are not stored);
    // the kTaps-1 halo rows before a sequence start are zeroed; a lane past the
    // last channel reads channel 0 and stores nothing.
    float w[4][kTaps];
    {
        const u32x4 *cw = reinterpret_cast<const u32x4 *>(a.conv + (int64_t)c0 * kTaps);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const u32x4 q = cw[c];
#pragma unroll
            for (int j = 0; j < kTaps; ++j) w[c][j] = __uint_as_float(q[j]);
        }
    }
    Raw rows[kRows];
    {
        const T *proj = reinterpret_cast<const T *>(a.proj) + c0;
        const int64_t first = t0 - (kTaps - 1);
        if (first >= 0 && t0 + kTileT <= a.tokens) {  // tile-uniform: every row exists
            const T *p = proj + first * a.ld;
#pragma unroll
            for (int r = 0; r < kRows; ++r, p += a.ld) rows[r] = *reinterpret_cast<const Raw *>(p);
        } else {
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                const int64_t t = first + r;
                const int64_t tc = t < 0 ? 0 : (t >= a.tokens ? a.tokens - 1 : t);
                rows[r] = *reinterpret_cast<const Raw *>(proj + tc * a.ld);
            }
        }
#pragma unroll
        for (int r = 0; r < kTaps - 1; ++r) {  // halo rows before the sequence start
            const uint32_t keep = first + r >= seq_start ? 0xffffffffu : 0u;
            rows[r] = rows[r] & keep;
        }
    }

    const int64_t kw = (int64_t)a.kh * a.kd;
    // this thread's output chunk of token t0 and the stride between tokens
    const int64_t dstride = is_qk ? a.ld_qk : a.ld_v;
    float *dst = (is_q ? a.q + c0 : is_k ? a.k + (c0 - kw) : a.v + (c0 - 2 * kw)) + t0 * dstride;
    const float qk_mul = is_q ? a.inv_sqrt_kd : 1.0f;
    // A later sequence starts inside the tile only when fewer than kTileT
    // positions remain in t0's sequence; only then do taps need a per-token mask.
    const bool inner_start = a.seq.d - s0 < (uint32_t)kTileT;
    auto run_tile = [&](auto masked) {
        // the window of unpacked rows t-3 .. t (row t - (kTaps-1) + j is tap j)
        float x[kTaps][4];
#pragma unroll
        for (int j = 0; j < kTaps - 1; ++j) Raw4<T>::unpack(rows[j], x[j + 1]);
        float *out = dst;
#pragma unroll
        for (int tt = 0; tt < kTileT; ++tt, out += dstride) {
#pragma unroll
            for (int j = 0; j < kTaps - 1; ++j)
#pragma unroll
                for (int c = 0; c < 4; ++c) x[j][c] = x[j + 1][c];
            Raw4<T>::unpack(rows[tt + kTaps - 1], x[kTaps - 1]);
            const int64_t t = t0 + tt;
            uint32_t s = 0;  // position of t in its sequence (masked tiles only)
            if constexpr (decltype(masked)::value)
                s = t < a.tokens ? (uint32_t)t - fastdiv((uint32_t)t, a.seq) * a.seq.d : 0u;
            float m[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                // tap j multiplies row t - (kTaps-1) + j; fused multiply-add per tap
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < kTaps; ++j) {
                    if constexpr (decltype(masked)::value) {
                        if (s >= (uint32_t)(kTaps - 1 - j)) acc = __builtin_fmaf(x[j][c], w[c][j], acc);
                    } else {
                        acc = __builtin_fmaf(x[j][c], w[c][j], acc);
                    }
                }
                m[c] = silu(acc);
            }
            if (is_qk) {  // L2 norm over the key head (an aligned group of LPH lanes)
                float ss = 0.0f;
#pragma unroll
                for (int c = 0; c < 4; ++c) ss = __builtin_fmaf(m[c], m[c], ss);
                ss = group_sum<LPH>(ss);
                // 1/(sqrt(ss + 1e-6) sqrt(kd)) for q, 1/sqrt(ss + 1e-6) for k, each
                // factor within an ulp or two of the correctly rounded one
                const float scale = __builtin_amdgcn_rsqf(ss + 1e-6f) * qk_mul;
#pragma unroll
                for (int c = 0; c < 4; ++c) m[c] = m[c] * scale;
            }
            if (live && t < a.tokens) store_chunk(out, m);
        }
    };
    if (!inner_start) run_tile(std::false_type{});
    else run_tile(std::true_type{});
}

// One wavefront per (token, segment); segments: q heads, k heads, the v block, the gates.
template <typename T>
__global__ __launch_bounds__(kBlock) void delta_prologue_general(Prologue a) {
    const int lane = threadIdx.x % kWave;
    const int64_t t = (int64_t)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (t >= a.tokens) return;  // uniform per wavefront
    const int seg = blockIdx.y;
    const T *proj = reinterpret_cast<const T *>(a.proj);
    const uint32_t s = (uint32_t)t - fastdiv((uint32_t)t, a.seq) * a.seq.d;
    const int64_t kw = (int64_t)a.kh * a.kd, vw = (int64_t)a.vh * a.vd;
    auto conv_silu = [&](int64_t c) {
        float acc = 0.0f;
        for (int j = 0; j < a.taps; ++j) {
            const int lag = a.taps - 1 - j;
            if ((int64_t)s >= lag) acc = acc + to_f32(proj[(t - lag) * a.ld + c]) * a.conv[c * a.taps + j];
        }
        return silu(acc);
    };
    if (seg < 2 * a.kh) {  // a q or k head
        const bool is_q = seg < a.kh;
        const int64_t c0 = (int64_t)seg * a.kd;
        float *dst = is_q ? a.q + t * a.ld_qk + c0 : a.k + t * a.ld_qk + (c0 - kw);
        float ss = 0.0f;
        for (int i = lane; i < a.kd; i += kWave) {
            const float m = conv_silu(c0 + i);
            dst[i] = m;
            ss += m * m;
        }
        ss = group_sum<kWave>(ss);
        const float scale = is_q ? 1.0f / (__builtin_sqrtf(ss + 1e-6f) * a.sqrt_kd)
                                 : 1.0f / __builtin_sqrtf(ss + 1e-6f);
        for (int i = lane; i < a.kd; i += kWave) dst[i] = dst[i] * scale;
    } else if (seg == 2 * a.kh) {  // the v block
        for (int64_t i = lane; i < vw; i += kWave) a.v[t * a.ld_v + i] = conv_silu(2 * kw + i);
    } else {  // gates
        for (int h = lane; h < a.vh; h += kWave) {
            a.beta[t * a.vh + h] = sigmoid_f(to_f32(proj[t * a.ld + a.b_off + h]));
            a.decay[t * a.vh + h] =
                a.a_decay[h] * softplus_f(to_f32(proj[t * a.ld + a.a_off + h]) + a.dt_bias[h]);
        }
    }
}

// An output of `width` floats per token row, rows `ld` floats apart.
struct OutRows {
    const float *p;
    int64_t width, ld;
    int64_t span(int64_t tokens) const { return ((tokens - 1) * ld + width) * 4; }
};

// Two outputs never write the same float: their spans do not overlap (separate
// buffers), or they share a row stride and are disjoint column blocks of the
// same rows (one [tokens, q|k|v] buffer).
bool disjoint_rows(const OutRows &a, const OutRows &b, int64_t tokens) {
    if (!overlaps(a.p, a.span(tokens), b.p, b.span(tokens))) return true;
    if (a.ld != b.ld) return false;
    const int64_t bytes = (const char *)b.p - (const char *)a.p;
    if (bytes % 4) return false;
    const int64_t d = ((bytes / 4) % a.ld + a.ld) % a.ld;  // b's column offset within a's rows
    return d >= a.width && d + b.width <= a.ld;
}

template <typename T, int TILE>
int32_t launch_fast(Prologue q, int lph, hipStream_t stream) {
    q.tiles = (uint32_t)ceil_div(q.tokens, TILE);
    q.chan_blocks = (uint32_t)(ceil_div(q.tiles, 8 * kXcdRun) * 8 * kXcdRun * q.blocks_per_tile);
    const int64_t blocks = (int64_t)q.chan_blocks + ceil_div(q.tokens, (int64_t)kGateTokens);
    const dim3 grid((uint32_t)blocks);
#define QDC_PRO(L)                                                                               \
    case L:                                                                                      \
        hipLaunchKernelGGL((delta_prologue_fast<T, L, TILE>), grid, dim3(kBlock), 0, stream, q); \
        return launch_status();
    switch (lph) {
        QDC_PRO(1)
        QDC_PRO(2)
        QDC_PRO(4)
        QDC_PRO(8)
        QDC_PRO(16)
        QDC_PRO(32)
        QDC_PRO(64)
        default:
            break;
    }
#undef QDC_PRO
    return kNoFastPath;
}

// Below this many workgroups with the large tiles (well under one per CU of the
// 256; counted as channel blocks plus one gates block per tile, the grid these
// measurements had) the launch takes 4-token tiles.  Measured on MI355X,
// graph-replayed: at the 0.8B DeltaNet dims (bf16, 7 workgroups per tile) 4-token tiles run 3.9
// and 4.9 us at 64 and 256 tokens against 6.1 and 6.2 with 12-token tiles (42
// and 154 large-tile workgroups); at the 4-layer synthetic dims (fp32, 2 per
// tile) 3.7-4.5 us at 64-512 tokens against 6.1-6.5 with 16-token tiles.
constexpr int64_t kSmallTileBelow = 160;

template <typename T>
int32_t launch(const Prologue &p, bool fast, hipStream_t stream) {
    const int lph = p.kd / 4;
    const int64_t bpt = ceil_div(p.chunks, kBlock);
    const int64_t big_tiles = ceil_div(p.tokens, tile_for<T>());
    const bool small = big_tiles * (bpt + 1) < kSmallTileBelow;
    const int64_t runs = ceil_div(small ? ceil_div(p.tokens, kSmallTile) : big_tiles, 8 * kXcdRun);
    const int64_t fast_blocks = runs * 8 * kXcdRun * bpt + ceil_div(p.tokens, (int64_t)kGateTokens);
    // the fast grid is one-dimensional: fewer than 2^32 work-items
    if (fast && p.kd % 4 == 0 && p.vd % 4 == 0 && p.taps == kTaps && lph <= kWave &&
        (lph & (lph - 1)) == 0 && fast_blocks * kBlock < ((int64_t)1 << 32)) {
        Prologue q = p;
        q.blocks_per_tile = (uint32_t)bpt;
        const int32_t st = small ? launch_fast<T, kSmallTile>(q, lph, stream)
                                 : launch_fast<T, tile_for<T>()>(q, lph, stream);
        if (st != kNoFastPath) return st;
    }
    const dim3 grid((uint32_t)ceil_div(p.tokens, kBlock / kWave), (uint32_t)(2 * p.kh + 2));
    hipLaunchKernelGGL((delta_prologue_general<T>), grid, dim3(kBlock), 0, stream, p);
    return launch_status();
}

}  // namespace
}  // namespace qdc

using namespace qdc;

extern "C" int32_t qdc_delta_prologue(float *q, float *k, float *v, float *beta, float *decay,
                                      const void *proj, int32_t proj_dtype, int64_t ld,
                                      const float *conv, int64_t taps, const float *a_decay,
                                      const float *dt_bias, int64_t tokens, int64_t seq_len,
                                      int64_t key_heads, int64_t key_dim, int64_t value_heads,
                                      int64_t value_dim, int64_t ld_qk, int64_t ld_v,
                                      hipStream_t stream) {
    if (!valid_dtype(proj_dtype)) return QDC_ERR_DTYPE;
    if (tokens < 0 || seq_len <= 0 || key_heads <= 0 || key_dim <= 0 || value_heads <= 0 ||
        value_dim <= 0 || taps <= 0 || taps > 64)
        return QDC_ERR_SHAPE;
    const int64_t kw = key_heads * key_dim, vw = value_heads * value_dim;
    const int64_t cq = 2 * kw + vw;
    if (ld < cq + vw + 2 * value_heads) return QDC_ERR_SHAPE;
    if (ld_qk < kw || ld_v < vw) return QDC_ERR_SHAPE;
    if (tokens == 0) return QDC_OK;
    if (tokens >= ((int64_t)1 << 26) || seq_len >= ((int64_t)1 << 31) || cq >= ((int64_t)1 << 28) ||
        key_heads > 32000)
        return QDC_ERR_SHAPE;
    if (!q || !k || !v || !beta || !decay || !proj || !conv || !a_decay || !dt_bias)
        return QDC_ERR_NULL;
    const int64_t es = elem_size(proj_dtype);
    const int64_t span_in = ((tokens - 1) * ld + ld) * es;
    const OutRows outs[3] = {{q, kw, ld_qk}, {k, kw, ld_qk}, {v, vw, ld_v}};
    for (int i = 0; i < 3; ++i) {
        if (overlaps(outs[i].p, outs[i].span(tokens), proj, span_in)) return QDC_ERR_ALIAS;
        for (int j = i + 1; j < 3; ++j)
            if (!disjoint_rows(outs[i], outs[j], tokens)) return QDC_ERR_ALIAS;
    }
    Prologue p{};
    p.proj = proj;
    p.ld = ld;
    p.a_off = cq + vw;
    p.b_off = cq + vw + value_heads;
    p.conv = conv;
    p.a_decay = a_decay;
    p.dt_bias = dt_bias;
    p.q = q;
    p.k = k;
    p.v = v;
    p.beta = beta;
    p.decay = decay;
    p.ld_qk = ld_qk;
    p.ld_v = ld_v;
    p.tokens = tokens;
    p.seq = make_fastdiv((uint32_t)seq_len);
    p.kh = (int)key_heads;
    p.kd = (int)key_dim;
    p.vh = (int)value_heads;
    p.vd = (int)value_dim;
    p.taps = (int)taps;
    p.chunks = (int)(cq / 4);
    p.qk_chunks = (int)(2 * kw / 4);
    // sqrt(Float32(key_dim)) of src/backbone.jl:313 / src/backbone_cpu.jl:516
    p.sqrt_kd = std::sqrt((float)key_dim);
    p.inv_sqrt_kd = 1.0f / p.sqrt_kd;
    // 4-channel pieces: 8-byte (bf16) or 16-byte (fp32) aligned projection rows
    const bool fast = ((uintptr_t)proj % (4 * es)) == 0 && (ld * es) % (4 * es) == 0 &&
                      aligned16(q) && aligned16(k) && aligned16(v) && aligned16(conv) && cq % 4 == 0 &&
                      ld_qk % 4 == 0 && ld_v % 4 == 0;
    if (proj_dtype == QDC_BF16) return launch<bf16_t>(p, fast, stream);
    return launch<float>(p, fast, stream);
}

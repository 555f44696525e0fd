// qdc_rope.hip -- per-head zero-centred RMSNorm fused with half-split partial
// RoPE for the Q and K heads of full attention (one launch for both), and the
// host-side RoPE table builder.
//
// Fast path (head_dim a power-of-two number >= 2 of 16-byte chunks, at most
// 128, rotary_dim/2 a multiple of the chunk): the row groups of
// qdc_rope_rows.hpp, Q rows on the first workgroups and K rows on the rest.
//
// General path (any shape/alignment): one wavefront per row; the normalised
// rotary block is staged in LDS so in-place operation stays correct.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "qdc_common.hpp"
#include "qdc_rope_rows.hpp"

namespace qdc {
namespace {

// Q rows take workgroups [0, q_blocks), K rows the rest (block-uniform branch);
// a lane group holds RPGQ heads of a Q token or one K head.
template <typename T, int LPR, int RPGQ>
__global__ __launch_bounds__(kBlock) void qk_norm_rope_fast(QKArgs<T> a) {
    const int hc = a.half / Elem<T>::kVec;
    if (2 * hc <= LPR && (hc & (hc - 1)) == 0) {
        if ((int64_t)blockIdx.x < a.q_blocks)
            qk_side_contig<T, LPR, RPGQ>(a, a.q, (int64_t)blockIdx.x);
        else
            qk_side_contig<T, LPR, 1>(a, a.k, (int64_t)blockIdx.x - a.q_blocks);
        return;
    }
    if ((int64_t)blockIdx.x < a.q_blocks)
        qk_side_paired<T, LPR, RPGQ>(a, a.q, (int64_t)blockIdx.x);
    else
        qk_side_paired<T, LPR, 1>(a, a.k, (int64_t)blockIdx.x - a.q_blocks);
}

constexpr int kMaxGeneralRotary = 1024;

template <typename T>
__global__ __launch_bounds__(kBlock) void qk_norm_rope_general(QKArgs<T> a) {
    __shared__ float staged[kBlock / kWave][kMaxGeneralRotary];
    const bool is_k = (int64_t)blockIdx.x >= a.q_blocks;
    const Side<T> &sd = is_k ? a.k : a.q;
    const int64_t block = is_k ? (int64_t)blockIdx.x - a.q_blocks : (int64_t)blockIdx.x;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int64_t row = block * (kBlock / kWave) + wave;
    const bool active = row < sd.rows;  // uniform per wavefront
    const int dim = a.dim, half = a.half;
    float *st = staged[wave];

    const T *in = sd.in;
    T *out = sd.out;
    float s = 0.0f;
    int64_t pos = 0;
    if (active) {
        const uint32_t t = fastdiv((uint32_t)row, sd.heads);
        const uint32_t h = (uint32_t)row - t * sd.heads.d;
        in += (int64_t)t * sd.in_tok + (int64_t)h * sd.in_head;
        const uint32_t tq = fastdiv(t, a.seq_len);
        const uint32_t sq = t - tq * a.seq_len.d;  // token within its sequence
        out += (int64_t)tq * sd.out_seq + (int64_t)sq * sd.out_tok + (int64_t)h * sd.out_head;
        pos = a.pos_offset + (int64_t)sq;
        float ss = 0.0f;
        for (int i = lane; i < dim; i += kWave) {
            const float v = to_f32(in[i]);
            ss += v * v;
        }
        ss = group_sum<kWave>(ss);
        s = rms_scale(ss, (float)dim, a.eps);
        for (int i = lane; i < 2 * half; i += kWave) st[i] = (to_f32(in[i]) * s) * (1.0f + to_f32(sd.w[i]));
    }
    __syncthreads();
    if (active) {
        for (int i = lane; i < dim; i += kWave) {
            float o;
            if (i < half) {
                const float c = a.cos[pos * half + i], sn = a.sin[pos * half + i];
                o = st[i] * c - st[i + half] * sn;
            } else if (i < 2 * half) {
                const float c = a.cos[pos * half + i - half], sn = a.sin[pos * half + i - half];
                o = st[i] * c + st[i - half] * sn;
            } else {
                o = (to_f32(in[i]) * s) * (1.0f + to_f32(sd.w[i]));
            }
            out[i] = from_f32<T>(o);
        }
    }
}

// Q heads of one token per lane group: the largest of 4, 2, 1 that divides the
// head count (4 measured ~5% faster than 1 on the 8 + 2 heads of 256 in bf16;
// 8 was slower).  K rows take one head per lane group: on those shapes 2.5%
// faster over the launch than both KV heads of a token in one group, since the
// K workgroups, last in the grid, then hold half the bytes each.
constexpr int kMaxRowsPerGroup = 4;
int rows_per_group(int64_t heads) {
    int r = 1;
    while (2 * r <= kMaxRowsPerGroup && heads % (2 * r) == 0) r *= 2;
    return r;
}

template <typename T, int LPR, int RPGQ>
int32_t launch_fast(QKArgs<T> a, hipStream_t stream) {
    constexpr int64_t gpb = kBlock / LPR;
    a.q_blocks = ceil_div(a.q.rows / RPGQ, gpb);
    const int64_t blocks = a.q_blocks + ceil_div(a.k.rows, gpb);
    hipLaunchKernelGGL((qk_norm_rope_fast<T, LPR, RPGQ>), dim3((uint32_t)blocks),
                       dim3(kBlock), 0, stream, a);
    return launch_status();
}

template <typename T, int LPR>
int32_t launch_lpr(QKArgs<T> a, int64_t heads, hipStream_t stream) {
    switch (rows_per_group(heads)) {
        case 4: return launch_fast<T, LPR, 4>(a, stream);
        case 2: return launch_fast<T, LPR, 2>(a, stream);
        default: return launch_fast<T, LPR, 1>(a, stream);
    }
}

template <typename T>
int32_t launch(QKArgs<T> a, int64_t heads, bool fast, hipStream_t stream) {
    constexpr int V = Elem<T>::kVec;
    const int64_t chunks = a.dim / V;
    // two chunks per lane: LPR = chunks / 2 lanes per row, a power of two <= 64
    const int64_t lpr = chunks / 2;
    if (fast && a.dim % V == 0 && a.half % V == 0 && chunks >= 2 && chunks % 2 == 0 && lpr <= kWave &&
        (lpr & (lpr - 1)) == 0) {
        switch (lpr) {
            case 1: return launch_lpr<T, 1>(a, heads, stream);
            case 2: return launch_lpr<T, 2>(a, heads, stream);
            case 4: return launch_lpr<T, 4>(a, heads, stream);
            case 8: return launch_lpr<T, 8>(a, heads, stream);
            case 16: return launch_lpr<T, 16>(a, heads, stream);
            case 32: return launch_lpr<T, 32>(a, heads, stream);
            case 64: return launch_lpr<T, 64>(a, heads, stream);
            default:
                break;
        }
    }
    // the general kernel stages the rotary block of each row in LDS
    if (2 * a.half > kMaxGeneralRotary) return QDC_ERR_SHAPE;
    const int64_t rpb = kBlock / kWave;
    a.q_blocks = ceil_div(a.q.rows, rpb);
    const int64_t blocks = a.q_blocks + ceil_div(a.k.rows, rpb);
    hipLaunchKernelGGL((qk_norm_rope_general<T>), dim3((uint32_t)blocks), dim3(kBlock), 0, stream,
                       a);
    return launch_status();
}

// A side's rows in memory: up to three (extent, stride) dimensions in
// elements (sequence, token within the sequence, head) over rows of head_dim
// contiguous elements.
struct Layout {
    int64_t n[3], stride[3];
};

// Rows never overlap: with the dimensions of extent > 1 sorted by stride, each
// stride reaches past everything the smaller ones span.
bool disjoint_rows(const Layout &l, int64_t head_dim) {
    int order[3], m = 0;
    for (int d = 0; d < 3; ++d) {
        if (l.n[d] <= 1) continue;
        if (l.stride[d] < 0) return false;
        order[m++] = d;
    }
    std::sort(order, order + m, [&](int x, int y) { return l.stride[x] < l.stride[y]; });
    int64_t span = head_dim;
    for (int i = 0; i < m; ++i) {
        const int d = order[i];
        if (l.stride[d] < span) return false;
        span += (l.n[d] - 1) * l.stride[d];
    }
    return true;
}

// Token t of `tokens` lies in sequence t / seq_len at position t % seq_len.
Layout side_layout(int64_t tokens, int64_t seq_len, int64_t heads, int64_t seq_stride,
                   int64_t tok, int64_t head) {
    const int64_t n_seq = (tokens + seq_len - 1) / seq_len;
    return Layout{{n_seq, std::min(tokens, seq_len), heads}, {seq_stride, tok, head}};
}

// Byte extent of a side: one past the last element any row touches.
int64_t span_bytes(int64_t tokens, int64_t seq_len, const Layout &l, int64_t head_dim,
                   int64_t es) {
    const int64_t last = tokens - 1, tq = last / seq_len;
    int64_t far = tq * l.stride[0] + (last - tq * seq_len) * l.stride[1];
    if (tq > 0) far = std::max(far, (tq - 1) * l.stride[0] + (seq_len - 1) * l.stride[1]);
    return (far + (l.n[2] - 1) * l.stride[2] + head_dim) * es;
}

int32_t qk_norm_rope(void *q_out, void *k_out, const void *q_in, const void *k_in,
                     const void *q_norm, const void *k_norm, const float *cos_table,
                     const float *sin_table, int64_t tokens, int64_t heads, int64_t kv_heads,
                     int64_t head_dim, int64_t rotary_dim, int64_t seq_len, int64_t pos_offset,
                     int64_t table_len, int64_t q_in_tok, int64_t q_in_head, int64_t q_out_seq,
                     int64_t q_out_tok, int64_t q_out_head, int64_t k_in_tok, int64_t k_in_head,
                     int64_t k_out_seq, int64_t k_out_tok, int64_t k_out_head, float eps,
                     int32_t dtype, hipStream_t stream) {
    if (!valid_dtype(dtype)) return QDC_ERR_DTYPE;
    if (tokens < 0 || heads < 0 || kv_heads < 0 || head_dim <= 0 || rotary_dim < 0 ||
        rotary_dim % 2 || rotary_dim > head_dim || seq_len <= 0 || pos_offset < 0 ||
        table_len < 0)
        return QDC_ERR_SHAPE;
    // up to a wavefront per (token, head) row in a grid of fewer than 2^32 work-items
    if (head_dim > INT32_MAX || seq_len >= ((int64_t)1 << 31) ||
        tokens * (heads + kv_heads) >= ((int64_t)1 << 26))
        return QDC_ERR_SHAPE;
    if (tokens == 0 || (heads == 0 && kv_heads == 0)) return QDC_OK;
    if (heads > 0 && (!q_out || !q_in || !q_norm)) return QDC_ERR_NULL;
    if (kv_heads > 0 && (!k_out || !k_in || !k_norm)) return QDC_ERR_NULL;
    if (rotary_dim > 0) {
        if (!cos_table || !sin_table) return QDC_ERR_NULL;
        if (pos_offset + std::min(tokens, seq_len) > table_len) return QDC_ERR_RANGE;
    }
    const int64_t es = elem_size(dtype);
    // Inputs are [tokens, heads] row grids; outputs may also split the tokens
    // into sequences of seq_len with their own stride.  Rows of a tensor must
    // not overlap (token-major, head-major (dim, tokens, heads) as the
    // reference AMDGPU layout, or head-major per sequence).
    const Layout qil{{1, tokens, heads}, {0, q_in_tok, q_in_head}};
    const Layout kil{{1, tokens, kv_heads}, {0, k_in_tok, k_in_head}};
    const Layout qol = side_layout(tokens, seq_len, heads, q_out_seq, q_out_tok, q_out_head);
    const Layout kol = side_layout(tokens, seq_len, kv_heads, k_out_seq, k_out_tok, k_out_head);
    if ((heads && (!disjoint_rows(qil, head_dim) || !disjoint_rows(qol, head_dim))) ||
        (kv_heads && (!disjoint_rows(kil, head_dim) || !disjoint_rows(kol, head_dim))))
        return QDC_ERR_SHAPE;
    struct View {
        const void *p;
        int64_t bytes;
        Layout l;
    };
    auto view = [&](const void *p, int64_t n_heads, int64_t seq, const Layout &l) {
        return View{p, n_heads ? span_bytes(tokens, seq, l, head_dim, es) : 0, l};
    };
    // an input's rows are one sequence of all the tokens
    const View qi = view(q_in, heads, tokens, qil), ki = view(k_in, kv_heads, tokens, kil);
    const View qo = view(q_out, heads, seq_len, qol), ko = view(k_out, kv_heads, seq_len, kol);
    // An output may coincide exactly with its own input (in place: same
    // pointer, and every row at the same place); any other overlap between an
    // output and an input or the other output is rejected.
    auto same_rows = [&](const View &o, const View &i) {
        const int64_t n_seq = o.l.n[0];
        return o.p == i.p && o.l.stride[1] == i.l.stride[1] && o.l.stride[2] == i.l.stride[2] &&
               (n_seq <= 1 || o.l.stride[0] == seq_len * i.l.stride[1]);
    };
    auto clash = [&](const View &o, const View &i, bool own) {
        if (own && same_rows(o, i)) return false;
        return overlaps(o.p, o.bytes, i.p, i.bytes);
    };
    if (clash(qo, qi, true) || clash(qo, ki, false) || clash(ko, ki, true) ||
        clash(ko, qi, false) || overlaps(qo.p, qo.bytes, ko.p, ko.bytes))
        return QDC_ERR_ALIAS;

    const bool fast = aligned16(q_out) && aligned16(q_in) && aligned16(q_norm) &&
                      aligned16(k_out) && aligned16(k_in) && aligned16(k_norm) &&
                      aligned16(cos_table) && aligned16(sin_table) &&
                      ((q_in_tok | q_in_head | q_out_seq | q_out_tok | q_out_head | k_in_tok |
                        k_in_head | k_out_seq | k_out_tok | k_out_head) *
                       es) % 16 == 0 &&
                      (rotary_dim / 2) % 4 == 0;
    if (!fast && rotary_dim > kMaxGeneralRotary) return QDC_ERR_SHAPE;

    auto fill = [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        QKArgs<T> a{};
        a.q = Side<T>{(const T *)q_in, (T *)q_out, (const T *)q_norm, q_in_tok, q_in_head,
                      q_out_tok, q_out_head, q_out_seq, tokens * heads,
                      make_fastdiv((uint32_t)std::max<int64_t>(heads, 1))};
        a.k = Side<T>{(const T *)k_in, (T *)k_out, (const T *)k_norm, k_in_tok, k_in_head,
                      k_out_tok, k_out_head, k_out_seq, tokens * kv_heads,
                      make_fastdiv((uint32_t)std::max<int64_t>(kv_heads, 1))};
        a.cos = cos_table;
        a.sin = sin_table;
        a.seq_len = make_fastdiv((uint32_t)seq_len);
        a.pos_offset = pos_offset;
        a.half = (int32_t)(rotary_dim / 2);
        a.dim = (int32_t)head_dim;
        a.eps = eps;
        return launch<T>(a, heads, fast, stream);
    };
    if (dtype == QDC_BF16) return fill((bf16_t *)nullptr);
    return fill((float *)nullptr);
}

}  // namespace
}  // namespace qdc

using namespace qdc;

extern "C" int32_t qdc_rope_tables(float *cos_table, float *sin_table, int64_t n_pos,
                                   int64_t rotary_dim, float theta) {
    if (n_pos < 0 || rotary_dim < 0 || rotary_dim % 2) return QDC_ERR_SHAPE;
    if (n_pos == 0 || rotary_dim == 0) return QDC_OK;
    if (!cos_table || !sin_table) return QDC_ERR_NULL;
    const int64_t half = rotary_dim / 2;
    for (int64_t i = 0; i < half; ++i) {
        // Float32 `^`, `inv`, `*` as in src/backbone_cpu.jl:92-95; Julia's Float32
        // pow/cos/sin evaluate in Float64 and round once.
        const float exponent = (float)(2 * i) / (float)rotary_dim;
        const float power = (float)std::pow((double)theta, (double)exponent);
        const float freq = 1.0f / power;
        for (int64_t p = 0; p < n_pos; ++p) {
            const float angle = freq * (float)p;
            cos_table[p * half + i] = (float)std::cos((double)angle);
            sin_table[p * half + i] = (float)std::sin((double)angle);
        }
    }
    return QDC_OK;
}

extern "C" int32_t qdc_qk_norm_rope(void *q_out, void *k_out, const void *q_in, const void *k_in,
                                    const void *q_norm, const void *k_norm,
                                    const float *cos_table, const float *sin_table, int64_t tokens,
                                    int64_t heads, int64_t kv_heads, int64_t head_dim,
                                    int64_t rotary_dim, int64_t seq_len, int64_t pos_offset,
                                    int64_t table_len, int64_t q_in_tok, int64_t q_in_head,
                                    int64_t q_out_tok, int64_t q_out_head, int64_t k_in_tok,
                                    int64_t k_in_head, int64_t k_out_tok, int64_t k_out_head,
                                    float eps, int32_t dtype, hipStream_t stream) {
    // one grid of token rows: sequence s starts at token s*seq_len (a stride
    // that is only used when tokens > seq_len)
    const bool several = seq_len > 0 && tokens > seq_len;
    return qk_norm_rope(q_out, k_out, q_in, k_in, q_norm, k_norm, cos_table, sin_table, tokens,
                        heads, kv_heads, head_dim, rotary_dim, seq_len, pos_offset, table_len,
                        q_in_tok, q_in_head, several ? seq_len * q_out_tok : 0, q_out_tok,
                        q_out_head, k_in_tok, k_in_head, several ? seq_len * k_out_tok : 0,
                        k_out_tok, k_out_head, eps, dtype, stream);
}

extern "C" int32_t qdc_qk_norm_rope_batched(
    void *q_out, void *k_out, const void *q_in, const void *k_in, const void *q_norm,
    const void *k_norm, const float *cos_table, const float *sin_table, int64_t tokens,
    int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t rotary_dim, int64_t seq_len,
    int64_t pos_offset, int64_t table_len, int64_t q_in_tok, int64_t q_in_head, int64_t q_out_seq,
    int64_t q_out_tok, int64_t q_out_head, int64_t k_in_tok, int64_t k_in_head, int64_t k_out_seq,
    int64_t k_out_tok, int64_t k_out_head, float eps, int32_t dtype, hipStream_t stream) {
    return qk_norm_rope(q_out, k_out, q_in, k_in, q_norm, k_norm, cos_table, sin_table, tokens,
                        heads, kv_heads, head_dim, rotary_dim, seq_len, pos_offset, table_len,
                        q_in_tok, q_in_head, q_out_seq, q_out_tok, q_out_head, k_in_tok, k_in_head,
                        k_out_seq, k_out_tok, k_out_head, eps, dtype, stream);
}

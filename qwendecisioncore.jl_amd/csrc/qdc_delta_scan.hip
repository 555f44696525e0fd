// qdc_delta_scan.hip -- the gated delta rule recurrence of the DeltaNet layers.
//
// Not one of the fused row kernels: it is the "existing path" recurrence of the
// reference's AMDGPU extension (delta_recurrent_kernel!, ext/amdgpu_delta.jl:37-81),
// provided so backbone_hidden runs at speed on long sequences.  Per (sequence
// b, value head h) with key head g = h / groups and state S [value_dim, key_dim]
// starting at zero, for each token t (cpu_delta_recurrent_step!,
// src/backbone_cpu.jl:681-705):
//     f = exp(decay[t]);  u = beta[t] * (v[t] - f * S k[t]);
//     S = f * S + u k[t]^T;  out[t] = S q[t]
//
// Mapping: a workgroup (4 wavefronts = 16 groups of 16 lanes) owns 16*R
// consecutive value rows of one (b, h); each 16-lane group owns R rows and splits
// the key dimension across its lanes, so both dot products per row and token
// reduce over 16 lanes with 4 DPP steps.  The state (R x KPL values per lane)
// stays in registers for the whole sequence.  Tokens are processed in chunks of
// kChunk: the chunk's k, q (key head g), v (the block's rows), beta and decay are
// staged in LDS by the whole workgroup, and the next chunk's global loads are
// issued before the current chunk's steps run, so the sequential steps read
// only LDS.  Outputs of a chunk are gathered in LDS and written as whole rows.
#include <type_traits>

#include "qdc_common.hpp"

namespace qdc {
namespace {

constexpr int kGroup = 16;                       // lanes per key split
constexpr int kGroupsPerBlock = kBlock / kGroup; // 16
constexpr int kChunk = 16;                       // tokens staged per LDS buffer

// Key component held in slot i of lane `lane`: blocks of 4 consecutive keys
// dealt round-robin over the 16 lanes (conflict-free 16-byte LDS reads) when a
// lane holds a multiple of 4 keys, else KPL consecutive keys.
template <int KPL> __device__ __forceinline__ int key_of(int lane, int i) {
    if constexpr (KPL % 4 == 0) return (i / 4) * (4 * kGroup) + lane * 4 + (i % 4);
    else return lane * KPL + i;
}

template <int KPL> __device__ __forceinline__ void read_keys(const float *row, int lane,
                                                             float (&out)[KPL]) {
    if constexpr (KPL % 4 == 0) {
#pragma unroll
        for (int i = 0; i < KPL; i += 4) {
            const f32x4 c = *reinterpret_cast<const f32x4 *>(row + key_of<KPL>(lane, i));
            out[i] = c.x; out[i + 1] = c.y; out[i + 2] = c.z; out[i + 3] = c.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < KPL; ++i) out[i] = row[key_of<KPL>(lane, i)];
    }
}

struct ScanArgs {
    void *out;
    const float *q, *k, *v, *beta, *decay;
    int S, H, KH, KD, vd, groups;
};

template <int KPL, int R, bool VEC, typename TO>
__global__ __launch_bounds__(kBlock) void delta_scan(ScanArgs a) {
    constexpr int KP = KPL * kGroup;             // padded key dimension
    constexpr int RB = R * kGroupsPerBlock;      // value rows per workgroup
    // chunk elements per thread for the staged loads (upper bounds)
    constexpr int KQ_ITEMS = VEC ? (kChunk * KP / 4 + kBlock - 1) / kBlock
                                 : (kChunk * KP + kBlock - 1) / kBlock;
    constexpr int V_ITEMS = (kChunk * RB + kBlock - 1) / kBlock;
    __shared__ __align__(16) float sk[2][kChunk][KP];
    __shared__ __align__(16) float sq[2][kChunk][KP];
    __shared__ float sv[2][kChunk][RB];
    __shared__ float sb[2][kChunk], sd[2][kChunk];
    __shared__ float so[kChunk][RB];

    const int tid = threadIdx.x;
    const int lane = tid % kGroup, grp = tid / kGroup;
    const int h = blockIdx.y, b = blockIdx.z;
    const int g = h / a.groups;
    const int row0 = blockIdx.x * RB;            // first value row of the workgroup
    const int KD = a.KD, S = a.S;
    const int64_t k_tok = (int64_t)a.KH * KD, v_tok = (int64_t)a.H * a.vd;
    const float *kb = a.k + (int64_t)b * S * k_tok + (int64_t)g * KD;
    const float *qb = a.q + (int64_t)b * S * k_tok + (int64_t)g * KD;
    const float *vb = a.v + (int64_t)b * S * v_tok + (int64_t)h * a.vd;
    const float *bb = a.beta + (int64_t)b * S * a.H + h;
    const float *db = a.decay + (int64_t)b * S * a.H + h;
    TO *ob = reinterpret_cast<TO *>(a.out) + (int64_t)b * S * v_tok + (int64_t)h * a.vd;

    // padded key components stay zero for the whole launch
    for (int i = tid; i < 2 * kChunk * KP; i += kBlock) {
        (&sk[0][0][0])[i] = 0.0f;
        (&sq[0][0][0])[i] = 0.0f;
    }

    // staged registers of one chunk
    using Item = typename std::conditional<VEC, f32x4, float>::type;
    Item rk[KQ_ITEMS], rq[KQ_ITEMS];
    float rv[V_ITEMS], rb = 0.0f, rd = 0.0f;
    const int kd4 = KD / 4;
    auto fetch = [&](int c) {  // global -> registers for chunk c
        const int t0 = c * kChunk;
        const int n = min(kChunk, S - t0);
#pragma unroll
        for (int p = 0; p < KQ_ITEMS; ++p) {
            const int idx = tid + p * kBlock;
            rk[p] = Item{};
            rq[p] = Item{};
            if constexpr (VEC) {
                const int tt = idx / kd4, j4 = idx - tt * kd4;
                if (tt < n) {
                    const int64_t off = (int64_t)(t0 + tt) * k_tok + j4 * 4;
                    rk[p] = *reinterpret_cast<const f32x4 *>(kb + off);
                    rq[p] = *reinterpret_cast<const f32x4 *>(qb + off);
                }
            } else {
                const int tt = idx / KD, j = idx - tt * KD;
                if (tt < n) {
                    const int64_t off = (int64_t)(t0 + tt) * k_tok + j;
                    rk[p] = kb[off];
                    rq[p] = qb[off];
                }
            }
        }
#pragma unroll
        for (int p = 0; p < V_ITEMS; ++p) {
            const int idx = tid + p * kBlock;
            const int tt = idx / RB, r = idx - tt * RB;
            rv[p] = (tt < n && row0 + r < a.vd) ? vb[(int64_t)(t0 + tt) * v_tok + row0 + r] : 0.0f;
        }
        if (tid < n) {
            rb = bb[(int64_t)(t0 + tid) * a.H];
            rd = db[(int64_t)(t0 + tid) * a.H];
        }
    };
    auto stage = [&](int c, int buf) {  // registers -> LDS buffer for chunk c
        const int n = min(kChunk, S - c * kChunk);
#pragma unroll
        for (int p = 0; p < KQ_ITEMS; ++p) {
            const int idx = tid + p * kBlock;
            if constexpr (VEC) {
                const int tt = idx / kd4, j4 = idx - tt * kd4;
                if (tt < n) {  // rows are staged in natural key order
                    *reinterpret_cast<f32x4 *>(&sk[buf][tt][j4 * 4]) = rk[p];
                    *reinterpret_cast<f32x4 *>(&sq[buf][tt][j4 * 4]) = rq[p];
                }
            } else {
                const int tt = idx / KD, j = idx - tt * KD;
                if (tt < n) {
                    sk[buf][tt][j] = rk[p];
                    sq[buf][tt][j] = rq[p];
                }
            }
        }
#pragma unroll
        for (int p = 0; p < V_ITEMS; ++p) {
            const int idx = tid + p * kBlock;
            const int tt = idx / RB;
            if (tt < kChunk) sv[buf][tt][idx - tt * RB] = rv[p];
        }
        if (tid < n) {
            sb[buf][tid] = rb;
            sd[buf][tid] = rd;
        }
    };

    float st[R][KPL];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < KPL; ++i) st[r][i] = 0.0f;

    const int chunks = (S + kChunk - 1) / kChunk;
    __syncthreads();  // zero padding written
    fetch(0);
    stage(0, 0);
    __syncthreads();
    for (int c = 0; c < chunks; ++c) {
        const int buf = c & 1;
        if (c + 1 < chunks) fetch(c + 1);  // in flight during this chunk's steps
        const int n = min(kChunk, S - c * kChunk);
        for (int tt = 0; tt < n; ++tt) {
            float kt[KPL], qt[KPL];
            read_keys<KPL>(&sk[buf][tt][0], lane, kt);
            read_keys<KPL>(&sq[buf][tt][0], lane, qt);
            const float bt = sb[buf][tt], f = __expf(sd[buf][tt]);
            float pred[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < KPL; ++i) s = __builtin_fmaf(st[r][i], kt[i], s);
                pred[r] = group_sum<kGroup>(s);
            }
            float o[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float u = bt * (sv[buf][tt][grp * R + r] - f * pred[r]);
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < KPL; ++i) {
                    st[r][i] = __builtin_fmaf(u, kt[i], f * st[r][i]);
                    s = __builtin_fmaf(st[r][i], qt[i], s);
                }
                o[r] = group_sum<kGroup>(s);
            }
            if (lane < R) {
                float mine = o[0];
#pragma unroll
                for (int r = 1; r < R; ++r) mine = lane == r ? o[r] : mine;
                so[tt][grp * R + lane] = mine;
            }
        }
        __syncthreads();  // steps done: `so` complete, buffer `buf` free
        if (c + 1 < chunks) stage(c + 1, buf ^ 1);
#pragma unroll
        for (int p = 0; p < V_ITEMS; ++p) {
            const int idx = tid + p * kBlock;
            const int tt = idx / RB, r = idx - tt * RB;
            if (tt < n && row0 + r < a.vd)
                ob[(int64_t)(c * kChunk + tt) * v_tok + row0 + r] = from_f32<TO>(so[tt][r]);
        }
        __syncthreads();  // next buffer staged, `so` read
    }
}

}  // namespace
}  // namespace qdc

using namespace qdc;

extern "C" int32_t qdc_delta_scan(void *out, int32_t out_dtype, const float *q, const float *k,
                                  const float *v, const float *beta, const float *decay,
                                  int64_t batch, int64_t seq, int64_t heads, int64_t key_heads,
                                  int64_t key_dim, int64_t value_dim, hipStream_t stream) {
    if (!valid_dtype(out_dtype)) return QDC_ERR_DTYPE;
    if (batch < 0 || seq < 0 || heads <= 0 || key_heads <= 0 || value_dim <= 0 ||
        heads % key_heads)
        return QDC_ERR_SHAPE;
    if (key_dim <= 0 || key_dim > 256) return QDC_ERR_SHAPE;
    if (batch == 0 || seq == 0) return QDC_OK;
    if (batch > 65535 || heads > 65535 || seq >= ((int64_t)1 << 31) ||
        value_dim >= ((int64_t)1 << 24))
        return QDC_ERR_SHAPE;
    if (!out || !q || !k || !v || !beta || !decay) return QDC_ERR_NULL;
    ScanArgs a{};
    a.out = out;
    a.q = q;
    a.k = k;
    a.v = v;
    a.beta = beta;
    a.decay = decay;
    a.S = (int)seq;
    a.H = (int)heads;
    a.KH = (int)key_heads;
    a.KD = (int)key_dim;
    a.vd = (int)value_dim;
    a.groups = (int)(heads / key_heads);
    // Two value rows per 16-lane group, or one when that leaves too few
    // workgroups to occupy the GPU (single sequences with few heads).
    const int64_t blocks2 = ceil_div(value_dim, 2 * kGroupsPerBlock) * heads * batch;
    const bool two = blocks2 >= 512;
    const int64_t rb = (two ? 2 : 1) * kGroupsPerBlock;
    const dim3 grid((uint32_t)ceil_div(value_dim, rb), (uint32_t)heads, (uint32_t)batch);
    const bool vec = aligned16(q) && aligned16(k) && key_dim % 4 == 0;
    const int64_t kpl = ceil_div(key_dim, kGroup);
#define QDC_SCAN(KPL, R, VEC, TO)                                                              \
    hipLaunchKernelGGL((delta_scan<KPL, R, VEC, TO>), grid, dim3(kBlock), 0, stream, a);      \
    return launch_status();
#define QDC_SCAN_R(KPL, VEC, TO)                                                               \
    if (two) { QDC_SCAN(KPL, 2, VEC, TO) }                                                     \
    QDC_SCAN(KPL, 1, VEC, TO)
#define QDC_SCAN_V(KPL, TO)                                                                    \
    if (vec) { QDC_SCAN_R(KPL, true, TO) }                                                     \
    QDC_SCAN_R(KPL, false, TO)
#define QDC_SCAN_K(TO)                                                                         \
    if (kpl <= 1) { QDC_SCAN_V(1, TO) }                                                        \
    if (kpl <= 2) { QDC_SCAN_V(2, TO) }                                                        \
    if (kpl <= 4) { QDC_SCAN_V(4, TO) }                                                        \
    if (kpl <= 8) { QDC_SCAN_V(8, TO) }                                                        \
    QDC_SCAN_V(16, TO)
    if (out_dtype == QDC_BF16) { QDC_SCAN_K(bf16_t) }
    QDC_SCAN_K(float)
#undef QDC_SCAN_K
#undef QDC_SCAN_V
#undef QDC_SCAN_R
#undef QDC_SCAN
}

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
    int64_t ld_qk, ld_v;  // elements between the token rows of q and k, and of v
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
    // input rows: q, k every ld_qk, v every ld_v elements; output rows contiguous
    const int64_t k_tok = a.ld_qk, vi_tok = a.ld_v, v_tok = (int64_t)a.H * a.vd;
    const float *kb = a.k + (int64_t)b * S * k_tok + (int64_t)g * KD;
    const float *qb = a.q + (int64_t)b * S * k_tok + (int64_t)g * KD;
    const float *vb = a.v + (int64_t)b * S * vi_tok + (int64_t)h * a.vd;
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
            rv[p] = (tt < n && row0 + r < a.vd) ? vb[(int64_t)(t0 + tt) * vi_tok + row0 + r] : 0.0f;
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

// ---------------------------------------------------------------------------
// Chunked form on the matrix cores (fp32 MFMA 16x16x4).  For a chunk of kC = 16
// tokens with state S0 (kept transposed, S^T [kd, vd]), log-decays d and their
// running sums g (g_i = d_0 + ... + d_i), the recurrence above is exactly
//     A[i][p] = beta_i exp(g_i - g_p) (k_i . k_p)   (p < i),  T = (I + A)^-1
//     U = T diag(beta) (V - diag(e^g) Z),   Z = K S0^T        (the deltas u_i)
//     O = diag(e^g) Q S0^T + P U,   P[i][p] = exp(g_i - g_p) (q_i . k_p)  (p <= i)
//     S^T <- e^(g_15) S^T + (diag(e^(g_15 - g)) K)^T U
// (a partial last chunk is padded with k = q = v = 0, beta = 0, d = 0).  A
// workgroup owns 64 value rows of one (sequence, head), 16 per row tile; the
// state of a tile lives in MFMA accumulator layout (lane l, register j:
// S^T[16a + 4(l/16) + j][16w + l%16]), which is also the B-operand layout the
// next chunk's S^T products read, so the state never leaves registers.
//
// Everything that does not involve the state (K K^T, Q K^T, A, P and the
// triangular inverse) is prepared ahead, overlapped with the state products.
// Per chunk c the workgroup runs two phases:
//     phase 1: Z, Q S0^T of chunk c (every wavefront); K K^T and Q K^T of chunk
//              c+1 split over the key dimension into four products, one per
//              SIMD; T diag(beta) of chunk c from A (the helper wavefront, the
//              last one); chunk c-1's outputs written from LDS (the others)
//     phase 2: U, O and the state update of chunk c (every wavefront); A and P
//              of chunk c+1 from the partial products (the last key part's
//              wavefronts, a quarter each); chunk c+2 staged (its loads were
//              issued in phase 1)
// with one barrier after each.  k, q, v live in three LDS buffers; P and the
// outputs in two.
constexpr int kC = 16;        // tokens per chunk: one MFMA tile edge
constexpr int kRowsWG = 64;   // value rows per workgroup, 16 per row tile
// LDS row stride of the v and output tiles: the four 16-lane groups of a
// wavefront read or write rows 4(l/16) + j, which 4 pad floats put on disjoint
// banks (an unpadded 64-float row put all four on the same banks; the padding
// measured 1-2.5% faster at the 0.8B shapes)
constexpr int kVS = kRowsWG + 4;

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Inclusive prefix sum over each 16-lane row of a wavefront (DPP row shifts;
// lanes shifted in from outside the row contribute 0).
__device__ __forceinline__ float row_prefix_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xf, 0xf, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xf, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xf, 0xf, true));
    return v;
}

// KSPLIT = 2 gives every 16-row tile two wavefronts, each holding half of the
// key blocks of the state: Z and Q S0^T are summed from the two halves through
// LDS, U is formed by both, O by the first, and each updates its own half of
// S^T.  That doubles the wavefronts (two per SIMD at the 0.8B shapes) so one
// wavefront's waits overlap the other's matrix work.
template <int KB, int KSPLIT, typename TO>
__global__ __launch_bounds__(kBlock * KSPLIT) void delta_scan_chunked(ScanArgs a) {
    constexpr int NT = kBlock * KSPLIT;      // threads per workgroup
    constexpr int KBW = KB / KSPLIT;         // key blocks of the state per wavefront
    static_assert(KB % KSPLIT == 0, "key blocks split evenly");
    static_assert(KB == 1 || KB % 2 == 0, "key blocks split into two halves");
    constexpr int KD = 16 * KB;             // key dimension
    constexpr int KS = KD + 4;              // LDS row stride of k/q rows (bank spread)
    constexpr int MS = kC + 1;              // row stride of the small matrices read by column
    constexpr int NB = 3;                   // k/q/v buffers: current, prepared, staging
    constexpr int KQ_ITEMS = (kC * KD / 4 + NT - 1) / NT;  // 16-byte loads per thread
    constexpr int kHelper = NT / kWave - 1;  // wavefront forming the inverse
    __shared__ __align__(16) float sK[NB][kC][KS];
    __shared__ __align__(16) float sQ[NB][kC][KS];
    __shared__ __align__(16) float sV[NB][kC][kVS];
    // per token: beta, the running log-decay sum g, e^g and e^(g_15 - g)
    __shared__ float sBeta[NB][kC], sG[NB][kC], sEg[NB][kC], sEt[NB][kC];
    __shared__ __align__(16) float sA[kC][kC];   // read as whole rows by the inverse
    // written and read as rows 4(l/16) + j by the 16-lane groups: a row stride of
    // 20 puts the four groups on disjoint banks
    constexpr int RS = kC + 4;
    __shared__ float sProd[4][kC][RS];           // K K^T and Q K^T, two key halves each
    __shared__ float sP[2][kC][MS], sTb[kC][MS];
    __shared__ float sT[kC][MS];                 // diagonal blocks of T (inverse)
    __shared__ float sO[2][kC][kVS];
    __shared__ float sPart[KSPLIT > 1 ? 2 * KSPLIT * 4 : 1][kC][RS];  // Z / Q S0^T halves

    const int tid = threadIdx.x;
    const int wv = tid / kWave, l = tid % kWave, lr = l % 16, lg = l / 16;
    const int w = wv % 4;                         // row tile of this wavefront
    const int kh = wv / 4;                        // key half (KSPLIT = 2)
    const int h = blockIdx.y, b = blockIdx.z;
    const int g = h / a.groups;
    const int row0 = blockIdx.x * kRowsWG;
    const int wrow = 16 * w;                      // this wavefront's rows within the workgroup
    const bool live = row0 + wrow < a.vd;         // value_dim % 16 == 0: whole tile or none
    const int S = a.S;
    // input rows: q, k every ld_qk, v every ld_v elements; output rows contiguous
    const int64_t k_tok = a.ld_qk, vi_tok = a.ld_v, v_tok = (int64_t)a.H * a.vd;
    const float *kb = a.k + (int64_t)b * S * k_tok + (int64_t)g * KD;
    const float *qb = a.q + (int64_t)b * S * k_tok + (int64_t)g * KD;
    const float *vb = a.v + (int64_t)b * S * vi_tok + (int64_t)h * a.vd + row0;
    const float *bb = a.beta + (int64_t)b * S * a.H + h;
    const float *db = a.decay + (int64_t)b * S * a.H + h;
    TO *ob = reinterpret_cast<TO *>(a.out) + (int64_t)b * S * v_tok + (int64_t)h * a.vd + row0;

    f32x4 rk[KQ_ITEMS], rq[KQ_ITEMS], rv;
    float rs = 0.0f;  // beta (threads 0..15) or decay (threads 16..31) of one token
    constexpr int kd4 = KD / 4;
    auto fetch = [&](int c) {
        const int t0 = c * kC, n = min(kC, S - t0);
#pragma unroll
        for (int p = 0; p < KQ_ITEMS; ++p) {
            const int idx = tid + p * NT;
            const int tt = idx / kd4, j4 = idx - tt * kd4;
            rk[p] = f32x4{0.f, 0.f, 0.f, 0.f};
            rq[p] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (tt < n) {
                const int64_t off = (int64_t)(t0 + tt) * k_tok + j4 * 4;
                rk[p] = *reinterpret_cast<const f32x4 *>(kb + off);
                rq[p] = *reinterpret_cast<const f32x4 *>(qb + off);
            }
        }
        {   // v: 16 tokens x 64 rows, one 16-byte piece per thread
            const int tt = tid / 16, r4 = (tid % 16) * 4;
            rv = f32x4{0.f, 0.f, 0.f, 0.f};
            if (tid < kC * kRowsWG / 4 && tt < n && row0 + r4 < a.vd)
                rv = *reinterpret_cast<const f32x4 *>(vb + (int64_t)(t0 + tt) * vi_tok + r4);
        }
        rs = 0.0f;
        if (tid < kC && tid < n) rs = bb[(int64_t)(t0 + tid) * a.H];
        else if (tid >= kC && tid < 2 * kC && tid - kC < n) rs = db[(int64_t)(t0 + tid - kC) * a.H];
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int p = 0; p < KQ_ITEMS; ++p) {
            const int idx = tid + p * NT;
            const int tt = idx / kd4, j4 = idx - tt * kd4;
            if (tt < kC) {
                *reinterpret_cast<f32x4 *>(&sK[buf][tt][j4 * 4]) = rk[p];
                *reinterpret_cast<f32x4 *>(&sQ[buf][tt][j4 * 4]) = rq[p];
            }
        }
        if (tid < kC * kRowsWG / 4) *reinterpret_cast<f32x4 *>(&sV[buf][tid / 16][(tid % 16) * 4]) = rv;
        // lanes 16..31 hold the 16 decays: one row of the wavefront
        const float g_run = row_prefix_sum(rs);
        const float g_last = __shfl(g_run, 2 * kC - 1, kWave);
        if (tid < kC) {
            sBeta[buf][tid] = rs;
        } else if (tid < 2 * kC) {
            sG[buf][tid - kC] = g_run;
            sEg[buf][tid - kC] = expf(g_run);
            sEt[buf][tid - kC] = expf(g_last - g_run);
        }
    };
    // One quarter of the next chunk's products (wavefront w of the first key
    // half, one per SIMD): w = 0, 1 -> K K^T, w = 2, 3 -> Q K^T, each over half
    // of the key dimension; lane l, register j holds entry [4(l/16) + j][l%16]
    auto products = [&](int buf) {
        const float(*x)[KS] = w < 2 ? sK[buf] : sQ[buf];
        const int half = w & 1;
        f32x4 part[4] = {};
        if constexpr (KB == 1) {
            const f32x4 xa = *reinterpret_cast<const f32x4 *>(&x[lr][4 * lg]);
            const f32x4 ka = *reinterpret_cast<const f32x4 *>(&sK[buf][lr][4 * lg]);
            part[0] = mfma4(half ? xa[2] : xa[0], half ? ka[2] : ka[0], part[0]);
            part[1] = mfma4(half ? xa[3] : xa[1], half ? ka[3] : ka[1], part[1]);
        } else {
#pragma unroll
            for (int ii = 0; ii < KB / 2; ++ii) {
                const int i = half * (KB / 2) + ii;
                const f32x4 xa = *reinterpret_cast<const f32x4 *>(&x[lr][16 * i + 4 * lg]);
                const f32x4 ka = *reinterpret_cast<const f32x4 *>(&sK[buf][lr][16 * i + 4 * lg]);
#pragma unroll
                for (int j = 0; j < 4; ++j) part[j] = mfma4(xa[j], ka[j], part[j]);
            }
        }
        const f32x4 acc = (part[0] + part[1]) + (part[2] + part[3]);
#pragma unroll
        for (int j = 0; j < 4; ++j) sProd[w][4 * lg + j][lr] = acc[j];
    };
    // A and P of the chunk in buffer `buf` from the partial products: wavefront
    // j of the four calling forms row 4(l/16) + j, column l%16 of both (nothing
    // reads them before the next barrier)
    auto finalize = [&](int buf, int pbn, int j) {
        const float *gs = sG[buf];
        const int i = 4 * lg + j;
        const float kk0 = sProd[0][i][lr], kk1 = sProd[1][i][lr];
        const float qk0 = sProd[2][i][lr], qk1 = sProd[3][i][lr];
        const float gi = gs[i], gp = gs[lr], bi = sBeta[buf][i];
        const bool keep = lr <= i;
        const float e = expf(keep ? gi - gp : 0.0f);
        sA[i][lr] = lr < i ? bi * e * (kk0 + kk1) : 0.0f;
        sP[pbn][i][lr] = keep ? e * (qk0 + qk1) : 0.0f;
    };
    // T = (I + A)^-1 of the chunk in buffer `buf`, stored as Tb = T diag(beta).
    // One wavefront.  Blocked: with A = [[A11, 0], [A21, A22]] in 8x8 blocks,
    // D = diag(T11, T22) comes from forward substitution on both diagonal blocks
    // at once (lane m < 16 owns column m of its block), and T = D - D (N D) with
    // N = [[0, 0], [A21, 0]] (two 16x16 products on the matrix cores;
    // T21 = -T22 A21 T11).
    auto inverse = [&](int buf) {
        if (l < kC) {  // D: the diagonal blocks, zeros elsewhere
            const int m = l, b0 = m & 8, mm = m & 7;
            float arow[8][8];
#pragma unroll
            for (int i = 1; i < 8; ++i)
#pragma unroll
                for (int p = 0; p < i; ++p) arow[i][p] = sA[b0 + i][b0 + p];
            __builtin_amdgcn_sched_barrier(0);  // all reads in flight before the first use
            float col[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) col[i] = i == mm ? 1.0f : 0.0f;
#pragma unroll
            for (int i = 1; i < 8; ++i) {
                float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                for (int p = 0; p < i; p += 2) {
                    s0 = __builtin_fmaf(arow[i][p], col[p], s0);
                    if (p + 1 < i) s1 = __builtin_fmaf(arow[i][p + 1], col[p + 1], s1);
                }
                if (i > mm) col[i] = -(s0 + s1);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                sT[b0 + i][m] = col[i];
                sT[(b0 ^ 8) + i][m] = 0.0f;
            }
        }
        // D is read across lanes below; LDS operations of one wavefront complete
        // in order, the fence keeps the compiler from reordering them
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // X = N D: k-slot s of step i is k = 4s + i (lane group l/16 = s)
        const f32x4 na = *reinterpret_cast<const f32x4 *>(&sA[lr][4 * lg]);
        const float bm = sBeta[buf][lr];
        float db[4], da[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            db[i] = sT[4 * lg + i][lr];  // D[k][lr]
            da[i] = sT[lr][4 * lg + i];  // D[lr][k]
        }
        const bool lower = lr >= 8 && lg < 2;  // N[lr][k] nonzero only for lr >= 8, k < 8
        f32x4 X = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) X = mfma4(lower ? na[i] : 0.0f, db[i], X);
        // Y = D X: X in accumulator layout (register i = row 4(l/16) + i) is the
        // B operand of that same k-slot order
        f32x4 Yd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) Yd = mfma4(da[i], X[i], Yd);
        // T = D - Y; entry (4(l/16) + j, l%16) of D is db[j]
#pragma unroll
        for (int j = 0; j < 4; ++j) sTb[4 * lg + j][lr] = (db[j] - Yd[j]) * bm;
    };
    // outputs of chunk cw (rows of sO[cw & 1]) to memory, by threads 0..nt-1
    auto write_out = [&](int cw, int nt) {
        const int n = min(kC, S - cw * kC);
        const float(*so)[kVS] = sO[cw & 1];
        for (int e = tid; e < kC * kRowsWG; e += nt) {
            const int tt = e / kRowsWG, r = e - tt * kRowsWG;
            if (tt < n && row0 + r < a.vd)
                ob[(int64_t)(cw * kC + tt) * v_tok + r] = from_f32<TO>(so[tt][r]);
        }
    };

    f32x4 st[KBW];  // state key blocks kh*KBW .. kh*KBW + KBW - 1
#pragma unroll
    for (int i = 0; i < KBW; ++i) st[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int chunks = (S + kC - 1) / kC;
    // prologue: chunks 0 and 1 staged, A and P of chunk 0 formed
    fetch(0);
    stage(0);
    if (chunks > 1) {
        fetch(1);
        stage(1);
    }
    __syncthreads();
    if (kh == 0) products(0);
    __syncthreads();
    if (kh == KSPLIT - 1) finalize(0, 0, w);
    __syncthreads();

    for (int c = 0; c < chunks; ++c) {
        const int buf = c % NB, nbuf = (c + 1) % NB, pb = c & 1;
        const bool ahead = c + 1 < chunks;
        // chunk c+2's loads land during both phases; the first key part issues
        // them after its matrix products so the two wavefronts of a SIMD do not
        // queue at the memory unit together
        if (kh != 0 && c + 2 < chunks) fetch(c + 2);

        // phase 1: the previous chunk's outputs or this chunk's inverse first (their
        // latency overlaps the other wavefront's matrix products), then Z = K S0^T
        // and Q S0^T (two chains each) and a quarter of the next chunk's K K^T /
        // Q K^T
        if (wv == kHelper) inverse(buf);
        else if (c > 0) write_out(c - 1, NT - kWave);  // the helper is the last wavefront
        f32x4 Z = {0.f, 0.f, 0.f, 0.f}, Y = {0.f, 0.f, 0.f, 0.f};
        if (live) {
            f32x4 z0 = {}, z1 = {}, y0 = {}, y1 = {};
#pragma unroll
            for (int i = 0; i < KBW; ++i) {
                const int kk = 16 * (kh * KBW + i) + 4 * lg;
                const f32x4 kv = *reinterpret_cast<const f32x4 *>(&sK[buf][lr][kk]);
                const f32x4 qv = *reinterpret_cast<const f32x4 *>(&sQ[buf][lr][kk]);
                z0 = mfma4(kv[0], st[i][0], z0);
                y0 = mfma4(qv[0], st[i][0], y0);
                z1 = mfma4(kv[1], st[i][1], z1);
                y1 = mfma4(qv[1], st[i][1], y1);
                z0 = mfma4(kv[2], st[i][2], z0);
                y0 = mfma4(qv[2], st[i][2], y0);
                z1 = mfma4(kv[3], st[i][3], z1);
                y1 = mfma4(qv[3], st[i][3], y1);
            }
            Z = z0 + z1;
            Y = y0 + y1;
            if constexpr (KSPLIT > 1) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    sPart[(0 * KSPLIT + kh) * 4 + w][4 * lg + j][lr] = Z[j];
                    sPart[(1 * KSPLIT + kh) * 4 + w][4 * lg + j][lr] = Y[j];
                }
            }
        }
        if (kh == 0 && c + 2 < chunks) fetch(c + 2);
        if (ahead && kh == 0) products(nbuf);
        __syncthreads();
        if constexpr (KSPLIT > 1) {  // add the other key half's partial products
            if (live) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    Z[j] += sPart[(0 * KSPLIT + (1 - kh)) * 4 + w][4 * lg + j][lr];
                    Y[j] += sPart[(1 * KSPLIT + (1 - kh)) * 4 + w][4 * lg + j][lr];
                }
            }
        }

        // phase 2: A and P of chunk c+1 first, then U, O and the state update of
        // chunk c; chunk c+2 staged
        if (ahead && kh == KSPLIT - 1) finalize(nbuf, pb ^ 1, w);
        if (live) {
            // R = V - diag(e^g) Z in accumulator layout = the B operand of U = Tb R
            f32x4 R;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float eg = sEg[buf][4 * lg + j];
                R[j] = sV[buf][4 * lg + j][wrow + lr] - eg * Z[j];
                Y[j] *= eg;  // Y = diag(e^g) Q S0^T
            }
            f32x4 U = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i) U = mfma4(sTb[lr][4 * lg + i], R[i], U);
            if (kh == 0) {
                f32x4 O = Y;
#pragma unroll
                for (int i = 0; i < 4; ++i) O = mfma4(sP[pb][lr][4 * lg + i], U[i], O);
#pragma unroll
                for (int j = 0; j < 4; ++j) sO[pb][4 * lg + j][wrow + lr] = O[j];
            }
            // state update; the decay weights e^(g_15 - g_tau) scale U's rows (the
            // lane's register i is token 4(l/16) + i)
            f32x4 Ue;
#pragma unroll
            for (int i = 0; i < 4; ++i) Ue[i] = U[i] * sEt[buf][4 * lg + i];
            const float gll = sEg[buf][kC - 1];
#pragma unroll
            for (int t = 0; t < KBW; ++t) {
                f32x4 acc = st[t] * gll;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc = mfma4(sK[buf][4 * lg + i][16 * (kh * KBW + t) + lr], Ue[i], acc);
                st[t] = acc;
            }
        }
        if (c + 2 < chunks) stage((c + 2) % NB);
        __syncthreads();
    }
    write_out(chunks - 1, NT);
}

}  // namespace
}  // namespace qdc

using namespace qdc;

extern "C" int32_t qdc_delta_scan(void *out, int32_t out_dtype, const float *q, const float *k,
                                  const float *v, const float *beta, const float *decay,
                                  int64_t batch, int64_t seq, int64_t heads, int64_t key_heads,
                                  int64_t key_dim, int64_t value_dim, int64_t ld_qk, int64_t ld_v,
                                  hipStream_t stream) {
    if (!valid_dtype(out_dtype)) return QDC_ERR_DTYPE;
    if (batch < 0 || seq < 0 || heads <= 0 || key_heads <= 0 || value_dim <= 0 ||
        heads % key_heads)
        return QDC_ERR_SHAPE;
    if (key_dim <= 0 || key_dim > 256) return QDC_ERR_SHAPE;
    if (ld_qk < key_heads * key_dim || ld_v < heads * value_dim) return QDC_ERR_SHAPE;
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
    a.ld_qk = ld_qk;
    a.ld_v = ld_v;
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
    // matrix-core chunked form: key_dim a multiple of 16 (<= 256), value_dim of 16
    if (key_dim % 16 == 0 && value_dim % 16 == 0 && aligned16(q) && aligned16(k) &&
        aligned16(v) && ld_qk % 4 == 0 && ld_v % 4 == 0) {
        const dim3 cgrid((uint32_t)ceil_div(value_dim, kRowsWG), (uint32_t)heads,
                         (uint32_t)batch);
#define QDC_CHUNKED(KB, KSPLIT)                                                                \
    if (key_dim == 16 * KB) {                                                                  \
        if (out_dtype == QDC_BF16)                                                             \
            hipLaunchKernelGGL((delta_scan_chunked<KB, KSPLIT, bf16_t>), cgrid,                \
                               dim3(kBlock * KSPLIT), 0, stream, a);                           \
        else                                                                                   \
            hipLaunchKernelGGL((delta_scan_chunked<KB, KSPLIT, float>), cgrid,                 \
                               dim3(kBlock * KSPLIT), 0, stream, a);                           \
        return launch_status();                                                                \
    }
        QDC_CHUNKED(1, 1)
        QDC_CHUNKED(2, 2)
        QDC_CHUNKED(4, 2)
        QDC_CHUNKED(8, 2)
        QDC_CHUNKED(16, 2)
#undef QDC_CHUNKED
    }
    const bool vec = aligned16(q) && aligned16(k) && key_dim % 4 == 0 && ld_qk % 4 == 0;
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

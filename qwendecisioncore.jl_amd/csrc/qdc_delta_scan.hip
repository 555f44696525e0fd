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
// Mapping: a wavefront is 4 groups of 16 lanes; each group owns R consecutive
// value rows of one (b, h) and splits the key dimension across its lanes (lane
// i holds key components i*KPL .. i*KPL+KPL-1, loaded as 16-byte chunks), so
// both dot products per row and token reduce over 16 lanes with 4 DPP steps and
// no cross-row traffic.  The state (R x KPL values per lane) stays in
// registers; the next token's k, q, v, beta and decay are loaded while the
// current token is computed.
#include "qdc_common.hpp"

namespace qdc {
namespace {

constexpr int kGroup = 16;        // lanes per key split
constexpr int kGroups = kWave / kGroup;
constexpr int kRowsPerGroup = 2;  // value rows per 16-lane group

template <int KPL> __device__ __forceinline__ void load_keys(const float *p, bool full, int valid,
                                                             float (&out)[KPL]) {
    if (KPL % 4 == 0 && full) {
#pragma unroll
        for (int i = 0; i < KPL; i += 4) {
            const f32x4 c = *reinterpret_cast<const f32x4 *>(p + i);
            out[i] = c.x; out[i + 1] = c.y; out[i + 2] = c.z; out[i + 3] = c.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < KPL; ++i) out[i] = i < valid ? p[i] : 0.0f;
    }
}

template <int KPL, typename TO>
__global__ __launch_bounds__(kWave) void delta_scan(
    TO *__restrict__ out, const float *__restrict__ q, const float *__restrict__ k,
    const float *__restrict__ v, const float *__restrict__ beta, const float *__restrict__ decay,
    int S, int H, int KH, int KD, int vd, int groups, bool vec) {
    constexpr int R = kRowsPerGroup;
    const int lane = threadIdx.x % kGroup;
    const int grp = threadIdx.x / kGroup;
    const int r0 = (blockIdx.x * kGroups + grp) * R;  // first value row of this group
    const int h = blockIdx.y, b = blockIdx.z;
    const int g = h / groups;
    // this lane's key components [j0, j0 + valid); lanes past key_dim hold zeros
    const int j0 = lane * KPL;
    const int valid = max(0, min(KPL, KD - j0));
    // 16-byte key loads need 16-byte aligned q/k and key_dim % 4 == 0 (checked on the host)
    const bool full = vec && valid == KPL;
    const int64_t k_tok = (int64_t)KH * KD, v_tok = (int64_t)H * vd, s_tok = H;
    const float *kp = k + (int64_t)b * S * k_tok + (int64_t)g * KD + min(j0, KD - 1);
    const float *qp = q + (int64_t)b * S * k_tok + (int64_t)g * KD + min(j0, KD - 1);
    const float *vp = v + (int64_t)b * S * v_tok + (int64_t)h * vd;
    const float *bp = beta + (int64_t)b * S * s_tok + h;
    const float *dp = decay + (int64_t)b * S * s_tok + h;
    TO *op = out + (int64_t)b * S * v_tok + (int64_t)h * vd;

    float st[R][KPL];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < KPL; ++i) st[r][i] = 0.0f;

    float kn[KPL], qn[KPL], vn[R], bn = 0.0f, dn = 0.0f;
    auto fetch = [&](int t) {
        load_keys<KPL>(kp + (int64_t)t * k_tok, full, valid, kn);
        load_keys<KPL>(qp + (int64_t)t * k_tok, full, valid, qn);
#pragma unroll
        for (int r = 0; r < R; ++r) vn[r] = r0 + r < vd ? vp[(int64_t)t * v_tok + r0 + r] : 0.0f;
        bn = bp[(int64_t)t * s_tok];
        dn = dp[(int64_t)t * s_tok];
    };
    if (S > 0) fetch(0);
    for (int t = 0; t < S; ++t) {
        float kt[KPL], qt[KPL], vt[R];
#pragma unroll
        for (int i = 0; i < KPL; ++i) {
            kt[i] = kn[i];
            qt[i] = qn[i];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) vt[r] = vn[r];
        const float bt = bn, f = __expf(dn);
        if (t + 1 < S) fetch(t + 1);

        float pred[R], o[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < KPL; ++i) s += st[r][i] * kt[i];
            pred[r] = group_sum<kGroup>(s);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float u = bt * (vt[r] - f * pred[r]);
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < KPL; ++i) {
                st[r][i] = f * st[r][i] + u * kt[i];
                s += st[r][i] * qt[i];
            }
            o[r] = group_sum<kGroup>(s);
        }
        // lane r of the group stores row r0 + r
        float mine = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) mine = lane == r ? o[r] : mine;
        if (lane < R && r0 + lane < vd) op[(int64_t)t * v_tok + r0 + lane] = from_f32<TO>(mine);
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
    const int rows_per_block = kGroups * kRowsPerGroup;
    const dim3 grid((uint32_t)ceil_div(value_dim, rows_per_block), (uint32_t)heads,
                    (uint32_t)batch);
    const int groups = (int)(heads / key_heads);
    const int S = (int)seq, H = (int)heads, KH = (int)key_heads, KD = (int)key_dim;
    const int vd = (int)value_dim;
#define QDC_SCAN(KPL, TO)                                                                       \
    hipLaunchKernelGGL((delta_scan<KPL, TO>), grid, dim3(kWave), 0, stream, (TO *)out, q, k, v,  \
                       beta, decay, S, H, KH, KD, vd, groups, vec);                              \
    return launch_status();
    const int64_t kpl = ceil_div(key_dim, kGroup);
    const bool vec = aligned16(q) && aligned16(k) && key_dim % 4 == 0;
    if (out_dtype == QDC_BF16) {
        if (kpl <= 1) { QDC_SCAN(1, bf16_t) }
        if (kpl <= 2) { QDC_SCAN(2, bf16_t) }
        if (kpl <= 4) { QDC_SCAN(4, bf16_t) }
        if (kpl <= 8) { QDC_SCAN(8, bf16_t) }
        QDC_SCAN(16, bf16_t)
    }
    if (kpl <= 1) { QDC_SCAN(1, float) }
    if (kpl <= 2) { QDC_SCAN(2, float) }
    if (kpl <= 4) { QDC_SCAN(4, float) }
    if (kpl <= 8) { QDC_SCAN(8, float) }
    QDC_SCAN(16, float)
#undef QDC_SCAN
}

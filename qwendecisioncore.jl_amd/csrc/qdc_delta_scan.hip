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
// Mapping: one wavefront per (b, h, group of R value rows).  Lane l holds the
// key components l, l+64, ... of each of its R state rows in registers; the
// two dot products per row and token are reduced across the wavefront (DPP
// inside 16-lane rows, permutes across them).  The next token's k, q, v, beta
// and decay are loaded while the current token is computed.
#include "qdc_common.hpp"

namespace qdc {
namespace {

constexpr int kRows = 8;  // value rows per wavefront

template <int KPL, typename TO>
__global__ __launch_bounds__(kWave) void delta_scan(
    TO *__restrict__ out, const float *__restrict__ q, const float *__restrict__ k,
    const float *__restrict__ v, const float *__restrict__ beta, const float *__restrict__ decay,
    int S, int H, int KH, int KD, int vd, int groups) {
    // lanes past key_dim hold zero key/query components and so add nothing
    const int lane = threadIdx.x;
    const int r0 = blockIdx.x * kRows;
    const int h = blockIdx.y, b = blockIdx.z;
    const int g = h / groups;
    // element strides of the [B, S, heads, dim] inputs
    const int64_t k_tok = (int64_t)KH * KD, v_tok = (int64_t)H * vd, s_tok = H;
    const float *kp = k + (int64_t)b * S * k_tok + (int64_t)g * KD + lane;
    const float *qp = q + (int64_t)b * S * k_tok + (int64_t)g * KD + lane;
    const float *vp = v + (int64_t)b * S * v_tok + (int64_t)h * vd + r0;
    const float *bp = beta + (int64_t)b * S * s_tok + h;
    const float *dp = decay + (int64_t)b * S * s_tok + h;
    TO *op = out + (int64_t)b * S * v_tok + (int64_t)h * vd + r0;
    const int rows = min(kRows, vd - r0);

    float st[kRows][KPL];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
#pragma unroll
        for (int i = 0; i < KPL; ++i) st[r][i] = 0.0f;

    // token-t operands, prefetched one token ahead
    float kn[KPL], qn[KPL], vn[kRows], bn = 0.0f, dn = 0.0f;
    auto fetch = [&](int t) {
#pragma unroll
        for (int i = 0; i < KPL; ++i) {
            const bool in = lane + i * kWave < KD;
            kn[i] = in ? kp[(int64_t)t * k_tok + i * kWave] : 0.0f;
            qn[i] = in ? qp[(int64_t)t * k_tok + i * kWave] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r) vn[r] = r < rows ? vp[(int64_t)t * v_tok + r] : 0.0f;
        bn = bp[(int64_t)t * s_tok];
        dn = dp[(int64_t)t * s_tok];
    };
    if (S > 0) fetch(0);
    for (int t = 0; t < S; ++t) {
        float kt[KPL], qt[KPL], vt[kRows];
#pragma unroll
        for (int i = 0; i < KPL; ++i) {
            kt[i] = kn[i];
            qt[i] = qn[i];
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r) vt[r] = vn[r];
        const float bt = bn, f = __expf(dn);
        if (t + 1 < S) fetch(t + 1);

        float pred[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < KPL; ++i) s += st[r][i] * kt[i];
            pred[r] = s;
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r) pred[r] = group_sum<kWave>(pred[r]);
        float o[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const float u = bt * (vt[r] - f * pred[r]);
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < KPL; ++i) {
                st[r][i] = f * st[r][i] + u * kt[i];
                s += st[r][i] * qt[i];
            }
            o[r] = s;
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r) o[r] = group_sum<kWave>(o[r]);
        // lane r stores row r: one coalesced store of the wavefront's rows
        float mine = 0.0f;
#pragma unroll
        for (int r = 0; r < kRows; ++r) mine = lane == r ? o[r] : mine;
        if (lane < rows) op[(int64_t)t * v_tok + lane] = from_f32<TO>(mine);
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
    const dim3 grid((uint32_t)ceil_div(value_dim, kRows), (uint32_t)heads, (uint32_t)batch);
    const int groups = (int)(heads / key_heads);
    const int S = (int)seq, H = (int)heads, KH = (int)key_heads, KD = (int)key_dim;
    const int vd = (int)value_dim;
#define QDC_SCAN(KPL, TO)                                                                       \
    hipLaunchKernelGGL((delta_scan<KPL, TO>), grid, dim3(kWave), 0, stream, (TO *)out, q, k, v,  \
                       beta, decay, S, H, KH, KD, vd, groups);                                   \
    return launch_status();
    if (out_dtype == QDC_BF16) {
        if (key_dim <= 64) { QDC_SCAN(1, bf16_t) }
        if (key_dim <= 128) { QDC_SCAN(2, bf16_t) }
        QDC_SCAN(4, bf16_t)
    }
    if (key_dim <= 64) { QDC_SCAN(1, float) }
    if (key_dim <= 128) { QDC_SCAN(2, float) }
    QDC_SCAN(4, float)
#undef QDC_SCAN
}

// qdc_rmsnorm.hip -- RMSNorm row kernels for gfx950:
//   qdc_rmsnorm          zero-centred (or plain) RMSNorm of strided rows
//   qdc_residual_rmsnorm residual = x + mixed, then zero-centred RMSNorm
//   qdc_gated_rmsnorm    DeltaNet output norm fused with silu(z)
//
// Fast path: a row of W elements is split into C = W*sizeof(T)/16 chunks of
// 16 bytes.  A group of LPR = min(C, 64) lanes owns a row; lane l holds chunks
// l, l+LPR, ... (CPL = C/LPR chunks, so every load instruction of the group is
// one contiguous LPR*16-byte segment).  The row stays in registers: HBM sees
// each input byte read once and each output byte written once.  The sum of
// squares is reduced across the group with xor-shuffles; 64/LPR rows share a
// wavefront, 4 wavefronts a workgroup.
//
// General path (any width, stride or alignment): one wavefront per row, scalar
// strided accesses, two passes over the row (the second from cache).
#include "qdc_common.hpp"

namespace qdc {
namespace {

enum class Mode { kPlain, kResidual, kGated };

// Row addressing: row r = (t, h) with t = r / heads, h = r % heads.
struct RowMap {
    FastDiv heads;
    int64_t x_tok, x_head;  // input (and residual-input `mixed` shares x's map)
    int64_t z_tok, z_head;  // gate input (gated mode)
    int64_t o_tok, o_head;  // output (and residual output)
};

template <typename T, int LPR, int CPL, Mode M, bool CENTERED>
__global__ __launch_bounds__(kBlock) void rms_rows_fast(
    T *out, T *res_out, const T *x, const T *mixed, const T *__restrict__ z,
    const T *__restrict__ w, int64_t rows, RowMap map, float width, float eps) {
    constexpr int V = Elem<T>::kVec;
    constexpr int RPB = kBlock / LPR;  // rows per workgroup
    const int lane = threadIdx.x % LPR;
    const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
    const bool active = row < rows;

    int64_t xo = 0, zo = 0, oo = 0;
    if (active) {
        const uint32_t t = fastdiv((uint32_t)row, map.heads);
        const uint32_t h = (uint32_t)row - t * map.heads.d;
        xo = (int64_t)t * map.x_tok + (int64_t)h * map.x_head;
        zo = (int64_t)t * map.z_tok + (int64_t)h * map.z_head;
        oo = (int64_t)t * map.o_tok + (int64_t)h * map.o_head;
    }

    // Issue every load of the row (x, mixed, gate, weights) before the first
    // dependent instruction so their latencies overlap.
    u32x4 xr[CPL], mr[M == Mode::kResidual ? CPL : 1], zr[M == Mode::kGated ? CPL : 1], wr[CPL];
    if (active) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) xr[c] = load_stream(x + xo + (c * LPR + lane) * V);
        if constexpr (M == Mode::kResidual) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) mr[c] = load_stream(mixed + xo + (c * LPR + lane) * V);
        }
        if constexpr (M == Mode::kGated) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) zr[c] = load_stream(z + zo + (c * LPR + lane) * V);
        }
#pragma unroll
        for (int c = 0; c < CPL; ++c) wr[c] = load_raw(w + (c * LPR + lane) * V);
    }

    float v[CPL][V];
    float ss = 0.0f;
    if (active) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            unpack(xr[c], v[c]);
            if constexpr (M == Mode::kResidual) {
                float m[V];
                unpack(mr[c], m);
#pragma unroll
                for (int j = 0; j < V; ++j) v[c][j] = v[c][j] + m[j];
                store_chunk(res_out + oo + (c * LPR + lane) * V, v[c]);
            }
#pragma unroll
            for (int j = 0; j < V; ++j) ss += v[c][j] * v[c][j];
        }
    }
    ss = group_sum<LPR>(ss);
    if (!active) return;
    const float s = rms_scale(ss, width, eps);

#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        float wv[V], o[V];
        unpack(wr[c], wv);
        if constexpr (M == Mode::kGated) {
            float g[V];
            unpack(zr[c], g);
#pragma unroll
            for (int j = 0; j < V; ++j) o[j] = ((v[c][j] * s) * wv[j]) * silu(g[j]);
        } else {
#pragma unroll
            for (int j = 0; j < V; ++j)
                o[j] = (v[c][j] * s) * (CENTERED ? (1.0f + wv[j]) : wv[j]);
        }
        store_chunk(out + oo + (c * LPR + lane) * V, o);
    }
}

// One wavefront per row, any width/stride/alignment.
template <typename T, Mode M, bool CENTERED>
__global__ __launch_bounds__(kBlock) void rms_rows_general(
    T *out, T *res_out, const T *x, const T *mixed, const T *__restrict__ z,
    const T *__restrict__ w,
    int64_t rows, RowMap map, int64_t width, float eps) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = (int64_t)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;  // uniform per wavefront
    const uint32_t t = fastdiv((uint32_t)row, map.heads);
    const uint32_t h = (uint32_t)row - t * map.heads.d;
    const T *xr = x + (int64_t)t * map.x_tok + (int64_t)h * map.x_head;
    const T *zr = z + (int64_t)t * map.z_tok + (int64_t)h * map.z_head;
    const int64_t oo = (int64_t)t * map.o_tok + (int64_t)h * map.o_head;
    float ss = 0.0f;
    for (int64_t i = lane; i < width; i += kWave) {
        float v = to_f32(xr[i]);
        if constexpr (M == Mode::kResidual) {
            v = v + to_f32(mixed[(xr - x) + i]);
            res_out[oo + i] = from_f32<T>(v);
        }
        ss += v * v;
    }
    ss = group_sum<kWave>(ss);
    const float s = rms_scale(ss, (float)width, eps);
    for (int64_t i = lane; i < width; i += kWave) {
        // the residual may overwrite x or mixed in place: read back what this
        // lane stored in the first pass
        const float v = M == Mode::kResidual ? to_f32(res_out[oo + i]) : to_f32(xr[i]);
        const float wv = to_f32(w[i]);
        float o;
        if constexpr (M == Mode::kGated) {
            o = ((v * s) * wv) * silu(to_f32(zr[i]));
        } else {
            o = (v * s) * (CENTERED ? (1.0f + wv) : wv);
        }
        out[oo + i] = from_f32<T>(o);
    }
}

template <typename T, int LPR, int CPL, Mode M, bool C>
int32_t launch_fast(T *out, T *res, const T *x, const T *mixed, const T *z, const T *w,
                    int64_t rows, const RowMap &map, int64_t width, float eps,
                    hipStream_t stream) {
    const int64_t blocks = ceil_div(rows, kBlock / LPR);
    hipLaunchKernelGGL((rms_rows_fast<T, LPR, CPL, M, C>), dim3((uint32_t)blocks), dim3(kBlock), 0,
                       stream, out, res, x, mixed, z, w, rows, map, (float)width, eps);
    return launch_status();
}

// Fast-path shapes by C = chunks per row: a lane holds 2 chunks (32 bytes in
// flight) for rows of up to 64 chunks and 4 chunks (64 bytes) for 128- and
// 256-chunk rows, which measured fastest on MI355X; wider rows use all 64
// lanes with C/64 chunks each.  kNoFastPath when no instantiation matches.
template <typename T, Mode M, bool C>
int32_t dispatch_fast(T *out, T *res, const T *x, const T *mixed, const T *z, const T *w,
                      int64_t rows, const RowMap &map, int64_t width, float eps,
                      hipStream_t stream) {
    const int64_t chunks = width / Elem<T>::kVec;
#define QDC_FAST(LPR, CPL)                                                                    \
    case LPR * CPL:                                                                           \
        return launch_fast<T, LPR, CPL, M, C>(out, res, x, mixed, z, w, rows, map, width, eps, \
                                              stream);
    switch (chunks) {
        QDC_FAST(1, 1)
        QDC_FAST(1, 2)
        QDC_FAST(2, 2)
        QDC_FAST(4, 2)
        QDC_FAST(8, 2)
        QDC_FAST(16, 2)
        QDC_FAST(32, 2)
        QDC_FAST(32, 4)
        QDC_FAST(64, 3)
        QDC_FAST(64, 4)
        QDC_FAST(64, 5)
        QDC_FAST(64, 6)
        QDC_FAST(64, 7)
        QDC_FAST(64, 8)
        QDC_FAST(64, 10)
        QDC_FAST(64, 12)
        QDC_FAST(64, 16)
        default:
            return kNoFastPath;
    }
#undef QDC_FAST
}

template <typename T, Mode M, bool C>
int32_t run(T *out, T *res, const T *x, const T *mixed, const T *z, const T *w, int64_t rows,
            const RowMap &map, int64_t width, float eps, bool fast, hipStream_t stream) {
    if (fast && width % Elem<T>::kVec == 0) {
        const int32_t rc = dispatch_fast<T, M, C>(out, res, x, mixed, z, w, rows, map, width, eps,
                                                  stream);
        if (rc != kNoFastPath) return rc;
    }
    const int64_t blocks = ceil_div(rows, kBlock / kWave);
    hipLaunchKernelGGL((rms_rows_general<T, M, C>), dim3((uint32_t)blocks), dim3(kBlock), 0, stream,
                       out, res, x, mixed, z, w, rows, map, width, eps);
    return launch_status();
}

template <Mode M, bool C>
int32_t run_dtype(int32_t dtype, void *out, void *res, const void *x, const void *mixed,
                  const void *z, const void *w, int64_t rows, const RowMap &map, int64_t width,
                  float eps, bool fast, hipStream_t stream) {
    if (dtype == QDC_BF16)
        return run<bf16_t, M, C>((bf16_t *)out, (bf16_t *)res, (const bf16_t *)x,
                                 (const bf16_t *)mixed, (const bf16_t *)z, (const bf16_t *)w, rows,
                                 map, width, eps, fast, stream);
    return run<float, M, C>((float *)out, (float *)res, (const float *)x, (const float *)mixed,
                            (const float *)z, (const float *)w, rows, map, width, eps, fast,
                            stream);
}

// Rows are addressed with 32-bit row indices in the kernels.
constexpr int64_t kMaxRows = (int64_t)1 << 31;

}  // namespace
}  // namespace qdc

using namespace qdc;

extern "C" int32_t qdc_rmsnorm(void *out, const void *x, const void *weight, int64_t rows,
                               int64_t width, int64_t ld_x, int64_t ld_out, float eps,
                               int32_t centered, int32_t dtype, hipStream_t stream) {
    if (!valid_dtype(dtype)) return QDC_ERR_DTYPE;
    if (rows < 0 || width < 0 || rows >= kMaxRows) return QDC_ERR_SHAPE;
    if (rows == 0 || width == 0) return QDC_OK;
    if (!out || !x || !weight) return QDC_ERR_NULL;
    if (ld_x < width || ld_out < width) return QDC_ERR_SHAPE;
    const int64_t es = elem_size(dtype);
    if (out != x && overlaps(out, ((rows - 1) * ld_out + width) * es, x,
                             ((rows - 1) * ld_x + width) * es))
        return QDC_ERR_ALIAS;
    if (out == x && ld_out != ld_x) return QDC_ERR_ALIAS;
    RowMap map{make_fastdiv(1), ld_x, 0, 0, 0, ld_out, 0};
    const bool fast = aligned16(out) && aligned16(x) && aligned16(weight) &&
                      (ld_x * es) % 16 == 0 && (ld_out * es) % 16 == 0;
    if (centered)
        return run_dtype<Mode::kPlain, true>(dtype, out, nullptr, x, nullptr, nullptr, weight, rows,
                                             map, width, eps, fast, stream);
    return run_dtype<Mode::kPlain, false>(dtype, out, nullptr, x, nullptr, nullptr, weight, rows,
                                          map, width, eps, fast, stream);
}

extern "C" int32_t qdc_residual_rmsnorm(void *residual, void *out, const void *x,
                                        const void *mixed, const void *weight, int64_t rows,
                                        int64_t width, float eps, int32_t dtype,
                                        hipStream_t stream) {
    if (!valid_dtype(dtype)) return QDC_ERR_DTYPE;
    if (rows < 0 || width < 0 || rows >= kMaxRows) return QDC_ERR_SHAPE;
    if (rows == 0 || width == 0) return QDC_OK;
    if (!residual || !out || !x || !mixed || !weight) return QDC_ERR_NULL;
    const int64_t bytes = rows * width * elem_size(dtype);
    if (overlaps(residual, bytes, out, bytes)) return QDC_ERR_ALIAS;
    for (const void *in : {x, mixed}) {
        if (residual != in && overlaps(residual, bytes, in, bytes)) return QDC_ERR_ALIAS;
        if (out != in && overlaps(out, bytes, in, bytes)) return QDC_ERR_ALIAS;
    }
    RowMap map{make_fastdiv(1), width, 0, 0, 0, width, 0};
    const bool fast = aligned16(residual) && aligned16(out) && aligned16(x) && aligned16(mixed) &&
                      aligned16(weight) && (width * elem_size(dtype)) % 16 == 0;
    return run_dtype<Mode::kResidual, true>(dtype, out, residual, x, mixed, nullptr, weight, rows,
                                            map, width, eps, fast, stream);
}

extern "C" int32_t qdc_gated_rmsnorm(void *out, const void *x, const void *z, const void *weight,
                                     int64_t tokens, int64_t heads, int64_t width, int64_t x_tok,
                                     int64_t z_tok, int64_t out_tok, float eps, int32_t dtype,
                                     hipStream_t stream) {
    if (!valid_dtype(dtype)) return QDC_ERR_DTYPE;
    if (tokens < 0 || heads < 0 || width < 0) return QDC_ERR_SHAPE;
    if (tokens == 0 || heads == 0 || width == 0) return QDC_OK;
    if (!out || !x || !z || !weight) return QDC_ERR_NULL;
    if (tokens * heads >= kMaxRows || heads >= kMaxRows) return QDC_ERR_SHAPE;
    if (x_tok < heads * width || z_tok < heads * width || out_tok < heads * width)
        return QDC_ERR_SHAPE;
    const int64_t es = elem_size(dtype);
    const int64_t span_o = ((tokens - 1) * out_tok + heads * width) * es;
    if (out != x && overlaps(out, span_o, x, ((tokens - 1) * x_tok + heads * width) * es))
        return QDC_ERR_ALIAS;
    if (out == x && out_tok != x_tok) return QDC_ERR_ALIAS;
    if (overlaps(out, span_o, z, ((tokens - 1) * z_tok + heads * width) * es)) return QDC_ERR_ALIAS;
    RowMap map{make_fastdiv((uint32_t)heads), x_tok, width, z_tok, width, out_tok, width};
    const bool fast = aligned16(out) && aligned16(x) && aligned16(z) && aligned16(weight) &&
                      (width * es) % 16 == 0 && (x_tok * es) % 16 == 0 &&
                      (z_tok * es) % 16 == 0 && (out_tok * es) % 16 == 0;
    return run_dtype<Mode::kGated, false>(dtype, out, nullptr, x, nullptr, z, weight,
                                          tokens * heads, map, width, eps, fast, stream);
}

// qdc_swiglu.hip -- SwiGLU out = silu(gate) * up for gfx950.
//
// Types: TI is gate and up, TO the output (the same type, or the split
// two-term bf16 form of fp32 values).
//
// Fast path: the [tokens, width] output is cut into 16-byte chunks numbered
// row-major; each thread handles kUnroll chunks spaced one workgroup apart,
// issuing all gate/up loads before any arithmetic.  Token/column of a chunk
// come from one multiply-high division by the chunks-per-row count, so gate
// and up may be separate tensors or the two halves of the packed gate||up
// GEMM output (ld = 2*width) without any extra copy.
#include <algorithm>

#include "qdc_common.hpp"

namespace qdc {
namespace {

constexpr int kUnroll = 1;

template <typename TI, typename TO>
__global__ __launch_bounds__(kBlock) void swiglu_fast(TO *out, const TI *gate, const TI *up,
                                                      uint32_t total_chunks, FastDiv per_row,
                                                      int64_t ld_gate, int64_t ld_up,
                                                      int64_t ld_out) {
    constexpr int V = Elem<TI>::kVec;
    const uint32_t base = blockIdx.x * (uint32_t)(kBlock * kUnroll) + threadIdx.x;
    float g[kUnroll][V], u[kUnroll][V];
    int64_t oo[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
        const uint32_t idx = base + (uint32_t)(k * kBlock);
        oo[k] = -1;
        if (idx < total_chunks) {
            const uint32_t t = fastdiv(idx, per_row);
            const int64_t col = (int64_t)(idx - t * per_row.d) * V;
            unpack(load_stream(gate + (int64_t)t * ld_gate + col), g[k]);
            unpack(load_stream(up + (int64_t)t * ld_up + col), u[k]);
            oo[k] = (int64_t)t * ld_out + col;
        }
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
        if (oo[k] < 0) continue;
        float o[V];
#pragma unroll
        for (int j = 0; j < V; ++j) o[j] = silu(g[k][j]) * u[k][j];
        store_chunk(out + oo[k], o);
    }
}

// Element-wise, any width/stride/alignment.
template <typename TI, typename TO>
__global__ __launch_bounds__(kBlock) void swiglu_general(TO *out, const TI *gate, const TI *up,
                                                         int64_t tokens, int64_t width,
                                                         int64_t ld_gate, int64_t ld_up,
                                                         int64_t ld_out) {
    const int64_t total = tokens * width;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kBlock) {
        const int64_t t = i / width, c = i - t * width;
        const float g = to_f32(gate[t * ld_gate + c]);
        const float u = to_f32(up[t * ld_up + c]);
        put_elem(out, t * ld_out + c, silu(g) * u);
    }
}

template <typename TI, typename TO>
int32_t launch(void *out, const void *gate, const void *up, int64_t tokens, int64_t width,
               int64_t ld_gate, int64_t ld_up, int64_t ld_out, bool fast, hipStream_t stream) {
    constexpr int V = Elem<TI>::kVec;
    const int64_t chunks = tokens * (width / V);
    if (fast && width % V == 0 && chunks < ((int64_t)1 << 31)) {
        const int64_t blocks = ceil_div(chunks, kBlock * kUnroll);
        hipLaunchKernelGGL((swiglu_fast<TI, TO>), dim3((uint32_t)blocks), dim3(kBlock), 0,
                           stream, (TO *)out, (const TI *)gate, (const TI *)up, (uint32_t)chunks,
                           make_fastdiv((uint32_t)(width / V)), ld_gate, ld_up, ld_out);
    } else {
        const int64_t blocks = std::min<int64_t>(ceil_div(tokens * width, kBlock), 1 << 20);
        hipLaunchKernelGGL((swiglu_general<TI, TO>), dim3((uint32_t)blocks), dim3(kBlock), 0,
                           stream, (TO *)out, (const TI *)gate, (const TI *)up, tokens, width,
                           ld_gate, ld_up, ld_out);
    }
    return launch_status();
}

}  // namespace
}  // namespace qdc

using namespace qdc;

extern "C" int32_t qdc_swiglu(void *out, const void *gate, const void *up, int64_t tokens,
                              int64_t width, int64_t ld_gate, int64_t ld_up, int64_t ld_out,
                              int32_t dtype, int32_t out_dtype, hipStream_t stream) {
    // out in dtype, or fp32 gate and up with the split output
    const bool split = dtype == QDC_F32 && out_dtype == QDC_BF16X2;
    if (!valid_dtype(dtype) || !(out_dtype == dtype || split)) return QDC_ERR_DTYPE;
    if (tokens < 0 || width < 0) return QDC_ERR_SHAPE;
    if (tokens == 0 || width == 0) return QDC_OK;
    if (!out || !gate || !up) return QDC_ERR_NULL;
    if (ld_gate < width || ld_up < width || ld_out < width) return QDC_ERR_SHAPE;
    if (width >= ((int64_t)1 << 31)) return QDC_ERR_SHAPE;
    if (split && !split_rows_ok(width, ld_out)) return QDC_ERR_SHAPE;
    const int64_t es = elem_size(dtype), eo = elem_size(out_dtype);
    const int64_t span_o = ((tokens - 1) * ld_out + width) * eo;
    // In place is allowed only element-for-element (same base, stride and type).
    if (!(out == gate && ld_out == ld_gate && !split) &&
        overlaps(out, span_o, gate, ((tokens - 1) * ld_gate + width) * es))
        return QDC_ERR_ALIAS;
    if (!(out == up && ld_out == ld_up && !split) &&
        overlaps(out, span_o, up, ((tokens - 1) * ld_up + width) * es))
        return QDC_ERR_ALIAS;
    const bool fast = aligned16(out) && aligned16(gate) && aligned16(up) &&
                      (ld_gate * es) % 16 == 0 && (ld_up * es) % 16 == 0 &&
                      (ld_out * eo) % 16 == 0;
    if (split)
        return launch<float, split_t>(out, gate, up, tokens, width, ld_gate, ld_up, ld_out, fast,
                                      stream);
    if (dtype == QDC_BF16)
        return launch<bf16_t, bf16_t>(out, gate, up, tokens, width, ld_gate, ld_up, ld_out, fast,
                                      stream);
    return launch<float, float>(out, gate, up, tokens, width, ld_gate, ld_up, ld_out, fast,
                                stream);
}

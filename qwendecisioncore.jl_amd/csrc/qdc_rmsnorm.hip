// qdc_rmsnorm.hip -- RMSNorm row kernels for gfx950:
//   qdc_rmsnorm          zero-centred (or plain) RMSNorm of strided rows
//   qdc_residual_rmsnorm residual = x + mixed, then zero-centred RMSNorm
//   qdc_gated_rmsnorm    DeltaNet output norm fused with silu(z)
//
// Types: TX is the row input (and the residual stream: x and the residual
// output), TM the `mixed` addend, TO the normalised output and the weight.
// The supported mixes keep the residual stream in fp32 while the activations
// fed to the GEMMs are bf16.
//
// Fast path: a row is split into G = width/V groups of V elements (V = 8 when
// every tensor is bf16, a 16-byte chunk; else 4: a 16-byte chunk of an fp32
// tensor, an 8-byte piece of a bf16 one; 8 elements of a mixed fp32/bf16 row
// per lane split each fp32 group over two accesses 32 bytes apart, which
// measured 12% slower with 7% more bytes written).  A set of LPR lanes owns a
// row; lane l holds groups l, l+LPR, ... (CPL groups), so each load or store
// instruction of the set covers one contiguous segment of every tensor.  All
// loads of a row (x, mixed, gate, weights) are issued before the first
// dependent instruction; streamed inputs use nontemporal loads.  The row
// stays in registers: HBM sees each input byte read once and each output byte
// written once.  The sum of squares is reduced across the LPR lanes (DPP inside
// 16-lane rows, lane swaps across them, and through LDS across the 2 or 4
// wavefronts of a row wider than 64 lanes); 64/LPR rows share a wavefront, 4
// wavefronts a workgroup.
//
// General path (any width, stride or alignment): one wavefront per row, scalar
// strided accesses, two passes over the row (the second from cache).
//
// Optional row mask (plain and residual modes): out row r is multiplied by
// keep[r], an int32 0/1, in fp32 before the store, as the reference's masked
// normalisation store does (ext/metal_normalization.jl:20-28).  The residual
// output is never masked.
#include <initializer_list>

#include "qdc_common.hpp"

namespace qdc {
namespace {

enum class Mode { kPlain, kResidual, kGated };

// Row addressing: row r = (t, h) with t = r / heads, h = r % heads.
struct RowMap {
    FastDiv heads;
    int64_t x_tok, x_head;  // input (the residual-mode addend shares x's map)
    int64_t z_tok, z_head;  // gate input (gated mode)
    int64_t o_tok, o_head;  // output (and residual output)
};

// 8 elements (one 16-byte chunk) per group when every tensor is bf16, else 4
// (16-byte fp32 chunks, 8-byte bf16 pieces)
template <typename TX, typename TM, typename TO> constexpr int group_elems() {
    return (sizeof(TX) == 2 && sizeof(TM) == 2 && sizeof(TO) == 2) ? 8 : 4;
}

template <typename TX, typename TM, typename TO, int LPR, int CPL, Mode M, bool CENTERED>
__global__ __launch_bounds__(kBlock) void rms_rows_fast(
    TO *out, TX *res_out, const TX *x, const TM *mixed, const Aux<TO> *__restrict__ z,
    const Aux<TO> *__restrict__ w, const int32_t *__restrict__ keep, int64_t rows, RowMap map,
    float width, float eps) {
    constexpr int V = group_elems<TX, TM, TO>();
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

    // Issue every load of the row before the first dependent instruction.
    Frag<TX, V> xr[CPL];
    Frag<TM, V> mr[M == Mode::kResidual ? CPL : 1];
    Frag<Aux<TO>, V> zr[M == Mode::kGated ? CPL : 1];
    Frag<Aux<TO>, V> wr[CPL];
    if (active) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) xr[c] = stream_frag<TX, V>(x + xo + (c * LPR + lane) * V);
        if constexpr (M == Mode::kResidual) {
#pragma unroll
            for (int c = 0; c < CPL; ++c)
                mr[c] = stream_frag<TM, V>(mixed + xo + (c * LPR + lane) * V);
        }
        if constexpr (M == Mode::kGated) {
#pragma unroll
            for (int c = 0; c < CPL; ++c)
                zr[c] = stream_frag<Aux<TO>, V>(z + zo + (c * LPR + lane) * V);
        }
#pragma unroll
        for (int c = 0; c < CPL; ++c) wr[c] = load_frag<Aux<TO>, V>(w + (c * LPR + lane) * V);
    }
    int32_t keep_row = 1;
    if (active && keep) keep_row = keep[row];

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
                store_frag(res_out + oo + (c * LPR + lane) * V, v[c]);
            }
#pragma unroll
            for (int j = 0; j < V; ++j) ss += v[c][j] * v[c][j];
        }
    }
    if constexpr (LPR <= kWave) {
        ss = group_sum<LPR>(ss);
    } else {  // a row over LPR / 64 wavefronts: their partial sums meet in LDS
        constexpr int WPR = LPR / kWave;
        __shared__ float part[kBlock / kWave];
        const int wave = threadIdx.x / kWave, first = wave - wave % WPR;
        ss = group_sum<kWave>(ss);
        if (threadIdx.x % kWave == 0) part[wave] = ss;
        __syncthreads();  // reached by every thread: inactive rows return below
        ss = part[first];
#pragma unroll
        for (int j = 1; j < WPR; ++j) ss += part[first + j];
    }
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
            if (keep) {
#pragma unroll
                for (int j = 0; j < V; ++j) o[j] = o[j] * (float)keep_row;
            }
        }
        store_frag(out + oo + (c * LPR + lane) * V, o);
    }
}

// One wavefront per row, any width/stride/alignment.
template <typename TX, typename TM, typename TO, Mode M, bool CENTERED>
__global__ __launch_bounds__(kBlock) void rms_rows_general(
    TO *out, TX *res_out, const TX *x, const TM *mixed, const Aux<TO> *__restrict__ z,
    const Aux<TO> *__restrict__ w, const int32_t *__restrict__ keep, int64_t rows, RowMap map,
    int64_t width, float eps) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = (int64_t)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;  // uniform per wavefront
    const uint32_t t = fastdiv((uint32_t)row, map.heads);
    const uint32_t h = (uint32_t)row - t * map.heads.d;
    const int64_t xo = (int64_t)t * map.x_tok + (int64_t)h * map.x_head;
    const int64_t zo = (int64_t)t * map.z_tok + (int64_t)h * map.z_head;
    const int64_t oo = (int64_t)t * map.o_tok + (int64_t)h * map.o_head;
    // The first pass only reads; the second recomputes x + mixed in fp32 (the
    // normalised output uses the unrounded sum, as the fast kernel does) and
    // then writes.  Element i is read before it is written, and only by this
    // lane, so the residual or the output may overwrite x or mixed in place.
    const float keep_row = keep ? (float)keep[row] : 1.0f;
    float ss = 0.0f;
    for (int64_t i = lane; i < width; i += kWave) {
        float v = to_f32(x[xo + i]);
        if constexpr (M == Mode::kResidual) v = v + to_f32(mixed[xo + i]);
        ss += v * v;
    }
    ss = group_sum<kWave>(ss);
    const float s = rms_scale(ss, (float)width, eps);
    for (int64_t i = lane; i < width; i += kWave) {
        float v = to_f32(x[xo + i]);
        if constexpr (M == Mode::kResidual) {
            v = v + to_f32(mixed[xo + i]);
            res_out[oo + i] = from_f32<TX>(v);
        }
        const float wv = to_f32(w[i]);
        float o;
        if constexpr (M == Mode::kGated) {
            o = ((v * s) * wv) * silu(to_f32(z[zo + i]));
        } else {
            o = (v * s) * (CENTERED ? (1.0f + wv) : wv);
            if (keep) o = o * keep_row;
        }
        put_elem(out, oo + i, o);
    }
}

struct Args {
    void *out, *res;
    const void *x, *mixed, *z, *w;
    int64_t rows, width;
    RowMap map;
    float eps;
    bool fast;
    const int32_t *keep = nullptr;  // per-row output mask (plain and residual modes)
};

template <typename TX, typename TM, typename TO, int LPR, int CPL, Mode M, bool C>
int32_t launch_fast(const Args &a, hipStream_t stream) {
    const int64_t blocks = ceil_div(a.rows, kBlock / LPR);
    hipLaunchKernelGGL((rms_rows_fast<TX, TM, TO, LPR, CPL, M, C>), dim3((uint32_t)blocks),
                       dim3(kBlock), 0, stream, (TO *)a.out, (TX *)a.res, (const TX *)a.x,
                       (const TM *)a.mixed, (const Aux<TO> *)a.z, (const Aux<TO> *)a.w, a.keep,
                       a.rows, a.map, (float)a.width, a.eps);
    return launch_status();
}

// Fast-path shapes by G = groups per row: a lane holds 2 groups for rows of up
// to 64 groups and 4 groups for 128-group rows (8 for plain all-bf16 128-group
// rows; the splits that measured fastest on MI355X); 256-group rows (fp32 rows
// of 1024) take 2 wavefronts of 2 groups per lane, 2-4% faster than 64 x 4 for
// the 16-byte-per-element residual rows (all fp32, or fp32 with a split output)
// and for fp32 rows to bf16, equal for the rest (32 x 8, 16 x 16 and 256 x 1
// were slower); rows of 192, 320, 384 and 448 groups take 64 lanes with 3-7
// groups each; wider rows 2 wavefronts (512-1536 groups: fp32 rows of
// 2048-6144 elements, 4-12 groups per lane) or 4 (2048-4096 groups, 8-16 per
// lane).  Measured on MI355X against one 64-lane wavefront per row with G/64
// groups per lane: 2-7% faster at 512-768 groups and 13-15% at 1024 (16 groups
// per lane took 256 VGPRs); 12-32 groups per lane in one wavefront took
// 200-256 VGPRs, with spills.  kNoFastPath when no instantiation matches.
template <typename TX, typename TM, typename TO, Mode M, bool C>
int32_t dispatch_fast(const Args &a, hipStream_t stream) {
    constexpr int V = group_elems<TX, TM, TO>();
    if (a.width % V) return kNoFastPath;
    // Plain all-bf16 rows of 128 groups (width 1024): 16 lanes x 8 groups, 16
    // rows per workgroup, measured ~5% faster than 32 x 4 (more bytes in flight
    // per wavefront at occupancy 3); the all-bf16 residual rows measured no
    // gain and keep 32 x 4.
    if constexpr (M == Mode::kPlain && sizeof(TX) == 2 && sizeof(TO) == 2) {
        if (a.width / V == 128) return launch_fast<TX, TM, TO, 16, 8, M, C>(a, stream);
    }
#define QDC_FAST(LPR, CPL) \
    case LPR * CPL:        \
        return launch_fast<TX, TM, TO, LPR, CPL, M, C>(a, stream);
    switch (a.width / V) {
        QDC_FAST(1, 1)
        QDC_FAST(1, 2)
        QDC_FAST(2, 2)
        QDC_FAST(4, 2)
        QDC_FAST(8, 2)
        QDC_FAST(16, 2)
        QDC_FAST(32, 2)
        QDC_FAST(32, 4)
        QDC_FAST(64, 3)
        QDC_FAST(128, 2)
        QDC_FAST(64, 5)
        QDC_FAST(64, 6)
        QDC_FAST(64, 7)
        QDC_FAST(128, 4)
        QDC_FAST(128, 5)
        QDC_FAST(128, 6)
        QDC_FAST(128, 8)
        QDC_FAST(128, 10)
        QDC_FAST(128, 12)
        QDC_FAST(256, 8)
        QDC_FAST(256, 10)
        QDC_FAST(256, 12)
        QDC_FAST(256, 16)
        default:
            return kNoFastPath;
    }
#undef QDC_FAST
}

template <typename TX, typename TM, typename TO, Mode M, bool C>
int32_t run(const Args &a, hipStream_t stream) {
    if (a.fast) {
        const int32_t rc = dispatch_fast<TX, TM, TO, M, C>(a, stream);
        if (rc != kNoFastPath) return rc;
    }
    const int64_t blocks = ceil_div(a.rows, kBlock / kWave);
    hipLaunchKernelGGL((rms_rows_general<TX, TM, TO, M, C>), dim3((uint32_t)blocks), dim3(kBlock),
                       0, stream, (TO *)a.out, (TX *)a.res, (const TX *)a.x, (const TM *)a.mixed,
                       (const Aux<TO> *)a.z, (const Aux<TO> *)a.w, a.keep, a.rows, a.map, a.width,
                       a.eps);
    return launch_status();
}

// A row takes up to 64 lanes (the general kernel one wavefront) and a grid
// holds fewer than 2^32 work-items, so rows < 2^26.
constexpr int64_t kMaxRows = (int64_t)1 << 26;

bool all16(std::initializer_list<const void *> ptrs) {
    for (const void *p : ptrs)
        if (!aligned16(p)) return false;
    return true;
}

// Shared by the plain and the masked entry points; `masked` requires keep.
int32_t rmsnorm(void *out, const void *x, const void *weight, const int32_t *keep, bool masked,
                int64_t rows, int64_t width, int64_t ld_x, int64_t ld_out, float eps,
                int32_t centered, int32_t x_dtype, int32_t out_dtype, hipStream_t stream) {
    const bool split = out_dtype == QDC_BF16X2;  // fp32 rows, bf16 weight
    if (!valid_dtype(x_dtype) || !(valid_dtype(out_dtype) || split)) return QDC_ERR_DTYPE;
    if (x_dtype == QDC_BF16 && out_dtype != QDC_BF16) return QDC_ERR_DTYPE;
    if (rows < 0 || width < 0 || rows >= kMaxRows) return QDC_ERR_SHAPE;
    if (rows == 0 || width == 0) return QDC_OK;
    if (!out || !x || !weight || (masked && !keep)) return QDC_ERR_NULL;
    if (ld_x < width || ld_out < width) return QDC_ERR_SHAPE;
    if (split && !split_rows_ok(width, ld_out)) return QDC_ERR_SHAPE;
    if (split && out == x) return QDC_ERR_ALIAS;
    const int64_t ex = elem_size(x_dtype), eo = elem_size(out_dtype);
    const int64_t span_x = ((rows - 1) * ld_x + width) * ex;
    const int64_t span_o = ((rows - 1) * ld_out + width) * eo;
    // in place: the same buffer, element type and stride
    if (out == x ? (ld_out != ld_x || ex != eo) : overlaps(out, span_o, x, span_x))
        return QDC_ERR_ALIAS;
    if (masked && overlaps(out, span_o, keep, rows * (int64_t)sizeof(int32_t)))
        return QDC_ERR_ALIAS;
    if (overlaps(out, span_o, weight, width * (split ? 2 : eo))) return QDC_ERR_ALIAS;
    Args a{out, nullptr, x, nullptr, nullptr, weight, rows, width,
           RowMap{make_fastdiv(1), ld_x, 0, 0, 0, ld_out, 0}, eps,
           all16({out, x, weight}) && (ld_x * ex) % 16 == 0 && (ld_out * eo) % 16 == 0};
    a.keep = masked ? keep : nullptr;
    if (centered) {
        if (split) return run<float, float, split_t, Mode::kPlain, true>(a, stream);
        if (x_dtype == QDC_BF16) return run<bf16_t, bf16_t, bf16_t, Mode::kPlain, true>(a, stream);
        if (out_dtype == QDC_BF16) return run<float, float, bf16_t, Mode::kPlain, true>(a, stream);
        return run<float, float, float, Mode::kPlain, true>(a, stream);
    }
    if (split) return run<float, float, split_t, Mode::kPlain, false>(a, stream);
    if (x_dtype == QDC_BF16) return run<bf16_t, bf16_t, bf16_t, Mode::kPlain, false>(a, stream);
    if (out_dtype == QDC_BF16) return run<float, float, bf16_t, Mode::kPlain, false>(a, stream);
    return run<float, float, float, Mode::kPlain, false>(a, stream);
}

// Shared by the plain and the masked entry points; `masked` requires keep.
int32_t residual_rmsnorm(void *residual, void *out, const void *x, const void *mixed,
                         const void *weight, const int32_t *keep, bool masked, int64_t rows,
                         int64_t width, float eps, int32_t residual_dtype, int32_t mixed_dtype,
                         int32_t out_dtype, hipStream_t stream) {
    // the split output takes an fp32 residual stream and an fp32 addend
    const bool split = out_dtype == QDC_BF16X2;
    if (split && (residual_dtype != QDC_F32 || mixed_dtype != QDC_F32)) return QDC_ERR_DTYPE;
    if (!valid_dtype(residual_dtype) || !valid_dtype(mixed_dtype) ||
        !(valid_dtype(out_dtype) || split))
        return QDC_ERR_DTYPE;
    const bool all_f32 =
        residual_dtype == QDC_F32 && mixed_dtype == QDC_F32 && out_dtype == QDC_F32;
    const bool all_bf16 =
        residual_dtype == QDC_BF16 && mixed_dtype == QDC_BF16 && out_dtype == QDC_BF16;
    // an fp32 residual stream may take a bf16 or fp32 addend and write either output
    const bool f32_stream = residual_dtype == QDC_F32;
    if (!all_bf16 && !f32_stream) return QDC_ERR_DTYPE;
    if (rows < 0 || width < 0 || rows >= kMaxRows) return QDC_ERR_SHAPE;
    if (rows == 0 || width == 0) return QDC_OK;
    if (!residual || !out || !x || !mixed || !weight || (masked && !keep)) return QDC_ERR_NULL;
    if (split && !split_rows_ok(width, width)) return QDC_ERR_SHAPE;
    const int64_t br = rows * width * elem_size(residual_dtype);
    const int64_t bm = rows * width * elem_size(mixed_dtype);
    const int64_t bo = rows * width * elem_size(out_dtype);
    // in place means the same buffer in the same element type
    if (overlaps(residual, br, out, bo)) return QDC_ERR_ALIAS;
    if (residual != x && overlaps(residual, br, x, br)) return QDC_ERR_ALIAS;
    if (residual == mixed ? residual_dtype != mixed_dtype : overlaps(residual, br, mixed, bm))
        return QDC_ERR_ALIAS;
    if (out == x ? out_dtype != residual_dtype : overlaps(out, bo, x, br)) return QDC_ERR_ALIAS;
    if (out == mixed ? out_dtype != mixed_dtype : overlaps(out, bo, mixed, bm))
        return QDC_ERR_ALIAS;
    const int64_t bk = rows * (int64_t)sizeof(int32_t);
    if (masked && (overlaps(out, bo, keep, bk) || overlaps(residual, br, keep, bk)))
        return QDC_ERR_ALIAS;
    const int64_t bw = width * (split ? 2 : elem_size(out_dtype));
    if (overlaps(out, bo, weight, bw) || overlaps(residual, br, weight, bw)) return QDC_ERR_ALIAS;
    Args a{out, residual, x, mixed, nullptr, weight, rows, width,
           RowMap{make_fastdiv(1), width, 0, 0, 0, width, 0}, eps,
           all16({residual, out, x, mixed, weight})};
    a.keep = masked ? keep : nullptr;
    if (split) return run<float, float, split_t, Mode::kResidual, true>(a, stream);
    if (all_f32) return run<float, float, float, Mode::kResidual, true>(a, stream);
    if (all_bf16) return run<bf16_t, bf16_t, bf16_t, Mode::kResidual, true>(a, stream);
    if (mixed_dtype == QDC_F32) return run<float, float, bf16_t, Mode::kResidual, true>(a, stream);
    if (out_dtype == QDC_BF16) return run<float, bf16_t, bf16_t, Mode::kResidual, true>(a, stream);
    return run<float, bf16_t, float, Mode::kResidual, true>(a, stream);
}

// out[i] = rms_scale(sum_squares[i], width, eps), the scale every row kernel
// applies to a row with that sum of squares.
__global__ __launch_bounds__(kBlock) void row_scale_map(float *out, const float *ss, int64_t n,
                                                        float width, float eps) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i < n) out[i] = rms_scale(ss[i], width, eps);
}

// Adds to *mismatches the number of bit patterns first + k, k < count, whose
// inv_sqrt_rn differs from the general expression 1.0f / sqrtf in any bit (two
// NaN results count as equal).  Grid-stride over k; one atomic per thread that
// found any.
constexpr uint32_t kCheckBlocks = 8192;
__global__ __launch_bounds__(kBlock) void row_scale_check(uint32_t first, uint64_t count,
                                                          unsigned long long *mismatches) {
    uint32_t n = 0;
    const uint64_t stride = (uint64_t)kCheckBlocks * kBlock;
    for (uint64_t k = (uint64_t)blockIdx.x * kBlock + threadIdx.x; k < count; k += stride) {
        const float x = __uint_as_float(first + (uint32_t)k);
        const float a = inv_sqrt_rn(x), b = 1.0f / __builtin_sqrtf(x);
        n += (__float_as_uint(a) != __float_as_uint(b)) && !(a != a && b != b);
    }
    if (n) atomicAdd(mismatches, (unsigned long long)n);
}

}  // namespace
}  // namespace qdc

using namespace qdc;

extern "C" int32_t qdc_row_scale(float *out, const float *sum_squares, int64_t n, float width,
                                 float eps, hipStream_t stream) {
    if (n < 0 || n >= ((int64_t)1 << 32) - kBlock) return QDC_ERR_SHAPE;
    if (n == 0) return QDC_OK;
    if (!out || !sum_squares) return QDC_ERR_NULL;
    if ((const void *)out != (const void *)sum_squares && overlaps(out, n * 4, sum_squares, n * 4))
        return QDC_ERR_ALIAS;
    hipLaunchKernelGGL(row_scale_map, dim3((uint32_t)ceil_div(n, kBlock)), dim3(kBlock), 0, stream,
                       out, sum_squares, n, width, eps);
    return launch_status();
}

extern "C" int32_t qdc_row_scale_check(uint32_t first, int64_t count, uint64_t *mismatches,
                                       hipStream_t stream) {
    if (count < 0 || count > ((int64_t)1 << 32) - (int64_t)first) return QDC_ERR_SHAPE;
    if (!mismatches) return QDC_ERR_NULL;
    if (count == 0) return QDC_OK;
    hipLaunchKernelGGL(row_scale_check, dim3(kCheckBlocks), dim3(kBlock), 0, stream, first,
                       (uint64_t)count, (unsigned long long *)mismatches);
    return launch_status();
}

extern "C" int32_t qdc_rmsnorm(void *out, const void *x, const void *weight, int64_t rows,
                               int64_t width, int64_t ld_x, int64_t ld_out, float eps,
                               int32_t centered, int32_t x_dtype, int32_t out_dtype,
                               hipStream_t stream) {
    return rmsnorm(out, x, weight, nullptr, false, rows, width, ld_x, ld_out, eps, centered,
                   x_dtype, out_dtype, stream);
}

extern "C" int32_t qdc_rmsnorm_masked(void *out, const void *x, const void *weight,
                                      const int32_t *token_mask, int64_t rows, int64_t width,
                                      int64_t ld_x, int64_t ld_out, float eps, int32_t centered,
                                      int32_t x_dtype, int32_t out_dtype, hipStream_t stream) {
    return rmsnorm(out, x, weight, token_mask, true, rows, width, ld_x, ld_out, eps, centered,
                   x_dtype, out_dtype, stream);
}

extern "C" int32_t qdc_residual_rmsnorm(void *residual, void *out, const void *x,
                                        const void *mixed, const void *weight, int64_t rows,
                                        int64_t width, float eps, int32_t residual_dtype,
                                        int32_t mixed_dtype, int32_t out_dtype,
                                        hipStream_t stream) {
    return residual_rmsnorm(residual, out, x, mixed, weight, nullptr, false, rows, width, eps,
                            residual_dtype, mixed_dtype, out_dtype, stream);
}

extern "C" int32_t qdc_residual_rmsnorm_masked(void *residual, void *out, const void *x,
                                               const void *mixed, const void *weight,
                                               const int32_t *token_mask, int64_t rows,
                                               int64_t width, float eps, int32_t residual_dtype,
                                               int32_t mixed_dtype, int32_t out_dtype,
                                               hipStream_t stream) {
    return residual_rmsnorm(residual, out, x, mixed, weight, token_mask, true, rows, width, eps,
                            residual_dtype, mixed_dtype, out_dtype, stream);
}

extern "C" int32_t qdc_gated_rmsnorm(void *out, const void *x, const void *z, const void *weight,
                                     int64_t tokens, int64_t heads, int64_t width, int64_t x_tok,
                                     int64_t z_tok, int64_t out_tok, float eps, int32_t dtype,
                                     int32_t out_dtype, hipStream_t stream) {
    // out in dtype, or bf16 x, z and weight with the split output
    const bool split = dtype == QDC_BF16 && out_dtype == QDC_BF16X2;
    if (!valid_dtype(dtype) || !(out_dtype == dtype || split)) return QDC_ERR_DTYPE;
    if (tokens < 0 || heads < 0 || width < 0) return QDC_ERR_SHAPE;
    if (tokens == 0 || heads == 0 || width == 0) return QDC_OK;
    if (!out || !x || !z || !weight) return QDC_ERR_NULL;
    if (tokens * heads >= kMaxRows || heads >= kMaxRows) return QDC_ERR_SHAPE;
    if (x_tok < heads * width || z_tok < heads * width || out_tok < heads * width)
        return QDC_ERR_SHAPE;
    if (split && !split_rows_ok(width, out_tok)) return QDC_ERR_SHAPE;
    const int64_t es = elem_size(dtype), eo = elem_size(out_dtype);
    const int64_t span_o = ((tokens - 1) * out_tok + heads * width) * eo;
    const int64_t span_x = ((tokens - 1) * x_tok + heads * width) * es;
    if (out == x ? (out_tok != x_tok || eo != es) : overlaps(out, span_o, x, span_x))
        return QDC_ERR_ALIAS;
    if (overlaps(out, span_o, z, ((tokens - 1) * z_tok + heads * width) * es))
        return QDC_ERR_ALIAS;
    if (overlaps(out, span_o, weight, width * es)) return QDC_ERR_ALIAS;
    const Args a{out, nullptr, x, nullptr, z, weight, tokens * heads, width,
                 RowMap{make_fastdiv((uint32_t)heads), x_tok, width, z_tok, width, out_tok, width},
                 eps,
                 all16({out, x, z, weight}) && (width * es) % 16 == 0 &&
                     (x_tok * es) % 16 == 0 && (z_tok * es) % 16 == 0 &&
                     (out_tok * eo) % 16 == 0};
    if (split) return run<bf16_t, bf16_t, split_t, Mode::kGated, false>(a, stream);
    if (dtype == QDC_BF16) return run<bf16_t, bf16_t, bf16_t, Mode::kGated, false>(a, stream);
    return run<float, float, float, Mode::kGated, false>(a, stream);
}

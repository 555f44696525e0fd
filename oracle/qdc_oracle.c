/*
 * qdc_oracle.c -- CPU restatement of the reference CPU path for the fused row
 * kernels.  TEST INFRASTRUCTURE ONLY (see qdc_oracle.h): the reference the HIP
 * library is compared with and the timed CPU baseline, never part of the
 * product path.
 *
 * Built with -ffp-contract=off so that every multiply and add rounds on its
 * own, as in the reference's Julia code (no FMA contraction there).  Row sums
 * of squares use 16 independent fp32 partial sums combined pairwise, the
 * reassociation Julia's `sum(abs2, v)` / `@simd` applies; the result differs
 * from a sequential sum only in the last bits.
 *
 * Threads (qdco_set_threads, default 1): rows are independent, so an OpenMP
 * loop over rows gives the same bits at any thread count; the timed CPU
 * baseline uses it for an all-cores figure.  SwiGLU over contiguous rows
 * restates the reference's own split instead: min(threads, cld(n, 65536))
 * workers, worker w taking the 256-element blocks w, w + workers, ...
 * (ext/QwenDecisionCoreLoopVectorizationExt.jl:194-205).
 */
#include "qdc_oracle.h"

#include <math.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void qdco_set_threads(int threads) { g_threads = threads < 1 ? 1 : threads; }
int qdco_threads(void) { return g_threads; }

/* src/safetensors.jl:28-30 */
float qdco_bf16_to_f32(uint16_t bits) {
    uint32_t wide = (uint32_t)bits << 16;
    float value;
    memcpy(&value, &wide, sizeof value);
    return value;
}

/* src/safetensors.jl:37-42: rounded = bits + 0x7fff + ((bits >> 16) & 1), keep the top half. */
uint16_t qdco_f32_to_bf16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, sizeof bits);
    uint32_t rounded = bits + 0x00007fffu + ((bits >> 16) & 1u);
    return (uint16_t)(rounded >> 16);
}

void qdco_bf16_to_f32_n(const uint16_t *in, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = qdco_bf16_to_f32(in[i]);
}

void qdco_f32_to_bf16_n(const float *in, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = qdco_f32_to_bf16(in[i]);
}

/* src/backbone.jl:56-64 with the id check of src/backbone.jl:417-418. */
int qdco_gather(void *out, const void *table, int64_t elem_bytes, const int32_t *ids,
                int64_t n_ids, int64_t vocab, int64_t hidden) {
    for (int64_t t = 0; t < n_ids; ++t)
        if (ids[t] < 0 || (int64_t)ids[t] >= vocab) return -1;
    const int64_t row_bytes = hidden * elem_bytes;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t t = 0; t < n_ids; ++t)
        memcpy((char *)out + t * row_bytes, (const char *)table + (int64_t)ids[t] * row_bytes,
               (size_t)row_bytes);
    return 0;
}

/* sum(abs2, v) in fp32 with @simd-style reassociation (16 partial sums). */
static float sum_squares(const float *v, int64_t n) {
    float acc[16] = {0};
    int64_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int j = 0; j < 16; ++j) acc[j] += v[i + j] * v[i + j];
    for (int j = 0; i < n; ++i, ++j) acc[j] += v[i] * v[i];
    for (int width = 8; width >= 1; width /= 2)
        for (int j = 0; j < width; ++j) acc[j] += acc[j + width];
    return acc[0];
}

/* inv(sqrt(sum/width + eps)) in fp32: src/backbone_cpu.jl:344. */
static float rms_scale(const float *row, int64_t width, float eps) {
    return 1.0f / sqrtf(sum_squares(row, width) / (float)width + eps);
}

/* cpu_rms! src/backbone_cpu.jl:333-350 (centred) and cpu_delta_rms! :352-362. */
void qdco_rms(float *out, int64_t ld_out, const float *x, int64_t ld_x, const float *w,
              int64_t rows, int64_t width, float eps, int centered) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float *in = x + r * ld_x;
        float *dst = out + r * ld_out;
        const float scale = rms_scale(in, width, eps);
        if (centered)
            for (int64_t i = 0; i < width; ++i) dst[i] = (in[i] * scale) * (1.0f + w[i]);
        else
            for (int64_t i = 0; i < width; ++i) dst[i] = (in[i] * scale) * w[i];
    }
}

/* src/backbone.jl:347-350; src/backbone_cpu.jl:321-328. */
void qdco_residual_rms(float *residual, float *out, const float *x, const float *mixed,
                       const float *w, int64_t rows, int64_t width, float eps) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float *res = residual + r * width;
        for (int64_t i = 0; i < width; ++i) res[i] = x[r * width + i] + mixed[r * width + i];
        const float scale = rms_scale(res, width, eps);
        for (int64_t i = 0; i < width; ++i) out[r * width + i] = (res[i] * scale) * (1.0f + w[i]);
    }
}

/* cpu_full_workspace src/backbone_cpu.jl:90-111.  Julia evaluates Float32 `^`,
 * `cos` and `sin` in Float64 and rounds once, which (float)pow/cos/sin of the
 * widened arguments restates. */
void qdco_rope_tables(float *cosines, float *sines, int64_t n_pos, int64_t rotary_dim, float theta) {
    const int64_t half = rotary_dim / 2;
    for (int64_t i = 0; i < half; ++i) {
        const float exponent = (float)(2 * i) / (float)rotary_dim;
        const float power = (float)pow((double)theta, (double)exponent);
        const float freq = 1.0f / power;
        for (int64_t p = 0; p < n_pos; ++p) {
            const float angle = freq * (float)p;
            cosines[p * half + i] = (float)cos((double)angle);
            sines[p * half + i] = (float)sin((double)angle);
        }
    }
}

/* cpu_full_rms! src/backbone_cpu.jl:113-123 then cpu_full_rope! :125-136. */
void qdco_qk_norm_rope(float *out, int64_t out_tok, int64_t out_head, const float *in,
                       int64_t in_tok, int64_t in_head, const float *w, const float *cosines,
                       const float *sines, int64_t tokens, int64_t heads, int64_t dim,
                       int64_t rotary_dim, int64_t seq_len, int64_t pos_offset, float eps) {
    const int64_t half = rotary_dim / 2;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t t = 0; t < tokens; ++t) {
        const int64_t pos = pos_offset + t % seq_len;
        const float *c = cosines + pos * half;
        const float *s = sines + pos * half;
        for (int64_t h = 0; h < heads; ++h) {
            const float *src = in + t * in_tok + h * in_head;
            float *dst = out + t * out_tok + h * out_head;
            const float scale = rms_scale(src, dim, eps);
            for (int64_t i = 0; i < dim; ++i) dst[i] = (src[i] * scale) * (1.0f + w[i]);
            for (int64_t i = 0; i < half; ++i) {
                const float a = dst[i], b = dst[half + i];
                dst[i] = a * c[i] - b * s[i];
                dst[half + i] = b * c[i] + a * s[i];
            }
        }
    }
}

/* native_silu src/backbone.jl:196-197. */
static float silu(float x) { return x * (1.0f / (1.0f + expf(-x))); }

/* ext/QwenDecisionCoreLoopVectorizationExt.jl:373-390; src/backbone_cpu.jl:750-755. */
void qdco_gated_rms(float *out, int64_t out_tok, const float *x, int64_t x_tok, const float *z,
                    int64_t z_tok, const float *w, int64_t tokens, int64_t heads, int64_t width,
                    float eps) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t t = 0; t < tokens; ++t)
        for (int64_t h = 0; h < heads; ++h) {
            const float *src = x + t * x_tok + h * width;
            const float *gate = z + t * z_tok + h * width;
            float *dst = out + t * out_tok + h * width;
            const float scale = rms_scale(src, width, eps);
            for (int64_t i = 0; i < width; ++i)
                dst[i] = ((src[i] * scale) * w[i]) * silu(gate[i]);
        }
}

/* ext/QwenDecisionCoreLoopVectorizationExt.jl:189-215 / :104-127 / :144-160. */
static void swiglu_range(float *out, const float *gate, const float *up, int64_t lo, int64_t hi) {
    for (int64_t i = lo; i < hi; ++i) {
        const float x = gate[i];
        out[i] = (x * (1.0f / (1.0f + expf(-x)))) * up[i];
    }
}

void qdco_swiglu(float *out, int64_t ld_out, const float *gate, int64_t ld_gate, const float *up,
                 int64_t ld_up, int64_t tokens, int64_t width) {
    const int64_t n = tokens * width;
    const int64_t blocks_needed = (n + 65535) / 65536;
    const int workers = (int)(g_threads < blocks_needed ? g_threads : blocks_needed);
    if (workers > 1 && ld_out == width && ld_gate == width && ld_up == width) {
#pragma omp parallel num_threads(workers)
        {
#ifdef _OPENMP
            const int64_t w = omp_get_thread_num(), nw = omp_get_num_threads();
#else
            const int64_t w = 0, nw = 1;
#endif
            for (int64_t b = 256 * w; b < n; b += 256 * nw)
                swiglu_range(out, gate, up, b, b + 256 < n ? b + 256 : n);
        }
        return;
    }
    for (int64_t t = 0; t < tokens; ++t) {
        const float *g = gate + t * ld_gate;
        const float *u = up + t * ld_up;
        float *dst = out + t * ld_out;
        for (int64_t i = 0; i < width; ++i) {
            const float x = g[i];
            dst[i] = (x * (1.0f / (1.0f + expf(-x)))) * u[i];
        }
    }
}

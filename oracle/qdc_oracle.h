/*
 * qdc_oracle.h -- CPU restatement of QwenDecisionCore.jl's CPU policy path for
 * the fused per-layer row kernels (embedding gather, zero-centred RMSNorm,
 * residual + RMSNorm, per-head q/k RMSNorm + partial RoPE, gated RMSNorm,
 * SwiGLU) and the bf16 <-> fp32 format.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is what the GPU kernels are
 * compared against and the timed CPU baseline.  Only tests/, the smoke() entry
 * and bench.py's cpu_baseline leg may load it.  The product path (the HIP
 * library) never links or calls it.
 *
 * Layout: row-major [rows, width], identical in memory to the reference's
 * column-major (width, rows) Julia matrices.  All arithmetic is fp32 in the
 * reference's operation order; bf16 data is handled by widening on input and
 * round-to-nearest-even on output, exactly as the reference's safetensors code.
 */
#ifndef QDC_ORACLE_H
#define QDC_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Threads for the row loops (default 1).  Rows are independent, so the
 * results do not depend on the count; used for the all-cores CPU figure. */
void qdco_set_threads(int threads);
int qdco_threads(void);

/* bf16 widen: bits << 16.  src/safetensors.jl:28-30 */
float qdco_bf16_to_f32(uint16_t bits);
/* bf16 narrow, RNE on the 16 dropped bits.  src/safetensors.jl:37-42 */
uint16_t qdco_f32_to_bf16(float value);
void qdco_bf16_to_f32_n(const uint16_t *in, float *out, int64_t n);
void qdco_f32_to_bf16_n(const float *in, uint16_t *out, int64_t n);

/* Embedding gather: out[t, :] = table[ids[t], :], a byte copy of each row.
 * src/backbone.jl:56-64 (CPU copyto! per column), ids 0-based and checked
 * against [0, vocab) first as src/backbone.jl:417-418.  Returns 0, or -1 with
 * nothing written when an id is out of range. */
int qdco_gather(void *out, const void *table, int64_t elem_bytes, const int32_t *ids,
                int64_t n_ids, int64_t vocab, int64_t hidden);

/* RMSNorm of each row: s = 1/sqrt(sum(x^2)/width + eps);
 * y = (x*s)*(1+w) when centered (cpu_rms! src/backbone_cpu.jl:333-350),
 * y = (x*s)*w otherwise (cpu_delta_rms! src/backbone_cpu.jl:352-362). */
void qdco_rms(float *out, int64_t ld_out, const float *x, int64_t ld_x, const float *w,
              int64_t rows, int64_t width, float eps, int centered);

/* residual = x + mixed; out = rms(residual) centred.
 * native_residual_rms src/backbone.jl:347-350; CPU src/backbone_cpu.jl:321-328. */
void qdco_residual_rms(float *residual, float *out, const float *x, const float *mixed,
                       const float *w, int64_t rows, int64_t width, float eps);

/* RoPE tables, layout [n_pos][rotary_dim/2]:
 * freq_i = inv(theta^(Float32(2i)/Float32(rotary_dim))), angle = freq_i*Float32(pos),
 * cos/sin of the fp32 angle rounded to fp32.  cpu_full_workspace
 * src/backbone_cpu.jl:90-111 (same arithmetic as native_rope src/backbone.jl:206-213). */
void qdco_rope_tables(float *cosines, float *sines, int64_t n_pos, int64_t rotary_dim, float theta);

/* Per-head centred RMSNorm then half-split partial RoPE, one (token, head) row
 * at a time: cpu_full_rms! src/backbone_cpu.jl:113-123 followed by
 * cpu_full_rope! src/backbone_cpu.jl:125-136.  Row (t, h) of the input starts at
 * in + t*in_tok + h*in_head (the q half of the q||gate projection when
 * in_head = 2*dim, src/backbone.jl:226-227).  Position of token t is
 * pos_offset + t % seq_len and indexes the tables. */
void qdco_qk_norm_rope(float *out, int64_t out_tok, int64_t out_head, const float *in,
                       int64_t in_tok, int64_t in_head, const float *w, const float *cosines,
                       const float *sines, int64_t tokens, int64_t heads, int64_t dim,
                       int64_t rotary_dim, int64_t seq_len, int64_t pos_offset, float eps);

/* Gated RMSNorm of each (token, head) row of width `width`:
 * y = ((x*s)*w)*silu(z), not centred.  cpu_delta_gate_output!
 * ext/QwenDecisionCoreLoopVectorizationExt.jl:373-390 and the scalar loop
 * src/backbone_cpu.jl:750-755; silu(z) as applied to z beforehand at
 * src/backbone_cpu.jl:518-520 with native_silu src/backbone.jl:196-197. */
void qdco_gated_rms(float *out, int64_t out_tok, const float *x, int64_t x_tok, const float *z,
                    int64_t z_tok, const float *w, int64_t tokens, int64_t heads, int64_t width,
                    float eps);

/* SwiGLU: out = (g * inv(1 + exp(-g))) * u.  cpu_portable_gate!
 * ext/QwenDecisionCoreLoopVectorizationExt.jl:189-215 (gate_blocks! :144-160,
 * exceptional lanes :104-127 use the same formula); native_mlp_gate!
 * src/backbone.jl:352-355. */
void qdco_swiglu(float *out, int64_t ld_out, const float *gate, int64_t ld_gate, const float *up,
                 int64_t ld_up, int64_t tokens, int64_t width);

#ifdef __cplusplus
}
#endif

#endif

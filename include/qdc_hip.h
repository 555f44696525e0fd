/*
 * qdc_hip.h -- C ABI of libqdc_hip.so: the fused per-layer row kernels of the
 * Qwen3.5 hybrid backbone forward, hand-written HIP for MI355X (gfx950).
 *
 * Conventions shared by every device entry point:
 *  - Tensors are device pointers to row-major data; "[rows, width]" here is the
 *    reference's column-major (width, rows) Julia matrix in the same memory.
 *    Strides ("tok", "head", "ld") are in elements, not bytes.
 *  - dtype arguments (QDC_F32 or QDC_BF16) select the element types of the
 *    call's tensors; the RMSNorm entry points take one per tensor role so an
 *    fp32 residual stream can feed bf16 activations.  Arithmetic is fp32; bf16
 *    results are rounded to nearest even.  RoPE tables are always fp32.
 *  - QDC_BF16X2 is an output type only (the split form of a GEMM input): each
 *    fp32 result v is written as two bf16 terms, hi = bf16(v) and
 *    lo = bf16(v - hi) (lo = 0 when hi is not finite), so hi + lo keeps about
 *    16 significant bits.  Element e of such an output takes the bf16 slots
 *    8*(e/4) + e%4 (hi) and 8*(e/4) + 4 + e%4 (lo): every aligned group of 4
 *    elements is one 16-byte piece [4 hi | 4 lo], 4 bytes per element, and
 *    strides stay in elements.  A row of K such elements is a bf16 row of 2K
 *    values; multiplied by a bf16 weight whose K rows are repeated in the same
 *    pattern (rows 8g+j and 8g+4+j both hold row 4g+j) it gives
 *    sum((hi + lo) * w).  Rows must hold whole groups: widths and output row
 *    strides a multiple of 4 (QDC_ERR_SHAPE otherwise).  Tensors read beside a
 *    split output in its dtype role (norm weights, the gated norm's z) are
 *    bf16.  Supported where each entry point says so.
 *  - The library never allocates or frees memory, keeps no pointer after
 *    return, has no mutable global state and never synchronises: work is
 *    enqueued on `stream` (0 = the null stream of the current device) and the
 *    caller keeps every buffer alive until that stream has completed it.
 *  - Return value: 0 on success; a negative qdc_status for an argument error
 *    detected on the host before anything is enqueued; a positive hipError_t
 *    when the launch itself failed.
 *  - Unaligned pointers/strides or unusual widths are accepted and take a
 *    slower general kernel; the fast kernels need 16-byte alignment.
 *  - Size limits (QDC_ERR_SHAPE beyond them) keep every launch grid below 2^32
 *    work-items: fewer than 2^26 rows for the RMSNorm entry points (tokens *
 *    heads for the gated norm), q rows + k rows for qdc_qk_norm_rope, q + k + v
 *    rows for qdc_attention_prepare, ids for the gather, score rows for the
 *    softmax and tokens for the DeltaNet prologue.
 */
#ifndef QDC_HIP_H
#define QDC_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    QDC_F32 = 0,
    QDC_BF16 = 1,
    QDC_BF16X2 = 2  /* output only: two bf16 terms per fp32 value */
} qdc_dtype;

typedef enum {
    QDC_OK = 0,
    QDC_ERR_NULL = -1,        /* a required pointer is NULL                  */
    QDC_ERR_SHAPE = -2,       /* negative / zero / inconsistent dimensions    */
    QDC_ERR_DTYPE = -3,       /* unsupported dtype or dtype combination       */
    QDC_ERR_RANGE = -4,       /* token id or position outside its table       */
    QDC_ERR_ALIAS = -5        /* an output overlaps an input it may not alias */
} qdc_status;

/*
 * Version of this header; qdc_version() returns the same string for the
 * library that was built from it, so a host can refuse a library whose entry
 * points it was not compiled against.  The minor number changes with any
 * signature change of an existing entry point (0.2.0: qdc_gated_rmsnorm and
 * qdc_swiglu take out_dtype before the stream; 0.3.0: qdc_delta_prologue and
 * qdc_delta_scan take the q/k and v row strides ld_qk, ld_v before the
 * stream), the patch number with added entry points (0.2.1: qdc_row_scale,
 * qdc_row_scale_check; 0.3.1: qdc_copy_pair).
 */
#define QDC_HIP_VERSION "qdc_hip 0.3.1"

/* Library version string ("qdc_hip <major>.<minor>.<patch>"), QDC_HIP_VERSION. */
const char *qdc_version(void);
/* Human-readable text for a status returned by any entry point. */
const char *qdc_status_string(int32_t status);

/*
 * Embedding gather: out[t, :] = table[ids[t], :] for t < n_ids.
 * Replaces native_gather / gather_kernel! (ext/amdgpu_workspace.jl:206-236;
 * generic src/backbone.jl:55, CPU :56-64).  A pure copy: bf16->bf16 and
 * f32->f32 move bits, bf16->f32 widens by <<16 (src/safetensors.jl:28-30), so
 * results are bit-exact.  ids are device int32, 0-based.  Ids are validated on
 * the host beforehand as in the reference (qdc_check_ids); an id outside
 * [0, vocab) that reaches the kernel writes a zero row and, when error_flag is
 * not NULL, sets *error_flag = 1 (device int32, cleared by the caller).
 */
int32_t qdc_embedding_gather(void *out, int32_t out_dtype, const void *table, int32_t table_dtype,
                             const int32_t *ids, int64_t n_ids, int64_t vocab, int64_t hidden,
                             int32_t *error_flag, hipStream_t stream);

/*
 * The embedding gather fused with the first layer's input RMSNorm, one pass
 * over the table rows: hidden[t, :] = table[ids[t], :] (fp32, the residual
 * stream; bf16 table entries widened exactly by <<16) and normed[t, :] =
 * zero-centred RMSNorm(hidden[t, :]) with `weight` (normed_dtype, as the
 * weight; QDC_BF16X2 with a bf16 weight), times token_mask[t] when
 * token_mask is not NULL (the DeltaNet input mask when the first layer is a
 * DeltaNet layer, as qdc_rmsnorm_masked).
 * Replaces native_gather (ext/amdgpu_workspace.jl:206-236) followed by the
 * first layer's native_rms (src/backbone.jl:364; ext/amdgpu_workspace.jl:
 * 113-149), which reads the gathered rows back.  Ids as qdc_embedding_gather
 * (an id outside [0, vocab) gives zero rows and sets *error_flag).  Outputs
 * contiguous [n_ids, width]; no overlap with an input.
 */
int32_t qdc_embedding_gather_rmsnorm(void *hidden, void *normed, const void *table,
                                     int32_t table_dtype, const int32_t *ids, const void *weight,
                                     int32_t normed_dtype, const int32_t *token_mask,
                                     int64_t n_ids, int64_t vocab, int64_t width, float eps,
                                     int32_t *error_flag, hipStream_t stream);

/*
 * Host-side id check of check_sequence / native_gather (src/backbone.jl:417-418,
 * ext/amdgpu_workspace.jl:223-224): QDC_OK when every ids[t] is in [0, vocab),
 * QDC_ERR_RANGE otherwise.  `ids` is host memory.
 */
int32_t qdc_check_ids(const int64_t *ids, int64_t n_ids, int64_t vocab);

/*
 * RMSNorm of `rows` rows of `width`: s = 1/sqrt(sum(x^2)/width + eps);
 * out = (x*s)*(1+w) if centered (zero-centred weight), else (x*s)*w.
 * Replaces native_rms / rms_kernel! (ext/amdgpu_workspace.jl:113-149; generic
 * src/backbone.jl:200-204; CPU cpu_rms! src/backbone_cpu.jl:333-350).  Serves
 * the input, post-attention and final norms, per-head q/k rows without RoPE
 * (rows = tokens*heads, width = head_dim) and, with centered = 0, the plain
 * DeltaNet output norm.  Row r reads x + r*ld_x and writes out + r*ld_out.
 * x_dtype is the type of x; out_dtype that of out and weight.  Supported:
 * f32->f32, bf16->bf16, f32->bf16 (an fp32 residual stream feeding bf16
 * GEMMs) and f32->bf16x2 (bf16 weight).  out may equal x when the type and
 * stride agree (not for a split output).
 */
int32_t qdc_rmsnorm(void *out, const void *x, const void *weight, int64_t rows, int64_t width,
                    int64_t ld_x, int64_t ld_out, float eps, int32_t centered, int32_t x_dtype,
                    int32_t out_dtype, hipStream_t stream);

/*
 * residual = x + mixed; out = zero-centred RMSNorm(residual) with weight, in
 * one pass over contiguous rows of `width`.  Replaces native_residual_rms
 * (ext/amdgpu_workspace.jl:157-166; generic src/backbone.jl:347-350; CPU
 * src/backbone_cpu.jl:321-328) and, called with the next layer's input-norm
 * weight, the residual add of native_layer (src/backbone.jl:358-366) fused
 * with that next norm.  residual_dtype types x and residual, mixed_dtype
 * mixed, out_dtype out and weight.  Supported: all bf16, or an f32 residual
 * stream with an f32 or bf16 addend and an f32 or bf16 output, or with an f32
 * addend and a bf16x2 output (bf16 weight).  The sum is formed and
 * normalised in fp32.  residual may equal x (or mixed of the same type); out
 * may equal x or mixed of the same type; out and residual must differ.
 */
int32_t qdc_residual_rmsnorm(void *residual, void *out, const void *x, const void *mixed,
                             const void *weight, int64_t rows, int64_t width, float eps,
                             int32_t residual_dtype, int32_t mixed_dtype, int32_t out_dtype,
                             hipStream_t stream);

/*
 * qdc_rmsnorm and qdc_residual_rmsnorm with the DeltaNet input mask fused into
 * the store: normalised row r is multiplied by (float)token_mask[r] in fp32
 * before it is rounded to out_dtype; the residual output is not masked.
 * token_mask is a device int32 vector of `rows` entries, 0 or 1 (the prepared
 * mask of native_prepare_mask, ext/amdgpu_workspace.jl:151-155, validated on
 * the host like the ids).  Replaces the separate `masked .= x .* mask` pass at
 * the head of delta_attention (ext/amdgpu_delta.jl:130-133; generic
 * src/backbone.jl:286): the norm producing a DeltaNet layer's input writes the
 * masked rows directly, as the reference's fused masked normalisation does
 * (residual_input_rms! and the first-layer fused_normalization,
 * ext/metal_normalization.jl:369-432, with native_layer_outputs(...,
 * Val(true)) skipping the multiply, src/backbone.jl:372-376).  Arguments and
 * status otherwise as the unmasked entry points; token_mask may not overlap an
 * output.
 */
int32_t qdc_rmsnorm_masked(void *out, const void *x, const void *weight,
                           const int32_t *token_mask, int64_t rows, int64_t width, int64_t ld_x,
                           int64_t ld_out, float eps, int32_t centered, int32_t x_dtype,
                           int32_t out_dtype, hipStream_t stream);

int32_t qdc_residual_rmsnorm_masked(void *residual, void *out, const void *x, const void *mixed,
                                    const void *weight, const int32_t *token_mask, int64_t rows,
                                    int64_t width, float eps, int32_t residual_dtype,
                                    int32_t mixed_dtype, int32_t out_dtype, hipStream_t stream);

/*
 * Per-head zero-centred RMSNorm fused with half-split partial RoPE, for the Q
 * heads and the K heads of full attention in one launch.
 * Replaces prepare_head_kernel! (ext/amdgpu_attention.jl:1-43, launches
 * :122-147); generic native_rms + native_rope (src/backbone.jl:200-235); CPU
 * cpu_full_rms! + cpu_full_rope! (src/backbone_cpu.jl:113-136).
 *   Q row (t, h), h < heads:    in  q_in  + t*q_in_tok  + h*q_in_head
 *                               out q_out + t*q_out_tok + h*q_out_head
 *   K row (t, g), g < kv_heads: likewise with k_*.
 * Rows of a tensor must not overlap (token-major, or head-major
 * (dim, tokens, heads) as the reference AMDGPU layout).
 * q_in_head = 2*head_dim reads q straight out of the interleaved q||gate
 * projection (src/backbone.jl:226-227).  For i < rotary_dim/2 the pair
 * (i, i+rotary_dim/2) is rotated by the angle of position
 * p = pos_offset + t % seq_len:  a' = a*cos - b*sin, b' = b*cos + a*sin, with
 * cos_table/sin_table fp32 [table_len, rotary_dim/2] (see qdc_rope_tables);
 * dims >= rotary_dim pass through normalised.  heads or kv_heads may be 0 to
 * process only one side (its pointers may then be NULL).  Outputs must not
 * overlap inputs unless out == in with identical strides.
 */
int32_t qdc_qk_norm_rope(void *q_out, void *k_out, const void *q_in, const void *k_in,
                         const void *q_norm, const void *k_norm, const float *cos_table,
                         const float *sin_table, int64_t tokens, int64_t heads, int64_t kv_heads,
                         int64_t head_dim, int64_t rotary_dim, int64_t seq_len, int64_t pos_offset,
                         int64_t table_len, int64_t q_in_tok, int64_t q_in_head, int64_t q_out_tok,
                         int64_t q_out_head, int64_t k_in_tok, int64_t k_in_head, int64_t k_out_tok,
                         int64_t k_out_head, float eps, int32_t dtype, hipStream_t stream);

/*
 * qdc_qk_norm_rope over a batch of sequences in one launch, each output with
 * its own stride between sequences: token t = s*seq_len + i (sequence s,
 * position pos_offset + i) writes
 *   Q row (t, h):  q_out + s*q_out_seq + i*q_out_tok + h*q_out_head
 * and likewise K.  Inputs are addressed as in qdc_qk_norm_rope.  With
 * q_out_seq = H*seq_len*head_dim, q_out_tok = head_dim and
 * q_out_head = seq_len*head_dim the output is head-major per sequence,
 * [batch, heads, seq_len, head_dim], the layout of batched attention
 * products; q_out_seq = seq_len*q_out_tok is qdc_qk_norm_rope.  The reference
 * runs one sequence per call (ext/amdgpu_attention.jl:108-147, output
 * (dim, tokens, heads)); this entry point does the same work for a batch in
 * one launch.  Arguments, checks and status otherwise as qdc_qk_norm_rope.
 */
int32_t qdc_qk_norm_rope_batched(void *q_out, void *k_out, const void *q_in, const void *k_in,
                                 const void *q_norm, const void *k_norm, const float *cos_table,
                                 const float *sin_table, int64_t tokens, int64_t heads,
                                 int64_t kv_heads, int64_t head_dim, int64_t rotary_dim,
                                 int64_t seq_len, int64_t pos_offset, int64_t table_len,
                                 int64_t q_in_tok, int64_t q_in_head, int64_t q_out_seq,
                                 int64_t q_out_tok, int64_t q_out_head, int64_t k_in_tok,
                                 int64_t k_in_head, int64_t k_out_seq, int64_t k_out_tok,
                                 int64_t k_out_head, float eps, int32_t dtype, hipStream_t stream);

/*
 * The attention prologue of a full-attention layer in one launch, for `batch`
 * sequences of `seq_len` tokens (token t = b*seq_len + s at position
 * pos_offset + s): each Q and K head row is normalised with its zero-centred
 * RMSNorm weight and rotated by half-split partial RoPE (as qdc_qk_norm_rope),
 * and each V head row is moved, into the layouts the two attention products
 * read as plain batched GEMMs:
 *   q_out [batch, heads, seq_len, head_dim]
 *   k_out [batch, kv_heads, head_dim, seq_len]   (K transposed)
 *   v_out [batch, kv_heads, seq_len, head_dim]
 * (contiguous).  Inputs: Q row (t, h) at q_in + t*q_in_tok + h*q_in_head
 * (q_in_head = 2*head_dim reads q out of the interleaved q||gate projection);
 * K row (t, g) at k_in + t*k_in_tok + g*head_dim, V row (t, g) at
 * v_in + t*v_in_tok + g*head_dim (inputs may share one packed projection).
 * Replaces prepare_head_kernel! for Q and for K and prepare_value_kernel!
 * (ext/amdgpu_attention.jl:1-59, launches :119-155): K and V are not expanded
 * per query head, since the heads/kv_heads query heads of KV head g are the
 * rows of one [heads/kv_heads * seq_len, head_dim] block of q_out.  heads a
 * multiple of kv_heads; tables as qdc_qk_norm_rope (pos_offset + seq_len <=
 * table_len); outputs may not overlap each other or an input.  heads = 0
 * prepares K and V only (q_out, q_in and q_norm are then unused and may be
 * NULL): the keys and values over a whole context for a query projected
 * apart, as the final-query attention of the last-token forward does
 * (cpu_final_full_attention, src/backbone_cpu.jl:984-1034).
 */
int32_t qdc_attention_prepare(void *q_out, void *k_out, void *v_out, const void *q_in,
                              const void *k_in, const void *v_in, const void *q_norm,
                              const void *k_norm, const float *cos_table, const float *sin_table,
                              int64_t batch, int64_t seq_len, int64_t heads, int64_t kv_heads,
                              int64_t head_dim, int64_t rotary_dim, int64_t pos_offset,
                              int64_t table_len, int64_t q_in_tok, int64_t q_in_head,
                              int64_t k_in_tok, int64_t v_in_tok, float eps, int32_t dtype,
                              hipStream_t stream);

/*
 * Host-side RoPE tables, fp32 [n_pos, rotary_dim/2] each, built the way the
 * reference CPU path builds them (cpu_full_workspace src/backbone_cpu.jl:90-111):
 * freq_i = 1/theta^(2i/rotary_dim) and angle = freq_i*pos in fp32, cos/sin of
 * that fp32 angle correctly rounded to fp32.  Host memory; the caller copies
 * them to the device once per (rotary_dim, theta, length).
 */
int32_t qdc_rope_tables(float *cos_table, float *sin_table, int64_t n_pos, int64_t rotary_dim,
                        float theta);

/*
 * Gated RMSNorm of the DeltaNet output, per (token, head) row of `width`:
 * out = ((x*s)*w)*silu(z), silu(z) = z/(1+exp(-z)), not centred.
 * Replaces the two-pass native_rms(...; centered=false) + broadcast
 * (ext/amdgpu_delta.jl:181-184; generic src/backbone.jl:339-341; CPU
 * cpu_delta_gate_output! ext/QwenDecisionCoreLoopVectorizationExt.jl:373-390).
 * Row (t, h) reads x + t*x_tok + h*width and z + t*z_tok + h*width (z may sit
 * inside the packed projection) and writes out + t*out_tok + h*width.
 * dtype types x, z and weight; out_dtype equals dtype, or is QDC_BF16X2 with
 * dtype QDC_BF16 (the out-projection input in the split form).  out may equal
 * x when their types and strides agree.
 */
int32_t qdc_gated_rmsnorm(void *out, const void *x, const void *z, const void *weight,
                          int64_t tokens, int64_t heads, int64_t width, int64_t x_tok,
                          int64_t z_tok, int64_t out_tok, float eps, int32_t dtype,
                          int32_t out_dtype, hipStream_t stream);

/*
 * SwiGLU: out[t, i] = silu(gate[t, i]) * up[t, i] for i < width.
 * Replaces mlp_gate_kernel! (ext/amdgpu_mlp.jl:63-75; generic native_mlp_gate!
 * src/backbone.jl:352-355; CPU cpu_portable_gate!
 * ext/QwenDecisionCoreLoopVectorizationExt.jl:189-215).  For the packed
 * gate||up GEMM output pass gate = packed, up = packed + width,
 * ld_gate = ld_up = 2*width; out is the down-projection input.  dtype types
 * gate and up; out_dtype equals dtype, or is QDC_BF16X2 with dtype QDC_F32
 * (the down-projection input in the split form).  out may equal gate or up
 * when its type and stride equal theirs.
 */
int32_t qdc_swiglu(void *out, const void *gate, const void *up, int64_t tokens, int64_t width,
                   int64_t ld_gate, int64_t ld_up, int64_t ld_out, int32_t dtype,
                   int32_t out_dtype, hipStream_t stream);

/*
 * Gated delta rule recurrence of the DeltaNet layers -- the "existing path"
 * recurrence (delta_recurrent_kernel!, ext/amdgpu_delta.jl:37-81; CPU
 * cpu_delta_recurrent_step! src/backbone_cpu.jl:681-705), not one of the fused
 * row kernels; provided so backbone_hidden runs at speed.  Per sequence b and
 * value head h (key head h / (heads / key_heads)), state S[value_dim, key_dim]
 * from zero, for t = 0..seq-1:  f = exp(decay);  u = beta*(v - f*S k);
 * S = f*S + u k^T;  out = S q.  fp32 inputs: q, k [batch, seq, key_heads,
 * key_dim] (q already L2-normalised and scaled) with their token rows ld_qk
 * elements apart, v [batch, seq, heads, value_dim] with rows ld_v apart
 * (ld_qk >= key_heads*key_dim, ld_v >= heads*value_dim: contiguous tensors
 * pass those widths, the column blocks of qdc_delta_prologue's one
 * [tokens, q|k|v] buffer pass its row length), beta and decay [batch, seq,
 * heads] contiguous; out [batch, seq, heads, value_dim] contiguous in
 * out_dtype.  key_dim 1..256.
 */
int32_t qdc_delta_scan(void *out, int32_t out_dtype, const float *q, const float *k,
                       const float *v, const float *beta, const float *decay, int64_t batch,
                       int64_t seq, int64_t heads, int64_t key_heads, int64_t key_dim,
                       int64_t value_dim, int64_t ld_qk, int64_t ld_v, hipStream_t stream);

/*
 * DeltaNet prologue in one pass over the packed projection rows
 * [q | k | v | z | a | b] (widths kh*kd, kh*kd, vh*vd, vh*vd, vh, vh; row
 * stride ld elements, proj_dtype): causal depthwise convolution of the qkv
 * block with `taps` taps per sequence of seq_len tokens (conv fp32
 * [channels, taps], tap 0 on the oldest row), SiLU, then per key head
 * q / (sqrt(sum(q^2) + 1e-6) * sqrt(kd)) and k / sqrt(sum(k^2) + 1e-6); v
 * passes through; beta = sigmoid(b), decay = a_decay * softplus(a + dt_bias).
 * Outputs fp32: q, k [tokens, kh*kd] with token rows ld_qk elements apart,
 * v [tokens, vh*vd] with rows ld_v apart (ld_qk >= kh*kd, ld_v >= vh*vd),
 * beta and decay [tokens, vh] contiguous.  Separate contiguous q, k, v pass
 * their widths; one [tokens, q|k|v] buffer (q, k, v its column blocks, the
 * layout the forward uses: each token's outputs one contiguous row) passes
 * its row length 2*kh*kd + vh*vd for both.  q, k and v may share rows only
 * as disjoint column blocks (QDC_ERR_ALIAS otherwise).  Replaces
 * causal_depthwise_kernel!, qk_normalize_kernel! and the beta/decay
 * broadcasts (ext/amdgpu_delta.jl:1-33, 83-113, 154-159; generic
 * src/backbone.jl:264-296; CPU src/backbone_cpu.jl:411-427, 501-533).
 */
int32_t qdc_delta_prologue(float *q, float *k, float *v, float *beta, float *decay,
                           const void *proj, int32_t proj_dtype, int64_t ld, const float *conv,
                           int64_t taps, const float *a_decay, const float *dt_bias,
                           int64_t tokens, int64_t seq_len, int64_t key_heads, int64_t key_dim,
                           int64_t value_heads, int64_t value_dim, int64_t ld_qk, int64_t ld_v,
                           hipStream_t stream);

/*
 * Masked, scaled softmax of attention score rows: scores fp32 [batch, heads,
 * queries, keys] (contiguous); query q of a row sits at position q + q_offset;
 * key i is visible when i <= position and (mask == NULL or mask[b * keys + i]
 * != 0); value = scores * scale if visible else -floatmax(Float32); probs =
 * exp(value - max) / sum (fp32 or bf16, contiguous like scores; may equal
 * scores when fp32).  A row with no visible key gets 1/keys everywhere.
 * Replaces attention_softmax_kernel! (ext/amdgpu_attention.jl:61-88, launch
 * :158-165; generic mask and softmax src/backbone.jl:237-242, 252-256).
 */
int32_t qdc_attention_softmax(void *probs, int32_t probs_dtype, const float *scores,
                              const int32_t *mask, int64_t batch, int64_t heads,
                              int64_t queries, int64_t keys, int64_t q_offset, float scale,
                              hipStream_t stream);

/*
 * Output-gate merge: out[t, h*head_dim + r] = values[b, h, s, r] *
 * sigmoid(gate[t*gate_tok + h*gate_head + r]) for t = b*seq + s; values fp32
 * [batch, heads, seq, head_dim] contiguous (the PV GEMM output), gate and out
 * in gate_dtype / out_dtype with the given token and head strides (elements);
 * out_dtype may be QDC_BF16X2 (the out-projection input in the split form).
 * Replaces merge_gate_kernel! (ext/amdgpu_attention.jl:90-106, launch :168-176;
 * generic src/backbone.jl:258-259).
 */
int32_t qdc_attention_gate(void *out, int32_t out_dtype, const float *values, const void *gate,
                           int32_t gate_dtype, int64_t batch, int64_t seq, int64_t heads,
                           int64_t head_dim, int64_t gate_tok, int64_t gate_head, int64_t out_tok,
                           hipStream_t stream);

/*
 * Plain device copy of `bytes` bytes (a multiple of 16; both pointers 16-byte
 * aligned, QDC_ERR_SHAPE otherwise; no overlap), one 16-byte chunk per thread
 * with nontemporal loads and stores.  No counterpart in the reference: it is
 * the single-launch bandwidth ceiling that the benchmark measures beside each
 * row kernel at the same byte count.
 */
int32_t qdc_copy(void *dst, const void *src, int64_t bytes, hipStream_t stream);

/*
 * qdc_copy in another launch shape: `chunks_per_thread` (1, 2, 4 or 8) 16-byte
 * chunks per thread in workgroups of `block` (256 or 512) threads, every load
 * before the first store; the k-th load instruction of a workgroup covers its
 * k-th run of `block` consecutive chunks.  Other values: QDC_ERR_SHAPE.
 * qdc_copy is (1, 256).  No counterpart in the reference: the benchmark times
 * several shapes beside each kernel and holds the kernel against the fastest.
 */
int32_t qdc_copy_grid(void *dst, const void *src, int64_t bytes, int32_t chunks_per_thread,
                      int32_t block, hipStream_t stream);

/*
 * Random-row copy: destination row i (row_bytes * repeat bytes, rows
 * contiguous) holds `repeat` copies of source row rows[i] (rows: device int32,
 * each in [0, n_src); one outside writes zeros).  row_bytes a multiple of 16,
 * repeat 1 to 4, both pointers 16-byte aligned, fewer than 2^31 chunks of 16
 * bytes (QDC_ERR_SHAPE otherwise); no overlap.  No counterpart in the
 * reference: the single-launch ceiling of the embedding gather's access
 * pattern (rows read at random places of a large table, written contiguously;
 * repeat = 2 writes as many bytes as the fp32-widening gather, repeat = 3 as
 * many as the gather fused with the first bf16 norm) that the benchmark times
 * beside the gathers.
 */
/*
 * Two copies in one launch: src0 -> dst0 (bytes0) and src1 -> dst1 (bytes1),
 * in the launch shapes of qdc_copy_grid; thread t moves its chunks of both
 * streams at the same offsets, every load before the first store.  No
 * destination may overlap a source or the other destination.  No counterpart
 * in the reference: the ceiling of a row kernel that reads two tensors and
 * writes two (the residual norm: x and the addend in, the residual stream and
 * the normalised rows out), which the benchmark times beside it.
 */
int32_t qdc_copy_pair(void *dst0, const void *src0, int64_t bytes0, void *dst1,
                      const void *src1, int64_t bytes1, int32_t chunks_per_thread, int32_t block,
                      hipStream_t stream);

int32_t qdc_copy_rows(void *dst, const void *src, const int32_t *rows, int64_t n_rows,
                      int64_t n_src, int64_t row_bytes, int32_t repeat, hipStream_t stream);

/*
 * Launches `workgroups` workgroups of 256 threads that do nothing (fewer than
 * 2^24 workgroups, QDC_ERR_SHAPE otherwise).  No counterpart in the reference:
 * the fixed cost of a launch of a row kernel's grid, which the benchmark times
 * beside the kernel and its same-size copy.
 */
int32_t qdc_empty(int64_t workgroups, hipStream_t stream);

/*
 * out[i] = 1 / sqrt(sum_squares[i] / width + eps), fp32, exactly as every
 * RMSNorm kernel of this library scales a row with that sum of squares: the
 * division (a multiply by 2^-k when width is a power of two), the add, then
 * RN(1 / RN(sqrt(.))) as 1.0f / sqrtf computes it (n < 2^32 - 256; out may
 * equal sum_squares).  No counterpart in the reference: it exposes the row
 * scale of cpu_rmsnorm! (src/backbone_cpu.jl:344) so that tests can compare it
 * with the CPU's correctly rounded square root and division.
 */
int32_t qdc_row_scale(float *out, const float *sum_squares, int64_t n, float width, float eps,
                      hipStream_t stream);

/*
 * Adds to *mismatches (a device uint64) the number of fp32 bit patterns
 * first + k, 0 <= k < count (count <= 2^32 - first), for which the row
 * kernels' 1 / sqrt(x) differs in any bit from the general expression
 * 1.0f / sqrtf(x) (two NaN results count as equal).  No counterpart in the
 * reference: a self-check of the short hardware-estimate sequence the row
 * kernels use for 2^-96 <= x < inf; a sweep of all 2^32 patterns finds none.
 */
int32_t qdc_row_scale_check(uint32_t first, int64_t count, uint64_t *mismatches,
                            hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif

# amdgpu_hip.jl -- QwenDecisionCore.jl's AMDGPU device methods on libqdc_hip.so.
#
# A drop-in for the Julia-authored kernels of the AMDGPU package extension
# (ext/QwenDecisionCoreAMDGPUExt.jl:1-45).  QwenBackbone(dir; device=:amdgpu),
# backbone_hidden and backbone_last_hidden keep their signatures; the row work of
# the forward runs in the hand-written gfx950 kernels of libqdc_hip.so, reached
# through `ccall`, while the GEMMs stay on rocBLAS (`native_linear`,
# `batched_matmul!`) as before.
#
# Wiring, in ext/QwenDecisionCoreAMDGPUExt.jl:
#     include("amdgpu_workspace.jl")   # keeps ForwardWorkspace, scratch, native_matmul,
#                                      # native_forward_scope, native_prepare_mask
#     include("amdgpu_mlp.jl")         # keeps PackedMLP, the weight packing, native_linear
#     include("amdgpu_hip.jl")         # this file, in place of amdgpu_delta.jl and
#                                      # amdgpu_attention.jl
# and delete from the two kept files the methods this file defines (Julia refuses
# to overwrite a method while a package precompiles):
#     native_rms              ext/amdgpu_workspace.jl:113-149  -> qdc_rmsnorm
#     native_residual_rms     ext/amdgpu_workspace.jl:157-166  -> qdc_residual_rmsnorm
#     native_hidden_forward   ext/amdgpu_workspace.jl:168-204  -> the layer loop below
#     native_gather           ext/amdgpu_workspace.jl:206-236  -> qdc_check_ids, qdc_embedding_gather
#     native_mlp              ext/amdgpu_mlp.jl:63-91          -> qdc_swiglu
# full_attention (ext/amdgpu_attention.jl:108-178) and delta_attention
# (ext/amdgpu_delta.jl:115-187) come from this file only.  native_hidden_states
# and native_delta_attention(..., ::Val{true}) are new methods for ROCArrays
# (their generic versions stay in src/backbone.jl:372-411).
#
# Arrays are column-major (width, rows), which is the library's row-major
# [rows, width] in the same memory, so pointers pass through unchanged and the
# element strides below are Julia's leading dimensions.  Everything is Float32,
# as the reference's AMDGPU path is (dtype code QDC_F32).

import Libdl

const QDC_F32 = Int32(0)
const QDC_BF16 = Int32(1)
const QDC_BF16X2 = Int32(2)  # output only: two bf16 terms per fp32 value

# ---------------------------------------------------------------- library --
# Loaded on first use, as src/cpu_mkl.jl:18-66 loads MKL: a missing library is
# an error at the first call, never a silent fallback.
const QDC_HANDLE = Ref{Ptr{Cvoid}}(C_NULL)
const QDC_SYMBOLS = Dict{Symbol,Ptr{Cvoid}}()
const QDC_LOCK = ReentrantLock()

qdc_library_path() = get(ENV, "QDC_HIP_LIBRARY", "libqdc_hip.so")

# QDC_HIP_VERSION of the header these bindings follow; a library built from
# another header is refused at load, since a changed signature would pass its
# arguments in the wrong slots without any error.
const QDC_HIP_VERSION = "qdc_hip 0.3.1"

function qdc_open()
    handle = Libdl.dlopen(qdc_library_path())
    built = unsafe_string(ccall(Libdl.dlsym(handle, :qdc_version), Cstring, ()))
    built == QDC_HIP_VERSION ||
        error("$(qdc_library_path()) is $built; these bindings need $QDC_HIP_VERSION")
    return handle
end

function qdc_sym(name::Symbol)
    lock(QDC_LOCK) do
        get!(QDC_SYMBOLS, name) do
            QDC_HANDLE[] == C_NULL && (QDC_HANDLE[] = qdc_open())
            Libdl.dlsym(QDC_HANDLE[], name)
        end
    end
end

qdc_status_string(status::Int32) =
    unsafe_string(ccall(qdc_sym(:qdc_status_string), Cstring, (Int32,), status))

qdc_version() = unsafe_string(ccall(qdc_sym(:qdc_version), Cstring, ()))

# Status -> exception: shape errors are DimensionMismatch, other argument errors
# ArgumentError (as the methods they replace throw them), launch failures error().
function qdc_check(status::Int32, what::AbstractString)
    status == 0 && return nothing
    text = qdc_status_string(status)
    status == Int32(-2) && throw(DimensionMismatch("$what: $text"))
    status < 0 && throw(ArgumentError("$what: $text"))
    error("$what: HIP error $status ($text)")
end

qdc_ptr(x::AMDGPU.ROCArray) = reinterpret(Ptr{Cvoid}, pointer(x))
qdc_fptr(x::AMDGPU.ROCArray{Float32}) = reinterpret(Ptr{Float32}, pointer(x))
qdc_iptr(x::AMDGPU.ROCArray{Int32}) = reinterpret(Ptr{Int32}, pointer(x))
qdc_stream() = reinterpret(Ptr{Cvoid}, AMDGPU.stream().stream)   # task-local HIP stream

# ------------------------------------------------------ the C entry points --
# One method per declaration of include/qdc_hip.h, same argument order and C
# types (the repository's tests parse these tuples against the header).

qdc_embedding_gather(out, out_dtype, table, table_dtype, ids, n_ids, vocab, hidden, error_flag,
                     stream) =
    ccall(qdc_sym(:qdc_embedding_gather), Int32,
          (Ptr{Cvoid}, Int32, Ptr{Cvoid}, Int32, Ptr{Int32}, Int64, Int64, Int64, Ptr{Int32},
           Ptr{Cvoid}),
          out, out_dtype, table, table_dtype, ids, n_ids, vocab, hidden, error_flag, stream)

qdc_embedding_gather_rmsnorm(hidden, normed, table, table_dtype, ids, weight, normed_dtype,
                             token_mask, n_ids, vocab, width, eps, error_flag, stream) =
    ccall(qdc_sym(:qdc_embedding_gather_rmsnorm), Int32,
          (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int32, Ptr{Int32}, Ptr{Cvoid}, Int32, Ptr{Int32},
           Int64, Int64, Int64, Float32, Ptr{Int32}, Ptr{Cvoid}),
          hidden, normed, table, table_dtype, ids, weight, normed_dtype, token_mask, n_ids, vocab,
          width, eps, error_flag, stream)

qdc_check_ids(ids::Vector{Int64}, vocab) =
    ccall(qdc_sym(:qdc_check_ids), Int32, (Ptr{Int64}, Int64, Int64), ids, length(ids), vocab)

qdc_rmsnorm(out, x, weight, rows, width, ld_x, ld_out, eps, centered, x_dtype, out_dtype,
            stream) =
    ccall(qdc_sym(:qdc_rmsnorm), Int32,
          (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Float32, Int32, Int32,
           Int32, Ptr{Cvoid}),
          out, x, weight, rows, width, ld_x, ld_out, eps, centered, x_dtype, out_dtype, stream)

qdc_residual_rmsnorm(residual, out, x, mixed, weight, rows, width, eps, residual_dtype,
                     mixed_dtype, out_dtype, stream) =
    ccall(qdc_sym(:qdc_residual_rmsnorm), Int32,
          (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Float32,
           Int32, Int32, Int32, Ptr{Cvoid}),
          residual, out, x, mixed, weight, rows, width, eps, residual_dtype, mixed_dtype,
          out_dtype, stream)

qdc_rmsnorm_masked(out, x, weight, token_mask, rows, width, ld_x, ld_out, eps, centered, x_dtype,
                   out_dtype, stream) =
    ccall(qdc_sym(:qdc_rmsnorm_masked), Int32,
          (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Int32}, Int64, Int64, Int64, Int64, Float32,
           Int32, Int32, Int32, Ptr{Cvoid}),
          out, x, weight, token_mask, rows, width, ld_x, ld_out, eps, centered, x_dtype,
          out_dtype, stream)

qdc_residual_rmsnorm_masked(residual, out, x, mixed, weight, token_mask, rows, width, eps,
                            residual_dtype, mixed_dtype, out_dtype, stream) =
    ccall(qdc_sym(:qdc_residual_rmsnorm_masked), Int32,
          (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Int32}, Int64, Int64,
           Float32, Int32, Int32, Int32, Ptr{Cvoid}),
          residual, out, x, mixed, weight, token_mask, rows, width, eps, residual_dtype,
          mixed_dtype, out_dtype, stream)

qdc_qk_norm_rope(q_out, k_out, q_in, k_in, q_norm, k_norm, cos_table, sin_table, tokens, heads,
                 kv_heads, head_dim, rotary_dim, seq_len, pos_offset, table_len, q_in_tok,
                 q_in_head, q_out_tok, q_out_head, k_in_tok, k_in_head, k_out_tok, k_out_head,
                 eps, dtype, stream) =
    ccall(qdc_sym(:qdc_qk_norm_rope), Int32,
          (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Float32},
           Ptr{Float32}, Int64, Int64, Int64, Int64, Int64, Int64, Int64, Int64, Int64, Int64,
           Int64, Int64, Int64, Int64, Int64, Int64, Float32, Int32, Ptr{Cvoid}),
          q_out, k_out, q_in, k_in, q_norm, k_norm, cos_table, sin_table, tokens, heads,
          kv_heads, head_dim, rotary_dim, seq_len, pos_offset, table_len, q_in_tok, q_in_head,
          q_out_tok, q_out_head, k_in_tok, k_in_head, k_out_tok, k_out_head, eps, dtype, stream)

qdc_qk_norm_rope_batched(q_out, k_out, q_in, k_in, q_norm, k_norm, cos_table, sin_table, tokens,
                         heads, kv_heads, head_dim, rotary_dim, seq_len, pos_offset, table_len,
                         q_in_tok, q_in_head, q_out_seq, q_out_tok, q_out_head, k_in_tok,
                         k_in_head, k_out_seq, k_out_tok, k_out_head, eps, dtype, stream) =
    ccall(qdc_sym(:qdc_qk_norm_rope_batched), Int32,
          (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Float32},
           Ptr{Float32}, Int64, Int64, Int64, Int64, Int64, Int64, Int64, Int64, Int64, Int64,
           Int64, Int64, Int64, Int64, Int64, Int64, Int64, Int64, Float32, Int32, Ptr{Cvoid}),
          q_out, k_out, q_in, k_in, q_norm, k_norm, cos_table, sin_table, tokens, heads,
          kv_heads, head_dim, rotary_dim, seq_len, pos_offset, table_len, q_in_tok, q_in_head,
          q_out_seq, q_out_tok, q_out_head, k_in_tok, k_in_head, k_out_seq, k_out_tok,
          k_out_head, eps, dtype, stream)

qdc_attention_prepare(q_out, k_out, v_out, q_in, k_in, v_in, q_norm, k_norm, cos_table,
                      sin_table, batch, seq_len, heads, kv_heads, head_dim, rotary_dim,
                      pos_offset, table_len, q_in_tok, q_in_head, k_in_tok, v_in_tok, eps, dtype,
                      stream) =
    ccall(qdc_sym(:qdc_attention_prepare), Int32,
          (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
           Ptr{Cvoid}, Ptr{Float32}, Ptr{Float32}, Int64, Int64, Int64, Int64, Int64, Int64,
           Int64, Int64, Int64, Int64, Int64, Int64, Float32, Int32, Ptr{Cvoid}),
          q_out, k_out, v_out, q_in, k_in, v_in, q_norm, k_norm, cos_table, sin_table, batch,
          seq_len, heads, kv_heads, head_dim, rotary_dim, pos_offset, table_len, q_in_tok,
          q_in_head, k_in_tok, v_in_tok, eps, dtype, stream)

qdc_rope_tables(cos_table, sin_table, n_pos, rotary_dim, theta) =
    ccall(qdc_sym(:qdc_rope_tables), Int32,
          (Ptr{Float32}, Ptr{Float32}, Int64, Int64, Float32),
          cos_table, sin_table, n_pos, rotary_dim, theta)

qdc_gated_rmsnorm(out, x, z, weight, tokens, heads, width, x_tok, z_tok, out_tok, eps, dtype,
                  out_dtype, stream) =
    ccall(qdc_sym(:qdc_gated_rmsnorm), Int32,
          (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Int64,
           Int64, Float32, Int32, Int32, Ptr{Cvoid}),
          out, x, z, weight, tokens, heads, width, x_tok, z_tok, out_tok, eps, dtype, out_dtype,
          stream)

qdc_swiglu(out, gate, up, tokens, width, ld_gate, ld_up, ld_out, dtype, out_dtype, stream) =
    ccall(qdc_sym(:qdc_swiglu), Int32,
          (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Int64, Int32, Int32,
           Ptr{Cvoid}),
          out, gate, up, tokens, width, ld_gate, ld_up, ld_out, dtype, out_dtype, stream)

qdc_delta_scan(out, out_dtype, q, k, v, beta, decay, batch, seq, heads, key_heads, key_dim,
               value_dim, ld_qk, ld_v, stream) =
    ccall(qdc_sym(:qdc_delta_scan), Int32,
          (Ptr{Cvoid}, Int32, Ptr{Float32}, Ptr{Float32}, Ptr{Float32}, Ptr{Float32},
           Ptr{Float32}, Int64, Int64, Int64, Int64, Int64, Int64, Int64, Int64, Ptr{Cvoid}),
          out, out_dtype, q, k, v, beta, decay, batch, seq, heads, key_heads, key_dim,
          value_dim, ld_qk, ld_v, stream)

qdc_delta_prologue(q, k, v, beta, decay, proj, proj_dtype, ld, conv, taps, a_decay, dt_bias,
                   tokens, seq_len, key_heads, key_dim, value_heads, value_dim, ld_qk, ld_v,
                   stream) =
    ccall(qdc_sym(:qdc_delta_prologue), Int32,
          (Ptr{Float32}, Ptr{Float32}, Ptr{Float32}, Ptr{Float32}, Ptr{Float32}, Ptr{Cvoid},
           Int32, Int64, Ptr{Float32}, Int64, Ptr{Float32}, Ptr{Float32}, Int64, Int64, Int64,
           Int64, Int64, Int64, Int64, Int64, Ptr{Cvoid}),
          q, k, v, beta, decay, proj, proj_dtype, ld, conv, taps, a_decay, dt_bias, tokens,
          seq_len, key_heads, key_dim, value_heads, value_dim, ld_qk, ld_v, stream)

qdc_attention_softmax(probs, probs_dtype, scores, mask, batch, heads, queries, keys, q_offset,
                      scale, stream) =
    ccall(qdc_sym(:qdc_attention_softmax), Int32,
          (Ptr{Cvoid}, Int32, Ptr{Float32}, Ptr{Int32}, Int64, Int64, Int64, Int64, Int64,
           Float32, Ptr{Cvoid}),
          probs, probs_dtype, scores, mask, batch, heads, queries, keys, q_offset, scale, stream)

qdc_attention_gate(out, out_dtype, values, gate, gate_dtype, batch, seq, heads, head_dim,
                   gate_tok, gate_head, out_tok, stream) =
    ccall(qdc_sym(:qdc_attention_gate), Int32,
          (Ptr{Cvoid}, Int32, Ptr{Float32}, Ptr{Cvoid}, Int32, Int64, Int64, Int64, Int64, Int64,
           Int64, Int64, Ptr{Cvoid}),
          out, out_dtype, values, gate, gate_dtype, batch, seq, heads, head_dim, gate_tok,
          gate_head, out_tok, stream)

# --------------------------------------------------------------- RoPE tables --
# Built on the host as cpu_full_workspace builds them (src/backbone_cpu.jl:90-111),
# uploaded once per (device, rotary_dim, theta) and grown to the longest
# sequence seen; a sequence of `tokens` reads positions 0..tokens-1 of it.
const QDC_ROPE = Dict{Tuple{Int,Int,Float32},Tuple{Any,Any,Int}}()
const QDC_ROPE_LOCK = ReentrantLock()

function qdc_device_rope_tables(tokens::Int, rotary_dim::Int, theta)
    key = (AMDGPU.device_id(AMDGPU.device()), rotary_dim, Float32(theta))
    lock(QDC_ROPE_LOCK) do
        entry = get(QDC_ROPE, key, nothing)
        if entry === nothing || entry[3] < tokens
            half = rotary_dim ÷ 2
            cos_h = Matrix{Float32}(undef, half, tokens)     # row-major [tokens, half]
            sin_h = similar(cos_h)
            qdc_check(qdc_rope_tables(cos_h, sin_h, tokens, rotary_dim, Float32(theta)),
                      "rope_tables")
            entry = (AMDGPU.ROCArray(cos_h), AMDGPU.ROCArray(sin_h), tokens)
            QDC_ROPE[key] = entry
        end
        return entry
    end
end

# ------------------------------------------------------------- row methods --
# native_rms / rms_kernel! (ext/amdgpu_workspace.jl:113-149)
function QwenDecisionCore.native_rms(input::AMDGPU.ROCArray{Float32}, weight, eps;
                                     centered = true)
    output = scratch(Float32, size(input))
    width = size(input, 1)
    rows = length(input) ÷ width
    qdc_check(qdc_rmsnorm(qdc_ptr(output), qdc_ptr(input), qdc_ptr(weight), rows, width, width,
                          width, Float32(eps), Int32(centered), QDC_F32, QDC_F32, qdc_stream()),
              "native_rms")
    return output
end

# native_residual_rms (ext/amdgpu_workspace.jl:157-166): one pass instead of two
function QwenDecisionCore.native_residual_rms(x::AMDGPU.ROCArray{Float32,2,ROCBuffer}, mixed,
                                              weight, eps)
    residual = scratch(Float32, size(x))
    output = scratch(Float32, size(x))
    qdc_check(qdc_residual_rmsnorm(qdc_ptr(residual), qdc_ptr(output), qdc_ptr(x),
                                   qdc_ptr(mixed), qdc_ptr(weight), size(x, 2), size(x, 1),
                                   Float32(eps), QDC_F32, QDC_F32, QDC_F32, qdc_stream()),
              "native_residual_rms")
    return residual, output
end

# native_gather / gather_kernel! (ext/amdgpu_workspace.jl:206-236): ids checked
# on the host with the reference's message, uploaded as Int32
function QwenDecisionCore.native_gather(embedding::AMDGPU.ROCArray{Float32},
                                        ids::Vector{<:Integer})
    host = Vector{Int64}(ids)
    qdc_check_ids(host, size(embedding, 2)) == 0 ||
        throw(ArgumentError("Token ID is outside the vocabulary."))
    device_ids = scratch(Int32, (length(ids),))
    copyto!(device_ids, Int32.(host))
    output = scratch(Float32, (size(embedding, 1), length(ids)))
    qdc_check(qdc_embedding_gather(qdc_ptr(output), QDC_F32, qdc_ptr(embedding), QDC_F32,
                                   qdc_iptr(device_ids), length(ids), size(embedding, 2),
                                   size(embedding, 1), Ptr{Int32}(C_NULL), qdc_stream()),
              "native_gather")
    return output
end

# mlp_gate_kernel! inside native_mlp(::PackedMLP) (ext/amdgpu_mlp.jl:63-91):
# gate and up read as the two halves of the packed GEMM output
function QwenDecisionCore.native_mlp(mlp::PackedMLP, x::AMDGPU.ROCArray{Float32,2,ROCBuffer})
    projected = QwenDecisionCore.native_linear(mlp.gate_up, x)     # (2width, tokens)
    width, tokens = size(projected, 1) ÷ 2, size(x, 2)
    gated = scratch(Float32, (width, tokens))
    qdc_check(qdc_swiglu(qdc_ptr(gated), qdc_ptr(projected), qdc_ptr(projected) + 4width, tokens,
                         width, 2width, 2width, width, QDC_F32, QDC_F32, qdc_stream()),
              "native_mlp")
    return QwenDecisionCore.native_linear(mlp.down, gated)
end

# ---------------------------------------------------------- full attention --
# full_attention (ext/amdgpu_attention.jl:108-178).  The two prepare_head_kernel!
# launches and prepare_value_kernel! become one qdc_attention_prepare call: q
# normalised and rotated into (dim, tokens, heads), K into its transpose
# (tokens, dim, kv_heads) and v into (dim, tokens, kv_heads), read in place from
# the three projections.  K and V are never expanded per query head: the
# `groups` query heads of KV head g are the contiguous block
# q[:, :, (g-1)*groups+1:g*groups], one (dim, tokens*groups) matrix, so both
# products run as plain strided batches over the KV heads.
function QwenDecisionCore.full_attention(attention, x::AMDGPU.ROCArray{Float32,2,ROCBuffer},
                                         mask, cfg)
    tokens = size(x, 2)
    dim, heads, kv_heads = cfg.head_dim, cfg.heads, cfg.kv_heads
    groups = heads ÷ kv_heads
    qgate = QwenDecisionCore.native_linear(attention.q, x)         # (2dim*heads, tokens)
    kp = QwenDecisionCore.native_linear(attention.k, x)            # (dim*kv_heads, tokens)
    vp = QwenDecisionCore.native_linear(attention.v, x)
    q = scratch(Float32, (dim, tokens, heads))
    kt = scratch(Float32, (tokens, dim, kv_heads))                 # K transposed
    v = scratch(Float32, (dim, tokens, kv_heads))
    cos_d, sin_d, table_len = cfg.rotary_dim > 0 ?
        qdc_device_rope_tables(tokens, cfg.rotary_dim, cfg.rope_theta) :
        (nothing, nothing, 0)
    cos_p = cos_d === nothing ? Ptr{Float32}(C_NULL) : qdc_fptr(cos_d)
    sin_p = sin_d === nothing ? Ptr{Float32}(C_NULL) : qdc_fptr(sin_d)
    qdc_check(qdc_attention_prepare(qdc_ptr(q), qdc_ptr(kt), qdc_ptr(v), qdc_ptr(qgate),
                                    qdc_ptr(kp), qdc_ptr(vp), qdc_ptr(attention.q_norm),
                                    qdc_ptr(attention.k_norm), cos_p, sin_p, 1, tokens, heads,
                                    kv_heads, dim, cfg.rotary_dim, 0, table_len, 2dim * heads,
                                    2dim, dim * kv_heads, dim * kv_heads, Float32(cfg.eps),
                                    QDC_F32, qdc_stream()), "prepare_heads")
    scores = scratch(Float32, (tokens, tokens, heads))              # (keys, queries, heads)
    batched_matmul!(reshape(scores, tokens, tokens * groups, kv_heads), kt,
                    reshape(q, dim, tokens * groups, kv_heads), 'N', 'N')
    device_mask = mask isa AMDGPU.ROCArray ? mask : QwenDecisionCore.native_prepare_mask(x, mask)
    # attention_softmax_kernel! (ext/amdgpu_attention.jl:61-88), in place
    qdc_check(qdc_attention_softmax(qdc_ptr(scores), QDC_F32, qdc_fptr(scores),
                                    qdc_iptr(device_mask), 1, heads, tokens, tokens, 0,
                                    inv(sqrt(Float32(dim))), qdc_stream()), "attention_softmax")
    values = scratch(Float32, (dim, tokens, heads))
    batched_matmul!(reshape(values, dim, tokens * groups, kv_heads), v,
                    reshape(scores, tokens, tokens * groups, kv_heads), 'N', 'N')
    # merge_gate_kernel! (ext/amdgpu_attention.jl:90-106): the gate is the second
    # half of each head's q||gate rows, read in place
    merged = scratch(Float32, (dim * heads, tokens))
    qdc_check(qdc_attention_gate(qdc_ptr(merged), QDC_F32, qdc_fptr(values),
                                 qdc_ptr(qgate) + 4dim, QDC_F32, 1, tokens, heads, dim,
                                 2dim * heads, 2dim, dim * heads, qdc_stream()), "merge_gate")
    return QwenDecisionCore.native_linear(attention.out, merged)
end

# ----------------------------------------------------------------- DeltaNet --
# delta_attention (ext/amdgpu_delta.jl:115-187) on an input whose masked tokens
# are already zero: the convolution + SiLU, the q/k normalisation and the
# beta/decay broadcasts become one qdc_delta_prologue pass over the packed
# projection, the recurrence one qdc_delta_scan, and the RMS + SiLU(z) broadcast
# pair one qdc_gated_rmsnorm reading z in place inside the projection.  q, k and
# v are the column blocks of one [q|k|v, tokens] buffer, so each token's
# prologue output is one contiguous column (row stride 2*kh*kd + vh*vd).
function amdgpu_delta_attention(attention, x::AMDGPU.ROCArray{Float32,2,ROCBuffer}, cfg)
    tokens = size(x, 2)
    kd, kh, vd, vh = cfg.key_dim, cfg.key_heads, cfg.value_dim, cfg.value_heads
    projected = QwenDecisionCore.native_linear(attention.packed_projection, x)
    ld = size(projected, 1)
    qkv_width = size(attention.qkv, 1)
    qkv_rows = 2 * kh * kd + vh * vd
    qkv = scratch(Float32, (qkv_rows, tokens))
    q = qdc_fptr(qkv)
    k = q + 4 * kh * kd
    v = q + 8 * kh * kd
    beta = scratch(Float32, (vh, tokens))
    decay = scratch(Float32, (vh, tokens))
    qdc_check(qdc_delta_prologue(q, k, v, qdc_fptr(beta), qdc_fptr(decay), qdc_ptr(projected),
                                 QDC_F32, ld, qdc_fptr(attention.conv), size(attention.conv, 1),
                                 qdc_fptr(attention.a_decay), qdc_fptr(attention.dt_bias), tokens,
                                 tokens, kh, kd, vh, vd, qkv_rows, qkv_rows, qdc_stream()),
              "delta_prologue")
    result = scratch(Float32, (vd, vh, tokens))
    qdc_check(qdc_delta_scan(qdc_ptr(result), QDC_F32, q, k, v, qdc_fptr(beta), qdc_fptr(decay),
                             1, tokens, vh, kh, kd, vd, qkv_rows, qkv_rows, qdc_stream()),
              "delta_scan")
    gated = scratch(Float32, (vd * vh, tokens))
    qdc_check(qdc_gated_rmsnorm(qdc_ptr(gated), qdc_ptr(result), qdc_ptr(projected) + 4qkv_width,
                                qdc_ptr(attention.norm), tokens, vh, vd, vd * vh, ld, vd * vh,
                                Float32(cfg.eps), QDC_F32, QDC_F32, qdc_stream()), "gated_rms")
    return QwenDecisionCore.native_linear(attention.out, gated)
end

# qdc_delta_scan keeps a key row per lane group in registers up to 256 wide; a
# wider key head is refused here rather than sent to a generic AMDGPU.jl path
# (the reference's ext/amdgpu_delta.jl:121-128 falls back to `invoke`).
check_key_dim(cfg) = cfg.key_dim <= 256 ||
    throw(ArgumentError("The HIP DeltaNet path supports key_dim <= 256, got $(cfg.key_dim)."))

function QwenDecisionCore.delta_attention(attention, x::AMDGPU.ROCArray{Float32,2,ROCBuffer},
                                          mask, cfg)
    check_key_dim(cfg)
    # called directly with an unmasked input (the layer loops below never do)
    device_mask = mask isa AMDGPU.ROCArray ? mask : QwenDecisionCore.native_prepare_mask(x, mask)
    masked = scratch(Float32, size(x))
    masked .= x .* reshape(device_mask, 1, :)
    return amdgpu_delta_attention(attention, masked, cfg)
end

# premasked input, as native_layer_outputs(..., Val(true)) passes it (src/backbone.jl:372-376)
function QwenDecisionCore.native_delta_attention(attention,
                                                 x::AMDGPU.ROCArray{Float32,2,ROCBuffer}, mask,
                                                 cfg, ::Val{true})
    check_key_dim(cfg)
    return amdgpu_delta_attention(attention, x, cfg)
end

# -------------------------------------------------------------- layer loops --
# native_hidden_states / native_hidden_forward (src/backbone.jl:390-411; AMDGPU
# ext/amdgpu_workspace.jl:168-204).  Each layer's MLP residual add is fused with
# the next layer's input norm (the final norm after the last layer) in one
# qdc_residual_rmsnorm pass, which writes the next residual stream and its norm
# straight into two ping-pong buffers outside the per-layer scratch banks; the
# norm producing a DeltaNet layer's input applies the token mask itself
# (qdc_*_masked), as the reference's Metal forward does with residual_input_rms!
# (ext/metal_normalization.jl:369-470).  `last_only` normalises only the last
# column (the last-token forward).
is_delta(layer) = layer.attention.kind != :full

function qdc_layer_norm!(hidden_out, normed_out, residual, mixed, weight, device_mask, masked,
                         eps, columns, first_column)
    width = size(residual, 1)
    offset = 4 * width * (first_column - 1)
    if masked
        qdc_check(qdc_residual_rmsnorm_masked(qdc_ptr(hidden_out) + offset,
                                              qdc_ptr(normed_out) + offset,
                                              qdc_ptr(residual) + offset, qdc_ptr(mixed) + offset,
                                              qdc_ptr(weight),
                                              qdc_iptr(device_mask) + 4 * (first_column - 1),
                                              columns, width, Float32(eps), QDC_F32, QDC_F32,
                                              QDC_F32, qdc_stream()), "residual_input_rms")
    else
        qdc_check(qdc_residual_rmsnorm(qdc_ptr(hidden_out) + offset, qdc_ptr(normed_out) + offset,
                                       qdc_ptr(residual) + offset, qdc_ptr(mixed) + offset,
                                       qdc_ptr(weight), columns, width, Float32(eps), QDC_F32,
                                       QDC_F32, QDC_F32, qdc_stream()), "residual_rms")
    end
end

function amdgpu_layers(hidden::AMDGPU.ROCArray{Float32}, layers, mask, final_norm, cfg,
                       last_only::Bool)
    width, tokens = size(hidden, 1), size(hidden, 2)
    device_mask = mask isa AMDGPU.ROCArray ? mask :
                  QwenDecisionCore.native_prepare_mask(hidden, mask)
    buffers = ((scratch(Float32, (width, tokens)), scratch(Float32, (width, tokens))),
               (scratch(Float32, (width, tokens)), scratch(Float32, (width, tokens))))
    normalized = buffers[1][2]
    first = layers[1]
    if is_delta(first)
        qdc_check(qdc_rmsnorm_masked(qdc_ptr(normalized), qdc_ptr(hidden),
                                     qdc_ptr(first.input_norm), qdc_iptr(device_mask), tokens,
                                     width, width, width, Float32(cfg.eps), Int32(1), QDC_F32,
                                     QDC_F32, qdc_stream()), "input_rms")
    else
        qdc_check(qdc_rmsnorm(qdc_ptr(normalized), qdc_ptr(hidden), qdc_ptr(first.input_norm),
                              tokens, width, width, width, Float32(cfg.eps), Int32(1), QDC_F32,
                              QDC_F32, qdc_stream()), "input_rms")
    end
    owner = get(task_local_storage(), WORKSPACE_KEY, nothing)
    for (index, layer) in enumerate(layers)
        destination = buffers[isodd(index) ? 2 : 1]
        last = index == length(layers)
        if owner !== nothing   # per-kind scratch banks, as ext/amdgpu_workspace.jl:183-195
            root_slots, root_cursor = owner.active_slots, owner.cursor
            owner.active_slots = get!(() -> Any[], owner.layer_slots, layer.attention.kind)
            owner.cursor = 0
        end
        try
            mixed = is_delta(layer) ?
                QwenDecisionCore.native_delta_attention(layer.attention, normalized, device_mask,
                                                        cfg, Val(true)) :
                QwenDecisionCore.full_attention(layer.attention, normalized, device_mask, cfg)
            residual, post = QwenDecisionCore.native_residual_rms(hidden, mixed, layer.post_norm,
                                                                  cfg.eps)
            mlp = QwenDecisionCore.native_mlp(layer.mlp, post)
            weight = last ? final_norm : layers[index+1].input_norm
            masked = !last && is_delta(layers[index+1])
            columns, from = last && last_only ? (1, tokens) : (tokens, 1)
            qdc_layer_norm!(destination[1], destination[2], residual, mlp, weight, device_mask,
                            masked, cfg.eps, columns, from)
        finally
            owner === nothing || ((owner.active_slots, owner.cursor) = (root_slots, root_cursor))
        end
        hidden, normalized = destination
    end
    return last_only ? view(normalized, :, tokens:tokens) : normalized
end

QwenDecisionCore.native_hidden_states(hidden::AMDGPU.ROCArray{Float32}, layers, mask,
                                      final_norm, cfg) =
    amdgpu_layers(hidden, layers, mask, final_norm, cfg, false)

QwenDecisionCore.native_hidden_forward(hidden::AMDGPU.ROCArray{Float32}, layers, mask,
                                       final_norm, cfg) =
    amdgpu_layers(hidden, layers, mask, final_norm, cfg, true)

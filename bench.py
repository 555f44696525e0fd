"""Benchmark of the fused per-layer row kernels on one MI355X.

A step is one launch of each fused kernel over its synthetic batch:

  rmsnorm_f32        x [8192, 1024] fp32, zero-centred RMSNorm
  rmsnorm_bf16       x [8192, 1024] bf16
  headnorm_f32       per-head q/k rows [81920, 256] fp32 (8192 tokens x 10 heads)
  headnorm_bf16      same in bf16
  qk_norm_rope_bf16  Q [8192, 8, 256] + K [8192, 2, 256] bf16, rotary 64 of 256,
                     theta 1e7, positions 0..2047 reset per sequence (4 x 2048)
  gather_bf16        16384 ids (8 x 2048) from a [248320, 1024] bf16 table
  swiglu_bf16        gate/up [16384, 3584] bf16 -> bf16
  gated_rms_bf16     DeltaNet output x, z [16384, 16, 128] bf16
  residual_rms_bf16  x, mixed [16384, 1024] bf16 -> residual, normalised

The same run measures the kernels that widen the path around the attention and
DeltaNet layers (reported under "widened", not in `value`):

  attn_softmax_bf16    masked softmax of scores [8, 8, 2048, 2048] fp32 -> bf16
                       (causally hidden scores are never read)
  attn_gate_bf16       PV output [8, 8, 2048, 256] fp32 x sigmoid(gate) -> bf16
  delta_prologue_bf16  DeltaNet conv + SiLU + q/k L2 norm + gates, 16384 tokens,
                       16 key/value heads of 128, packed bf16 projection -> fp32
  delta_scan_bf16      gated delta rule over 8 x 2048 tokens, 16 heads 128 x 128
                       (chunked form on the fp32 matrix cores; reported in
                       TFLOP/s against the dense fp32 MFMA peak too)

Beside each fused row kernel the run times the library's plain streaming copy
of the same total bytes, half read and half written, in the same way and in
several launch shapes (qdc_copy, qdc_copy_grid): `copy_pct_peak` is what the
fastest single launch of that size reaches (`copy_shape`), and `pct_of_copy`
the kernel's bandwidth as a share of it (`pct_of_one_chunk_copy` against the
one-chunk-per-thread shape alone).  The residual norms whose two inputs and two
outputs have the same sizes are also held against a copy of those two streams
in one launch (qdc_copy_pair, the same launch shapes): `pair_copy_us`,
`pct_of_pair_copy`.

Inputs are resident in HBM before timing.  Every kernel cycles through
several input/output buffer sets totalling more than 512 MB, so the 256 MB
last-level cache cannot serve repeated launches.  The K launches of each
kernel are captured once in a HIP graph (no host launch overhead between the
few-microsecond kernels) and replayed between HIP events recorded on the same
stream; a kernel's average launch duration is its replay time / K.  value =
total algorithmic bytes of the K steps / total time of the fused row kernels (GB/s).  Algorithmic bytes
= inputs read once + outputs written once + parameter vectors (+ RoPE tables).

The CPU baseline times the C oracle (a single-threaded restatement of the
reference CPU path, fp32 arithmetic as in the reference) on a quarter of each
kernel's rows, repeated to at least 10 s, on this machine's host cores, then
the same mix on every host core the process may use (OpenMP over rows,
`all_cores`, at least 5 s) as an upper bound for a threaded CPU path.
With the end-to-end run, `backbone.cpu` times the oracle's backbone_hidden of
one 2048-token sequence of the same backbone in fp32 on the host (the
reference runs one sequence per call) and `backbone.speedup_vs_cpu` compares.

`decision` follows the reference's own inference benchmark (backbone_last_hidden
of one sequence of 64, 128, 256 and 512 tokens on its synthetic 4-layer model's
shapes, host in and out, median of 21 per length, aggregate = sum of medians),
eager and served from recorded HIP graphs, with the oracle on one host thread
beside it and the reference's published figures for the same protocol.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu] [--no-e2e]
                       [--no-decision | --decision-only]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "qwendecisioncore.jl_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "achieved HBM GB/s (% of peak) per fused kernel; backbone_hidden tokens/s"
PEAK_GBS = 8000.0            # MI355X HBM3E
MFMA_F32_PEAK_TF = 157.3     # MI355X dense fp32 matrix-core peak
ROTATE_BYTES = 640 << 20     # > 2x the 256 MB last-level cache
PMC_FILE = os.path.join(ROOT, "profiles", "pmc_traffic.json")


def _sets(set_bytes: int) -> int:
    return max(2, math.ceil(ROTATE_BYTES / set_bytes))


def _qkv_views(tokens, heads, dim, dev):
    """q, k, v [tokens, heads, dim] fp32 as the column blocks of one
    [tokens, q|k|v] buffer (the DeltaNet prologue's output layout in the
    forward)."""
    import torch
    w = heads * dim
    qkv = torch.empty((tokens, 3 * w), dtype=torch.float32, device=dev)
    return tuple(qkv[:, i * w:(i + 1) * w].view(tokens, heads, dim) for i in range(3))


class Kernel:
    """One fused kernel at its benchmark shape with rotating buffer sets."""

    def __init__(self, name, symbol, algo_bytes, make_set, launch, shape, dtype, group="hot",
                 flops=None, launches=None, ceiling=None, workgroups=None, pair=None):
        self.name, self.symbol, self.algo_bytes = name, symbol, algo_bytes
        self.shape, self.dtype = shape, dtype
        # (bytes0, bytes1): a kernel that reads two tensors and writes two of the
        # same sizes is also held against qdc_copy_pair of those two streams
        self.pair = pair
        # (make_set, launch) of a plain kernel with this kernel's access pattern
        # and bytes, timed beside it as its ceiling (None: the contiguous copy)
        self.ceiling = ceiling
        # workgroups of the kernel's launch grid (the rocprofv3 trace's Grid_Size
        # / 256 confirms it), for the empty-launch floor timed beside it
        self.workgroups = workgroups
        # "hot": the fused row kernels at the per-kernel shapes; "next": widened;
        # "forward": the fused row kernels as the 0.8B-like forward launches them
        self.group, self.flops = group, flops
        self.launches = launches  # launches per forward ("forward" group)
        self.launch = launch
        self.sets = [make_set(i) for i in range(_sets(algo_bytes) if algo_bytes else 1)]
        self.graph = None
        self.avg_ms = None

    def run(self, i):
        self.launch(self.sets[i % len(self.sets)])


def row_copy_ceiling(dev, g, table, n, repeat):
    """The random-row copy (qdc_copy_rows) of the same table: n rows at
    uniformly random places, written contiguously `repeat` times (repeat 2
    writes as many bytes as the fp32-widening gather).  Bytes: the rows read,
    the rows written and the int32 row indices, as the gather's."""
    import torch
    from qdc_amd import ops
    vocab, hidden = table.shape
    row_bytes = hidden * table.element_size()

    def make_set(i):
        return (torch.randint(0, vocab, (n,), generator=g, device=dev, dtype=torch.int32),
                torch.empty((n, hidden * repeat), dtype=table.dtype, device=dev))

    return make_set, lambda s: ops.device_copy_rows(s[1], table, s[0], repeat)


def build_kernels(dev):
    import torch
    from qdc_amd import ops

    g = torch.Generator(device=dev)
    g.manual_seed(0)
    bf, f32 = torch.bfloat16, torch.float32

    def randn(shape, dtype, scale=1.0):
        return (torch.randn(shape, generator=g, device=dev, dtype=f32) * scale).to(dtype)

    kernels = []

    def rms(name, rows, width, dtype, rows_per_wg):
        es = 2 if dtype == bf else 4
        w = randn((width,), dtype, 0.02)
        kernels.append(Kernel(
            name, "rms_rows_fast", 2 * rows * width * es + width * es,
            lambda i: (randn((rows, width), dtype), torch.empty((rows, width), dtype=dtype, device=dev)),
            lambda s: ops.native_rms(s[0], w, 1e-6, out=s[1]), [rows, width], str(dtype)[6:],
            workgroups=rows // rows_per_wg))

    # rows per workgroup of rms_rows_fast: 256 / lanes per row (64 lanes x 4 groups
    # for fp32 rows of 1024, 16 x 8 for bf16 rows of 1024, 32 x 2 and 16 x 2 for
    # fp32 and bf16 rows of 256)
    rms("rmsnorm_f32", 8192, 1024, f32, 2)   # 2 wavefronts per 1024-wide fp32 row
    rms("rmsnorm_bf16", 8192, 1024, bf, 16)
    rms("headnorm_f32", 81920, 256, f32, 8)
    rms("headnorm_bf16", 81920, 256, bf, 16)

    T, H, KV, hd, rd, seq = 8192, 8, 2, 256, 64, 2048
    qn, kn = randn((hd,), bf, 0.02), randn((hd,), bf, 0.02)
    tables = ops.rope_tables(seq, rd, 1e7, dev)
    kernels.append(Kernel(
        "qk_norm_rope_bf16", "qk_norm_rope_fast",
        2 * T * (H + KV) * hd * 2 + 2 * hd * 2 + 2 * seq * (rd // 2) * 4,
        lambda i: (randn((T, H, hd), bf), randn((T, KV, hd), bf),
                   torch.empty((T, H, hd), dtype=bf, device=dev),
                   torch.empty((T, KV, hd), dtype=bf, device=dev)),
        lambda s: ops.prepare_heads(s[0], s[1], qn, kn, tables, rd, 1e-6, seq_len=seq,
                                    q_out=s[2], k_out=s[3]),
        [T, H, KV, hd, rd, seq], "bfloat16",
        # 16-lane groups of 4 Q heads / 1 K head, 16 groups per workgroup
        workgroups=T * H // 4 // 16 + T * KV // 16))

    vocab, hidden, n = 248320, 1024, 16384
    table = randn((vocab, hidden), bf, 0.02)
    kernels.append(Kernel(
        "gather_bf16", "gather_flat", 2 * n * hidden * 2 + n * 4,
        lambda i: (torch.randint(0, vocab, (n,), generator=g, device=dev, dtype=torch.int32),
                   torch.empty((n, hidden), dtype=bf, device=dev)),
        lambda s: ops.native_gather(table, s[0], out=s[1]), [vocab, hidden, n], "bfloat16",
        ceiling=row_copy_ceiling(dev, g, table, n, 1)))

    Ti, I = 16384, 3584
    kernels.append(Kernel(
        "swiglu_bf16", "swiglu_fast", 3 * Ti * I * 2,
        lambda i: (randn((Ti, I), bf), randn((Ti, I), bf), torch.empty((Ti, I), dtype=bf, device=dev)),
        lambda s: ops.native_mlp_gate(s[0], s[1], out=s[2]), [Ti, I], "bfloat16"))

    Tg, Hg, Wg = 16384, 16, 128
    wg = randn((Wg,), bf, 1.0)
    kernels.append(Kernel(
        "gated_rms_bf16", "rms_rows_fast", 3 * Tg * Hg * Wg * 2 + Wg * 2,
        lambda i: (randn((Tg, Hg, Wg), bf), randn((Tg, Hg, Wg), bf),
                   torch.empty((Tg, Hg, Wg), dtype=bf, device=dev)),
        lambda s: ops.native_gated_rms(s[0], s[1], wg, 1e-6, out=s[2]), [Tg, Hg, Wg], "bfloat16"))

    Tr, Hr = 16384, 1024
    wr = randn((Hr,), bf, 0.02)
    kernels.append(Kernel(
        "residual_rms_bf16", "rms_rows_fast", 4 * Tr * Hr * 2 + Hr * 2,
        lambda i: (randn((Tr, Hr), bf), randn((Tr, Hr), bf),
                   torch.empty((Tr, Hr), dtype=bf, device=dev), torch.empty((Tr, Hr), dtype=bf, device=dev)),
        lambda s: ops.native_residual_rms(s[0], s[1], wr, 1e-6, residual=s[2], out=s[3]),
        [Tr, Hr], "bfloat16", workgroups=Tr // 8,  # 32 lanes x 4 groups per row
        pair=(Tr * Hr * 2, Tr * Hr * 2)))  # x -> residual, mixed -> normalised

    # Attention row work of one full-attention layer (8 sequences of 2048, 8 heads).
    # Softmax: the causally visible scores are read (the rest are -floatmax by
    # definition and never loaded), every probability is written.
    Ba, Ha, Sa = 8, 8, 2048
    amask = torch.ones((Ba, Sa), dtype=torch.int32, device=dev)
    kernels.append(Kernel(
        "attn_softmax_bf16", "softmax_rows_fast",
        Ba * Ha * Sa * (Sa + 1) // 2 * 4 + Ba * Ha * Sa * Sa * 2 + Ba * Sa * 4,
        lambda i: (randn((Ba, Ha, Sa, Sa), f32),
                   torch.empty((Ba, Ha, Sa, Sa), dtype=bf, device=dev)),
        lambda s: ops.attention_softmax(s[0], amask, 0.0625, out=s[1]), [Ba, Ha, Sa, Sa],
        "float32->bfloat16", group="next"))
    hda = 256
    kernels.append(Kernel(
        "attn_gate_bf16", "gate_merge_fast",
        Ba * Ha * Sa * hda * 4 + 2 * Ba * Sa * Ha * hda * 2,
        lambda i: (randn((Ba, Ha, Sa, hda), f32), randn((Ba * Sa, Ha, 2 * hda), bf),
                   torch.empty((Ba * Sa, Ha * hda), dtype=bf, device=dev)),
        lambda s: ops.attention_gate(s[0], s[1][:, :, hda:], out=s[2]), [Ba * Sa, Ha, hda],
        "bfloat16", group="next"))

    # DeltaNet prologue of one layer: 16384 tokens, 16 key/value heads of 128,
    # packed projection [qkv | z | a | b] in bf16 (z is not read), fp32 outputs
    # q, k, v as the column blocks of one [T, q|k|v] buffer, as the forward
    # writes them; rows padded to a multiple of 256 columns as the backbone
    # packs the weight.
    Tp, hp, dp = 16384, 16, 128
    cqp = 3 * hp * dp
    widthp = -(-(cqp + hp * dp + 2 * hp) // 256) * 256
    convp = randn((cqp, 4), f32, 0.5)
    a_dec = -torch.exp(randn((hp,), f32, 0.5))
    dtb = randn((hp,), f32)
    kernels.append(Kernel(
        "delta_prologue_bf16", "delta_prologue_fast",
        Tp * (cqp + 2 * hp) * 2 + Tp * (cqp + 2 * hp) * 4 + cqp * 4 * 4 + 2 * hp * 4,
        lambda i: (randn((Tp, widthp), bf), *_qkv_views(Tp, hp, dp, dev),
                   torch.empty((Tp, hp), dtype=f32, device=dev),
                   torch.empty((Tp, hp), dtype=f32, device=dev)),
        lambda s: ops.delta_prologue(s[0], convp, a_dec, dtb, 2048, hp, dp, hp, dp, out=s[1:]),
        [Tp, hp, dp], "bfloat16->float32", group="next"))

    # DeltaNet recurrence of one layer (not a row kernel: bound by the sequential
    # per-token state update, reported with its bytes for reference)
    Bs, Ss = 8, 2048

    def scan_set(i):  # q, k, v read from one [tokens, q|k|v] buffer, as in the forward
        qkv = torch.empty((Bs, Ss, 3, hp, dp), dtype=f32, device=dev)
        qkv[:, :, 0] = torch.nn.functional.normalize(randn((Bs, Ss, hp, dp), f32),
                                                     dim=-1) / math.sqrt(dp)
        qkv[:, :, 1] = torch.nn.functional.normalize(randn((Bs, Ss, hp, dp), f32), dim=-1)
        qkv[:, :, 2] = randn((Bs, Ss, hp, dp), f32)
        return (qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2],
                torch.sigmoid(randn((Bs, Ss, hp), f32)), -torch.rand((Bs, Ss, hp), generator=g,
                                                                        device=dev),
                torch.empty((Bs, Ss, hp, dp), dtype=bf, device=dev))
    kernels.append(Kernel(
        "delta_scan_bf16", "delta_scan",
        Bs * Ss * hp * dp * 4 * 3 + Bs * Ss * hp * 4 * 2 + Bs * Ss * hp * dp * 2,
        scan_set,
        lambda s: ops.delta_scan(s[0], s[1], s[2], s[3], s[4], bf, out=s[5]),
        [Bs, Ss, hp, dp], "float32->bfloat16", group="next",
        # chunked form per (token, head): 2 kd vd each for K S^T, Q S^T and the
        # state update, 64 (kd + vd) for K K^T, Q K^T, U and O = 7 kd vd at 128 x 128
        flops=Bs * Ss * hp * (6 * dp * dp + 64 * (dp + dp))))
    return kernels


def build_forward_kernels(dev):
    """The fused row kernels exactly as one bf16 forward of the 0.8B-like
    backbone launches them (8 x 2048 = 16384 tokens; fp32 residual stream, bf16
    GEMM activations, q/k read in place from the packed projection and written
    head-major per sequence, z read in place from the DeltaNet projection),
    each over rotating buffer sets like the per-kernel benchmark."""
    import torch
    from qdc_amd import ops
    from qdc_amd.config import qwen35_08b_config
    cfg = qwen35_08b_config()
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    bf, f32 = torch.bfloat16, torch.float32

    def randn(shape, dtype, scale=1.0):
        return (torch.randn(shape, generator=g, device=dev, dtype=f32) * scale).to(dtype)

    B, S = E2E_BATCH, E2E_SEQ
    T, Hd, I = B * S, cfg.hidden, cfg.intermediate
    n_full = sum(1 for k in cfg.layer_types if k == "full_attention")
    n_delta = len(cfg.layer_types) - n_full
    n_layers = len(cfg.layer_types)
    ks = []
    wb, wf = randn((Hd,), bf, 0.02), randn((Hd,), f32, 0.02)
    table = randn((cfg.vocab, Hd), bf, 0.02)
    # the gather fused with the first input norm, as the forward launches it:
    # bf16 table rows -> fp32 residual rows + bf16 normalised rows
    ks.append(Kernel(
        "fwd_gather_rms_bf16", "gather_rms_fast", T * Hd * (2 + 4 + 2) + T * 4 + Hd * 2,
        lambda i: (torch.randint(0, cfg.vocab, (T,), generator=g, device=dev, dtype=torch.int32),
                   torch.empty((T, Hd), dtype=f32, device=dev),
                   torch.empty((T, Hd), dtype=bf, device=dev)),
        lambda s: ops.native_gather_rms(table, s[0], wb, 1e-6, hidden=s[1], normed=s[2]),
        [T, Hd], "bfloat16->float32,bfloat16", group="forward", launches=1,
        ceiling=row_copy_ceiling(dev, g, table, T, 3)))
    # the two launches it replaces, at the same shapes (not launched by the forward)
    ks.append(Kernel(
        "fwd_gather_bf16_f32", "gather_widen", T * Hd * 2 + T * Hd * 4 + T * 4,
        lambda i: (torch.randint(0, cfg.vocab, (T,), generator=g, device=dev, dtype=torch.int32),
                   torch.empty((T, Hd), dtype=f32, device=dev)),
        lambda s: ops.native_gather(table, s[0], out=s[1], out_dtype=f32), [T, Hd],
        "bfloat16->float32", group="standalone",
        ceiling=row_copy_ceiling(dev, g, table, T, 2)))
    ks.append(Kernel(
        "fwd_input_rms_f32_bf16", "rms_rows_fast", T * Hd * (4 + 2) + Hd * 2,
        lambda i: (randn((T, Hd), f32), torch.empty((T, Hd), dtype=bf, device=dev)),
        lambda s: ops.native_rms(s[0], wb, 1e-6, out=s[1]), [T, Hd], "float32->bfloat16",
        group="standalone"))
    ks.append(Kernel(
        "fwd_residual_rms_f32_bf16", "rms_rows_fast", T * Hd * (4 + 4 + 4 + 2) + Hd * 2,
        lambda i: (randn((T, Hd), f32), randn((T, Hd), f32),
                   torch.empty((T, Hd), dtype=f32, device=dev),
                   torch.empty((T, Hd), dtype=bf, device=dev)),
        lambda s: ops.native_residual_rms(s[0], s[1], wb, 1e-6, residual=s[2], out=s[3]),
        [T, Hd], "float32->float32,bfloat16", group="forward", launches=2 * n_layers - 1))
    ks.append(Kernel(
        "fwd_final_rms_f32", "rms_rows_fast", T * Hd * 4 * 4 + Hd * 4,
        lambda i: (randn((T, Hd), f32), randn((T, Hd), f32),
                   torch.empty((T, Hd), dtype=f32, device=dev),
                   torch.empty((T, Hd), dtype=f32, device=dev)),
        lambda s: ops.native_residual_rms(s[0], s[1], wf, 1e-6, residual=s[2], out=s[3]),
        [T, Hd], "float32", group="forward", launches=1, pair=(T * Hd * 4, T * Hd * 4)))
    hd, nh, kv, rd = cfg.head_dim, cfg.heads, cfg.kv_heads, cfg.rotary_dim
    qn, kn = randn((hd,), bf, 0.02), randn((hd,), bf, 0.02)
    tables = ops.rope_tables(S, rd, cfg.rope_theta, dev)
    qkv_w = 2 * hd * nh + 2 * hd * kv

    def prep_launch(s):  # the packed projection [q | k | v | gate] as the forward lays it out
        ops.attention_prepare(s[0][:, :hd * nh].view(T, nh, hd),
                              s[0][:, hd * nh:hd * (nh + kv)].view(T, kv, hd),
                              s[0][:, hd * (nh + kv):hd * (nh + 2 * kv)].view(T, kv, hd),
                              qn, kn, tables, rd, 1e-6, B, out=s[1:])
    ks.append(Kernel(
        "fwd_attention_prepare_bf16", "attention_prepare_fast",
        2 * T * (nh + 2 * kv) * hd * 2 + 2 * hd * 2 + 2 * S * (rd // 2) * 4,
        lambda i: (randn((T, qkv_w), bf), torch.empty((B, nh, S, hd), dtype=bf, device=dev),
                   torch.empty((B, kv, hd, S), dtype=bf, device=dev),
                   torch.empty((B, kv, S, hd), dtype=bf, device=dev)),
        prep_launch, [B, S, nh, kv, hd, rd], "bfloat16", group="forward", launches=n_full))
    vh, vd = cfg.value_heads, cfg.value_dim
    cq = 2 * cfg.key_dim * cfg.key_heads + vh * vd
    pw = -(-(cq + vh * vd + 2 * vh) // 256) * 256
    wg = randn((vd,), bf, 1.0)
    ks.append(Kernel(
        "fwd_gated_rms_bf16", "rms_rows_fast", 3 * T * vh * vd * 2 + vd * 2,
        lambda i: (randn((T, vh, vd), bf), randn((T, pw), bf),
                   torch.empty((T, vh, vd), dtype=bf, device=dev)),
        lambda s: ops.native_gated_rms(s[0], s[1][:, cq:cq + vh * vd].view(T, vh, vd), wg, 1e-6,
                                       out=s[2]),
        [T, vh, vd], "bfloat16", group="forward", launches=n_delta))
    ks.append(Kernel(
        "fwd_swiglu_bf16", "swiglu_fast", 3 * T * I * 2,
        lambda i: (randn((T, 2 * I), bf), torch.empty((T, I), dtype=bf, device=dev)),
        lambda s: ops.native_mlp_gate(s[0][:, :I], s[0][:, I:], out=s[1]), [T, I], "bfloat16",
        group="forward", launches=n_layers))
    # the split GEMM-input variants (bf16 weights, split_gemm_inputs="all"): each
    # output element is two bf16 terms (4 bytes); `launches` counts them per
    # forward in that mode ("mlp" launches the residual norm 24 times and SwiGLU)
    X2 = ops.BF16X2
    ks.append(Kernel(
        "fwd_gather_rms_split", "gather_rms_fast", T * Hd * (2 + 4 + 4) + T * 4 + Hd * 2,
        lambda i: (torch.randint(0, cfg.vocab, (T,), generator=g, device=dev, dtype=torch.int32),
                   torch.empty((T, Hd), dtype=f32, device=dev),
                   torch.empty((T, 2 * Hd), dtype=bf, device=dev)),
        lambda s: ops.native_gather_rms(table, s[0], wb, 1e-6, hidden=s[1], normed=s[2],
                                        normed_dtype=X2),
        [T, Hd], "bfloat16->float32,bf16x2", group="split", launches=1,
        ceiling=row_copy_ceiling(dev, g, table, T, 4)))
    ks.append(Kernel(
        "fwd_residual_rms_f32_split", "rms_rows_fast", T * Hd * (4 + 4 + 4 + 4) + Hd * 2,
        lambda i: (randn((T, Hd), f32), randn((T, Hd), f32),
                   torch.empty((T, Hd), dtype=f32, device=dev),
                   torch.empty((T, 2 * Hd), dtype=bf, device=dev)),
        lambda s: ops.native_residual_rms(s[0], s[1], wb, 1e-6, residual=s[2], out=s[3],
                                          out_dtype=X2),
        [T, Hd], "float32->float32,bf16x2", group="split", launches=2 * n_layers - 1))
    ks.append(Kernel(
        "fwd_gated_rms_split", "rms_rows_fast", T * vh * vd * (2 + 2 + 4) + vd * 2,
        lambda i: (randn((T, vh, vd), bf), randn((T, pw), bf),
                   torch.empty((T, vh, 2 * vd), dtype=bf, device=dev)),
        lambda s: ops.native_gated_rms(s[0], s[1][:, cq:cq + vh * vd].view(T, vh, vd), wg, 1e-6,
                                       out=s[2], out_dtype=X2),
        [T, vh, vd], "bfloat16->bf16x2", group="split", launches=n_delta))
    ks.append(Kernel(
        "fwd_gate_merge_split", "gate_merge_fast", T * nh * hd * (4 + 2 + 4),
        lambda i: (randn((B, nh, S, hd), f32), randn((T, qkv_w), bf),
                   torch.empty((T, 2 * nh * hd), dtype=bf, device=dev)),
        lambda s: ops.attention_gate(s[0], s[1][:, hd * (nh + 2 * kv):].view(T, nh, hd),
                                     out_dtype=X2, out=s[2]),
        [B, S, nh, hd], "float32,bfloat16->bf16x2", group="split", launches=n_full))
    ks.append(Kernel(
        "fwd_swiglu_f32_split", "swiglu_fast", T * I * (4 + 4 + 4),
        lambda i: (randn((T, 2 * I), f32), torch.empty((T, 2 * I), dtype=bf, device=dev)),
        lambda s: ops.native_mlp_gate(s[0][:, :I], s[0][:, I:], out=s[1], out_dtype=X2),
        [T, I], "float32->bf16x2", group="split", launches=n_layers))
    return ks


def capture(kernels, steps):
    """One HIP graph per kernel holding `steps` launches over its rotating sets;
    a replay must reproduce the eager result exactly."""
    import torch
    stream = torch.cuda.Stream()
    for k in kernels:
        torch.cuda.synchronize()
        k.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(k.graph, stream=stream):
            for i in range(steps):
                k.run(i)
    torch.cuda.synchronize()


def check_replay(kernels, steps):
    """Replay output == eager output for the last set each graph wrote."""
    import torch
    for k in kernels:
        s = k.sets[(steps - 1) % len(k.sets)]
        outs = [t for t in s if t.dtype != torch.int32][-2:]
        k.graph.replay()
        torch.cuda.synchronize()
        replayed = [o.clone() for o in outs]
        k.run(steps - 1)
        torch.cuda.synchronize()
        for a, b in zip(replayed, outs):
            if not torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                               b.view(torch.int16) if b.dtype == torch.bfloat16 else b):
                raise RuntimeError(f"graph replay of {k.name} differs from the eager launch")


def time_gpu(kernels, steps):
    import torch
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in kernels]
    start.record(stream)
    for k, (a, b) in zip(kernels, marks):
        a.record(stream)
        k.graph.replay()
        b.record(stream)
    end.record(stream)
    torch.cuda.synchronize()
    for k, (a, b) in zip(kernels, marks):
        k.avg_ms = a.elapsed_time(b) / steps
    return start.elapsed_time(end)


def empty_floors(kernels, steps, warmup):
    """For each kernel with a known grid, qdc_empty over the same number of
    workgroups, graph-replayed like the kernels: the fixed cost of the launch."""
    import torch
    from qdc_amd import ops
    empties = [Kernel(f"empty_{k.name}", "empty_grid", 0, lambda i: (),
                      lambda st, n=k.workgroups, d=torch.device("cuda:0"): ops.empty_launch(n, d),
                      [k.workgroups], "-") for k in kernels if k.workgroups]
    for i in range(warmup):
        for e in empties:
            e.run(i)
    capture(empties, steps)
    for e in empties:
        e.graph.replay()
    time_gpu(empties, steps)
    return {e.name[len("empty_"):]: e for e in empties}


# Launch shapes of the copy ceiling, (16-byte chunks per thread, threads per
# workgroup): qdc_copy's one chunk per thread and the qdc_copy_grid shapes that
# measured faster at some sizes (2 or 4 chunks per thread at 33-67 MB,
# 512-thread workgroups at 352 MB).  Each kernel is held against the fastest.
COPY_SHAPES = ((1, 256), (2, 256), (4, 256), (1, 512))


def copy_ceilings(dev, kernels, steps, warmup):
    """For each kernel, the library's plain streaming copy (qdc_copy /
    qdc_copy_grid: 16-byte chunks, nontemporal) of the same total bytes, half
    read and half written, graph-replayed over rotating buffers like the
    kernels, in every shape of COPY_SHAPES (sharing one set of buffers): what
    a single launch moving that many bytes reaches on this GPU.  Returns
    {kernel: (fastest copy, random-row copy or None, {shape: copy}, fastest two-stream
    copy or None, {shape: two-stream copy})}; the two-stream copies (qdc_copy_pair)
    only for kernels with a `pair`."""
    import torch
    from qdc_amd import ops
    copies = []
    for k in kernels:
        side = (k.algo_bytes // 2) // 16 * 16
        bufs = {}

        def make_set(i, side=side, bufs=bufs):
            if i not in bufs:
                bufs[i] = (torch.empty(side, dtype=torch.uint8, device=dev),
                           torch.empty(side, dtype=torch.uint8, device=dev))
            return bufs[i]

        for cpt, blk in COPY_SHAPES:
            copies.append(Kernel(
                f"copy{cpt}x{blk}_{k.name}", "copy_chunks" if (cpt, blk) == (1, 256) else "copy_grid",
                2 * side, make_set,
                lambda st, cpt=cpt, blk=blk: ops.device_copy(st[1], st[0], cpt, blk), [side], "u8"))
        if k.ceiling is not None:  # the same access pattern as a plain copy
            make_set, launch = k.ceiling
            copies.append(Kernel(f"rows_{k.name}", "copy_rows", k.algo_bytes, make_set, launch,
                                 k.shape, k.dtype))
        if k.pair is not None:  # two streams, each read and written, in one launch
            b0, b1 = k.pair
            pbufs = {}

            def make_pair(i, b0=b0, b1=b1, pbufs=pbufs):
                if i not in pbufs:
                    pbufs[i] = tuple(torch.empty(n, dtype=torch.uint8, device=dev)
                                     for n in (b0, b0, b1, b1))
                return pbufs[i]

            for cpt, blk in COPY_SHAPES:
                copies.append(Kernel(
                    f"pair{cpt}x{blk}_{k.name}", "copy_pair", 2 * (b0 + b1), make_pair,
                    lambda st, cpt=cpt, blk=blk: ops.device_copy_pair(st[1], st[0], st[3], st[2],
                                                                      cpt, blk),
                    [b0, b1], "u8"))
    for i in range(warmup):
        for c in copies:
            c.run(i)
    capture(copies, steps)
    for c in copies:  # one untimed replay
        c.graph.replay()
    time_gpu(copies, steps)
    by_name = {c.name: c for c in copies}
    out = {}
    for k in kernels:
        shapes = {f"{cpt}x{blk}": by_name[f"copy{cpt}x{blk}_{k.name}"] for cpt, blk in COPY_SHAPES}
        best = min(shapes.values(), key=lambda c: c.avg_ms)
        pairs = {f"{cpt}x{blk}": by_name[f"pair{cpt}x{blk}_{k.name}"] for cpt, blk in COPY_SHAPES
                 if f"pair{cpt}x{blk}_{k.name}" in by_name}
        pair = min(pairs.values(), key=lambda c: c.avg_ms) if pairs else None
        out[k.name] = (best, by_name.get(f"rows_{k.name}"), shapes, pair, pairs)
    return out


PAIR_ROUNDS = 3


def paired_ratios(kernels, ceilings, rounds=PAIR_ROUNDS):
    """Each kernel's graph replayed right before its ceilings' graphs (the
    same-size copy, the random-row copy and the two-stream copy where there are
    those), in `rounds`
    rounds over all kernels: the median over rounds of ceiling time / kernel
    time.  Back to back, a kernel and its ceiling run in the same clock and
    memory state, which the separate timing phases above do not ensure."""
    import torch
    stream = torch.cuda.current_stream()
    ratios = {k.name: ([], [], []) for k in kernels}
    for _ in range(rounds):
        marks = []
        for k in kernels:
            c, rows, _, pair = ceilings[k.name][:4]
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
            ev[0].record(stream)
            k.graph.replay()
            ev[1].record(stream)
            c.graph.replay()
            ev[2].record(stream)
            if rows is not None:
                rows.graph.replay()
            ev[3].record(stream)
            if pair is not None:
                pair.graph.replay()
            ev[4].record(stream)
            marks.append((k, rows is not None, pair is not None, ev))
        torch.cuda.synchronize()
        for k, has_rows, has_pair, ev in marks:
            t_k = ev[0].elapsed_time(ev[1])
            ratios[k.name][0].append(ev[1].elapsed_time(ev[2]) / t_k)
            if has_rows:
                ratios[k.name][1].append(ev[2].elapsed_time(ev[3]) / t_k)
            if has_pair:
                ratios[k.name][2].append(ev[3].elapsed_time(ev[4]) / t_k)
    med = lambda v: sorted(v)[len(v) // 2] if v else None  # noqa: E731
    return {name: (med(a), med(b), med(c)) for name, (a, b, c) in ratios.items()}


CALIB_BYTES = 512 << 20


def calibrate(dev):
    """Plain device-to-device copies of CALIB_BYTES each (torch's copy kernel):
    the reference point that scales FETCH_SIZE / WRITE_SIZE to bytes."""
    import torch
    src = [torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev) for _ in range(2)]
    dst = [torch.empty_like(s) for s in src]
    for i in range(4):
        dst[i % 2].copy_(src[i % 2])
    torch.cuda.synchronize()
    print(f"calibration: 4 copies of {CALIB_BYTES} bytes", file=sys.stderr, flush=True)


E2E_BATCH, E2E_SEQ = 8, 2048


def fused_sequence(cfg, dev, tokens, split=None):
    """The fused row-kernel launches of one bf16 forward at `tokens` tokens
    (gather + first input norm, 2 residual norms per layer, SwiGLU per layer, the
    attention prologue per full-attention layer, gated norm per DeltaNet layer)
    on buffers of the forward's shapes and strides.  `split="mlp"` launches them
    as the forward with split MLP inputs does: the post-attention norm writes
    the split output, SwiGLU reads fp32 gate/up and writes the split output."""
    import torch
    from qdc_amd import ops
    bf, f32 = torch.bfloat16, torch.float32
    if split not in (None, "mlp"):
        raise ValueError("split must be None or 'mlp'")
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    rn = lambda shape, dt: torch.randn(shape, generator=g, device=dev).to(dt)  # noqa: E731
    H = cfg.hidden
    table = rn((cfg.vocab, H), bf)
    ids = torch.randint(0, cfg.vocab, (tokens,), generator=g, device=dev, dtype=torch.int32)
    w = rn((H,), bf)
    h, mixed = rn((tokens, H), f32), rn((tokens, H), f32)
    res, normed = torch.empty_like(h), torch.empty((tokens, H), dtype=bf, device=dev)
    mlp_in = ops.BF16X2 if split else None
    gu = rn((tokens, 2 * cfg.intermediate), f32 if split else bf)
    act = torch.empty((tokens, (2 if split else 1) * cfg.intermediate), dtype=bf, device=dev)
    post = torch.empty((tokens, 2 * H), dtype=bf, device=dev) if split else normed
    hd, nh, kv = cfg.head_dim, cfg.heads, cfg.kv_heads
    qkv = rn((tokens, 2 * hd * nh + 2 * hd * kv), bf)
    qn = rn((hd,), bf)
    # the layouts the forward writes for the attention products
    n_seq = tokens // E2E_SEQ
    prep_out = (torch.empty((n_seq, nh, E2E_SEQ, hd), dtype=bf, device=dev),
                torch.empty((n_seq, kv, hd, E2E_SEQ), dtype=bf, device=dev),
                torch.empty((n_seq, kv, E2E_SEQ, hd), dtype=bf, device=dev))
    tables = ops.rope_tables(E2E_SEQ, cfg.rotary_dim, cfg.rope_theta, dev)
    vw = cfg.value_dim * cfg.value_heads
    cq = 2 * cfg.key_dim * cfg.key_heads + vw
    proj = rn((tokens, cq + vw + 2 * cfg.value_heads), bf)
    dx = rn((tokens, cfg.value_heads, cfg.value_dim), bf)
    gated = torch.empty_like(dx)
    wv = rn((cfg.value_dim,), bf)
    I = cfg.intermediate

    def run():
        ops.native_gather_rms(table, ids, w, 1e-6, hidden=h, normed=normed)
        for kind in cfg.layer_types:
            if kind == "full_attention":
                ops.attention_prepare(qkv[:, :hd * nh].view(tokens, nh, hd),
                                      qkv[:, hd * nh:hd * (nh + kv)].view(tokens, kv, hd),
                                      qkv[:, hd * (nh + kv):hd * (nh + 2 * kv)].view(tokens, kv, hd),
                                      qn, qn, tables, cfg.rotary_dim, 1e-6, n_seq, out=prep_out)
            else:
                ops.native_gated_rms(dx, proj[:, cq:cq + vw].view(tokens, cfg.value_heads,
                                                                  cfg.value_dim), wv, 1e-6,
                                     out=gated)
            ops.native_residual_rms(h, mixed, w, 1e-6, residual=res, out=post, out_dtype=mlp_in)
            ops.native_mlp_gate(gu[:, :I], gu[:, I:], out=act, out_dtype=mlp_in)
            ops.native_residual_rms(res, mixed, w, 1e-6, residual=h, out=normed)
    return run


def widened_sequence(cfg, dev, batch, seq):
    """The widened kernels of one bf16 forward: per full-attention layer the
    masked softmax and the gate merge, per DeltaNet layer the prologue and the
    recurrence, on buffers of the forward's shapes."""
    import torch
    from qdc_amd import ops
    bf, f32 = torch.bfloat16, torch.float32
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    rn = lambda shape, dt: torch.randn(shape, generator=g, device=dev).to(dt)  # noqa: E731
    T = batch * seq
    H, hd = cfg.heads, cfg.head_dim
    scores = rn((batch, H, seq, seq), f32)
    probs = torch.empty(scores.shape, dtype=bf, device=dev)
    mask = None  # as in the forward: no padding
    values = rn((batch, H, seq, hd), f32)
    qgate = rn((T, H, 2 * hd), bf)
    merged = torch.empty((T, H * hd), dtype=bf, device=dev)
    kh, kd, vh, vd = cfg.key_heads, cfg.key_dim, cfg.value_heads, cfg.value_dim
    cq = 2 * kh * kd + vh * vd
    proj = rn((T, cq + vh * vd + 2 * vh), bf)
    conv = rn((cq, cfg.conv_kernel), f32)
    a_dec, dtb = -torch.exp(rn((vh,), f32)), rn((vh,), f32)
    qkv = torch.empty((T, cq), dtype=f32, device=dev)  # the forward's [T, q|k|v] rows
    outs = [qkv[:, :kh * kd].view(T, kh, kd), qkv[:, kh * kd:2 * kh * kd].view(T, kh, kd),
            qkv[:, 2 * kh * kd:].view(T, vh, vd)]
    outs += [torch.empty((T, vh), dtype=f32, device=dev) for _ in range(2)]
    scanned = torch.empty((batch, seq, vh, vd), dtype=bf, device=dev)
    scale = 1.0 / math.sqrt(hd)

    def run():
        for kind in cfg.layer_types:
            if kind == "full_attention":
                ops.attention_softmax(scores, mask, scale, out=probs)
                ops.attention_gate(values, qgate[:, :, hd:], out=merged)
            else:
                q, k, v, beta, decay = ops.delta_prologue(proj, conv, a_dec, dtb, seq, kh, kd,
                                                          vh, vd, out=outs)
                ops.delta_scan(q.view(batch, seq, kh, kd), k.view(batch, seq, kh, kd),
                               v.view(batch, seq, vh, vd), beta.view(batch, seq, vh),
                               decay.view(batch, seq, vh), out=scanned)
    return run


def _graph_ms(run):
    """Time one replay of `run` captured in a HIP graph (after one eager call)."""
    import torch
    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=torch.cuda.Stream()):
        run()
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b)


def e2e_benchmark(dev, steps=3, warmup=1):
    """backbone_hidden of the random-init Qwen3.5-0.8B-like backbone (24 layers,
    bf16 weights/activations, fp32 residual stream) on 8 sequences of 2048."""
    import torch
    from qdc_amd import backbone
    from qdc_amd.config import qwen35_08b_config
    from qdc_amd.weights import random_device_weights
    cfg = qwen35_08b_config()
    weights = random_device_weights(cfg, seed=0, device=dev, dtype=torch.bfloat16)
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    ids = torch.randint(0, cfg.vocab, (E2E_BATCH, E2E_SEQ), generator=g, device=dev,
                        dtype=torch.int32)
    mask = None  # no padding: every token is kept (the forward then does no masking work)

    def forward_ms(split, dtype=torch.bfloat16):
        model = backbone.QwenBackbone.from_weights(weights, cfg, dev, dtype,
                                                   split_gemm_inputs=split)
        for _ in range(warmup):
            out = model.forward(ids, mask)
        torch.cuda.synchronize()
        if not torch.isfinite(out).all():
            raise RuntimeError("non-finite backbone output")
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            model.forward(ids, mask)
        end.record()
        torch.cuda.synchronize()
        del model, out
        torch.cuda.empty_cache()
        return start.elapsed_time(end) / steps

    # headline: bf16 weights with the MLP's two GEMM inputs split, the fastest
    # bf16-weight mode that meets the 1e-2 end-to-end bar at 24 layers
    ms = forward_ms("mlp")
    all_split_ms = forward_ms("all")
    bf16_ms = forward_ms(False)
    # the same weights widened to fp32 (exact), fp32 activations and GEMMs
    fp32_ms = forward_ms(False, torch.float32)
    del weights
    torch.cuda.empty_cache()
    # this library's kernels of one forward, replayed from graphs on buffers of
    # the forward's shapes: the fused row kernels (as the headline mode and as
    # all-bf16 storage launch them), then the widened kernels
    fused_ms = _graph_ms(fused_sequence(cfg, dev, E2E_BATCH * E2E_SEQ, split="mlp"))
    torch.cuda.empty_cache()
    fused_bf16_ms = _graph_ms(fused_sequence(cfg, dev, E2E_BATCH * E2E_SEQ))
    torch.cuda.empty_cache()
    widened_ms = _graph_ms(widened_sequence(cfg, dev, E2E_BATCH, E2E_SEQ))
    torch.cuda.empty_cache()
    tps = lambda v: round(E2E_BATCH * E2E_SEQ / (v / 1e3), 1)  # noqa: E731
    return {"workload": "random-init Qwen3.5-0.8B-like backbone, 24 layers (18 DeltaNet + 6 full), "
                        "hidden 1024, vocab 248320, bf16 weights, fp32 residual stream, the MLP's "
                        "two GEMM inputs split into two bf16 terms (split_gemm_inputs='mlp')",
            "mode": "split_gemm_inputs='mlp'",
            "end_to_end_vs_fp32_oracle": {"24 layers, 64 tokens": 3.00e-3,
                                          "full size, first 64 positions": [3.11e-3, 3.13e-3],
                                          "bar": 1e-2, "meets_1e-2_end_to_end": True},
            "batch": E2E_BATCH, "seq_len": E2E_SEQ, "ms_per_forward": round(ms, 3),
            "tokens_per_s": tps(ms),
            "fused_kernels_ms": round(fused_ms, 3),
            "fused_kernel_time_share": round(fused_ms / ms, 4),
            "widened_kernels_ms": round(widened_ms, 3),
            "widened_kernel_time_share": round(widened_ms / ms, 4),
            "split_gemm_inputs_all": {
                "note": "every GEMM input split (split_gemm_inputs='all'): 2.31e-3 from the fp32 "
                        "oracle at 24 layers, within the 1e-2 bar",
                "ms_per_forward": round(all_split_ms, 3), "tokens_per_s": tps(all_split_ms)},
            "bf16_storage": {
                "note": "all-bf16 storage (bf16 GEMM inputs, no split): faster, but misses the "
                        "1e-2 end-to-end bar at 24 layers (1.40e-2 against the oracle with the "
                        "same storage points, 2.05e-2 against the fp32 oracle; the two xfails "
                        "of the GPU suite), so it is not the headline",
                "meets_1e-2_end_to_end": False,
                "end_to_end_24_layers": {"vs_same_storage_oracle": 1.40e-2, "vs_fp32_oracle": 2.05e-2},
                "ms_per_forward": round(bf16_ms, 3), "tokens_per_s": tps(bf16_ms),
                "fused_kernels_ms": round(fused_bf16_ms, 3),
                "fused_kernel_time_share": round(fused_bf16_ms / bf16_ms, 4),
                "widened_kernel_time_share": round(widened_ms / bf16_ms, 4)},
            "fp32": {
                "note": "the same weights widened to fp32 (exactly), fp32 activations and GEMMs: "
                        "the mode within 1e-5 of the fp32 oracle end to end",
                "ms_per_forward": round(fp32_ms, 3), "tokens_per_s": tps(fp32_ms)},
            "steps": steps, "warmup": warmup}


def cpu_backbone(n_tokens=None):
    """The oracle's backbone_hidden of one sequence of E2E_SEQ tokens (the
    reference runs one sequence per call) on the host: the same random-init
    0.8B-like backbone in fp32 (numpy GEMMs on the host BLAS threads, the
    oracle's row ops on one thread, as the reference CPU path with Julia's
    default single thread).  Weights are drawn on the host (seed 0)."""
    import numpy as np
    from oracle import forward
    from qdc_amd.config import qwen35_08b_config
    from qdc_amd.weights import random_weights
    n = n_tokens or E2E_SEQ
    cfg = qwen35_08b_config()
    weights = random_weights(cfg, seed=0)
    ids = np.random.default_rng(2).integers(0, cfg.vocab, size=n)
    t0 = time.perf_counter()
    hidden = forward.backbone_hidden(weights, cfg.as_dict(), ids, np.ones(n, np.int64))
    secs = time.perf_counter() - t0
    if not np.isfinite(hidden).all():
        raise RuntimeError("non-finite oracle backbone output")
    return {"tokens_per_s": round(n / secs, 1), "seconds": round(secs, 2),
            "sample": (f"oracle backbone_hidden, fp32, one sequence of {n} tokens, numpy GEMMs "
                       f"on the host BLAS threads, row ops on 1 thread, on '{cpu_model()}' "
                       f"({len(os.sched_getaffinity(0))} cores usable)")}


DECISION_LENGTHS = (64, 128, 256, 512)
# The reference's published numbers for the same protocol on its own hardware
# (benchmark/results/inference-next-15-2026-10-24.txt): aggregate of the four
# medians, backbone_last_hidden, Julia and BLAS on one thread.
DECISION_REFERENCE = {"cuda_rtx3060_ms": 6.421419, "cpu_xeon_e5_2699v3_1thread_ms": 115.952651,
                      "source": "benchmark/results/inference-next-15-2026-10-24.txt"}


def _median_ms(f, warm=4, samples=21):
    import statistics
    for _ in range(warm):
        f()
    times = []
    for _ in range(samples):
        t0 = time.perf_counter()
        f()
        times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times)


def decision_latency(dev, samples=21):
    """The reference's inference benchmark protocol (benchmark/inference.jl) on
    its synthetic model's shapes (benchmark/synthetic.jl: 4 layers, 3 DeltaNet +
    1 full attention, hidden 256, intermediate 512, fp32): backbone_last_hidden
    of one sequence of 64, 128, 256 and 512 tokens, ids (0..n-1) mod 256 and an
    all-ones mask from the host, the [hidden] result back on the host; 4 warm
    calls, then the median of 21 timed calls per length; the aggregate is the sum
    of the four medians.  Timed eager (one launch per op) and served from
    recorded HIP graphs (qdc_amd.graphs; recording, which also picks the faster
    GEMM library per length, excluded, as the reference excludes its CUDA graph
    recording).  Every graph result is checked against the eager result (1e-5
    normwise, fp32)."""
    import numpy as np
    import torch
    from qdc_amd import backbone
    from qdc_amd.config import synthetic_inference_config
    from qdc_amd.graphs import LastHiddenGraphs
    from qdc_amd.weights import random_weights
    cfg = synthetic_inference_config()
    model = backbone.QwenBackbone.from_weights(random_weights(cfg, seed=42), cfg, dev,
                                               torch.float32)
    graphs = LastHiddenGraphs(model, max_graphs=len(DECISION_LENGTHS))
    eager, graphed, libraries = {}, {}, {}
    for n in DECISION_LENGTHS:
        ids = np.arange(n) % min(256, cfg.vocab)
        mask = np.ones(n, np.int64)
        want = backbone.backbone_last_hidden(model, ids, mask)
        got = graphs(ids, mask)
        err = float(np.linalg.norm(got - want) / np.linalg.norm(want))
        if not err <= 1e-5:   # fp32: the products may come from the other GEMM library
            raise RuntimeError(f"graph-replayed last hidden is {err:.2e} from the eager one at {n}")
        entry = graphs.entry(n, False)
        libraries[n] = None if entry is None else entry.library
        eager[n] = _median_ms(lambda: backbone.backbone_last_hidden(model, ids, mask),
                              samples=samples)
        graphed[n] = _median_ms(lambda: graphs(ids, mask), samples=samples)
    agg_e, agg_g = sum(eager.values()), sum(graphed.values())
    return {"workload": "backbone_last_hidden, one sequence of 64/128/256/512 tokens, the "
                        "reference's synthetic inference model shapes (4 layers: 3 DeltaNet + 1 "
                        "full, hidden 256, intermediate 512), fp32, host ids in, host [hidden] out",
            "eager_ms": {str(n): round(v, 4) for n, v in eager.items()},
            "graph_ms": {str(n): round(v, 4) for n, v in graphed.items()},
            "aggregate_eager_ms": round(agg_e, 4), "aggregate_graph_ms": round(agg_g, 4),
            "graph_keys_eager": sorted(str(k) for k in graphs.eager_keys),
            "graph_gemm_library": {str(n): v for n, v in libraries.items()},
            "reference_published": DECISION_REFERENCE,
            "note": "the reference's figures are from other hardware (an RTX 3060 and a Xeon "
                    "E5-2699 v3); same protocol and model shapes, not the same machine"}


def cpu_decision(samples=5):
    """The oracle's forward of the same synthetic model on the host, one thread
    (BLAS limited to one thread as the reference's `julia -t 1` run), median of
    `samples` per length after one warm call; the last row is the result."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import forward
    from qdc_amd.config import synthetic_inference_config
    from qdc_amd.weights import random_weights
    cfg = synthetic_inference_config()
    weights = random_weights(cfg, seed=42)
    per = {}
    with threadpool_limits(limits=1):
        for n in DECISION_LENGTHS:
            ids = np.arange(n) % min(256, cfg.vocab)
            mask = np.ones(n, np.int64)
            per[n] = _median_ms(lambda: forward.backbone_hidden(weights, cfg.as_dict(), ids,
                                                                mask)[-1],
                                warm=1, samples=samples)
    return {"ms": {str(n): round(v, 3) for n, v in per.items()},
            "aggregate_ms": round(sum(per.values()), 3), "cores": 1, "kind": "port",
            "sample": f"oracle backbone_hidden (numpy, fp32) on 1 thread of '{cpu_model()}', "
                      f"median of {samples} per length"}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(min_seconds=10.0, all_cores_seconds=5.0):
    """The C oracle (single thread, fp32 as the reference CPU path) on a quarter
    of each kernel's rows; GB/s over the same algorithmic bytes (bf16 kernels
    counted at their bf16 sizes, which favours the CPU).  `all_cores` repeats
    the mix with the oracle's row loops on every host core the process may use
    (OpenMP; SwiGLU split into the reference's interleaved 256-element blocks),
    an upper bound for a multi-threaded CPU path."""
    import numpy as np
    from oracle import qdc_oracle as O

    rng = np.random.default_rng(0)

    def rnd(*shape, scale=1.0):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))

    jobs = []
    for name, rows, width, es in (("rmsnorm_f32", 2048, 1024, 4), ("rmsnorm_bf16", 2048, 1024, 2),
                                  ("headnorm_f32", 20480, 256, 4), ("headnorm_bf16", 20480, 256, 2)):
        x, w = rnd(rows, width), rnd(width, scale=0.02)
        jobs.append((name, 2 * rows * width * es + width * es, lambda x=x, w=w: O.rms(x, w, 1e-6)))
    T, H, KV, hd, rd = 2048, 8, 2, 256, 64
    q, k, qn = rnd(T, H, hd), rnd(T, KV, hd), rnd(hd, scale=0.02)
    cos, sin = O.rope_tables(2048, rd, 1e7)
    jobs.append(("qk_norm_rope_bf16", 2 * T * (H + KV) * hd * 2 + 2 * hd * 2 + 2 * 2048 * 32 * 4,
                 lambda: (O.qk_norm_rope(q, qn, cos, sin, rd, 1e-6),
                          O.qk_norm_rope(k, qn, cos, sin, rd, 1e-6))))
    table = rng.integers(0, 1 << 16, size=(248320, 1024), dtype=np.uint16)
    ids = rng.integers(0, 248320, size=4096)
    jobs.append(("gather_bf16", 2 * 4096 * 1024 * 2 + 4096 * 4, lambda: O.gather(table, ids)))
    gt, ut = rnd(4096, 3584), rnd(4096, 3584)
    jobs.append(("swiglu_bf16", 3 * 4096 * 3584 * 2, lambda: O.swiglu(gt, ut)))
    xg, zg, wg = rnd(4096, 16, 128), rnd(4096, 16, 128), rnd(128)
    jobs.append(("gated_rms_bf16", 3 * 4096 * 16 * 128 * 2 + 256, lambda: O.gated_rms(xg, zg, wg, 1e-6)))
    xr, mr, wr = rnd(4096, 1024), rnd(4096, 1024), rnd(1024, scale=0.02)
    jobs.append(("residual_rms_bf16", 4 * 4096 * 1024 * 2 + 2048,
                 lambda: O.residual_rms(xr, mr, wr, 1e-6)))
    def timed(seconds):
        per, total_bytes, total_s, reps = {}, 0, 0.0, 0
        while total_s < seconds or reps == 0:
            for name, nbytes, fn in jobs:
                t0 = time.perf_counter()
                fn()
                dt = time.perf_counter() - t0
                b, s = per.get(name, (0, 0.0))
                per[name] = (b + nbytes, s + dt)
                total_bytes += nbytes
                total_s += dt
            reps += 1
        return total_bytes / total_s / 1e9, reps, total_s, {
            k: round(b / s / 1e9, 3) for k, (b, s) in per.items()}

    gbs, reps, secs, per = timed(min_seconds)
    cores = len(os.sched_getaffinity(0))
    previous = O.set_threads(cores)
    try:
        gbs_all, reps_all, secs_all, per_all = timed(all_cores_seconds)
    finally:
        O.set_threads(previous)
    return {
        "value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": (f"C oracle, 1 thread, fp32 arithmetic, on 1/4 of each kernel's rows "
                   f"(same kernel mix), {reps} passes in {secs:.1f} s on '{cpu_model()}' "
                   f"({os.cpu_count()} logical CPUs visible)"),
        "per_kernel_gbs": per,
        "all_cores": {"value": round(gbs_all, 3), "unit": "GB/s", "cores": cores,
                      "sample": f"same mix, OpenMP over rows, {reps_all} passes in {secs_all:.1f} s",
                      "per_kernel_gbs": per_all},
    }


def _pmc():
    try:
        with open(PMC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def load_traffic(name):
    """HBM bytes per launch of a kernel counted by rocprofv3 (FETCH_SIZE +
    WRITE_SIZE, calibrated) in the profiling run recorded in PMC_FILE; not
    counted by this run."""
    entry = _pmc().get("kernels", {}).get(name)
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def traffic_source():
    """Where the traffic figures of this line come from."""
    data = _pmc()
    if not data:
        return None
    return {"file": os.path.relpath(PMC_FILE, ROOT), "summary": data.get("source"),
            "commit": data.get("commit"), "commands": data.get("commands"),
            "note": "counted by rocprofv3 --pmc in that profiling run of bench.py, not in this run"}


# ------------------------------------------------- profile summaries ------
def _dispatches(path, counter=None):
    """rocprofv3 CSV rows in dispatch order: (signature, duration us, value)."""
    import csv
    out = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if counter is not None and r.get("Counter_Name") != counter:
                continue
            sig = (r["Kernel_Name"], int(r.get("Grid_Size") or r.get("Grid_Size_X")),
                   int(r.get("Workgroup_Size") or r.get("Workgroup_Size_X")))
            dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            val = float(r["Counter_Value"]) if counter is not None else None
            out.append((int(r["Dispatch_Id"]), sig, dur, val))
    out.sort(key=lambda d: d[0])
    return [d[1:] for d in out]


def _runs(disp, steps):
    """Consecutive dispatches of one signature, cut into runs of `steps` where
    a run is a whole multiple of it (graph replays of adjacent kernels that
    share a signature)."""
    runs = []
    for d in disp:
        if runs and runs[-1][0][0] == d[0]:
            runs[-1].append(d)
        else:
            runs.append([d])
    out = []
    for r in runs:
        if len(r) > steps and len(r) % steps == 0:
            out += [r[i:i + steps] for i in range(0, len(r), steps)]
        else:
            out.append(r)
    return out


def _find_passes(runs, names, steps, start=0):
    """The untimed and timed replay passes of `names` (in order): the first
    place from `start` where 2*len(names) runs of `steps` dispatches follow
    one another with the second half repeating the first half's signatures.
    Returns ({name: [untimed run, timed run]}, index after the passes)."""
    n = len(names)
    for i in range(start, len(runs) - 2 * n + 1):
        block = runs[i:i + 2 * n]
        if all(len(r) == steps for r in block) and \
                all(block[j][0][0] == block[n + j][0][0] for j in range(n)):
            return {name: [block[j], block[n + j]] for j, name in enumerate(names)}, i + 2 * n
    raise RuntimeError(f"no replay passes of {n} kernels x {steps} launches found")


def summarize_profiles(out_dir, commit):
    """Write profiles/fused_kernels_trace_pmc.md, profiles/pmc_traffic.json,
    profiles/launch_ceilings.md and profiles/kernel_stats_bench.txt from the
    outputs of the three rocprofv3 runs named in PROFILE_COMMANDS under
    `out_dir` (each bench run's stdout beside its rocprofv3 directory, its
    stderr holding the timed order of the kernels)."""
    import csv
    import statistics

    def bench_line(name):
        with open(os.path.join(out_dir, name)) as f:
            return json.loads([ln for ln in f if ln.startswith("{")][-1])

    def order(name):
        with open(os.path.join(out_dir, name)) as f:
            return [ln.split(": ", 1)[1].strip().split(",") for ln in f
                    if ln.startswith("timed order: ")][-1]

    line = bench_line("prof_k_bench.json")
    names = order("prof_k_bench.err")
    fwd = line["forward_shapes"]
    groups = {"hot": list(line["kernels"]), "fwd": list(fwd["kernels"]),
              "alone": list(fwd.get("standalone", {}).get("kernels", {})),
              "split": list(fwd.get("split_gemm_inputs", {}).get("kernels", {}))}
    entry = {**line["kernels"], **line.get("widened", {}), **fwd["kernels"],
             **fwd.get("standalone", {}).get("kernels", {}),
             **fwd.get("split_gemm_inputs", {}).get("kernels", {})}
    steps = line["steps"]
    # the ceilings and floors in the order bench.py times them
    ceil_names = []
    for k in groups["hot"] + [k for g in ("fwd", "alone", "split") for k in groups[g]
                              if k not in groups["hot"]]:
        ceil_names += [f"copy{cpt}x{blk}_{k}" for cpt, blk in COPY_SHAPES]
        if "ceiling_us" in entry[k]:
            ceil_names.append("rows_" + k)
        if "pair_copy_us" in entry[k]:
            ceil_names += [f"pair{cpt}x{blk}_{k}" for cpt, blk in COPY_SHAPES]
    floor_names = ["empty_" + k for k in groups["hot"] if "empty_us" in entry[k]]

    runs = _runs(_dispatches(os.path.join(out_dir, "prof_k", "trace_kernel_trace.csv")), steps)
    kp, nxt = _find_passes(runs, names, steps)
    cp, nxt = _find_passes(runs, ceil_names, steps, nxt)
    fp, _ = _find_passes(runs, floor_names, steps, nxt)
    timed = {**{k: v[1] for k, v in kp.items()}, **{k: v[1] for k, v in cp.items()},
             **{k: v[1] for k, v in fp.items()}}

    # HBM traffic: FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of the two
    # replay passes of the PMC runs, scaled by the calibration copies
    traffic = {}
    scale = {}
    for counter, sub, stem in (("FETCH_SIZE", "pmc_fetch", "fetch"),
                               ("WRITE_SIZE", "pmc_write", "write")):
        disp = _dispatches(os.path.join(out_dir, sub, f"{stem}_counter_collection.csv"), counter)
        calib = [d for d in disp[:40] if "copyBuffer" in d[0][0]]
        counted = sum(d[2] for d in calib) * 1024
        scale[counter] = 4 * CALIB_BYTES / counted if counted else 1.0
        pl = bench_line(f"{sub}_bench.json")
        pruns = _runs(disp, pl["steps"])
        pp, _ = _find_passes(pruns, order(f"{sub}.err"), pl["steps"])
        for k, (a, b) in pp.items():
            traffic.setdefault(k, {})[counter] = statistics.median(
                [d[2] for d in a + b]) * 1024 * scale[counter]

    pmc = {"source": "profiles/fused_kernels_trace_pmc.md", "commit": commit,
           "commands": [c.replace("$R/", "") for c in PROFILE_COMMANDS],
           "scale_fetch": scale["FETCH_SIZE"], "scale_write": scale["WRITE_SIZE"],
           "kernels": {}}
    rows = []
    for k in names:
        e = entry[k]
        durs = [d[1] for d in timed[k]]
        avg, mn = sum(durs) / len(durs), min(durs)
        t = traffic.get(k, {})
        rd, wr = t.get("FETCH_SIZE"), t.get("WRITE_SIZE")
        if rd is not None and wr is not None:
            pmc["kernels"][k] = {"hbm_bytes_per_launch": int(rd + wr), "read_bytes": int(rd),
                                 "write_bytes": int(wr), "avg_us_trace": round(avg, 3)}
        gbs = e["bytes"] / avg / 1e3
        rows.append(f"| {k} | {e.get('launches_per_forward', '')} | {avg:.2f} | {mn:.2f} | "
                    f"{e['us']:.2f} | {e['bytes'] / 1e6:.2f} | "
                    + (f"{rd / 1e6:.2f} | {wr / 1e6:.2f} | {(rd + wr) / e['bytes']:.3f} | "
                       if rd is not None and wr is not None else " |  |  | ")
                    + f"{gbs:.0f} | {100 * gbs / PEAK_GBS:.1f} |")
    with open(os.path.join(ROOT, "profiles", "pmc_traffic.json"), "w") as f:
        json.dump(pmc, f, indent=1)
        f.write("\n")
    cmds = "\n".join(PROFILE_COMMANDS)
    with open(os.path.join(ROOT, "profiles", "fused_kernels_trace_pmc.md"), "w") as f:
        f.write(f"""# Fused row kernels and widened kernels: rocprofv3 kernel trace and HBM traffic (bench.py shapes)

Workload: `bench.py` kernel benchmark (each kernel at its benchmark shape, {steps} steps per kernel
captured in a HIP graph, rotating buffer sets > 640 MB per kernel). The rows follow the bench's
timed order: the fused row kernels at their per-kernel benchmark shapes, the widened kernels
(attention softmax and gate merge, DeltaNet prologue and recurrence), then the `fwd_*` rows, the
fused row kernels exactly as one forward of the 0.8B-like backbone launches them (8 x 2048 tokens;
"per fwd" = launches per forward), the two launches `fwd_gather_rms_bf16` fuses, at the same shapes
(not launched by the forward), and the split-output kernels of the split-GEMM-input forward.

Commands (run from `/tmp` with `TMPDIR=/tmp`, `$R` = repository root), commit {commit}; each
bench run's stdout and stderr saved beside its rocprofv3 directory, then
`python bench.py --summarize-profiles $R/gpurun_out --commit {commit}` wrote this file,
`pmc_traffic.json`, `launch_ceilings.md` and `kernel_stats_bench.txt`:

```
{cmds}
```

Counter calibration: `--calibrate` runs four 512 MiB device copies (`__amd_rocclr_copyBuffer`);
FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are scaled so that those copies read and write
their bytes: fetch x {scale['FETCH_SIZE']:.4f}, write x {scale['WRITE_SIZE']:.4f}. Per-kernel counter values
are the median over the kernel's dispatches in the two graph replays of its PMC run; trace
durations are the {steps} launches of the timed replay; "bench us" is the HIP-event average of the
traced bench run (it includes the graph's gap between nodes).

| kernel (bench name) | per fwd | avg us (trace) | min us | bench us | algorithmic MB | HBM read MB | HBM write MB | traffic / algorithmic | GB/s (algo / avg) | % of 8 TB/s |
|---|---|---|---|---|---|---|---|---|---|---|
""" + "\n".join(rows) + "\n")

    # single-launch ceilings, from the same trace
    def avg(name):
        r = timed.get(name)
        return None if r is None else sum(d[1] for d in r) / len(r)

    lrows = []
    for k in groups["hot"] + [k for g in ("fwd", "alone", "split") for k in groups[g]
                              if k not in groups["hot"]]:
        e = entry[k]
        # the copy shape that was fastest by HIP events in the same run
        cn = f"copy{e.get('copy_shape', '1x256')}_{k}"
        ku, cu, ru, eu = avg(k), avg(cn), avg("rows_" + k), avg("empty_" + k)
        pu = avg(f"pair{e['pair_copy_shape']}_{k}") if "pair_copy_shape" in e else None
        wg = timed[k][0][0][1] // timed[k][0][0][2]
        cwg = timed[cn][0][0][1] // timed[cn][0][0][2]
        kb, cb = e["bytes"], (e["bytes"] // 2) // 16 * 16 * 2
        lrows.append(f"| {k} | {kb / 1e6:.1f} | {wg} | {ku:.2f} | {e.get('copy_shape', '1x256')} | "
                     f"{cu:.2f} | {cwg} | "
                     f"{'' if ru is None else f'{ru:.2f}'} | {'' if eu is None else f'{eu:.2f}'} | "
                     f"{100 * kb / ku / 1e3 / PEAK_GBS:.1f} | {100 * cb / cu / 1e3 / PEAK_GBS:.1f} | "
                     f"{100 * (kb / ku) / (cb / cu):.1f} | "
                     f"{e.get('pct_of_copy_paired', '')} | {e.get('pct_of_ceiling_paired', '')} | "
                     + ("|  |  |" if pu is None else
                        f"{e['pair_copy_shape']} {pu:.2f} | {100 * pu / ku:.1f} | "
                        f"{e.get('pct_of_pair_copy_paired', '')} |"))
    with open(os.path.join(ROOT, "profiles", "launch_ceilings.md"), "w") as f:
        f.write(f"""# Single-launch ceilings: each fused kernel beside a copy of its bytes and an empty launch of its grid

Same trace as `fused_kernels_trace_pmc.md` (commit {commit}; command there). Every row is the
average over the {steps} launches of a timed graph replay, from the trace's own timestamps. For each
kernel the same run times, in the same way:

- a copy of the kernel's algorithmic bytes, half read and half written, nontemporal 16-byte
  chunks, in each launch shape of `COPY_SHAPES` (chunks per thread x threads per workgroup:
  `qdc_copy` and `qdc_copy_grid`); the table shows the shape that was fastest by HIP events in
  the same run (`copy shape`), and each kernel is held against it;
- for the gathers, `qdc_copy_rows`: the same table, the same number of rows read at uniformly
  random places and written contiguously 1, 2 or 3 times (the gather's access pattern and bytes);
- for the per-kernel configurations of the RMSNorm family and the q/k kernel, `qdc_empty` over
  the kernel's own grid (workgroups of 256 threads that do nothing): the fixed cost of the launch;
- for the residual norms whose two inputs and two outputs have the same sizes (the all-bf16
  per-kernel configuration and the forward's all-fp32 final norm), `qdc_copy_pair`: their two
  streams, each read and written, copied in one launch in each of the same launch shapes (the
  fastest shown; "two-stream copy").

The "paired" columns are the bench line's paired ratios of the same run: the kernel's graph
replayed right before its ceilings' graphs, median of three rounds (HIP events; ceiling time /
kernel time).

| kernel | MB | workgroups | kernel us | copy shape | copy us | copy workgroups | random-row copy us | empty us (same grid) | kernel % of 8 TB/s | copy % of 8 TB/s | kernel % of copy | paired % of copy | paired % of random-row copy | two-stream copy shape, us | kernel % of two-stream copy | paired % of two-stream copy |
|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|
""" + "\n".join(lrows) + "\n")

    # rocprofv3 --stats of the library's kernels
    with open(os.path.join(out_dir, "prof_k", "trace_kernel_stats.csv"), newline="") as f:
        st = [r for r in csv.DictReader(f) if "qdc::" in r["Name"]]
    with open(os.path.join(ROOT, "profiles", "kernel_stats_bench.txt"), "w") as f:
        f.write(f"""rocprofv3 --kernel-trace --stats summary (kernel_stats.csv) of the bench kernel run, library kernels only
Command (from /tmp with TMPDIR=/tmp, $R = repository root), commit {commit}:
  {PROFILE_COMMANDS[0]}
Averages cover every call of a symbol (warmup, eager checks and graph replays; a symbol shared by
several shapes averages them all). The per-shape timed-replay averages are in
fused_kernels_trace_pmc.md; copy_chunks, copy_rows<R> and empty_grid are the benchmark's ceilings
(launch_ceilings.md); "% time" is of all kernels in the run.

calls    avg us    min us    max us % time  kernel
""")
        for r in st:
            f.write(f"{int(r['Calls']):5d} {float(r['AverageNs']) / 1e3:9.2f} "
                    f"{float(r['MinNs']) / 1e3:9.2f} {float(r['MaxNs']) / 1e3:9.2f} "
                    f"{float(r['Percentage']):6.2f}  {r['Name'][:150]}\n")


def _kernel_label(name, gemm="hipBLASLt GEMM"):
    """A table label for a traced kernel: the library's kernels by function
    name, Tensile GEMMs by their output type, the runtime's copy kernels."""
    import re
    m = re.search(r"qdc::\(anonymous namespace\)::(\w+)", name)
    if m:
        return f"`{m.group(1)}`"
    if name.startswith("Cijk_"):
        code = name.split("_")[3]
        out = {"B": "bf16", "S": "fp32", "H": "fp16"}.get(code[1:2], code) if len(code) == 3 else None
        return f"{gemm} {out} out" if out else f"{gemm}s (Tensile kernels of the kept library)"
    if "copyBuffer" in name:
        return "runtime copy"
    m = re.search(r"at::native::(?:\(anonymous namespace\)::)?(\w+)", name)
    return f"torch `{m.group(1)}`" if m else name[:40]


def _trace_rows(path):
    import csv
    with open(path, newline="") as f:
        rows = list(csv.DictReader(f))
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    grid = "Grid_Size_X" if "Grid_Size_X" in rows[0] else "Grid_Size"
    return [(r["Kernel_Name"], int(r[grid]), int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
            for r in rows]


def _kernel_table(segments, per, gemm="hipBLASLt GEMM", unit_ms=True):
    """Markdown rows: label, launches and time per forward (summed over the
    segments, divided by `per`; ms with the share of kernel time, or µs), and
    the total kernel time per forward in ms."""
    from collections import OrderedDict
    acc = OrderedDict()
    for seg in segments:
        for name, _, t0, t1 in seg:
            label = _kernel_label(name, gemm)
            n, t = acc.get(label, (0, 0))
            acc[label] = (n + 1, t + (t1 - t0))
    total = sum(t for _, t in acc.values())
    out = []
    for label, (n, t) in sorted(acc.items(), key=lambda kv: -kv[1][1]):
        if unit_ms:
            out.append(f"| {label} | {n // per} | {t / per / 1e6:.3f} | {100 * t / total:.1f}% |")
        else:
            out.append(f"| {label} | {n // per} | {t / per / 1e3:.1f} |")
    return out, total / per / 1e6


def summarize_forward(out_dir, commit):
    """Write profiles/backbone_forward_kernels.md, other_modes_forward.md
    and decision_latency_kernels.md from the end-to-end and decision traces
    under `out_dir` (FORWARD_COMMANDS) and the untraced bench line of the same
    commit in `out_dir`/bench.log."""
    rows = _trace_rows(os.path.join(out_dir, "prof_e2e", "e2e_kernel_trace.csv"))
    starts = [i for i, r in enumerate(rows) if "gather_rms" in r[0]]
    untraced = json.loads([ln for ln in open(os.path.join(out_dir, "bench.log"))
                           if ln.startswith("{")][-1])
    b = untraced["backbone"]
    # e2e_benchmark's order: the headline "mlp" mode, "all", all-bf16 storage, fp32
    modes = [("mlp", starts[0:5], b["ms_per_forward"]),
             ("all", starts[4:9], b["split_gemm_inputs_all"]["ms_per_forward"]),
             ("all-bf16 storage", starts[8:13], b["bf16_storage"]["ms_per_forward"])]
    cmd = FORWARD_COMMANDS[0]
    tables = {}
    for mode, st, ms in modes:
        # the first and second timed forwards (after one warm-up forward)
        segs = [rows[st[1]:st[2]], rows[st[2]:st[3]]]
        t, busy = _kernel_table(segs, 2)
        span = sum((s[-1][3] - s[0][2]) for s in segs) / 2 / 1e6
        tables[mode] = (t, busy, span, ms)
    hdr = "| kernel | launches / forward | ms / forward | share of kernel time |\n|---|---|---|---|\n"
    t, busy, span, ms = tables["mlp"]
    with open(os.path.join(ROOT, "profiles", "backbone_forward_kernels.md"), "w") as f:
        f.write(f"""# backbone_hidden forward: per-kernel time (random-init Qwen3.5-0.8B-like, bf16 weights, split MLP inputs, 8 x 2048 tokens)

Command (run from `/tmp` with `TMPDIR=/tmp`, `$R` = repository root), commit {commit}; then
`python bench.py --summarize-forward $R/gpurun_out --commit {commit}` (with the untraced bench line
of the same commit in `gpurun_out/bench.log`) wrote this file, `other_modes_forward.md` and
`decision_latency_kernels.md`:

```
{cmd}
```

The headline mode: bf16 weights, the MLP's two GEMM inputs (the post-attention norm's output and
SwiGLU's) written as two bf16 terms, the MLP gate/up GEMM writing fp32 for SwiGLU
(`split_gemm_inputs="mlp"`, within 1e-2 of the fp32 oracle end to end). The trace covers the whole
run; the table sums the kernels of the first and second timed forwards of `bench.py`'s end-to-end
benchmark (each forward starts with its one gather launch, the gather fused with the first input
norm) and divides by two. 24 layers: 18 DeltaNet + 6 full attention, hidden 1024, 16384 tokens
per forward. GEMMs are labelled by the output type of their Tensile kernel. The same run
continues with the other modes, summarised in `other_modes_forward.md`.

forward span {span:.3f} ms, kernels busy {busy:.3f} ms under the tracer; untraced, the bench line of
the same commit gives {ms:.3f} ms per forward

""" + hdr + "\n".join(t) + """

`rms_rows_fast` covers the 24 post-attention residual norms (fp32 residual stream, split output),
the 23 residual + next-input norms (bf16 output), the 18 DeltaNet gated norms and the residual +
final norm (fp32). `swiglu_fast` reads the fp32 gate/up GEMM output and writes the split form
(704 MB per launch).
""")
    with open(os.path.join(ROOT, "profiles", "other_modes_forward.md"), "w") as f:
        f.write(f"""# backbone_hidden forward in the other bf16-weight modes: per-kernel time (random-init Qwen3.5-0.8B-like, 8 x 2048 tokens)

Command (run from `/tmp` with `TMPDIR=/tmp`, `$R` = repository root), commit {commit} -- the same
run as `backbone_forward_kernels.md`:

```
{cmd}
```

`bench.py`'s end-to-end benchmark runs the same weights and tokens with `split_gemm_inputs="mlp"`
(the headline, `backbone_forward_kernels.md`), then `"all"` (every GEMM input written as two bf16
terms; projection weights with their input rows repeated, twice the inner dimension), then
all-bf16 storage (no split; misses the 1e-2 end-to-end bar at 24 layers), one warm-up and three
timed forwards each. Each table sums the kernels of the first and second timed forwards of its
mode and divides by two. In both split modes the MLP gate/up GEMM writes fp32 and SwiGLU reads
it, so `swiglu_fast` moves 704 MB per launch instead of 352 MB. The split-output kernels alone,
at these shapes beside their copy ceilings and with counted HBM traffic, are in
`fused_kernels_trace_pmc.md` and `launch_ceilings.md` (`fwd_*_split`).
""")
        for mode in ("all", "all-bf16 storage", "mlp"):
            t, busy, span, ms = tables[mode]
            f.write(f"""
## {mode}: forward span {span:.3f} ms, kernels busy {busy:.3f} ms (untraced: {ms:.3f} ms)

""" + hdr + "\n".join(t) + "\n")

    # decision latency: the last graph replay of each length
    rows = _trace_rows(os.path.join(out_dir, "prof_dec", "dec_kernel_trace.csv"))
    starts = [i for i, r in enumerate(rows) if "gather_rms" in r[0]]
    segs = {}
    for j, i in enumerate(starts):
        a = i - 1 if i > 0 and "copyBuffer" in rows[i - 1][0] else i   # the ids copied in
        end = starts[j + 1] - 1 if j + 1 < len(starts) else len(rows)
        if end > a and "copyBuffer" not in rows[end - 1][0] and j + 1 < len(starts):
            end += 1  # the next start has no copy-in of its own
        segs[rows[i][1]] = rows[a:end]  # keyed by the gather's grid: one per length
    d = untraced["decision"]
    lengths = sorted(d["graph_ms"], key=int)
    with open(os.path.join(ROOT, "profiles", "decision_latency_kernels.md"), "w") as f:
        f.write(f"""# Single-sequence last-token latency: kernels of one graph replay per length

Workload: `bench.py --decision-only`, the reference's inference benchmark protocol
(`benchmark/inference.jl`) on its synthetic model's shapes (`benchmark/synthetic.jl`: 4 layers,
3 DeltaNet + 1 full attention, hidden 256, intermediate 512, fp32): `backbone_last_hidden` of one
sequence of 64, 128, 256 and 512 tokens served from recorded HIP graphs (`qdc_amd.graphs`).

Command (run from `/tmp` with `TMPDIR=/tmp`, `$R` = repository root), commit {commit}; summary as in
`backbone_forward_kernels.md`:

```
{FORWARD_COMMANDS[1]}
```

Each table is the last graph replay of its length. "Kernel µs" sums the kernel durations in the
trace; the untraced median per call of the same commit (`bench.py`'s decision section: the
host-to-device copy of the ids, the graph launch, the kernels, the device-to-host copy of the
result and the stream synchronisation) is in each heading. GEMM library kept per length:
{d.get("graph_gemm_library")} ("cublas" is rocBLAS, "cublaslt" hipBLASLt, in torch's names).
""")
        for n, grid in zip(lengths, sorted(segs)):
            seg = segs[grid]
            t, busy = _kernel_table([seg], 1, gemm="GEMM", unit_ms=False)
            t = [ln.replace("| runtime copy |", "| runtime copy (ids in, result out) |") for ln in t]
            f.write(f"""
## {n} tokens: {len(seg)} kernels, {busy * 1e3:.1f} kernel µs (untraced: {d["graph_ms"][n] * 1e3:.0f} µs per call)

| kernel | launches | µs |
|---|---|---|
""" + "\n".join(t) + "\n")


FORWARD_COMMANDS = [
    "rocprofv3 --kernel-trace --stats --output-format csv -d $R/gpurun_out/prof_e2e -o e2e "
    "-- python -u $R/bench.py --no-cpu --only swiglu_bf16 --steps 2 --warmup 1",
    "rocprofv3 --kernel-trace --stats --output-format csv -d $R/gpurun_out/prof_dec -o dec "
    "-- python -u $R/bench.py --decision-only --no-cpu",
]


PROFILE_COMMANDS = [
    "rocprofv3 --kernel-trace --stats --output-format csv -d $R/gpurun_out/prof_k -o trace "
    "-- python -u $R/bench.py --no-cpu --no-e2e",
    "rocprofv3 --pmc FETCH_SIZE --output-format csv -d $R/gpurun_out/pmc_fetch -o fetch "
    "-- python -u $R/bench.py --no-cpu --no-e2e --steps 2 --warmup 1 --calibrate",
    "rocprofv3 --pmc WRITE_SIZE --output-format csv -d $R/gpurun_out/pmc_write -o write "
    "-- python -u $R/bench.py --no-cpu --no-e2e --steps 2 --warmup 1 --calibrate",
]


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma-separated kernel names (profiling runs)")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end backbone run")
    ap.add_argument("--no-decision", action="store_true",
                    help="skip the single-sequence last-token latency run (--no-e2e skips it too)")
    ap.add_argument("--decision-only", action="store_true",
                    help="run only the single-sequence last-token latency run (profiling runs)")
    ap.add_argument("--calibrate", action="store_true",
                    help="first run 4 plain 512 MiB device copies (scales the PMC byte counters)")
    ap.add_argument("--summarize-profiles", metavar="DIR", default="",
                    help="write the profiles/ summaries from rocprofv3 outputs under DIR (no GPU)")
    ap.add_argument("--summarize-forward", metavar="DIR", default="",
                    help="write the forward and decision-latency summaries from traces under DIR")
    ap.add_argument("--commit", default="", help="commit the profiled tree was at (summaries)")
    args = ap.parse_args()
    if args.summarize_profiles:
        summarize_profiles(args.summarize_profiles, args.commit)
        return
    if args.summarize_forward:
        summarize_forward(args.summarize_forward, args.commit)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the row kernels need no exchange; see the sharding notes)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.decision_only:
        line = {"decision": decision_latency(dev)}
        if not args.no_cpu:
            line["decision"]["cpu"] = cpu_decision()
        print(json.dumps(line), flush=True)
        return
    if args.calibrate:
        calibrate(dev)
    kernels = build_kernels(dev) + build_forward_kernels(dev)
    if args.only:
        keep = set(args.only.split(","))
        kernels = [k for k in kernels if k.name in keep]
    for i in range(args.warmup):
        for k in kernels:
            k.run(i)
    # the order of the timed graph replays, for matching a rocprofv3 trace
    print("timed order: " + ",".join(k.name for k in kernels), file=sys.stderr, flush=True)
    capture(kernels, args.steps)
    check_replay(kernels, args.steps)
    for k in kernels:  # one untimed replay
        k.graph.replay()
    time_gpu(kernels, args.steps)
    hot = [k for k in kernels if k.group == "hot"] or kernels
    fwd = [k for k in kernels if k.group == "forward"]
    alone = [k for k in kernels if k.group == "standalone"]
    split = [k for k in kernels if k.group == "split"]
    ceilings = copy_ceilings(dev, hot + [k for k in fwd + alone + split if k not in hot],
                             args.steps, args.warmup)
    floors = empty_floors(hot, args.steps, args.warmup)
    paired = paired_ratios([k for k in kernels if k.name in ceilings], ceilings)
    hot_ms = sum(k.avg_ms for k in hot) * args.steps
    step_bytes = sum(k.algo_bytes for k in hot)
    value = step_bytes * args.steps / (hot_ms / 1e3) / 1e9

    def entry(k):
        e = {"shape": k.shape, "dtype": k.dtype, "bytes": k.algo_bytes,
             "us": round(k.avg_ms * 1e3, 3),
             "gbs": round(k.algo_bytes / (k.avg_ms / 1e3) / 1e9, 1),
             "pct_peak": round(100 * k.algo_bytes / (k.avg_ms / 1e3) / 1e9 / PEAK_GBS, 1)}
        t = load_traffic(k.name)
        if t is not None:  # counted in the profiling run named by traffic_source
            e.update(hbm_bytes_counted=t, traffic_per_algorithmic=round(t / k.algo_bytes, 4))
        c, rows, shapes, pair, pairs = ceilings.get(k.name, (None,) * 5)
        if c is not None:  # the same bytes as one plain streaming copy launch, fastest shape
            copy_gbs = c.algo_bytes / (c.avg_ms / 1e3) / 1e9
            one = shapes["1x256"]
            e.update(copy_us=round(c.avg_ms * 1e3, 3),
                     copy_shape=c.name.split("_", 1)[0][len("copy"):],
                     copy_pct_peak=round(100 * copy_gbs / PEAK_GBS, 1),
                     pct_of_copy=round(100 * e["gbs"] / copy_gbs, 1),
                     copy_us_by_shape={n: round(x.avg_ms * 1e3, 3) for n, x in shapes.items()},
                     pct_of_one_chunk_copy=round(100 * one.avg_ms / k.avg_ms, 1))
        if rows is not None:  # the same access pattern as a plain random-row copy
            e.update(ceiling="random-row copy (qdc_copy_rows), same table, bytes and row count",
                     ceiling_us=round(rows.avg_ms * 1e3, 3),
                     ceiling_pct_peak=round(100 * rows.algo_bytes / (rows.avg_ms / 1e3) / 1e9
                                            / PEAK_GBS, 1),
                     pct_of_ceiling=round(100 * rows.avg_ms / k.avg_ms, 1))
        if pair is not None:  # its two streams as one two-stream copy launch, fastest shape
            e.update(pair_copy="qdc_copy_pair of the kernel's two streams, each read and written "
                               "(bytes " + " + ".join(str(b) for b in k.pair) + ")",
                     pair_copy_us=round(pair.avg_ms * 1e3, 3),
                     pair_copy_shape=pair.name.split("_", 1)[0][len("pair"):],
                     pair_copy_us_by_shape={n: round(x.avg_ms * 1e3, 3) for n, x in pairs.items()},
                     pct_of_pair_copy=round(100 * pair.avg_ms / k.avg_ms, 1))
        pc, prow, ppair = paired.get(k.name, (None, None, None))
        if pc is not None:  # the kernel and its ceilings replayed back to back
            e.update(pct_of_copy_paired=round(100 * pc, 1))
        if prow is not None:
            e.update(pct_of_ceiling_paired=round(100 * prow, 1))
        if ppair is not None:
            e.update(pct_of_pair_copy_paired=round(100 * ppair, 1))
        f = floors.get(k.name)
        if f is not None:  # an empty launch of the same grid
            e.update(workgroups=k.workgroups, empty_us=round(f.avg_ms * 1e3, 3))
        if k.flops:
            tf = k.flops / (k.avg_ms / 1e3) / 1e12
            e.update(bound="mfma", tflops=round(tf, 2), mfma_f32_peak_tflops=MFMA_F32_PEAK_TF,
                     pct_mfma_peak=round(100 * tf / MFMA_F32_PEAK_TF, 1))
        return e

    per = {k.name: entry(k) for k in hot}
    widened = {k.name: entry(k) for k in kernels if k.group == "next"}
    dom = max(hot, key=lambda k: k.avg_ms)
    achieved = dom.algo_bytes / (dom.avg_ms / 1e3) / 1e9
    traffic = load_traffic(dom.name)
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(hot_ms / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        # the arithmetic type; every kernel computes in fp32 whatever it stores
        "dtype": "f32", "storage_dtypes": {k.name: k.dtype for k in hot},
        "data": "synthetic",
        "config": {"workload": "fused row kernels of one Qwen3.5-0.8B-like layer set: "
                               + ", ".join(k.name for k in hot),
                   "storage": "bf16 and fp32 as named per kernel", "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "kernel": dom.name, "achieved": round(achieved, 1),
                     "peak": PEAK_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_GBS, 4),
                     "traffic": traffic, "algorithmic_bytes": dom.algo_bytes,
                     "traffic_source": traffic_source()},
        "kernels": per,
    }
    if widened:
        line["widened"] = widened
    if fwd:
        fb = sum(k.launches * k.algo_bytes for k in fwd)
        fs = sum(k.launches * k.avg_ms for k in fwd) / 1e3
        line["forward_shapes"] = {
            "workload": "the fused row kernels as one forward of the Qwen3.5-0.8B-like backbone "
                        "launches them (8 x 2048 tokens, bf16, fp32 residual stream)",
            "kernels": {k.name: dict(entry(k), launches_per_forward=k.launches) for k in fwd},
            "gbs_forward_weighted": round(fb / fs / 1e9, 1),
            "pct_peak_forward_weighted": round(100 * fb / fs / 1e9 / PEAK_GBS, 1)}
        if alone:
            line["forward_shapes"]["standalone"] = {
                "note": "the gather and the first input norm as two launches at the forward's "
                        "shapes; the forward runs them fused (fwd_gather_rms_bf16)",
                "kernels": {k.name: entry(k) for k in alone}}
    if split:
        sb = sum(k.launches * k.algo_bytes for k in split)
        ss = sum(k.launches * k.avg_ms for k in split) / 1e3
        line.setdefault("forward_shapes", {})["split_gemm_inputs"] = {
            "note": "the kernels that write GEMM inputs, as the forward with bf16 weights and "
                    "split_gemm_inputs='all' launches them: every output element as two bf16 "
                    "terms (4 bytes); SwiGLU reads the fp32 gate/up GEMM output",
            "kernels": {k.name: dict(entry(k), launches_per_forward=k.launches) for k in split},
            "gbs_forward_weighted": round(sb / ss / 1e9, 1),
            "pct_peak_forward_weighted": round(100 * sb / ss / 1e9 / PEAK_GBS, 1)}
    if not args.no_e2e:
        for k in kernels:  # release the kernel benchmark's buffers first
            k.sets, k.graph = None, None
        torch.cuda.empty_cache()
        line["backbone"] = e2e_benchmark(dev)
    if not (args.no_e2e or args.no_decision or args.only):
        line["decision"] = decision_latency(dev)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
        if "backbone" in line:
            line["backbone"]["cpu"] = cpu_backbone()
            line["backbone"]["speedup_vs_cpu"] = round(
                line["backbone"]["tokens_per_s"] / line["backbone"]["cpu"]["tokens_per_s"], 1)
        if "decision" in line:
            line["decision"]["cpu"] = cpu_decision()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

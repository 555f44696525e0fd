"""GPU parity of every fused row kernel against the CPU oracle, through the
C ABI (qdc_amd.ops -> libqdc_hip.so).

Bars: gather bit-exact; everything else normwise relative error (Julia
isapprox semantics) <= 1e-5 in fp32 and <= 1e-2 in bf16, where bf16 runs use
bf16-representable inputs and the oracle computes in fp32 on the same values.
Shapes cover the benchmark configurations at full size, the reference's small
and ragged cases, strided / packed layouts, in-place calls and the general
(unaligned / odd-width) kernels.
"""
import numpy as np
import pytest
import torch

from conftest import normwise
from oracle import qdc_oracle as O

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from qdc_amd import ops  # noqa: F401  (fails loudly if the library is missing)
    yield
    torch.cuda.synchronize()


def host(shape, seed, scale=1.0, dtype=torch.float32):
    """Seeded N(0, scale) fp32 values, made bf16-representable for bf16 runs."""
    x = (np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(scale))
    return O.round_bf16(x) if dtype == torch.bfloat16 else x


def dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV).to(dtype)


def back(t):
    return t.float().cpu().numpy()


def report(name, got, exp, dtype):
    err = normwise(got, exp)
    print(f"{name}: normwise {err:.3e} maxabs {np.abs(got - exp).max() if got.size else 0:.3e}",
          flush=True)
    assert err <= TOL[dtype], (name, err)


DTYPES = [torch.float32, torch.bfloat16]


# ------------------------------------------------------------------ RMSNorm --
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,width", [(8192, 1024), (81920, 256), (17, 7), (1, 1), (3, 1000),
                                        (33, 2560), (5, 4096), (257, 128), (2, 8), (9, 64),
                                        # rows over 2 or 4 wavefronts (fp32 from 2048;
                                        # bf16 from 4096)
                                        (6, 2048), (9, 5120), (4, 8192), (3, 10240), (2, 16384)])
@pytest.mark.parametrize("centered", [True, False])
def test_rmsnorm(dtype, rows, width, centered):
    from qdc_amd import ops
    x = host((rows, width), 1, 1.0, dtype)
    w = host((width,), 2, 0.02, dtype)
    got = back(ops.native_rms(dev(x, dtype), dev(w, dtype), 1e-6, centered=centered))
    report(f"rms {rows}x{width} {dtype} c={centered}", got, O.rms(x, w, 1e-6, centered), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_rmsnorm_strided_misaligned_inplace_empty(dtype):
    from qdc_amd import ops
    x = host((64, 1040), 3, 1.0, dtype)
    w = host((1024,), 4, 0.02, dtype)
    big = dev(x, dtype)
    # rows of 1024 inside rows of 1040 (aligned stride) and shifted by one element
    for off in (0, 1):
        view = big[:, off:off + 1024]
        got = back(ops.native_rms(view, dev(w, dtype), 1e-6))
        report(f"rms strided off={off}", got, O.rms(x[:, off:off + 1024], w, 1e-6), dtype)
    t = dev(x[:, :1024], dtype).contiguous()
    ops.native_rms(t, dev(w, dtype), 1e-6, out=t)
    report("rms in place", back(t), O.rms(x[:, :1024], w, 1e-6), dtype)
    empty = torch.empty((0, 1024), dtype=dtype, device=DEV)
    assert ops.native_rms(empty, dev(w, dtype), 1e-6).shape == (0, 1024)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,width", [(8192, 1024), (16384, 1024), (17, 7), (65, 256), (3, 3000),
                                        (5, 5120)])
def test_residual_rmsnorm(dtype, rows, width):
    from qdc_amd import ops
    x = host((rows, width), 5, 1.0, dtype)
    m = host((rows, width), 6, 1.0, dtype)
    w = host((width,), 7, 0.02, dtype)
    res, out = ops.native_residual_rms(dev(x, dtype), dev(m, dtype), dev(w, dtype), 1e-6)
    # the residual is x + mixed rounded once; the norm uses the unrounded fp32 sum
    exp_res, exp_out = O.residual_rms(x, m, w, 1e-6)
    if dtype == torch.bfloat16:
        exp_res = O.round_bf16(exp_res)
    report(f"residual {rows}x{width}", back(res), exp_res, dtype)
    report(f"residual-norm {rows}x{width}", back(out), exp_out, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("width", [1024, 1000])
def test_residual_rmsnorm_in_place(dtype, width):
    from qdc_amd import ops
    x = host((37, width), 8, 1.0, dtype)
    m = host((37, width), 9, 1.0, dtype)
    w = host((width,), 10, 0.02, dtype)
    exp_res, exp_out = O.residual_rms(x, m, w, 1e-6)
    if dtype == torch.bfloat16:
        exp_res = O.round_bf16(exp_res)
    xt, mt = dev(x, dtype), dev(m, dtype)
    # residual over x, normalised output over mixed (the reference reuses buffers this way)
    ops.native_residual_rms(xt, mt, dev(w, dtype), 1e-6, residual=xt, out=mt)
    report("residual in place", back(xt), exp_res, dtype)
    report("residual-norm in place", back(mt), exp_out, dtype)


# ------------------------------------------------------- q/k norm + RoPE ----
QK_CASES = [
    # tokens, heads, kv, head_dim, rotary, seq_len, theta
    (8192, 8, 2, 256, 64, 2048, 1e7),   # Qwen3.5-0.8B-like, 4 sequences of 2048
    (128, 4, 1, 64, 16, 128, 1e7),      # 2-layer plumbing backbone
    (65, 2, 1, 4, 4, 65, 1e4),          # reference fixture shape (general kernel)
    (40, 3, 1, 64, 0, 40, 1e7),         # no rotation
    (33, 2, 2, 128, 128, 11, 1e4),      # full rotary, sequences of 11
    (19, 2, 1, 96, 24, 19, 1e6),        # 12-wide halves: general kernel
    (9, 3, 1, 16, 16, 5, 1e4),          # two bf16 chunks per row: one lane per row
    (7, 2, 1, 24, 16, 7, 1e4),          # odd chunk count: general kernel
    (21, 4, 2, 256, 48, 7, 1e6),        # rotary chunks not a power of two: pair-dealt lanes
    (37, 8, 2, 256, 64, 16, 1e7),       # 0.8B heads, sequences of 16 with a partial last one
    (12, 2, 1, 4, 2, 12, 1e4),          # rotary 2 of head_dim 4 (the reference's partial case)
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", QK_CASES)
def test_qk_norm_rope(dtype, case):
    from qdc_amd import ops
    T, H, KV, hd, rd, seq, theta = case
    qgate = host((T, H, 2 * hd), 11, 1.0, dtype)   # interleaved q||gate projection
    k = host((T, KV, hd), 12, 1.0, dtype)
    qn = host((hd,), 13, 0.02, dtype)
    kn = host((hd,), 14, 0.02, dtype)
    tables = ops.rope_tables(seq, rd, theta, DEV)
    qg = dev(qgate, dtype)
    q_view = qg[:, :, :hd]
    qo, ko = ops.prepare_heads(q_view, dev(k, dtype), dev(qn, dtype), dev(kn, dtype), tables, rd,
                               1e-6, seq_len=seq)
    cos, sin = O.rope_tables(seq, rd, theta)
    report(f"q {case}", back(qo), O.qk_norm_rope(qgate[:, :, :hd], qn, cos, sin, rd, 1e-6, seq), dtype)
    report(f"k {case}", back(ko), O.qk_norm_rope(k, kn, cos, sin, rd, 1e-6, seq), dtype)
    # the gate half of the projection is untouched
    assert torch.equal(qg[:, :, hd:], dev(qgate, dtype)[:, :, hd:])


@pytest.mark.parametrize("dtype", DTYPES)
def test_qk_norm_rope_offset_inplace_one_side(dtype):
    from qdc_amd import ops
    T, H, hd, rd = 48, 4, 256, 64
    q = host((T, H, hd), 15, 2.0, dtype)
    qn = host((hd,), 16, 0.02, dtype)
    tables = ops.rope_tables(200, rd, 1e7, DEV)
    cos, sin = O.rope_tables(200, rd, 1e7)
    qt = dev(q, dtype)
    # Q only, positions 100.., in place
    ops.prepare_heads(qt, None, dev(qn, dtype), None, tables, rd, 1e-6, seq_len=T, pos_offset=100,
                      q_out=qt)
    report("q offset in place", back(qt), O.qk_norm_rope(q, qn, cos, sin, rd, 1e-6, T, 100), dtype)
    with pytest.raises(ValueError):
        ops.prepare_heads(qt, None, dev(qn, dtype), None, tables, rd, 1e-6, seq_len=T,
                          pos_offset=160)


# ----------------------------------------------------------- gated norm -----
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("tokens,heads,width", [(16384, 16, 128), (128, 4, 128), (17, 4, 128),
                                                (1, 4, 128), (129, 4, 128), (9, 3, 100),
                                                (5, 2, 8)])
def test_gated_rmsnorm(dtype, tokens, heads, width):
    from qdc_amd import ops
    x = host((tokens, heads, width), 17, 1.0, dtype)
    z = host((tokens, heads, width), 18, 1.0, dtype)
    w = host((width,), 19, 0.02, dtype)
    got = back(ops.native_gated_rms(dev(x, dtype), dev(z, dtype), dev(w, dtype), 1e-6))
    report(f"gated {tokens}x{heads}x{width}", got, O.gated_rms(x, z, w, 1e-6), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_gated_rmsnorm_z_in_packed_projection(dtype):
    """z read straight from the packed [qkv | z | a | b] projection."""
    from qdc_amd import ops
    T, H, W, qkv = 257, 16, 128, 6144
    proj = host((T, qkv + H * W + 2 * H), 20, 1.0, dtype)
    x = host((T, H, W), 21, 1.0, dtype)
    w = host((W,), 22, 1.0, dtype)
    pt = dev(proj, dtype)
    z_view = pt[:, qkv:qkv + H * W].view(T, H, W)
    xt = dev(x, dtype)
    ops.native_gated_rms(xt, z_view, dev(w, dtype), 1e-6, out=xt)   # in place over x
    exp = O.gated_rms(x, proj[:, qkv:qkv + H * W].reshape(T, H, W), w, 1e-6)
    report("gated packed z, in place", back(xt), exp, dtype)


# ---------------------------------------------------------------- SwiGLU ----
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("tokens,width", [(16384, 3584), (128, 768), (17, 16), (3, 1001), (1, 8)])
def test_swiglu(dtype, tokens, width):
    from qdc_amd import ops
    g = host((tokens, width), 23, 1.0, dtype)
    u = host((tokens, width), 24, 1.0, dtype)
    got = back(ops.native_mlp_gate(dev(g, dtype), dev(u, dtype)))
    report(f"swiglu {tokens}x{width}", got, O.swiglu(g, u), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_swiglu_packed_inplace_special(dtype):
    from qdc_amd import ops
    T, I = 300, 3584
    packed = host((T, 2 * I), 25, 3.0, dtype)
    special = np.array([0.0, -0.0, -100.0, 100.0, 1e-30, -1e-30, 80.0, -20.0, 88.0, -88.0, 1e-12,
                        3.0, np.inf, -np.inf], np.float32)
    packed[0, :special.size] = special
    if dtype == torch.bfloat16:
        packed = O.round_bf16(packed)
    pt = dev(packed, dtype)
    got = back(ops.native_mlp_gate(pt[:, :I], pt[:, I:]))
    exp = O.swiglu(packed[:, :I], packed[:, I:])
    finite = np.isfinite(exp)
    report("swiglu packed", np.where(finite, got, 0), np.where(finite, exp, 0), dtype)
    assert np.array_equal(np.isnan(got), np.isnan(exp)) and np.array_equal(
        got[np.isinf(exp)], exp[np.isinf(exp)])
    g = dev(packed[:, :I], dtype).contiguous()
    ops.native_mlp_gate(g, dev(packed[:, I:], dtype).contiguous(), out=g)  # native_mlp_gate!
    assert np.array_equal(back(g), got, equal_nan=True)


# ---------------------------------------------------------------- gather ----
@pytest.mark.parametrize("table_dtype,out_dtype", [(torch.bfloat16, torch.bfloat16),
                                                   (torch.bfloat16, torch.float32),
                                                   (torch.float32, torch.float32)])
@pytest.mark.parametrize("vocab,hidden,n", [(248320, 1024, 16384), (4096, 256, 128), (64, 8, 65),
                                            (100, 12, 33), (50, 1000, 7)])
def test_gather_bit_exact(table_dtype, out_dtype, vocab, hidden, n):
    from qdc_amd import ops
    rng = np.random.default_rng(26)
    if table_dtype == torch.bfloat16:
        bits = rng.integers(0, 1 << 16, size=(vocab, hidden), dtype=np.uint16)
        table = torch.from_numpy(bits.view(np.int16)).to(DEV).view(torch.bfloat16)
        exp_bits = bits
    else:
        vals = rng.standard_normal((vocab, hidden), dtype=np.float32)
        table = torch.from_numpy(vals).to(DEV)
        exp_bits = vals.view(np.uint32)
    ids = rng.integers(0, vocab, size=n)
    ids[:3] = [0, vocab - 1, 0][:min(3, n)]
    out = ops.native_gather(table, ids, out_dtype=out_dtype)
    torch.cuda.synchronize()
    got = out.cpu()
    exp = O.gather(exp_bits, ids)
    if table_dtype == torch.bfloat16 and out_dtype == torch.float32:
        exp = (exp.astype(np.uint32) << 16)
        assert np.array_equal(got.view(torch.int32).numpy().view(np.uint32), exp)
    elif table_dtype == torch.bfloat16:
        assert np.array_equal(got.view(torch.int16).numpy().view(np.uint16), exp)
    else:
        assert np.array_equal(got.view(torch.int32).numpy().view(np.uint32), exp)


def test_gather_checks_and_device_ids():
    from qdc_amd import ops
    table = torch.arange(64 * 8, dtype=torch.float32, device=DEV).view(64, 8)
    with pytest.raises(ValueError):
        ops.native_gather(table, [1, 64])
    with pytest.raises(ValueError):
        ops.native_gather(table, [-1])
    assert ops.native_gather(table, []).shape == (0, 8)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    ids = torch.tensor([3, 99, 5, -7], dtype=torch.int32, device=DEV)
    out = ops.native_gather(table, ids, error_flag=flag)
    torch.cuda.synchronize()
    assert flag.item() == 1
    exp = table.cpu().numpy()
    got = out.cpu().numpy()
    assert np.array_equal(got[0], exp[3]) and np.array_equal(got[2], exp[5])
    assert not got[1].any() and not got[3].any()
    # without a flag (the kernel form with no atomic): the same rows, bf16 too
    for t in (table, table.to(torch.bfloat16)):
        out = ops.native_gather(t, ids).cpu()
        assert torch.equal(out[0], t[3].cpu()) and torch.equal(out[2], t[5].cpu())
        assert not out[1].any() and not out[3].any()


def test_gather_widening_invalid_ids_mid_wavefront():
    """The fp32-widening gather (lanes exchange half chunks) with out-of-range
    device ids inside a wavefront: those rows are zero, the flag is set, every
    other row is the widened table row bit for bit; rows narrower and wider
    than a wavefront's 64 chunks."""
    from qdc_amd import ops
    rng = np.random.default_rng(31)
    for vocab, hidden, n in ((40, 64, 37), (300, 1024, 9), (7, 8, 130)):
        bits = rng.integers(0, 1 << 16, size=(vocab, hidden), dtype=np.uint16)
        table = torch.from_numpy(bits.view(np.int16)).to(DEV).view(torch.bfloat16)
        ids = rng.integers(0, vocab, size=n).astype(np.int32)
        bad = [1, n // 2, n - 1]
        ids[bad] = [vocab, -1, vocab + 5]
        flag = torch.zeros(1, dtype=torch.int32, device=DEV)
        out = ops.native_gather(table, torch.from_numpy(ids).to(DEV), out_dtype=torch.float32,
                                error_flag=flag)
        torch.cuda.synchronize()
        assert flag.item() == 1
        got = out.cpu().view(torch.int32).numpy().view(np.uint32)
        ok = np.setdiff1d(np.arange(n), bad)
        assert np.array_equal(got[ok], bits[ids[ok]].astype(np.uint32) << 16), (vocab, hidden)
        assert not got[bad].any()


def test_device_copy_rows():
    """The random-row copy the benchmark holds the gathers against: each
    output row is `repeat` copies of the indexed table row's bytes; an index
    outside the table gives zeros."""
    from qdc_amd import ops
    rng = np.random.default_rng(32)
    for vocab, hidden, n, repeat in ((248320, 1024, 16384, 1), (248320, 1024, 16384, 2),
                                     (248320, 1024, 4096, 3), (50, 24, 33, 2), (9, 8, 5, 4)):
        bits = rng.integers(0, 1 << 16, size=(vocab, hidden), dtype=np.uint16)
        table = torch.from_numpy(bits.view(np.int16)).to(DEV)
        rows = rng.integers(0, vocab, size=n).astype(np.int32)
        rows[-1] = vocab  # outside: zeros
        dst = torch.full((n, hidden * repeat), 7, dtype=torch.int16, device=DEV)
        ops.device_copy_rows(dst, table, torch.from_numpy(rows).to(DEV), repeat)
        torch.cuda.synchronize()
        got = dst.cpu().numpy().view(np.uint16).reshape(n, repeat, hidden)
        for k in range(repeat):
            assert np.array_equal(got[:-1, k], bits[rows[:-1]]), (vocab, hidden, repeat)
        assert not got[-1].any()
    with pytest.raises(ValueError):
        ops.device_copy_rows(torch.empty((3, 8), dtype=torch.int16, device=DEV),
                             torch.empty((4, 8), dtype=torch.int16, device=DEV),
                             torch.zeros(3, dtype=torch.int32, device=DEV), repeat=2)


# Every fast-path row shape of the RMSNorm family (groups per row G = lanes x
# groups per lane; 4 elements per group when any tensor is fp32, 8 when all are
# bf16), once per type mix, against the oracle: a wrong dispatch entry or a
# broken multi-wavefront reduction shows at its own width.
RMS_FAST_GROUPS = [1, 2, 4, 8, 16, 32, 64, 128, 192, 256, 320, 384, 448, 512, 640, 768, 1024,
                   1280, 1536, 2048, 2560, 3072, 4096]


@pytest.mark.parametrize("groups", RMS_FAST_GROUPS)
@pytest.mark.parametrize("mix", ["f32", "bf16", "f32->bf16", "residual f32+bf16->bf16"])
def test_rmsnorm_every_fast_shape(groups, mix):
    from qdc_amd import ops
    bf, f32 = torch.bfloat16, torch.float32
    width = groups * (8 if mix == "bf16" else 4)
    rows = 5
    x = host((rows, width), 71, 1.0, bf if mix == "bf16" else f32)
    out_dtype = f32 if mix == "f32" else bf
    w = host((width,), 72, 0.02, out_dtype)
    if mix.startswith("residual"):
        m = host((rows, width), 73, 1.0, bf)
        res, got = ops.native_residual_rms(dev(x, f32), dev(m, bf), dev(w, bf), 1e-6)
        exp_res, exp = O.residual_rms(x, m, w, 1e-6)
        assert np.array_equal(back(res), exp_res)
    else:
        got = ops.native_rms(dev(x, bf if mix == "bf16" else f32), dev(w, out_dtype), 1e-6)
        exp = O.rms(x, w, 1e-6)
    report(f"rms {mix} G={groups} width={width}", back(got), exp, out_dtype)


@pytest.mark.parametrize("groups", RMS_FAST_GROUPS)
@pytest.mark.parametrize("mix", ["f32->split", "residual f32+f32->split", "gated bf16->split"])
def test_rmsnorm_every_fast_shape_split_output(groups, mix):
    """The same fast-path shapes (4 elements per group) with the split two-term
    bf16 output: hi + lo within the fp32 bar of the oracle's fp32 result."""
    from qdc_amd import ops
    bf, f32 = torch.bfloat16, torch.float32
    width, rows = groups * 4, 5
    w = host((width,), 72, 0.02, bf)
    if mix.startswith("gated"):
        x = host((rows, 1, width), 74, 1.0, bf)
        z = host((rows, 1, width), 75, 1.0, bf)
        got = ops.native_gated_rms(dev(x, bf), dev(z, bf), dev(w, bf), 1e-6,
                                   out_dtype=ops.BF16X2).view(rows, 2 * width)
        exp = O.gated_rms(x, z, w, 1e-6).reshape(rows, width)
    elif mix.startswith("residual"):
        x, m = host((rows, width), 71), host((rows, width), 73)
        res, got = ops.native_residual_rms(dev(x, f32), dev(m, f32), dev(w, bf), 1e-6,
                                           out_dtype=ops.BF16X2)
        exp_res, exp = O.residual_rms(x, m, w, 1e-6)
        assert np.array_equal(back(res), exp_res)
    else:
        x = host((rows, width), 71)
        got = ops.native_rms(dev(x, f32), dev(w, bf), 1e-6, out_dtype=ops.BF16X2)
        exp = O.rms(x, w, 1e-6)
    bits = got.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    report(f"rms {mix} G={groups} width={width}", O.join_split(bits), exp, f32)


# ------------------------------------------- fp32 residual stream mixes ------
@pytest.mark.parametrize("rows,width", [(16384, 1024), (33, 256), (5, 1000), (7, 5120),
                                        (3, 12288)])
def test_rmsnorm_fp32_to_bf16(rows, width):
    """fp32 rows normalised into a bf16 output with a bf16 weight."""
    from qdc_amd import ops
    x = host((rows, width), 27, 1.0)
    w = host((width,), 28, 0.02, torch.bfloat16)
    got = ops.native_rms(dev(x, torch.float32), dev(w, torch.bfloat16), 1e-6)
    assert got.dtype == torch.bfloat16
    report(f"rms f32->bf16 {rows}x{width}", back(got), O.rms(x, w, 1e-6), torch.bfloat16)


@pytest.mark.parametrize("mixed_dtype,out_dtype", [(torch.bfloat16, torch.bfloat16),
                                                    (torch.bfloat16, torch.float32),
                                                    (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("rows,width", [(16384, 1024), (65, 256), (3, 3000), (9, 6144),
                                        (4, 8192)])
def test_residual_rmsnorm_fp32_stream(mixed_dtype, out_dtype, rows, width):
    """fp32 residual stream + bf16 or fp32 addend -> fp32 residual, normalised
    output in the weight's dtype (bf16 for the next GEMM, fp32 for the final norm)."""
    from qdc_amd import ops
    x = host((rows, width), 29, 1.0)
    m = host((rows, width), 30, 1.0, mixed_dtype)
    w = host((width,), 31, 0.02, out_dtype)
    res, out = ops.native_residual_rms(dev(x, torch.float32), dev(m, mixed_dtype),
                                       dev(w, out_dtype), 1e-6)
    assert res.dtype == torch.float32 and out.dtype == out_dtype
    exp_res, exp_out = O.residual_rms(x, m, w, 1e-6)
    # x + mixed is one fp32 addition of the same values: bit-exact
    assert np.array_equal(back(res), exp_res)
    report(f"residual f32+bf16 -> {out_dtype} {rows}x{width}", back(out), exp_out, out_dtype)


# ------------------------------------------------- DeltaNet input mask ------
def _same_bits_or_nan(a, b):
    """Julia isequal on fp32 arrays: NaN equals NaN, -0 differs from +0."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | ((a.view(np.uint32) == b.view(np.uint32)) & ~np.isnan(a))))


def _exact_rows(width):
    """Rows whose sum of squares is exact in any summation order, so the
    normalised values are fixed bit for bit: zeros; 1e20 (the sum overflows to
    inf, scale 0); an inf (NaN there, zeros elsewhere); a NaN (all NaN); fp32
    denormals 2^-130 (squares underflow to 0: a flush-to-zero would show);
    2^-60 (squares 2^-120, exact partial sums); 3.0 and alternating +-1.5.
    All values are bf16-representable."""
    rows = [np.zeros(width), np.full(width, 1e20)]
    r = np.full(width, 3.0)
    r[width // 2] = np.inf
    rows.append(r)
    r = np.full(width, 2.0)
    r[0] = np.nan
    rows.append(r)
    rows += [np.full(width, 2.0 ** -130), np.full(width, 2.0 ** -60), np.full(width, 3.0),
             np.where(np.arange(width) % 2 == 0, 1.5, -1.5)]
    return O.round_bf16(np.array(rows, dtype=np.float32))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("width", [1024, 1000, 7, 4096, 5120])
def test_norm_special_rows_bit_exact(dtype, width):
    """Zero, overflowing, inf, NaN, denormal and exactly-summable rows through
    the plain, residual and gated norms: bit for bit (NaN-aware) equal to the
    oracle, on the fast kernels (width 1024) and the general ones (1000, 7).
    The gate z is 0, +100 or -100, where silu is exactly 0, z and -0."""
    from qdc_amd import ops
    x = _exact_rows(width)
    w = host((width,), 45, 0.02, dtype)
    # a bf16 output is the fp32 result rounded once to nearest even
    rnd = O.round_bf16 if dtype == torch.bfloat16 else (lambda e: e)
    with np.errstate(all="ignore"):
        got = back(ops.native_rms(dev(x, dtype), dev(w, dtype), 1e-6))
        assert _same_bits_or_nan(got, rnd(O.rms(x, w, 1e-6))), "rms"
        got = back(ops.native_rms(dev(x, dtype), dev(w, dtype), 1e-6, centered=False))
        assert _same_bits_or_nan(got, rnd(O.rms(x, w, 1e-6, False))), "rms not centred"
        zero = np.zeros_like(x)
        res, out = ops.native_residual_rms(dev(x, dtype), dev(zero, dtype), dev(w, dtype), 1e-6)
        exp_res, exp_out = O.residual_rms(x, zero, w, 1e-6)
        assert _same_bits_or_nan(back(res), exp_res), "residual"
        assert _same_bits_or_nan(back(out), rnd(exp_out)), "residual norm"
        z = np.resize(np.array([0.0, 100.0, -100.0], np.float32), x.shape)
        got = back(ops.native_gated_rms(dev(x, dtype).view(len(x), 1, width),
                                        dev(z, dtype).view(len(x), 1, width), dev(w, dtype), 1e-6))
        exp = O.gated_rms(x.reshape(len(x), 1, width), z.reshape(len(x), 1, width), w, 1e-6)
        assert _same_bits_or_nan(got.reshape(x.shape), rnd(exp.reshape(x.shape))), "gated"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hd,rd", [(256, 64), (96, 24)])
def test_qk_norm_rope_special_rows_bit_exact(dtype, hd, rd):
    """The same exactly-summable and special rows as q and k heads (one token
    each, positions 0..7): normalisation and rotation use the oracle's
    operation order and its bit-equal tables, so q and k agree bit for bit
    (fast kernel at head_dim 256, general kernel at 96)."""
    from qdc_amd import ops
    x = _exact_rows(hd)
    T = len(x)
    qn = host((hd,), 46, 0.02, dtype)
    kn = host((hd,), 47, 0.02, dtype)
    tables = ops.rope_tables(T, rd, 1e7, DEV)
    cos, sin = O.rope_tables(T, rd, 1e7)
    rnd = O.round_bf16 if dtype == torch.bfloat16 else (lambda e: e)
    xs = x.reshape(T, 1, hd)
    with np.errstate(all="ignore"):
        qo, ko = ops.prepare_heads(dev(xs, dtype), dev(xs, dtype), dev(qn, dtype), dev(kn, dtype),
                                   tables, rd, 1e-6, seq_len=T)
        assert _same_bits_or_nan(back(qo), rnd(O.qk_norm_rope(xs, qn, cos, sin, rd, 1e-6, T))), "q"
        assert _same_bits_or_nan(back(ko), rnd(O.qk_norm_rope(xs, kn, cos, sin, rd, 1e-6, T))), "k"


@pytest.mark.parametrize("x_dtype,out_dtype", [(torch.float32, torch.float32),
                                                (torch.bfloat16, torch.bfloat16),
                                                (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("rows,width", [(16384, 1024), (65, 256), (33, 1000), (3, 7), (9, 5120)])
def test_masked_norms(x_dtype, out_dtype, rows, width):
    """The DeltaNet input mask (src/backbone.jl:286) fused into the norms that
    produce that input.  Each masked row is the unmasked kernel's row times its
    0/1 entry, bit for bit (-0, and NaN from a masked inf, included); the
    residual output is not masked; and the finite rows match the oracle's norm
    followed by the reference's ``x .* mask``.  Widths 1000 and 7 take the
    general kernels."""
    from qdc_amd import ops
    keep = (np.random.default_rng(40).random(rows) < 0.7).astype(np.int32)
    keep[0] = 0
    keep[-1] = 1
    x = host((rows, width), 41, 1.0, x_dtype)
    m = host((rows, width), 42, 1.0, out_dtype)
    w = host((width,), 43, 0.02, out_dtype)
    special = 1 if rows > 2 else None
    if special is not None:  # masked row holding an inf: 0 * inf = NaN, as in the reference
        keep[special] = 0
        x[special, 0] = np.inf
    finite = np.ones(rows, bool)
    if special is not None:
        finite[special] = False
    km = torch.from_numpy(keep).to(DEV)
    xt, mt, wt = dev(x, x_dtype), dev(m, out_dtype), dev(w, out_dtype)
    with np.errstate(all="ignore"):
        plain = back(ops.native_rms(xt, wt, 1e-6))
        masked = back(ops.native_rms(xt, wt, 1e-6, token_mask=km))
        assert _same_bits_or_nan(masked, plain * keep[:, None].astype(np.float32))
        exp = O.rms(x, w, 1e-6) * keep[:, None].astype(np.float32)
        report(f"masked rms {rows}x{width} {x_dtype}->{out_dtype}", masked[finite], exp[finite],
               out_dtype)
        res0, out0 = ops.native_residual_rms(xt, mt, wt, 1e-6)
        res1, out1 = ops.native_residual_rms(xt, mt, wt, 1e-6, token_mask=km)
        assert _same_bits_or_nan(back(res1), back(res0))
        assert _same_bits_or_nan(back(out1), back(out0) * keep[:, None].astype(np.float32))
        exp_res, exp_out = O.residual_rms(x, m, w, 1e-6)
        report(f"masked residual-norm {rows}x{width}", back(out1)[finite],
               (exp_out * keep[:, None].astype(np.float32))[finite], out_dtype)
    with pytest.raises(ValueError):
        ops.native_rms(xt, wt, 1e-6, token_mask=km[:-1])
    with pytest.raises(ValueError):
        ops.native_rms(xt, wt, 1e-6, token_mask=km.to(torch.int64))


# ------------------------------------------- fast and general kernels ------
def _shifted(t):
    """The same values starting one element past a 16-byte boundary (the
    general kernels take them)."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    buf[1:] = t.reshape(-1)
    out = buf[1:].view(t.shape)
    assert out.data_ptr() % 16 != 0
    return out


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("op", ["rms", "residual", "gated", "qk", "swiglu", "gather",
                                "prologue", "softmax", "gate"])
def test_fast_and_general_kernels_agree(dtype, op):
    """Each op at its Qwen3.5-0.8B-like shape through both of its kernels --
    aligned inputs take the fast kernel, the same values one element off a
    16-byte boundary the general one -- as the reference checks each CPU policy
    against the generic path (test/backbone.jl:36-75): both within the op's bar
    of the oracle and close to each other (the gather bit for bit)."""
    from oracle import forward
    from qdc_amd import ops
    bar = dtype  # tolerance class of the outputs
    if op == "prologue":  # bf16 or fp32 projection -> fp32 q, k, v
        B, S, KH, kd, H, vd = 2, 1024, 16, 128, 16, 128
        kw, vw = KH * kd, H * vd
        cq = 2 * kw + vw
        width = cq + vw + 2 * H
        x = host((B * S, width), 67, 1.0, dtype)
        conv = host((cq, 4), 68, 0.5)
        a_decay, dt_bias = -np.exp(host((H,), 69, 0.5)), host((H,), 70, 1.0)
        dconv, da, dd = (dev(t, torch.float32) for t in (conv, a_decay, dt_bias))

        def run(xt):
            parts = ops.delta_prologue(xt, dconv, da, dd, S, KH, kd, H, vd)
            return torch.cat([t.reshape(-1) for t in parts[:3]])
        per = [forward.delta_prologue(r[:, :cq], conv, r[:, cq + vw:cq + vw + H],
                                      r[:, cq + vw + H:width], a_decay, dt_bias, KH, kd, H, vd)
               for r in (x[b * S:(b + 1) * S] for b in range(B))]
        exp = np.concatenate([np.concatenate([p[i] for p in per]).reshape(-1) for i in range(3)])
        bar = torch.float32
    elif op == "softmax":
        x, mask = _softmax_inputs((1, 8, 2048, 2048, 0, "rand"))
        scale = float(1.0 / np.sqrt(np.float32(256)))
        dmask = dev(mask, torch.int32)
        run = lambda xt: ops.attention_softmax(xt, dmask, scale, out_dtype=dtype)  # noqa: E731
        exp = forward.attention_softmax(x, mask, np.float32(scale))
        x = x.astype(np.float32)
    elif op == "gate":
        B, S, H, hd = 1, 2048, 8, 256
        x = host((B, H, S, hd), 71, 1.0)
        qgate = host((B * S, H, 2 * hd), 72, 2.0, dtype)
        gv = dev(qgate, dtype)[:, :, hd:]
        run = lambda xt: ops.attention_gate(xt, gv, out_dtype=dtype)  # noqa: E731
        exp = forward.attention_gate(x, qgate[:, :, hd:])
    elif op == "rms":
        x, w = host((8192, 1024), 51, 1.0, dtype), host((1024,), 52, 0.02, dtype)
        run = lambda xt: ops.native_rms(xt, dev(w, dtype), 1e-6)  # noqa: E731
        exp = O.rms(x, w, 1e-6)
    elif op == "residual":
        x, m = host((8192, 1024), 53, 1.0, dtype), host((8192, 1024), 54, 1.0, dtype)
        w = host((1024,), 55, 0.02, dtype)
        run = lambda xt: ops.native_residual_rms(xt, dev(m, dtype), dev(w, dtype), 1e-6)[1]  # noqa: E731
        exp = O.residual_rms(x, m, w, 1e-6)[1]
    elif op == "gated":
        x, z = host((2048, 16, 128), 56, 1.0, dtype), host((2048, 16, 128), 57, 1.0, dtype)
        w = host((128,), 58, 1.0, dtype)
        run = lambda xt: ops.native_gated_rms(xt, dev(z, dtype), dev(w, dtype), 1e-6)  # noqa: E731
        exp = O.gated_rms(x, z, w, 1e-6)
    elif op == "qk":
        T, H, KV, hd, rd, seq = 4096, 8, 2, 256, 64, 2048
        x, kx = host((T, H, hd), 59, 1.0, dtype), host((T, KV, hd), 60, 1.0, dtype)
        qn, kn = host((hd,), 61, 0.02, dtype), host((hd,), 62, 0.02, dtype)
        tables = ops.rope_tables(seq, rd, 1e7, DEV)
        kt = dev(kx, dtype)

        def run(xt):
            qo, ko = ops.prepare_heads(xt, kt, dev(qn, dtype), dev(kn, dtype), tables, rd, 1e-6,
                                       seq_len=seq)
            return torch.cat([qo.reshape(-1), ko.reshape(-1)])
        cos, sin = O.rope_tables(seq, rd, 1e7)
        exp = np.concatenate([O.qk_norm_rope(x, qn, cos, sin, rd, 1e-6, seq).reshape(-1),
                              O.qk_norm_rope(kx, kn, cos, sin, rd, 1e-6, seq).reshape(-1)])
    elif op == "swiglu":
        x, u = host((4096, 3584), 63, 1.0, dtype), host((4096, 3584), 64, 1.0, dtype)
        run = lambda xt: ops.native_mlp_gate(xt, dev(u, dtype))  # noqa: E731
        exp = O.swiglu(x, u)
    else:  # gather: the table is the aligned input; shift the output instead
        table = host((4096, 1024), 65, 0.02, dtype)
        ids = np.random.default_rng(66).integers(0, 4096, size=2048)
        tt = dev(table, dtype)
        fast = back(ops.native_gather(tt, ids))
        general = _shifted(torch.zeros((2048, 1024), dtype=dtype, device=DEV))
        ops.native_gather(tt, ids, out=general)
        exp = table[ids]
        assert np.array_equal(fast, exp) and np.array_equal(back(general), exp)
        return
    xt = dev(x, torch.float32 if op in ("softmax", "gate") else dtype)
    fast, general = back(run(xt)), back(run(_shifted(xt)))
    report(f"{op} fast kernel", fast, exp, bar)
    report(f"{op} general kernel", general, exp, bar)
    assert normwise(fast, general) <= (1e-6 if bar == torch.float32 else 2e-3)


def _kernel_chain(seed):
    """Inputs drawn from seeds seed .. seed+16 and a closure running a chain of
    the library's kernels on them (gather, RMSNorm, q/k norm + RoPE, SwiGLU,
    gated norm, residual norm, DeltaNet prologue and scan, softmax, gate merge);
    it allocates its outputs on the current stream."""
    from qdc_amd import ops
    dt = torch.bfloat16
    r = lambda shape, k, scale=1.0: dev(host(shape, seed + k, scale, dt), dt)  # noqa: E731
    T, hidden, H, KV, hd, rd = 256, 1024, 8, 2, 256, 64
    table = r((512, hidden), 0, 0.02)
    ids = torch.from_numpy(np.random.default_rng(seed).integers(0, 512, T).astype(np.int32)).to(DEV)
    w = r((hidden,), 1, 0.02)
    qg, kx = r((T, H, 2 * hd), 2), r((T, KV, hd), 3)
    qn, kn = r((hd,), 4, 0.02), r((hd,), 5, 0.02)
    tables = ops.rope_tables(T, rd, 1e7, DEV)
    gu = r((T, 2 * 3584), 6)
    gx, gz, gw = r((T, 16, 128), 7), r((T, 16, 128), 8), r((128,), 9)
    mixed = r((T, hidden), 10)
    KH, kd, VH, vd = 16, 128, 16, 128
    cq = 2 * KH * kd + VH * vd
    proj = r((T, cq + VH * vd + 2 * VH), 11)
    conv = dev(host((cq, 4), seed + 12, 0.5), torch.float32)
    a_dec = dev(-np.exp(host((VH,), seed + 13, 0.5)), torch.float32)
    dt_b = dev(host((VH,), seed + 14, 1.0), torch.float32)
    scores = dev(host((1, H, T, T), seed + 15, 4.0), torch.float32)
    values = dev(host((1, H, T, hd), seed + 16, 1.0), torch.float32)

    def chain():
        h = ops.native_gather(table, ids, out_dtype=torch.float32)
        n = ops.native_rms(h, w.float(), 1e-6)
        qo, ko = ops.prepare_heads(qg[:, :, :hd], kx, qn, kn, tables, rd, 1e-6, seq_len=T)
        a = ops.native_mlp_gate(gu[:, :3584], gu[:, 3584:])
        g = ops.native_gated_rms(gx, gz, gw, 1e-6)
        res, nr = ops.native_residual_rms(h, mixed, w, 1e-6)
        q, k, v, beta, decay = ops.delta_prologue(proj, conv, a_dec, dt_b, T, KH, kd, VH, vd)
        o = ops.delta_scan(q.view(1, T, KH, kd), k.view(1, T, KH, kd), v.view(1, T, VH, vd),
                           beta.view(1, T, VH), decay.view(1, T, VH), dt)
        p = ops.attention_softmax(scores, None, 0.0625, out_dtype=dt)
        m = ops.attention_gate(values, qg[:, :, hd:], out_dtype=dt)
        return [n, qo, ko, a, g, res, nr, o, p, m]
    return chain


def test_graph_replays_match_eager():
    """The kernel chain captured once in a HIP graph and replayed three times,
    with eager work on other buffers in between: every replay equals the eager
    run bit for bit (the kernels clear nothing with memset and keep no state
    between calls)."""
    chain = _kernel_chain(81)
    eager = [t.clone() for t in chain()]
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        chain()  # warm up on the capture stream
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            outs = chain()
    for rep in range(3):
        for t in outs:
            t.fill_(float("nan"))  # a replay must rewrite every output
        graph.replay()
        torch.cuda.synchronize()
        other = chain()  # eager work between replays, on freshly allocated outputs
        torch.cuda.synchronize()
        for i, (got, exp) in enumerate(zip(outs, eager)):
            assert torch.equal(got, exp), (rep, i)
            assert torch.equal(other[i], exp), (rep, i)


def _bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


def test_concurrent_threads_on_own_streams_match_serial():
    """Two host threads, each on its own stream, run the kernel chain ten times
    on different inputs at the same time (the C calls release the GIL): every
    result equals the serial run bit for bit.  The library keeps no mutable
    state and launches only on the stream it is given."""
    import threading
    chains = [_kernel_chain(100), _kernel_chain(200)]
    serial = [[t.clone() for t in c()] for c in chains]
    torch.cuda.synchronize()
    results, errors = [None, None], []

    def worker(i):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                for _ in range(10):
                    outs = chains[i]()
                stream.synchronize()
            results[i] = outs
        except Exception as e:  # reported after the join
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i in range(2):
        for j, (got, exp) in enumerate(zip(results[i], serial[i])):
            assert torch.equal(_bits(got), _bits(exp)), (i, j)


# ------------------------------------------------ DeltaNet recurrence --------
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,S,KH,H,kd,vd,dscale", [
    (2, 37, 2, 4, 128, 128, 2.0), (3, 64, 16, 16, 128, 128, 2.0),   # matrix-core chunked form
    (1, 33, 1, 2, 64, 48, 2.0), (2, 16, 1, 1, 16, 16, 2.0), (1, 50, 2, 2, 32, 16, 2.0),
    (1, 300, 1, 1, 256, 32, 2.0), (1, 40, 1, 2, 128, 128, 40.0),    # strong decay
    (2, 20, 1, 2, 128, 80, 2.0),                                    # two chunks, 80 rows
    (1, 2048, 1, 2, 128, 128, 0.05),                # a whole 0.8B-shaped sequence, weak decay
    (1, 5, 1, 2, 64, 20, 2.0), (1, 9, 1, 1, 256, 8, 2.0),           # recurrent kernel
    (2, 65, 1, 2, 2, 2, 2.0), (1, 17, 2, 6, 96, 33, 2.0)])
def test_delta_scan(out_dtype, B, S, KH, H, kd, vd, dscale):
    from oracle import forward
    from qdc_amd import ops
    rng = np.random.default_rng(32)
    q = rng.standard_normal((B, S, KH, kd), dtype=np.float32)
    k = rng.standard_normal((B, S, KH, kd), dtype=np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True) * np.float32(np.sqrt(kd))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, S, H, vd), dtype=np.float32)
    beta = rng.random((B, S, H), dtype=np.float32)
    decay = -rng.random((B, S, H), dtype=np.float32) * np.float32(dscale)
    got = back(ops.delta_scan(*(dev(a, torch.float32) for a in (q, k, v, beta, decay)),
                              out_dtype=out_dtype))
    exp = np.stack([forward.delta_recurrence(q[b], k[b], v[b], beta[b], decay[b])
                    for b in range(B)])
    report(f"delta scan {B}x{S} kh{KH} h{H} kd{kd} vd{vd} decay*{dscale}", got, exp, out_dtype)
    # the same inputs as the column blocks of one [B, S, q|k|v] buffer, the
    # prologue's layout in the forward (row strides ld_qk = ld_v = the row
    # length): bit-identical to the contiguous inputs
    kw, vw = KH * kd, H * vd
    qkv = torch.from_numpy(np.concatenate([q.reshape(B, S, kw), k.reshape(B, S, kw),
                                           v.reshape(B, S, vw)], axis=-1)).to(DEV)
    strided = back(ops.delta_scan(qkv[..., :kw].view(B, S, KH, kd),
                                  qkv[..., kw:2 * kw].view(B, S, KH, kd),
                                  qkv[..., 2 * kw:].view(B, S, H, vd), dev(beta, torch.float32),
                                  dev(decay, torch.float32), out_dtype=out_dtype))
    assert np.array_equal(strided, got, equal_nan=True)


@pytest.mark.parametrize("B,S,KH,H,kd,vd", [(2, 50, 2, 4, 128, 128), (1, 300, 1, 1, 64, 32)])
def test_delta_scan_chunked_matches_recurrent(B, S, KH, H, kd, vd):
    """The two forms of the recurrence agree, as the reference checks its chunked
    and recurrent DeltaNet paths (test/backbone.jl:162-185): the same values go
    through the matrix-core chunked kernel (aligned inputs) and the token
    recurrence (q shifted by one element, so not 16-byte aligned)."""
    from oracle import forward
    from qdc_amd import ops
    rng = np.random.default_rng(33)
    q = rng.standard_normal((B, S, KH, kd), dtype=np.float32)
    k = rng.standard_normal((B, S, KH, kd), dtype=np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True) * np.float32(np.sqrt(kd))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, S, H, vd), dtype=np.float32)
    beta = rng.random((B, S, H), dtype=np.float32)
    decay = -rng.random((B, S, H), dtype=np.float32) * np.float32(2.0)
    args = [dev(a, torch.float32) for a in (q, k, v, beta, decay)]
    chunked = back(ops.delta_scan(*args))
    shifted = torch.empty(q.size + 1, dtype=torch.float32, device=DEV)
    shifted[1:] = args[0].reshape(-1)
    q_off = shifted[1:].view(q.shape)
    assert q_off.data_ptr() % 16 != 0
    recurrent = back(ops.delta_scan(q_off, *args[1:]))
    exp = np.stack([forward.delta_recurrence(q[b], k[b], v[b], beta[b], decay[b])
                    for b in range(B)])
    report(f"chunked {B}x{S} kd{kd}", chunked, exp, torch.float32)
    report(f"recurrent {B}x{S} kd{kd}", recurrent, exp, torch.float32)
    assert normwise(chunked, recurrent) <= 2e-6


# ------------------------------------------------ DeltaNet prologue ----------
# (B, S, KH, kd, H, vd, taps, pad): pad > 0 widens the row stride by pad elements
PROLOGUE_CASES = [
    (2, 1024, 16, 128, 16, 128, 4, 0),   # Qwen3.5-0.8B DeltaNet dims: 12/8-token tiles
    (1, 200, 16, 128, 16, 128, 4, 0),    # the same dims, one short sequence: 4-token tiles
    (2, 37, 2, 128, 4, 128, 4, 0),       # sequences break inside a (4-token) tile
    (3, 5, 1, 64, 2, 32, 4, 8),          # strided rows
    (7, 1, 2, 16, 2, 8, 4, 0),           # every token starts a sequence
    (2, 33, 1, 8, 4, 16, 4, 0),          # one lane per key head
    (1, 65, 2, 2, 2, 2, 4, 0),           # fixture-sized heads: general kernel
    (2, 19, 2, 96, 4, 40, 4, 0),         # kd/8 not a power of two: general kernel
    (2, 21, 1, 64, 2, 64, 3, 0),         # three taps: general kernel
    (1, 17, 1, 64, 2, 64, 4, 3),         # odd row stride: general kernel
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", PROLOGUE_CASES)
def test_delta_prologue(dtype, case):
    from oracle import forward
    from qdc_amd import ops
    B, S, KH, kd, H, vd, taps, pad = case
    kw, vw = KH * kd, H * vd
    cq = 2 * kw + vw
    width = cq + vw + 2 * H
    T = B * S
    proj = host((T, width + pad), 41, 1.0, dtype)
    conv = host((cq, taps), 42, 0.5)
    a_decay = -np.exp(host((H,), 43, 0.5))
    dt_bias = host((H,), 44, 1.0)
    # wide gate inputs so both softplus branches and saturated sigmoids occur
    proj[:, cq + vw:width] *= np.float32(8)
    proj = O.round_bf16(proj) if dtype == torch.bfloat16 else proj
    d_proj = dev(proj, dtype)[:, :width]
    got = [back(t) for t in ops.delta_prologue(d_proj, dev(conv, torch.float32),
                                               dev(a_decay, torch.float32),
                                               dev(dt_bias, torch.float32), S, KH, kd, H, vd)]
    exp = [[], [], [], [], []]
    for b in range(B):
        rows = proj[b * S:(b + 1) * S]
        parts = forward.delta_prologue(rows[:, :cq], conv, rows[:, cq + vw:cq + vw + H],
                                       rows[:, cq + vw + H:width], a_decay, dt_bias, KH, kd, H, vd)
        for i, part in enumerate(parts):
            exp[i].append(part)
    for name, g, e in zip(("q", "k", "v", "beta", "decay"), got, exp):
        e = np.concatenate(e)
        assert g.shape == e.shape, (name, g.shape, e.shape)
        report(f"prologue {name} {case} {dtype}", g, e, torch.float32)
    # q, k, v written as the column blocks of one [T, q|k|v] buffer (the
    # forward's layout): the same values, bit for bit
    il = ops.delta_prologue(d_proj, dev(conv, torch.float32), dev(a_decay, torch.float32),
                            dev(dt_bias, torch.float32), S, KH, kd, H, vd, interleaved=True)
    assert il[0].stride(0) == cq and il[1].data_ptr() == il[0].data_ptr() + 4 * kw
    for name, g, t in zip(("q", "k", "v", "beta", "decay"), got, il):
        assert np.array_equal(back(t), g, equal_nan=True), name


@pytest.mark.parametrize("KH,kd,H,vd,pad", [(1, 8, 1, 8, 2),    # fast kernel
                                            (1, 6, 1, 6, 0)])   # general kernel
def test_delta_prologue_special_values(KH, kd, H, vd, pad):
    """The q/k normalisation special values of test/backbone.jl:304-312 (0, -0,
    NaN, Inf, floatmax and the smallest denormal) through the prologue: every
    token its own sequence and the convolution the current-row tap, so each head
    sees silu(x) with x the special value (2^-148 becomes 2^-149)."""
    from oracle import forward
    from qdc_amd import ops
    kw, vw = KH * kd, H * vd
    cq = 2 * kw + vw
    width = cq + vw + 2 * H
    specials = [0.0, -0.0, np.nan, np.inf, float(np.finfo(np.float32).max), 2.0 ** -148]
    T = len(specials)
    proj = np.zeros((T, width + pad), np.float32)
    proj[:, :cq] = np.array(specials, np.float32)[:, None]
    conv = np.zeros((cq, 4), np.float32)
    conv[:, 3] = 1.0
    a_decay = np.full((H,), -1.0, np.float32)
    dt_bias = np.zeros((H,), np.float32)
    got = [back(t) for t in ops.delta_prologue(dev(proj, torch.float32)[:, :width],
                                               dev(conv, torch.float32),
                                               dev(a_decay, torch.float32),
                                               dev(dt_bias, torch.float32), 1, KH, kd, H, vd)]
    for t in range(T):
        row = proj[t:t + 1]
        exp = forward.delta_prologue(row[:, :cq], conv, row[:, cq + vw:cq + vw + H],
                                     row[:, cq + vw + H:width], a_decay, dt_bias, KH, kd, H, vd)
        for name, g, e in zip(("q", "k", "v"), got[:3], exp[:3]):
            assert _same_bits_or_nan(g[t], e[0]), (name, specials[t], g[t], e[0])


# ------------------------------------------------ attention row work ---------
# (B, H, Q, K, q_offset, mask kind): "rand" = 30% of keys masked, "none" = no mask,
# "dead" = some sequences whose first keys are all masked (rows with no visible key)
SOFTMAX_CASES = [
    (2, 8, 2048, 2048, 0, "rand"),   # Qwen3.5-0.8B full attention, 2 of the 8 sequences
    (1, 3, 37, 37, 0, "rand"),
    (2, 2, 5, 8, 0, "dead"),
    (1, 2, 16, 100, 84, "rand"),     # a chunk of queries at the end of a 100-key context
    (1, 1, 7, 2560, 2553, "none"),   # more keys than one wavefront holds: 2 per row
    (1, 2, 40, 4096, 4056, "rand"),  # 2 wavefronts per row
    (2, 1, 20, 8192, 0, "dead"),     # 4 per row, rows with no visible key
    (1, 1, 12, 20000, 19988, "rand"),  # 16 per row (1024-thread workgroups), a partial chunk span
    (1, 1, 6, 32768, 32762, "none"),   # the longest rows of the register path
    (1, 1, 3, 33000, 32997, "none"),   # longer rows: general kernel
    (1, 1, 5, 2561, 2556, "none"),   # long rows with keys % 4 != 0: general kernel
    (1, 2, 9, 13, 4, "rand"),        # keys % 4 != 0: general kernel
]


def _softmax_inputs(case):
    B, H, Q, K, off, kind = case
    scores = host((B, H, Q, K), 51, 4.0)
    mask = None
    if kind != "none":
        mask = (np.random.default_rng(52).random((B, K)) > 0.3).astype(np.int32)
        if kind == "dead":
            mask[1, :4] = 0
    return scores, mask


@pytest.mark.parametrize("out_dtype", DTYPES)
@pytest.mark.parametrize("case", SOFTMAX_CASES)
def test_attention_softmax(out_dtype, case):
    from oracle import forward
    from qdc_amd import ops
    B, H, Q, K, off, kind = case
    scores, mask = _softmax_inputs(case)
    scale = 1.0 / np.sqrt(np.float32(256))
    got = ops.attention_softmax(dev(scores, torch.float32),
                                dev(mask, torch.int32) if mask is not None else None,
                                float(scale), off, out_dtype=out_dtype)
    exp = forward.attention_softmax(scores, mask, np.float32(scale), off)
    got = back(got)
    report(f"softmax {case} -> {out_dtype}", got, exp, out_dtype)
    if out_dtype == torch.float32:
        # causally hidden keys are exactly zero unless the row sees no key at all
        pos = np.arange(Q)[:, None] + off
        hidden = np.broadcast_to(np.arange(K)[None, :] > pos, got.shape)
        dead = np.isclose(exp, 1.0 / K).all(-1, keepdims=True)
        assert np.all(got[hidden & ~np.broadcast_to(dead, got.shape)] == 0)


@pytest.mark.parametrize("case", [(2, 4, 64, 64, 0, "rand"), (1, 2, 8, 4096, 4088, "rand")])
def test_attention_softmax_in_place(case):
    from oracle import forward
    from qdc_amd import ops
    scores, mask = _softmax_inputs(case)
    d = dev(scores, torch.float32)
    out = ops.attention_softmax(d, dev(mask, torch.int32), 0.0625, case[4], out=d)
    assert out.data_ptr() == d.data_ptr()
    report(f"softmax in place {case}", back(d),
           forward.attention_softmax(scores, mask, 0.0625, case[4]), torch.float32)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,S,H,hd", [(8, 2048, 8, 256), (2, 37, 4, 64), (1, 5, 3, 12),
                                      (3, 1, 2, 8)])
def test_attention_gate(dtype, B, S, H, hd):
    from oracle import forward
    from qdc_amd import ops
    values = host((B, H, S, hd), 61, 1.0)
    qgate = host((B * S, H, 2 * hd), 62, 2.0, dtype)      # interleaved q||gate projection
    got = ops.attention_gate(dev(values, torch.float32), dev(qgate, dtype)[:, :, hd:])
    assert got.dtype == dtype and got.shape == (B * S, H * hd)
    exp = forward.attention_gate(values, qgate[:, :, hd:])
    report(f"gate {B}x{S} h{H} hd{hd} {dtype}", back(got), exp, dtype)


def test_attention_gate_fp32_out_from_bf16_gate():
    from oracle import forward
    from qdc_amd import ops
    B, S, H, hd = 2, 33, 8, 256
    values = host((B, H, S, hd), 63, 1.0)
    gate = host((B * S, H, hd), 64, 2.0, torch.bfloat16)
    got = ops.attention_gate(dev(values, torch.float32), dev(gate, torch.bfloat16),
                             out_dtype=torch.float32)
    report("gate bf16 -> f32", back(got), forward.attention_gate(values, gate), torch.float32)


def test_qk_norm_rope_head_major_output():
    # the reference AMDGPU layout (dim, tokens, heads): q/k written head-major
    from qdc_amd import ops
    T, H, KV, hd, rd, seq = 40, 4, 2, 64, 16, 20
    qgate = host((T, H, 2 * hd), 71, 1.0)
    k = host((T, KV, hd), 72, 1.0)
    qn, kn = host((hd,), 73, 0.02), host((hd,), 74, 0.02)
    tables = ops.rope_tables(seq, rd, 1e7, DEV)
    q_hm = torch.empty((H, T, hd), device=DEV)
    k_hm = torch.empty((KV, T, hd), device=DEV)
    ops.prepare_heads(dev(qgate, torch.float32)[:, :, :hd], dev(k, torch.float32),
                      dev(qn, torch.float32), dev(kn, torch.float32), tables, rd, 1e-6,
                      seq_len=seq, q_out=q_hm.permute(1, 0, 2), k_out=k_hm.permute(1, 0, 2))
    cos, sin = O.rope_tables(seq, rd, 1e7)
    report("q head-major", back(q_hm).transpose(1, 0, 2),
           O.qk_norm_rope(qgate[:, :, :hd], qn, cos, sin, rd, 1e-6, seq), torch.float32)
    report("k head-major", back(k_hm).transpose(1, 0, 2),
           O.qk_norm_rope(k, kn, cos, sin, rd, 1e-6, seq), torch.float32)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,S,H,KV,hd,rd", [(8, 2048, 8, 2, 256, 64), (3, 37, 4, 1, 64, 16),
                                            (2, 9, 2, 2, 128, 128), (3, 5, 3, 1, 96, 24)])
def test_qk_norm_rope_batched_head_major(dtype, B, S, H, KV, hd, rd):
    """All sequences of a batch in one launch, written head-major per sequence
    ([B, H, S, hd], the layout of the batched attention products): each
    sequence equals the one-sequence call bit for bit (the reference runs one
    sequence per call) and matches the oracle.  Cases cover the contiguous and
    pair-dealt fast kernels and the general kernel (head_dim 96)."""
    from qdc_amd import ops
    T = B * S
    qgate = host((T, H, 2 * hd), 75, 1.0, dtype)
    k = host((T, KV, hd), 76, 1.0, dtype)
    qn, kn = host((hd,), 77, 0.02, dtype), host((hd,), 78, 0.02, dtype)
    tables = ops.rope_tables(S, rd, 1e6, DEV)
    qg, kk = dev(qgate, dtype), dev(k, dtype)
    qw, kw = dev(qn, dtype), dev(kn, dtype)
    q_hm = torch.full((B, H, S, hd), float("nan"), dtype=dtype, device=DEV)
    k_hm = torch.full((B, KV, S, hd), float("nan"), dtype=dtype, device=DEV)
    ops.prepare_heads(qg[:, :, :hd], kk, qw, kw, tables, rd, 1e-6, seq_len=S,
                      q_out=q_hm.permute(0, 2, 1, 3), k_out=k_hm.permute(0, 2, 1, 3))
    for b in range(B):
        rows = slice(b * S, (b + 1) * S)
        qo, ko = ops.prepare_heads(qg[rows, :, :hd], kk[rows], qw, kw, tables, rd, 1e-6,
                                   seq_len=S)
        assert torch.equal(q_hm[b].permute(1, 0, 2), qo), b
        assert torch.equal(k_hm[b].permute(1, 0, 2), ko), b
    cos, sin = O.rope_tables(S, rd, 1e6)
    take = slice(0, min(T, 4096))  # oracle on the first sequences only
    got_q = back(q_hm).transpose(0, 2, 1, 3).reshape(T, H, hd)[take]
    got_k = back(k_hm).transpose(0, 2, 1, 3).reshape(T, KV, hd)[take]
    report("q batched", got_q, O.qk_norm_rope(qgate[take, :, :hd], qn, cos, sin, rd, 1e-6, S), dtype)
    report("k batched", got_k, O.qk_norm_rope(k[take], kn, cos, sin, rd, 1e-6, S), dtype)


def test_device_copy():
    """The streaming copy the benchmark uses as its per-size ceiling moves
    every byte (sizes not a multiple of a workgroup's 4 KB included)."""
    from qdc_amd import ops
    for nbytes in (16, 4096 + 48, 33_554_432):
        src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=DEV)
        dst = torch.zeros_like(src)
        ops.device_copy(dst, src)
        torch.cuda.synchronize()
        assert torch.equal(dst, src), nbytes
    with pytest.raises(ValueError):
        ops.device_copy(torch.empty(32, dtype=torch.uint8, device=DEV),
                        torch.empty(24, dtype=torch.uint8, device=DEV))


@pytest.mark.parametrize("cpt,block", [(1, 256), (2, 256), (4, 256), (8, 256), (1, 512), (2, 512),
                                       (4, 512), (8, 512)])
def test_device_copy_shapes(cpt, block):
    """Every launch shape of the copy ceiling (qdc_copy_grid) moves every byte,
    with a last workgroup that is partly past the end and one that is whole, and
    touches nothing after the destination."""
    from qdc_amd import ops
    for nbytes in (16, cpt * block * 16 * 3, cpt * block * 16 * 3 + 4096 + 48, 16_777_216 + 16):
        src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=DEV)
        dst = torch.zeros(nbytes + 4096, dtype=torch.uint8, device=DEV)
        ops.device_copy(dst[:nbytes], src, cpt, block)
        torch.cuda.synchronize()
        assert torch.equal(dst[:nbytes], src), (cpt, block, nbytes)
        assert not dst[nbytes:].any(), (cpt, block, nbytes)
    with pytest.raises(ValueError):   # not a launch shape of the library
        ops.device_copy(torch.empty(32, dtype=torch.uint8, device=DEV),
                        torch.empty(32, dtype=torch.uint8, device=DEV), 3, 256)


@pytest.mark.parametrize("cpt,block", [(1, 256), (2, 256), (4, 256), (8, 256), (1, 512),
                                       (4, 512)])
def test_device_copy_pair(cpt, block):
    """Both streams of the two-copy ceiling (qdc_copy_pair) arrive byte for byte,
    with equal and unequal sizes (the shorter stream ending inside a workgroup,
    or empty) and nothing written past either destination."""
    from qdc_amd import ops
    span = cpt * block * 16
    for n0, n1 in ((span * 3, span * 3), (span * 3 + 4096 + 48, span + 32), (16, span * 2 + 16),
                   (33_554_432, 33_554_432), (span, 0)):
        s0 = torch.randint(0, 256, (n0,), dtype=torch.uint8, device=DEV)
        s1 = torch.randint(0, 256, (n1,), dtype=torch.uint8, device=DEV)
        d0 = torch.zeros(n0 + 4096, dtype=torch.uint8, device=DEV)
        d1 = torch.zeros(n1 + 4096, dtype=torch.uint8, device=DEV)
        ops.device_copy_pair(d0[:n0], s0, d1[:n1], s1, cpt, block)
        torch.cuda.synchronize()
        assert torch.equal(d0[:n0], s0) and torch.equal(d1[:n1], s1), (cpt, block, n0, n1)
        assert not d0[n0:].any() and not d1[n1:].any(), (cpt, block, n0, n1)


# ---------------------------------------------------------------- row scale --
def test_row_scale_check_every_pattern():
    """The row kernels take 1/sqrt(x) from the hardware square root and
    reciprocal estimates with one-ulp corrections for 2^-96 <= x < inf; over
    all 2^32 fp32 bit patterns it equals the general 1.0f / sqrtf(x) in every
    bit (qdc_row_scale_check counts the differences on the device)."""
    from qdc_amd import _lib
    lib = _lib.lib()
    count = torch.zeros(1, dtype=torch.int64, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    step = 1 << 30
    for first in range(0, 1 << 32, step):
        assert lib.qdc_row_scale_check(first, step, count.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert int(count.item()) == 0


@pytest.mark.parametrize("width,eps", [(1.0, 0.0), (256.0, 1e-6), (1000.0, 1e-6), (3.0, 1e-5)])
def test_row_scale_matches_numpy(width, eps):
    """qdc_row_scale, the scale the row kernels apply, against numpy's correctly
    rounded float32 divide, add, square root and reciprocal, bit for bit, on 4M
    random bit patterns and the boundary values (zeros, denormals, 2^-96 and its
    neighbours, the largest finite value, infinities, NaN, negatives)."""
    from qdc_amd import _lib
    lib = _lib.lib()
    special = np.array([0, 0x80000000, 1, 0x007FFFFF, 0x00800000, 0x0F7FFFFF, 0x0F800000,
                        0x0F800001, 0x2F800000, 0x3F800000, 0x3F800001, 0x7F7FFFFF, 0x7F800000,
                        0xFF800000, 0x7FC00000, 0xBF800000, 0x358637BD], dtype=np.uint32)
    bits = np.random.default_rng(11).integers(0, 1 << 32, size=1 << 22, dtype=np.uint64)
    x = np.concatenate([special, bits.astype(np.uint32)]).view(np.float32)
    with np.errstate(all="ignore"):
        exp = np.float32(1) / np.sqrt(x / np.float32(width) + np.float32(eps))
    xd = torch.from_numpy(x).to(DEV)
    out = torch.empty_like(xd)
    assert lib.qdc_row_scale(out.data_ptr(), xd.data_ptr(), x.size, width, eps,
                             torch.cuda.current_stream().cuda_stream) == 0
    got = out.cpu().numpy()
    same = (got.view(np.uint32) == exp.view(np.uint32)) | (np.isnan(got) & np.isnan(exp))
    assert same.all(), x[~same][:8]


# ------------------------------------------------------ attention prologue ----
PREP_CASES = [
    # B, S, H, KV, hd, rotary, packed [q|k|v|gate] (else q read from interleaved q||gate), offset
    (8, 2048, 8, 2, 256, 64, True, 0),     # the 0.8B-like forward: fast path, bf16 LPR 16
    (2, 200, 8, 2, 256, 64, False, 0),     # a partial 64-token tile at each sequence end
    (3, 40, 4, 1, 64, 16, True, 0),        # the plumbing shape: LPR 4 (bf16) / 8 (fp32)
    (2, 96, 4, 2, 128, 0, True, 0),        # no rotation
    (1, 37, 4, 2, 64, 16, True, 0),        # seq not a multiple of a chunk: general path
    (2, 16, 2, 1, 24, 8, False, 3),        # head_dim not a multiple of a chunk: general path
    (3, 72, 8, 2, 128, 32, True, 5),       # fast path with an offset: partial K and V tiles
    (5, 8, 4, 2, 64, 16, True, 0),         # shortest bf16 fast path: one 8-token K and V tile
    (1, 4, 2, 1, 64, 16, False, 2),        # 4 tokens: fp32 fast path (bf16: general path)
    (2, 136, 8, 2, 256, 64, True, 0),      # last K tile of 8 tokens: rows and pieces past the end skipped
    (2, 200, 4, 2, 512, 128, True, 1),     # 512-wide heads: bf16 LPR 32 (8 rows per lane group); fp32 general path
    (3, 40, 8, 2, 64, 16, True, 2),        # 8 heads: two 4-head Q row groups per token
    (2, 72, 16, 4, 128, 32, False, 0),     # 16 heads, 4 KV heads, q read out of interleaved q||gate rows
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", PREP_CASES)
def test_attention_prepare(dtype, case):
    """q, k normalised + rotated and v moved by one launch into [B, H, S, hd],
    K transposed [B, KV, hd, S] and [B, KV, S, hd], against the oracle's q/k
    norm + RoPE per sequence (positions restart at every sequence, shifted by
    the case's offset) and the v rows themselves (bit for bit)."""
    from qdc_amd import ops
    B, S, H, KV, hd, rd, packed, pos_offset = case
    T = B * S
    width = (2 * H + 2 * KV) * hd
    proj = host((T, width), 41, 1.0, dtype)
    qn, kn = host((hd,), 42, 0.02, dtype), host((hd,), 43, 0.02, dtype)
    if packed:   # [q | k | v | gate]
        qv, kv_ = proj[:, :H * hd].reshape(T, H, hd), proj[:, H * hd:(H + KV) * hd]
        vv = proj[:, (H + KV) * hd:(H + 2 * KV) * hd]
    else:        # [q0 g0 q1 g1 ... | k | v]
        qv = proj[:, :2 * H * hd].reshape(T, H, 2 * hd)[:, :, :hd]
        kv_, vv = proj[:, 2 * H * hd:(2 * H + KV) * hd], proj[:, (2 * H + KV) * hd:]
    kv_, vv = kv_.reshape(T, KV, hd), vv.reshape(T, KV, hd)
    d = dev(proj, dtype)
    if packed:
        qd = d[:, :H * hd].view(T, H, hd)
        kd, vd = d[:, H * hd:(H + KV) * hd].view(T, KV, hd), d[:, (H + KV) * hd:(H + 2 * KV) * hd].view(T, KV, hd)
    else:
        qd = d[:, :2 * H * hd].view(T, H, 2 * hd)[:, :, :hd]
        kd = d[:, 2 * H * hd:(2 * H + KV) * hd].view(T, KV, hd)
        vd = d[:, (2 * H + KV) * hd:].view(T, KV, hd)
    tables = ops.rope_tables(S + pos_offset, rd, 1e7, DEV) if rd else None
    q_out, k_t, v_out = ops.attention_prepare(qd, kd, vd, dev(qn, dtype), dev(kn, dtype), tables, rd,
                                              1e-6, B, pos_offset=pos_offset)
    torch.cuda.synchronize()
    cos, sin = O.rope_tables(S + pos_offset, rd, 1e7) if rd else (np.zeros((1, 0), np.float32),) * 2
    exp_q = O.qk_norm_rope(np.ascontiguousarray(qv), qn, cos, sin, rd, 1e-6, S, pos_offset)
    exp_k = O.qk_norm_rope(np.ascontiguousarray(kv_), kn, cos, sin, rd, 1e-6, S, pos_offset)
    got_q = back(q_out).transpose(0, 2, 1, 3).reshape(T, H, hd)
    got_k = back(k_t).transpose(0, 3, 1, 2).reshape(T, KV, hd)
    report(f"prepare q {case}", got_q, exp_q, dtype)
    report(f"prepare k {case}", got_k, exp_k, dtype)
    got_v = v_out.permute(0, 2, 1, 3).reshape(T, KV, hd)
    assert torch.equal(got_v, vd.contiguous()), case


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", [PREP_CASES[i] for i in (0, 1, 2, 4, 6, 9)])
def test_attention_prepare_kv_only(dtype, case):
    """heads = 0 (``q=None``): K transposed and V head-major only, for a query
    projected apart (final-query attention).  Bit-identical to the K and V of
    the launch with Q rows, on the fast path's K and V tiles and on the
    general path."""
    from qdc_amd import ops
    B, S, H, KV, hd, rd, packed, pos_offset = case
    T = B * S
    proj = dev(host((T, (2 * H + 2 * KV) * hd), 44, 1.0, dtype), dtype)
    qd = proj[:, :H * hd].view(T, H, hd)
    kd = proj[:, H * hd:(H + KV) * hd].view(T, KV, hd)
    vd = proj[:, (H + KV) * hd:(H + 2 * KV) * hd].view(T, KV, hd)
    qn, kn = dev(host((hd,), 45, 0.02, dtype), dtype), dev(host((hd,), 46, 0.02, dtype), dtype)
    tables = ops.rope_tables(S + pos_offset, rd, 1e7, DEV) if rd else None
    _, k_full, v_full = ops.attention_prepare(qd, kd, vd, qn, kn, tables, rd, 1e-6, B,
                                              pos_offset=pos_offset)
    none, k_t, v_out = ops.attention_prepare(None, kd, vd, None, kn, tables, rd, 1e-6, B,
                                             pos_offset=pos_offset)
    torch.cuda.synchronize()
    assert none is None
    assert torch.equal(k_t, k_full), case
    assert torch.equal(v_out, v_full), case


def test_attention_prepare_checks():
    from qdc_amd import ops
    T, H, KV, hd = 64, 4, 2, 64
    q = torch.zeros((T, H, hd), device=DEV)
    k = torch.zeros((T, KV, hd), device=DEV)
    v = torch.zeros((T, KV, hd), device=DEV)
    w = torch.zeros(hd, device=DEV)
    tables = ops.rope_tables(16, 16, 1e4, DEV)
    with pytest.raises(ValueError):     # sequences of 32 need 32 table rows
        ops.attention_prepare(q, k, v, w, w, tables, 16, 1e-6, 2)
    with pytest.raises(ValueError):     # tokens not a multiple of batch
        ops.attention_prepare(q, k, v, w, w, ops.rope_tables(64, 16, 1e4, DEV), 16, 1e-6, 3)
    with pytest.raises(ValueError):     # output overlapping an input
        out = (q.view(1, H, T, hd), torch.empty((1, KV, hd, T), device=DEV),
               torch.empty((1, KV, T, hd), device=DEV))
        ops.attention_prepare(q, k, v, w, w, ops.rope_tables(64, 16, 1e4, DEV), 16, 1e-6, 1, out=out)


# ------------------------------------------------- gather + first input norm --
GATHER_RMS_FAST_GROUPS = [2, 4, 8, 16, 32, 64, 128, 256, 320, 384, 512, 640, 768, 1024]


@pytest.mark.parametrize("groups", GATHER_RMS_FAST_GROUPS)
@pytest.mark.parametrize("table_dtype,normed", [(torch.bfloat16, "split"), (torch.float32, "split"),
                                                (torch.bfloat16, torch.float32)])
def test_gather_rms_every_fast_shape(groups, table_dtype, normed):
    """Every fast-path width of the fused gather + first norm (4 elements per
    group) for the type mixes the width table is not otherwise run with: bf16
    or fp32 table rows into the split output, and bf16 rows into an fp32 norm.
    hidden bit-exact; normed within the fp32 bar."""
    from qdc_amd import ops
    width, vocab, n = groups * 4, 97, 19
    table = host((vocab, width), 81, 0.02, torch.bfloat16)
    ids = np.random.default_rng(82).integers(0, vocab, size=n).astype(np.int32)
    split = normed == "split"
    wdt = torch.bfloat16 if split else normed
    w = host((width,), 83, 0.02, wdt)
    hidden, got = ops.native_gather_rms(dev(table, table_dtype), dev(ids, torch.int32), dev(w, wdt),
                                        1e-6, normed_dtype=ops.BF16X2 if split else None)
    rows = O.gather(table, ids)
    assert np.array_equal(back(hidden), rows)
    if split:
        got = O.join_split(got.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))
    else:
        got = back(got)
    report(f"gather_rms {table_dtype}->{normed} width={width}", got, O.rms(rows, w, 1e-6),
           torch.float32)


@pytest.mark.parametrize("table_dtype,norm_dtype", [(torch.bfloat16, torch.bfloat16),
                                                    (torch.float32, torch.float32),
                                                    (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("vocab,width,n", [(248320, 1024, 16384), (4096, 256, 129), (64, 8, 65),
                                           (100, 12, 33), (50, 1000, 7), (30, 4096, 5),
                                           (60, 512, 70), (40, 2048, 9), (45, 2560, 11),
                                           (35, 1280, 6)])
def test_gather_rms(table_dtype, norm_dtype, vocab, width, n):
    """hidden = the gathered rows widened to fp32 bit for bit; normed = their
    zero-centred RMSNorm (oracle, fp32 1e-5 / bf16 1e-2), masked rows times
    their 0/1 entry bit for bit; out-of-range device ids give zero rows and
    set the flag."""
    from qdc_amd import ops
    rng = np.random.default_rng(51)
    table = host((vocab, width), 52, 0.02, table_dtype)
    w = host((width,), 53, 0.02, norm_dtype)
    ids = rng.integers(0, vocab, size=n).astype(np.int32)
    ids[:2] = [0, vocab - 1][:min(2, n)]
    dt, dw, di = dev(table, table_dtype), dev(w, norm_dtype), dev(ids, torch.int32)
    hidden, normed = ops.native_gather_rms(dt, di, dw, 1e-6)
    torch.cuda.synchronize()
    rows = table[ids]
    assert np.array_equal(back(hidden).view(np.uint32), rows.view(np.uint32))
    report(f"gather_rms {vocab}x{width} n={n}", back(normed), O.rms(rows, w, 1e-6), norm_dtype)
    mask = (rng.random(n) > 0.3).astype(np.int32)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    h2, masked = ops.native_gather_rms(dt, di, dw, 1e-6, token_mask=dev(mask, torch.int32),
                                       error_flag=flag)
    torch.cuda.synchronize()
    assert flag.item() == 0 and torch.equal(h2, hidden)
    got, plain = back(masked), back(normed)
    assert np.array_equal(got[mask == 1].view(np.uint32), plain[mask == 1].view(np.uint32))
    assert not got[mask == 0].any()
    if n > 3:
        bad = ids.copy()
        bad[[1, n - 1]] = [vocab, -3]
        h3, n3 = ops.native_gather_rms(dt, dev(bad, torch.int32), dw, 1e-6, error_flag=flag)
        torch.cuda.synchronize()
        assert flag.item() == 1
        hb, nb = back(h3), back(n3)
        assert not hb[[1, n - 1]].any() and not nb[[1, n - 1]].any()
        keep = np.setdiff1d(np.arange(n), [1, n - 1])
        assert np.array_equal(hb[keep].view(np.uint32), rows[keep].view(np.uint32))

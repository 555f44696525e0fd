"""GPU parity of the split two-term bf16 outputs (QDC_BF16X2) of the kernels
that write GEMM inputs, through the C ABI, against the oracle.

A split output holds hi = bf16(v) and lo = bf16(v - hi) of each fp32 result v,
every aligned group of 4 elements as [4 hi | 4 lo]; hi + lo is within 2^-17
(7.6e-6) of v relative.  Bars: hi + lo within the fp32 bar (1e-5 normwise) of
the oracle's fp32 result and per element within 3e-5 relative (a missing lo
term is up to 2^-9 relative); hi equal to bf16(oracle)
except where the fp32 value sits on a rounding boundary (at most 0.1% of the
elements); rows whose result is fixed bit for bit (exact sums, zeros, inf, NaN,
denormals) equal the oracle's split form bit for bit.  The GEMM test checks
that a split row times ``ops.split_weight(w)`` is the fp32 row times ``w``.
"""
import numpy as np
import pytest
import torch

from conftest import normwise
from oracle import qdc_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF, F32 = torch.bfloat16, torch.float32


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from qdc_amd import ops  # noqa: F401  (fails loudly if the library is missing)
    yield
    torch.cuda.synchronize()


def host(shape, seed, scale=1.0, dtype=F32):
    x = (np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(scale))
    return O.round_bf16(x) if dtype == BF else x


def dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV).to(dtype)


def bits(t):
    """bf16 bit patterns of a device tensor."""
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def terms(b):
    """(hi, lo) fp32 arrays of split bit patterns [..., 2K]."""
    lead, k2 = b.shape[:-1], b.shape[-1]
    g = O.bf16_to_f32(b).reshape(*lead, k2 // 8, 2, 4)
    return g[..., 0, :].reshape(*lead, k2 // 2), g[..., 1, :].reshape(*lead, k2 // 2)


def check_split(name, got, exp):
    b = bits(got)
    assert b.shape == exp.shape[:-1] + (2 * exp.shape[-1],), (name, b.shape, exp.shape)
    dec = O.join_split(b)
    hi, _ = terms(b)
    err = normwise(dec, exp)
    flips = float(np.mean(hi != O.round_bf16(exp))) if exp.size else 0.0
    worst = float(np.max(np.abs(dec - exp) / np.maximum(np.abs(exp), 1e-30))) if exp.size else 0.0
    print(f"{name}: normwise {err:.3e} worst elementwise {worst:.2e} hi flips {flips:.1e}",
          flush=True)
    assert err <= 1e-5, (name, err)
    assert np.all(np.abs(dec - exp) <= 3e-5 * np.abs(exp) + 1e-37), name
    assert flips <= 1e-3, (name, flips)


def _same_bits_or_nan(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | ((a.view(np.uint32) == b.view(np.uint32)) & ~np.isnan(a))))


def check_split_exact(name, got, exp):
    """Bit for bit (NaN-aware) equal to the oracle's split form of ``exp``."""
    with np.errstate(all="ignore"):
        gh, gl = terms(bits(got))
        eh, el = terms(O.split_bf16(exp))
    assert _same_bits_or_nan(gh, eh), (name, "hi")
    assert _same_bits_or_nan(gl, el), (name, "lo")


# ------------------------------------------------------------------ RMSNorm --
# fast kernels (1024, 4096 over 4 wavefronts, 12), the general kernel (1000, 20)
@pytest.mark.parametrize("rows,width", [(8192, 1024), (5, 4096), (33, 12), (17, 1000), (3, 20)])
@pytest.mark.parametrize("centered", [True, False])
def test_rms_split(rows, width, centered):
    from qdc_amd import ops
    x = host((rows, width), 1)
    w = host((width,), 2, 0.02, BF)
    got = ops.native_rms(dev(x, F32), dev(w, BF), 1e-6, centered=centered, out_dtype=ops.BF16X2)
    check_split(f"rms split {rows}x{width} c={centered}", got, O.rms(x, w, 1e-6, centered))


def test_rms_split_strided_and_masked():
    """Rows of 1024 inside rows of 1040, into split rows inside wider rows; and
    the masked entry point (masked rows are exact zeros)."""
    from qdc_amd import ops
    x = host((64, 1040), 3)
    w = host((1024,), 4, 0.02, BF)
    out = torch.full((64, 2 * 1040), 7.0, dtype=BF, device=DEV)
    ops.native_rms(dev(x, F32)[:, :1024], dev(w, BF), 1e-6, out=out[:, :2048],
                   out_dtype=ops.BF16X2)
    check_split("rms split strided", out[:, :2048], O.rms(x[:, :1024], w, 1e-6))
    assert torch.all(out[:, 2048:] == 7.0)  # nothing written past the rows
    keep = (np.arange(64) % 3 != 0).astype(np.int32)
    got = ops.native_rms(dev(x[:, :1024], F32), dev(w, BF), 1e-6,
                         token_mask=torch.from_numpy(keep).to(DEV), out_dtype=ops.BF16X2)
    exp = O.rms(x[:, :1024], w, 1e-6) * keep[:, None].astype(np.float32)
    check_split("rms split masked", got, exp)
    assert np.all(O.join_split(bits(got))[keep == 0] == 0)  # masked rows: +-0


@pytest.mark.parametrize("rows,width", [(16384, 1024), (7, 1000), (9, 2048)])
@pytest.mark.parametrize("masked", [False, True])
def test_residual_rms_split(rows, width, masked):
    from qdc_amd import ops
    x = host((rows, width), 5)
    m = host((rows, width), 6)
    w = host((width,), 7, 0.02, BF)
    keep = (np.arange(rows) % 4 != 1).astype(np.int32)
    res, out = ops.native_residual_rms(dev(x, F32), dev(m, F32), dev(w, BF), 1e-6,
                                       token_mask=torch.from_numpy(keep).to(DEV) if masked
                                       else None, out_dtype=ops.BF16X2)
    exp_res, exp = O.residual_rms(x, m, w, 1e-6)
    assert np.array_equal(res.cpu().numpy(), exp_res)
    if masked:
        exp = exp * keep[:, None].astype(np.float32)
    check_split(f"residual rms split {rows}x{width} masked={masked}", out, exp)


@pytest.mark.parametrize("width", [1024, 1000, 4096])
def test_norm_special_rows_split_bit_exact(width):
    """The exactly-summable and special rows (zeros, overflow, inf, NaN,
    denormals) through the plain, residual and gated norms with split outputs:
    bit for bit the oracle's split form of its fp32 result."""
    from qdc_amd import ops
    from test_gpu_ops import _exact_rows
    x = _exact_rows(width)
    w = host((width,), 45, 0.02, BF)
    with np.errstate(all="ignore"):
        got = ops.native_rms(dev(x, F32), dev(w, BF), 1e-6, out_dtype=ops.BF16X2)
        check_split_exact("rms", got, O.rms(x, w, 1e-6))
        zero = np.zeros_like(x)
        res, out = ops.native_residual_rms(dev(x, F32), dev(zero, F32), dev(w, BF), 1e-6,
                                           out_dtype=ops.BF16X2)
        check_split_exact("residual", out, O.residual_rms(x, zero, w, 1e-6)[1])
        z = np.resize(np.array([0.0, 100.0, -100.0], np.float32), x.shape)
        got = ops.native_gated_rms(dev(x, BF).view(len(x), 1, width),
                                   dev(z, BF).view(len(x), 1, width), dev(w, BF), 1e-6,
                                   out_dtype=ops.BF16X2)
        exp = O.gated_rms(x.reshape(len(x), 1, width), z.reshape(len(x), 1, width), w, 1e-6)
        check_split_exact("gated", got.view(len(x), 2 * width), exp.reshape(x.shape))


# ------------------------------------------------------ gather + first norm --
@pytest.mark.parametrize("table_dtype", [BF, F32])
@pytest.mark.parametrize("width", [1024, 1000, 256])
def test_gather_rms_split(table_dtype, width):
    from qdc_amd import ops
    vocab, n = 4096, 777
    table = host((vocab, width), 8, 0.02, BF)
    w = host((width,), 9, 0.02, BF)
    ids = np.random.default_rng(10).integers(0, vocab, size=n).astype(np.int32)
    keep = (np.arange(n) % 5 != 2).astype(np.int32)
    hidden, normed = ops.native_gather_rms(dev(table, table_dtype), dev(ids, torch.int32),
                                           dev(w, BF), 1e-6,
                                           token_mask=torch.from_numpy(keep).to(DEV),
                                           normed_dtype=ops.BF16X2)
    h = O.gather(table, ids)
    assert np.array_equal(hidden.cpu().numpy(), h)
    check_split(f"gather rms split {table_dtype} {width}", normed,
                O.rms(h, w, 1e-6) * keep[:, None].astype(np.float32))


# -------------------------------------------------------------- gated norm --
@pytest.mark.parametrize("tokens,heads,width", [(2048, 16, 128), (37, 3, 100), (5, 2, 8)])
def test_gated_rms_split(tokens, heads, width):
    """x bf16 (the recurrence output) and z read in place inside a packed
    bf16 projection [q | z | tail] (fast at widths 128 and 8; the general
    kernel at 100, whose bf16 rows are not 16-byte multiples)."""
    from qdc_amd import ops
    x = host((tokens, heads, width), 11, 1.0, BF)
    packed = host((tokens, heads * width * 2 + 8), 12, 1.0, BF)
    w = host((width,), 13, 0.5, BF)
    pk = dev(packed, BF)
    z = pk[:, heads * width:2 * heads * width].view(tokens, heads, width)
    got = ops.native_gated_rms(dev(x, BF), z, dev(w, BF), 1e-6, out_dtype=ops.BF16X2)
    assert got.shape == (tokens, heads, 2 * width)
    zn = packed[:, heads * width:2 * heads * width].reshape(tokens, heads, width)
    exp = O.gated_rms(x, zn, w, 1e-6)
    check_split(f"gated split {tokens}x{heads}x{width}", got.view(tokens, -1),
                exp.reshape(tokens, -1))


# ------------------------------------------------------------------ SwiGLU --
@pytest.mark.parametrize("tokens,width", [(16384, 3584), (33, 1000), (4, 12)])
def test_swiglu_split(tokens, width):
    """fp32 gate and up read as the two halves of the packed gate||up GEMM output."""
    from qdc_amd import ops
    packed = host((tokens, 2 * width), 14, 2.0)
    pk = dev(packed, F32)
    got = ops.native_mlp_gate(pk[:, :width], pk[:, width:], out_dtype=ops.BF16X2)
    check_split(f"swiglu split {tokens}x{width}", got,
                O.swiglu(packed[:, :width], packed[:, width:]))


def test_swiglu_split_general_and_specials():
    """Inputs one element off 16-byte alignment (the general kernel), and the
    special values of the reference's exceptional lanes (|x| beyond 80, tiny,
    inf, NaN) on the fast kernel."""
    from qdc_amd import ops
    tokens, width = 9, 64
    buf = host((tokens * 2 * width + 1,), 15, 3.0)
    g = dev(buf, F32)[1:].view(tokens, 2 * width)
    got = ops.native_mlp_gate(g[:, :width], g[:, width:], out_dtype=ops.BF16X2)
    gh = buf[1:].reshape(tokens, 2 * width)
    check_split("swiglu split general", got, O.swiglu(gh[:, :width], gh[:, width:]))
    special = np.array([0.0, -0.0, 1e-30, -1e-30, 85.0, -85.0, 100.0, -100.0, np.inf, -np.inf,
                        np.nan, 1e30], np.float32)
    gate = np.resize(special, (12, 16))
    up = np.resize(np.array([1.0, -2.0, 3.0, np.inf], np.float32), (12, 16))
    with np.errstate(all="ignore"):
        got = ops.native_mlp_gate(dev(gate, F32), dev(up, F32), out_dtype=ops.BF16X2)
        exp = O.swiglu(gate, up)
        hi, lo = terms(bits(got))
        fin = np.isfinite(exp)
        # specials: hi carries inf / NaN, lo is +0
        assert _same_bits_or_nan(hi[~fin], O.round_bf16(exp[~fin]))
        assert np.all(lo[~fin] == 0) and not np.any(np.signbit(lo[~fin]))
        dec = hi[fin] + lo[fin]
        assert np.all(np.abs(dec - exp[fin]) <= 3e-5 * np.abs(exp[fin]) + 1e-37)


# ------------------------------------------------------- attention gate merge --
@pytest.mark.parametrize("B,S,H,hd", [(8, 2048, 8, 256), (2, 5, 3, 12)])
def test_attention_gate_split(B, S, H, hd):
    """values fp32 [B, H, S, hd]; gate the bf16 gate block of a packed [q | gate]
    projection (fast at head_dim 256, general at 12)."""
    from qdc_amd import ops
    values = host((B, H, S, hd), 16)
    packed = host((B * S, 2 * H * hd), 17, 2.0, BF)
    pk = dev(packed, BF)
    gate = pk[:, H * hd:].view(B * S, H, hd)
    got = ops.attention_gate(dev(values, F32), gate, out_dtype=ops.BF16X2)
    from oracle import forward
    exp = forward.attention_gate(values, packed[:, H * hd:].reshape(B * S, H, hd))
    check_split(f"gate merge split {B}x{S}x{H}x{hd}", got, exp.reshape(B * S, H * hd))


# ------------------------------------------------------------------- GEMM ---
@pytest.mark.parametrize("k,n", [(1024, 3072), (3584, 1024)])
def test_split_rows_times_split_weight(k, n):
    """A split row times ``split_weight(w)`` (bf16 x bf16, fp32 accumulate, one
    GEMM of inner dimension 2k) is the fp32 row times ``w``: the kernels' piece
    layout and the weight's repeated rows agree."""
    from qdc_amd import ops
    rows = 256
    x = host((rows, k), 18)
    w = host((k, n), 19, 0.02, BF)
    x2 = ops.native_rms(dev(x, F32), dev(np.zeros(k, np.float32), BF), 1e-6,
                        out_dtype=ops.BF16X2)
    xs = O.rms(x, np.zeros(k, np.float32), 1e-6)
    got = torch.mm(x2, ops.split_weight(dev(w, BF)), out_dtype=torch.float32).cpu().numpy()
    exp = (xs.astype(np.float64) @ w.astype(np.float64))
    err = normwise(got, exp)
    plain = torch.mm(dev(xs, BF), dev(w, BF), out_dtype=torch.float32).cpu().numpy()
    print(f"split GEMM {k}x{n}: normwise {err:.2e} (plain bf16 input {normwise(plain, exp):.2e})",
          flush=True)
    assert err <= 1e-5
    # join_split reads the pieces back as the oracle does
    assert np.array_equal(ops.join_split(x2).cpu().numpy(), O.join_split(bits(x2)))

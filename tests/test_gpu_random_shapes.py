"""Seeded random shapes through every fused row kernel's GPU parity test.

The hand-picked cases of ``test_gpu_ops.py`` and ``test_gpu_split.py`` cover
the benchmark shapes, each fast-path width and the known edge cases; this file
draws further valid shapes from a fixed seed (widths small and odd, around the
fast-path widths and up to 6000; row counts up to a few hundred; strides,
offsets, head layouts, masks, output types) and runs them through the same
test bodies, so each case is checked against the oracle at the same bars
(fp32 1e-5, bf16 1e-2, split outputs 1e-5, gathers and moved values bit-exact).
The case list is fixed for a given count: a failure names a reproducible case.
"""
import os

import numpy as np
import pytest
import torch

import test_gpu_ops as G
import test_gpu_split as GS

pytestmark = pytest.mark.gpu

F32, BF = torch.float32, torch.bfloat16
# cases per kernel (QDC_RANDOM_CASES widens the sweep: 80 per kernel, 2240 cases, all pass)
N = int(os.environ.get("QDC_RANDOM_CASES", "20"))


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from qdc_amd import ops  # noqa: F401  (fails loudly if the library is missing)
    yield
    torch.cuda.synchronize()


def _width(rng, quantum=1, top=6000):
    """Small, medium or large, a multiple of `quantum` half of the time."""
    mid = min(1200, top)
    ranges = [(1, 41), (41, mid)] + ([(1200, top)] if top > 1200 else [])
    lo, hi = ranges[int(rng.integers(0, len(ranges)))]
    w = int(rng.integers(lo, hi))
    if quantum > 1 and rng.random() < 0.5:
        w = max(quantum, w // quantum * quantum)
    return w


def _cases(seed, make):
    rng = np.random.default_rng(seed)
    return [make(rng) for _ in range(N)]


# ------------------------------------------------------------------ norms ---
RMS = _cases(101, lambda r: (int(r.integers(1, 300)), _width(r, 8), bool(r.random() < 0.5)))


@pytest.mark.parametrize("dtype", [F32, BF])
@pytest.mark.parametrize("rows,width,centered", RMS)
def test_random_rmsnorm(dtype, rows, width, centered):
    G.test_rmsnorm(dtype, rows, width, centered)


RES = _cases(102, lambda r: (int(r.integers(1, 300)), _width(r, 8)))


@pytest.mark.parametrize("dtype", [F32, BF])
@pytest.mark.parametrize("rows,width", RES)
def test_random_residual_rmsnorm(dtype, rows, width):
    G.test_residual_rmsnorm(dtype, rows, width)


MIX = _cases(103, lambda r: (int(r.integers(1, 300)), _width(r, 4),
                             [BF, F32][int(r.integers(0, 2))], [BF, F32][int(r.integers(0, 2))]))


@pytest.mark.parametrize("rows,width,mixed_dtype,out_dtype", MIX)
def test_random_residual_rmsnorm_fp32_stream(rows, width, mixed_dtype, out_dtype):
    G.test_residual_rmsnorm_fp32_stream(mixed_dtype, out_dtype, rows, width)


MASK = _cases(104, lambda r: (int(r.integers(1, 200)), _width(r, 8, 3000),
                              [(F32, F32), (BF, BF), (F32, BF)][int(r.integers(0, 3))]))


@pytest.mark.parametrize("rows,width,types", MASK)
def test_random_masked_norms(rows, width, types):
    G.test_masked_norms(types[0], types[1], rows, width)


GATED = _cases(105, lambda r: (int(r.integers(1, 200)), int(r.integers(1, 20)),
                               _width(r, 8, 600)))


@pytest.mark.parametrize("dtype", [F32, BF])
@pytest.mark.parametrize("tokens,heads,width", GATED)
def test_random_gated_rmsnorm(dtype, tokens, heads, width):
    G.test_gated_rmsnorm(dtype, tokens, heads, width)


# ------------------------------------------------------------- SwiGLU, gather --
SWI = _cases(106, lambda r: (int(r.integers(1, 200)), _width(r, 8)))


@pytest.mark.parametrize("dtype", [F32, BF])
@pytest.mark.parametrize("tokens,width", SWI)
def test_random_swiglu(dtype, tokens, width):
    G.test_swiglu(dtype, tokens, width)


GATHER = _cases(107, lambda r: (int(r.integers(1, 3000)), _width(r, 8, 3000),
                                int(r.integers(1, 400))))


@pytest.mark.parametrize("types", [(BF, BF), (BF, F32), (F32, F32)])
@pytest.mark.parametrize("vocab,hidden,n", GATHER)
def test_random_gather(types, vocab, hidden, n):
    G.test_gather_bit_exact(types[0], types[1], vocab, hidden, n)


GRMS = _cases(108, lambda r: (int(r.integers(5, 2000)), _width(r, 8, 4200),
                              int(r.integers(1, 300))))


@pytest.mark.parametrize("types", [(BF, BF), (F32, F32), (F32, BF)])
@pytest.mark.parametrize("vocab,width,n", GRMS)
def test_random_gather_rms(types, vocab, width, n):
    G.test_gather_rms(types[0], types[1], vocab, width, n)


# --------------------------------------------------------------- q/k + RoPE --
def _qk_case(r):
    hd = 2 * int(r.integers(1, 160))
    rd = 2 * int(r.integers(0, hd // 2 + 1))
    T = int(r.integers(1, 300))
    return (T, int(r.integers(1, 9)), int(r.integers(1, 5)), hd, rd, int(r.integers(1, T + 1)),
            float(r.choice([1e4, 1e6, 1e7])))


QK = _cases(109, _qk_case)


@pytest.mark.parametrize("dtype", [F32, BF])
@pytest.mark.parametrize("case", QK)
def test_random_qk_norm_rope(dtype, case):
    G.test_qk_norm_rope(dtype, case)


def _prep_case(r):
    hd = int(r.choice([4, 8, 16, 24, 32, 64, 96, 128, 256]))
    KV = int(r.integers(1, 4))
    return (int(r.integers(1, 5)), int(r.integers(1, 150)), KV * int(r.integers(1, 5)), KV, hd,
            2 * int(r.integers(0, hd // 2 + 1)), bool(r.random() < 0.5), int(r.integers(0, 9)))


PREP = _cases(110, _prep_case)


@pytest.mark.parametrize("dtype", [F32, BF])
@pytest.mark.parametrize("case", PREP)
def test_random_attention_prepare(dtype, case):
    G.test_attention_prepare(dtype, case)


# ---------------------------------------------------------- attention, DeltaNet --
def _softmax_case(r):
    K = _width(r, 4, 36000)
    Q = int(r.integers(1, 24))
    return (int(r.integers(1, 3)), int(r.integers(1, 4)), Q, K, int(r.integers(0, K + 1)),
            str(r.choice(["rand", "none", "dead"])))


SOFTMAX = _cases(111, _softmax_case)


@pytest.mark.parametrize("out_dtype", [F32, BF])
@pytest.mark.parametrize("case", SOFTMAX)
def test_random_attention_softmax(out_dtype, case):
    if case[5] == "dead" and case[0] < 2:  # the "dead" rows are drawn in the second sequence
        case = (2,) + case[1:]
    G.test_attention_softmax(out_dtype, case)


GATE = _cases(112, lambda r: (int(r.integers(1, 4)), int(r.integers(1, 100)),
                              int(r.integers(1, 10)), _width(r, 8, 300)))


@pytest.mark.parametrize("dtype", [F32, BF])
@pytest.mark.parametrize("B,S,H,hd", GATE)
def test_random_attention_gate(dtype, B, S, H, hd):
    G.test_attention_gate(dtype, B, S, H, hd)


def _prologue_case(r):
    KH = int(r.integers(1, 5))
    kd = int(r.choice([2, 6, 8, 16, 32, 64, 96, 128]))
    return (int(r.integers(1, 4)), int(r.integers(1, 90)), KH, kd, KH * int(r.integers(1, 4)),
            int(r.choice([2, 8, 16, 40, 64, 128])), int(r.choice([3, 4, 4, 4])),
            int(r.choice([0, 0, 1, 8])))


PROLOGUE = _cases(113, _prologue_case)


@pytest.mark.parametrize("dtype", [F32, BF])
@pytest.mark.parametrize("case", PROLOGUE)
def test_random_delta_prologue(dtype, case):
    G.test_delta_prologue(dtype, case)


# ------------------------------------------------------------ split outputs --
SPLIT_RMS = _cases(114, lambda r: (int(r.integers(1, 300)), _width(r, 4) // 4 * 4 or 4,
                                   bool(r.random() < 0.5)))


@pytest.mark.parametrize("rows,width,flag", SPLIT_RMS)
def test_random_split_norms(rows, width, flag):
    GS.test_rms_split(rows, width, flag)
    GS.test_residual_rms_split(rows, width, flag)


SPLIT_OTHER = _cases(115, lambda r: (int(r.integers(1, 150)), int(r.integers(1, 12)),
                                     (_width(r, 8, 800) // 4 * 4) or 4))


@pytest.mark.parametrize("tokens,heads,width", SPLIT_OTHER)
def test_random_split_gated_swiglu_gate(tokens, heads, width):
    GS.test_gated_rms_split(tokens, heads, width)
    GS.test_swiglu_split(tokens, width)
    GS.test_attention_gate_split(1, tokens, heads, width)

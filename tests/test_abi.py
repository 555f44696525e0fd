"""C-ABI checks that need no GPU: the library loads, exports every entry point
declared in include/qdc_hip.h, and rejects bad arguments on the host (with the
documented status) before anything would be enqueued.  Only calls that fail
validation are made, so no kernel is ever launched here."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from oracle import qdc_oracle as O
from qdc_amd import _lib

HEADER = os.path.join(ROOT, "include", "qdc_hip.h")
F32, BF16, X2 = _lib.QDC_F32, _lib.QDC_BF16, _lib.QDC_BF16X2
NULL_S = None
FAKE = 0x10000  # a non-null, 16-byte aligned address never dereferenced by validation


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(qdc_\w+)\s*\(", text, re.M)))


def test_exports_match_header():
    lib = _lib.lib()
    names = declared()
    assert len(names) == 26, names
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, name
    assert set(_lib.SIGNATURES) == set(names)
    assert _lib.version().startswith("qdc_hip ")


def test_version_matches_the_header():
    """qdc_version() is the QDC_HIP_VERSION of the header the library was built
    from (0.2.0: out_dtype added to qdc_gated_rmsnorm and qdc_swiglu; 0.2.1:
    qdc_row_scale and qdc_row_scale_check added; 0.3.0: q/k and v row strides
    added to qdc_delta_prologue and qdc_delta_scan; 0.3.1: qdc_copy_pair added)."""
    m = re.search(r'#define\s+QDC_HIP_VERSION\s+"([^"]+)"', open(HEADER).read())
    assert m and re.fullmatch(r"qdc_hip \d+\.\d+\.\d+", m.group(1))
    assert _lib.version() == m.group(1) == "qdc_hip 0.3.1"


def test_status_strings():
    for code, name in _lib.STATUS.items():
        assert _lib.status_string(code)
    assert "NULL" in _lib.status_string(-1)


def test_rope_tables_match_oracle_bitwise():
    for n_pos, rd, theta in ((2048, 64, 1e7), (128, 16, 1e7), (65, 4, 1e4), (7, 2, 10.0)):
        cos = np.empty((n_pos, rd // 2), np.float32)
        sin = np.empty((n_pos, rd // 2), np.float32)
        assert _lib.lib().qdc_rope_tables(cos.ctypes.data, sin.ctypes.data, n_pos, rd, theta) == 0
        oc, os_ = O.rope_tables(n_pos, rd, theta)
        assert np.array_equal(cos, oc) and np.array_equal(sin, os_)
    lib = _lib.lib()
    assert lib.qdc_rope_tables(None, None, 4, 3, 1e4) == -2
    assert lib.qdc_rope_tables(None, None, 4, 4, 1e4) == -1
    assert lib.qdc_rope_tables(None, None, 0, 4, 1e4) == 0


def test_check_ids():
    lib = _lib.lib()
    ids = np.array([0, 5, 4095], np.int64)
    assert lib.qdc_check_ids(ids.ctypes.data, 3, 4096) == 0
    assert lib.qdc_check_ids(ids.ctypes.data, 3, 4095) == -4
    neg = np.array([3, -1], np.int64)
    assert lib.qdc_check_ids(neg.ctypes.data, 2, 10) == -4
    assert lib.qdc_check_ids(None, 0, 10) == 0
    assert lib.qdc_check_ids(None, 2, 10) == -1


def test_rmsnorm_validation():
    lib = _lib.lib()
    rms = lambda *a: lib.qdc_rmsnorm(*a, None)  # noqa: E731
    assert rms(FAKE, FAKE, FAKE, 4, 8, 8, 8, 1e-6, 1, 7, F32) == -3
    assert rms(FAKE, FAKE, FAKE, 4, 8, 8, 8, 1e-6, 1, BF16, F32) == -3  # bf16 -> f32 not offered
    assert rms(FAKE, FAKE, FAKE, -1, 8, 8, 8, 1e-6, 1, F32, F32) == -2
    assert rms(FAKE, FAKE, FAKE, 4, 8, 4, 8, 1e-6, 1, F32, F32) == -2  # ld < width
    assert rms(None, FAKE, FAKE, 4, 8, 8, 8, 1e-6, 1, F32, F32) == -1
    assert rms(FAKE, FAKE, None, 4, 8, 8, 8, 1e-6, 1, BF16, BF16) == -1
    assert rms(None, None, None, 0, 8, 8, 8, 1e-6, 1, F32, F32) == 0  # nothing to do
    assert rms(FAKE + 16, FAKE, FAKE, 4, 8, 8, 8, 1e-6, 1, F32, F32) == -5  # partial overlap
    assert rms(FAKE, FAKE, FAKE, 4, 8, 8, 16, 1e-6, 1, F32, F32) == -5  # in place, other stride
    assert rms(FAKE, FAKE, FAKE, 4, 8, 8, 8, 1e-6, 1, F32, BF16) == -5  # in place, other type
    # up to a wavefront per row in a grid of fewer than 2^32 work-items: rows < 2^26
    assert rms(FAKE, FAKE * 2, FAKE, 1 << 26, 8, 8, 8, 1e-6, 1, F32, F32) == -2
    assert rms(FAKE, FAKE * 2, FAKE, 4, 8, 8, 8, 1e-6, 1, F32, F32) == -5  # out on the weight
    # the split output: fp32 rows only, whole groups of 4, never in place
    assert rms(FAKE, FAKE * 2, FAKE * 3, 4, 8, 8, 8, 1e-6, 1, BF16, X2) == -3
    assert rms(FAKE, FAKE * 2, FAKE * 3, 4, 6, 6, 6, 1e-6, 1, F32, X2) == -2
    assert rms(FAKE, FAKE * 2, FAKE * 3, 4, 8, 8, 10, 1e-6, 1, F32, X2) == -2
    assert rms(FAKE, FAKE, FAKE * 3, 4, 8, 8, 8, 1e-6, 1, F32, X2) == -5
    assert rms(FAKE, FAKE * 2, FAKE * 3, 0, 8, 8, 8, 1e-6, 1, F32, X2) == 0


def test_residual_validation():
    lib = _lib.lib()
    f = lambda *a: lib.qdc_residual_rmsnorm(*a, None)  # noqa: E731
    A, B, C, D, W = FAKE, FAKE * 2, FAKE * 3, FAKE * 4, FAKE * 5
    assert f(A, B, C, D, W, 4, 8, 1e-6, 9, F32, F32) == -3
    assert f(A, B, C, D, W, 4, 8, 1e-6, BF16, F32, F32) == -3  # bf16 stream, f32 addend
    assert f(A, B, C, D, W, 4, 8, 1e-6, BF16, BF16, F32) == -3  # bf16 stream, f32 output
    assert f(A, B, C, None, W, 4, 8, 1e-6, F32, F32, F32) == -1
    assert f(A, A, C, D, W, 4, 8, 1e-6, F32, F32, F32) == -5  # residual and out coincide
    assert f(A, B, A + 4, D, W, 4, 8, 1e-6, F32, F32, F32) == -5  # residual overlaps x partially
    assert f(A, B, C, B, W, 4, 8, 1e-6, F32, BF16, F32) == -5  # out on mixed of another type
    assert f(A, B, C, D, W, 0, 8, 1e-6, F32, F32, F32) == 0
    assert f(A, B, C, D, W, 1 << 26, 8, 1e-6, F32, F32, F32) == -2  # rows < 2^26
    assert f(A, B, C, D, A + 8, 4, 8, 1e-6, F32, F32, F32) == -5  # weight inside residual
    # the split output: fp32 residual and addend, whole groups of 4, not in place
    assert f(A, B, C, D, W, 4, 8, 1e-6, F32, BF16, X2) == -3
    assert f(A, B, C, D, W, 4, 8, 1e-6, BF16, BF16, X2) == -3
    assert f(A, B, C, D, W, 4, 6, 1e-6, F32, F32, X2) == -2
    assert f(A, C, C, D, W, 4, 8, 1e-6, F32, F32, X2) == -5  # out on x
    assert f(A, B, C, D, W, 0, 8, 1e-6, F32, F32, X2) == 0


def test_masked_norm_validation():
    """The masked entry points validate like the unmasked ones, require the
    mask, and refuse a mask that overlaps an output."""
    lib = _lib.lib()
    rms = lambda *a: lib.qdc_rmsnorm_masked(*a, None)  # noqa: E731
    K = FAKE * 8
    assert rms(FAKE, FAKE, FAKE, K, 4, 8, 8, 8, 1e-6, 1, 7, F32) == -3
    assert rms(FAKE, FAKE, FAKE, None, 4, 8, 8, 8, 1e-6, 1, F32, F32) == -1  # mask required
    assert rms(None, None, None, None, 0, 8, 8, 8, 1e-6, 1, F32, F32) == 0  # nothing to do
    assert rms(FAKE, FAKE * 2, FAKE * 3, FAKE + 16, 4, 8, 8, 8, 1e-6, 1, F32, F32) == -5
    assert rms(FAKE, FAKE * 2, FAKE * 3, K, 1 << 26, 8, 8, 8, 1e-6, 1, F32, F32) == -2
    f = lambda *a: lib.qdc_residual_rmsnorm_masked(*a, None)  # noqa: E731
    A, B, C, D, W = FAKE, FAKE * 2, FAKE * 3, FAKE * 4, FAKE * 5
    assert f(A, B, C, D, W, None, 4, 8, 1e-6, F32, F32, F32) == -1  # mask required
    assert f(A, B, C, D, W, K, 4, 8, 1e-6, BF16, F32, F32) == -3
    assert f(A, B, C, D, W, B + 8, 4, 8, 1e-6, F32, F32, F32) == -5  # mask inside out
    assert f(A, B, C, D, W, A + 8, 4, 8, 1e-6, F32, F32, F32) == -5  # mask inside residual
    assert f(A, B, C, D, W, None, 0, 8, 1e-6, F32, F32, F32) == 0
    assert f(A, B, C, D, W, K, 1 << 26, 8, 1e-6, F32, F32, F32) == -2


def test_gated_validation():
    lib = _lib.lib()
    g = lambda *a: lib.qdc_gated_rmsnorm(*a, None)  # noqa: E731
    f = lambda *a: g(*a, a[-1])  # noqa: E731  (out in the input dtype)
    A, X, Z, W = FAKE, FAKE * 2, FAKE * 3, FAKE * 4
    assert f(A, X, Z, W, 4, 2, 8, 16, 16, 16, 1e-6, 3) == -3
    assert f(A, X, Z, W, 4, 2, 8, 8, 16, 16, 1e-6, F32) == -2  # token stride < heads*width
    assert f(A, X, None, W, 4, 2, 8, 16, 16, 16, 1e-6, F32) == -1
    assert f(Z, X, Z, W, 4, 2, 8, 16, 16, 16, 1e-6, F32) == -5  # out on z
    assert f(W, X, Z, W, 4, 2, 8, 16, 16, 16, 1e-6, F32) == -5  # out on the weight
    assert f(A, X, Z, W, 0, 2, 8, 16, 16, 16, 1e-6, F32) == 0
    assert f(A, X, Z, W, 1 << 25, 2, 8, 16, 16, 16, 1e-6, F32) == -2  # tokens * heads < 2^26
    # the split output: bf16 inputs only, whole groups of 4 per row
    assert g(A, X, Z, W, 4, 2, 8, 16, 16, 16, 1e-6, F32, X2) == -3
    assert g(A, X, Z, W, 4, 2, 8, 16, 16, 16, 1e-6, BF16, F32) == -3
    assert g(A, X, Z, W, 4, 2, 6, 12, 12, 12, 1e-6, BF16, X2) == -2  # width 6
    assert g(A, X, Z, W, 4, 2, 8, 16, 16, 18, 1e-6, BF16, X2) == -2  # token stride 18
    assert g(X, X, Z, W, 4, 2, 8, 16, 16, 16, 1e-6, BF16, X2) == -5  # in place, other type
    assert g(A, X, Z, W, 0, 2, 8, 16, 16, 16, 1e-6, BF16, X2) == 0


def test_swiglu_validation():
    lib = _lib.lib()
    g = lambda *a: lib.qdc_swiglu(*a, None)  # noqa: E731
    f = lambda *a: g(*a, a[-1])  # noqa: E731  (out in the input dtype)
    O_, G, U = FAKE, FAKE * 2, FAKE * 3
    assert f(O_, G, U, 4, 8, 8, 8, 8, 5) == -3
    assert g(O_, G, U, 4, 8, 8, 8, 8, F32, BF16) == -3  # no f32 -> bf16
    assert g(O_, G, U, 4, 8, 8, 8, 8, BF16, X2) == -3  # split output from f32 only
    assert g(O_, G, U, 4, 6, 6, 6, 6, F32, X2) == -2  # width 6: not whole groups
    assert g(O_, G, U, 4, 8, 16, 16, 10, F32, X2) == -2  # output stride 10
    assert g(G, G, U, 4, 8, 8, 8, 8, F32, X2) == -5  # in place, other type
    assert g(O_, G, U, 0, 8, 8, 8, 8, F32, X2) == 0
    assert f(O_, G, U, 4, 8, 4, 8, 8, F32) == -2
    assert f(O_, None, U, 4, 8, 8, 8, 8, F32) == -1
    assert f(G + 4, G, U, 4, 8, 8, 8, 8, F32) == -5
    assert f(G, G, U, 4, 8, 8, 8, 16, F32) == -5  # in place with another stride
    assert f(O_, G, U, 4, 0, 8, 8, 8, F32) == 0


def test_gather_validation():
    lib = _lib.lib()
    f = lambda *a: lib.qdc_embedding_gather(*a, None, None)  # noqa: E731
    O_, T, I = FAKE, FAKE * 2, FAKE * 3
    assert f(O_, BF16, T, F32, I, 4, 16, 8) == -3  # f32 -> bf16 is not a copy
    assert f(O_, F32, T, 9, I, 4, 16, 8) == -3
    assert f(O_, F32, T, F32, None, 4, 16, 8) == -1
    assert f(O_, F32, T, F32, I, -4, 16, 8) == -2
    assert f(O_, F32, T, F32, I, 4, 0, 8) == -4
    assert f(T + 64, F32, T, F32, I, 4, 16, 8) == -5  # output inside the table
    assert f(O_, F32, T, F32, I, 0, 16, 8) == 0


def test_qk_norm_rope_validation():
    lib = _lib.lib()
    Q, K, QI, KI, QN, KN, C, S = (FAKE * i for i in range(1, 9))

    def f(tokens=8, heads=2, kv=1, hd=16, rd=8, seq=8, off=0, tl=8,
          qs=(64, 32, 32, 16), ks=(16, 16, 16, 16), dtype=F32, q=Q, k=K, qi=QI, ki=KI, c=C):
        return lib.qdc_qk_norm_rope(q, k, qi, ki, QN, KN, c, S, tokens, heads, kv, hd, rd, seq,
                                    off, tl, *qs, *ks, 1e-6, dtype, None)
    assert f(dtype=4) == -3
    assert f(rd=7) == -2
    assert f(rd=32) == -2  # rotary > head_dim
    assert f(seq=0) == -2
    assert f(tl=7) == -4  # position 7 is outside a 7-row table
    assert f(off=1) == -4
    assert f(c=None) == -1
    assert f(qs=(64, 8, 32, 16)) == -2  # head stride < head_dim
    assert f(q=KI) == -5  # q output on the k input
    assert f(k=Q + 32) == -5  # the two outputs overlap
    assert f(tokens=0) == 0
    # q rows + k rows < 2^26 (up to a wavefront per row, fewer than 2^32 work-items)
    assert f(tokens=1 << 24, kv=2, ks=(32, 16, 32, 16)) == -2


def test_qk_norm_rope_batched_validation():
    """Output strides per sequence: rows of a tensor may not overlap, an
    output may replace its input only row for row, and sequences laid out
    head-major per sequence ([batch, heads, seq, head_dim]) are accepted."""
    lib = _lib.lib()
    Q, K, QI, KI, QN, KN, C, S = (FAKE * i for i in range(1, 9))
    B, L, H, KV, hd = 3, 4, 2, 1, 16
    # head-major per sequence: (seq, tok, head) strides
    qhm, khm = (H * L * hd, hd, L * hd), (KV * L * hd, hd, L * hd)

    def f(tokens=B * L, qs=(2 * H * hd, 2 * hd) + qhm, ks=(hd, hd) + khm, q=Q, k=K, qi=QI,
          ki=KI, seq=L, dtype=F32):
        return lib.qdc_qk_norm_rope_batched(q, k, qi, ki, QN, KN, C, S, tokens, H, KV, hd, 8, seq,
                                            0, L, *qs, *ks, 1e-6, dtype, None)
    # a grid that would launch is not called here: only rejected layouts
    assert f(dtype=4) == -3
    assert f(qs=(2 * H * hd, 2 * hd, H * L * hd - 1, hd, L * hd)) == -2  # sequences overlap
    assert f(qs=(2 * H * hd, 2 * hd, H * L * hd, hd, hd)) == -2  # heads overlap tokens
    assert f(ks=(hd, hd, 0, hd, L * hd)) == -2  # every sequence on the first
    assert f(k=Q + 4 * (H * L * hd - 1)) == -5  # k output inside the q output
    assert f(q=QI) == -5  # not the same rows as the input: rejected in place
    assert f(tokens=0) == 0
    # partial last sequence: the q output's extent ends at the last head of its last
    # sequence's third token; a k output starting one element before that end overlaps
    T = 2 * L + 3
    far = max(2 * qhm[0] + 2 * qhm[1], qhm[0] + (L - 1) * qhm[1]) + (H - 1) * qhm[2] + hd
    assert f(tokens=T, k=Q + 4 * (far - 1)) == -5
    # the flat entry point's checks agree with a sequence stride of seq_len * token stride
    flat = lib.qdc_qk_norm_rope(Q, K, QI, KI, QN, KN, C, S, B * L, H, KV, hd, 8, L, 0, L,
                                2 * H * hd, 2 * hd, hd, B * L * hd - 1, hd, hd, hd, hd,
                                1e-6, F32, None)
    assert flat == -2  # q heads overlap (head stride below the token span)


def test_delta_scan_validation():
    lib = _lib.lib()
    f = lambda *a: lib.qdc_delta_scan(*a, None)  # noqa: E731
    P = FAKE
    # ..., batch, seq, heads, key_heads, key_dim, value_dim, ld_qk, ld_v
    assert f(P, 7, P, P, P, P, P, 1, 4, 2, 1, 128, 128, 128, 256) == -3
    assert f(P, F32, P, P, P, P, P, 1, 4, 3, 2, 128, 128, 256, 384) == -2  # heads not a multiple
    assert f(P, F32, P, P, P, P, P, 1, 4, 2, 1, 320, 128, 320, 256) == -2  # key_dim above 256
    assert f(P, F32, P, P, P, P, P, 1, 4, 2, 1, 128, 128, 127, 256) == -2  # q/k rows too short
    assert f(P, F32, P, P, P, P, P, 1, 4, 2, 1, 128, 128, 128, 255) == -2  # v rows too short
    assert f(P, F32, P, None, P, P, P, 1, 4, 2, 1, 128, 128, 512, 512) == -1
    assert f(None, F32, None, None, None, None, None, 0, 4, 2, 1, 128, 128, 128, 256) == 0


@pytest.mark.timeout(300)
def test_fastdiv_exhaustive(tmp_path):
    """The multiply-high division used for row/token indexing, compiled for the
    host from the same header, against integer division."""
    src = tmp_path / "fastdiv_check.cpp"
    src.write_text(r'''
#include "qdc_common.hpp"
#include <cstdio>
#include <random>
int main() {
    std::mt19937_64 rng(1);
    uint32_t divisors[4096]; int nd = 0;
    for (uint32_t d = 1; d <= 2100; ++d) divisors[nd++] = d;
    for (int k = 2; k <= 31; ++k) for (int e = -2; e <= 2; ++e) {
        long long d = (1ll << k) + e; if (d >= 1 && d <= (1ll << 31)) divisors[nd++] = (uint32_t)d; }
    const uint32_t extra[] = {448, 3584, 16384, 81920, 262144, 248320, 2147483647u};
    for (uint32_t d : extra) divisors[nd++] = d;
    long long checked = 0;
    for (int i = 0; i < nd; ++i) {
        const uint32_t d = divisors[i];
        const qdc::FastDiv f = qdc::make_fastdiv(d);
        auto one = [&](uint32_t n) {
            if (n > 0x7fffffffu) return true;
            ++checked;
            return qdc::fastdiv(n, f) == n / d;
        };
        const uint32_t edge[] = {0u, 1u, d - 1, d, d + 1, 2 * d - 1, 2 * d, 0x7fffffffu,
                                 0x7fffffffu - 1, (0x7fffffffu / d) * d, (0x7fffffffu / d) * d - 1};
        for (uint32_t n : edge) if (!one(n)) { printf("FAIL d=%u n=%u\n", d, n); return 1; }
        for (int r = 0; r < 20000; ++r) {
            const uint32_t n = (uint32_t)(rng() & 0x7fffffffu);
            if (!one(n)) { printf("FAIL d=%u n=%u\n", d, n); return 1; }
        }
    }
    printf("ok %lld\n", checked);
    return 0;
}
''')
    exe = tmp_path / "fastdiv_check"
    inc = os.path.join(ROOT, "qwendecisioncore.jl_amd", "csrc")
    subprocess.run(["/opt/rocm/bin/hipcc", "-O2", "-std=c++17", f"-I{inc}",
                    f"-I{os.path.join(ROOT, 'include')}", str(src), "-o", str(exe)],
                   check=True, capture_output=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=240)
    assert run.returncode == 0 and run.stdout.startswith("ok"), run.stdout


def test_delta_prologue_validation():
    lib = _lib.lib()
    # q, k, v, beta, decay, proj, dtype, ld, conv, taps, a_decay, dt_bias, tokens, seq,
    # kh, kd, vh, vd, ld_qk, ld_v: kh=1 kd=8 vh=2 vd=8 -> qkv 32 channels, row width
    # 32 + 16 + 4 = 52; separate q, k [16, 8] and v [16, 16] outputs
    pro = lambda *a: lib.qdc_delta_prologue(*a, None)  # noqa: E731
    ok = (FAKE, FAKE + 4096, FAKE + 8192, FAKE + 12288, FAKE + 16384, FAKE + 65536, F32, 52,
          FAKE + 131072, 4, FAKE, FAKE, 16, 8, 1, 8, 2, 8, 8, 16)

    def call(**kw):
        args = list(ok)
        names = ["q", "k", "v", "beta", "decay", "proj", "dtype", "ld", "conv", "taps",
                 "a_decay", "dt_bias", "tokens", "seq", "kh", "kd", "vh", "vd", "ld_qk", "ld_v"]
        for key, val in kw.items():
            args[names.index(key)] = val
        return pro(*args)

    assert call(dtype=5) == -3
    assert call(ld=51) == -2                 # narrower than q|k|v|z|a|b
    assert call(seq=0) == -2
    assert call(taps=0) == -2
    assert call(kd=0) == -2
    assert call(tokens=-1) == -2
    assert call(tokens=1 << 26) == -2
    assert call(q=None) == -1
    assert call(conv=None) == -1
    assert call(tokens=0, q=None, proj=None) == 0
    assert call(v=FAKE + 65536 + 64) == -5   # output inside the projection
    assert call(ld_qk=7) == -2               # q/k rows narrower than kh*kd
    assert call(ld_v=15) == -2               # v rows narrower than vh*vd
    # one [16, q|k|v] buffer of 32-float rows: q, k, v its column blocks
    assert call(k=FAKE + 28, v=FAKE + 64, ld_qk=32, ld_v=32) == -5  # k overlaps q's columns
    assert call(k=FAKE + 32, v=FAKE + 64, ld_qk=32, ld_v=24) == -5  # v rows share q's memory
    assert call(k=FAKE + 32, v=FAKE + 96, ld_qk=32, ld_v=32) == -5  # v wraps into the next row
    assert call(k=FAKE, ld_qk=8) == -5       # k is q


def test_attention_softmax_validation():
    lib = _lib.lib()
    # probs, dtype, scores, mask, batch, heads, queries, keys, q_offset, scale
    sm = lambda *a: lib.qdc_attention_softmax(*a, None)  # noqa: E731
    assert sm(FAKE, 7, FAKE + 65536, None, 1, 2, 8, 8, 0, 0.5) == -3
    assert sm(FAKE, F32, FAKE + 65536, None, 1, -2, 8, 8, 0, 0.5) == -2
    assert sm(FAKE, F32, FAKE + 65536, None, 1, 2, 8, 8, -1, 0.5) == -2
    assert sm(FAKE, F32, FAKE + 65536, None, 1 << 20, 64, 1, 8, 0, 0.5) == -2  # 2^26 rows
    assert sm(None, F32, FAKE, None, 1, 2, 8, 8, 0, 0.5) == -1
    assert sm(None, F32, None, None, 0, 2, 8, 8, 0, 0.5) == 0
    assert sm(FAKE, BF16, FAKE, None, 1, 2, 8, 8, 0, 0.5) == -5     # in place needs fp32
    assert sm(FAKE + 64, F32, FAKE, None, 1, 2, 8, 8, 0, 0.5) == -5  # partial overlap
    assert sm(FAKE, F32, FAKE + 65536, FAKE + 16, 1, 2, 8, 8, 0, 0.5) == -5  # writes the mask


def test_attention_prepare_validation():
    lib = _lib.lib()
    ins = [FAKE + (1 + i) * 65536 for i in range(3)]        # q_in, k_in, v_in
    outs = [FAKE + (4 + i) * 65536 for i in range(3)]       # q_out, k_t, v_out
    norms = [FAKE + 7 * 65536, FAKE + 7 * 65536 + 256]      # q_norm, k_norm
    tabs = [FAKE + 8 * 65536, FAKE + 9 * 65536]             # cos, sin

    def prep(heads=4, kv=2, batch=2, seq=8, dim=64, rotary=16, pos=0, table_len=8,
             q=True, k_out=True, q_out_at=None):
        qi, ki, vi = ins
        qo, ko, vo = outs
        qo = qo if q_out_at is None else q_out_at
        return lib.qdc_attention_prepare(qo if q else None, ko if k_out else None, vo,
                                         qi if q else None, ki, vi, norms[0] if q else None,
                                         norms[1], *tabs, batch, seq, heads, kv, dim, rotary, pos,
                                         table_len, 2 * heads * dim if q else 0,
                                         dim if q else 0, 2 * kv * dim, 2 * kv * dim, 1e-6, F32,
                                         None)

    assert prep(heads=-1) == -2
    assert prep(heads=3) == -2                      # not a multiple of kv_heads
    assert prep(kv=0) == -2
    assert prep(q=False, batch=0) == 0              # nothing to do
    assert prep(table_len=7) == -4                  # positions 0..7 need 8 table rows
    assert prep(q=False) == -1                      # q pointers NULL with heads > 0
    assert prep(q=False, heads=0, k_out=False) == -1
    # heads = 0: K and V only, the q pointers NULL; the range check comes after
    # the pointer checks, so reaching it shows NULL q passes
    assert prep(q=False, heads=0, table_len=7) == -4
    assert prep(q_out_at=ins[1]) == -5              # q output over the k input


def test_attention_gate_validation():
    lib = _lib.lib()
    # out, out dtype, values, gate, gate dtype, batch, seq, heads, dim, gate_tok, gate_head, out_tok
    ga = lambda *a: lib.qdc_attention_gate(*a, None)  # noqa: E731
    assert ga(FAKE, 9, FAKE + 65536, FAKE + 131072, F32, 1, 4, 2, 8, 32, 16, 16) == -3
    assert ga(FAKE, F32, FAKE + 65536, FAKE + 131072, F32, 1, 4, 0, 8, 32, 16, 16) == -2
    assert ga(FAKE, F32, FAKE + 65536, FAKE + 131072, F32, 1, 4, 2, 8, 32, 4, 16) == -2
    assert ga(FAKE, F32, FAKE + 65536, FAKE + 131072, F32, 1, 4, 2, 8, 32, 16, 8) == -2
    assert ga(None, F32, FAKE + 65536, FAKE + 131072, F32, 1, 4, 2, 8, 32, 16, 16) == -1
    assert ga(None, F32, None, None, F32, 0, 4, 2, 8, 32, 16, 16) == 0
    assert ga(FAKE + 65536 + 32, F32, FAKE + 65536, FAKE + 131072, F32, 1, 4, 2, 8, 32, 16,
              16) == -5
    # the split output: whole groups of 4 per (token, head) row
    assert ga(FAKE, X2, FAKE + 65536, FAKE + 131072, BF16, 1, 4, 2, 6, 24, 12, 12) == -2
    assert ga(FAKE, X2, FAKE + 65536, FAKE + 131072, BF16, 1, 4, 2, 8, 32, 16, 18) == -2
    assert ga(None, X2, None, None, BF16, 0, 4, 2, 8, 32, 16, 16) == 0


def test_gather_rmsnorm_validation():
    lib = _lib.lib()
    # hidden, normed, table, table dtype, ids, weight, normed dtype, mask, n, vocab, width, eps
    gr = lambda *a: lib.qdc_embedding_gather_rmsnorm(*a, None, None)  # noqa: E731
    H, N, T, I, W = (FAKE * i for i in range(1, 6))
    assert gr(H, N, T, 7, I, W, F32, None, 4, 16, 8, 1e-6) == -3
    assert gr(H, N, T, BF16, I, W, 7, None, 4, 16, 8, 1e-6) == -3
    assert gr(H, N, T, BF16, None, W, BF16, None, 4, 16, 8, 1e-6) == -1
    assert gr(H, N, T, BF16, I, W, BF16, None, 4, 0, 8, 1e-6) == -4
    assert gr(H, H + 32, T, BF16, I, W, BF16, None, 4, 16, 8, 1e-6) == -5
    assert gr(H, N, T, BF16, I, N + 4, BF16, None, 4, 16, 8, 1e-6) == -5  # weight in normed
    assert gr(H, N, T, BF16, I, W, X2, None, 4, 16, 6, 1e-6) == -2  # split: width 6
    assert gr(H, N, T, BF16, I, H + 32, X2, None, 4, 16, 8, 1e-6) == -5
    assert gr(H, N, T, BF16, I, W, X2, None, 0, 16, 8, 1e-6) == 0


def test_copy_validation():
    lib = _lib.lib()
    f = lambda *a: lib.qdc_copy(*a, None)  # noqa: E731
    assert f(FAKE, FAKE * 2, 24) == -2           # not a multiple of 16
    assert f(FAKE, FAKE * 2, -16) == -2
    assert f(FAKE + 8, FAKE * 2, 32) == -2       # misaligned destination
    assert f(None, FAKE, 32) == -1
    assert f(None, None, 0) == 0
    assert f(FAKE, FAKE + 16, 64) == -5          # overlapping
    assert f(FAKE, FAKE * 2, 1 << 37) == -2      # 2^33 chunks: grid over 2^32 work-items


def test_copy_grid_validation():
    lib = _lib.lib()
    cg = lambda *a: lib.qdc_copy_grid(*a, None)  # noqa: E731
    assert cg(FAKE, FAKE + (1 << 20), 4096, 3, 256) == -2     # chunks per thread
    assert cg(FAKE, FAKE + (1 << 20), 4096, 2, 128) == -2     # block
    assert cg(FAKE, FAKE + (1 << 20), 4100, 2, 256) == -2     # not whole chunks
    assert cg(FAKE + 8, FAKE + (1 << 20), 4096, 2, 256) == -2  # misaligned
    assert cg(None, FAKE, 4096, 4, 512) == -1
    assert cg(FAKE, FAKE + 2048, 4096, 8, 256) == -5          # overlap
    assert cg(None, None, 0, 8, 512) == 0


def test_copy_rows_validation():
    lib = _lib.lib()
    cr = lambda *a: lib.qdc_copy_rows(*a, None)  # noqa: E731
    assert cr(FAKE, FAKE, FAKE, 4, 10, 24, 1) == -2        # row bytes not a multiple of 16
    assert cr(FAKE, FAKE, FAKE, 4, 10, 32, 5) == -2        # repeat 1 to 4
    assert cr(FAKE, FAKE, FAKE, -1, 10, 32, 1) == -2
    assert cr(FAKE, FAKE, FAKE, 1 << 28, 10, 1 << 8, 1) == -2   # 2^32 chunks
    assert cr(None, FAKE, FAKE, 4, 10, 32, 1) == -1
    assert cr(FAKE, FAKE, None, 4, 10, 32, 1) == -1
    assert cr(FAKE + 8, FAKE, FAKE, 4, 10, 32, 1) == -2    # misaligned
    assert cr(FAKE, FAKE + 64, 0x900000, 4, 10, 32, 2) == -5   # dst overlaps the table
    assert cr(None, None, None, 0, 10, 32, 1) == 0


def test_copy_pair_validation():
    lib = _lib.lib()
    cp = lambda *a: lib.qdc_copy_pair(*a, None)  # noqa: E731
    A, B, C, D = FAKE, FAKE + (1 << 20), FAKE + (2 << 20), FAKE + (3 << 20)
    assert cp(A, B, 32, C, D, 16, 3, 256) == -2          # not a launch shape
    assert cp(A, B, 32, C, D, 16, 1, 128) == -2
    assert cp(A, B, 24, C, D, 16, 1, 256) == -2          # not a multiple of 16
    assert cp(A, B, 32, C, D, -16, 1, 256) == -2
    assert cp(None, B, 32, C, D, 16, 1, 256) == -1
    assert cp(A, B, 32, C, None, 16, 1, 256) == -1
    assert cp(None, None, 0, C, D, 0, 1, 256) == 0       # nothing to copy
    assert cp(A + 8, B, 32, C, D, 16, 1, 256) == -2      # misaligned
    assert cp(A, A + 16, 32, C, D, 16, 1, 256) == -5     # dst0 overlaps src0
    assert cp(A, B, 32, C, A + 16, 16, 1, 256) == -5     # src1 inside dst0
    assert cp(A, B, 32, A + 16, D, 16, 1, 256) == -5     # the destinations overlap


def test_empty_validation():
    lib = _lib.lib()
    assert lib.qdc_empty(-1, None) == -2
    assert lib.qdc_empty(1 << 24, None) == -2
    assert lib.qdc_empty(0, None) == 0


def test_row_scale_validation():
    lib = _lib.lib()
    rs = lambda *a: lib.qdc_row_scale(*a, None)  # noqa: E731
    assert rs(FAKE, FAKE, -1, 1.0, 0.0) == -2
    assert rs(FAKE, FAKE, (1 << 32) - 256, 1.0, 0.0) == -2
    assert rs(None, FAKE, 4, 1.0, 0.0) == -1
    assert rs(FAKE, None, 4, 1.0, 0.0) == -1
    assert rs(FAKE, FAKE + 4, 4, 1.0, 0.0) == -5     # partial overlap
    assert rs(None, None, 0, 1.0, 0.0) == 0
    ck = lambda *a: lib.qdc_row_scale_check(*a, None)  # noqa: E731
    assert ck(0, -1, FAKE) == -2
    assert ck(0, (1 << 32) + 1, FAKE) == -2
    assert ck(16, (1 << 32) - 15, FAKE) == -2         # past the last pattern
    assert ck(0, 1 << 32, None) == -1
    assert ck(5, 0, FAKE) == 0


def test_c_host_program_host_only(tmp_path):
    """include/qdc_hip.h compiles as C99 with gcc, a plain C program links
    against the library, and its host-only checks (version, status strings,
    argument errors found before any launch) pass; the same program runs its
    device checks in tests/test_gpu_c_host.py."""
    src = os.path.join(ROOT, "tests", "c_host", "qdc_c_host.c")
    exe = tmp_path / "qdc_c_host"
    lib = os.path.join(ROOT, "qwendecisioncore.jl_amd", "lib")
    subprocess.run(["gcc", "-std=c99", "-O1", "-Wall", "-Wextra", "-Werror",
                    "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I" + os.path.join(ROOT, "include"), src, "-o", str(exe), "-L" + lib,
                    "-lqdc_hip", "-L/opt/rocm/lib", "-lamdhip64", "-lm", "-Wl,-rpath," + lib,
                    "-Wl,-rpath,/opt/rocm/lib"], check=True)
    r = subprocess.run([str(exe), "--host-only"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout

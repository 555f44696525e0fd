"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

Checks, per oracle function:
  * the reference's own golden data: test/fixtures/native (5 PyTorch cases of
    reference.json and 21 of cuda_reference.json) end to end at the reference's
    tolerance (atol = rtol = 2e-5, test/backbone.jl:1-34) -- covers gather, all
    RMSNorm variants, full-rotary RoPE, gated norm and SwiGLU together;
  * an independent implementation (transformers' Qwen3.5 modules) for partial
    RoPE (rotary 16 of 64 and 64 of 256, positions reset per sequence), the
    norms, SwiGLU with special values and a 2-layer backbone;
  * the bf16 known-answer tests of test/safetensors.jl:23-25;
  * the reference's q/k normalisation cases (sine ramps, special values:
    test/backbone.jl:290-312);
  * closed forms and invariants (exact scale invariance, identity rotations,
    pair-norm preservation, silu(x) - silu(-x) = x, byte-equal gathers);
  * planted mistakes: each mutant of the oracle must fail the fixture.
"""
import numpy as np
import pytest

from conftest import isapprox, normwise, ramp
from oracle import forward
from oracle import qdc_oracle as O


def fixture_logits(fx, cases=None):
    out = []
    for name, ids, mask, expected in (cases or fx["cases"]):
        got = np.stack([fx["readout"] @ forward.backbone_hidden(fx["weights"], fx["cfg"], ids[r],
                                                                mask[r])[-1]
                        for r in range(ids.shape[0])])
        out.append((name, got, expected))
    return out


def test_fixture_end_to_end(native_fixture):
    assert len(native_fixture["cases"]) == 26
    for name, got, expected in fixture_logits(native_fixture):
        assert isapprox(got, expected, 2e-5, 2e-5), (name, normwise(got, expected))


def test_fixture_input_validation(native_fixture):
    W, cfg = native_fixture["weights"], native_fixture["cfg"]
    for ids, mask in (([1, 2], [1]), ([], []), ([1, 2], [1, 2, 0]), ([64], [1]), ([-1], [1]),
                      ([1, 2], [1, 2])):
        with pytest.raises(ValueError):
            forward.backbone_hidden(W, cfg, ids, mask)


MUTANTS = {
    "rms weight not centred": ("rms", lambda x, w, eps, centered=True:
                               _np_rms(x, w, eps, not centered)),
    "residual rms eps dropped": ("residual_rms", lambda x, m, w, eps:
                                 (x + m, _np_rms(x + m, w, 0.0, True))),
    "rope sin sign": ("qk_norm_rope", lambda x, w, c, s, rd, eps, seq_len=None, pos_offset=0:
                      _orig["qk_norm_rope"](x, w, c, -s, rd, eps, seq_len, pos_offset)),
    "rope pairs interleaved": ("qk_norm_rope", lambda x, w, c, s, rd, eps, seq_len=None,
                               pos_offset=0: _np_rope_interleaved(x, w, c, s, rd, eps)),
    "residual not added": ("residual_rms", lambda x, m, w, eps: (x + m, _np_rms(x, w, eps, True))),
    "swiglu gate sigmoid only": ("swiglu", lambda g, u: (1 / (1 + np.exp(-g))).astype(np.float32) * u),
    "gated norm centred": ("gated_rms", lambda x, z, w, eps: _orig["gated_rms"](x, z, w + 1, eps)),
    "gated norm no silu": ("gated_rms", lambda x, z, w, eps: _np_rms(x, w, eps, False) * z),
    "gather off by one": ("gather", lambda t, ids: _orig["gather"](t, (np.asarray(ids) + 1) % t.shape[0])),
}
_orig = {name: getattr(O, name) for name in ("rms", "qk_norm_rope", "residual_rms", "swiglu",
                                             "gated_rms", "gather")}


def _np_rms(x, w, eps, centered):
    x = x.astype(np.float32)
    s = 1 / np.sqrt((x * x).sum(-1, keepdims=True) / np.float32(x.shape[-1]) + np.float32(eps))
    return ((x * s) * ((1 + w) if centered else w)).astype(np.float32)


def _np_rope_interleaved(x, w, c, s, rd, eps):
    y = _np_rms(x, w, eps, True)
    T = x.shape[0]
    for i in range(rd // 2):
        a, b = y[..., 2 * i].copy(), y[..., 2 * i + 1].copy()
        ci, si = c[:T, i][:, None], s[:T, i][:, None]
        y[..., 2 * i], y[..., 2 * i + 1] = a * ci - b * si, b * ci + a * si
    return y


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_fixture_catches_planted_mistakes(native_fixture, monkeypatch, mutant):
    name, fn = MUTANTS[mutant]
    monkeypatch.setattr(O, name, fn)
    # two cases with masks, holes and 65 tokens are enough to expose each mutant
    cases = [c for c in native_fixture["cases"] if c[0].startswith(("ref04", "cuda13"))]
    bad = [n for n, got, exp in fixture_logits(native_fixture, cases)
           if not isapprox(got, exp, 2e-5, 2e-5)]
    assert bad, f"planted mistake '{mutant}' went unnoticed"


def test_bf16_known_answers():
    # test/safetensors.jl:23-25
    assert O.f32_to_bf16(np.float32([1.0, -2.0, 0.0])).tolist() == [0x3F80, 0xC000, 0x0000]
    # round to nearest, ties to even, on the 16 dropped bits
    bits = np.array([0x3F808000, 0x3F818000, 0x3F808001, 0x3F807FFF, 0x7F7FFFFF], np.uint32)
    assert O.f32_to_bf16(bits.view(np.float32)).tolist() == [0x3F80, 0x3F82, 0x3F81, 0x3F80, 0x7F80]
    # widening is exact: every bf16 pattern round-trips
    allbits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    wide = O.bf16_to_f32(allbits)
    assert np.array_equal(wide.view(np.uint32), allbits.astype(np.uint32) << 16)
    finite = np.isfinite(wide)
    assert np.array_equal(O.f32_to_bf16(wide[finite]), allbits[finite])


def test_split_bf16_pinned():
    """The two-term bf16 form (hi = bf16(x), lo = bf16(x - hi)) by its defining
    properties: a known answer with the piece layout, the unique decomposition
    of any a + b with bf16 a and |b| below half an ulp of a, the 2^-17 bound,
    and the non-finite and signed-zero cases."""
    # 1 + 2^-8 + 2^-12 rounds up to 1 + 2^-7; the rest, -15 * 2^-12, is a bf16 value
    x = np.float32([1 + 2.0 ** -8 + 2.0 ** -12, 1.0, -3.0, 0.5, 2.0, 0.0, 3 * 2.0 ** -10, -7.25])
    b = O.split_bf16(x)
    assert b.shape == (16,)
    assert b[:4].tolist() == [0x3F81, 0x3F80, 0xC040, 0x3F00]            # hi of elements 0..3
    assert O.bf16_to_f32(b[4:8]).tolist() == [-15 * 2.0 ** -12, 0.0, 0.0, 0.0]  # their lo
    assert b[8:12].tolist() == O.f32_to_bf16(x[4:]).tolist()             # hi of elements 4..7
    assert np.array_equal(O.join_split(b), x)
    # unique decomposition: a + b (exact in fp32) splits back into (a, b) bit for bit
    rng = np.random.default_rng(5)
    n = 200000
    a = O.round_bf16(rng.standard_normal(n).astype(np.float32) *
                     np.exp2(rng.integers(-60, 60, n)).astype(np.float32))
    ulp = np.exp2(np.floor(np.log2(np.abs(a))) - 7).astype(np.float32)
    # |b| in [2^-8, 0.499] ulps of a: a + b spans at most 24 bits, so it is exact
    mag = rng.uniform(2.0 ** -8, 0.499, n) * rng.choice([-1.0, 1.0], n)
    lo = O.round_bf16((mag * ulp).astype(np.float32))
    # (below a power of two the next binade's half ulp is smaller: keep a off them)
    keep = np.frexp(a)[0] != np.float32(np.sign(a) * 0.5)
    a, lo = a[keep], lo[keep]
    a, lo = a[:len(a) // 8 * 8], lo[:len(a) // 8 * 8]
    xs = (a + lo).astype(np.float32)
    assert np.array_equal(xs.astype(np.float64), a.astype(np.float64) + lo.astype(np.float64))
    g = O.split_bf16(xs.reshape(-1, 8)).reshape(-1, 2, 4)
    assert np.array_equal(O.bf16_to_f32(g[:, 0]).reshape(-1), a)
    assert np.array_equal(O.bf16_to_f32(g[:, 1]).reshape(-1), lo)
    # any normal fp32 value: hi is bf16(x) and |x - (hi + lo)| <= 2^-17 |x| (|x - hi| is
    # at most half a bf16 ulp, 2^-8 |x|, and lo rounds that rest to 8 bits)
    y = (rng.standard_normal(n) * np.exp2(rng.integers(-100, 100, n))).astype(np.float32)
    g = O.split_bf16(y.reshape(-1, 8)).reshape(-1, 2, 4)
    assert np.array_equal(g[:, 0].reshape(-1), O.f32_to_bf16(y))
    err = np.abs(O.round_split(y).astype(np.float64) - y) / np.abs(y)
    assert err.max() <= 2.0 ** -17 and err.max() > 2.0 ** -18
    # non-finite hi (inf, NaN, FLT_MAX rounding up to inf) gets lo = +0; -0 splits to (-0, +0)
    sp = np.float32([np.inf, -np.inf, np.nan, np.finfo(np.float32).max, -0.0, 1e-40, 0, 0])
    with np.errstate(invalid="ignore"):
        g = O.split_bf16(sp).reshape(2, 2, 4)
    hi, lo = O.bf16_to_f32(g[:, 0]).reshape(-1), g[:, 1].reshape(-1)
    assert hi[0] == np.inf and hi[1] == -np.inf and np.isnan(hi[2]) and hi[3] == np.inf
    assert lo[:4].tolist() == [0, 0, 0, 0]
    assert g[1, 0, 0] == 0x8000 and lo[4] == 0x0000
    # a denormal: hi = bf16(x), lo = bf16(x - hi)
    h5 = O.bf16_to_f32(g[1, 0, 1:2])
    assert g[1, 0, 1] == O.f32_to_bf16(sp[5:6])[0]
    assert lo[5] == O.f32_to_bf16((sp[5:6] - h5).astype(np.float32))[0]
    with pytest.raises(ValueError):
        O.split_bf16(np.zeros(6, np.float32))


def test_transformers_rms(transformers_golden):
    for width in (7, 256, 1024):
        got = O.rms(ramp(np.sin, (17, width)), ramp(np.cos, (width,), 0.1), 1e-6)
        assert normwise(got, transformers_golden[f"rms/{width}"]) < 1e-6


def test_transformers_gated(transformers_golden):
    got = O.gated_rms(ramp(np.sin, (17, 4, 128)), ramp(np.cos, (17, 4, 128), 3.0),
                      ramp(np.cos, (128,)), 1e-6)
    assert normwise(got, transformers_golden["gated/out"]) < 1e-6


@pytest.mark.parametrize("tag", ["hd64", "hd256"])
def test_transformers_partial_rope(transformers_golden, tag):
    hd, rot, heads, kv, seqs, seq = (int(v) for v in transformers_golden[f"rope/{tag}/meta"])
    T = seqs * seq
    cos, sin = O.rope_tables(seq, rot, 1e7)
    q = O.qk_norm_rope(ramp(np.sin, (T, heads, hd), 2.0), ramp(np.cos, (hd,), 0.05), cos, sin, rot,
                       1e-6, seq_len=seq)
    k = O.qk_norm_rope(ramp(np.cos, (T, kv, hd), 2.0), ramp(np.sin, (hd,), 0.05), cos, sin, rot,
                       1e-6, seq_len=seq)
    assert normwise(q, transformers_golden[f"rope/{tag}/q"]) < 1e-6
    assert normwise(k, transformers_golden[f"rope/{tag}/k"]) < 1e-6


def test_transformers_swiglu(transformers_golden):
    gate = transformers_golden["swiglu/gate"]
    up = ramp(np.cos, (9, 64), 2.0)
    got = O.swiglu(gate, up)
    exp = transformers_golden["swiglu/out"]
    assert normwise(got, exp) < 1e-6
    # special values of the first row: 0, -0, -100, 100, +-1e-30, 80, -20, +-88, 1e-12, 3
    np.testing.assert_allclose(got[0, :12], exp[0, :12], rtol=2e-6, atol=1e-37)


def test_transformers_plumbing_backbone(transformers_golden):
    import dataclasses
    from qdc_amd.config import plumbing_config
    from qdc_amd.weights import random_weights
    vocab, T, seed = (int(v) for v in transformers_golden["model/meta"])
    cfg = dataclasses.replace(plumbing_config(), vocab=vocab)
    W = random_weights(cfg, seed=seed)
    got = forward.backbone_hidden(W, cfg.as_dict(), transformers_golden["model/ids"],
                                  np.ones(T, np.int8))
    assert normwise(got, transformers_golden["model/hidden"]) < 2e-6


def test_gather_bruteforce():
    rng = np.random.default_rng(0)
    for dtype in (np.float32, np.uint16):
        table = rng.integers(0, 1 << 16, size=(37, 24)).astype(dtype)
        ids = rng.integers(0, 37, size=101)
        got = O.gather(table, ids)
        assert got.tobytes() == b"".join(table[i].tobytes() for i in ids)
    for bad in ([37], [-1], [0, 5, 99]):
        with pytest.raises(ValueError):
            O.gather(table, bad)
    assert O.gather(table, []).shape == (0, 24)


def test_rms_closed_forms():
    # constant rows: s = 1/sqrt(c^2 + eps)
    c = np.float32(0.75)
    w = ramp(np.cos, (7,), 0.1)
    got = O.rms(np.full((3, 7), c, np.float32), w, 1e-6)
    exp = (c * (np.float32(1) / np.sqrt(c * c + np.float32(1e-6)))) * (np.float32(1) + w)
    np.testing.assert_allclose(got, np.broadcast_to(exp, (3, 7)), rtol=2e-7)
    # with eps = 0 scaling by a power of two is exact
    x = ramp(np.sin, (5, 1024))
    w = ramp(np.cos, (1024,))
    assert np.array_equal(O.rms(x, w, 0.0), O.rms(x * np.float32(8), w, 0.0))
    assert np.array_equal(O.rms(x, w, 0.0, centered=False), O.rms(x / np.float32(4), w, 0.0, False))
    # widths 1 / 7 / 1024 and n = 0 / 1 / 17, as test/backbone.jl:387-413
    for width in (1, 7, 1024):
        for n in (0, 1, 17):
            x = ramp(np.sin, (n, width))
            w = ramp(np.cos, (width,))
            np.testing.assert_allclose(O.rms(x, w, 1e-6), _np_rms(x, w, 1e-6, True), rtol=3e-6,
                                       atol=1e-7)


# the special values of test/backbone.jl:303-312 (fp32 denormal included)
NORM_SPECIALS = [0.0, -0.0, np.nan, np.inf, float(np.finfo(np.float32).max),
                 float(np.nextafter(np.float32(0), np.float32(1)))]


def _same_bits_or_nan(a, b):
    """Julia isequal on fp32 arrays: NaN equals NaN, -0 differs from +0."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | ((a.view(np.uint32) == b.view(np.uint32)) & ~np.isnan(a))))


def test_normalize_heads_reference_cases():
    """The DeltaNet q/k normalisation against test/backbone.jl:290-312: sine
    ramps over widths 1/7/16/128, 1 or 3 heads, n = 0/1/65 and both multipliers
    against the division form at 2e-6, and special values that must match it
    exactly (Julia isequal)."""
    F32 = np.float32
    for width in (1, 7, 16, 128):
        for heads in (1, 3):
            for n in (0, 1, 65):
                for mult in (F32(1), np.sqrt(F32(width))):
                    x = np.sin(np.arange(1, width * heads * n + 1, dtype=F32)).astype(F32)
                    x = x.reshape(n, heads, width)  # column-major (width, heads, n)
                    exp = x / (np.sqrt((x * x).sum(-1, keepdims=True) + F32(1e-6)) * mult)
                    np.testing.assert_allclose(forward.normalize_heads(x, mult), exp,
                                               atol=2e-6, rtol=2e-6)
    for v in NORM_SPECIALS:
        x = np.full((3, 2, 8), v, np.float32)
        with np.errstate(over="ignore", invalid="ignore"):
            exp = (x / np.sqrt((x * x).sum(-1, keepdims=True, dtype=np.float32)
                               + np.float32(1e-6))).astype(np.float32)
        assert _same_bits_or_nan(forward.normalize_heads(x, np.float32(1)), exp), v


def test_rope_closed_forms():
    T, H, hd, rd = 40, 3, 64, 16
    cos, sin = O.rope_tables(T, rd, 1e7)
    # freq_0 = 1: column 0 holds cos/sin of the position itself
    np.testing.assert_array_equal(cos[:, 0], np.cos(np.arange(T, dtype=np.float64)).astype(np.float32))
    np.testing.assert_array_equal(sin[:, 0], np.sin(np.arange(T, dtype=np.float64)).astype(np.float32))
    assert np.allclose(cos * cos + sin * sin, 1, atol=1e-6)
    assert np.array_equal(cos[0], np.ones(rd // 2, np.float32))
    x = ramp(np.sin, (T, H, hd))
    w = ramp(np.cos, (hd,), 0.1)
    normed = O.rms(x, w, 1e-6)
    # rotary 0 is the plain per-head norm (test/backbone.jl:359); position 0 is identity
    np.testing.assert_array_equal(O.qk_norm_rope(x, w, cos[:, :0], sin[:, :0], 0, 1e-6), normed)
    got = O.qk_norm_rope(x, w, cos, sin, rd, 1e-6)
    np.testing.assert_array_equal(got[0], normed[0])
    # dims >= rotary pass through, pair norms are preserved
    np.testing.assert_array_equal(got[..., rd:], normed[..., rd:])
    h = rd // 2
    pair = lambda y: y[..., :h] ** 2 + y[..., h:rd] ** 2  # noqa: E731
    np.testing.assert_allclose(pair(got), pair(normed), rtol=1e-5, atol=1e-7)
    # against a float64 rotation by the fp32 angle freq_i * pos
    freq = (np.float32(1) / np.float32(1e7) ** (np.arange(0, rd, 2, dtype=np.float32) / np.float32(rd)))
    ang = (freq[None, :] * np.arange(T, dtype=np.float32)[:, None]).astype(np.float64)
    a, b = normed[..., :h].astype(np.float64), normed[..., h:rd].astype(np.float64)
    c64, s64 = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    exp = np.concatenate([a * c64 - b * s64, b * c64 + a * s64], -1)
    assert normwise(got[..., :rd], exp) < 1e-6
    # positions reset per sequence and the offset shifts them
    two = O.qk_norm_rope(np.concatenate([x, x]), w, cos, sin, rd, 1e-6, seq_len=T)
    np.testing.assert_array_equal(two[:T], two[T:])
    cos2, sin2 = O.rope_tables(2 * T, rd, 1e7)
    shifted = O.qk_norm_rope(x[5:], w, cos2, sin2, rd, 1e-6, seq_len=T, pos_offset=5)
    np.testing.assert_array_equal(shifted, O.qk_norm_rope(x, w, cos2, sin2, rd, 1e-6)[5:])


def test_swiglu_invariants():
    g = ramp(np.sin, (4, 256), 6.0)
    u = np.ones_like(g)
    # silu(x) - silu(-x) = x
    np.testing.assert_allclose(O.swiglu(g, u) - O.swiglu(-g, u), g, rtol=1e-6, atol=1e-6)
    assert np.array_equal(O.swiglu(np.zeros((2, 8), np.float32), u[:2, :8]), np.zeros((2, 8)))
    # silu(x)*u is linear in u
    u2 = ramp(np.cos, (4, 256))
    np.testing.assert_array_equal(O.swiglu(g, u2 * np.float32(2)), O.swiglu(g, u2) * np.float32(2))


# mistakes planted in the attention and DeltaNet row work of oracle/forward.py
_fwd = {name: getattr(forward, name) for name in ("attention_softmax", "attention_gate",
                                                  "delta_prologue")}
FORWARD_MUTANTS = {
    "softmax mask ignored": ("attention_softmax", lambda s, m, scale, q_offset=0:
                             _fwd["attention_softmax"](s, None, scale, q_offset)),
    "softmax scale dropped": ("attention_softmax", lambda s, m, scale, q_offset=0:
                              _fwd["attention_softmax"](s, m, 1.0, q_offset)),
    "softmax not causal": ("attention_softmax", lambda s, m, scale, q_offset=0:
                           _fwd["attention_softmax"](s, m, scale, q_offset + s.shape[-1])),
    "gate not applied": ("attention_gate", lambda v, g: _fwd["attention_gate"](v, g * 0 + 80)),
    "prologue q not scaled": ("delta_prologue", lambda *a: (lambda r: (r[0] * np.float32(
        np.sqrt(a[7])), *r[1:]))(_fwd["delta_prologue"](*a))),
    "prologue decay sign": ("delta_prologue", lambda *a: (lambda r: (*r[:4], -r[4]))(
        _fwd["delta_prologue"](*a))),
}


@pytest.mark.parametrize("mutant", sorted(FORWARD_MUTANTS))
def test_goldens_catch_planted_forward_mistakes(native_fixture, transformers_golden, monkeypatch,
                                                mutant):
    # the fixture checks the last position under masks; the transformers golden
    # checks every position of an unmasked sequence (causality)
    import dataclasses
    from qdc_amd.config import plumbing_config
    from qdc_amd.weights import random_weights
    name, fn = FORWARD_MUTANTS[mutant]
    monkeypatch.setattr(forward, name, fn)
    cases = [c for c in native_fixture["cases"] if c[0].startswith(("ref04", "cuda13"))]
    bad = [n for n, got, exp in fixture_logits(native_fixture, cases)
           if not isapprox(got, exp, 2e-5, 2e-5)]
    vocab, T, seed = (int(v) for v in transformers_golden["model/meta"])
    cfg = dataclasses.replace(plumbing_config(), vocab=vocab)
    got = forward.backbone_hidden(random_weights(cfg, seed=seed), cfg.as_dict(),
                                  transformers_golden["model/ids"], np.ones(T, np.int8))
    if normwise(got, transformers_golden["model/hidden"]) >= 2e-6:
        bad.append("transformers plumbing")
    assert bad, f"planted mistake '{mutant}' went unnoticed"


def test_attention_softmax_against_scipy():
    from scipy.special import softmax
    rng = np.random.default_rng(5)
    B, H, Q, K = 2, 3, 9, 12
    scores = rng.standard_normal((B, H, Q, K), dtype=np.float32) * np.float32(4)
    mask = (rng.random((B, K)) > 0.3).astype(np.int32)
    mask[1, :] = 0
    mask[1, 7] = 1          # batch 1: queries 0..3 (offset 3) see no unmasked key
    for q_offset in (0, 3):
        got = forward.attention_softmax(scores, mask, 0.125, q_offset)
        for b in range(B):
            for h in range(H):
                for q in range(Q):
                    vis = [i for i in range(K) if i <= q + q_offset and mask[b, i]]
                    row = got[b, h, q]
                    if not vis:  # no visible key: uniform over every key (reference behaviour)
                        assert np.array_equal(row, np.full(K, np.float32(1) / np.float32(K)))
                        continue
                    exp = np.zeros(K, np.float64)
                    exp[vis] = softmax(scores[b, h, q, vis].astype(np.float64) * 0.125)
                    assert np.abs(row - exp).max() < 1e-6
                    assert np.all(row[[i for i in range(K) if i not in vis]] == 0)


def test_attention_gate_against_scipy():
    from scipy.special import expit
    rng = np.random.default_rng(6)
    B, H, S, hd = 2, 3, 5, 4
    values = rng.standard_normal((B, H, S, hd), dtype=np.float32)
    gate = rng.standard_normal((B * S, H, hd), dtype=np.float32) * np.float32(3)
    got = forward.attention_gate(values, gate)
    for b in range(B):
        for s in range(S):
            for h in range(H):
                exp = values[b, h, s] * expit(gate[b * S + s, h].astype(np.float64))
                assert np.abs(got[b * S + s, h * hd:(h + 1) * hd] - exp).max() < 1e-6


def test_threaded_oracle_is_bit_identical():
    """The oracle's OpenMP row loops (used for the all-cores CPU figure) give
    the single-thread bits; SwiGLU over more than 65536 elements takes the
    reference's interleaved 256-element block split, with a ragged last block."""
    rng = np.random.default_rng(9)
    g = rng.standard_normal((301, 700), dtype=np.float32) * np.float32(4)
    u = rng.standard_normal((301, 700), dtype=np.float32)
    x = rng.standard_normal((257, 96), dtype=np.float32)
    w = rng.standard_normal(96, dtype=np.float32) * np.float32(0.02)
    q = rng.standard_normal((33, 3, 96), dtype=np.float32)
    cos, sin = O.rope_tables(33, 32, 1e4)
    z = rng.standard_normal((41, 4, 96), dtype=np.float32)
    table = rng.standard_normal((500, 96), dtype=np.float32)
    ids = rng.integers(0, 500, size=77)

    def run():
        return [O.swiglu(g, u), O.rms(x, w, 1e-6), O.rms(x, w, 1e-6, False),
                *O.residual_rms(x, x[::-1].copy(), w, 1e-6),
                O.qk_norm_rope(q, w, cos, sin, 32, 1e-6, 11),
                O.gated_rms(z, z[::-1].copy(), w, 1e-6), O.gather(table, ids)]

    assert g.size > 65536 and g.size % 256
    single = run()
    previous = O.set_threads(4)
    try:
        threaded = run()
    finally:
        O.set_threads(previous)
    for a, b in zip(single, threaded):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))

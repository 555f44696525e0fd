"""Host-side argument checks of the ``qdc_amd.ops`` wrappers, on the CPU.

Every wrapper must reject a caller-supplied output of the wrong dtype or on
another device before anything reaches the library: a bf16 ``out`` given to an
fp32 kernel would be written past its end on the device, and a host ``out``
would hand a host pointer to the kernel.  Here the library is replaced by a
stub that fails the test if any entry point is reached, and ``meta`` tensors
stand in for device tensors (``ops._device`` is switched to accept them), so a
missing check shows up as a stub call instead of a launch.
"""
import pytest
import torch

from qdc_amd import ops

F32, BF16 = torch.float32, torch.bfloat16


class _Stub:
    def __getattr__(self, name):
        raise AssertionError(f"{name} reached the library")


@pytest.fixture
def no_launch(monkeypatch):
    def device(*tensors):
        dev = tensors[0].device
        if dev.type != "meta":
            raise ValueError("device tensors required")
        for t in tensors:
            if t.device != dev:
                raise ValueError(f"tensors on different devices: {dev} vs {t.device}")

    monkeypatch.setattr(ops, "_device", device)
    monkeypatch.setattr(ops, "lib", lambda: _Stub())
    monkeypatch.setattr(ops, "_stream", lambda t: 0)


def d(*shape, dtype=F32):
    return torch.empty(shape, dtype=dtype, device="meta")


def host(*shape, dtype=F32):
    return torch.empty(shape, dtype=dtype)


def _calls():
    """(name, valid call, [invalid calls]) per wrapper: the valid call must reach
    the library (the stub), every invalid one must raise ValueError first."""
    tables = (d(8, 4), d(8, 4))
    return [
        ("native_gather_rms",
         lambda **kw: ops.native_gather_rms(d(10, 16, dtype=BF16), d(4, dtype=torch.int32),
                                            d(16, dtype=BF16), 1e-6, **kw),
         [dict(hidden=d(4, 16, dtype=BF16)), dict(hidden=host(4, 16)),
          dict(normed=d(4, 16)), dict(normed=host(4, 16, dtype=BF16)),
          dict(error_flag=d(1)), dict(error_flag=host(1, dtype=torch.int32)),
          dict(token_mask=d(4, dtype=torch.int64))]),
        ("attention_prepare",
         lambda **kw: ops.attention_prepare(d(8, 2, 16), d(8, 1, 16), d(8, 1, 16), d(16), d(16),
                                            tables, 8, 1e-6, 2, **kw),
         [dict(out=(d(2, 2, 4, 16), d(2, 1, 16, 4), d(2, 1, 4, 16, dtype=BF16))),
          dict(out=(d(2, 2, 4, 16), host(2, 1, 16, 4), d(2, 1, 4, 16))),
          dict(out=(d(2, 2, 4, 16), d(2, 1, 4, 16), d(2, 1, 4, 16))),
          dict(out=(d(2, 2, 4, 16), d(2, 1, 16, 4)))]),
        # K and V only (q=None): the final-query attention's context
        ("attention_prepare_kv",
         lambda **kw: ops.attention_prepare(kw.pop("q", None), d(8, 1, 16), d(8, 1, 16),
                                            kw.pop("q_norm", None), d(16), tables, 8, 1e-6, 2,
                                            **kw),
         [dict(q_norm=d(16)),
          dict(out=(d(2, 2, 4, 16), d(2, 1, 16, 4), d(2, 1, 4, 16))),
          dict(out=(None, d(2, 1, 4, 16), d(2, 1, 4, 16))),
          dict(out=(None, d(2, 1, 16, 4, dtype=BF16), d(2, 1, 4, 16)))]),
        ("device_copy_rows",
         lambda **kw: ops.device_copy_rows(kw.get("dst", d(4, 16, dtype=BF16)),
                                           d(10, 16, dtype=BF16), d(4, dtype=torch.int32)),
         [dict(dst=host(4, 16, dtype=BF16)), dict(dst=d(4, 8, dtype=BF16))]),
        ("native_gather",
         lambda **kw: ops.native_gather(d(10, 16, dtype=BF16), d(4, dtype=torch.int32), **kw),
         [dict(out=d(4, 16, dtype=F32)),                      # bf16 table -> bf16 out expected
          dict(out=host(4, 16, dtype=BF16)),
          dict(out_dtype=F32, out=d(4, 16, dtype=BF16)),
          dict(error_flag=host(1, dtype=torch.int32)),
          dict(error_flag=d(1, dtype=torch.int64))]),
        ("native_rms",
         lambda **kw: ops.native_rms(d(8, 64), d(64, dtype=BF16), 1e-6, **kw),
         [dict(out=d(8, 64, dtype=F32)), dict(out=host(8, 64, dtype=BF16)),
          dict(token_mask=host(8, dtype=torch.int32)), dict(token_mask=d(8, dtype=torch.int64))]),
        ("native_residual_rms",
         lambda **kw: ops.native_residual_rms(d(8, 64), d(8, 64, dtype=BF16), d(64, dtype=BF16),
                                              1e-6, **kw),
         [dict(residual=d(8, 64, dtype=BF16)), dict(residual=host(8, 64)),
          dict(out=d(8, 64, dtype=F32)), dict(out=host(8, 64, dtype=BF16))]),
        ("native_gated_rms",
         lambda **kw: ops.native_gated_rms(d(4, 2, 16, dtype=BF16), d(4, 2, 16, dtype=BF16),
                                           d(16, dtype=BF16), 1e-6, **kw),
         [dict(out=d(4, 2, 16, dtype=F32)), dict(out=host(4, 2, 16, dtype=BF16))]),
        ("prepare_heads",
         lambda **kw: ops.prepare_heads(d(8, 2, 16), d(8, 1, 16), d(16), d(16), tables, 8, 1e-6,
                                        **kw),
         [dict(q_out=d(8, 2, 16, dtype=BF16)), dict(k_out=d(8, 1, 16, dtype=BF16)),
          dict(q_out=host(8, 2, 16)), dict(k_out=host(8, 1, 16)),
          dict(q_out=d(1, 8, 2, 16, dtype=BF16))]),
        ("native_mlp_gate",
         lambda **kw: ops.native_mlp_gate(d(4, 16), d(4, 16), **kw),
         [dict(out=d(4, 16, dtype=BF16)), dict(out=host(4, 16))]),
        ("delta_scan",
         lambda **kw: ops.delta_scan(d(1, 4, 2, 8), d(1, 4, 2, 8), d(1, 4, 2, 8), d(1, 4, 2),
                                     d(1, 4, 2), **kw),
         [dict(out=host(1, 4, 2, 8)), dict(out=d(1, 4, 2, 8, dtype=torch.float16))]),
        ("delta_prologue",
         lambda **kw: ops.delta_prologue(d(4, 3 * 16 + 16 + 4, dtype=BF16), d(48, 4), d(2), d(2),
                                         4, 1, 16, 2, 8, **kw),
         [dict(out=(host(4, 1, 16), d(4, 1, 16), d(4, 2, 8), d(4, 2), d(4, 2))),
          dict(out=(d(4, 1, 16), d(4, 1, 16), d(4, 2, 8), d(4, 2), host(4, 2))),
          dict(out=(d(4, 1, 16, dtype=BF16), d(4, 1, 16), d(4, 2, 8), d(4, 2), d(4, 2)))]),
        ("attention_softmax",
         lambda **kw: ops.attention_softmax(d(1, 2, 4, 4), None, 0.5, **kw),
         [dict(out=host(1, 2, 4, 4)), dict(out=d(1, 2, 4, 4, dtype=torch.float16))]),
        ("attention_gate",
         lambda **kw: ops.attention_gate(d(1, 2, 4, 8), d(4, 2, 8, dtype=BF16), **kw),
         [dict(out=host(4, 16, dtype=BF16)), dict(out=d(4, 16, dtype=torch.float16))]),
        # split two-term bf16 outputs: bf16 buffers with twice the last axis
        ("native_gather_rms split",
         lambda **kw: ops.native_gather_rms(d(10, 16, dtype=BF16), d(4, dtype=torch.int32),
                                            d(16, dtype=BF16), 1e-6, normed_dtype=ops.BF16X2,
                                            **kw),
         [dict(normed=d(4, 16, dtype=BF16)), dict(normed=d(4, 32)),
          dict(normed=host(4, 32, dtype=BF16))]),
        ("native_rms split",
         lambda **kw: ops.native_rms(d(8, 64), d(64, dtype=BF16), 1e-6, out_dtype=ops.BF16X2,
                                     **kw),
         [dict(out=d(8, 64, dtype=BF16)), dict(out=d(8, 128)), dict(out=host(8, 128, dtype=BF16))]),
        ("native_residual_rms split",
         lambda **kw: ops.native_residual_rms(d(8, 64), d(8, 64), d(64, dtype=BF16), 1e-6,
                                              out_dtype=ops.BF16X2, **kw),
         [dict(out=d(8, 64, dtype=BF16)), dict(out=d(8, 128)), dict(out=host(8, 128, dtype=BF16))]),
        ("native_gated_rms split",
         lambda **kw: ops.native_gated_rms(d(4, 2, 16, dtype=BF16), d(4, 2, 16, dtype=BF16),
                                           d(16, dtype=BF16), 1e-6, out_dtype=ops.BF16X2, **kw),
         [dict(out=d(4, 2, 16, dtype=BF16)), dict(out=d(4, 2, 32)),
          dict(out=host(4, 2, 32, dtype=BF16))]),
        ("native_mlp_gate split",
         lambda **kw: ops.native_mlp_gate(d(4, 16), d(4, 16), out_dtype=ops.BF16X2, **kw),
         [dict(out=d(4, 16, dtype=BF16)), dict(out=d(4, 32)), dict(out=host(4, 32, dtype=BF16))]),
        ("attention_gate split",
         lambda **kw: ops.attention_gate(d(1, 2, 4, 8), d(4, 2, 8, dtype=BF16),
                                         out_dtype=ops.BF16X2, **kw),
         [dict(out=d(4, 16, dtype=BF16)), dict(out=d(4, 32)), dict(out=host(4, 32, dtype=BF16))]),
    ]


@pytest.mark.parametrize("name,call,bad", _calls(), ids=[c[0] for c in _calls()])
def test_outputs_checked_before_launch(no_launch, name, call, bad):
    with pytest.raises(AssertionError, match="reached the library"):
        call()
    for kwargs in bad:
        with pytest.raises(ValueError):
            call(**kwargs)


def test_host_tensors_rejected(no_launch):
    with pytest.raises(ValueError):
        ops.native_rms(host(8, 64), host(64), 1e-6)
    with pytest.raises(ValueError):
        ops.native_mlp_gate(d(4, 16), host(4, 16))


def test_split_argument_checks(no_launch):
    """The split output takes the input types its kernels implement; anything
    else raises before the library is reached."""
    X2 = ops.BF16X2
    with pytest.raises(ValueError, match="unknown out_dtype"):
        ops.native_rms(d(8, 64), d(64, dtype=BF16), 1e-6, out_dtype="bf16x3")
    with pytest.raises(ValueError):
        ops.native_rms(d(8, 64), d(64), 1e-6, out_dtype=X2)                # fp32 weight
    with pytest.raises(ValueError):
        ops.native_rms(d(8, 64, dtype=BF16), d(64, dtype=BF16), 1e-6, out_dtype=X2)
    with pytest.raises(ValueError):
        ops.native_residual_rms(d(8, 64), d(8, 64, dtype=BF16), d(64, dtype=BF16), 1e-6,
                                out_dtype=X2)                              # bf16 addend
    with pytest.raises(ValueError):
        ops.native_gated_rms(d(4, 2, 16), d(4, 2, 16), d(16), 1e-6, out_dtype=X2)
    with pytest.raises(ValueError):
        ops.native_mlp_gate(d(4, 16, dtype=BF16), d(4, 16, dtype=BF16), out_dtype=X2)
    with pytest.raises(ValueError):
        ops.native_gather_rms(d(10, 16, dtype=BF16), d(4, dtype=torch.int32), d(16), 1e-6,
                              normed_dtype=X2)                             # fp32 weight


def test_split_weight_and_join_on_cpu():
    """split_weight repeats each input row into its hi and lo slots, and
    join_split adds the two terms back, on plain CPU tensors."""
    w = torch.arange(8 * 3, dtype=torch.float32).reshape(8, 3).to(BF16)
    w2 = ops.split_weight(w)
    assert w2.shape == (16, 3)
    for g in range(2):
        for j in range(4):
            assert torch.equal(w2[8 * g + j], w[4 * g + j])
            assert torch.equal(w2[8 * g + 4 + j], w[4 * g + j])
    with pytest.raises(ValueError):
        ops.split_weight(torch.zeros(6, 3, dtype=BF16))
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0, 0.5, 0.25, -1.0, 0.0]], dtype=BF16)
    assert torch.equal(ops.join_split(x), torch.tensor([[1.5, 2.25, 2.0, 4.0]]))
    with pytest.raises(ValueError):
        ops.join_split(torch.zeros(1, 8))
    # the product identity the layout exists for: [hi | lo] pieces times the
    # repeated rows equal (hi + lo) times the rows
    hi = torch.tensor([[1.0, -2.0, 0.5, 3.0, 8.0, 1.0, -1.0, 2.0]]).to(BF16)
    lo = torch.tensor([[2.0 ** -9, 0.0, -(2.0 ** -12), 2.0 ** -8, 0.0, 2.0 ** -10, 0.0,
                        -(2.0 ** -9)]]).to(BF16)
    xs = torch.cat([hi.view(1, 2, 4), lo.view(1, 2, 4)], 2).reshape(1, 16)
    wk = torch.randn(8, 5).to(BF16)
    got = xs.float() @ ops.split_weight(wk).float()
    exp = (hi.float() + lo.float()) @ wk.float()
    assert torch.allclose(got, exp, rtol=0, atol=1e-6)


def test_backbone_split_mode_checks():
    """The split GEMM-input modes are bf16-only, named, and need rows of whole
    4-element groups; all of it is checked before any weight is touched."""
    import dataclasses

    from qdc_amd import backbone
    from qdc_amd.config import plumbing_config
    cfg = plumbing_config()
    with pytest.raises(ValueError, match="bfloat16"):
        backbone.QwenBackbone(cfg, {}, "cpu", torch.float32, split_gemm_inputs=True)
    with pytest.raises(ValueError, match="split_gemm_inputs"):
        backbone.QwenBackbone(cfg, {}, "cpu", torch.bfloat16, split_gemm_inputs="attention")
    odd = dataclasses.replace(cfg, value_dim=6)
    with pytest.raises(ValueError, match="multiples of 4"):
        backbone.QwenBackbone(odd, {}, "cpu", torch.bfloat16, split_gemm_inputs="all")
    with pytest.raises(KeyError):  # "mlp" does not split the 6-wide value rows: it proceeds
        backbone.QwenBackbone(odd, {}, "cpu", torch.bfloat16, split_gemm_inputs="mlp")


def test_split_output_strides_checked(no_launch):
    """A caller-supplied split output whose rows are not whole 16-byte pieces
    apart (a bf16 stride that is not a multiple of 8) is rejected before the
    stride is halved for the C ABI."""
    X2 = ops.BF16X2
    odd = torch.empty((8, 140), dtype=BF16, device="meta")[:, :128]      # stride 140
    with pytest.raises(ValueError, match="multiple of 8"):
        ops.native_rms(d(8, 64), d(64, dtype=BF16), 1e-6, out=odd, out_dtype=X2)
    with pytest.raises(ValueError, match="multiple of 8"):
        ops.native_mlp_gate(d(8, 64), d(8, 64), out=odd, out_dtype=X2)
    gated = torch.empty((8, 1, 140), dtype=BF16, device="meta")[:, :, :128]
    with pytest.raises(ValueError, match="multiple of 8"):
        ops.native_gated_rms(d(8, 1, 64, dtype=BF16), d(8, 1, 64, dtype=BF16),
                             d(64, dtype=BF16), 1e-6, out=gated, out_dtype=X2)
    merged = torch.empty((4, 36), dtype=BF16, device="meta")[:, :32]
    with pytest.raises(ValueError, match="multiple of 8"):
        ops.attention_gate(d(1, 2, 4, 8), d(4, 2, 8, dtype=BF16), out=merged, out_dtype=X2)


def test_native_sequence_start(monkeypatch):
    """The first kept token of a row (``ext/QwenDecisionCoreAMDGPUExt.jl:17-24``):
    leading zeros are skipped, the last token always stays, and
    ``QDC_AMDGPU_TRIM_PADDING`` other than "1" turns the trim off."""
    import numpy as np
    from qdc_amd.backbone import native_sequence_start
    mask = np.array([[1, 1, 0, 1], [0, 0, 1, 1], [0, 0, 0, 0], [0, 0, 0, 1], [0, 1, 0, 1]])
    monkeypatch.delenv("QDC_AMDGPU_TRIM_PADDING", raising=False)
    assert [native_sequence_start(mask, r) for r in range(5)] == [0, 2, 3, 3, 1]
    monkeypatch.setenv("QDC_AMDGPU_TRIM_PADDING", "1")
    assert native_sequence_start(mask, 1) == 2
    monkeypatch.setenv("QDC_AMDGPU_TRIM_PADDING", "0")
    assert [native_sequence_start(mask, r) for r in range(5)] == [0] * 5


def test_parameter_vectors_checked_before_launch(no_launch):
    """Norm weights, RoPE tables and the DeltaNet parameters are read by the
    kernels as contiguous vectors of a known length: a shorter or strided one,
    or a table of the wrong width, dtype or device, raises ValueError before
    the library is reached (the kernels would read past their ends)."""
    tables = (d(8, 4), d(8, 4))
    q, k, v = d(8, 2, 16), d(8, 1, 16), d(8, 1, 16)
    proj = d(4, 3 * 16 + 16 + 4, dtype=BF16)
    bad = [
        lambda: ops.native_residual_rms(d(8, 16), d(8, 16), d(32)[::2], 1e-6),
        lambda: ops.native_residual_rms(d(8, 16), d(8, 16), d(15), 1e-6),
        lambda: ops.native_gated_rms(d(4, 2, 16, dtype=BF16), d(4, 2, 16, dtype=BF16),
                                     d(8, dtype=BF16), 1e-6),
        lambda: ops.native_gated_rms(d(4, 2, 16, dtype=BF16), d(4, 2, 16, dtype=BF16),
                                     d(32, dtype=BF16)[::2], 1e-6),
        lambda: ops.prepare_heads(q, k, d(8), d(16), tables, 8, 1e-6),
        lambda: ops.prepare_heads(q, k, d(16), d(32)[::2], tables, 8, 1e-6),
        lambda: ops.prepare_heads(q, k, d(16), d(16), (d(8, 3), d(8, 3)), 8, 1e-6),
        lambda: ops.prepare_heads(q, k, d(16), d(16), (d(8, 4), d(7, 4)), 8, 1e-6),
        lambda: ops.prepare_heads(q, k, d(16), d(16), (d(8, 4, dtype=BF16),) * 2, 8, 1e-6),
        lambda: ops.prepare_heads(q, k, d(16), d(16), None, 8, 1e-6),
        lambda: ops.attention_prepare(q, k, v, d(32)[::2], d(16), tables, 8, 1e-6, 2),
        lambda: ops.attention_prepare(q, k, v, d(16), d(16), (d(8, 4), host(8, 4)), 8, 1e-6, 2),
        lambda: ops.delta_prologue(proj, d(40, 4), d(2), d(2), 4, 1, 16, 2, 8),
        lambda: ops.delta_prologue(proj, d(48, 4), d(3), d(2), 4, 1, 16, 2, 8),
        lambda: ops.delta_prologue(proj, d(48, 4), d(2), d(4)[::2], 4, 1, 16, 2, 8),
        lambda: ops.delta_prologue(d(4, 60, dtype=BF16), d(48, 4), d(2), d(2), 4, 1, 16, 2, 8),
    ]
    for i, call in enumerate(bad):
        with pytest.raises(ValueError):
            call()

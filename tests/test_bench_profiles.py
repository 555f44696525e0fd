"""The profile-summary matching of bench.py on synthetic dispatch lists (CPU):
graph replays are found as runs of `steps` dispatches, adjacent kernels that
share a signature are split apart, and the timed pass is the second of two
identical consecutive passes."""
import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402


def _d(sig, n, dur=1.0):
    return [((sig, 1, 1), dur, None)] * n


def test_runs_split_adjacent_same_signature():
    disp = _d("a", 2) + _d("b", 4) + _d("a", 3)
    runs = bench._runs(disp, 2)
    assert [len(r) for r in runs] == [2, 2, 2, 3]
    assert [r[0][0][0] for r in runs] == ["a", "b", "b", "a"]


def test_find_passes_takes_the_second_identical_pass():
    steps = 3
    # eager warmup, check pass (replay + one eager launch each), untimed, timed
    disp = _d("x", 1) + _d("y", 1) + _d("x", 4) + _d("y", 4)
    disp += _d("x", steps, 1.0) + _d("y", steps, 1.0)      # untimed
    disp += _d("x", steps, 2.0) + _d("y", steps, 5.0)      # timed
    disp += _d("c", 1)
    passes, end = bench._find_passes(bench._runs(disp, steps), ["kx", "ky"], steps)
    assert [d[1] for d in passes["kx"][1]] == [2.0] * steps
    assert [d[1] for d in passes["ky"][1]] == [5.0] * steps
    assert [d[1] for d in passes["ky"][0]] == [1.0] * steps


def test_find_passes_with_a_shared_signature_and_failure():
    steps = 2
    disp = _d("s", steps * 2) + _d("s", steps * 2)  # two kernels of one signature, two passes
    passes, _ = bench._find_passes(bench._runs(disp, steps), ["k1", "k2"], steps)
    assert set(passes) == {"k1", "k2"}
    with pytest.raises(RuntimeError):
        bench._find_passes(bench._runs(_d("a", 5), steps), ["k1"], steps)


def test_kernel_labels():
    """Trace kernel names as the forward tables label them."""
    assert bench._kernel_label("void qdc::(anonymous namespace)::rms_rows_fast<float>(x)") == \
        "`rms_rows_fast`"
    assert bench._kernel_label("Cijk_Ailk_Bljk_BBS_BH_Bias_HA_S_SAV") == "hipBLASLt GEMM bf16 out"
    assert bench._kernel_label("Cijk_Ailk_Bljk_BSS_BH_Bias_S_HA") == "hipBLASLt GEMM fp32 out"
    assert bench._kernel_label("Cijk_Ailk_Bljk_SB_MT32x32x64", "GEMM") == \
        "GEMMs (Tensile kernels of the kept library)"
    assert bench._kernel_label("__amd_rocclr_copyBuffer") == "runtime copy"

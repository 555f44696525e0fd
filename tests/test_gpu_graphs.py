"""Graph-replayed last-token forward (``qdc_amd.graphs.LastHiddenGraphs``)
against the eager ``backbone_last_hidden`` and the CPU oracle.

Recorded with the eager forward's own GEMM library, every replay equals the
eager forward of the same inputs bit for bit, with eager work and
synchronisations between replays; each length is replayed several times with
different ids, masked and unmasked, under a graph cache smaller than the number
of keys (recordings are evicted and made again).  Recorded with the faster of
the two GEMM libraries (the default), results stay within fp32 rounding of the
eager forward (1e-5 normwise in fp32, 1e-2 in bf16), fp32 within 1e-5 of the
oracle, and replays of the same inputs are identical to each other.
"""
import numpy as np
import pytest
import torch

from conftest import normwise
from oracle import forward

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.synchronize()


def _bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def _check_replays(model, graphs, cfg, lengths, reps, seed, oracle_weights=None, exact=True,
                   tol=1e-5):
    from qdc_amd import backbone
    from qdc_amd.graphs import MEMSET_NODE
    rng = np.random.default_rng(seed)
    for n in lengths:
        for rep in range(reps):
            ids = rng.integers(0, cfg.vocab, size=n)
            mask = np.ones(n, np.int64)
            if rep % 3 == 2:
                mask[: max(1, n // 8)] = 0      # a padded prefix: the masked graph
            print(f"graph replay n={n} rep={rep} masked={not mask.all()}", flush=True)
            got = graphs(ids, mask)
            exp = backbone.backbone_last_hidden(model, ids, mask)   # eager, in between
            again = graphs(ids, mask)
            torch.cuda.synchronize()
            assert got.shape == (cfg.hidden,)
            assert np.array_equal(_bits(got), _bits(again)), (n, rep)
            if exact:
                assert np.array_equal(_bits(got), _bits(exp)), (n, rep, normwise(got, exp))
            else:
                assert normwise(got, exp) <= tol, (n, rep, normwise(got, exp))
            if oracle_weights is not None and rep == 0:
                ref = forward.backbone_hidden(oracle_weights, cfg.as_dict(), ids, mask)[-1]
                assert normwise(got, ref) <= 1e-5, (n, normwise(got, ref))
    for key, e in graphs._entries.items():
        assert MEMSET_NODE not in e.nodes, key
        assert 0 in e.nodes, key            # kernel nodes were recorded
    assert graphs._entries, "no key was served from a recorded graph"
    print("graphs kept " + ", ".join(f"{k}: {e.library} {e.replay_ms:.3f} ms"
                                     for k, e in graphs._entries.items())
          + f"; eager keys {sorted(graphs.eager_keys)}", flush=True)


def _synthetic_model(dtype, seed=11, split=False):
    from qdc_amd import backbone
    from qdc_amd.config import synthetic_inference_config
    from qdc_amd.weights import random_weights
    cfg = synthetic_inference_config()
    weights = random_weights(cfg, seed=seed)
    if dtype == torch.bfloat16:
        from oracle import qdc_oracle as O
        weights = {k: O.round_bf16(v) for k, v in weights.items()}
    return cfg, weights, backbone.QwenBackbone.from_weights(weights, cfg, "cuda:0", dtype,
                                                            split_gemm_inputs=split)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_graph_replays_match_eager(dtype):
    """The reference's inference-benchmark model shapes (4 layers, hidden 256),
    recorded with the eager forward's GEMM library: bit for bit."""
    from qdc_amd.graphs import LastHiddenGraphs
    cfg, weights, model = _synthetic_model(dtype)
    graphs = LastHiddenGraphs(model, max_graphs=3, gemm_libraries=None)
    _check_replays(model, graphs, cfg, (64, 128, 37, 512), 3, 5,
                   oracle_weights=weights if dtype == torch.float32 else None)
    assert len(graphs._entries) <= 3


@pytest.mark.parametrize("split", ["all", "mlp"])
def test_graph_replays_split_gemm_inputs(split):
    """bf16 weights with split GEMM inputs: the split-output kernels recorded and
    replayed bit for bit against eager, and the replay within 1e-2 of the fp32
    oracle."""
    from qdc_amd.graphs import LastHiddenGraphs
    cfg, weights, model = _synthetic_model(torch.bfloat16, seed=13, split=split)
    graphs = LastHiddenGraphs(model, max_graphs=2, gemm_libraries=None)
    _check_replays(model, graphs, cfg, (64, 200), 3, 6)
    rng = np.random.default_rng(7)
    ids, mask = rng.integers(0, cfg.vocab, size=96), np.ones(96, np.int64)
    ref = forward.backbone_hidden(weights, cfg.as_dict(), ids, mask)[-1]
    assert normwise(graphs(ids, mask), ref) <= 1e-2
    # recorded with both GEMM libraries (twice-as-deep split GEMMs on rocBLAS
    # too), the faster kept: within bf16 rounding of the eager forward
    both = LastHiddenGraphs(model, max_graphs=2)
    _check_replays(model, both, cfg, (64, 200), 2, 8, exact=False, tol=1e-2)
    assert normwise(both(ids, mask), ref) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_graph_gemm_library_choice(dtype):
    """Recorded with both GEMM libraries, the faster kept: within fp32 rounding
    of the eager forward, and torch's library setting restored."""
    from qdc_amd.graphs import LastHiddenGraphs
    cfg, weights, model = _synthetic_model(dtype, seed=12)
    before = torch.backends.cuda.preferred_blas_library()
    graphs = LastHiddenGraphs(model, max_graphs=8)
    _check_replays(model, graphs, cfg, (64, 256, 512), 3, 6, exact=False,
                   tol=1e-5 if dtype == torch.float32 else 1e-2,
                   oracle_weights=weights if dtype == torch.float32 else None)
    assert torch.backends.cuda.preferred_blas_library() == before
    assert {e.library for e in graphs._entries.values()} <= {"cublaslt", "cublas"}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_graph_replays_full_size_model(dtype):
    """The 24-layer Qwen3.5-0.8B-like backbone at short lengths (small GEMMs,
    where the libraries pick other kernels than at 16384 tokens).  bf16 recorded
    with the eager forward's GEMM library: bit for bit.  fp32 recorded with both
    libraries: within 1e-5 of the eager forward (two bf16 evaluations with
    different GEMM kernels drift apart over 24 layers through rounding flips, so
    the library choice is held to fp32's bar)."""
    from qdc_amd import backbone
    from qdc_amd.config import qwen35_08b_config
    from qdc_amd.graphs import LastHiddenGraphs
    from qdc_amd.weights import random_device_weights
    cfg = qwen35_08b_config()
    weights = random_device_weights(cfg, seed=3, device="cuda:0", dtype=dtype)
    model = backbone.QwenBackbone.from_weights(weights, cfg, "cuda:0", dtype)
    del weights
    exact = dtype == torch.bfloat16
    graphs = LastHiddenGraphs(model, max_graphs=4,
                              gemm_libraries=None if exact else ("cublaslt", "cublas"))
    _check_replays(model, graphs, cfg, (16, 96), 3, 9, exact=exact)
    del graphs, model
    torch.cuda.empty_cache()


def test_graph_all_masked_and_single_token():
    """Edge masks and lengths through the graph path (eager GEMM library: bit for
    bit): a sequence with every token masked (no visible key in any attention
    row), one with only its last token kept, and a single token."""
    from qdc_amd import backbone
    from qdc_amd.graphs import LastHiddenGraphs
    cfg, weights, model = _synthetic_model(torch.float32, seed=13)
    graphs = LastHiddenGraphs(model, gemm_libraries=None)
    rng = np.random.default_rng(14)
    for n, mask in ((40, np.zeros(40, np.int64)), (40, np.r_[np.zeros(39, np.int64), 1]),
                    (1, np.ones(1, np.int64))):
        ids = rng.integers(0, cfg.vocab, size=n)
        got = graphs(ids, mask)
        exp = backbone.backbone_last_hidden(model, ids, mask)
        assert np.array_equal(_bits(got), _bits(exp)), (n, mask.sum())
        ref = forward.backbone_hidden(weights, cfg.as_dict(), ids, mask)[-1]
        assert normwise(got, ref) <= 1e-5, (n, normwise(got, ref))
    assert set(graphs._entries) == {(40, True), (1, False)}


def test_graph_input_checks():
    from qdc_amd import backbone
    from qdc_amd.config import synthetic_inference_config
    from qdc_amd.graphs import LastHiddenGraphs
    from qdc_amd.weights import random_weights
    cfg = synthetic_inference_config()
    model = backbone.QwenBackbone.from_weights(random_weights(cfg, seed=1), cfg, "cuda:0")
    graphs = LastHiddenGraphs(model, gemm_libraries=None)
    for ids, mask in (([1, 2], [1]), ([], []), ([1, 256], [1, 1]), ([-1], [1]), ([1, 2], [1, 2])):
        with pytest.raises(ValueError):
            graphs(ids, mask)
    assert not graphs._entries        # nothing recorded for rejected inputs
    row = graphs(np.array([[3, 4, 5, 6]]), np.ones((1, 4), np.int64))   # a [1, S] array
    assert np.array_equal(_bits(row), _bits(backbone.backbone_last_hidden(model, [3, 4, 5, 6],
                                                                         [1, 1, 1, 1])))
    with pytest.raises(ValueError):
        LastHiddenGraphs(model, max_graphs=0)
    with pytest.raises(ValueError):
        LastHiddenGraphs(model, trials=0)

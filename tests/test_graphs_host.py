"""Host logic of the graph-replayed last-token forward (``qdc_amd.graphs``) on the
CPU, with recording replaced by a stub: the cache keys, least-recently-used
eviction, the eager fallback for a recording that holds a memset node, and the
input checks made before anything is recorded."""
import types

import numpy as np
import pytest

from qdc_amd import graphs as G
from qdc_amd.config import synthetic_inference_config


class _Model:
    def __init__(self):
        self.cfg = synthetic_inference_config()
        self.vocab = self.cfg.vocab
        self.device = "cpu"


def _stub(monkeypatch, memset_keys=()):
    recorded = []

    def record(self, seq_len, masked):   # None: every recording held a memset node
        recorded.append((seq_len, masked))
        if (seq_len, masked) in memset_keys:
            return None
        return types.SimpleNamespace(nodes=[0, 1, 0], key=(seq_len, masked))

    monkeypatch.setattr(G.LastHiddenGraphs, "_record", record)
    return recorded


def test_keys_and_eviction(monkeypatch):
    recorded = _stub(monkeypatch)
    g = G.LastHiddenGraphs(_Model(), max_graphs=2)
    a = g.entry(64, False)
    assert a.key == (64, False) and g.entry(64, False) is a      # kept, not recorded again
    g.entry(64, True)                                           # masked: its own key
    g.entry(64, False)                                          # (64, False) most recent now
    g.entry(128, False)                                         # evicts (64, True)
    assert list(g._entries) == [(64, False), (128, False)]
    assert recorded == [(64, False), (64, True), (128, False)]
    g.entry(64, True)                                           # recorded again
    assert recorded[-1] == (64, True) and len(g._entries) == 2


def test_key_without_usable_recording_served_eagerly(monkeypatch):
    recorded = _stub(monkeypatch, memset_keys={(37, False)})
    g = G.LastHiddenGraphs(_Model())
    assert g.entry(37, False) is None
    assert (37, False) in g.eager_keys and (37, False) not in g._entries
    assert g.entry(37, False) is None and recorded == [(37, False)]   # not recorded twice
    assert g.entry(38, False) is not None


def test_inputs_checked_before_recording(monkeypatch):
    recorded = _stub(monkeypatch)
    g = G.LastHiddenGraphs(_Model())
    for ids, mask in (([1, 2], [1]), ([], []), ([1, 256], [1, 1]), ([-1], [1]),
                      ([1, 2], [1, 2]), (np.ones((2, 3), int), np.ones((2, 3), int))):
        with pytest.raises(ValueError):
            g(ids, mask)
    assert recorded == []
    with pytest.raises(ValueError):
        G.LastHiddenGraphs(_Model(), max_graphs=0)
    with pytest.raises(ValueError):
        G.LastHiddenGraphs(_Model(), trials=0)

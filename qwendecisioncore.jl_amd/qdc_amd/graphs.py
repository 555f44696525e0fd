"""HIP-graph replay of the last-token forward, for a decision model that scores
one prompt after another.

A short single sequence is launch-bound: one forward of a 4-layer hybrid model
is ~48 kernel launches of a few microseconds each, and the host work of
issuing them (Python, ctypes, torch dispatch) costs more than the kernels.
:class:`LastHiddenGraphs` records the whole forward of
:func:`backbone.backbone_last_hidden` once per (sequence length, masked or not)
into a HIP graph with static device buffers for the ids and the mask, then
serves each call with one host-to-device copy of the inputs, one graph launch
and one device-to-host copy of the ``[hidden]`` result.  The reference's CUDA
backend records CUDA graphs for the same calls (``benchmark/README.md``: "CUDA
graph recording [is] excluded" from its ``backbone_last_hidden`` timing).
Each key is recorded with both of torch's GEMM libraries on ROCm and the
recording that replays faster is kept: at a few hundred tokens the products
are small, and the library whose kernels are tiled for large problems can
leave most of the chip idle.

Every captured graph is inspected before first use: a graph holding a memset
node is dropped and its key served eagerly, since memset nodes in replayed
graphs have produced wrong results after the first replay on this platform.
The forward's own kernels clear nothing with memsets; the check guards the
library calls inside it (GEMMs) whose node kinds are not under this package's
control.
"""
from __future__ import annotations

import ctypes
import re
import threading
from collections import OrderedDict

import numpy as np
import torch

from . import backbone as bb

MEMSET_NODE, CHILD_GRAPH_NODE = 2, 4   # hipGraphNodeTypeMemset, hipGraphNodeTypeGraph
_hip_lib = None


def _hip():
    """The HIP runtime this process already runs (the copy torch loaded), by its
    exact path so that no second runtime is mapped."""
    global _hip_lib
    if _hip_lib is None:
        path = "libamdhip64.so.7"
        try:
            with open("/proc/self/maps") as f:
                found = re.findall(r"(/\S*libamdhip64\.so\S*)", f.read())
            if found:
                path = found[0]
        except OSError:
            pass
        lib = ctypes.CDLL(path)
        vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        lib.hipGraphGetNodes.argtypes = [vp, ctypes.POINTER(vp), ctypes.POINTER(sz)]
        lib.hipGraphGetNodes.restype = i32
        lib.hipGraphNodeGetType.argtypes = [vp, ctypes.POINTER(i32)]
        lib.hipGraphNodeGetType.restype = i32
        lib.hipGraphChildGraphNodeGetGraph.argtypes = [vp, ctypes.POINTER(vp)]
        lib.hipGraphChildGraphNodeGetGraph.restype = i32
        _hip_lib = lib
    return _hip_lib


def _ok(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed with hipError_t {status}")


def node_types(graph: int) -> list:
    """The hipGraphNodeType of every node of a hipGraph_t, child graphs included."""
    hip = _hip()
    n = ctypes.c_size_t(0)
    _ok(hip.hipGraphGetNodes(graph, None, ctypes.byref(n)), "hipGraphGetNodes")
    nodes = (ctypes.c_void_p * max(n.value, 1))()
    _ok(hip.hipGraphGetNodes(graph, nodes, ctypes.byref(n)), "hipGraphGetNodes")
    types = []
    for node in nodes[:n.value]:
        t = ctypes.c_int(-1)
        _ok(hip.hipGraphNodeGetType(node, ctypes.byref(t)), "hipGraphNodeGetType")
        types.append(t.value)
        if t.value == CHILD_GRAPH_NODE:
            child = ctypes.c_void_p()
            _ok(hip.hipGraphChildGraphNodeGetGraph(node, ctypes.byref(child)),
                "hipGraphChildGraphNodeGetGraph")
            types.extend(node_types(child.value))
    return types


class _Entry:
    """One recorded forward: static inputs, the graph, its output and a pinned
    host copy of it."""

    def __init__(self, model: bb.QwenBackbone, seq_len: int, masked: bool):
        dev = model.device
        self.ids = torch.zeros((1, seq_len), dtype=torch.int32, device=dev)
        self.mask = torch.ones((1, seq_len), dtype=torch.int32, device=dev) if masked else None
        self.ids_host = torch.zeros((1, seq_len), dtype=torch.int32, pin_memory=True)
        self.mask_host = (torch.ones((1, seq_len), dtype=torch.int32, pin_memory=True)
                          if masked else None)
        self.out_host = torch.empty(model.cfg.hidden, dtype=torch.float32, pin_memory=True)
        self.graph = None
        self.out = None
        self.nodes = []
        self.library = None     # the GEMM library the graph was recorded with
        self.replay_ms = None   # its measured replay time


class LastHiddenGraphs:
    """``backbone_last_hidden`` served from recorded HIP graphs.

    ``graphs(ids, mask)`` returns what ``backbone.backbone_last_hidden(model,
    ids, mask)`` returns, after the same host checks (``check_sequence``).  One
    graph per (sequence length, mask with zeros or not) is recorded on first use
    and kept, least recently used first out beyond ``max_graphs``.

    GEMMs: each key is recorded once per library in ``gemm_libraries`` (torch's
    preferred BLAS library, ``"cublaslt"`` = hipBLASLt and ``"cublas"`` =
    rocBLAS on ROCm; the process-wide setting is restored after recording) and
    the recording with the fastest replay is kept.  At short sequences the two
    libraries pick very different kernels for the same small products (the
    large-problem tiles of one can leave most of the chip idle).  All other
    kernels are the eager forward's, so results equal the eager forward's bit
    for bit when the kept library is the one the eager forward uses, and within
    fp32 rounding of the products otherwise.  ``gemm_libraries=None`` records
    with the current library only.

    A recording holding a memset node is not used; a key with no usable
    recording is served by the eager forward (``eager_keys``).  One call at a
    time per instance (a lock, as the reference's per-model lock); the model's
    weights must not change while graphs exist."""

    def __init__(self, model: bb.QwenBackbone, max_graphs: int = 8,
                 gemm_libraries=("cublaslt", "cublas"), trials: int = 5):
        if max_graphs < 1:
            raise ValueError("max_graphs must be at least 1.")
        if trials < 1:
            raise ValueError("trials must be at least 1.")
        self.model = model
        self.max_graphs = max_graphs
        self.gemm_libraries = tuple(gemm_libraries) if gemm_libraries else None
        self.trials = trials
        self._entries: OrderedDict = OrderedDict()
        self.eager_keys: set = set()
        self._lock = threading.Lock()
        self._stream = None   # the recording stream, made at the first recording

    def _forward(self, e: _Entry) -> torch.Tensor:
        return self.model.forward(e.ids, e.mask, last_only=True)[0]

    def _record_one(self, seq_len: int, masked: bool) -> _Entry:
        e = _Entry(self.model, seq_len, masked)
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=self.model.device)
        cur = torch.cuda.current_stream(self.model.device)
        self._stream.wait_stream(cur)
        with torch.cuda.stream(self._stream):
            for _ in range(2):    # library handles, RoPE tables and workspaces first
                self._forward(e)
        cur.wait_stream(self._stream)
        torch.cuda.synchronize(self.model.device)
        graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(graph, stream=self._stream):
            e.out = self._forward(e)
        e.nodes = node_types(graph.raw_cuda_graph())
        graph.instantiate()
        e.graph = graph
        return e

    def _replay_ms(self, e: _Entry) -> float:
        stream = torch.cuda.current_stream(self.model.device)
        e.graph.replay()                       # first replay: uploads the graph
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(self.trials):
            e.graph.replay()
        end.record(stream)
        end.synchronize()
        return start.elapsed_time(end) / self.trials

    def _record(self, seq_len: int, masked: bool):
        """The fastest usable recording of this key over the GEMM libraries, or
        None when every recording holds a memset node."""
        backends = torch.backends.cuda
        previous = backends.preferred_blas_library()
        best = None
        try:
            with torch.cuda.device(self.model.device):
                for library in self.gemm_libraries or (previous,):
                    backends.preferred_blas_library(library)
                    e = self._record_one(seq_len, masked)
                    if MEMSET_NODE in e.nodes:
                        continue
                    e.library = str(library)
                    e.replay_ms = self._replay_ms(e)
                    if best is None or e.replay_ms < best.replay_ms:
                        best = e
        finally:
            backends.preferred_blas_library(previous)
        return best

    def entry(self, seq_len: int, masked: bool):
        """The recorded forward for this key (recording it now if needed), or
        None when the key is served eagerly."""
        key = (seq_len, masked)
        if key in self.eager_keys:
            return None
        e = self._entries.get(key)
        if e is None:
            e = self._record(seq_len, masked)
            if e is None:
                self.eager_keys.add(key)
                return None
            self._entries[key] = e
            while len(self._entries) > self.max_graphs:
                self._entries.popitem(last=False)
        self._entries.move_to_end(key)
        return e

    def __call__(self, ids, mask) -> np.ndarray:
        ids, mask = bb._host_sequence(self.model, ids, mask)
        with self._lock:
            masked = not bool(mask.all())
            e = self.entry(ids.size, masked)
            if e is None:
                return bb.backbone_last_hidden(self.model, ids, mask)
            with torch.cuda.device(self.model.device):
                stream = torch.cuda.current_stream(self.model.device)
                e.ids_host[0].numpy()[:] = ids
                e.ids.copy_(e.ids_host, non_blocking=True)
                if masked:
                    e.mask_host[0].numpy()[:] = mask
                    e.mask.copy_(e.mask_host, non_blocking=True)
                e.graph.replay()
                e.out_host.copy_(e.out.float(), non_blocking=True)
                stream.synchronize()
                return e.out_host.numpy().copy()

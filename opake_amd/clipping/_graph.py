"""HIP-graph replay of the ghost clip -> sum step.

The counterpart of the reference's ``CudaGraphChunkCompiler``
(packages/opake-engine/src/opake/api/engine/clipping/_cuda_graph.py:1-219):
each distinct operand signature of :func:`ghost_clip_captured` -- the norm,
clip-factor and clipped-sum kernels of every layer -- is captured once as a
HIP graph (``torch.cuda.CUDAGraph`` on ROCm) and replayed afterwards, which
removes the per-call Python and launch overhead of steps made of many small
layers.

Rules, as in the reference:

* the capture key is every operand's shape, stride and dtype plus the
  layers' names, row segments and options; a new signature is captured anew
  (up to ``max_graphs``, then it runs eagerly);
* before every replay the operands are copied into the graph's static input
  buffers, and the outputs are cloned on return (the next replay overwrites
  them);
* warm-up runs before the first capture happen on a side stream, so one-time
  initialisation (library load, cached device tables) is not recorded;
* the graph holds no noise: like the reference's chunk kernel it produces the
  clipped sum, and the noise mechanism is applied to the result afterwards (the
  noise key changes every step, a replayed graph would repeat it).

Every device table a kernel reads comes from a content-keyed cache that keeps
its pinned host source alive, so the recorded copies stay valid; each graph
entry also holds every table its capture used, so none is freed while the
graph can replay; the leaf, norm, clip-factor and clipped-sum kernels record
no memset.
"""

from __future__ import annotations

import torch

from opake_amd import _tables
from opake_amd.clipping._model import DirectCapture, LinearCapture, ghost_clip_captured
from opake_amd.exceptions import ConfigurationError
from opake_amd.types import clipped


def _tensor_key(t: torch.Tensor) -> tuple:
    return (tuple(t.shape), tuple(t.stride()), t.dtype, str(t.device))


def _signature(captures) -> tuple:
    key = []
    for c in captures:
        if isinstance(c, LinearCapture):
            key.append(("linear", c.name, _tensor_key(c.A), _tensor_key(c.G), c.has_bias,
                        None if c.segments is None else tuple(c.segments), c.param_dtype,
                        c.norm_method))
        elif isinstance(c, DirectCapture):
            key.append(("direct", tuple((n, _tensor_key(t)) for n, t in sorted(c.grads.items()))))
        else:
            raise ConfigurationError(f"unsupported capture {type(c).__name__}")
    return tuple(key)


def _static_copy(captures):
    out = []
    for c in captures:
        if isinstance(c, LinearCapture):
            out.append(LinearCapture(name=c.name, A=c.A.detach().clone(), G=c.G.detach().clone(),
                                     has_bias=c.has_bias, segments=c.segments,
                                     param_dtype=c.param_dtype, norm_method=c.norm_method))
        else:
            out.append(DirectCapture({n: t.detach().clone() for n, t in c.grads.items()}))
    return out


def _tensors(captures):
    ts = []
    for c in captures:
        if isinstance(c, LinearCapture):
            ts.extend([c.A, c.G])
        else:
            ts.extend(t for _, t in sorted(c.grads.items()))
    return ts


class GraphedGhostClip:
    """``ghost_clip_captured(captures, clipping_norm=..., normalize_by=...,
    dtype=...)`` replayed from a HIP graph per operand signature.

    One instance owns one graph memory pool shared by its captures; use one
    per training run.  Calling it returns a ``ClippedPytree`` (clones of the
    graph's outputs).
    """

    def __init__(self, *, clipping_norm, normalize_by: float = 1.0,
                 dtype: torch.dtype | None = None, warmup_runs: int = 2, max_graphs: int = 4):
        if warmup_runs < 1:
            raise ConfigurationError("warmup_runs must be >= 1")
        if isinstance(max_graphs, bool) or not isinstance(max_graphs, int) or max_graphs < 1:
            raise ConfigurationError(f"max_graphs must be a positive integer; got {max_graphs!r}.")
        self.clipping_norm = clipping_norm
        self.normalize_by = normalize_by
        self.dtype = dtype
        self.warmup_runs = warmup_runs
        self.max_graphs = max_graphs
        self.captures = 0
        self.replays = 0
        self._pool = None
        self._graphs: dict = {}

    def _eager(self, captures):
        return ghost_clip_captured(captures, clipping_norm=self.clipping_norm,
                                   normalize_by=self.normalize_by, dtype=self.dtype)

    def _capture(self, captures):
        static = _static_copy(captures)
        device = _tensors(static)[0].device
        with torch.cuda.device(device):
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(self.warmup_runs):
                    self._eager(static)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            if self._pool is None:
                self._pool = torch.cuda.graph_pool_handle()
            graph = torch.cuda.CUDAGraph()
            # The device tables the captured kernels read (cache hits made
            # during warm-up included) stay referenced by the entry, so a
            # later eviction from the table cache cannot free them.
            with _tables.keep_alive() as tables, torch.cuda.graph(graph, pool=self._pool):
                out = self._eager(static)
            torch.cuda.synchronize()
        self.captures += 1
        return graph, static, out, tables

    def __call__(self, captures):
        key = _signature(captures)
        entry = self._graphs.get(key)
        if entry is None:
            if self.captures >= self.max_graphs:
                return self._eager(captures)
            entry = self._graphs[key] = self._capture(captures)
        graph, static, out, _ = entry
        torch._foreach_copy_(_tensors(static), [t.detach() for t in _tensors(captures)])
        graph.replay()
        self.replays += 1
        tree = {k: v.clone() for k, v in out.pytree.items()}
        return clipped(tree, max_norm=out.max_norm)


__all__ = ["GraphedGhostClip"]

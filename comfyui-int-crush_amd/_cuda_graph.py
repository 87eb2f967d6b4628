"""hipGraph replay of the INT8 linear (prep + quantize + GEMM).

Counterpart of the reference's _cuda_graph.py:80-297 with the same contract:
one runner per qualifying INT8 Linear, an LRU of at most four captured
graphs keyed (M, N, K, dtype, has_bias), static input/intermediate/output
buffers owned by the cache entry, a bias-identity check before replay, and
no-clone replay that returns the static output buffer (the caller consumes
it before the next replay, as in sequential inference).

On ROCm `torch.cuda.CUDAGraph` records a hipGraph.  The captured work is two
kernel launches of libintcrush_gfx950.so (the fused prep+quantize kernel and
the W8A8 GEMM) on the capture stream; neither allocates, synchronises or
clears memory, so the graph holds kernel nodes only.
"""
from __future__ import annotations

import logging
from collections import OrderedDict

import torch

from . import _hip_runtime as _rt

log = logging.getLogger(__name__)

__all__ = ["CudaGraphRunner", "HipGraphRunner"]


class _GraphEntry:
    """A captured graph and the buffers it reads and writes; every one of them
    must stay referenced for the graph's lifetime (_cuda_graph.py:30-77)."""

    __slots__ = ("graph", "static_x", "static_x_int8", "static_s_a", "static_out", "bias_snapshot", "_no_clone")

    def __init__(self, graph, static_x, static_x_int8, static_s_a, static_out, bias_snapshot, no_clone=False):
        self.graph = graph
        self.static_x = static_x
        self.static_x_int8 = static_x_int8
        self.static_s_a = static_s_a
        self.static_out = static_out
        self.bias_snapshot = bias_snapshot
        self._no_clone = no_clone

    def replay(self, x_2d: torch.Tensor) -> torch.Tensor:
        self.static_x.copy_(x_2d)
        self.graph.replay()
        return self.static_out if self._no_clone else self.static_out.clone()


class CudaGraphRunner:
    """Per-layer graph cache for the INT8 path (_cuda_graph.py:80-297).

    Reads the layer's quantized weight, scales and preparation tensors once;
    `run(x, bias, compute_dtype)` returns [M, out_features] in compute_dtype.
    """

    _MAX_CACHED_SHAPES: int = 4

    def __init__(self, layer, safe_no_clone: bool = True, max_cached_shapes: int | None = None) -> None:
        self._layer = layer
        self._w_int8: torch.Tensor = layer.weight._qdata
        self._s_w: torch.Tensor = layer.weight._params.scale
        self._zp = layer.weight._params.zp
        self._rot_size: int = layer._intcrush_rot_size if layer._intcrush_rot_need else 0
        self._safe_no_clone = safe_no_clone
        self._max_cached = max_cached_shapes if max_cached_shapes is not None else self._MAX_CACHED_SHAPES
        self._graphs: OrderedDict[tuple, _GraphEntry] = OrderedDict()

    # ── public API ────────────────────────────────────────────────────────
    def run(self, x: torch.Tensor, bias: torch.Tensor | None, compute_dtype: torch.dtype) -> torch.Tensor:
        x_2d = x.reshape(-1, x.shape[-1])
        M, K = x_2d.shape
        N = self._w_int8.shape[0]
        if self._zp is not None:
            return self._run_eager(x_2d, bias, compute_dtype)
        key = (M, N, K, x.dtype, bias is not None)
        entry = self._graphs.get(key)
        if entry is not None:
            if entry.bias_snapshot is bias:
                self._graphs.move_to_end(key)
                return entry.replay(x_2d)
            del self._graphs[key]  # bias object changed: capture again
        out = self._run_eager(x_2d, bias, compute_dtype)
        self._capture(key, x_2d, bias, compute_dtype)
        while len(self._graphs) > self._max_cached:
            self._graphs.popitem(last=False)
            log.debug("[INT-Crush] evicted the oldest graph entry")
        return out

    def invalidate(self) -> None:
        self._graphs.clear()

    def cached_keys(self) -> list[tuple]:
        return list(self._graphs.keys())

    # ── internals ─────────────────────────────────────────────────────────
    def _prep_and_quantize(self, x_2d, bias, compute_dtype, *, s_a_out=None, x_int8_out=None, out=None):
        st = self._layer._intcrush_state(x_2d)
        # at the GEMM's width (the layer's prepared width unless it is padded
        # to a multiple of 128 for the MFMA kernels)
        q, s_a = _rt.rotate_quantize(x_2d, rot_size=self._rot_size, w_in=st.k_gemm, smoothrot=st.smoothrot,
                                     perm=st.perm_gemm, smooth=st.smooth_gemm, s_a_out=s_a_out,
                                     x_int8_out=x_int8_out)
        wq, ws = st.gemm_weights(self._w_int8, self._s_w)
        return _rt.fused_int8_gemm_dequant(q, wq, ws, s_a, bias=bias, out_dtype=compute_dtype, out=out)

    def _run_eager(self, x_2d, bias, compute_dtype):
        return self._prep_and_quantize(x_2d, bias, compute_dtype)

    def _capture(self, key, x_2d, bias, compute_dtype) -> None:
        M, K = x_2d.shape
        N = self._w_int8.shape[0]
        dev = x_2d.device
        static_x = torch.empty(M, K, dtype=x_2d.dtype, device=dev)
        static_x_int8 = torch.empty(M, self._layer._intcrush_state(x_2d).k_gemm, dtype=torch.int8, device=dev)
        static_s_a = torch.empty(M, dtype=torch.float32, device=dev)
        static_out = torch.empty(M, N, dtype=compute_dtype, device=dev)
        static_x.copy_(x_2d)
        # every per-layer preparation tensor exists before capture starts
        self._layer._intcrush_state(static_x)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._prep_and_quantize(static_x, bias, compute_dtype, s_a_out=static_s_a,
                                    x_int8_out=static_x_int8, out=static_out)
        self._graphs[key] = _GraphEntry(graph, static_x, static_x_int8, static_s_a, static_out, bias,
                                        no_clone=self._safe_no_clone)
        log.debug("[INT-Crush] captured hipGraph M=%d N=%d K=%d dtype=%s bias=%s", M, N, K, compute_dtype,
                  bias is not None)


HipGraphRunner = CudaGraphRunner

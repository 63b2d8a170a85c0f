"""MetalComputeProvider — the VectorCore integration façade over the C ABI.

Reference: Integration/MetalComputeProvider.swift (batchDistance :119-154, findNearest
:174-217, selectTopK :219-226, the BatchKernelProvider conformance :228-269, distanceMatrix
:270-).  VectorCore's `Operations.findNearest` / `batchDistance` reach the GPU through it.

Semantics kept from the reference:
  * batchDistance: euclidean -> L2 distance (sqrt of L2^2), cosine -> 1 - similarity (the GPU
    rule: FLT_MIN floor, NaN-preserving clamp), dotProduct -> the raw dot product;
  * findNearest(metric: SupportedDistanceMetric): the min(k, count) nearest candidates as
    (index, distance) pairs, nearest first; for dotProduct "nearest" is the largest dot
    (selectTopK's largerIsCloser) and the value returned is the raw dot;
  * the BatchKernelProvider conformance (metric objects of VectorCore): EuclideanDistance and
    CosineDistance as above, DotProductDistance as VectorCore defines it, -dot, ascending;
  * distanceMatrix: row i is batchDistance(queries[i], candidates).
Every distance and selection runs in libva_hip.so (va_l2_all_pairs, va_cosine_all_pairs,
va_dot_all_pairs, va_fused_topk); ties order by candidate index (the reference's sort leaves
them unspecified).  The reference computes manhattan and chebyshev on the CPU (Accelerate); this
build has no CPU path and no GPU kernel for them, so they raise VectorError("unsupported").
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import Enum

import numpy as np

from . import _lib
from .context import GPUContext, VectorError, dptr
from .kernels import _as_matrix


def _torch():
    import torch

    return torch


class SupportedDistanceMetric(str, Enum):
    """VectorCore's SupportedDistanceMetric."""

    euclidean = "euclidean"
    cosine = "cosine"
    dotProduct = "dotProduct"
    manhattan = "manhattan"
    chebyshev = "chebyshev"


# VectorCore's DistanceMetric types, as the BatchKernelProvider conformance sees them
class EuclideanDistance:
    pass


class CosineDistance:
    pass


class DotProductDistance:
    """VectorCore's dot-product distance: -dot (smaller is nearer)."""


@dataclass
class Configuration:
    """MetalComputeProvider.Configuration: the reference's routing knobs.  Every operation runs on
    the GPU here, so preferGPU must stay True and there is no CPU fallback to enable."""

    preferGPU: bool = True
    fallbackToCPU: bool = False

    def validate(self):
        if not self.preferGPU or self.fallbackToCPU:
            raise VectorError("unsupported", "this build computes on the GPU only (no CPU path)")


class MetalComputeProvider:
    def __init__(self, context: GPUContext | None = None, configuration: Configuration | None = None):
        self.configuration = configuration or Configuration()
        self.configuration.validate()
        self.context = context or GPUContext(0)

    @classmethod
    def makeDefault(cls) -> "MetalComputeProvider":
        return cls()

    # -- helpers --------------------------------------------------------------------------------
    def _operands(self, queries, candidates):
        q = _as_matrix(queries, "query")
        x = _as_matrix(candidates, "candidates")
        if x.shape[1] != q.shape[1]:
            raise VectorError.invalidInput(f"All candidates must match the query dimension ({q.shape[1]})")
        c = self.context
        return q, x, c.buffer(q), c.buffer(x)

    @staticmethod
    def _check_metric(metric) -> SupportedDistanceMetric:
        m = SupportedDistanceMetric(metric)
        if m in (SupportedDistanceMetric.manhattan, SupportedDistanceMetric.chebyshev):
            raise VectorError("unsupported", f"{m.value} has no GPU kernel in this build")
        return m

    def _matrix(self, q, x, qd, xd, m: SupportedDistanceMetric) -> np.ndarray:
        torch = _torch()
        c = self.context
        out = c.empty((q.shape[0], x.shape[0]), torch.float32)
        c.order_after_torch()
        Q, N, D = q.shape[0], x.shape[0], q.shape[1]
        if m is SupportedDistanceMetric.euclidean:
            st = c.lib.va_l2_all_pairs(c.handle, dptr(qd), dptr(xd), dptr(out), Q, N, D, 1)
        elif m is SupportedDistanceMetric.cosine:
            st = c.lib.va_cosine_all_pairs(c.handle, dptr(qd), dptr(xd), dptr(out), Q, N, D, 1)
        else:
            st = c.lib.va_dot_all_pairs(c.handle, dptr(qd), dptr(xd), dptr(out), Q, N, D, 0)
        c.check(st, "MetalComputeProvider.batchDistance")
        c.synchronize()
        return out.cpu().numpy()

    def _topk(self, q, x, qd, xd, k: int, va_metric: int):
        torch = _torch()
        c = self.context
        Q = q.shape[0]
        idx = c.empty((Q, k), torch.int32)
        dist = c.empty((Q, k), torch.float32)
        c.order_after_torch()
        c.check(c.lib.va_fused_topk(c.handle, va_metric, dptr(qd), dptr(xd), Q, x.shape[0], q.shape[1], k, dptr(idx),
                                    dptr(dist)), "MetalComputeProvider.findNearest")
        c.synchronize()
        return idx.cpu().numpy().view(np.uint32), dist.cpu().numpy()

    # -- batch distance ---------------------------------------------------------------------------
    def batchDistance(self, query, candidates, metric) -> list[float]:
        """Distance from `query` to each candidate, in candidate order (MetalComputeProvider.swift:119-154).
        `metric`: a SupportedDistanceMetric, or a VectorCore metric object (the conformance,
        :228-253: DotProductDistance gives -dot)."""
        if len(candidates) == 0:
            return []
        neg = isinstance(metric, DotProductDistance)
        m = self._conformance_metric(metric)
        q, x, qd, xd = self._operands([query], candidates)
        row = self._matrix(q, x, qd, xd, m)[0]
        return (-row if neg else row).tolist()

    def distanceMatrix(self, queries, candidates, metric) -> list[list[float]]:
        """queries x candidates; row i is batchDistance(queries[i], candidates)."""
        if len(queries) == 0 or len(candidates) == 0:
            return []
        m = self._check_metric(metric)
        q, x, qd, xd = self._operands(queries, candidates)
        return self._matrix(q, x, qd, xd, m).tolist()

    # -- k nearest neighbours ------------------------------------------------------------------------
    def _conformance_metric(self, metric) -> SupportedDistanceMetric:
        if isinstance(metric, EuclideanDistance):
            return SupportedDistanceMetric.euclidean
        if isinstance(metric, CosineDistance):
            return SupportedDistanceMetric.cosine
        if isinstance(metric, DotProductDistance):
            return SupportedDistanceMetric.dotProduct
        return self._check_metric(metric)

    def findNearest(self, query, candidates, k: int, metric) -> list[tuple[int, float]]:
        """The min(k, count) nearest candidates as (index, distance), nearest first
        (MetalComputeProvider.swift:174-217; with a VectorCore metric object, :255-265)."""
        return self.findNearestBatch([query], candidates, k, metric)[0] if k > 0 and len(candidates) else []

    def findNearestBatch(self, queries, candidates, k: int, metric) -> list[list[tuple[int, float]]]:
        """findNearest for every query, in one GPU dispatch."""
        if k <= 0 or len(candidates) == 0 or len(queries) == 0:
            return [[] for _ in range(len(queries))]
        vc_dot = isinstance(metric, DotProductDistance)
        m = self._conformance_metric(metric)
        q, x, qd, xd = self._operands(queries, candidates)
        kk = min(k, x.shape[0], _lib.VA_MAX_K)
        if k > _lib.VA_MAX_K and x.shape[0] > _lib.VA_MAX_K:
            raise VectorError.invalidInput(f"k {k} exceeds maximum supported k {_lib.VA_MAX_K}")
        vm = {SupportedDistanceMetric.euclidean: _lib.VA_METRIC_L2, SupportedDistanceMetric.cosine: _lib.VA_METRIC_COSINE,
              SupportedDistanceMetric.dotProduct: _lib.VA_METRIC_DOT}[m]
        idx, dist = self._topk(q, x, qd, xd, kk, vm)
        out = []
        for r in range(q.shape[0]):
            pairs = []
            for i, d in zip(idx[r], dist[r]):
                if i == _lib.VA_SENTINEL_INDEX:
                    break
                d = float(d)
                # va_fused_topk's DOT distance is -dot: the enum's dotProduct reports the raw dot
                # (largest first), VectorCore's DotProductDistance the -dot itself (ascending)
                pairs.append((int(i), d if (m is not SupportedDistanceMetric.dotProduct or vc_dot) else -d))
            out.append(pairs)
        return out

"""Distance and top-K kernels — host mirror of the reference's Metal4 kernel wrappers.

Each class keeps the reference's name and tiers:
  * ``encode(...)``   device tensors in, enqueue only (the encode(into:) tier);
  * ``execute(...)``  device tensors in, outputs allocated, waits (executeAndWait);
  * ``compute(...)`` / ``findNearestNeighbors(...)`` / ``select(...)`` host arrays in and out.
All arithmetic runs in libva_hip.so; this module only validates, allocates and converts.
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import IntEnum

import numpy as np

from . import _lib
from .context import GPUContext, VectorError, dptr


def _torch():
    import torch

    return torch


def _as_matrix(rows, name: str) -> np.ndarray:
    """[[Float]] (or a 2-D array) -> contiguous float32 matrix, with the reference's checks."""
    if rows is None or len(rows) == 0:
        raise VectorError.invalidInput(f"Empty input {name}")
    if isinstance(rows, np.ndarray):
        m = np.ascontiguousarray(rows, dtype=np.float32)
        if m.ndim != 2:
            raise VectorError.invalidInput(f"{name} must be 2-D")
        return m
    dim = len(rows[0])
    if any(len(r) != dim for r in rows):
        raise VectorError.invalidInput("Dimension mismatch in input vectors")
    return np.ascontiguousarray(np.asarray(rows, dtype=np.float32).reshape(len(rows), dim))


# ---------------------------------------------------------------------------------------
# 1:1 distances
# ---------------------------------------------------------------------------------------
class L2DistanceKernel:
    """1:1 L2 distance (Kernels/Metal4/L2DistanceKernel.swift:19-90)."""

    name = "L2DistanceKernel"

    def __init__(self, context: GPUContext):
        self.context = context

    def encode(self, queries, targets, distances, numQueries: int, dimension: int, computeSqrt: bool = True):
        c = self.context
        c.check(
            c.lib.va_l2_pairs(c.handle, dptr(queries), dptr(targets), dptr(distances), numQueries, dimension,
                              int(bool(computeSqrt))),
            "L2DistanceKernel.encode",
        )

    def compute(self, queries, targets, computeSqrt: bool = True) -> np.ndarray:
        q = _as_matrix(queries, "queries")
        t = _as_matrix(targets, "targets")
        if q.shape != t.shape:
            raise VectorError.invalidInput("queries and targets must pair 1:1")
        c = self.context
        dq, dt = c.buffer(q), c.buffer(t)
        out = c.empty((q.shape[0],), _torch().float32)
        c.order_after_torch()
        self.encode(dq, dt, out, q.shape[0], q.shape[1], computeSqrt)
        c.synchronize()
        return out.cpu().numpy()

    def allPairs(self, queries, database, computeSqrt: bool = True) -> np.ndarray:
        """Q x N matrix (the l2AllPairs test helper's replication, done natively)."""
        return _all_pairs(self.context, "va_l2_all_pairs", queries, database, int(bool(computeSqrt)))


class CosineSimilarityKernel:
    """1:1 cosine similarity (Kernels/Metal4/CosineSimilarityKernel.swift:19-91)."""

    name = "CosineSimilarityKernel"

    def __init__(self, context: GPUContext):
        self.context = context

    def encode(self, queries, targets, similarities, numQueries: int, dimension: int, outputDistance: bool = False):
        c = self.context
        c.check(
            c.lib.va_cosine_pairs(c.handle, dptr(queries), dptr(targets), dptr(similarities), numQueries, dimension,
                                  int(bool(outputDistance))),
            "CosineSimilarityKernel.encode",
        )

    def compute(self, queries, targets, outputDistance: bool = False) -> np.ndarray:
        q = _as_matrix(queries, "queries")
        t = _as_matrix(targets, "targets")
        if q.shape != t.shape:
            raise VectorError.invalidInput("queries and targets must pair 1:1")
        c = self.context
        dq, dt = c.buffer(q), c.buffer(t)
        out = c.empty((q.shape[0],), _torch().float32)
        c.order_after_torch()
        self.encode(dq, dt, out, q.shape[0], q.shape[1], outputDistance)
        c.synchronize()
        return out.cpu().numpy()

    def allPairs(self, queries, database, outputDistance: bool = False) -> np.ndarray:
        return _all_pairs(self.context, "va_cosine_all_pairs", queries, database, int(bool(outputDistance)))


def _all_pairs(c: GPUContext, fn: str, queries, database, flag: int) -> np.ndarray:
    q = _as_matrix(queries, "queries")
    x = _as_matrix(database, "database")
    if q.shape[1] != x.shape[1]:
        raise VectorError.invalidInput("Dimension mismatch in input vectors")
    dq, dx = c.buffer(q), c.buffer(x)
    out = c.empty((q.shape[0], x.shape[0]), _torch().float32)
    c.order_after_torch()
    c.check(getattr(c.lib, fn)(c.handle, dptr(dq), dptr(dx), dptr(out), q.shape[0], x.shape[0], q.shape[1], flag), fn)
    c.synchronize()
    return out.cpu().numpy()


# ---------------------------------------------------------------------------------------
# all-pairs dot product
# ---------------------------------------------------------------------------------------
@dataclass
class DotProductParameters:
    """DotProductParameters (Kernels/Metal4/DotProductKernel.swift:25-96)."""

    numQueries: int
    numDatabase: int
    dimension: int
    absoluteValue: bool = False

    @property
    def isGEMV(self) -> bool:
        return self.numQueries == 1


class DotProductKernel:
    """All-pairs dot product (Kernels/Metal4/DotProductKernel.swift:136-362)."""

    name = "DotProductKernel"
    optimizedDimensions = [384, 512, 768, 1536]

    def __init__(self, context: GPUContext):
        self.context = context

    def encode(self, queries, database, output, parameters: DotProductParameters):
        c = self.context
        p = parameters
        c.check(
            c.lib.va_dot_all_pairs(c.handle, dptr(queries), dptr(database), dptr(output), p.numQueries,
                                   p.numDatabase, p.dimension, int(bool(p.absoluteValue))),
            "DotProductKernel.encode",
        )

    def execute(self, queries, database, parameters: DotProductParameters):
        c = self.context
        out = c.empty((parameters.numQueries, parameters.numDatabase), _torch().float32)
        c.order_after_torch()
        self.encode(queries, database, out, parameters)
        c.synchronize()
        return out

    def compute(self, queries, database, absoluteValue: bool = False) -> np.ndarray:
        return _all_pairs(self.context, "va_dot_all_pairs", queries, database, int(bool(absoluteValue)))

    def computeSingle(self, query, database, absoluteValue: bool = False) -> np.ndarray:
        return self.compute([list(query)], database, absoluteValue)[0]


# ---------------------------------------------------------------------------------------
# fused distance + top-k
# ---------------------------------------------------------------------------------------
class Metric(IntEnum):
    """Distances the fused kernel ranks by (ascending)."""

    euclideanSquared = _lib.VA_METRIC_L2SQ
    cosine = _lib.VA_METRIC_COSINE
    dotProduct = _lib.VA_METRIC_DOT
    euclidean = _lib.VA_METRIC_L2


@dataclass
class FusedL2TopKParameters:
    """FusedL2TopKParameters (Kernels/Metal4/FusedL2TopKKernel.swift:25-86).

    The reference throws for dimension > 768 and k > 128 (limits of its shader); this
    library accepts any dimension and k <= VA_MAX_K (1024).
    """

    numQueries: int
    numDataset: int
    dimension: int
    k: int
    maxK = _lib.VA_MAX_K

    def __post_init__(self):
        if self.numQueries <= 0:
            raise VectorError.invalidInput(f"numQueries must be positive, got {self.numQueries}")
        if self.numDataset <= 0:
            raise VectorError.invalidInput(f"numDataset must be positive, got {self.numDataset}")
        if self.dimension <= 0:
            raise VectorError.invalidInput(f"dimension must be positive, got {self.dimension}")
        if self.k <= 0:
            raise VectorError.invalidInput(f"k must be positive, got {self.k}")
        if self.k > self.maxK:
            raise VectorError.invalidInput(f"k {self.k} exceeds maximum supported k {self.maxK}")


@dataclass
class Metal4FusedL2Config:
    """Metal4FusedL2Config (FusedL2TopKKernel.swift:91-136).  Only includeDistances matters:
    the scan never materialises the distance matrix, so the matrix-size knobs are moot."""

    includeDistances: bool = True


class Metal4FusedL2TopKResult:
    """Metal4FusedL2TopKResult (FusedL2TopKKernel.swift:140-179)."""

    def __init__(self, indices, distances, numQueries: int, k: int):
        self.indices = indices
        self.distances = distances
        self.numQueries = numQueries
        self.k = k
        self._host = None

    def _fetch(self):
        if self._host is None:
            idx = self.indices.cpu().numpy().view(np.uint32).reshape(self.numQueries, self.k)
            dist = None if self.distances is None else self.distances.cpu().numpy().reshape(self.numQueries, self.k)
            self._host = (idx, dist)
        return self._host

    def results(self, queryIndex: int) -> list[tuple[int, float]]:
        if queryIndex >= self.numQueries:
            return []
        idx, dist = self._fetch()
        out = []
        for i in range(self.k):
            j = int(idx[queryIndex, i])
            if j != _lib.VA_SENTINEL_INDEX:  # skip sentinel values
                out.append((j, float(dist[queryIndex, i]) if dist is not None else 0.0))
        return out

    def allResults(self) -> list[list[tuple[int, float]]]:
        return [self.results(q) for q in range(self.numQueries)]


class FusedL2TopKKernel:
    """Fused distance + exact top-k (Kernels/Metal4/FusedL2TopKKernel.swift:205-1150).

    ``metric`` extends the reference (L2^2 only) with cosine (1 - s), dot (-dot) and L2.
    """

    name = "FusedL2TopKKernel"

    def __init__(self, context: GPUContext):
        self.context = context

    def encode(self, queries, dataset, outputIndices, outputDistances, parameters: FusedL2TopKParameters,
               metric: Metric = Metric.euclideanSquared):
        c = self.context
        p = parameters
        c.check(
            c.lib.va_fused_topk(c.handle, int(metric), dptr(queries), dptr(dataset), p.numQueries, p.numDataset,
                                p.dimension, p.k, dptr(outputIndices), dptr(outputDistances)),
            "FusedL2TopKKernel.encode",
        )

    def execute(self, queries, dataset, parameters: FusedL2TopKParameters,
                config: Metal4FusedL2Config = Metal4FusedL2Config(),
                metric: Metric = Metric.euclideanSquared) -> Metal4FusedL2TopKResult:
        torch = _torch()
        c = self.context
        p = parameters
        idx = c.empty((p.numQueries, p.k), torch.int32)
        dist = c.empty((p.numQueries, p.k), torch.float32) if config.includeDistances else None
        c.order_after_torch()
        self.encode(queries, dataset, idx, dist, p, metric)
        c.synchronize()
        return Metal4FusedL2TopKResult(idx, dist, p.numQueries, p.k)

    def encodeStreamed(self, queries, hostDataset, outputIndices, outputDistances, parameters: FusedL2TopKParameters,
                       metric: Metric = Metric.euclideanSquared, chunkRows: int = 0):
        """The same search over a dataset in host memory (a contiguous float32 CPU tensor, pinned for
        overlapped uploads), streamed through the device in chunks of ``chunkRows`` rows (0 = ~512 MiB)
        and merged into a running top-k: the reference's chunked fallback with GPU merge
        (FusedL2TopKKernel.swift:765-931).  Synchronous."""
        c = self.context
        p = parameters
        if hostDataset.is_cuda or not hostDataset.is_contiguous():
            raise VectorError.invalidInput("hostDataset must be a contiguous host tensor")
        c.check(
            c.lib.va_fused_topk_streamed(c.handle, int(metric), dptr(queries), int(hostDataset.data_ptr()),
                                         p.numQueries, p.numDataset, p.dimension, p.k, int(chunkRows),
                                         dptr(outputIndices), dptr(outputDistances)),
            "FusedL2TopKKernel.encodeStreamed",
        )

    def executeStreamed(self, queries, hostDataset, parameters: FusedL2TopKParameters,
                        metric: Metric = Metric.euclideanSquared, chunkRows: int = 0) -> Metal4FusedL2TopKResult:
        torch = _torch()
        c = self.context
        p = parameters
        idx = c.empty((p.numQueries, p.k), torch.int32)
        dist = c.empty((p.numQueries, p.k), torch.float32)
        c.order_after_torch()
        self.encodeStreamed(queries, hostDataset, idx, dist, p, metric, chunkRows)
        return Metal4FusedL2TopKResult(idx, dist, p.numQueries, p.k)

    def findNearestNeighbors(self, queries, dataset, k: int, includeDistances: bool = True,
                             metric: Metric = Metric.euclideanSquared) -> list[list[tuple[int, float]]]:
        q = _as_matrix(queries, "arrays")
        x = _as_matrix(dataset, "arrays")
        if q.shape[1] != x.shape[1]:
            raise VectorError.invalidInput("Dimension mismatch in input vectors")
        params = FusedL2TopKParameters(q.shape[0], x.shape[0], q.shape[1], k)
        c = self.context
        res = self.execute(c.buffer(q), c.buffer(x), params, Metal4FusedL2Config(includeDistances), metric)
        return res.allResults()


# The reference's alias (VectorAccelerate.swift:288)
FusedTopKKernel = FusedL2TopKKernel


# ---------------------------------------------------------------------------------------
# top-k selection and merge
# ---------------------------------------------------------------------------------------
class Metal4SelectionMode(IntEnum):
    """Metal4SelectionMode (Kernels/Metal4/TopKSelectionKernel.swift:23-29)."""

    minimum = _lib.VA_SELECT_MIN
    maximum = _lib.VA_SELECT_MAX


class TopKSelectionKernel:
    """Row-wise top-k of a value matrix (Kernels/Metal4/TopKSelectionKernel.swift:150-440).

    Unlike the reference's value-only heap (unspecified tie order) the selection is exact
    with ties to the lower index.
    """

    name = "TopKSelectionKernel"
    maxK = _lib.VA_MAX_K

    def __init__(self, context: GPUContext):
        self.context = context

    def encode(self, values, outputIndices, outputValues, batchSize: int, numElements: int, k: int,
               mode: Metal4SelectionMode = Metal4SelectionMode.minimum):
        c = self.context
        c.check(
            c.lib.va_topk_select(c.handle, dptr(values), batchSize, numElements, k, int(mode), dptr(outputIndices),
                                 dptr(outputValues)),
            "TopKSelectionKernel.encode",
        )

    def select(self, values, k: int, mode: Metal4SelectionMode = Metal4SelectionMode.minimum,
               sorted: bool = True) -> list[list[tuple[int, float]]]:
        torch = _torch()
        m = _as_matrix(values, "values")
        rows, n = m.shape
        if k <= 0:
            raise VectorError.invalidInput(f"k must be positive, got {k}")
        kk = min(k, self.maxK)
        c = self.context
        dv = c.buffer(m)
        idx = c.empty((rows, kk), torch.int32)
        val = c.empty((rows, kk), torch.float32)
        c.order_after_torch()
        self.encode(dv, idx, val, rows, n, kk, mode)
        c.synchronize()
        hi = idx.cpu().numpy().view(np.uint32)
        hv = val.cpu().numpy()
        out = []
        for r in range(rows):
            out.append([(int(hi[r, i]), float(hv[r, i])) for i in range(kk) if hi[r, i] != _lib.VA_SENTINEL_INDEX])
        return out

    def selectSingle(self, values, k: int, mode: Metal4SelectionMode = Metal4SelectionMode.minimum):
        return self.select([list(values)], k, mode)[0]


class TopKMergeKernel:
    """Merge two sorted top-k lists (TopKMergeKernel / merge_topk_sorted_kernel,
    Metal/Shaders/SearchAndRetrieval.metal:320-385)."""

    name = "TopKMergeKernel"

    def __init__(self, context: GPUContext):
        self.context = context

    def encode(self, aIdx, aDist, bIdx, bDist, outIdx, outDist, numQueries: int, k: int, chunkBase: int):
        c = self.context
        c.check(
            c.lib.va_topk_merge(c.handle, dptr(aIdx), dptr(aDist), dptr(bIdx), dptr(bDist), numQueries, k,
                                chunkBase, dptr(outIdx), dptr(outDist)),
            "TopKMergeKernel.encode",
        )

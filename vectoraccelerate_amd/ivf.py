"""IVF-Flat search pipeline — host mirror of IVFSearchPipeline / IVFSearchConfiguration.

Reference: Index/Kernels/IVF/IVFKernels.swift:28-107 (configuration), IVFSearchPipeline.swift:
45-612 (pipeline, IVFGPUIndexStructure), IVFKernels.swift:245-290 (IVFSearchResult).
The index structure is a ``va_ivf`` handle (device CSR lists) built by ``va_ivf_build``.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from .context import GPUContext, VectorError, dptr
from .kernels import _as_matrix


def _torch():
    import torch

    return torch


@dataclass
class IVFSearchConfiguration:
    numCentroids: int
    nprobe: int = 8
    dimension: int = 0
    metric: str = "euclidean"

    def __post_init__(self):
        self.nprobe = min(self.nprobe, self.numCentroids)  # IVFKernels.swift:62

    def validate(self):
        if self.numCentroids < 1:
            raise VectorError.invalidInput(f"numCentroids must be at least 1, got {self.numCentroids}")
        if self.nprobe < 1:
            raise VectorError.invalidInput(f"nprobe must be at least 1, got {self.nprobe}")
        if self.nprobe > self.numCentroids:
            raise VectorError.invalidInput(f"nprobe ({self.nprobe}) cannot exceed numCentroids ({self.numCentroids})")
        if not 1 <= self.dimension <= 4096:
            raise VectorError.invalidInput(f"dimension must be 1-4096, got {self.dimension}")

    @classmethod
    def small(cls, dimension: int):
        return cls(256, 8, dimension)

    @classmethod
    def standard(cls, dimension: int):
        return cls(1024, 16, dimension)

    @classmethod
    def large(cls, dimension: int):
        return cls(4096, 32, dimension)


class IVFGPUIndexStructure:
    """Owns a va_ivf handle: centroids + CSR-ordered list vectors on the device."""

    def __init__(self, context: GPUContext, handle: C.c_void_p, numCentroids: int, totalVectors: int, dimension: int):
        self.context = context
        self._h = handle
        self.numCentroids = numCentroids
        self.totalVectors = totalVectors
        self.dimension = dimension

    @property
    def handle(self):
        return self._h

    def lists(self) -> tuple[np.ndarray, np.ndarray]:
        """(offsets[C+1], row ids[N]) of the CSR structure."""
        c = self.context
        off = np.empty(self.numCentroids + 1, np.uint32)
        ids = np.empty(self.totalVectors, np.uint32)
        c.check(c.lib.va_ivf_get_lists(c.handle, self._h, off.ctypes.data_as(C.c_void_p),
                                       ids.ctypes.data_as(C.c_void_p)), "va_ivf_get_lists")
        return off, ids

    def add(self, vectors, firstId: int):
        """Append rows (device tensor [n x D]) to their nearest lists, ids firstId + i (va_ivf_add)."""
        c = self.context
        if vectors.shape[0] == 0:
            return
        if vectors.shape[1] != self.dimension:
            raise VectorError.dimensionMismatch(self.dimension, vectors.shape[1])
        x = vectors.contiguous()
        c.order_after_torch()
        c.check(c.lib.va_ivf_add(c.handle, self._h, dptr(x), x.shape[0], x.shape[1], int(firstId)), "va_ivf_add")
        self.totalVectors += x.shape[0]

    def listCount(self, listIndex: int) -> int:
        off, _ = self.lists()
        return int(off[listIndex + 1] - off[listIndex])

    def close(self):
        if getattr(self, "_h", None) is not None:
            self.context.lib.va_ivf_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class IVFSearchResult:
    def __init__(self, indices, distances, numQueries: int, k: int):
        self.indices = indices
        self.distances = distances
        self.numQueries = numQueries
        self.k = k

    def results(self, queryIndex: int) -> list[tuple[int, float]]:
        idx = self.indices.cpu().numpy().view(np.uint32)[queryIndex]
        dist = self.distances.cpu().numpy()[queryIndex]
        return [(int(i), float(d)) for i, d in zip(idx, dist) if i != _lib.VA_SENTINEL_INDEX]

    def allResults(self):
        return [self.results(q) for q in range(self.numQueries)]


class IVFSearchPipeline:
    """Coarse probe -> list-major scan -> exact top-k, L2^2 (IVFSearchPipeline.swift:45-568)."""

    def __init__(self, context: GPUContext, configuration: IVFSearchConfiguration):
        configuration.validate()
        self.context = context
        self.configuration = configuration

    def prepareIndexStructure(self, centroids, vectors) -> IVFGPUIndexStructure:
        """Assign every vector to its nearest centroid and lay the lists out on the device."""
        c = self.context
        cen = centroids if hasattr(centroids, "is_cuda") else c.buffer(_as_matrix(centroids, "centroids"))
        x = vectors if hasattr(vectors, "is_cuda") else c.buffer(_as_matrix(vectors, "vectors"))
        if cen.shape[1] != x.shape[1]:
            raise VectorError.dimensionMismatch(cen.shape[1], x.shape[1])
        if cen.shape[0] != self.configuration.numCentroids:
            raise VectorError.invalidInput(
                f"Number of centroids ({cen.shape[0]}) must match numCentroids ({self.configuration.numCentroids})")
        h = C.c_void_p()
        c.order_after_torch()
        c.check(c.lib.va_ivf_build(c.handle, dptr(cen), cen.shape[0], dptr(x), x.shape[0], x.shape[1], C.byref(h)),
                "va_ivf_build")
        return IVFGPUIndexStructure(c, h, cen.shape[0], x.shape[0], x.shape[1])

    def _queries(self, queries, structure):
        c = self.context
        q = queries if hasattr(queries, "is_cuda") else c.buffer(_as_matrix(queries, "queries"))
        if q.shape[1] != structure.dimension:
            raise VectorError.dimensionMismatch(structure.dimension, q.shape[1])
        return q

    def findNearestCentroids(self, queries, structure: IVFGPUIndexStructure, nprobe: int | None = None):
        torch = _torch()
        c = self.context
        q = self._queries(queries, structure)
        nprobe = nprobe or self.configuration.nprobe
        probes = c.empty((q.shape[0], nprobe), torch.int32)
        c.order_after_torch()
        c.check(c.lib.va_ivf_probe(c.handle, structure.handle, dptr(q), q.shape[0], nprobe, dptr(probes)),
                "va_ivf_probe")
        c.synchronize()
        return probes

    def searchLists(self, queries, structure: IVFGPUIndexStructure, probes, k: int) -> IVFSearchResult:
        torch = _torch()
        c = self.context
        q = self._queries(queries, structure)
        p = probes if hasattr(probes, "is_cuda") else c.buffer(np.asarray(probes, np.uint32).view(np.int32))
        idx = c.empty((q.shape[0], k), torch.int32)
        dist = c.empty((q.shape[0], k), torch.float32)
        c.order_after_torch()
        c.check(c.lib.va_ivf_scan(c.handle, structure.handle, dptr(q), q.shape[0], dptr(p), p.shape[1], k, dptr(idx),
                                  dptr(dist)), "va_ivf_scan")
        c.synchronize()
        return IVFSearchResult(idx, dist, q.shape[0], k)

    def encodeSearch(self, queries, structure: IVFGPUIndexStructure, outIdx, outDist, k: int):
        c = self.context
        c.check(c.lib.va_ivf_search(c.handle, structure.handle, dptr(queries), queries.shape[0],
                                    self.configuration.nprobe, k, dptr(outIdx), dptr(outDist)), "va_ivf_search")

    def search(self, queries, structure: IVFGPUIndexStructure, k: int) -> IVFSearchResult:
        torch = _torch()
        if k <= 0:
            raise VectorError.invalidInput("k must be positive")
        c = self.context
        q = self._queries(queries, structure)
        idx = c.empty((q.shape[0], k), torch.int32)
        dist = c.empty((q.shape[0], k), torch.float32)
        c.order_after_torch()
        self.encodeSearch(q, structure, idx, dist, k)
        c.synchronize()
        return IVFSearchResult(idx, dist, q.shape[0], k)

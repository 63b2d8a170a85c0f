"""K-means clustering pipeline — host mirror of KMeansPipeline / KMeansConfiguration.

Reference: Index/Kernels/Clustering/ClusteringKernels.swift:60-120 (KMeansConfiguration),
ClusteringKernels.swift:165-240 (KMeansResult), KMeansPipeline.swift:102-270 (fit) and
KMeansPlusPlusKernel.swift:94-203 (k-means++ seeding).  The iterations run in
``va_kmeans_fit`` and the seeding in ``va_kmeans_plusplus`` (libva_hip.so); this module only
checks arguments, moves data and wraps results.
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
class KMeansConfiguration:
    """ClusteringKernels.swift:60-120.  Only the euclidean metric and full-batch Lloyd
    iterations are implemented (the reference's pipeline uses no other)."""

    numClusters: int
    dimension: int
    maxIterations: int = 100
    convergenceThreshold: float = 1e-4
    metric: str = "euclidean"
    enableProfiling: bool = False
    batchSize: int = 0
    initialization: str = "kMeansPlusPlus"
    seed: int = 0x5EED

    def validate(self):
        if self.numClusters < 1:
            raise VectorError.invalidInput(f"numClusters must be positive, got {self.numClusters}")
        if self.dimension < 1:
            raise VectorError.invalidInput(f"dimension must be positive, got {self.dimension}")
        if self.metric != "euclidean":
            raise VectorError("unsupported", f"k-means metric {self.metric!r} (only euclidean)")
        if self.batchSize != 0:
            raise VectorError("unsupported", "mini-batch k-means (batchSize != 0)")


class KMeansResult:
    """ClusteringKernels.swift:165-240: device tensors plus the fit's summary."""

    def __init__(self, centroids, assignments, distances, clusterCounts, numClusters, numVectors, dimension,
                 iterations, converged, inertia, maxMovement):
        self.centroids = centroids
        self.assignments = assignments
        self.distances = distances
        self.clusterCounts = clusterCounts
        self.numClusters = numClusters
        self.numVectors = numVectors
        self.dimension = dimension
        self.iterations = iterations
        self.converged = converged
        self.inertia = inertia
        self.maxMovement = maxMovement

    def extractCentroids(self) -> list[list[float]]:
        return self.centroids.cpu().numpy().tolist()

    def extractAssignments(self) -> list[int]:
        return self.assignments.cpu().numpy().view(np.uint32).astype(np.int64).tolist()

    def extractClusterCounts(self) -> list[int]:
        return self.clusterCounts.cpu().numpy().view(np.uint32).astype(np.int64).tolist()


class KMeansPlusPlusKernel:
    """KMeansPlusPlusKernel.swift:94-203: D^2 seeding on the device."""

    def __init__(self, context: GPUContext):
        self.context = context

    def selectCentroidsBuffer(self, vectors, k: int, seed: int = 0x5EED):
        """(centroids [k x D] device tensor, row ids [k] numpy)."""
        torch = _torch()
        c = self.context
        x = vectors if hasattr(vectors, "is_cuda") else c.buffer(_as_matrix(vectors, "vectors"))
        if x.shape[0] < k:
            raise VectorError.invalidInput(f"Not enough vectors ({x.shape[0]}) for {k} clusters")
        if k <= 0:
            raise VectorError.invalidInput("k must be positive")
        cen = c.empty((k, x.shape[1]), torch.float32)
        idx = c.empty((k,), torch.int32)
        c.order_after_torch()
        c.check(c.lib.va_kmeans_plusplus(c.handle, dptr(x), x.shape[0], x.shape[1], k, C.c_uint64(seed), dptr(cen),
                                         dptr(idx)), "va_kmeans_plusplus")
        return cen, idx.cpu().numpy().view(np.uint32).copy()

    def selectCentroids(self, vectors, k: int, seed: int = 0x5EED) -> list[int]:
        return self.selectCentroidsBuffer(vectors, k, seed)[1].astype(np.int64).tolist()


class KMeansPipeline:
    """Lloyd k-means on the device (KMeansPipeline.swift:102-270)."""

    def __init__(self, context: GPUContext, configuration: KMeansConfiguration):
        configuration.validate()
        self.context = context
        self.configuration = configuration

    def fit(self, vectors, initialCentroids=None) -> KMeansResult:
        torch = _torch()
        c = self.context
        cfg = self.configuration
        if not hasattr(vectors, "is_cuda") and len(vectors) == 0:
            raise VectorError.invalidInput("Vectors cannot be empty")
        x = vectors if hasattr(vectors, "is_cuda") else c.buffer(_as_matrix(vectors, "vectors"))
        if x.shape[0] == 0:
            raise VectorError.invalidInput("Vectors cannot be empty")
        if x.shape[1] != cfg.dimension:
            raise VectorError.dimensionMismatch(cfg.dimension, x.shape[1])
        if initialCentroids is not None:
            init = initialCentroids if hasattr(initialCentroids, "is_cuda") else c.buffer(
                _as_matrix(initialCentroids, "initialCentroids"))
            if init.shape[0] != cfg.numClusters:
                raise VectorError.invalidInput(
                    f"Initial centroids count ({init.shape[0]}) must match numClusters ({cfg.numClusters})")
            if init.shape[1] != cfg.dimension:
                raise VectorError.dimensionMismatch(cfg.dimension, init.shape[1])
        else:
            init, _ = KMeansPlusPlusKernel(c).selectCentroidsBuffer(x, cfg.numClusters, cfg.seed)
        N, D = x.shape
        K = cfg.numClusters
        cen = c.empty((K, D), torch.float32)
        assign = c.empty((N,), torch.int32)
        dist = c.empty((N,), torch.float32)
        counts = c.empty((K,), torch.int32)
        info = _lib.KMeansInfo()
        c.order_after_torch()
        c.check(c.lib.va_kmeans_fit(c.handle, dptr(x), N, D, K, dptr(init), cfg.maxIterations,
                                    C.c_float(cfg.convergenceThreshold), dptr(cen), dptr(assign), dptr(dist),
                                    dptr(counts), C.byref(info)), "va_kmeans_fit")
        return KMeansResult(cen, assign, dist, counts, K, N, D, int(info.iterations), bool(info.converged),
                            float(info.inertia), float(info.max_movement))

"""AcceleratedVectorIndex — the reference's index actor over the native index of libva_hip.so.

Reference: Index/AcceleratedVectorIndex.swift (init :166-237, insert :481-700, remove
:771-833, compact :834-893, search :895-1000, searchUnfiltered :1103-1186, searchFiltered
:1188-1265, searchBatchGPU :1278-1374, searchIVF :1378-1431); handles
(Index/Types/VectorHandle.swift:33-70, Index/Internal/HandleAllocator.swift:39-242).

Storage, stable handles, deletions, compaction, IVF training and lists, routing and every search
(flat or IVF, plain or filtered) are the native index (``va_index_*``): its rows live on the device
with an fp16 shadow for the screening scan, deleted rows are excluded inside every scan (the IVF
list scan included), and a filter is applied to round after round of not-yet-examined nearest
rows, so no result is short however many rows are deleted or rejected.  This module keeps what
the reference keeps in Swift beside the index: metadata and the Python-facing result types.
"""
from __future__ import annotations

import ctypes as C
import math
import time
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .context import DeviceRows, GPUContext, VectorError, dptr

_METRICS = {"euclidean": _lib.VA_METRIC_L2SQ, "cosine": _lib.VA_METRIC_COSINE, "dotProduct": _lib.VA_METRIC_DOT}


def _torch():
    import torch

    return torch


@dataclass(frozen=True, order=True)
class VectorHandle:
    """Opaque stable identifier of an inserted vector (VectorHandle.swift:33-70)."""

    stableID: int

    @property
    def isValid(self) -> bool:
        return self.stableID != 0xFFFFFFFF


VectorHandle.invalid = VectorHandle(0xFFFFFFFF)


@dataclass
class IndexSearchResult:
    id: VectorHandle
    distance: float  # L2^2 (the metric's distance for cosine / dotProduct indexes)

    @property
    def euclideanDistance(self) -> float:
        return math.sqrt(self.distance)


@dataclass
class SearchResults:
    results: list = field(default_factory=list)
    candidatesSearched: int = 0
    searchTimeNanos: int = 0
    isExhaustive: bool = True

    @property
    def count(self) -> int:
        return len(self.results)


@dataclass
class IndexConfiguration:
    """IndexConfiguration (Index/Types/IndexConfiguration.swift): flat or IVF.

    The reference's GPU search is L2^2 only (AcceleratedVectorIndex.validateMetricSupport); the
    flat index here also accepts "cosine" (1 - similarity) and "dotProduct" (-dot) distances."""

    dimension: int
    capacity: int = 10_000
    metric: str = "euclidean"
    indexType: tuple = ("flat",)
    routingThreshold: int = 0

    @classmethod
    def flat(cls, dimension: int, capacity: int = 10_000, metric: str = "euclidean"):
        return cls(dimension, capacity, metric)

    @classmethod
    def ivf(cls, dimension: int, nlist: int, nprobe: int, capacity: int = 100_000, routingThreshold: int = 0):
        return cls(dimension, capacity, "euclidean", ("ivf", nlist, nprobe), routingThreshold)

    def validate(self):
        if self.dimension <= 0:
            raise VectorError.invalidInput(f"dimension must be positive, got {self.dimension}")
        if self.capacity <= 0:
            raise VectorError.invalidInput(f"capacity must be positive, got {self.capacity}")
        if self.metric not in _METRICS:
            raise VectorError("unsupported", f"metric {self.metric} is not supported by the index")
        if self.indexType[0] == "ivf":
            if self.metric != "euclidean":
                raise VectorError("unsupported", "IVF indexes search by L2^2 only")
            nlist, nprobe = self.indexType[1], self.indexType[2]
            if nlist < 1 or nprobe < 1 or nprobe > nlist:
                raise VectorError.invalidInput(f"invalid IVF parameters nlist={nlist} nprobe={nprobe}")


class AcceleratedVectorIndex:
    def __init__(self, configuration: IndexConfiguration, context: GPUContext | None = None):
        configuration.validate()
        self.configuration = configuration
        self.context = context or GPUContext(0)
        c = self.context
        h = C.c_void_p()
        if configuration.indexType[0] == "ivf":
            _, nlist, nprobe = configuration.indexType
            c.check(c.lib.va_index_create_ivf(c.handle, configuration.dimension, configuration.capacity, nlist, nprobe,
                                              configuration.routingThreshold, C.byref(h)), "va_index_create_ivf")
        else:
            c.check(c.lib.va_index_create(c.handle, configuration.dimension, configuration.capacity, C.byref(h)),
                    "va_index_create")
        self._h = h
        self._metric = _METRICS[configuration.metric]
        self._metadata: dict[int, object] = {}

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            self.context.lib.va_index_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- properties ------------------------------------------------------------------------
    def _info(self) -> _lib.IndexInfo:
        info = _lib.IndexInfo()
        self.context.check(self.context.lib.va_index_get_info(self._h, C.byref(info)), "va_index_get_info")
        return info

    def _rows(self) -> DeviceRows:
        info = self._info()
        return DeviceRows(info.rows or 0, info.slots, info.dimension)

    @property
    def count(self) -> int:
        return int(self._info().count)

    @property
    def dimension(self) -> int:
        return self.configuration.dimension

    @property
    def isEmpty(self) -> bool:
        return self.count == 0

    @property
    def capacity(self) -> int:
        return int(self._info().capacity)

    @property
    def isIVF(self) -> bool:
        return self.configuration.indexType[0] == "ivf"

    @property
    def isTrained(self) -> bool:
        return bool(self._info().trained)

    # -- mutation ----------------------------------------------------------------------------
    def insert(self, vector=None, metadata=None, vectors=None):
        """insert(vector) -> VectorHandle, or insert(vectors=[...]) -> [VectorHandle].

        A trained IVF index appends the new vectors to their nearest lists."""
        batch = vectors is not None
        c = self.context
        if batch and getattr(vectors, "is_cuda", False):
            # rows already on the device (fp32 [n x D] tensor): no host round trip
            torch = _torch()
            if vectors.dim() != 2 or vectors.shape[1] != self.dimension:
                raise VectorError.dimensionMismatch(self.dimension, vectors.shape[-1])
            dev = vectors.to(torch.float32).contiguous()
            n = dev.shape[0]
        else:
            arr = np.asarray(vectors if batch else [vector], np.float32)
            if arr.ndim != 2 or arr.shape[1] != self.dimension:
                got = arr.shape[-1] if arr.ndim >= 1 else 0
                raise VectorError.dimensionMismatch(self.dimension, got)
            n = arr.shape[0]
            dev = c.buffer(np.ascontiguousarray(arr)) if n else None
        if n == 0:
            return []
        out = np.zeros(n, np.uint32)
        c.order_after_torch()
        c.check(c.lib.va_index_insert(c.handle, self._h, dptr(dev), n, out.ctypes.data), "va_index_insert")
        handles = [VectorHandle(int(h)) for h in out]
        if metadata is not None and not batch:
            self._metadata[handles[0].stableID] = metadata
        c.synchronize()  # the staged input buffer is released on return
        return handles if batch else handles[0]

    def remove(self, handle):
        """remove(handle) or remove([handles]) -> number removed (AcceleratedVectorIndex.swift:771-833).

        The slot stays in place (and in its IVF list) and is excluded from every search until
        compact()."""
        hs = handle if isinstance(handle, (list, tuple)) else [handle]
        if not isinstance(handle, (list, tuple)) and not self.contains(handle):
            raise VectorError.invalidInput(f"invalid handle {handle.stableID}")
        ids = np.asarray([h.stableID for h in hs], np.uint32)
        removed = C.c_uint32(0)
        c = self.context
        c.check(c.lib.va_index_remove(c.handle, self._h, ids.ctypes.data, len(ids), C.byref(removed)), "va_index_remove")
        for h in hs:
            self._metadata.pop(h.stableID, None)
        return int(removed.value)

    def compact(self):
        """Drop deleted slots; handles keep their stable ids (AcceleratedVectorIndex.swift:834-893).
        A trained IVF index rebuilds its lists from the trained centroids."""
        c = self.context
        c.check(c.lib.va_index_compact(c.handle, self._h), "va_index_compact")

    def vector(self, handle: VectorHandle):
        if not self.contains(handle):
            return None
        out = np.zeros(self.dimension, np.float32)
        c = self.context
        c.check(c.lib.va_index_get_vector(c.handle, self._h, handle.stableID, out.ctypes.data), "va_index_get_vector")
        return out.tolist()

    def metadata(self, handle: VectorHandle):
        return self._metadata.get(handle.stableID)

    def contains(self, handle: VectorHandle) -> bool:
        return bool(self.context.lib.va_index_contains(self._h, handle.stableID))

    # -- IVF ---------------------------------------------------------------------------------
    def train(self, centroids=None, seed: int = 0x5EED):
        """Train the IVF centroids; the lists are then built from the stored vectors (va_index_train).

        Without ``centroids``: k-means on the device over the live vectors (compacted first) with
        k-means++ seeding, 25 iterations at most, threshold 0.001, as IVFStructure.train
        (Index/Internal/IVFStructure.swift:202-259) called by AcceleratedVectorIndex.train
        (AcceleratedVectorIndex.swift:406-446).  With ``centroids`` ([nlist x D]): installs them.
        A flat index has nothing to train (the reference returns at once, :405-407)."""
        c = self.context
        cen = None
        if centroids is not None and self.isIVF:
            nlist = self.configuration.indexType[1]
            if getattr(centroids, "is_cuda", False):
                cen = centroids.to(_torch().float32).contiguous()
            else:
                cen = c.buffer(np.ascontiguousarray(np.asarray(centroids, np.float32)))
            if tuple(cen.shape) != (nlist, self.dimension):
                raise VectorError.invalidInput(f"centroids must be {nlist} x {self.dimension}")
            c.order_after_torch()
        c.check(c.lib.va_index_train(c.handle, self._h, dptr(cen) if cen is not None else None, int(seed)),
                "va_index_train")

    def centroids(self) -> np.ndarray | None:
        """The trained centroids [nlist x D] (host copy), or None."""
        info = self._info()
        if not info.trained:
            return None
        out = np.empty((info.nlist, info.dimension), np.float32)
        c = self.context
        c.check(c.lib.va_buffer_download(c.handle, out.ctypes.data, info.centroids, out.nbytes), "va_buffer_download")
        c.synchronize()
        return out

    def lists(self) -> tuple[np.ndarray, np.ndarray] | None:
        """(offsets[nlist + 1], slots[slots]) of the inverted lists (CSR order), or None."""
        info = self._info()
        if not info.lists:
            return None
        off = np.empty(info.nlist + 1, np.uint32)
        ids = np.empty(info.slots, np.uint32)
        c = self.context
        c.check(c.lib.va_ivf_get_lists(c.handle, info.lists, off.ctypes.data, ids.ctypes.data), "va_ivf_get_lists")
        return off, ids

    def probes(self, queries) -> np.ndarray:
        """The nprobe lists each query probes [Q x nprobe] (va_ivf_probe over the index's lists)."""
        torch = _torch()
        info = self._info()
        if not info.lists:
            raise VectorError.invalidInput("the index has no inverted lists (untrained or empty)")
        c = self.context
        q = c.buffer(np.asarray(queries, np.float32).reshape(-1, self.dimension))
        out = c.empty((q.shape[0], info.nprobe), torch.int32)
        c.order_after_torch()
        c.check(c.lib.va_ivf_probe(c.handle, info.lists, dptr(q), q.shape[0], info.nprobe, dptr(out)), "va_ivf_probe")
        c.synchronize()
        return out.cpu().numpy().view(np.uint32)

    def _use_ivf(self) -> bool:
        return bool(self._info().ivf_routed)

    # -- search --------------------------------------------------------------------------------
    def _topk(self, q_dev, k: int):
        """The k nearest live vectors per query row (va_index_search: flat or IVF)."""
        torch = _torch()
        c = self.context
        Q = q_dev.shape[0]
        idx = c.empty((Q, k), torch.int32)
        dist = c.empty((Q, k), torch.float32)
        c.order_after_torch()
        c.check(c.lib.va_index_search(c.handle, self._h, self._metric, dptr(q_dev), Q, k, dptr(idx), dptr(dist)),
                "va_index_search")
        c.synchronize()
        ids = idx.cpu().numpy().view(np.uint32)
        ds = dist.cpu().numpy()
        out = []
        for row, drow in zip(ids, ds):
            keep = row != _lib.VA_SENTINEL_INDEX
            out.append(([int(h) for h in row[keep]], [float(x) for x in drow[keep]]))
        return out

    def _results(self, hs, ds):
        return [IndexSearchResult(VectorHandle(h), d) for h, d in zip(hs, ds)]

    def _filtered(self, q: np.ndarray, k: int, filt):
        c = self.context
        q_dev = c.buffer(q.reshape(1, -1))
        meta = self._metadata

        def accept(h, _user):
            try:
                return 1 if filt(VectorHandle(int(h)), meta.get(int(h))) else 0
            except Exception:  # a raising filter rejects the vector
                return 0

        cb = _lib.INDEX_FILTER(accept)
        hs = np.zeros(k, np.uint32)
        ds = np.zeros(k, np.float32)
        n, examined = C.c_uint32(0), C.c_uint32(0)
        c.order_after_torch()
        c.check(c.lib.va_index_search_filtered(c.handle, self._h, self._metric, dptr(q_dev), k, cb, None,
                                               hs.ctypes.data, ds.ctypes.data, C.byref(n), C.byref(examined)),
                "va_index_search_filtered")
        return self._results([int(h) for h in hs[:n.value]], [float(x) for x in ds[:n.value]]), int(examined.value)

    def _effective_k(self, k: int, live: int) -> int:
        if k <= 0:
            raise VectorError.invalidInput(f"k must be positive, got {k}")
        eff = min(k, live)
        if eff > _lib.VA_MAX_K:
            # FusedL2TopKParameters rejects k > maxK (Kernels/Metal4/FusedL2TopKKernel.swift:57-79)
            raise VectorError.invalidInput(f"k {eff} exceeds maximum supported k {_lib.VA_MAX_K}")
        return eff

    def search(self, query=None, k: int = 10, filter=None, queries=None):
        """search(query, k[, filter]) -> SearchResults; search(queries=[...], k) -> [SearchResults]."""
        if queries is not None:
            return self._search_batch(queries, k, filter)
        q = np.asarray(query, np.float32).reshape(-1)
        if q.shape[0] != self.dimension:
            raise VectorError.dimensionMismatch(self.dimension, q.shape[0])
        live = self.count
        if k <= 0:
            raise VectorError.invalidInput(f"k must be positive, got {k}")
        if live == 0:
            return SearchResults()
        ivf = self._use_ivf()
        t0 = time.perf_counter_ns()
        if filter is not None:
            res, examined = self._filtered(q, min(k, live), filter)
            return SearchResults(res, examined, time.perf_counter_ns() - t0, not ivf)
        effective_k = self._effective_k(k, live)
        hs, ds = self._topk(self.context.buffer(q.reshape(1, -1)), effective_k)[0]
        return SearchResults(self._results(hs, ds), live, time.perf_counter_ns() - t0, not ivf)

    def _search_batch(self, queries, k, filter):
        qs = np.asarray(queries, np.float32)
        if qs.size == 0:
            return []
        if qs.ndim != 2 or qs.shape[1] != self.dimension:
            raise VectorError.dimensionMismatch(self.dimension, qs.shape[-1])
        if k <= 0:
            raise VectorError.invalidInput(f"k must be positive, got {k}")
        live = self.count
        if live == 0:
            return [SearchResults() for _ in range(qs.shape[0])]
        if filter is not None:
            return [self.search(q, k, filter) for q in qs]
        effective_k = self._effective_k(k, live)
        ivf = self._use_ivf()
        t0 = time.perf_counter_ns()
        rows = self._topk(self.context.buffer(qs), effective_k)
        dt = time.perf_counter_ns() - t0
        return [SearchResults(self._results(hs, ds), live, dt, not ivf) for hs, ds in rows]

    def searchDevice(self, queries_dev, k: int, out_handles, out_dist):
        """encode tier of the search: device queries [Q x D] -> device handles / distances
        [Q x k] (uint32 / fp32 tensors), enqueued on the context's stream (va_index_search)."""
        c = self.context
        Q = queries_dev.shape[0]
        c.order_after_torch()
        c.check(c.lib.va_index_search(c.handle, self._h, self._metric, dptr(queries_dev), Q, k, dptr(out_handles),
                                      dptr(out_dist)), "va_index_search")

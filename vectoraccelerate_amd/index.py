"""AcceleratedVectorIndex — the reference's index actor over the native index of libva_hip.so.

Reference: Index/AcceleratedVectorIndex.swift (init :166-237, insert :481-700, remove
:771-833, compact :834-893, search :895-1000, searchUnfiltered :1103-1186, searchFiltered
:1188-1265, searchBatchGPU :1278-1374, searchIVF :1378-1431); handles
(Index/Types/VectorHandle.swift:33-70, Index/Internal/HandleAllocator.swift:39-242).

Storage, stable handles, deletions, compaction and the flat searches (plain and filtered) are the
native index (``va_index_*``): its rows live on the device with an fp16 shadow for the screening
scan, deleted rows are excluded inside the scan, and a filter is applied to round after round of
not-yet-examined nearest rows, so no result is short however many rows are deleted or rejected.
This module keeps what the reference keeps in Swift: metadata, the IVF configuration, routing
and the IVF lists (built over the index's slots with va_ivf_*).
"""
from __future__ import annotations

import ctypes as C
import math
import time
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .context import DeviceRows, GPUContext, VectorError, dptr
from .ivf import IVFGPUIndexStructure, IVFSearchConfiguration, IVFSearchPipeline

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
        c.check(c.lib.va_index_create(c.handle, configuration.dimension, configuration.capacity, C.byref(h)),
                "va_index_create")
        self._h = h
        self._metric = _METRICS[configuration.metric]
        self._metadata: dict[int, object] = {}
        # slot -> stable id and the deletion flags, mirrored for the IVF path (whose lists hold slots)
        self._slot_handle: list[int] = []
        self._deleted_slots: set[int] = set()
        self._ivf: IVFGPUIndexStructure | None = None
        self._ivf_dirty = True
        self._centroids = None
        if configuration.indexType[0] == "ivf":
            _, nlist, nprobe = configuration.indexType
            self._ivf_pipe = IVFSearchPipeline(self.context, IVFSearchConfiguration(nlist, nprobe,
                                                                                    configuration.dimension))

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            if self._ivf is not None:
                self._ivf.close()
                self._ivf = None
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
        return self._centroids is not None

    # -- mutation ----------------------------------------------------------------------------
    def insert(self, vector=None, metadata=None, vectors=None):
        """insert(vector) -> VectorHandle, or insert(vectors=[...]) -> [VectorHandle]."""
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
        first = self._info().slots
        out = np.zeros(n, np.uint32)
        c.order_after_torch()
        c.check(c.lib.va_index_insert(c.handle, self._h, dptr(dev), n, out.ctypes.data), "va_index_insert")
        handles = [VectorHandle(int(h)) for h in out]
        self._slot_handle.extend(int(h) for h in out)
        if metadata is not None and not batch:
            self._metadata[handles[0].stableID] = metadata
        if self._ivf is not None and not self._ivf_dirty:
            # built lists: append the new slots to their nearest lists (va_ivf_add) instead of a rebuild
            self._ivf.add(self._rows().rows(first, first + n), first)
        else:
            self._ivf_dirty = True
        c.synchronize()  # the staged input buffer is released on return
        return handles if batch else handles[0]

    def remove(self, handle):
        """remove(handle) or remove([handles]) -> number removed (AcceleratedVectorIndex.swift:771-833).

        The IVF lists are left as they are: removed slots are skipped when results are collected."""
        hs = handle if isinstance(handle, (list, tuple)) else [handle]
        if not isinstance(handle, (list, tuple)) and not self.contains(handle):
            raise VectorError.invalidInput(f"invalid handle {handle.stableID}")
        ids = np.asarray([h.stableID for h in hs], np.uint32)
        live = [h.stableID for h in hs if self.contains(h)]
        slot_of = {hid: s for s, hid in enumerate(self._slot_handle)} if live else {}
        removed = C.c_uint32(0)
        c = self.context
        c.check(c.lib.va_index_remove(c.handle, self._h, ids.ctypes.data, len(ids), C.byref(removed)), "va_index_remove")
        for hid in live:
            self._deleted_slots.add(slot_of[hid])
            self._metadata.pop(hid, None)
        return int(removed.value)

    def compact(self):
        """Drop deleted slots; handles keep their stable ids (AcceleratedVectorIndex.swift:834-893)."""
        if not self._deleted_slots:
            return
        c = self.context
        c.check(c.lib.va_index_compact(c.handle, self._h), "va_index_compact")
        self._slot_handle = [h for s, h in enumerate(self._slot_handle) if s not in self._deleted_slots]
        self._deleted_slots.clear()
        self._ivf_dirty = True

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
        """Train the IVF centroids; the lists are then built from the stored vectors.

        Without ``centroids``: k-means on the device over the live vectors (compacted first) with
        k-means++ seeding, 25 iterations at most, threshold 0.001, as IVFStructure.train
        (Index/Internal/IVFStructure.swift:202-259) called by AcceleratedVectorIndex.train
        (AcceleratedVectorIndex.swift:406-446).  With ``centroids`` ([nlist x D]): installs them.
        """
        if not self.isIVF:
            raise VectorError.invalidInput("train() needs an IVF index")
        nlist = self.configuration.indexType[1]
        if centroids is None:
            from .clustering import KMeansConfiguration, KMeansPipeline

            live = self.count
            if live == 0:
                raise VectorError.invalidInput("Cannot train IVF index with no vectors")
            if live < nlist:
                raise VectorError.invalidInput(f"Need at least {nlist} vectors for {nlist} clusters, got {live}")
            self.compact()  # the live rows are then slots [0, count)
            cfg = KMeansConfiguration(nlist, self.dimension, maxIterations=25, convergenceThreshold=0.001, seed=seed)
            self._centroids = KMeansPipeline(self.context, cfg).fit(self._rows()).centroids
        else:
            cen = np.asarray(centroids, np.float32)
            if cen.shape != (nlist, self.dimension):
                raise VectorError.invalidInput(f"centroids must be {nlist} x {self.dimension}")
            self._centroids = self.context.buffer(cen)
        self._ivf_dirty = True

    def _ivf_structure(self) -> IVFGPUIndexStructure:
        if self._ivf is None or self._ivf_dirty:
            if self._ivf is not None:
                self._ivf.close()
            self._ivf = self._ivf_pipe.prepareIndexStructure(self._centroids, self._rows())
            self._ivf_dirty = False
        return self._ivf

    def _use_ivf(self) -> bool:
        if not (self.isIVF and self.isTrained):
            return False
        t = self.configuration.routingThreshold
        return not (t > 0 and self.count < t)

    def _ivf_topk(self, q_dev, k: int):
        """IVF: the k nearest live slots per query row, as (handle lists, distance lists)."""
        if len(self._deleted_slots) and k + len(self._deleted_slots) > _lib.VA_MAX_K:
            # over-fetching past the removed slots would exceed VA_MAX_K: drop them first
            self.compact()
        fetch = min(k + len(self._deleted_slots), _lib.VA_MAX_K)
        res = self._ivf_pipe.search(q_dev, self._ivf_structure(), fetch)
        ids = res.indices.cpu().numpy().view(np.uint32)
        d = res.distances.cpu().numpy()
        out = []
        for row, drow in zip(ids, d):
            hs, ds = [], []
            for s, dist in zip(row, drow):
                s = int(s)
                if s == _lib.VA_SENTINEL_INDEX or s in self._deleted_slots:
                    continue
                hs.append(self._slot_handle[s])
                ds.append(float(dist))
                if len(hs) == k:
                    break
            out.append((hs, ds))
        return out

    # -- search --------------------------------------------------------------------------------
    def _flat_topk(self, q_dev, k: int):
        """Flat: the k nearest live vectors per query row (va_index_search)."""
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

    def search(self, query=None, k: int = 10, filter=None, queries=None):
        """search(query, k[, filter]) -> SearchResults; search(queries=[...], k) -> [SearchResults]."""
        if queries is not None:
            return self._search_batch(queries, k, filter)
        q = np.asarray(query, np.float32).reshape(-1)
        if q.shape[0] != self.dimension:
            raise VectorError.dimensionMismatch(self.dimension, q.shape[0])
        if k <= 0:
            raise VectorError.invalidInput(f"k must be positive, got {k}")
        live = self.count
        if live == 0:
            return SearchResults()
        t0 = time.perf_counter_ns()
        if filter is not None and not self._use_ivf():
            res, examined = self._filtered(q, k, filter)
            return SearchResults(res, examined, time.perf_counter_ns() - t0, True)
        effective_k = min(k, live, _lib.VA_MAX_K)
        q_dev = self.context.buffer(q.reshape(1, -1))
        if self._use_ivf():
            if filter is None:
                hs, ds = self._ivf_topk(q_dev, effective_k)[0]
                return SearchResults(self._results(hs, ds), live, time.perf_counter_ns() - t0, False)
            # IVF with a filter: iterative over-fetch within VA_MAX_K (searchFiltered)
            fetch = min(2 * k, live, _lib.VA_MAX_K)
            while True:
                hs, ds = self._ivf_topk(q_dev, fetch)[0]
                res = [r for r in self._results(hs, ds) if filter(r.id, self._metadata.get(r.id.stableID))]
                if len(res) >= k or fetch >= min(live, _lib.VA_MAX_K):
                    return SearchResults(res[:k], len(hs), time.perf_counter_ns() - t0, False)
                fetch = min(fetch * 2, live, _lib.VA_MAX_K)
        hs, ds = self._flat_topk(q_dev, effective_k)[0]
        return SearchResults(self._results(hs, ds), live, time.perf_counter_ns() - t0, True)

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
        t0 = time.perf_counter_ns()
        effective_k = min(k, live, _lib.VA_MAX_K)
        q_dev = self.context.buffer(qs)
        ivf = self._use_ivf()
        rows = self._ivf_topk(q_dev, effective_k) if ivf else self._flat_topk(q_dev, effective_k)
        dt = time.perf_counter_ns() - t0
        return [SearchResults(self._results(hs, ds), live, dt, not ivf) for hs, ds in rows]

    def searchDevice(self, queries_dev, k: int, out_handles, out_dist):
        """encode tier of the flat search: device queries [Q x D] -> device handles / distances
        [Q x k] (uint32 / fp32 tensors), enqueued on the context's stream (va_index_search)."""
        c = self.context
        Q = queries_dev.shape[0]
        c.order_after_torch()
        c.check(c.lib.va_index_search(c.handle, self._h, self._metric, dptr(queries_dev), Q, k, dptr(out_handles),
                                      dptr(out_dist)), "va_index_search")

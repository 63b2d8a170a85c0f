"""AcceleratedVectorIndex — host semantics of the reference's index actor over the C ABI.

Reference: Index/AcceleratedVectorIndex.swift (init :166-237, insert :481-700, remove
:771-833, compact :834-893, search :895-1000, searchUnfiltered :1103-1186, searchFiltered
:1188-1265, searchBatchGPU :1278-1374, searchIVF :1378-1431); handles
(Index/Types/VectorHandle.swift:33-70, Index/Internal/HandleAllocator.swift:39-242).

Storage is a growable row-major fp32 device buffer (slots); handles are stable ids that survive
compaction; deletions are a host mask honoured by over-fetching (fetchK = k + deletedCount).
Every distance and selection runs in libva_hip.so (va_fused_topk / va_ivf_*); this module only
keeps the bookkeeping the reference keeps on the host.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .context import GPUContext, VectorError, dptr
from .ivf import IVFGPUIndexStructure, IVFSearchConfiguration, IVFSearchPipeline
from .kernels import FusedL2TopKKernel, FusedL2TopKParameters, Metric


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
    distance: float  # L2^2

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
    """IndexConfiguration (Index/Types/IndexConfiguration.swift): flat or IVF, L2^2 only."""

    dimension: int
    capacity: int = 10_000
    metric: str = "euclidean"
    indexType: tuple = ("flat",)
    routingThreshold: int = 0

    @classmethod
    def flat(cls, dimension: int, capacity: int = 10_000):
        return cls(dimension, capacity)

    @classmethod
    def ivf(cls, dimension: int, nlist: int, nprobe: int, capacity: int = 100_000, routingThreshold: int = 0):
        return cls(dimension, capacity, "euclidean", ("ivf", nlist, nprobe), routingThreshold)

    def validate(self):
        if self.dimension <= 0:
            raise VectorError.invalidInput(f"dimension must be positive, got {self.dimension}")
        if self.capacity <= 0:
            raise VectorError.invalidInput(f"capacity must be positive, got {self.capacity}")
        if self.metric != "euclidean":
            # AcceleratedVectorIndex.validateMetricSupport: GPU search is L2^2 only
            raise VectorError("unsupported", f"metric {self.metric} is not supported by the index")
        if self.indexType[0] == "ivf":
            nlist, nprobe = self.indexType[1], self.indexType[2]
            if nlist < 1 or nprobe < 1 or nprobe > nlist:
                raise VectorError.invalidInput(f"invalid IVF parameters nlist={nlist} nprobe={nprobe}")


class AcceleratedVectorIndex:
    def __init__(self, configuration: IndexConfiguration, context: GPUContext | None = None):
        configuration.validate()
        self.configuration = configuration
        self.context = context or GPUContext(0)
        torch = _torch()
        self._storage = self.context.empty((configuration.capacity, configuration.dimension), torch.float32)
        self._slots = 0                     # allocated slots (deleted included)
        self._slot_handle: list[int] = []   # slot -> stable id
        self._handle_slot: dict[int, int] = {}
        self._deleted = np.zeros(configuration.capacity, bool)
        self._deleted_count = 0
        self._next_id = 0
        self._metadata: dict[int, object] = {}
        self._kernel = FusedL2TopKKernel(self.context)
        self._ivf: IVFGPUIndexStructure | None = None
        self._ivf_dirty = True
        self._centroids = None
        if configuration.indexType[0] == "ivf":
            _, nlist, nprobe = configuration.indexType
            self._ivf_pipe = IVFSearchPipeline(self.context, IVFSearchConfiguration(nlist, nprobe,
                                                                                    configuration.dimension))

    # -- properties ------------------------------------------------------------------------
    @property
    def count(self) -> int:
        return self._slots - self._deleted_count

    @property
    def dimension(self) -> int:
        return self.configuration.dimension

    @property
    def isEmpty(self) -> bool:
        return self.count == 0

    @property
    def capacity(self) -> int:
        return self._storage.shape[0]

    @property
    def isIVF(self) -> bool:
        return self.configuration.indexType[0] == "ivf"

    @property
    def isTrained(self) -> bool:
        return self._centroids is not None

    # -- mutation ----------------------------------------------------------------------------
    def _grow(self, need: int):
        torch = _torch()
        cap = self._storage.shape[0]
        if need <= cap:
            return
        new_cap = max(need, cap * 2)
        s = self.context.empty((new_cap, self.dimension), torch.float32)
        s[:self._slots] = self._storage[:self._slots]
        self._storage = s
        self._deleted = np.concatenate([self._deleted, np.zeros(new_cap - cap, bool)])

    def insert(self, vector=None, metadata=None, vectors=None):
        """insert(vector) -> VectorHandle, or insert(vectors=[...]) -> [VectorHandle]."""
        torch = _torch()
        batch = vectors is not None
        arr = np.asarray(vectors if batch else [vector], np.float32)
        if arr.ndim != 2 or arr.shape[1] != self.dimension:
            got = arr.shape[-1] if arr.ndim >= 1 else 0
            raise VectorError.dimensionMismatch(self.dimension, got)
        n = arr.shape[0]
        self._grow(self._slots + n)
        self._storage[self._slots:self._slots + n] = torch.from_numpy(arr).to(self._storage.device)
        handles = []
        for i in range(n):
            hid = self._next_id
            self._next_id += 1
            self._slot_handle.append(hid)
            self._handle_slot[hid] = self._slots + i
            if metadata is not None and not batch:
                self._metadata[hid] = metadata
            handles.append(VectorHandle(hid))
        first = self._slots
        self._slots += n
        if self._ivf is not None and not self._ivf_dirty:
            # built lists: append the new rows to their nearest lists (va_ivf_add) instead of a rebuild
            self._ivf.add(self._storage[first:first + n], first)
        else:
            self._ivf_dirty = True
        return handles if batch else handles[0]

    def remove(self, handle):
        """remove(handle) or remove([handles]) -> number removed (AcceleratedVectorIndex.swift:771-833)."""
        hs = handle if isinstance(handle, (list, tuple)) else [handle]
        removed = 0
        for h in hs:
            slot = self._handle_slot.pop(h.stableID, None)
            if slot is None:
                if not isinstance(handle, (list, tuple)):
                    raise VectorError.invalidInput(f"invalid handle {h.stableID}")
                continue
            self._deleted[slot] = True
            self._deleted_count += 1
            self._metadata.pop(h.stableID, None)
            removed += 1
        self._ivf_dirty = True
        return removed

    def compact(self):
        """Drop deleted slots; handles keep their stable ids (AcceleratedVectorIndex.swift:834-893)."""
        torch = _torch()
        keep = np.nonzero(~self._deleted[:self._slots])[0]
        if len(keep) == self._slots:
            return
        idx = torch.from_numpy(keep.astype(np.int64)).to(self._storage.device)
        self._storage[:len(keep)] = self._storage[idx].clone()
        self._slot_handle = [self._slot_handle[s] for s in keep]
        self._handle_slot = {h: i for i, h in enumerate(self._slot_handle)}
        self._slots = len(keep)
        self._deleted[:] = False
        self._deleted_count = 0
        self._ivf_dirty = True

    def vector(self, handle: VectorHandle):
        slot = self._handle_slot.get(handle.stableID)
        return None if slot is None else self._storage[slot].cpu().numpy().tolist()

    def metadata(self, handle: VectorHandle):
        return self._metadata.get(handle.stableID)

    def contains(self, handle: VectorHandle) -> bool:
        return handle.stableID in self._handle_slot

    # -- IVF ---------------------------------------------------------------------------------
    def train(self, centroids=None, seed: int = 0x5EED):
        """Train the IVF centroids; the lists are then built from the stored vectors.

        Without ``centroids``: k-means on the device over the live (not deleted) vectors with
        k-means++ seeding, 25 iterations at most, threshold 0.001, as IVFStructure.train
        (Index/Internal/IVFStructure.swift:202-259) called by AcceleratedVectorIndex.train
        (AcceleratedVectorIndex.swift:406-446).  With ``centroids`` ([nlist x D]): installs them.
        """
        if not self.isIVF:
            raise VectorError.invalidInput("train() needs an IVF index")
        nlist = self.configuration.indexType[1]
        if centroids is None:
            from .clustering import KMeansConfiguration, KMeansPipeline

            live = np.nonzero(~self._deleted[:self._slots])[0]
            if live.size == 0:
                raise VectorError.invalidInput("Cannot train IVF index with no vectors")
            if live.size < nlist:
                raise VectorError.invalidInput(
                    f"Need at least {nlist} vectors for {nlist} clusters, got {live.size}")
            torch = _torch()
            rows = self._storage[torch.as_tensor(live, device=self._storage.device)].contiguous()
            cfg = KMeansConfiguration(nlist, self.dimension, maxIterations=25, convergenceThreshold=0.001, seed=seed)
            self._centroids = KMeansPipeline(self.context, cfg).fit(rows).centroids
        else:
            c = np.asarray(centroids, np.float32)
            if c.shape != (nlist, self.dimension):
                raise VectorError.invalidInput(f"centroids must be {nlist} x {self.dimension}")
            self._centroids = self.context.buffer(c)
        self._ivf_dirty = True

    def _ivf_structure(self) -> IVFGPUIndexStructure:
        if self._ivf is None or self._ivf_dirty:
            if self._ivf is not None:
                self._ivf.close()
            self._ivf = self._ivf_pipe.prepareIndexStructure(self._centroids, self._storage[:self._slots])
            self._ivf_dirty = False
        return self._ivf

    def _use_ivf(self) -> bool:
        if not (self.isIVF and self.isTrained):
            return False
        t = self.configuration.routingThreshold
        return not (t > 0 and self.count < t)

    # -- search --------------------------------------------------------------------------------
    def _raw_topk(self, q_dev, fetch_k: int):
        """Slot ids and L2^2 distances of the fetch_k nearest slots for every query row."""
        torch = _torch()
        Q = q_dev.shape[0]
        if self._use_ivf():
            st = self._ivf_structure()
            res = self._ivf_pipe.search(q_dev, st, fetch_k)
            return res.indices.cpu().numpy().view(np.uint32), res.distances.cpu().numpy()
        idx = self.context.empty((Q, fetch_k), torch.int32)
        dist = self.context.empty((Q, fetch_k), torch.float32)
        c = self.context
        c.order_after_torch()
        self._kernel.encode(q_dev, self._storage, idx, dist,
                            FusedL2TopKParameters(Q, self._slots, self.dimension, fetch_k), Metric.euclideanSquared)
        c.synchronize()
        return idx.cpu().numpy().view(np.uint32), dist.cpu().numpy()

    def _collect(self, ids, dists, k, filt=None, seen=None):
        out = []
        for s, d in zip(ids, dists):
            s = int(s)
            if s == _lib.VA_SENTINEL_INDEX or s >= self._slots:
                continue
            if seen is not None:
                if s in seen:
                    continue
                seen.add(s)
            if self._deleted[s]:
                continue
            hid = self._slot_handle[s]
            h = VectorHandle(hid)
            if filt is not None and not filt(h, self._metadata.get(hid)):
                continue
            out.append(IndexSearchResult(h, float(d)))
            if len(out) >= k:
                break
        return out

    def search(self, query=None, k: int = 10, filter=None, queries=None):
        """search(query, k[, filter]) -> SearchResults; search(queries=[...], k) -> [SearchResults]."""
        if queries is not None:
            return self._search_batch(queries, k, filter)
        q = np.asarray(query, np.float32).reshape(-1)
        if q.shape[0] != self.dimension:
            raise VectorError.dimensionMismatch(self.dimension, q.shape[0])
        if k <= 0:
            raise VectorError.invalidInput(f"k must be positive, got {k}")
        if self.count == 0:
            return SearchResults()
        t0 = time.perf_counter_ns()
        q_dev = self.context.buffer(q.reshape(1, -1))
        effective_k = min(k, self.count)
        if filter is None:
            fetch = min(effective_k + self._deleted_count, self._slots, _lib.VA_MAX_K)
            ids, d = self._raw_topk(q_dev, fetch)
            res = self._collect(ids[0], d[0], effective_k)
            return SearchResults(res, self._slots, time.perf_counter_ns() - t0, not self._use_ivf())
        # iterative over-fetch (searchFiltered): double fetchK until k results pass the filter
        seen: set[int] = set()
        results: list[IndexSearchResult] = []
        fetch = min(k * 2, self._slots, _lib.VA_MAX_K)
        while True:
            ids, d = self._raw_topk(q_dev, fetch)
            results += self._collect(ids[0], d[0], k - len(results), filter, seen)
            nxt = min(fetch * 2, self._slots, _lib.VA_MAX_K)
            if len(results) >= k or nxt == fetch or len(seen) >= self._slots:
                break
            fetch = nxt
        return SearchResults(results[:k], len(seen), time.perf_counter_ns() - t0, not self._use_ivf())

    def _search_batch(self, queries, k, filter):
        qs = np.asarray(queries, np.float32)
        if qs.size == 0:
            return []
        if qs.ndim != 2 or qs.shape[1] != self.dimension:
            raise VectorError.dimensionMismatch(self.dimension, qs.shape[-1])
        if self.count == 0:
            return [SearchResults() for _ in range(qs.shape[0])]
        if filter is not None:
            return [self.search(q, k, filter) for q in qs]
        t0 = time.perf_counter_ns()
        effective_k = min(k, self.count)
        fetch = min(effective_k + self._deleted_count, self._slots, _lib.VA_MAX_K)
        ids, d = self._raw_topk(self.context.buffer(qs), fetch)
        dt = time.perf_counter_ns() - t0
        return [SearchResults(self._collect(ids[r], d[r], effective_k), self._slots, dt, not self._use_ivf())
                for r in range(qs.shape[0])]

"""Product quantization — host mirror of Metal4ProductQuantizationKernel and its types.

Reference: Kernels/Metal4/ProductQuantizationKernel.swift:23-60 (Metal4PQConfig), :62-107
(Metal4PQModel), :109-140 (Metal4EncodedVectors), :221-560 (the kernel: train, encode,
computeDistances, trainAndEncode, findNearestNeighbors).  Every step runs in libva_hip.so
(va_pq_*); this module checks arguments and wraps device tensors.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from .context import GPUContext, VectorError, dptr
from .kernels import _as_matrix


def _torch():
    import torch

    return torch


@dataclass
class Metal4PQConfig:
    dimension: int
    M: int = 8
    K: int = 256
    trainIterations: int = 25
    convergenceThreshold: float = 0.001

    def __post_init__(self):
        if self.M < 1 or self.dimension % self.M != 0:
            raise VectorError.invalidInput("Dimension must be divisible by M")
        if not 1 <= self.K <= 256:
            raise VectorError.invalidInput("K must be <= 256 for uint8 encoding")

    @property
    def D_sub(self) -> int:
        return self.dimension // self.M

    @property
    def compressionRatio(self) -> float:
        return self.dimension * 32 / (self.M * 8)


class Metal4PQModel:
    """Trained codebooks [M x K x D_sub] on the device."""

    def __init__(self, codebooks, config: Metal4PQConfig, iterations: int = 0):
        self.codebooks = codebooks
        self.config = config
        self.iterations = iterations

    def decodeCentroid(self, subspace: int, code: int) -> list[float]:
        if subspace >= self.config.M:
            return []
        return self.codebooks[subspace, code].cpu().numpy().tolist()


class Metal4EncodedVectors:
    """Codes [N x M] bytes on the device."""

    def __init__(self, codes, count: int, config: Metal4PQConfig):
        self.codes = codes
        self.count = count
        self.config = config

    def decode(self, index: int, model: Metal4PQModel) -> list[float]:
        if index >= self.count:
            return []
        code = self.codes[index].cpu().numpy()
        cb = model.codebooks.cpu().numpy()
        return np.concatenate([cb[m, code[m]] for m in range(self.config.M)]).tolist()


class ProductQuantizationKernel:
    """Metal4ProductQuantizationKernel (ProductQuantizationKernel.swift:221-560)."""

    def __init__(self, context: GPUContext):
        self.context = context

    def _dev(self, a, what):
        return a if hasattr(a, "is_cuda") else self.context.buffer(_as_matrix(a, what))

    def train(self, data, config: Metal4PQConfig, seed: int = 0x5EED, initialCodebooks=None) -> Metal4PQModel:
        torch = _torch()
        c = self.context
        x = self._dev(data, "data")
        if x.shape[1] != config.dimension:
            raise VectorError.dimensionMismatch(config.dimension, x.shape[1])
        cb = c.empty((config.M, config.K, config.D_sub), torch.float32)
        init = None
        if initialCodebooks is not None:
            init = initialCodebooks if hasattr(initialCodebooks, "is_cuda") else c.buffer(
                np.ascontiguousarray(initialCodebooks, np.float32))
        it = C.c_uint32(0)
        c.order_after_torch()
        c.check(c.lib.va_pq_train(c.handle, dptr(x), x.shape[0], x.shape[1], config.M, config.K,
                                  config.trainIterations, C.c_float(config.convergenceThreshold), C.c_uint64(seed),
                                  dptr(init), dptr(cb), C.byref(it)), "va_pq_train")
        return Metal4PQModel(cb, config, int(it.value))

    def encode(self, vectors, model: Metal4PQModel) -> Metal4EncodedVectors:
        torch = _torch()
        c = self.context
        cfg = model.config
        x = self._dev(vectors, "vectors")
        if x.shape[1] != cfg.dimension:
            raise VectorError.dimensionMismatch(cfg.dimension, x.shape[1])
        codes = c.empty((x.shape[0], cfg.M), torch.uint8)
        c.order_after_torch()
        c.check(c.lib.va_pq_encode(c.handle, dptr(x), x.shape[0], x.shape[1], cfg.M, cfg.K, dptr(model.codebooks),
                                   dptr(codes)), "va_pq_encode")
        c.synchronize()
        return Metal4EncodedVectors(codes, x.shape[0], cfg)

    def trainAndEncode(self, data, config: Metal4PQConfig, seed: int = 0x5EED):
        model = self.train(data, config, seed)
        return model, self.encode(data, model)

    def computeDistanceTables(self, queries, model: Metal4PQModel):
        torch = _torch()
        c = self.context
        cfg = model.config
        q = self._dev(queries, "queries")
        if q.shape[1] != cfg.dimension:
            raise VectorError.dimensionMismatch(cfg.dimension, q.shape[1])
        t = c.empty((q.shape[0], cfg.M, cfg.K), torch.float32)
        c.order_after_torch()
        c.check(c.lib.va_pq_distance_tables(c.handle, dptr(q), q.shape[0], q.shape[1], cfg.M, cfg.K,
                                            dptr(model.codebooks), dptr(t)), "va_pq_distance_tables")
        c.synchronize()
        return t

    def computeDistances(self, queries, encodedVectors: Metal4EncodedVectors, model: Metal4PQModel):
        """Squared ADC distances [Q x N] (computeDistances, :409-478, batched over queries)."""
        torch = _torch()
        c = self.context
        cfg = model.config
        t = self.computeDistanceTables(queries, model)
        out = c.empty((t.shape[0], encodedVectors.count), torch.float32)
        c.order_after_torch()
        c.check(c.lib.va_pq_adc_distances(c.handle, dptr(t), t.shape[0], dptr(encodedVectors.codes),
                                          encodedVectors.count, cfg.M, cfg.K, dptr(out)), "va_pq_adc_distances")
        c.synchronize()
        return out

    def search(self, queries, encodedDatabase: Metal4EncodedVectors, model: Metal4PQModel, k: int):
        """(indices [Q x k] int32 view of uint32, distances [Q x k] = sqrt of the ADC sum)."""
        torch = _torch()
        c = self.context
        cfg = model.config
        q = self._dev(queries, "queries")
        if q.shape[1] != cfg.dimension:
            raise VectorError.dimensionMismatch(cfg.dimension, q.shape[1])
        idx = c.empty((q.shape[0], k), torch.int32)
        dist = c.empty((q.shape[0], k), torch.float32)
        c.order_after_torch()
        c.check(c.lib.va_pq_search(c.handle, dptr(q), q.shape[0], q.shape[1], cfg.M, cfg.K, dptr(model.codebooks),
                                   dptr(encodedDatabase.codes), encodedDatabase.count, k, dptr(idx), dptr(dist)),
                "va_pq_search")
        c.synchronize()
        return idx, dist

    def findNearestNeighbors(self, query, encodedDatabase: Metal4EncodedVectors, model: Metal4PQModel, k: int):
        """[(index, distance)] of one query (findNearestNeighbors, :504-540)."""
        q = np.asarray(query, np.float32).reshape(1, -1)
        idx, dist = self.search(q, encodedDatabase, model, k)
        i = idx.cpu().numpy().view(np.uint32)[0]
        d = dist.cpu().numpy()[0]
        return [(int(a), float(b)) for a, b in zip(i, d) if a != 0xFFFFFFFF]

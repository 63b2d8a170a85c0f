"""Scalar-int8 and binary quantization kernels — host mirror of the reference's wrappers.

ScalarQuantizationKernel   Kernels/Metal4/ScalarQuantizationKernel.swift:169-520
BinaryQuantizationKernel   Kernels/Metal4/BinaryQuantizationKernel.swift:19-401
HammingDistanceKernel      Kernels/Metal4/HammingDistanceKernel.swift:19-363
All arithmetic (min/max, quantize, scans, packing, Hamming) runs in libva_hip.so.
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import IntEnum

import numpy as np

from . import _lib
from .context import GPUContext, VectorError, dptr
from .kernels import _as_matrix


def _torch():
    import torch

    return torch


# ---------------------------------------------------------------------------------------
# scalar int8
# ---------------------------------------------------------------------------------------
class Metal4QuantizationType(IntEnum):
    """Metal4QuantizationType (ScalarQuantizationKernel.swift:22-32)."""

    symmetric = 0
    asymmetric = 1
    perChannel = 2
    dynamic = 3


class Metal4BitWidth(IntEnum):
    int8 = 8


@dataclass
class Metal4QuantizationResult:
    """Metal4QuantizationResult (ScalarQuantizationKernel.swift:99-118)."""

    quantizedData: bytes
    scale: float
    zeroPoint: int | None
    bitWidth: Metal4BitWidth
    compressionRatio: float


@dataclass
class PerDimensionParameters:
    """Per-dimension affine int8 parameters (min, max, scale, int32 zero point)."""

    min: np.ndarray
    max: np.ndarray
    scale: np.ndarray
    zeroPoint: np.ndarray


class ScalarQuantizationKernel:
    """int8 quantize / dequantize and the int8 top-k scan.

    ``quantize(data, type)`` keeps the reference's global-parameter API (its parameters are
    computed on the CPU there too, ScalarQuantizationKernel.swift:496-520); the per-dimension
    API (``computePerDimensionParameters`` / ``quantizePerDimension`` / ``searchTopK``) is the
    search path's min/max affine map with an int32 zero point.
    """

    name = "ScalarQuantizationKernel"

    def __init__(self, context: GPUContext):
        self.context = context

    # -- encode tier (device tensors) ---------------------------------------------------------
    def encodeComputeParameters(self, x, numVectors: int, dimension: int, outMin, outMax, outScale, outZeroPoint):
        c = self.context
        c.check(c.lib.va_sq_params_per_dim(c.handle, dptr(x), numVectors, dimension, dptr(outMin), dptr(outMax),
                                           dptr(outScale), dptr(outZeroPoint)), "va_sq_params_per_dim")

    def encodeQuantize(self, x, codes, scale, zeroPoint, numVectors: int, dimension: int):
        c = self.context
        c.check(c.lib.va_sq_quantize_i8(c.handle, dptr(x), numVectors, dimension, dptr(scale), dptr(zeroPoint),
                                        dptr(codes)), "va_sq_quantize_i8")

    def encodeDequantize(self, codes, out, scale, zeroPoint, numVectors: int, dimension: int):
        c = self.context
        c.check(c.lib.va_sq_dequantize_i8(c.handle, dptr(codes), numVectors, dimension, dptr(scale),
                                          dptr(zeroPoint), dptr(out)), "va_sq_dequantize_i8")

    def encodeScanTopK(self, queryCodes, databaseCodes, outIdx, outDist, numQueries: int, numDatabase: int,
                       dimension: int, k: int):
        c = self.context
        c.check(c.lib.va_i8_scan_topk(c.handle, dptr(queryCodes), dptr(databaseCodes), numQueries, numDatabase,
                                      dimension, k, dptr(outIdx), dptr(outDist)), "va_i8_scan_topk")

    # -- execute tier ----------------------------------------------------------------------------
    def computePerDimensionParameters(self, x) -> PerDimensionParameters:
        torch = _torch()
        c = self.context
        dx = x if hasattr(x, "is_cuda") else c.buffer(_as_matrix(x, "data"))
        n, d = dx.shape
        mn = c.empty((d,), torch.float32)
        mx = c.empty((d,), torch.float32)
        sc = c.empty((d,), torch.float32)
        zp = c.empty((d,), torch.int32)
        c.order_after_torch()
        self.encodeComputeParameters(dx, n, d, mn, mx, sc, zp)
        c.synchronize()
        return PerDimensionParameters(mn.cpu().numpy(), mx.cpu().numpy(), sc.cpu().numpy(), zp.cpu().numpy())

    def quantizePerDimension(self, x, params: PerDimensionParameters):
        """Codes (device int8 tensor) of x under per-dimension parameters."""
        torch = _torch()
        c = self.context
        dx = x if hasattr(x, "is_cuda") else c.buffer(_as_matrix(x, "data"))
        n, d = dx.shape
        if params.scale.shape[0] != d:
            raise VectorError.dimensionMismatch(params.scale.shape[0], d)
        codes = c.empty((n, d), torch.int8)
        sc = c.buffer(np.asarray(params.scale, np.float32))
        zp = c.buffer(np.asarray(params.zeroPoint, np.int32))
        c.order_after_torch()
        self.encodeQuantize(dx, codes, sc, zp, n, d)
        c.synchronize()
        return codes

    def dequantizePerDimension(self, codes, params: PerDimensionParameters):
        torch = _torch()
        c = self.context
        n, d = codes.shape
        out = c.empty((n, d), torch.float32)
        sc = c.buffer(np.asarray(params.scale, np.float32))
        zp = c.buffer(np.asarray(params.zeroPoint, np.int32))
        c.order_after_torch()
        self.encodeDequantize(codes, out, sc, zp, n, d)
        c.synchronize()
        return out

    def searchTopK(self, queryCodes, databaseCodes, k: int):
        """Exact int8 scan: distance = -dot (int32); returns (indices uint32, distances int32)."""
        torch = _torch()
        c = self.context
        q = queryCodes if hasattr(queryCodes, "is_cuda") else c.buffer(np.asarray(queryCodes, np.int8))
        x = databaseCodes if hasattr(databaseCodes, "is_cuda") else c.buffer(np.asarray(databaseCodes, np.int8))
        if q.shape[1] != x.shape[1]:
            raise VectorError.dimensionMismatch(x.shape[1], q.shape[1])
        idx = c.empty((q.shape[0], k), torch.int32)
        dist = c.empty((q.shape[0], k), torch.int32)
        c.order_after_torch()
        self.encodeScanTopK(q, x, idx, dist, q.shape[0], x.shape[0], q.shape[1], k)
        c.synchronize()
        return idx.cpu().numpy().view(np.uint32), dist.cpu().numpy()

    # -- the reference's global-parameter API ----------------------------------------------------
    @staticmethod
    def _global_params(data: np.ndarray, qtype: Metal4QuantizationType):
        """computeQuantizationParams (ScalarQuantizationKernel.swift:496-520), int8 branch."""
        mn = np.float32(data.min()) if data.size else np.float32(0)
        mx = np.float32(data.max()) if data.size else np.float32(0)
        if qtype == Metal4QuantizationType.asymmetric:
            scale = np.float32(max(np.float32(mx - mn) / np.float32(255.0), np.float32(1e-8)))
            r = float(-(mn / scale))
            zp = int(np.clip(np.sign(r) * np.floor(abs(r) + 0.5), -128, 127))  # Int8(clamping: round(.))
            return scale, zp
        absmax = np.float32(max(abs(mn), abs(mx)))
        return np.float32(max(absmax / np.float32(127.0), np.float32(1e-8))), None

    def quantize(self, data, bitWidth: Metal4BitWidth = Metal4BitWidth.int8,
                 type: Metal4QuantizationType = Metal4QuantizationType.symmetric) -> Metal4QuantizationResult:
        arr = np.ascontiguousarray(np.asarray(data, np.float32).reshape(-1))
        if arr.size == 0:
            raise VectorError.invalidInput("Empty input data")
        scale, zp = self._global_params(arr, type)
        p = PerDimensionParameters(np.zeros(1, np.float32), np.zeros(1, np.float32), np.array([scale], np.float32),
                                   np.array([zp or 0], np.int32))
        codes = self.quantizePerDimension(self.context.buffer(arr.reshape(-1, 1)), p)
        raw = codes.cpu().numpy().reshape(-1).tobytes()
        return Metal4QuantizationResult(raw, float(scale), zp if type == Metal4QuantizationType.asymmetric else None,
                                        bitWidth, float(arr.size * 4) / float(len(raw)))

    def dequantize(self, result: Metal4QuantizationResult, count: int) -> np.ndarray:
        codes = np.frombuffer(result.quantizedData, np.int8)[:count].reshape(-1, 1)
        p = PerDimensionParameters(np.zeros(1, np.float32), np.zeros(1, np.float32),
                                   np.array([result.scale], np.float32), np.array([result.zeroPoint or 0], np.int32))
        out = self.dequantizePerDimension(self.context.buffer(codes), p)
        return out.cpu().numpy().reshape(-1)


ScalarQuantKernel = ScalarQuantizationKernel


# ---------------------------------------------------------------------------------------
# binary
# ---------------------------------------------------------------------------------------
class Metal4BinaryVector:
    """Bit-packed binary vector (BinaryQuantizationKernel.swift:23-75): LSB-first words."""

    def __init__(self, data, dimension: int):
        self.data = [int(w) & 0xFFFFFFFF for w in data]
        self.dimension = int(dimension)
        self.numWords = (self.dimension + 31) // 32

    def asBoolArray(self) -> list[bool]:
        return [self.bit(i) for i in range(self.dimension)]

    def bit(self, index: int) -> bool:
        if index < 0 or index >= self.dimension:
            return False
        w = index // 32
        return w < len(self.data) and bool((self.data[w] >> (index % 32)) & 1)

    def asFloatArray(self) -> list[float]:
        return [1.0 if b else 0.0 for b in self.asBoolArray()]

    def hammingDistance(self, other: "Metal4BinaryVector") -> int:
        """The reference's CPU method on the value type (BinaryQuantizationKernel.swift:65-74)."""
        if self.dimension != other.dimension:
            return -1
        return sum(bin((self.data[i] if i < len(self.data) else 0) ^ (other.data[i] if i < len(other.data) else 0))
                   .count("1") for i in range(self.numWords))


class Metal4BinaryVectorBatch:
    def __init__(self, vectors: list[Metal4BinaryVector]):
        if not vectors:
            raise VectorError.invalidInput("Cannot create empty batch")
        if any(v.dimension != vectors[0].dimension for v in vectors):
            raise VectorError.invalidInput("All vectors must have same dimension")
        self.vectors = vectors
        self.dimension = vectors[0].dimension
        self.numWords = vectors[0].numWords

    @property
    def count(self) -> int:
        return len(self.vectors)

    def vector(self, index: int):
        return self.vectors[index] if 0 <= index < len(self.vectors) else None

    def codes(self) -> np.ndarray:
        return np.array([v.data for v in self.vectors], dtype=np.uint32).reshape(self.count, self.numWords)


@dataclass
class Metal4BinaryQuantizationResult:
    binaryVectors: Metal4BinaryVectorBatch
    compressionRatio: float
    originalBytes: int
    compressedBytes: int


@dataclass
class Metal4HammingDistanceResult:
    distances: list[float]


class BinaryQuantizationKernel:
    """Sign-bit quantization (x > 0) and Hamming distances (BinaryQuantizationKernel.swift:79-401)."""

    name = "BinaryQuantizationKernel"

    def __init__(self, context: GPUContext):
        self.context = context

    def encodeQuantize(self, x, codes, numVectors: int, dimension: int):
        c = self.context
        c.check(c.lib.va_bq_pack(c.handle, dptr(x), numVectors, dimension, dptr(codes)), "va_bq_pack")

    def pack(self, x):
        """Device codes [N x ceil(D/32)] (int32 tensor holding uint32 words)."""
        torch = _torch()
        c = self.context
        dx = x if hasattr(x, "is_cuda") else c.buffer(_as_matrix(x, "vectors"))
        n, d = dx.shape
        codes = c.empty((n, (d + 31) // 32), torch.int32)
        c.order_after_torch()
        self.encodeQuantize(dx, codes, n, d)
        c.synchronize()
        return codes

    def quantize(self, vectors=None, config=None, vector=None):
        if vector is not None:
            return self.quantize([list(vector)]).binaryVectors.vectors[0]
        m = _as_matrix(vectors, "vectors")
        if m.shape[1] == 0:
            raise VectorError.invalidInput("Input vectors cannot be empty")
        words = self.pack(m).cpu().numpy().view(np.uint32)
        batch = Metal4BinaryVectorBatch([Metal4BinaryVector(words[i].tolist(), m.shape[1]) for i in range(m.shape[0])])
        orig = m.size * 4
        comp = words.size * 4
        return Metal4BinaryQuantizationResult(batch, orig / comp, orig, comp)

    @staticmethod
    def compressionRatio(dimension: int) -> float:
        return (dimension * 4) / (((dimension + 31) // 32) * 4)

    def computeHammingDistances(self, query: Metal4BinaryVector,
                                candidates: Metal4BinaryVectorBatch) -> Metal4HammingDistanceResult:
        if query.dimension != candidates.dimension:
            raise VectorError.invalidInput("Query and candidate dimensions must match")
        m = HammingDistanceKernel(self.context).computeBitPacked(np.array([query.data], np.uint32),
                                                                 candidates.codes())
        return Metal4HammingDistanceResult([float(v) for v in m[0]])


BinaryQuantKernel = BinaryQuantizationKernel


class HammingDistanceKernel:
    """Q x N Hamming distances on bit-packed codes and the exact Hamming top-k
    (HammingDistanceKernel.swift:150-363; nearestNeighbors :114-120)."""

    name = "HammingDistanceKernel"

    def __init__(self, context: GPUContext):
        self.context = context

    def encodeBitPacked(self, queries, dataset, out, numQueries: int, numDataset: int, words: int):
        c = self.context
        c.check(c.lib.va_hamming_matrix(c.handle, dptr(queries), dptr(dataset), numQueries, numDataset, words,
                                        dptr(out)), "va_hamming_matrix")

    def encodeTopK(self, queries, dataset, outIdx, outDist, numQueries: int, numDataset: int, words: int, k: int):
        c = self.context
        c.check(c.lib.va_hamming_topk(c.handle, dptr(queries), dptr(dataset), numQueries, numDataset, words, k,
                                      dptr(outIdx), dptr(outDist)), "va_hamming_topk")

    def _dev_codes(self, codes):
        if hasattr(codes, "is_cuda"):
            return codes
        return self.context.buffer(np.ascontiguousarray(np.asarray(codes, np.uint32)).view(np.int32))

    def computeBitPacked(self, queries, dataset) -> np.ndarray:
        torch = _torch()
        c = self.context
        q, x = self._dev_codes(queries), self._dev_codes(dataset)
        if q.shape[1] != x.shape[1]:
            raise VectorError.invalidInput("Query and dataset word counts must match")
        out = c.empty((q.shape[0], x.shape[0]), torch.int32)
        c.order_after_torch()
        self.encodeBitPacked(q, x, out, q.shape[0], x.shape[0], q.shape[1])
        c.synchronize()
        return out.cpu().numpy().view(np.uint32)

    def nearestNeighbors(self, queries, dataset, k: int):
        """Exact top-k by (Hamming distance, index): (indices uint32, distances uint32)."""
        torch = _torch()
        c = self.context
        q, x = self._dev_codes(queries), self._dev_codes(dataset)
        idx = c.empty((q.shape[0], k), torch.int32)
        dist = c.empty((q.shape[0], k), torch.int32)
        c.order_after_torch()
        self.encodeTopK(q, x, idx, dist, q.shape[0], x.shape[0], q.shape[1], k)
        c.synchronize()
        return idx.cpu().numpy().view(np.uint32), dist.cpu().numpy().view(np.uint32)

    @staticmethod
    def packBinary(bits) -> list[int]:
        """packBinary (HammingDistanceKernel.swift): LSB-first uint32 words of a bool vector."""
        words = [0] * ((len(bits) + 31) // 32)
        for i, b in enumerate(bits):
            if b:
                words[i // 32] |= 1 << (i % 32)
        return words

    def distance(self, a, b) -> int:
        return int(self.distanceMatrix([a], [b])[0][0])

    def distanceMatrix(self, queries, dataset) -> np.ndarray:
        qa = np.array([self.packBinary(v) for v in queries], np.uint32)
        xa = np.array([self.packBinary(v) for v in dataset], np.uint32)
        return self.computeBitPacked(qa, xa).astype(np.float32)

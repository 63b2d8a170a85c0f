"""vectoraccelerate_amd — MI355X (gfx950) flat/IVF vector search behind VectorAccelerate's API.

The product is ``libva_hip.so`` (hand-written HIP, C ABI in ``include/va_hip.h``).  This
package is the host-side mirror of the reference's kernel / index classes over that ABI.
"""
from ._lib import VA_MAX_K, VA_SENTINEL_INDEX, LibraryMissing
from .context import GPUContext, Metal4Context, VectorError
from .kernels import (
    CosineSimilarityKernel,
    DotProductKernel,
    DotProductParameters,
    FusedL2TopKKernel,
    FusedL2TopKParameters,
    FusedTopKKernel,
    L2DistanceKernel,
    Metal4FusedL2Config,
    Metal4FusedL2TopKResult,
    Metal4SelectionMode,
    Metric,
    TopKMergeKernel,
    TopKSelectionKernel,
)
from .index import (
    AcceleratedVectorIndex,
    IndexConfiguration,
    IndexSearchResult,
    SearchResults,
    VectorHandle,
)
from .clustering import KMeansConfiguration, KMeansPipeline, KMeansPlusPlusKernel, KMeansResult
from .provider import (
    CosineDistance,
    DotProductDistance,
    EuclideanDistance,
    MetalComputeProvider,
    SupportedDistanceMetric,
)
from .pq import Metal4EncodedVectors, Metal4PQConfig, Metal4PQModel, ProductQuantizationKernel
from .ivf import IVFGPUIndexStructure, IVFSearchConfiguration, IVFSearchPipeline, IVFSearchResult
from .quantization import (
    BinaryQuantizationKernel,
    BinaryQuantKernel,
    HammingDistanceKernel,
    Metal4BinaryVector,
    Metal4BinaryVectorBatch,
    Metal4QuantizationType,
    PerDimensionParameters,
    ScalarQuantizationKernel,
    ScalarQuantKernel,
)

__all__ = [
    "MetalComputeProvider",
    "SupportedDistanceMetric",
    "EuclideanDistance",
    "CosineDistance",
    "DotProductDistance",
    "AcceleratedVectorIndex",
    "IndexConfiguration",
    "IndexSearchResult",
    "SearchResults",
    "VectorHandle",
    "IVFGPUIndexStructure",
    "KMeansConfiguration",
    "KMeansPipeline",
    "KMeansPlusPlusKernel",
    "KMeansResult",
    "Metal4EncodedVectors",
    "Metal4PQConfig",
    "Metal4PQModel",
    "ProductQuantizationKernel",
    "IVFSearchConfiguration",
    "IVFSearchPipeline",
    "IVFSearchResult",
    "BinaryQuantizationKernel",
    "BinaryQuantKernel",
    "HammingDistanceKernel",
    "Metal4BinaryVector",
    "Metal4BinaryVectorBatch",
    "Metal4QuantizationType",
    "PerDimensionParameters",
    "ScalarQuantizationKernel",
    "ScalarQuantKernel",
    "VA_MAX_K",
    "VA_SENTINEL_INDEX",
    "LibraryMissing",
    "GPUContext",
    "Metal4Context",
    "VectorError",
    "CosineSimilarityKernel",
    "DotProductKernel",
    "DotProductParameters",
    "FusedL2TopKKernel",
    "FusedL2TopKParameters",
    "FusedTopKKernel",
    "L2DistanceKernel",
    "Metal4FusedL2Config",
    "Metal4FusedL2TopKResult",
    "Metal4SelectionMode",
    "Metric",
    "TopKMergeKernel",
    "TopKSelectionKernel",
]

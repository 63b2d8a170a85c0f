"""Writes the golden fixtures of the search path into tests/golden/*.json.

The fixtures are the known answers stated in gifton/VectorAccelerate's own XCTest suites,
restated as data (inputs + expected outputs).  Nothing here runs or imports the reference:
each expected value is the one the cited test asserts.  Re-run with
``python tests/golden/make_golden.py`` after editing.
"""
from __future__ import annotations

import json
from pathlib import Path

HERE = Path(__file__).resolve().parent
INF = float("inf")

FIXTURES = {
    # Global int8 quantization (ScalarQuantizationKernel.quantize with computeQuantizationParams,
    # Kernels/Metal4/ScalarQuantizationKernel.swift:496-520; codes by quantize_int8_kernel,
    # DataTransformations.metal:188-200).  The reference's tests assert only round trips
    # (KernelTests.swift:1775-1787) and order (:1850-1862); these cases are closed forms chosen so
    # that scale and codes are exact: a range of 255 or absMax of 127 gives scale 1 (254: 2).
    "sq_global": {
        "kind": "sq_global",
        "cases": [
            # absMax 127 -> scale 1; rint: 63.5 -> 64 (half even), -2.5 -> -2
            {"data": [-127, 63.5, 1, 0, -2.5], "asymmetric": False, "scale": 1.0, "zero_point": 0,
             "codes": [-127, 64, 1, 0, -2]},
            # absMax 254 -> scale 2: -2.5 / 2 = -1.25 -> -1
            {"data": [254, -2.5], "asymmetric": False, "scale": 2.0, "zero_point": 0, "codes": [127, -1]},
            # range 255 -> scale 1, zero point -round(-1) = 1; 254 + 1 saturates at 127
            {"data": [-1, 254, 0], "asymmetric": True, "scale": 1.0, "zero_point": 1, "codes": [0, 127, 1]},
            # Swift round is half away from zero: -round(-2.5) = 3 (half even would give 2)
            {"data": [-2.5, 252.5], "asymmetric": True, "scale": 1.0, "zero_point": 3, "codes": [0, 127]},
            # Int8(clamping:): -round(1000) = -1000 saturates to -128; codes saturate at 127
            {"data": [1000, 1255], "asymmetric": True, "scale": 1.0, "zero_point": -128, "codes": [127, 127]},
            # ... and -round(-300) = 300 saturates to 127
            {"data": [-300, -45], "asymmetric": True, "scale": 1.0, "zero_point": 127, "codes": [-128, 82]},
            # the 1e-8 scale floor: constant data and a tiny range
            {"data": [0, 0, 0], "asymmetric": True, "scale": 1e-8, "zero_point": 0, "codes": [0, 0, 0]},
            {"data": [1e-9, 2e-9], "asymmetric": False, "scale": 1e-8, "zero_point": 0, "codes": [0, 0]},
        ],
    },
    # Tests/VectorAccelerateTests/KernelTests.swift:806-835 (testBasicNearestNeighbors)
    "fused_topk_basic": {
        "kind": "flat_topk", "metric": 0, "k": 2,
        "queries": [[0, 0, 0, 0]],
        "dataset": [[1, 0, 0, 0], [2, 0, 0, 0], [0.5, 0, 0, 0], [3, 0, 0, 0]],
        "expected_idx": [[2, 0]], "expected_dist": [[0.25, 1.0]],
    },
    # FlatIndexSearchTests.swift:101-138 (testSearchResultsAreOrdered)
    "flat_ordering": {
        "kind": "flat_topk", "metric": 0, "k": 5,
        "queries": [[0, 0, 0, 0]],
        "dataset": [[3, 0, 0, 0], [1, 0, 0, 0], [2, 0, 0, 0], [0.5, 0, 0, 0], [4, 0, 0, 0]],
        "expected_idx": [[3, 1, 2, 0, 4]], "expected_dist": [[0.25, 1, 4, 9, 16]],
    },
    # FlatIndexSearchTests.swift:141-170 (ordering with negative values; the two distance-1
    # entries are ordered by the (distance, index) tie rule, Metal4Common.h:142-159)
    "flat_ordering_ties": {
        "kind": "flat_topk", "metric": 0, "k": 4,
        "queries": [[0, 0, 0, 0]],
        "dataset": [[-2, 0, 0, 0], [1, 0, 0, 0], [-1, 0, 0, 0], [0, 0, 0, 0]],
        "expected_idx": [[3, 1, 2, 0]], "expected_dist": [[0, 1, 1, 4]],
    },
    # FlatIndexSearchTests.swift:577-610 (L2^2 = 25 and 30)
    "flat_l2sq_25": {
        "kind": "flat_topk", "metric": 0, "k": 1,
        "queries": [[0, 0, 0, 0]], "dataset": [[3, 4, 0, 0]],
        "expected_idx": [[0]], "expected_dist": [[25.0]],
    },
    "flat_l2sq_30": {
        "kind": "flat_topk", "metric": 0, "k": 1,
        "queries": [[0, 0, 0, 0]], "dataset": [[1, 2, 3, 4]],
        "expected_idx": [[0]], "expected_dist": [[30.0]],
    },
    # FlatIndexSearchTests.swift:613-630 (L2^2 between points = 50)
    "flat_l2sq_50": {
        "kind": "flat_topk", "metric": 0, "k": 1,
        "queries": [[4, 6, 8]], "dataset": [[1, 2, 3]],
        "expected_idx": [[0]], "expected_dist": [[50.0]],
    },
    # FlatIndexSearchTests.swift:633-646 (exact match = 0)
    "flat_exact_match": {
        "kind": "flat_topk", "metric": 0, "k": 1,
        "queries": [[1.5, 2.5, 3.5, 4.5]], "dataset": [[1.5, 2.5, 3.5, 4.5]],
        "expected_idx": [[0]], "expected_dist": [[0.0]],
    },
    # KernelTests.swift:621-645 (testBasicTopKMinimum)
    "topk_min": {
        "kind": "topk_rows", "mode": "minimum", "k": 3,
        "values": [[5, 2, 8, 1, 9, 3], [7, 4, 0.5, 6, 2.5, 1.5]],
        "expected_idx": [[3, 1, 5], [2, 5, 4]], "expected_values": [[1, 2, 3], [0.5, 1.5, 2.5]],
    },
    # KernelTests.swift:647-660 (testBasicTopKMaximum)
    "topk_max": {
        "kind": "topk_rows", "mode": "maximum", "k": 3,
        "values": [[5, 2, 8, 1, 9, 3]],
        "expected_idx": [[4, 2, 0]], "expected_values": [[9, 8, 5]],
    },
    # KernelTests.swift:662-671 (testSingleQuery: 0..99, k=5)
    "topk_single": {
        "kind": "topk_rows", "mode": "minimum", "k": 5,
        "values": [list(range(100))],
        "expected_idx": [[0, 1, 2, 3, 4]], "expected_values": [[0, 1, 2, 3, 4]],
    },
    # KernelTests.swift:3490-3497 (packBinary [t,f,t,f,f,f,f,f] = 0b101) and :3499-3505 (64 x true)
    "bq_pack_basic": {
        "kind": "bq_pack",
        "vectors": [[1, -1, 1, -1, -1, -1, -1, -1]],
        "expected_codes": [[5]],
    },
    "bq_pack_64_true": {
        "kind": "bq_pack",
        "vectors": [[1.0] * 64],
        "expected_codes": [[4294967295, 4294967295]],
    },
    # KernelTests.swift:1933-1985 (identical 0, opposite 4, partial 2)
    "hamming_basic": {
        "kind": "hamming",
        "queries": [[1, 1, 1, 1], [1, 1, -1, -1]],
        "dataset": [[1, 1, 1, 1], [-1, -1, -1, -1], [1, -1, 1, -1]],
        "expected": [[0, 4, 2], [2, 2, 2]],
    },
    # KernelTests.swift:3463-3480 (testDistanceMatrix: [t,f] vs [[t,f],[f,f],[t,t]] -> 0,1,1)
    "hamming_matrix": {
        "kind": "hamming",
        "queries": [[1, -1], [-1, 1]],
        "dataset": [[1, -1], [-1, -1], [1, 1]],
        "expected": [[0, 1, 1], [2, 1, 1]],
    },
    # per-dimension min/max int8 map (ScalarQuantizationKernel.swift:513-518 asymmetric scale,
    # DataTransformations.metal:188-200 code rule) on a hand-checked 3 x 2 case, in fp32:
    # dim 0: min -1, max 1, scale = float32(2/255) (rounded up), -1/scale = -127.49999,
    #        zp = -128 - round(-127.49999) = -1 -> codes rint(-128.49999) = -128,
    #        rint(126.49999) = 126, rint(-1) = -1
    # dim 1: min 0, max 255, scale 1, zp = -128 -> codes -128, 127, -128 + 100
    "sq_per_dim": {
        "kind": "sq",
        "vectors": [[-1, 0], [1, 255], [0, 100]],
        "expected_zero_point": [-1, -128],
        "expected_codes": [[-128, -128], [126, 127], [-1, -28]],
    },
}


def main() -> None:
    for name, fx in FIXTURES.items():
        (HERE / f"{name}.json").write_text(json.dumps(fx, indent=1) + "\n")
    print(f"wrote {len(FIXTURES)} fixtures to {HERE}")


if __name__ == "__main__":
    main()

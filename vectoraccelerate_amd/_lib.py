"""ctypes binding of libva_hip.so (the C ABI declared in include/va_hip.h).

The library is built in-tree by ``vectoraccelerate_amd/build.py``.  Loading fails loudly
when it is missing: there is no CPU fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libva_hip.so"

VA_OK = 0
VA_ERR_INVALID_ARG = 1
VA_ERR_DIMENSION_MISMATCH = 2
VA_ERR_OOM = 3
VA_ERR_HIP = 4
VA_ERR_UNSUPPORTED = 5

VA_METRIC_L2SQ = 0
VA_METRIC_COSINE = 1
VA_METRIC_DOT = 2
VA_METRIC_L2 = 3

VA_SELECT_MIN = 0
VA_SELECT_MAX = 1

VA_OPT_CANDIDATE_CAP = 1
VA_OPT_SAMPLE_ROWS = 2
VA_OPT_SCREEN = 3
VA_OPT_SAMPLE_RANK = 4

VA_SENTINEL_INDEX = 0xFFFFFFFF
VA_MAX_K = 1024
VA_I8_MAX_DIM = 131071  # va_i8_scan_topk: the int32 dot of two code vectors stays exact
VA_NOALLOC_SCRATCH_BYTES = 64 << 20

VA_PROBE_FP32 = 0
VA_PROBE_FP16 = 1
VA_PROBE_INT8 = 2
VA_PROBE_FP4 = 3
VA_PROBE_LDS = 4
VA_PROBE_HBM = 5

_p = C.c_void_p
_u32 = C.c_uint32
_u64 = C.c_uint64
_i32 = C.c_int
_st = C.c_int

# name -> (restype, argtypes); must list every entry point of include/va_hip.h
SIGNATURES: dict[str, tuple] = {
    "va_abi_version": (C.c_int, []),
    "va_status_string": (C.c_char_p, [_st]),
    "va_context_create": (_st, [_i32, C.POINTER(_p)]),
    "va_context_create_with_stream": (_st, [_i32, _p, C.POINTER(_p)]),
    "va_context_destroy": (_st, [_p]),
    "va_context_stream": (_p, [_p]),
    "va_context_device": (C.c_int, [_p]),
    "va_context_synchronize": (_st, [_p]),
    "va_last_error_message": (C.c_char_p, [_p]),
    "va_context_set_option": (_st, [_p, _i32, _u64]),
    "va_context_set_profiling": (_st, [_p, _i32]),
    "va_context_last_scan": (_st, [_p, _p]),
    "va_context_scan_totals": (_st, [_p, _p, C.POINTER(C.c_uint32)]),
    "va_context_reset_scan_totals": (_st, [_p]),
    "va_buffer_alloc": (_st, [_p, C.c_size_t, C.POINTER(_p)]),
    "va_buffer_free": (_st, [_p, _p]),
    "va_buffer_upload": (_st, [_p, _p, _p, C.c_size_t]),
    "va_buffer_download": (_st, [_p, _p, _p, C.c_size_t]),
    "va_l2_pairs": (_st, [_p, _p, _p, _p, _u32, _u32, _i32]),
    "va_cosine_pairs": (_st, [_p, _p, _p, _p, _u32, _u32, _i32]),
    "va_l2_all_pairs": (_st, [_p, _p, _p, _p, _u32, _u32, _u32, _i32]),
    "va_cosine_all_pairs": (_st, [_p, _p, _p, _p, _u32, _u32, _u32, _i32]),
    "va_dot_all_pairs": (_st, [_p, _p, _p, _p, _u32, _u32, _u32, _i32]),
    "va_fused_topk": (_st, [_p, _i32, _p, _p, _u32, _u32, _u32, _u32, _p, _p]),
    "va_fused_topk_streamed": (_st, [_p, _i32, _p, _p, _u32, _u32, _u32, _u32, _u32, _p, _p]),
    "va_fused_topk_noalloc": (_st, [_p, _i32, _p, _p, _u32, _u32, _u32, _u32, _p, _p]),
    "va_topk_select": (_st, [_p, _p, _u32, _u32, _u32, _i32, _p, _p]),
    "va_topk_merge": (_st, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _p, _p]),
    "va_sq_params_per_dim": (_st, [_p, _p, _u32, _u32, _p, _p, _p, _p]),
    "va_sq_quantize_i8": (_st, [_p, _p, _u64, _u32, _p, _p, _p]),
    "va_sq_dequantize_i8": (_st, [_p, _p, _u64, _u32, _p, _p, _p]),
    "va_i8_scan_topk": (_st, [_p, _p, _p, _u32, _u32, _u32, _u32, _p, _p]),
    "va_bq_pack": (_st, [_p, _p, _u32, _u32, _p]),
    "va_hamming_matrix": (_st, [_p, _p, _p, _u32, _u32, _u32, _p]),
    "va_hamming_topk": (_st, [_p, _p, _p, _u32, _u32, _u32, _u32, _p, _p]),
    "va_ivf_build": (_st, [_p, _p, _u32, _p, _u32, _u32, C.POINTER(_p)]),
    "va_ivf_destroy": (_st, [_p]),
    "va_ivf_add": (_st, [_p, _p, _p, _u32, _u32, _u32]),
    "va_ivf_get_lists": (_st, [_p, _p, _p, _p]),
    "va_ivf_probe": (_st, [_p, _p, _p, _u32, _u32, _p]),
    "va_ivf_scan": (_st, [_p, _p, _p, _u32, _p, _u32, _u32, _p, _p]),
    "va_ivf_search": (_st, [_p, _p, _p, _u32, _u32, _u32, _p, _p]),
    "va_index_create": (_st, [_p, _u32, _u32, C.POINTER(_p)]),
    "va_index_create_ivf": (_st, [_p, _u32, _u32, _u32, _u32, _u32, C.POINTER(_p)]),
    "va_index_train": (_st, [_p, _p, _p, _u64]),
    "va_index_destroy": (_st, [_p]),
    "va_index_insert": (_st, [_p, _p, _p, _u32, _p]),
    "va_index_remove": (_st, [_p, _p, _p, _u32, C.POINTER(_u32)]),
    "va_index_compact": (_st, [_p, _p]),
    "va_index_get_info": (_st, [_p, _p]),
    "va_index_contains": (C.c_int, [_p, _u32]),
    "va_index_get_vector": (_st, [_p, _p, _u32, _p]),
    "va_index_search": (_st, [_p, _p, _i32, _p, _u32, _u32, _p, _p]),
    "va_index_search_filtered": (_st, [_p, _p, _i32, _p, _u32, _p, _p, _p, _p, C.POINTER(_u32), C.POINTER(_u32)]),
    "va_kmeans_fit": (_st, [_p, _p, _u32, _u32, _u32, _p, _u32, C.c_float, _p, _p, _p, _p, _p]),
    "va_kmeans_plusplus": (_st, [_p, _p, _u32, _u32, _u32, _u64, _p, _p]),
    "va_pq_train": (_st, [_p, _p, _u32, _u32, _u32, _u32, _u32, C.c_float, _u64, _p, _p, C.POINTER(_u32)]),
    "va_pq_encode": (_st, [_p, _p, _u32, _u32, _u32, _u32, _p, _p]),
    "va_pq_distance_tables": (_st, [_p, _p, _u32, _u32, _u32, _u32, _p, _p]),
    "va_pq_adc_distances": (_st, [_p, _p, _u32, _p, _u32, _u32, _u32, _p]),
    "va_pq_search": (_st, [_p, _p, _u32, _u32, _u32, _u32, _p, _p, _u32, _u32, _p, _p]),
    "va_probe_mfma": (_st, [_p, _i32, _i32, _u32, _p]),
}



class ScanTimings(C.Structure):
    """va_scan_timings (include/va_hip.h)."""

    _fields_ = [
        ("sample_ms", C.c_float),
        ("scan_ms", C.c_float),
        ("select_ms", C.c_float),
        ("fallback_ms", C.c_float),
        ("total_ms", C.c_float),
        ("sample_rows", C.c_uint32),
        ("candidate_cap", C.c_uint32),
        ("overflow_rows", C.c_uint32),
        ("scan_launches", C.c_uint32),
        ("screened", C.c_uint32),
        ("rerank_rows", C.c_uint32),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class IndexInfo(C.Structure):
    """va_index_info (include/va_hip.h)."""

    _fields_ = [
        ("count", C.c_uint32),
        ("deleted", C.c_uint32),
        ("slots", C.c_uint32),
        ("dimension", C.c_uint32),
        ("capacity", C.c_uint64),
        ("rows", C.c_void_p),
        ("next_handle", C.c_uint32),
        ("nlist", C.c_uint32),
        ("nprobe", C.c_uint32),
        ("routing_threshold", C.c_uint32),
        ("trained", C.c_uint32),
        ("ivf_routed", C.c_uint32),
        ("centroids", C.c_void_p),
        ("lists", C.c_void_p),
    ]


class ProbeResult(C.Structure):
    """va_probe_result (include/va_hip.h)."""

    _fields_ = [
        ("ops_per_second", C.c_double),
        ("engine_mhz", C.c_double),
        ("ms", C.c_double),
        ("ops", C.c_double),
    ]


# int (*va_index_filter)(uint32_t handle, void* user)
INDEX_FILTER = C.CFUNCTYPE(C.c_int, C.c_uint32, C.c_void_p)


class KMeansInfo(C.Structure):
    """va_kmeans_info (include/va_hip.h)."""

    _fields_ = [
        ("iterations", C.c_uint32),
        ("converged", C.c_int32),
        ("inertia", C.c_double),
        ("max_movement", C.c_float),
    ]


_LIB: C.CDLL | None = None


class LibraryMissing(RuntimeError):
    """libva_hip.so is not built: run ``python -c 'import __graft_entry__ as g; g.build()'``."""


def load(path: Path | None = None) -> C.CDLL:
    """Load (once) and type libva_hip.so.  Raises when the library is absent."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise LibraryMissing(f"{p} not found; build it with vectoraccelerate_amd/build.py")
    # PyTorch-ROCm wheels ship their own libamdhip64.so.  Loading torch first makes this
    # library bind to that same HIP runtime; loading ours first would put a second runtime
    # in the process and torch's device initialisation would then fail.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:  # a missing export raises AttributeError at its first use
            continue
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib

"""numpy wrapper of the CPU oracle (oracle/libva_oracle.so) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.
The product path (vectoraccelerate_amd / libva_hip.so) never does.  Each function restates
the reference semantics cited in oracle/va_oracle.h.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# VA_ORACLE_LIB: another build of the same source (the sanitizer build of run_sanitized.sh)
LIB = Path(os.environ.get("VA_ORACLE_LIB", HERE / "libva_oracle.so"))

L2SQ, COSINE, DOT, L2 = 0, 1, 2, 3
SENTINEL = 0xFFFFFFFF

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = C.CDLL(str(LIB))
        _lib.vo_distance.restype = C.c_double
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


_i = C.c_int64


def num_threads() -> int:
    return int(lib().vo_num_threads())


def l2_pairs(q, t, compute_sqrt=False):
    q, t = _f32(q), _f32(t)
    out = np.empty(q.shape[0], np.float32)
    lib().vo_l2_pairs(_p(q), _p(t), _i(q.shape[0]), _i(q.shape[1]), C.c_int(int(compute_sqrt)), _p(out))
    return out


def cosine_pairs(q, t, output_distance=False):
    q, t = _f32(q), _f32(t)
    out = np.empty(q.shape[0], np.float32)
    lib().vo_cosine_pairs(_p(q), _p(t), _i(q.shape[0]), _i(q.shape[1]), C.c_int(int(output_distance)), _p(out))
    return out


MATRIX_KIND = {"l2sq": 0, "l2": 1, "cos_sim": 2, "cos_dist": 3, "dot": 4, "abs_dot": 5}


def distance_matrix(kind: str, q, x):
    q, x = _f32(q), _f32(x)
    out = np.empty((q.shape[0], x.shape[0]), np.float32)
    lib().vo_distance_matrix(C.c_int(MATRIX_KIND[kind]), _p(q), _p(x), _i(q.shape[0]), _i(x.shape[0]),
                             _i(q.shape[1]), _p(out))
    return out


def distance(metric: int, q, x) -> float:
    q, x = _f32(q), _f32(x)
    return float(lib().vo_distance(C.c_int(metric), _p(q), _p(x), _i(q.shape[0])))


def topk_rows(values, k, mode_max=False):
    v = _f32(values)
    Q, N = v.shape
    idx = np.empty((Q, k), np.uint32)
    val = np.empty((Q, k), np.float32)
    lib().vo_topk_rows(_p(v), _i(Q), _i(N), _i(k), C.c_int(int(mode_max)), _p(idx), _p(val))
    return idx, val


def flat_topk(metric: int, q, x, k, accum_double=True):
    q, x = _f32(q), _f32(x)
    Q, D = q.shape
    idx = np.empty((Q, k), np.uint32)
    dist = np.empty((Q, k), np.float32)
    lib().vo_flat_topk(C.c_int(metric), _p(q), _p(x), _i(Q), _i(x.shape[0]), _i(D), _i(k),
                       C.c_int(int(accum_double)), _p(idx), _p(dist))
    return idx, dist


def topk_merge(a_idx, a_d, b_idx, b_d, chunk_base):
    a_idx = np.ascontiguousarray(a_idx, np.uint32)
    b_idx = np.ascontiguousarray(b_idx, np.uint32)
    a_d, b_d = _f32(a_d), _f32(b_d)
    Q, k = a_idx.shape
    oi = np.empty((Q, k), np.uint32)
    od = np.empty((Q, k), np.float32)
    lib().vo_topk_merge(_p(a_idx), _p(a_d), _p(b_idx), _p(b_d), _i(Q), _i(k), C.c_uint32(chunk_base), _p(oi), _p(od))
    return oi, od


def sq_params_per_dim(x):
    x = _f32(x)
    N, D = x.shape
    mn = np.empty(D, np.float32)
    mx = np.empty(D, np.float32)
    sc = np.empty(D, np.float32)
    zp = np.empty(D, np.int32)
    lib().vo_sq_params_per_dim(_p(x), _i(N), _i(D), _p(mn), _p(mx), _p(sc), _p(zp))
    return mn, mx, sc, zp


def sq_global_params(x, asymmetric: bool):
    """(scale, zero point) of the global int8 quantization (zero point 0 when symmetric)."""
    x = _f32(np.asarray(x, np.float32).reshape(-1))
    scale = np.empty(1, np.float32)
    zp = np.empty(1, np.int32)
    lib().vo_sq_global_params(_p(x), _i(x.size), C.c_int(int(asymmetric)), _p(scale), _p(zp))
    return np.float32(scale[0]), int(zp[0])


def sq_global_quantize(x, asymmetric: bool):
    """Global int8 codes of a flat array: (codes, scale, zero point)."""
    scale, zp = sq_global_params(x, asymmetric)
    flat = np.asarray(x, np.float32).reshape(-1, 1)
    return sq_quantize(flat, [scale], [zp]).reshape(-1), scale, zp


def sq_quantize(x, scale, zp):
    x = _f32(x)
    N, D = x.shape
    scale = _f32(scale)
    zp = np.ascontiguousarray(zp, np.int32)
    out = np.empty((N, D), np.int8)
    lib().vo_sq_quantize(_p(x), _i(N), _i(D), _p(scale), _p(zp), _p(out))
    return out


def sq_dequantize(codes, scale, zp):
    codes = np.ascontiguousarray(codes, np.int8)
    N, D = codes.shape
    out = np.empty((N, D), np.float32)
    lib().vo_sq_dequantize(_p(codes), _i(N), _i(D), _p(_f32(scale)), _p(np.ascontiguousarray(zp, np.int32)), _p(out))
    return out


def i8_topk(qc, xc, k):
    qc = np.ascontiguousarray(qc, np.int8)
    xc = np.ascontiguousarray(xc, np.int8)
    Q, D = qc.shape
    idx = np.empty((Q, k), np.uint32)
    dist = np.empty((Q, k), np.int32)
    lib().vo_i8_topk(_p(qc), _p(xc), _i(Q), _i(xc.shape[0]), _i(D), _i(k), _p(idx), _p(dist))
    return idx, dist


def i8_dot_matrix(qc, xc):
    qc = np.ascontiguousarray(qc, np.int8)
    xc = np.ascontiguousarray(xc, np.int8)
    out = np.empty((qc.shape[0], xc.shape[0]), np.int32)
    lib().vo_i8_dot_matrix(_p(qc), _p(xc), _i(qc.shape[0]), _i(xc.shape[0]), _i(qc.shape[1]), _p(out))
    return out


def bq_pack(x):
    x = _f32(x)
    N, D = x.shape
    W = (D + 31) // 32
    out = np.empty((N, W), np.uint32)
    lib().vo_bq_pack(_p(x), _i(N), _i(D), _p(out))
    return out


def hamming_matrix(q, x):
    q = np.ascontiguousarray(q, np.uint32)
    x = np.ascontiguousarray(x, np.uint32)
    out = np.empty((q.shape[0], x.shape[0]), np.uint32)
    lib().vo_hamming_matrix(_p(q), _p(x), _i(q.shape[0]), _i(x.shape[0]), _i(q.shape[1]), _p(out))
    return out


def hamming_topk(q, x, k):
    q = np.ascontiguousarray(q, np.uint32)
    x = np.ascontiguousarray(x, np.uint32)
    Q, W = q.shape
    idx = np.empty((Q, k), np.uint32)
    dist = np.empty((Q, k), np.uint32)
    lib().vo_hamming_topk(_p(q), _p(x), _i(Q), _i(x.shape[0]), _i(W), _i(k), _p(idx), _p(dist))
    return idx, dist


def ivf_assign(x, c):
    x, c = _f32(x), _f32(c)
    out = np.empty(x.shape[0], np.int32)
    lib().vo_ivf_assign(_p(x), _i(x.shape[0]), _p(c), _i(c.shape[0]), _i(x.shape[1]), _p(out))
    return out


def ivf_csr(lists, C_):
    lists = np.ascontiguousarray(lists, np.int32)
    off = np.empty(C_ + 1, np.uint32)
    ids = np.empty(lists.shape[0], np.uint32)
    lib().vo_ivf_csr(_p(lists), _i(lists.shape[0]), _i(C_), _p(off), _p(ids))
    return off, ids


def ivf_probe(q, c, nprobe):
    q, c = _f32(q), _f32(c)
    out = np.empty((q.shape[0], nprobe), np.uint32)
    lib().vo_ivf_probe(_p(q), _i(q.shape[0]), _p(c), _i(c.shape[0]), _i(q.shape[1]), _i(nprobe), _p(out))
    return out


def ivf_scan(q, x, offsets, ids, probes, k):
    q, x = _f32(q), _f32(x)
    offsets = np.ascontiguousarray(offsets, np.uint32)
    ids = np.ascontiguousarray(ids, np.uint32)
    probes = np.ascontiguousarray(probes, np.uint32)
    Q, D = q.shape
    idx = np.empty((Q, k), np.uint32)
    dist = np.empty((Q, k), np.float32)
    lib().vo_ivf_scan(_p(q), _i(Q), _p(x), _i(D), _p(offsets), _p(ids), _i(offsets.shape[0] - 1), _p(probes),
                      _i(probes.shape[1]), _i(k), _p(idx), _p(dist))
    return idx, dist


def kmeans_fit(x, init, max_iter, threshold):
    """Lloyd k-means: (centroids, assignments, distances, counts, iterations, converged, inertia,
    max_movement)."""
    x, init = _f32(x), _f32(init)
    N, D = x.shape
    C_ = init.shape[0]
    cen = np.empty((C_, D), np.float32)
    assign = np.empty(N, np.uint32)
    dist = np.empty(N, np.float32)
    counts = np.empty(C_, np.uint32)
    iu = np.empty(2, np.uint32)
    fi = np.empty(2, np.float32)
    lib().vo_kmeans_fit(_p(x), _i(N), _i(D), _i(C_), _p(init), _i(max_iter), C.c_float(threshold), _p(cen),
                        _p(assign), _p(dist), _p(counts), _p(iu), _p(fi))
    return cen, assign, dist, counts, int(iu[0]), bool(iu[1]), float(fi[0]), float(fi[1])


def kmeans_update(x, assign, dist, old):
    """One k-means update given an assignment: (centroids, counts)."""
    x, old, dist = _f32(x), _f32(old), _f32(dist)
    assign = np.ascontiguousarray(assign, np.uint32)
    N, D = x.shape
    C_ = old.shape[0]
    cen = np.empty((C_, D), np.float32)
    counts = np.empty(C_, np.uint32)
    lib().vo_kmeans_update(_p(x), _i(N), _i(D), _i(C_), _p(assign), _p(dist), _p(old), _p(cen), _p(counts))
    return cen, counts


def kmeans_plusplus(x, k, seed):
    """Row ids chosen by k-means++ D^2 sampling with splitmix64(seed) draws."""
    x = _f32(x)
    idx = np.empty(k, np.uint32)
    lib().vo_kmeans_plusplus(_p(x), _i(x.shape[0]), _i(x.shape[1]), _i(k), C.c_uint64(seed), _p(idx))
    return idx


def pq_sub_l2sq(v, c):
    v, c = _f32(v), _f32(c)
    lib().vo_pq_sub_l2sq.restype = C.c_float
    return float(lib().vo_pq_sub_l2sq(_p(v), _p(c), _i(v.shape[0])))


def pq_encode(x, cb, M, K):
    x, cb = _f32(x), _f32(cb)
    codes = np.empty((x.shape[0], M), np.uint8)
    lib().vo_pq_encode(_p(x), _i(x.shape[0]), _i(x.shape[1]), _i(M), _i(K), _p(cb), _p(codes))
    return codes


def pq_tables(q, cb, M, K):
    q, cb = _f32(q), _f32(cb)
    t = np.empty((q.shape[0], M, K), np.float32)
    lib().vo_pq_tables(_p(q), _i(q.shape[0]), _i(q.shape[1]), _i(M), _i(K), _p(cb), _p(t))
    return t


def pq_adc(tables, codes):
    tables = _f32(tables)
    codes = np.ascontiguousarray(codes, np.uint8)
    Q, M, K = tables.shape
    out = np.empty((Q, codes.shape[0]), np.float32)
    lib().vo_pq_adc(_p(tables), _i(Q), _p(codes), _i(codes.shape[0]), _i(M), _i(K), _p(out))
    return out


def pq_search(q, cb, codes, M, K, k):
    q, cb = _f32(q), _f32(cb)
    codes = np.ascontiguousarray(codes, np.uint8)
    idx = np.empty((q.shape[0], k), np.uint32)
    dist = np.empty((q.shape[0], k), np.float32)
    lib().vo_pq_search(_p(q), _i(q.shape[0]), _i(q.shape[1]), _i(M), _i(K), _p(cb), _p(codes), _i(codes.shape[0]),
                       _i(k), _p(idx), _p(dist))
    return idx, dist


def pq_train(x, cb_init, M, K, iterations, threshold):
    """(codebooks [M x K x D/M], rounds run)."""
    x = _f32(x)
    cb = np.array(cb_init, np.float32, copy=True, order="C")
    lib().vo_pq_train.restype = C.c_int64
    it = lib().vo_pq_train(_p(x), _i(x.shape[0]), _i(x.shape[1]), _i(M), _i(K), _i(iterations),
                           C.c_float(threshold), _p(cb))
    return cb, int(it)

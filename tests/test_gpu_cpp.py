"""The C++ host mirror (include/vectoraccelerate.hpp) end to end: tests/cpp/va_example runs the
flat top-k (L2^2, cosine), IVF build + add + search, k-means, PQ, the provider and the flat and IVF
AcceleratedVectorIndex through the C++ classes; its outputs are compared with the CPU oracle."""
from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
EXE = ROOT / "tests" / "cpp" / "va_example"


def test_cpp_header_compiles():
    """CPU check: the header builds stand-alone with warnings on."""
    proc = subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-fsyntax-only", f"-I{ROOT / 'include'}",
                           "-x", "c++", str(ROOT / "include" / "vectoraccelerate.hpp")], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr


@pytest.mark.gpu
def test_cpp_mirror_matches_oracle(tmp_path, oracle):
    from tests.helpers import L2SQ, check_topk
    from tests.test_gpu_ivf import clustered

    if not EXE.exists():
        from vectoraccelerate_amd.build import build_cpp_example

        build_cpp_example()
    Q, N, D, C, k, nprobe = 24, 6000, 32, 16, 10, 4
    c, x, q = clustered(C, D, N, Q, seed=77)
    for name, arr in (("q", q), ("x", x), ("c", c)):
        arr.astype(np.float32).tofile(tmp_path / f"{name}.bin")
    print(f"cpp example Q={Q} N={N} D={D} C={C}", flush=True)
    proc = subprocess.run([str(EXE), str(tmp_path), str(Q), str(N), str(D), str(C), str(k), str(nprobe)],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr
    rd = lambda n, t: np.fromfile(tmp_path / f"{n}.bin", dtype=t)  # noqa: E731
    oi, od = oracle.flat_topk(L2SQ, q, x, k)
    check_topk(L2SQ, q, x, k, rd("l2_idx", np.uint32).reshape(Q, k), rd("l2_dist", np.float32).reshape(Q, k), oi, od)
    oi, od = oracle.flat_topk(oracle.COSINE, q, x, k)
    check_topk(oracle.COSINE, q, x, k, rd("cos_idx", np.uint32).reshape(Q, k), None, oi, od)
    off, ids = oracle.ivf_csr(oracle.ivf_assign(x, c), C)
    probes = oracle.ivf_probe(q, c, nprobe)
    ii, _ = oracle.ivf_scan(q, x, off, ids, probes, k)
    np.testing.assert_array_equal(rd("ivf_idx", np.uint32).reshape(Q, k), ii)
    kc, ka, *_ = oracle.kmeans_fit(x, c, 5, 0.0)
    np.testing.assert_array_equal(rd("km_assign", np.uint32), ka)
    np.testing.assert_array_equal(rd("km_cen", np.float32).reshape(C, D), kc)
    cb = rd("pq_cb", np.float32).reshape(4, 16, D // 4)
    codes = rd("pq_codes", np.uint8).reshape(N, 4)
    np.testing.assert_array_equal(codes, oracle.pq_encode(x, cb, 4, 16))
    pi, _ = oracle.pq_search(q, cb, codes, 4, 16, k)
    np.testing.assert_array_equal(rd("pq_idx", np.uint32).reshape(Q, k), pi)
    assert (tmp_path / "error_kind.txt").read_text() == "invalidInput"
    # MetalComputeProvider: sqrt L2, 1 - cosine similarity, raw dot; nearest first
    np.testing.assert_allclose(rd("prov_l2", np.float32), np.sqrt(((x - q[0]) ** 2).sum(1)), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(rd("prov_cos", np.float32), oracle.distance_matrix("cos_dist", q[:1], x)[0], atol=1e-4)
    np.testing.assert_allclose(rd("prov_dot", np.float32), x.astype(np.float64) @ q[0].astype(np.float64), rtol=1e-4,
                               atol=1e-3)
    nn = rd("prov_nn_idx", np.uint32).reshape(3, Q, k)
    nd = rd("prov_nn_dist", np.float32).reshape(3, Q, k)
    oi, od = oracle.flat_topk(oracle.L2, q, x, k)
    check_topk(oracle.L2, q, x, k, nn[0], nd[0], oi, od)
    oi, od = oracle.flat_topk(oracle.COSINE, q, x, k)
    check_topk(oracle.COSINE, q, x, k, nn[1], nd[1], oi, od)
    oi, od = oracle.flat_topk(oracle.DOT, q, x, k)
    check_topk(oracle.DOT, q, x, k, nn[2], -nd[2], oi, od)  # raw dot reported, largest first
    # AcceleratedVectorIndex: the live vectors (every 7th removed) in handle space
    live = np.array([i for i in range(N) if i % 7], np.int64)
    gi = rd("index_idx", np.uint32).reshape(Q, k).astype(np.int64)
    assert np.isin(gi, live).all()
    oi, od = oracle.flat_topk(L2SQ, q, x[live], k)
    check_topk(L2SQ, q, x[live], k, np.searchsorted(live, gi).astype(np.uint32), None, oi, od)
    odd_live = np.array([i for i in live if i % 2 == 1], np.int64)
    gf = rd("index_filtered_idx", np.uint32).astype(np.int64)
    assert gf.shape == (k,) and np.isin(gf, odd_live).all()
    oi, od = oracle.flat_topk(L2SQ, q[:1], x[odd_live], k)
    check_topk(L2SQ, q[:1], x[odd_live], k, np.searchsorted(odd_live, gf)[None].astype(np.uint32), None, oi, od)
    removed, count, c0, c1 = (tmp_path / "index_counts.txt").read_text().split()
    assert (int(removed), int(count), c0, c1) == (len(range(0, N, 7)), len(live), "0", "1")
    # AcceleratedVectorIndex (IVF): lists = the oracle's assignment + CSR of every row; results =
    # the oracle's scan of the oracle's probes over the live rows (every 5th removed)
    assert (tmp_path / "ivx_state.txt").read_text().split() == ["1", "1", str(N - len(range(0, N, 5)))]
    np.testing.assert_array_equal(rd("ivx_off", np.uint32), off)
    np.testing.assert_array_equal(rd("ivx_ids", np.uint32), ids)
    keep = ids % 5 != 0
    lens = np.bincount(np.repeat(np.arange(C), np.diff(off.astype(np.int64)))[keep], minlength=C)
    loff = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    vi, vd = oracle.ivf_scan(q, x, loff, ids[keep], probes, k)
    check_topk(L2SQ, q, x, k, rd("ivx_idx", np.uint32).reshape(Q, k), rd("ivx_dist", np.float32).reshape(Q, k), vi,
               vd)

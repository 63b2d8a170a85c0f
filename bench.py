"""Benchmark of the flat/IVF search hot path on one MI355X.

Headline (the JSON line's ``value``) = BASELINE.json configs[1]: flat cosine top-100 over
N=1,000,000 x d=1536 fp32 (rows N(0,1) then L2-normalised), Q=1024 queries = database rows +
N(0, 0.05) noise, renormalised.  A "step" is one AcceleratedVectorIndex.search
(va_index_search) over the resident index, whose fp32 rows and fp16 shadow are built at insert
outside the timed region (threshold sample -> fp16 MFMA screening scan -> exact fp32 rerank of
the band the screen's error bound leaves open -> selection; no step waits on the host).  The
same search on the fp32 scan alone is timed beside it and must return the same ids and
distances bit for bit (``fp32_scan_only``, ``screened_equals_fp32_scan``).  The other configs
are measured the same way at full size and reported under ``extra`` (configs[2] int8 top-10,
configs[3] binary top-100, configs[4] IVF-Flat top-10, PQ ADC, IVF training; configs[0] is the
CPU-runnable parity case covered by the tests).

CPU baseline: the C oracle's float-accumulation port of the reference CPU path
(CPUTopK / AccelerateFallback), timed on this host's cores on a bounded query sample.
Prints ONE JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"]
PEAK = {
    "fp32_mfma_tflops": 157.3,
    "int8_mfma_tops": 5000.0,
    # 32-bit integer VALU, 256 CU x 64 lanes/clk x 2.4 GHz (no packed xor/popcount exists).
    # The Hamming scan issues 2 of these per word and measures ~6% above this figure, as does a
    # standalone xor + popcount instruction stream, so it is a floor of the real issue rate.
    "valu_int32_tops": 39.3,
    # dense fp4 (e2m1) MFMA, MI355X published figure (fp6 the same)
    "fp4_mfma_tflops": 10100.0,
    # dense fp16 MFMA, MI355X published figure
    "fp16_mfma_tflops": 2500.0,
    "hbm_gbs": 8000.0,
    # host link of the MI355X board (PCIe 5.0 x16, one direction)
    "pcie5_x16_gbs": 64.0,
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--workload", default="all",
                   choices=["all", "c2", "c3", "c4", "c5", "kmeans", "pq", "ceiling", "small"],
                   help="all = configs[1] headline + configs[2..4] extras")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines (profiling runs)")
    p.add_argument("--no-extra", action="store_true", help="headline only (no L2 top-10 extra)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="first run a plain 1 GiB device copy (reference point for rocprofv3 FETCH/WRITE_SIZE)")
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


COUNTERS_SCREEN16 = "profiles/counters__screen16_filter__configs1_cosine_top100.txt"
COUNTERS_SCREEN = "profiles/counters__screen_filter__configs1_cosine_top100.txt"
COUNTERS_FP32 = "profiles/counters__dist_gemm_filter__configs1_cosine_top100.txt"
COUNTERS_I8 = "profiles/counters__i8_resq16_filter__configs2_int8_top10.txt"
COUNTERS_HAMMING = "profiles/counters__hamming_mfma_filter__configs3_binary_top100.txt"
COUNTERS_IVF16 = {"192 queries x 256 rows, LDS-staged (full pass, lists probed by more than 96 queries)":
                  "profiles/counters__ivf16_big__configs4_ivfflat_top10.txt",
                  "96 resident queries x 1024 rows (full pass, 33-96 queries)": "profiles/counters__ivf16_resq__configs4_ivfflat_top10.txt",
                  "64-query tiles (sample pass)": "profiles/counters__ivf16_wide64__configs4_ivfflat_top10.txt",
                  "32-query tiles": "profiles/counters__ivf16_wide32__configs4_ivfflat_top10.txt",
                  "16-query tiles": "profiles/counters__ivf16_narrow__configs4_ivfflat_top10.txt"}
COUNTERS_IVF = {"2x2 tiles": "profiles/counters__ivf_list_scan_2x2__configs4_ivfflat_top10.txt",
                "4x1 tiles": "profiles/counters__ivf_list_scan_4x1__configs4_ivfflat_top10.txt",
                "16-query tiles": "profiles/counters__ivf_small_tiles__configs4_ivfflat_top10.txt"}
COUNTERS_PQ = "profiles/counters__pq_adc_filter__10Mx16codes_K256_Q1024.txt"
COUNTERS_SMALL = "profiles/counters__screen16_small_filter__1Mx768_l2_top10.txt"
CEILING_PROFILE = "profiles/mfma_ceiling__probe_fp32_fp16_int8_fp4.txt"


def counters(rel: str) -> dict:
    """Per-launch figures of a committed rocprofv3 counter summary (mfma_busy_pct, hbm_gbs,
    traffic_bytes_per_launch, ...); empty when the file is absent."""
    f = ROOT / rel
    out = {}
    if not f.exists():
        return out
    for line in f.read_text().splitlines():
        if ":" in line and not line.startswith(("#", "rocprofv3")):
            key, val = line.split(":", 1)
            try:
                out[key.strip()] = float(val.split()[0])
            except (ValueError, IndexError):
                pass
    return out


def counted(rel: str) -> dict:
    """The counted MFMA-busy and HBM figures of a committed counter summary, for a roofline."""
    c = counters(rel)
    return {"mfma_busy": c.get("mfma_busy_pct"), "hbm_gbs": c.get("hbm_gbs"),
            "traffic": c.get("traffic_bytes_per_launch"), "counters_source": rel}


def timed(ctx, fn, steps: int, warmup: int, scan_timings: bool = True, phase_reps: int = 3):
    """Run `warmup` untimed steps, then time exactly `steps` steps between synchronisations.
    With scan_timings, the timed loop runs at profiling level 2 (the library records two hipEvents
    around each scan phase on its stream, which nothing waits for inside the loop: the scan
    kernel's mean duration over exactly the timed steps), and `phase_reps` more steps after it at
    level 1 give the breakdown of the other phases and the counts (outside the timed loop).
    Without, the timed loop runs with profiling off (level 1 is restored after it)."""
    import torch

    for _ in range(warmup):
        fn()
    ctx.synchronize()
    torch.cuda.synchronize()
    if scan_timings:
        ctx.set_profiling(2)
        ctx.reset_scan_totals()
    else:
        ctx.set_profiling(0)
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    ctx.synchronize()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    if not scan_timings:
        ctx.set_profiling(True)
        return ms, None
    total, n = ctx.scan_totals()
    ctx.set_profiling(True)
    ctx.reset_scan_totals()
    for _ in range(phase_reps):
        fn()
    ctx.synchronize()
    ftotal, fn_ = ctx.scan_totals()
    return ms, (total, n, ctx.last_scan_timings(), ftotal, fn_)


def mean_phases(phases):
    """Mean phase times per scan: the scan phase over the timed loop, the other phases over the
    level-1 steps after it (from timed()), with the last scan's sizes."""
    if not phases:
        return {}
    total, n, last, ftotal, fn_ = phases
    fn_ = max(fn_, 1)
    out = {k: float(ftotal[k]) / fn_ for k in ("sample_ms", "select_ms", "fallback_ms", "total_ms")}
    out["scan_ms_phase_steps"] = float(ftotal["scan_ms"]) / fn_
    # (a scan with no sample phase records nothing at level 2: its time comes from the level-1 steps)
    out["scan_ms"] = float(total["scan_ms"]) / n if n else out["scan_ms_phase_steps"]
    out["scans"] = n
    out.update({k: last[k] for k in ("sample_rows", "candidate_cap", "overflow_rows", "screened", "rerank_rows")
                if k in last})
    return out


PROBES = (("fp32", 0, "fp32_mfma_tflops", 1500), ("fp16", 1, "fp16_mfma_tflops", 3000),
          ("int8", 2, "int8_mfma_tops", 3000), ("fp4", 3, "fp4_mfma_tflops", 3000))


def run_ceiling(ctx):
    """The board's sustained MFMA rate per instruction the scans use (va_probe_mfma: register-only
    loops on every SIMD, random and constant operands) with the engine clock, beside the datasheet
    peak.  Outside every timed region."""
    import ctypes as C

    from vectoraccelerate_amd import _lib

    out = {}
    # the LDS read bandwidth the screens' fragment reads draw on (bytes per clock per CU)
    r = _lib.ProbeResult()
    ctx.check(ctx.lib.va_probe_mfma(ctx.handle, _lib.VA_PROBE_LDS, 1, 20000, C.byref(r)), "va_probe_mfma")
    import torch

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    bpc = r.ops_per_second / (cus * r.engine_mhz * 1e6) if r.engine_mhz else None
    out["lds_read"] = {"tb_per_s": r.ops_per_second / 1e12, "engine_mhz": r.engine_mhz, "bytes_per_clk_per_cu": bpc,
                       "cus": cus, "ms": r.ms}
    log(f"LDS read (ds_read_b128, 8 waves per CU): {r.ops_per_second / 1e12:.1f} TB/s = "
        f"{bpc:.0f} B/clk per CU at {r.engine_mhz:.0f} MHz")
    # the HBM read bandwidth the HBM-bound scans draw on: a 4 GiB streaming read
    r = _lib.ProbeResult()
    ctx.check(ctx.lib.va_probe_mfma(ctx.handle, _lib.VA_PROBE_HBM, 1, 4096, C.byref(r)), "va_probe_mfma")
    out["hbm_read"] = {"gb_per_s": r.ops_per_second / 1e9, "frac_of_datasheet": r.ops_per_second / 1e9 / PEAK["hbm_gbs"],
                       "bytes": r.ops, "ms": r.ms, "engine_mhz": r.engine_mhz}
    log(f"HBM read (16-byte loads, 4 GiB): {r.ops_per_second / 1e9:.0f} GB/s = "
        f"{100 * r.ops_per_second / 1e9 / PEAK['hbm_gbs']:.1f}% of {PEAK['hbm_gbs']:.0f}")
    for name, kind, peak_key, iters in PROBES:
        row = {"datasheet_peak": PEAK[peak_key], "unit": "TOP/s" if name == "int8" else "TFLOP/s"}
        for rnd, label in ((1, "random"), (0, "constant")):
            r = _lib.ProbeResult()
            ctx.check(ctx.lib.va_probe_mfma(ctx.handle, kind, rnd, iters, C.byref(r)), "va_probe_mfma")
            t = r.ops_per_second / 1e12
            row[label] = {"rate": t, "frac_of_datasheet": t / PEAK[peak_key], "engine_mhz": r.engine_mhz, "ms": r.ms}
        out[name] = row
        log(f"MFMA ceiling {name}: random {row['random']['rate']:.1f} ({100 * row['random']['frac_of_datasheet']:.1f}% "
            f"of {PEAK[peak_key]:.0f}) at {row['random']['engine_mhz']:.0f} MHz; constant {row['constant']['rate']:.1f} "
            f"({100 * row['constant']['frac_of_datasheet']:.1f}%) at {row['constant']['engine_mhz']:.0f} MHz")
    return out


def with_hbm_ceiling(obj, ceil: dict | None):
    """Every HBM-bound roofline dict inside obj gets the measured HBM read rate beside the datasheet
    peak (the probe's streaming read, in this run)."""
    if not ceil or "hbm_read" not in ceil:
        return
    if isinstance(obj, dict):
        if obj.get("bound") == "hbm" and obj.get("achieved"):
            m = ceil["hbm_read"]["gb_per_s"]
            obj["measured_ceiling"] = {"instruction": "16-byte streaming loads", "rate": m, "unit": "GB/s",
                                       "frac_of_measured": obj["achieved"] / m, "profile": CEILING_PROFILE}
        for v in obj.values():
            with_hbm_ceiling(v, ceil)
    elif isinstance(obj, list):
        for v in obj:
            with_hbm_ceiling(v, ceil)


def with_ceiling(roof: dict, ceil: dict | None, name: str) -> dict:
    """A roofline dict with the measured ceiling of its instruction beside the datasheet peak."""
    if not ceil or name not in ceil or not roof.get("achieved"):
        return roof
    m = ceil[name]["random"]["rate"]
    roof["measured_ceiling"] = {"instruction": name, "rate": m, "operands": "random",
                                "engine_mhz": ceil[name]["random"]["engine_mhz"],
                                "frac_of_measured": roof["achieved"] / m, "profile": CEILING_PROFILE}
    return roof


def run_small_batches(ctx, a, ix, qpool, metric: int, k: int, label: str):
    """Index searches with Q = 1, 10, 100 (the reference's published batch scaling,
    Guides/03-Accelerated-Search/01-Flat-Search-On-GPU.md:300-308) over a resident index: the
    small-batch screen over the fp16 shadow, checked bit for bit against the fp32-only scan."""
    import torch

    from vectoraccelerate_amd import _lib

    info = ix._info()
    N, D = info.slots, info.dimension
    shadow_bytes = float(N) * D * 2
    out = {}
    for Q in (1, 10, 100):
        q = qpool[:Q].contiguous()
        idx = ctx.empty((Q, k), torch.int32)
        dist = ctx.empty((Q, k), torch.float32)

        def step():
            ctx.check(ctx.lib.va_index_search(ctx.handle, ix._h, metric, q.data_ptr(), Q, k, idx.data_ptr(),
                                              dist.data_ptr()), "va_index_search")

        ms, ph = timed(ctx, step, max(20, a.steps), 3)
        phm = mean_phases(ph)
        i32 = ctx.empty((Q, k), torch.int32)
        d32 = ctx.empty((Q, k), torch.float32)
        ctx.set_option(_lib.VA_OPT_SCREEN, 1)
        try:
            def step32():
                ctx.check(ctx.lib.va_index_search(ctx.handle, ix._h, metric, q.data_ptr(), Q, k, i32.data_ptr(),
                                                  d32.data_ptr()), "va_index_search")

            ms32, ph32 = timed(ctx, step32, max(10, a.steps // 2), 2)
        finally:
            ctx.set_option(_lib.VA_OPT_SCREEN, 0)
        same = bool(torch.equal(idx, i32)) and bool(torch.equal(dist.view(torch.int32), d32.view(torch.int32)))
        if not same:
            raise SystemExit(f"{label} Q={Q}: the small-batch screen differs from the fp32 scan")
        scan_ms = phm.get("scan_ms") or ms
        gbs_scan = shadow_bytes / (scan_ms * 1e-3) / 1e9
        gbs_search = shadow_bytes / (ms * 1e-3) / 1e9
        out[f"Q{Q}"] = {
            "ms_per_search": ms, "qps": Q / (ms * 1e-3), "phases_ms": phm,
            "fp32_scan_only_ms": ms32, "equals_fp32_scan": same,
            "roofline": {"bound": "hbm", "achieved": gbs_scan, "peak": PEAK["hbm_gbs"], "unit": "GB/s",
                         "frac": gbs_scan / PEAK["hbm_gbs"], "kernel": "screen16_small_kernel (screen pass)",
                         "algorithmic": f"the fp16 shadow read once: N*D*2 = {shadow_bytes:.4g} B per search",
                         "whole_search_gbs": gbs_search, "whole_search_frac": gbs_search / PEAK["hbm_gbs"],
                         "whole_search_over_roofline": ms / (shadow_bytes / (PEAK["hbm_gbs"] * 1e9) * 1e3),
                         **(counted(COUNTERS_SMALL) if Q <= 32 else {})},
        }
        log(f"{label} Q={Q}: {ms:.3f} ms/search = {Q / (ms * 1e-3):.0f} QPS (fp32 scan only {ms32:.3f} ms); screen "
            f"pass {scan_ms:.3f} ms = {gbs_scan:.0f} GB/s ({100 * gbs_scan / PEAK['hbm_gbs']:.1f}% HBM); whole "
            f"search {ms / (shadow_bytes / 8e12 * 1e3):.2f}x the shadow's HBM time; identical: {same}")
        del idx, dist, i32, d32
    return out


def run_c2(ctx, a, cpu: bool, extra_l2: bool):
    import numpy as np
    import torch

    from vectoraccelerate_amd import (AcceleratedVectorIndex, FusedL2TopKKernel, FusedL2TopKParameters,
                                      IndexConfiguration, Metric, _lib)

    N, D, Q, k = 1_000_000, 1536, 1024, 100
    log(f"configs[1]: generating N={N} D={D} Q={Q}")
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(N, D, device="cuda", generator=g, dtype=torch.float32)
    x /= x.norm(dim=1, keepdim=True)
    gq = torch.Generator(device="cuda").manual_seed(1)
    src = torch.randint(0, N, (Q,), device="cuda", generator=gq)
    q = x[src] + 0.05 * torch.randn(Q, D, device="cuda", generator=gq, dtype=torch.float32)
    q /= q.norm(dim=1, keepdim=True)
    q = q.contiguous()
    torch.cuda.synchronize()
    # the index (AcceleratedVectorIndex over va_index_*): rows and their fp16 shadow are built at
    # insert time, outside the timed region
    t0 = time.perf_counter()
    ix = AcceleratedVectorIndex(IndexConfiguration.flat(D, N, metric="cosine"), ctx)
    ix.insert(vectors=x)
    ctx.synchronize()
    insert_s = time.perf_counter() - t0
    rows = ix._rows()
    del x
    torch.cuda.empty_cache()
    idx = ctx.empty((Q, k), torch.int32)
    dist = ctx.empty((Q, k), torch.float32)
    ms, phases = timed(ctx, lambda: ix.searchDevice(q, k, idx, dist), a.steps, a.warmup)
    ph = mean_phases(phases)
    flops = 2.0 * Q * N * D
    tflops = flops / (ph["scan_ms"] * 1e-3) / 1e12
    screened = bool(ph.get("screened", 0))
    peak = PEAK["fp16_mfma_tflops"] if screened else PEAK["fp32_mfma_tflops"]
    cnt = counters(COUNTERS_SCREEN16 if screened else COUNTERS_FP32)
    res = {
        "ms_per_step": ms,
        "qps": Q / (ms * 1e-3),
        "phases_ms": ph,
        "scan_tflops": tflops,
        "index_insert_s": insert_s,
        "rank1_is_source_row": float((idx[:, 0].long() == src).float().mean().item()),
        "roofline": {
            "bound": "mfma", "achieved": tflops, "peak": peak, "unit": "TFLOP/s",
            "frac": tflops / peak,
            "traffic": cnt.get("traffic_bytes_per_launch"),
            "mfma_busy": cnt.get("mfma_busy_pct"),
            "hbm_gbs": cnt.get("hbm_gbs"),
            "counters_source": COUNTERS_SCREEN16 if screened else COUNTERS_FP32,
            "kernel": ("screen16_kernel (fp16 MFMA screening scan over the index's fp16 shadow; exact fp32 "
                       "rerank of a proven band)" if screened else "dist_gemm_kernel<4, 1, true, 2, true, false> (fp32 scan)"),
            "algorithmic": f"2*Q*N*D = {flops:.4g} FLOP per launch",
            "fp32_mfma_equivalent_frac": tflops / PEAK["fp32_mfma_tflops"],
            "power_limited_ceiling": ("a register-only loop of the same fp16 MFMA on random operands (the "
                                      "measured_ceiling below, probed in this run) runs at 0.6-0.66 of the "
                                      "2.5 PFLOP/s peak with the engine clock at 1.6-1.65 GHz; the scan runs "
                                      "its LDS reads at about 160 of the ~225 B/clk per CU the LDS delivers"),
        },
    }
    log(f"configs[1] cosine top-100 (index search): {ms:.3f} ms/step = {res['qps']:.0f} QPS; scan "
        f"{ph['scan_ms']:.3f} ms = {tflops:.1f} TFLOP/s ({100 * tflops / peak:.1f}% of the "
        f"{'fp16' if screened else 'fp32'} MFMA peak)")
    # the same search on the fp32 scan alone: the same ids and distances, bit for bit
    idx32 = ctx.empty((Q, k), torch.int32)
    dist32 = ctx.empty((Q, k), torch.float32)
    ctx.set_option(_lib.VA_OPT_SCREEN, 1)
    try:
        ms32, ph32 = timed(ctx, lambda: ix.searchDevice(q, k, idx32, dist32), max(3, a.steps // 2), 1)
    finally:
        ctx.set_option(_lib.VA_OPT_SCREEN, 0)
    s32 = mean_phases(ph32)["scan_ms"]
    same = bool(torch.equal(idx, idx32)) and bool(torch.equal(dist.view(torch.int32), dist32.view(torch.int32)))
    c32 = counters(COUNTERS_FP32)
    res["fp32_scan_only"] = {
        "ms_per_step": ms32, "qps": Q / (ms32 * 1e-3), "scan_ms": s32,
        "scan_tflops": flops / (s32 * 1e-3) / 1e12,
        "mfma_frac": flops / (s32 * 1e-3) / 1e12 / PEAK["fp32_mfma_tflops"],
        "kernel": "dist_gemm_kernel<4, 1, true, 2, true, false>",
        "traffic": c32.get("traffic_bytes_per_launch"), "mfma_busy": c32.get("mfma_busy_pct"),
        "counters_source": COUNTERS_FP32,
    }
    res["screened_equals_fp32_scan"] = same
    log(f"configs[1] fp32 scan only: {ms32:.3f} ms/step, scan {s32:.3f} ms; screened result identical: {same}")
    if not same:
        raise SystemExit("screened search differs from the fp32 scan")
    del idx32, dist32
    # the raw-pointer search (va_fused_topk over the fp32 rows, converting them to fp16 in the
    # scan): the same result again
    kern = FusedL2TopKKernel(ctx)
    params = FusedL2TopKParameters(Q, N, D, k)
    idxr = ctx.empty((Q, k), torch.int32)
    distr = ctx.empty((Q, k), torch.float32)
    msr, phr = timed(ctx, lambda: kern.encode(q, rows, idxr, distr, params, Metric.cosine), max(3, a.steps // 2), 1)
    sr = mean_phases(phr)["scan_ms"]
    same_r = bool(torch.equal(idx, idxr)) and bool(torch.equal(dist.view(torch.int32), distr.view(torch.int32)))
    cr = counters(COUNTERS_SCREEN)
    res["raw_fused_topk"] = {
        "ms_per_step": msr, "qps": Q / (msr * 1e-3), "scan_ms": sr, "scan_tflops": flops / (sr * 1e-3) / 1e12,
        "kernel": "screen_kernel<1> (fp32 rows converted in the scan)", "equals_index_search": same_r,
        "mfma_busy": cr.get("mfma_busy_pct"), "traffic": cr.get("traffic_bytes_per_launch"),
        "counters_source": COUNTERS_SCREEN,
    }
    log(f"configs[1] va_fused_topk over the fp32 rows: {msr:.3f} ms/step, scan {sr:.3f} ms; identical: {same_r}")
    if not same_r:
        raise SystemExit("va_fused_topk differs from the index search")
    # end to end: host queries in, host ids and distances out (pinned buffers, copies on the
    # context's stream), timed around the whole call
    qh = torch.empty((Q, D), dtype=torch.float32, pin_memory=True)
    qh.copy_(q)
    oh_i = torch.empty((Q, k), dtype=torch.int32, pin_memory=True)
    oh_d = torch.empty((Q, k), dtype=torch.float32, pin_memory=True)
    qd = ctx.empty((Q, D), torch.float32)
    stream = ctx.torch_stream()

    def e2e():
        with torch.cuda.stream(stream):
            qd.copy_(qh, non_blocking=True)
        ix.searchDevice(qd, k, idxr, distr)
        with torch.cuda.stream(stream):
            oh_i.copy_(idxr, non_blocking=True)
            oh_d.copy_(distr, non_blocking=True)

    mse, _ = timed(ctx, e2e, max(3, a.steps // 2), 1, scan_timings=False)
    same_e = bool(torch.equal(oh_i, idx.cpu())) and bool(torch.equal(oh_d.view(torch.int32), dist.cpu().view(torch.int32)))
    res["end_to_end"] = {"ms_per_step": mse, "qps": Q / (mse * 1e-3), "equals_resident": same_e,
                         "host_bytes_per_step": Q * D * 4 + Q * k * 8,
                         "what": "pinned host queries -> device -> index search -> pinned host ids + distances"}
    log(f"configs[1] end to end (host queries in, host results out): {mse:.3f} ms/step = {Q / (mse * 1e-3):.0f} "
        f"QPS; identical: {same_e}")
    del qh, oh_i, oh_d, qd
    if extra_l2:
        # the same search with the database in pinned host memory, streamed through the device
        # (va_fused_topk_streamed): bound by the host link, not by HBM or the MFMA
        xh = torch.empty((N, D), dtype=torch.float32, pin_memory=True)
        ctx.check(ctx.lib.va_buffer_download(ctx.handle, xh.data_ptr(), rows.data_ptr(), N * D * 4),
                  "va_buffer_download")
        ctx.synchronize()
        idx_s = ctx.empty((Q, k), torch.int32)
        dist_s = ctx.empty((Q, k), torch.float32)
        ms_s, _ = timed(ctx, lambda: kern.encodeStreamed(q, xh, idx_s, dist_s, params, Metric.cosine), 2, 1,
                        scan_timings=False)
        same_s = bool(torch.equal(idx, idx_s)) and bool(torch.equal(dist.view(torch.int32), dist_s.view(torch.int32)))
        gbs = N * D * 4 / (ms_s * 1e-3) / 1e9
        res["host_resident_streamed"] = {
            "ms_per_step": ms_s, "qps": Q / (ms_s * 1e-3), "host_to_device_gbs": gbs,
            "host_link_peak_gbs": PEAK["pcie5_x16_gbs"], "host_link_frac": gbs / PEAK["pcie5_x16_gbs"],
            "chunk_rows": "auto (~512 MiB chunks)", "equals_resident": same_s,
        }
        log(f"configs[1] streamed from pinned host memory: {ms_s:.1f} ms/step = {Q / (ms_s * 1e-3):.0f} QPS, "
            f"{gbs:.1f} GB/s host->device; identical to the resident search: {same_s}")
        del xh, idx_s, dist_s
        idx10 = ctx.empty((Q, 10), torch.int32)
        dist10 = ctx.empty((Q, 10), torch.float32)
        p10 = FusedL2TopKParameters(Q, N, D, 10)
        ms10, ph10 = timed(ctx, lambda: kern.encode(q, rows, idx10, dist10, p10, Metric.euclideanSquared),
                           max(3, a.steps // 2), 1)
        s10 = mean_phases(ph10)["scan_ms"]
        res["l2sq_top10_same_shape_raw"] = {"ms_per_step": ms10, "qps": Q / (ms10 * 1e-3), "scan_ms": s10,
                                            "scan_tflops": flops / (s10 * 1e-3) / 1e12,
                                            "mfma_frac": flops / (s10 * 1e-3) / 1e12 / peak}
        log(f"configs[1] shape, L2^2 top-10 (va_fused_topk): {ms10:.3f} ms/step, scan {s10:.3f} ms")
        # the metric's own wording through the index: flat L2^2 top-10 at 1M x 1536, Q=1024
        ixi = ctx.empty((Q, 10), torch.int32)
        ixd = ctx.empty((Q, 10), torch.float32)

        def l2_index():
            ctx.check(ctx.lib.va_index_search(ctx.handle, ix._h, _lib.VA_METRIC_L2SQ, q.data_ptr(), Q, 10,
                                              ixi.data_ptr(), ixd.data_ptr()), "va_index_search")

        msi, phi = timed(ctx, l2_index, a.steps, a.warmup)
        si = mean_phases(phi)
        same_i = bool(torch.equal(ixi, idx10)) and bool(torch.equal(ixd.view(torch.int32), dist10.view(torch.int32)))
        ti = flops / (si["scan_ms"] * 1e-3) / 1e12
        res["l2sq_top10_index_search"] = {
            "ms_per_step": msi, "qps": Q / (msi * 1e-3), "phases_ms": si, "scan_tflops": ti,
            "mfma_frac": ti / PEAK["fp16_mfma_tflops"], "equals_fused_topk": same_i,
            "what": "the metric's wording (flat L2^2 top-10 @1M x 1536, Q=1024) through va_index_search "
                    "(screen16_kernel over the shadow)"}
        log(f"configs[1] shape, L2^2 top-10 through the index: {msi:.3f} ms/step = {Q / (msi * 1e-3):.0f} QPS, scan "
            f"{si['scan_ms']:.3f} ms; identical to va_fused_topk: {same_i}")
        if not same_i:
            raise SystemExit("L2^2 index search differs from va_fused_topk")
        del ixi, ixd
        res["small_batches"] = run_small_batches(ctx, a, ix, q, _lib.VA_METRIC_COSINE, 100,
                                                 "configs[1] shape (1M x 1536 cosine top-100)")
    if cpu:
        from oracle import oracle

        nq = 512
        log(f"configs[1] CPU baseline: {nq} queries on {oracle.num_threads()} threads")
        xh = np.empty((N, D), np.float32)
        ctx.check(ctx.lib.va_buffer_download(ctx.handle, xh.ctypes.data, rows.data_ptr(), N * D * 4),
                  "va_buffer_download")
        ctx.synchronize()
        qh = q[:nq].cpu().numpy()
        t0 = time.perf_counter()
        ci, _ = oracle.flat_topk(oracle.COSINE, qh, xh, k, accum_double=False)
        dt = time.perf_counter() - t0
        gi = idx[:nq].cpu().numpy().view(np.uint32)
        res["cpu_baseline"] = {
            "value": nq / dt, "unit": "queries/s", "cores": oracle.num_threads(), "kind": "port",
            "sample": (f"{nq} of the {Q} configs[1] queries against the full {N}x{D} database; C port of "
                       "AccelerateFallback.batchCosineSimilarity + CPUTopK's bounded heap (float accumulation)"),
            "seconds": dt,
            "topk_id_overlap_with_gpu": float(np.mean([len(set(gi[r]) & set(ci[r])) / k for r in range(nq)])),
        }
        log(f"configs[1] CPU baseline: {nq / dt:.2f} QPS ({dt:.1f} s)")
        del xh
    del q, rows
    ix.close()
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------------------
# scalar int8, 10M x 512, Q = 4096, top-10
# ---------------------------------------------------------------------------------------
def run_c3(ctx, a, cpu: bool):
    import numpy as np
    import torch

    from vectoraccelerate_amd import ScalarQuantizationKernel

    N, D, Q, k = 10_000_000, 512, 4096, 10
    log(f"configs[2]: generating N={N} D={D} Q={Q}")
    g = torch.Generator(device="cuda").manual_seed(2)
    s = torch.rand(D, device="cuda", generator=g) * 1.5 + 0.5  # U(0.5, 2) per dimension
    x = (torch.rand(N, D, device="cuda", generator=g) * 2 - 1).mul_(s)  # U(-1, 1) * s_d
    qf = ((torch.rand(Q, D, device="cuda", generator=g) * 2 - 1) * s).contiguous()
    torch.cuda.synchronize()
    sq = ScalarQuantizationKernel(ctx)
    mn, mx = ctx.empty((D,), torch.float32), ctx.empty((D,), torch.float32)
    sc, zp = ctx.empty((D,), torch.float32), ctx.empty((D,), torch.int32)
    codes = ctx.empty((N, D), torch.int8)
    qcodes = ctx.empty((Q, D), torch.int8)
    ctx.order_after_torch()

    def quantize_db():
        sq.encodeComputeParameters(x, N, D, mn, mx, sc, zp)
        sq.encodeQuantize(x, codes, sc, zp, N, D)

    qms, _ = timed(ctx, quantize_db, 2, 1, scan_timings=False)
    sq.encodeQuantize(qf, qcodes, sc, zp, Q, D)
    ctx.synchronize()
    del x, qf
    torch.cuda.empty_cache()
    idx = ctx.empty((Q, k), torch.int32)
    dist = ctx.empty((Q, k), torch.int32)
    ms, phases = timed(ctx, lambda: sq.encodeScanTopK(qcodes, codes, idx, dist, Q, N, D, k), max(3, a.steps // 2), 1)
    ph = mean_phases(phases)
    ops = 2.0 * Q * N * D
    tops = ops / (ph["scan_ms"] * 1e-3) / 1e12
    res = {
        "workload": "configs[2]: int8 top-10, N=10,000,000 x d=512, Q=4096, per-dimension min/max affine codes",
        "ms_per_step": ms, "qps": Q / (ms * 1e-3), "phases_ms": ph,
        "quantize_database_ms": qms,
        "quantize_hbm_gbs": (N * D * 4 * 2 + N * D) / (qms * 1e-3) / 1e9,
        "roofline": {"bound": "mfma", "achieved": tops, "peak": PEAK["int8_mfma_tops"], "unit": "TOP/s",
                     "frac": tops / PEAK["int8_mfma_tops"], "kernel": "i8_resq16_kernel<512, 16, 4>",
                     "algorithmic": f"2*Q*N*D = {ops:.4g} int ops per launch", **counted(COUNTERS_I8)},
    }
    log(f"configs[2] int8 top-10: {ms:.3f} ms/step = {res['qps']:.0f} QPS; scan {ph['scan_ms']:.3f} ms = "
        f"{tops:.0f} TOP/s; quantize 10M x 512 in {qms:.2f} ms")
    if cpu:
        from oracle import oracle

        nq = 64
        xh = codes.cpu().numpy()
        qh = qcodes[:nq].cpu().numpy()
        t0 = time.perf_counter()
        ci, cd = oracle.i8_topk(qh, xh, k)
        dt = time.perf_counter() - t0
        gi = idx[:nq].cpu().numpy().view(np.uint32)
        res["cpu_baseline"] = {"value": nq / dt, "unit": "queries/s", "cores": oracle.num_threads(), "kind": "port",
                               "sample": f"{nq} queries x the full 10M x 512 int8 database (int32 dot + heap)",
                               "seconds": dt, "ids_bit_exact_vs_gpu": bool(np.array_equal(gi, ci))}
        log(f"configs[2] CPU baseline: {nq / dt:.2f} QPS; ids bit-exact vs GPU: {np.array_equal(gi, ci)}")
        del xh
    del codes
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------------------
# binary Hamming, 50M x 768 bits, Q = 256, top-100
# ---------------------------------------------------------------------------------------
def run_c4(ctx, a, cpu: bool):
    import numpy as np
    import torch

    from vectoraccelerate_amd import HammingDistanceKernel

    N, W, Q, k = 50_000_000, 24, 256, 100
    log(f"configs[3]: generating N={N} x {W} words, Q={Q}")
    # sign bits of i.i.d. N(0,1) floats are i.i.d. fair bits: draw the packed words directly
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randint(-2**31, 2**31 - 1, (N, W), device="cuda", generator=g, dtype=torch.int32)
    q = torch.randint(-2**31, 2**31 - 1, (Q, W), device="cuda", generator=g, dtype=torch.int32)
    torch.cuda.synchronize()
    h = HammingDistanceKernel(ctx)
    idx = ctx.empty((Q, k), torch.int32)
    dist = ctx.empty((Q, k), torch.int32)
    ctx.order_after_torch()
    ms, phases = timed(ctx, lambda: h.encodeTopK(q, x, idx, dist, Q, N, W, k), max(3, a.steps // 2), 1)
    ph = mean_phases(phases)
    # the filter scan computes a.b of bit vectors on the fp4 MFMA: 2 ops per bit per pair
    flops = 2.0 * Q * N * W * 32
    tflops = flops / (ph["scan_ms"] * 1e-3) / 1e12
    valu_equiv = 2.0 * Q * N * W / (ph["scan_ms"] * 1e-3) / 1e12
    gbs = N * W * 4 / (ph["scan_ms"] * 1e-3) / 1e9
    res = {
        "workload": "configs[3]: binary Hamming top-100, N=50,000,000 x 768 bits (96 B), Q=256",
        "ms_per_step": ms, "qps": Q / (ms * 1e-3), "phases_ms": ph,
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": PEAK["fp4_mfma_tflops"], "unit": "TFLOP/s",
                     "frac": tflops / PEAK["fp4_mfma_tflops"], "kernel": "hamming_mfma_kernel<24>",
                     "note": "Hamming = |a| + |b| - 2 a.b with a.b of {0,1} vectors on the fp4 MFMA (exact: "
                             "integer sums in fp32); the xor + popcount VALU scan it replaces is bound by VALU "
                             "issue (2 instructions per 32-bit word per pair, valu_equivalent_tops vs 39.3 "
                             "peak). The database is read from HBM once (hbm_frac).",
                     "algorithmic": f"2 ops per bit per (query, row) pair: {flops:.4g} per launch",
                     "valu_equivalent_tops": valu_equiv,
                     "hbm_gbs_database_once": gbs, "hbm_frac": gbs / PEAK["hbm_gbs"], **counted(COUNTERS_HAMMING)},
    }
    log(f"configs[3] binary top-100: {ms:.3f} ms/step = {res['qps']:.0f} QPS; scan {ph['scan_ms']:.3f} ms = "
        f"{tflops:.0f} TFLOP/s fp4 MFMA ({100 * tflops / PEAK['fp4_mfma_tflops']:.1f}%), {gbs:.0f} GB/s")
    if cpu:
        from oracle import oracle

        nq = 32
        xh = x.cpu().numpy().view(np.uint32)
        qh = q[:nq].cpu().numpy().view(np.uint32)
        t0 = time.perf_counter()
        ci, cd = oracle.hamming_topk(qh, xh, k)
        dt = time.perf_counter() - t0
        gi = idx[:nq].cpu().numpy().view(np.uint32)
        res["cpu_baseline"] = {"value": nq / dt, "unit": "queries/s", "cores": oracle.num_threads(), "kind": "port",
                               "sample": f"{nq} queries x the full 50M-code database (popcount + stable top-k)",
                               "seconds": dt, "ids_bit_exact_vs_gpu": bool(np.array_equal(gi, ci))}
        log(f"configs[3] CPU baseline: {nq / dt:.2f} QPS; ids bit-exact vs GPU: {np.array_equal(gi, ci)}")
        del xh
    del x
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------------------
# IVF-Flat, 4096 lists, 4M x 768, Zipf(1.1) cluster sizes, Q=1024, nprobe 32
# ---------------------------------------------------------------------------------------
def ivf_phases(ctx, fn, reps: int = 3) -> dict:
    """Phase times of the IVF list scan (the last scan of each search), averaged over a few
    searches run after a timed loop (each read waits for its search)."""
    keys = ("sample_ms", "scan_ms", "select_ms", "fallback_ms", "total_ms")
    acc = {k: 0.0 for k in keys}
    last = {}
    for _ in range(reps):
        fn()
        ctx.synchronize()
        last = ctx.last_scan_timings()
        for k in keys:
            acc[k] += float(last[k]) / reps
    acc.update({k: last[k] for k in ("candidate_cap", "overflow_rows", "screened", "rerank_rows") if k in last})
    return acc


def run_c5(ctx, a, cpu: bool):
    import numpy as np
    import torch

    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline, _lib

    C, D, N, Q, nprobe, k = 4096, 768, 4_000_000, 1024, 32, 10
    log(f"configs[4]: generating C={C} N={N} D={D} Q={Q}")
    g = torch.Generator(device="cuda").manual_seed(4)
    cen = torch.randn(C, D, device="cuda", generator=g) * 4.0
    p = 1.0 / torch.arange(1, C + 1, device="cuda", dtype=torch.float64) ** 1.1
    p = (p / p.sum()).float()
    lab = torch.multinomial(p, N, replacement=True, generator=g)
    x = cen[lab] + torch.randn(N, D, device="cuda", generator=g)
    qlab = torch.multinomial(p, Q, replacement=True, generator=g)
    q = (cen[qlab] + torch.randn(Q, D, device="cuda", generator=g)).contiguous()
    torch.cuda.synchronize()
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(C, nprobe, D))
    t0 = time.perf_counter()
    st = pipe.prepareIndexStructure(cen, x)
    build_s = time.perf_counter() - t0
    off, ids = st.lists()
    probes = pipe.findNearestCentroids(q, st).cpu().numpy().view(np.uint32)
    sizes = np.diff(off.astype(np.int64))
    cand = int(sizes[probes].sum())
    distinct = np.unique(probes)
    idx = ctx.empty((Q, k), torch.int32)
    dist = ctx.empty((Q, k), torch.float32)
    step = lambda: pipe.encodeSearch(q, st, idx, dist, k)  # noqa: E731
    ms, _ = timed(ctx, step, max(20, a.steps), 3, scan_timings=False)
    ph = ivf_phases(ctx, step)
    # the same search on the fp32 list scan alone: the same ids and distances, bit for bit
    idx32 = ctx.empty((Q, k), torch.int32)
    dist32 = ctx.empty((Q, k), torch.float32)
    step32 = lambda: pipe.encodeSearch(q, st, idx32, dist32, k)  # noqa: E731
    ctx.set_option(_lib.VA_OPT_SCREEN, 1)
    try:
        ms32, _ = timed(ctx, step32, max(3, a.steps // 2), 1, scan_timings=False)
        ph32 = ivf_phases(ctx, step32)
    finally:
        ctx.set_option(_lib.VA_OPT_SCREEN, 0)
    same = bool(torch.equal(idx, idx32)) and bool(torch.equal(dist.view(torch.int32), dist32.view(torch.int32)))
    flops = 2.0 * Q * C * D + 2.0 * D * cand
    tflops = flops / (ms * 1e-3) / 1e12
    b_min = float(sizes[distinct].sum()) * D * 4 + C * D * 4
    # the screened main pass streams the fp16 shadow of every probed list (each row block once,
    # its query blocks on neighbouring waves) and the fp16 queries
    b16 = float(sizes[distinct].sum()) * D * 2 + Q * D * 2
    gbs = b16 / (ph["scan_ms"] * 1e-3) / 1e9
    screened = bool(ph.get("screened", 0))
    res = {
        "workload": "configs[4]: IVF-Flat L2^2 top-10, 4096 lists, N=4,000,000 x d=768 (Zipf 1.1), Q=1024, nprobe 32",
        "ms_per_step": ms, "qps": Q / (ms * 1e-3), "build_s": build_s, "phases_ms": ph,
        "candidates_scanned": cand, "largest_list": int(sizes.max()),
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK["hbm_gbs"], "unit": "GB/s",
                     "frac": gbs / PEAK["hbm_gbs"],
                     "kernel": ("screened list scan: ivf16_big_kernel (lists probed by more than 96 queries), then "
                                "ivf16_narrow_kernel / ivf16_wide_kernel<1> / ivf16_resq_kernel concurrently (fp16 shadow "
                                "rows on the fp16 MFMA), timed as one phase" if screened else "fp32 list scan"),
                     "algorithmic": f"fp16 shadow of the distinct probed lists + fp16 queries = {b16 / 1e9:.2f} GB "
                                    f"per search (fp32 rows: {b_min / 1e9:.2f} GB)",
                     "counted": {name: counted(rel) for name, rel in COUNTERS_IVF16.items()},
                     "whole_search_fp32_equivalent_tflops": tflops,
                     "whole_search_fp32_mfma_frac": tflops / PEAK["fp32_mfma_tflops"],
                     "fp32_work": f"2QCD + 2D*sum|L_p| = {flops:.4g} FLOP"},
        "fp32_list_scan_only": {"ms_per_step": ms32, "qps": Q / (ms32 * 1e-3), "phases_ms": ph32,
                                "whole_search_tflops": flops / (ms32 * 1e-3) / 1e12,
                                "counted": {name: counted(rel) for name, rel in COUNTERS_IVF.items()}},
        "screened_equals_fp32_list_scan": same,
    }
    if not same:
        raise SystemExit("screened IVF search differs from the fp32 list scan")
    del idx32, dist32
    log(f"configs[4] IVF top-10: {ms:.3f} ms/step = {res['qps']:.0f} QPS ({tflops:.1f} TFLOP/s fp32-equivalent); "
        f"list scan {ph['scan_ms']:.3f} ms = {gbs:.0f} GB/s of fp16 rows; fp32 list scan {ms32:.3f} ms/step; "
        f"identical: {same}; {cand / 1e6:.1f}M candidates; build {build_s:.1f} s")
    if cpu:
        from oracle import oracle

        nq = 128
        xh = x.cpu().numpy()
        qh = q[:nq].cpu().numpy()
        ch = cen.cpu().numpy()
        t0 = time.perf_counter()
        op = oracle.ivf_probe(qh, ch, nprobe)
        ci, cd = oracle.ivf_scan(qh, xh, off, ids, op, k)
        dt = time.perf_counter() - t0
        gi = idx[:nq].cpu().numpy().view(np.uint32)
        res["cpu_baseline"] = {"value": nq / dt, "unit": "queries/s", "cores": oracle.num_threads(), "kind": "port",
                               "sample": f"{nq} queries: exact coarse probe + list scan over the same lists",
                               "seconds": dt,
                               "topk_id_overlap_with_gpu": float(np.mean([len(set(gi[r]) & set(ci[r])) / k
                                                                          for r in range(nq)]))}
        log(f"configs[4] CPU baseline: {nq / dt:.2f} QPS")
        del xh
    st.close()
    del x, cen, q
    torch.cuda.empty_cache()
    return res


def run_kmeans(ctx, a, cpu: bool):
    """IVF training at configs[4]'s shape: 4096 centroids, d=768, on a 262,144-point sample of
    the configs[4] construction; 10 Lloyd iterations (threshold 0, so all ten run)."""
    import numpy as np
    import torch

    from vectoraccelerate_amd import KMeansConfiguration, KMeansPipeline, KMeansPlusPlusKernel

    C, D, N, iters = 4096, 768, 262_144, 10
    g = torch.Generator(device="cuda").manual_seed(14)
    cen = torch.randn(C, D, device="cuda", generator=g) * 4.0
    p = 1.0 / torch.arange(1, C + 1, device="cuda", dtype=torch.float64) ** 1.1
    lab = torch.multinomial((p / p.sum()).float(), N, replacement=True, generator=g)
    x = (cen[lab] + torch.randn(N, D, device="cuda", generator=g)).contiguous()
    del cen, lab
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    init, _ = KMeansPlusPlusKernel(ctx).selectCentroidsBuffer(x, C, 7)
    pp_s = time.perf_counter() - t0
    pipe = KMeansPipeline(ctx, KMeansConfiguration(C, D, maxIterations=iters, convergenceThreshold=0.0))
    KMeansPipeline(ctx, KMeansConfiguration(C, D, maxIterations=1, convergenceThreshold=0.0)).fit(x, init)  # warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    r = pipe.fit(x, init)
    fit_s = time.perf_counter() - t0
    ms_it = fit_s * 1e3 / r.iterations
    flops = 2.0 * N * C * D
    tflops = flops / (ms_it * 1e-3) / 1e12
    res = {
        "workload": "IVF training (k-means) at configs[4]'s shape: 4096 centroids, d=768, 262,144 points, "
                    "k-means++ seeding then 10 Lloyd iterations",
        "ms_per_iteration": ms_it, "kmeanspp_s": pp_s, "iterations": r.iterations, "inertia": r.inertia,
        "assignment_tflops_effective": tflops,
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": PEAK["fp32_mfma_tflops"], "unit": "TFLOP/s",
                     "frac": tflops / PEAK["fp32_mfma_tflops"],
                     "kernel": "whole Lloyd iteration (assignment GEMM + grouping + means + convergence)",
                     "algorithmic": f"2NCD = {flops:.4g} FLOP per iteration"},
    }
    log(f"k-means C={C} D={D} N={N}: {ms_it:.2f} ms/iteration ({tflops:.1f} TFLOP/s effective), "
        f"k-means++ {pp_s:.2f} s, inertia {r.inertia:.4g}")
    if cpu:
        from oracle import oracle

        ns = 4096
        xh = x[:ns].cpu().numpy()
        ih = init.cpu().numpy()
        t0 = time.perf_counter()
        oracle.kmeans_fit(xh, ih, 1, 0.0)
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": ns * C * D * 2 / dt / 1e12, "unit": "TFLOP/s (assignment)",
                               "cores": oracle.num_threads(), "kind": "port",
                               "sample": f"one Lloyd iteration of {ns} points against the same 4096 centroids",
                               "seconds": dt}
        log(f"k-means CPU baseline: {ns} points, one iteration in {dt:.2f} s")
    del x, init, r
    torch.cuda.empty_cache()
    return res


def run_pq(ctx, a, cpu: bool):
    """PQ ADC search: 10M database rows coded with M=16 sub-quantizers of K=256 (d=768, 48 values
    per sub-vector), Q=1024, top-10.  Codes are synthetic (uniform bytes) and the codebooks random;
    the scan's cost does not depend on how the codes were made.  Encoding is timed on 1M rows."""
    import numpy as np
    import torch

    from vectoraccelerate_amd import Metal4EncodedVectors, Metal4PQConfig, Metal4PQModel, ProductQuantizationKernel

    N, D, M, K, Q, k = 10_000_000, 768, 16, 256, 1024, 10
    g = torch.Generator(device="cuda").manual_seed(21)
    cfg = Metal4PQConfig(D, M, K)
    cb = torch.randn(M, K, D // M, device="cuda", generator=g)
    codes = torch.randint(0, 256, (N, M), device="cuda", dtype=torch.uint8, generator=g)
    q = torch.randn(Q, D, device="cuda", generator=g)
    pq = ProductQuantizationKernel(ctx)
    model = Metal4PQModel(cb, cfg)
    enc = Metal4EncodedVectors(codes, N, cfg)
    idx = ctx.empty((Q, k), torch.int32)
    dist = ctx.empty((Q, k), torch.float32)

    def step():
        ctx.check(ctx.lib.va_pq_search(ctx.handle, q.data_ptr(), Q, D, M, K, cb.data_ptr(), codes.data_ptr(), N, k,
                                       idx.data_ptr(), dist.data_ptr()), "va_pq_search")

    ms, ph = timed(ctx, step, max(3, a.steps // 2), 1)
    tim = mean_phases(ph)
    lookups = float(Q) * N * M
    scan_ms = tim.get("scan_ms") if tim else None
    rate = lookups / (scan_ms * 1e-3) / 1e12 if scan_ms else None
    # LDS: 128 bytes per clock per CU = 32 four-byte words; 256 CUs at 2.4 GHz = 19.66 T words/s.
    # The filter pass reads fp16 pair tables: one 4-byte word carries two queries' entries (and one
    # 128-bit read four words, eight queries), so the fraction is counted per word (two lookups).
    lds_peak = 256 * 32 * 2.4e9 / 1e12
    reads = rate / 2 if rate else None
    xe = torch.randn(1_000_000, D, device="cuda", generator=g)
    ce = ctx.empty((1_000_000, M), torch.uint8)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ctx.check(ctx.lib.va_pq_encode(ctx.handle, xe.data_ptr(), 1_000_000, D, M, K, cb.data_ptr(), ce.data_ptr()),
              "va_pq_encode")
    ctx.synchronize()
    enc_s = time.perf_counter() - t0
    res = {
        "workload": "PQ ADC top-10: 10M rows x M=16 codes (K=256, d=768), Q=1024 (synthetic codes, random codebooks)",
        "ms_per_step": ms, "qps": Q / (ms * 1e-3), "scan_timings": tim,
        "encode_rows_per_s": 1_000_000 / enc_s,
        "roofline": {"bound": "lds", "achieved": reads, "peak": lds_peak, "unit": "T 4-byte LDS reads/s",
                     "frac": (reads / lds_peak) if reads else None, "kernel": "pq_adc_screen<16> (filter pass)",
                     "lookups_per_s_T": rate,
                     "algorithmic": f"Q*N*M = {lookups:.4g} table lookups per scan = {lookups / 2:.4g} 4-byte LDS "
                                    "words (fp16 pair tables, entry-major: one word serves two queries, one "
                                    "128-bit read eight; exact fp32 re-score of the passes)",
                     **counted(COUNTERS_PQ)},
    }
    log(f"PQ ADC top-10: {ms:.3f} ms/step = {res['qps']:.0f} QPS; filter scan {scan_ms} ms = "
        f"{rate if rate is None else round(rate, 2)} T lookups/s = {reads if reads is None else round(reads / lds_peak, 3)} "
        f"of the LDS read rate; encode {res['encode_rows_per_s']:.3g} rows/s")
    if cpu:
        from oracle import oracle

        nq = 16
        ch = codes.cpu().numpy()
        qh = q[:nq].cpu().numpy()
        cbh = cb.cpu().numpy()
        t0 = time.perf_counter()
        oi, od = oracle.pq_search(qh, cbh, ch, M, K, k)
        dt = time.perf_counter() - t0
        gi = idx[:nq].cpu().numpy().view(np.uint32)
        res["cpu_baseline"] = {"value": nq / dt, "unit": "queries/s", "cores": oracle.num_threads(), "kind": "port",
                               "sample": f"{nq} queries: tables + ADC over all 10M codes + heap top-k", "seconds": dt,
                               "ids_equal_gpu": bool((gi == oi).all())}
        log(f"PQ CPU baseline: {nq / dt:.2f} QPS; ids equal: {res['cpu_baseline']['ids_equal_gpu']}")
    del codes, q, cb, xe, ce
    torch.cuda.empty_cache()
    return res


def run_small_768(ctx, a):
    """The reference's own batch-scaling shape: flat L2^2 top-10 over 1M x 768 N(0,1) rows with
    Q = 1, 10, 100 (Guides/03-Accelerated-Search/01-Flat-Search-On-GPU.md:300-308), through the index."""
    import torch

    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration, _lib

    N, D = 1_000_000, 768
    g = torch.Generator(device="cuda").manual_seed(30)
    x = torch.randn(N, D, device="cuda", generator=g)
    q = torch.randn(100, D, device="cuda", generator=g).contiguous()
    ix = AcceleratedVectorIndex(IndexConfiguration.flat(D, N), ctx)
    ix.insert(vectors=x)
    del x
    torch.cuda.empty_cache()
    res = run_small_batches(ctx, a, ix, q, _lib.VA_METRIC_L2SQ, 10, "1M x 768 L2^2 top-10")
    res["workload"] = "flat L2^2 top-10, N=1,000,000 x d=768 N(0,1) rows, Q in {1, 10, 100} (index search)"
    ix.close()
    torch.cuda.empty_cache()
    return res


def main() -> int:
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (every box in this build has one); --gpus {a.gpus} is not supported",
              file=sys.stderr)
        return 2
    import torch

    from vectoraccelerate_amd import GPUContext

    if a.copy_calibration:
        src_t = torch.ones(1 << 28, device="cuda", dtype=torch.float32)  # 1 GiB
        dst_t = torch.empty_like(src_t)
        dst_t.copy_(src_t)
        torch.cuda.synchronize()
        log("copy calibration: 1 GiB read + 1 GiB written by one copy kernel")
        del src_t, dst_t
    ctx = GPUContext(0)
    ctx.set_profiling(True)
    cpu = not a.no_cpu
    extra = {}
    ceil = run_ceiling(ctx) if a.workload in ("all", "ceiling") else None
    if ceil:
        extra["mfma_ceiling"] = ceil
    if a.workload == "ceiling":
        ctx.close()
        print(json.dumps({"metric": METRIC, "value": None, "extra": extra}), flush=True)
        return 0
    if a.workload in ("all", "small"):
        extra["small_batches_1Mx768"] = run_small_768(ctx, a)
    if a.workload in ("all", "c2"):
        c2 = run_c2(ctx, a, cpu, extra_l2=not a.no_extra)
    else:
        c2 = None
    if a.workload in ("all", "c3"):
        extra["configs2_int8"] = run_c3(ctx, a, cpu)
    if a.workload in ("all", "c4"):
        extra["configs3_binary"] = run_c4(ctx, a, cpu)
    if a.workload in ("all", "c5"):
        extra["configs4_ivf"] = run_c5(ctx, a, cpu)
    if a.workload in ("all", "kmeans"):
        extra["ivf_training_kmeans"] = run_kmeans(ctx, a, cpu)
    if a.workload in ("all", "pq"):
        extra["pq_adc"] = run_pq(ctx, a, cpu)
    for key, name in (("configs2_int8", "int8"), ("configs3_binary", "fp4"), ("ivf_training_kmeans", "fp32")):
        if key in extra and "roofline" in extra[key]:
            with_ceiling(extra[key]["roofline"], ceil, name)
    with_hbm_ceiling(extra, ceil)
    if c2 is not None:
        with_hbm_ceiling(c2, ceil)
    ctx.close()
    if c2 is None:
        print(json.dumps({"metric": METRIC, "value": None, "extra": extra}), flush=True)
        return 0
    cpu_base = c2.pop("cpu_baseline", None)
    roof = with_ceiling(c2.pop("roofline"), ceil, "fp16" if c2["phases_ms"].get("screened") else "fp32")
    line = {
        "metric": METRIC,
        "value": c2["qps"],
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": c2["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (torch seeded generators, BASELINE configs constructions)",
        "config": {
            "workload": "BASELINE configs[1]: flat cosine top-100, N=1,000,000 x d=1536 fp32, Q=1024",
            "search": "AcceleratedVectorIndex.search over the native index (va_index_search)",
            "N": 1_000_000, "D": 1536, "Q": 1024, "k": 100, "metric": "cosine (1 - s)",
            "parallelism": "single GPU",
        },
        "roofline": roof,
        "cpu_baseline": cpu_base,
        "extra": {"configs1_cosine_top100": c2, **extra},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

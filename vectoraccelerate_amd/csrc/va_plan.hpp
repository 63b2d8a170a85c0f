// va_plan.hpp — the host-side sizing of the top-k scans: sample sizes, candidate and rerank
// capacities, the device fallback's buffers, the scratch each search carves and the IVF tile
// shapes.  No HIP dependency (like va_keys.hpp), so a host-only test program can include it and
// check the arithmetic under AddressSanitizer and UndefinedBehaviorSanitizer at the extreme
// shapes (k = 1024, N near 2^32, the fixed 64 MiB block of the allocation-free entry point).
#pragma once

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>

#include "va_keys.hpp"

namespace va {

// Scratch carves are rounded to 256 bytes.
inline size_t scratch_round(size_t b) { return (b + 255) & ~size_t(255); }

// ---- the sampled exact scan (va_scan.hip) ------------------------------------------------------
constexpr uint32_t kMinSample = 16384;
// Bytes of dense keys one launch may write (the threshold sample, the dense path, the overflow
// rescan): 256 MiB, or a quarter of a fixed scratch block (fixed_bytes > 0).
inline size_t dense_budget_for(size_t fixed_bytes) {
    constexpr size_t kArena = 256ull << 20;
    return fixed_bytes ? std::min(kArena, fixed_bytes / 4) : kArena;
}

struct ScanPlan {
    uint64_t S = 0;       // sample rows (every stride-th row); S >= N: the dense path
    bool direct = false;  // dense keys of every row, no sample
    uint32_t stride = 1;
    uint64_t cap = 0;     // candidate capacity per query (a multiple of 64, at most N rounded up)
    uint32_t qs = 1;      // queries per sample launch
};

// Sample size N/64 (so that a threshold at the sample's r-th key keeps ~64 r candidates per
// query), at least kMinSample rows, the dense sample's Q S keys capped at the budget; candidate
// capacity max(3k, k + 32) ceil(N / S) + 1024.  opt_* override (0 = automatic).
inline ScanPlan plan_scan_for(uint64_t budget, uint64_t opt_sample_rows, uint64_t opt_candidate_cap, uint32_t Q,
                              uint32_t N, uint32_t k) {
    ScanPlan p;
    const uint64_t q = std::max<uint32_t>(Q, 1);
    p.S = opt_sample_rows ? opt_sample_rows
                          : std::max<uint64_t>(kMinSample, std::min<uint64_t>(N / 64, budget / 4 / q));
    p.direct = p.S >= N;
    if (p.direct) return p;
    p.stride = uint32_t(N / p.S);
    const uint64_t ratio = (uint64_t(N) + p.S - 1) / p.S;
    uint64_t cap = opt_candidate_cap ? opt_candidate_cap : std::max<uint64_t>(3ull * k, uint64_t(k) + 32) * ratio + 1024;
    cap = std::min<uint64_t>(cap, N);
    p.cap = (cap + 63) & ~uint64_t(63);
    p.qs = uint32_t(std::max<uint64_t>(1, std::min<uint64_t>(q, budget / (p.S * 4))));
    return p;
}

// The order statistic of the sample that becomes a query's threshold: k, or the smallest rank r
// whose Poisson(k S / N) tail P(>= r) is below 1e-4 (a list left with fewer than k candidates is
// checked and sent to the fallback).  A deletion mask keeps rank k.  opt_rank > 0 sets r (capped
// at k).
inline uint32_t sample_rank_for(uint64_t opt_rank, uint32_t k, uint64_t S, uint32_t N, bool masked) {
    if (masked || k <= 1) return k;
    if (opt_rank) return uint32_t(std::min<uint64_t>(opt_rank, k));
    const double lam = double(k) * double(S) / double(std::max<uint32_t>(N, 1));
    double term = std::exp(-lam), cdf = term;  // P(X = r - 1), P(X <= r - 1)
    uint32_t r = 1;
    while (r < k && 1.0 - cdf > 1e-4) {
        term *= lam / double(r);
        cdf += term;
        ++r;
    }
    return r;
}

// ---- the device fallback (va_fallback.hpp) ------------------------------------------------------
constexpr int kFbPasses = 5;
constexpr uint32_t kFbGrid = 1024;  // workgroups per pass (4 waves each)
constexpr uint32_t kFbTieBins = 4096;
constexpr uint32_t kFbKeyBins = 2048;

// List capacity and id shift for ids below N, `rows` rows in all (0: N) and top-k.  The id-edge
// pass keeps fewer than k ties plus one id bin, which holds at most min(2^ishift, rows).
inline void fb_geometry(uint32_t N, uint32_t k, uint32_t& ishift, uint32_t& cap, uint32_t rows = 0) {
    ishift = 0;
    while ((uint64_t(N) >> ishift) >= kFbTieBins) ++ishift;
    const uint64_t bin = std::min<uint64_t>(uint64_t(1) << ishift, rows ? rows : N);
    cap = uint32_t((uint64_t(k) + bin + 63) / 64 * 64);
}
inline size_t fb_bytes(uint32_t rmax, uint32_t N, uint32_t k, uint32_t rows = 0) {
    uint32_t ishift, cap;
    fb_geometry(N, k, ishift, cap, rows);
    return scratch_round(uint64_t(rmax) * kFbKeyBins * 4) + scratch_round(uint64_t(rmax) * kFbTieBins * 4) +
           scratch_round(uint64_t(rmax) * 8 * 4) + scratch_round(uint64_t(rmax) * 4) +
           scratch_round(uint64_t(rmax) * cap * 4) * 2 + scratch_round(8 * 4);
}
// Whether the fallback's buffers fit beside `need` bytes (always, with the grow-only arena).
inline bool fb_fits_in(size_t fixed_bytes, size_t need, uint32_t rows, uint32_t N, uint32_t k) {
    return !fixed_bytes || need + fb_bytes(rows, N, k) <= fixed_bytes;
}

// ---- scratch of the scan drivers (the sum of their carves, in carve order) --------------------
// exact_topk_scan's sampled path (without the fallback)
inline size_t exact_scan_need(uint32_t Q, const ScanPlan& p) {
    return scratch_round(uint64_t(Q) * 4) * 3 + scratch_round(uint64_t(Q) * p.cap * 4) * 2 + scratch_round(256) +
           scratch_round(uint64_t(p.qs) * p.S * 4);
}
// The rerank capacity of the screened scan: k plus the band of rows whose interval straddles the
// k-th bound, at least 2k + 256, rounded to 128 rows, at most N.
inline uint64_t screen_rerank_cap(uint32_t N, uint32_t k, uint64_t cap) {
    return std::min<uint64_t>(N, (std::max<uint64_t>(2ull * k + 256, cap / 4) + 127) / 128 * 128);
}
// screened_topk_scan (without the fallback); Dp = the fp16 row pitch in halves
inline size_t screened_scan_need(uint32_t Q, uint32_t Dp, const ScanPlan& p, uint64_t rcap) {
    const size_t q4 = scratch_round(uint64_t(Q) * 4);
    return q4 * 6 + scratch_round(256) + scratch_round(uint64_t(Q) * 16) * 2 + scratch_round(uint64_t(Q) * Dp * 2) +
           scratch_round(uint64_t(p.qs) * p.S * 4) + scratch_round(p.S * 4) + scratch_round(uint64_t(Q) * p.cap * 4) * 3 +
           scratch_round(uint64_t(Q) * rcap * 4) * 2;
}

// ---- IVF (va_ivf.hip) --------------------------------------------------------------------------
// Threshold sample: a prefix of every probed list (rows in insertion order, so a prefix is an
// unbiased subset) of at least 1/64 of its rows and at least 32 rows: every list is sampled at
// rate >= 1/64, so a query's candidate count stays within about 64 k; the floor gives short lists
// a few rows.  (A floor of 128 sampled 13% of configs[4]'s probed rows; 32 measured 0.1 ms faster
// per search, the looser threshold's extra candidates included.)
constexpr uint32_t kIvfSampleRate = 64;
constexpr uint32_t kIvfSampleMin = 32;
VA_HD inline uint32_t ivf_sample_rows(uint32_t n) {
    // (64-bit sum: a list of more than 2^32 - 64 rows would wrap)
    const uint32_t s = uint32_t((uint64_t(n) + kIvfSampleRate - 1) / kIvfSampleRate);
    const uint32_t m = s > kIvfSampleMin ? s : kIvfSampleMin;
    return n < m ? n : m;
}
// Candidate capacity of the fp32 list scan: max(3k, k + 32) * 64 + 1024, at most the rows of the
// nprobe longest lists (top_rows); the screened scan adds 7 times it (at most 16,384 of it per 7).
inline uint64_t ivf_fp32_cap(uint64_t opt_cap, uint32_t k, uint64_t top_rows) {
    const uint64_t cap = opt_cap ? opt_cap : std::max<uint64_t>(3ull * k, uint64_t(k) + 32) * kIvfSampleRate + 1024;
    return std::max<uint64_t>(1, std::min<uint64_t>(cap, top_rows));
}
inline uint64_t ivf_screen_cap(uint64_t opt_cap, uint32_t k, uint64_t top_rows) {
    const uint64_t cap32 = std::max<uint64_t>(3ull * k, uint64_t(k) + 32) * kIvfSampleRate + 1024;
    const uint64_t cap = opt_cap ? opt_cap : cap32 + 7 * std::min<uint64_t>(cap32, 16384);
    return std::max<uint64_t>(1, std::min<uint64_t>(cap, top_rows));
}
inline uint64_t ivf_rerank_cap(uint32_t k, uint64_t cap, uint64_t top_rows) {
    return std::max<uint64_t>(1, std::min<uint64_t>(top_rows, (std::max<uint64_t>(2ull * k + 256, cap / 4) + 127) / 128 * 128));
}

// Tile shapes of the fp32 list scan: shape s has wq x wn waves = (32 wq) x (128 wn) per tile.
// Relative cost per wave tile measured on the box (shapes with more waves share their LDS stages
// across more MFMA work and run more workgroups per CU, except 1 x 4, whose 87 KB of LDS leaves
// one workgroup per CU).  The one- and two-wave shapes keep lists with few queries or few rows
// from paying for a 4-wave tile.  Group kSmallGroup is the 16-query tiles of ivf_small_kernel.
constexpr int kShapes = 5;
constexpr int kSmallGroup = kShapes;
constexpr int kGroups = kShapes + 1;
constexpr uint32_t kSmallListQueries = 16;
constexpr uint32_t kSmallTileQueries = 16, kSmallTileRows = 128;
VA_HD inline int shape_wq(int s) { return s == 0 ? 4 : (s <= 2 ? 2 : 1); }
VA_HD inline int shape_wn(int s) { return s == 1 ? 2 : (s == 4 ? 4 : 1); }
VA_HD inline uint32_t shape_cost(int s) {
    return s == 0 ? 100u : s == 1 ? 120u : s == 2 ? 135u : s == 3 ? 175u : 195u;  // per wave tile, relative
}
// the shape of least estimated time for a list probed by nq queries with nrows rows
VA_HD inline int shape_for(uint32_t nq, uint32_t nrows) {
    int best = 0;
    uint64_t best_cost = ~0ull;
    for (int i = 0; i < kShapes; ++i) {
        const uint32_t wq = uint32_t(shape_wq(i)), wn = uint32_t(shape_wn(i));
        const uint64_t cost = uint64_t((uint64_t(nq) + 32 * wq - 1) / (32 * wq)) *
                              ((uint64_t(nrows) + 128 * wn - 1) / (128 * wn)) * (wq * wn) * shape_cost(i);
        if (cost < best_cost) {
            best = i;
            best_cost = cost;
        }
    }
    return best;
}
VA_HD inline void group_tile(int g, uint32_t& TQ, uint32_t& TN) {
    if (g == kSmallGroup) {
        TQ = kSmallTileQueries;
        TN = kSmallTileRows;
    } else {
        TQ = 32u * uint32_t(shape_wq(g));
        TN = 128u * uint32_t(shape_wn(g));
    }
}

}  // namespace va

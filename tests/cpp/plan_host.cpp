// Host check of the scan planning arithmetic (vectoraccelerate_amd/csrc/va_plan.hpp): sample sizes,
// candidate / rerank capacities, the device fallback's buffers, the scratch the drivers carve and
// the IVF tile shapes, at the extreme shapes (k up to 1024, N up to 2^32 - 1, query batches up to
// 2^20, fp16 pitches up to 131,072 halves, the fixed 64 MiB block).  Every size is recomputed in
// 128-bit integers, so a wrapped 64-bit product fails; tests/test_plan.py builds this with g++
// (under AddressSanitizer + UndefinedBehaviorSanitizer in oracle/run_sanitized.sh) and runs it.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../vectoraccelerate_amd/csrc/va_plan.hpp"

using namespace va;
typedef unsigned __int128 u128;

static int failures = 0;
#define CHECK(cond, ...)                                   \
    do {                                                   \
        if (!(cond)) {                                     \
            if (failures < 40) {                           \
                std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
                std::printf(__VA_ARGS__);                  \
                std::printf("\n");                         \
            }                                              \
            ++failures;                                    \
        }                                                  \
    } while (0)

static u128 rnd(u128 b) { return (b + 255) / 256 * 256; }

// P(X >= r) for X ~ Poisson(lam), summed from the upper tail with log-gamma terms (a different
// route from the recurrence in sample_rank_for)
static double poisson_tail(double lam, uint32_t r) {
    if (r == 0) return 1.0;
    double s = 0.0;
    for (uint32_t i = r; i < r + 2000; ++i) {
        const double t = std::exp(double(i) * std::log(lam) - lam - std::lgamma(double(i) + 1.0));
        s += t;
        if (t < 1e-30 && double(i) > lam) break;
    }
    return s;
}

int main() {
    const uint32_t Qs[] = {1, 7, 32, 191, 192, 1024, 4096, 65535, 1u << 20};
    const uint32_t Ns[] = {1, 100, 16384, 16385, 50000, 1000000, 10000000, 50000000, 0xFFFFFFFEu, 0xFFFFFFFFu};
    const uint32_t ks[] = {1, 10, 64, 100, 1023, 1024};
    const size_t fixed[] = {0, 64ull << 20};
    const uint64_t opt_S[] = {0, 4096, 20000};
    const uint64_t opt_cap[] = {0, 64, 100000};
    const uint32_t Dps[] = {64, 768, 1536, 131072};

    // dense budget: the arena's 256 MiB, or a quarter of a fixed block
    CHECK(dense_budget_for(0) == (256ull << 20), "arena budget");
    CHECK(dense_budget_for(64ull << 20) == (16ull << 20), "fixed-block budget");

    uint64_t plans = 0;
    for (size_t fb : fixed)
        for (uint64_t oS : opt_S)
            for (uint64_t oc : opt_cap)
                for (uint32_t Q : Qs)
                    for (uint32_t N : Ns)
                        for (uint32_t k : ks) {
                            if (k > N) continue;
                            const uint64_t budget = dense_budget_for(fb);
                            const ScanPlan p = plan_scan_for(budget, oS, oc, Q, N, k);
                            ++plans;
                            const uint64_t autoS =
                                std::max<uint64_t>(kMinSample, std::min<uint64_t>(N / 64, budget / 4 / Q));
                            CHECK(p.S == (oS ? oS : autoS), "S Q=%u N=%u", Q, N);
                            CHECK(p.direct == (p.S >= N), "direct Q=%u N=%u", Q, N);
                            if (p.direct) continue;
                            CHECK(p.stride >= 1 && u128(p.S) * p.stride <= N, "stride Q=%u N=%u S=%llu", Q, N,
                                  (unsigned long long)p.S);
                            CHECK(p.cap % 64 == 0 && p.cap >= 64, "cap multiple of 64");
                            CHECK(p.cap <= u128(N) + 63, "cap beyond N Q=%u N=%u k=%u", Q, N, k);
                            if (!oc) CHECK(p.cap >= std::min<uint64_t>(N, uint64_t(k) + 32), "cap below k N=%u k=%u", N, k);
                            CHECK(p.qs >= 1 && p.qs <= Q, "qs range Q=%u qs=%u", Q, p.qs);
                            if (p.qs > 1) CHECK(u128(p.qs) * p.S * 4 <= budget, "sample launch over budget");
                            // scratch sums: no wrapped products (recomputed in 128 bits)
                            const u128 ex = rnd(u128(Q) * 4) * 3 + rnd(u128(Q) * p.cap * 4) * 2 + rnd(256) +
                                            rnd(u128(p.qs) * p.S * 4);
                            CHECK(u128(exact_scan_need(Q, p)) == ex, "exact_scan_need Q=%u N=%u", Q, N);
                            for (uint32_t Dp : Dps) {
                                const uint64_t rcap = screen_rerank_cap(N, k, p.cap);
                                CHECK(rcap <= N && rcap >= std::min<uint64_t>(N, 2ull * k + 256), "rcap N=%u k=%u", N, k);
                                const u128 sn = rnd(u128(Q) * 4) * 6 + rnd(256) + rnd(u128(Q) * 16) * 2 +
                                                rnd(u128(Q) * Dp * 2) + rnd(u128(p.qs) * p.S * 4) + rnd(u128(p.S) * 4) +
                                                rnd(u128(Q) * p.cap * 4) * 3 + rnd(u128(Q) * rcap * 4) * 2;
                                CHECK(u128(screened_scan_need(Q, Dp, p, rcap)) == sn, "screened_scan_need Q=%u N=%u Dp=%u",
                                      Q, N, Dp);
                            }
                            // the threshold's rank
                            for (int masked = 0; masked < 2; ++masked) {
                                const uint32_t r = sample_rank_for(0, k, p.S, N, masked != 0);
                                CHECK(r >= 1 && r <= k, "rank range k=%u r=%u", k, r);
                                if (masked || k <= 1) {
                                    CHECK(r == k, "masked or k <= 1 keeps rank k");
                                    continue;
                                }
                                const double lam = double(k) * double(p.S) / double(N);
                                if (r < k) CHECK(poisson_tail(lam, r) < 1e-4 * (1 + 1e-9), "tail at r=%u lam=%g", r, lam);
                                if (r > 1) CHECK(poisson_tail(lam, r - 1) >= 1e-4 * (1 - 1e-9), "r=%u not minimal lam=%g", r, lam);
                                CHECK(sample_rank_for(5, k, p.S, N, false) == std::min<uint32_t>(5, k), "opt rank");
                            }
                        }
    // the rank grows with the sample fraction
    for (uint32_t k : ks) {
        uint32_t prev = 0;
        for (uint64_t S = 16384; S <= 1000000; S *= 2) {
            const uint32_t r = sample_rank_for(0, k, S, 1000000, false);
            CHECK(r >= prev, "rank not monotone in S (k=%u)", k);
            prev = r;
        }
    }

    // device fallback buffers
    for (uint32_t N : Ns)
        for (uint32_t k : ks)
            for (uint32_t rows : {0u, 1u, 300u, 1u << 20}) {
                uint32_t ishift, cap;
                fb_geometry(N, k, ishift, cap, rows);
                CHECK((uint64_t(N) >> ishift) < kFbTieBins, "tie bins N=%u", N);
                if (ishift) CHECK((uint64_t(N) >> (ishift - 1)) >= kFbTieBins, "ishift not minimal N=%u", N);
                const uint64_t bin = std::min<uint64_t>(uint64_t(1) << ishift, rows ? rows : N);
                CHECK(cap % 64 == 0 && cap >= k + bin, "fb cap N=%u k=%u", N, k);
                for (uint32_t rmax : {1u, 1024u, 4096u, 1u << 20}) {
                    const u128 fbb = rnd(u128(rmax) * 2048 * 4) + rnd(u128(rmax) * kFbTieBins * 4) + rnd(u128(rmax) * 32) +
                                     rnd(u128(rmax) * 4) + rnd(u128(rmax) * cap * 4) * 2 + rnd(32);
                    CHECK(u128(fb_bytes(rmax, N, k, rows)) == fbb, "fb_bytes rmax=%u N=%u k=%u", rmax, N, k);
                    // the fixed 64 MiB block: fits exactly when the sum does
                    const size_t blk = 64ull << 20;
                    // (fb_fits_in sizes the fallback for ids over all N rows: rows = 0)
                    const u128 fb0 = u128(fb_bytes(rmax, N, k));
                    for (size_t need : {size_t(0), size_t(1) << 20, size_t(60) << 20})
                        CHECK(fb_fits_in(blk, need, rmax, N, k) == (u128(need) + fb0 <= blk), "fb_fits_in");
                    CHECK(fb_fits_in(0, size_t(1) << 40, rmax, N, k), "the arena always fits");
                }
            }
    // configs[1] through the allocation-free block: 1024 queries of k = 100 over 1M rows need more
    // than 64 MiB for the fallback's buffers (the entry point then rejects or synchronises)
    {
        const ScanPlan p = plan_scan_for(dense_budget_for(64ull << 20), 0, 0, 1024, 1000000, 100);
        std::printf("configs[1] in the 64 MiB block: scan %zu B, fallback %zu B\n", exact_scan_need(1024, p),
                    fb_bytes(1024, 1000000, 100));
    }

    // IVF
    for (uint32_t n : {0u, 1u, 127u, 128u, 129u, 8191u, 8192u, 8193u, 642000u, 0xFFFFFFFFu}) {
        const uint32_t s = ivf_sample_rows(n);
        CHECK(s <= n && s >= std::min<uint32_t>(n, kIvfSampleMin) && u128(s) * kIvfSampleRate + kIvfSampleRate > n,
              "ivf_sample_rows n=%u s=%u", n, s);
    }
    for (uint32_t k : ks)
        for (uint64_t top : {uint64_t(1), uint64_t(100), uint64_t(65536), uint64_t(1) << 33})
            for (uint64_t oc : opt_cap) {
                const uint64_t c32 = ivf_fp32_cap(oc, k, top), cs = ivf_screen_cap(oc, k, top);
                CHECK(c32 >= 1 && c32 <= top && cs >= 1 && cs <= top, "ivf caps k=%u top=%llu", k, (unsigned long long)top);
                if (!oc) CHECK(cs >= c32, "screen cap below the fp32 cap");
                const uint64_t rc = ivf_rerank_cap(k, cs, top);
                CHECK(rc >= 1 && rc <= top, "ivf rerank cap");
            }
    const uint32_t nqs[] = {1, 16, 17, 32, 33, 64, 65, 128, 129, 1000, 0xFFFFFFFFu};
    const uint32_t nrs[] = {1, 127, 128, 129, 511, 512, 513, 100000, 642000, 0xFFFFFFFFu};
    for (uint32_t nq : nqs)
        for (uint32_t nr : nrs) {
            const int s = shape_for(nq, nr);
            CHECK(s >= 0 && s < kShapes, "shape range");
            // brute force in 128 bits: the first shape of least cost
            u128 best = ~u128(0);
            int bi = -1;
            for (int i = 0; i < kShapes; ++i) {
                const u128 wq = u128(shape_wq(i)), wn = u128(shape_wn(i));
                const u128 c = ((u128(nq) + 32 * wq - 1) / (32 * wq)) * ((u128(nr) + 128 * wn - 1) / (128 * wn)) * wq * wn *
                               shape_cost(i);
                if (c < best) {
                    best = c;
                    bi = i;
                }
            }
            CHECK(s == bi, "shape_for(%u, %u) = %d, brute force %d", nq, nr, s, bi);
            uint32_t TQ, TN;
            group_tile(s, TQ, TN);
            CHECK(TQ == 32u * uint32_t(shape_wq(s)) && TN == 128u * uint32_t(shape_wn(s)), "group_tile");
        }
    uint32_t TQ, TN;
    group_tile(kSmallGroup, TQ, TN);
    CHECK(TQ == kSmallTileQueries && TN == kSmallTileRows, "small group tile");

    std::printf("%llu plans checked\n", (unsigned long long)plans);
    if (failures) {
        std::printf("%d failures\n", failures);
        return 1;
    }
    std::printf("plan_host: %llu plans checked, ok\n", (unsigned long long)plans);
    return 0;
}

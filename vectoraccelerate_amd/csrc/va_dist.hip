// va_dist.hip — fp32 distance GEMM on CDNA4 MFMA (v_mfma_f32_32x32x2_f32).
//
// One kernel computes every Q x N distance family of the search path:
//   dist(q, x) from the contraction q.x and the squared norms |q|^2, |x|^2, where the
//   norms are accumulated on the VALU from the same LDS fragments that feed the MFMA
//   (no separate norm pass over the database).
// Replaces the reference's per-pair scalar loops: l2_distance_kernel
// (Metal/Shaders/L2Distance.metal:34-91), dot_product_kernel (DotProduct.metal:29-96) and the
// distance loop of fused_l2_topk (AdvancedTopK.metal:238-242).
//
// Tile geometry (256 threads = 4 wave64):
//   wave tile      = 32 queries x 128 database rows = 4 MFMA blocks of 32x32, 64 acc/lane
//   workgroup tile = (32*WQ) queries x (128*WN) rows, WQ*WN = 4
//   K loop         = LDS stages of KC=16 d-values, double buffered, one barrier per stage
// MFMA operand map: A = database rows (M), B = queries (N).  The contraction index is
// permuted so one ds_read_b128 per lane feeds four MFMA steps: at step s of an 8-wide
// d-group, lane half h supplies d = d0 + 4h + s for both A and B.
// Output map of a 32x32 block (lane l, acc v): row m = 8*(v/4) + 4*(l/32) + v%4,
// column n = l%32 — so each lane owns ONE query and 64 database rows.
#include <cfloat>

#include <algorithm>

#include "va_distop.hpp"
#include "va_internal.hpp"

namespace va {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int KC = 16;               // d-values per LDS stage
#ifndef VA_DIST_SWZ
#define VA_DIST_SWZ 1
#endif
#ifndef VA_DIST_WPE
#define VA_DIST_WPE 2      // waves per SIMD the register-staged kernel is compiled for
#endif
#ifndef VA_DIST_DMA_WPE
#define VA_DIST_DMA_WPE 4  // ... and the direct-load kernel
#endif
#ifndef VA_DIST_DMA
#define VA_DIST_DMA 1
#endif
#ifndef VA_DIST_DMA_SLOTS
#define VA_DIST_DMA_SLOTS 2  // LDS ring slots of the direct-load kernel (stages in flight + 1)
#endif
#if VA_DIST_SWZ
// 64-byte rows, unpadded: 16-byte chunk c of row r sits at chunk c ^ ((r >> 2) & 3).
// ds_read_b128 / ds_write_b128 serve 16 lanes per clock across 64 banks; the 16 rows of a
// fragment read (and the 4 x 4 chunks of a 16-lane write) land in 16 distinct bank groups.
constexpr int LDS_STRIDE = KC;
__device__ __forceinline__ int lds_chunk(int row, int c) { return c ^ ((row >> 2) & 3); }
#else
constexpr int LDS_STRIDE = KC + 4;   // 80-byte rows: conflict-free ds_read_b128 / ds_write_b128
__device__ __forceinline__ int lds_chunk(int row, int c) { return c; }
#endif

// WQ x WN waves of 64 lanes; each wave owns 32 queries x 128 rows (4 MFMA blocks).
template <int WQ, int WN>
struct Tile {
    static constexpr int NW = WQ * WN;
    static constexpr int NT = 64 * NW;
    static constexpr int TQ = 32 * WQ;
    static constexpr int TN = 128 * WN;
    static constexpr int ROWS = TQ + TN;
    static constexpr int CHUNKS = ROWS * (KC / 4);
    static constexpr int CPT = (CHUNKS + NT - 1) / NT;
    static constexpr int STAGE = ROWS * LDS_STRIDE;
    // register-staged loads: a one-wave tile keeps one LDS stage (the next stage waits in
    // registers), 44 KB instead of 87 KB, so three workgroups share a CU instead of one
    static constexpr int NSTAGE = NW == 1 ? 1 : 2;
    static constexpr size_t LDS_BYTES = size_t(NSTAGE * STAGE + NW * 128) * sizeof(float);
    // direct-to-LDS loads: 16-row groups of 1 KiB (one wave-wide load each), the same number
    // per wave (the last few may be padding), two ring slots
    static constexpr int GROUPS = ROWS / 16;
    static constexpr int GPW = (GROUPS + NW - 1) / NW;
    static constexpr int DSTAGE = GPW * NW * 256;  // floats per slot
    static constexpr size_t DMA_LDS_BYTES = size_t(VA_DIST_DMA_SLOTS * DSTAGE + NW * 128) * sizeof(float);
};

// DMA = true: the stages move global -> LDS by direct buffer loads (no register staging, so
// fewer VGPRs and more waves per SIMD); needs 16-byte rows (VEC) and the swizzled 64-byte LDS
// rows.  DMA = false: register-staged loads, any row alignment.
// One tile: queries qs + i (i < qc; through qrow when given) x database rows at positions
// rs + j (j < rc).  Every wave of the workgroup calls it with the same tile.
// LOOP: called once per iteration of the planned launch's tile loop.  The thread index then goes
// through an opaque move, so that nothing derived from it is hoisted out of the loop and held
// across the whole tile (the main loop has no register to spare).
// (the planned launches are the IVF list scans: L2^2, the distance fixed at compile time)
template <int WQ, int WN, bool VEC, int OUT, bool DMA, bool LOOP = false>
__device__ __forceinline__ void dist_tile(const DistArgs& a, uint32_t qs, uint32_t qc, uint32_t rs, uint32_t rc) {
    const int op = LOOP ? int(OP_L2SQ) : int(a.op);
    using T = Tile<WQ, WN>;
    extern __shared__ float lds[];
    float* nrm = lds + (DMA ? VA_DIST_DMA_SLOTS * T::DSTAGE : T::NSTAGE * T::STAGE);  // [waves][128] squared norms of the wave's rows

    int tid = int(threadIdx.x);
    if constexpr (LOOP) asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"(tid));
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wq = wave % WQ;
    const int wn = wave / WQ;
    const int l32 = lane & 31;
    const int hh = lane >> 5;

    f32x16 acc[4];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[b][v] = 0.0f;
    float qss = 0.0f;
    float xss[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // fragment rows start at multiples of 32, so every fragment row shares l32's chunk swizzle
    const int boff = (wq * 32 + l32) * LDS_STRIDE;
    const int aoff = (T::TQ + wn * 128 + l32) * LDS_STRIDE;
    int koff[KC / 8];
#pragma unroll
    for (int g = 0; g < KC / 8; ++g) koff[g] = 4 * lds_chunk(l32, 2 * g + hh);
    // one 16-value stage of MFMAs from an LDS slot; norms accumulate from the same fragments
    auto compute = [&](const float* st) {
#pragma unroll
        for (int g = 0; g < KC / 8; ++g) {
            const f32x4v bv = *reinterpret_cast<const f32x4v*>(st + boff + koff[g]);
            qss = fmaf(bv[0], bv[0], qss);
            qss = fmaf(bv[1], bv[1], qss);
            qss = fmaf(bv[2], bv[2], qss);
            qss = fmaf(bv[3], bv[3], qss);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const f32x4v av = *reinterpret_cast<const f32x4v*>(st + aoff + b * 32 * LDS_STRIDE + koff[g]);
                xss[b] = fmaf(av[0], av[0], xss[b]);
                xss[b] = fmaf(av[1], av[1], xss[b]);
                xss[b] = fmaf(av[2], av[2], xss[b]);
                xss[b] = fmaf(av[3], av[3], xss[b]);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[0], bv[0], acc[b], 0, 0, 0);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[1], bv[1], acc[b], 0, 0, 0);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[2], bv[2], acc[b], 0, 0, 0);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[3], bv[3], acc[b], 0, 0, 0);
            }
        }
    };
    const int nstages = int((a.D + KC - 1) / KC);
    if constexpr (DMA) {
        // 16-row group gi of a slot is rows 16*gi .. 16*gi+15 (queries first, then database
        // rows); lane L loads row 16*gi + L/4, physical chunk L%4 = logical chunk
        // (L%4) ^ swizzle(row).  Rows outside the tile and columns past D load from an offset
        // past the descriptor and land as zeros.
        // every offset below addresses a real row (checked by the launcher to stay under
        // kDmaMaxBytes), so the descriptors only need to bound kDmaSkip
        const dma_rsrc qres = make_dma_rsrc(a.q, kDmaMaxBytes);
        const dma_rsrc xres = make_dma_rsrc(a.x + int64_t(rs) * a.ldx, kDmaMaxBytes);
        uint32_t base[T::GPW], colb[T::GPW];
#pragma unroll
        for (int i = 0; i < T::GPW; ++i) {
            const int row = 16 * (wave + T::NW * i) + (lane >> 2);
            const int c = lds_chunk(row, lane & 3);
            colb[i] = uint32_t(4 * c);
            base[i] = kDmaSkip;
            if (row < T::TQ) {
                if (uint32_t(row) < qc) {
                    const uint32_t r = a.qrow ? a.qrow[qs + row] : qs + row;
                    base[i] = uint32_t(int64_t(r) * a.ldq * 4) + 16u * uint32_t(c);
                }
            } else if (row < T::ROWS) {
                const uint32_t jr = uint32_t(row - T::TQ);
                if (jr < rc) base[i] = uint32_t(int64_t(jr) * a.ldx * 4) + 16u * uint32_t(c);
            }
        }
        const uint32_t lds0 = lds_addr_of(lds);
        auto issue = [&](uint32_t d0, int slot) {
#pragma unroll
            for (int i = 0; i < T::GPW; ++i) {
                const uint32_t voff = (base[i] != kDmaSkip && d0 + colb[i] < a.D) ? base[i] + d0 * 4u : kDmaSkip;
                const int grp = wave + T::NW * i;
                lds_dma16(16 * grp < T::TQ ? qres : xres, voff,
                          lds0 + uint32_t(slot * T::DSTAGE + grp * 256) * 4u);
            }
        };
        if constexpr (VA_DIST_DMA_SLOTS == 2) {
            issue(0, 0);
            wait_vmcnt<0>();
            __syncthreads();
            for (int s = 0; s < nstages; ++s) {
                const bool more = (s + 1) < nstages;
                if (more) issue(uint32_t(s + 1) * KC, (s + 1) & 1);  // slot last read before the previous barrier
                compute(lds + (s & 1) * T::DSTAGE);
                if (more) wait_vmcnt<0>();
                __syncthreads();
            }
        } else {
            // three slots: stage s+2 loads while stage s computes
            issue(0, 0);
            if (nstages > 1) issue(KC, 1);
            int slot = 0;
            for (int s = 0; s < nstages; ++s) {
                if (s + 1 < nstages) wait_vmcnt<T::GPW>();
                else wait_vmcnt<0>();
                __syncthreads();  // stage s visible; every wave is past the reads of slot (s + 2) % 3
                if (s + 2 < nstages) issue(uint32_t(s + 2) * KC, slot == 0 ? 2 : slot - 1);
                compute(lds + slot * T::DSTAGE);
                slot = slot == 2 ? 0 : slot + 1;
            }
            __syncthreads();  // the epilogue reuses LDS only after every wave's last reads
        }
    } else {
        // source row pointers of this thread's load chunks (fixed across stages)
        const float* src[T::CPT];
        int ldsoff[T::CPT];
        uint32_t colv[T::CPT];
#pragma unroll
        for (int j = 0; j < T::CPT; ++j) {
            const int c = tid + T::NT * j;
            src[j] = nullptr;
            ldsoff[j] = -1;
            colv[j] = 0;
            if (c < T::CHUNKS) {
                const int row = c >> 2;
                const int col = (c & 3) * 4;
                ldsoff[j] = row * LDS_STRIDE + 4 * lds_chunk(row, col / 4);
                colv[j] = uint32_t(col);
                if (row < T::TQ) {
                    if (uint32_t(row) < qc) {
                        const uint32_t r = a.qrow ? a.qrow[qs + row] : qs + row;
                        src[j] = a.q + int64_t(r) * a.ldq + col;
                    }
                } else {
                    const uint32_t jr = uint32_t(row - T::TQ);
                    if (jr < rc) {
                        const int64_t xr = a.gather ? int64_t(a.gather[int64_t(qs) * a.gcap + rs + jr])
                                                    : int64_t(rs + jr);
                        src[j] = a.x + xr * a.ldx + col;
                    }
                }
            }
        }

        f32x4v pre[T::CPT];
        auto load = [&](uint32_t d0) {
#pragma unroll
            for (int j = 0; j < T::CPT; ++j) {
                f32x4v v = {0.0f, 0.0f, 0.0f, 0.0f};
                const uint32_t d = d0 + colv[j];
                if (src[j]) {
                    if (VEC) {
                        if (d < a.D) v = *reinterpret_cast<const f32x4v*>(src[j] + d0);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (d + e < a.D) v[e] = src[j][d0 + e];
                    }
                }
                pre[j] = v;
            }
        };
        auto store = [&](float* stage) {
#pragma unroll
            for (int j = 0; j < T::CPT; ++j)
                if (ldsoff[j] >= 0) *reinterpret_cast<f32x4v*>(stage + ldsoff[j]) = pre[j];
        };

        load(0);
        store(lds);
        __syncthreads();
        for (int s = 0; s < nstages; ++s) {
            const bool more = (s + 1) < nstages;
            if (more) load(uint32_t(s + 1) * KC);
            if constexpr (T::NSTAGE == 1) {
                compute(lds);
                __syncthreads();  // every read of the stage is done before it is overwritten
                if (more) store(lds);
            } else {
                compute(lds + (s & 1) * T::STAGE);
                if (more) store(lds + ((s + 1) & 1) * T::STAGE);
            }
            __syncthreads();
        }
    }

    // combine the two lane halves of every partial sum of squares
    const float qq = qss + __shfl_xor(qss, 32);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const float t = xss[b] + __shfl_xor(xss[b], 32);
        if (hh == 0) nrm[wave * 128 + b * 32 + l32] = t;
    }
    __syncthreads();

    const uint32_t li = uint32_t(wq * 32 + l32);  // query slot of this lane in the tile
    if (li >= qc) return;
    const uint32_t orow = qs + li;                                   // dense output row
    if (OUT == OUT_ARGMIN) {
        // the lane's 64 rows in increasing id order, strict < : ties keep the lower row id; the two
        // lane halves hold the same query and the other rows of each 8-row group
        uint32_t bk = 0xFFFFFFFFu, bi = 0xFFFFFFFFu;
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int mloc = b * 32 + 8 * j + 4 * hh;
                const f32x4v xx = *reinterpret_cast<const f32x4v*>(nrm + wave * 128 + mloc);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t r = uint32_t(wn * 128 + mloc + e);
                    const uint32_t key = key_of_float(apply_op(op, acc[b][4 * j + e], qq, xx[e]));
                    if (r < rc && key < bk && key < 0xFFFFFFFEu) {  // NaN distances never win
                        bk = key;
                        bi = rs + r;
                    }
                }
            }
        unsigned long long best = (static_cast<unsigned long long>(bk) << 32) | bi;
        const unsigned long long other =
            (static_cast<unsigned long long>(uint32_t(__shfl_xor(int(bk), 32))) << 32) | uint32_t(__shfl_xor(int(bi), 32));
        best = other < best ? other : best;
        if (hh == 0 && best != ~0ull) atomicMin(a.best + orow, best);
        return;
    }
    const uint32_t qi = (OUT == OUT_FILTER && a.qrow) ? a.qrow[orow] : orow;  // query id (filter)
    if (OUT == OUT_FILTER) {
        const uint32_t thr = a.thr[qi];
        // Keys of passing values are reserved with one atomic and written; the direct-load
        // kernel does this for half of the lane's 64 values at a time, which keeps its
        // epilogue within the main loop's 128-VGPR budget (4 waves per SIMD).
        constexpr int HALVES = DMA ? 2 : 1;
        constexpr int NB = 4 / HALVES;  // MFMA blocks per half
#pragma unroll
        for (int h = 0; h < HALVES; ++h) {
            uint64_t pass = 0;  // bit 16(b - NB h) + 4j + e
            uint32_t keys[16 * NB];
#pragma unroll
            for (int bb = 0; bb < NB; ++bb)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int b = NB * h + bb;
                    const int mloc = b * 32 + 8 * j + 4 * hh;
                    const f32x4v xx = *reinterpret_cast<const f32x4v*>(nrm + wave * 128 + mloc);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t key = key_of_float(apply_op(op, acc[b][4 * j + e], qq, xx[e]));
                        keys[16 * bb + 4 * j + e] = key;
                        const bool p = (uint32_t(wn * 128 + mloc + e) < rc) & (key <= thr);
                        pass |= uint64_t(p) << (16 * bb + 4 * j + e);
                    }
                }
            if (!pass) continue;
            uint32_t pos = atomicAdd(a.cnt + qi, uint32_t(__popcll(pass)));
#pragma unroll
            for (int t = 0; t < 16 * NB; ++t) {
                if (!((pass >> t) & 1)) continue;
                if (pos < a.cap) {
                    const int b = NB * h + (t >> 4), j = (t >> 2) & 3, e = t & 3;
                    const uint32_t p = rs + uint32_t(wn * 128 + b * 32 + 8 * j + 4 * hh + e);
                    const int64_t o = int64_t(qi) * a.cap + pos;
                    a.cand_key[o] = keys[t];
                    a.cand_id[o] = a.ids ? a.ids[p] : a.id_base + p;
                }
                ++pos;
            }
        }
        return;
    }

#pragma unroll
    for (int b = 0; b < 4; ++b) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int mloc = b * 32 + 8 * j + 4 * hh;
            const f32x4v xx = *reinterpret_cast<const f32x4v*>(nrm + wave * 128 + mloc);
            float val[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) val[e] = apply_op(op, acc[b][4 * j + e], qq, xx[e]);
            const uint32_t jr = uint32_t(wn * 128 + mloc);  // row slot of acc element e = 0
            if (OUT == OUT_KEYS) {
                uint32_t* o = a.out_k + int64_t(orow) * a.ldo + rs + jr;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (jr + e < rc) o[e] = key_of_float(val[e]);
            } else {
                float* o = a.out_f + int64_t(orow) * a.ldo + rs + jr;
                if (jr + 3 < rc && ((a.ldo & 3) == 0) && ((reinterpret_cast<uintptr_t>(o) & 15) == 0)) {
                    f32x4v w = {val[0], val[1], val[2], val[3]};
                    *reinterpret_cast<f32x4v*>(o) = w;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (jr + e < rc) o[e] = val[e];
                }
            }
        }
    }
}

// PLAN: a device-planned list-major launch (a.plan): a fixed grid loops over the tiles of the
// plan, each decoded from the plan's per-list tile counts.
template <int WQ, int WN, bool VEC, int OUT, bool DMA, bool PLAN>
__global__ __launch_bounds__(64 * WQ * WN, DMA ? VA_DIST_DMA_WPE : VA_DIST_WPE) void dist_gemm_kernel(DistArgs a) {
    using T = Tile<WQ, WN>;
    static_assert(!DMA || (VEC && LDS_STRIDE == KC), "direct loads need 16-byte rows and unpadded LDS rows");
    if constexpr (PLAN) {
        const uint32_t total = a.plan.pre[a.plan.C];
        for (uint32_t t = blockIdx.x; t < total; t += gridDim.x) {
            uint32_t qs, qc, rs, rc;
            plan_tile(a.plan, t, uint32_t(T::TQ), uint32_t(T::TN), qs, qc, rs, rc);
            dist_tile<WQ, WN, VEC, OUT, DMA, true>(a, qs, qc, rs, rc);
            __syncthreads();  // the tile's LDS is read to the end before the next tile's loads
        }
        return;
    } else {
        // XCD-aware order: workgroup w runs on XCD w % 8.  XCD x takes database tiles x, x+8, ...
        // and runs every query block of a tile back to back, so each tile crosses the fabric once
        // and is reused from that XCD's L2 (the grid is padded to a multiple of 8 tiles).
        const uint32_t nqb = a.gather ? 1u : (a.Q + T::TQ - 1) / T::TQ;
        const uint32_t xcd = blockIdx.x % kXcds, seq = blockIdx.x / kXcds;
        const uint32_t qb = seq % nqb;
        const uint32_t tb = (seq / nqb) * kXcds + xcd;
        if (!a.gather && tb * uint32_t(T::TN) >= a.N) return;  // padding workgroup
        // Tile extent.  Flat launches derive it from blockIdx; gather launches take one query and
        // up to 128 rows of its gather list.
        uint32_t qs = qb * T::TQ, rs = tb * T::TN, qc, rc;
        if (a.gather) {
            qs = blockIdx.x / a.gtiles;
            rs = (blockIdx.x % a.gtiles) * uint32_t(T::TN);
            const uint32_t m = min(a.gcount[qs], a.gcap);
            if (rs >= m) return;  // empty tile (uniform)
            qc = 1;
            rc = min(uint32_t(T::TN), m - rs);
        } else {
            qc = min(uint32_t(T::TQ), a.Q - qs);
            rc = min(uint32_t(T::TN), a.N - rs);
        }
        dist_tile<WQ, WN, VEC, OUT, DMA>(a, qs, qc, rs, rc);
    }
}

template <int WQ, int WN, bool VEC, int OUT, bool DMA, bool PLAN = false>
va_status launch_tile(va_context* ctx, const DistArgs& a) {
    using T = Tile<WQ, WN>;
    const uint64_t nqb = (a.Q + T::TQ - 1) / T::TQ;
    const uint64_t ntb = (a.N + T::TN - 1) / T::TN;
    const uint64_t grid = PLAN ? a.plan.grid
                          : a.gather ? uint64_t(a.Q) * a.gtiles : nqb * ((ntb + kXcds - 1) / kXcds) * kXcds;
    if (grid == 0) return VA_OK;
    if (grid > 0x7FFFFFFFull) return fail(ctx, VA_ERR_INVALID_ARG, "distance grid too large (%llu tiles)", (unsigned long long)grid);
    auto kern = &dist_gemm_kernel<WQ, WN, VEC, OUT, DMA, PLAN>;
    const size_t lds_bytes = DMA ? T::DMA_LDS_BYTES : T::LDS_BYTES;
    if (lds_bytes > 65536) {
        VA_CHECK_HIP(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes)));
    }
    kern<<<dim3(uint32_t(grid)), dim3(T::NT), lds_bytes, ctx->stream>>>(a);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

// Direct loads address rows through 32-bit offsets below kDmaMaxBytes: every query row the
// launch can name, and every row of one tile relative to the tile's first row.
template <int WQ, int WN>
bool dma_fits(const DistArgs& a, bool vec) {
    if (!VA_DIST_DMA || !vec || LDS_STRIDE != KC) return false;
    const uint64_t qrows = a.qrow ? a.q_rows : a.Q;
    if (qrows == 0) return false;
    const uint64_t tn = a.plan.pre ? Tile<WQ, WN>::TN : std::min<uint64_t>(Tile<WQ, WN>::TN, a.N);
    return (qrows - 1) * uint64_t(a.ldq) * 4 + uint64_t(a.D) * 4 <= kDmaMaxBytes &&
           (tn - 1) * uint64_t(a.ldx) * 4 + uint64_t(a.D) * 4 <= kDmaMaxBytes;
}

template <int WQ, int WN, int OUT>
va_status launch_shape(va_context* ctx, const DistArgs& a, bool vec) {
    if (a.plan.pre) {
        if constexpr (OUT == OUT_FILTER) {
            if constexpr (LDS_STRIDE == KC)
                if (dma_fits<WQ, WN>(a, vec)) return launch_tile<WQ, WN, true, OUT, true, true>(ctx, a);
            return vec ? launch_tile<WQ, WN, true, OUT, false, true>(ctx, a)
                       : launch_tile<WQ, WN, false, OUT, false, true>(ctx, a);
        }
        return fail(ctx, VA_ERR_INVALID_ARG, "launch_dist: planned launches are filter launches");
    }
    if constexpr (LDS_STRIDE == KC)
        if (dma_fits<WQ, WN>(a, vec)) return launch_tile<WQ, WN, true, OUT, true>(ctx, a);
    return vec ? launch_tile<WQ, WN, true, OUT, false>(ctx, a) : launch_tile<WQ, WN, false, OUT, false>(ctx, a);
}

}  // namespace

va_status launch_dist(va_context* ctx, const DistArgs& a) {
    if (a.plan.pre ? a.plan.grid == 0 : (a.Q == 0 || a.N == 0)) return VA_OK;
    const bool vec = (a.D % 4 == 0) && (a.ldq % 4 == 0) && (a.ldx % 4 == 0) &&
                     ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) && ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0);
    if (a.gather) {
        // rows come from anywhere in the database (64-bit addresses): register-staged loads
        if (a.out != OUT_KEYS || a.plan.pre || a.qrow || a.gtiles == 0 || a.gcap == 0 || !a.gcount)
            return fail(ctx, VA_ERR_INVALID_ARG, "launch_dist: malformed gather launch");
        return vec ? launch_tile<1, 1, true, OUT_KEYS, false>(ctx, a) : launch_tile<1, 1, false, OUT_KEYS, false>(ctx, a);
    }
    const int wq = a.wq ? a.wq : (a.Q <= 32 ? 1 : (a.Q <= 64 ? 2 : 4));
    const int wn = a.wn ? a.wn : 4 / wq;
#define VA_DIST_CASE(W, N, O) \
    if (wq == W && wn == N && a.out == O) return launch_shape<W, N, O>(ctx, a, vec);
    VA_DIST_CASE(1, 4, OUT_VALUES) VA_DIST_CASE(1, 4, OUT_KEYS) VA_DIST_CASE(1, 4, OUT_FILTER)
    VA_DIST_CASE(2, 2, OUT_VALUES) VA_DIST_CASE(2, 2, OUT_KEYS) VA_DIST_CASE(2, 2, OUT_FILTER)
    VA_DIST_CASE(4, 1, OUT_VALUES) VA_DIST_CASE(4, 1, OUT_KEYS) VA_DIST_CASE(4, 1, OUT_FILTER)
    VA_DIST_CASE(1, 4, OUT_ARGMIN) VA_DIST_CASE(2, 2, OUT_ARGMIN) VA_DIST_CASE(4, 1, OUT_ARGMIN)
    // small list-major tiles (one or two waves) for sparse IVF work
    VA_DIST_CASE(1, 1, OUT_FILTER) VA_DIST_CASE(2, 1, OUT_FILTER)
#undef VA_DIST_CASE
    return fail(ctx, VA_ERR_INVALID_ARG, "launch_dist: no %dx%d tile for output mode %d", wq, wn, int(a.out));
}

}  // namespace va

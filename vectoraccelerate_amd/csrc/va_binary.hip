// va_binary.hip — binary (sign-bit) quantization and Hamming scan on CDNA4.
//
//   pack : bit d = (x_d > 0), word w bit b = dimension 32w+b (binaryQuantize,
//          Metal/Shaders/QuantizationShaders.metal:132-160).  One wave per row; each lane reads
//          one float and __ballot turns 64 consecutive dimensions into two words, so every
//          load is a fully coalesced 256-byte wave access (the reference's shader has one
//          thread per vector striding through the row, and no bounds guard).
//   scan : Hamming distance sum(popcount(q ^ x)) with v_xor + v_bcnt (accumulating popcount)
//          on the VALU.  One database row per lane, held in VGPRs (128-bit loads); the query
//          words are wave-uniform and come through scalar loads, so each (query, row) pair
//          costs 2 VALU ops per 32-bit word.  Feeds the shared exact top-k driver with the
//          distance itself as the key (ties -> lower index, HammingDistanceKernel.swift:114-120).
#include <algorithm>

#include "va_fallback.hpp"
#include "va_internal.hpp"

namespace va {
namespace {

constexpr uint32_t kMaxWords = 32;  // register-resident rows up to D = 1024

__global__ __launch_bounds__(256) void pack_kernel(const float* __restrict__ x, uint32_t N, uint32_t D, uint32_t W,
                                                   uint32_t* __restrict__ codes) {
    const int lane = threadIdx.x & 63;
    const uint32_t waves = gridDim.x * 4;
    for (uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6); r < N; r += waves) {
        const float* row = x + uint64_t(r) * D;
        uint32_t* out = codes + uint64_t(r) * W;
        for (uint32_t c = 0; c * 64 < D; ++c) {
            const uint32_t d = c * 64 + uint32_t(lane);
            const bool bit = (d < D) && (row[d] > 0.0f);
            const uint64_t m = __ballot(bit);
            if (lane == 0) {
                out[2 * c] = uint32_t(m);
                if (2 * c + 1 < W) out[2 * c + 1] = uint32_t(m >> 32);
            }
        }
    }
}

__global__ __launch_bounds__(256) void hamming_matrix_kernel(const uint32_t* __restrict__ q,
                                                             const uint32_t* __restrict__ x, uint32_t N, uint32_t W,
                                                             uint32_t* __restrict__ out) {
    const uint32_t qi = blockIdx.y;
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    if (j >= N) return;
    const uint32_t* qw = q + uint64_t(qi) * W;
    const uint32_t* xw = x + uint64_t(j) * W;
    uint32_t d = 0;
    for (uint32_t w = 0; w < W; ++w) d += __popc(qw[w] ^ xw[w]);
    out[uint64_t(qi) * N + j] = d;
}

struct HamArgs {
    const uint32_t* q = nullptr;
    const uint32_t* qrow = nullptr;  // optional query indirection
    uint32_t q0 = 0, nq = 0;
    const uint32_t* x = nullptr;
    uint32_t c0 = 0, cols = 0, stride = 1;  // rows c0 + j*stride, j < cols
    uint32_t W = 0;
    uint32_t* out_k = nullptr;
    int64_t ldo = 0;
    const uint32_t* thr = nullptr;
    uint32_t* cnt = nullptr;
    uint32_t* cand_key = nullptr;
    uint32_t* cand_id = nullptr;
    uint32_t cap = 0;
};

// wave-uniform word load through the scalar data cache (read-only constant address space)
__device__ __forceinline__ uint32_t uniform_load(const uint32_t* p) {
    return *(const __attribute__((address_space(4))) uint32_t*)(p);
}

// WC > 0: compile-time word count (fully unrolled; query words arrive in wide scalar loads);
// WC = 0: any W <= kMaxWords.
template <int WC, bool FILTER>
__global__ __launch_bounds__(256) void hamming_scan_kernel(HamArgs a) {
    constexpr uint32_t WR = WC > 0 ? uint32_t(WC) : kMaxWords;
    const uint32_t W = WC > 0 ? uint32_t(WC) : a.W;
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    const bool valid = j < a.cols;
    const uint32_t row = a.c0 + (valid ? j : 0) * a.stride;
    // the row, word by word, in VGPRs (uint4 loads; rows are 16-byte aligned when W % 4 == 0)
    uint32_t xr[WR];
    const uint32_t* xp = a.x + uint64_t(row) * W;
    if ((W & 3) == 0) {
#pragma unroll
        for (uint32_t w = 0; w < WR; w += 4) {
            if (w < W) {
                const uint4 v = *reinterpret_cast<const uint4*>(xp + w);
                xr[w] = v.x;
                xr[w + 1] = v.y;
                xr[w + 2] = v.z;
                xr[w + 3] = v.w;
            }
        }
    } else {
#pragma unroll
        for (uint32_t w = 0; w < WR; ++w)
            if (w < W) xr[w] = xp[w];
    }
#pragma unroll 2
    for (uint32_t i = 0; i < a.nq; ++i) {
        const uint32_t qr = a.qrow ? uniform_load(a.qrow + i) : a.q0 + i;
        const uint32_t* qw = a.q + uint64_t(qr) * W;
        uint32_t d = 0;
#pragma unroll
        for (uint32_t w = 0; w < WR; ++w)
            if (w < W) d += __popc(xr[w] ^ uniform_load(qw + w));
        if (!valid) continue;
        if (FILTER) {
            const uint32_t qi = a.q0 + i;
            if (d <= uniform_load(a.thr + qi)) {
                const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
                if (pos < a.cap) {
                    const int64_t o = int64_t(qi) * a.cap + pos;
                    a.cand_key[o] = d;
                    a.cand_id[o] = row;
                }
            }
        } else {
            a.out_k[int64_t(i) * a.ldo + j] = d;
        }
    }
}

// rows longer than kMaxWords words: the row is re-read from L1/L2 for every query
template <bool FILTER>
__global__ __launch_bounds__(256) void hamming_scan_wide_kernel(HamArgs a) {
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    if (j >= a.cols) return;
    const uint32_t row = a.c0 + j * a.stride;
    const uint32_t* xp = a.x + uint64_t(row) * a.W;
    for (uint32_t i = 0; i < a.nq; ++i) {
        const uint32_t qr = a.qrow ? a.qrow[i] : a.q0 + i;
        const uint32_t* qw = a.q + uint64_t(qr) * a.W;
        uint32_t d = 0;
        for (uint32_t w = 0; w < a.W; ++w) d += __popc(xp[w] ^ qw[w]);
        if (FILTER) {
            const uint32_t qi = a.q0 + i;
            if (d <= a.thr[qi]) {
                const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
                if (pos < a.cap) {
                    const int64_t o = int64_t(qi) * a.cap + pos;
                    a.cand_key[o] = d;
                    a.cand_id[o] = row;
                }
            }
        } else {
            a.out_k[int64_t(i) * a.ldo + j] = d;
        }
    }
}

// ---------------------------------------------------------------------------------------
// Filter scan on the fp4 MFMA (large Q, rows of 8/16/24 words)
// ---------------------------------------------------------------------------------------
// Hamming distance as |a| + |b| - 2 a.b over {0,1} vectors: a.b is a dot product of bits,
// which the gfx950 matrix cores compute exactly with every bit widened to an fp4 (e2m1)
// value 0 or a power of two whose products with the other side's are 1.0
// (v_mfma_scale_f32_32x32x64_f8f6f4, unit scales, fp32 sums of integers <= 1024).  fp4 runs the 32x32x64 MFMA at 8 dense TFLOP/s-equivalents per CU per clock pair
// of the int8 rate, so the 2·Q·N·32W bit products cost a fraction of the xor + popcount
// VALU scan, which is bound by VALU issue (two ops per word per pair).
// Layout and pipeline follow i8_resq_kernel: a workgroup keeps 256 queries resident in LDS
// (already widened: 16 bytes per 32-bit word, rows padded to 16W + 16 bytes, which puts the
// 16 rows of one ds_read_b128 clock in 16 distinct bank groups) and streams a contiguous range
// of 256-row tiles past them; each of its eight waves owns 32 rows of a tile and loads them
// straight into registers (lane: row l % 32, half h = l / 32 of its words, 16-byte loads;
// the next tile in flight while this one computes), widens one 32-bit word per k-step into
// the A fragment and runs 8 MFMAs against the 8 resident query blocks.  K mapping: k-step s
// takes word h·W/2 + s of the half, widened by the same bit-to-slot assignment on both sides
// (widen_row, widen_query).  No workgroup barrier after the query load.  Filter epilogue as in
// i8_resq_kernel: a pass is d <= tau, tested in the form 512 + a.b - |x|/2 >= 512 + (|q| -
// tau)/2 with the accumulators started from 512 - |x|/2, a per-lane maximum first; passes go to
// a per-wave LDS list flushed when full.
namespace hmf {
constexpr int TQ = 256, NW = 8, WR = 32, TN = NW * WR, LCAP = 80;
constexpr int STAGE = NW * LCAP * 12;
constexpr int PA = NW * WR * 4;  // per-wave row popcounts
constexpr int PB = TQ * 4;       // query popcounts
// resident queries, chunk-major: 16-byte chunk c (of W) of query r at c * 4096 + r * 16, so the
// fragments of all 8 query blocks of one k-step lie within a 16-bit DS offset of one address
constexpr int qbytes(int W) { return TQ * 16 * W; }
constexpr int rows_bytes(int W) { return NW * WR * (W + 1) * 4; }  // per-wave row words, rows W + 1 apart
constexpr size_t lds_bytes(int W) { return size_t(qbytes(W)) + STAGE + PA + PB + rows_bytes(W); }
}  // namespace hmf

// 32 bits -> 32 fp4 (e2m1) nibbles in four dwords: nibble i of dword j holds bit 4i + j of the
// word.  A dot product does not depend on which k slot a bit goes to as long as rows and queries
// use the same assignment, nor on how a set bit's value splits between the two sides as long as
// every product is 1.  A row bit stays where the mask finds it: nibble bit 0, 1 or 2 is e2m1 0.5,
// 1.0 or 2.0 (bit 3 is the sign, so bit 4i + 3 moves down one place): five VALU ops per word,
// which matters because this scan's VALU work adds to its MFMA time.  The query side (widened
// once, at load) carries the reciprocal weights 2.0, 1.0, 0.5, 0.5.
__device__ __forceinline__ uint4 widen_row(uint32_t w) {
    return {w & 0x11111111u, w & 0x22222222u, w & 0x44444444u, (w >> 1) & 0x44444444u};
}
__device__ __forceinline__ uint4 widen_query(uint32_t w) {
    return {(w << 2) & 0x44444444u, w & 0x22222222u, (w >> 2) & 0x11111111u, (w >> 3) & 0x11111111u};
}

typedef int i32x8h __attribute__((ext_vector_type(8)));
typedef int i32x4h __attribute__((ext_vector_type(4)));
// an fp4 MFMA operand: the instruction reads the first four registers of the eight
__device__ __forceinline__ i32x8h fp4_operand(const i32x4h& v) { return i32x8h{v[0], v[1], v[2], v[3], 0, 0, 0, 0}; }
typedef float f32x16h __attribute__((ext_vector_type(16)));
typedef float f32x4h __attribute__((ext_vector_type(4)));

template <int W>
__global__ __launch_bounds__(512, 2) void hamming_mfma_kernel(HamArgs a, uint32_t R) {
    using namespace hmf;
    constexpr int HW = W / 2;  // words per lane half = k-steps per tile
    constexpr int QB = qbytes(W);
    extern __shared__ __attribute__((aligned(16))) char lds8[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, hh = lane >> 5;
    const uint32_t Q = a.nq, N = a.cols;

    const uint32_t nqb = (Q + TQ - 1) / TQ;
    const uint32_t xcd = blockIdx.x % kXcds, seq = blockIdx.x / kXcds;
    const uint32_t qb = seq % nqb;
    const uint32_t range = (seq / nqb) * kXcds + xcd;
    const uint32_t ntiles = (N + TN - 1) / TN;
    const uint32_t tpr = (ntiles + R - 1) / R;
    const uint32_t t0 = range * tpr;
    if (t0 >= ntiles) return;  // the whole workgroup: no range left
    const uint32_t tcount = min(tpr, ntiles - t0);
    const uint32_t q0 = qb * TQ;
    const uint32_t qn = min(uint32_t(TQ), Q - q0);

    float* s_pa = reinterpret_cast<float*>(lds8 + QB + STAGE) + wave * WR;
    float* s_pb = reinterpret_cast<float*>(lds8 + QB + STAGE + PA);
    uint32_t* s_rw = reinterpret_cast<uint32_t*>(lds8 + QB + STAGE + PA + PB) + wave * WR * (W + 1);
    // resident queries, widened: word w of query r -> chunk 2 (w % HW) + w / HW
    for (int e = tid; e < TQ * W; e += 512) {
        const int r = e / W, w = e % W;
        const uint32_t v = uint32_t(r) < qn ? a.q[uint64_t(q0 + r) * W + w] : 0u;
        const int c = 2 * (w % HW) + w / HW;
        *reinterpret_cast<uint4*>(lds8 + c * 4096 + r * 16) = widen_query(v);
    }
    for (int r = tid; r < TQ; r += 512) {
        uint32_t pb = 0;
        if (uint32_t(r) < qn)
            for (int w = 0; w < W; ++w) pb += __popc(a.q[uint64_t(q0 + r) * W + w]);
        s_pb[r] = float(pb);
    }
    __syncthreads();  // resident queries visible; the only workgroup barrier
    // pass iff 2 a.b - |x| >= |q| - tau, i.e. 512 + a.b - |x|/2 >= 512 + (|q| - tau)/2 (halves of
    // integers below 2^24: exact).  The accumulators start from 512 - |x|/2, so the left side is
    // what they hold, and every value on either side is a positive float (|x|, |q|, tau <= 32 W
    // <= 768), whose bit patterns order like the values: the quick test is an unsigned maximum.
    // tau >= 32 W passes everything (0); padding never passes (+inf)
    float cq[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const uint32_t ql = uint32_t(u * 32 + l32);
        const uint32_t t = a.thr[q0 + (ql < qn ? ql : 0u)];
        cq[u] = ql >= qn ? __builtin_inff() : (t >= uint32_t(32 * W) ? 0.0f : 512.0f + 0.5f * (s_pb[ql] - float(t)));
    }

    // ---- this wave's rows -------------------------------------------------------------------
    // lane: row l32 of the wave's 32, words [hh HW, hh HW + HW); rows past N read as zeros
    auto load_tile = [&](uint32_t lt, uint32_t (&xw)[HW]) {
        const uint64_t r0 = uint64_t(t0 + lt) * TN + uint32_t(wave) * WR;
        const uint32_t rows = r0 < N ? uint32_t(min(uint64_t(WR), uint64_t(N) - r0)) : 0u;
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint32_t*>(a.x + r0 * W), 0, int(rows * uint32_t(W) * 4u), 0x00020000);
        const uint32_t off = (uint32_t(l32) * W + uint32_t(hh) * HW) * 4u;
#pragma unroll
        for (int i = 0; i < HW / 4; ++i) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16u * i, 0, 0);
            xw[4 * i] = uint32_t(v[0]);
            xw[4 * i + 1] = uint32_t(v[1]);
            xw[4 * i + 2] = uint32_t(v[2]);
            xw[4 * i + 3] = uint32_t(v[3]);
        }
    };
    const char* qrd = lds8 + hh * 4096 + l32 * 16;
    // The query fragments are the same for every tile; an opaque per-tile zero in their
    // address keeps the compiler from hoisting all 8 x W/2 of them out of the tile loop into
    // registers (it would spill them).
    uint32_t qz = 0;
    auto rd_q = [&](int st, int u) { return *reinterpret_cast<const i32x4h*>(qrd + qz + st * 8192 + u * 512); };

    // ---- filter epilogue ------------------------------------------------------------------
    uint32_t* s_qi = reinterpret_cast<uint32_t*>(lds8 + QB) + wave * 3 * LCAP;
    uint32_t* s_key = s_qi + LCAP;
    uint32_t* s_id = s_key + LCAP;
    uint32_t lc = 0;  // staged passes (wave-uniform)
    auto flush = [&]() {
        for (uint32_t b0 = 0; b0 < lc; b0 += 64) {
            const uint32_t e = b0 + uint32_t(lane);
            if (e < lc) {
                const uint32_t qi = s_qi[e];
                const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
                if (pos < a.cap) {
                    a.cand_key[int64_t(qi) * a.cap + pos] = s_key[e];
                    a.cand_id[int64_t(qi) * a.cap + pos] = s_id[e];
                }
            }
        }
        lc = 0;
    };
    f32x16h acc[8];
    // Lane value v of a block is row 8 (v >> 2) + 4 hh + (v & 3) of the wave's 32; it holds
    // 512 + a.b - |x|/2 at the end of a tile.  The passes of block u of a tile whose first row id is
    // r0 and whose rows past N start at lim (this lane half's view) go to the staging list.
    auto block_passes = [&](int u, uint32_t r0, int32_t lim) {
        const float c = cq[u];
        // an opaque zero: without it the compiler precomputes this rare path's per-block query
        // values for all 8 blocks ahead of the loop and spills them
        uint32_t oz;
        asm volatile("v_mov_b32 %0, 0" : "=v"(oz));
        const uint32_t ql = uint32_t(u * 32 + l32) + oz;
        uint32_t vm = 0;
#pragma unroll
        for (int v = 0; v < 16; ++v) vm |= __ballot(acc[u][v] >= c) ? (1u << v) : 0u;
#pragma unroll 1
        while (vm) {
            const uint32_t v = __builtin_ctz(vm);
            vm &= vm - 1;
            const float sv = acc[u][v];
            const uint32_t roff = 8 * (v >> 2) + (v & 3);
            const bool p = sv >= c && int32_t(roff) < lim;
            const uint64_t mk = __ballot(p);
            if (!mk) continue;
            const uint32_t n = uint32_t(__popcll(mk));
            if (lc + n > uint32_t(LCAP)) flush();  // wave-uniform
            if (p) {
                const uint32_t e =
                    lc + __builtin_amdgcn_mbcnt_hi(uint32_t(mk >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(mk), 0u));
                s_qi[e] = q0 + ql;
                s_key[e] = uint32_t(s_pb[ql] + 1024.0f - 2.0f * sv);  // |q| + |x| - 2 a.b, exact
                s_id[e] = r0 + roff + 4 * uint32_t(hh);
            }
            lc += n;
        }
    };

    // ---- main loop ------------------------------------------------------------------------
    // A tile's row words go through a per-wave LDS buffer (rows W + 1 words apart: the 32 rows
    // of one read fall in distinct banks), so the middle k-steps are a rolled loop that reads
    // its word by step index.  The first k-step takes its word from registers and its starting
    // values (512 - |x|/2 of each accumulator's row) from LDS, written at the end of the previous
    // tile; the last k-step is followed, in the same basic block, by the next tile's row counts
    // and by this tile's quick test (one maximum per block and lane, no branch per block), whose
    // VALU work overlaps the last MFMAs; only a tile with a possible pass branches to the
    // staging code.
    uint32_t xw[HW], xn[HW];
    load_tile(0, xw);
    i32x4h bq[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) bq[u] = rd_q(0, u);
    uint32_t* myrow = s_rw + l32 * (W + 1) + hh * HW;
    auto widen_operand = [&](uint32_t w) {
        const uint4 d = widen_row(w);
        return fp4_operand(i32x4h{int(d.x), int(d.y), int(d.z), int(d.w)});
    };
    // 512 - |x|/2 of the tile's rows into LDS: the two halves of a row are the lane pair (l, l + 32),
    // which both store the same value (no branch)
    auto row_counts = [&]() {
        uint32_t pa = 0;
#pragma unroll
        for (int i = 0; i < HW; ++i) pa += __popc(xw[i]);
        s_pa[l32] = 512.0f - 0.5f * float(pa + __shfl_xor(pa, 32));
    };
    row_counts();
    for (uint32_t lt = 0; lt < tcount; ++lt) {
#pragma unroll
        for (int i = 0; i < HW; ++i) myrow[i] = xw[i];
        f32x16h c0;  // 512 - |x|/2 of the row of each accumulator value
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4h t = *reinterpret_cast<const f32x4h*>(s_pa + 8 * g + 4 * hh);
#pragma unroll
            for (int e = 0; e < 4; ++e) c0[4 * g + e] = t[e];
        }
        asm volatile("v_mov_b32 %0, 0" : "=v"(qz));
        // One k-step: block u's MFMA, then the read of its fragment for the next step, a full
        // step (8 MFMAs) ahead of its use; the row word of the step after next is read at the
        // start.  Scheduling barriers keep this program order: left alone, the scheduler moves
        // every read behind the step's last MFMA and the next step waits for all of them.
        uint32_t word = 0;
        auto k_step = [&](const i32x8h& af, const f32x16h* init, int nq, int nw) {
            if (nw >= 0) word = myrow[nw];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                acc[u] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af, fp4_operand(bq[u]), init ? *init : acc[u],
                                                                         4, 4, 0, 127, 0, 127);
                bq[u] = rd_q(nq, u);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        k_step(widen_operand(xw[0]), &c0, 1, 1);  // accumulators start from 512 - |x|/2
        load_tile(lt + 1 < tcount ? lt + 1 : lt, xn);  // the next tile in flight
        // keeps those loads here: with no store after them the compiler would sink them below
        // the k-steps, next to their use, and the tile would wait for HBM
        asm volatile("" ::: "memory");
#pragma unroll 1
        for (int st = 1; st < HW - 1; ++st) k_step(widen_operand(word), nullptr, st + 1, st + 1);
        k_step(widen_operand(word), nullptr, 0, -1);  // the last step; the next tile starts at step 0
#pragma unroll
        for (int i = 0; i < HW; ++i) xw[i] = xn[i];
        if (lt + 1 < tcount) row_counts();
        uint32_t hit = 0;  // blocks with a lane whose best value passes (wave-uniform)
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            uint32_t m = __float_as_uint(acc[u][0]);
#pragma unroll
            for (int v = 1; v < 16; ++v) m = max(m, __float_as_uint(acc[u][v]));
            hit |= __ballot(m >= __float_as_uint(cq[u])) ? (1u << u) : 0u;
        }
        if (hit) {
            const uint64_t r64 = uint64_t(t0 + lt) * TN + uint32_t(wave) * WR;
            const int32_t lim = int32_t(r64 < N ? min(uint64_t(N) - r64, uint64_t(WR)) : 0) - 4 * hh;
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (hit & (1u << u)) block_passes(u, uint32_t(r64), lim);  // ids below N fit 32 bits
        }
    }
    flush();
}

// The fp4 MFMA filter scan needs whole 16-byte loads of each half row (W % 8 == 0), rows
// whose widened queries fit the LDS with the row buffers (W <= 24), enough queries to fill a
// 256-query block reasonably and dense rows.
bool hmf_ok(const HamArgs& a) {
#ifndef VA_HAM_MFMA
#define VA_HAM_MFMA 1
#endif
    return VA_HAM_MFMA && !a.qrow && a.q0 == 0 && a.c0 == 0 && a.stride == 1 && a.nq > 192 &&
           (a.W == 8 || a.W == 16 || a.W == 24) && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
           uint64_t(a.cols) * a.W * 4 <= 0xFFFFFFFFFFFFull;
}

template <int W>
va_status launch_hmf_w(va_context* ctx, const HamArgs& a) {
    using namespace hmf;
    const uint32_t nqb = (a.nq + TQ - 1) / TQ;
    const uint32_t per = (uint32_t(std::max(ctx->num_cus, 8)) + nqb - 1) / nqb;
    const uint32_t R = std::max<uint32_t>(kXcds, (per + kXcds - 1) / kXcds * kXcds);
    const uint64_t grid = uint64_t(nqb) * R;
    if (grid > 0x7FFFFFFFull) return fail(ctx, VA_ERR_INVALID_ARG, "Hamming scan grid too large");
    auto kern = &hamming_mfma_kernel<W>;
    VA_CHECK_HIP(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes(W))));
    kern<<<dim3(uint32_t(grid)), dim3(512), lds_bytes(W), ctx->stream>>>(a, R);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status launch_hmf(va_context* ctx, const HamArgs& a) {
    switch (a.W) {
        case 8: return launch_hmf_w<8>(ctx, a);
        case 16: return launch_hmf_w<16>(ctx, a);
        default: return launch_hmf_w<24>(ctx, a);
    }
}

va_status launch_ham(va_context* ctx, const HamArgs& a, bool filter) {
    if (a.nq == 0 || a.cols == 0) return VA_OK;
    if (filter && hmf_ok(a)) return launch_hmf(ctx, a);
    const dim3 grid((a.cols + 255) / 256);
    const bool aligned = (a.W & 3) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0;
    if (a.W <= kMaxWords && (aligned || (a.W & 3) != 0)) {
#define VA_HAM_CASE(WC)                                                                       \
    if (filter)                                                                               \
        hamming_scan_kernel<WC, true><<<grid, dim3(256), 0, ctx->stream>>>(a);               \
    else                                                                                      \
        hamming_scan_kernel<WC, false><<<grid, dim3(256), 0, ctx->stream>>>(a);
        if (a.W == 8 && aligned) {
            VA_HAM_CASE(8)
        } else if (a.W == 16 && aligned) {
            VA_HAM_CASE(16)
        } else if (a.W == 24 && aligned) {
            VA_HAM_CASE(24)
        } else if (a.W == 32 && aligned) {
            VA_HAM_CASE(32)
        } else {
            VA_HAM_CASE(0)
        }
#undef VA_HAM_CASE
    } else {
        if (filter)
            hamming_scan_wide_kernel<true><<<grid, dim3(256), 0, ctx->stream>>>(a);
        else
            hamming_scan_wide_kernel<false><<<grid, dim3(256), 0, ctx->stream>>>(a);
    }
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

struct HamProducer final : KeyProducer {
    va_context* ctx;
    const uint32_t* q;
    const uint32_t* x;
    uint32_t Q, N, W;
    va_status fallback_pass(const FbArgs& a, int pass) override {
        return fb_launch_pass(ctx, FbHam{q, x, N, W}, a, pass);
    }
    // distances are at most 32 W
    uint32_t key_bits() const override { return 32u - uint32_t(__builtin_clz(32u * W)); }
    va_status dense(const uint32_t* qrow, uint32_t q0, uint32_t nq, uint32_t c0, uint32_t cols, uint32_t stride,
                    uint32_t* out_k, int64_t ldo) override {
        HamArgs a;
        a.q = q;
        a.qrow = qrow;
        a.q0 = q0;
        a.nq = nq;
        a.x = x;
        a.c0 = c0;
        a.cols = cols;
        a.stride = stride;
        a.W = W;
        a.out_k = out_k;
        a.ldo = ldo;
        return launch_ham(ctx, a, false);
    }
    va_status filter(const uint32_t* thr, uint32_t* cnt, uint32_t* ckey, uint32_t* cid, uint32_t cap) override {
        HamArgs a;
        a.q = q;
        a.q0 = 0;
        a.nq = Q;
        a.x = x;
        a.c0 = 0;
        a.cols = N;
        a.stride = 1;
        a.W = W;
        a.thr = thr;
        a.cnt = cnt;
        a.cand_key = ckey;
        a.cand_id = cid;
        a.cap = cap;
        return launch_ham(ctx, a, true);
    }
};

}  // namespace
}  // namespace va

extern "C" {

va_status va_bq_pack(va_context* ctx, const float* x, uint32_t num_vectors, uint32_t dim, uint32_t* codes) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, x && codes, "va_bq_pack: NULL pointer");
    VA_REQUIRE(ctx, num_vectors > 0 && dim > 0, "Input vectors cannot be empty");
    va::DeviceGuard g(ctx->device);
    const uint32_t W = (dim + 31) / 32;
    const uint32_t blocks = std::min<uint32_t>((num_vectors + 3) / 4, 65536);
    va::pack_kernel<<<dim3(blocks), dim3(256), 0, ctx->stream>>>(x, num_vectors, dim, W, codes);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status va_hamming_matrix(va_context* ctx, const uint32_t* query_codes, const uint32_t* database_codes,
                            uint32_t num_queries, uint32_t num_database, uint32_t words, uint32_t* out) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, query_codes && database_codes && out, "va_hamming_matrix: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0 && num_database > 0 && words > 0, "va_hamming_matrix: empty input");
    VA_REQUIRE(ctx, num_queries <= 65535, "va_hamming_matrix: at most 65535 queries per call");
    va::DeviceGuard g(ctx->device);
    va::hamming_matrix_kernel<<<dim3((num_database + 255) / 256, num_queries), dim3(256), 0, ctx->stream>>>(
        query_codes, database_codes, num_database, words, out);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status va_hamming_topk(va_context* ctx, const uint32_t* query_codes, const uint32_t* database_codes,
                          uint32_t num_queries, uint32_t num_database, uint32_t words, uint32_t k, uint32_t* out_idx,
                          uint32_t* out_dist) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, query_codes && database_codes && out_idx, "va_hamming_topk: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0 && num_database > 0 && words > 0, "va_hamming_topk: empty input");
    VA_REQUIRE(ctx, k > 0 && k <= VA_MAX_K, "k must be in [1, %u], got %u", VA_MAX_K, k);
    va::DeviceGuard g(ctx->device);
    va::HamProducer p;
    p.ctx = ctx;
    p.q = query_codes;
    p.x = database_codes;
    p.Q = num_queries;
    p.N = num_database;
    p.W = words;
    va::ScanOutputs o;
    o.idx = out_idx;
    o.key = out_dist;
    o.key_kind = 3;
    return va::exact_topk_scan(ctx, p, num_queries, num_database, k, o);
}

}  // extern "C"

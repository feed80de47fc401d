// Decode W4A16 GEMV for M <= 16 rows on the strip layout, with an optional fused SwiGLU epilogue.
//
// Work split. A wave owns S strips (S = 2: the gate and up strips of 16 channels when fused, or two adjacent
// strips) over a contiguous run of the K tiles of its split; `wps` waves share a strip group's K range and add
// their partial sums through LDS at the end. A workgroup holds `nu` strip groups over one K range (split), so
// the activation chunk it stages in LDS once serves nu * S strips: for M > 1 that chunk is M times larger
// than for one row, and sharing it is what keeps its L2 -> LDS traffic below the weight traffic. Splits bound
// the staged chunk and, with several rows, widen narrow grids; their fp32 partials are added by sum_splits,
// which applies SwiGLU when fused.
//
// Streaming. Each wave keeps a ring of KB steps (S strip tiles and their scale/zero records per step) in
// flight: the tile of step i + KB is requested as soon as step i has consumed its registers, and each step
// waits only for its own loads (in-order vmcnt). A strip tile is 1 KiB read with one 16-byte load per lane,
// so every wave load is fully coalesced; weights use non-temporal loads. With several rows the ring holds 8
// tiles (4 where the records or the four-row folds need the registers), which keeps the register count near
// 100, so four or more waves fit per SIMD and every workgroup of a decode launch is resident at once (the
// launch streams without a second round of workgroups). With one row the launch picks the ring depth (3, 4
// or 8 steps; strip pairs at most 4) from its wave count so that about kRingSteps steps are in flight over
// the whole launch: more than that only lengthens the memory queues and the launch's tail (measured on the
// Llama-3-8B, Qwen2.5-14B and Llama-3.2-1B projections: down at 2048 waves 7.3 us with 4 steps against 7.6
// with 8, at 2560 waves 9.8 us with 3 against 11.2 with 8, and at 1024 waves 4.6 us with 8 against 4.8
// with 4). Few rows keep 4 steps.
//
// Math per strip tile (4 MFMA steps of 32 K): the B operand is bias + q straight from the nibbles
// (hm_device.hpp), A is the activation rows from LDS. One row:
//   P = sum_k x'_k (bias + q'_k)       (q' = q, or 16 q on the fp16 odd pairs with x' = x / 16)
//     = sum_k x_k q_k + Xb,            Xb = bias * sum_k x'_k
// and per group, with scale s and zero z of the column, sum_k x_k (q_k - z) s = s (P - Xb - z X), X = sum_k x_k.
// Xb and X per group are computed when the wave stages x. This is the reference's per-tile factorization
// s (sum q x - z sum x) (kernels/gpu/src/gemv_w4a16.cu:91-98, src/cpu_avx_kernels/w4a16_gemv_avx_packed.cpp:242-253),
// applied to MFMA partial sums. Two to four rows (and five to eight, two rows per lane group) take the same math: A
// row r is x row r / 4, so lane group h of the MFMA output holds row h and folds it as one row does (the fp16 odd pairs'
// operand takes bias 64 so that the rows go to LDS unscaled, by DMA, and the group sums are made from LDS). Several
// rows (the rest): each 32-K step runs a second MFMA of the same A fragment against the constant operand -(bias + z)
// (the fp16 odd pairs take bias 64, so x needs no scaling), so the chain holds P = sum_k x_k (q_k - z) exactly in its
// products and the fold is one FMA s P per row: no per-group activation sums, and x goes to LDS as it is, by DMA. The MFMA pipe has the room (it is idle most of the time in a
// decode GEMV); the VALU has not. One LDS read of an A fragment feeds the MFMAs of all S strips.
//
// Output: plain y = round(sum) (or, accumulating, y = round(y + round(sum)): a residual add), fused
// act = round(SiLU(gate) * up) with fp32 math and one rounding (kernels/gpu/src/silu_mul.cu:10-30), or fp32
// partials per split. One row may stage RMSNorm(x) * w instead of x (the layer-boundary norm).
#include "hm_device.hpp"
#include "hm_internal.hpp"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdlib>
#include <exception>
#include <unordered_map>

namespace hm {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr size_t kXBudget = 64 * 1024;   // staged activation bytes per workgroup at one row (bounds a split's K range)
constexpr size_t kLdsMax = kGemvLdsMax;   // LDS of one workgroup
constexpr int64_t kRowsInFlight = 5120;  // weight tiles in flight over a multi-row launch the planner aims for (5 MiB)
constexpr int64_t kUnitsPerCu = 4;       // (strip group, split) units per CU a multi-row K split may make at most
constexpr int kNormChunks = 4;           // RMSNorm in the staging: rows of up to 4 x 2048 columns
constexpr int64_t kRingSteps = 8192;     // ring steps in flight over a one-row launch (8 MiB of single-strip tiles)

// Ring depth of a one-row launch of `waves` waves: the deepest of 8, 4 and 3 steps that keeps at most
// kRingSteps steps in flight, and 3 beyond that.
int ring_depth(int64_t waves) { return waves * 8 <= kRingSteps ? 8 : waves * 4 <= kRingSteps ? 4 : 3; }

struct GemvArgs {
    const uint4 *quant;
    const uint32_t *meta;
    const uint16_t *x;
    uint16_t *y;
    float *partial; // [splits][m][ncols] fp32, or nullptr when the call has one split
    int64_t ldx, ldy;
    int kt_pitch;
    int kt_begin, kt_count, kt_per_split;
    int strip_begin; // first strip of the call
    int groups;      // strip groups (S strips each) of the call
    int m;
    int ncols; // 16 * strips of the call (row length of `partial`)
    int nu;    // strip groups per workgroup
    int wps;   // waves per strip group
    // One row, whole K: the staged activation is RMSNorm(x) * norm_w (the norm of hm_rmsnorm, same rounding).
    const uint16_t *norm_w;
    float norm_eps;
    bool accumulate; // plain output: y = round(y + round(sum)) (a residual add) instead of y = round(sum)
    // K-split pair (one row, two splits): split 1 reads a second matrix over x[k0, k0 + 128 kt_count2).
    const uint4 *quant2;
    const uint32_t *meta2;
    int kt_pitch2, kt_count2;
    int k0;
    // One row, fused: units > 0 deals (strip pair, K half) units evenly over the workgroups, workgroup b running
    // units b * units .. b * units + units - 1 (unit u: pair u / 2, half u % 2); a pair whose two units fall in
    // two workgroups (odd units) writes both halves' fp32 sums to pair_spill instead of its act columns.
    int units;
    // One row, plain: pair_units > 0 (odd) means x is the act of such a launch with that many units per
    // workgroup, whose split pairs' columns are formed from pair_spill while x is staged.
    int pair_units;
    float *pair_spill;
};

// v plus v of another lane of the same row of 16 (DPP control CTRL).
template <int CTRL> __device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum of v over aligned groups of N (1, 2, 4, 8 or 16) consecutive lanes, in every lane of the group, by DPP
// butterflies within a row of 16 lanes: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror.
template <int N> __device__ __forceinline__ float group_sum(float v) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group of lanes");
    if constexpr (N >= 2) {
        v = dpp_add<0xB1>(v);
    }
    if constexpr (N >= 4) {
        v = dpp_add<0x4E>(v);
    }
    if constexpr (N >= 8) {
        v = dpp_add<0x141>(v);
    }
    if constexpr (N >= 16) {
        v = dpp_add<0x140>(v);
    }
    return v;
}

// B operand of one 32-K step for several rows: bias + q in all eight K positions. fp16: 1024 + q in the even
// pairs and 64 + q in the odd pairs, whose nibbles sit at bits 4..7 of each half (under the exponent of 64 the
// mantissa step is 1/16, so 16 q reads as q); bf16: 128 + q (magic_operand).
template <class T> __device__ __forceinline__ uint4 rows_operand(uint32_t w, const MagicRegs &c, uint32_t odd_magic) {
    if constexpr (T::kWide) {
        const uint32_t u = w >> 8;
        return uint4{(w & c.lo) | c.magic, (w & c.hi) | odd_magic, (u & c.lo) | c.magic, (u & c.hi) | odd_magic};
    } else {
        return magic_operand<T>(w, c);
    }
}

// The matching constant operand -(bias + z) for the zero point z of record r (bits 16..23, at most 16): every
// value exact, so one MFMA of it against the same activations takes sum_k x_k (bias + z) off the step's sum.
template <class T> __device__ __forceinline__ uint4 zero_operand(uint32_t r) {
    const uint32_t z2 = __builtin_amdgcn_perm(0u, r, 0x0C020C02u); // z in both 16-bit halves
    if constexpr (T::kWide) {
        const uint32_t e = z2 | 0xE400E400u;        // -(1024 + z)
        const uint32_t o = (z2 << 4) | 0xD400D400u; // -(64 + z)
        return uint4{e, o, e, o};
    } else {
        const uint32_t e = z2 | 0xC300C300u; // -(128 + z)
        return uint4{e, e, e, e};
    }
}

// MT: rows the instantiation serves. 1: one row. kFewRows (2..4 rows) and 2 kFewRows (5..8 rows): the one-row math
// and streaming with R = MT / 4 rows per lane group of the MFMA output: A row r reads x row r R / 4, so lane group h
// holds rows R h .. R h + R - 1 (D elements 4 e / R, e < R) and folds each as one row does (R = 1: no more fold work
// per step than one row). 16: several rows (up to 16) on the zero-point math.
//
// Dynamic LDS. One row: xs [kc + 8] 16-bit, sums [kc / G + 1] float2 (Xb, X), the RMSNorm's four partial sums,
// red [waves][S][16] float, then (pair_units > 0) the formed columns of the split's split pairs, 16 per pair in
// pair order. Few rows: xs [m][xst] with xst = kc rounded up to 512 + 8, sums [m][kc / G + 1], 16 bytes, red
// [waves][S][m][16]. Several rows: per K tile of the split a block of rows_pad = 4 ceil(m / 4) rows of 256 bytes, the
// 16-byte chunk c of row r at slot c ^ (r % 16) (rows past m hold row m - 1), and after the multiply, over its
// front, red [wps - 1][nu][S][4][64 lanes] float: the sums of each strip group's waves past the first.
// RING: ring depth in steps for one or few rows (group >= 64), at most 8 tiles; the other instantiations
// size their ring themselves and take RING = 0. PAIRS (one row): kUnitsOut, the fused launch by units (a.units
// waves per workgroup of WGS = 1024); kUnitsIn, the plain launch whose x holds such a launch's split pairs.
constexpr int kUnitsOut = 1, kUnitsIn = 2;
constexpr int kFewRows = 4;
template <class T, int MT, int G, int S, bool FUSED, int WGS, int RING, int PAIRS = 0>
__global__ void __launch_bounds__(WGS) __attribute__((amdgpu_waves_per_eu(4))) gemv_kernel(GemvArgs a) {
    static_assert(MT == 1 || MT == kFewRows || MT == 2 * kFewRows || MT == 16, "row modes");
    static_assert(PAIRS == 0 || (MT == 1 && (PAIRS == kUnitsOut ? FUSED && WGS == 1024 : !FUSED && S == 1)), "pair modes");
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr bool FEW = MT == kFewRows || MT == 2 * kFewRows;
    constexpr bool ONE = MT == 1 || FEW; // the one-row math (one or few rows)
    constexpr int RPL = FEW ? MT / 4 : 1; // rows per lane group (few rows)
    constexpr int QE = 4 / RPL;           // D elements per row in a lane (few rows)
    constexpr int ROWS = ONE ? RPL : 4;   // D elements per lane that can hold a real row
    constexpr int GPT = 128 / G;           // groups per strip tile
    constexpr int SPG = 4 / GPT;           // MFMA steps per group
    // Ring depth in steps: 8 tiles in flight per wave, fewer where the records (group < 128) and the
    // four-row folds (M > 1) need the registers.
    constexpr int kInFlight = (!ONE && (S == 1 || GPT > 1)) ? 4 : 8; // strip tiles
    constexpr int KB_SIZED = kInFlight / S / (GPT == 4 ? 2 : 1) > 0 ? kInFlight / S / (GPT == 4 ? 2 : 1) : 1;
    constexpr int KB = RING > 0 ? RING : KB_SIZED;
    static_assert(RING == 0 || (ONE && GPT < 4 && S * RING <= 8), "a chosen ring depth is for one or few rows, groups of 64 or 128, at most 8 tiles");
    constexpr int CPG = G / 8;             // 8-element activation chunks per group
    constexpr int kPre = 4;                // chunks per thread fetched ahead of the weights
    // Weight loads are non-temporal. Plain loads in the Llama-3-8B down GEMV (ring of 4) look 0.5 us faster per layer
    // when six layers rotate, but only because the six down matrices (184 MB) then stay in the 256 MB Infinity Cache:
    // with 12 or 32 layers rotating, as in a whole model, the layer is 0.3-0.5 us faster with non-temporal loads
    // (21.25 against 20.78 us at 12, 21.27 against 21.02 at 32).

    const int tid = threadIdx.x;
    const int wave = uniform(tid >> 6);
    const int lane = tid & 63;
    const int m = MT == 1 ? 1 : a.m; // the one-row instantiation is launched for m = 1 only, the few-row ones for 2..4, 5..8
    const int col = lane & 15;
    const int h = lane >> 4;

    const int split = blockIdx.y;
    const bool second = a.quant2 != nullptr && split == 1; // the pair's second matrix
    const int kt0 = second ? 0 : a.kt_begin + split * a.kt_per_split;
    const int nkt = second ? a.kt_count2 : min(a.kt_per_split, a.kt_begin + a.kt_count - kt0);
    const int kc = nkt * 128; // K values of this split
    const int kg = kc / G;    // groups of this split
    const int64_t xk0 = second ? static_cast<int64_t>(a.k0) : static_cast<int64_t>(kt0 - a.kt_begin) * 128;

    // One row: x padded by 16 bytes and the group sums by 8 (the layout the fold reads). Few rows: each row's x
    // rounded up to whole 1 KiB transfers (512 K) and padded by 16 bytes, so the four rows one MFMA operand read
    // touches fall on different banks; its group sums likewise one row after another.
    const int xst = FEW ? ((kc + 511) & ~511) + 8 : kc + 8;
    const int sst = kg + 1;
    const int xrows = FEW ? m : 1;
    uint16_t *xs = reinterpret_cast<uint16_t *>(smem);
    float2 *sums = reinterpret_cast<float2 *>(smem + xrows * xst * 2);
    const int norm_off = (xrows * (xst * 2 + sst * static_cast<int>(sizeof(float2))) + 15) & ~15; // 4 floats past the staging
    // Several rows: bytes per K tile of the staged chunk.
    const int rows_pad = (m + 3) & ~3;
    const int tstride = rows_pad * 256;
    // One row: the cross-wave sums get their own space past the norm's partials, so a wave that has finished its
    // multiply writes them while others still read the staging (no barrier before the writes). Several rows:
    // they reuse the staging space, which the 144 KiB chunk leaves no room beside.
    float *red = reinterpret_cast<float *>(smem + (ONE ? norm_off + 16 : 0));

    // This wave's strip group and its contiguous run [tb, te) of the split's tiles. Groups past the end of
    // the call (a partial last workgroup) read the last group and are not stored. Units (one row, fused): the
    // wave's unit gives its pair and its K half (a.wps == 2).
    constexpr bool by_units = PAIRS == kUnitsOut;
    const int unit = static_cast<int>(blockIdx.x) * a.units + wave;
    const int grp = by_units ? 0 : wave % a.nu;
    const int wi = by_units ? unit & 1 : wave / a.nu;
    const int gidx = min(by_units ? unit >> 1 : static_cast<int>(blockIdx.x) * a.nu + grp, a.groups - 1);
    const int strip0 = a.strip_begin + gidx * S;
    const uint4 *qp[S];
    const uint32_t *mp[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int64_t tile0 = static_cast<int64_t>(strip0 + s) * (second ? a.kt_pitch2 : a.kt_pitch) + kt0;
        qp[s] = (second ? a.quant2 : a.quant) + tile0 * 64;
        mp[s] = (second ? a.meta2 : a.meta) + tile0 * 16 * GPT;
    }
    const int tpw = (nkt + a.wps - 1) / a.wps;
    const int tb = wi * tpw;
    const int te = min(tb + tpw, nkt);
    const int last = te - 1; // >= 0: a wave past the split's end gets te = nkt >= 1 and reads only zero-weighted tiles

    // Activation staging. One row: each wave stages the K range of its own tiles, so no workgroup barrier
    // stands between the weight stream and the multiply (waves of other strip groups with the same range write
    // the same values). Chunks are 8 consecutive K; consecutive lanes take consecutive chunks, so one group's
    // chunks are G / 8 consecutive lanes. Several rows: the workgroup copies the whole chunk once for its nu
    // strip groups, memory to LDS without registers (below).
    const int st_lo = tb * 16;
    const int st_hi = max(te, tb) * 16;
    // Memory requests go out in this order: the activation chunks (one row: held in registers; several rows:
    // the LDS transfers), then the first KB steps of the wave's ring. Staging waits for the activations only.
    // RMSNorm of the row (one row, whole K): waves 0..3 take the norm's chunks of the 256 threads of the
    // separate RMSNorm kernel (thread t: elements 8t + 2048j), so its sum of squares is formed in the same order.
    const bool norm = MT == 1 && a.norm_w != nullptr;
    const int hcols = a.kt_count * 128;
    uint4 nx[kNormChunks];
    if (norm && wave < 4) {
#pragma unroll
        for (int j = 0; j < kNormChunks; ++j) {
            const int c = (wave * 64 + lane) * 8 + j * 2048;
            nx[j] = *reinterpret_cast<const uint4 *>(a.x + min(c, hcols - 8));
        }
    }
    uint4 xv[kPre], wv[kPre] = {};
    // Positions of this thread's next kPre chunks of the wave's range and whether each is staged (chunks past the
    // end re-read a valid one, branch-free, and are not staged).
    int pc8[kPre];
    bool pval[kPre];
    auto positions = [&](int base) {
#pragma unroll
        for (int c = 0; c < kPre; ++c) {
            const int idx = st_lo + base + c * 64 + lane;
            pval[c] = idx < st_hi;
            pc8[c] = st_hi > st_lo ? min(idx, st_hi - 1) : 0;
        }
    };
    auto fetch = [&]() {
#pragma unroll
        for (int c = 0; c < kPre; ++c) {
            xv[c] = *reinterpret_cast<const uint4 *>(a.x + xk0 + pc8[c] * 8);
            if (norm) {
                wv[c] = *reinterpret_cast<const uint4 *>(a.norm_w + xk0 + pc8[c] * 8);
            }
        }
    };
    // Split pairs of the producing launch (one row, plain, pair_units = U odd): pair p of x's columns is split
    // when p % U == (U - 1) / 2, and split pair U j + (U - 1) / 2 has the fp32 sums of its column c at pair_spill
    // [16 j + c] = {gate, up of half 0, gate, up of half 1}. The wave's split pairs' columns t (16 per pair) are
    // taken four per lane, t = lane + 64 i, their sums loaded ahead of the weights; before staging each is formed
    // as round(SiLU(g0 + g1) * (u0 + u1)), the rounding of the producer's other pairs, into the LDS area `formed`
    // (the split's split pairs in order, 16 columns each), which the staging reads in place of x.
    constexpr bool forms = PAIRS == kUnitsIn;
    // Columns per lane loaded ahead: 16 split pairs, what a wave's range holds when the down GEMV runs 8 waves
    // per strip (a range of R pairs holds at most R / U + 1, and R is about 16 U there: the Llama-3-8B layer
    // gives 16); a longer range forms the rest after, each load waited for in turn.
    constexpr int kFormPre = 4;
    const int pu = forms ? a.pair_units : 1;
    const int phalf = (pu - 1) >> 1;
    const int cb = static_cast<int>(xk0 >> 3);                       // x chunk of the split's first K
    const int js = (cb / 2 + phalf) / pu;                             // the split's first split pair
    const int ja = uniform(((cb + st_lo) / 2 + phalf) / pu);          // this wave's first split pair
    const int ncols_form = forms ? 16 * (uniform(((cb + st_hi) / 2 + phalf) / pu) - ja) : 0;
    uint16_t *formed = reinterpret_cast<uint16_t *>(smem + norm_off + 16 + (WGS / 64) * S * 16 * static_cast<int>(sizeof(float)));
    const float4 *spill4 = reinterpret_cast<const float4 *>(a.pair_spill) + static_cast<int64_t>(ja) * 16;
    float4 fsum[kFormPre];
    if constexpr (MT == 1) {
        positions(0);
        fetch();
        if constexpr (forms) {
            if (ncols_form > 0) { // columns past the range re-read its last one
#pragma unroll
                for (int i = 0; i < kFormPre; ++i) {
                    fsum[i] = spill4[min(lane + 64 * i, ncols_form - 1)];
                }
            }
        }
    } else if constexpr (FEW) {
        // Few rows: each row's chunks of the wave's range go memory to LDS without registers, in whole 1 KiB
        // transfers of 64 chunks aligned to the split's chunk 0 (chunks past the range hold the same x as any wave
        // staging them writes; past the split's last row the buffer reads zeros). The group sums follow from LDS.
        const uint32_t ldx2 = static_cast<uint32_t>(a.ldx) * 2u;
        const __amdgpu_buffer_rsrc_t xr =
            buffer_rsrc(a.x + xk0, static_cast<uint32_t>(m - 1) * ldx2 + static_cast<uint32_t>(kc) * 2u);
        const int blo = st_lo >> 6, bhi = (st_hi + 63) >> 6;
        for (int r = 0; r < m; ++r) {
            for (int b = blo; b < bhi; ++b) {
                const uint32_t voff = static_cast<uint32_t>(r) * ldx2 + static_cast<uint32_t>(64 * b + lane) * 16u;
                lds_dma16(xr, reinterpret_cast<uint8_t *>(xs + r * xst + 512 * b), voff, 0u);
            }
        }
    } else {
        // Transfer p (1 KiB): K tile p / (rows_pad / 4), rows 4 (p % (rows_pad / 4)) + h; lane l fills slot l % 16
        // of its row with chunk (l % 16) ^ row. Rows past m read row m - 1.
        constexpr int WAVES = WGS / 64;
        const int rblocks = rows_pad >> 2;
        const uint32_t ldx2 = static_cast<uint32_t>(a.ldx) * 2u;
        const __amdgpu_buffer_rsrc_t xr =
            buffer_rsrc(a.x + xk0, static_cast<uint32_t>(m - 1) * ldx2 + static_cast<uint32_t>(kc) * 2u);
        for (int p = wave; p < nkt * rblocks; p += WAVES) {
            const int t = p / rblocks;
            const int rb = p - t * rblocks;
            const int row = 4 * rb + h;
            const uint32_t voff = static_cast<uint32_t>(min(row, m - 1)) * ldx2 + static_cast<uint32_t>(col ^ row) * 16u;
            lds_dma16(xr, smem + t * tstride + rb * 1024, voff, static_cast<uint32_t>(t) * 256u);
        }
    }

    // Scale/zero records travel in blocks of RB consecutive tiles: lane l loads the records of tile
    // i + l / 16 (column l % 16), so one coalesced load covers RB tiles (the records of consecutive tiles
    // are contiguous), and step u takes its column's record from lane 16 (u % RB) + col.
    constexpr int RB = KB < 4 ? KB : 4;
    static_assert(KB % RB == 0, "the ring holds whole record blocks");
    const int rsub = min(lane >> 4, RB - 1);
    uint4 wq[KB][S];
    // Record blocks of the round being multiplied (rv) and of the next round (rn): a round's steps read rv
    // while the next round's block is already in flight.
    uint32_t rv[KB / RB][S][GPT], rn[KB / RB][S][GPT];
    auto advance = [&]() {
#pragma unroll
        for (int b = 0; b < KB / RB; ++b) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
#pragma unroll
                for (int g = 0; g < GPT; ++g) {
                    rv[b][s][g] = rn[b][s][g];
                }
            }
        }
    };
    // Step u of the ring <- local tile i (already clamped to [0, last]): records (every RB steps), then the weights.
    auto load = [&](int u, int i) {
        if (u % RB == 0) {
            const int64_t ri = static_cast<int64_t>(min(i + rsub, last)) * 16 + col;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                if constexpr (GPT == 1) {
                    rn[u / RB][s][0] = mp[s][ri];
                } else if constexpr (GPT == 2) {
                    const uint2 r = *reinterpret_cast<const uint2 *>(mp[s] + ri * 2);
                    rn[u / RB][s][0] = r.x;
                    rn[u / RB][s][1] = r.y;
                } else {
                    const uint4 r = *reinterpret_cast<const uint4 *>(mp[s] + ri * 4);
                    rn[u / RB][s][0] = r.x;
                    rn[u / RB][s][1] = r.y;
                    rn[u / RB][s][2] = r.z;
                    rn[u / RB][s][3] = r.w;
                }
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const u32x4_t *src = reinterpret_cast<const u32x4_t *>(qp[s] + i * 64 + lane);
            const u32x4_t v = __builtin_nontemporal_load(src);
            wq[u][s] = uint4{v.x, v.y, v.z, v.w};
        }
    };
#pragma unroll
    for (int u = 0; u < KB; ++u) {
        load(u, min(tb + u, last));
    }
    __builtin_amdgcn_sched_barrier(0);
    advance();
    if constexpr (FEW) {
        // This wave's transfers are in LDS once at most the ring's loads are outstanding (vmcnt counts in issue
        // order); the wave reads only rows it transferred itself.
        wait_vmcnt<KB * S + (KB / RB) * S>();
    } else if constexpr (!ONE) {
        // As above; the barrier then covers every wave's transfers.
        wait_vmcnt<KB * S + (KB / RB) * S>();
        lds_barrier();
    }

    float nscale = 1.0f;
    if (norm) {
        float *npart = reinterpret_cast<float *>(smem + norm_off);
        if (wave < 4) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < kNormChunks; ++j) {
                const int c = (wave * 64 + lane) * 8 + j * 2048;
                if (c < hcols) {
                    const uint32_t w[4] = {nx[j].x, nx[j].y, nx[j].z, nx[j].w};
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        const float v = T::to_float(k & 1 ? w[k >> 1] >> 16 : w[k >> 1] & 0xFFFFu);
                        ss += v * v;
                    }
                }
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                ss += __shfl_xor(ss, off);
            }
            if (lane == 0) {
                npart[wave] = ss;
            }
        }
        lds_barrier();
        float total = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            total += npart[w];
        }
        nscale = 1.0f / sqrtf(total / static_cast<float>(hcols) + a.norm_eps);
    }

    // 1. One row: stage x into LDS (fp16: odd pairs scaled by 1/16) with the per-group sums. Consecutive lanes
    //    take consecutive 8-element chunks, so one group is G / 8 consecutive lanes. (Few rows: x is in LDS as it is,
    //    the fp16 odd pairs' operand taking bias 64 instead, rows_operand; the group sums follow below.)
    auto stage = [&](int c8, uint4 v, uint4 g, bool valid) {
        float sa = 0.0f, sb = 0.0f;
        if (norm) { // v <- round(v * scale * g) element-wise, as the RMSNorm kernel stores it
            uint32_t vw[4] = {v.x, v.y, v.z, v.w};
            const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float lo = T::to_float(vw[i] & 0xFFFFu) * nscale * T::to_float(gw[i] & 0xFFFFu);
                const float hi = T::to_float(vw[i] >> 16) * nscale * T::to_float(gw[i] >> 16);
                vw[i] = static_cast<uint32_t>(T::from_float(lo)) | (static_cast<uint32_t>(T::from_float(hi)) << 16);
            }
            v = uint4{vw[0], vw[1], vw[2], vw[3]};
        }
        if (valid) {
            if constexpr (T::kWide) {
                // fp16: sums of the even / odd pairs with v_dot2_f32_f16 against (1, 1)
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                const h2 one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
                sa = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, v.z), one, __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, v.x), one, 0.0f, false), false);
                sb = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, v.w), one, __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, v.y), one, 0.0f, false), false);
            } else {
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const float lo = T::to_float(w[p] & 0xFFFFu), hi = T::to_float(w[p] >> 16);
                    if (p & 1) {
                        sb += lo + hi;
                    } else {
                        sa += lo + hi;
                    }
                }
            }
            if constexpr (T::kWide) {
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                const h2 sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
                v.y = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v.y) * sixteenth);
                v.w = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v.w) * sixteenth);
            }
            *reinterpret_cast<uint4 *>(xs + c8 * 8) = v;
        }
        // Sum over the CPG consecutive lanes of a group with DPP (no LDS crossbar): pairs, quads, eights, sixteens.
        sa = group_sum<CPG>(sa);
        sb = group_sum<CPG>(sb);
        if (valid && (c8 % CPG) == 0) {
            const float xb = T::kWide ? (1024.0f * sa + 64.0f * sb) : T::kBias * (sa + sb);
            sums[c8 / CPG] = make_float2(xb, sa + sb);
        }
    };
    // x's chunk c8 of the split, or its formed chunk when it belongs to a split pair. pr / pu as the high word of
    // pr ceil(2^32 / pu): exact for 2 <= pu <= 16 and pr < 2^24 (checked exhaustively; pairs of x number K / 16).
    const uint32_t pu_inv = forms ? 0xFFFFFFFFu / static_cast<uint32_t>(pu) + 1u : 0u;
    auto x_chunk = [&](int c8, uint4 v) {
        if constexpr (forms) {
            const int k8 = cb + c8;
            const int pr = k8 >> 1;
            const int q = static_cast<int>(__umulhi(static_cast<uint32_t>(pr), pu_inv));
            if (pr - q * pu == phalf) {
                v = reinterpret_cast<const uint4 *>(formed)[(q - js) * 2 + (k8 & 1)];
            }
        }
        return v;
    };
    if constexpr (MT == 1) {
        if constexpr (forms) {
            uint16_t *fw = formed + (ja - js) * 16;
            auto form = [&](int t, float4 v) {
                if (t < ncols_form) {
                    fw[t] = T::from_float(silu((0.0f + v.x) + v.z) * ((0.0f + v.y) + v.w));
                }
            };
#pragma unroll
            for (int i = 0; i < kFormPre; ++i) {
                form(lane + 64 * i, fsum[i]);
            }
            for (int t = lane + 64 * kFormPre; t < ncols_form; t += 64) {
                form(t, spill4[t]);
            }
        }
#pragma unroll
        for (int c = 0; c < kPre; ++c) {
            stage(pc8[c], x_chunk(pc8[c], xv[c]), wv[c], pval[c]); // all lanes take part in the shuffles
        }
        for (int base = kPre * 64; st_lo + base < st_hi; base += kPre * 64) {
            positions(base);
            fetch(); // long ranges only: these chunks wait behind the first ring steps
#pragma unroll
            for (int c = 0; c < kPre; ++c) {
                stage(pc8[c], x_chunk(pc8[c], xv[c]), wv[c], pval[c]);
            }
        }
        // The wave reads only what it wrote; LDS operations of one wave complete in order.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    } else if constexpr (FEW) {
        // Group sums of the staged rows: one lane per (row, group) of the wave's range, adding the group's chunks in
        // order from a lane-dependent first chunk (consecutive lanes' groups are 2 G bytes apart, so starting at
        // chunk lane % CPG spreads one read over the banks); no shuffles. Against the one-row staging's shuffle sums
        // over 64 chunks at a time: the Llama-3-8B down at 4 / 5 rows 10.7 / 11.4 -> 9.5 / 9.8 us, Qwen2.5-14B's at 4
        // rows 13.7 -> 12.7, Llama-3.2-1B's 6.3 / 6.8 -> 5.7 / 5.9.
        const int ng = (st_hi - st_lo) / CPG; // groups of the wave's range in one row
        const int g0 = st_lo / CPG;
        const float inv_ng = 1.0f / static_cast<float>(max(ng, 1));
        for (int base = 0; base < m * ng; base += 64) {
            const int idx = base + lane;
            int r = static_cast<int>(static_cast<float>(idx) * inv_ng); // idx / ng, corrected below
            r += (r + 1) * ng <= idx ? 1 : 0;
            r -= r * ng > idx ? 1 : 0;
            if (idx < m * ng) {
                const int gi = g0 + idx - r * ng;
                const uint16_t *src = xs + r * xst + gi * G;
                float sa = 0.0f, sb = 0.0f;
#pragma unroll
                for (int t = 0; t < CPG; ++t) {
                    const uint4 v = *reinterpret_cast<const uint4 *>(src + ((t + lane) % CPG) * 8);
                    if constexpr (T::kWide) {
                        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                        const h2 one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
                        sa = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, v.z), one, __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, v.x), one, sa, false), false);
                        sb = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, v.w), one, __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, v.y), one, sb, false), false);
                    } else {
                        typedef __bf16 b2 __attribute__((ext_vector_type(2)));
                        const b2 one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
                        sa = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, v.z), one, __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, v.x), one, sa, false), false);
                        sb = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, v.w), one, __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, v.y), one, sb, false), false);
                    }
                }
                const float xb = T::kWide ? (1024.0f * sa + 64.0f * sb) : T::kBias * (sa + sb);
                sums[r * sst + gi] = make_float2(xb, sa + sb);
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }

    // 2. Multiply.
    const MagicRegs magic = magic_regs<T>();
    float acc[S][ROWS];
#pragma unroll
    for (int e = 0; e < ROWS; ++e) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            acc[s][e] = 0.0f;
        }
    }
    // One row: the lane's K offset in the staged row. Few rows: in row col / QE (A row r is x row r / QE), and the
    // group sums of the lane's D rows RPL h + e; rows past the last repeat it and are not stored.
    const uint16_t *xa = xs + (FEW ? min(col / QE, m - 1) * xst : 0) + 8 * h;
    int soff[RPL];
#pragma unroll
    for (int e = 0; e < RPL; ++e) {
        soff[e] = FEW ? min(RPL * h + e, m - 1) * sst : 0;
    }
    // Several rows: the A-operand row of this lane (rows past rows_pad read the last staged row; they only feed
    // D rows >= m, which are never stored) and its slot offsets per 32-K step; the magic of the fp16 odd pairs.
    const int arow = min(col, rows_pad - 1);
    uint32_t aoff[4];
#pragma unroll
    for (int mu = 0; mu < 4; ++mu) {
        aoff[mu] = static_cast<uint32_t>(arow * 256 + (((4 * mu + h) ^ arow) << 4));
    }
    uint32_t odd_magic = 0x54005400u;
    asm volatile("" : "+v"(odd_magic));

    // One row: the x fragments and group sums of a step's tile are read from LDS one step ahead (read_x), so a step's
    // first MFMA does not wait for the LDS (Llama-3-8B layer 21.06 -> 20.75 us, Qwen2.5-14B 26.25 -> 25.36, Llama-3.2-1B
    // 10.23 -> 9.93). Issuing the next step's record permutes a step ahead as well, or forcing either ahead of the
    // step's MFMAs with a scheduling barrier, measured slower.
    uint4 xf[4];
    float2 xg[RPL][GPT];
    auto read_x = [&](int i) {
        const int ic = min(i, last);
#pragma unroll
        for (int mu = 0; mu < 4; ++mu) {
            xf[mu] = *reinterpret_cast<const uint4 *>(xa + ic * 128 + 32 * mu);
        }
#pragma unroll
        for (int g = 0; g < GPT; ++g) {
#pragma unroll
            for (int e = 0; e < RPL; ++e) {
                xg[e][g] = sums[soff[e] + ic * GPT + g];
            }
        }
    };
    if constexpr (ONE) {
        read_x(tb);
    }
    // One row, one step: the S tiles of local tile i (unclamped: tiles past the wave's run are weighted by zero).
    auto step = [&](int u, int i) {
        // Tiles past the wave's run are dropped by a select, not a zero weight: a wave without tiles reads
        // LDS that no wave of its range staged, and NaN * 0 would survive.
        const bool live = i < te;
        uint4 av[4];
        float2 xsum[RPL][GPT];
#pragma unroll
        for (int mu = 0; mu < 4; ++mu) {
            av[mu] = xf[mu];
        }
#pragma unroll
        for (int e = 0; e < RPL; ++e) {
#pragma unroll
            for (int g = 0; g < GPT; ++g) {
                xsum[e][g] = xg[e][g];
            }
        }
        uint32_t rr[S][GPT];
#pragma unroll
        for (int s = 0; s < S; ++s) {
#pragma unroll
            for (int g = 0; g < GPT; ++g) {
                rr[s][g] = static_cast<uint32_t>(__shfl(static_cast<int>(rv[u / RB][s][g]), 16 * (u % RB) + col));
            }
        }
        read_x(i + 1);
        float4_t p[S];
#pragma unroll
        for (int mu = 0; mu < 4; ++mu) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const uint32_t word = mu == 0 ? wq[u][s].x : mu == 1 ? wq[u][s].y : mu == 2 ? wq[u][s].z : wq[u][s].w;
                if (mu % SPG == 0) {
                    p[s] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
                }
                p[s] = T::mfma16(av[mu], (FEW ? rows_operand<T>(word, magic, odd_magic) : magic_operand<T>(word, magic)), p[s]);
            }
            if (mu % SPG == SPG - 1) {
                const int g = mu / SPG;
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const float sc = T::to_float(rr[s][g] & 0xFFFFu);
                    const float z = static_cast<float>((rr[s][g] >> 16) & 0xFFu);
#pragma unroll
                    for (int e = 0; e < RPL; ++e) {
                        const float t = __builtin_fmaf(-z, xsum[e][g].y, p[s][QE * e] - xsum[e][g].x);
                        const float upd = __builtin_fmaf(sc, t, acc[s][e]);
                        acc[s][e] = live ? upd : acc[s][e];
                    }
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // Several rows, one live step: the S tiles of local tile i. Each 32-K step chains the MFMA of bias + q and
    // the MFMA of -(bias + z) into the group's sum P = sum_k x_k (q_k - z); the fold adds s P per row.
    auto step_rows = [&](int u, int i) {
        const uint8_t *at = smem + i * tstride;
        float4_t p[S];
        uint4 bz[S];
        float sc[S];
#pragma unroll
        for (int mu = 0; mu < 4; ++mu) {
            const uint4 av = *reinterpret_cast<const uint4 *>(at + aoff[mu]);
            if (mu % SPG == 0) {
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const uint32_t rr = static_cast<uint32_t>(__shfl(static_cast<int>(rv[u / RB][s][mu / SPG]), 16 * (u % RB) + col));
                    sc[s] = T::to_float(rr & 0xFFFFu);
                    bz[s] = zero_operand<T>(rr);
                    p[s] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
                }
            }
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const uint32_t word = mu == 0 ? wq[u][s].x : mu == 1 ? wq[u][s].y : mu == 2 ? wq[u][s].z : wq[u][s].w;
                p[s] = T::mfma16(av, rows_operand<T>(word, magic, odd_magic), p[s]);
            }
#pragma unroll
            for (int s = 0; s < S; ++s) {
                p[s] = T::mfma16(av, bz[s], p[s]);
            }
            if (mu % SPG == SPG - 1) {
#pragma unroll
                for (int s = 0; s < S; ++s) {
#pragma unroll
                    for (int e = 0; e < ROWS; ++e) {
                        acc[s][e] = __builtin_fmaf(sc[s], p[s][e], acc[s][e]);
                    }
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // One row: the same round count for every wave of the workgroup, the steps past a wave's run dropped by a
    // select. Several rows: the wave's own count, so every step of a full round is live, and the last round
    // skips its dead steps by a (wave-uniform) branch.
    const int rounds = ONE ? (tpw + KB - 1) / KB : max(1, (te - tb + KB - 1) / KB);
    for (int r = 0; r + 1 < rounds; ++r) {
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const int i = tb + r * KB + u;
            if constexpr (ONE) {
                step(u, i);
            } else {
                step_rows(u, i);
            }
            load(u, min(i + KB, last));
        }
        advance();
    }
#pragma unroll
    for (int u = 0; u < KB; ++u) {
        const int i = tb + (rounds - 1) * KB + u;
        if constexpr (ONE) {
            step(u, i);
        } else if (i < te) {
            step_rows(u, i);
        }
    }

    // 3. Add the waves of each strip group, then write.
    if constexpr (!ONE) {
        // Several rows: the group's first wave (K range 0) writes the outputs straight from its accumulators
        // (lane: column col, rows 4 h + e), after adding those of the group's other waves in order of their K
        // ranges, which they leave in LDS lane by lane; a group of one wave needs neither LDS nor a barrier.
        // The sums are the same as adding every wave's share to zero in that order (no share is -0).
        const int gg = static_cast<int>(blockIdx.x) * a.nu + grp;
        if (a.wps > 1) {
            __syncthreads(); // red reuses the staging space
            if (wi > 0) {
                float *rw = red + ((wi - 1) * a.nu + grp) * (S * ROWS * 64) + lane;
#pragma unroll
                for (int s = 0; s < S; ++s) {
#pragma unroll
                    for (int e = 0; e < ROWS; ++e) {
                        rw[(s * ROWS + e) * 64] = acc[s][e];
                    }
                }
            }
            __syncthreads();
            if (wi == 0) {
                for (int w = 1; w < a.wps; ++w) {
                    const float *rr = red + ((w - 1) * a.nu + grp) * (S * ROWS * 64) + lane;
#pragma unroll
                    for (int s = 0; s < S; ++s) {
#pragma unroll
                        for (int e = 0; e < ROWS; ++e) {
                            acc[s][e] += rr[(s * ROWS + e) * 64];
                        }
                    }
                }
            }
        }
        if (wi == 0 && gg < a.groups) {
#pragma unroll
            for (int e = 0; e < ROWS; ++e) {
                const int row = 4 * h + e;
                if (row >= m) {
                    continue;
                }
                if (a.partial != nullptr) {
                    float *pr = a.partial + (static_cast<int64_t>(split) * m + row) * a.ncols + gg * S * 16 + col;
#pragma unroll
                    for (int s = 0; s < S; ++s) {
                        pr[s * 16] = acc[s][e];
                    }
                } else if constexpr (FUSED) {
                    a.y[row * a.ldy + gg * 16 + col] = T::from_float(silu(acc[0][e]) * acc[1][e]);
                } else {
#pragma unroll
                    for (int s = 0; s < S; ++s) {
                        uint16_t *yp = a.y + row * a.ldy + (gg * S + s) * 16 + col;
                        const uint16_t yv = T::from_float(acc[s][e]);
                        *yp = a.accumulate ? T::from_float(T::to_float(*yp) + T::to_float(yv)) : yv;
                    }
                }
            }
        }
        return;
    }
    if constexpr (by_units) {
        {
            // The halves' sums meet in red [wave][S][16]. A pair whose partner wave is in this workgroup is
            // finished by its first half; a split pair (the last wave's first half, the first wave's second half)
            // leaves both halves' sums in the spill.
            if (h == 0) {
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    red[(wave * S + s) * 16 + col] = acc[s][0];
                }
            }
            __syncthreads();
            const int pair = unit >> 1;
            if (h == 0 && pair < a.groups) {
                if (wi == 0 ? wave + 1 == a.units : wave == 0) {
                    float *sp = a.pair_spill + (static_cast<int64_t>(pair / a.units) * 16 + col) * 4 + wi * 2;
                    *reinterpret_cast<float2 *>(sp) = make_float2(acc[0][0], acc[1][0]);
                } else if (wi == 0) {
                    float v[S];
#pragma unroll
                    for (int s = 0; s < S; ++s) {
                        v[s] = (0.0f + red[(wave * S + s) * 16 + col]) + red[((wave + 1) * S + s) * 16 + col];
                    }
                    a.y[gidx * 16 + col] = T::from_float(silu(v[0]) * v[1]);
                }
            }
            return;
        }
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int e = 0; e < ROWS; ++e) {
            const int row = FEW ? RPL * h + e : 4 * h + e; // one row: lanes 0..15; few rows: lane group h holds rows RPL h + e
            if (row < m) {
                red[((wave * S + s) * m + row) * 16 + col] = acc[s][e];
            }
        }
    }
    __syncthreads();
    constexpr int OUT_S = FUSED ? 1 : S; // outputs per (group, row, column)
    const int outs = a.nu * OUT_S * m * 16;
    for (int o = tid; o < outs; o += WGS) {
        const int c = o & 15;
        int rest = o >> 4;
        const int row = rest % m;
        rest /= m;
        const int s_out = rest % OUT_S;
        const int g = rest / OUT_S;
        const int gg = static_cast<int>(blockIdx.x) * a.nu + g;
        if (gg >= a.groups) {
            continue;
        }
        float v[S];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            float t = 0.0f;
            for (int w = 0; w < a.wps; ++w) {
                t += red[(((w * a.nu + g) * S + s) * m + row) * 16 + c];
            }
            v[s] = t;
        }
        if (a.partial != nullptr) {
            float *pr = a.partial + (static_cast<int64_t>(split) * m + row) * a.ncols + gg * S * 16 + c;
            if constexpr (FUSED) {
                pr[0] = v[0];
                pr[16] = v[1];
            } else {
                pr[s_out * 16] = v[s_out];
            }
        } else if constexpr (FUSED) {
            a.y[row * a.ldy + gg * 16 + c] = T::from_float(silu(v[0]) * v[1]);
        } else {
            uint16_t *yp = a.y + row * a.ldy + (gg * S + s_out) * 16 + c;
            const uint16_t yv = T::from_float(v[s_out]);
            *yp = a.accumulate ? T::from_float(T::to_float(*yp) + T::to_float(yv)) : yv;
        }
    }
}

// Adds the split partials [splits][m][ncols]; fused: ncols alternate gate and up per 16 columns and the
// output is SiLU(gate) * up per channel (ncols / 2 channels). Four consecutive outputs per thread, so every split
// is read with 16-byte loads (ncols is a multiple of 16, and four consecutive channels of a fused call lie in one
// group of 16 gate and 16 up columns).
template <class T, bool FUSED>
__global__ void __launch_bounds__(256) sum_splits(const float *__restrict__ partial, uint16_t *__restrict__ y, int64_t ldy, int m,
                                                  int ncols, int splits, bool accumulate, bool pairwise) {
    const int quads = (FUSED ? ncols / 2 : ncols) / 4;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= static_cast<int64_t>(m) * quads) {
        return;
    }
    const int row = static_cast<int>(idx / quads);
    const int c = 4 * static_cast<int>(idx - static_cast<int64_t>(row) * quads);
    const int cg = FUSED ? (c >> 4) * 32 + (c & 15) : c; // gate (or plain) column of output c
    const float4 *pr = reinterpret_cast<const float4 *>(partial + static_cast<int64_t>(row) * ncols + cg);
    const int64_t split4 = static_cast<int64_t>(m) * ncols / 4; // float4s per split
    uint16_t *yr = y + row * ldy + c;
    auto lanes = [](const float4 &v) { return std::array<float, 4>{v.x, v.y, v.z, v.w}; };
    if (!FUSED && pairwise) {
        // A K-split pair: each share's sum is rounded, then they are added with one more rounding, as
        // round(round(x0 W0) + round(x1 W1)) (plain outputs only).
        std::array<float, 4> v = lanes(pr[0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = T::to_float(T::from_float(v[i]));
        }
        for (int s = 1; s < splits; ++s) {
            const std::array<float, 4> p = lanes(pr[s * split4]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = T::to_float(T::from_float(v[i] + T::to_float(T::from_float(p[i]))));
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            yr[i] = T::from_float(v[i]);
        }
        return;
    }
    // Eight splits' loads are in flight at once (a load per split and a wait per add would put the splits'
    // memory latencies in series); the sums still run in split order.
    constexpr int kBatch = 8;
    std::array<float, 4> g{0.0f, 0.0f, 0.0f, 0.0f}, u{0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < splits; s0 += kBatch) {
        float4 gv[kBatch], uv[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int s = min(s0 + j, splits - 1); // past the last split: re-read it, not added
            gv[j] = pr[s * split4];
            uv[j] = FUSED ? pr[s * split4 + 4] : float4{};
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            if (s0 + j < splits) {
                const std::array<float, 4> a = lanes(gv[j]), b = lanes(uv[j]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    g[i] += a[i];
                    u[i] += b[i];
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint16_t out = T::from_float(FUSED ? silu(g[i]) * u[i] : g[i]);
        yr[i] = accumulate ? T::from_float(T::to_float(yr[i]) + T::to_float(out)) : out;
    }
}

template <class T, int MT, int G, int S, bool FUSED, int WGS, int RING, int PAIRS>
hipError_t launch_w(const GemvArgs &a, dim3 grid, size_t lds, hipStream_t s, unsigned block) {
    auto kern = gemv_kernel<T, MT, G, S, FUSED, WGS, RING, PAIRS>;
    // One attribute call per instantiation; a function-local static is initialized once even when several
    // host threads launch at the same time.
    static const hipError_t configured =
        hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (configured != hipSuccess) {
        return configured;
    }
    hipLaunchKernelGGL(kern, grid, dim3(block), lds, s, a);
    return hipGetLastError();
}

// block: threads per workgroup, WGS or (units) fewer.
template <class T, int MT, int G, int S, bool FUSED, int WGS, int PAIRS = 0>
hipError_t launch_r(const GemvArgs &a, dim3 grid, int ring, size_t lds, hipStream_t s, unsigned block = WGS) {
    if constexpr ((MT == kFewRows || MT == 2 * kFewRows) && G != 32) {
        (void)ring;
        return launch_w<T, MT, G, S, FUSED, WGS, 4, PAIRS>(a, grid, lds, s, block); // 4 steps in flight
    } else if constexpr (MT == 1 && G != 32) {
        // Strip pairs stop at 4 steps (8 tiles): measured slower with 8 (Llama-3.2-1B gate_up at 512 waves:
        // 7.2 us against 6.6).
        constexpr int deep = S == 2 ? 4 : 8;
        switch (ring) {
        case 3:
            return launch_w<T, MT, G, S, FUSED, WGS, 3, PAIRS>(a, grid, lds, s, block);
        case 8:
            return launch_w<T, MT, G, S, FUSED, WGS, deep, PAIRS>(a, grid, lds, s, block);
        default:
            return launch_w<T, MT, G, S, FUSED, WGS, 4, PAIRS>(a, grid, lds, s, block);
        }
    } else {
        return launch_w<T, MT, G, S, FUSED, WGS, 0, PAIRS>(a, grid, lds, s, block);
    }
}

template <class T, int MT, int G, int S, bool FUSED>
hipError_t launch_s(const GemvArgs &a, dim3 grid, int waves, int ring, size_t lds, hipStream_t s) {
    if constexpr (MT == 1 && FUSED) {
        if (a.units > 0) { // `units` waves of the 16-wave instantiation
            return launch_r<T, MT, G, S, FUSED, 1024, kUnitsOut>(a, grid, ring, lds, s, 64u * static_cast<unsigned>(a.units));
        }
    }
    if constexpr (MT == 1 && !FUSED && S == 1) {
        if (a.pair_units > 0) {
            switch (waves) {
            case 4:
                return launch_r<T, MT, G, S, FUSED, 256, kUnitsIn>(a, grid, ring, lds, s);
            case 8:
                return launch_r<T, MT, G, S, FUSED, 512, kUnitsIn>(a, grid, ring, lds, s);
            default:
                return launch_r<T, MT, G, S, FUSED, 1024, kUnitsIn>(a, grid, ring, lds, s);
            }
        }
    }
    if (a.units > 0 || a.pair_units > 0) {
        return hipErrorInvalidConfiguration;
    }
    switch (waves) {
    case 4:
        return launch_r<T, MT, G, S, FUSED, 256>(a, grid, ring, lds, s);
    case 8:
        return launch_r<T, MT, G, S, FUSED, 512>(a, grid, ring, lds, s);
    default:
        return launch_r<T, MT, G, S, FUSED, 1024>(a, grid, ring, lds, s);
    }
}

template <class T, int MT, int G>
hipError_t launch_g(const GemvArgs &a, bool fused, int strips_per_wave, dim3 grid, int waves, int ring, size_t lds, hipStream_t s) {
    if (fused) {
        return launch_s<T, MT, G, 2, true>(a, grid, waves, ring, lds, s);
    }
    if (strips_per_wave == 2) {
        return launch_s<T, MT, G, 2, false>(a, grid, waves, ring, lds, s);
    }
    return launch_s<T, MT, G, 1, false>(a, grid, waves, ring, lds, s);
}

template <class T, int MT>
hipError_t launch_m(const GemvArgs &a, int group, bool fused, int spw, dim3 grid, int waves, int ring, size_t lds, hipStream_t s) {
    if constexpr (MT == 2 * kFewRows) { // groups of 128 only (the planner's rule): no other group is instantiated
        return group == 128 ? launch_g<T, MT, 128>(a, fused, spw, grid, waves, ring, lds, s) : hipErrorInvalidConfiguration;
    } else {
        switch (group) {
        case 32:
            return launch_g<T, MT, 32>(a, fused, spw, grid, waves, ring, lds, s);
        case 64:
            return launch_g<T, MT, 64>(a, fused, spw, grid, waves, ring, lds, s);
        default:
            return launch_g<T, MT, 128>(a, fused, spw, grid, waves, ring, lds, s);
        }
    }
}

template <class T>
hipError_t launch_dtype(const GemvArgs &a, bool few, int group, bool fused, int spw, dim3 grid, int waves, int ring, size_t lds,
                        hipStream_t s) {
    if (a.m <= 1) {
        return launch_m<T, 1>(a, group, fused, spw, grid, waves, ring, lds, s);
    }
    if (few) {
        return a.m <= kFewRows ? launch_m<T, kFewRows>(a, group, fused, spw, grid, waves, ring, lds, s)
                               : launch_m<T, 2 * kFewRows>(a, group, fused, spw, grid, waves, ring, lds, s);
    }
    return launch_m<T, 16>(a, group, fused, spw, grid, waves, ring, lds, s);
}

} // namespace

namespace {

GemvPlan plan_gemv_uncached(const GemvCall &c, int64_t cus, bool allow_few = true) {
    GemvPlan p;
    const int64_t strips = c.fused ? 2 * (c.n / 16) : c.n / 16;
    // Few rows (no RMSNorm staging): the one-row launch shape and math, the rows staged one after another. Two to
    // four rows always (against the several-row kernels, with the group sums made by shuffles, Llama-3-8B layer at
    // M = 2 / 3 / 4: 24.1 / 24.5 / 25.0 -> 21.5 / 22.6 / 23.3 us, Llama-3.2-1B 14.4 / 14.3 / 14.7 -> 11.6 / 12.2 / 12.9,
    // Qwen2.5-14B 30.4 / 29.3 / 29.8 -> 28.5 / 28.5 / 30.0; the per-lane group sums took 0.4-1.9 us more off at 2..4
    // rows). Five to eight rows (two per lane group, groups of 128) only where the several-row plan
    // splits K and the rows fit LDS whole: the projections with K = 2048..4096 and N = 1024..6144 at M = 5 / 8
    // 7.1-8.7 -> 5.3-6.9 / 6.3-8.3 us, the Llama-3-8B and Llama-3.2-1B downs at 5 rows 11.4 / 7.9 -> 11.3 / 6.9; a
    // K split of the staged rows (Llama-3-8B down at 6 / 8 rows: 11.9 / 12.0 -> 14.7 / 16.2) and the large fused
    // gate_ups that the several-row kernel runs unsplit (Llama-3-8B at 8 rows: 15.1 -> 16.4) measured slower.
    // Staging the rows after the ring's first loads instead of before measured 1.4-2.5 us slower per layer.
    auto few_stage = [&](int64_t kts) {
        const int64_t kc = kts * 128;
        return static_cast<size_t>(c.m) * (static_cast<size_t>(((kc + 511) & ~int64_t{511}) + 8) * 2 +
                                           static_cast<size_t>(kc / c.w.group + 1) * sizeof(float2));
    };
    const size_t few_red = static_cast<size_t>(16 * 2 * c.m * 16) * sizeof(float); // the cross-wave sums of 16 waves
    bool few = false;
    if (allow_few && c.m >= 2 && c.norm_w == nullptr) {
        if (c.m <= kFewRows) {
            few = true;
        } else if (c.m <= 2 * kFewRows && c.w.group == 128 && few_stage(c.kt_count) + 16 + few_red <= kLdsMax) {
            few = plan_gemv_uncached(c, cus, false).splits > 1;
        }
    }
    const int64_t xrows = few ? c.m : 1;
    p.spw = c.fused ? 2 : (c.m > 1 && !few && strips % 2 == 0 ? 2 : 1);
    p.groups = strips / p.spw;
    // Staged activation bytes of a split of kts K tiles: one or few rows, x and its group sums per row (few rows:
    // x rounded up to whole 1 KiB transfers); several rows, rows_pad rows of x (m rounded up to a multiple of 4).
    auto stage_bytes = [&](int64_t kts) {
        const int64_t kc = kts * 128;
        if (few) {
            return few_stage(kts);
        }
        if (c.m == 1) {
            return static_cast<size_t>(kc + 8) * 2 + static_cast<size_t>(kc / c.w.group + 1) * sizeof(float2);
        }
        return static_cast<size_t>((c.m + 3) & ~int64_t{3}) * kc * 2;
    };
    // Several rows: LDS for the cross-wave sums, a lane-contiguous block of S x 4 rows for each wave past the
    // first of a strip group (over the staging space, after the multiply).
    auto rows_red = [&](int64_t wps, int64_t nu) { return static_cast<size_t>((wps - 1) * nu * p.spw * 4 * 64) * sizeof(float); };
    auto set_splits = [&](int64_t splits) {
        splits = std::min<int64_t>(std::max<int64_t>(splits, 1), c.kt_count);
        p.kt_per_split = (c.kt_count + splits - 1) / splits;
        p.splits = (c.kt_count + p.kt_per_split - 1) / p.kt_per_split;
    };
    p.wps = 1;
    p.nu = 1;
    p.few = few;
    if (c.m == 1 || few) {
        // K split only to bound the staged chunk (kXBudget: 256 K tiles at one row; few rows: the LDS less the
        // largest cross-wave sums, 16 waves x 2 strips x m rows).
        const int64_t max_tiles = static_cast<int64_t>(kXBudget) / 256;
        set_splits((c.kt_count + max_tiles - 1) / max_tiles);
        while (few && p.splits < c.kt_count && stage_bytes(p.kt_per_split) + 16 + few_red > kLdsMax) {
            set_splits(p.splits + 1);
        }
        // Waves per strip group: up to 8, keeping at least 8 K tiles per wave (16 with a strip pair: measured
        // on the Llama-3-8B gate_up, 32-tile wave runs in 448 workgroups beat 16-tile runs in 896); strip
        // groups per workgroup: enough for 4 waves.
        const int64_t min_run = 8 * p.spw;
        while (p.wps < 8 && p.kt_per_split >= 2 * min_run * p.wps) {
            p.wps *= 2;
        }
        // Strip pairs whose four-wave workgroups would leave CUs idle split K in two anyway (Llama-3.2-1B
        // gate_up: 512 pairs, 16 tiles; 256 workgroups of two pairs measured 6.0 us against 7.0 us for 128 of four).
        if (c.fused && p.wps == 1 && p.kt_per_split >= 16 && p.groups < 4 * cus) {
            p.wps = 2;
        }
        while (p.nu * p.wps < 4) {
            p.nu *= 2;
        }
        // Between one and two strip groups per CU (Qwen2.5-14B down: 320 strips), workgroups of twice the strips
        // run one round on fewer CUs: measured 11.2 µs against 12.1 µs for 320 workgroups.
        if (!c.fused && p.groups > cus && p.groups < 2 * cus && p.nu * p.wps <= 8) {
            p.nu *= 2;
        }
        // Few rows: the staged rows bound the workgroups a CU holds; where the grid would take more than one round of
        // them, workgroups of more strip groups share each staged chunk (Llama-3-8B down at 5..8 rows: two K splits
        // of 256 strips in 256 workgroups of two).
        while (few && p.nu * p.wps < 16) {
            const size_t lds = stage_bytes(p.kt_per_split) + 16 + static_cast<size_t>(p.nu * p.wps * p.spw * c.m * 16) * sizeof(float);
            const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(static_cast<int64_t>(kLdsMax / lds), 16 / (p.nu * p.wps)));
            if ((p.groups + p.nu - 1) / p.nu * p.splits <= per_cu * cus) {
                break;
            }
            p.nu *= 2;
        }
        // Units: given a spill for the pairs it may split, a fused call deals its (pair, K half) units evenly over
        // the CUs, ceil(2 pairs / CUs) waves per workgroup, where whole pairs per workgroup leave CUs with
        // unequal work (Llama-3-8B gate_up: 896 pairs in 448 workgroups of two put four pairs on 192 CUs and
        // two on the rest; seven halves on every CU: 12.72 us against 13.38 us under a kernel trace, while the down
        // GEMV that forms the split pairs takes 8.64 us against 7.79).
        if (c.m == 1 && c.fused && c.pair_spill != nullptr && p.splits == 1 && p.wps <= 2 && c.kt_count >= 2) {
            const int64_t u = (2 * p.groups + cus - 1) / cus;
            if (u >= 4 && u <= 16) {
                p.units = static_cast<int>(u);
                p.wps = 2;
                p.nu = 1;
            }
        }
    } else {
        // Several rows: the launch shape (K splits, waves per strip group, strip groups per workgroup) of least
        // cost over the candidates that fit LDS, where the cost multiplies
        //   the CU imbalance (the busiest CU's workgroups against the mean),
        //   the distance of the weight loads in flight over the launch (each wave holds min(ring, its run) steps
        //   of S tiles) from kRowsInFlight tiles: sqrt(target / in flight) below it and (in flight / target)^0.05
        //   above (more only lengthens the memory queues and the tail),
        //   1 + 0.05 x the staged activation bytes per weight byte (rows_pad / (4 nu S)),
        //   1 + 0.5 x the split's fp32 partial traffic per weight byte (written and read: 16 splits m / K), and
        //   1 + 0.25 per extra round of workgroups;
        // ties go to fewer splits, then to more waves per workgroup. The weights and exponents are fitted to
        // sweeps of every (splits, nu, wps) on the gate_up and down projections of Llama-3-8B, Qwen2.5-14B and
        // Llama-3.2-1B at 2, 4, 8, 12 and 16 rows (one graph of 60 launches per shape, the graphs' replays
        // interleaved, weights streamed from HBM): the rule's choice is within 5% of the best measured shape on all
        // 30 of them and 1.1% on average, against 10.8% (at worst 65%) for the rules it replaced.
        const int64_t rows_pad = (c.m + 3) & ~int64_t{3};
        const int gpt = static_cast<int>(128 / c.w.group);
        const int ring = std::max(1, (p.spw == 1 || gpt > 1 ? 4 : 8) / p.spw / (gpt == 4 ? 2 : 1)); // the kernel's KB
        double best = -1.0;
        for (int64_t sp = 1; sp <= std::min<int64_t>(c.kt_count, 16); ++sp) {
            const int64_t ktp = (c.kt_count + sp - 1) / sp;
            if ((c.kt_count + ktp - 1) / ktp != sp || (sp > 1 && sp * p.groups > kUnitsPerCu * cus)) {
                continue; // a split count that a smaller count already gives, or partials past the bound
            }
            const size_t stage = stage_bytes(ktp);
            for (int wps = 1; wps <= 4; wps *= 2) {
                for (int nu = 1; nu <= 8; nu *= 2) {
                    const int waves = nu * wps;
                    const size_t lds = std::max(stage, rows_red(wps, nu));
                    if ((waves != 4 && waves != 8 && waves != 16) || lds > kLdsMax) {
                        continue;
                    }
                    const int64_t wgs = (p.groups + nu - 1) / nu * sp;
                    const int64_t per_cu = std::min<int64_t>(static_cast<int64_t>(kLdsMax / lds), 16 / waves);
                    const int64_t rounds = (wgs + cus * per_cu - 1) / (cus * per_cu);
                    const int64_t tpw = (ktp + wps - 1) / wps;
                    const double inflight = static_cast<double>(p.groups * sp * wps * std::min<int64_t>(ring, tpw) * p.spw);
                    const double imb = static_cast<double>((wgs + cus - 1) / cus * cus) / static_cast<double>(wgs);
                    const double r = inflight / static_cast<double>(kRowsInFlight);
                    const double partial = sp > 1 ? 16.0 * static_cast<double>(sp * c.m) / static_cast<double>(c.kt_count * 128) : 0.0;
                    const double cost = imb * (r < 1.0 ? std::sqrt(1.0 / r) : std::pow(r, 0.05)) *
                                        (1.0 + 0.05 * static_cast<double>(rows_pad) / (4.0 * nu * p.spw)) * (1.0 + 0.5 * partial) *
                                        (1.0 + 0.25 * static_cast<double>(rounds - 1));
                    // Candidates come in order of splits, so equal costs keep fewer splits; within the same
                    // splits an equal cost takes the larger workgroup.
                    const bool lower = best < 0.0 || cost < best * (1.0 - 1e-9);
                    const bool tie_bigger = !lower && cost <= best * (1.0 + 1e-9) && sp == p.splits && waves > p.nu * p.wps;
                    if (lower || tie_bigger) {
                        best = cost;
                        p.kt_per_split = ktp;
                        p.splits = sp;
                        p.wps = wps;
                        p.nu = nu;
                    }
                }
            }
        }
        if (best < 0.0) {
            // No candidate within the partial bound: a long K whose staged chunk needs more splits than the bound allows
            // (K = 28672, N = 8192 at 12 or 16 rows). Take the fewest splits whose chunk fits LDS, one wave per strip
            // group and four groups per workgroup; the partial buffer follows this plan (gemv_partial_bound).
            const int64_t max_kt = std::max<int64_t>(1, static_cast<int64_t>(kLdsMax) / (rows_pad * 256));
            set_splits((c.kt_count + max_kt - 1) / max_kt);
            p.wps = 1;
            p.nu = 4;
        }
    }
    p.waves = p.units > 0 ? p.units : p.nu * p.wps;
    const size_t stage = stage_bytes(p.kt_per_split);
    const bool one_math = c.m == 1 || few;
    const size_t red = one_math ? static_cast<size_t>(p.waves) * p.spw * xrows * 16 * sizeof(float) : rows_red(p.wps, p.nu);
    // One or few rows: the staging, the RMSNorm's four partial sums (16 bytes), then the cross-wave sums; several
    // rows: the sums reuse the staging space.
    const size_t stage16 = (stage + 15) & ~static_cast<size_t>(15);
    p.lds = one_math ? stage16 + 16 + red : std::max(stage16, red);
    if (c.m == 1 && c.pair_units > 0) { // the split's split pairs' formed columns, 32 bytes a pair
        p.lds += static_cast<size_t>(32 * (p.kt_per_split * 8 / c.pair_units + 1));
    }
    p.partial_bytes = p.splits > 1 ? static_cast<size_t>(p.splits) * c.m * strips * 16 * sizeof(float) : 0;
    return p;
}

// The plan's inputs: the call's rows, columns, K tiles, fusion, group, pair spill and pair units, and the device's
// CU count.
struct PlanKey {
    int64_t m, n, kt_count, cus;
    int32_t group, pair_units;
    bool fused, spill;
    bool operator==(const PlanKey &o) const {
        return m == o.m && n == o.n && kt_count == o.kt_count && cus == o.cus && group == o.group && pair_units == o.pair_units &&
               fused == o.fused && spill == o.spill;
    }
};
struct PlanKeyHash {
    size_t operator()(const PlanKey &k) const {
        uint64_t h = 1469598103934665603ull;
        for (const uint64_t v : {static_cast<uint64_t>(k.m), static_cast<uint64_t>(k.n), static_cast<uint64_t>(k.kt_count),
                                 static_cast<uint64_t>(k.cus), static_cast<uint64_t>(k.group), static_cast<uint64_t>(k.pair_units),
                                 static_cast<uint64_t>(k.fused) | (static_cast<uint64_t>(k.spill) << 1)}) {
            h = (h ^ v) * 1099511628211ull;
        }
        return static_cast<size_t>(h);
    }
};

} // namespace

// Plans are cached per host thread (the several-row planner weighs up to a few hundred launch shapes, 1-3 us on the
// host, and each call plans twice), so repeated eager calls of one shape plan once.
GemvPlan plan_gemv(const GemvCall &c) {
    const int64_t cus = device_topology().cus;
    const PlanKey key{c.m, c.n, c.kt_count, cus, static_cast<int32_t>(c.w.group), static_cast<int32_t>(c.pair_units), c.fused,
                      c.pair_spill != nullptr};
    thread_local std::unordered_map<PlanKey, GemvPlan, PlanKeyHash> cache;
    const auto it = cache.find(key);
    if (it != cache.end()) {
        return it->second;
    }
    if (cache.size() >= 4096) {
        cache.clear();
    }
    const GemvPlan p = plan_gemv_uncached(c, cus);
    try {
        cache.emplace(key, p);
    } catch (const std::exception &) {
        // a failed host allocation only leaves the plan uncached
    }
    return p;
}

size_t gemv_pair_spill_bytes(int64_t channels) {
    // Split pairs are pairs U j + (U - 1) / 2 for odd U >= 5: at most pairs / 5 + 1, 64 floats each.
    return static_cast<size_t>(channels / 16 / 5 + 1) * 64 * sizeof(float);
}

size_t gemv_partial_bound(const GemvCall &c) {
    // With several rows a split launch has at most kUnitsPerCu (strip group, split) units per CU, whatever range
    // of the call's columns it covers.
    const GemvPlan p = plan_gemv(c);
    const size_t narrow = c.m > 1 ? static_cast<size_t>(kUnitsPerCu * device_topology().cus) * p.spw * c.m * 16 * sizeof(float) : 0;
    return std::max(p.partial_bytes, narrow);
}

namespace {

GemvArgs make_args(const GemvCall &c, const GemvPlan &p) {
    GemvArgs a{};
    a.quant = reinterpret_cast<const uint4 *>(c.w.quant);
    a.meta = c.w.meta;
    a.x = c.x;
    a.y = c.y;
    a.partial = p.splits > 1 ? c.partial : nullptr;
    a.ldx = c.ldx;
    a.ldy = c.ldy;
    a.kt_pitch = static_cast<int>(c.w.kt_pitch());
    a.kt_begin = static_cast<int>(c.kt_begin);
    a.kt_count = static_cast<int>(c.kt_count);
    a.kt_per_split = static_cast<int>(p.kt_per_split);
    a.strip_begin = static_cast<int>(c.strip_begin);
    a.groups = static_cast<int>(p.groups);
    a.m = static_cast<int>(c.m);
    a.ncols = static_cast<int>(p.groups * p.spw * 16);
    a.nu = p.nu;
    a.wps = p.wps;
    a.norm_w = c.norm_w;
    a.norm_eps = c.norm_eps;
    a.accumulate = c.accumulate;
    a.units = p.units;
    a.pair_units = c.pair_units;
    a.pair_spill = c.pair_spill;
    return a;
}

hipError_t launch_args(const GemvArgs &a, const GemvCall &c, const GemvPlan &p, unsigned splits, hipStream_t stream) {
    if (p.units > 0 ? (p.units > 16 || p.wps != 2 || splits != 1) : (p.waves != 4 && p.waves != 8 && p.waves != 16)) {
        return hipErrorInvalidConfiguration;
    }
    const dim3 grid(static_cast<unsigned>(p.units > 0 ? (2 * p.groups + p.units - 1) / p.units : (p.groups + p.nu - 1) / p.nu), splits);
    const int group = static_cast<int>(c.w.group);
    const int ring = ring_depth(static_cast<int64_t>(grid.x) * grid.y * p.waves);
    return c.w.dtype == 1 ? launch_dtype<F16>(a, p.few, group, c.fused, p.spw, grid, p.waves, ring, p.lds, stream)
                          : launch_dtype<BF16>(a, p.few, group, c.fused, p.spw, grid, p.waves, ring, p.lds, stream);
}

} // namespace

hipError_t launch_gemv(const GemvCall &c, hipStream_t stream) {
    // A consumer of pair units takes the odd counts a fused plan makes (5..15; its index arithmetic divides by the
    // count as a multiply-high, exact for 2..16).
    if (c.pair_units != 0 && (c.m != 1 || c.fused || c.pair_units < 5 || c.pair_units > 15 || c.pair_units % 2 == 0 ||
                              c.pair_spill == nullptr)) {
        return hipErrorInvalidValue;
    }
    const GemvPlan p = plan_gemv(c);
    const GemvArgs a = make_args(c, p);
    const hipError_t e = launch_args(a, c, p, static_cast<unsigned>(p.splits), stream);
    if (e != hipSuccess || p.splits == 1) {
        return e;
    }
    return launch_sum_splits(c.partial, c.y, c.ldy, c.m, a.ncols, static_cast<int>(p.splits), c.fused, c.w.dtype, stream, c.accumulate);
}

bool gemv_pair_supported(const GemvCall &c0, const GemvCall &c1) {
    return c0.m == 1 && c1.m == 1 && !c0.fused && !c1.fused && c0.n == c1.n && c0.strip_begin == c1.strip_begin &&
           c0.w.group == c1.w.group && c0.w.dtype == c1.w.dtype && c0.norm_w == nullptr && c1.norm_w == nullptr &&
           !c0.accumulate && !c1.accumulate && c1.kt_begin == 0 && plan_gemv(c0).splits == 1 && plan_gemv(c1).splits == 1;
}

size_t gemv_pair_partial_bytes(const GemvCall &c0) { return 2 * static_cast<size_t>(c0.m) * static_cast<size_t>(c0.n) * sizeof(float); }

hipError_t launch_gemv_pair(const GemvCall &c0, const GemvCall &c1, int64_t k0, hipStream_t stream) {
    // The launch shape of the longer share (its LDS covers the shorter one's staging); split s runs share s.
    GemvPlan p = plan_gemv(c0.kt_count >= c1.kt_count ? c0 : c1);
    p.splits = 2;
    GemvArgs a = make_args(c0, p);
    a.partial = c0.partial;
    a.kt_per_split = static_cast<int>(c0.kt_count);
    a.quant2 = reinterpret_cast<const uint4 *>(c1.w.quant);
    a.meta2 = c1.w.meta;
    a.kt_pitch2 = static_cast<int>(c1.w.kt_pitch());
    a.kt_count2 = static_cast<int>(c1.kt_count);
    a.k0 = static_cast<int>(k0);
    const hipError_t e = launch_args(a, c0, p, 2u, stream);
    if (e != hipSuccess) {
        return e;
    }
    return launch_sum_splits(c0.partial, c0.y, c0.ldy, c0.m, a.ncols, 2, false, c0.w.dtype, stream, false, true);
}

hipError_t launch_sum_splits(const float *partial, uint16_t *y, int64_t ldy, int64_t m, int ncols, int splits, bool fused,
                             int dtype, hipStream_t stream, bool accumulate, bool pairwise) {
    const int64_t total = m * (fused ? ncols / 2 : ncols) / 4; // four outputs per thread
    const dim3 blocks(static_cast<unsigned>((total + 255) / 256));
    const int mi = static_cast<int>(m);
    if (dtype == 1) {
        if (fused) {
            hipLaunchKernelGGL((sum_splits<F16, true>), blocks, dim3(256), 0, stream, partial, y, ldy, mi, ncols, splits, accumulate, pairwise);
        } else {
            hipLaunchKernelGGL((sum_splits<F16, false>), blocks, dim3(256), 0, stream, partial, y, ldy, mi, ncols, splits, accumulate, pairwise);
        }
    } else {
        if (fused) {
            hipLaunchKernelGGL((sum_splits<BF16, true>), blocks, dim3(256), 0, stream, partial, y, ldy, mi, ncols, splits, accumulate, pairwise);
        } else {
            hipLaunchKernelGGL((sum_splits<BF16, false>), blocks, dim3(256), 0, stream, partial, y, ldy, mi, ncols, splits, accumulate, pairwise);
        }
    }
    return hipGetLastError();
}

} // namespace hm

// Prefill W4A16 GEMM on the strip layout: v_mfma_f32_16x16x32 with the weights dequantized in registers.
//
// The B operand of v_mfma_f32_16x16x32 (lane l: column l % 16, K 8 (l / 16) .. + 7 of a 32-K step) is the
// strip layout itself (hm_device.hpp): one 16-byte load per lane brings a strip tile's four 32-K steps. So
// each wave loads the nibbles of its own strips straight from memory into registers (no LDS, and no other
// wave dequantizes the same columns), turns each step's dword into (q - z) * s in the activation type, and
// multiplies it with activation fragments read from LDS. The weight rounding to fp16 / bf16 happens once per
// weight, as in the reference GEMM (src/hipkernels/w4a16_gemm_packed.cu:491-497); accumulation is fp32.
//
// Workgroup = WN waves side by side over a BM x (32 WN) output tile (4 waves over 64 x 128 or 128 x 128, or 8
// waves over 128 x 256); a wave owns all BM = 16 RBW rows of 2 strips (32 columns), so each dequantized B
// operand feeds RBW MFMAs (8 at BM = 128: about two VALU instructions per MFMA). The activation tile (BM x 128
// per K tile) goes from memory straight into LDS (buffer_load ... lds, no registers) and serves all WN waves;
// its 16-byte chunks are XOR-swizzled by row so that an MFMA operand read touches 16 distinct bank groups; one
// barrier per K tile (per two K tiles for the 128 x 256 tiles).
//
// Software pipeline: while the MFMAs of 32-K step mu run, the VALU builds the B operands of step mu + 1 (of the
// next K tile at mu = 3) and the LDS delivers the activation fragments of step mu + 1; sched_group_barrier
// interleaves one MFMA with two VALU instructions. K tile kt + LOOK's weights and activations are requested at the
// start of K tile kt: LOOK = 1 (two buffers) for the 128 x 128 tiles, 3 (four buffers) for the 64-row tiles, whose
// small grids expose each workgroup's own latency, and 2 (four buffers, one barrier per two K tiles) for the
// 128 x 256 tiles.
//
// Tiles are dealt to XCDs in contiguous runs (workgroup i runs on XCD i % 8 on an MI355X) of an order that walks bands of 4
// row tiles column by column, so the workgroups resident on one XCD share both activation rows and weight
// columns in its L2.
//
// D element i of lane l is row 4 (l / 16) + i, column l % 16. Fused (gate_up, strips alternating gate / up
// per 16 channels): a wave's two strips are the gate and up columns of the same channels in the same lanes, so
// the epilogue writes SiLU(gate) * up with fp32 math and one rounding (kernels/gpu/src/gemm_w4a16.cu:229-275
// fuses the same way). Every output element accumulates in the same order for any M and tile shape. Small
// grids (under 128 workgroups, or 4-wave grids under two workgroups per CU) split the K range instead
// (blockIdx.y = split): each split writes fp32 partials and sum_splits adds them in split order, SwiGLU when
// fused.
#include "hm_device.hpp"
#include "hm_internal.hpp"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace hm {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct GemmArgs {
    const uint4 *quant;
    const uint32_t *meta;
    const uint16_t *x;
    uint16_t *y;
    float *partial; // [splits][m][ncols] fp32 when the K range is split
    int64_t ldx, ldy;
    int kt_pitch;
    int kt_begin, kt_count, kt_per_split;
    int strip_begin;
    int m;
    int ncols; // 16 * strips of the call
    int tiles_m, tiles_n;
    int accumulate; // plain output: y = round(y + round(sum)) instead of y = round(sum)
    int group_m;    // tile order: bands of group_m row tiles, column-major inside a band (1: row-major)
    int xcds;       // XCDs of the device: the dispatcher places workgroup i on XCD i % xcds
};

// Per (strip, group) dequantization constants, made once per K tile from the scale/zero record.
template <class T> struct Deq;
// fp16: d2 = (1024 + z) in both halves, s2 = s in both halves.
// fp16 with the wide nibble positions: pairs 1 and 3 of a dword come out as 1024 + 16 q, so they take
// d2w = 1024 + 16 z and s2w = s / 16 (exact for s >= 2^-10; smaller scales lose their low bits in s / 16).
template <> struct Deq<F16> {
    uint32_t d2, s2, d2w, s2w;
};
// bf16: s and -(128 + z) s in fp32 (both exact).
template <> struct Deq<BF16> {
    float s, ds;
};

__device__ __forceinline__ Deq<F16> make_deq(uint32_t rec, F16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t z = (rec >> 16) & 0xFFu;
    const uint32_t d = 0x6400u + z;      // fp16 bits of 1024 + z (z <= 16)
    const uint32_t dw = 0x6400u + 16u * z; // fp16 bits of 1024 + 16 z
    const uint32_t sb = rec & 0xFFFFu;
    const h2 s16 = __builtin_bit_cast(h2, sb | (sb << 16)) * h2{static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
    return Deq<F16>{d | (d << 16), sb | (sb << 16), dw | (dw << 16), __builtin_bit_cast(uint32_t, s16)};
}

__device__ __forceinline__ Deq<BF16> make_deq(uint32_t rec, BF16) {
    const float s = bf16_bits_to_float(rec & 0xFFFFu);
    return Deq<BF16>{s, -static_cast<float>((rec >> 16) & 0xFFu) * s};
}

// B operand of one 32-K step from one strip dword: (q - z) * s in the activation type.
// fp16: (1024 + q) - (1024 + z) is exact, one rounding in the multiply by s.
__device__ __forceinline__ uint4 dequant_operand(uint32_t w, const Deq<F16> &q, const MagicRegs &m) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 d2 = __builtin_bit_cast(h2, q.d2);
    const h2 s2 = __builtin_bit_cast(h2, q.s2);
    const h2 d2w = __builtin_bit_cast(h2, q.d2w);
    const h2 s2w = __builtin_bit_cast(h2, q.s2w);
    const uint32_t u = w >> 8;
    // dword i holds K elements 2i, 2i + 1 (nibbles i and 4 + i); (16 (q - z)) (s / 16) = (q - z) s exactly
    uint4 b;
    b.x = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, (w & m.lo) | m.magic) - d2) * s2);
    b.y = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, (w & m.hi) | m.magic) - d2w) * s2w);
    b.z = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, (u & m.lo) | m.magic) - d2) * s2);
    b.w = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, (u & m.hi) | m.magic) - d2w) * s2w);
    return b;
}

// bf16: exact (q - z) * s in fp32 (q * s and z * s carry at most 12 significant bits, so one FMA of them is
// exact), then one round to nearest even (v_cvt_pk_bf16_f32). The nibbles go to bytes with two masks (bytes of
// w & 0x0F0F0F0F hold nibbles 0, 2, 4, 6; of (w >> 4) & 0x0F0F0F0F nibbles 1, 3, 5, 7) and each byte to fp32
// with one v_cvt_f32_ubyte, as gfx950 has no packed bf16 arithmetic.
__device__ __forceinline__ uint4 dequant_operand(uint32_t w, const Deq<BF16> &q, const MagicRegs &m) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    (void)m;
    uint32_t e = w & 0x0F0F0F0Fu;        // nibbles 0, 2, 4, 6
    uint32_t o = (w >> 4) & 0x0F0F0F0Fu; // nibbles 1, 3, 5, 7
    // Opaque to the optimizer, which would otherwise fold the masks into per-byte shifts and masks instead of
    // the byte-selecting conversions.
    asm volatile("" : "+v"(e), "+v"(o));
    auto pair = [&](uint32_t src, int b0) __attribute__((always_inline)) {
        const float lo = static_cast<float>(static_cast<uint8_t>(src >> (8 * b0)));
        const float hi = static_cast<float>(static_cast<uint8_t>(src >> (8 * (b0 + 2))));
        const f2 r = {__builtin_fmaf(lo, q.s, q.ds), __builtin_fmaf(hi, q.s, q.ds)};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(r, b2));
    };
    // dword i holds K elements 2i, 2i + 1 (nibbles i and 4 + i)
    return uint4{pair(e, 0), pair(o, 0), pair(e, 1), pair(o, 1)};
}

template <class T, int G, int NSW> struct BTile {
    u32x4_t w[NSW];           // strip dwords of one K tile
    uint32_t r[NSW][128 / G]; // scale/zero records of its groups
};

template <class T, int G, bool FUSED, int RBW, int NSW, int WN, int DEPTH, int KPB = 1>
__global__ void __launch_bounds__(WN * 64) __attribute__((amdgpu_waves_per_eu(2))) gemm_kernel(GemmArgs a) {
    constexpr int WGS = WN * 64;
    constexpr int BM = RBW * 16;
    constexpr int BN = WN * NSW * 16;
    constexpr int GPT = 128 / G;
    constexpr int SPG = 4 / GPT;       // 32-K steps per group
    constexpr int ADMA = BM * 16 / WGS; // 1 KiB activation transfers per wave per K tile
    static_assert(ADMA * WGS == BM * 16, "activation transfers");
    // K tiles in flight: DEPTH - 1 tiles ahead of the one being multiplied, each with its weights in registers
    // and its activations in one of DEPTH LDS buffers. Per K tile a wave issues NB weight/record loads and ADMA
    // activation transfers, in that order; all of them count in vmcnt, in order.
    static_assert(DEPTH == 2 || DEPTH == 4, "pipeline depth");
    // KPB = 2: one barrier per two K tiles. Four LDS buffers, K tiles requested two ahead; the barrier after each odd
    // K tile waits for everything in flight (the next two tiles), and the buffer an iteration fills two tiles ahead was
    // last read before the previous barrier.
    static_assert(KPB == 1 || (KPB == 2 && DEPTH == 4), "two K tiles per barrier: four buffers");
    constexpr int LOOK = KPB == 2 ? 2 : DEPTH - 1; // K tiles requested ahead of the one being multiplied
    constexpr int NB = 2 * NSW;
    constexpr int AHEAD = KPB == 2 ? 0 : (DEPTH - 2) * (NB + ADMA); // loads issued after tile kt + 1's activations at iteration kt
    // Activation tile of one K tile: BM rows of 128 halves (256 B), 16-byte chunks XOR-swizzled by row
    // (chunk c of row r at slot c ^ (r % 16)), so the 16 rows one MFMA operand read touches fall on distinct banks.
    // Two separate arrays (not one [2][...]) so that the compiler can tell the buffers apart and does not
    // make reads of one wait for the transfers into the other.
    __shared__ __align__(1024) uint8_t as0[BM * 256];
    __shared__ __align__(1024) uint8_t as1[BM * 256];
    __shared__ __align__(1024) uint8_t as2[DEPTH > 2 ? BM * 256 : 16];
    __shared__ __align__(1024) uint8_t as3[DEPTH > 2 ? BM * 256 : 16];
    auto abuf = [&](int buf) __attribute__((always_inline)) { return buf == 0 ? as0 : buf == 1 ? as1 : buf == 2 ? as2 : as3; };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int col = lane & 15;
    const int h = lane >> 4;

    // Workgroup -> tile: XCD x = blockIdx.x % xcds takes a contiguous run of the tile order (row-major, or bands
    // of group_m row tiles walked column by column).
    const int nt = a.tiles_m * a.tiles_n;
    const int qx = nt / a.xcds, rx = nt % a.xcds;
    const int xcd = static_cast<int>(blockIdx.x) % a.xcds;
    const int lin = xcd * qx + min(xcd, rx) + static_cast<int>(blockIdx.x) / a.xcds;
    int tm, tn;
    if (a.group_m > 1) {
        const int band_tiles = a.group_m * a.tiles_n;
        const int band = lin / band_tiles;
        const int idx = lin - band * band_tiles;
        const int rows_in_band = min(a.group_m, a.tiles_m - band * a.group_m);
        tm = band * a.group_m + idx % rows_in_band;
        tn = idx / rows_in_band;
    } else {
        tm = lin / a.tiles_n;
        tn = lin - tm * a.tiles_n;
    }
    const int row0 = tm * BM;
    // K split (small grids only): this workgroup's K tiles [kt_lo, kt_lo + nkt) of the call.
    const int split = static_cast<int>(blockIdx.y);
    const int kt_lo = split * a.kt_per_split;
    const int nkt = min(a.kt_per_split, a.kt_count - kt_lo);

    // Buffer resources with per-wave bases; per K tile only the scalar offset moves.
    const int sbase = tn * (BN / 16) + wave * NSW; // first strip of this wave within the call
    const int64_t tile0 = static_cast<int64_t>(a.strip_begin + sbase) * a.kt_pitch + a.kt_begin + kt_lo;
    const uint32_t qstrip = static_cast<uint32_t>(a.kt_pitch) * 1024u;
    const uint32_t mstrip = static_cast<uint32_t>(a.kt_pitch) * 64u * GPT;
    const __amdgpu_buffer_rsrc_t qr = buffer_rsrc(reinterpret_cast<const uint8_t *>(a.quant) + tile0 * 1024, NSW * qstrip);
    const __amdgpu_buffer_rsrc_t mr = buffer_rsrc(reinterpret_cast<const uint8_t *>(a.meta) + tile0 * 64 * GPT, NSW * mstrip);
    const uint32_t ldx2 = static_cast<uint32_t>(a.ldx) * 2u;
    const int rows_here = min(BM, a.m - row0);
    if (rows_here <= 0) {
        return; // never for a consistent plan (its last tile row starts below M); a guard against one that is not
    }
    // x column 0 is the call's first K (kt_begin), as for the GEMV.
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(reinterpret_cast<const uint8_t *>(a.x) + static_cast<int64_t>(row0) * a.ldx * 2 +
                                                      static_cast<int64_t>(kt_lo) * 256,
                                                  static_cast<uint32_t>(rows_here - 1) * ldx2 + static_cast<uint32_t>(nkt) * 256u);
    // Transfer j of this wave fills LDS bytes [(wave * ADMA + j) KiB, +1 KiB): lane l -> slot p = 64 (wave ADMA + j) + l,
    // row p / 16, swizzled chunk p % 16 (so source chunk (p % 16) ^ (row % 16)). Rows past M read row M - 1.
    uint32_t xoff[ADMA];
#pragma unroll
    for (int j = 0; j < ADMA; ++j) {
        const int p = (wave * ADMA + j) * 64 + lane;
        const int r = p >> 4;
        const int c = (p & 15) ^ (r & 15);
        xoff[j] = static_cast<uint32_t>(min(r, rows_here - 1)) * ldx2 + static_cast<uint32_t>(c) * 16u;
    }
    const uint32_t qoff = static_cast<uint32_t>(lane) * 16u;
    const uint32_t moff = static_cast<uint32_t>(col) * GPT * 4u;

    auto load_b = [&](int kt, BTile<T, G, NSW> &bt) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < NSW; ++s) {
            const uint32_t mo = moff + s * mstrip;
            const uint32_t ms = static_cast<uint32_t>(kt) * (64u * GPT);
            if constexpr (GPT == 1) {
                bt.r[s][0] = __builtin_amdgcn_raw_buffer_load_b32(mr, mo, ms, 0);
            } else if constexpr (GPT == 2) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b64(mr, mo, ms, 0);
                bt.r[s][0] = v[0];
                bt.r[s][1] = v[1];
            } else {
                const auto v = __builtin_amdgcn_raw_buffer_load_b128(mr, mo, ms, 0);
                bt.r[s][0] = v[0];
                bt.r[s][1] = v[1];
                bt.r[s][2] = v[2];
                bt.r[s][3] = v[3];
            }
        }
#pragma unroll
        for (int s = 0; s < NSW; ++s) {
            bt.w[s] = __builtin_amdgcn_raw_buffer_load_b128(qr, qoff + s * qstrip, static_cast<uint32_t>(kt) * 1024u, 0);
        }
    };
    // Activation chunks of K tile kt straight into LDS buffer buf (no registers).
    auto load_a = [&](int kt, int buf) __attribute__((always_inline)) {
        const uint32_t so = static_cast<uint32_t>(kt) * 256u;
#pragma unroll
        for (int j = 0; j < ADMA; ++j) {
            lds_dma16(xr, abuf(buf) + (wave * ADMA + j) * 1024, xoff[j], so);
        }
    };

    float4_t acc[RBW][NSW];
#pragma unroll
    for (int rb = 0; rb < RBW; ++rb) {
#pragma unroll
        for (int s = 0; s < NSW; ++s) {
            acc[rb][s] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    const MagicRegs magic = magic_regs<T>();

    // Software pipeline over the 32-K steps: while the MFMAs of step mu run, the VALU builds the B operands of
    // step mu + 1 (of the next K tile when mu = 3) and the LDS delivers the activation fragments of step mu + 1.
    struct BOps {
        uint4 v[NSW];
    };
    struct AFr {
        uint4 v[RBW];
    };
    // B operands of step mu of tile bt with the constants dqg of its group; the constants are rebuilt when a group starts.
    auto dequant_step = [&](const BTile<T, G, NSW> &bt, Deq<T> (&dqg)[NSW], int mu, BOps &o) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < NSW; ++s) {
            if (mu % SPG == 0) {
                dqg[s] = make_deq(bt.r[s][mu / SPG], T{});
            }
            o.v[s] = dequant_operand(bt.w[s][mu], dqg[s], magic);
        }
    };
    // Fragment of row block rb, step mu: row rb * 16 + col, chunk 4 mu + h at its swizzled slot.
    const uint32_t aread = static_cast<uint32_t>(col) * 256u;
    auto read_a = [&](int buf, int mu, AFr &f) __attribute__((always_inline)) {
        const uint8_t *ab = abuf(buf) + aread + (((4 * mu + h) ^ col) << 4);
#pragma unroll
        for (int rb = 0; rb < RBW; ++rb) {
            f.v[rb] = *reinterpret_cast<const uint4 *>(ab + rb * 4096);
        }
    };

    // One K tile in pipeline slot `buf` (kt % DEPTH). On entry `op` holds step 0's B operands of `cur`, `dq` the
    // constants of `cur`, `fa` step 0's activation fragments; on exit the same for K tile kt + 1 (slot `nb`). The
    // tile DEPTH - 1 ahead goes into slot `lb` (that of K tile kt - 1, whose registers and LDS buffer were last
    // read before the previous barrier).
    auto iteration = [&](int kt, int buf, int nb, const BTile<T, G, NSW> &cur, const BTile<T, G, NSW> &nxt, BTile<T, G, NSW> &ld, int lb,
                         Deq<T> (&dq)[NSW], BOps &op, AFr &fa, auto odd) __attribute__((always_inline)) {
        constexpr bool kOdd = decltype(odd)::value; // KPB = 2: kt is odd (a barrier follows)
        const int ktn = min(kt + LOOK, nkt - 1); // the last iterations re-request the last tile; nothing reads it
        load_b(ktn, ld);
        load_a(ktn, lb);
#pragma unroll
        for (int mu = 0; mu < 4; ++mu) {
            BOps on;
            AFr fn;
            if (mu < 3) {
                read_a(buf, mu + 1, fn);
                dequant_step(cur, dq, mu + 1, on);
            } else {
                if constexpr (KPB == 2) {
                    // nxt's weights: at an odd kt they were requested one iteration ago, before nxt's and this
                    // iteration's transfers; at an even kt the barrier before this iteration already waited for them.
                    wait_vmcnt<kOdd ? 2 * ADMA + NB : ADMA + NB>();
                } else {
                    wait_vmcnt<ADMA + AHEAD>(); // nxt's weights (the transfers issued after them may still run)
                }
                dequant_step(nxt, dq, 0, on);
            }
            // strip-major: the operand of the last strip, finished at the end of the previous step, is needed last
#pragma unroll
            for (int s = 0; s < NSW; ++s) {
#pragma unroll
                for (int rb = 0; rb < RBW; ++rb) {
                    acc[rb][s] = T::mfma16(fa.v[rb], op.v[s], acc[rb][s]);
                }
            }
#pragma unroll
            for (int i = 0; i < RBW * NSW; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0); // then a share of the next step's operand build
            }
            __builtin_amdgcn_sched_barrier(0);
            op = on;
            if (mu < 3) {
                fa = fn;
            }
        }
        // The next tile's activations: this wave's transfers done, then everyone's.
        if constexpr (KPB == 1 || kOdd) {
            wait_vmcnt<AHEAD>();
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
        read_a(nb, 0, fa);
    };

    BTile<T, G, NSW> b[DEPTH];
#pragma unroll
    for (int t = 0; t < LOOK; ++t) {
        load_b(min(t, nkt - 1), b[t]);
        load_a(min(t, nkt - 1), t);
    }
    Deq<T> dq[NSW];
    BOps op;
    AFr fa;
    if constexpr (KPB == 2) {
        wait_vmcnt<2 * ADMA + NB>(); // tile 0's weights (tile 0's transfers and tile 1's loads may still run)
    } else {
        wait_vmcnt<ADMA + AHEAD>();
    }
    dequant_step(b[0], dq, 0, op);
    wait_vmcnt<AHEAD>();
    asm volatile("s_barrier" ::: "memory");
    read_a(0, 0, fa);
    // DEPTH K tiles per trip, so the register sets and LDS buffers rotate without copies.
    auto one = [&](int k, auto u) __attribute__((always_inline)) {
        constexpr int U = decltype(u)::value;
        using Parity = std::integral_constant<bool, U % 2 == 1>;
        iteration(k, U, (U + 1) % DEPTH, b[U], b[(U + 1) % DEPTH], b[(U + LOOK) % DEPTH], (U + LOOK) % DEPTH, dq, op, fa, Parity{});
    };
    int kt = 0;
    for (; kt + DEPTH - 1 < nkt; kt += DEPTH) {
        one(kt, std::integral_constant<int, 0>{});
        one(kt + 1, std::integral_constant<int, 1>{});
        if constexpr (DEPTH == 4) {
            one(kt + 2, std::integral_constant<int, 2>{});
            one(kt + 3, std::integral_constant<int, 3>{});
        }
    }
    if (kt < nkt) {
        one(kt, std::integral_constant<int, 0>{});
    }
    if constexpr (DEPTH == 4) {
        if (kt + 1 < nkt) {
            one(kt + 1, std::integral_constant<int, 1>{});
        }
        if (kt + 2 < nkt) {
            one(kt + 2, std::integral_constant<int, 2>{});
        }
    }

    if (a.partial != nullptr) {
        // K split: fp32 partials [split][m][ncols] (strip order, so a fused call's gate and up columns alternate
        // per 16), added by sum_splits. Rows past M fall outside the buffer and are dropped: the row offset is
        // part of the vector offset, which the buffer range check covers (the scalar offset is not checked).
        const uint32_t ldp4 = static_cast<uint32_t>(a.ncols) * 4u;
        const __amdgpu_buffer_rsrc_t pr =
            buffer_rsrc(a.partial + (static_cast<int64_t>(split) * a.m + row0) * a.ncols, static_cast<uint32_t>(rows_here) * ldp4);
        const uint32_t pcol = static_cast<uint32_t>(4 * h) * ldp4 + static_cast<uint32_t>(sbase * 16 + col) * 4u;
#pragma unroll
        for (int rb = 0; rb < RBW; ++rb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t ro = static_cast<uint32_t>(rb * 16 + i) * ldp4;
#pragma unroll
                for (int s = 0; s < NSW; ++s) {
                    // Element first: a bit cast of a vector element expression reads element 0.
                    const float v = acc[rb][s][i];
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), pr, pcol + ro + s * 64u, 0, 0);
                }
            }
        }
        return;
    }
    // Epilogue through a buffer covering this tile's valid rows: stores of rows past M fall outside it and are
    // dropped by the buffer range check, so no per-row branch. The row offset goes into the vector offset: the
    // range check covers the vector and instruction offsets, not the scalar offset.
    const uint32_t ldy2 = static_cast<uint32_t>(a.ldy) * 2u;
    const __amdgpu_buffer_rsrc_t yr = buffer_rsrc(a.y + static_cast<int64_t>(row0) * a.ldy, static_cast<uint32_t>(rows_here) * ldy2);
    const uint32_t ycol = static_cast<uint32_t>(4 * h) * ldy2 + static_cast<uint32_t>(FUSED ? sbase / 2 * 16 + col : sbase * 16 + col) * 2u;
#pragma unroll
    for (int rb = 0; rb < RBW; ++rb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t ro = static_cast<uint32_t>(rb * 16 + i) * ldy2;
            if constexpr (FUSED) {
#pragma unroll
                for (int s = 0; s < NSW; s += 2) {
                    const uint16_t v = T::from_float(silu(acc[rb][s][i]) * acc[rb][s + 1][i]);
                    __builtin_amdgcn_raw_buffer_store_b16(v, yr, ycol + ro + (s / 2) * 32u, 0, 0);
                }
            } else {
#pragma unroll
                for (int s = 0; s < NSW; ++s) {
                    uint16_t v = T::from_float(acc[rb][s][i]);
                    if (a.accumulate) {
                        v = T::from_float(T::to_float(__builtin_amdgcn_raw_buffer_load_b16(yr, ycol + ro + s * 32u, 0, 0)) + T::to_float(v));
                    }
                    __builtin_amdgcn_raw_buffer_store_b16(v, yr, ycol + ro + s * 32u, 0, 0);
                }
            }
        }
    }
}

template <class T, int G, int RBW, int NSW, int WN, int DEPTH, int KPB = 1>
hipError_t launch_cfg(const GemmArgs &a, bool fused, dim3 grid, hipStream_t s) {
    if (fused) {
        hipLaunchKernelGGL((gemm_kernel<T, G, true, RBW, NSW, WN, DEPTH, KPB>), grid, dim3(WN * 64), 0, s, a);
    } else {
        hipLaunchKernelGGL((gemm_kernel<T, G, false, RBW, NSW, WN, DEPTH, KPB>), grid, dim3(WN * 64), 0, s, a);
    }
    return hipGetLastError();
}

template <class T, int G> hipError_t launch_g(const GemmArgs &a, bool fused, int cfg, dim3 grid, hipStream_t s) {
    switch (cfg) {
    case 2:
        // 128 x 256, 8 waves of 128 x 32, 2 K tiles ahead in 4 buffers, one barrier per 2 K tiles (against one per K
        // tile, the same bits: Llama-3-8B M = 2048 gate_up 398.0 -> 392.9 us, down 193.9 -> 192.1, M = 512 down 67.9 ->
        // 66.1; Qwen2.5-14B layer at M = 1024 426.7 -> 416.4)
        return launch_cfg<T, G, 8, 2, 8, 4, 2>(a, fused, grid, s);
    case 1:
        return launch_cfg<T, G, 8, 2, 4, 2>(a, fused, grid, s); // 128 x 128, 4 waves of 128 x 32, 1 K tile ahead
    default:
        return launch_cfg<T, G, 4, 2, 4, 4>(a, fused, grid, s); // 64 x 128, 4 waves of 64 x 32, 3 K tiles ahead
    }
}

template <class T> hipError_t launch_t(const GemmArgs &a, int group, bool fused, int cfg, dim3 grid, hipStream_t s) {
    switch (group) {
    case 32:
        return launch_g<T, 32>(a, fused, cfg, grid, s);
    case 64:
        return launch_g<T, 64>(a, fused, cfg, grid, s);
    default:
        return launch_g<T, 128>(a, fused, cfg, grid, s);
    }
}

} // namespace

GemmPlan plan_gemm(const GemmCall &c) {
    GemmPlan p;
    const int64_t cus = device_topology().cus;
    const int64_t cols = c.fused ? 2 * c.n : c.n;
    const int64_t rows128 = (c.m + 127) / 128;
    // 128 x 128 tiles from 160 of them (5/8 of the CUs: measured on the Llama-3-8B and Qwen2.5-14B projections
    // at M = 256..2048, the taller tiles win once their grid is that large), else 64 x 128 (4 waves each).
    // 128 x 256 tiles (8 waves, one workgroup per CU; each staged activation tile feeds twice the strips) where
    // their grid is one round of 160..256 workgroups or six and more rounds: measured 4-7% faster there, and
    // 2-34% slower for one to six partial rounds and for small grids, where the 4-wave tiles balance better.
    // All three accumulate every output element in the same order, so without a K split a row block computed
    // alone gives the same bits as inside a larger call.
    p.cfg = rows128 * (cols / 128) >= 5 * cus / 8 ? 1 : 0;
    const int64_t wide = cols % 256 == 0 ? rows128 * (cols / 256) : 0;
    // A fused gate_up of 1.5 to 2 rounds of 128 x 256 tiles takes them too (the layer at M = 512: Llama-3-8B
    // -3.6%, Qwen2.5-14B -4.6%, bf16 -2.7%); the long-K down projections at such grids stay at 128 x 128
    // (15% slower otherwise).
    if (p.cfg == 1 && ((wide >= 5 * cus / 8 && wide <= cus) || wide >= 6 * cus || (c.fused && wide >= 3 * cus / 2 && wide < 2 * cus))) {
        p.cfg = 2;
    }
    // A plain long-K (down) projection of more than 128 rows whose 128 x 256 grid is under half the CUs takes
    // 128 x 256 tiles and splits K toward one round of them (below): Llama-3-8B down at M = 256 / 512, 8 / 4 splits
    // of 256 workgroups against 4 / 2 splits of 64 x 128 tiles, the layer 96.5 / 186.7 -> 94.2 / 176.1 µs.
    if (!c.fused && rows128 >= 2 && c.kt_count >= 64 && cols % 256 == 0 && wide < cus / 2) {
        p.cfg = 2;
    }
    // Tile shape of each configuration; launch_g instantiates the kernel with the same shape.
    const int64_t bm = p.cfg >= 1 ? 128 : 64;
    const int64_t bn = p.cfg == 2 ? 256 : 128;
    p.tiles_m = (c.m + bm - 1) / bm;
    p.tiles_n = cols / bn;
    p.kt_per_split = c.kt_count;
    p.splits = 1;
    p.partial_bytes = 0;
    // Grids of under 128 workgroups (a down projection at up to 128 rows) split K toward 256 workgroups, and
    // 4-wave grids of 128 to 511 workgroups (under two per CU: the down projection at 256..512 rows) toward 512,
    // with at least 8 K tiles per split (24 in the larger grids, where the partials' traffic must stay small
    // against each split's work) and fp32 partials within kGemmPartialMax. Measured on the Llama-3-8B layer,
    // against no split: M = 256 / 384 / 512 126.5 / 172.6 / 203.1 -> 102.7 / 164.4 / 196.7 µs (fp16), the bf16 and
    // Qwen2.5-14B shapes alike; aiming the small grids at 512 too was 2.7% slower at M = 128, and splitting
    // 32 K tiles in two (a 1024-column projection at M = 2048) slower. A row block's bits then depend on whether
    // its call splits (grids that do not split keep them).
    const int64_t wgs = p.tiles_m * p.tiles_n;
    const bool small = wgs < cus / 2;
    const int64_t aim = small ? cus : ((p.cfg == 0 || p.cfg == 1) && wgs < 2 * cus ? 2 * cus : 0);
    if (aim > 0 && c.kt_count >= 16) {
        int64_t splits = std::min<int64_t>((aim + wgs - 1) / wgs, c.kt_count / (small ? 8 : 24));
        while (splits > 1 && static_cast<size_t>(splits) * c.m * cols * sizeof(float) > kGemmPartialMax) {
            --splits;
        }
        if (splits > 1) {
            p.kt_per_split = (c.kt_count + splits - 1) / splits;
            p.splits = (c.kt_count + p.kt_per_split - 1) / p.kt_per_split;
            p.partial_bytes = static_cast<size_t>(p.splits) * c.m * cols * sizeof(float);
        }
    }
    return p;
}

hipError_t launch_gemm(const GemmCall &c, hipStream_t stream) {
    const GemmPlan p = plan_gemm(c);
    GemmArgs a;
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
    a.m = static_cast<int>(c.m);
    a.ncols = static_cast<int>(c.fused ? 2 * c.n : c.n);
    a.tiles_m = static_cast<int>(p.tiles_m);
    a.tiles_n = static_cast<int>(p.tiles_n);
    a.accumulate = c.accumulate && !c.fused ? 1 : 0;
    // Tile order: bands of 4 row tiles, column-major inside a band, so the 32 workgroups resident on one XCD
    // hold about 4 row blocks x 8 column blocks: 4 x 32 KiB of activations and 8 x 16 KiB of weights per K tile
    // through its L2, against 32 + 32 x 16 KiB in row-major order. Measured (same bits): Llama-3-8B layer at
    // M = 512 / 1024 / 2048 -2.2 / -1.7 / -1.7%, Qwen2.5-14B at M = 1024 / 2048 -1.7%; bands of 2 gained 1.2-1.4%,
    // of 8 and 16 less or nothing.
    a.group_m = 4;
    a.xcds = device_topology().xcds;
    const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n), static_cast<unsigned>(p.splits));
    const int group = static_cast<int>(c.w.group);
    hipError_t e = c.w.dtype == 1 ? launch_t<F16>(a, group, c.fused, p.cfg, grid, stream)
                                  : launch_t<BF16>(a, group, c.fused, p.cfg, grid, stream);
    if (e != hipSuccess || p.splits == 1) {
        return e;
    }
    return launch_sum_splits(c.partial, c.y, c.ldy, c.m, a.ncols, static_cast<int>(p.splits), c.fused, c.w.dtype, stream, c.accumulate);
}

} // namespace hm

// Prefill W4A16 GEMM on the strip layout: v_mfma_f32_16x16x32 with the weights dequantized in registers.
//
// The B operand of v_mfma_f32_16x16x32 (lane l: column l % 16, K 8 (l / 16) .. + 7 of a 32-K step) is the
// strip layout itself (hm_device.hpp): one 16-byte load per lane brings a strip tile's four 32-K steps. So
// each wave loads the nibbles of its own 4 strips straight from memory into registers (no LDS, and no other
// wave dequantizes the same columns), turns each step's dword into (q - z) * s in the activation type, and
// multiplies it with activation fragments read from LDS. The weight rounding to fp16 / bf16 happens once per
// weight, as in the reference GEMM (src/hipkernels/w4a16_gemm_packed.cu:491-497); accumulation is fp32.
//
// Workgroup = WM x WN waves over a BM x BN output tile, BM = WM * RBW * 16 rows, BN = WN * 64 columns; a wave
// owns RBW row blocks of 16 x its 4 strips. The activation tile (BM x 128 per K tile) is double-buffered in
// LDS: the next K tile's activation chunks and strip tiles are requested before the current one is
// multiplied, written to the other buffer after it, and one barrier per K tile separates the two.
//
// Tiles are dealt to XCDs in contiguous runs (workgroup i runs on XCD i % 8), row tile outermost, so the
// workgroups resident on one XCD share activation rows in its L2 while the weights stream.
//
// D element i of lane l is row 4 (l / 16) + i, column l % 16. Fused (gate_up, strips alternating gate / up
// per 16 channels): a wave's strips 2j and 2j + 1 are the gate and up columns of the same channels in the same
// lanes, so the epilogue writes SiLU(gate) * up with fp32 math and one rounding
// (kernels/gpu/src/gemm_w4a16.cu:229-275 fuses the same way). K splits write fp32 partials instead, which the
// split reduction adds (and applies SwiGLU to when fused).
#include "hm_device.hpp"
#include "hm_internal.hpp"

#include <algorithm>
#include <cstdlib>

namespace hm {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kAStride = 128 + 8; // halves per staged activation row (padding spreads LDS banks)

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
};

// Per (strip, group) dequantization constants, made once per K tile from the scale/zero record.
template <class T> struct Deq;
// fp16: d2 = (1024 + z) in both halves, s2 = s in both halves.
template <> struct Deq<F16> {
    uint32_t d2, s2;
};
// bf16: s and -(128 + z) s in fp32 (both exact).
template <> struct Deq<BF16> {
    float s, ds;
};

__device__ __forceinline__ Deq<F16> make_deq(uint32_t rec, F16) {
    const uint32_t d = 0x6400u | ((rec >> 16) & 0xFFu); // fp16 bits of 1024 + z (z < 16)
    const uint32_t sb = rec & 0xFFFFu;
    return Deq<F16>{d | (d << 16), sb | (sb << 16)};
}

__device__ __forceinline__ Deq<BF16> make_deq(uint32_t rec, BF16) {
    const float s = bf16_bits_to_float(rec & 0xFFFFu);
    return Deq<BF16>{s, -(128.0f + static_cast<float>((rec >> 16) & 0xFFu)) * s};
}

// B operand of one 32-K step from one strip dword: (q - z) * s in the activation type.
// fp16: (1024 + q) - (1024 + z) is exact, one rounding in the multiply by s.
__device__ __forceinline__ uint4 dequant_operand(uint32_t w, const Deq<F16> &q, const MagicRegs &m) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 d2 = __builtin_bit_cast(h2, q.d2);
    const h2 s2 = __builtin_bit_cast(h2, q.s2);
    uint4 b;
    uint32_t *o = reinterpret_cast<uint32_t *>(&b);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t v = ((w >> (4 * i)) & m.lo) | m.magic;
        o[i] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, v) - d2) * s2);
    }
    return b;
}

// bf16: exact (q - z) * s in fp32, then one round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint4 dequant_operand(uint32_t w, const Deq<BF16> &q, const MagicRegs &m) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    uint4 b;
    uint32_t *o = reinterpret_cast<uint32_t *>(&b);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t v = ((w >> (4 * i)) & m.lo) | m.magic;
        const f2 r = {__builtin_fmaf(__uint_as_float(v << 16), q.s, q.ds), __builtin_fmaf(__uint_as_float(v & 0xFFFF0000u), q.s, q.ds)};
        o[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, b2));
    }
    return b;
}

template <class T, int G, int NSW> struct BTile {
    u32x4_t w[NSW];                  // strip dwords of one K tile
    uint32_t r[NSW][128 / G];        // scale/zero records of its groups
};

template <class T, int G, bool FUSED, int WM, int WN, int RBW, int NSW, int OCC>
__global__ void __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(OCC))) gemm_kernel(GemmArgs a) {
    constexpr int WGS = WM * WN * 64;
    constexpr int BM = WM * RBW * 16;
    constexpr int BN = WN * NSW * 16;
    constexpr int GPT = 128 / G;
    constexpr int SPG = 4 / GPT;       // 32-K steps per group
    constexpr int ACH = BM * 16 / WGS; // 16-byte activation chunks per thread per K tile
    constexpr int AH = ACH / 2;
    static_assert(AH * 2 == ACH, "activation halves");
    __shared__ __align__(16) uint16_t as[2][BM * kAStride];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int wm = wave / WN;
    const int wn = wave % WN;
    const int col = lane & 15;
    const int h = lane >> 4;

    // Workgroup -> tile: XCD x = blockIdx.x % 8 takes a contiguous run of the row-major tile order.
    const int nt = a.tiles_m * a.tiles_n;
    const int q8 = nt / 8, r8 = nt % 8;
    const int xcd = static_cast<int>(blockIdx.x) % 8;
    const int lin = xcd * q8 + min(xcd, r8) + static_cast<int>(blockIdx.x) / 8;
    const int tm = lin / a.tiles_n;
    const int tn = lin - tm * a.tiles_n;
    const int row0 = tm * BM;
    const int nkt = a.kt_count;

    // Byte offsets (32-bit) from uniform bases, so loads take the scalar-base + vector-offset form.
    const uint8_t *qb = reinterpret_cast<const uint8_t *>(a.quant);
    const uint8_t *mb = reinterpret_cast<const uint8_t *>(a.meta);
    const uint8_t *xb = reinterpret_cast<const uint8_t *>(a.x);
    const int sbase = tn * (BN / 16) + wn * NSW; // strip index within the call
    const uint32_t tile0 = static_cast<uint32_t>(a.strip_begin + sbase) * a.kt_pitch + a.kt_begin;
    const uint32_t qoff = tile0 * 1024u + lane * 16u;
    const uint32_t moff = (tile0 * 16u + col) * GPT * 4u;
    const uint32_t qstrip = static_cast<uint32_t>(a.kt_pitch) * 1024u;
    const uint32_t mstrip = static_cast<uint32_t>(a.kt_pitch) * 64u * GPT;
    uint32_t aoff[ACH]; // activation chunk c = tid + WGS j: row c / 16 (rows past M read row M - 1), K 8 (c % 16)
#pragma unroll
    for (int j = 0; j < ACH; ++j) {
        const int c = tid + WGS * j;
        const uint32_t gr = static_cast<uint32_t>(min(row0 + (c >> 4), a.m - 1));
        aoff[j] = (gr * static_cast<uint32_t>(a.ldx) + static_cast<uint32_t>((c & 15) * 8)) * 2u;
    }

    u32x4_t av[AH];
    auto load_a = [&](int kt, int half) __attribute__((always_inline)) {
        const uint8_t *xk = xb + static_cast<uint32_t>(kt) * 256u;
#pragma unroll
        for (int j = 0; j < AH; ++j) {
            av[j] = *reinterpret_cast<const u32x4_t *>(xk + aoff[half * AH + j]);
        }
    };
    auto store_a = [&](int buf, int half) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < AH; ++j) {
            const int c = tid + WGS * (half * AH + j);
            *reinterpret_cast<u32x4_t *>(as[buf] + (c >> 4) * kAStride + (c & 15) * 8) = av[j];
        }
    };
    auto load_b = [&](int kt, BTile<T, G, NSW> &bt) __attribute__((always_inline)) {
        const uint8_t *mk = mb + static_cast<uint32_t>(kt) * (64u * GPT);
        const uint8_t *qk = qb + static_cast<uint32_t>(kt) * 1024u;
#pragma unroll
        for (int s = 0; s < NSW; ++s) {
            if constexpr (GPT == 1) {
                bt.r[s][0] = *reinterpret_cast<const uint32_t *>(mk + moff + s * mstrip);
            } else if constexpr (GPT == 2) {
                const uint2 v = *reinterpret_cast<const uint2 *>(mk + moff + s * mstrip);
                bt.r[s][0] = v.x;
                bt.r[s][1] = v.y;
            } else {
                const uint4 v = *reinterpret_cast<const uint4 *>(mk + moff + s * mstrip);
                bt.r[s][0] = v.x;
                bt.r[s][1] = v.y;
                bt.r[s][2] = v.z;
                bt.r[s][3] = v.w;
            }
        }
#pragma unroll
        for (int s = 0; s < NSW; ++s) {
            bt.w[s] = *reinterpret_cast<const u32x4_t *>(qk + qoff + s * qstrip);
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

    // One K tile: multiply `cur` with activation buffer `buf` while K tile `ktn` is requested into `nxt` and
    // the other buffer.
    auto iteration = [&](int kt, int buf, const BTile<T, G, NSW> &cur, BTile<T, G, NSW> &nxt) __attribute__((always_inline)) {
        const int ktn = min(kt + 1, nkt - 1); // the last iteration re-requests its own tile; nothing reads it
        load_a(ktn, 0);
        load_b(ktn, nxt);
        Deq<T> dq[NSW][GPT];
#pragma unroll
        for (int s = 0; s < NSW; ++s) {
#pragma unroll
            for (int g = 0; g < GPT; ++g) {
                dq[s][g] = make_deq(cur.r[s][g], T{});
            }
        }
        const uint16_t *ab = as[buf] + (wm * RBW * 16 + col) * kAStride + 8 * h;
#pragma unroll
        for (int mu = 0; mu < 4; ++mu) {
            uint4 bv[NSW];
#pragma unroll
            for (int s = 0; s < NSW; ++s) {
                bv[s] = dequant_operand(cur.w[s][mu], dq[s][mu / SPG], magic);
            }
#pragma unroll
            for (int rb = 0; rb < RBW; ++rb) {
                const uint4 a4 = *reinterpret_cast<const uint4 *>(ab + rb * 16 * kAStride + 32 * mu);
#pragma unroll
                for (int s = 0; s < NSW; ++s) {
                    acc[rb][s] = T::mfma16(a4, bv[s], acc[rb][s]);
                }
            }
            if (mu == 1) {
                store_a(buf ^ 1, 0); // that buffer was last read before the previous barrier
                load_a(ktn, 1);
            }
            __builtin_amdgcn_sched_barrier(0); // one 32-K step's fragments live at a time
        }
        store_a(buf ^ 1, 1);
        lds_barrier();
    };

    BTile<T, G, NSW> b0, b1;
    load_a(0, 0);
    load_b(0, b0);
    store_a(0, 0);
    load_a(0, 1);
    store_a(0, 1);
    lds_barrier();
    // Two K tiles per trip, so the register sets alternate without copies.
    int kt = 0;
    for (; kt + 1 < nkt; kt += 2) {
        iteration(kt, 0, b0, b1);
        iteration(kt + 1, 1, b1, b0);
    }
    if (kt < nkt) {
        iteration(kt, 0, b0, b1);
    }

    // Epilogue.
#pragma unroll
    for (int rb = 0; rb < RBW; ++rb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = row0 + wm * RBW * 16 + rb * 16 + 4 * h + i;
            if (row >= a.m) {
                continue;
            }
            if constexpr (FUSED) {
#pragma unroll
                for (int s = 0; s < NSW; s += 2) {
                    const int ch = (sbase + s) / 2 * 16 + col;
                    a.y[static_cast<int64_t>(row) * a.ldy + ch] = T::from_float(silu(acc[rb][s][i]) * acc[rb][s + 1][i]);
                }
            } else {
#pragma unroll
                for (int s = 0; s < NSW; ++s) {
                    a.y[static_cast<int64_t>(row) * a.ldy + (sbase + s) * 16 + col] = T::from_float(acc[rb][s][i]);
                }
            }
        }
    }
}

template <class T, int G, int WM, int WN, int RBW, int NSW, int OCC>
hipError_t launch_cfg(const GemmArgs &a, bool fused, dim3 grid, hipStream_t s) {
    if (fused) {
        hipLaunchKernelGGL((gemm_kernel<T, G, true, WM, WN, RBW, NSW, OCC>), grid, dim3(WM * WN * 64), 0, s, a);
    } else {
        hipLaunchKernelGGL((gemm_kernel<T, G, false, WM, WN, RBW, NSW, OCC>), grid, dim3(WM * WN * 64), 0, s, a);
    }
    return hipGetLastError();
}

template <class T, int G> hipError_t launch_g(const GemmArgs &a, bool fused, int cfg, dim3 grid, hipStream_t s) {
    switch (cfg) {
    case 2:
        return launch_cfg<T, G, 2, 2, 8, 4, 1>(a, fused, grid, s); // 256 x 128, 4 waves of 128 x 64
    case 1:
        return launch_cfg<T, G, 2, 2, 4, 4, 2>(a, fused, grid, s); // 128 x 128, 4 waves of 64 x 64
    default:
        return launch_cfg<T, G, 1, 2, 4, 4, 2>(a, fused, grid, s); // 64 x 128, 2 waves of 64 x 64
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

constexpr int kCUs = 256;

} // namespace

GemmPlan plan_gemm(const GemmCall &c) {
    GemmPlan p;
    const int64_t cols = c.fused ? 2 * c.n : c.n;
    // 128 x 128 tiles (4 waves) when their grid fills the chip, else 64 x 128 (2 waves). The K range is never
    // split: every output element then accumulates in the same order for any M and tile shape, so a row block
    // computed alone gives the same bits as inside a larger call.
    p.cfg = ((c.m + 127) / 128) * (cols / 128) >= kCUs ? 1 : 0;
    if (const char *v = std::getenv("HM_GEMM_CFG")) { // tuning override
        const int cfg = std::atoi(v);
        if (cfg >= 0 && cfg <= 2) {
            p.cfg = cfg;
        }
    }
    const int64_t bm = p.cfg == 2 ? 256 : p.cfg == 1 ? 128 : 64;
    const int64_t bn = 128;
    p.tiles_m = (c.m + bm - 1) / bm;
    p.tiles_n = cols / bn;
    p.kt_per_split = c.kt_count;
    p.splits = 1;
    p.partial_bytes = 0;
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
    const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n), static_cast<unsigned>(p.splits));
    const int group = static_cast<int>(c.w.group);
    hipError_t e = c.w.dtype == 1 ? launch_t<F16>(a, group, c.fused, p.cfg, grid, stream)
                                  : launch_t<BF16>(a, group, c.fused, p.cfg, grid, stream);
    if (e != hipSuccess || p.splits == 1) {
        return e;
    }
    return launch_sum_splits(c.partial, c.y, c.ldy, c.m, a.ncols, static_cast<int>(p.splits), c.fused, c.w.dtype, stream);
}

} // namespace hm

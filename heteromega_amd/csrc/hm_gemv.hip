// Decode W4A16 GEMV for M <= 16 rows on the strip layout, with an optional fused SwiGLU epilogue.
//
// Work split. Workgroup = `waves` wave64s over one unit: one strip (16 columns) or, fused, a strip pair
// (gate and up of the same 16 channels). The unit's K tiles are dealt to its waves round-robin. A wave reads
// one 1 KiB strip tile per step with one 16-byte load per lane, so each wave load instruction is fully
// coalesced. A wave requests its tiles in batches of up to 16 (one memory round trip per batch), after the
// activation chunks that the workgroup stages in LDS.
//
// Math per strip tile (4 MFMA steps of 32 K): the B operand is bias + q straight from the nibbles
// (hm_device.hpp), A is the activation rows from LDS (rows >= m are zero), so
//   P = sum_k x'_k (bias + q'_k)       (q' = q, or 16 q on the fp16 odd pairs with x' = x / 16)
//     = sum_k x_k q_k + Xb,            Xb = bias * sum_k x'_k
// and per group, with scale s and zero z of the column, sum_k x_k (q_k - z) s = s (P - Xb - z X), X = sum_k x_k.
// Xb and X per (row, group) are computed once when the workgroup stages x. This is the reference's
// per-tile factorization s (sum q x - z sum x) (kernels/gpu/src/gemv_w4a16.cu:91-98,
// src/cpu_avx_kernels/w4a16_gemv_avx_packed.cpp:242-253), applied to MFMA partial sums.
//
// Output: the waves of a strip add their partials through LDS. Plain: y = round(sum) or an fp32 partial for
// split-K. Fused: act = round(SiLU(gate) * up), fp32 math, one rounding (kernels/gpu/src/silu_mul.cu:10-30).
#include "hm_device.hpp"
#include "hm_internal.hpp"

#include <algorithm>

namespace hm {
namespace {


typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct GemvArgs {
    const uint4 *quant;
    const uint32_t *meta;
    const uint16_t *x;
    uint16_t *y;
    float *partial;
    int64_t ldx, ldy;
    int kt_pitch;
    int kt_begin, kt_count, kt_per_split;
    int strip_begin;
    int m;
    int n; // output columns or channels (row length of `partial`)
};

// Dynamic LDS: xs [m][KC] 16-bit, sums [m][KC / G] float2 (Xb, X), red [waves][m][16] float.
template <class T, int MT, int G, bool FUSED, int WGS>
__global__ void __launch_bounds__(WGS) gemv_kernel(GemvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NS = FUSED ? 2 : 1;
    constexpr int ROWS = MT < 4 ? MT : 4; // D elements per lane that can hold a real row
    constexpr int GPT = 128 / G;          // groups per strip tile
    constexpr int SPG = 4 / GPT;          // MFMA steps per group
    constexpr int KB = G >= 64 ? 16 : 8;  // weight tiles per wave per batch

    const int tid = threadIdx.x;
    const int waves = WGS / 64;
    const int wave = uniform(tid >> 6);
    const int lane = tid & 63;
    const int m = a.m;

    const int split = blockIdx.y;
    const int kt0 = a.kt_begin + split * a.kt_per_split;
    const int nkt = min(a.kt_per_split, a.kt_begin + a.kt_count - kt0);
    const int kc = nkt * 128;       // K values of this split
    const int kg = kc / G;          // groups of this split
    const int64_t xk0 = static_cast<int64_t>(kt0 - a.kt_begin) * 128;

    // Row strides padded by 16 bytes (x) and 8 bytes (sums) so that lanes reading different rows of one MFMA
    // operand or fold hit different LDS banks.
    const int xst = kc + 8;  // staged row stride, 16-bit elements
    const int sst = kg + 1;  // sums row stride, float2
    uint16_t *xs = reinterpret_cast<uint16_t *>(smem);
    float2 *sums = reinterpret_cast<float2 *>(smem + static_cast<size_t>(m) * xst * 2);
    float *red = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(sums) + static_cast<size_t>(m) * sst * sizeof(float2));

    // Tile stream of this wave: strip `strip`, a contiguous run of its local tiles.
    const int wps = waves / NS;          // waves per strip
    const int j = FUSED ? (wave & 1) : 0; // strip of this wave within the unit
    const int wi = FUSED ? (wave >> 1) : wave;
    const int strip = a.strip_begin + blockIdx.x * NS + j;
    const uint4 *qp = a.quant + (static_cast<int64_t>(strip) * a.kt_pitch + kt0) * 64; // wave-uniform base
    const int col = lane & 15;
    const int h = lane >> 4;
    const uint32_t *mp = a.meta + ((static_cast<int64_t>(strip) * a.kt_pitch + kt0) * 16 + col) * GPT;
    // Each wave of a strip takes a contiguous run of tiles [tb, te).
    const int tpw = (nkt + wps - 1) / wps;
    const int tb = wi * tpw;
    const int te = min(tb + tpw, nkt);

    // Memory requests go out in this order: the activation chunks this thread stages (up to kPre, held in
    // registers), then the wave's whole first batch of weight tiles and records. Staging then waits for the
    // activations only, so it costs one round trip and never waits for the weights. (LDS DMA loads would
    // save the registers, but the compiler then waits for vmcnt(0) before every LDS read.)
    constexpr int CPG = G / 8;              // 8-element activation chunks per group
    constexpr int kPre = MT == 1 ? 4 : 8;   // chunks per thread staged ahead of the weights
    const int chunks_row = kc / 8;
    const int total = m * chunks_row;
    uint4 xv[kPre];
    auto fetch = [&](int base) { // branch-free: chunks past the end re-read the last one and are not staged
#pragma unroll
        for (int c = 0; c < kPre; ++c) {
            const int idx = min(base + c * WGS + tid, total - 1);
            const int row = idx / chunks_row;
            xv[c] = *reinterpret_cast<const uint4 *>(a.x + row * a.ldx + xk0 + (idx - row * chunks_row) * 8);
        }
    };
    fetch(0);

    // A batch is KB consecutive tiles from i0. Indices past the wave's run are clamped to its last tile, so
    // the batch has no branches and the compiler can wait for each tile's loads separately (s_waitcnt vmcnt
    // counting down) instead of for all of them; the clamped copies are weighted by zero.
    uint4 wq[KB];
    uint32_t rq[KB][GPT];
    // The small record loads go first: folds then wait for them without waiting for the weight tiles.
    auto load = [&](int i0) {
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const int i = max(min(i0 + u, te - 1), 0); // a wave without tiles loads tile te - 1 >= 0 and skips it
            if constexpr (GPT == 1) {
                rq[u][0] = mp[i * 16];
            } else if constexpr (GPT == 2) {
                const uint2 r = *reinterpret_cast<const uint2 *>(mp + i * 32);
                rq[u][0] = r.x;
                rq[u][1] = r.y;
            } else {
                const uint4 r = *reinterpret_cast<const uint4 *>(mp + i * 64);
                rq[u][0] = r.x;
                rq[u][1] = r.y;
                rq[u][2] = r.z;
                rq[u][3] = r.w;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const int i = max(min(i0 + u, te - 1), 0);
            const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(qp + i * 64 + lane));
            wq[u] = uint4{v.x, v.y, v.z, v.w};
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    load(tb);

    // 1. Stage x into LDS (fp16: odd pairs scaled by 1/16) with the per-group sums. Consecutive lanes take
    //    consecutive 8-element chunks of a row, so one group is G / 8 consecutive lanes.
    auto stage = [&](int idx, uint4 v, bool valid) {
        float sa = 0.0f, sb = 0.0f;
        int row = 0, c8 = 0;
        if (valid) {
            row = idx / chunks_row;
            c8 = idx - row * chunks_row;
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
            if constexpr (T::kWide) {
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                const h2 sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
                v.y = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v.y) * sixteenth);
                v.w = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v.w) * sixteenth);
            }
            *reinterpret_cast<uint4 *>(xs + row * xst + c8 * 8) = v;
        }
#pragma unroll
        for (int off = 1; off < CPG; off <<= 1) {
            sa += __shfl_xor(sa, off);
            sb += __shfl_xor(sb, off);
        }
        if (valid && (c8 % CPG) == 0) {
            const float xb = T::kWide ? (1024.0f * sa + 64.0f * sb) : T::kBias * (sa + sb);
            sums[row * sst + c8 / CPG] = make_float2(xb, sa + sb);
        }
    };
#pragma unroll
    for (int c = 0; c < kPre; ++c) {
        const int idx = c * WGS + tid;
        stage(idx, xv[c], idx < total); // all lanes take part in the shuffles
    }
    for (int base = kPre * WGS; base < total; base += kPre * WGS) {
        fetch(base); // large M only: these chunks wait behind the weight batch
#pragma unroll
        for (int c = 0; c < kPre; ++c) {
            const int idx = base + c * WGS + tid;
            stage(idx, xv[c], idx < total);
        }
    }
    lds_barrier(); // not __syncthreads(): its fence would wait for the weight batch too

    // 2. Multiply.
    // A-operand row of this lane. Rows >= m read row m - 1 instead of zeros: they only feed D rows >= m,
    // which are never stored.
    const int arow = min(lane & 15, m - 1);
    const uint16_t *xa = xs + arow * xst + 8 * h;
    const MagicRegs magic = magic_regs<T>();

    float acc[ROWS];
#pragma unroll
    for (int e = 0; e < ROWS; ++e) {
        acc[e] = 0.0f;
    }
    int srow[ROWS]; // rows of the D elements, clamped to a staged row
#pragma unroll
    for (int e = 0; e < ROWS; ++e) {
        srow[e] = min(4 * h + e, m - 1);
    }

    auto compute = [&](int i0) {
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const int i = min(i0 + u, te - 1);
            const float live = (i0 + u < te) ? 1.0f : 0.0f;
            const uint32_t words[4] = {wq[u].x, wq[u].y, wq[u].z, wq[u].w};
            float4_t p = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int mu = 0; mu < 4; ++mu) {
                const uint4 av = *reinterpret_cast<const uint4 *>(xa + i * 128 + 32 * mu);
                const uint4 bv = magic_operand<T>(words[mu], magic);
                if (mu % SPG == 0) {
                    p = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
                }
                p = T::mfma16(av, bv, p);
                if (mu % SPG == SPG - 1) {
                    const int g = mu / SPG;
                    const uint32_t rr = rq[u][g];
                    const float s = T::to_float(rr & 0xFFFFu) * live;
                    const float z = static_cast<float>((rr >> 16) & 0xFFu);
                    const int gl = i * GPT + g; // local group index
#pragma unroll
                    for (int e = 0; e < ROWS; ++e) {
                        const float2 xsum = sums[srow[e] * sst + gl];
                        const float t = __builtin_fmaf(-z, xsum.y, p[e] - xsum.x);
                        acc[e] = __builtin_fmaf(s, t, acc[e]);
                    }
                }
            }
        }
    };

    for (int i0 = tb; i0 < te; i0 += KB) {
        compute(i0);
        if (i0 + KB < te) {
            load(i0 + KB);
        }
    }

    // 3. Add the waves of each strip, then write.
#pragma unroll
    for (int e = 0; e < ROWS; ++e) {
        const int row = 4 * h + e;
        if (row < m) {
            red[(wave * m + row) * 16 + col] = acc[e];
        }
    }
    __syncthreads();
    for (int o = tid; o < m * 16; o += WGS) {
        const int row = o >> 4;
        const int c = o & 15;
        float v[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            float t = 0.0f;
            for (int w = 0; w < wps; ++w) {
                t += red[((w * NS + s) * m + row) * 16 + c];
            }
            v[s] = t;
        }
        const int out_col = blockIdx.x * 16 + c;
        if constexpr (FUSED) {
            a.y[row * a.ldy + out_col] = T::from_float(silu(v[0]) * v[1]);
        } else if (a.partial != nullptr) {
            a.partial[(static_cast<int64_t>(split) * m + row) * a.n + out_col] = v[0];
        } else {
            a.y[row * a.ldy + out_col] = T::from_float(v[0]);
        }
    }
}

template <class T>
__global__ void __launch_bounds__(256) sum_splits(const float *__restrict__ partial, uint16_t *__restrict__ y, int64_t ldy, int m,
                                                  int n, int splits) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= static_cast<int64_t>(m) * n) {
        return;
    }
    const int row = static_cast<int>(idx / n);
    const int c = static_cast<int>(idx - static_cast<int64_t>(row) * n);
    float v = 0.0f;
    for (int s = 0; s < splits; ++s) {
        v += partial[(static_cast<int64_t>(s) * m + row) * n + c];
    }
    y[row * ldy + c] = T::from_float(v);
}

template <class T, int MT, int G, bool FUSED, int WGS>
hipError_t launch_w(const GemvArgs &a, dim3 grid, size_t lds, hipStream_t s) {
    auto kern = gemv_kernel<T, MT, G, FUSED, WGS>;
    static bool configured = false; // one attribute call per instantiation
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) {
            return e;
        }
        configured = true;
    }
    hipLaunchKernelGGL(kern, grid, dim3(WGS), lds, s, a);
    return hipGetLastError();
}

// Fused (gate/up pairs) runs 4 or 8 waves per workgroup, plain 4, 8 or 16.
template <class T, int MT, int G> hipError_t launch_g(const GemvArgs &a, bool fused, dim3 grid, int threads, size_t lds, hipStream_t s) {
    if (fused) {
        return threads >= 512 ? launch_w<T, MT, G, true, 512>(a, grid, lds, s) : launch_w<T, MT, G, true, 256>(a, grid, lds, s);
    }
    if constexpr (G == 128 && MT == 1) { // other shapes need more registers than 16 waves per CU allow
        if (threads >= 1024) {
            return launch_w<T, MT, G, false, 1024>(a, grid, lds, s);
        }
    }
    return threads >= 512 ? launch_w<T, MT, G, false, 512>(a, grid, lds, s) : launch_w<T, MT, G, false, 256>(a, grid, lds, s);
}

template <class T, int MT> hipError_t launch_m(const GemvArgs &a, int group, bool fused, dim3 grid, int threads, size_t lds, hipStream_t s) {
    switch (group) {
    case 32:
        return launch_g<T, MT, 32>(a, fused, grid, threads, lds, s);
    case 64:
        return launch_g<T, MT, 64>(a, fused, grid, threads, lds, s);
    default:
        return launch_g<T, MT, 128>(a, fused, grid, threads, lds, s);
    }
}

template <class T> hipError_t launch_dtype(const GemvArgs &a, int group, bool fused, dim3 grid, int threads, size_t lds, hipStream_t s) {
    if (a.m <= 1) {
        return launch_m<T, 1>(a, group, fused, grid, threads, lds, s);
    }
    if (a.m <= 4) {
        return launch_m<T, 4>(a, group, fused, grid, threads, lds, s);
    }
    return launch_m<T, 16>(a, group, fused, grid, threads, lds, s);
}

constexpr size_t kLdsBudget = 96 * 1024;

} // namespace

namespace {
// Waves per workgroup that a launch uses for c.waves.
int effective_waves(const GemvCall &c) {
    if (c.fused) {
        return c.waves >= 8 ? 8 : 4;
    }
    return (c.waves >= 16 && c.w.group == 128 && c.m == 1) ? 16 : c.waves >= 8 ? 8 : 4;
}

// LDS of one workgroup that stages kt_per_split K tiles.
size_t lds_for(const GemvCall &c, int64_t kt_per_split) {
    const int64_t kc = kt_per_split * 128;
    const size_t xs = static_cast<size_t>(c.m) * (kc + 8) * 2;
    const size_t sums = static_cast<size_t>(c.m) * (kc / c.w.group + 1) * sizeof(float2);
    const size_t red = static_cast<size_t>(effective_waves(c)) * c.m * 16 * sizeof(float);
    return xs + sums + red;
}
} // namespace

size_t gemv_lds_bytes(const GemvCall &c, int splits) { return lds_for(c, (c.kt_count + splits - 1) / splits); }

int gemv_pick_splits(const GemvCall &c) {
    if (c.fused) {
        return 1; // the SwiGLU epilogue needs whole sums
    }
    int splits = 1;
    while (gemv_lds_bytes(c, splits) > kLdsBudget && splits < c.kt_count) {
        ++splits;
    }
    return splits;
}

size_t gemv_partial_bytes(const GemvCall &c) {
    const int splits = gemv_pick_splits(c);
    return splits > 1 ? static_cast<size_t>(splits) * c.m * c.n * sizeof(float) : 0;
}

hipError_t launch_gemv(const GemvCall &c, hipStream_t stream) {
    GemvArgs a;
    a.quant = reinterpret_cast<const uint4 *>(c.w.quant);
    a.meta = c.w.meta;
    a.x = c.x;
    a.y = c.y;
    a.ldx = c.ldx;
    a.ldy = c.ldy;
    a.kt_pitch = static_cast<int>(c.w.kt_pitch());
    a.kt_begin = static_cast<int>(c.kt_begin);
    a.kt_count = static_cast<int>(c.kt_count);
    a.strip_begin = static_cast<int>(c.strip_begin);
    a.m = static_cast<int>(c.m);
    a.n = static_cast<int>(c.n);
    const int splits = c.splits > 0 ? c.splits : 1;
    a.kt_per_split = static_cast<int>((c.kt_count + splits - 1) / splits);
    const int real_splits = static_cast<int>((c.kt_count + a.kt_per_split - 1) / a.kt_per_split);
    a.partial = real_splits > 1 ? c.partial : nullptr;
    const int units = static_cast<int>(c.n / 16);
    const dim3 grid(units, real_splits);
    const int threads = effective_waves(c) * 64;
    const size_t lds = lds_for(c, a.kt_per_split);
    const int group = static_cast<int>(c.w.group);
    hipError_t e = c.w.dtype == 1 ? launch_dtype<F16>(a, group, c.fused, grid, threads, lds, stream)
                                  : launch_dtype<BF16>(a, group, c.fused, grid, threads, lds, stream);
    if (e != hipSuccess || real_splits == 1) {
        return e;
    }
    const int64_t total = c.m * c.n;
    if (c.w.dtype == 1) {
        hipLaunchKernelGGL(sum_splits<F16>, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, c.partial, c.y,
                           c.ldy, static_cast<int>(c.m), static_cast<int>(c.n), real_splits);
    } else {
        hipLaunchKernelGGL(sum_splits<BF16>, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, c.partial, c.y,
                           c.ldy, static_cast<int>(c.m), static_cast<int>(c.n), real_splits);
    }
    return hipGetLastError();
}

} // namespace hm

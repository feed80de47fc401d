// Prefill W4A16 GEMM on the strip layout: v_mfma_f32_32x32x16 with the weights dequantized in registers.
//
// Workgroup = 4 waves (2 x 2) over a BM x BN output tile; each wave owns (BM / 2) x (BN / 2) as 32 x 32 MFMA
// blocks. Per 128-K step the workgroup stages the activation tile (BM x 128, row-major with a padded stride)
// and the raw strip tiles (BN / 16 KiB of nibbles plus their scale/zero records) in LDS, then each wave turns
// its B fragments into (q - z) * s in the activation type and runs the MFMAs with fp32 accumulation.
// The weight rounding to fp16 / bf16 happens once per weight, as in the reference GEMM
// (src/hipkernels/w4a16_gemm_packed.cu:491-497).
//
// MFMA 32x32x16 operands (gfx950): A lane l holds row l % 32, K 8 (l / 32) .. + 7; B lane l holds column l % 32,
// the same K; D element 4 jj + ii of lane l is row 8 jj + 4 (l / 32) + ii, column l % 32.
//
// Fused (gate_up, strips alternating gate / up per 16 channels): a 32-column block is 16 gate and 16 up columns
// of the same channels, so lane l and lane l ^ 16 hold gate and up of one (row, channel); the epilogue writes
// SiLU(gate) * up, fp32 math and one rounding (kernels/gpu/src/gemm_w4a16.cu:229-275 fuses the same way).
#include "hm_device.hpp"
#include "hm_internal.hpp"

namespace hm {
namespace {

constexpr int kAStride = 128 + 8; // halves per staged activation row (padding spreads LDS banks)

struct GemmArgs {
    const uint4 *quant;
    const uint32_t *meta;
    const uint16_t *x;
    uint16_t *y;
    int64_t ldx, ldy;
    int kt_pitch;
    int kt_begin, kt_count;
    int strip_begin;
    int m;
};

template <class T> __device__ __forceinline__ uint4 dequant_operand(uint32_t w, uint32_t rec);

// fp16: (bias + q) - (bias + z) is exact, one rounding in the multiply by s.
template <> __device__ __forceinline__ uint4 dequant_operand<F16>(uint32_t w, uint32_t rec) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const _Float16 s = __builtin_bit_cast(_Float16, static_cast<uint16_t>(rec & 0xFFFFu));
    const _Float16 d = static_cast<_Float16>(1024.0f + static_cast<float>((rec >> 16) & 0xFFu));
    const h2 s2 = {s, s};
    const h2 d2 = {d, d};
    uint4 b;
    uint32_t *o = reinterpret_cast<uint32_t *>(&b);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t v = ((w >> (4 * i)) & 0x000F000Fu) | F16::kMagic;
        o[i] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, v) - d2) * s2);
    }
    return b;
}

// bf16: exact (q - z) * s in fp32, then one round to nearest even.
template <> __device__ __forceinline__ uint4 dequant_operand<BF16>(uint32_t w, uint32_t rec) {
    const float s = bf16_bits_to_float(rec & 0xFFFFu);
    const float ds = -(128.0f + static_cast<float>((rec >> 16) & 0xFFu)) * s;
    uint4 b;
    uint32_t *o = reinterpret_cast<uint32_t *>(&b);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t v = ((w >> (4 * i)) & 0x000F000Fu) | BF16::kMagic;
        const float lo = __builtin_fmaf(__uint_as_float(v << 16), s, ds);
        const float hi = __builtin_fmaf(__uint_as_float(v & 0xFFFF0000u), s, ds);
        o[i] = static_cast<uint32_t>(float_to_bf16_bits(lo)) | (static_cast<uint32_t>(float_to_bf16_bits(hi)) << 16);
    }
    return b;
}

template <class T, int BM, int BN, int G, bool FUSED>
__global__ void __launch_bounds__(256) gemm_kernel(GemmArgs a) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int RB = WM / 32, CB = WN / 32;
    constexpr int NSTRIP = BN / 16;
    constexpr int GPT = 128 / G;
    __shared__ __align__(16) uint16_t as[BM * kAStride];
    __shared__ __align__(16) uint32_t bs[NSTRIP * 256];        // raw strip tiles, 1 KiB each
    __shared__ __align__(16) uint32_t ms[NSTRIP * GPT * 16];   // records of the tile's groups

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = (wave >> 1) * WM;
    const int wn0 = (wave & 1) * WN;
    const int m0 = blockIdx.y * BM;
    const int strip0 = a.strip_begin + blockIdx.x * NSTRIP;

    float16_t acc[RB][CB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
#pragma unroll
        for (int c = 0; c < CB; ++c) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                acc[r][c][e] = 0.0f;
            }
        }
    }

    const int l32 = lane & 31;
    const int hi = lane >> 5;

    for (int i = 0; i < a.kt_count; ++i) {
        const int t = a.kt_begin + i;
        // Stage A: BM rows x 128 K, 16 chunks of 8 per row.
        for (int c = tid; c < BM * 16; c += 256) {
            const int row = c >> 4;
            const int k8 = c & 15;
            uint4 v = {0u, 0u, 0u, 0u};
            if (m0 + row < a.m) {
                v = *reinterpret_cast<const uint4 *>(a.x + static_cast<int64_t>(m0 + row) * a.ldx + static_cast<int64_t>(i) * 128 + k8 * 8);
            }
            *reinterpret_cast<uint4 *>(as + row * kAStride + k8 * 8) = v;
        }
        // Stage B: NSTRIP tiles of 64 uint4.
        for (int c = tid; c < NSTRIP * 64; c += 256) {
            const int sj = c >> 6;
            const int l = c & 63;
            const uint4 v = a.quant[(static_cast<int64_t>(strip0 + sj) * a.kt_pitch + t) * 64 + l];
            *reinterpret_cast<uint4 *>(bs + c * 4) = v;
        }
        for (int c = tid; c < NSTRIP * GPT * 16; c += 256) {
            const int sj = c / (GPT * 16);
            const int r = c % (GPT * 16);
            ms[c] = a.meta[((static_cast<int64_t>(strip0 + sj) * a.kt_pitch + t) * 16 + (r & 15)) * GPT + r / 16];
        }
        __syncthreads();

#pragma unroll 2
        for (int nu = 0; nu < 8; ++nu) {
            const int kl = 16 * nu + 8 * hi; // K offset of this lane's 8 values inside the tile
            uint4 av[RB];
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                av[r] = *reinterpret_cast<const uint4 *>(as + (wm0 + 32 * r + l32) * kAStride + kl);
            }
            uint4 bv[CB];
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                const int colb = wn0 + 32 * c + l32; // column inside the block tile
                const int sj = colb >> 4;
                const int mu = kl >> 5;
                const int hh = (kl >> 3) & 3;
                const uint32_t w = bs[sj * 256 + ((hh << 4) | (colb & 15)) * 4 + mu];
                const uint32_t rec = ms[(sj * GPT + kl / G) * 16 + (colb & 15)];
                bv[c] = dequant_operand<T>(w, rec);
            }
#pragma unroll
            for (int r = 0; r < RB; ++r) {
#pragma unroll
                for (int c = 0; c < CB; ++c) {
                    acc[r][c] = T::mfma32(av[r], bv[c], acc[r][c]);
                }
            }
        }
        __syncthreads();
    }

    // Epilogue.
#pragma unroll
    for (int r = 0; r < RB; ++r) {
#pragma unroll
        for (int c = 0; c < CB; ++c) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm0 + 32 * r + 8 * (e >> 2) + 4 * hi + (e & 3);
                const float v = acc[r][c][e];
                if constexpr (FUSED) {
                    const float other = __shfl_xor(v, 16);
                    if ((l32 & 16) == 0 && row < a.m) {
                        // channel: half of the block's first column, plus this lane's gate column
                        const int ch = (blockIdx.x * BN + wn0 + 32 * c) / 2 + l32;
                        a.y[static_cast<int64_t>(row) * a.ldy + ch] = T::from_float(silu(v) * other);
                    }
                } else {
                    if (row < a.m) {
                        const int colg = blockIdx.x * BN + wn0 + 32 * c + l32;
                        a.y[static_cast<int64_t>(row) * a.ldy + colg] = T::from_float(v);
                    }
                }
            }
        }
    }
}

template <class T, int BM, int BN, int G>
hipError_t launch_fg(const GemmArgs &a, bool fused, dim3 grid, hipStream_t s) {
    if (fused) {
        hipLaunchKernelGGL((gemm_kernel<T, BM, BN, G, true>), grid, dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL((gemm_kernel<T, BM, BN, G, false>), grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

template <class T, int BM, int BN>
hipError_t launch_t(const GemmArgs &a, int group, bool fused, dim3 grid, hipStream_t s) {
    switch (group) {
    case 32:
        return launch_fg<T, BM, BN, 32>(a, fused, grid, s);
    case 64:
        return launch_fg<T, BM, BN, 64>(a, fused, grid, s);
    default:
        return launch_fg<T, BM, BN, 128>(a, fused, grid, s);
    }
}

} // namespace

hipError_t launch_gemm(const GemmCall &c, hipStream_t stream) {
    constexpr int BM = 128, BN = 128;
    GemmArgs a;
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
    // Columns of the weight block: n (plain) or 2 n (fused). Must be a multiple of BN.
    const int64_t cols = c.fused ? 2 * c.n : c.n;
    const dim3 grid(static_cast<unsigned>(cols / BN), static_cast<unsigned>((c.m + BM - 1) / BM));
    const int group = static_cast<int>(c.w.group);
    return c.w.dtype == 1 ? launch_t<F16, BM, BN>(a, group, c.fused, grid, stream) : launch_t<BF16, BM, BN>(a, group, c.fused, grid, stream);
}

} // namespace hm

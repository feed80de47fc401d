// Device helpers shared by the gfx950 kernels: 16-bit float conversions, the
// strip-layout constants and the MFMA wrappers.
//
// Strip layout (one matrix W[K, N], y = x W, int4 q, group size g | 128):
//   quant plane: strip s = n / 16, K tile t = k / 128, 1 KiB per (s, t):
//     byte ((s * kt_pitch + t) * 64 + L) * 16 + 4 * mu holds, for lane L and dword mu in 0..3,
//     column 16 s + (L & 15) and K = 128 t + 32 mu + 8 (L >> 4) + e, e = 0..7,
//     nibble p(e) = e / 2 for even e and 4 + e / 2 for odd e.
//   That is the B-operand order of v_mfma_f32_16x16x32_{f16,bf16}: lane L holds column
//   L & 15 and 8 consecutive K of one 32-K step. With the nibble order, masking a dword
//   with 0x000F000F (after a shift by 4 i) gives the pair (e = 2 i, e = 2 i + 1) in the
//   two 16-bit halves, so OR-ing the exponent of 1024 (fp16) or 128 (bf16) makes the
//   operand without a conversion instruction.
//   meta plane: one uint32 record per (strip, column, group), blocked like the quant plane: the records of
//   tile (s, t) are 16 columns x (128 / g) groups, contiguous, groups innermost, so a lane's records for a
//   tile are one 4-, 8- or 16-byte load and a wave's records for a tile share one cache line or two:
//     record ((s * kt_pitch + t) * 16 + (n & 15)) * (128 / g) + (k % 128) / g = scale bits | zero << 16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hm {

constexpr int kTileK = 128;      // K rows per strip tile
constexpr int kStrip = 16;       // columns per strip
constexpr int kTileBytes = 1024; // nibble bytes per strip tile

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b) { return __uint_as_float(b << 16); }

// Round to nearest even; NaN stays NaN (quiet bit set).
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return static_cast<uint16_t>((u >> 16) | 0x40u);
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Activation / scale element type. kMagic is the exponent pattern that turns a nibble in
// the low mantissa bits into bias + q. kWide is true when the nibble at bits 4..7 of each
// half also fits the mantissa (fp16: 1024 + 16 q), which saves a shift per pair.
struct F16 {
    static constexpr uint32_t kMagic = 0x64006400u;
    static constexpr float kBias = 1024.0f;
    static constexpr bool kWide = true;
    __device__ static __forceinline__ float to_float(uint32_t bits) { return half_bits_to_float(bits); }
    __device__ static __forceinline__ uint16_t from_float(float f) { return float_to_half_bits(f); }
    __device__ static __forceinline__ float4_t mfma16(uint4 a, uint4 b, float4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                       0, 0, 0);
    }
};

struct BF16 {
    static constexpr uint32_t kMagic = 0x43004300u;
    static constexpr float kBias = 128.0f;
    static constexpr bool kWide = false;
    __device__ static __forceinline__ float to_float(uint32_t bits) { return bf16_bits_to_float(bits); }
    __device__ static __forceinline__ uint16_t from_float(float f) { return float_to_bf16_bits(f); }
    __device__ static __forceinline__ float4_t mfma16(uint4 a, uint4 b, float4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                        c, 0, 0, 0);
    }
};

// Nibble position of K offset e (0..7) inside a strip dword.
__host__ __device__ __forceinline__ int nibble_of(int e) { return (e & 1) ? 4 + (e >> 1) : (e >> 1); }

// Loop-invariant constants of the operand build, held in VGPRs. With all three operands in registers,
// instruction selection turns (w & mask) | bits into one v_and_or_b32 (gfx9 VOP3 takes no literal). The
// empty asm only hides the constant values from the optimizer; it runs once per kernel.
struct MagicRegs {
    uint32_t lo, hi, magic;
};

template <class T> __device__ __forceinline__ MagicRegs magic_regs() {
    MagicRegs r{0x000F000Fu, 0x00F000F0u, T::kMagic};
    asm volatile("" : "+v"(r.lo), "+v"(r.hi), "+v"(r.magic));
    return r;
}

// B operand of one 32-K MFMA step from one strip dword: eight values bias + q_e (F16 with
// kWide: the odd pairs hold bias + 16 q_e, and the caller scales the matching activations by 1/16).
template <class T> __device__ __forceinline__ uint4 magic_operand(uint32_t w, const MagicRegs &c) {
    uint4 b;
    if constexpr (T::kWide) {
        const uint32_t u = w >> 8;
        b.x = (w & c.lo) | c.magic;
        b.y = (w & c.hi) | c.magic;
        b.z = (u & c.lo) | c.magic;
        b.w = (u & c.hi) | c.magic;
    } else {
        b.x = (w & c.lo) | c.magic;
        b.y = ((w >> 4) & c.lo) | c.magic;
        b.z = ((w >> 8) & c.lo) | c.magic;
        b.w = ((w >> 12) & c.lo) | c.magic;
    }
    return b;
}

// Buffer resource over [base, base + bytes): loads past the end return zero instead of faulting.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// 16 bytes per lane from a buffer straight into LDS at lds + 16 * lane (buffer_load_dwordx4 ... lds); the
// transfer counts in vmcnt until the bytes are in LDS. The host pass of hipcc does not instantiate kernels that
// name this builtin, so only the device pass sees it.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff, uint32_t soff) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, voff, soff, 0, 0);
#else
    (void)r, (void)lds, (void)voff, (void)soff;
#endif
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations and is a compiler memory
// barrier, but unlike __syncthreads() it does not wait for the wave's outstanding global loads (the
// workgroup-scope fence of __syncthreads() waits for vmcnt(0)).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// s_waitcnt vmcnt(n) alone (gfx9 encoding: vmcnt bits [3:0] and [15:14], expcnt and lgkmcnt left at "no wait").
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Wave-uniform value as a scalar (lets the compiler keep wave indices and tile loops in SGPRs).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// SiLU with the hardware reciprocal (v_rcp_f32, 1 ulp) in place of an IEEE division: the result is rounded to
// fp16 / bf16 next, far coarser than the reciprocal's error. g -> -inf gives -0, g -> +inf gives g.
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

} // namespace hm

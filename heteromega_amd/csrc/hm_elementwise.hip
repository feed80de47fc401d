// Elementwise operators around the FFN: SiLU-and-multiply, RMSNorm, residual adds. fp32 math, one rounding
// per stored value, 16-byte accesses.
#include "hm_device.hpp"
#include "hm_internal.hpp"

namespace hm {
namespace {

template <class T> __device__ __forceinline__ void load8(const uint16_t *p, float o[8]) {
    const uint4 v = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o[2 * i] = T::to_float(w[i] & 0xFFFFu);
        o[2 * i + 1] = T::to_float(w[i] >> 16);
    }
}

// Eight fp32 partials (two 16-byte loads).
__device__ __forceinline__ void load8_f32(const float *p, float o[8]) {
    const float4 a = *reinterpret_cast<const float4 *>(p);
    const float4 b = *reinterpret_cast<const float4 *>(p + 4);
    o[0] = a.x, o[1] = a.y, o[2] = a.z, o[3] = a.w, o[4] = b.x, o[5] = b.y, o[6] = b.z, o[7] = b.w;
}

template <class T> __device__ __forceinline__ void store8(uint16_t *p, const float v[8]) {
    uint4 o;
    uint32_t *w = reinterpret_cast<uint32_t *>(&o);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w[i] = static_cast<uint32_t>(T::from_float(v[2 * i])) | (static_cast<uint32_t>(T::from_float(v[2 * i + 1])) << 16);
    }
    *reinterpret_cast<uint4 *>(p) = o;
}

// act[r, c] = SiLU(gate) * up. Blocked: gate column c, up column n + c. Interleaved (per 64 channels): gate
// column (c / 64) * 128 + c % 64, up 64 columns later (kernels/gpu/src/silu_mul.cu:10-30).
template <class T>
__global__ void __launch_bounds__(256) silu_mul_kernel(const uint16_t *__restrict__ gu, int64_t ld_in, uint16_t *__restrict__ act,
                                                       int64_t ld_out, int64_t rows, int64_t n, bool interleaved) {
    const int64_t per_row = n / 8;
    const int64_t total = rows * per_row;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t r = i / per_row;
        const int64_t c = (i - r * per_row) * 8;
        const int64_t gc = interleaved ? (c / 64) * 128 + c % 64 : c;
        const int64_t uc = interleaved ? gc + 64 : n + c;
        float g[8], u[8], o[8];
        load8<T>(gu + r * ld_in + gc, g);
        load8<T>(gu + r * ld_in + uc, u);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            o[k] = silu(g[k]) * u[k];
        }
        store8<T>(act + r * ld_out + c, o);
    }
}

// Block sum over 256 threads.
__device__ __forceinline__ float block_sum(float v, float *scratch) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        v += __shfl_xor(v, off);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        scratch[wave] = v;
    }
    lds_barrier(); // LDS only: the block's global stores need not complete here
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        t += scratch[w];
    }
    lds_barrier();
    return t;
}

// One row per block. ADD: x += y first (stored rounded), and the norm reads the rounded x, as the model's
// x.add_ then RMSNorm does (src/unified_llm_w4a16_hetero/unified_llm_w4a16.cpp:2815-2821, :2892).
// Rows of up to kCached * 2048 columns stay in registers: x, y and the weight are requested in one round
// trip and x is not read back after its residual update.
constexpr int kCached = 4;

// With a second addend zr (may be null): x = round((x + y) + z), the order of the reference's residual_norm
// (kernels/gpu/src/residual_norm.cu:45-49).
template <class T, bool ADD>
__device__ __forceinline__ void rmsnorm_cached(uint16_t *__restrict__ out, uint16_t *__restrict__ xr, const uint16_t *__restrict__ yr,
                                               const uint16_t *__restrict__ zr, const uint16_t *__restrict__ w, int64_t cols, float eps,
                                               float *scratch) {
    float v[kCached][8], g[kCached][8];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < kCached; ++j) {
        const int64_t c = threadIdx.x * 8 + j * 2048;
        if (c < cols) {
            load8<T>(xr + c, v[j]);
            load8<T>(w + c, g[j]);
            if constexpr (ADD) {
                float a[8];
                load8<T>(yr + c, a);
                if (zr != nullptr) {
                    float b[8];
                    load8<T>(zr + c, b);
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        v[j][k] = T::to_float(T::from_float((v[j][k] + a[k]) + b[k]));
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        v[j][k] = T::to_float(T::from_float(v[j][k] + a[k]));
                    }
                }
                store8<T>(xr + c, v[j]);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                ss += v[j][k] * v[j][k];
            }
        }
    }
    const float total = block_sum(ss, scratch);
    const float scale = 1.0f / sqrtf(total / static_cast<float>(cols) + eps);
#pragma unroll
    for (int j = 0; j < kCached; ++j) {
        const int64_t c = threadIdx.x * 8 + j * 2048;
        if (c < cols) {
            float o[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                o[k] = v[j][k] * scale * g[j][k];
            }
            store8<T>(out + c, o);
        }
    }
}

template <class T, bool ADD>
__global__ void __launch_bounds__(256) rmsnorm_kernel(uint16_t *__restrict__ out, int64_t ld_out, uint16_t *__restrict__ x, int64_t ldx,
                                                      const uint16_t *__restrict__ y, int64_t ldy, const uint16_t *__restrict__ z,
                                                      int64_t ldz, const uint16_t *__restrict__ w, int64_t cols, float eps) {
    __shared__ float scratch[4];
    const int64_t r = blockIdx.x;
    uint16_t *xr = x + r * ldx;
    if (cols <= kCached * 2048) {
        rmsnorm_cached<T, ADD>(out + r * ld_out, xr, ADD ? y + r * ldy : nullptr, ADD && z != nullptr ? z + r * ldz : nullptr, w, cols, eps,
                               scratch);
        return;
    }
    float ss = 0.0f;
    for (int64_t c = threadIdx.x * 8; c < cols; c += 256 * 8) {
        float v[8];
        load8<T>(xr + c, v);
        if constexpr (ADD) {
            float a[8];
            load8<T>(y + r * ldy + c, a);
            if (z != nullptr) {
                float b[8];
                load8<T>(z + r * ldz + c, b);
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    v[k] = T::to_float(T::from_float((v[k] + a[k]) + b[k]));
                }
            } else {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    v[k] = T::to_float(T::from_float(v[k] + a[k]));
                }
            }
            store8<T>(xr + c, v);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            ss += v[k] * v[k];
        }
    }
    const float total = block_sum(ss, scratch);
    const float scale = 1.0f / sqrtf(total / static_cast<float>(cols) + eps);
    for (int64_t c = threadIdx.x * 8; c < cols; c += 256 * 8) {
        float v[8], g[8], o[8];
        load8<T>(xr + c, v);
        load8<T>(w + c, g);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            o[k] = v[k] * scale * g[k];
        }
        store8<T>(out + r * ld_out + c, o);
    }
}

template <class T>
__global__ void __launch_bounds__(256) residual_add2_kernel(uint16_t *__restrict__ x, int64_t ldx, const uint16_t *__restrict__ a, int64_t lda,
                                                            const uint16_t *__restrict__ b, int64_t ldb, int64_t rows, int64_t cols) {
    const int64_t per_row = cols / 8;
    const int64_t total = rows * per_row;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t r = i / per_row;
        const int64_t c = (i - r * per_row) * 8;
        float v[8], t[8];
        load8<T>(x + r * ldx + c, v);
        if (a != nullptr) {
            load8<T>(a + r * lda + c, t);
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                t[k] = 0.0f;
            }
        }
        if (b != nullptr) {
            float u[8];
            load8<T>(b + r * ldb + c, u);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                t[k] += u[k];
            }
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            v[k] += t[k];
        }
        store8<T>(x + r * ldx + c, v);
    }
}

// x += a + b with each partial 16-bit (the activation type) or fp32 (the reference's residual_add2 takes either,
// kernels/gpu/src/residual_add.cu:9-31): the partials are added first, then the residual, one rounding.
template <class T, bool A32, bool B32>
__global__ void __launch_bounds__(256) residual_add2_mixed_kernel(uint16_t *__restrict__ x, int64_t ldx, const void *__restrict__ a, int64_t lda,
                                                                  const void *__restrict__ b, int64_t ldb, int64_t rows, int64_t cols) {
    const int64_t per_row = cols / 8;
    const int64_t total = rows * per_row;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t r = i / per_row;
        const int64_t c = (i - r * per_row) * 8;
        float v[8], t[8], u[8];
        load8<T>(x + r * ldx + c, v);
        if constexpr (A32) {
            load8_f32(static_cast<const float *>(a) + r * lda + c, t);
        } else {
            load8<T>(static_cast<const uint16_t *>(a) + r * lda + c, t);
        }
        if constexpr (B32) {
            load8_f32(static_cast<const float *>(b) + r * ldb + c, u);
        } else {
            load8<T>(static_cast<const uint16_t *>(b) + r * ldb + c, u);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            v[k] += t[k] + u[k];
        }
        store8<T>(x + r * ldx + c, v);
    }
}

// Nonfinite scan: 8 elements per thread, element (r, c) checked for c < cols (all) or c % stride == 0 (sampled);
// the least row-major index r * cols + c of a nonfinite one goes to *first by an unsigned atomic min. *first starts
// at kNoIndex (find_init, a kernel rather than a memset so that the scan can be captured in a graph), which read as
// an int64 is -1, the answer when nothing is found.
constexpr unsigned long long kNoIndex = ~0ull;
__global__ void find_init(unsigned long long *first) { *first = kNoIndex; }
template <bool FP16>
__global__ void __launch_bounds__(256) find_nonfinite_kernel(const uint16_t *__restrict__ x, int64_t ld, int64_t rows, int64_t cols, int64_t stride,
                                                             unsigned long long *first) {
    const uint32_t mask = FP16 ? 0x7C00u : 0x7F80u;
    const int64_t per_row = (cols + 8 * stride - 1) / (8 * stride); // groups of 8 checked elements per row
    const int64_t total = rows * per_row;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t r = i / per_row;
        const int64_t c0 = (i - r * per_row) * 8 * stride;
        unsigned long long hit = kNoIndex;
        for (int k = 7; k >= 0; --k) { // highest first, so the least index is kept
            const int64_t c = c0 + k * stride;
            if (c < cols && (x[r * ld + c] & mask) == mask) {
                hit = static_cast<unsigned long long>(r * cols + c);
            }
        }
        if (hit != kNoIndex) {
            atomicMin(first, hit);
        }
    }
}

dim3 grid_for(int64_t work) {
    const int64_t blocks = (work + 255) / 256;
    return dim3(static_cast<unsigned>(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192));
}

} // namespace

hipError_t launch_silu_mul(const uint16_t *gate_up, int64_t ld_in, uint16_t *act, int64_t ld_out, int64_t rows, int64_t n,
                           bool interleaved, int dtype, hipStream_t stream) {
    const int64_t work = rows * (n / 8);
    if (work == 0) {
        return hipSuccess;
    }
    if (dtype == 1) {
        hipLaunchKernelGGL(silu_mul_kernel<F16>, grid_for(work), dim3(256), 0, stream, gate_up, ld_in, act, ld_out, rows, n, interleaved);
    } else {
        hipLaunchKernelGGL(silu_mul_kernel<BF16>, grid_for(work), dim3(256), 0, stream, gate_up, ld_in, act, ld_out, rows, n, interleaved);
    }
    return hipGetLastError();
}

hipError_t launch_rmsnorm(uint16_t *out, int64_t ld_out, const uint16_t *x, int64_t ldx, const uint16_t *weight, int64_t rows,
                          int64_t cols, float eps, int dtype, hipStream_t stream) {
    if (rows == 0) {
        return hipSuccess;
    }
    uint16_t *xm = const_cast<uint16_t *>(x); // not written without ADD
    if (dtype == 1) {
        hipLaunchKernelGGL((rmsnorm_kernel<F16, false>), dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, out, ld_out, xm, ldx,
                           static_cast<const uint16_t *>(nullptr), int64_t(0), static_cast<const uint16_t *>(nullptr), int64_t(0), weight, cols,
                           eps);
    } else {
        hipLaunchKernelGGL((rmsnorm_kernel<BF16, false>), dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, out, ld_out, xm, ldx,
                           static_cast<const uint16_t *>(nullptr), int64_t(0), static_cast<const uint16_t *>(nullptr), int64_t(0), weight, cols,
                           eps);
    }
    return hipGetLastError();
}

hipError_t launch_residual_rmsnorm(uint16_t *x, int64_t ldx, const uint16_t *y, int64_t ldy, const uint16_t *z, int64_t ldz,
                                   const uint16_t *weight, uint16_t *normed, int64_t ld_normed, int64_t rows, int64_t cols, float eps, int dtype,
                                   hipStream_t stream) {
    if (rows == 0) {
        return hipSuccess;
    }
    if (dtype == 1) {
        hipLaunchKernelGGL((rmsnorm_kernel<F16, true>), dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, normed, ld_normed, x, ldx, y,
                           ldy, z, ldz, weight, cols, eps);
    } else {
        hipLaunchKernelGGL((rmsnorm_kernel<BF16, true>), dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, normed, ld_normed, x, ldx,
                           y, ldy, z, ldz, weight, cols, eps);
    }
    return hipGetLastError();
}

hipError_t launch_residual_add2_mixed(uint16_t *x, int64_t ldx, const void *a, int64_t lda, bool a32, const void *b, int64_t ldb, bool b32,
                                      int64_t rows, int64_t cols, int dtype, hipStream_t stream) {
    const int64_t work = rows * (cols / 8);
    if (work == 0) {
        return hipSuccess;
    }
    const dim3 g = grid_for(work);
    auto kern = dtype == 1 ? (a32 ? (b32 ? residual_add2_mixed_kernel<F16, true, true> : residual_add2_mixed_kernel<F16, true, false>)
                                  : (b32 ? residual_add2_mixed_kernel<F16, false, true> : residual_add2_mixed_kernel<F16, false, false>))
                           : (a32 ? (b32 ? residual_add2_mixed_kernel<BF16, true, true> : residual_add2_mixed_kernel<BF16, true, false>)
                                  : (b32 ? residual_add2_mixed_kernel<BF16, false, true> : residual_add2_mixed_kernel<BF16, false, false>));
    hipLaunchKernelGGL(kern, g, dim3(256), 0, stream, x, ldx, a, lda, b, ldb, rows, cols);
    return hipGetLastError();
}

hipError_t launch_find_nonfinite(const uint16_t *x, int64_t ld, int64_t rows, int64_t cols, int64_t stride, int dtype, int64_t *first,
                                 hipStream_t stream) {
    unsigned long long *f = reinterpret_cast<unsigned long long *>(first);
    hipLaunchKernelGGL(find_init, dim3(1), dim3(1), 0, stream, f);
    const int64_t work = rows * ((cols + 8 * stride - 1) / (8 * stride));
    if (work > 0) {
        if (dtype == 1) {
            hipLaunchKernelGGL(find_nonfinite_kernel<true>, grid_for(work), dim3(256), 0, stream, x, ld, rows, cols, stride, f);
        } else {
            hipLaunchKernelGGL(find_nonfinite_kernel<false>, grid_for(work), dim3(256), 0, stream, x, ld, rows, cols, stride, f);
        }
    }
    return hipGetLastError();
}

hipError_t launch_residual_add2(uint16_t *x, int64_t ldx, const uint16_t *a, int64_t lda, const uint16_t *b, int64_t ldb, int64_t rows,
                                int64_t cols, int dtype, hipStream_t stream) {
    const int64_t work = rows * (cols / 8);
    if (work == 0) {
        return hipSuccess;
    }
    if (dtype == 1) {
        hipLaunchKernelGGL(residual_add2_kernel<F16>, grid_for(work), dim3(256), 0, stream, x, ldx, a, lda, b, ldb, rows, cols);
    } else {
        hipLaunchKernelGGL(residual_add2_kernel<BF16>, grid_for(work), dim3(256), 0, stream, x, ldx, a, lda, b, ldb, rows, cols);
    }
    return hipGetLastError();
}

} // namespace hm

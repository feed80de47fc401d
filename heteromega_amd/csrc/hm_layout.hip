// One-time weight conversion into the strip layout (hm_device.hpp), and back.
//
// Sources:
//   - the reference's 4352-byte tiles. Tile (tile column c, tile row r) of a tiles_k x tiles_n matrix sits at
//     index (c / 8 + sum_{g < c % 8} ceil((tiles_n - g) / 8)) * tiles_k + r
//     (kernels/gpu/src/pack_w4a16.cpp:100-107). Inside a tile, byte ((a * 8 + cc) * 8 + b) * 4 + j holds row
//     a * 8 + b, column cc * 8 + 2 j (low nibble) and cc * 8 + 2 j + 1 (high nibble) (pack_w4a16.cpp:38-49);
//     bytes 4096 + 2 i hold the bf16 scale of column i, byte 4224 + (i / 8) * 16 + i % 8 its zero (:51-61).
//   - logical tensors q [K, N], scales and zeros [K / group, N].
// One thread writes one strip dword (8 K values of one column); one thread per record writes the metadata.
#include "hm_device.hpp"
#include "hm_internal.hpp"

namespace hm {
namespace {

__device__ __forceinline__ int64_t tile_index(int64_t c, int64_t r, int64_t tiles_k, int64_t tiles_n) {
    int64_t before = c / 8;
    for (int64_t g = 0; g < c % 8; ++g) {
        before += (tiles_n - g + 7) / 8;
    }
    return before * tiles_k + r;
}

// Source column of output column n: plain (one source) or fused (strip 2j <- src 0, strip 2j + 1 <- src 1).
__device__ __forceinline__ void source_column(int64_t n, bool fused, int &which, int64_t &src_col) {
    if (fused) {
        const int64_t s = n >> 4;
        which = static_cast<int>(s & 1);
        src_col = ((s >> 1) << 4) | (n & 15);
    } else {
        which = 0;
        src_col = n;
    }
}

// Packed column of source column c (TileSource::col_mode).
__device__ __forceinline__ int64_t packed_column(const TileSource &src, int64_t c) {
    if (src.col_mode == 0) {
        return c + src.col_offset;
    }
    return ((c >> 6) << 7) + (src.col_mode == 2 ? 64 : 0) + (c & 63);
}

__device__ __forceinline__ void check_zero(uint32_t z, uint32_t *bad_zero) {
    if (z > kMaxZero && bad_zero != nullptr) {
        atomicOr(bad_zero, 1u);
    }
}

__device__ __forceinline__ uint32_t bf16_bits_to_dtype(uint32_t bits, int dtype) {
    if (dtype == 1) { // fp16 plane from bf16 tiles: round to nearest even
        return float_to_half_bits(bf16_bits_to_float(bits));
    }
    return bits;
}

__global__ void __launch_bounds__(256)
    repack_tiles_quant(TileSource s0, TileSource s1, bool fused, uint32_t *__restrict__ quant, int64_t kt, int64_t total) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) {
        return;
    }
    const int mu = static_cast<int>(idx & 3);
    const int lane = static_cast<int>((idx >> 2) & 63);
    const int64_t st = idx >> 8;
    const int64_t t = st % kt;
    const int64_t s = st / kt;
    int which;
    int64_t n_src;
    source_column(s * 16 + (lane & 15), fused, which, n_src);
    const TileSource &src = which ? s1 : s0;
    n_src = packed_column(src, n_src);
    const uint8_t *tile = src.tiles + tile_index(n_src >> 6, t, src.tiles_k, src.tiles_n) * 4352;
    const int a = 4 * mu + (lane >> 4); // 8-row block of the 128-row tile
    const int cn = static_cast<int>(n_src & 63);
    const int cc = cn >> 3, j = (cn & 7) >> 1, shift = 4 * (cn & 1);
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t q = (tile[((a * 8 + cc) * 8 + e) * 4 + j] >> shift) & 0xFu;
        word |= q << (4 * nibble_of(e));
    }
    quant[idx] = word;
}

__global__ void __launch_bounds__(256)
    repack_tiles_meta(TileSource s0, TileSource s1, bool fused, uint32_t *__restrict__ meta, int64_t kt, int64_t total, int dtype,
                      uint32_t *bad_zero) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) {
        return;
    }
    const int col = static_cast<int>(idx & 15); // group size 128: one record per column and tile
    const int64_t t = (idx >> 4) % kt;
    const int64_t s = (idx >> 4) / kt;
    int which;
    int64_t n_src;
    source_column(s * 16 + col, fused, which, n_src);
    const TileSource &src = which ? s1 : s0;
    n_src = packed_column(src, n_src);
    const uint8_t *tile = src.tiles + tile_index(n_src >> 6, t, src.tiles_k, src.tiles_n) * 4352;
    const int cn = static_cast<int>(n_src & 63);
    const uint32_t sbits = static_cast<uint32_t>(tile[4096 + 2 * cn]) | (static_cast<uint32_t>(tile[4096 + 2 * cn + 1]) << 8);
    const uint32_t z = tile[4224 + (cn >> 3) * 16 + (cn & 7)];
    check_zero(z, bad_zero);
    meta[idx] = bf16_bits_to_dtype(sbits, dtype) | (z << 16);
}

__global__ void __launch_bounds__(256)
    repack_logical_quant(LogicalSource s0, LogicalSource s1, bool fused, uint32_t *__restrict__ quant, int64_t kt, int64_t total) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) {
        return;
    }
    const int mu = static_cast<int>(idx & 3);
    const int lane = static_cast<int>((idx >> 2) & 63);
    const int64_t st = idx >> 8;
    const int64_t t = st % kt;
    const int64_t s = st / kt;
    int which;
    int64_t n_src;
    source_column(s * 16 + (lane & 15), fused, which, n_src);
    const LogicalSource &src = which ? s1 : s0;
    const int64_t k0 = t * 128 + 32 * mu + 8 * (lane >> 4);
    const uint8_t *q = src.q + k0 * src.ld + n_src;
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        word |= (static_cast<uint32_t>(q[e * src.ld]) & 0xFu) << (4 * nibble_of(e));
    }
    quant[idx] = word;
}

__global__ void __launch_bounds__(256)
    repack_logical_meta(LogicalSource s0, LogicalSource s1, bool fused, uint32_t *__restrict__ meta, int64_t kt, int gpt, int64_t total,
                        uint32_t *bad_zero) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) {
        return;
    }
    const int gi = static_cast<int>(idx % gpt);
    const int col = static_cast<int>((idx / gpt) & 15);
    const int64_t st = idx / (gpt * 16);
    const int64_t g = (st % kt) * gpt + gi;
    const int64_t s = st / kt;
    int which;
    int64_t n_src;
    source_column(s * 16 + col, fused, which, n_src);
    const LogicalSource &src = which ? s1 : s0;
    const uint32_t sbits = src.scales[g * src.ld + n_src];
    const uint32_t z = src.zeros[g * src.ld + n_src];
    check_zero(z, bad_zero);
    meta[idx] = sbits | (z << 16);
}

__global__ void __launch_bounds__(256)
    unpack_quant(const uint32_t *__restrict__ quant, uint8_t *__restrict__ q, int64_t N, int64_t kt, int64_t total) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) {
        return;
    }
    const int mu = static_cast<int>(idx & 3);
    const int lane = static_cast<int>((idx >> 2) & 63);
    const int64_t st = idx >> 8;
    const int64_t t = st % kt;
    const int64_t s = st / kt;
    const int64_t n = s * 16 + (lane & 15);
    const int64_t k0 = t * 128 + 32 * mu + 8 * (lane >> 4);
    const uint32_t word = quant[idx];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        q[(k0 + e) * N + n] = static_cast<uint8_t>((word >> (4 * nibble_of(e))) & 0xFu);
    }
}

__global__ void __launch_bounds__(256) unpack_meta(const uint32_t *__restrict__ meta, uint16_t *__restrict__ scales,
                                                   uint8_t *__restrict__ zeros, int64_t N, int64_t kt, int gpt, int64_t total) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) {
        return;
    }
    const int gi = static_cast<int>(idx % gpt);
    const int col = static_cast<int>((idx / gpt) & 15);
    const int64_t st = idx / (gpt * 16);
    const int64_t g = (st % kt) * gpt + gi;
    const int64_t s = st / kt;
    const uint32_t rec = meta[idx];
    scales[g * N + s * 16 + col] = static_cast<uint16_t>(rec & 0xFFFFu);
    zeros[g * N + s * 16 + col] = static_cast<uint8_t>(rec >> 16);
}

// One thread per strip dword: the 8 K values of one column, (q - z) s exact in fp32 and rounded once to the
// activation type (the reference's dequantize_packed computes (w - z) * s in bf16 arithmetic: one rounding of the
// exact product, unified_llm_w4a16.cpp:770-777). Transposed output [N, K] takes the 8 values as one 16-byte store.
template <class T>
__global__ void __launch_bounds__(256) dequantize_kernel(const uint32_t *__restrict__ quant, const uint32_t *__restrict__ meta,
                                                          uint16_t *__restrict__ out, int64_t ld, bool transposed, int64_t kt,
                                                          int gpt, int group, int64_t total) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) {
        return;
    }
    const int mu = static_cast<int>(idx & 3);
    const int lane = static_cast<int>((idx >> 2) & 63);
    const int64_t st = idx >> 8;
    const int64_t t = st % kt;
    const int64_t s = st / kt;
    const int col = lane & 15;
    const int64_t n = s * 16 + col;
    const int kin = 32 * mu + 8 * (lane >> 4); // K offset inside the tile; 8 values never straddle a group
    const uint32_t rec = meta[((s * kt + t) * 16 + col) * gpt + kin / group];
    const float sc = T::to_float(rec & 0xFFFFu);
    const float z = static_cast<float>((rec >> 16) & 0xFFu);
    const uint32_t word = quant[idx];
    uint16_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        v[e] = T::from_float((static_cast<float>((word >> (4 * nibble_of(e))) & 0xFu) - z) * sc);
    }
    const int64_t k0 = t * 128 + kin;
    if (transposed) {
        uint4 o;
        o.x = v[0] | (static_cast<uint32_t>(v[1]) << 16);
        o.y = v[2] | (static_cast<uint32_t>(v[3]) << 16);
        o.z = v[4] | (static_cast<uint32_t>(v[5]) << 16);
        o.w = v[6] | (static_cast<uint32_t>(v[7]) << 16);
        *reinterpret_cast<uint4 *>(out + n * ld + k0) = o;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            out[(k0 + e) * ld + n] = v[e];
        }
    }
}

dim3 blocks_for(int64_t total) { return dim3(static_cast<unsigned>((total + 255) / 256)); }

} // namespace

hipError_t launch_repack_tiles(const TileSource *src, int nsrc, bool fused, uint8_t *quant, uint32_t *meta, int64_t K,
                               int64_t N, int dtype, uint32_t *bad_zero, hipStream_t stream) {
    const TileSource s0 = src[0];
    const TileSource s1 = nsrc > 1 ? src[1] : src[0];
    const int64_t kt = K / 128;
    const int64_t words = (N / 16) * kt * 256;
    if (words > 0) {
        hipLaunchKernelGGL(repack_tiles_quant, blocks_for(words), dim3(256), 0, stream, s0, s1, fused,
                           reinterpret_cast<uint32_t *>(quant), kt, words);
    }
    const int64_t records = (N / 16) * kt * 16;
    if (records > 0) {
        hipLaunchKernelGGL(repack_tiles_meta, blocks_for(records), dim3(256), 0, stream, s0, s1, fused, meta, kt, records, dtype, bad_zero);
    }
    return hipGetLastError();
}

hipError_t launch_repack_logical(const LogicalSource *src, int nsrc, bool fused, uint8_t *quant, uint32_t *meta,
                                 int64_t K, int64_t N, int64_t group, uint32_t *bad_zero, hipStream_t stream) {
    const LogicalSource s0 = src[0];
    const LogicalSource s1 = nsrc > 1 ? src[1] : src[0];
    const int64_t kt = K / 128;
    const int64_t words = (N / 16) * kt * 256;
    if (words > 0) {
        hipLaunchKernelGGL(repack_logical_quant, blocks_for(words), dim3(256), 0, stream, s0, s1, fused,
                           reinterpret_cast<uint32_t *>(quant), kt, words);
    }
    const int64_t groups = K / group;
    const int64_t records = (N / 16) * groups * 16;
    if (records > 0) {
        hipLaunchKernelGGL(repack_logical_meta, blocks_for(records), dim3(256), 0, stream, s0, s1, fused, meta, kt,
                           static_cast<int>(128 / group), records, bad_zero);
    }
    return hipGetLastError();
}

hipError_t launch_unpack(const Planes &p, uint8_t *q, uint16_t *scales, uint8_t *zeros, hipStream_t stream) {
    const int64_t kt = p.K / 128;
    const int64_t words = (p.N / 16) * kt * 256;
    if (words > 0) {
        hipLaunchKernelGGL(unpack_quant, blocks_for(words), dim3(256), 0, stream, reinterpret_cast<const uint32_t *>(p.quant), q,
                           p.N, kt, words);
    }
    const int64_t groups = p.K / p.group;
    const int64_t records = (p.N / 16) * groups * 16;
    if (records > 0) {
        hipLaunchKernelGGL(unpack_meta, blocks_for(records), dim3(256), 0, stream, p.meta, scales, zeros, p.N, kt,
                           static_cast<int>(128 / p.group), records);
    }
    return hipGetLastError();
}

hipError_t launch_dequantize(const Planes &p, uint16_t *out, int64_t ld, bool transposed, hipStream_t stream) {
    const int64_t kt = p.K / 128;
    const int64_t words = (p.N / 16) * kt * 256;
    if (words > 0) {
        const int gpt = static_cast<int>(128 / p.group);
        if (p.dtype == 1) {
            hipLaunchKernelGGL(dequantize_kernel<F16>, blocks_for(words), dim3(256), 0, stream, reinterpret_cast<const uint32_t *>(p.quant),
                               p.meta, out, ld, transposed, kt, gpt, static_cast<int>(p.group), words);
        } else {
            hipLaunchKernelGGL(dequantize_kernel<BF16>, blocks_for(words), dim3(256), 0, stream, reinterpret_cast<const uint32_t *>(p.quant),
                               p.meta, out, ld, transposed, kt, gpt, static_cast<int>(p.group), words);
        }
    }
    return hipGetLastError();
}

} // namespace hm

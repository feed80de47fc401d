// Host-side declarations shared by the C ABI (hm_api.cpp) and the kernel files.
#pragma once

#include "../../include/hm_w4a16.h"

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

namespace hm {

// Records the message of a failed C ABI call for hm_last_error() on this thread and returns s.
hm_status set_error(hm_status s, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Compute units and XCDs of the current device (queried once per device; 256 and 8 on an MI355X). Launch planning
// sizes grids by the CU count; the GEMM deals tiles to XCDs, onto which the dispatcher places workgroup i at i % xcds.
struct Topology {
    int64_t cus = 256;
    int xcds = 8;
};
Topology device_topology();

// Device planes of one repacked matrix (layout: hm_device.hpp).
struct Planes {
    const uint8_t *quant = nullptr; // (N/16) * (K/128) KiB
    const uint32_t *meta = nullptr; // (N/16) * (K/group) * 16 records
    int64_t K = 0, N = 0, group = 128;
    int dtype = 0; // hm_dtype
    int64_t kt_pitch() const { return K / 128; }
};

// One source matrix of a repack: the reference tiles or logical tensors of a [K, N] matrix.
// Column c of the source is packed column c + col_offset (col_mode 0), or, in a gate_up matrix interleaved per 64
// channels (the reference's GateUpLayout::kInterleaved, kernels/gpu/include/heteromega/gpu_ffn.hpp:43-46), the gate
// column (c / 64) * 128 + c % 64 (col_mode 1) or the up column 64 more (col_mode 2).
struct TileSource {
    const uint8_t *tiles = nullptr;
    int64_t tiles_k = 0, tiles_n = 0; // of the whole packed matrix
    int64_t col_offset = 0;
    int col_mode = 0;
};
// Largest zero point the repack accepts (GPTQ checkpoints store z - 1, so z reaches 16 after adding the one back).
constexpr uint32_t kMaxZero = 16;
struct LogicalSource {
    const uint8_t *q = nullptr;      // [K, ld] row-major
    const uint16_t *scales = nullptr; // [K/group, ld]
    const uint8_t *zeros = nullptr;   // [K/group, ld]
    int64_t ld = 0;
};

// Repack launches. `fused` interleaves two sources per 16 columns (strip 2j from src[0], 2j + 1 from src[1]);
// then N counts the columns of the result (2x the columns taken from each source). A zero point above kMaxZero
// sets bit 0 of *bad_zero (device memory, may be null).
hipError_t launch_repack_tiles(const TileSource *src, int nsrc, bool fused, uint8_t *quant, uint32_t *meta, int64_t K,
                               int64_t N, int dtype, uint32_t *bad_zero, hipStream_t stream);
hipError_t launch_repack_logical(const LogicalSource *src, int nsrc, bool fused, uint8_t *quant, uint32_t *meta,
                                 int64_t K, int64_t N, int64_t group, uint32_t *bad_zero, hipStream_t stream);
hipError_t launch_unpack(const Planes &p, uint8_t *q, uint16_t *scales, uint8_t *zeros, hipStream_t stream);
// Dequantized weights round((q - z) s) in the activation type: [N, K] (transposed, the orientation of the
// reference's dequantize_packed) or [K, N], leading dimension ld.
hipError_t launch_dequantize(const Planes &p, uint16_t *out, int64_t ld, bool transposed, hipStream_t stream);

// Decode GEMV (M <= 16) on strips [strip_begin, strip_begin + n/16) and K tiles [kt_begin, kt_begin + kt_count).
// fused: pairs of strips (gate, up) -> act = SiLU(gate) * up, n = output channels.
struct GemvCall {
    Planes w;
    const uint16_t *x = nullptr;
    int64_t ldx = 0;
    uint16_t *y = nullptr;
    int64_t ldy = 0;
    int64_t m = 1;
    int64_t strip_begin = 0;
    int64_t n = 0; // output columns (plain) or channels (fused)
    int64_t kt_begin = 0, kt_count = 0;
    bool fused = false;
    float *partial = nullptr; // split-K partials (GemvPlan::partial_bytes)
    // One row over the whole K (kt_begin 0, K <= 8192): stage RMSNorm(x) * norm_w instead of x.
    const uint16_t *norm_w = nullptr;
    float norm_eps = 0.0f;
    bool accumulate = false; // plain output: y = round(y + round(x W)) (residual add into y)
    // Strip-pair spill (gemv_pair_spill_bytes(n) bytes), for a one-row fused call whose act only a following
    // one-row plain call reads. Given one, the fused call may deal its pairs' K halves evenly over the CUs
    // (GemvPlan::units waves per workgroup): a pair whose halves land in two workgroups writes their fp32 sums here
    // and leaves its act columns unwritten. The plain call over that act then passes the same spill and
    // pair_units = the fused plan's units (when odd; even units split no pair) and forms those columns itself.
    float *pair_spill = nullptr;
    int pair_units = 0;
};
// Launch shape of a GemvCall: strips per wave, strip groups, K split, waves per strip group, strip groups per
// workgroup, LDS bytes and the fp32 partial buffer the split needs (0 without a split). units > 0: the one-row
// fused launch of (pair, K half) units, `units` waves per workgroup.
struct GemvPlan {
    int spw = 1;
    int64_t groups = 0;
    int64_t splits = 1, kt_per_split = 0;
    int wps = 1, nu = 1, waves = 4;
    int units = 0;
    bool few = false; // 2..8 rows on the one-row math and launch shape (else several rows: m > 1)
    size_t lds = 0;
    size_t partial_bytes = 0;
};
GemvPlan plan_gemv(const GemvCall &c);
constexpr size_t kGemvLdsMax = 160 * 1024; // LDS of one workgroup
// Bytes of the strip-pair spill of a one-row fused call over `channels` channels.
size_t gemv_pair_spill_bytes(int64_t channels);
// The largest partial buffer of a call like c over any range of c's columns (narrower ranges split K more).
size_t gemv_partial_bound(const GemvCall &c);
hipError_t launch_gemv(const GemvCall &c, hipStream_t stream);
// A K-split pair at one row in one launch: split 0 runs c0, split 1 runs c1 (x advanced by k0 elements), and the
// split sum forms round(round(c0) + round(c1)) into c0.y. c0.partial holds gemv_pair_partial_bytes(c0).
bool gemv_pair_supported(const GemvCall &c0, const GemvCall &c1);
size_t gemv_pair_partial_bytes(const GemvCall &c0);
hipError_t launch_gemv_pair(const GemvCall &c0, const GemvCall &c1, int64_t k0, hipStream_t stream);

// Prefill GEMM (MFMA 16x16x32) with the same operand conventions; fused writes SiLU(gate) * up.
struct GemmCall {
    Planes w;
    const uint16_t *x = nullptr;
    int64_t ldx = 0;
    uint16_t *y = nullptr;
    int64_t ldy = 0;
    int64_t m = 0;
    int64_t strip_begin = 0;
    int64_t n = 0;
    int64_t kt_begin = 0, kt_count = 0;
    bool fused = false;
    float *partial = nullptr; // split-K partials (GemmPlan::partial_bytes)
    bool accumulate = false;  // plain output: y = round(y + round(x W))
};
// Tile configuration (2: 128 x 256 tiles, 8 waves; 1: 128 x 128, 4 waves; 0: 64 x 128, 4 waves). The GEMM splits
// K only for grids of under 128 workgroups and 4-wave grids of under 512, with fp32 partials of at most
// kGemmPartialMax bytes.
constexpr size_t kGemmPartialMax = 32u << 20;
struct GemmPlan {
    int cfg = 1;
    int64_t tiles_m = 0, tiles_n = 0;
    int64_t splits = 1, kt_per_split = 0;
    size_t partial_bytes = 0;
};
GemmPlan plan_gemm(const GemmCall &c);
hipError_t launch_gemm(const GemmCall &c, hipStream_t stream);

// Adds split-K partials [splits][m][ncols] into y [m, ncols] (or, fused, y [m, ncols / 2] = SiLU(gate) * up
// with gate and up alternating per 16 columns).
// pairwise (plain only): each split's sum rounded, then added in split order with one rounding per add.
hipError_t launch_sum_splits(const float *partial, uint16_t *y, int64_t ldy, int64_t m, int ncols, int splits, bool fused,
                             int dtype, hipStream_t stream, bool accumulate = false, bool pairwise = false);

hipError_t launch_silu_mul(const uint16_t *gate_up, int64_t ld_in, uint16_t *act, int64_t ld_out, int64_t rows, int64_t n,
                           bool interleaved, int dtype, hipStream_t stream);
hipError_t launch_rmsnorm(uint16_t *out, int64_t ld_out, const uint16_t *x, int64_t ldx, const uint16_t *weight,
                          int64_t rows, int64_t cols, float eps, int dtype, hipStream_t stream);
hipError_t launch_residual_add2(uint16_t *x, int64_t ldx, const uint16_t *a, int64_t lda, const uint16_t *b, int64_t ldb,
                                int64_t rows, int64_t cols, int dtype, hipStream_t stream);
// x = round(x + y) (z null) or round((x + y) + z), then normed = RMSNorm(x) * weight.
hipError_t launch_residual_rmsnorm(uint16_t *x, int64_t ldx, const uint16_t *y, int64_t ldy, const uint16_t *z, int64_t ldz,
                                   const uint16_t *weight, uint16_t *normed, int64_t ld_normed, int64_t rows, int64_t cols, float eps, int dtype,
                                   hipStream_t stream);
// x += a + b with a and b each 16-bit (the activation type) or fp32.
hipError_t launch_residual_add2_mixed(uint16_t *x, int64_t ldx, const void *a, int64_t lda, bool a32, const void *b, int64_t ldb, bool b32,
                                      int64_t rows, int64_t cols, int dtype, hipStream_t stream);
// *first (device int64) = least row-major index r * cols + c of a nonfinite element with c % stride == 0, or -1.
hipError_t launch_find_nonfinite(const uint16_t *x, int64_t ld, int64_t rows, int64_t cols, int64_t stride, int dtype, int64_t *first,
                                 hipStream_t stream);

} // namespace hm

// The reference's C++ operator surface for the W4A16 FFN, served by the engine's C ABI (include/hm_w4a16.h).
//
// A maintainer of the reference links this translation unit (hm_reference_api.cpp) with libhmw4a16.so in place of
// src/hipkernels/w4a16_gemv_packed.cu, w4a16_gemm_packed.cu and kernels/gpu/src/{gemv,gemm}_w4a16.cu, gpu_ffn.cpp,
// pack_w4a16.cpp, residual_add.cu and residual_norm.cu: the FFN operators of gpu_ffn.hpp and the finite check of
// merged_ffn_contract.hpp are all declared here. What this file does not provide is off the FFN path: the prefill
// attention (sdpa_bf16, sdpa_v_tiles, sdpa_store_v), the CPU reducer residual_add2_cpu and MergedFfnConfig::load (the
// NPU artifact manifest), so a build that uses those keeps the reference's own files for them.
// Declarations keep the reference's names, argument order and defaults (include/hipkernels/w4a16_gemm_packed.hpp:38-52;
// kernels/gpu/include/heteromega/gpu_ffn.hpp:17-242). Argument errors raise c10::Error (TORCH_CHECK), launch errors
// std::runtime_error, as the reference's do.
//
// Packed weights stay the reference's 4352-byte tiles in the caller's tensors. The first call on a packed tensor
// repacks it into the engine's layout and keeps that copy, keyed by the tensor's address and the block it computes,
// for as long as the tensor's storage lives unchanged: a copy made from a storage that has since been freed (its
// address reused by other weights) or written in place (its version counter moved) is repacked on the next call.
// The repack enqueues on the caller's stream and waits for it, so the first call per packed tensor must come before
// any graph capture on that stream (under capture it raises c10::Error instead).
#pragma once

#include <hip/hip_runtime_api.h>
#include <torch/torch.h>

#include <cstdint>
#include <mutex>
#include <unordered_map>
#include <vector>

namespace hipkernels {

// output [M, out_features] = input [M, in_features] @ W, W the packed [in_features, out_features] matrix.
void w4a16_gemm_fused_packed(torch::Tensor &output, const torch::Tensor &input, const torch::Tensor &packed_params, int64_t in_features,
                             int64_t out_features, hipStream_t stream = 0);

// The same on the leading in_features x out_features block of a packed [128 packed_tiles_k, 64 packed_tiles_n] matrix.
// fuse_activation: the matrix is a gate_up interleaved per 64 channels and output [M, out_features / 2] = SiLU(gate) * up.
void w4a16_gemm_fused_packed_tiles(torch::Tensor &output, const torch::Tensor &input, const torch::Tensor &packed_params,
                                   int64_t in_features, int64_t out_features, int64_t packed_tiles_k, int64_t packed_tiles_n,
                                   hipStream_t stream = 0, bool fuse_activation = false);

// output [1, out_features] = input [1, in_features] @ W[:, start_col : start_col + out_features] of a packed
// [in_features, total_out_features] matrix (total_out_features = -1: out_features).
void w4a16_gemv_fused_packed(torch::Tensor &output, const torch::Tensor &input, const torch::Tensor &packed_params, int64_t in_features,
                             int64_t out_features, int64_t total_out_features = -1, int64_t start_col = 0, hipStream_t stream = 0);

} // namespace hipkernels

namespace heteromega {

constexpr int64_t kTileK = 128;
constexpr int64_t kTileN = 64;
constexpr int64_t kTileBytes = 4352;

// Rows a reference GEMM input had to hold; the engine needs no padding and keeps the function for callers.
inline int64_t padded_rows(int64_t m) { return (m + kTileK - 1) / kTileK * kTileK; }

enum class GateUpLayout {
    kBlocked,     // [gate 0..n) | up 0..n)]
    kInterleaved, // per 64 channels: their 64 gate columns, then their 64 up columns
};

// One device's packed share of an FFN layer, channels [begin, end) (gpu_ffn.hpp:53-71).
struct FfnSliceWeights {
    torch::Tensor gate_up; // packed [H, 2 * stored_channels()], column order `layout`
    torch::Tensor down;    // packed [stored_channels(), H]
    int64_t begin = 0;
    int64_t end = 0;
    int64_t hidden = 0;
    GateUpLayout layout = GateUpLayout::kBlocked;
    int64_t packed_channels = 0; // channels in the packed tensors; 0 means channels()

    int64_t channels() const { return end - begin; }
    int64_t stored_channels() const { return packed_channels > 0 ? packed_channels : channels(); }
    // The same slice with its tensors on `device`.
    FfnSliceWeights to(const torch::Device &device) const;
    // The same tensors, used for channels [begin, begin + n) only (n a multiple of 128; n < stored needs kInterleaved).
    FfnSliceWeights prefix(int64_t n) const;
};

// ---- Weight packing (gpu_ffn.hpp:27-98) ----

// The reference's 4352-byte tiles of a [K, N] matrix (K % 128 == 0, N % 64 == 0): qweight [K, N] values 0..15,
// scales [K / 128, N] (bf16), zeros [K / 128, N] (int8). Returns a flat uint8 CPU tensor (hm_pack_w4a16).
torch::Tensor pack_w4a16(const torch::Tensor &qweight, const torch::Tensor &scales, const torch::Tensor &zeros);

// One layer's quantized FFN tensors in [in_features, out_features] order (H hidden, I intermediate).
struct FfnLayerQuant {
    torch::Tensor gate_q, gate_s, gate_z; // [H, I], [H / 128, I], [H / 128, I]
    torch::Tensor up_q, up_s, up_z;       // [H, I], [H / 128, I], [H / 128, I]
    torch::Tensor down_q, down_s, down_z; // [I, H], [I / 128, H], [I / 128, H]
};

// Packs channels [begin, end) (multiples of 128) of a layer: gate_up [H, 2n] in `layout` order, down [n, H]; CPU tensors.
FfnSliceWeights pack_ffn_slice(const FfnLayerQuant &layer, int64_t begin, int64_t end, GateUpLayout layout = GateUpLayout::kBlocked);

int64_t packed_tile_index(int64_t c, int64_t r, int64_t tiles_k, int64_t tiles_n);

// pack_ffn_slice from already packed gate [hidden, inter], up [hidden, inter] and down [inter, hidden]: whole tiles copied on
// the tensors' device, the same bytes as pack_ffn_slice; for [0, inter) the result's down is `down` itself.
FfnSliceWeights slice_packed_ffn(const torch::Tensor &gate, const torch::Tensor &up, const torch::Tensor &down, int64_t hidden, int64_t inter,
                                 int64_t begin, int64_t end, GateUpLayout layout = GateUpLayout::kBlocked);

// act[m, j] = SiLU(gate[m, j]) * up[m, j], gate and up columns of gate_up in `layout` order; fp32 math, one rounding.
void silu_mul(const torch::Tensor &gate_up, torch::Tensor &act, hipStream_t stream, GateUpLayout layout = GateUpLayout::kBlocked);

// out[1, n] = x[1, k] @ W[:k, :n] of a packed [packed_k, packed_n] matrix. split_k is chosen by the engine.
void gemv_w4a16(torch::Tensor &out, const torch::Tensor &x, const torch::Tensor &packed, int64_t k, int64_t n, int64_t packed_k,
                int64_t packed_n, int split_k, hipStream_t stream);

// out[M, n] = x[M, k] @ W[:k, :n] of a packed [packed_k, packed_n] matrix.
void gemm_w4a16(torch::Tensor &out, const torch::Tensor &x, const torch::Tensor &packed, int64_t k, int64_t n, int64_t packed_k,
                int64_t packed_n, hipStream_t stream);
bool gemm_w4a16_supports(int64_t m, int64_t k, int64_t n);

// The FFN of n channels as one pass: gate_up packed [h, 2 * stored] (kInterleaved), down packed [stored, h].
bool gemm_w4a16_ffn_supports(int64_t m, int64_t h, int64_t n);
void gemm_w4a16_ffn(torch::Tensor &y, const torch::Tensor &x, const torch::Tensor &gate_up, const torch::Tensor &down, int64_t h, int64_t n,
                    int64_t stored, hipStream_t stream);

// The engine keeps no prepared GEMM input: its GEMM reads the input rows from memory. Matrices stay where they are.
torch::Tensor gemm_uncached_weights(const torch::Tensor &packed);

// The reference prepares a GEMM input once for several GEMMs of one x (Q, K and V; gpu_ffn.hpp:117-127). The engine's
// GEMM needs no preparation, so this only keeps the bookkeeping: while one lives on a thread, gemm_w4a16 and
// packed_linear GEMM calls with the marked x, k and stream count as hits.
class GemmInputReuse {
  public:
    GemmInputReuse();
    ~GemmInputReuse();
    GemmInputReuse(const GemmInputReuse &) = delete;
    GemmInputReuse &operator=(const GemmInputReuse &) = delete;
    void mark_prepared(const void *x, int64_t k, hipStream_t stream);
    int hits() const;
};
// The reference's prepared-input buffers have no counterpart here: raises c10::Error (its callers, the reference's
// residual_norm and sdpa kernels, are replaced by calls that write the GEMM input rows to memory).
void gemm_input_buffers(int64_t m, int64_t k, hipStream_t stream, float **sums, uint16_t **tiles);

// ---- Between two GEMMs (gpu_ffn.hpp:132-141) ----

// Any M > 0 and H a multiple of 8 (the reference's kernel needs M % 16 == 0 and H == 4096).
bool residual_norm_supports(int64_t m, int64_t h);
// x = round((x + a) + b) (a and b may be null; without a, x is left as it is), then RMSNorm(x) * weight is written to
// gemm_x (the rows the next GEMM reads, stride normed_stride) and, if non-null and different, to normed; then
// gemm_input.mark_prepared(gemm_x, h, stream). One dispatch (hm_residual2_rmsnorm), no host wait.
void residual_norm_bf16(uint16_t *x, const uint16_t *a, const uint16_t *b, const uint16_t *weight, uint16_t *normed, const void *gemm_x,
                        GemmInputReuse &gemm_input, int64_t m, int64_t h, int64_t x_stride, int64_t a_stride, int64_t b_stride,
                        int64_t normed_stride, float eps, hipStream_t stream);

// x [M, H] (bf16 or fp16) += y_g + y_n, each partial of x's type or fp32; partials first, then the residual, one rounding.
void residual_add2(torch::Tensor &x, const torch::Tensor &y_g, const torch::Tensor &y_n, hipStream_t stream);

enum class GemvKernel { kHeteroMega, kHeteroMosaic };
enum class GemmKernel { kHeteroMosaic, kHeteroMega };

// HETEROMEGA_GEMM=fast at the first call gives kHeteroMega, else kHeteroMosaic (gpu_ffn.hpp:196-197). Both choices run the
// engine's GEMM; callers keep the value for their own path decisions.
GemmKernel configured_gemm_kernel();

struct LinearOptions {
    int64_t packed_k = 0;           // rows of the whole packed matrix; 0 means k
    int64_t packed_n = 0;           // columns of the whole packed matrix; 0 means n
    GemvKernel gemv = GemvKernel::kHeteroMega;
    int gemv_split_k = 0;
    bool fuse_activation = false;   // gate/up only: write SiLU(gate) * up [M, n / 2]
    GemmKernel gemm = GemmKernel::kHeteroMosaic;
};

// out[M, n] = in[M, k] @ W[:k, :n]; the kernel choices in `opt` all run the engine's kernels.
void packed_linear(torch::Tensor &out, const torch::Tensor &in, const torch::Tensor &packed, int64_t k, int64_t n, hipStream_t stream,
                   const LinearOptions &opt = {});

// Scratch of gpu_ffn_slice_forward, allocated once for the largest M and the most channels (gpu_ffn.hpp:172-180): the
// reference's three tensors with their sizes ([padded_rows(M), 2n], [.., n], [.., H], bf16). The engine takes its
// workspace from gate_up's storage (the larger of the three); `workspace` is grown only when that is too small.
struct GpuFfnBuffers {
    torch::Tensor gate_up; // [rows, 2n] bf16
    torch::Tensor act;     // [rows, n] bf16
    torch::Tensor x_pad;   // [rows, H] bf16 (the engine needs no padded copy of x_norm)
    torch::Tensor workspace; // uint8, only when gate_up's storage is smaller than the engine's workspace
    std::vector<torch::Tensor> retired; // outgrown workspaces, kept while enqueued work may still read them

    static GpuFfnBuffers allocate(int64_t max_m, int64_t channels, int64_t hidden, const torch::Device &device);
};

// The GPU share of one FFN layer: y [M, H] = FFN of x_norm [M, H] over w's channels. Enqueues, does not synchronize.
void gpu_ffn_slice_forward(const FfnSliceWeights &w, const torch::Tensor &x_norm, GpuFfnBuffers &buf, torch::Tensor &y, hipStream_t stream);

// The GPU FFN of every layer of a model (gpu_ffn.hpp:219-242).
class GpuFfnModel {
  public:
    // Adds the next layer from the reference's packed gate [H, I], up [H, I] and down [I, H] (bf16 activations).
    void add_layer(const torch::Tensor &gate, const torch::Tensor &up, const torch::Tensor &down, int64_t hidden, int64_t inter);
    // GPU channels for prefill (M > 1) and decode (M == 1): multiples of 128 in (0, I].
    void set_split(int64_t s_prefill, int64_t s_decode);
    int64_t layers() const { return static_cast<int64_t>(layers_.size()); }
    int64_t channels(int64_t m) const { return m > 1 ? s_prefill_ : s_decode_; }
    // y = the GPU share of layer `layer` for x_norm (bf16 [M, H], contiguous); enqueues on `stream`.
    void forward(int64_t layer, const torch::Tensor &x_norm, torch::Tensor &y, hipStream_t stream);
    ~GpuFfnModel();

  private:
    std::vector<void *> layers_; // hm_ffn handles
    int64_t inter_ = 0;
    int64_t s_prefill_ = 0;
    int64_t s_decode_ = 0;
    std::mutex mutex_;
    std::unordered_map<hipStream_t, torch::Tensor> workspaces_;
    std::vector<torch::Tensor> retired_; // outgrown workspaces, kept while enqueued work may still read them
};

// ---- The merged FFN's nonfinite check (include/heteromega/merged_ffn_contract.hpp:13-39) ----

// HETEROMEGA_FFN_FINITE_CHECK: full (every element) or sampled (every row at one in kFiniteSampleStride columns).
enum class FiniteCheck { kFull, kSampled };
constexpr int64_t kFiniteSampleStride = 64;
// nullptr, "" and "full" give kFull, "sampled" kSampled; anything else throws std::invalid_argument.
FiniteCheck parse_finite_check(const char *value);
// Row-major bf16 bits in host memory: the index of the first checked element with all 8 exponent bits set, or -1.
int64_t find_nonfinite_bf16(const uint16_t *bits, int64_t rows, int64_t columns, FiniteCheck mode);
// The same check of a device tensor [M, N] (bf16 or fp16, contiguous last dimension) where it lies: the first index is
// written to `first` (a device int64 tensor of one element), enqueued on `stream` without a host wait.
void find_nonfinite_device(const torch::Tensor &t, FiniteCheck mode, torch::Tensor &first, hipStream_t stream);

} // namespace heteromega

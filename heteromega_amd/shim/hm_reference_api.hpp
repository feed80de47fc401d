// The reference's C++ operator surface for the W4A16 FFN, served by the engine's C ABI (include/hm_w4a16.h).
//
// A maintainer of the reference links this translation unit (hm_reference_api.cpp) with libhmw4a16.so in place of
// src/hipkernels/w4a16_gemv_packed.cu, w4a16_gemm_packed.cu and kernels/gpu/src/{gemv,gemm}_w4a16.cu, gpu_ffn.cpp:
// the call sites in unified_llm_w4a16.cpp (:1054-1065) and the HeteroMega model integration compile unchanged.
// Declarations keep the reference's names, argument order and defaults (include/hipkernels/w4a16_gemm_packed.hpp:38-52;
// kernels/gpu/include/heteromega/gpu_ffn.hpp:17-242). Argument errors raise c10::Error (TORCH_CHECK), launch errors
// std::runtime_error, as the reference's do.
//
// Packed weights stay the reference's 4352-byte tiles in the caller's tensors. The first call on a packed tensor
// repacks it into the engine's layout once and keeps that copy for the life of the process, keyed by the tensor's
// address and the block it computes: as in the reference, packed parameters are loaded once and not rewritten.
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
    // The same tensors, used for channels [begin, begin + n) only (n a multiple of 128; n < stored needs kInterleaved).
    FfnSliceWeights prefix(int64_t n) const;
};

int64_t packed_tile_index(int64_t c, int64_t r, int64_t tiles_k, int64_t tiles_n);

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

enum class GemvKernel { kHeteroMega, kHeteroMosaic };
enum class GemmKernel { kHeteroMosaic, kHeteroMega };

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

// Scratch of gpu_ffn_slice_forward: the engine's workspace for up to max_m rows.
struct GpuFfnBuffers {
    torch::Tensor workspace; // uint8, grown on demand
    std::vector<torch::Tensor> retired; // outgrown buffers, kept while enqueued work may still read them
    int64_t max_m = 0;
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

} // namespace heteromega

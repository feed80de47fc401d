// The reference's hipkernels:: and heteromega:: FFN operators over the engine's C ABI (declarations and contract:
// hm_reference_api.hpp). No kernels here: every call validates, finds (or makes, once) the engine's repacked copy
// of the packed tensor, and enqueues the engine's launch on the caller's stream.
#include "hm_reference_api.hpp"

#include "../../include/hm_w4a16.h"

#include <cstring>
#include <functional>
#include <stdexcept>
#include <string>
#include <tuple>

namespace {

// Argument errors as TORCH_CHECK (c10::Error), device errors as std::runtime_error: the reference's split between
// its TORCH_CHECKs (pack_w4a16.cpp:11-16) and its launch checks (w4a16_gemv_packed.cu:197-200).
void check(hm_status s) {
    if (s == HM_OK) {
        return;
    }
    if (s == HM_INVALID_ARGUMENT || s == HM_UNSUPPORTED || s == HM_WORKSPACE_TOO_SMALL) {
        TORCH_CHECK(false, hm_last_error());
    }
    throw std::runtime_error(std::string("W4A16 engine: ") + hm_last_error());
}

hm_dtype dtype_of(const torch::Tensor &t) {
    TORCH_CHECK(t.scalar_type() == torch::kBFloat16 || t.scalar_type() == torch::kHalf, "activations must be bfloat16 or float16, got ",
                t.scalar_type());
    return t.scalar_type() == torch::kHalf ? HM_FP16 : HM_BF16;
}

void check_packed(const torch::Tensor &p, int64_t pk, int64_t pn, const char *what) {
    TORCH_CHECK(p.is_cuda() && p.scalar_type() == torch::kUInt8 && p.is_contiguous(), what, ": packed parameters must be a contiguous device uint8 tensor");
    const int64_t bytes = hm_packed_bytes(pk, pn);
    TORCH_CHECK(bytes > 0 && p.numel() == bytes, what, ": a packed [", pk, ", ", pn, "] matrix has ", bytes, " bytes, got ", p.numel());
}

// Rows and leading dimension of a [..., width] activation with a contiguous last dimension.
std::pair<int64_t, int64_t> rows_ld(const torch::Tensor &t, const char *what) {
    TORCH_CHECK(t.is_cuda() && t.dim() >= 1 && t.stride(-1) == 1, what, ": needs a device tensor with a contiguous last dimension");
    const int64_t width = t.size(-1);
    const int64_t rows = width > 0 ? t.numel() / width : 0;
    const int64_t ld = t.dim() >= 2 && t.size(-2) > 1 ? t.stride(-2) : width;
    return {rows, ld};
}

// Repacked copies, one per packed tensor and use, kept for the life of the process.
struct Key {
    const void *ptr;
    int64_t a, b, c, d;
    int kind, dtype;
    bool operator==(const Key &o) const {
        return ptr == o.ptr && a == o.a && b == o.b && c == o.c && d == o.d && kind == o.kind && dtype == o.dtype;
    }
};
struct KeyHash {
    size_t operator()(const Key &k) const {
        size_t h = std::hash<const void *>()(k.ptr);
        for (int64_t v : {k.a, k.b, k.c, k.d, static_cast<int64_t>(k.kind), static_cast<int64_t>(k.dtype)}) {
            h = h * 1000003u ^ std::hash<int64_t>()(v);
        }
        return h;
    }
};
std::mutex g_mu;
std::unordered_map<Key, void *, KeyHash> g_repacked;

template <class Make> void *cached(const Key &key, Make make) {
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_repacked.find(key);
    if (it != g_repacked.end()) {
        return it->second;
    }
    void *h = make();
    g_repacked.emplace(key, h);
    return h;
}

// The whole packed [pk, pn] matrix, repacked once; calls compute any leading block of it.
hm_weights *matrix(const torch::Tensor &packed, int64_t pk, int64_t pn, hm_dtype dt, hipStream_t s, const char *what) {
    check_packed(packed, pk, pn, what);
    return static_cast<hm_weights *>(cached(Key{packed.data_ptr(), pk, pn, 0, 0, 0, dt}, [&]() {
        hm_weights *w = nullptr;
        check(hm_weights_from_tiles(packed.data_ptr<uint8_t>(), pk, pn, pk, pn, dt, s, &w));
        return static_cast<void *>(w);
    }));
}

// A gate_up matrix packed [pk, 2 stored] in `layout` order, repacked once as a fused matrix of all stored channels.
hm_weights *gate_up_matrix(const torch::Tensor &packed, int64_t pk, int64_t stored, heteromega::GateUpLayout layout, hm_dtype dt, hipStream_t s,
                           const char *what) {
    check_packed(packed, pk, 2 * stored, what);
    const int32_t lay = layout == heteromega::GateUpLayout::kInterleaved ? HM_GATE_UP_INTERLEAVED : HM_GATE_UP_BLOCKED;
    return static_cast<hm_weights *>(cached(Key{packed.data_ptr(), pk, stored, 0, 0, 1 + lay, dt}, [&]() {
        hm_weights *w = nullptr;
        check(hm_weights_from_gate_up_tiles(packed.data_ptr<uint8_t>(), pk, stored, pk, stored, lay, dt, s, &w));
        return static_cast<void *>(w);
    }));
}

// The FFN layer of a gate_up [h, 2 stored] and down [stored, h] pair, all stored channels.
hm_ffn *ffn_layer(const torch::Tensor &gate_up, const torch::Tensor &down, int64_t h, int64_t stored, heteromega::GateUpLayout layout, hm_dtype dt,
                  hipStream_t s) {
    check_packed(gate_up, h, 2 * stored, "gate_up");
    check_packed(down, stored, h, "down");
    const int32_t lay = layout == heteromega::GateUpLayout::kInterleaved ? HM_GATE_UP_INTERLEAVED : HM_GATE_UP_BLOCKED;
    return static_cast<hm_ffn *>(cached(Key{gate_up.data_ptr(), h, stored, reinterpret_cast<int64_t>(down.data_ptr()), 0, 3 + lay, dt}, [&]() {
        hm_ffn *f = nullptr;
        check(hm_ffn_from_gate_up_tiles(gate_up.data_ptr<uint8_t>(), down.data_ptr<uint8_t>(), h, stored, stored, lay, dt, s, &f));
        return static_cast<void *>(f);
    }));
}

// Per-stream workspace, grown as needed (the reference keeps its scratch per stream under a mutex, gpu_ffn.cpp:142-156).
// A replaced buffer is kept, not freed: work already enqueued on the stream may still read it, and the caching
// allocator would hand a freed block to its own stream at once.
std::mutex g_ws_mu;
std::unordered_map<hipStream_t, torch::Tensor> g_ws;
std::vector<torch::Tensor> g_ws_retired;

void *workspace(hipStream_t s, size_t bytes, const torch::Device &dev) {
    if (bytes == 0) {
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_ws_mu);
    torch::Tensor &t = g_ws[s];
    if (!t.defined() || static_cast<size_t>(t.numel()) < bytes + 256 || t.device() != dev) {
        if (t.defined()) {
            g_ws_retired.push_back(t);
        }
        t = torch::empty({static_cast<int64_t>(bytes + 256)}, torch::TensorOptions().dtype(torch::kUInt8).device(dev));
    }
    const uintptr_t p = reinterpret_cast<uintptr_t>(t.data_ptr());
    return reinterpret_cast<void *>((p + 255) & ~static_cast<uintptr_t>(255));
}

void linear(torch::Tensor &out, const torch::Tensor &in, hm_weights *w, int64_t k, int64_t n, int64_t col0, hipStream_t s) {
    const auto [m, ldx] = rows_ld(in, "input");
    const auto [mo, ldy] = rows_ld(out, "output");
    TORCH_CHECK(mo == m, "output rows ", mo, " != input rows ", m);
    TORCH_CHECK(in.scalar_type() == out.scalar_type(), "input and output dtypes differ");
    const size_t bytes = hm_linear_workspace_bytes(w, m, k, n);
    check(hm_linear(w, out.data_ptr(), ldy, in.data_ptr(), ldx, m, k, n, col0, workspace(s, bytes, in.device()), bytes, s));
}

void swiglu(torch::Tensor &act, const torch::Tensor &in, hm_weights *w, int64_t k, int64_t channels, hipStream_t s) {
    const auto [m, ldx] = rows_ld(in, "input");
    const auto [mo, lda] = rows_ld(act, "output");
    TORCH_CHECK(mo == m, "output rows ", mo, " != input rows ", m);
    const size_t bytes = hm_linear_swiglu_workspace_bytes(w, m, k, channels);
    check(hm_linear_swiglu(w, act.data_ptr(), lda, in.data_ptr(), ldx, m, k, 0, channels, workspace(s, bytes, in.device()), bytes, s));
}

void ffn_forward(hm_ffn *f, torch::Tensor &y, const torch::Tensor &x, int64_t channels, hipStream_t s) {
    const auto [m, ldx] = rows_ld(x, "x");
    const auto [my, ldy] = rows_ld(y, "y");
    TORCH_CHECK(my == m, "y rows ", my, " != x rows ", m);
    const size_t bytes = hm_ffn_workspace_bytes(f, m);
    check(hm_ffn_forward(f, y.data_ptr(), ldy, x.data_ptr(), ldx, m, 0, channels, workspace(s, bytes, x.device()), bytes, s));
}

} // namespace

namespace hipkernels {

void w4a16_gemm_fused_packed(torch::Tensor &output, const torch::Tensor &input, const torch::Tensor &packed_params, int64_t in_features,
                             int64_t out_features, hipStream_t stream) {
    hm_weights *w = matrix(packed_params, in_features, out_features, dtype_of(input), stream, "w4a16_gemm_fused_packed");
    linear(output, input, w, in_features, out_features, 0, stream);
}

void w4a16_gemm_fused_packed_tiles(torch::Tensor &output, const torch::Tensor &input, const torch::Tensor &packed_params,
                                   int64_t in_features, int64_t out_features, int64_t packed_tiles_k, int64_t packed_tiles_n,
                                   hipStream_t stream, bool fuse_activation) {
    const int64_t pk = packed_tiles_k * 128, pn = packed_tiles_n * 64;
    if (fuse_activation) {
        // gate/up interleaved per 64 channels (w4a16_gemm_packed.cu:549-578): out_features columns are out_features / 2 channels
        TORCH_CHECK(out_features % 2 == 0 && pn % 128 == 0, "w4a16_gemm_fused_packed_tiles: a fused gate_up needs whole 64-channel pairs");
        hm_weights *w = gate_up_matrix(packed_params, pk, pn / 2, heteromega::GateUpLayout::kInterleaved, dtype_of(input), stream,
                                       "w4a16_gemm_fused_packed_tiles");
        swiglu(output, input, w, in_features, out_features / 2, stream);
        return;
    }
    hm_weights *w = matrix(packed_params, pk, pn, dtype_of(input), stream, "w4a16_gemm_fused_packed_tiles");
    linear(output, input, w, in_features, out_features, 0, stream);
}

void w4a16_gemv_fused_packed(torch::Tensor &output, const torch::Tensor &input, const torch::Tensor &packed_params, int64_t in_features,
                             int64_t out_features, int64_t total_out_features, int64_t start_col, hipStream_t stream) {
    const int64_t width = total_out_features == -1 ? out_features : total_out_features;
    hm_weights *w = matrix(packed_params, in_features, width, dtype_of(input), stream, "w4a16_gemv_fused_packed");
    linear(output, input, w, in_features, out_features, start_col, stream);
}

} // namespace hipkernels

namespace heteromega {

FfnSliceWeights FfnSliceWeights::prefix(int64_t n) const {
    TORCH_CHECK(n > 0 && n <= stored_channels() && n % kTileK == 0, "FfnSliceWeights::prefix: n must be a multiple of 128 in (0, ",
                stored_channels(), "], got ", n);
    TORCH_CHECK(n == stored_channels() || layout == GateUpLayout::kInterleaved,
                "FfnSliceWeights::prefix: a shorter prefix needs GateUpLayout::kInterleaved");
    FfnSliceWeights w = *this;
    w.packed_channels = stored_channels();
    w.end = begin + n;
    return w;
}

int64_t packed_tile_index(int64_t c, int64_t r, int64_t tiles_k, int64_t tiles_n) { return hm_packed_tile_index(c, r, tiles_k, tiles_n); }

void silu_mul(const torch::Tensor &gate_up, torch::Tensor &act, hipStream_t stream, GateUpLayout layout) {
    TORCH_CHECK(gate_up.dim() == 2 && act.dim() == 2 && gate_up.size(0) == act.size(0) && gate_up.size(1) == 2 * act.size(1),
                "silu_mul: gate_up must be [M, 2n] and act [M, n]");
    TORCH_CHECK(gate_up.scalar_type() == act.scalar_type(), "silu_mul: dtypes differ");
    check(hm_silu_mul(gate_up.data_ptr(), gate_up.stride(0), act.data_ptr(), act.stride(0), act.size(0), act.size(1),
                      layout == GateUpLayout::kInterleaved ? HM_GATE_UP_INTERLEAVED : HM_GATE_UP_BLOCKED, dtype_of(act), stream));
}

void gemv_w4a16(torch::Tensor &out, const torch::Tensor &x, const torch::Tensor &packed, int64_t k, int64_t n, int64_t packed_k,
                int64_t packed_n, int split_k, hipStream_t stream) {
    (void)split_k; // the engine plans its own K split
    linear(out, x, matrix(packed, packed_k, packed_n, dtype_of(x), stream, "gemv_w4a16"), k, n, 0, stream);
}

void gemm_w4a16(torch::Tensor &out, const torch::Tensor &x, const torch::Tensor &packed, int64_t k, int64_t n, int64_t packed_k,
                int64_t packed_n, hipStream_t stream) {
    linear(out, x, matrix(packed, packed_k, packed_n, dtype_of(x), stream, "gemm_w4a16"), k, n, 0, stream);
}

bool gemm_w4a16_supports(int64_t m, int64_t k, int64_t n) { return m > 0 && k > 0 && k % 128 == 0 && n > 0 && n % (m > 16 ? 128 : 16) == 0; }

bool gemm_w4a16_ffn_supports(int64_t m, int64_t h, int64_t n) { return m > 0 && h > 0 && h % 128 == 0 && n > 0 && n % 128 == 0; }

void gemm_w4a16_ffn(torch::Tensor &y, const torch::Tensor &x, const torch::Tensor &gate_up, const torch::Tensor &down, int64_t h, int64_t n,
                    int64_t stored, hipStream_t stream) {
    TORCH_CHECK(n <= stored, "gemm_w4a16_ffn: n = ", n, " exceeds the ", stored, " stored channels");
    ffn_forward(ffn_layer(gate_up, down, h, stored, GateUpLayout::kInterleaved, dtype_of(x), stream), y, x, n, stream);
}

void packed_linear(torch::Tensor &out, const torch::Tensor &in, const torch::Tensor &packed, int64_t k, int64_t n, hipStream_t stream,
                   const LinearOptions &opt) {
    const int64_t pk = opt.packed_k > 0 ? opt.packed_k : k;
    const int64_t pn = opt.packed_n > 0 ? opt.packed_n : n;
    if (opt.fuse_activation) {
        TORCH_CHECK(n % 2 == 0 && pn % 128 == 0, "packed_linear: a fused gate_up needs whole 64-channel pairs");
        swiglu(out, in, gate_up_matrix(packed, pk, pn / 2, GateUpLayout::kInterleaved, dtype_of(in), stream, "packed_linear"), k, n / 2, stream);
        return;
    }
    linear(out, in, matrix(packed, pk, pn, dtype_of(in), stream, "packed_linear"), k, n, 0, stream);
}

GpuFfnBuffers GpuFfnBuffers::allocate(int64_t max_m, int64_t channels, int64_t hidden, const torch::Device &device) {
    (void)channels;
    (void)hidden;
    GpuFfnBuffers b;
    b.max_m = max_m;
    b.workspace = torch::empty({0}, torch::TensorOptions().dtype(torch::kUInt8).device(device));
    return b;
}

void gpu_ffn_slice_forward(const FfnSliceWeights &w, const torch::Tensor &x_norm, GpuFfnBuffers &buf, torch::Tensor &y, hipStream_t stream) {
    hm_ffn *f = ffn_layer(w.gate_up, w.down, w.hidden, w.stored_channels(), w.layout, dtype_of(x_norm), stream);
    const auto [m, ldx] = rows_ld(x_norm, "x_norm");
    const auto [my, ldy] = rows_ld(y, "y");
    TORCH_CHECK(my == m, "y rows ", my, " != x_norm rows ", m);
    const size_t bytes = hm_ffn_workspace_bytes(f, m);
    if (!buf.workspace.defined() || static_cast<size_t>(buf.workspace.numel()) < bytes + 256) {
        if (buf.workspace.defined()) {
            buf.retired.push_back(buf.workspace);
        }
        buf.workspace = torch::empty({static_cast<int64_t>(bytes + 256)}, torch::TensorOptions().dtype(torch::kUInt8).device(x_norm.device()));
    }
    const uintptr_t p = (reinterpret_cast<uintptr_t>(buf.workspace.data_ptr()) + 255) & ~static_cast<uintptr_t>(255);
    check(hm_ffn_forward(f, y.data_ptr(), ldy, x_norm.data_ptr(), ldx, m, 0, w.channels(), reinterpret_cast<void *>(p), bytes, stream));
}

void GpuFfnModel::add_layer(const torch::Tensor &gate, const torch::Tensor &up, const torch::Tensor &down, int64_t hidden, int64_t inter) {
    check_packed(gate, hidden, inter, "gate");
    check_packed(up, hidden, inter, "up");
    check_packed(down, inter, hidden, "down");
    TORCH_CHECK(layers_.empty() || inter == inter_, "GpuFfnModel::add_layer: every layer must have ", inter_, " channels");
    hm_ffn *f = nullptr;
    check(hm_ffn_from_tiles(gate.data_ptr<uint8_t>(), up.data_ptr<uint8_t>(), down.data_ptr<uint8_t>(), hidden, inter, HM_BF16, nullptr, &f));
    layers_.push_back(f);
    inter_ = inter;
    if (s_prefill_ == 0) {
        s_prefill_ = s_decode_ = inter;
    }
}

void GpuFfnModel::set_split(int64_t s_prefill, int64_t s_decode) {
    for (int64_t s : {s_prefill, s_decode}) {
        TORCH_CHECK(s > 0 && s <= inter_ && s % kTileK == 0, "GpuFfnModel::set_split: splits must be multiples of 128 in (0, ", inter_, "], got ", s);
    }
    s_prefill_ = s_prefill;
    s_decode_ = s_decode;
}

void GpuFfnModel::forward(int64_t layer, const torch::Tensor &x_norm, torch::Tensor &y, hipStream_t stream) {
    TORCH_CHECK(layer >= 0 && layer < layers(), "GpuFfnModel::forward: layer ", layer, " of ", layers());
    hm_ffn *f = static_cast<hm_ffn *>(layers_[layer]);
    const auto [m, ldx] = rows_ld(x_norm, "x_norm");
    const auto [my, ldy] = rows_ld(y, "y");
    TORCH_CHECK(my == m, "y rows ", my, " != x_norm rows ", m);
    const size_t bytes = hm_ffn_workspace_bytes(f, m);
    void *ws = nullptr;
    {
        std::lock_guard<std::mutex> lock(mutex_);
        torch::Tensor &t = workspaces_[stream];
        if (!t.defined() || static_cast<size_t>(t.numel()) < bytes + 256) {
            if (t.defined()) {
                retired_.push_back(t);
            }
            t = torch::empty({static_cast<int64_t>(bytes + 256)}, torch::TensorOptions().dtype(torch::kUInt8).device(x_norm.device()));
        }
        ws = reinterpret_cast<void *>((reinterpret_cast<uintptr_t>(t.data_ptr()) + 255) & ~static_cast<uintptr_t>(255));
    }
    check(hm_ffn_forward(f, y.data_ptr(), ldy, x_norm.data_ptr(), ldx, m, 0, channels(m), ws, bytes, stream));
}

GpuFfnModel::~GpuFfnModel() {
    for (void *f : layers_) {
        hm_ffn_destroy(static_cast<hm_ffn *>(f));
    }
}

} // namespace heteromega

// The reference's hipkernels:: and heteromega:: FFN operators over the engine's C ABI (declarations and contract:
// hm_reference_api.hpp). No kernels here: every call validates, finds (or makes, once) the engine's repacked copy
// of the packed tensor, and enqueues the engine's launch on the caller's stream.
#include "hm_reference_api.hpp"

#include "../../include/hm_w4a16.h"

#include <cstdlib>
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

// Repacked copies, one per packed tensor and use. An entry remembers the storage it was made from (a weak
// reference: the cache keeps no weights alive) and the tensors' version counters. It is used only while that
// storage is alive and unchanged: a freed tensor whose address the allocator hands to new weights, or weights
// rewritten in place, make the entry stale, and it is repacked from the current contents (the old copy freed).
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
// Identity of one source tensor at the time of the repack.
struct Source {
    c10::weak_intrusive_ptr<c10::StorageImpl> storage;
    int64_t version = 0;
    explicit Source(const torch::Tensor &t) : storage(t.storage().getWeakStorageImpl()), version(t._version()) {}
    bool matches(const torch::Tensor &t) const {
        return !storage.expired() && storage._unsafe_get_target() == t.storage().unsafeGetStorageImpl() && version == t._version();
    }
};
struct Entry {
    std::vector<Source> sources;
    void *handle = nullptr;
    void (*destroy)(void *) = nullptr;
};
std::mutex g_mu;
std::unordered_map<Key, Entry, KeyHash> g_repacked;

void destroy_weights(void *h) { hm_weights_destroy(static_cast<hm_weights *>(h)); }
void destroy_ffn(void *h) { hm_ffn_destroy(static_cast<hm_ffn *>(h)); }

// The repack enqueues on the caller's stream and then waits for it (the engine checks the zero points it read), so
// it cannot be captured into a graph: the first call per packed tensor must come before any capture.
void check_not_capturing(hipStream_t s, const char *what) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    TORCH_CHECK(hipStreamIsCapturing(s, &status) == hipSuccess && status == hipStreamCaptureStatusNone, what,
                ": the first call on a packed tensor repacks it and cannot run under stream capture; call it once before capturing");
}

template <class Make>
void *cached(const Key &key, std::initializer_list<const torch::Tensor *> tensors, void (*destroy)(void *), hipStream_t s, const char *what,
             Make make) {
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_repacked.find(key);
    if (it != g_repacked.end()) {
        bool fresh = it->second.sources.size() == tensors.size();
        size_t i = 0;
        for (const torch::Tensor *t : tensors) {
            fresh = fresh && it->second.sources[i++].matches(*t);
        }
        if (fresh) {
            return it->second.handle;
        }
        check_not_capturing(s, what);
        // hipFree in the destroy call waits for the device, so work still enqueued on the stale copy finishes first.
        it->second.destroy(it->second.handle);
        g_repacked.erase(it);
    } else {
        check_not_capturing(s, what);
    }
    Entry e;
    for (const torch::Tensor *t : tensors) {
        e.sources.emplace_back(*t);
    }
    e.handle = make();
    e.destroy = destroy;
    void *h = e.handle;
    g_repacked.emplace(key, std::move(e));
    return h;
}

// The whole packed [pk, pn] matrix, repacked once; calls compute any leading block of it.
hm_weights *matrix(const torch::Tensor &packed, int64_t pk, int64_t pn, hm_dtype dt, hipStream_t s, const char *what) {
    check_packed(packed, pk, pn, what);
    return static_cast<hm_weights *>(cached(Key{packed.data_ptr(), pk, pn, 0, 0, 0, dt}, {&packed}, destroy_weights, s, what, [&]() {
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
    return static_cast<hm_weights *>(cached(Key{packed.data_ptr(), pk, stored, 0, 0, 1 + lay, dt}, {&packed}, destroy_weights, s, what, [&]() {
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
    const Key key{gate_up.data_ptr(), h, stored, reinterpret_cast<int64_t>(down.data_ptr()), 0, 3 + lay, dt};
    return static_cast<hm_ffn *>(cached(key, {&gate_up, &down}, destroy_ffn, s, "FFN layer", [&]() {
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

// GemmInputReuse bookkeeping of this thread (see the header): the marked input and the GEMM calls that used it.
struct InputReuse {
    bool active = false;
    const void *x = nullptr;
    int64_t k = 0;
    hipStream_t stream = nullptr;
    int hits = 0;
};
thread_local InputReuse t_reuse;

void note_gemm_input(const torch::Tensor &in, int64_t k, hipStream_t s) {
    if (t_reuse.active && t_reuse.x == in.data_ptr() && t_reuse.k == k && t_reuse.stream == s) {
        ++t_reuse.hits;
    }
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
    note_gemm_input(x, k, stream);
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
    if (in.numel() > in.size(-1)) { // a GEMM (M > 1) with the kHeteroMega choice reads the prepared input in the reference
        note_gemm_input(in, k, stream);
    }
}

GpuFfnBuffers GpuFfnBuffers::allocate(int64_t max_m, int64_t channels, int64_t hidden, const torch::Device &device) {
    TORCH_CHECK(max_m > 0 && channels > 0 && hidden > 0, "GpuFfnBuffers::allocate: sizes must be positive");
    const auto opt = torch::TensorOptions().dtype(torch::kBFloat16).device(device);
    const int64_t rows = padded_rows(max_m);
    GpuFfnBuffers b;
    b.gate_up = torch::empty({rows, 2 * channels}, opt);
    b.act = torch::empty({rows, channels}, opt);
    b.x_pad = torch::empty({rows, hidden}, opt);
    return b;
}

void gpu_ffn_slice_forward(const FfnSliceWeights &w, const torch::Tensor &x_norm, GpuFfnBuffers &buf, torch::Tensor &y, hipStream_t stream) {
    hm_ffn *f = ffn_layer(w.gate_up, w.down, w.hidden, w.stored_channels(), w.layout, dtype_of(x_norm), stream);
    const auto [m, ldx] = rows_ld(x_norm, "x_norm");
    const auto [my, ldy] = rows_ld(y, "y");
    TORCH_CHECK(my == m, "y rows ", my, " != x_norm rows ", m);
    const size_t bytes = hm_ffn_workspace_bytes(f, m);
    // The engine's workspace: gate_up's storage when it holds it (the reference's own scratch for this call), else a
    // buffer grown in buf.workspace.
    const bool own = buf.gate_up.defined() && buf.gate_up.device() == x_norm.device() && buf.gate_up.nbytes() >= bytes + 256;
    if (!own && (!buf.workspace.defined() || static_cast<size_t>(buf.workspace.numel()) < bytes + 256 || buf.workspace.device() != x_norm.device())) {
        if (buf.workspace.defined()) {
            buf.retired.push_back(buf.workspace);
        }
        buf.workspace = torch::empty({static_cast<int64_t>(bytes + 256)}, torch::TensorOptions().dtype(torch::kUInt8).device(x_norm.device()));
    }
    void *base = own ? buf.gate_up.data_ptr() : buf.workspace.data_ptr();
    const uintptr_t p = (reinterpret_cast<uintptr_t>(base) + 255) & ~static_cast<uintptr_t>(255);
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

// ---- Weight packing ----

torch::Tensor pack_w4a16(const torch::Tensor &qweight, const torch::Tensor &scales, const torch::Tensor &zeros) {
    TORCH_CHECK(qweight.dim() == 2 && scales.dim() == 2 && zeros.dim() == 2, "pack_w4a16: qweight [K, N], scales and zeros [K / 128, N]");
    const int64_t K = qweight.size(0), N = qweight.size(1);
    TORCH_CHECK(K % kTileK == 0 && N % kTileN == 0, "pack_w4a16: K must be a multiple of 128 and N of 64, got ", K, "x", N);
    TORCH_CHECK(scales.size(0) == K / kTileK && scales.size(1) == N && zeros.size(0) == K / kTileK && zeros.size(1) == N,
                "pack_w4a16: scales and zeros must be [K / 128, N]");
    const auto q = qweight.to(torch::kCPU, torch::kUInt8).contiguous();
    const auto sc = scales.to(torch::kCPU, torch::kBFloat16).contiguous();
    const auto z = zeros.to(torch::kCPU, torch::kInt8).contiguous();
    auto out = torch::empty({hm_packed_bytes(K, N)}, torch::kUInt8);
    check(hm_pack_w4a16(q.data_ptr<uint8_t>(), reinterpret_cast<const uint16_t *>(sc.data_ptr()), z.data_ptr<int8_t>(), K, N,
                        out.data_ptr<uint8_t>()));
    return out;
}

FfnSliceWeights pack_ffn_slice(const FfnLayerQuant &layer, int64_t begin, int64_t end, GateUpLayout layout) {
    TORCH_CHECK(layer.gate_q.dim() == 2 && layer.down_q.dim() == 2, "pack_ffn_slice: gate_q [H, I] and down_q [I, H]");
    const int64_t hidden = layer.gate_q.size(0), inter = layer.gate_q.size(1);
    TORCH_CHECK(0 <= begin && begin < end && end <= inter && begin % kTileK == 0 && end % kTileK == 0,
                "pack_ffn_slice: channels [", begin, ", ", end, ") must be multiples of 128 within [0, ", inter, "]");
    TORCH_CHECK(layer.down_q.size(0) == inter && layer.down_q.size(1) == hidden, "pack_ffn_slice: down_q must be [I, H]");
    const int64_t n = end - begin;
    // [rows, n] gate and up columns -> [rows, 2n] in the layout's column order.
    const auto join = [&](const torch::Tensor &g, const torch::Tensor &u) {
        const torch::Tensor gs = g.slice(1, begin, end), us = u.slice(1, begin, end);
        if (layout == GateUpLayout::kBlocked) {
            return torch::cat({gs, us}, 1);
        }
        const int64_t r = gs.size(0);
        return torch::stack({gs.reshape({r, n / kTileN, kTileN}), us.reshape({r, n / kTileN, kTileN})}, 2).reshape({r, 2 * n});
    };
    FfnSliceWeights w;
    w.gate_up = pack_w4a16(join(layer.gate_q, layer.up_q), join(layer.gate_s, layer.up_s), join(layer.gate_z, layer.up_z));
    w.down = pack_w4a16(layer.down_q.slice(0, begin, end), layer.down_s.slice(0, begin / kTileK, end / kTileK),
                        layer.down_z.slice(0, begin / kTileK, end / kTileK));
    w.begin = begin;
    w.end = end;
    w.hidden = hidden;
    w.layout = layout;
    return w;
}

FfnSliceWeights slice_packed_ffn(const torch::Tensor &gate, const torch::Tensor &up, const torch::Tensor &down, int64_t hidden, int64_t inter,
                                 int64_t begin, int64_t end, GateUpLayout layout) {
    TORCH_CHECK(hidden > 0 && inter > 0 && hidden % kTileK == 0 && inter % kTileK == 0, "slice_packed_ffn: hidden and inter must be multiples of 128");
    TORCH_CHECK(0 <= begin && begin < end && end <= inter && begin % kTileK == 0 && end % kTileK == 0,
                "slice_packed_ffn: channels [", begin, ", ", end, ") must be multiples of 128 within [0, ", inter, "]");
    const int64_t matrix_bytes = hm_packed_bytes(hidden, inter);
    for (const torch::Tensor *t : {&gate, &up, &down}) {
        TORCH_CHECK(t->defined() && t->scalar_type() == torch::kUInt8 && t->is_contiguous() && t->numel() == matrix_bytes &&
                        t->device() == gate.device(),
                    "slice_packed_ffn: gate, up and down must be contiguous uint8 packed matrices of ", matrix_bytes, " bytes on one device");
    }
    const int64_t tiles_k = hidden / kTileK, tiles_n = inter / kTileN, n = end - begin, half = n / kTileN, out_n = 2 * half;
    const int64_t gate_tiles = tiles_k * tiles_n;
    // Destination tile -> source tile (gate's tiles, then up's), placed by the packed order of the result.
    std::vector<int64_t> src(static_cast<size_t>(tiles_k * out_n));
    for (int64_t c = 0; c < out_n; ++c) {
        const bool is_up = layout == GateUpLayout::kBlocked ? c >= half : (c & 1) == 1;
        const int64_t col = begin / kTileN + (layout == GateUpLayout::kBlocked ? c % half : c / 2);
        for (int64_t r = 0; r < tiles_k; ++r) {
            src[hm_packed_tile_index(c, r, tiles_k, out_n)] = (is_up ? gate_tiles : 0) + hm_packed_tile_index(col, r, tiles_k, tiles_n);
        }
    }
    const auto gather = [](const torch::Tensor &tiles, const std::vector<int64_t> &idx) {
        const auto i = torch::tensor(idx, torch::kInt64).to(tiles.device());
        return tiles.index_select(0, i).reshape({-1});
    };
    FfnSliceWeights w;
    w.gate_up = gather(torch::cat({gate.view({-1, kTileBytes}), up.view({-1, kTileBytes})}), src);
    if (begin == 0 && end == inter) {
        w.down = down;
    } else {
        const int64_t dk = inter / kTileK, dn = hidden / kTileN, rows = n / kTileK;
        std::vector<int64_t> didx(static_cast<size_t>(rows * dn));
        for (int64_t c = 0; c < dn; ++c) {
            for (int64_t r = 0; r < rows; ++r) {
                didx[hm_packed_tile_index(c, r, rows, dn)] = hm_packed_tile_index(c, begin / kTileK + r, dk, dn);
            }
        }
        w.down = gather(down.view({-1, kTileBytes}), didx);
    }
    w.begin = begin;
    w.end = end;
    w.hidden = hidden;
    w.layout = layout;
    return w;
}

FfnSliceWeights FfnSliceWeights::to(const torch::Device &device) const {
    FfnSliceWeights w = *this;
    w.gate_up = gate_up.to(device);
    w.down = down.to(device);
    return w;
}

// ---- GEMM input, layer boundary ----

torch::Tensor gemm_uncached_weights(const torch::Tensor &packed) { return packed; }

GemmInputReuse::GemmInputReuse() { t_reuse = InputReuse{true}; }
GemmInputReuse::~GemmInputReuse() { t_reuse = InputReuse{}; }
void GemmInputReuse::mark_prepared(const void *x, int64_t k, hipStream_t stream) {
    t_reuse.x = x;
    t_reuse.k = k;
    t_reuse.stream = stream;
}
int GemmInputReuse::hits() const { return t_reuse.hits; }

void gemm_input_buffers(int64_t m, int64_t k, hipStream_t stream, float **sums, uint16_t **tiles) {
    (void)m, (void)k, (void)stream;
    if (sums != nullptr) {
        *sums = nullptr;
    }
    if (tiles != nullptr) {
        *tiles = nullptr;
    }
    TORCH_CHECK(false, "gemm_input_buffers: the engine's GEMM reads its input rows from memory and keeps no prepared input");
}

bool residual_norm_supports(int64_t m, int64_t h) { return m > 0 && h > 0 && h % 8 == 0; }

void residual_norm_bf16(uint16_t *x, const uint16_t *a, const uint16_t *b, const uint16_t *weight, uint16_t *normed, const void *gemm_x,
                        GemmInputReuse &gemm_input, int64_t m, int64_t h, int64_t x_stride, int64_t a_stride, int64_t b_stride,
                        int64_t normed_stride, float eps, hipStream_t stream) {
    TORCH_CHECK(residual_norm_supports(m, h), "residual_norm_bf16: unsupported shape ", m, ", ", h);
    uint16_t *out = gemm_x != nullptr ? static_cast<uint16_t *>(const_cast<void *>(gemm_x)) : normed;
    TORCH_CHECK(out != nullptr, "residual_norm_bf16: needs gemm_x or normed to write the normalized rows to");
    check(hm_residual2_rmsnorm(x, x_stride, a, a_stride, b, b_stride, weight, out, normed_stride, m, h, eps, HM_BF16, stream));
    if (normed != nullptr && normed != out) {
        const size_t pitch = static_cast<size_t>(normed_stride) * 2;
        const hipError_t e = hipMemcpy2DAsync(normed, pitch, out, pitch, static_cast<size_t>(h) * 2, static_cast<size_t>(m), hipMemcpyDeviceToDevice, stream);
        if (e != hipSuccess) {
            throw std::runtime_error(std::string("residual_norm_bf16: copy of the normalized rows failed: ") + hipGetErrorString(e));
        }
    }
    gemm_input.mark_prepared(gemm_x, h, stream);
}

void residual_add2(torch::Tensor &x, const torch::Tensor &y_g, const torch::Tensor &y_n, hipStream_t stream) {
    TORCH_CHECK(x.dim() == 2 && x.is_cuda() && x.stride(1) == 1, "residual_add2: x must be a device [M, H] tensor with a contiguous last dimension");
    const hm_dtype dt = dtype_of(x);
    const auto operand = [&](const torch::Tensor &t, const char *name) {
        TORCH_CHECK(t.dim() == 2 && t.size(0) == x.size(0) && t.size(1) == x.size(1) && t.stride(1) == 1 && t.device() == x.device(), "residual_add2: ",
                    name, " must match x");
        TORCH_CHECK(t.scalar_type() == x.scalar_type() || t.scalar_type() == torch::kFloat32, "residual_add2: ", name, " must be of x's type or fp32");
        return t.scalar_type() == torch::kFloat32 ? 1 : 0;
    };
    const int32_t g32 = operand(y_g, "y_g"), n32 = operand(y_n, "y_n");
    check(hm_residual_add2_mixed(x.data_ptr(), x.stride(0), y_g.data_ptr(), y_g.stride(0), g32, y_n.data_ptr(), y_n.stride(0), n32, x.size(0),
                                 x.size(1), dt, stream));
}

GemmKernel configured_gemm_kernel() {
    static const GemmKernel kernel = [] {
        const char *v = std::getenv("HETEROMEGA_GEMM");
        return v != nullptr && std::string(v) == "fast" ? GemmKernel::kHeteroMega : GemmKernel::kHeteroMosaic;
    }();
    return kernel;
}

// ---- Nonfinite check ----

FiniteCheck parse_finite_check(const char *value) {
    if (value == nullptr || *value == '\0' || std::string(value) == "full") {
        return FiniteCheck::kFull;
    }
    if (std::string(value) == "sampled") {
        return FiniteCheck::kSampled;
    }
    throw std::invalid_argument(std::string("merged FFN: HETEROMEGA_FFN_FINITE_CHECK must be full or sampled, not ") + value);
}

int64_t find_nonfinite_bf16(const uint16_t *bits, int64_t rows, int64_t columns, FiniteCheck mode) {
    return hm_find_nonfinite(bits, rows, columns, columns, HM_BF16, mode == FiniteCheck::kSampled ? 1 : 0);
}

void find_nonfinite_device(const torch::Tensor &t, FiniteCheck mode, torch::Tensor &first, hipStream_t stream) {
    TORCH_CHECK(t.is_cuda() && t.dim() == 2 && t.stride(1) == 1, "find_nonfinite_device: t must be a device [M, N] tensor with a contiguous last dimension");
    TORCH_CHECK(first.is_cuda() && first.scalar_type() == torch::kInt64 && first.numel() == 1, "find_nonfinite_device: first must be one device int64");
    check(hm_find_nonfinite_device(t.data_ptr(), t.size(0), t.size(1), t.stride(0), dtype_of(t), mode == FiniteCheck::kSampled ? 1 : 0,
                                   first.data_ptr<int64_t>(), stream));
}

} // namespace heteromega

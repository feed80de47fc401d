// Python access to the reference-signature C++ operators (hm_reference_api.hpp), so that tests call the very
// functions a C++ caller of the reference would: torch tensors in, the HIP stream as an integer (the pattern of
// the reference's experiments/ffn_partition/gpu_bindings.cpp:9-44).
#include <torch/extension.h>

#include "hm_reference_api.hpp"

namespace {

hipStream_t as_stream(uint64_t s) { return reinterpret_cast<hipStream_t>(s); }

heteromega::GateUpLayout layout_of(const std::string &name) {
    TORCH_CHECK(name == "blocked" || name == "interleaved", "layout must be 'blocked' or 'interleaved'");
    return name == "interleaved" ? heteromega::GateUpLayout::kInterleaved : heteromega::GateUpLayout::kBlocked;
}

} // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "The reference's hipkernels:: and heteromega:: FFN operators over the MI355X engine";
    m.def("w4a16_gemm_fused_packed", [](torch::Tensor out, const torch::Tensor &in, const torch::Tensor &packed, int64_t k, int64_t n,
                                         uint64_t stream) { hipkernels::w4a16_gemm_fused_packed(out, in, packed, k, n, as_stream(stream)); });
    m.def("w4a16_gemm_fused_packed_tiles",
          [](torch::Tensor out, const torch::Tensor &in, const torch::Tensor &packed, int64_t k, int64_t n, int64_t tiles_k, int64_t tiles_n,
             uint64_t stream, bool fuse) { hipkernels::w4a16_gemm_fused_packed_tiles(out, in, packed, k, n, tiles_k, tiles_n, as_stream(stream), fuse); });
    m.def("w4a16_gemv_fused_packed", [](torch::Tensor out, const torch::Tensor &in, const torch::Tensor &packed, int64_t k, int64_t n,
                                         int64_t total_n, int64_t start_col, uint64_t stream) {
        hipkernels::w4a16_gemv_fused_packed(out, in, packed, k, n, total_n, start_col, as_stream(stream));
    });
    m.def("gemv_w4a16", [](torch::Tensor out, const torch::Tensor &x, const torch::Tensor &packed, int64_t k, int64_t n, int64_t pk, int64_t pn,
                           int split_k, uint64_t stream) { heteromega::gemv_w4a16(out, x, packed, k, n, pk, pn, split_k, as_stream(stream)); });
    m.def("gemm_w4a16", [](torch::Tensor out, const torch::Tensor &x, const torch::Tensor &packed, int64_t k, int64_t n, int64_t pk, int64_t pn,
                           uint64_t stream) { heteromega::gemm_w4a16(out, x, packed, k, n, pk, pn, as_stream(stream)); });
    m.def("gemm_w4a16_supports", &heteromega::gemm_w4a16_supports);
    m.def("gemm_w4a16_ffn_supports", &heteromega::gemm_w4a16_ffn_supports);
    m.def("gemm_w4a16_ffn", [](torch::Tensor y, const torch::Tensor &x, const torch::Tensor &gate_up, const torch::Tensor &down, int64_t h, int64_t n,
                               int64_t stored, uint64_t stream) { heteromega::gemm_w4a16_ffn(y, x, gate_up, down, h, n, stored, as_stream(stream)); });
    m.def("silu_mul", [](const torch::Tensor &gate_up, torch::Tensor act, uint64_t stream, const std::string &layout) {
        heteromega::silu_mul(gate_up, act, as_stream(stream), layout_of(layout));
    });
    m.def("packed_linear", [](torch::Tensor out, const torch::Tensor &in, const torch::Tensor &packed, int64_t k, int64_t n, uint64_t stream,
                              int64_t packed_k, int64_t packed_n, bool fuse) {
        heteromega::LinearOptions opt;
        opt.packed_k = packed_k;
        opt.packed_n = packed_n;
        opt.fuse_activation = fuse;
        heteromega::packed_linear(out, in, packed, k, n, as_stream(stream), opt);
    });
    m.def("gpu_ffn_slice_forward", [](const torch::Tensor &gate_up, const torch::Tensor &down, int64_t begin, int64_t end, int64_t hidden,
                                      const std::string &layout, int64_t packed_channels, const torch::Tensor &x_norm, torch::Tensor y,
                                      uint64_t stream) {
        heteromega::FfnSliceWeights w;
        w.gate_up = gate_up;
        w.down = down;
        w.begin = begin;
        w.end = end;
        w.hidden = hidden;
        w.layout = layout_of(layout);
        w.packed_channels = packed_channels;
        auto buf = heteromega::GpuFfnBuffers::allocate(x_norm.size(0), w.channels(), hidden, x_norm.device());
        heteromega::gpu_ffn_slice_forward(w, x_norm, buf, y, as_stream(stream));
        // kept alive by the caller until the stream has run the launch
        return pybind11::make_tuple(buf.gate_up, buf.act, buf.x_pad, buf.workspace.defined() ? buf.workspace : torch::Tensor());
    });
    m.def("pack_w4a16", &heteromega::pack_w4a16);
    m.def("pack_ffn_slice", [](const std::vector<torch::Tensor> &t, int64_t begin, int64_t end, const std::string &layout) {
        TORCH_CHECK(t.size() == 9, "pack_ffn_slice: gate q/s/z, up q/s/z, down q/s/z");
        heteromega::FfnLayerQuant q{t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7], t[8]};
        const auto w = heteromega::pack_ffn_slice(q, begin, end, layout_of(layout));
        return pybind11::make_tuple(w.gate_up, w.down, w.begin, w.end, w.hidden);
    });
    m.def("slice_packed_ffn", [](const torch::Tensor &gate, const torch::Tensor &up, const torch::Tensor &down, int64_t hidden, int64_t inter,
                                 int64_t begin, int64_t end, const std::string &layout, const std::string &device) {
        auto w = heteromega::slice_packed_ffn(gate, up, down, hidden, inter, begin, end, layout_of(layout));
        if (!device.empty()) {
            w = w.to(torch::Device(device));
        }
        return pybind11::make_tuple(w.gate_up, w.down, w.begin, w.end, w.hidden);
    });
    m.def("residual_add2", [](torch::Tensor x, const torch::Tensor &y_g, const torch::Tensor &y_n, uint64_t stream) {
        heteromega::residual_add2(x, y_g, y_n, as_stream(stream));
    });
    m.def("residual_norm_supports", &heteromega::residual_norm_supports);
    // Tensors stand for the reference's raw pointers (an undefined tensor for a null one). After the boundary, one
    // gemm_w4a16 per packed [h, n] matrix in gemm_w reads gemm_x, as the reference's Q/K/V GEMMs do; returns the reuse's
    // hits and their outputs.
    m.def("residual_norm_bf16", [](torch::Tensor x, const std::optional<torch::Tensor> &a, const std::optional<torch::Tensor> &b,
                                   const torch::Tensor &weight, const std::optional<torch::Tensor> &normed, torch::Tensor gemm_x, float eps,
                                   uint64_t stream, const std::vector<torch::Tensor> &gemm_w, int64_t n) {
        auto ptr = [](const std::optional<torch::Tensor> &t) { return t ? reinterpret_cast<uint16_t *>(t->data_ptr()) : nullptr; };
        heteromega::GemmInputReuse reuse;
        const int64_t m = x.size(0), h = x.size(1);
        heteromega::residual_norm_bf16(reinterpret_cast<uint16_t *>(x.data_ptr()), ptr(a), ptr(b), reinterpret_cast<const uint16_t *>(weight.data_ptr()),
                                       ptr(normed), gemm_x.data_ptr(), reuse, m, h, x.stride(0), a ? a->stride(0) : 0, b ? b->stride(0) : 0,
                                       gemm_x.stride(0), eps, as_stream(stream));
        std::vector<torch::Tensor> outs;
        for (const auto &w : gemm_w) {
            auto out = torch::empty({m, n}, gemm_x.options());
            heteromega::gemm_w4a16(out, gemm_x, w, h, n, h, n, as_stream(stream));
            outs.push_back(out);
        }
        return pybind11::make_tuple(reuse.hits(), outs);
    });
    m.def("gemm_input_buffers", [](int64_t m, int64_t k, uint64_t stream) {
        float *sums = nullptr;
        uint16_t *tiles = nullptr;
        heteromega::gemm_input_buffers(m, k, as_stream(stream), &sums, &tiles);
    });
    m.def("configured_gemm_kernel", []() { return heteromega::configured_gemm_kernel() == heteromega::GemmKernel::kHeteroMega ? "fast" : "mosaic"; });
    m.def("gemm_uncached_weights", &heteromega::gemm_uncached_weights);
    m.def("parse_finite_check", [](const std::string &v, bool null) {
        return heteromega::parse_finite_check(null ? nullptr : v.c_str()) == heteromega::FiniteCheck::kSampled ? "sampled" : "full";
    });
    m.def("find_nonfinite_bf16", [](const torch::Tensor &bits, bool sampled) {
        TORCH_CHECK(bits.device().is_cpu() && bits.dim() == 2 && bits.is_contiguous() && bits.element_size() == 2, "CPU [rows, columns] 16-bit tensor");
        return heteromega::find_nonfinite_bf16(reinterpret_cast<const uint16_t *>(bits.data_ptr()), bits.size(0), bits.size(1),
                                               sampled ? heteromega::FiniteCheck::kSampled : heteromega::FiniteCheck::kFull);
    });
    m.def("find_nonfinite_device", [](const torch::Tensor &t, bool sampled, torch::Tensor first, uint64_t stream) {
        heteromega::find_nonfinite_device(t, sampled ? heteromega::FiniteCheck::kSampled : heteromega::FiniteCheck::kFull, first, as_stream(stream));
    });
    pybind11::class_<heteromega::GpuFfnModel>(m, "GpuFfnModel")
        .def(pybind11::init<>())
        .def("add_layer", &heteromega::GpuFfnModel::add_layer)
        .def("set_split", &heteromega::GpuFfnModel::set_split)
        .def("layers", &heteromega::GpuFfnModel::layers)
        .def("channels", &heteromega::GpuFfnModel::channels)
        .def("forward", [](heteromega::GpuFfnModel &self, int64_t layer, const torch::Tensor &x_norm, torch::Tensor y, uint64_t stream) {
            self.forward(layer, x_norm, y, as_stream(stream));
        });
}

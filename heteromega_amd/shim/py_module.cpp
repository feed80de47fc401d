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
        return buf.workspace; // kept alive by the caller until the stream has run the launch
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

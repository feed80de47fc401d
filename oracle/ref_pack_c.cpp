// Test infrastructure only (a checker, never on the product path): a C interface to the reference's own packing code,
// kernels/gpu/src/pack_w4a16.cpp:9-176 (pack_w4a16, pack_ffn_slice, packed_tile_index, slice_packed_ffn), which
// oracle/build_ref.py compiles from its place under the reference tree together with this file into
// oracle/_ref/libref_pack.so. The tests call it through ctypes on host buffers to pin the oracle's and the engine's
// packers byte for byte against the reference's. Nothing here is the reference's code: it only wraps raw buffers in
// CPU tensors, calls the reference's functions and copies their results out.
#include "heteromega/gpu_ffn.hpp"

#include <cstdint>
#include <cstring>
#include <exception>

namespace {

torch::Tensor host(const void *p, int64_t rows, int64_t cols, torch::ScalarType t) {
    return torch::from_blob(const_cast<void *>(p), {rows, cols}, torch::TensorOptions().dtype(t)).clone();
}

void copy_out(const torch::Tensor &t, uint8_t *out) {
    const auto c = t.contiguous().to(torch::kCPU);
    std::memcpy(out, c.data_ptr(), static_cast<size_t>(c.numel()) * c.element_size());
}

} // namespace

extern "C" {

// out (K / 128 * N / 64 * 4352 bytes) = heteromega::pack_w4a16(q [K, N] u8, scales [K/128, N] bf16 bits, zeros int8). 0 on success.
int ref_pack_w4a16(const uint8_t *q, const uint16_t *scales, const int8_t *zeros, int64_t K, int64_t N, uint8_t *out) {
    try {
        copy_out(heteromega::pack_w4a16(host(q, K, N, torch::kUInt8), host(scales, K / 128, N, torch::kBFloat16),
                                        host(zeros, K / 128, N, torch::kInt8)),
                 out);
        return 0;
    } catch (const std::exception &) {
        return 1;
    }
}

int64_t ref_packed_tile_index(int64_t c, int64_t r, int64_t tiles_k, int64_t tiles_n) {
    return heteromega::packed_tile_index(c, r, tiles_k, tiles_n);
}

// heteromega::pack_ffn_slice of a layer given as nine host arrays (gate/up [H, I], down [I, H], groups of 128);
// gate_up_out holds H / 128 * 2n / 64 tiles and down_out n / 128 * H / 64 tiles (n = end - begin).
int ref_pack_ffn_slice(const uint8_t *gq, const uint16_t *gs, const int8_t *gz, const uint8_t *uq, const uint16_t *us, const int8_t *uz,
                       const uint8_t *dq, const uint16_t *ds, const int8_t *dz, int64_t H, int64_t I, int64_t begin, int64_t end, int interleaved,
                       uint8_t *gate_up_out, uint8_t *down_out) {
    try {
        heteromega::FfnLayerQuant L;
        L.gate_q = host(gq, H, I, torch::kUInt8), L.gate_s = host(gs, H / 128, I, torch::kBFloat16), L.gate_z = host(gz, H / 128, I, torch::kInt8);
        L.up_q = host(uq, H, I, torch::kUInt8), L.up_s = host(us, H / 128, I, torch::kBFloat16), L.up_z = host(uz, H / 128, I, torch::kInt8);
        L.down_q = host(dq, I, H, torch::kUInt8), L.down_s = host(ds, I / 128, H, torch::kBFloat16), L.down_z = host(dz, I / 128, H, torch::kInt8);
        const auto w = heteromega::pack_ffn_slice(L, begin, end, interleaved ? heteromega::GateUpLayout::kInterleaved : heteromega::GateUpLayout::kBlocked);
        copy_out(w.gate_up, gate_up_out);
        copy_out(w.down, down_out);
        return 0;
    } catch (const std::exception &) {
        return 1;
    }
}

// heteromega::slice_packed_ffn on host copies of packed gate [H, I], up [H, I] and down [I, H].
int ref_slice_packed_ffn(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int64_t H, int64_t I, int64_t begin, int64_t end,
                         int interleaved, uint8_t *gate_up_out, uint8_t *down_out) {
    try {
        const int64_t bytes = (H / 128) * (I / 64) * 4352;
        const auto t = [&](const uint8_t *p) { return host(p, 1, bytes, torch::kUInt8).view({bytes}); };
        const auto w = heteromega::slice_packed_ffn(t(gate), t(up), t(down), H, I, begin, end,
                                                    interleaved ? heteromega::GateUpLayout::kInterleaved : heteromega::GateUpLayout::kBlocked);
        copy_out(w.gate_up, gate_up_out);
        copy_out(w.down, down_out);
        return 0;
    } catch (const std::exception &) {
        return 1;
    }
}

} // extern "C"

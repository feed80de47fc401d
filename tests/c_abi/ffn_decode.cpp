// A C++ host over the C ABI alone (include/hm_w4a16.h; no Python, no torch), as the reference's C++ model
// integration would call it: packs a small SwiGLU FFN layer into the reference's 4352-byte tiles on the host
// (hm_pack_w4a16), repacks it on the GPU (hm_ffn_from_tiles), runs hm_ffn_forward at M = 1, 3, 16 and 48 (the
// one-row, few-row, several-row and GEMM paths) and checks the output against a float64 evaluation of the same
// weights computed here. Prints PASS and exits 0
// on success; exits 2 when no GPU is visible.
#include "hm_w4a16.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

namespace {

uint16_t bf16_bits(float f) { // round to nearest even (finite inputs)
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

float bf16_value(uint16_t b) {
    const uint32_t u = static_cast<uint32_t>(b) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// One [K, N] W4A16 matrix, group 128: q and z uniform 0..15, scales bf16 U(0.001, 0.02).
struct Matrix {
    int K = 0, N = 0;
    std::vector<uint8_t> q;
    std::vector<uint16_t> s;
    std::vector<int8_t> z;
    std::vector<double> w; // (q - z) * s
};

Matrix random_matrix(int K, int N, std::mt19937 &rng) {
    Matrix m;
    m.K = K;
    m.N = N;
    std::uniform_int_distribution<int> nib(0, 15);
    std::uniform_real_distribution<float> sc(0.001f, 0.02f);
    m.q.resize(static_cast<size_t>(K) * N);
    m.s.resize(static_cast<size_t>(K / 128) * N);
    m.z.resize(m.s.size());
    for (auto &v : m.q) v = static_cast<uint8_t>(nib(rng));
    for (auto &v : m.s) v = bf16_bits(sc(rng));
    for (auto &v : m.z) v = static_cast<int8_t>(nib(rng));
    m.w.resize(m.q.size());
    for (int k = 0; k < K; ++k) {
        for (int n = 0; n < N; ++n) {
            const size_t g = static_cast<size_t>(k / 128) * N + n;
            m.w[static_cast<size_t>(k) * N + n] = (static_cast<double>(m.q[static_cast<size_t>(k) * N + n]) - m.z[g]) * bf16_value(m.s[g]);
        }
    }
    return m;
}

#define CHECK_HM(call)                                                                                   \
    do {                                                                                                 \
        const hm_status st_ = (call);                                                                    \
        if (st_ != HM_OK) {                                                                              \
            std::fprintf(stderr, "%s: status %d: %s\n", #call, static_cast<int>(st_), hm_last_error()); \
            return 1;                                                                                    \
        }                                                                                                \
    } while (0)

#define CHECK_HIP(call)                                                                  \
    do {                                                                                 \
        const hipError_t e_ = (call);                                                    \
        if (e_ != hipSuccess) {                                                          \
            std::fprintf(stderr, "%s: %s\n", #call, hipGetErrorString(e_));              \
            return 1;                                                                    \
        }                                                                                \
    } while (0)

} // namespace

int main() {
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
        std::fprintf(stderr, "no GPU visible\n");
        return 2;
    }
    const int H = 1024, I = 2048, MaxM = 48;
    std::mt19937 rng(1234);
    const Matrix mats[3] = {random_matrix(H, I, rng), random_matrix(H, I, rng), random_matrix(I, H, rng)};

    // Host packing into the reference format, then the device copies the repack reads.
    uint8_t *tiles[3] = {};
    for (int i = 0; i < 3; ++i) {
        const int64_t bytes = hm_packed_bytes(mats[i].K, mats[i].N);
        if (bytes <= 0) {
            std::fprintf(stderr, "hm_packed_bytes rejected [%d, %d]\n", mats[i].K, mats[i].N);
            return 1;
        }
        std::vector<uint8_t> packed(static_cast<size_t>(bytes));
        CHECK_HM(hm_pack_w4a16(mats[i].q.data(), mats[i].s.data(), mats[i].z.data(), mats[i].K, mats[i].N, packed.data()));
        CHECK_HIP(hipMalloc(&tiles[i], packed.size()));
        CHECK_HIP(hipMemcpy(tiles[i], packed.data(), packed.size(), hipMemcpyHostToDevice));
    }
    hm_ffn *ffn = nullptr;
    CHECK_HM(hm_ffn_from_tiles(tiles[0], tiles[1], tiles[2], H, I, HM_BF16, nullptr, &ffn));
    const size_t ws_bytes = hm_ffn_workspace_bytes(ffn, MaxM);
    void *ws = nullptr;
    uint16_t *dx = nullptr, *dy = nullptr;
    CHECK_HIP(hipMalloc(&ws, ws_bytes));
    CHECK_HIP(hipMalloc(&dx, static_cast<size_t>(MaxM) * H * 2));
    CHECK_HIP(hipMalloc(&dy, static_cast<size_t>(MaxM) * H * 2));

    std::normal_distribution<float> normal(0.0f, 1.0f);
    for (const int M : {1, 3, 16, MaxM}) {
        std::vector<uint16_t> x(static_cast<size_t>(M) * H), y(x.size());
        for (auto &v : x) v = bf16_bits(normal(rng));
        CHECK_HIP(hipMemcpy(dx, x.data(), x.size() * 2, hipMemcpyHostToDevice));
        CHECK_HM(hm_ffn_forward(ffn, dy, H, dx, H, M, 0, I, ws, ws_bytes, nullptr));
        CHECK_HIP(hipDeviceSynchronize());
        CHECK_HIP(hipMemcpy(y.data(), dy, y.size() * 2, hipMemcpyDeviceToHost));

        // float64 reference: act = bf16(SiLU(x Wg) * (x Wu)), y = act Wd.
        double err2 = 0.0, ref2 = 0.0, max_err = 0.0, max_ref = 0.0;
        std::vector<double> act(I);
        for (int r = 0; r < M; ++r) {
            for (int c = 0; c < I; ++c) {
                double g = 0.0, u = 0.0;
                for (int k = 0; k < H; ++k) {
                    const double xv = bf16_value(x[static_cast<size_t>(r) * H + k]);
                    g += xv * mats[0].w[static_cast<size_t>(k) * I + c];
                    u += xv * mats[1].w[static_cast<size_t>(k) * I + c];
                }
                act[c] = bf16_value(bf16_bits(static_cast<float>(g / (1.0 + std::exp(-g)) * u)));
            }
            for (int n = 0; n < H; ++n) {
                double ref = 0.0;
                for (int c = 0; c < I; ++c) {
                    ref += act[c] * mats[2].w[static_cast<size_t>(c) * H + n];
                }
                const double got = bf16_value(y[static_cast<size_t>(r) * H + n]);
                if (!std::isfinite(got)) {
                    std::fprintf(stderr, "M=%d: non-finite output at row %d column %d\n", M, r, n);
                    return 1;
                }
                err2 += (got - ref) * (got - ref);
                ref2 += ref * ref;
                max_err = std::fmax(max_err, std::fabs(got - ref));
                max_ref = std::fmax(max_ref, std::fabs(ref));
            }
        }
        const double max_rel = max_err / max_ref, rel_l2 = std::sqrt(err2 / ref2);
        std::printf("M=%d: max_rel=%.3e rel_l2=%.3e\n", M, max_rel, rel_l2);
        if (!(max_rel <= 1e-2 && rel_l2 <= 5e-3)) { // the bf16 bar of the Python parity tests
            std::fprintf(stderr, "M=%d: outside tolerance\n", M);
            return 1;
        }
    }
    CHECK_HM(hm_ffn_destroy(ffn));
    for (uint8_t *t : tiles) CHECK_HIP(hipFree(t));
    CHECK_HIP(hipFree(ws));
    CHECK_HIP(hipFree(dx));
    CHECK_HIP(hipFree(dy));
    std::printf("PASS\n");
    return 0;
}

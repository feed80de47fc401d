// C ABI of the W4A16 FFN engine (include/hm_w4a16.h): validation, allocation at create time, dispatch.
#include "../../include/hm_w4a16.h"
#include "hm_internal.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <mutex>
#include <string>

struct hm_weights {
    hm::Planes p;
    void *buffer = nullptr;
    int64_t bytes = 0;
    int64_t quant_bytes = 0, meta_bytes = 0;
    uint32_t *status = nullptr; // device word after the planes: the repack's out-of-range zero flag
    bool fused = false;         // gate_up: strips alternate gate / up per 16 channels (N = 2 x channels)
};

struct hm_ffn {
    hm_weights gate_up; // [H, 2 I], strips alternate gate / up per 16 channels
    hm_weights down;    // [I, H]
    int64_t hidden = 0, inter = 0;
    size_t decode_partial[17] = {}; // largest split-partial buffer of any call of 1..m rows (m <= 16), planned at creation
};

namespace {

// The last error message of this thread: a fixed buffer, so that reporting an error allocates nothing.
thread_local char g_error[512];

hm_status vfail(hm_status s, const char *fmt, va_list ap) {
    std::vsnprintf(g_error, sizeof(g_error), fmt, ap);
    return s;
}

hm_status fail(hm_status s, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vfail(s, fmt, ap);
    va_end(ap);
    return s;
}

hm_status hip_fail(hipError_t e, const char *what) {
    return fail(e == hipErrorOutOfMemory ? HM_OUT_OF_MEMORY : HM_HIP_ERROR, "%s: %s", what, hipGetErrorString(e));
}

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

bool valid_group(int64_t g) { return g == 32 || g == 64 || g == 128; }

int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// Allocates both planes of a K x N matrix in one device buffer.
hm_status alloc_planes(hm_weights *w, int64_t K, int64_t N, int64_t group, int dtype) {
    w->p.K = K;
    w->p.N = N;
    w->p.group = group;
    w->p.dtype = dtype;
    w->quant_bytes = K * N / 2;
    w->meta_bytes = (N / 16) * (K / group) * 16 * 4;
    const int64_t meta_off = round_up(w->quant_bytes, 256);
    const int64_t status_off = round_up(meta_off + w->meta_bytes, 256);
    w->bytes = status_off + 256;
    const hipError_t e = hipMalloc(&w->buffer, static_cast<size_t>(w->bytes));
    if (e != hipSuccess) {
        w->buffer = nullptr;
        return hip_fail(e, "hipMalloc of the repacked weights");
    }
    w->p.quant = static_cast<const uint8_t *>(w->buffer);
    w->p.meta = reinterpret_cast<const uint32_t *>(static_cast<uint8_t *>(w->buffer) + meta_off);
    w->status = reinterpret_cast<uint32_t *>(static_cast<uint8_t *>(w->buffer) + status_off);
    return HM_OK;
}

// Clears the zero-point flag before a repack (load time only, never inside a captured graph).
hm_status begin_repack(hm_weights *w, hipStream_t s) {
    const hipError_t e = hipMemsetAsync(w->status, 0, sizeof(uint32_t), s);
    return e == hipSuccess ? HM_OK : hip_fail(e, "clearing the repack status");
}

// Waits for the repack and reports zero points outside 0..16: the kernels read zeros as unsigned bytes and build
// 1024 + z and 1024 + 16 z in fp16, exact only for small z; the reference's GPU reads tile zeros as int8
// (w4a16_gemv_packed.cu:86-87) and its CPU as uint8 (w4a16_gemv_avx_packed.cpp:122-124), which agree on 0..127.
hm_status end_repack(const hm_weights *w, hipStream_t s, const char *what) {
    uint32_t flag = 0;
    hipError_t e = hipMemcpyAsync(&flag, w->status, sizeof(flag), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) {
        e = hipStreamSynchronize(s);
    }
    if (e != hipSuccess) {
        return hip_fail(e, "repack");
    }
    if (flag != 0) {
        return fail(HM_INVALID_ARGUMENT, "%s: zero points must lie in 0..%u", what, hm::kMaxZero);
    }
    return HM_OK;
}

void free_planes(hm_weights *w) {
    if (w->buffer != nullptr) {
        (void)hipFree(w->buffer);
        w->buffer = nullptr;
    }
}

hm_status check_dtype(hm_dtype dtype) {
    if (dtype != HM_BF16 && dtype != HM_FP16) {
        return fail(HM_INVALID_ARGUMENT, "dtype must be HM_BF16 or HM_FP16, got %d", static_cast<int>(dtype));
    }
    return HM_OK;
}

hm_status check_tile_source(const uint8_t *tiles, int64_t packed_k, int64_t packed_n, int64_t K, int64_t N, const char *what) {
    if (tiles == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "%s: null packed matrix", what);
    }
    if (packed_k <= 0 || packed_n <= 0 || packed_k % 128 || packed_n % 64) {
        return fail(HM_INVALID_ARGUMENT, "%s: packed matrix [%lld, %lld] must be multiples of 128 x 64", what,
                    static_cast<long long>(packed_k), static_cast<long long>(packed_n));
    }
    if (K <= 0 || N <= 0 || K % 128 || N % 16 || K > packed_k || N > packed_n) {
        return fail(HM_INVALID_ARGUMENT, "%s: block [%lld, %lld] must be multiples of 128 x 16 inside [%lld, %lld]", what,
                    static_cast<long long>(K), static_cast<long long>(N), static_cast<long long>(packed_k),
                    static_cast<long long>(packed_n));
    }
    return HM_OK;
}

// A reference gate_up matrix packed [packed_k, 2 stored] in `layout` order (kernels/gpu/include/heteromega/gpu_ffn.hpp:
// 43-71: FfnSliceWeights.gate_up); the engine takes channels [0, channels) over K rows.
hm_status check_gate_up_source(const uint8_t *gate_up, int64_t packed_k, int64_t stored, int64_t K, int64_t channels, int32_t layout,
                               const char *what) {
    if (layout != HM_GATE_UP_BLOCKED && layout != HM_GATE_UP_INTERLEAVED) {
        return fail(HM_INVALID_ARGUMENT, "%s: layout must be HM_GATE_UP_BLOCKED or HM_GATE_UP_INTERLEAVED, got %d", what, static_cast<int>(layout));
    }
    if (stored <= 0 || stored % 64) {
        return fail(HM_INVALID_ARGUMENT, "%s: stored channels %lld must be a positive multiple of 64", what, static_cast<long long>(stored));
    }
    if (channels <= 0 || channels % 16 || channels > stored) {
        return fail(HM_INVALID_ARGUMENT, "%s: channels %lld must be a positive multiple of 16 within the %lld stored", what,
                    static_cast<long long>(channels), static_cast<long long>(stored));
    }
    return check_tile_source(gate_up, packed_k, 2 * stored, K, 2 * channels, what);
}

// The gate and up halves of a reference gate_up matrix as the two sources of a fused repack.
void gate_up_sources(const uint8_t *gate_up, int64_t packed_k, int64_t stored, int32_t layout, hm::TileSource gu[2]) {
    for (int i = 0; i < 2; ++i) {
        gu[i].tiles = gate_up;
        gu[i].tiles_k = packed_k / 128;
        gu[i].tiles_n = 2 * stored / 64;
        if (layout == HM_GATE_UP_INTERLEAVED) {
            gu[i].col_mode = 1 + i; // per 64 channels: 64 gate columns, then 64 up columns
        } else {
            gu[i].col_offset = i * stored; // [gate 0..stored) | up 0..stored)]
        }
    }
}

hm_status check_logical(const uint8_t *q, const uint16_t *s, const uint8_t *z, int64_t K, int64_t N, int64_t group,
                        const char *what) {
    if (q == nullptr || s == nullptr || z == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "%s: null tensor", what);
    }
    if (!valid_group(group)) {
        return fail(HM_INVALID_ARGUMENT, "%s: group must be 32, 64 or 128, got %lld", what, static_cast<long long>(group));
    }
    if (K <= 0 || N <= 0 || K % 128 || N % 16) {
        return fail(HM_INVALID_ARGUMENT, "%s: [%lld, %lld] must be multiples of 128 x 16", what, static_cast<long long>(K),
                    static_cast<long long>(N));
    }
    return HM_OK;
}

// Rows beyond this use the MFMA GEMM; up to it, the decode GEMV.
constexpr int64_t kGemvMaxRows = 16;

hm_status run_linear(const hm::Planes &p, void *y, int64_t ldy, const void *x, int64_t ldx, int64_t M, int64_t strip_begin,
                     int64_t n, int64_t kt_begin, int64_t kt_count, bool fused, void *workspace, size_t workspace_bytes,
                     hipStream_t stream, bool accumulate = false) {
    if (M <= kGemvMaxRows) {
        hm::GemvCall c;
        c.w = p;
        c.x = static_cast<const uint16_t *>(x);
        c.ldx = ldx;
        c.y = static_cast<uint16_t *>(y);
        c.ldy = ldy;
        c.m = M;
        c.strip_begin = strip_begin;
        c.n = n;
        c.kt_begin = kt_begin;
        c.kt_count = kt_count;
        c.fused = fused;
        c.accumulate = accumulate;
        const size_t need = hm::plan_gemv(c).partial_bytes;
        if (need > workspace_bytes) {
            return fail(HM_WORKSPACE_TOO_SMALL, "workspace of %zu bytes, need %zu", workspace_bytes, need);
        }
        c.partial = static_cast<float *>(workspace);
        const hipError_t e = hm::launch_gemv(c, stream);
        return e == hipSuccess ? HM_OK : hip_fail(e, "gemv launch");
    }
    const int64_t cols = fused ? 2 * n : n;
    if (cols % 128) {
        return fail(HM_UNSUPPORTED, "GEMM path (M > %lld) needs %s a multiple of %d, got %lld", static_cast<long long>(kGemvMaxRows),
                    fused ? "channels" : "n", fused ? 64 : 128, static_cast<long long>(n));
    }
    hm::GemmCall c;
    c.w = p;
    c.x = static_cast<const uint16_t *>(x);
    c.ldx = ldx;
    c.y = static_cast<uint16_t *>(y);
    c.ldy = ldy;
    c.m = M;
    c.strip_begin = strip_begin;
    c.n = n;
    c.kt_begin = kt_begin;
    c.kt_count = kt_count;
    c.fused = fused;
    c.accumulate = accumulate;
    const size_t need = hm::plan_gemm(c).partial_bytes;
    if (need > workspace_bytes) {
        return fail(HM_WORKSPACE_TOO_SMALL, "workspace of %zu bytes, need %zu", workspace_bytes, need);
    }
    c.partial = static_cast<float *>(workspace);
    const hipError_t e = hm::launch_gemm(c, stream);
    return e == hipSuccess ? HM_OK : hip_fail(e, "gemm launch");
}

// Workspace for any call of M rows over up to n columns (any column range within them) and kt_count K tiles.
size_t linear_workspace(const hm::Planes &p, int64_t M, int64_t n, int64_t kt_count, bool fused) {
    if (M > kGemvMaxRows) {
        // A narrower column range has a smaller grid and may split K further: the largest plan over every width
        // (at most kGemmPartialMax). More K tiles never split less, so kt_count itself bounds the K ranges.
        hm::GemmCall c;
        c.w = p;
        c.m = M;
        c.kt_count = kt_count;
        c.fused = fused;
        size_t need = 0;
        for (int64_t w = fused ? 64 : 128; w <= n; w += fused ? 64 : 128) {
            c.n = w;
            need = std::max(need, hm::plan_gemm(c).partial_bytes);
        }
        return need;
    }
    hm::GemvCall c;
    c.w = p;
    c.m = M;
    c.n = n;
    c.kt_count = kt_count;
    c.fused = fused;
    return hm::gemv_partial_bound(c);
}

hm_status check_activation(const void *x, int64_t ldx, int64_t width, const char *what) {
    if (x == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "%s: null pointer", what);
    }
    if (!aligned(x, 16) || ldx % 8 || ldx < width) {
        return fail(HM_INVALID_ARGUMENT, "%s: needs 16-byte alignment and a leading dimension that is a multiple of 8 and >= %lld (got %lld)",
                    what, static_cast<long long>(width), static_cast<long long>(ldx));
    }
    return HM_OK;
}

hm_status check_output(const void *y, int64_t ldy, int64_t width, const char *what) {
    if (y == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "%s: null pointer", what);
    }
    if (!aligned(y, 2) || ldy < width) {
        return fail(HM_INVALID_ARGUMENT, "%s: leading dimension %lld < %lld", what, static_cast<long long>(ldy), static_cast<long long>(width));
    }
    return HM_OK;
}

hm_status check_channels(const hm_ffn *f, int64_t b, int64_t e) {
    if (b < 0 || b >= e || e > f->inter || b % 128 || e % 128) {
        return fail(HM_INVALID_ARGUMENT, "channel range [%lld, %lld) must be a nonempty range of multiples of 128 inside [0, %lld)",
                    static_cast<long long>(b), static_cast<long long>(e), static_cast<long long>(f->inter));
    }
    return HM_OK;
}

} // namespace

namespace {

hm_status check_ffn_shape(int64_t hidden, int64_t inter, const char *what) {
    if (hidden <= 0 || inter <= 0 || hidden % 128 || inter % 128) {
        return fail(HM_INVALID_ARGUMENT, "%s: hidden and inter must be positive multiples of 128, got %lld, %lld", what,
                    static_cast<long long>(hidden), static_cast<long long>(inter));
    }
    return HM_OK;
}

void destroy_ffn(hm_ffn *f) {
    free_planes(&f->gate_up);
    free_planes(&f->down);
    delete f;
}

// An FFN layer with both planes allocated (gate_up [H, 2 I] fused, down [I, H]).
hm_status new_ffn(int64_t hidden, int64_t inter, int64_t group, hm_dtype dtype, hm_ffn **out) {
    auto *f = new (std::nothrow) hm_ffn;
    if (f == nullptr) {
        return fail(HM_OUT_OF_MEMORY, "host allocation of a layer handle failed");
    }
    f->hidden = hidden;
    f->inter = inter;
    hm_status st = alloc_planes(&f->gate_up, hidden, 2 * inter, group, dtype);
    if (st == HM_OK && (st = alloc_planes(&f->down, inter, hidden, group, dtype)) != HM_OK) {
        free_planes(&f->gate_up);
    }
    if (st != HM_OK) {
        delete f;
        return st;
    }
    f->gate_up.fused = true;
    *out = f;
    return HM_OK;
}

// Runs the repack launches of a new layer (launches(flag) enqueues them with the zero-point flag), waits for them
// and publishes the layer, or frees it on any failure.
template <class Launches> hm_status fill_ffn(hm_ffn *f, hipStream_t s, const char *what, hm_ffn **out, Launches launches) {
    hm_status st = begin_repack(&f->gate_up, s);
    if (st == HM_OK) {
        const hipError_t e = launches(f->gate_up.status);
        st = e != hipSuccess ? hip_fail(e, "repack launch") : end_repack(&f->gate_up, s, what);
    }
    if (st != HM_OK) {
        destroy_ffn(f);
        return st;
    }
    for (int64_t m = 1; m <= kGemvMaxRows; ++m) {
        const size_t d = linear_workspace(f->down.p, m, f->hidden, f->inter / 128, false);
        const size_t g = linear_workspace(f->gate_up.p, m, f->inter, f->hidden / 128, true);
        f->decode_partial[m] = std::max({f->decode_partial[m - 1], d, g});
    }
    *out = f;
    return HM_OK;
}

// gate_up from two tile sources (separate gate and up matrices, or the halves of one gate_up matrix), down from a
// packed [down_k, down_n] matrix whose leading [inter, hidden] block is the layer's.
hm_status build_ffn_from_tiles(const hm::TileSource gu[2], const uint8_t *down, int64_t down_k, int64_t down_n, int64_t hidden, int64_t inter,
                               hm_dtype dtype, hipStream_t s, const char *what, hm_ffn **out) {
    hm_ffn *f = nullptr;
    hm_status st = new_ffn(hidden, inter, 128, dtype, &f);
    if (st != HM_OK) {
        return st;
    }
    hm::TileSource d;
    d.tiles = down;
    d.tiles_k = down_k / 128;
    d.tiles_n = down_n / 64;
    return fill_ffn(f, s, what, out, [&](uint32_t *flag) {
        hipError_t e = hm::launch_repack_tiles(gu, 2, true, const_cast<uint8_t *>(f->gate_up.p.quant), const_cast<uint32_t *>(f->gate_up.p.meta),
                                               hidden, 2 * inter, dtype, flag, s);
        if (e == hipSuccess) {
            e = hm::launch_repack_tiles(&d, 1, false, const_cast<uint8_t *>(f->down.p.quant), const_cast<uint32_t *>(f->down.p.meta), inter,
                                        hidden, dtype, flag, s);
        }
        return e;
    });
}

size_t one_row_spill_bytes(int64_t channels) { return static_cast<size_t>(round_up(static_cast<int64_t>(hm::gemv_pair_spill_bytes(channels)), 256)); }

} // namespace

hm::Topology hm::device_topology() {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static Topology cache[kMaxDevices];
    static bool known[kMaxDevices] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        return Topology{};
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!known[dev]) {
        Topology t;
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) {
            t.cus = v;
        }
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeNumberOfXccs, dev) == hipSuccess && v > 0) {
            t.xcds = v;
        }
        cache[dev] = t;
        known[dev] = true;
    }
    return cache[dev];
}

hm_status hm::set_error(hm_status s, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vfail(s, fmt, ap);
    va_end(ap);
    return s;
}

extern "C" {

int hm_abi_version(void) { return HM_ABI_VERSION; }

const char *hm_last_error(void) { return g_error; }

int64_t hm_packed_bytes(int64_t K, int64_t N) {
    if (K <= 0 || N <= 0 || K % 128 || N % 64) {
        return -1;
    }
    return (K / 128) * (N / 64) * 4352;
}

int64_t hm_packed_tile_index(int64_t c, int64_t r, int64_t tiles_k, int64_t tiles_n) {
    if (tiles_k <= 0 || tiles_n <= 0 || c < 0 || c >= tiles_n || r < 0 || r >= tiles_k) {
        return -1;
    }
    int64_t before = c / 8;
    for (int64_t g = 0; g < c % 8; ++g) {
        before += (tiles_n - g + 7) / 8;
    }
    return before * tiles_k + r;
}

hm_status hm_pack_w4a16(const uint8_t *q, const uint16_t *scales, const int8_t *zeros, int64_t K, int64_t N, uint8_t *out) {
    if (q == nullptr || scales == nullptr || zeros == nullptr || out == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_pack_w4a16: null pointer");
    }
    if (K <= 0 || N <= 0 || K % 128 || N % 64) {
        return fail(HM_INVALID_ARGUMENT, "hm_pack_w4a16: K must be a multiple of 128 and N of 64, got %lldx%lld",
                    static_cast<long long>(K), static_cast<long long>(N));
    }
    for (int64_t i = 0; i < (K / 128) * N; ++i) {
        if (zeros[i] < 0 || zeros[i] > static_cast<int>(hm::kMaxZero)) {
            return fail(HM_INVALID_ARGUMENT, "hm_pack_w4a16: zero point %d at [%lld, %lld] is outside 0..%u", static_cast<int>(zeros[i]),
                        static_cast<long long>(i / N), static_cast<long long>(i % N), hm::kMaxZero);
        }
    }
    const int64_t tiles_k = K / 128, tiles_n = N / 64;
    for (int64_t c = 0; c < tiles_n; ++c) {
        for (int64_t r = 0; r < tiles_k; ++r) {
            uint8_t *tile = out + hm_packed_tile_index(c, r, tiles_k, tiles_n) * 4352;
            // Byte ((a * 8 + cc) * 8 + b) * 4 + j: row 8 a + b, columns 8 cc + 2 j (low) and + 1 (high).
            for (int byte = 0; byte < 4096; ++byte) {
                const int j = byte & 3, b = (byte >> 2) & 7, cc = (byte >> 5) & 7, a = byte >> 8;
                const uint8_t *row = q + (r * 128 + a * 8 + b) * N + c * 64 + cc * 8 + 2 * j;
                tile[byte] = static_cast<uint8_t>((row[0] & 0x0F) | ((row[1] & 0x0F) << 4));
            }
            std::memcpy(tile + 4096, scales + r * N + c * 64, 128);
            for (int i = 0; i < 64; ++i) {
                const uint8_t z = static_cast<uint8_t>(zeros[r * N + c * 64 + i]);
                tile[4224 + (i >> 3) * 16 + (i & 7)] = z;
                tile[4224 + (i >> 3) * 16 + 8 + (i & 7)] = z;
            }
        }
    }
    return HM_OK;
}

hm_status hm_awq_unpack(const int32_t *packed, int64_t rows, int64_t cols8, uint8_t *out) {
    if (packed == nullptr || out == nullptr || rows <= 0 || cols8 <= 0) {
        return fail(HM_INVALID_ARGUMENT, "hm_awq_unpack: bad arguments");
    }
    static const int order[8] = {0, 4, 1, 5, 2, 6, 3, 7};
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t j = 0; j < cols8; ++j) {
            const uint32_t v = static_cast<uint32_t>(packed[r * cols8 + j]);
            for (int k = 0; k < 8; ++k) {
                out[r * cols8 * 8 + 8 * j + k] = static_cast<uint8_t>((v >> (4 * order[k])) & 0xFu);
            }
        }
    }
    return HM_OK;
}

hm_status hm_gptq_unpack(const int32_t *packed, int64_t rows8, int64_t cols, uint8_t *out) {
    if (packed == nullptr || out == nullptr || rows8 <= 0 || cols <= 0) {
        return fail(HM_INVALID_ARGUMENT, "hm_gptq_unpack: bad arguments");
    }
    for (int64_t r = 0; r < rows8; ++r) {
        for (int64_t c = 0; c < cols; ++c) {
            const uint32_t v = static_cast<uint32_t>(packed[r * cols + c]);
            for (int k = 0; k < 8; ++k) {
                out[(8 * r + k) * cols + c] = static_cast<uint8_t>((v >> (4 * k)) & 0xFu);
            }
        }
    }
    return HM_OK;
}

hm_status hm_gptq_unpack_zeros(const int32_t *packed, int64_t groups, int64_t cols8, int32_t add_one, uint8_t *out) {
    if (packed == nullptr || out == nullptr || groups <= 0 || cols8 <= 0) {
        return fail(HM_INVALID_ARGUMENT, "hm_gptq_unpack_zeros: bad arguments");
    }
    for (int64_t g = 0; g < groups; ++g) {
        for (int64_t j = 0; j < cols8; ++j) {
            const uint32_t v = static_cast<uint32_t>(packed[g * cols8 + j]);
            for (int k = 0; k < 8; ++k) {
                out[g * cols8 * 8 + 8 * j + k] = static_cast<uint8_t>(((v >> (4 * k)) & 0xFu) + (add_one ? 1 : 0));
            }
        }
    }
    return HM_OK;
}

hm_status hm_weights_from_tiles(const uint8_t *tiles, int64_t packed_k, int64_t packed_n, int64_t K, int64_t N, hm_dtype dtype,
                                void *stream, hm_weights **out) {
    if (out == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_weights_from_tiles: null output handle");
    }
    *out = nullptr;
    hm_status st = check_dtype(dtype);
    if (st != HM_OK || (st = check_tile_source(tiles, packed_k, packed_n, K, N, "hm_weights_from_tiles")) != HM_OK) {
        return st;
    }
    auto *w = new (std::nothrow) hm_weights;
    if (w == nullptr) {
        return fail(HM_OUT_OF_MEMORY, "host allocation of a weights handle failed");
    }
    if ((st = alloc_planes(w, K, N, 128, dtype)) != HM_OK) {
        delete w;
        return st;
    }
    hm::TileSource src;
    src.tiles = tiles;
    src.tiles_k = packed_k / 128;
    src.tiles_n = packed_n / 64;
    const hipStream_t s = as_stream(stream);
    if ((st = begin_repack(w, s)) == HM_OK) {
        const hipError_t e = hm::launch_repack_tiles(&src, 1, false, const_cast<uint8_t *>(w->p.quant), const_cast<uint32_t *>(w->p.meta), K,
                                                     N, dtype, w->status, s);
        st = e != hipSuccess ? hip_fail(e, "repack launch") : end_repack(w, s, "hm_weights_from_tiles");
    }
    if (st != HM_OK) {
        free_planes(w);
        delete w;
        return st;
    }
    *out = w;
    return HM_OK;
}

hm_status hm_weights_from_logical(const uint8_t *q, const uint16_t *scales, const uint8_t *zeros, int64_t K, int64_t N, int64_t group,
                                  hm_dtype dtype, void *stream, hm_weights **out) {
    if (out == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_weights_from_logical: null output handle");
    }
    *out = nullptr;
    hm_status st = check_dtype(dtype);
    if (st != HM_OK || (st = check_logical(q, scales, zeros, K, N, group, "hm_weights_from_logical")) != HM_OK) {
        return st;
    }
    auto *w = new (std::nothrow) hm_weights;
    if (w == nullptr) {
        return fail(HM_OUT_OF_MEMORY, "host allocation of a weights handle failed");
    }
    if ((st = alloc_planes(w, K, N, group, dtype)) != HM_OK) {
        delete w;
        return st;
    }
    hm::LogicalSource src;
    src.q = q;
    src.scales = scales;
    src.zeros = zeros;
    src.ld = N;
    const hipStream_t s = as_stream(stream);
    if ((st = begin_repack(w, s)) == HM_OK) {
        const hipError_t e = hm::launch_repack_logical(&src, 1, false, const_cast<uint8_t *>(w->p.quant), const_cast<uint32_t *>(w->p.meta),
                                                       K, N, group, w->status, s);
        st = e != hipSuccess ? hip_fail(e, "repack launch") : end_repack(w, s, "hm_weights_from_logical");
    }
    if (st != HM_OK) {
        free_planes(w);
        delete w;
        return st;
    }
    *out = w;
    return HM_OK;
}

hm_status hm_weights_from_gate_up_tiles(const uint8_t *gate_up, int64_t packed_k, int64_t stored, int64_t K, int64_t channels,
                                        int32_t layout, hm_dtype dtype, void *stream, hm_weights **out) {
    if (out == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_weights_from_gate_up_tiles: null output handle");
    }
    *out = nullptr;
    hm_status st = check_dtype(dtype);
    if (st != HM_OK || (st = check_gate_up_source(gate_up, packed_k, stored, K, channels, layout, "hm_weights_from_gate_up_tiles")) != HM_OK) {
        return st;
    }
    auto *w = new (std::nothrow) hm_weights;
    if (w == nullptr) {
        return fail(HM_OUT_OF_MEMORY, "host allocation of a weights handle failed");
    }
    if ((st = alloc_planes(w, K, 2 * channels, 128, dtype)) != HM_OK) {
        delete w;
        return st;
    }
    w->fused = true;
    hm::TileSource gu[2];
    gate_up_sources(gate_up, packed_k, stored, layout, gu);
    const hipStream_t s = as_stream(stream);
    if ((st = begin_repack(w, s)) == HM_OK) {
        const hipError_t e = hm::launch_repack_tiles(gu, 2, true, const_cast<uint8_t *>(w->p.quant), const_cast<uint32_t *>(w->p.meta), K,
                                                     2 * channels, dtype, w->status, s);
        st = e != hipSuccess ? hip_fail(e, "repack launch") : end_repack(w, s, "hm_weights_from_gate_up_tiles");
    }
    if (st != HM_OK) {
        free_planes(w);
        delete w;
        return st;
    }
    *out = w;
    return HM_OK;
}

hm_status hm_weights_dequantize(const hm_weights *w, void *out, int64_t ld_out, int32_t transposed, void *stream) {
    if (w == nullptr || out == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_weights_dequantize: null pointer");
    }
    const int64_t width = transposed ? w->p.K : w->p.N;
    if (ld_out < width || (transposed && (ld_out % 8 || !aligned(out, 16))) || !aligned(out, 2)) {
        return fail(HM_INVALID_ARGUMENT,
                    "hm_weights_dequantize: leading dimension %lld must be >= %lld (and, transposed, a multiple of 8 with 16-byte alignment)",
                    static_cast<long long>(ld_out), static_cast<long long>(width));
    }
    const hipError_t e = hm::launch_dequantize(w->p, static_cast<uint16_t *>(out), ld_out, transposed != 0, as_stream(stream));
    return e == hipSuccess ? HM_OK : hip_fail(e, "dequantize launch");
}

hm_status hm_weights_to_logical(const hm_weights *w, uint8_t *q, uint16_t *scales, uint8_t *zeros, void *stream) {
    if (w == nullptr || q == nullptr || scales == nullptr || zeros == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_weights_to_logical: null pointer");
    }
    const hipError_t e = hm::launch_unpack(w->p, q, scales, zeros, as_stream(stream));
    return e == hipSuccess ? HM_OK : hip_fail(e, "unpack launch");
}

hm_status hm_weights_info(const hm_weights *w, int64_t *K, int64_t *N, int64_t *group, int32_t *dtype, int64_t *device_bytes) {
    if (w == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_weights_info: null handle");
    }
    if (K) *K = w->p.K;
    if (N) *N = w->p.N;
    if (group) *group = w->p.group;
    if (dtype) *dtype = w->p.dtype;
    if (device_bytes) *device_bytes = w->bytes;
    return HM_OK;
}

hm_status hm_weights_planes(const hm_weights *w, const void **quant, int64_t *quant_bytes, const void **meta, int64_t *meta_bytes) {
    if (w == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_weights_planes: null handle");
    }
    if (quant) *quant = w->p.quant;
    if (quant_bytes) *quant_bytes = w->quant_bytes;
    if (meta) *meta = w->p.meta;
    if (meta_bytes) *meta_bytes = w->meta_bytes;
    return HM_OK;
}

hm_status hm_weights_destroy(hm_weights *w) {
    if (w != nullptr) {
        free_planes(w);
        delete w;
    }
    return HM_OK;
}

hm_status hm_weights_concat(const hm_weights *const *parts, int32_t count, void *stream, hm_weights **out) {
    if (out == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_weights_concat: null output handle");
    }
    *out = nullptr;
    if (parts == nullptr || count <= 0) {
        return fail(HM_INVALID_ARGUMENT, "hm_weights_concat: no parts");
    }
    int64_t n = 0;
    for (int32_t i = 0; i < count; ++i) {
        const hm_weights *w = parts[i];
        if (w == nullptr) {
            return fail(HM_INVALID_ARGUMENT, "hm_weights_concat: part %d is null", static_cast<int>(i));
        }
        if (w->fused) {
            return fail(HM_INVALID_ARGUMENT, "hm_weights_concat: part %d is a fused gate_up matrix", static_cast<int>(i));
        }
        if (w->p.K != parts[0]->p.K || w->p.group != parts[0]->p.group || w->p.dtype != parts[0]->p.dtype) {
            return fail(HM_INVALID_ARGUMENT, "hm_weights_concat: part %d has K %lld, group %lld, dtype %d; part 0 has %lld, %lld, %d",
                        static_cast<int>(i), static_cast<long long>(w->p.K), static_cast<long long>(w->p.group), w->p.dtype,
                        static_cast<long long>(parts[0]->p.K), static_cast<long long>(parts[0]->p.group), parts[0]->p.dtype);
        }
        n += w->p.N;
    }
    auto *c = new (std::nothrow) hm_weights;
    if (c == nullptr) {
        return fail(HM_OUT_OF_MEMORY, "host allocation of a weights handle failed");
    }
    hm_status st = alloc_planes(c, parts[0]->p.K, n, parts[0]->p.group, parts[0]->p.dtype);
    if (st != HM_OK) {
        delete c;
        return st;
    }
    // Both planes are strip-major (a strip's K tiles, then the next strip), so the parts' planes concatenate.
    int64_t qo = 0, mo = 0;
    for (int32_t i = 0; i < count; ++i) {
        const hm_weights *w = parts[i];
        hipError_t e = hipMemcpyAsync(const_cast<uint8_t *>(c->p.quant) + qo, w->p.quant, static_cast<size_t>(w->quant_bytes),
                                      hipMemcpyDeviceToDevice, as_stream(stream));
        if (e == hipSuccess) {
            e = hipMemcpyAsync(reinterpret_cast<uint8_t *>(const_cast<uint32_t *>(c->p.meta)) + mo, w->p.meta,
                               static_cast<size_t>(w->meta_bytes), hipMemcpyDeviceToDevice, as_stream(stream));
        }
        if (e != hipSuccess) {
            free_planes(c);
            delete c;
            return hip_fail(e, "hm_weights_concat copy");
        }
        qo += w->quant_bytes;
        mo += w->meta_bytes;
    }
    *out = c;
    return HM_OK;
}

size_t hm_linear_workspace_bytes(const hm_weights *w, int64_t M, int64_t k, int64_t n) {
    if (w == nullptr || M <= 0 || k <= 0 || n <= 0) {
        return 0;
    }
    return linear_workspace(w->p, M, n, k / 128, false);
}

hm_status hm_linear(const hm_weights *w, void *y, int64_t ldy, const void *x, int64_t ldx, int64_t M, int64_t k, int64_t n, int64_t col_begin,
                    void *workspace, size_t workspace_bytes, void *stream) {
    if (w == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_linear: null weights");
    }
    if (w->fused) {
        return fail(HM_INVALID_ARGUMENT, "hm_linear: a fused gate_up matrix runs through hm_linear_swiglu");
    }
    if (M <= 0 || k <= 0 || n <= 0 || k % 128 || n % 16 || col_begin < 0 || col_begin % 16 || k > w->p.K || col_begin + n > w->p.N) {
        return fail(HM_INVALID_ARGUMENT, "hm_linear: block k=%lld, columns [%lld, %lld) must be multiples of 128 / 16 inside [%lld, %lld]",
                    static_cast<long long>(k), static_cast<long long>(col_begin), static_cast<long long>(col_begin + n),
                    static_cast<long long>(w->p.K), static_cast<long long>(w->p.N));
    }
    hm_status st = check_activation(x, ldx, k, "hm_linear x");
    if (st != HM_OK || (st = check_output(y, ldy, n, "hm_linear y")) != HM_OK) {
        return st;
    }
    return run_linear(w->p, y, ldy, x, ldx, M, col_begin / 16, n, 0, k / 128, false, workspace, workspace_bytes, as_stream(stream));
}

size_t hm_linear_swiglu_workspace_bytes(const hm_weights *w, int64_t M, int64_t k, int64_t channels) {
    if (w == nullptr || !w->fused || M <= 0 || k <= 0 || channels <= 0) {
        return 0;
    }
    return linear_workspace(w->p, M, channels, k / 128, true);
}

hm_status hm_linear_swiglu(const hm_weights *w, void *act, int64_t ld_act, const void *x, int64_t ldx, int64_t M, int64_t k, int64_t ch_begin,
                           int64_t ch_end, void *workspace, size_t workspace_bytes, void *stream) {
    if (w == nullptr || !w->fused) {
        return fail(HM_INVALID_ARGUMENT, "hm_linear_swiglu: needs a fused gate_up matrix (hm_weights_from_gate_up_tiles)");
    }
    const int64_t channels = w->p.N / 2;
    if (M <= 0 || k <= 0 || k % 128 || k > w->p.K || ch_begin < 0 || ch_begin >= ch_end || ch_end > channels || ch_begin % 16 || ch_end % 16) {
        return fail(HM_INVALID_ARGUMENT, "hm_linear_swiglu: k=%lld (multiple of 128, <= %lld) and channels [%lld, %lld) (multiples of 16 within %lld)",
                    static_cast<long long>(k), static_cast<long long>(w->p.K), static_cast<long long>(ch_begin), static_cast<long long>(ch_end),
                    static_cast<long long>(channels));
    }
    hm_status st = check_activation(x, ldx, k, "hm_linear_swiglu x");
    if (st != HM_OK || (st = check_output(act, ld_act, ch_end - ch_begin, "hm_linear_swiglu act")) != HM_OK) {
        return st;
    }
    return run_linear(w->p, act, ld_act, x, ldx, M, 2 * (ch_begin / 16), ch_end - ch_begin, 0, k / 128, true, workspace, workspace_bytes,
                      as_stream(stream));
}

size_t hm_linear_k_split_workspace_bytes(const hm_weights *w0, const hm_weights *w1, int64_t M, int64_t k0, int64_t k1, int64_t n) {
    if (w0 == nullptr || w1 == nullptr || M <= 0 || k0 <= 0 || k1 <= 0 || n <= 0) {
        return 0;
    }
    // The two launches run one after the other on one stream and share the workspace; at one row the pair may
    // run as one launch with a partial sum per share.
    const size_t pair = M == 1 ? 2 * static_cast<size_t>(n) * sizeof(float) : 0;
    return std::max({linear_workspace(w0->p, M, n, k0 / 128, false), linear_workspace(w1->p, M, n, k1 / 128, false), pair});
}

hm_status hm_linear_k_split(const hm_weights *w0, const hm_weights *w1, void *y, int64_t ldy, const void *x, int64_t ldx, int64_t M,
                            int64_t k0, int64_t k1, int64_t n, void *workspace, size_t workspace_bytes, void *stream) {
    if (w0 == nullptr || w1 == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_linear_k_split: null weights");
    }
    if (w0->p.dtype != w1->p.dtype) {
        return fail(HM_INVALID_ARGUMENT, "hm_linear_k_split: the two shares have different activation types");
    }
    if (M <= 0 || k0 <= 0 || k1 <= 0 || n <= 0 || k0 % 128 || k1 % 128 || n % 16 || k0 > w0->p.K || k1 > w1->p.K || n > w0->p.N ||
        n > w1->p.N) {
        return fail(HM_INVALID_ARGUMENT,
                    "hm_linear_k_split: k0=%lld, k1=%lld (multiples of 128) and n=%lld (multiple of 16) must fit [%lld, %lld] and [%lld, %lld]",
                    static_cast<long long>(k0), static_cast<long long>(k1), static_cast<long long>(n), static_cast<long long>(w0->p.K),
                    static_cast<long long>(w0->p.N), static_cast<long long>(w1->p.K), static_cast<long long>(w1->p.N));
    }
    hm_status st = check_activation(x, ldx, k0 + k1, "hm_linear_k_split x");
    if (st != HM_OK || (st = check_output(y, ldy, n, "hm_linear_k_split y")) != HM_OK) {
        return st;
    }
    const hipStream_t s = as_stream(stream);
    // One row: both shares in one GEMV launch (split s runs share s), their rounded sums added by the split sum.
    if (M == 1) {
        hm::GemvCall c0, c1;
        c0.w = w0->p;
        c1.w = w1->p;
        c0.x = static_cast<const uint16_t *>(x);
        c1.x = c0.x + k0;
        c0.ldx = c1.ldx = ldx;
        c0.y = c1.y = static_cast<uint16_t *>(y);
        c0.ldy = c1.ldy = ldy;
        c0.n = c1.n = n;
        c0.kt_count = k0 / 128;
        c1.kt_count = k1 / 128;
        if (hm::gemv_pair_supported(c0, c1)) {
            const size_t need = hm::gemv_pair_partial_bytes(c0);
            if (need > workspace_bytes) {
                return fail(HM_WORKSPACE_TOO_SMALL, "workspace of %zu bytes, need %zu", workspace_bytes, need);
            }
            c0.partial = static_cast<float *>(workspace);
            const hipError_t e = hm::launch_gemv_pair(c0, c1, k0, s);
            return e == hipSuccess ? HM_OK : hip_fail(e, "gemv pair launch");
        }
    }
    // Share 0 writes y = round(x[:, :k0] W0); share 1 adds in its epilogue: y = round(y + round(x[:, k0:] W1)).
    if ((st = run_linear(w0->p, y, ldy, x, ldx, M, 0, n, 0, k0 / 128, false, workspace, workspace_bytes, s)) != HM_OK) {
        return st;
    }
    const uint16_t *x1 = static_cast<const uint16_t *>(x) + k0;
    return run_linear(w1->p, y, ldy, x1, ldx, M, 0, n, 0, k1 / 128, false, workspace, workspace_bytes, s, true);
}

hm_status hm_ffn_from_tiles(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int64_t hidden, int64_t inter, hm_dtype dtype,
                            void *stream, hm_ffn **out) {
    return hm_ffn_from_tiles_padded(gate, up, down, hidden, inter, hidden, inter, dtype, stream, out);
}

hm_status hm_ffn_from_tiles_padded(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int64_t hidden, int64_t inter,
                                   int64_t packed_hidden, int64_t packed_inter, hm_dtype dtype, void *stream, hm_ffn **out) {
    if (out == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_ffn_from_tiles: null output handle");
    }
    *out = nullptr;
    hm_status st = check_dtype(dtype);
    if (st != HM_OK || (st = check_ffn_shape(hidden, inter, "hm_ffn_from_tiles")) != HM_OK) {
        return st;
    }
    if ((st = check_tile_source(gate, packed_hidden, packed_inter, hidden, inter, "gate")) != HM_OK ||
        (st = check_tile_source(up, packed_hidden, packed_inter, hidden, inter, "up")) != HM_OK ||
        (st = check_tile_source(down, packed_inter, packed_hidden, inter, hidden, "down")) != HM_OK) {
        return st;
    }
    hm::TileSource gu[2];
    gu[0].tiles = gate;
    gu[1].tiles = up;
    gu[0].tiles_k = gu[1].tiles_k = packed_hidden / 128;
    gu[0].tiles_n = gu[1].tiles_n = packed_inter / 64;
    return build_ffn_from_tiles(gu, down, packed_inter, packed_hidden, hidden, inter, dtype, as_stream(stream), "hm_ffn_from_tiles", out);
}

hm_status hm_ffn_from_gate_up_tiles(const uint8_t *gate_up, const uint8_t *down, int64_t hidden, int64_t inter, int64_t stored, int32_t layout,
                                    hm_dtype dtype, void *stream, hm_ffn **out) {
    if (out == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_ffn_from_gate_up_tiles: null output handle");
    }
    *out = nullptr;
    hm_status st = check_dtype(dtype);
    if (st != HM_OK || (st = check_ffn_shape(hidden, inter, "hm_ffn_from_gate_up_tiles")) != HM_OK ||
        (st = check_gate_up_source(gate_up, hidden, stored, hidden, inter, layout, "gate_up")) != HM_OK ||
        (st = check_tile_source(down, stored, hidden, inter, hidden, "down")) != HM_OK) {
        return st;
    }
    hm::TileSource gu[2];
    gate_up_sources(gate_up, hidden, stored, layout, gu);
    return build_ffn_from_tiles(gu, down, stored, hidden, hidden, inter, dtype, as_stream(stream), "hm_ffn_from_gate_up_tiles", out);
}

hm_status hm_ffn_from_logical(const uint8_t *gate_q, const uint16_t *gate_s, const uint8_t *gate_z, const uint8_t *up_q, const uint16_t *up_s,
                              const uint8_t *up_z, const uint8_t *down_q, const uint16_t *down_s, const uint8_t *down_z, int64_t hidden,
                              int64_t inter, int64_t group, hm_dtype dtype, void *stream, hm_ffn **out) {
    if (out == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_ffn_from_logical: null output handle");
    }
    *out = nullptr;
    hm_status st = check_dtype(dtype);
    if (st != HM_OK || (st = check_logical(gate_q, gate_s, gate_z, hidden, inter, group, "gate")) != HM_OK ||
        (st = check_logical(up_q, up_s, up_z, hidden, inter, group, "up")) != HM_OK ||
        (st = check_logical(down_q, down_s, down_z, inter, hidden, group, "down")) != HM_OK) {
        return st;
    }
    hm_ffn *f = nullptr;
    if ((st = new_ffn(hidden, inter, group, dtype, &f)) != HM_OK) {
        return st;
    }
    hm::LogicalSource gu[2];
    gu[0].q = gate_q;
    gu[0].scales = gate_s;
    gu[0].zeros = gate_z;
    gu[1].q = up_q;
    gu[1].scales = up_s;
    gu[1].zeros = up_z;
    gu[0].ld = gu[1].ld = inter;
    hm::LogicalSource d;
    d.q = down_q;
    d.scales = down_s;
    d.zeros = down_z;
    d.ld = hidden;
    const hipStream_t s = as_stream(stream);
    return fill_ffn(f, s, "hm_ffn_from_logical", out, [&](uint32_t *flag) {
        hipError_t e = hm::launch_repack_logical(gu, 2, true, const_cast<uint8_t *>(f->gate_up.p.quant),
                                                 const_cast<uint32_t *>(f->gate_up.p.meta), hidden, 2 * inter, group, flag, s);
        if (e == hipSuccess) {
            e = hm::launch_repack_logical(&d, 1, false, const_cast<uint8_t *>(f->down.p.quant), const_cast<uint32_t *>(f->down.p.meta), inter,
                                          hidden, group, flag, s);
        }
        return e;
    });
}

hm_status hm_ffn_info(const hm_ffn *f, int64_t *hidden, int64_t *inter, int64_t *group, int32_t *dtype) {
    if (f == nullptr) {
        return fail(HM_INVALID_ARGUMENT, "hm_ffn_info: null handle");
    }
    if (hidden) *hidden = f->hidden;
    if (inter) *inter = f->inter;
    if (group) *group = f->down.p.group;
    if (dtype) *dtype = f->down.p.dtype;
    return HM_OK;
}

hm_status hm_ffn_destroy(hm_ffn *f) {
    if (f != nullptr) {
        destroy_ffn(f);
    }
    return HM_OK;
}

size_t hm_ffn_workspace_bytes(const hm_ffn *f, int64_t max_m) {
    if (f == nullptr || max_m <= 0) {
        return 0;
    }
    // The one-row layout (act, the strip-pair spill, partials) fits in the same bytes as every wider one.
    const size_t act = static_cast<size_t>(round_up(max_m * f->inter * 2, 256)) + one_row_spill_bytes(f->inter);
    // The largest partial buffer of any M up to max_m and any channel range: the GEMV's (M <= 16, planned when the
    // layer was made) and, above, the GEMM's small-grid K split, which never needs more than kGemmPartialMax.
    if (max_m <= kGemvMaxRows) {
        return act + f->decode_partial[max_m];
    }
    return act + std::max(hm::kGemmPartialMax, f->decode_partial[kGemvMaxRows]);
}

namespace {

// One row through the two GEMVs: act = SwiGLU(x W_gate_up) over channels [ch_begin, ch_end) (of RMSNorm(x) *
// norm_w when norm_w is given; hidden <= 8192), then y = act W_down (accumulate: y += it, rounded). Workspace:
// act, the strip-pair spill, then split partials. With the spill the gate_up GEMV may deal its strip pairs' K
// halves evenly over the CUs; the down GEMV then forms the act columns of the pairs two workgroups share.
hm_status one_row_ffn(const hm_ffn *f, void *y, int64_t ldy, const void *x, int64_t ldx, int64_t ch_begin, int64_t ch_end,
                      const void *norm_w, float eps, bool accumulate, void *workspace, size_t workspace_bytes, hipStream_t s) {
    const int64_t n = ch_end - ch_begin;
    const size_t act_bytes = static_cast<size_t>(round_up(n * 2, 256));
    const size_t spill_bytes = one_row_spill_bytes(n);
    if (workspace_bytes < act_bytes + spill_bytes) {
        return fail(HM_WORKSPACE_TOO_SMALL, "one-row FFN: workspace of %zu bytes, need %zu before partials", workspace_bytes,
                    act_bytes + spill_bytes);
    }
    uint16_t *act = static_cast<uint16_t *>(workspace);
    float *spill = reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) + act_bytes);
    void *rest = static_cast<uint8_t *>(workspace) + act_bytes + spill_bytes;
    const size_t rest_bytes = workspace_bytes - act_bytes - spill_bytes;
    hm::GemvCall c;
    c.w = f->gate_up.p;
    c.x = static_cast<const uint16_t *>(x);
    c.ldx = ldx;
    c.y = act;
    c.ldy = n;
    c.m = 1;
    c.strip_begin = 2 * (ch_begin / 16);
    c.n = n;
    c.kt_count = f->hidden / 128;
    c.fused = true;
    c.norm_w = static_cast<const uint16_t *>(norm_w);
    c.norm_eps = eps;
    c.pair_spill = spill;
    c.partial = static_cast<float *>(rest);
    hm::GemvPlan gp = hm::plan_gemv(c);
    hm::GemvCall d;
    d.w = f->down.p;
    d.x = act;
    d.ldx = n;
    d.y = static_cast<uint16_t *>(y);
    d.ldy = ldy;
    d.m = 1;
    d.n = f->hidden;
    d.kt_begin = ch_begin / 128;
    d.kt_count = n / 128;
    d.accumulate = accumulate;
    d.partial = c.partial;
    if (gp.units % 2 == 1) {
        d.pair_spill = spill;
        d.pair_units = gp.units;
        // The down GEMV forms the split pairs in every strip group of a workgroup; with more than one, or more LDS
        // than a workgroup has, the gate_up keeps whole pairs per workgroup (Qwen2.5-14B, two down strip groups
        // per workgroup: 26.9 us a layer against 26.0).
        const hm::GemvPlan dp = hm::plan_gemv(d);
        if (dp.nu > 1 || dp.lds > hm::kGemvLdsMax) {
            c.pair_spill = nullptr;
            gp = hm::plan_gemv(c);
            d.pair_spill = nullptr;
            d.pair_units = 0;
        }
    }
    const size_t need = std::max(gp.partial_bytes, hm::plan_gemv(d).partial_bytes);
    if (need > rest_bytes) {
        return fail(HM_WORKSPACE_TOO_SMALL, "one-row FFN: %zu bytes for partials, need %zu", rest_bytes, need);
    }
    hipError_t e = hm::launch_gemv(c, s);
    if (e != hipSuccess) {
        return hip_fail(e, "one-row gate_up launch");
    }
    e = hm::launch_gemv(d, s);
    return e == hipSuccess ? HM_OK : hip_fail(e, "one-row down launch");
}

} // namespace

hm_status hm_ffn_gate_up(const hm_ffn *f, void *act, int64_t ld_act, const void *x, int64_t ldx, int64_t M, int64_t ch_begin, int64_t ch_end,
                         void *workspace, size_t workspace_bytes, void *stream) {
    if (f == nullptr || M <= 0) {
        return fail(HM_INVALID_ARGUMENT, "hm_ffn_gate_up: null handle or M <= 0");
    }
    hm_status st = check_channels(f, ch_begin, ch_end);
    if (st != HM_OK || (st = check_activation(x, ldx, f->hidden, "hm_ffn_gate_up x")) != HM_OK ||
        (st = check_output(act, ld_act, ch_end - ch_begin, "hm_ffn_gate_up act")) != HM_OK) {
        return st;
    }
    return run_linear(f->gate_up.p, act, ld_act, x, ldx, M, 2 * (ch_begin / 16), ch_end - ch_begin, 0, f->hidden / 128, true, workspace,
                      workspace_bytes, as_stream(stream));
}

hm_status hm_ffn_down(const hm_ffn *f, void *y, int64_t ldy, const void *act, int64_t ld_act, int64_t M, int64_t ch_begin, int64_t ch_end,
                      void *workspace, size_t workspace_bytes, void *stream) {
    if (f == nullptr || M <= 0) {
        return fail(HM_INVALID_ARGUMENT, "hm_ffn_down: null handle or M <= 0");
    }
    hm_status st = check_channels(f, ch_begin, ch_end);
    if (st != HM_OK || (st = check_activation(act, ld_act, ch_end - ch_begin, "hm_ffn_down act")) != HM_OK ||
        (st = check_output(y, ldy, f->hidden, "hm_ffn_down y")) != HM_OK) {
        return st;
    }
    return run_linear(f->down.p, y, ldy, act, ld_act, M, 0, f->hidden, ch_begin / 128, (ch_end - ch_begin) / 128, false, workspace,
                      workspace_bytes, as_stream(stream));
}

hm_status hm_ffn_forward(const hm_ffn *f, void *y, int64_t ldy, const void *x, int64_t ldx, int64_t M, int64_t ch_begin, int64_t ch_end,
                         void *workspace, size_t workspace_bytes, void *stream) {
    if (f == nullptr || M <= 0) {
        return fail(HM_INVALID_ARGUMENT, "hm_ffn_forward: null handle or M <= 0");
    }
    hm_status st = check_channels(f, ch_begin, ch_end);
    if (st != HM_OK) {
        return st;
    }
    const size_t need = hm_ffn_workspace_bytes(f, M);
    if (workspace == nullptr || workspace_bytes < need || !aligned(workspace, 256)) {
        return fail(HM_WORKSPACE_TOO_SMALL, "hm_ffn_forward: workspace must be 256-byte aligned with >= %zu bytes (got %zu)", need,
                    workspace_bytes);
    }
    if (M == 1) {
        if ((st = check_activation(x, ldx, f->hidden, "hm_ffn_forward x")) != HM_OK ||
            (st = check_output(y, ldy, f->hidden, "hm_ffn_forward y")) != HM_OK) {
            return st;
        }
        return one_row_ffn(f, y, ldy, x, ldx, ch_begin, ch_end, nullptr, 0.0f, false, workspace, workspace_bytes, as_stream(stream));
    }
    const int64_t n = ch_end - ch_begin;
    const size_t act_bytes = static_cast<size_t>(round_up(M * f->inter * 2, 256));
    void *act = workspace;
    void *rest = static_cast<uint8_t *>(workspace) + act_bytes;
    const size_t rest_bytes = workspace_bytes - act_bytes;
    if ((st = hm_ffn_gate_up(f, act, n, x, ldx, M, ch_begin, ch_end, rest, rest_bytes, stream)) != HM_OK) {
        return st;
    }
    return hm_ffn_down(f, y, ldy, act, n, M, ch_begin, ch_end, rest, rest_bytes, stream);
}

size_t hm_ffn_block_workspace_bytes(const hm_ffn *f, int64_t max_m) {
    if (f == nullptr || max_m <= 0) {
        return 0;
    }
    // normed and y rows for the separate-kernel path, then the FFN's own workspace.
    return 2 * static_cast<size_t>(round_up(max_m * f->hidden * 2, 256)) + hm_ffn_workspace_bytes(f, max_m);
}

hm_status hm_ffn_block_forward(const hm_ffn *f, void *x, int64_t ldx, const void *norm_weight, float eps, int64_t M, void *workspace,
                               size_t workspace_bytes, void *stream) {
    if (f == nullptr || M <= 0) {
        return fail(HM_INVALID_ARGUMENT, "hm_ffn_block_forward: null handle or M <= 0");
    }
    hm_status st = check_activation(x, ldx, f->hidden, "hm_ffn_block_forward x");
    if (st != HM_OK) {
        return st;
    }
    if (norm_weight == nullptr || !aligned(norm_weight, 16) || !(eps >= 0.0f)) {
        return fail(HM_INVALID_ARGUMENT, "hm_ffn_block_forward: norm_weight must be 16-byte aligned and eps >= 0");
    }
    const size_t need = hm_ffn_block_workspace_bytes(f, M);
    if (workspace == nullptr || workspace_bytes < need || !aligned(workspace, 256)) {
        return fail(HM_WORKSPACE_TOO_SMALL, "hm_ffn_block_forward: workspace must be 256-byte aligned with >= %zu bytes (got %zu)", need,
                    workspace_bytes);
    }
    const size_t rows_bytes = static_cast<size_t>(round_up(M * f->hidden * 2, 256));
    uint16_t *normed = static_cast<uint16_t *>(workspace);
    uint16_t *y = reinterpret_cast<uint16_t *>(static_cast<uint8_t *>(workspace) + rows_bytes);
    void *ffn_ws = static_cast<uint8_t *>(workspace) + 2 * rows_bytes;
    const size_t ffn_bytes = workspace_bytes - 2 * rows_bytes;
    const hipStream_t s = as_stream(stream);
    const hm_dtype dtype = static_cast<hm_dtype>(f->gate_up.p.dtype);
    if (M == 1 && f->hidden <= 8192) {
        // Two launches: the gate_up GEMV stages RMSNorm(x) * weight, the down GEMV adds its output into x.
        return one_row_ffn(f, x, ldx, x, ldx, 0, f->inter, norm_weight, eps, true, ffn_ws, ffn_bytes, s);
    }
    // Several rows: RMSNorm, the gate_up projection, then the down projection adding its rounded output into x
    // (x = round(x + round(act W)), in its epilogue or in the split sum: the bits of hm_ffn_forward followed by
    // hm_residual_add2, one launch fewer).
    (void)y;
    const size_t act_bytes = static_cast<size_t>(round_up(M * f->inter * 2, 256));
    void *act = ffn_ws;
    void *rest = static_cast<uint8_t *>(ffn_ws) + act_bytes;
    const size_t rest_bytes = ffn_bytes - act_bytes;
    if ((st = hm_rmsnorm(normed, f->hidden, x, ldx, norm_weight, M, f->hidden, eps, dtype, stream)) != HM_OK ||
        (st = hm_ffn_gate_up(f, act, f->inter, normed, f->hidden, M, 0, f->inter, rest, rest_bytes, stream)) != HM_OK) {
        return st;
    }
    return run_linear(f->down.p, x, ldx, act, f->inter, M, 0, f->hidden, 0, f->inter / 128, false, rest, rest_bytes, s, true);
}

hm_status hm_silu_mul(const void *gate_up, int64_t ld_in, void *act, int64_t ld_out, int64_t rows, int64_t n, int32_t layout, hm_dtype dtype,
                      void *stream) {
    hm_status st = check_dtype(dtype);
    if (st != HM_OK) {
        return st;
    }
    const bool inter = layout == HM_GATE_UP_INTERLEAVED;
    if (gate_up == nullptr || act == nullptr || rows < 0 || n <= 0 || n % (inter ? 64 : 8) || ld_in % 8 || ld_out % 8 || ld_in < 2 * n ||
        ld_out < n || !aligned(gate_up, 16) || !aligned(act, 16) || (layout != HM_GATE_UP_BLOCKED && !inter)) {
        return fail(HM_INVALID_ARGUMENT, "hm_silu_mul: gate_up [rows, 2n] and act [rows, n] must be 16-byte aligned, n a multiple of %d",
                    inter ? 64 : 8);
    }
    const hipError_t e = hm::launch_silu_mul(static_cast<const uint16_t *>(gate_up), ld_in, static_cast<uint16_t *>(act), ld_out, rows, n,
                                             inter, dtype, as_stream(stream));
    return e == hipSuccess ? HM_OK : hip_fail(e, "silu_mul launch");
}

hm_status hm_rmsnorm(void *out, int64_t ld_out, const void *x, int64_t ldx, const void *weight, int64_t rows, int64_t cols, float eps, hm_dtype dtype,
                     void *stream) {
    hm_status st = check_dtype(dtype);
    if (st != HM_OK) {
        return st;
    }
    if (out == nullptr || x == nullptr || weight == nullptr || rows < 0 || cols <= 0 || cols % 8 || ld_out % 8 || ldx % 8 || ldx < cols ||
        ld_out < cols || !aligned(out, 16) || !aligned(x, 16) || !aligned(weight, 16) || !(eps >= 0.0f)) {
        return fail(HM_INVALID_ARGUMENT, "hm_rmsnorm: rows of a multiple of 8 columns, 16-byte aligned, eps >= 0");
    }
    const hipError_t e = hm::launch_rmsnorm(static_cast<uint16_t *>(out), ld_out, static_cast<const uint16_t *>(x), ldx,
                                            static_cast<const uint16_t *>(weight), rows, cols, eps, dtype, as_stream(stream));
    return e == hipSuccess ? HM_OK : hip_fail(e, "rmsnorm launch");
}

hm_status hm_residual_add2(void *x, int64_t ldx, const void *a, int64_t lda, const void *b, int64_t ldb, int64_t rows, int64_t cols,
                           hm_dtype dtype, void *stream) {
    hm_status st = check_dtype(dtype);
    if (st != HM_OK) {
        return st;
    }
    if (x == nullptr || rows < 0 || cols <= 0 || cols % 8 || ldx % 8 || ldx < cols || !aligned(x, 16) ||
        (a != nullptr && (lda % 8 || lda < cols || !aligned(a, 16))) || (b != nullptr && (ldb % 8 || ldb < cols || !aligned(b, 16)))) {
        return fail(HM_INVALID_ARGUMENT, "hm_residual_add2: rows of a multiple of 8 columns, 16-byte aligned");
    }
    const hipError_t e = hm::launch_residual_add2(static_cast<uint16_t *>(x), ldx, static_cast<const uint16_t *>(a), lda,
                                                  static_cast<const uint16_t *>(b), ldb, rows, cols, dtype, as_stream(stream));
    return e == hipSuccess ? HM_OK : hip_fail(e, "residual_add2 launch");
}

hm_status hm_residual_rmsnorm(void *x, int64_t ldx, const void *y, int64_t ldy, const void *weight, void *normed, int64_t ld_normed, int64_t rows,
                              int64_t cols, float eps, hm_dtype dtype, void *stream) {
    hm_status st = check_dtype(dtype);
    if (st != HM_OK) {
        return st;
    }
    if (x == nullptr || y == nullptr || weight == nullptr || normed == nullptr || rows < 0 || cols <= 0 || cols % 8 || ldx % 8 || ldy % 8 ||
        ld_normed % 8 || ldx < cols || ldy < cols || ld_normed < cols || !aligned(x, 16) || !aligned(y, 16) || !aligned(weight, 16) ||
        !aligned(normed, 16) || !(eps >= 0.0f)) {
        return fail(HM_INVALID_ARGUMENT, "hm_residual_rmsnorm: rows of a multiple of 8 columns, 16-byte aligned, eps >= 0");
    }
    const hipError_t e = hm::launch_residual_rmsnorm(static_cast<uint16_t *>(x), ldx, static_cast<const uint16_t *>(y), ldy, nullptr, 0,
                                                     static_cast<const uint16_t *>(weight), static_cast<uint16_t *>(normed), ld_normed, rows,
                                                     cols, eps, dtype, as_stream(stream));
    return e == hipSuccess ? HM_OK : hip_fail(e, "residual_rmsnorm launch");
}

hm_status hm_residual2_rmsnorm(void *x, int64_t ldx, const void *a, int64_t lda, const void *b, int64_t ldb, const void *weight, void *normed,
                               int64_t ld_normed, int64_t rows, int64_t cols, float eps, hm_dtype dtype, void *stream) {
    hm_status st = check_dtype(dtype);
    if (st != HM_OK) {
        return st;
    }
    if (x == nullptr || weight == nullptr || normed == nullptr || rows < 0 || cols <= 0 || cols % 8 || ldx % 8 || ld_normed % 8 ||
        ldx < cols || ld_normed < cols || !aligned(x, 16) || !aligned(weight, 16) || !aligned(normed, 16) || !(eps >= 0.0f) ||
        (a != nullptr && (lda % 8 || lda < cols || !aligned(a, 16))) || (a != nullptr && b != nullptr && (ldb % 8 || ldb < cols || !aligned(b, 16)))) {
        return fail(HM_INVALID_ARGUMENT, "hm_residual2_rmsnorm: rows of a multiple of 8 columns, 16-byte aligned, eps >= 0");
    }
    const hipStream_t s = as_stream(stream);
    // Without a, x stays as it is (b is not read) and the call is the plain RMSNorm.
    const hipError_t e =
        a == nullptr ? hm::launch_rmsnorm(static_cast<uint16_t *>(normed), ld_normed, static_cast<const uint16_t *>(x), ldx,
                                          static_cast<const uint16_t *>(weight), rows, cols, eps, dtype, s)
                     : hm::launch_residual_rmsnorm(static_cast<uint16_t *>(x), ldx, static_cast<const uint16_t *>(a), lda,
                                                   static_cast<const uint16_t *>(b), ldb, static_cast<const uint16_t *>(weight),
                                                   static_cast<uint16_t *>(normed), ld_normed, rows, cols, eps, dtype, s);
    return e == hipSuccess ? HM_OK : hip_fail(e, "residual2_rmsnorm launch");
}

hm_status hm_residual_add2_mixed(void *x, int64_t ldx, const void *a, int64_t lda, int32_t a_fp32, const void *b, int64_t ldb, int32_t b_fp32,
                                 int64_t rows, int64_t cols, hm_dtype dtype, void *stream) {
    hm_status st = check_dtype(dtype);
    if (st != HM_OK) {
        return st;
    }
    if (x == nullptr || a == nullptr || b == nullptr || rows < 0 || cols <= 0 || cols % 8 || ldx % 8 || lda % 8 || ldb % 8 || ldx < cols ||
        lda < cols || ldb < cols || !aligned(x, 16) || !aligned(a, 16) || !aligned(b, 16)) {
        return fail(HM_INVALID_ARGUMENT, "hm_residual_add2_mixed: x, a and b rows of a multiple of 8 columns, 16-byte aligned");
    }
    const hipError_t e = hm::launch_residual_add2_mixed(static_cast<uint16_t *>(x), ldx, a, lda, a_fp32 != 0, b, ldb, b_fp32 != 0, rows, cols,
                                                        dtype, as_stream(stream));
    return e == hipSuccess ? HM_OK : hip_fail(e, "residual_add2_mixed launch");
}

int64_t hm_find_nonfinite(const void *bits, int64_t rows, int64_t cols, int64_t ld, hm_dtype dtype, int32_t sampled) {
    if (bits == nullptr || rows <= 0 || cols <= 0 || ld < cols || check_dtype(dtype) != HM_OK) {
        return -1;
    }
    const uint16_t mask = dtype == HM_FP16 ? 0x7C00u : 0x7F80u;
    const int64_t stride = sampled ? HM_FINITE_SAMPLE_STRIDE : 1;
    const uint16_t *p = static_cast<const uint16_t *>(bits);
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < cols; c += stride) {
            if ((p[r * ld + c] & mask) == mask) {
                return r * cols + c;
            }
        }
    }
    return -1;
}

hm_status hm_find_nonfinite_device(const void *x, int64_t rows, int64_t cols, int64_t ld, hm_dtype dtype, int32_t sampled, int64_t *first,
                                   void *stream) {
    hm_status st = check_dtype(dtype);
    if (st != HM_OK) {
        return st;
    }
    if (x == nullptr || first == nullptr || rows < 0 || cols <= 0 || ld < cols || !aligned(first, 8)) {
        return fail(HM_INVALID_ARGUMENT, "hm_find_nonfinite_device: x [rows, cols] with ld >= cols and an 8-byte aligned device int64");
    }
    const hipError_t e = hm::launch_find_nonfinite(static_cast<const uint16_t *>(x), ld, rows, cols, sampled ? HM_FINITE_SAMPLE_STRIDE : 1,
                                                   dtype, first, as_stream(stream));
    return e == hipSuccess ? HM_OK : hip_fail(e, "find_nonfinite launch");
}

hm_status hm_partition_check(int64_t intermediate, int64_t npu_channels, int64_t alignment) {
    if (intermediate <= 0 || alignment <= 0) {
        return fail(HM_INVALID_ARGUMENT, "partition: intermediate_channels and alignment must be positive integers");
    }
    if (npu_channels < 0 || npu_channels > intermediate) {
        return fail(HM_INVALID_ARGUMENT, "partition: npu_channels must lie within the FFN width");
    }
    if (intermediate % alignment || npu_channels % alignment) {
        return fail(HM_INVALID_ARGUMENT, "partition: FFN width and NPU channel count must satisfy alignment");
    }
    return HM_OK;
}

hm_status hm_partition_from_ratio(int64_t intermediate, double npu_ratio, int64_t alignment, int64_t *npu_channels) {
    if (npu_channels == nullptr || intermediate <= 0 || alignment <= 0) {
        return fail(HM_INVALID_ARGUMENT, "partition: intermediate_channels and alignment must be positive integers");
    }
    if (!std::isfinite(npu_ratio) || npu_ratio < 0.0 || npu_ratio > 1.0) {
        return fail(HM_INVALID_ARGUMENT, "partition: npu_ratio must be finite and in [0, 1]");
    }
    const double units = static_cast<double>(intermediate) * npu_ratio / static_cast<double>(alignment);
    *npu_channels = static_cast<int64_t>(std::floor(units + 0.5)) * alignment;
    return hm_partition_check(intermediate, *npu_channels, alignment);
}

} // extern "C"

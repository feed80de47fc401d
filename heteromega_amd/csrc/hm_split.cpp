// Split descriptors of the reference's hetero executor, planned on the host and executed with every share on the
// GPU (declarations: include/hm_w4a16.h). The reference keys its kernel configs by {forM, forK, forN, layer_id,
// chunk_id} and derives a split type from the shapes when it loads them (src/unified_llm_w4a16_hetero/
// npuSetup.cpp:1283-1291); its executor then splits a projection by rows, columns or K between the GPU and the
// other devices (hetero_compute.cpp:189-259, 282-447, 497-560, 633-805). Here the same table drives the same
// partition, each share one launch of this engine on the caller's stream.
#include "../../include/hm_w4a16.h"
#include "hm_internal.hpp"

#include <algorithm>
#include <array>
#include <cstdint>
#include <cstring>
#include <exception>
#include <limits>
#include <map>
#include <mutex>
#include <new>

struct hm_split_table {
    std::map<std::array<int32_t, 5>, hm_split_desc> entries;
    mutable std::mutex mu;
};

namespace {

hm_split_desc make_desc(int32_t npuM, int32_t npuK, int32_t npuN, int32_t cpuN, int32_t cpuThreads, int32_t config, int32_t split_type) {
    hm_split_desc d;
    d.hw_idx = -1;
    d.inst_idx = -1;
    d.npuM = npuM;
    d.npuK = npuK;
    d.npuN = npuN;
    d.cpuN = cpuN;
    d.cpuThreads = cpuThreads;
    d.config = config;
    d.split_type = split_type;
    return d;
}

// The column shares of a GEMV entry as the reference resolves them (hetero_compute.cpp:503-532): both dropped when
// they exceed N, cpuN dropped unless a multiple of 64 (its AVX tiles).
void gemv_shares(const hm_split_desc &d, int64_t N, int64_t &npuN, int64_t &cpuN) {
    npuN = std::max<int64_t>(d.npuN, 0);
    cpuN = std::max<int64_t>(d.cpuN, 0);
    if (npuN + cpuN > N) {
        npuN = 0;
        cpuN = 0;
    }
    if (cpuN % 64 != 0) {
        cpuN = 0;
    }
}

// Pieces of one split: (row begin, rows, column begin, columns).
struct Piece {
    int64_t r0, rows, c0, cols;
};

int plan_pieces(const hm_split_desc *d, int64_t M, int64_t N, Piece out[3]) {
    if (d == nullptr) {
        out[0] = Piece{0, M, 0, N};
        return 1;
    }
    int n = 0;
    auto add = [&](int64_t r0, int64_t rows, int64_t c0, int64_t cols) {
        if (rows > 0 && cols > 0) {
            out[n++] = Piece{r0, rows, c0, cols};
        }
    };
    if (M == 1 && d->split_type <= 0) {
        // GEMV: the GPU's columns first (the reference launches them before the other devices' shares), then the
        // NPU's [0, npuN) and the CPU's [npuN, npuN + cpuN), here on the GPU too.
        int64_t npuN = 0, cpuN = 0;
        gemv_shares(*d, N, npuN, cpuN);
        add(0, 1, npuN + cpuN, N - npuN - cpuN);
        add(0, 1, 0, npuN);
        add(0, 1, npuN, cpuN);
        return n;
    }
    if (d->split_type == -1) {
        const int64_t npu_m = std::min<int64_t>(std::max<int64_t>(d->npuM, 0), M);
        add(0, M - npu_m, 0, N); // the GPU takes [0, M - npuM) (hetero_compute.cpp:205-213)
        add(M - npu_m, npu_m, 0, N);
        return n;
    }
    if (d->split_type == -2) {
        const int64_t npu_n = std::min<int64_t>(std::max<int64_t>(d->npuN, 0), N);
        add(0, M, npu_n, N - npu_n);
        add(0, M, 0, npu_n);
        return n;
    }
    out[0] = Piece{0, M, 0, N};
    return 1;
}

} // namespace

extern "C" {

int32_t hm_split_type(int32_t forM, int32_t forK, int32_t forN, int32_t npuM, int32_t npuK, int32_t npuN) {
    if (forK != npuK) {
        return npuK; // K split, taking precedence
    }
    if (forM != npuM && forN == npuN) {
        return -1; // M split
    }
    if (forN != npuN) {
        return -2; // N split
    }
    return -1; // the loader's default
}

int32_t hm_layer_id(const char *layer_type) {
    if (layer_type == nullptr) {
        return 0;
    }
    static const struct {
        const char *name;
        int32_t id;
    } ids[] = {{"qkv", 8}, {"q", 1}, {"k", 2}, {"v", 3}, {"o", 4}, {"gate", 5}, {"up", 6}, {"down", 7}};
    for (const auto &e : ids) {
        if (std::strcmp(layer_type, e.name) == 0) {
            return e.id;
        }
    }
    return 0;
}

namespace {

// Inserts or replaces an entry; false when the host allocation fails (no exception leaves the C ABI).
bool store(hm_split_table *t, const std::array<int32_t, 5> &key, const hm_split_desc &d) {
    try {
        std::lock_guard<std::mutex> lock(t->mu);
        t->entries[key] = d;
        return true;
    } catch (const std::exception &) {
        return false;
    }
}

} // namespace

hm_status hm_split_table_create(hm_split_table **out) {
    if (out == nullptr) {
        return hm::set_error(HM_INVALID_ARGUMENT, "hm_split_table_create: null output handle");
    }
    *out = new (std::nothrow) hm_split_table;
    return *out != nullptr ? HM_OK : hm::set_error(HM_OUT_OF_MEMORY, "hm_split_table_create: host allocation failed");
}

hm_status hm_split_table_destroy(hm_split_table *t) {
    delete t;
    return HM_OK;
}

hm_status hm_split_table_add_gemm(hm_split_table *t, int32_t forM, int32_t forK, int32_t forN, int32_t layer_id, int32_t chunk_id,
                                  int32_t npuM, int32_t npuK, int32_t npuN, int32_t config, int32_t *stored) {
    if (stored != nullptr) {
        *stored = 0;
    }
    if (t == nullptr) {
        return hm::set_error(HM_INVALID_ARGUMENT, "hm_split_table_add_gemm: null table");
    }
    if (forM <= 0 || forK <= 0 || forN <= 0 || npuM < 0 || npuK <= 0 || npuN <= 0) {
        return hm::set_error(HM_INVALID_ARGUMENT, "hm_split_table_add_gemm: sizes must be positive (forM %d forK %d forN %d, npuM %d npuK %d npuN %d)",
                             forM, forK, forN, npuM, npuK, npuN);
    }
    if (npuK > forK) {
        return hm::set_error(HM_INVALID_ARGUMENT, "hm_split_table_add_gemm: npuK %d exceeds forK %d", npuK, forK);
    }
    const int32_t split = hm_split_type(forM, forK, forN, npuM, npuK, npuN);
    if (split > 0 && (split % 128 != 0 || (forK - split) % 128 != 0)) {
        return hm::set_error(HM_INVALID_ARGUMENT, "hm_split_table_add_gemm: K split %d + %d must be multiples of 128", split, forK - split);
    }
    if (npuM == 0) {
        return HM_OK; // GPU-only in the reference: the loader skips it (npuSetup.cpp:1312-1319)
    }
    if (!store(t, {forM, forK, forN, layer_id, chunk_id}, make_desc(npuM, npuK, npuN, 0, 1, config, split))) {
        return hm::set_error(HM_OUT_OF_MEMORY, "hm_split_table_add_gemm: host allocation failed");
    }
    if (stored != nullptr) {
        *stored = 1;
    }
    return HM_OK;
}

hm_status hm_split_table_add_gemv(hm_split_table *t, int32_t forK, int32_t forN, int32_t layer_id, int32_t chunk_id, int32_t npuN, int32_t cpuN,
                                  int32_t cpuThreads, int32_t config) {
    if (t == nullptr) {
        return hm::set_error(HM_INVALID_ARGUMENT, "hm_split_table_add_gemv: null table");
    }
    if (forK <= 0 || forN <= 0 || npuN < 0 || cpuN < 0 || cpuThreads < 0) {
        return hm::set_error(HM_INVALID_ARGUMENT, "hm_split_table_add_gemv: forK %d, forN %d must be positive, npuN %d, cpuN %d, cpuThreads %d not negative",
                             forK, forN, npuN, cpuN, cpuThreads);
    }
    if (!store(t, {1, forK, forN, layer_id, chunk_id}, make_desc(1, forK, npuN, cpuN, cpuThreads, config, 0))) {
        return hm::set_error(HM_OUT_OF_MEMORY, "hm_split_table_add_gemv: host allocation failed");
    }
    return HM_OK;
}

hm_status hm_split_table_find(const hm_split_table *t, int32_t M, int32_t K, int32_t N, int32_t layer_id, int32_t chunk_id, hm_split_desc *out) {
    if (t == nullptr || out == nullptr) {
        return hm::set_error(HM_INVALID_ARGUMENT, "hm_split_table_find: null pointer");
    }
    std::lock_guard<std::mutex> lock(t->mu);
    const auto it = t->entries.find({M, K, N, layer_id, chunk_id});
    if (it == t->entries.end()) {
        return hm::set_error(HM_INVALID_ARGUMENT, "hm_split_table_find: no entry for {%d, %d, %d, %d, %d}", M, K, N, layer_id, chunk_id);
    }
    *out = it->second;
    return HM_OK;
}

int64_t hm_split_table_size(const hm_split_table *t) {
    if (t == nullptr) {
        return 0;
    }
    std::lock_guard<std::mutex> lock(t->mu);
    return static_cast<int64_t>(t->entries.size());
}

size_t hm_linear_split_workspace_bytes(const hm_split_desc *d, const hm_weights *w0, const hm_weights *w1, int64_t M, int64_t K, int64_t N) {
    if (w0 == nullptr || M <= 0 || K <= 0 || N <= 0) {
        return 0;
    }
    if (d != nullptr && d->split_type > 0) {
        return hm_linear_k_split_workspace_bytes(w0, w1, M, d->split_type, K - d->split_type, N);
    }
    Piece p[3];
    const int n = plan_pieces(d, M, N, p);
    size_t need = 0;
    for (int i = 0; i < n; ++i) {
        need = std::max(need, hm_linear_workspace_bytes(w0, p[i].rows, K, p[i].cols));
    }
    return need;
}

hm_status hm_linear_split(const hm_split_desc *d, const hm_weights *w0, const hm_weights *w1, void *y, int64_t ldy, const void *x, int64_t ldx,
                          int64_t M, int64_t K, int64_t N, void *workspace, size_t workspace_bytes, void *stream) {
    if (w0 == nullptr || y == nullptr || x == nullptr || M <= 0 || K <= 0 || N <= 0) {
        return hm::set_error(HM_INVALID_ARGUMENT, "hm_linear_split: null pointer or empty shape");
    }
    if (d != nullptr && d->split_type > 0) {
        if (w1 == nullptr) {
            return hm::set_error(HM_INVALID_ARGUMENT, "hm_linear_split: a K split (K0 = %d) needs the second share's matrix", d->split_type);
        }
        if (d->split_type >= K) {
            return hm::set_error(HM_INVALID_ARGUMENT, "hm_linear_split: K0 = %d must lie inside K = %lld", d->split_type, static_cast<long long>(K));
        }
        return hm_linear_k_split(w0, w1, y, ldy, x, ldx, M, d->split_type, K - d->split_type, N, workspace, workspace_bytes, stream);
    }
    Piece p[3];
    const int n = plan_pieces(d, M, N, p);
    for (int i = 0; i < n; ++i) {
        uint16_t *yp = static_cast<uint16_t *>(y) + p[i].r0 * ldy;
        const uint16_t *xp = static_cast<const uint16_t *>(x) + p[i].r0 * ldx;
        // column shares write their own columns of y from column c0 of the matrix
        const hm_status st = hm_linear(w0, yp + p[i].c0, ldy, xp, ldx, p[i].rows, K, p[i].cols, p[i].c0, workspace, workspace_bytes, stream);
        if (st != HM_OK) {
            return st;
        }
    }
    return HM_OK;
}

hm_status hm_merged_ffn_check(int64_t m, int64_t hidden, int64_t intermediate, int64_t npu_channels, uint64_t *activation_bytes,
                              uint64_t *intermediate_bytes, uint64_t *weight_bytes) {
    if (m <= 0 || hidden <= 0 || intermediate <= 0 || npu_channels <= 0) {
        return hm::set_error(HM_INVALID_ARGUMENT, "merged FFN: nonpositive size");
    }
    if (m % 512 || hidden % 128 || intermediate % 128 || npu_channels % 256 || npu_channels >= intermediate || npu_channels > 8192) {
        return hm::set_error(HM_INVALID_ARGUMENT, "merged FFN: incompatible shape or channel partition");
    }
    // checked_product: a * b must stay within INT64_MAX (and size_t)
    const uint64_t limit = static_cast<uint64_t>(std::min<uint64_t>(std::numeric_limits<size_t>::max(), static_cast<uint64_t>(INT64_MAX)));
    bool ok = true;
    auto product = [&](uint64_t a, uint64_t b) -> uint64_t {
        if (a == 0 || b == 0 || a > limit / b) {
            ok = false;
            return 0;
        }
        return a * b;
    };
    const uint64_t act = product(product(static_cast<uint64_t>(m), static_cast<uint64_t>(hidden)), 2);
    const uint64_t mid = product(product(static_cast<uint64_t>(m), static_cast<uint64_t>(npu_channels)), 2);
    const uint64_t wts = product(product(static_cast<uint64_t>(hidden / 128), static_cast<uint64_t>(intermediate / 64)), 4352);
    if (!ok) {
        return hm::set_error(HM_INVALID_ARGUMENT, "merged FFN: invalid or overflowing buffer size");
    }
    if (activation_bytes != nullptr) *activation_bytes = act;
    if (intermediate_bytes != nullptr) *intermediate_bytes = mid;
    if (weight_bytes != nullptr) *weight_bytes = wts;
    return HM_OK;
}

int32_t hm_merged_ffn_supports(int64_t m, int64_t hidden, int64_t intermediate, int64_t rows, int64_t h, int64_t inter) {
    return rows > 1 && rows == m && h == hidden && inter == intermediate ? 1 : 0;
}

} // extern "C"

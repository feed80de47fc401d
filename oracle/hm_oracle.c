/*
 * CPU oracle of the W4A16 FFN hot path. TEST INFRASTRUCTURE ONLY: imported by tests/, by
 * __graft_entry__.smoke() as the checker and by bench.py's cpu_baseline leg. Nothing in the
 * product (heteromega_amd/) links or calls it.
 *
 * A plain-C restatement of the reference's byte and bit semantics:
 *   - bf16 rounding (npu/ffn/reference.py:26-35; kernels/gpu/src/bf16_device.hpp:15-22)
 *   - IEEE binary16 rounding (round to nearest even), for fp16 outputs
 *   - the 4352-byte tile packer (kernels/gpu/src/pack_w4a16.cpp:9-66), in its own loop order
 *   - the tile index (pack_w4a16.cpp:100-107)
 *   - a tile decoder that follows the consumer's address formulas
 *     (src/hipkernels/w4a16_gemv_packed.cu:34-75 and :84-90)
 *   - AWQ int32 unpack (py/unified_llm_w4a16/llama3_8b_w4a16_model.py:325-358)
 *   - the reference AVX-512 CPU GEMV on packed tiles (src/cpu_avx_kernels/w4a16_gemv_avx_packed.cpp:28-292),
 *     restated with the same tile walk, factorization, conversions and parallel grain; scalar fallback
 *     (:255-281) when the CPU lacks AVX-512. This is the reported CPU baseline.
 *   - the model-path SwiGLU between the CPU GEMVs: torch::silu_ then mul_ on bf16
 *     (src/unified_llm_w4a16_hetero/unified_llm_w4a16.cpp:2881-2883), each rounding to bf16.
 *   - a float64 FFN block at one row (RMSNorm, SwiGLU FFN, residual add) with the engine's rounding points,
 *     for full-size layer stacks without float64 weight matrices in memory.
 *   - emulations of the rounding points of the reference's GPU kernels (fp16-accumulating decode GEMV,
 *     bf16-dequantizing prefill GEMM), to attribute disagreements with them.
 * Float reference math (dequantize, matmul, SwiGLU, RMSNorm) also lives in oracle/oracle.py (numpy, float64).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <immintrin.h>
#include <omp.h>

/* ---- 16-bit floats ---------------------------------------------------------------------------- */

static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* bf16 round to nearest even; infinities kept; NaN stays NaN with the quiet bit (reference.py:26-35). */
uint16_t or_bf16_from_f32(float f) {
    const uint32_t u = f32_bits(f);
    if ((u & 0x7F800000u) == 0x7F800000u) {
        uint32_t hi = u & 0xFFFF0000u;
        if (u & 0x007FFFFFu) {
            hi |= 0x00400000u;
        }
        return (uint16_t)(hi >> 16);
    }
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

float or_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* IEEE binary16, round to nearest even, overflow to infinity, subnormals kept. */
uint16_t or_f16_from_f32(float f) {
    const uint32_t u = f32_bits(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) { /* inf or NaN (NaN keeps a quiet payload bit) */
        return (uint16_t)(sign | 0x7C00u | (a > 0x7F800000u ? 0x0200u : 0u));
    }
    const int e = (int)(a >> 23);
    if (e == 0) {
        return sign; /* f32 subnormals are far below the f16 range */
    }
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u; /* value = m * 2^(E - 23) */
    const int E = e - 127;
    const int ulp_exp = E >= -14 ? E - 10 : -24;    /* last kept bit: normal or subnormal f16 */
    const int shift = ulp_exp - (E - 23);
    if (shift > 24) {
        return sign;
    }
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) {
        ++q;
    }
    if (E >= -14) {
        int e16 = E + 15;
        if (q == 2048u) {
            q = 1024u;
            ++e16;
        }
        if (e16 >= 31) {
            return (uint16_t)(sign | 0x7C00u);
        }
        return (uint16_t)(sign | ((uint32_t)e16 << 10) | (q - 1024u));
    }
    return (uint16_t)(sign | q); /* subnormal; q == 1024 is the smallest normal's encoding */
}

float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    if (e == 0x1Fu) {
        return bits_f32(sign | 0x7F800000u | (m << 13));
    }
    if (e == 0) {
        return (sign ? -1.0f : 1.0f) * ldexpf((float)m, -24);
    }
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

void or_bf16_round_array(const float *in, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_bf16_from_f32(in[i]);
}

void or_f16_round_array(const float *in, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_f16_from_f32(in[i]);
}

/* ---- 4352-byte tiles ----------------------------------------------------------------------------- */

/* Column group g holds tile columns g, g + 8, ...; storage runs over groups, then columns, then rows. */
int64_t or_tile_index(int64_t c, int64_t r, int64_t tiles_k, int64_t tiles_n) {
    int64_t t = 0;
    for (int64_t g = 0; g < 8; ++g) {
        for (int64_t cc = g; cc < tiles_n; cc += 8) {
            if (cc == c) {
                return t + r;
            }
            t += tiles_k;
        }
    }
    return -1;
}

/* Packs q [K, N] u8, scales [K/128, N] bf16 bits, zeros [K/128, N] u8. Returns 0 or -1 on bad shape. */
int or_pack_tiles(const uint8_t *q, const uint16_t *s, const uint8_t *z, int64_t K, int64_t N, uint8_t *out) {
    if (K <= 0 || N <= 0 || K % 128 || N % 64) {
        return -1;
    }
    const int64_t tiles_k = K / 128, tiles_n = N / 64;
    uint8_t *tile = out;
    for (int64_t g = 0; g < 8; ++g) {
        for (int64_t c = g; c < tiles_n; c += 8) {
            for (int64_t r = 0; r < tiles_k; ++r, tile += 4352) {
                for (int row = 0; row < 128; ++row) {
                    for (int col = 0; col < 64; col += 2) {
                        const int a = row >> 3, b = row & 7, cc = col >> 3, j = (col & 7) >> 1;
                        const uint8_t lo = q[(r * 128 + row) * N + c * 64 + col] & 0x0F;
                        const uint8_t hi = q[(r * 128 + row) * N + c * 64 + col + 1] & 0x0F;
                        tile[((a * 8 + cc) * 8 + b) * 4 + j] = (uint8_t)(lo | (hi << 4));
                    }
                }
                for (int col = 0; col < 64; ++col) {
                    const uint16_t sb = s[r * N + c * 64 + col];
                    tile[4096 + 2 * col] = (uint8_t)(sb & 0xFF);
                    tile[4096 + 2 * col + 1] = (uint8_t)(sb >> 8);
                    const uint8_t zb = z[r * N + c * 64 + col];
                    tile[4224 + (col / 8) * 16 + (col % 8)] = zb;
                    tile[4224 + (col / 8) * 16 + 8 + (col % 8)] = zb;
                }
            }
        }
    }
    return 0;
}

/* Decodes with the consumer's formulas: block bx, base_z = sum over earlier column groups of
 * ceil((tiles_n - g) / 8) * tiles_k + (bx / 8) * tiles_k; per K tile, thread (warp, lane) reads byte
 * (sr << 8) + (warp << 5) + lane for rows sr * 8 + lane / 4 and columns warp * 8 + (lane % 4) * 2 + {0, 1};
 * scale of column i at 4096 + 2 i, zero at 4224 + (i / 8) * 16 + i % 8. Also returns the duplicated zero
 * copy (+8) so tests can check it. */
int or_unpack_tiles(const uint8_t *packed, int64_t K, int64_t N, uint8_t *q, uint16_t *s, uint8_t *z, uint8_t *z_dup) {
    if (K <= 0 || N <= 0 || K % 128 || N % 64) {
        return -1;
    }
    const int64_t tiles_k = K / 128, tiles_n = N / 64;
    for (int64_t bx = 0; bx < tiles_n; ++bx) {
        int64_t tbg = 0;
        for (int64_t g = 0; g < bx % 8; ++g) {
            tbg += ((tiles_n + 7 - g) / 8) * tiles_k;
        }
        const int64_t base_z = tbg + (bx / 8) * tiles_k;
        for (int64_t kt = 0; kt < tiles_k; ++kt) {
            const uint8_t *w = packed + (base_z + kt) * 4352;
            for (int warp = 0; warp < 8; ++warp) {
                for (int lane = 0; lane < 32; ++lane) {
                    const int row_in = lane >> 2, pair = lane & 3;
                    const int out0 = warp * 8 + pair * 2;
                    for (int sr = 0; sr < 16; ++sr) {
                        const uint8_t byte = w[(sr << 8) + (warp << 5) + lane];
                        const int64_t row = kt * 128 + sr * 8 + row_in;
                        q[row * N + bx * 64 + out0] = byte & 0x0F;
                        q[row * N + bx * 64 + out0 + 1] = (byte >> 4) & 0x0F;
                    }
                }
            }
            for (int i = 0; i < 64; ++i) {
                s[kt * N + bx * 64 + i] = (uint16_t)(w[4096 + 2 * i] | (w[4096 + 2 * i + 1] << 8));
                z[kt * N + bx * 64 + i] = w[4224 + (i / 8) * 16 + i % 8];
                if (z_dup) {
                    z_dup[kt * N + bx * 64 + i] = w[4224 + (i / 8) * 16 + 8 + i % 8];
                }
            }
        }
    }
    return 0;
}

/* AWQ: qweight [In, Out/8] int32 -> [In, Out] u8. The model transposes to [Out/8, In], splits each
 * word into 8 parts with shifts 4 * [0, 4, 1, 5, 2, 6, 3, 7][k] (part k), stacks them last, permutes to
 * [Out/8, 8, In] and views [Out, In]: output feature 8 j + k takes part k of word column j.
 * qzeros [G, Out/8] follows the same part order without the transpose. */
void or_awq_unpack(const int32_t *packed, int64_t rows, int64_t cols8, uint8_t *out) {
    static const int shift_of_part[8] = {0, 16, 4, 20, 8, 24, 12, 28};
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t j = 0; j < cols8; ++j) {
            const uint32_t w = (uint32_t)packed[r * cols8 + j];
            for (int k = 0; k < 8; ++k) {
                out[r * (cols8 * 8) + j * 8 + k] = (uint8_t)((w >> shift_of_part[k]) & 0x0Fu);
            }
        }
    }
}

/* ---- Reference AVX-512 CPU GEMV on packed tiles (the CPU baseline) --------------------------------- */

/* One 64-column tile bx of y = x W over all K tiles, scalar fallback of the reference (:255-281). */
static void gemv_tile_scalar(const uint16_t *x, const uint8_t *packed, int64_t K, int64_t tiles_k, int64_t tiles_n, int64_t bx,
                             float acc[64]) {
    int64_t tbg = 0;
    for (int64_t g = 0; g < bx % 8; ++g) tbg += ((tiles_n + 7 - g) / 8) * tiles_k;
    const int64_t base_z = tbg + (bx / 8) * tiles_k;
    for (int c = 0; c < 64; ++c) acc[c] = 0.0f;
    for (int64_t kt = 0; kt < tiles_k; ++kt) {
        const uint8_t *w = packed + (base_z + kt) * 4352;
        float sc[64], zr[64];
        for (int i = 0; i < 64; ++i) {
            sc[i] = or_bf16_to_f32((uint16_t)(w[4096 + 2 * i] | (w[4096 + 2 * i + 1] << 8)));
            zr[i] = (float)w[4224 + (i / 8) * 16 + (i % 8)];
        }
        const int64_t row_start = kt * 128;
        const int r_limit = (int)(row_start + 128 > K ? K - row_start : 128);
        for (int r = 0; r < r_limit; ++r) {
            const float in = or_bf16_to_f32(x[row_start + r]);
            const int SR = r >> 3, IR = r & 7;
            for (int c = 0; c < 64; ++c) {
                const int SC = c >> 3, IC = c & 7;
                const uint8_t byte = w[((SR * 8 + SC) << 5) + (IR << 2) + (IC >> 1)];
                const int q4 = (IC & 1) ? ((byte >> 4) & 0x0F) : (byte & 0x0F);
                acc[c] += ((float)q4 - zr[c]) * sc[c] * in;
            }
        }
    }
}

/* bf16 -> fp32 of 16 values: the bits shifted up by 16 (what _mm512_cvtpbh_ps does). */
#if defined(__GNUC__)
__attribute__((target("avx512f,avx512bw,avx512vl")))
#endif
static inline __m512 cvt_bf16x16(__m256i raw) {
    return _mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu16_epi32(raw), 16));
}

#if defined(__GNUC__)
__attribute__((target("avx512f,avx512bw,avx512vl")))
#endif
static void gemv_tile_avx512(const uint16_t *x, const uint8_t *packed, int64_t K, int64_t tiles_k, int64_t tiles_n, int64_t bx,
                             float acc[64]) {
    int64_t tbg = 0;
    for (int64_t g = 0; g < bx % 8; ++g) tbg += ((tiles_n + 7 - g) / 8) * tiles_k;
    const int64_t base_z = tbg + (bx / 8) * tiles_k;
    for (int c = 0; c < 64; ++c) acc[c] = 0.0f;
    for (int64_t kt = 0; kt < tiles_k; ++kt) {
        const uint8_t *w = packed + (base_z + kt) * 4352;
        const uint16_t *scale = (const uint16_t *)(w + 4096);
        const uint8_t *zero = w + 4224;
        const int64_t row_start = kt * 128;
        const int r_limit = (int)(row_start + 128 > K ? K - row_start : 128);
        /* 1. Sum of the tile's 128 inputs, 16 at a time, then the remainder. */
        __m512 v_sum = _mm512_setzero_ps();
        int r = 0;
        for (; r + 16 <= r_limit; r += 16) {
            const __m256i raw = _mm256_loadu_si256((const __m256i *)(x + row_start + r));
            v_sum = _mm512_add_ps(v_sum, cvt_bf16x16(raw));
        }
        float input_sum = _mm512_reduce_add_ps(v_sum);
        for (; r < r_limit; ++r) input_sum += or_bf16_to_f32(x[row_start + r]);
        const __m512 v_input_sum = _mm512_set1_ps(input_sum);
        /* 2. Four chunks of 16 columns. */
        for (int chunk = 0; chunk < 4; ++chunk) {
            const int c_start = chunk * 16;
            const __m512 v_s = cvt_bf16x16(_mm256_loadu_si256((const __m256i *)(scale + c_start)));
            uint16_t zb[16];
            for (int i = 0; i < 16; ++i) {
                const int c = c_start + i;
                zb[i] = or_bf16_from_f32((float)zero[(c / 8) * 16 + (c % 8)]);
            }
            const __m512 v_z = cvt_bf16x16(_mm256_loadu_si256((const __m256i *)zb));
            __m512 a0 = _mm512_setzero_ps(), a1 = _mm512_setzero_ps(), a2 = _mm512_setzero_ps(), a3 = _mm512_setzero_ps();
            const int sc0 = chunk * 2, sc1 = chunk * 2 + 1;
            for (int sr = 0; sr < 16; ++sr) {
                const int r_base = sr * 8;
                if (r_base >= r_limit) break;
                const uint8_t *p0 = w + (sr * 8 + sc0) * 32;
                const uint8_t *p1 = w + (sr * 8 + sc1) * 32;
                for (int qd = 0; qd < 2; ++qd) {
                    const int r_quad = qd * 4;
                    if (r_base + r_quad >= r_limit) break;
                    const __m128i v0 = _mm_loadu_si128((const __m128i *)(p0 + r_quad * 4));
                    const __m128i v1 = _mm_loadu_si128((const __m128i *)(p1 + r_quad * 4));
                    const __m128i pair0 = _mm_unpacklo_epi32(v0, v1); /* rows 0, 1: 16 columns each */
                    const __m128i pair1 = _mm_unpackhi_epi32(v0, v1); /* rows 2, 3 */
                    const __m128i mask = _mm_set1_epi8(0x0F);
                    {
                        const __m128i lo = _mm_and_si128(pair0, mask);
                        const __m128i hi = _mm_and_si128(_mm_srli_epi16(pair0, 4), mask);
                        const __m128i u8lo = _mm_unpacklo_epi8(lo, hi), u8hi = _mm_unpackhi_epi8(lo, hi);
                        const int ir = r_quad;
                        const __m512 in0 = _mm512_set1_ps(or_bf16_to_f32(x[row_start + r_base + ir]));
                        const __m512 f0 = _mm512_cvtepi32_ps(_mm512_cvtepu16_epi32(_mm256_cvtepu8_epi16(u8lo)));
                        if (qd == 0) a0 = _mm512_fmadd_ps(f0, in0, a0);
                        else a2 = _mm512_fmadd_ps(f0, in0, a2);
                        if (r_base + ir + 1 < r_limit) {
                            const __m512 in1 = _mm512_set1_ps(or_bf16_to_f32(x[row_start + r_base + ir + 1]));
                            const __m512 f1 = _mm512_cvtepi32_ps(_mm512_cvtepu16_epi32(_mm256_cvtepu8_epi16(u8hi)));
                            if (qd == 0) a1 = _mm512_fmadd_ps(f1, in1, a1);
                            else a3 = _mm512_fmadd_ps(f1, in1, a3);
                        }
                    }
                    if (r_base + r_quad + 2 < r_limit) {
                        const __m128i lo = _mm_and_si128(pair1, mask);
                        const __m128i hi = _mm_and_si128(_mm_srli_epi16(pair1, 4), mask);
                        const __m128i u8lo = _mm_unpacklo_epi8(lo, hi), u8hi = _mm_unpackhi_epi8(lo, hi);
                        const int ir = r_quad + 2;
                        const __m512 in0 = _mm512_set1_ps(or_bf16_to_f32(x[row_start + r_base + ir]));
                        const __m512 f0 = _mm512_cvtepi32_ps(_mm512_cvtepu16_epi32(_mm256_cvtepu8_epi16(u8lo)));
                        if (qd == 0) a2 = _mm512_fmadd_ps(f0, in0, a2);
                        else a0 = _mm512_fmadd_ps(f0, in0, a0);
                        if (r_base + ir + 1 < r_limit) {
                            const __m512 in1 = _mm512_set1_ps(or_bf16_to_f32(x[row_start + r_base + ir + 1]));
                            const __m512 f1 = _mm512_cvtepi32_ps(_mm512_cvtepu16_epi32(_mm256_cvtepu8_epi16(u8hi)));
                            if (qd == 0) a3 = _mm512_fmadd_ps(f1, in1, a3);
                            else a1 = _mm512_fmadd_ps(f1, in1, a1);
                        }
                    }
                }
            }
            const __m512 unscaled = _mm512_add_ps(_mm512_add_ps(a0, a1), _mm512_add_ps(a2, a3));
            const __m512 scaled = _mm512_mul_ps(_mm512_sub_ps(unscaled, _mm512_mul_ps(v_z, v_input_sum)), v_s);
            _mm512_storeu_ps(acc + c_start, _mm512_add_ps(_mm512_loadu_ps(acc + c_start), scaled));
        }
    }
}

/* The reference's AVX-512 branch is compiled under __AVX512F__ and uses 512-bit float/integer ops and
 * bf16 widening (a 16-bit shift); AVX-512 F, BW and VL cover every instruction of the restatement. */
int or_cpu_has_avx512(void) {
#if defined(__GNUC__)
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("avx512vl");
#else
    return 0;
#endif
}

/* y[start_col, end_col) of y = x W, x bf16 [K], W packed [K, N] (N = all columns of the packed matrix),
 * parallel over 64-column tiles like at::parallel_for(start_tile, end_tile, 1, ...). Output is bf16 and,
 * as in the reference, indexed by absolute column. use_avx: -1 auto, 0 scalar, 1 AVX-512. Returns the
 * branch that ran (1 AVX-512, 0 scalar). */
int or_cpu_gemv_packed(const uint16_t *x, const uint8_t *packed, int64_t K, int64_t N, int64_t start_col, int64_t end_col, uint16_t *y,
                       int threads, int use_avx) {
    const int64_t tiles_k = (K + 127) / 128, tiles_n = (N + 63) / 64;
    if (end_col < 0) end_col = N;
    int64_t start_tile = start_col / 64, end_tile = (end_col + 63) / 64;
    if (start_tile < 0) start_tile = 0;
    if (end_tile > tiles_n) end_tile = tiles_n;
    const int avx = use_avx < 0 ? or_cpu_has_avx512() : (use_avx && or_cpu_has_avx512());
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int64_t bx = start_tile; bx < end_tile; ++bx) {
        float acc[64];
        if (avx) gemv_tile_avx512(x, packed, K, tiles_k, tiles_n, bx, acc);
        else gemv_tile_scalar(x, packed, K, tiles_k, tiles_n, bx, acc);
        for (int c = 0; c < 64; ++c) {
            if (bx * 64 + c < N) y[bx * 64 + c] = or_bf16_from_f32(acc[c]);
        }
    }
    return avx;
}

/* torch::silu_(gate) then gate.mul_(up) on bf16: SiLU in fp32 of the bf16 value, rounded; product in fp32
 * of the two bf16 values, rounded. */
void or_silu_mul_bf16_model(uint16_t *gate, const uint16_t *up, int64_t n, int threads) {
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int64_t i = 0; i < n; ++i) {
        const float g = or_bf16_to_f32(gate[i]);
        const float s = or_bf16_to_f32(or_bf16_from_f32(g / (1.0f + expf(-g))));
        gate[i] = or_bf16_from_f32(s * or_bf16_to_f32(up[i]));
    }
}

/* Decode FFN on the CPU, as the model's cpu path runs it: gate GEMV, up GEMV, silu_ and mul_, down GEMV.
 * gate_up_scratch holds 2 * inter bf16 values. Returns the GEMV branch used. */
int or_cpu_ffn_decode(const uint16_t *x, const uint8_t *gate, const uint8_t *up, const uint8_t *down, int64_t hidden, int64_t inter,
                      uint16_t *gate_up_scratch, uint16_t *y, int threads, int use_avx) {
    uint16_t *g = gate_up_scratch, *u = gate_up_scratch + inter;
    int avx = or_cpu_gemv_packed(x, gate, hidden, inter, 0, inter, g, threads, use_avx);
    or_cpu_gemv_packed(x, up, hidden, inter, 0, inter, u, threads, use_avx);
    or_silu_mul_bf16_model(g, u, inter, threads);
    or_cpu_gemv_packed(g, down, inter, hidden, 0, hidden, y, threads, use_avx);
    return avx;
}

/* ---- rounding from double ------------------------------------------------------------------------
 * Direct round to nearest even from a double: rounding to float first and then to 16 bits would round
 * twice and move values that sit within a float ulp of a 16-bit tie. */

static uint16_t round16_from_f64(double d, int mant_bits, int exp_bias, int max_exp, uint16_t inf_bits, uint16_t nan_bits) {
    const uint16_t sign = signbit(d) ? 0x8000u : 0u;
    if (isnan(d)) return (uint16_t)(sign | nan_bits);
    const double a = fabs(d);
    if (a == 0.0) return sign;
    if (isinf(a)) return (uint16_t)(sign | inf_bits);
    int e;
    (void)frexp(a, &e);
    int E = e - 1; /* a = 1.f * 2^E */
    const int min_exp = 1 - exp_bias;
    if (E < min_exp) { /* subnormal: quantum 2^(min_exp - mant_bits) */
        const double r = nearbyint(ldexp(a, mant_bits - min_exp));
        return (uint16_t)(sign | (uint16_t)r); /* r == 2^mant_bits is the smallest normal's encoding */
    }
    double r = nearbyint(ldexp(a, mant_bits - E)); /* in [2^mant_bits, 2^(mant_bits + 1)] */
    if (r == ldexp(1.0, mant_bits + 1)) {
        r = ldexp(1.0, mant_bits);
        ++E;
    }
    if (E > max_exp) return (uint16_t)(sign | inf_bits);
    return (uint16_t)(sign | ((uint32_t)(E + exp_bias) << mant_bits) | ((uint32_t)r - (1u << mant_bits)));
}

uint16_t or_f16_from_f64(double d) { return round16_from_f64(d, 10, 15, 15, 0x7C00u, 0x7E00u); }

uint16_t or_bf16_from_f64(double d) { return round16_from_f64(d, 7, 127, 127, 0x7F80u, 0x7FC0u); }

static inline double bits_to_f64(uint16_t b, int dtype) { return dtype == 1 ? (double)or_f16_to_f32(b) : (double)or_bf16_to_f32(b); }

static inline uint16_t f64_to_bits(double d, int dtype) { return dtype == 1 ? or_f16_from_f64(d) : or_bf16_from_f64(d); }

static inline double silu_f64(double v) {
    const double e = exp(-fabs(v));
    return v >= 0 ? v / (1.0 + e) : v * e / (1.0 + e);
}

/* out[n] (+)= sum_k x[k] (q[k][n] - z[k / group][n]) s[k / group][n] for n in [n0, n1), in float64, as the
 * reference's per-tile factorization s (sum q x - z sum x) (kernels/gpu/src/gemv_w4a16.cu:91-98) applied per
 * group. q [K, N] row-major, s (dtype bits) and z [K / group, N]. */
static void matvec_f64(const double *x, const uint8_t *q, const uint16_t *s, const uint8_t *z, int64_t K, int64_t N, int64_t group,
                       int dtype, int64_t n0, int64_t n1, double *out) {
    const int64_t w = n1 - n0;
    double p[64];
    for (int64_t c = 0; c < w; ++c) out[n0 + c] = 0.0;
    for (int64_t g = 0; g < K / group; ++g) {
        double xs = 0.0;
        for (int64_t c = 0; c < w; ++c) p[c] = 0.0;
        for (int64_t k = g * group; k < (g + 1) * group; ++k) {
            const uint8_t *row = q + k * N + n0;
            xs += x[k];
            for (int64_t c = 0; c < w; ++c) p[c] += x[k] * (double)row[c];
        }
        for (int64_t c = 0; c < w; ++c) {
            const double sc = bits_to_f64(s[g * N + n0 + c], dtype);
            out[n0 + c] += sc * (p[c] - (double)z[g * N + n0 + c] * xs);
        }
    }
}

/* One pre-norm FFN block at one row in float64 with the engine's rounding points (SwiGLU and RMSNorm numerics of
 * kernels/gpu/src/silu_mul.cu:10-30 and src/hipkernels/rmsnorm.cu:25-62, layer as unified_llm_w4a16.cpp:2867-2892):
 *   normed = round(x * rsqrt(mean(x^2) + eps) * w)      (norm_w == NULL: normed = x, no rounding)
 *   act    = round(SiLU(normed Wg) * (normed Wu))
 *   y      = round(act Wd),  x_out = round(x + y)
 * x, norm_w, the scales and every *_bits output are 16-bit `dtype` values (0 bf16, 1 fp16); g_raw, u_raw, y_raw
 * (may be NULL) receive the unrounded float64 sums. Parallel over 64-column chunks. */
void or_ffn_block_f64(const uint16_t *x, const uint16_t *norm_w, double eps, const uint8_t *gq, const uint16_t *gs, const uint8_t *gz,
                      const uint8_t *uq, const uint16_t *us, const uint8_t *uz, const uint8_t *dq, const uint16_t *ds, const uint8_t *dz,
                      int64_t hidden, int64_t inter, int64_t group, int dtype, int threads, uint16_t *normed_bits, uint16_t *act_bits,
                      uint16_t *y_bits, uint16_t *x_out_bits, double *g_raw, double *u_raw, double *y_raw) {
    if (threads < 1) threads = 1;
    double *xn = (double *)malloc(sizeof(double) * (size_t)hidden);
    double *g = (double *)malloc(sizeof(double) * (size_t)inter);
    double *u = (double *)malloc(sizeof(double) * (size_t)inter);
    double *act = (double *)malloc(sizeof(double) * (size_t)inter);
    double *y = (double *)malloc(sizeof(double) * (size_t)hidden);
    double ss = 0.0;
    for (int64_t k = 0; k < hidden; ++k) {
        const double v = bits_to_f64(x[k], dtype);
        ss += v * v;
    }
    const double r = 1.0 / sqrt(ss / (double)hidden + eps);
    for (int64_t k = 0; k < hidden; ++k) {
        const double v = bits_to_f64(x[k], dtype);
        if (norm_w != NULL) {
            const uint16_t b = f64_to_bits(v * r * bits_to_f64(norm_w[k], dtype), dtype);
            if (normed_bits != NULL) normed_bits[k] = b;
            xn[k] = bits_to_f64(b, dtype);
        } else {
            xn[k] = v;
        }
    }
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (int64_t c = 0; c < (inter + 63) / 64; ++c) {
        const int64_t n0 = c * 64, n1 = n0 + 64 < inter ? n0 + 64 : inter;
        matvec_f64(xn, gq, gs, gz, hidden, inter, group, dtype, n0, n1, g);
        matvec_f64(xn, uq, us, uz, hidden, inter, group, dtype, n0, n1, u);
        for (int64_t n = n0; n < n1; ++n) {
            const uint16_t b = f64_to_bits(silu_f64(g[n]) * u[n], dtype);
            act_bits[n] = b;
            act[n] = bits_to_f64(b, dtype);
        }
    }
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (int64_t c = 0; c < (hidden + 63) / 64; ++c) {
        const int64_t n0 = c * 64, n1 = n0 + 64 < hidden ? n0 + 64 : hidden;
        matvec_f64(act, dq, ds, dz, inter, hidden, group, dtype, n0, n1, y);
    }
    for (int64_t h = 0; h < hidden; ++h) {
        const uint16_t yb = f64_to_bits(y[h], dtype);
        y_bits[h] = yb;
        if (x_out_bits != NULL) x_out_bits[h] = f64_to_bits(bits_to_f64(x[h], dtype) + bits_to_f64(yb, dtype), dtype);
    }
    if (g_raw != NULL) memcpy(g_raw, g, sizeof(double) * (size_t)inter);
    if (u_raw != NULL) memcpy(u_raw, u, sizeof(double) * (size_t)inter);
    if (y_raw != NULL) memcpy(y_raw, y, sizeof(double) * (size_t)hidden);
    free(xn);
    free(g);
    free(u);
    free(act);
    free(y);
}

/* ---- rounding points of the reference's GPU kernels -----------------------------------------------
 * These emulate, on the CPU, where the reference's HIP kernels round. They need an RDNA GPU to run, so their
 * exact output bits cannot be pinned here; the emulations make a disagreement with them attributable. */

/* The reference decode GEMV w4a16_gemv_kernel_packed (src/hipkernels/w4a16_gemv_packed.cu:24-176) on logical
 * weights: x (bf16) to fp16; scale (bf16) and zero to fp16; w = fp16((q - z) * s); per lane four fp16
 * accumulators, lane (row b of each 8-row block) taking rows sr * 8 + b of every K tile into accumulator sr % 4
 * with an fp16 fused multiply-add, K tiles in order; then fp16 (a0 + a1) + (a2 + a3), to fp32, and the shuffle
 * tree ((v0 + v1) + (v2 + v3)) + ((v4 + v5) + (v6 + v7)) over the 8 lanes in fp32; bf16 output.
 * q [K, N], s bf16 bits [K / 128, N], z [K / 128, N]; group 128 (the tile height). */
void or_hm_gemv_emul(const uint16_t *x_bf16, const uint8_t *q, const uint16_t *s, const uint8_t *z, int64_t K, int64_t N, uint16_t *y_bf16,
                     int threads) {
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int64_t n = 0; n < N; ++n) {
        float v[8];
        for (int b = 0; b < 8; ++b) {
            double acc[4] = {0.0, 0.0, 0.0, 0.0}; /* fp16 values */
            for (int64_t kt = 0; kt < K / 128; ++kt) {
                const double s16 = (double)or_f16_to_f32(or_f16_from_f32(or_bf16_to_f32(s[kt * N + n])));
                const double z16 = (double)or_f16_to_f32(or_f16_from_f32((float)(int8_t)z[kt * N + n]));
                for (int sr = 0; sr < 16; ++sr) {
                    const int64_t row = kt * 128 + sr * 8 + b;
                    const double w = (double)or_f16_to_f32(or_f16_from_f64(((double)q[row * N + n] - z16) * s16));
                    const double xv = (double)or_f16_to_f32(or_f16_from_f32(or_bf16_to_f32(x_bf16[row])));
                    acc[sr % 4] = (double)or_f16_to_f32(or_f16_from_f64(w * xv + acc[sr % 4]));
                }
            }
            const double a01 = (double)or_f16_to_f32(or_f16_from_f64(acc[0] + acc[1]));
            const double a23 = (double)or_f16_to_f32(or_f16_from_f64(acc[2] + acc[3]));
            v[b] = or_f16_to_f32(or_f16_from_f64(a01 + a23));
        }
        const float t = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
        y_bf16[n] = or_bf16_from_f32(t);
    }
}

/* The reference prefill GEMM w4a16_gemm_rocwmma_packed (src/hipkernels/w4a16_gemm_packed.cu:380-613) on logical
 * weights: each weight rounded once to bf16((q - z) * s) with the product in fp32 (:491-497), bf16 x bf16
 * products accumulated in fp32 over 16-K steps in K order (one rounding per 16-K step: the sum inside a step
 * is formed exactly here), fp32 result. q [K, N], s bf16 bits and z [K / group, N], x bf16 [M, K];
 * out fp32 [M, N]. */
void or_hm_gemm_emul(const uint16_t *x_bf16, const uint8_t *q, const uint16_t *s, const uint8_t *z, int64_t M, int64_t K, int64_t N,
                     int64_t group, float *out, int threads) {
    if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
    {
        float *acc = (float *)malloc(sizeof(float) * (size_t)M);
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            for (int64_t m = 0; m < M; ++m) acc[m] = 0.0f;
            for (int64_t k0 = 0; k0 < K; k0 += 16) {
                double wv[16];
                for (int j = 0; j < 16; ++j) {
                    const int64_t k = k0 + j;
                    const float sc = or_bf16_to_f32(s[(k / group) * N + n]);
                    wv[j] = (double)or_bf16_to_f32(or_bf16_from_f32((float)((int)q[k * N + n] - (int)z[(k / group) * N + n]) * sc));
                }
                for (int64_t m = 0; m < M; ++m) {
                    double step = 0.0;
                    for (int j = 0; j < 16; ++j) step += wv[j] * (double)or_bf16_to_f32(x_bf16[m * K + k0 + j]);
                    acc[m] = (float)((double)acc[m] + step);
                }
            }
            for (int64_t m = 0; m < M; ++m) out[m * N + n] = acc[m];
        }
        free(acc);
    }
}

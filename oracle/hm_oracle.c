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
 * Float reference math (dequantize, matmul, SwiGLU, RMSNorm) lives in oracle/oracle.py (numpy, float64).
 */
#include <math.h>
#include <stdint.h>
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

/*
 * hm_w4a16.h - C ABI of the MI355X (gfx950) W4A16 SwiGLU FFN engine.
 *
 * Plain C: pointers, sizes and status codes only. All tensors are caller-owned
 * memory; the `stream` arguments are hipStream_t values passed as void*
 * (NULL means the default stream). Compute entry points enqueue work on that
 * stream and return without synchronizing; they never allocate.
 *
 * Element types: activations, outputs and per-group scales are 16-bit floats,
 * either bf16 (the reference operator surface) or fp16 (hm_dtype). They are
 * passed as raw uint16_t bits. Quantized weights are unsigned int4 (0..15)
 * with unsigned int4 zero points, dequantized as (q - z) * s.
 *
 * Errors: every function that can fail returns an hm_status; the message of
 * the last failure on the calling thread is available from hm_last_error().
 * This replaces the reference's TORCH_CHECK / std::exit / std::runtime_error
 * paths (kernels/gpu/src/pack_w4a16.cpp:11-16, unified_llm_w4a16.cpp:889-891,
 * src/hipkernels/w4a16_gemv_packed.cu:197-200).
 */
#ifndef HM_W4A16_H
#define HM_W4A16_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HM_ABI_VERSION 1

typedef enum hm_status {
    HM_OK = 0,
    HM_INVALID_ARGUMENT = 1, /* shape, alignment, range or pointer check failed */
    HM_UNSUPPORTED = 2,      /* valid request that this build does not implement */
    HM_HIP_ERROR = 3,        /* a HIP runtime call or kernel launch failed */
    HM_OUT_OF_MEMORY = 4,    /* a create/repack call could not allocate device memory */
    HM_WORKSPACE_TOO_SMALL = 5
} hm_status;

/* The *_FORCE_INT32_ enumerators are no values: they make each enumeration span every 32-bit value, so that a value
 * outside the list that a caller passes is still a value of the type in C++ and the library rejects it with
 * HM_INVALID_ARGUMENT (C++ gives an enumeration without them only the values of its enumerators' bit width). */
typedef enum hm_dtype {
    HM_BF16 = 0, /* reference surface: include/hipkernels/w4a16_gemm_packed.hpp:31-33 */
    HM_FP16 = 1,
    HM_DTYPE_FORCE_INT32_ = -2147483647 - 1
} hm_dtype;

/* Column order of a reference-packed gate_up matrix
 * (kernels/gpu/include/heteromega/gpu_ffn.hpp:43-46). */
typedef enum hm_gate_up_layout {
    HM_GATE_UP_BLOCKED = 0,     /* [gate 0..n) | up 0..n) ] */
    HM_GATE_UP_INTERLEAVED = 1, /* per 64 channels: 64 gate columns, then 64 up columns */
    HM_GATE_UP_LAYOUT_FORCE_INT32_ = -2147483647 - 1
} hm_gate_up_layout;

int hm_abi_version(void);
const char *hm_last_error(void);

/* ---------------------------------------------------------------------------
 * Reference 4352-byte tile format (host memory, no GPU needed).
 * A [K, N] matrix is (K/128) x (N/64) tiles of 4096 nibble bytes, 64 bf16
 * scales and 128 zero bytes, in column-group order.
 * ------------------------------------------------------------------------- */

/* Bytes of a packed [K, N] matrix: (K/128)*(N/64)*4352, or -1 if K%128 or N%64.
 * Replaces MergedFfnConfig::weight_bytes (include/heteromega/merged_ffn_contract.hpp:60). */
int64_t hm_packed_bytes(int64_t K, int64_t N);

/* Position of tile (tile column c, tile row r) in a packed matrix of
 * tiles_k x tiles_n tiles, or -1 when out of range.
 * Replaces heteromega::packed_tile_index (kernels/gpu/src/pack_w4a16.cpp:100-107). */
int64_t hm_packed_tile_index(int64_t c, int64_t r, int64_t tiles_k, int64_t tiles_n);

/* Packs q [K, N] (uint8 0..15), scales [K/128, N] (bf16 bits) and zeros
 * [K/128, N] (int8 0..15), all row-major host arrays, into hm_packed_bytes(K, N)
 * bytes at `out`. Replaces heteromega::pack_w4a16 (kernels/gpu/src/pack_w4a16.cpp:9-66)
 * and the packers it mirrors (py/unified_llm_w4a16/llama3_8b_w4a16_model.py:546-656,
 * src/unified_llm_w4a16_hetero/unified_llm_w4a16.cpp:1242-1387). */
hm_status hm_pack_w4a16(const uint8_t *q, const uint16_t *scales, const int8_t *zeros, int64_t K, int64_t N,
                        uint8_t *out);

/* Unpacks AWQ int32 tensors (host): qweight [K, N/8] -> q [K, N] uint8, and
 * qzeros [G, N/8] -> zeros [G, N] uint8, nibble order 0,4,1,5,2,6,3,7.
 * Replaces _unpack_awq_qweight / _unpack_awq_qzeros
 * (py/unified_llm_w4a16/llama3_8b_w4a16_model.py:325-358). */
hm_status hm_awq_unpack(const int32_t *packed, int64_t rows, int64_t cols8, uint8_t *out);

/* GPTQ qweight [rows8, cols] int32 -> out [8 * rows8, cols] uint8: nibble k of
 * word (r, c) is row 8 r + k, column c (sequential order along the input
 * dimension). Restates _unpack_gptq_qweight + _unpack_packed_out_in2_to_in_out
 * (py/unified_llm_w4a16/llama3_8b_w4a16_model.py:361-378, :398-407). Host memory. */
hm_status hm_gptq_unpack(const int32_t *packed, int64_t rows8, int64_t cols, uint8_t *out);

/* GPTQ qzeros [groups, cols8] int32 -> out [groups, 8 * cols8] uint8: nibble k
 * of word (g, j) is column 8 j + k; add_one adds the 1 that GPTQ checkpoints
 * subtract when storing (zeros then range 1..16; the engine keeps the zero as a
 * byte). Restates _unpack_gptq_qzeros (llama3_8b_w4a16_model.py:381-395)
 * without its transpose (the engine's zeros are [K / group, N]). Host memory. */
hm_status hm_gptq_unpack_zeros(const int32_t *packed, int64_t groups, int64_t cols8, int32_t add_one, uint8_t *out);

/* ---------------------------------------------------------------------------
 * Repacked weights on the device (CDNA4 strip layout). Created once at load
 * time; the forward entry points read only this layout.
 * ------------------------------------------------------------------------- */
typedef struct hm_weights hm_weights;

/* From a reference-packed matrix already in device memory: `tiles` holds the
 * packed [packed_k, packed_n] matrix (hm_packed_bytes(packed_k, packed_n) bytes).
 * The repacked matrix is its leading [K, N] block (K%128 == 0, N%16 == 0).
 * Group size is 128 (the tile height). Replaces the packed_params_ buffer that
 * QuantizedLinearImpl owns (unified_llm_w4a16.cpp:854) as the kernels' input. */
hm_status hm_weights_from_tiles(const uint8_t *tiles, int64_t packed_k, int64_t packed_n, int64_t K, int64_t N,
                                hm_dtype dtype, void *stream, hm_weights **out);

/* From logical device tensors: q [K, N] uint8 (0..15), scales [K/group, N]
 * (dtype bits), zeros [K/group, N] uint8 (0..15), row-major. group in
 * {32, 64, 128}. Covers what the 4352-byte layout cannot hold: a tile stores one
 * scale/zero row per 128 K rows, so group 64 or 32 weights need this entry. */
hm_status hm_weights_from_logical(const uint8_t *q, const uint16_t *scales, const uint8_t *zeros, int64_t K,
                                  int64_t N, int64_t group, hm_dtype dtype, void *stream, hm_weights **out);

/* Zero points. The engine reads every zero point as an unsigned byte and accepts 0..16 (int4 zeros, and 1..16 for
 * GPTQ checkpoints that store z - 1); the create calls above and below return HM_INVALID_ARGUMENT for any other
 * value, after waiting for the repack on `stream` (they are load-time calls). The reference's GPU GEMV reads tile
 * zeros as int8 (src/hipkernels/w4a16_gemv_packed.cu:86-87), its CPU GEMV as uint8
 * (src/cpu_avx_kernels/w4a16_gemv_avx_packed.cpp:122-124); both agree with this on 0..16. */

/* A gate_up matrix as the reference stores it for the fused FFN: packed [packed_k, 2 stored] with the gate and up
 * columns of `stored` channels in `layout` order (HM_GATE_UP_INTERLEAVED: per 64 channels 64 gate columns then 64
 * up columns; HM_GATE_UP_BLOCKED: all gate columns, then all up columns), kernels/gpu/include/heteromega/
 * gpu_ffn.hpp:43-71 (FfnSliceWeights.gate_up), as read by the FUSE_ACT GEMM (src/hipkernels/w4a16_gemm_packed.cu:
 * 549-578). The result is the fused gate_up of channels [0, channels) over the leading K rows (K % 128 == 0,
 * channels % 16 == 0, channels <= stored, stored % 64 == 0); it runs through hm_linear_swiglu, not hm_linear. */
hm_status hm_weights_from_gate_up_tiles(const uint8_t *gate_up, int64_t packed_k, int64_t stored, int64_t K, int64_t channels,
                                        int32_t layout, hm_dtype dtype, void *stream, hm_weights **out);

/* The dequantized weights round((q - z) * s) in the activation type (one rounding of the exact product), as
 * QuantizedLinearImpl::dequantize_packed returns them (src/unified_llm_w4a16_hetero/unified_llm_w4a16.cpp:710-790):
 * transposed != 0 writes [N, K] (the reference's [out, in] orientation, its transpose at :789), else [K, N]; ld_out is
 * the leading dimension of `out` (transposed: a multiple of 8, 16-byte aligned). A fused gate_up matrix comes out
 * with its columns alternating gate / up per 16 channels. */
hm_status hm_weights_dequantize(const hm_weights *w, void *out, int64_t ld_out, int32_t transposed, void *stream);

/* Writes the logical tensors back (device pointers, same shapes as above).
 * Round trip from_logical -> to_logical is bit-exact. */
hm_status hm_weights_to_logical(const hm_weights *w, uint8_t *q, uint16_t *scales, uint8_t *zeros, void *stream);

hm_status hm_weights_info(const hm_weights *w, int64_t *K, int64_t *N, int64_t *group, int32_t *dtype,
                          int64_t *device_bytes);

/* Device pointers of the two planes (nibble tiles, scale/zero records) and their sizes. */
hm_status hm_weights_planes(const hm_weights *w, const void **quant, int64_t *quant_bytes, const void **meta,
                            int64_t *meta_bytes);

hm_status hm_weights_destroy(hm_weights *w);

/* Columns of `count` matrices with the same K, group and dtype side by side in one new matrix
 * [K, N_0 + N_1 + ...], so projections that read the same input (an attention block's Q, K and V) run as one
 * hm_linear launch whose output holds their columns in order. The reference reads the input of Q, K and V
 * three times and reuses only its prepared GEMM layout (GemmInputReuse, kernels/gpu/include/heteromega/
 * gpu_ffn.hpp:117-127; QuantizedLinear calls at src/unified_llm_w4a16_hetero/unified_llm_w4a16.cpp:2795).
 * The parts are copied (device to device on `stream`) and stay owned by the caller. */
hm_status hm_weights_concat(const hm_weights *const *parts, int32_t count, void *stream, hm_weights **out);

/* ---------------------------------------------------------------------------
 * One projection: y[M, n] = x[M, k] @ W[:k, :n].
 * Replaces hipkernels::w4a16_gemv_fused_packed / w4a16_gemm_fused_packed[_tiles]
 * (include/hipkernels/w4a16_gemm_packed.hpp:38-52) and heteromega::gemv_w4a16,
 * gemm_w4a16, packed_linear (kernels/gpu/include/heteromega/gpu_ffn.hpp:99-199).
 * x and y are row-major with leading dimensions ldx, ldy (elements). The
 * block is the leading k x n of the repacked matrix (k%128 == 0, n%16 == 0).
 * col_begin selects columns [col_begin, col_begin + n) instead (the
 * reference GEMV's start_col, w4a16_gemv_packed.cu:178-194); it must be a
 * multiple of 16. No input padding to 128 rows is needed.
 * ------------------------------------------------------------------------- */
size_t hm_linear_workspace_bytes(const hm_weights *w, int64_t M, int64_t k, int64_t n);
hm_status hm_linear(const hm_weights *w, void *y, int64_t ldy, const void *x, int64_t ldx, int64_t M, int64_t k,
                    int64_t n, int64_t col_begin, void *workspace, size_t workspace_bytes, void *stream);

/* SwiGLU projection on a fused gate_up matrix (hm_weights_from_gate_up_tiles):
 *   act[M, ch_end - ch_begin] = SiLU(x[M, k] Wg[:k, ch]) * (x Wu[:k, ch]), fp32 sums, one rounding.
 * Replaces hipkernels::w4a16_gemm_fused_packed_tiles with fuse_activation = true
 * (include/hipkernels/w4a16_gemm_packed.hpp:41-49, src/hipkernels/w4a16_gemm_packed.cu:549-578, which rounds gate and
 * up to bf16 first). Channels are multiples of 16 (M <= 16) or of 64 (M > 16). */
size_t hm_linear_swiglu_workspace_bytes(const hm_weights *w, int64_t M, int64_t k, int64_t channels);
hm_status hm_linear_swiglu(const hm_weights *w, void *act, int64_t ld_act, const void *x, int64_t ldx, int64_t M, int64_t k, int64_t ch_begin,
                           int64_t ch_end, void *workspace, size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------
 * K split of one projection over two packed matrices (the pre-saved K-split
 * pair, W0 = rows [0, k0) and W1 = rows [k0, k0 + k1) of W):
 *   y[M, n] = round(round(x[:, :k0] W0[:, :n]) + round(x[:, k0:k0+k1] W1[:, :n])).
 * Replaces hetero_matmul_out_gemm_packed_K and hetero_matmul_out_gemv_packed_K
 * (src/unified_llm_w4a16_hetero/hetero_compute.cpp:282-447 and 633-805), which
 * give the K0 share to the NPU or, GPU-only, run both shares and sum their
 * rounded outputs (output_2d.add_(temp_output), :437 and :800). Both shares run
 * on the GPU here. At M = 1 (same group size) both shares run in one GEMV
 * launch, each writing an fp32 partial that the split sum rounds and adds;
 * otherwise share 0 writes y and share 1 adds into y in its epilogue (no
 * temporary output, no extra pass). k0, k1 multiples of 128, n of 16; the two
 * matrices have the same activation type. M <= 16 uses the GEMV.
 * ------------------------------------------------------------------------- */
size_t hm_linear_k_split_workspace_bytes(const hm_weights *w0, const hm_weights *w1, int64_t M, int64_t k0, int64_t k1,
                                         int64_t n);
hm_status hm_linear_k_split(const hm_weights *w0, const hm_weights *w1, void *y, int64_t ldy, const void *x, int64_t ldx,
                            int64_t M, int64_t k0, int64_t k1, int64_t n, void *workspace, size_t workspace_bytes,
                            void *stream);

/* ---------------------------------------------------------------------------
 * One SwiGLU FFN layer: y = (SiLU(x Wg) * (x Wu)) Wd over the channels
 * [ch_begin, ch_end) of the layer (the row/column partition: the GPU share of
 * the reference's channel split, kernels/gpu/src/gpu_ffn.cpp:77-119 and
 * src/unified_llm_w4a16_hetero/merged_ffn.cpp:235-236). Channel bounds are
 * multiples of 128. SiLU(g)*u is computed in fp32 and rounded once to the
 * activation dtype (kernels/gpu/src/silu_mul.cu:10-30 semantics).
 * ------------------------------------------------------------------------- */
typedef struct hm_ffn hm_ffn;

/* From reference-packed device matrices gate [H, I], up [H, I], down [I, H]
 * (replaces GpuFfnModel::add_layer, kernels/gpu/src/gpu_ffn.cpp:122-130). */
hm_status hm_ffn_from_tiles(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int64_t hidden,
                            int64_t inter, hm_dtype dtype, void *stream, hm_ffn **out);

/* Same from matrices stored padded: gate / up packed as [packed_hidden,
 * packed_inter], down as [packed_inter, packed_hidden] (the reference's
 * padPackedWeights rounds both up to multiples of 2048 with zeros,
 * llama3_8b_w4a16_model.py:546-608); the layer is their leading block. */
hm_status hm_ffn_from_tiles_padded(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int64_t hidden,
                                   int64_t inter, int64_t packed_hidden, int64_t packed_inter, hm_dtype dtype,
                                   void *stream, hm_ffn **out);

/* From the reference's fused-FFN tensors: gate_up packed [hidden, 2 stored] in `layout` order (see
 * hm_weights_from_gate_up_tiles) and down packed [stored, hidden]; the layer is channels [0, inter) of them
 * (inter % 128 == 0, inter <= stored: the reference's FfnSliceWeights with its prefix(),
 * kernels/gpu/include/heteromega/gpu_ffn.hpp:55-71, and the inputs of heteromega::gemm_w4a16_ffn,
 * kernels/gpu/src/gemm_w4a16.cu:463-502). */
hm_status hm_ffn_from_gate_up_tiles(const uint8_t *gate_up, const uint8_t *down, int64_t hidden, int64_t inter, int64_t stored,
                                    int32_t layout, hm_dtype dtype, void *stream, hm_ffn **out);

/* From logical device tensors (see hm_weights_from_logical), any group in {32, 64, 128}:
 * gate/up q [H, I], s/z [H/group, I]; down q [I, H], s/z [I/group, H]. */
hm_status hm_ffn_from_logical(const uint8_t *gate_q, const uint16_t *gate_s, const uint8_t *gate_z,
                              const uint8_t *up_q, const uint16_t *up_s, const uint8_t *up_z,
                              const uint8_t *down_q, const uint16_t *down_s, const uint8_t *down_z, int64_t hidden,
                              int64_t inter, int64_t group, hm_dtype dtype, void *stream, hm_ffn **out);

hm_status hm_ffn_info(const hm_ffn *f, int64_t *hidden, int64_t *inter, int64_t *group, int32_t *dtype);
hm_status hm_ffn_destroy(hm_ffn *f);

/* Workspace for hm_ffn_forward with up to max_m rows (the SwiGLU activation
 * [max_m, I], the one-row gate_up's fp32 sums of strip pairs that two of its
 * workgroups share (about 3.2 I bytes), and split-K partials: the decode GEMV's for
 * up to 16 rows, and 32 MiB from 17 rows, the most a small GEMM grid's K split
 * writes). Nothing in it has to start at zero. Replaces GpuFfnBuffers
 * (gpu_ffn.hpp:172-180). */
size_t hm_ffn_workspace_bytes(const hm_ffn *f, int64_t max_m);

/* y [M, H] (ldy) = FFN over channels [ch_begin, ch_end) of x [M, H] (ldx). */
hm_status hm_ffn_forward(const hm_ffn *f, void *y, int64_t ldy, const void *x, int64_t ldx, int64_t M,
                         int64_t ch_begin, int64_t ch_end, void *workspace, size_t workspace_bytes, void *stream);

/* hm_ffn_forward without a workspace argument: the scratch (SwiGLU activation and split partials) is a static
 * device array of HM_STATIC_SCRATCH_BYTES that the library holds on each GPU it runs on until the process ends.
 * No counterpart in the reference: it is for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc); the call itself allocates nothing. The scratch must hold
 * hm_ffn_workspace_bytes(f, M): decode rows (M <= 16) of the Llama-3-8B and Qwen2.5-14B layers need about
 * 3.3 MB; prefill rows (M > 16) need more than the scratch and return HM_WORKSPACE_TOO_SMALL, as does any
 * request above HM_STATIC_SCRATCH_BYTES. Calls on one GPU share its scratch: calls that overlap in time on one
 * GPU (different streams or threads) race; calls on one stream are ordered and safe. */
#define HM_STATIC_SCRATCH_BYTES (8u << 20)
hm_status hm_ffn_forward_static(const hm_ffn *f, void *y, int64_t ldy, const void *x, int64_t ldx, int64_t M, int64_t ch_begin,
                                int64_t ch_end, void *stream);

/* The first half alone: act [M, ch_end - ch_begin] (ld_act) = SiLU(x Wg) * (x Wu). */
hm_status hm_ffn_gate_up(const hm_ffn *f, void *act, int64_t ld_act, const void *x, int64_t ldx, int64_t M,
                         int64_t ch_begin, int64_t ch_end, void *workspace, size_t workspace_bytes, void *stream);

/* The second half alone: y [M, H] = act [M, ch_end - ch_begin] @ Wd[ch_begin:ch_end, :]. */
hm_status hm_ffn_down(const hm_ffn *f, void *y, int64_t ldy, const void *act, int64_t ld_act, int64_t M,
                      int64_t ch_begin, int64_t ch_end, void *workspace, size_t workspace_bytes, void *stream);

/* Workspace for hm_ffn_block_forward with up to max_m rows. */
size_t hm_ffn_block_workspace_bytes(const hm_ffn *f, int64_t max_m);

/* One pre-norm FFN block of a layer stack, in place: x [M, H] (ldx) += FFN(RMSNorm(x) * norm_weight), eps as in
 * hm_rmsnorm. This is the model's FFN block with the layer-boundary norm and residual add
 * (src/unified_llm_w4a16_hetero/unified_llm_w4a16.cpp:2867-2892 with kernels/gpu/src/residual_norm.cu:25-98).
 * One row (H <= 8192) runs as two launches: the gate_up GEMV normalizes x while staging it and the down GEMV
 * adds its rounded output into x. Other M run hm_rmsnorm, the gate_up projection and a down projection that adds
 * its rounded output into x (x = round(x + round(act Wd))). Either way the result equals hm_rmsnorm, hm_ffn_forward
 * and hm_residual_add2 bit for bit. Needs hm_ffn_block_workspace_bytes(f, M) bytes of workspace. */
hm_status hm_ffn_block_forward(const hm_ffn *f, void *x, int64_t ldx, const void *norm_weight, float eps, int64_t M,
                               void *workspace, size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------
 * Elementwise operators next to the FFN.
 * ------------------------------------------------------------------------- */

/* act[m, j] = SiLU(gate[m, j]) * up[m, j], fp32 math, one rounding. gate and up
 * are columns of gate_up [rows, 2n] in `layout` order. Replaces heteromega::silu_mul
 * (kernels/gpu/src/silu_mul.cu:34-57). */
hm_status hm_silu_mul(const void *gate_up, int64_t ld_in, void *act, int64_t ld_out, int64_t rows, int64_t n,
                      int32_t layout, hm_dtype dtype, void *stream);

/* out = x * rsqrt(mean(x^2) + eps) * weight per row (fp32 math, one rounding).
 * Replaces launch_rmsnorm (src/hipkernels/rmsnorm.cu:65-103, non-gemma). */
hm_status hm_rmsnorm(void *out, int64_t ld_out, const void *x, int64_t ldx, const void *weight, int64_t rows,
                     int64_t cols, float eps, hm_dtype dtype, void *stream);

/* x += a + b per element (a or b may be NULL), fp32 math, one rounding.
 * Replaces heteromega::residual_add2 (kernels/gpu/src/residual_add.cu:9-73). */
hm_status hm_residual_add2(void *x, int64_t ldx, const void *a, int64_t lda, const void *b, int64_t ldb,
                           int64_t rows, int64_t cols, hm_dtype dtype, void *stream);

/* One dispatch between FFN layers: x += y (residual), then normed = RMSNorm(x) * weight.
 * The layer-boundary fusion of kernels/gpu/src/residual_norm.cu:25-98 without its GEMM input prep. */
hm_status hm_residual_rmsnorm(void *x, int64_t ldx, const void *y, int64_t ldy, const void *weight, void *normed,
                              int64_t ld_normed, int64_t rows, int64_t cols, float eps, hm_dtype dtype, void *stream);

/* The same with two addends: x = round((x + a) + b) (b may be NULL), then normed = RMSNorm(x) * weight; with a
 * NULL, x is left as it is and only the norm runs. Replaces heteromega::residual_norm_bf16
 * (kernels/gpu/include/heteromega/gpu_ffn.hpp:136-141, kernels/gpu/src/residual_norm.cu:25-106) without its
 * prepared GEMM input: the engine's GEMM reads its input rows from memory. */
hm_status hm_residual2_rmsnorm(void *x, int64_t ldx, const void *a, int64_t lda, const void *b, int64_t ldb, const void *weight,
                               void *normed, int64_t ld_normed, int64_t rows, int64_t cols, float eps, hm_dtype dtype,
                               void *stream);

/* x += a + b per element with each partial either in x's type (a_fp32 / b_fp32 = 0) or fp32 (1): the partials are
 * added first, then the residual, fp32 math, one rounding. Replaces heteromega::residual_add2 with fp32 partials
 * (kernels/gpu/include/heteromega/gpu_ffn.hpp:162-163, kernels/gpu/src/residual_add.cu:48-73). */
hm_status hm_residual_add2_mixed(void *x, int64_t ldx, const void *a, int64_t lda, int32_t a_fp32, const void *b,
                                 int64_t ldb, int32_t b_fp32, int64_t rows, int64_t cols, hm_dtype dtype, void *stream);

/* ---------------------------------------------------------------------------
 * Nonfinite scan (the merged FFN's failure check).
 * ------------------------------------------------------------------------- */

/* Columns between the checked ones of a sampled scan (include/heteromega/merged_ffn_contract.hpp:18). */
#define HM_FINITE_SAMPLE_STRIDE 64

/* Host memory: the least row-major index r * cols + c of an element of rows x cols 16-bit values (row stride ld)
 * whose exponent bits are all set (inf or NaN), checking every column (sampled = 0) or every
 * HM_FINITE_SAMPLE_STRIDE-th (sampled = 1); -1 when there is none or the arguments are invalid. Replaces
 * heteromega::find_nonfinite_bf16 with FiniteCheck::kFull / kSampled (merged_ffn_contract.hpp:13-39) and covers fp16. */
int64_t hm_find_nonfinite(const void *bits, int64_t rows, int64_t cols, int64_t ld, hm_dtype dtype, int32_t sampled);

/* The same scan of device memory, enqueued on `stream`: *first (a device int64) receives the index or -1. No
 * allocation and no host wait: an output can be checked where it lies, without a copy to the host. */
hm_status hm_find_nonfinite_device(const void *x, int64_t rows, int64_t cols, int64_t ld, hm_dtype dtype, int32_t sampled,
                                   int64_t *first, void *stream);

/* ---------------------------------------------------------------------------
 * Partition descriptor (host). The other device's share is [0, npu_channels),
 * the GPU's is [npu_channels, intermediate), as in npu/ffn/reference.py:121-151.
 * On this build every share runs on the GPU; npu_channels = 0 is the GPU-only case.
 * ------------------------------------------------------------------------- */

/* Checks 0 <= npu_channels <= intermediate and the alignment (reference.py:127-133). */
hm_status hm_partition_check(int64_t intermediate, int64_t npu_channels, int64_t alignment);

/* Rounds intermediate * ratio to the nearest multiple of alignment, ties up
 * (FFNPartition.from_ratio, reference.py:135-144). */
hm_status hm_partition_from_ratio(int64_t intermediate, double npu_ratio, int64_t alignment, int64_t *npu_channels);

/* ---------------------------------------------------------------------------
 * Split descriptors of the reference's hetero executor (host, no GPU needed to plan).
 * A projection's config entry is keyed by {forM, forK, forN, layer_id, chunk_id} (NPUKey) and holds the other
 * device's shares {npuM, npuK, npuN, cpuN, cpuThreads, config} plus a split_type derived from the shapes
 * (NPUValue; include/unified_llm_w4a16_hetero/npuSetup.hpp:93-109). On this build every share runs on the GPU:
 * hm_linear_split executes the split an entry describes as GPU launches, so a config table written for the
 * reference drives the same partition here.
 * ------------------------------------------------------------------------- */
typedef struct hm_split_desc {
    int32_t hw_idx, inst_idx; /* the other device's contexts in the reference; unused here (-1) */
    int32_t npuM, npuK, npuN, cpuN, cpuThreads, config;
    int32_t split_type; /* > 0: K split at K0 = split_type; -1: M split; -2: N split; 0: GEMV column shares */
} hm_split_desc;

/* split_type of a kernel config (src/unified_llm_w4a16_hetero/npuSetup.cpp:1283-1291): npuK when forK != npuK
 * (a K split, taking precedence), -1 when only M differs, -2 when N differs, -1 otherwise. */
int32_t hm_split_type(int32_t forM, int32_t forK, int32_t forN, int32_t npuM, int32_t npuK, int32_t npuN);

/* layer_id of a layer name: qkv 8, q 1, k 2, v 3, o 4, gate 5, up 6, down 7, anything else 0
 * (get_layer_id, npuSetup.cpp:635-653). */
int32_t hm_layer_id(const char *layer_type);

typedef struct hm_split_table hm_split_table; /* config_map (npuSetup.hpp:114) */
hm_status hm_split_table_create(hm_split_table **out);
hm_status hm_split_table_destroy(hm_split_table *t);
/* A GEMM entry as the config loader makes it (npuSetup.cpp:1283-1467): split_type by hm_split_type, cpuN 0,
 * cpuThreads 1. Rejected: negative or zero sizes, npuK > forK (a K share past the projection), K splits whose shares
 * are not multiples of 128. Entries with npuM == 0 are GPU-only in the reference and are not stored (returns HM_OK
 * and *stored = 0). */
hm_status hm_split_table_add_gemm(hm_split_table *t, int32_t forM, int32_t forK, int32_t forN, int32_t layer_id, int32_t chunk_id,
                                  int32_t npuM, int32_t npuK, int32_t npuN, int32_t config, int32_t *stored);
/* A GEMV entry (M = 1) with column shares (npuSetup.cpp:1763: {-1, -1, npuM, npuK, 0, cpuN, threads, config, 0}). */
hm_status hm_split_table_add_gemv(hm_split_table *t, int32_t forK, int32_t forN, int32_t layer_id, int32_t chunk_id, int32_t npuN, int32_t cpuN,
                                  int32_t cpuThreads, int32_t config);
/* Exact-key lookup (find_config_entry, src/unified_llm_w4a16_hetero/hetero_compute.cpp:98-106): HM_OK and *out, or
 * HM_INVALID_ARGUMENT when no entry has this key (chunk -1 is not a wildcard). */
hm_status hm_split_table_find(const hm_split_table *t, int32_t M, int32_t K, int32_t N, int32_t layer_id, int32_t chunk_id, hm_split_desc *out);
int64_t hm_split_table_size(const hm_split_table *t);

/* y [M, N] = x [M, K] @ W, split as `d` describes, every share on the GPU, in the order the reference launches them:
 *   d NULL: one launch (the reference's GPU default path).
 *   split_type > 0 (K split, hetero_matmul_out_gem{m,v}_packed_K, hetero_compute.cpp:282-447, 633-805): w0 holds rows
 *     [0, K0) and w1 rows [K0, K) with K0 = split_type; y = round(round(x0 W0) + round(x1 W1)) (hm_linear_k_split).
 *   M == 1 otherwise (hetero_matmul_out_gemv_packed_M, :497-560): columns [0, npuN), [npuN, npuN + cpuN) and the rest,
 *     with both shares dropped when npuN + cpuN > N and cpuN dropped unless a multiple of 64, as the reference does.
 *     (The reference sizes the GPU's columns before it drops such a cpuN, :516-538, and leaves those columns
 *     unwritten; here the GPU's share covers them.)
 *   split_type -1 (M split, :189-259): rows [0, M - npuM) and [M - npuM, M) (npuM clamped to M).
 *   split_type -2 (N split): columns [0, npuN) and [npuN, N).
 * Column and row shares of one projection give the bits of the unsplit launch where the launches do not split K
 * differently (the GEMM splits K only for grids under two workgroups per CU). */
size_t hm_linear_split_workspace_bytes(const hm_split_desc *d, const hm_weights *w0, const hm_weights *w1, int64_t M, int64_t K, int64_t N);
hm_status hm_linear_split(const hm_split_desc *d, const hm_weights *w0, const hm_weights *w1, void *y, int64_t ldy, const void *x, int64_t ldx,
                          int64_t M, int64_t K, int64_t N, void *workspace, size_t workspace_bytes, void *stream);

/* The merged-FFN deployment contract's shape and partition rules (MergedFfnConfig::load and its buffer sizes,
 * include/heteromega/merged_ffn_contract.hpp:41-127): m a positive multiple of 512, hidden and intermediate of 128,
 * npu_channels a positive multiple of 256 below intermediate and at most 8192. Sizes: activations m * hidden * 2,
 * intermediate m * npu_channels * 2, weights (hidden / 128) * (intermediate / 64) * 4352 bytes, each product checked
 * for overflow (checked_product). The artifact fields (xclbin hashes, layouts, fifo depths) describe NPU binaries and
 * have no counterpart here. */
hm_status hm_merged_ffn_check(int64_t m, int64_t hidden, int64_t intermediate, int64_t npu_channels, uint64_t *activation_bytes,
                              uint64_t *intermediate_bytes, uint64_t *weight_bytes);
/* MergedFfnConfig::supports: rows > 1 and the exact shape of the contract. */
int32_t hm_merged_ffn_supports(int64_t m, int64_t hidden, int64_t intermediate, int64_t rows, int64_t h, int64_t inter);

#ifdef __cplusplus
}
#endif

#endif /* HM_W4A16_H */

/*
 * eif_quantize_bitnet.h -- ternary (BitNet b1.58) kernel API, served by libbitllm_hip.so on one MI355X.
 *
 * Every declaration below keeps the exact symbol name, argument order and types of the reference header
 * include/eif_quantize_bitnet.h of tevfik/bitllm.c, so a C99 caller (src/eif_tinyllm.c, src/eif_qwen35.c) links
 * against this library instead of src/eif_quantize_bitnet.c without a source change. The line after each
 * declaration names the reference declaration it replaces.
 *
 * Conventions kept from the reference:
 *   - all pointers are caller-owned HOST memory; calls are synchronous and return when outputs are written;
 *   - scales == NULL means 1.0, bias == NULL means 0.0, invalid sizes are a silent no-op;
 *   - 2-bit code format: column c lives in byte c>>2 at bits 2*(c&3); 01 = +1, 10 = -1, 00 and 11 = 0.
 * What differs: the arithmetic runs as HIP kernels on the GPU. Weight buffers (and the block scales of
 * eif_matmul_bitnet_block_f32) are uploaded once and kept resident, keyed by (host pointer, size); call
 * eif_hip_forget_host_weights() after rewriting such a buffer in place. Without a usable GPU the compute entry points print a diagnostic and abort(): there is no CPU path.
 */
#ifndef EIF_QUANTIZE_BITNET_H
#define EIF_QUANTIZE_BITNET_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Decode one 2-bit code (pos 0..3) of a packed byte to {-1,0,+1}.   ref: include/eif_quantize_bitnet.h:32 */
int8_t eif_unpack_ternary(uint8_t byte, int pos);

/* Pack count values in {-1,0,+1} into (count+3)/4 bytes.            ref: include/eif_quantize_bitnet.h:41 */
size_t eif_pack_ternary(const int8_t *ternary, uint8_t *packed, size_t count);

/* Base-3 pack: 5 values per byte as sum(code_i * 3^i).              ref: include/eif_quantize_bitnet.h:54 */
size_t eif_pack_ternary_dense(const int8_t *ternary, uint8_t *packed, size_t count);

/* y[r] = scales[r] * sum_c w[r,c] * x[c] + bias[r]; FP32 activations. ref: include/eif_quantize_bitnet.h:72-78 */
void eif_matmul_bitnet_f32(const uint8_t *weights, const float *scales, const float *input, const float *bias,
                           float *output, int rows, int cols);

/* As eif_matmul_bitnet_f32 with base-3 packed rows of (cols+4)/5 bytes. ref: include/eif_quantize_bitnet.h:94-100 */
void eif_matmul_bitnet_dense_f32(const uint8_t *weights, const float *scales, const float *input,
                                 const float *bias, float *output, int rows, int cols);

/* INT8 in, INT8 out: isum = bias[r] + sum w*x (int32), y = clamp(round_away(isum * sw*sin/sout)).
 *                                                                   ref: include/eif_quantize_bitnet.h:120-128 */
void eif_matmul_bitnet_int8(const uint8_t *weights, float scale_w, const int8_t *input, float scale_in,
                            const int32_t *bias, int8_t *output, float scale_out, int rows, int cols);

/* Gate and up projections of one FFN in one call (per-row scales, no bias).
 *                                                                   ref: include/eif_quantize_bitnet.h:134-137 */
void eif_matmul_bitnet_f32_w1w3(float *out_w1, float *out_w3, const uint8_t *w1, const uint8_t *w3,
                                const float *scale_w1, const float *scale_w3, const float *input, int hidden_dim,
                                int dim);

/* Per-vector absmax INT8: scale = amax*(1/127), q = trunc(x*(127/amax) +- 0.5) clamped to [-128,127];
 * amax < 1e-12 gives q = 0 and scale 1.                              ref: include/eif_quantize_bitnet.h:151-154 */
void eif_quantize_activation_i8(const float *x_f32, int8_t *x_i8, float *out_scale, int n);

/* INT8 activations x ternary, exact int32 row sums: y = isum * (scales[r]*scale_in) + bias[r].
 *                                                                   ref: include/eif_quantize_bitnet.h:171-178 */
void eif_matmul_bitnet_i8xternary_f32(const uint8_t *weights, const float *scales, const int8_t *input_i8,
                                      float scale_in, const float *bias, float *output, int rows, int cols);

/* eif_quantize_activation_i8 followed by eif_matmul_bitnet_i8xternary_f32.
 *                                                                   ref: include/eif_quantize_bitnet.h:186-192 */
void eif_matmul_bitnet_act_quant_f32(const uint8_t *weights, const float *scales, const float *input_f32,
                                     const float *bias, float *output, int rows, int cols);

/* Group-scaled ternary GEMV, FP32 activations: y[r] = sum_b block_scales[r*nb+b] * sum_{c in b} w*x + bias[r],
 * nb = ceil(cols/block_size), block_size <= 0 means 64.               ref: include/eif_quantize_bitnet.h:209-216 */
void eif_matmul_bitnet_block_f32(const uint8_t *weights, const float *block_scales, int block_size,
                                 const float *input, const float *bias, float *output, int rows, int cols);

/* Reorder packed rows so each 4-row block stores byte g of its rows contiguously; tail rows are copied.
 * Returns the bytes written (rows * ((cols+3)/4)), 0 on invalid input. ref: include/eif_quantize_bitnet.h:230-233 */
size_t eif_interleave_weights_4rows(const uint8_t *src_row_major, uint8_t *dst_interleaved, int rows, int cols);

/* eif_matmul_bitnet_f32 on the 4-row interleaved layout. Every column is used (no 4096-column cap).
 *                                                                   ref: include/eif_quantize_bitnet.h:240-246 */
void eif_matmul_bitnet_tmac_interleaved_f32(const uint8_t *interleaved_weights, const float *scales,
                                           const float *input, const float *bias, float *output, int rows,
                                           int cols);

/* Largest power of two <= 1024 dividing n.                          ref: include/eif_quantize_bitnet.h:252 */
int eif_hadamard_block_size(int n);

/* Largest multiple of 32 <= max_group dividing n; 0 = one scale per row. ref: include/eif_quantize_bitnet.h:258 */
int eif_bitnet_group_size(int n, int max_group);

/* In place x <- FWHT_block(x * signs) * (1/sqrt(block)), butterflies h = 1, 2, ..., block/2. signs may be NULL.
 * No-op unless x != NULL, block > 0 and n % block == 0. A block that is not a power of two is rejected (no-op)
 * instead of writing out of range.                                  ref: include/eif_quantize_bitnet.h:272 */
void eif_hadamard_rotate_f32(float *x, const float *signs, int n, int block);

#ifdef __cplusplus
}
#endif

#endif /* EIF_QUANTIZE_BITNET_H */

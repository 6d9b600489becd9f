/*
 * eif_quant_linear.h -- the INT8 / INT4 row-scaled GEMVs that the reference engines call but keep in their
 * own translation units, exported here so a drop-in needs only a few-line edit at the call sites.
 *
 *   tinyllm_matmul_int8_rowscale  keeps the exported signature of include/eif_tinyllm.h:384-385 (note: in_dim
 *                                 (cols) comes before out_dim (rows)); body src/eif_tinyllm.c:1651-1721.
 *   eif_int4_gemv_f32             replaces the file-static int4_gemv of src/eif_qwen35.c:293-352 (call sites
 *                                 src/eif_qwen35.c:436-437 via linear_gemv, :927-929 for a tied INT4 head).
 *   eif_int8_gemv_f32             replaces the file-static int8_gemv of src/eif_qwen35.c:384-419 (LM head :925).
 *
 * Host pointers, synchronous, FP32 activations (the reference x86 semantics); weights are kept resident on
 * the GPU keyed by (host pointer, size). INT4 rows hold (cols+1)/2 bytes, even column in the HIGH nibble,
 * value = nibble - 8 (producer src/eif_qwen35_gguf.c:249-253).
 */
#ifndef EIF_QUANT_LINEAR_H
#define EIF_QUANT_LINEAR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* y[r] = scales[r] * sum_c w[r*cols+c] * x[c]; scales may be NULL (1.0).   ref: include/eif_tinyllm.h:384-385 */
void tinyllm_matmul_int8_rowscale(float *y, const int8_t *w, const float *x, int in_dim, int out_dim,
                                  const float *scales);

/* out[r] = sc[r] * sum_c (nibble(r,c) - 8) * x[c].                          ref: src/eif_qwen35.c:293-352 */
void eif_int4_gemv_f32(float *out, const uint8_t *W, const float *sc, const float *x, int rows, int cols);

/* out[r] = sc[r] * sum_c W[r,c] * x[c].                                     ref: src/eif_qwen35.c:384-419 */
void eif_int8_gemv_f32(float *out, const int8_t *W, const float *sc, const float *x, int rows, int cols);

#ifdef __cplusplus
}
#endif

#endif /* EIF_QUANT_LINEAR_H */

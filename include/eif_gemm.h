/*
 * eif_gemm.h -- FP32 NT GEMM and row softmax, served by libbitllm_hip.so on one MI355X.
 *
 * Same symbols, argument order and types as the reference header include/eif_gemm.h of tevfik/bitllm.c
 * (the prefill GEMM that src/eif_qwen35.c:1034-1065 calls). Pointers are caller-owned host memory and the calls
 * are synchronous; the arithmetic runs on the GPU. Without a usable GPU the calls abort with a diagnostic.
 */
#ifndef EIF_GEMM_H
#define EIF_GEMM_H

#ifdef __cplusplus
extern "C" {
#endif

/* Epilogue selectors.                                               ref: include/eif_gemm.h:13-14 */
#define EIF_GEMM_ACT_NONE 0
#define EIF_GEMM_ACT_GELU_TANH 1

/* C[M,N] = act(A[M,K] W[N,K]^T + bias) (accumulate == 0), or C += A W^T + bias (accumulate != 0, act NONE).
 * Contiguous row-major operands; bias may be NULL.                  ref: include/eif_gemm.h:22-23 */
void eif_gemm_f32_nt(const float *A, const float *W, const float *bias, float *C, int M, int N, int K, int act,
                     int accumulate);

/* As eif_gemm_f32_nt with row strides (in floats) lda, ldw, ldc.     ref: include/eif_gemm.h:26-27 */
void eif_gemm_f32_nt_ld(const float *A, int lda, const float *W, int ldw, const float *bias, float *C, int ldc,
                        int M, int N, int K, int act, int accumulate);

/* S[r, :cols] <- softmax(scale * S[r, :cols]) in place, rows ld floats apart.  ref: include/eif_gemm.h:30 */
void eif_softmax_rows_f32(float *S, int rows, int cols, int ld, float scale);

#ifdef __cplusplus
}
#endif

#endif /* EIF_GEMM_H */

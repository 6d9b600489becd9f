/*
 * oracle.h -- declarations of the CPU oracle (oracle.c). TEST INFRASTRUCTURE ONLY: loaded by tests/, smoke()
 * and the CPU-baseline leg of bench.py, never by the product library.
 */
#ifndef BITLLM_ORACLE_H
#define BITLLM_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
int8_t orc_unpack_ternary(uint8_t byte, int pos);
size_t orc_pack_ternary(const int8_t *v, uint8_t *packed, size_t count);
size_t orc_pack_ternary_dense(const int8_t *v, uint8_t *packed, size_t count);
int orc_hadamard_block_size(int n);
int orc_bitnet_group_size(int n, int max_group);
float orc_wht_norm_exact(int block);
float orc_wht_norm_fastmath(int block);
int orc_hadamard_rotate(float *x, const float *signs, int n, int block, float norm);
void orc_quantize_activation_i8(const float *x, int8_t *q, float *out_scale, int n);
int orc_prep_rows(const float *x, int ldx, const float *signs, int M, int K, int wht_block, float norm, int8_t *xq, int ldq, float *xs, float *xrot, int ldr);
void orc_ternary_acc_i32(const uint8_t *w, const int8_t *xq, int ldq, int M, int rows, int cols, int group, int32_t *acc);
void orc_ternary_gemv_grouped(const uint8_t *w, const float *gscales, int group, const int8_t *xq, int ldq, const float *xs, const float *bias, float *y, int ldy, int M, int rows, int cols);
void orc_matmul_bitnet_i8xternary_f32(const uint8_t *w, const float *scales, const int8_t *xq, float scale_in, const float *bias, float *y, int rows, int cols);
void orc_ternary_gemv_rowscale(const uint8_t *w, const float *scales, const int8_t *xq, int ldq, const float *xs, const float *bias, float *y, int ldy, int M, int rows, int cols);
void orc_matmul_bitnet_act_quant_f32(const uint8_t *w, const float *scales, const float *x, const float *bias, float *y, int rows, int cols);
void orc_matmul_bitnet_int8(const uint8_t *w, float scale_w, const int8_t *x, float scale_in, const int32_t *bias, int8_t *y, float scale_out, int rows, int cols);
void orc_int8_acc_i32(const int8_t *w, const int8_t *xq, int ldq, int M, int rows, int cols, int32_t *acc);
void orc_int4_acc_i32(const uint8_t *w, const int8_t *xq, int ldq, int M, int rows, int cols, int32_t *acc);
void orc_int8_gemv_i8act(const int8_t *w, const float *scales, const int8_t *xq, int ldq, const float *xs, const float *bias, float *y, int ldy, int M, int rows, int cols);
void orc_int4_gemv_i8act(const uint8_t *w, const float *scales, const int8_t *xq, int ldq, const float *xs, const float *bias, float *y, int ldy, int M, int rows, int cols);
void orc_matmul_bitnet_f32(const uint8_t *w, const float *scales, const float *x, const float *bias, float *y, int rows, int cols);
void orc_matmul_bitnet_block_f32(const uint8_t *w, const float *bs, int block_size, const float *x, const float *bias, float *y, int rows, int cols);
void orc_matmul_bitnet_f32_w1w3(float *o1, float *o3, const uint8_t *w1, const uint8_t *w3, const float *s1, const float *s3, const float *x, int hidden, int dim);
void orc_matmul_bitnet_dense_f32(const uint8_t *w, const float *scales, const float *x, const float *bias, float *y, int rows, int cols);
size_t orc_interleave_weights_4rows(const uint8_t *src, uint8_t *dst, int rows, int cols);
void orc_matmul_bitnet_tmac_interleaved_f32(const uint8_t *il, const float *scales, const float *x, const float *bias, float *y, int rows, int cols);
void orc_int8_rowscale_f32(float *y, const int8_t *w, const float *x, int cols, int rows, const float *scales);
void orc_int4_gemv_f32(float *out, const uint8_t *w, const float *sc, const float *x, int rows, int cols);
void orc_quant_rows(const float *x, int ldx, int rows, int cols, int bits, uint8_t *dst, float *scales);
void orc_gguf_ternary_rows(int type, const uint8_t *src, int rows, int cols, uint8_t *codes, float *scales);
void orc_gemm_f32_nt_ld(const float *A, int lda, const float *W, int ldw, const float *bias, float *C, int ldc, int M, int N, int K, int act, int accumulate);
void orc_softmax_rows_f32(float *S, int rows, int cols, int ld, float scale);
int orc_num_threads(void);

/* One BitNet-b1.58 decoder step (decode_oracle.c). */
float orc_round_f16(float v);
#define ORC_LIN_INT8 0
#define ORC_LIN_F32 1
typedef struct orc_bitnet_cfg {
    int dim, hidden, n_layers, n_heads, n_kv_heads, head_dim, vocab, seq_len;
    float rope_theta, rms_eps, sub_eps;
    int wht_dim, wht_q, wht_hidden;            /* WHT blocks of the inputs of wq/wk/wv/w1/w3, wo, w2 (0: none) */
    float wht_norm_dim, wht_norm_q, wht_norm_hidden;
    int g_q, g_o, g_13, g_2;                   /* ternary groups of wq/wk/wv, wo, w1/w3, w2 */
} orc_bitnet_cfg;
typedef struct orc_bitnet_weights {            /* reference formats, per-layer arrays concatenated over layers */
    const int8_t *emb;                         /* [vocab, dim] */
    const float *emb_scale;                    /* [vocab] or NULL */
    const uint8_t *wq, *wk, *wv, *wo, *w1, *w3, *w2;
    const float *gq, *gk, *gv, *go, *g1, *g3, *g2;
    const float *rms_att, *rms_ffn, *rms_sub_att, *rms_sub_ffn, *rms_final;
    const float *signs_dim, *signs_q, *signs_hidden;
    const int8_t *wcls;                        /* [vocab, dim] */
    const float *wcls_scale;                   /* [vocab] */
} orc_bitnet_weights;
/* kcache / vcache: [n_layers, seq_len, kv_dim] floats. Returns 0, or -1 on bad arguments. */
int orc_bitnet_forward(const orc_bitnet_cfg *c, const orc_bitnet_weights *w, float *kcache, float *vcache, int token,
                       int pos, int mode, float *logits);
#ifdef __cplusplus
}
#endif
#endif

/*
 * eif_hip_decode.h -- BitNet-b1.58 decoder on one MI355X, built on the quantized-linear kernels of eif_hip.h.
 *
 * Replaces the token loop of the reference's tinyllm engine for the BitNet path: tinyllm_forward /
 * tinyllm_forward_embedding_ex (src/eif_tinyllm.c:371-857, :1502-1506) and its greedy sampler
 * tinyllm_sample_greedy (src/eif_tinyllm.c:1519-1530). One token step is 5 launches per layer plus 3:
 *   per layer: [RMSNorm + WHT + INT8] QKV GEMV | RoPE + fp16 KV append + attention over up to eight chunks of
 *              the positions per head, one share each |
 *              [shares combined + sub-RMSNorm + WHT + INT8] O GEMV + residual | [RMSNorm + WHT + INT8] gate/up GEMV |
 *              [SiLU(gate) * up + sub-RMSNorm + WHT + INT8] down GEMV + residual
 *   RMSNorm + INT8 prep | INT8 head GEMV with per-tile maxima | argmax (greedy) or the next prompt token,
 *   position + 1, the next token's embedding row (INT8 table x per-token scale)
 * The position and the current token live in device memory, so the step is captured once as a HIP graph and
 * replayed per token with no host work in between.
 *
 * Weights are passed in the reference's formats (host pointers): 2-bit ternary rows as eif_pack_ternary writes
 * them with grouped FP32 scales [rows, cols / group] (tinyllm_weights_t.bitnet_gscale, include/eif_tinyllm.h),
 * RMSNorm weights, +-1 rotation signs, an INT8 embedding with per-token scales and an INT8 head with per-row
 * scales. Compute: the linears on int8 activations (the contract of eif_hip_qlinear_prep), fp32 everything
 * else, the KV cache in fp16. Calls on one model are not thread-safe; the stream argument orders them.
 */
#ifndef EIF_HIP_DECODE_H
#define EIF_HIP_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct eif_hip_bitnet eif_hip_bitnet;

typedef struct eif_hip_bitnet_config {
    int dim, hidden, n_layers, n_heads, n_kv_heads, head_dim, vocab, seq_len;
    float rope_theta;                       /* RoPE base (half-split pairs, src/eif_tinyllm.c:476-507) */
    float rms_eps;                          /* attention / FFN / final RMSNorm epsilon */
    float sub_eps;                          /* sub-norm epsilon (1e-5 in the reference) */
    int wht_dim, wht_q, wht_hidden;         /* WHT blocks of the inputs of wq/wk/wv/w1/w3, wo, w2 (0: none) */
    float wht_norm_dim, wht_norm_q, wht_norm_hidden;   /* their scales, e.g. eif_hip_wht_norm(block) */
    int g_q, g_o, g_13, g_2;                /* ternary groups of wq/wk/wv, wo, w1/w3, w2 (0: one scale per row) */
} eif_hip_bitnet_config;

typedef struct eif_hip_bitnet_layer {       /* one layer, host pointers */
    const uint8_t *wq, *wk, *wv, *wo, *w1, *w3, *w2;
    const float *gq, *gk, *gv, *go, *g1, *g3, *g2;
    const float *rms_att, *rms_ffn, *rms_sub_att, *rms_sub_ffn;   /* NULL = 1 */
} eif_hip_bitnet_layer;

typedef struct eif_hip_bitnet_globals {    /* host pointers */
    const int8_t *emb;                      /* [vocab, dim] */
    const float *emb_scale;                 /* [vocab] or NULL (= 1) */
    const float *rms_final;                 /* [dim] or NULL */
    const float *signs_dim, *signs_q, *signs_hidden;   /* or NULL */
    const int8_t *wcls;                     /* [vocab, dim] */
    const float *wcls_scale;                /* [vocab] or NULL */
} eif_hip_bitnet_globals;

/* A BitNet-b1.58 model file in the reference's SVLM or TTML/TLLM layout (what tinyllm_load_quantized_model
 * reads, src/eif_tinyllm.c:2442-2556, laid out as tinyllm_setup_quantized_pointers expects, :2663-2731,
 * configured as src/eif_llm.c:321-351 reads it: SVLM with RoPE theta 100000, the file's group bound and
 * Hadamard flag; TTML with the file's theta, or tinyllm's default by vocabulary when it is 0, and one scale per
 * row) -> a ready model, weights repacked into the GPU layout. seq_len <= 0 takes the file's (512 when an SVLM
 * file has none). A TTML file with rope_interleaved set has the rows of wq and wk reordered within each head for
 * the decoder's half-split pairs (as eif_hip_bitnet_load_gguf, eif_hip_gguf.h). Files that are not BitNet
 * return EIF_HIP_E_ARG.                                                                                  */
int eif_hip_bitnet_load_svlm(eif_hip_bitnet **out, const char *path, int seq_len);

/* Allocates the model (weights are set separately). Limits: head_dim 32, 64 or 128, n_heads a multiple of
 * n_kv_heads, seq_len <= 4096, dim / q_dim / hidden multiples of 32 with the WHT blocks dividing them.      */
int eif_hip_bitnet_create(eif_hip_bitnet **out, const eif_hip_bitnet_config *cfg);
int eif_hip_bitnet_set_layer(eif_hip_bitnet *m, int layer, const eif_hip_bitnet_layer *w);
int eif_hip_bitnet_set_globals(eif_hip_bitnet *m, const eif_hip_bitnet_globals *g);

/* Starts a sequence: clears the KV cache, uploads the prompt (n_prompt >= 1 ids), position 0. The globals
 * must be set.                                                                                          */
int eif_hip_bitnet_reset(eif_hip_bitnet *m, const int *prompt, int n_prompt, void *stream);

/* How a token step runs: on = 0 (the default) as separate launches per linear and attention, replayed as a HIP
 * graph; on = 1 the layer stack as one persistent kernel (one workgroup per CU, grid barriers between the stages,
 * the next layer's weight tiles streamed into LDS while the current layer computes; src/eif_tinyllm.c:371-857's
 * layer loop), then the head GEMV and the sampler. Both give the same bits. The persistent form is slower on
 * MI355X at the BitNet-2B shape (1.72 against 1.14 ms per token): every stage's fused activation prep is a
 * dependent chain of 1.8-4.5 us that the separate launches overlap with their weight loads, while the persistent
 * kernel, whose weights are already in LDS, waits for it and for a grid barrier of about 1.8 us per stage.
 * Shapes outside the persistent kernel (head_dim other than 128, row-scaled ternary matrices, ...) always take
 * the separate launches. on = -1 only queries. Returns 1 when steps run persistent, 0 when not, or a negative
 * error (all layers and the globals must be set); EIF_HIP_E_LIMIT when one workgroup of the kernel cannot be
 * resident on a CU. A persistent step that gives up waiting at a grid barrier (all workgroups could not run at
 * once, e.g. other work held CUs) makes the next eif_hip_bitnet_tokens / _logits / _position return
 * EIF_HIP_E_DEVICE; its position, KV cache and tokens are then undefined, and eif_hip_bitnet_reset must be
 * called before the model is used again.                                                                */
int eif_hip_bitnet_set_persistent(eif_hip_bitnet *m, int on);

/* Runs n token steps from the current position. The step at position p consumes the current token and
 * makes the next: the prompt's token p + 1 while the prompt lasts, the argmax of the logits after. Each
 * made token is stored at index p + 1 of the sequence. Steps past seq_len return EIF_HIP_E_LIMIT.
 * use_graph != 0 replays the step as a HIP graph (captured on the first such call) on the stream.       */
int eif_hip_bitnet_steps(eif_hip_bitnet *m, int n, int use_graph, void *stream);

/* Runs the next n prompt tokens (positions p .. p + n - 1, all within the prompt) as one batch: every linear
 * through the prep + int8-MFMA GEMM of the n rows (the prefill of tinyllm_forward_batch_embeddings,
 * src/eif_tinyllm.c:930-1500), RoPE and KV append for the batch, causal attention on fp32 MFMAs per
 * 16-token block. The state afterwards is that of n token steps: the KV cache holds the n positions, the logits are the last
 * token's, and the current token is the prompt's next or, at the prompt's end, the argmax. Batch buffers
 * for n tokens are allocated on the first call with that n (not during graph capture).               */
int eif_hip_bitnet_prefill(eif_hip_bitnet *m, int n, void *stream);

/* The sequence so far (ids at positions 0 .. n-1) and the logits of the last step, copied to the host
 * (synchronous).                                                                                        */
int eif_hip_bitnet_tokens(eif_hip_bitnet *m, int *out, int n, void *stream);
int eif_hip_bitnet_logits(eif_hip_bitnet *m, float *out, void *stream);
int eif_hip_bitnet_position(eif_hip_bitnet *m, void *stream);   /* current position, or a negative error */

/* Cached keys and values of one layer at positions [pos0, pos0 + n), as floats in the reference's cache layout
 * [position][kv_head * head_dim + i] (src/eif_tinyllm.c:414-418), copied to the host (synchronous).           */
int eif_hip_bitnet_kv_cache(eif_hip_bitnet *m, int layer, int pos0, int n, float *k, float *v, void *stream);

/* The model's configuration (e.g. of a model read from a file).                                          */
int eif_hip_bitnet_get_config(const eif_hip_bitnet *m, eif_hip_bitnet_config *out);

/* Bytes of weights, scales and norms resident on the device, and the KV bytes one step reads at position p. */
size_t eif_hip_bitnet_weight_bytes(const eif_hip_bitnet *m);
size_t eif_hip_bitnet_kv_bytes(const eif_hip_bitnet *m, int p);

void eif_hip_bitnet_destroy(eif_hip_bitnet *m);

#ifdef __cplusplus
}
#endif
#endif

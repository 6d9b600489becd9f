/*
 * eif_hip_gguf.h -- BitNet-b1.58 models in GGUF files, read as the reference's GGUF loader reads them, then into
 * the GPU decoder (eif_hip_decode.h).
 *
 * The reference reads a GGUF causal model in two passes: tinyllm_read_gguf_config (src/eif_tinyllm.c:2843-3009)
 * takes the configuration from the metadata, and tinyllm_load_gguf (:3529-3838) converts every tensor into its own
 * weight formats (load_embedding_tensor :3276-3349, load_projection_tensor :3351-3527, load_rmsnorm :3112-3130).
 * Here eif_gguf_bitnet_open does both on the host and holds the result in the reference's formats, one scale per
 * row; eif_hip_bitnet_load_gguf hands that to the decoder. Only BitNet files are taken: those whose probe
 * projection (blk.0.attn_q.weight, else blk.0.ffn_down.weight, else the first quantized blk.0 weight) is TL1 or
 * TL2, which is what makes the reference run a GGUF file as BitNet (:3650-3662).
 *
 * What is refused (EIF_HIP_E_ARG) where the reference would read out of bounds or produce a model this decoder
 * does not run: a truncated or malformed container, a metadata value of an unexpected type for a key that is
 * read, a missing or misshapen projection, embedding or norm tensor, a tensor of another type than TL1 / TL2 /
 * Q8_0 / F32 / F16 / Q4_0 / Q4_1 / Q4_K / Q6_K (TL only for projections) or whose rows are not whole blocks, Q/K/V
 * biases, no token list (vocabulary 0).
 * Host code only; no call here touches the GPU except eif_hip_bitnet_load_gguf.
 */
#ifndef EIF_HIP_GGUF_H
#define EIF_HIP_GGUF_H

#include <stdint.h>

#include "eif_hip_decode.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct eif_gguf_bitnet eif_gguf_bitnet;   /* a converted model, host memory */

typedef struct eif_gguf_bitnet_info {
    char arch[64];          /* general.architecture ("" when absent) */
    uint32_t version;       /* container version */
    uint32_t alignment;     /* data alignment (general.alignment, 32 when absent) */
    int dim, hidden, n_layers, n_heads, n_kv_heads, head_dim, vocab, seq_len;
    float rope_theta;       /* rope.freq_base; when absent or <= 0: 1e6 for "qwen" in the architecture or path,
                             * else 1e4 (src/eif_tinyllm.c:2993-2999) */
    int rope_interleaved;   /* 1 for the llama, granite, minicpm and smollm architectures (:3614-3617) */
    int proj_type;          /* GGUF type of the probe projection: 34 (TL1) or 35 (TL2) */
    int emb_type;           /* GGUF type of token_embd.weight */
    int head_type;          /* GGUF type of output.weight / lm_head.weight; -1: tied to the embedding */
} eif_gguf_bitnet_info;

/* Reads and converts a GGUF BitNet model (the reference's arithmetic throughout):
 *  - configuration: <arch>.embedding_length, .feed_forward_length, .block_count, .attention.head_count,
 *    .attention.head_count_kv (0: head_count), .attention.key_length (0: dim / heads), .context_length (<= 0:
 *    2048, at most 4096), any key holding "rope.freq_base" / "rope_freq_base", the vocabulary from the count of
 *    tokenizer.ggml.tokens; <arch> is the architecture read so far ("llama" before general.architecture);
 *  - projections: TL1 / TL2 blocks copied, Q8_0 by sign, row scale = the block scales summed in order times
 *    1 / blocks (eif_gguf_ternary_rows); F32 / F16 / Q4_0 / Q4_1 / Q4_K / Q6_K ternarized by the row's absolute
 *    mean gamma = sum |x| * (1 / cols), code = +1 / -1 where x / gamma > 0.5 / < -0.5 (the sum in the order the
 *    reference's -ffast-math build forms it: sequential for F32 / F16, eight lanes for block types);
 *  - token_embd.weight and output.weight (else lm_head.weight, else tied): per row s = max|x| * (1 / 127) and
 *    q = round-half-away(x * (127 / max|x|)) clamped to [-128, 127] (s = 1, q = round(x) when s < 1e-12);
 *    Q8_0, Q4_0, Q4_1, Q4_K and Q6_K blocks dequantised first (ggml's block layouts). The reference's source writes s = max / 127, inv = 1 / s and the projections'
 *    mean as a division; these follow its -ffast-math build, which computes them as above;
 *  - attn_norm / ffn_norm / output_norm (else norm) weights: F32 or F16, 1 when absent or of another type. The
 *    reference reads no sub-norm tensors for GGUF models; they act as weight 1.                            */
int eif_gguf_bitnet_open(eif_gguf_bitnet **out, const char *path);
void eif_gguf_bitnet_close(eif_gguf_bitnet *m);
int eif_gguf_bitnet_get_info(const eif_gguf_bitnet *m, eif_gguf_bitnet_info *info);
/* Host pointers into the converted model, valid until eif_gguf_bitnet_close: 2-bit rows as the file holds them
 * (before any RoPE reordering), one scale per row (g* = [rows]), sub-norms NULL.                          */
int eif_gguf_bitnet_get_layer(const eif_gguf_bitnet *m, int layer, eif_hip_bitnet_layer *lw);
int eif_gguf_bitnet_get_globals(const eif_gguf_bitnet *m, eif_hip_bitnet_globals *g);

/* A GGUF BitNet model -> a ready decoder (the configuration above, RMSNorm epsilon 1e-6 above 120000 tokens of
 * vocabulary else 1e-5, no rotation, one scale per row). seq_len <= 0 takes the file's. A model whose RoPE
 * rotates interleaved pairs has the rows of wq and wk reordered within each head (row 2j -> j, 2j+1 -> j +
 * head_dim / 2, scales alike): the decoder's half-split rotation of the reordered rows is the interleaved
 * rotation of the file's rows, and q.k over a head is the same sum in another order.                        */
int eif_hip_bitnet_load_gguf(eif_hip_bitnet **out, const char *path, int seq_len);

#ifdef __cplusplus
}
#endif

#endif /* EIF_HIP_GGUF_H */

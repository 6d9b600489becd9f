/*
 * eif_hip_qwen35.h -- Qwen3.5 model files (the reference's QWN5 image, include/eif_qwen35.h:32-110) into resident
 * GPU weights for the quantized linears of eif_hip.h.
 *
 * The image is what qwen35_load maps (src/eif_qwen35.c:1223-1481): a 48-byte header, the 128-byte config block,
 * one layer-type byte per layer, then the weights, scales and norms regions. eif_qwen35_parse restates its
 * layout walk on the host and reports where every array lies; eif_hip_qwen35_load reads a file, parses it and
 * uploads every quantized linear (ternary 2-bit with row or group scales, ternary base-3 as 2-bit rows, INT4 with
 * row scales) and the tied embedding / LM head into the layouts of eif_hip_qweight_create, so the engine's
 * linear_gemv calls (src/eif_qwen35.c:421-444) become eif_hip_qlinear / eif_hip_qlinear_prep on them. FP32
 * matrices (the dt/beta projections of a grouped file, an FP32 LM) stay with the host: their handle is NULL.
 */
#ifndef EIF_HIP_QWEN35_H
#define EIF_HIP_QWEN35_H

#include <stddef.h>
#include <stdint.h>

#include "eif_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Matrix kinds of a layer. DeltaNet layers: DN_*; full-attention layers: FA_* (FA_Q holds the query rows and
 * their gate rows, 2 n_heads head_dim of them); every layer: FF_*. */
enum {
    EIF_Q35_DN_QKV = 0, EIF_Q35_DN_Z, EIF_Q35_DN_OUT, EIF_Q35_DN_B, EIF_Q35_DN_A,
    EIF_Q35_FA_Q, EIF_Q35_FA_K, EIF_Q35_FA_V, EIF_Q35_FA_O,
    EIF_Q35_FF_GATE, EIF_Q35_FF_UP, EIF_Q35_FF_DOWN,
    EIF_Q35_KINDS
};

/* Storage of one matrix: QWEN35_QTYPE_* for linears (0 FP32, 1 INT4, 2 ternary 2-bit, 3 ternary base-3), and
 * for the embedding its QWEN35_EMBED_* type mapped the same way (INT8 embeddings: qtype 4). */
enum { EIF_Q35_FP32 = 0, EIF_Q35_INT4 = 1, EIF_Q35_TERN2 = 2, EIF_Q35_TERN3 = 3, EIF_Q35_INT8 = 4 };

/* Byte offsets into the image (0: absent; offset 0 is the header, never an array). */
typedef struct eif_qwen35_tensor {
    size_t codes;     /* rows of the matrix */
    size_t scales;    /* its scales: [rows] per row, [rows, cols / group] grouped; 0 for FP32 */
    int rows, cols;
    int qtype;        /* EIF_Q35_* */
    int group;        /* ternary scale group, 0: one scale per row */
} eif_qwen35_tensor;

typedef struct eif_qwen35_layout {
    int32_t config[32];               /* the config block as stored (qwen35_config_t) */
    uint8_t layer_types[24];          /* 0 DeltaNet, 1 full attention */
    int n_layers;
    eif_qwen35_tensor embed;          /* token embedding [vocab, dim], also the tied LM head */
    eif_qwen35_tensor lin[24][EIF_Q35_KINDS];
    /* FP32 vectors (byte offsets, 0: absent) */
    size_t rms_att[24], rms_ffn[24], rms_final;
    size_t sub_att[24], sub_ffn[24];  /* SubLN before o_proj (full attention) and down_proj */
    size_t conv[24], dt_bias[24], a_log[24], delta_norm[24];   /* DeltaNet layers */
    size_t q_norm[24], k_norm[24];    /* full-attention layers */
    size_t signs_dim, signs_hid;      /* Hadamard signs (hadamard_block > 0) */
    int hadamard_block;
    size_t weights_end, scales_end, norms_end;   /* end of the data each region's walk reaches */
} eif_qwen35_layout;

/* Walk the layout of a QWN5 image of `bytes` bytes (host memory), with the reference loader's checks (magic and
 * version, region offsets in the file, the configuration's bounds, ternary_group and hadamard_block rules) and
 * one more: every array lies inside its region and the file. EIF_HIP_E_ARG on a malformed image. Host only.    */
int eif_qwen35_parse(const void *image, size_t bytes, eif_qwen35_layout *out);

typedef struct eif_hip_qwen35 eif_hip_qwen35;

/* Read and parse a QWN5 file, upload every quantized linear and the embedding / tied head. Synchronous.       */
int eif_hip_qwen35_load(eif_hip_qwen35 **out, const char *path, void *stream);

/* A llama.cpp-style Qwen3.5 text GGUF (bytes in memory) -> the QWN5 image the loader reads, as the reference's
 * qwen35_gguf_build_image builds it (src/eif_qwen35_gguf.c:262-454; eif_hip_qwen35_load calls it for a GGUF path,
 * as qwen35_load does, src/eif_qwen35.c:1236-1246): F32 / F16 / BF16 / Q8_0 / Q4_0 / Q4_K / Q5_K / Q6_K tensors
 * dequantised, the linears requantised to INT4 rows and the tied embedding to INT8 rows (quant_rows as the
 * reference's -ffast-math build computes it: s = max(1e-8, max |x|) * (1 / qmax), q = round-half-even(x / s)
 * through inv = 1 / s), ssm_a stored as A_log = logf(-ssm_a). The builder's limits are the reference's: 24
 * layers, tied head, as many key as value heads, RMSNorm epsilon 1e-6. Host only. *image is released with
 * eif_qwen35_image_free.                                                                                 */
int eif_qwen35_gguf_image(const void *file, size_t bytes, void **image, size_t *image_bytes);
void eif_qwen35_image_free(void *image);
void eif_hip_qwen35_destroy(eif_hip_qwen35 *m);

/* The parsed layout (offsets into the file's bytes). */
const eif_qwen35_layout *eif_hip_qwen35_get_layout(const eif_hip_qwen35 *m);
/* Resident weight of layer `layer`, kind EIF_Q35_*; NULL where the layer has no such matrix or it is FP32. */
const eif_hip_qweight *eif_hip_qwen35_linear(const eif_hip_qwen35 *m, int layer, int kind);
/* The embedding as a weight: the tied LM head (NULL for an FP32 embedding). */
const eif_hip_qweight *eif_hip_qwen35_head(const eif_hip_qwen35 *m);

/* Kind of the tied head for eif_hip_qwen35_linear_batch. */
#define EIF_Q35_HEAD (-1)

/* The prefill's batched linear on a resident matrix (replaces linear_gemm, src/eif_qwen35.c:1034-1065, as
 * prefill_chunk calls it, :1067-1153): y [M, ldy] = the matrix of layer `layer`, kind EIF_Q35_* (EIF_Q35_HEAD: the
 * tied head), times the M FP32 rows of spec (device memory; the engine's Hadamard rotation either applied by the
 * caller, as prefill_chunk's had_rows does, or asked of the prep through spec->signs / wht_block), on the
 * INT8-activation contract: each row quantised to INT8 (absmax), then the GEMV or the int8-MFMA GEMM by token
 * count and shape (eif_hip_qlinear_prep). EIF_HIP_E_ARG for a kind the layer lacks or an FP32 matrix. */
int eif_hip_qwen35_linear_batch(const eif_hip_qwen35 *m, int layer, int kind, const eif_hip_prep_spec *spec,
                                const float *bias, float *y, int ldy, int M, void *stream);
/* Device copy of an FP32 vector of the norms region (norms, sub-norms, Hadamard signs) by its layout offset;
 * NULL for 0 or an offset outside the region. */
const float *eif_hip_qwen35_vector(const eif_hip_qwen35 *m, size_t offset);

#ifdef __cplusplus
}
#endif

#endif

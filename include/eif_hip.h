/*
 * eif_hip.h -- device-pointer core of libbitllm_hip.so (gfx950 / MI355X).
 *
 * The host-pointer symbols of eif_quantize_bitnet.h, eif_gemm.h and eif_quant_linear.h wrap this layer. It has
 * no counterpart in the reference: it is the seam for callers whose activations stay in HBM (the
 * decode loop that replaces src/eif_tinyllm.c:371-857 and the qwen35 prefill that replaces
 * src/eif_qwen35.c:1034-1065). All pointers are DEVICE pointers; `stream` is a hipStream_t (NULL = the null
 * stream); every call is asynchronous on that stream and returns 0 or a negative EIF_HIP_E_* code.
 *
 * Integer contract (bit-exact with the CPU oracle):
 *   prep:   v = x*signs (if signs), butterflies h = 1,2,..,block/2 (a+b, a-b), v *= norm; amax = max|v|;
 *           amax < 1e-12 -> q = 0, xs = 1; else xs = amax*(1/127), q = trunc(v*(127/amax) +- 0.5) in [-128,127]
 *           (src/eif_quantize_bitnet.c:1032-1060, :1646-1677).
 *   linear: per (token m, row r, group g) acc = sum_{c in g} w[r,c]*xq[m,c] in int32 (exact);
 *           grouped ternary:  y = xs[m] * sum_g s[r,g]*(float)acc_g (+ bias[r])   (FP32, rel. 1e-5)
 *           row-scaled:       isum = sum_g acc_g; y = ((float)isum * xs[m]) * s[r] (+ bias[r]), the order the
 *                             reference build evaluates src/eif_quantize_bitnet.c:1199-1200 in.
 */
#ifndef EIF_HIP_H
#define EIF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    EIF_HIP_OK = 0,
    EIF_HIP_E_ARG = -1,     /* invalid size, pointer or combination */
    EIF_HIP_E_DEVICE = -2,  /* no usable gfx950 device / HIP runtime error */
    EIF_HIP_E_NOMEM = -3,   /* device allocation failed */
    EIF_HIP_E_LIMIT = -4    /* request beyond a documented maximum */
};

/* Weight formats of eif_hip_qweight_create. */
enum {
    EIF_HIP_W_TERNARY = 1, /* 2-bit codes, reference layout rows of (cols+3)/4 bytes */
    EIF_HIP_W_INT8 = 2,    /* int8 [rows, cols] row-major */
    EIF_HIP_W_INT4 = 3     /* 4-bit, reference layout rows of (cols+1)/2 bytes, even col = high nibble, v = n-8 */
};

/* Paths of eif_hip_qlinear_ex. */
enum { EIF_HIP_PATH_AUTO = 0, EIF_HIP_PATH_GEMV = 1, EIF_HIP_PATH_GEMM = 2 };

typedef struct eif_hip_qweight eif_hip_qweight;

/* Select device `device` for this thread and check it is gfx950. */
int eif_hip_init(int device);

/* Human-readable text of a return code. */
const char *eif_hip_strerror(int code);

/* The per-element WHT scale the reference build uses for `block`: on x86 the value its -O3 -ffast-math code
 * computes for 1.0f/sqrtf(block) (rsqrtss + one Newton step), elsewhere the correctly rounded value.
 * ref: src/eif_quantize_bitnet.c:1554, CMakeLists.txt:19 */
float eif_hip_wht_norm(int block);

/* Correctly rounded 1/sqrt(block) in float. */
float eif_hip_wht_norm_exact(int block);

/* Activation prep for M rows of K floats (row stride ldx): optional sign flip + blockwise WHT (wht_block = 0:
 * no rotation; else a power of two dividing K) + per-row absmax INT8. Writes xq [M, ldq] (ldq >= K, the bytes
 * [K, ldq) are zeroed), xs [M], and, if xrot != NULL, the rotated FP32 rows [M, ldr]. xq/xs may be NULL to
 * rotate only. K <= 12288 runs as one fused kernel; larger K needs xrot.                               */
int eif_hip_prep_rows(const float *x, int ldx, const float *signs, int M, int K, int wht_block, float norm,
                      int8_t *xq, int ldq, float *xs, float *xrot, int ldr, void *stream);

/* Upload/repack a weight matrix into the GPU layout (kept in HBM until eif_hip_qweight_destroy).
 *   codes, scales: host pointers (src_on_device = 0) or device pointers (src_on_device = 1);
 *   EIF_HIP_W_TERNARY: group > 0 (multiple of 32) -> scales [rows, ceil(cols/group)];
 *                      group == 0 -> row scales [rows] (NULL = 1);
 *   EIF_HIP_W_INT8/INT4: group must be 0, row scales [rows] (NULL = 1).
 * Synchronous (returns after the copy and repack completed).                                            */
int eif_hip_qweight_create(eif_hip_qweight **out, int fmt, int rows, int cols, int group, const void *codes,
                           const float *scales, int src_on_device, void *stream);
void eif_hip_qweight_destroy(eif_hip_qweight *w);

/* Shape of a weight: rows, cols, padded cols (the minimum ldq for activations), group, and device bytes. */
int eif_hip_qweight_info(const eif_hip_qweight *w, int *rows, int *cols, int *kpad, int *group, size_t *bytes);

/* y[m, r] for m < M, r < rows (row stride ldy), activations xq [M, ldq] (ldq >= kpad, multiple of 16) with
 * per-row scales xs [M]; bias [rows] or NULL. Auto path: the GEMV or the int8-MFMA GEMM by token count and
 * shape (see eif_hip_set_gemm_min_tokens); the GEMM from eif_hip_gemm_min_tokens() tokens on.            */
int eif_hip_qlinear(const eif_hip_qweight *w, const int8_t *xq, int ldq, const float *xs, const float *bias,
                    float *y, int ldy, int M, void *stream);
int eif_hip_qlinear_ex(const eif_hip_qweight *w, const int8_t *xq, int ldq, const float *xs, const float *bias,
                       float *y, int ldy, int M, int path, void *stream);

/* eif_hip_qlinear_ex that allocates nothing (no counterpart in the reference; for callers that cannot call
 * hipMalloc: code under HIP graph capture, tight serving loops, harnesses that forbid allocation). The GEMM's
 * split-along-K partials go to a fixed scratch in the library's device memory, eif_hip_qlinear_noalloc_max_bytes()
 * bytes (32 MiB) per device, instead of a per-stream workspace allocated on first use; a call whose split needs more
 * returns EIF_HIP_E_LIMIT and launches nothing. Results are those of eif_hip_qlinear_ex (the same split, the same
 * bits). Every call on a device shares that device's scratch, which keeps the last call's contents: calls that
 * overlap on one device (other streams, other threads) race and must be serialized by the caller.       */
int eif_hip_qlinear_ex_noalloc(const eif_hip_qweight *w, const int8_t *xq, int ldq, const float *xs,
                               const float *bias, float *y, int ldy, int M, int path, void *stream);
size_t eif_hip_qlinear_noalloc_max_bytes(void);

/* Exact int32 accumulators of the same kernels: grouped ternary -> acc [M, rows, ngroups]; row-scaled -> acc
 * [M, rows]. For parity tests.                                                                          */
int eif_hip_qlinear_acc(const eif_hip_qweight *w, const int8_t *xq, int ldq, int32_t *acc, int M, int path,
                        void *stream);

/* Prep fused into the GEMV: y = linear(prep(x)) for M <= 8 FP32 rows x [M, ldx] of K = cols (K % 32 == 0,
 * rows and signs 16-byte aligned, ldx % 4 == 0, K <= 16384), with the prep contract above (signs, wht_block <= 1024,
 * norm). One launch; the result equals eif_hip_prep_rows followed by eif_hip_qlinear bit for bit. M > 8
 * returns EIF_HIP_E_LIMIT (use the two calls).                                                         */
int eif_hip_qlinear_f32(const eif_hip_qweight *w, const float *x, int ldx, const float *signs, int wht_block,
                        float norm, const float *bias, float *y, int ldy, int M, void *stream);
int eif_hip_qlinear_f32_acc(const eif_hip_qweight *w, const float *x, int ldx, const float *signs, int wht_block,
                            float norm, int32_t *acc, int M, void *stream);

/* What the fused prep does before the rotation (eif_hip_qlinear_prep):
 *   EIF_HIP_PRE_NONE        the rows as given;
 *   EIF_HIP_PRE_RMS         RMSNorm: (x * (1 / sqrtf(sum(x^2) / K + eps))) * norm_w, the decoder's pre-norm
 *                           (src/eif_tinyllm.c:196-330, weight NULL = 1);
 *   EIF_HIP_PRE_SWIGLU_RMS  h = (x * (1 / (1 + expf(-x)))) * x2 (SiLU gate times up, src/eif_tinyllm.c:776-780), then
 *                           RMSNorm of h (the BitNet sub-norm before the down projection).            */
#define EIF_HIP_PRE_NONE 0
#define EIF_HIP_PRE_RMS 1
#define EIF_HIP_PRE_SWIGLU_RMS 2

typedef struct eif_hip_prep_spec {
    const float *x;       /* [M, ldx] FP32 rows (device), 16-byte aligned */
    int ldx;              /* row stride in floats, a multiple of 4, >= K */
    const float *x2;      /* EIF_HIP_PRE_SWIGLU_RMS: up-projection rows [M, ldx]; else ignored */
    const float *norm_w;  /* RMSNorm weight [K] or NULL (= 1) */
    float eps;            /* RMSNorm epsilon */
    int pre;              /* EIF_HIP_PRE_* */
    const float *signs;   /* [K] or NULL */
    int wht_block;        /* 0: no rotation; else a power of two <= 1024 dividing K */
    float wht_norm;       /* the WHT scale, e.g. eif_hip_wht_norm(wht_block) */
} eif_hip_prep_spec;

/* eif_hip_qlinear_f32 with a pre-op: y = linear(prep(pre(x))) (+ bias). M <= 8 rows: one launch (a row-scaled
 * matrix of 65536 rows or more at M = 1, e.g. a vocabulary head: a prep launch, then the GEMV of the prepped row,
 * with the same output bits); the bias may then be the residual stream itself (y == bias: each output reads its
 * own bias element first). More rows (a prompt batch): the prep of eif_hip_prep_spec_rows into a per-stream
 * workspace, then eif_hip_qlinear on the auto path (the GEMV or the int8-MFMA GEMM by token count and shape),
 * the same bits as those two calls; the bias must not overlap y, and a stream's first such call must be made
 * outside graph capture (it allocates the workspace; inside a capture it returns EIF_HIP_E_LIMIT).      */
int eif_hip_qlinear_prep(const eif_hip_qweight *w, const eif_hip_prep_spec *spec, const float *bias, float *y,
                         int ldy, int M, void *stream);

/* The gated FFN input of one layer in one launch: w stacks the gate projection (rows 0 .. rows/2 - 1) over the up
 * projection (rows rows/2 .. rows - 1); y[m, r] = SiLU(g) * u = (g * (1 / (1 + expf(-g)))) * u for r < rows / 2,
 * g and u the outputs eif_hip_qlinear_prep gives for rows r and rows/2 + r (src/eif_tinyllm.c:776-780). Fed to a
 * down projection with EIF_HIP_PRE_RMS, these rows give the bits of EIF_HIP_PRE_SWIGLU_RMS on the two halves.
 * M <= 8; a ternary g128 matrix whose half is a multiple of 32 rows, the WHT-128 or none; other shapes return
 * EIF_HIP_E_LIMIT (use eif_hip_qlinear_prep and the SwiGLU pre-op). No counterpart in the reference, which
 * computes the two halves and then SiLU(g) * u in its token loop.                                       */
int eif_hip_qlinear_prep_glu(const eif_hip_qweight *w, const eif_hip_prep_spec *spec, float *y, int ldy, int M,
                             void *stream);

/* The prep of a spec on its own, for any M (e.g. a prompt batch before the MFMA GEMM of eif_hip_qlinear):
 * M rows of K columns (K % 32 == 0) -> xq [M, ldq] int8 (ldq >= K, a multiple of 16, zeros past K) and
 * xs [M]. The codes and scales equal those the fused prep of eif_hip_qlinear_prep stages.              */
int eif_hip_prep_spec_rows(const eif_hip_prep_spec *spec, int K, int8_t *xq, int ldq, float *xs, int M,
                           void *stream);
int eif_hip_qlinear_prep_acc(const eif_hip_qweight *w, const eif_hip_prep_spec *spec, int32_t *acc, int M,
                             void *stream);

/* FP32 weight rows -> the INT8 / INT4 row-scaled formats eif_hip_qweight_create takes, with the arithmetic of the
 * reference's GGUF import, quant_rows (src/eif_qwen35_gguf.c:225-258), as its -ffast-math build computes it: per
 * row s = max(1e-8, max |x|) * (1 / qmax) (qmax 127 for bits 8, 7 for bits 4), q = round-half-even(x * (1 / s))
 * clamped to [-128, 127] / [-8, 7];
 * bits 4 packs columns (2i, 2i+1) into byte i as ((a + 8) << 4) | (b + 8), a zero column padding an odd count.
 * x [rows, ldx] FP32, dst [rows, cols or (cols + 1) / 2] bytes and scales [rows], all device memory.   */
int eif_hip_quant_rows(const float *x, int ldx, int rows, int cols, int bits, uint8_t *dst, float *scales,
                       void *stream);

/* BitNet projection tensors of a GGUF file -> the reference's 2-bit ternary rows with one scale per row, as the
 * reference's GGUF loader converts them (load_projection_tensor, src/eif_tinyllm.c:3351-3400): TL1 / TL2
 * (gguf_type 34 / 35: 32-column blocks of an fp16 scale and 8 bytes of codes, copied) or Q8_0 (gguf_type 8:
 * blocks of an fp16 scale and 32 int8 values, coded by sign); scale = the row's block scales summed in order, times
 * 1 / blocks (the reference's mean as its -ffast-math build computes it). Host
 * memory in and out: codes [rows, (cols + 3) / 4], scales [rows]. (The reference copies a TL row's last block past
 * the row's end when cols % 32 != 0; this stops at the row's end.)                                      */
int eif_gguf_ternary_rows(int gguf_type, const void *src, int rows, int cols, uint8_t *codes, float *scales);
/* The same conversion, then the resident row-scaled ternary weight (host src).                          */
int eif_hip_qweight_from_gguf_ternary(eif_hip_qweight **out, int gguf_type, const void *src, int rows, int cols,
                                      void *stream);

/* Drop the device copies the host-pointer ABI keeps for the weight or block-scale buffer at host_ptr (NULL: all
 * of them). Call it after rewriting such a buffer in place or before freeing it.                          */
void eif_hip_forget_host_weights(const void *host_ptr);

/* Bound on the device bytes of those copies (0: three quarters of the device's memory, the default); returns the
 * previous setting. A copy that would exceed it first evicts the least recently used copies that no call is
 * using; a later call needing an evicted buffer uploads it again.                                       */
size_t eif_hip_set_host_weight_cache_limit(size_t bytes);
/* Device bytes those copies hold now.                                                                   */
size_t eif_hip_host_weight_cache_bytes(void);

/* What the host-pointer ABI (eif_quantize_bitnet.h, eif_gemm.h, eif_quant_linear.h) does when a call fails
 * (no usable gfx950 device, a HIP error). Its functions return void, as the reference's do.
 *   EIF_HIP_HOST_ABORT (the default): print the call and the error, then abort().
 *   EIF_HIP_HOST_RECORD: return from the failing call with its outputs not (or not fully) written, and record the
 *   error for the calling thread (eif_hip_host_last_error).
 * The mode applies to all threads. Returns the previous mode, or -1 for an unknown one.                 */
#define EIF_HIP_HOST_ABORT 0
#define EIF_HIP_HOST_RECORD 1
int eif_hip_set_host_error_mode(int mode);

/* The calling thread's last error recorded by the host-pointer ABI (EIF_HIP_OK if none), cleared by this call;
 * msg (may be NULL) receives its description, at most len bytes with the terminating NUL.              */
int eif_hip_host_last_error(char *msg, size_t len);

/* Token count from which the auto path always uses the MFMA GEMM (default 64); returns the previous value.
 * Below it the auto path takes the GEMV for up to 8 tokens and, from 9 tokens on, where one workgroup stages
 * 16 token rows of the weight's columns and the shape favours it: group-scaled ternary of fewer than 256
 * 16-row tiles and 24 steps of K up to 16 tokens; row-scaled INT8 / INT4 up to 16 tokens; up to 32 tokens
 * vocabulary-sized ones (the streaming GEMV), INT8 ones of 8192 rows or 16 steps of 128 columns and more, and
 * INT4 ones of 32,768 rows and more; matrices of fewer than 2048 rows at any batch. The GEMM otherwise.     */
int eif_hip_set_gemm_min_tokens(int m);
int eif_hip_gemm_min_tokens(void);

/* Waves that split one 16-row tile's columns in the GEMV (1..16; 0 = chosen from the shape, the default);
 * returns the previous setting. A tuning knob: results do not depend on it.                              */
int eif_hip_set_gemv_ksplit(int k);

/* 16-row tiles per workgroup of the GEMV (1 or 4; 0 = chosen from the shape, the default); returns the
 * previous setting. A tuning knob: results do not depend on it.                                          */
int eif_hip_set_gemv_row_tiles(int rt);

/* Token rows per GEMV workgroup for batches above 8 tokens (1, 2, 4, 8, 16, 32 or 64; 0 = 32, halved until the
 * shape's staged rows fit, the default): a workgroup decodes each weight step once for all its rows (up to 4
 * MFMA token tiles of 16), and a larger batch is cut into chunks of that many rows, whose workgroups share
 * each weight tile through L2. Returns the previous setting. A tuning knob: results do not depend on it.   */
int eif_hip_set_gemv_token_chunk(int m);

/* The streaming GEMV of vocabulary-sized row-scaled INT4 / INT8 matrices (65,536 rows or more, prepped
 * activations, 4 to 32 token rows, 8 or 16 steps of K): waves per CU of its launch (1..32, which also takes 1
 * to 3 token rows; 0 = the default, 8; -1 = off, such matrices then take the GEMV above). Such matrices keep a
 * tile-major copy of their codes, which the stream reads (a load instruction covers 1 KB of whole lines);
 * -2 - wpc (-2 .. -34) asks for the same launch on the row-tile layout instead. Returns the previous setting.
 * A tuning knob: results do not depend on it.                                                             */
int eif_hip_set_gemv_stream(int wpc);

/* The row-pair GEMV of row-scaled INT4 / INT8 matrices at one token row, rows of whole 512-byte runs (INT4 K a
 * multiple of 1024 up to 4096, INT8 of 512 up to 2560): each half-wave reads 512 contiguous bytes of a row and
 * the products are v_dot4_i32_i8 on the resident layout. 0 = used for 16,384 rows or 20 MB of codes or more (the
 * default), 1 = for every such shape, -1 = off. Returns the previous setting. A tuning knob: results do not depend on it.     */
int eif_hip_set_gemv_rowpair(int mode);

/* Row tiles (of 4 rows) a wave takes at a time in the FP32-activation GEMVs of the host-pointer ABI (1 or 2;
 * 0 = chosen from the shape, the default); returns the previous setting. A tuning knob: results do not
 * depend on it.                                                                                          */
int eif_hip_set_f32_tiles_per_wave(int tw);

/* Waves that split one row tile's columns in those GEMVs (1, 2, 3, 4 or 8; 0 = chosen from the shape, the default);
 * returns the previous setting. A tuning knob: results depend on it only through the order of FP32 sums.   */
int eif_hip_set_f32_ksplit(int ks);

/* Fewest columns per thread of the prep fused into the GEMV (4, 8 or 16; 0 = chosen from the shape, the
 * default): more columns, fewer waves per workgroup. Returns the previous setting. A tuning knob: results do
 * not depend on it (with an RMSNorm pre-op, as for the other shape knobs, its sum of squares is added in
 * another order).                                                                                       */
int eif_hip_set_gemv_prep_cols(int e);

/* Splits along K of the GEMM (1..16; 0 = chosen from the shape, the default); returns the previous setting.
 * A split GEMM adds the per-split FP32 partials of grouped ternary in split order (deterministic, within
 * 1e-5 of the oracle; unsplit launches match it bit for bit); integer sums do not depend on it. Each tile's last
 * split adds them in the same launch. Splits use a per-stream workspace allocated on first use outside graph
 * capture.                                                                                              */
int eif_hip_set_gemm_split(int k);

/* Token tiles of 16 tokens per GEMM workgroup (1, 2 or 4; 0 = chosen from the batch, the default: 1 up to 16
 * tokens, 2 up to 32, else 4). Returns the previous setting. A tuning knob: results do not depend on it.     */
int eif_hip_set_gemm_token_tiles(int tt);

/* Steps of K whose loads the GEMM keeps in flight per workgroup (2, 4 or 8; 0 = chosen from the launch, the
 * default: 4 or 8 for launches of few workgroups, 2 for more than two per CU; 8 is taken as 4 for 64-token
 * tiles, and the panel form below takes at least 4). Returns the previous setting. A tuning knob: results do
 * not depend on it.                                                                                      */
int eif_hip_set_gemm_prefetch(int pf);

/* The GEMM's panel form, which stages a workgroup's whole activation panel (and its rows' group scales) in LDS
 * once and runs the K loop without barriers: 0 = chosen from the launch (the default: launches whose panel
 * workgroups all fit the CUs' LDS at once, grouped ternary split along K, with long K loops or more
 * workgroups than CUs, and unsplit INT8 / INT4 launches of one to four workgroups per CU), 1 = wherever its
 * LDS fits, -1 = never. Returns the previous setting. A tuning knob: results do not depend on it.          */
int eif_hip_set_gemm_panel(int mode);

#ifdef __cplusplus
}
#endif

#endif /* EIF_HIP_H */

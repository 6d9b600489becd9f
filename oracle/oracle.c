/*
 * oracle.c -- CPU restatement of tevfik/bitllm.c's quantized-linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this
 * library, as the checker / the timed CPU baseline. Nothing in the product (libbitllm_hip.so) links or calls it.
 *
 * Two builds of this one file (oracle/Makefile):
 *   liboracle.so       checker: -O2 -fno-fast-math -ffp-contract=off; every FP operation is written out in the
 *                      order it is meant, fmaf() only where a fused multiply-add is part of the contract.
 *   liboracle_port.so  CPU baseline: the reference flags -O3 -mavx2 -mfma -ffast-math -fopenmp
 *                      (CMakeLists.txt:19); OpenMP row loops as the reference.
 *
 * Each function names the reference lines it restates. Parity pins (tests/test_oracle_*.py) per function:
 *   orc_unpack/pack_ternary(_dense)     KAT tests/test_all_features.c:72-89, brute force over all 256 bytes
 *   orc_hadamard_block/group_size       KAT tests/test_bitnet_hadamard.c:34-36 + brute force over n
 *   orc_hadamard_rotate                 Sylvester matrix + involution (tests/test_bitnet_hadamard.c:43-62),
 *                                       bit-exact vs the compiled reference (oracle/_ref) given its norm
 *   orc_wht_norm_fastmath               bit-exact vs the compiled reference for every power of two <= 2^14
 *   orc_quantize_activation_i8          closed form, ties, amax < 1e-12, bit-exact vs compiled reference
 *   orc_*_acc_i32                       int64 numpy brute force (exact), KAT 4x8 of test_all_features.c:104-186
 *   orc_matmul_bitnet_i8xternary_f32    bit-exact vs compiled reference
 *   orc_matmul_bitnet_int8              bit-exact vs compiled reference
 *   orc_int8/int4_gemv_i8act            int32 sums vs int64 brute force; FP32 outputs within 1e-6 of the float64
 *                                       closed form acc*xs[m]*s[r] + bias[r] (normalised by |acc|*xs*s + |bias|),
 *                                       a planted xs / scale-index / bias-order mistake failing it
 *   FP32-activation GEMVs, GEMM, softmax  float64 references with the reference tests' bounds
 *                                       (test_int8_gemv.c:10-44, test_q35_int4.c:24-33, test_gemm.c:9-34)
 *   orc_quant_rows                      numpy float32 restatement, nibble order of test_q35_int4.c:20,
 *                                       closed-form bounds (|x - q s| <= s / 2, the largest |x| at +-qmax);
 *                                       bit-exact vs the compiled reference's GGUF image builder
 *   orc_gguf_ternary_rows               numpy restatement: the codes byte for byte, every fp16 scale value
 *                                       against numpy's binary16, the block order sum times 1 / blocks;
 *                                       bit-exact vs the compiled reference's GGUF loader
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#if defined(__x86_64__)
#include <immintrin.h>
#endif
#if defined(_OPENMP)
#include <omp.h>
#endif

#include "oracle.h"

#if defined(ORC_PORT)
#define ORC_PAR_ROWS _Pragma("omp parallel for schedule(static)")
#else
#define ORC_PAR_ROWS
#endif
/* Exact integer row sums (every row's int32 accumulators are independent of the others and of any order):
 * split over threads whenever OpenMP is on, the checker build included; the results are the same bits. */
#if defined(_OPENMP)
#define ORC_PAR_INT _Pragma("omp parallel for schedule(static)")
#else
#define ORC_PAR_INT
#endif

/* ---- a1: 2-bit codes.  src/eif_quantize_bitnet.c:15-41, format include/eif_quantize_bitnet.h:4-11 ---- */

int8_t orc_unpack_ternary(uint8_t byte, int pos)
{
    unsigned code = (byte >> (2 * pos)) & 3u;
    return code == 1u ? 1 : (code == 2u ? -1 : 0);
}

size_t orc_pack_ternary(const int8_t *v, uint8_t *packed, size_t count)
{
    size_t nb = (count + 3) / 4;
    for (size_t b = 0; b < nb; b++) {
        unsigned byte = 0;
        for (unsigned p = 0; p < 4; p++) {
            size_t i = 4 * b + p;
            unsigned code = 0;
            if (i < count) code = v[i] > 0 ? 1u : (v[i] < 0 ? 2u : 0u);
            byte |= code << (2 * p);
        }
        packed[b] = (uint8_t)byte;
    }
    return nb;
}

/* base 3, 5 trits per byte, trit i weighs 3^i.  src/eif_quantize_bitnet.c:92-112 */
size_t orc_pack_ternary_dense(const int8_t *v, uint8_t *packed, size_t count)
{
    size_t nb = (count + 4) / 5;
    for (size_t b = 0; b < nb; b++) {
        unsigned byte = 0, mul = 1;
        for (unsigned p = 0; p < 5; p++) {
            size_t i = 5 * b + p;
            unsigned code = 0;
            if (i < count) code = v[i] > 0 ? 1u : (v[i] < 0 ? 2u : 0u);
            byte += code * mul;
            mul *= 3;
        }
        packed[b] = (uint8_t)byte;
    }
    return nb;
}

static int8_t dense_trit(uint8_t byte, int i)
{
    unsigned t = byte;
    for (int k = 0; k < i; k++) t /= 3;
    t %= 3;
    return t == 1 ? 1 : (t == 2 ? -1 : 0);
}

/* ---- a2: size helpers.  src/eif_quantize_bitnet.c:1527-1541 ---- */

int orc_hadamard_block_size(int n)
{
    int b = 1;
    while (n > 0 && n % (2 * b) == 0 && 2 * b <= 1024) b *= 2;
    return b;
}

int orc_bitnet_group_size(int n, int max_group)
{
    if (max_group <= 0 || max_group >= n) return 0;
    for (int g = max_group - max_group % 32; g >= 32; g -= 32)
        if (n % g == 0) return g;
    return 0;
}

/* ---- a3: WHT norm. The reference writes 1.0f / sqrtf((float)block) (src/eif_quantize_bitnet.c:1554) and
 * builds with -O3 -mavx2 -mfma -ffast-math (CMakeLists.txt:19); gcc then emits rsqrtss followed by one
 * Newton step r = fma(a*x0, x0, -3) * (x0 * -0.5). orc_wht_norm_fastmath evaluates that sequence; its
 * rsqrtss estimate is the host CPU's, like the reference's. ---- */

float orc_wht_norm_exact(int block) { return (float)(1.0 / sqrt((double)block)); }

float orc_wht_norm_fastmath(int block)
{
#if defined(__x86_64__)
    float a = (float)block;
    float x0 = _mm_cvtss_f32(_mm_rsqrt_ss(_mm_set_ss(a)));
    float e0 = a * x0;
    float e1 = fmaf(e0, x0, -3.0f);
    float e2 = x0 * -0.5f;
    return e1 * e2;
#else
    return orc_wht_norm_exact(block);
#endif
}

/* ---- a3: blockwise WHT, in place.  src/eif_quantize_bitnet.c:1646-1677 (scalar), :1544-1593 (AVX2: the same
 * per-element operations). Returns 0 on success, -1 for the reference's silent no-op cases, -2 for a block
 * that is not a power of two (the reference writes out of range there; the restatement refuses). ---- */

int orc_hadamard_rotate(float *x, const float *signs, int n, int block, float norm)
{
    if (!x || block <= 0 || n % block != 0) return -1;
    if (block & (block - 1)) return -2;
    if (signs)
        for (int i = 0; i < n; i++) x[i] = x[i] * signs[i];
    for (int base = 0; base < n; base += block) {
        float *v = x + base;
        for (int h = 1; h < block; h *= 2)
            for (int i = 0; i < block; i += 2 * h)
                for (int j = i; j < i + h; j++) {
                    float a = v[j], b = v[j + h];
                    v[j] = a + b;
                    v[j + h] = a - b;
                }
        for (int i = 0; i < block; i++) v[i] = v[i] * norm;
    }
    return 0;
}

/* ---- a4: absmax INT8.  src/eif_quantize_bitnet.c:1032-1060. The scale is amax * (1/127) with the reciprocal
 * rounded to float, which is what the -ffast-math build computes for amax / 127.0f; 127/amax stays a correctly
 * rounded division; q*inv and the +-0.5 are separate roundings (no FMA contraction in the reference). ---- */

void orc_quantize_activation_i8(const float *x, int8_t *q, float *out_scale, int n)
{
    float amax = 0.0f;
    for (int i = 0; i < n; i++) {
        float v = fabsf(x[i]);
        if (v > amax) amax = v;
    }
    if (amax < 1e-12f) {
        memset(q, 0, (size_t)(n > 0 ? n : 0));
        if (out_scale) *out_scale = 1.0f;
        return;
    }
    const float recip127 = 1.0f / 127.0f;
    float scale = amax * recip127;
    float inv = 127.0f / amax;
    if (out_scale) *out_scale = scale;
    for (int i = 0; i < n; i++) {
        float t = x[i] * inv;
        float r = t >= 0.0f ? t + 0.5f : t - 0.5f;
        long v = (long)r;
        if (v > 127) v = 127;
        if (v < -128) v = -128;
        q[i] = (int8_t)v;
    }
}

/* Fused prep of M rows (the GPU's first kernel): optional WHT with the given norm, then a4.
 * wht_block == 0 skips the rotation (and the signs). xrot (optional) receives the rotated rows. */
int orc_prep_rows(const float *x, int ldx, const float *signs, int M, int K, int wht_block, float norm,
                  int8_t *xq, int ldq, float *xs, float *xrot, int ldr)
{
    float *tmp = (float *)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
    if (!tmp) return -3;
    int rc = 0;
    for (int m = 0; m < M && rc == 0; m++) {
        memcpy(tmp, x + (size_t)m * ldx, sizeof(float) * (size_t)K);
        if (wht_block > 0) rc = orc_hadamard_rotate(tmp, signs, K, wht_block, norm);
        if (rc) break;
        if (xrot) memcpy(xrot + (size_t)m * ldr, tmp, sizeof(float) * (size_t)K);
        if (xq) {
            orc_quantize_activation_i8(tmp, xq + (size_t)m * ldq, xs ? xs + m : NULL, K);
            for (int c = K; c < ldq; c++) xq[(size_t)m * ldq + c] = 0;
        }
    }
    free(tmp);
    return rc;
}

/* ---- exact int32 accumulators (new contract; integer sums are order-free) ---- */

/* acc[m, r, g] = sum_{c in group g} w[r,c] * xq[m,c], groups of `group` columns (last one partial).
 * group <= 0 or >= cols: one group per row. w: reference 2-bit rows of (cols+3)/4 bytes. */
void orc_ternary_acc_i32(const uint8_t *w, const int8_t *xq, int ldq, int M, int rows, int cols, int group,
                         int32_t *acc)
{
    const int rb = (cols + 3) / 4;
    const int g = (group > 0 && group < cols) ? group : cols;
    const int ng = (cols + g - 1) / g;
    ORC_PAR_INT
    for (int r = 0; r < rows; r++)
        for (int m = 0; m < M; m++) {
            const int8_t *xm = xq + (size_t)m * ldq;
            for (int gi = 0; gi < ng; gi++) {
                int32_t s = 0;
                int c1 = (gi + 1) * g < cols ? (gi + 1) * g : cols;
                for (int c = gi * g; c < c1; c++) s += orc_unpack_ternary(w[(size_t)r * rb + c / 4], c & 3) * xm[c];
                acc[((size_t)m * rows + r) * ng + gi] = s;
            }
        }
}

/* Grouped ternary x INT8 (the GPU linear's FP32 contract): per (m, r): t = 0; for g in order:
 * t = fmaf((float)acc_g, s[r,g], t); y = t * xs[m]; with bias: y = y + bias[r].
 * Design precedents: src/eif_quantize_bitnet.c:1227-1296 (group-ordered total += block_sum * scale) and the
 * aarch64 int8 x group-scale kernel src/eif_qwen35.c:228-290. */
void orc_ternary_gemv_grouped(const uint8_t *w, const float *gscales, int group, const int8_t *xq, int ldq,
                              const float *xs, const float *bias, float *y, int ldy, int M, int rows, int cols)
{
    const int g = (group > 0 && group < cols) ? group : cols;
    const int ng = (cols + g - 1) / g;
    int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)M * rows * ng);
    if (!acc) return;
    orc_ternary_acc_i32(w, xq, ldq, M, rows, cols, g, acc);
    for (int m = 0; m < M; m++)
        for (int r = 0; r < rows; r++) {
            float t = 0.0f;
            for (int gi = 0; gi < ng; gi++)
                t = fmaf((float)acc[((size_t)m * rows + r) * ng + gi], gscales ? gscales[(size_t)r * ng + gi] : 1.0f, t);
            float v = t * xs[m];
            if (bias) v = v + bias[r];
            y[(size_t)m * ldy + r] = v;
        }
    free(acc);
}

/* ---- a5: INT8 x ternary, per-row scale.  src/eif_quantize_bitnet.c:1143-1203 (int32 sum: :1063-1105).
 * The source line ((float)isum * (scale_row * scale_in)) + bias is compiled by the reference build
 * (-O3 -mavx2 -mfma -ffast-math) as ((float)isum * scale_in) * scale_row, then a separate add of the bias
 * when bias != NULL (no FMA); this restatement evaluates that order. ---- */

void orc_matmul_bitnet_i8xternary_f32(const uint8_t *w, const float *scales, const int8_t *xq, float scale_in,
                                      const float *bias, float *y, int rows, int cols)
{
    const int rb = (cols + 3) / 4;
    ORC_PAR_ROWS
    for (int r = 0; r < rows; r++) {
        int32_t s = 0;
        for (int c = 0; c < cols; c++) s += orc_unpack_ternary(w[(size_t)r * rb + c / 4], c & 3) * xq[c];
        float v = ((float)s * scale_in) * (scales ? scales[r] : 1.0f);
        if (bias) v = v + bias[r];
        y[r] = v;
    }
}

/* Batched a5 over M token rows with per-token scales xs (the GPU row-scaled ternary contract). */
void orc_ternary_gemv_rowscale(const uint8_t *w, const float *scales, const int8_t *xq, int ldq, const float *xs,
                               const float *bias, float *y, int ldy, int M, int rows, int cols)
{
    for (int m = 0; m < M; m++)
        orc_matmul_bitnet_i8xternary_f32(w, scales, xq + (size_t)m * ldq, xs[m], bias, y + (size_t)m * ldy, rows,
                                         cols);
}

/* ---- a6: quantize then a5.  src/eif_quantize_bitnet.c:1205-1224 ---- */
void orc_matmul_bitnet_act_quant_f32(const uint8_t *w, const float *scales, const float *x, const float *bias,
                                     float *y, int rows, int cols)
{
    int8_t *q = (int8_t *)malloc((size_t)(cols > 0 ? cols : 1));
    float s = 1.0f;
    if (!q) return;
    orc_quantize_activation_i8(x, q, &s, cols);
    orc_matmul_bitnet_i8xternary_f32(w, scales, q, s, bias, y, rows, cols);
    free(q);
}

/* ---- a10: INT8 in / INT8 out.  src/eif_quantize_bitnet.c:986-1030 ---- */
void orc_matmul_bitnet_int8(const uint8_t *w, float scale_w, const int8_t *x, float scale_in, const int32_t *bias,
                            int8_t *y, float scale_out, int rows, int cols)
{
    const int rb = (cols + 3) / 4;
    float eff = (scale_w * scale_in) / (scale_out > 1e-12f ? scale_out : 1.0f);
    for (int r = 0; r < rows; r++) {
        int32_t s = bias ? bias[r] : 0;
        for (int c = 0; c < cols; c++) s += orc_unpack_ternary(w[(size_t)r * rb + c / 4], c & 3) * x[c];
        float v = (float)s * eff;
        long q = (long)(v >= 0.0f ? v + 0.5f : v - 0.5f);
        if (q > 127) q = 127;
        if (q < -128) q = -128;
        y[r] = (int8_t)q;
    }
}

/* ---- INT8 / INT4 weights x INT8 activations (new contract): exact int32 row sums, then the a5 epilogue
 * y = ((float)isum * xs[m]) * s[r] (+ bias) applied to the a14/a15 weights. ---- */

static inline int int4_val(const uint8_t *row, int c)
{
    uint8_t b = row[c >> 1];
    return (c & 1) ? (int)(b & 0x0F) - 8 : (int)(b >> 4) - 8;
}

void orc_int8_acc_i32(const int8_t *w, const int8_t *xq, int ldq, int M, int rows, int cols, int32_t *acc)
{
    ORC_PAR_INT
    for (int r = 0; r < rows; r++)
        for (int m = 0; m < M; m++) {
            int32_t s = 0;
            for (int c = 0; c < cols; c++) s += (int32_t)w[(size_t)r * cols + c] * xq[(size_t)m * ldq + c];
            acc[(size_t)m * rows + r] = s;
        }
}

void orc_int4_acc_i32(const uint8_t *w, const int8_t *xq, int ldq, int M, int rows, int cols, int32_t *acc)
{
    const int pc = (cols + 1) / 2;
    ORC_PAR_INT
    for (int r = 0; r < rows; r++)
        for (int m = 0; m < M; m++) {
            int32_t s = 0;
            for (int c = 0; c < cols; c++) s += int4_val(w + (size_t)r * pc, c) * xq[(size_t)m * ldq + c];
            acc[(size_t)m * rows + r] = s;
        }
}

/* Row-scaled FP32 epilogue of the INT8 / INT4 linears on INT8 activations:
 * y = ((float)isum * xs[m]) * s[r] + bias[r]: the int32 sum times the activation scale, then the row scale, the
 * order of the reference's INT8-activation INT4 GEMV (src/eif_qwen35.c:221-224, aarch64), then the bias. The
 * x86 reference has no INT8-activation INT8/INT4 kernel, so these bits are this library's contract; the float64
 * closed form pins them (tests/test_oracle_pins.py).
 * ORC_PLANT_ROWSCALE (tests only, default 0) plants one mistake so the closed-form pin can be shown to catch it:
 * 1 = xs[0] for every token, 2 = the row scale indexed by token, 3 = the bias added before the xs multiply. */
#ifndef ORC_PLANT_ROWSCALE
#define ORC_PLANT_ROWSCALE 0
#endif
static void rowscale_epilogue(const int32_t *acc, const float *scales, const float *xs, const float *bias,
                              float *y, int ldy, int M, int rows)
{
    for (int m = 0; m < M; m++)
        for (int r = 0; r < rows; r++) {
            const float xsm = ORC_PLANT_ROWSCALE == 1 ? xs[0] : xs[m];
            const int si = ORC_PLANT_ROWSCALE == 2 ? m : r;
            const float b = bias ? bias[r] : 0.0f;
            float v;
            if (ORC_PLANT_ROWSCALE == 3) {
                v = (((float)acc[(size_t)m * rows + r] + b) * xsm) * (scales ? scales[si] : 1.0f);
            } else {
                v = ((float)acc[(size_t)m * rows + r] * xsm) * (scales ? scales[si] : 1.0f);
                if (bias) v = v + b;
            }
            y[(size_t)m * ldy + r] = v;
        }
}

void orc_int8_gemv_i8act(const int8_t *w, const float *scales, const int8_t *xq, int ldq, const float *xs,
                         const float *bias, float *y, int ldy, int M, int rows, int cols)
{
    int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)M * rows);
    if (!acc) return;
    orc_int8_acc_i32(w, xq, ldq, M, rows, cols, acc);
    rowscale_epilogue(acc, scales, xs, bias, y, ldy, M, rows);
    free(acc);
}

void orc_int4_gemv_i8act(const uint8_t *w, const float *scales, const int8_t *xq, int ldq, const float *xs,
                         const float *bias, float *y, int ldy, int M, int rows, int cols)
{
    int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)M * rows);
    if (!acc) return;
    orc_int4_acc_i32(w, xq, ldq, M, rows, cols, acc);
    rowscale_epilogue(acc, scales, xs, bias, y, ldy, M, rows);
    free(acc);
}

/* ---- FP32-activation paths (what the reference engines run on x86). Sequential sums; the reference's
 * vector lanes sum in another order, so comparisons use the reference tests' normalised bounds. ---- */

/* a8: src/eif_quantize_bitnet.c:834-892 (AVX2 :290-375). */
void orc_matmul_bitnet_f32(const uint8_t *w, const float *scales, const float *x, const float *bias, float *y,
                           int rows, int cols)
{
    const int rb = (cols + 3) / 4;
    ORC_PAR_ROWS
    for (int r = 0; r < rows; r++) {
        float s = 0.0f;
        for (int c = 0; c < cols; c++) {
            int v = orc_unpack_ternary(w[(size_t)r * rb + c / 4], c & 3);
            if (v > 0) s += x[c];
            else if (v < 0) s -= x[c];
        }
        y[r] = s * (scales ? scales[r] : 1.0f) + (bias ? bias[r] : 0.0f);
    }
}

/* a7: src/eif_quantize_bitnet.c:1356-1420 (AVX2 :1227-1296). block_size <= 0 means 64. */
void orc_matmul_bitnet_block_f32(const uint8_t *w, const float *bs, int block_size, const float *x,
                                 const float *bias, float *y, int rows, int cols)
{
    if (block_size <= 0) block_size = 64;
    const int rb = (cols + 3) / 4, nb = (cols + block_size - 1) / block_size;
    ORC_PAR_ROWS
    for (int r = 0; r < rows; r++) {
        float total = 0.0f;
        for (int b = 0; b < nb; b++) {
            float s = 0.0f;
            int c1 = (b + 1) * block_size < cols ? (b + 1) * block_size : cols;
            for (int c = b * block_size; c < c1; c++) {
                int v = orc_unpack_ternary(w[(size_t)r * rb + c / 4], c & 3);
                if (v > 0) s += x[c];
                else if (v < 0) s -= x[c];
            }
            total += s * (bs ? bs[(size_t)r * nb + b] : 1.0f);
        }
        y[r] = total + (bias ? bias[r] : 0.0f);
    }
}

/* a9: src/eif_quantize_bitnet.c:894-942. All 2*hidden rows are computed (the reference skips a trailing
 * 2*hidden % 4 remainder); a NULL scale means 1. */
void orc_matmul_bitnet_f32_w1w3(float *o1, float *o3, const uint8_t *w1, const uint8_t *w3, const float *s1,
                                const float *s3, const float *x, int hidden, int dim)
{
    orc_matmul_bitnet_f32(w1, s1, x, NULL, o1, hidden, dim);
    orc_matmul_bitnet_f32(w3, s3, x, NULL, o3, hidden, dim);
}

/* a11: src/eif_quantize_bitnet.c:944-983. */
void orc_matmul_bitnet_dense_f32(const uint8_t *w, const float *scales, const float *x, const float *bias, float *y,
                                 int rows, int cols)
{
    const int rb = (cols + 4) / 5;
    ORC_PAR_ROWS
    for (int r = 0; r < rows; r++) {
        float s = 0.0f;
        for (int c = 0; c < cols; c++) s += x[c] * (float)dense_trit(w[(size_t)r * rb + c / 5], c % 5);
        y[r] = s * (scales ? scales[r] : 1.0f) + (bias ? bias[r] : 0.0f);
    }
}

/* a12 layout: src/eif_quantize_bitnet.c:1422-1456. */
size_t orc_interleave_weights_4rows(const uint8_t *src, uint8_t *dst, int rows, int cols)
{
    if (!src || !dst || rows <= 0 || cols <= 0) return 0;
    const int ng = (cols + 3) / 4;
    size_t off = 0;
    int r = 0;
    for (; r < (rows & ~3); r += 4)
        for (int g = 0; g < ng; g++)
            for (int k = 0; k < 4; k++) dst[off++] = src[(size_t)(r + k) * ng + g];
    for (; r < rows; r++) {
        memcpy(dst + off, src + (size_t)r * ng, (size_t)ng);
        off += (size_t)ng;
    }
    return off;
}

/* a12 GEMV: src/eif_quantize_bitnet.c:1458-1520, without its input-pointer LUT cache and 1024-group cap. */
void orc_matmul_bitnet_tmac_interleaved_f32(const uint8_t *il, const float *scales, const float *x,
                                           const float *bias, float *y, int rows, int cols)
{
    const int ng = (cols + 3) / 4;
    for (int r = 0; r < rows; r++) {
        const uint8_t *p;
        size_t stride;
        if (r < (rows & ~3)) {
            p = il + (size_t)(r & ~3) * ng + (r & 3);
            stride = 4;
        } else {
            p = il + (size_t)(rows & ~3) * ng + (size_t)(r - (rows & ~3)) * ng;
            stride = 1;
        }
        float s = 0.0f;
        for (int g = 0; g < ng; g++) {
            uint8_t b = p[(size_t)g * stride];
            for (int k = 0; k < 4; k++) {
                int c = 4 * g + k;
                if (c >= cols) break;
                int v = orc_unpack_ternary(b, k);
                if (v > 0) s += x[c];
                else if (v < 0) s -= x[c];
            }
        }
        y[r] = s * (scales ? scales[r] : 1.0f) + (bias ? bias[r] : 0.0f);
    }
}

/* a14: src/eif_tinyllm.c:1651-1721 (x86 AVX2), scalar :1863-1874. Argument order as the reference. */
void orc_int8_rowscale_f32(float *y, const int8_t *w, const float *x, int cols, int rows, const float *scales)
{
    ORC_PAR_ROWS
    for (int r = 0; r < rows; r++) {
        float s = 0.0f;
        for (int c = 0; c < cols; c++) s += (float)w[(size_t)r * cols + c] * x[c];
        y[r] = s * (scales ? scales[r] : 1.0f);
    }
}

/* a15: src/eif_qwen35.c:293-352. */
void orc_int4_gemv_f32(float *out, const uint8_t *w, const float *sc, const float *x, int rows, int cols)
{
    const int pc = (cols + 1) / 2;
    ORC_PAR_ROWS
    for (int r = 0; r < rows; r++) {
        float s = 0.0f;
        for (int c = 0; c < cols; c++) s += (float)int4_val(w + (size_t)r * pc, c) * x[c];
        out[r] = (sc ? sc[r] : 1.0f) * s;
    }
}

/* ---- a18: FP32 NT GEMM + softmax.  src/eif_gemm.c:103-186, :188-218 ---- */

static float gelu_tanh(float v)
{
    const float k = 0.7978845608028654f;
    return 0.5f * v * (1.0f + tanhf(k * (v + 0.044715f * v * v * v)));
}

void orc_gemm_f32_nt_ld(const float *A, int lda, const float *W, int ldw, const float *bias, float *C, int ldc,
                        int M, int N, int K, int act, int accumulate)
{
    if (M <= 0 || N <= 0) return;
    ORC_PAR_ROWS
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float s = 0.0f;
            for (int k = 0; k < K; k++) s += A[(size_t)i * lda + k] * W[(size_t)j * ldw + k];
            float v = s + (bias ? bias[j] : 0.0f);
            if (accumulate) C[(size_t)i * ldc + j] += v;
            else C[(size_t)i * ldc + j] = act == 1 ? gelu_tanh(v) : v;
        }
}

void orc_softmax_rows_f32(float *S, int rows, int cols, int ld, float scale)
{
    for (int r = 0; r < rows; r++) {
        float *x = S + (size_t)r * ld;
        float mx = -INFINITY, sum = 0.0f;
        for (int c = 0; c < cols; c++) mx = fmaxf(mx, x[c]);
        for (int c = 0; c < cols; c++) {
            x[c] = expf((x[c] - mx) * scale);
            sum += x[c];
        }
        float inv = 1.0f / sum;
        for (int c = 0; c < cols; c++) x[c] *= inv;
    }
}

/* ---- CPU baseline helper: thread count the OpenMP build runs with. ---- */
int orc_num_threads(void)
{
#if defined(_OPENMP)
    return omp_get_max_threads();
#else
    return 1;
#endif
}


/* Row-wise symmetric quantisation of FP32 rows to INT8 or INT4 with one scale per row: the reference's GGUF import,
 * quant_rows (src/eif_qwen35_gguf.c:225-258) after its dequant_row. amax = max(1e-8, max |x|), s = amax / qmax
 * (qmax 127 or 7), inv = 1 / s, q = nearbyintf(x * inv) clamped to [-128, 127] or [-8, 7]; INT4 packs columns
 * (2i, 2i+1) into byte i as ((a + 8) << 4) | (b + 8), a zero column padding an odd count. */
void orc_quant_rows(const float *x, int ldx, int rows, int cols, int bits, uint8_t *dst, float *scales)
{
    const size_t rb = bits == 8 ? (size_t)cols : (size_t)(cols + 1) / 2;
    /* s = amax * (1 / qmax): the reference build (-ffast-math) multiplies by the reciprocal where its source divides
     * (bit-exact vs the images of the compiled qwen35_gguf_build_image, tests/test_qwen35_gguf.py) */
    const float rq = bits == 8 ? 1.0f / 127.0f : 1.0f / 7.0f;
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * ldx;
        float amax = 1e-8f;
        for (int c = 0; c < cols; c++) {
            const float a = fabsf(xr[c]);
            if (a > amax) amax = a;
        }
        const float sc = amax * rq, inv = 1.0f / sc;
        scales[r] = sc;
        uint8_t *o = dst + (size_t)r * rb;
        if (bits == 8) {
            for (int c = 0; c < cols; c++) {
                int q = (int)nearbyintf(xr[c] * inv);
                q = q > 127 ? 127 : (q < -128 ? -128 : q);
                ((int8_t *)o)[c] = (int8_t)q;
            }
        } else {
            for (int c = 0; c < cols; c += 2) {
                int a = (int)nearbyintf(xr[c] * inv);
                int b = c + 1 < cols ? (int)nearbyintf(xr[c + 1] * inv) : 0;
                a = a > 7 ? 7 : (a < -8 ? -8 : a);
                b = b > 7 ? 7 : (b < -8 ? -8 : b);
                o[c / 2] = (uint8_t)(((a + 8) << 4) | ((b + 8) & 0x0F));
            }
        }
    }
}


/* BitNet projection tensors of a GGUF file -> 2-bit ternary rows with one scale per row: the reference's
 * load_projection_tensor (src/eif_tinyllm.c:3351-3400) for TL1/TL2 (types 34/35: blocks of an fp16 scale and 8
 * code bytes, copied) and Q8_0 (type 8: blocks of an fp16 scale and 32 int8, coded by sign); scale = the sum of the
 * block scales in block order over the block count; the fp16 conversion is the reference's (include/eif_gguf.h:
 * 57-80). A TL row's copy stops at the row's end. */
static float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)(h & 0x8000)) << 16, exp = (h >> 10) & 0x1F, mant = h & 0x03FF;
    if (exp == 0) {
        if (mant == 0) return sign ? -0.0f : 0.0f;
        while (!(mant & 0x0400)) { mant <<= 1; exp--; }
        exp++;
        mant &= ~0x0400u;
    } else if (exp == 31) {
        return mant == 0 ? (sign ? -INFINITY : INFINITY) : NAN;
    }
    exp = exp + (127 - 15);
    uint32_t u = sign | (exp << 23) | (mant << 13);
    float out;
    memcpy(&out, &u, 4);
    return out;
}

void orc_gguf_ternary_rows(int type, const uint8_t *src, int rows, int cols, uint8_t *codes, float *scales)
{
    const int blocks = (cols + 31) / 32;
    const size_t rb = (size_t)(cols + 3) / 4, bb = type == 8 ? 34 : 10;
    for (int r = 0; r < rows; r++) {
        const uint8_t *rs = src + (size_t)r * blocks * bb;
        uint8_t *rd = codes + (size_t)r * rb;
        memset(rd, 0, rb);
        float s_sum = 0.0f;
        for (int b = 0; b < blocks; b++) {
            const uint8_t *blk = rs + (size_t)b * bb;
            uint16_t h;
            memcpy(&h, blk, 2);
            s_sum += orc_f16_to_f32(h);
            if (type != 8) {
                for (int i = 0; i < 8 && (size_t)b * 8 + i < rb; i++) rd[b * 8 + i] = blk[2 + i];
            } else {
                const int count = b == blocks - 1 ? cols - b * 32 : 32;
                for (int i = 0; i < count; i++) {
                    const int c = b * 32 + i;
                    const int8_t v = (int8_t)blk[2 + i];
                    const uint8_t code = v > 0 ? 1 : (v < 0 ? 2 : 0);
                    rd[c / 4] |= (uint8_t)(code << ((c % 4) * 2));
                }
            }
        }
        /* the reference as its build compiles it: -ffast-math turns s_sum / blocks, blocks loop-invariant, into a
         * multiply by the reciprocal (bit-exact vs the compiled reference, tests/test_gguf_model.py) */
        scales[r] = blocks > 0 ? s_sum * (1.0f / (float)blocks) : 1.0f;
    }
}

// hip_common.h -- shared helpers of libbitllm_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/eif_hip.h"

#define EIF_DEV __device__ __forceinline__

typedef int v4i __attribute__((ext_vector_type(4)));

// Return-code plumbing for the C ABI: every HIP call is checked, a failure maps to EIF_HIP_E_DEVICE.
#define EIF_HIP_TRY(expr)                                                                                      \
    do {                                                                                                       \
        hipError_t e__ = (expr);                                                                               \
        if (e__ != hipSuccess) {                                                                               \
            fprintf(stderr, "libbitllm_hip: %s failed: %s (%s:%d)\n", #expr, hipGetErrorString(e__), __FILE__, \
                    __LINE__);                                                                                 \
            return EIF_HIP_E_DEVICE;                                                                           \
        }                                                                                                      \
    } while (0)

// Checks the launch that was just enqueued (configuration errors surface here, not at execution).
#define EIF_HIP_LAUNCHED() EIF_HIP_TRY(hipGetLastError())

static inline int eif_ceil_div(int a, int b) { return (a + b - 1) / b; }
static inline int eif_round_up(int a, int b) { return eif_ceil_div(a, b) * b; }

// Device-side wave64 reductions (xor butterflies; exact for max and for integers).
EIF_DEV float eif_wave_max(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

EIF_DEV float eif_wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Greedy argmax of a row-scaled GEMV's outputs as one 64-bit key, folded over the workgroups by atomic max:
// the high word orders the value (IEEE order mapped to unsigned; -0 taken as +0; NaN taken as -inf, so it never
// beats a number), the low word is ~row, so of equal values the first row wins. The key of a row past the
// matrix (row 0x7fffffff, value -inf) loses to every real row.
EIF_DEV unsigned long long eif_argmax_key(float v, int row)
{
    if (v != v) v = -INFINITY;
    if (v == 0.0f) v = 0.0f;
    const uint32_t u = __float_as_uint(v);
    const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)k << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)row);
}
inline __host__ __device__ int eif_argmax_key_row(unsigned long long key)
{
    return (int)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
}
// The keys are folded into kArgmaxSlots slots kArgmaxStride keys (256 bytes) apart, a tile's into slot tile %
// kArgmaxSlots: device-scope atomics on one address serialise (8,016 tiles of a 128,256-row head on one key took
// 61 us more than the GEMV), on separate lines they proceed in parallel; the reader folds the slots.
constexpr int kArgmaxSlots = 64, kArgmaxStride = 32;

// Decode attention: the positions of a head are split into at most kAttnShares chunks, each leaving a share
// (unnormalized output, running maximum, sum) that the next linear's prep combines.
constexpr int kAttnShares = 8;

// v <- v of lane (l ^ LX): DPP only for LX <= 8 (quad_perm, row_half_mirror, row_mirror compositions).
template <int LX>
EIF_DEV float xlane(float v)
{
    int i = __float_as_int(v);
    if constexpr (LX == 1) {
        i = __builtin_amdgcn_update_dpp(0, i, 0xB1, 0xF, 0xF, false);            // quad_perm [1,0,3,2]
    } else if constexpr (LX == 2) {
        i = __builtin_amdgcn_update_dpp(0, i, 0x4E, 0xF, 0xF, false);            // quad_perm [2,3,0,1]
    } else if constexpr (LX == 4) {
        i = __builtin_amdgcn_update_dpp(0, i, 0x141, 0xF, 0xF, false);           // row_half_mirror: l ^ 7
        i = __builtin_amdgcn_update_dpp(0, i, 0x1B, 0xF, 0xF, false);            // quad_perm [3,2,1,0]: ^ 3
    } else if constexpr (LX == 8) {
        i = __builtin_amdgcn_update_dpp(0, i, 0x140, 0xF, 0xF, false);           // row_mirror: l ^ 15
        i = __builtin_amdgcn_update_dpp(0, i, 0x141, 0xF, 0xF, false);           // row_half_mirror: ^ 7
    } else {
        return __shfl_xor(v, LX, 64);
    }
    return __int_as_float(i);
}

// Internal launchers shared between translation units (defined in the .hip files).
namespace eif {
int launch_prep_rows(const float *x, int ldx, const float *signs, int M, int K, int wht_block, float norm,
                     int8_t *xq, int ldq, float *xs, float *xrot, int ldr, hipStream_t st);
int launch_rotate_rows(float *x, int ldx, const float *signs, int M, int K, int wht_block, float norm,
                       hipStream_t st);
int launch_quant_rows(const float *x, int ldx, int M, int K, int8_t *xq, int ldq, float *xs, hipStream_t st);

int qlinear_scaled(const eif_hip_qweight *w, const float *scales, const int8_t *xq, int ldq, const float *xs,
                   const float *bias, float *y, int ldy, int M, int path, hipStream_t st);
int qweight_row_tiles(const eif_hip_qweight *w);
// The GPU layout of a resident weight (qlinear.hip): codes W (rows padded to 64, wld bytes per row), scales
// ([rows, G] grouped, [rows] row-scaled or NULL), format, group (0: row-scaled), steps of the layout along K.
struct QView {
    const uint8_t *W;
    const float *scales;
    int fmt, rows, cols, group, ud, kpad, rows_pad, nsteps, wld, G;
};
int qweight_view(const eif_hip_qweight *w, QView *v);
// The device's fixed scratch of eif_hip_qlinear_ex_noalloc (qlinear.hip) and its split GEMM counters, set up once
// per device.
int scratch_init(int device, float **out, int **cnt = nullptr);
// The fused-prep linear of one token row (M = 1) whose input row is combined from attention shares in the prep:
// column c = h hd + d is sum_s e^(M_s - M) O_s[d] / sum_s e^(M_s - M) L_s over the shares s of head h, M = max_s M_s,
// with sh_o [K / hd][kAttnShares][hd] the outputs O_s and sh_ml [K / hd][2 kAttnShares] the maxima M_s, then the
// sums L_s (a share with M_s = -inf weighs 0). spec->x and spec->ldx are ignored; ternary weights only.
int qlinear_prep_shares(const eif_hip_qweight *w, const eif_hip_prep_spec *spec, const float *sh_o,
                        const float *sh_ml, int hd, const float *bias, float *y, int ldy, hipStream_t st);
int qlinear_argmax(const eif_hip_qweight *w, const int8_t *xq, int ldq, const float *xs, float *y,
                   unsigned long long *amax_key, hipStream_t st);

// FP32-activation GEMVs on the row-tile layout (f32linear.hip). Formats of the resident copy and the reference
// layouts it is made from.
constexpr int kF32Tern = 0, kF32Int4 = 1, kF32Int8 = 2;
constexpr int kSrcTernRow = 0;   // 2-bit row-major, (cols + 3) / 4 bytes a row, 01 = +1, 10 = -1, 00 / 11 = 0
constexpr int kSrcTernIl = 1;    // the same codes in the 4-row interleaved layout (src/eif_quantize_bitnet.c:1422-1456)
constexpr int kSrcDense = 2;     // base 3, (cols + 4) / 5 bytes a row, trit i of a byte weighs 3^i, 1 = +1, 2 = -1
constexpr int kSrcInt4 = 3;      // (cols + 1) / 2 bytes a row, even column in the high nibble, value nibble - 8
constexpr int kSrcInt8 = 4;      // cols signed bytes a row
size_t f32_tiles_bytes(int fmt, int rows, int cols);
// Whether a matrix of cols columns and block scales of `block` columns (0: one scale a row) has the row-tile path.
bool f32_tiles_fit(int cols, int block);
// Bytes of the [tile][block][4 rows] copy of block scales [rows, ceil(cols / block)], and the launch making it.
size_t f32_scales_bytes(int rows, int cols, int block);
int launch_f32_scales(const float *scales, void *dst, int rows, int cols, int block, hipStream_t st);
int launch_f32_repack(int src_fmt, const uint8_t *src, void *dst, int rows, int cols, hipStream_t st);
// y = W x (+ bias) on the row-tile copy Wt: block > 0 (ternary only) with block scales in the copy of
// launch_f32_scales, else scales [rows] (NULL = 1). x 16-byte aligned. EIF_HIP_E_LIMIT when f32_tiles_fit is false.
int launch_f32_tiles(int fmt, const void *Wt, const float *scales, int block, const float *x, const float *bias,
                     float *y, int rows, int cols, hipStream_t st);
int launch_tern_f32(const uint8_t *W, const float *scales, int mode, int block, const float *x, const float *bias,
                    float *y, int rows, int cols, int il, hipStream_t st);
int launch_dense_f32(const uint8_t *W, const float *scales, const float *x, const float *bias, float *y, int rows,
                     int cols, hipStream_t st);
int launch_int8_f32(const int8_t *W, const float *scales, const float *x, float *y, int rows, int cols,
                    hipStream_t st);
int launch_int4_f32(const uint8_t *W, const float *scales, const float *x, float *y, int rows, int cols,
                    hipStream_t st);
int launch_tern_int8_out(const uint8_t *W, const int8_t *x, const int32_t *bias, int8_t *y, float eff, int rows,
                         int cols, hipStream_t st);
int launch_gemm_f32_nt(const float *A, int lda, const float *W, int ldw, const float *bias, float *C, int ldc, int M,
                       int N, int K, int act, int accumulate, hipStream_t st);
int launch_softmax_rows(float *S, int rows, int cols, int ld, float scale, hipStream_t st);
}  // namespace eif

// f32linear.hip -- GEMVs with FP32 activations on the reference weight layouts (what the reference engines run
// on x86), plus the INT8-in/INT8-out ternary GEMV. One wave per output row, four rows per workgroup; lanes
// stride over the packed row bytes and the row sum is a wave reduction. These serve the host-pointer drop-in
// symbols; the FP32 sums are within the reference tests' normalised bounds (summation order differs).
#include "hip_common.h"

namespace {

constexpr int kRowsPerBlock = 4;

EIF_DEV float tern_val(unsigned byte, int pos)
{
    unsigned code = (byte >> (2 * pos)) & 3u;
    return code == 1u ? 1.0f : (code == 2u ? -1.0f : 0.0f);
}

EIF_DEV int tern_ival(unsigned byte, int pos)
{
    unsigned code = (byte >> (2 * pos)) & 3u;
    return code == 1u ? 1 : (code == 2u ? -1 : 0);
}

// Address of packed byte j of row r: row-major, or the 4-row interleaved layout of
// src/eif_quantize_bitnet.c:1422-1456 (full 4-row blocks interleaved byte by byte, tail rows row-major).
EIF_DEV const uint8_t *row_byte(const uint8_t *W, int rows, int rb, int r, int j, bool il)
{
    if (il && r < (rows & ~3)) return W + (size_t)(r & ~3) * rb + 4 * (size_t)j + (r & 3);
    return W + (size_t)r * rb + j;
}

// mode 0: per-row scale (scales[r] or 1); mode 1: block scales [rows, ceil(cols/block)] (NULL = 1).
// src/eif_quantize_bitnet.c:834-892 (mode 0), :1356-1420 (mode 1), :1458-1520 (il = true).
__global__ __launch_bounds__(64 * kRowsPerBlock) void tern_f32_kernel(const uint8_t *__restrict__ W,
                                                                      const float *__restrict__ scales, int mode,
                                                                      int block, const float *__restrict__ x,
                                                                      const float *__restrict__ bias,
                                                                      float *__restrict__ y, int rows, int cols,
                                                                      int il)
{
    const int r = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int rb = (cols + 3) / 4, nb = mode ? (cols + block - 1) / block : 1;
    float acc = 0.0f;
    for (int j = lane; j < rb; j += 64) {
        const unsigned byte = *row_byte(W, rows, rb, r, j, il != 0);
        const int c0 = 4 * j;
        if (mode == 0 || (block % 4 == 0)) {
            float s = 0.0f;
#pragma unroll
            for (int p = 0; p < 4; ++p)
                if (c0 + p < cols) s = fmaf(tern_val(byte, p), x[c0 + p], s);
            const float bsc = (mode && scales) ? scales[(size_t)r * nb + c0 / block] : 1.0f;
            acc = fmaf(s, bsc, acc);
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p)
                if (c0 + p < cols) {
                    const float bsc = scales ? scales[(size_t)r * nb + (c0 + p) / block] : 1.0f;
                    acc = fmaf(tern_val(byte, p) * x[c0 + p], bsc, acc);
                }
        }
    }
    acc = eif_wave_sum(acc);
    if (lane == 0) {
        float out = mode ? acc : acc * (scales ? scales[r] : 1.0f);
        y[r] = out + (bias ? bias[r] : 0.0f);
    }
}

// Base-3 rows of (cols+4)/5 bytes, trit i of a byte weighs 3^i.  src/eif_quantize_bitnet.c:944-983
__global__ __launch_bounds__(64 * kRowsPerBlock) void dense_f32_kernel(const uint8_t *__restrict__ W,
                                                                       const float *__restrict__ scales,
                                                                       const float *__restrict__ x,
                                                                       const float *__restrict__ bias,
                                                                       float *__restrict__ y, int rows, int cols)
{
    const int r = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int rb = (cols + 4) / 5;
    float acc = 0.0f;
    for (int j = lane; j < rb; j += 64) {
        unsigned t = W[(size_t)r * rb + j];
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const unsigned d = t % 3u;
            t /= 3u;
            const int c = 5 * j + i;
            if (c < cols && d) acc = d == 1u ? acc + x[c] : acc - x[c];
        }
    }
    acc = eif_wave_sum(acc);
    if (lane == 0) y[r] = acc * (scales ? scales[r] : 1.0f) + (bias ? bias[r] : 0.0f);
}

// INT8 row-scaled, FP32 activations.  src/eif_tinyllm.c:1651-1721, src/eif_qwen35.c:384-419
__global__ __launch_bounds__(64 * kRowsPerBlock) void int8_f32_kernel(const int8_t *__restrict__ W,
                                                                      const float *__restrict__ scales,
                                                                      const float *__restrict__ x,
                                                                      float *__restrict__ y, int rows, int cols)
{
    const int r = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int8_t *wr = W + (size_t)r * cols;
    float acc = 0.0f;
    for (int c = lane; c < cols; c += 64) acc = fmaf((float)wr[c], x[c], acc);
    acc = eif_wave_sum(acc);
    if (lane == 0) y[r] = acc * (scales ? scales[r] : 1.0f);
}

// INT4 row-scaled, FP32 activations; even column = high nibble, value = nibble - 8.  src/eif_qwen35.c:293-352
__global__ __launch_bounds__(64 * kRowsPerBlock) void int4_f32_kernel(const uint8_t *__restrict__ W,
                                                                      const float *__restrict__ scales,
                                                                      const float *__restrict__ x,
                                                                      float *__restrict__ y, int rows, int cols)
{
    const int r = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int pc = (cols + 1) / 2;
    const uint8_t *wr = W + (size_t)r * pc;
    float acc = 0.0f;
    for (int j = lane; j < pc; j += 64) {
        const unsigned b = wr[j];
        const int c = 2 * j;
        acc = fmaf((float)((int)(b >> 4) - 8), x[c], acc);
        if (c + 1 < cols) acc = fmaf((float)((int)(b & 15u) - 8), x[c + 1], acc);
    }
    acc = eif_wave_sum(acc);
    if (lane == 0) y[r] = (scales ? scales[r] : 1.0f) * acc;
}

// INT8 in, INT8 out: exact int32 row sum, then the reference's rounding.  src/eif_quantize_bitnet.c:986-1030
__global__ __launch_bounds__(64 * kRowsPerBlock) void tern_int8_out_kernel(const uint8_t *__restrict__ W,
                                                                           const int8_t *__restrict__ x,
                                                                           const int32_t *__restrict__ bias,
                                                                           int8_t *__restrict__ y, float eff,
                                                                           int rows, int cols)
{
    const int r = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int rb = (cols + 3) / 4;
    int acc = 0;
    for (int j = lane; j < rb; j += 64) {
        const unsigned byte = W[(size_t)r * rb + j];
#pragma unroll
        for (int p = 0; p < 4; ++p)
            if (4 * j + p < cols) acc += tern_ival(byte, p) * (int)x[4 * j + p];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) {
        const int isum = acc + (bias ? bias[r] : 0);
        const float v = (float)isum * eff;
        long q = (long)(v >= 0.0f ? v + 0.5f : v - 0.5f);
        q = q > 127 ? 127 : (q < -128 ? -128 : q);
        y[r] = (int8_t)q;
    }
}

inline dim3 row_grid(int rows) { return dim3((unsigned)eif_ceil_div(rows, kRowsPerBlock)); }

}  // namespace

namespace eif {

int launch_tern_f32(const uint8_t *W, const float *scales, int mode, int block, const float *x, const float *bias,
                    float *y, int rows, int cols, int il, hipStream_t st)
{
    if (rows <= 0 || cols <= 0) return EIF_HIP_OK;
    tern_f32_kernel<<<row_grid(rows), 64 * kRowsPerBlock, 0, st>>>(W, scales, mode, block, x, bias, y, rows, cols,
                                                                    il);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

int launch_dense_f32(const uint8_t *W, const float *scales, const float *x, const float *bias, float *y, int rows,
                     int cols, hipStream_t st)
{
    if (rows <= 0 || cols <= 0) return EIF_HIP_OK;
    dense_f32_kernel<<<row_grid(rows), 64 * kRowsPerBlock, 0, st>>>(W, scales, x, bias, y, rows, cols);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

int launch_int8_f32(const int8_t *W, const float *scales, const float *x, float *y, int rows, int cols,
                    hipStream_t st)
{
    if (rows <= 0 || cols <= 0) return EIF_HIP_OK;
    int8_f32_kernel<<<row_grid(rows), 64 * kRowsPerBlock, 0, st>>>(W, scales, x, y, rows, cols);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

int launch_int4_f32(const uint8_t *W, const float *scales, const float *x, float *y, int rows, int cols,
                    hipStream_t st)
{
    if (rows <= 0 || cols <= 0) return EIF_HIP_OK;
    int4_f32_kernel<<<row_grid(rows), 64 * kRowsPerBlock, 0, st>>>(W, scales, x, y, rows, cols);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

int launch_tern_int8_out(const uint8_t *W, const int8_t *x, const int32_t *bias, int8_t *y, float eff, int rows,
                         int cols, hipStream_t st)
{
    if (rows <= 0 || cols <= 0) return EIF_HIP_OK;
    tern_int8_out_kernel<<<row_grid(rows), 64 * kRowsPerBlock, 0, st>>>(W, x, bias, y, eff, rows, cols);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

}  // namespace eif

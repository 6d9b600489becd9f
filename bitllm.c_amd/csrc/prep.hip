// prep.hip -- activation prep: sign flip + blockwise Walsh-Hadamard rotation + per-row absmax INT8.
//
// Restates src/eif_quantize_bitnet.c:1646-1677 (rotation) and :1032-1060 (quantization) as one kernel per token
// row. The row is staged in LDS; every butterfly stage h = 1, 2, ..., block/2 is one pass over the pairs
// (a+b, a-b) followed by a barrier, so each element sees exactly the reference's sequence of IEEE operations and
// the result is bit-identical whatever the thread mapping. The library is built with -ffp-contract=off, so
// q = v*inv and q +- 0.5 stay two roundings as in the reference; 127/amax is a correctly rounded division.
#include "hip_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kLdsMaxFloats = 12288;   // fused path: whole row in 48 KiB of LDS
constexpr int kSegFloats = 8192;       // rotation-only path: segment per workgroup

EIF_DEV void wht_lds(float *v, int n, int block)
{
    // n is a multiple of block, block a power of two; pairs (a, a+h) never leave their block.
    for (int h = 1, lh = 0; h < block; h <<= 1, ++lh) {
        for (int p = threadIdx.x; p < (n >> 1); p += kThreads) {
            int i = p >> lh;
            int a = (i << (lh + 1)) + (p - (i << lh));
            float va = v[a], vb = v[a + h];
            v[a] = va + vb;
            v[a + h] = va - vb;
        }
        __syncthreads();
    }
}

EIF_DEV float block_max(float m, float *red)
{
    m = eif_wave_max(m);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = m;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kThreads / 64; ++i) r = fmaxf(r, red[i]);
    return r;
}

EIF_DEV int8_t quant_one(float v, float inv)
{
    float t = v * inv;
    float r = t >= 0.0f ? t + 0.5f : t - 0.5f;
    int q = (int)r;
    q = q > 127 ? 127 : (q < -128 ? -128 : q);
    return (int8_t)q;
}

// One workgroup per row m. Dynamic LDS: K floats.
__global__ __launch_bounds__(kThreads) void prep_rows_kernel(const float *__restrict__ x, int ldx,
                                                             const float *__restrict__ signs, int K, int block,
                                                             float norm, int8_t *__restrict__ xq, int ldq,
                                                             float *__restrict__ xs, float *__restrict__ xrot,
                                                             int ldr)
{
    extern __shared__ float sv[];
    __shared__ float red[kThreads / 64];
    const int m = blockIdx.x;
    const float *xr = x + (size_t)m * ldx;

    for (int i = threadIdx.x; i < K; i += kThreads) {
        float v = xr[i];
        if (block > 0 && signs) v = v * signs[i];
        sv[i] = v;
    }
    __syncthreads();
    if (block > 1) wht_lds(sv, K, block);

    float amax = 0.0f;
    for (int i = threadIdx.x; i < K; i += kThreads) {
        float v = sv[i];
        if (block > 0) {
            v = v * norm;
            sv[i] = v;
        }
        if (xrot) xrot[(size_t)m * ldr + i] = v;
        amax = fmaxf(amax, fabsf(v));
    }
    if (!xq) return;
    amax = block_max(amax, red);

    int8_t *qr = xq + (size_t)m * ldq;
    if (amax < 1e-12f) {
        for (int i = threadIdx.x; i < ldq; i += kThreads) qr[i] = 0;
        if (threadIdx.x == 0 && xs) xs[m] = 1.0f;
        return;
    }
    const float inv = 127.0f / amax;
    if (threadIdx.x == 0 && xs) xs[m] = amax * (1.0f / 127.0f);
    for (int i = threadIdx.x; i < ldq; i += kThreads) qr[i] = i < K ? quant_one(sv[i], inv) : (int8_t)0;
}

// Rotation only, in place, for rows longer than the fused kernel's LDS: grid (M, segments of kSegFloats).
__global__ __launch_bounds__(kThreads) void rotate_rows_kernel(float *__restrict__ x, int ldx,
                                                               const float *__restrict__ signs, int K, int block,
                                                               float norm, int seg)
{
    __shared__ float sv[kSegFloats];
    const int m = blockIdx.x, s0 = blockIdx.y * seg;
    const int n = (K - s0) < seg ? (K - s0) : seg;
    float *xr = x + (size_t)m * ldx + s0;
    for (int i = threadIdx.x; i < n; i += kThreads) {
        float v = xr[i];
        if (signs) v = v * signs[s0 + i];
        sv[i] = v;
    }
    __syncthreads();
    if (block > 1) wht_lds(sv, n, block);
    for (int i = threadIdx.x; i < n; i += kThreads) xr[i] = sv[i] * norm;
}

// Quantization only (any K): one workgroup per row, two passes over global memory.
__global__ __launch_bounds__(kThreads) void quant_rows_kernel(const float *__restrict__ x, int ldx, int K,
                                                              int8_t *__restrict__ xq, int ldq,
                                                              float *__restrict__ xs)
{
    __shared__ float red[kThreads / 64];
    const int m = blockIdx.x;
    const float *xr = x + (size_t)m * ldx;
    float amax = 0.0f;
    for (int i = threadIdx.x; i < K; i += kThreads) amax = fmaxf(amax, fabsf(xr[i]));
    amax = block_max(amax, red);
    int8_t *qr = xq + (size_t)m * ldq;
    if (amax < 1e-12f) {
        for (int i = threadIdx.x; i < ldq; i += kThreads) qr[i] = 0;
        if (threadIdx.x == 0 && xs) xs[m] = 1.0f;
        return;
    }
    const float inv = 127.0f / amax;
    if (threadIdx.x == 0 && xs) xs[m] = amax * (1.0f / 127.0f);
    for (int i = threadIdx.x; i < ldq; i += kThreads) qr[i] = i < K ? quant_one(xr[i], inv) : (int8_t)0;
}

// Blocks longer than a segment: the same stages, one launch per stage over global memory.
// mode 0: x *= signs; mode 1: butterfly stage h; mode 2: x *= norm. Grid: (pairs or elements / 256, M).
__global__ __launch_bounds__(kThreads) void wht_global_kernel(float *__restrict__ x, int ldx,
                                                              const float *__restrict__ signs, int K, int mode,
                                                              int lh, float norm)
{
    float *xr = x + (size_t)blockIdx.y * ldx;
    const int p = blockIdx.x * kThreads + threadIdx.x;
    if (mode == 1) {
        if (p >= (K >> 1)) return;
        const int h = 1 << lh, i = p >> lh;
        const int a = (i << (lh + 1)) + (p - (i << lh));
        const float va = xr[a], vb = xr[a + h];
        xr[a] = va + vb;
        xr[a + h] = va - vb;
        return;
    }
    if (p >= K) return;
    xr[p] = mode == 0 ? xr[p] * signs[p] : xr[p] * norm;
}

bool is_pow2(int b) { return b > 0 && (b & (b - 1)) == 0; }

}  // namespace

namespace eif {

int launch_rotate_rows(float *x, int ldx, const float *signs, int M, int K, int block, float norm, hipStream_t st)
{
    if (M <= 0 || K <= 0) return EIF_HIP_OK;
    if (!x || ldx < K || !is_pow2(block) || K % block != 0) return EIF_HIP_E_ARG;
    if (block > kSegFloats) {
        dim3 ge(eif_ceil_div(K, kThreads), M), gp(eif_ceil_div(K / 2, kThreads), M);
        if (signs) {
            wht_global_kernel<<<ge, kThreads, 0, st>>>(x, ldx, signs, K, 0, 0, norm);
            EIF_HIP_LAUNCHED();
        }
        for (int lh = 0; (1 << lh) < block; ++lh) {
            wht_global_kernel<<<gp, kThreads, 0, st>>>(x, ldx, signs, K, 1, lh, norm);
            EIF_HIP_LAUNCHED();
        }
        wht_global_kernel<<<ge, kThreads, 0, st>>>(x, ldx, signs, K, 2, 0, norm);
        EIF_HIP_LAUNCHED();
        return EIF_HIP_OK;
    }
    const int seg = (kSegFloats / block) * block;
    dim3 grid(M, eif_ceil_div(K, seg));
    rotate_rows_kernel<<<grid, kThreads, 0, st>>>(x, ldx, signs, K, block, norm, seg);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

int launch_quant_rows(const float *x, int ldx, int M, int K, int8_t *xq, int ldq, float *xs, hipStream_t st)
{
    if (M <= 0 || K <= 0) return EIF_HIP_OK;
    if (!x || !xq || ldx < K || ldq < K) return EIF_HIP_E_ARG;
    quant_rows_kernel<<<M, kThreads, 0, st>>>(x, ldx, K, xq, ldq, xs);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

int launch_prep_rows(const float *x, int ldx, const float *signs, int M, int K, int block, float norm,
                     int8_t *xq, int ldq, float *xs, float *xrot, int ldr, hipStream_t st)
{
    if (M <= 0 || K <= 0) return EIF_HIP_OK;
    if (!x || ldx < K || block < 0) return EIF_HIP_E_ARG;
    if (block > 0 && (!is_pow2(block) || K % block != 0)) return EIF_HIP_E_ARG;
    if (xq && (ldq < K || !xs)) return EIF_HIP_E_ARG;
    if (xrot && ldr < K) return EIF_HIP_E_ARG;
    if (K <= kLdsMaxFloats) {
        prep_rows_kernel<<<M, kThreads, (size_t)K * sizeof(float), st>>>(x, ldx, signs, K, block, norm, xq, ldq,
                                                                          xs, xrot, ldr);
        EIF_HIP_LAUNCHED();
        return EIF_HIP_OK;
    }
    // Long rows: rotate into xrot (required), then quantize from it.
    if (!xrot) return EIF_HIP_E_LIMIT;
    EIF_HIP_TRY(hipMemcpy2DAsync(xrot, (size_t)ldr * sizeof(float), x, (size_t)ldx * sizeof(float),
                                 (size_t)K * sizeof(float), M, hipMemcpyDeviceToDevice, st));
    if (block > 0) {
        int rc = launch_rotate_rows(xrot, ldr, signs, M, K, block, norm, st);
        if (rc) return rc;
    }
    if (xq) return launch_quant_rows(xrot, ldr, M, K, xq, ldq, xs, st);
    return EIF_HIP_OK;
}

}  // namespace eif

extern "C" int eif_hip_prep_rows(const float *x, int ldx, const float *signs, int M, int K, int wht_block,
                                 float norm, int8_t *xq, int ldq, float *xs, float *xrot, int ldr, void *stream)
{
    return eif::launch_prep_rows(x, ldx, signs, M, K, wht_block, norm, xq, ldq, xs, xrot, ldr,
                                 (hipStream_t)stream);
}

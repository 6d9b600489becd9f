// gemm_f32.hip -- C = act(A W^T + bias) / C += A W^T + bias in FP32, and the row softmax of eif_gemm.h.
// Reference: src/eif_gemm.c:103-186 (GEMM, GELU-tanh epilogue :97-101), :188-218 (softmax).
// 64x64 output tile per 256-thread workgroup, 4x4 outputs per thread, K staged 16 at a time through LDS.
#include "hip_common.h"
#include "../../include/eif_gemm.h"

namespace {

constexpr int kTile = 64, kKT = 16;

EIF_DEV float gelu_tanh(float v)
{
    const float k = 0.7978845608028654f;
    return 0.5f * v * (1.0f + tanhf(k * (v + 0.044715f * v * v * v)));
}

__global__ __launch_bounds__(256) void gemm_f32_nt_kernel(const float *__restrict__ A, int lda,
                                                          const float *__restrict__ W, int ldw,
                                                          const float *__restrict__ bias, float *__restrict__ C,
                                                          int ldc, int M, int N, int K, int act, int accumulate)
{
    __shared__ float As[kKT][kTile + 1];
    __shared__ float Ws[kKT][kTile + 1];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int m0 = blockIdx.y * kTile, n0 = blockIdx.x * kTile;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += kKT) {
        for (int i = threadIdx.x; i < kTile * kKT; i += 256) {
            const int rr = i / kKT, kk = i % kKT;
            const int gm = m0 + rr, gn = n0 + rr, gk = k0 + kk;
            As[kk][rr] = (gm < M && gk < K) ? A[(size_t)gm * lda + gk] : 0.0f;
            Ws[kk][rr] = (gn < N && gk < K) ? W[(size_t)gn * ldw + gk] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kKT; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Ws[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int gm = m0 + ty + 16 * i, gn = n0 + tx + 16 * j;
            if (gm >= M || gn >= N) continue;
            const float v = acc[i][j] + (bias ? bias[gn] : 0.0f);
            float *c = C + (size_t)gm * ldc + gn;
            if (accumulate)
                *c += v;
            else
                *c = act == EIF_GEMM_ACT_GELU_TANH ? gelu_tanh(v) : v;
        }
}

__global__ __launch_bounds__(256) void softmax_rows_kernel(float *__restrict__ S, int cols, int ld, float scale)
{
    __shared__ float red[4];
    float *x = S + (size_t)blockIdx.x * ld;
    float mx = -INFINITY;
    for (int c = threadIdx.x; c < cols; c += 256) mx = fmaxf(mx, x[c]);
    mx = eif_wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float sum = 0.0f;
    for (int c = threadIdx.x; c < cols; c += 256) {
        const float e = expf((x[c] - mx) * scale);
        x[c] = e;
        sum += e;
    }
    sum = eif_wave_sum(sum);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sum;
    __syncthreads();
    const float inv = 1.0f / (red[0] + red[1] + red[2] + red[3]);
    for (int c = threadIdx.x; c < cols; c += 256) x[c] *= inv;
}

}  // namespace

namespace eif {

int launch_gemm_f32_nt(const float *A, int lda, const float *W, int ldw, const float *bias, float *C, int ldc, int M,
                       int N, int K, int act, int accumulate, hipStream_t st)
{
    if (M <= 0 || N <= 0) return EIF_HIP_OK;
    dim3 grid(eif_ceil_div(N, kTile), eif_ceil_div(M, kTile));
    gemm_f32_nt_kernel<<<grid, 256, 0, st>>>(A, lda, W, ldw, bias, C, ldc, M, N, K, act, accumulate);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

int launch_softmax_rows(float *S, int rows, int cols, int ld, float scale, hipStream_t st)
{
    if (rows <= 0 || cols <= 0) return EIF_HIP_OK;
    softmax_rows_kernel<<<rows, 256, 0, st>>>(S, cols, ld, scale);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

}  // namespace eif

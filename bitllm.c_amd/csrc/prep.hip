// prep.hip -- activation prep: sign flip + blockwise Walsh-Hadamard rotation + per-row absmax INT8.
//
// Restates src/eif_quantize_bitnet.c:1646-1677 (rotation) and :1032-1060 (quantization) as one kernel per token
// row. Every butterfly stage h = 1, 2, ..., block/2 applies the reference's (a+b, a-b) to each pair, so each
// element sees exactly the reference's sequence of IEEE operations and the result is bit-identical whatever the
// thread mapping. The hot kernel (prep_rows_t32_kernel) keeps the row in registers, 32 elements per thread; the
// general kernels stage it in LDS. The library is built with -ffp-contract=off, so q = v*inv and q +- 0.5 stay
// two roundings as in the reference; 127/amax is a correctly rounded division.
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

// Lane exchange v <- v of lane (l ^ LX). LX = 1, 2: DPP quad permutes (no LDS traffic); larger: bpermute.
template <int LX>
EIF_DEV float lane_xor(float v)
{
    if constexpr (LX == 1)
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    else if constexpr (LX == 2)
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    else
        return __shfl_xor(v, LX, 64);
}

// Prep with a compile-time block (1 <= BLOCK <= 2048, or 0 = no rotation) for K % 32 == 0, K <= 8192*NCH.
// Thread t owns the 32 consecutive elements [8192*c + 32t, +32) of chunk c: butterfly stages h < 32 are
// in-register; stage h >= 32 pairs lane l with lane l ^ (h/32) (DPP for h = 32, 64), the lower partner keeping
// a+b and the upper one a-b -- exactly the reference's operations, so the result is bit-identical. One barrier
// (the absmax) per row.
template <int BLOCK, int NCH>
__global__ __launch_bounds__(kThreads) void prep_rows_t32_kernel(const float *__restrict__ x, int ldx,
                                                                 const float *__restrict__ signs, int K, float norm,
                                                                 int8_t *__restrict__ xq, int ldq,
                                                                 float *__restrict__ xs, float *__restrict__ xrot,
                                                                 int ldr)
{
    constexpr int E = 32;
    __shared__ float red[kThreads / 64];
    const int m = blockIdx.x, t = threadIdx.x;
    const float *xr = x + (size_t)m * ldx;
    float v[NCH][E];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int i0 = 8192 * c + E * t;
        if (i0 < K) {
#pragma unroll
            for (int q = 0; q < E / 4; ++q) {
                const float4 a = *reinterpret_cast<const float4 *>(xr + i0 + 4 * q);
                v[c][4 * q] = a.x, v[c][4 * q + 1] = a.y, v[c][4 * q + 2] = a.z, v[c][4 * q + 3] = a.w;
            }
            if (BLOCK > 0 && signs) {
#pragma unroll
                for (int q = 0; q < E / 4; ++q) {
                    const float4 s = *reinterpret_cast<const float4 *>(signs + i0 + 4 * q);
                    v[c][4 * q] = v[c][4 * q] * s.x, v[c][4 * q + 1] = v[c][4 * q + 1] * s.y;
                    v[c][4 * q + 2] = v[c][4 * q + 2] * s.z, v[c][4 * q + 3] = v[c][4 * q + 3] * s.w;
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e) v[c][e] = 0.0f;
        }
    }
#pragma unroll
    for (int h = 1; h < (BLOCK < E ? BLOCK : E); h <<= 1)
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int e = 0; e < E; ++e)
                if ((e & h) == 0) {
                    const float a = v[c][e], b = v[c][e + h];
                    v[c][e] = a + b;
                    v[c][e + h] = a - b;
                }
    auto cross = [&](auto lxc) {
        constexpr int LX = decltype(lxc)::value;
        const bool upper = (t & LX) != 0;
        float o[NCH][E];
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int e = 0; e < E; ++e) o[c][e] = lane_xor<LX>(v[c][e]);
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int e = 0; e < E; ++e) v[c][e] = upper ? o[c][e] - v[c][e] : v[c][e] + o[c][e];
    };
    if constexpr (BLOCK > 32) cross(std::integral_constant<int, 1>{});
    if constexpr (BLOCK > 64) cross(std::integral_constant<int, 2>{});
    if constexpr (BLOCK > 128) cross(std::integral_constant<int, 4>{});
    if constexpr (BLOCK > 256) cross(std::integral_constant<int, 8>{});
    if constexpr (BLOCK > 512) cross(std::integral_constant<int, 16>{});
    if constexpr (BLOCK > 1024) cross(std::integral_constant<int, 32>{});

    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int i0 = 8192 * c + E * t;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            if constexpr (BLOCK > 0) v[c][e] = v[c][e] * norm;
            amax = fmaxf(amax, fabsf(v[c][e]));   // elements past K are zero
        }
        if (xrot && i0 < K) {
            float *o = xrot + (size_t)m * ldr + i0;
#pragma unroll
            for (int q = 0; q < E / 4; ++q)
                *reinterpret_cast<float4 *>(o + 4 * q) =
                    make_float4(v[c][4 * q], v[c][4 * q + 1], v[c][4 * q + 2], v[c][4 * q + 3]);
        }
    }
    if (!xq) return;
    amax = block_max(amax, red);
    const bool zero = amax < 1e-12f;
    const float inv = zero ? 0.0f : 127.0f / amax;
    if (t == 0 && xs) xs[m] = zero ? 1.0f : amax * (1.0f / 127.0f);
    int8_t *qr = xq + (size_t)m * ldq;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int i0 = 8192 * c + E * t;
        if (i0 >= K) continue;
        uint32_t w[E / 4];
#pragma unroll
        for (int q = 0; q < E / 4; ++q) {
            uint32_t d = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) d |= (uint32_t)(uint8_t)(zero ? 0 : quant_one(v[c][4 * q + b], inv)) << (8 * b);
            w[q] = d;
        }
#pragma unroll
        for (int q = 0; q < E / 16; ++q)
            *reinterpret_cast<uint4 *>(qr + i0 + 16 * q) = make_uint4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
    }
    for (int i = K + t; i < ldq; i += kThreads) qr[i] = 0;
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
    const bool aligned = ((uintptr_t)x & 15) == 0 && ldx % 4 == 0 && ((uintptr_t)signs & 15) == 0 &&
                         (!xq || (((uintptr_t)xq & 15) == 0 && ldq % 16 == 0)) &&
                         (!xrot || (((uintptr_t)xrot & 15) == 0 && ldr % 4 == 0));
    if (aligned && K % 32 == 0 && K <= 16384 && block <= 2048) {
        const int nch = K <= 8192 ? 1 : 2;
        int lb = -1;
        for (int b = block; b > 0; b >>= 1) ++lb;
#define EIF_PREP_T32(B)                                                                                         \
    case B:                                                                                                     \
        if (nch == 1)                                                                                           \
            prep_rows_t32_kernel<(1 << B), 1>                                          \
                <<<M, kThreads, 0, st>>>(x, ldx, signs, K, norm, xq, ldq, xs, xrot, ldr);                       \
        else                                                                                                    \
            prep_rows_t32_kernel<(1 << B), 2>                                          \
                <<<M, kThreads, 0, st>>>(x, ldx, signs, K, norm, xq, ldq, xs, xrot, ldr);                       \
        break;
        switch (lb) {
        case -1:
            if (nch == 1)
                prep_rows_t32_kernel<0, 1><<<M, kThreads, 0, st>>>(x, ldx, signs, K, norm, xq, ldq, xs, xrot, ldr);
            else
                prep_rows_t32_kernel<0, 2><<<M, kThreads, 0, st>>>(x, ldx, signs, K, norm, xq, ldq, xs, xrot, ldr);
            break;
            EIF_PREP_T32(0)
            EIF_PREP_T32(1)
            EIF_PREP_T32(2)
            EIF_PREP_T32(3)
            EIF_PREP_T32(4)
            EIF_PREP_T32(5)
            EIF_PREP_T32(6)
            EIF_PREP_T32(7)
            EIF_PREP_T32(8)
            EIF_PREP_T32(9)
            EIF_PREP_T32(10)
            EIF_PREP_T32(11)
        }
#undef EIF_PREP_T32
        EIF_HIP_LAUNCHED();
        return EIF_HIP_OK;
    }
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

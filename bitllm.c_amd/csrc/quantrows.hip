// quantrows.hip -- FP32 weight rows -> the INT8 / INT4 row-scaled formats of eif_hip_qweight_create, on the GPU.
//
// The arithmetic of the reference's GGUF import, quant_rows (src/eif_qwen35_gguf.c:225-258), applied to rows it
// has dequantised: amax = max(1e-8, max |x|), s = amax * (1 / qmax) (qmax 127 for INT8, 7 for INT4), inv = 1 / s,
// q = round-half-even(x * inv) clamped to the format's range (the source writes s = amax / qmax; the reference's
// -ffast-math build multiplies by the reciprocal, which is what its images hold); INT4 stores columns (2i, 2i+1) in byte i as
// ((a + 8) << 4) | (b + 8), a zero column padding an odd count. A NaN input takes the code the reference's x86
// conversion gives it after the clamp (the lowest).
#include "hip_common.h"

namespace {

EIF_DEV int round_code(float v, int lo, int hi)
{
    if (!(v == v)) return lo;
    const int q = (int)rintf(v);
    return q > hi ? hi : (q < lo ? lo : q);
}

// One workgroup per row: the row's absmax (NaN ignored, as the reference's comparison ignores it), then the codes.
__global__ __launch_bounds__(256) void quant_rows_kernel(const float *x, int ldx, int cols, int bits, uint8_t *dst,
                                                         size_t rb, float *scales)
{
    __shared__ float red[4];
    const int r = blockIdx.x, t = threadIdx.x;
    const float *xr = x + (size_t)r * ldx;
    float m = 0.0f;
    for (int c = t; c < cols; c += blockDim.x) m = fmaxf(m, fabsf(xr[c]));
    m = eif_wave_max(m);
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), 1e-8f);
    const float rq = bits == 8 ? 1.0f / 127.0f : 1.0f / 7.0f;
    const float sc = amax * rq, inv = 1.0f / sc;
    if (t == 0) scales[r] = sc;
    uint8_t *o = dst + (size_t)r * rb;
    if (bits == 8) {
        for (int c = t; c < cols; c += blockDim.x) o[c] = (uint8_t)(int8_t)round_code(xr[c] * inv, -128, 127);
    } else {
        for (size_t i = t; i < rb; i += blockDim.x) {
            const int c = (int)(2 * i);
            const int a = round_code(xr[c] * inv, -8, 7);
            const int b = c + 1 < cols ? round_code(xr[c + 1] * inv, -8, 7) : 0;
            o[i] = (uint8_t)(((a + 8) << 4) | ((b + 8) & 0x0F));
        }
    }
}

}  // namespace

extern "C" int eif_hip_quant_rows(const float *x, int ldx, int rows, int cols, int bits, uint8_t *dst, float *scales,
                                  void *stream)
{
    if (rows < 0 || cols < 1 || (bits != 4 && bits != 8) || ldx < cols) return EIF_HIP_E_ARG;
    if (rows == 0) return EIF_HIP_OK;
    if (!x || !dst || !scales) return EIF_HIP_E_ARG;
    const size_t rb = bits == 8 ? (size_t)cols : (size_t)(cols + 1) / 2;
    quant_rows_kernel<<<rows, 256, 0, (hipStream_t)stream>>>(x, ldx, cols, bits, dst, rb, scales);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

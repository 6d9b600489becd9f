/*
 * eif_gpu_bitnet.h -- the reference's GPU seat for the ternary GEMV, served by libbitllm_hip.so on one MI355X.
 *
 * The reference's optional GPU backend (include/eif_gpu.h of tevfik/bitllm.c) declares
 * eif_gpu_matmul_bitnet_f32 as the plug-in point for this GEMV. Its own definition is a stub that returns
 * false, so every caller runs its CPU kernel (src/eif_gpu.c:897-902). This library exports the symbol with the
 * seat's contract. A build that drops the stub from src/eif_gpu.c and links libbitllm_hip.so gets the MI355X
 * kernel. The context type below has the reference's layout (include/eif_gpu.h:31-36), and a translation unit
 * that already included the reference header keeps that one.
 */
#ifndef EIF_GPU_BITNET_H
#define EIF_GPU_BITNET_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef EIF_GPU_H
typedef struct {
    bool is_available;
    char backend_name[64];
    char device_name[256];
    void *internal_handle;
} eif_gpu_context_t;
#endif

/* output[r] = scales[r] * sum_c W[r][c] input[c] + bias[r] (scales NULL = 1, bias NULL = 0), W in the 2-bit
 * row-major format of eif_matmul_bitnet_f32, all pointers host memory. ctx is not read (it may be NULL).
 * Returns true when the GPU computed the output, and false when the caller must run its CPU kernel: no usable
 * gfx950 device, invalid sizes, or a HIP error during the call. The call never aborts, whatever
 * eif_hip_set_host_error_mode says: a failure is recorded for the calling thread (eif_hip_host_last_error) and
 * false returned. The weights stay resident, as for eif_matmul_bitnet_f32.
 *                                                                        ref: include/eif_gpu.h:55-70 */
bool eif_gpu_matmul_bitnet_f32(eif_gpu_context_t *ctx, const uint8_t *weights, const float *scales,
                               const float *input, const float *bias, float *output, int rows, int cols);

#ifdef __cplusplus
}
#endif

#endif

// gguf_ternary.cpp -- BitNet projection tensors of a GGUF file (TL1 / TL2 ternary blocks, or Q8_0 taken by sign)
// -> the reference's 2-bit rows with one scale per row, and from there a resident ternary weight.
//
// The conversion of the reference's GGUF loader, load_projection_tensor (src/eif_tinyllm.c:3351-3400):
//   TL1 / TL2 (types 34, 35): 32-column blocks of 10 bytes, an fp16 scale then 8 bytes of 2-bit codes in the
//     reference's own packing, copied as they are; row scale = sum of the block scales in block order times
//     1 / blocks (the reference's s_sum / blocks as its -ffast-math build computes it: blocks is loop-invariant,
//     so the division becomes a multiply by the reciprocal)
//   Q8_0 (type 8): 32-column blocks of 34 bytes, an fp16 scale then 32 int8 values; code +1 / -1 / 0 by the
//     value's sign; row scale as above
// The reference copies a TL row's last block whole, past the row's end when cols is not a multiple of 32; here
// the copy stops at the row's end.
#include <cstring>
#include <new>
#include <vector>

#include "../../include/eif_hip.h"
#include "host_formats.h"

using eif::half_to_float;

extern "C" int eif_gguf_ternary_rows(int gguf_type, const void *src, int rows, int cols, uint8_t *codes,
                                     float *scales)
{
    if (!src || !codes || !scales || rows < 0 || cols < 1) return EIF_HIP_E_ARG;
    if (gguf_type != 8 && gguf_type != 34 && gguf_type != 35) return EIF_HIP_E_ARG;
    const int blocks = (cols + 31) / 32;
    const size_t rb = (size_t)(cols + 3) / 4, bb = gguf_type == 8 ? 34 : 10;
    const uint8_t *s = static_cast<const uint8_t *>(src);
    for (int r = 0; r < rows; r++) {
        const uint8_t *rs = s + (size_t)r * blocks * bb;
        uint8_t *rd = codes + (size_t)r * rb;
        if (gguf_type == 8) std::memset(rd, 0, rb);
        float sum = 0.0f;
        for (int b = 0; b < blocks; b++) {
            const uint8_t *blk = rs + (size_t)b * bb;
            uint16_t h;
            std::memcpy(&h, blk, 2);
            sum += half_to_float(h);
            if (gguf_type != 8) {
                const size_t off = (size_t)b * 8, n = off + 8 <= rb ? 8 : rb - off;
                std::memcpy(rd + off, blk + 2, n);
            } else {
                const int8_t *q = reinterpret_cast<const int8_t *>(blk + 2);
                const int count = b == blocks - 1 ? cols - b * 32 : 32;
                for (int i = 0; i < count; i++) {
                    const int c = b * 32 + i;
                    const uint8_t code = q[i] > 0 ? 1 : (q[i] < 0 ? 2 : 0);
                    rd[c / 4] |= (uint8_t)(code << ((c % 4) * 2));
                }
            }
        }
        scales[r] = blocks > 0 ? sum * (1.0f / (float)blocks) : 1.0f;
    }
    return EIF_HIP_OK;
}

extern "C" int eif_hip_qweight_from_gguf_ternary(eif_hip_qweight **out, int gguf_type, const void *src, int rows,
                                                 int cols, void *stream)
{
    if (!out || rows < 1 || cols < 1) return EIF_HIP_E_ARG;
    std::vector<uint8_t> codes;
    std::vector<float> scales;
    try {
        codes.resize((size_t)rows * ((cols + 3) / 4));
        scales.resize(rows);
    } catch (...) {
        return EIF_HIP_E_NOMEM;
    }
    const int rc = eif_gguf_ternary_rows(gguf_type, src, rows, cols, codes.data(), scales.data());
    if (rc) return rc;
    return eif_hip_qweight_create(out, EIF_HIP_W_TERNARY, rows, cols, 0, codes.data(), scales.data(), 0, stream);
}

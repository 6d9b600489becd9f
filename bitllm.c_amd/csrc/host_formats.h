// host_formats.h -- host-side helpers shared by the model-file readers (gguf_ternary.cpp, gguf_model.cpp,
// svlm.cpp): IEEE binary16 decoding and the reordering of q / k rows from interleaved to half-split RoPE pairs.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <vector>

namespace eif {

inline float half_to_float(uint16_t h)   // IEEE binary16 -> binary32, exact
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu, bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {   // subnormal: normalise
            int e = -1;
            do {
                mant <<= 1;
                ++e;
            } while (!(mant & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3FFu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Rows of a q or k projection ordered for RoPE on interleaved pairs (2j, 2j+1) -> ordered for half-split pairs
// (j, j + head_dim / 2): within each head, row 2j moves to j and row 2j + 1 to j + head_dim / 2, with its scale
// (one per row). Rotating the reordered output by half-split pairs equals rotating the original by interleaved
// pairs (the same cos / sin index j per pair, src/eif_tinyllm.c:481-507), and q.k over a head sums the same
// products. codes: [n_heads * head_dim, row_bytes]; scales: [n_heads * head_dim] or NULL.
inline void rope_rows_to_half_split(uint8_t *codes, size_t row_bytes, float *scales, int n_heads, int head_dim)
{
    const int half = head_dim / 2;
    std::vector<uint8_t> tmp((size_t)head_dim * row_bytes);
    std::vector<float> ts((size_t)head_dim);
    for (int h = 0; h < n_heads; ++h) {
        uint8_t *c = codes + (size_t)h * head_dim * row_bytes;
        float *s = scales ? scales + (size_t)h * head_dim : nullptr;
        for (int j = 0; j < half; ++j) {
            std::memcpy(&tmp[(size_t)j * row_bytes], c + (size_t)(2 * j) * row_bytes, row_bytes);
            std::memcpy(&tmp[(size_t)(j + half) * row_bytes], c + (size_t)(2 * j + 1) * row_bytes, row_bytes);
            if (s) ts[j] = s[2 * j], ts[j + half] = s[2 * j + 1];
        }
        std::memcpy(c, tmp.data(), tmp.size());
        if (s) std::memcpy(s, ts.data(), ts.size() * sizeof(float));
    }
}

}  // namespace eif

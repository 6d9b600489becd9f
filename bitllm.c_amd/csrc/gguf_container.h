// gguf_container.h -- host-side pieces of the GGUF container shared by the model-file readers (gguf_model.cpp,
// qwen35_gguf.cpp): the file mapped read-only, bounds-checked reads, value skipping, block geometry and the
// dequantisation of one row.
//
// GGUF, little-endian: 'GGUF', version u32, tensor count u64, metadata count u64; the metadata pairs (key string,
// value type u32, value); per tensor its name string, dimension count u32, dimensions u64 (the first is the row
// length), ggml type u32 and offset u64 from the data start; the data start is the end of the tensor table
// rounded up to general.alignment. A string is a u64 length then its bytes; value types 0/1 u8/i8, 2/3 u16/i16,
// 4/5/6 u32/i32/f32, 7 bool, 8 string, 9 array (element type u32, count u64, elements), 10/11/12 u64/i64/f64.
#pragma once

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <string>

#include "host_formats.h"

namespace eif {
namespace gguf {

constexpr uint32_t kMagic = 0x46554747u;
constexpr int kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ4_1 = 3, kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kBF16 = 30,
              kTL1 = 34, kTL2 = 35;

struct Mapped {   // a file, memory-mapped read-only
    const uint8_t *p = nullptr;
    size_t n = 0;
    Mapped() = default;
    Mapped(const Mapped &) = delete;
    Mapped &operator=(const Mapped &) = delete;
    ~Mapped()
    {
        if (p) munmap(const_cast<uint8_t *>(p), n);
    }
    bool open(const char *path)
    {
        const int fd = ::open(path, O_RDONLY);
        if (fd < 0) return false;
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size <= 0) {
            ::close(fd);
            return false;
        }
        void *a = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        if (a == MAP_FAILED) return false;
        p = static_cast<const uint8_t *>(a), n = (size_t)st.st_size;
        return true;
    }
};

struct Cursor {   // bounds-checked reads; ok turns false at the first read past the end
    const uint8_t *b;
    size_t n, at = 0;
    bool ok = true;
    template <class T>
    T get()
    {
        T v{};
        if (!ok || n - at < sizeof(T)) {
            ok = false;
            return v;
        }
        std::memcpy(&v, b + at, sizeof(T));
        at += sizeof(T);
        return v;
    }
    void skip(uint64_t k)
    {
        if (!ok || k > n - at) {
            ok = false;
            return;
        }
        at += (size_t)k;
    }
    std::string str()
    {
        const uint64_t l = get<uint64_t>();
        if (!ok || l > n - at) {
            ok = false;
            return {};
        }
        std::string s(reinterpret_cast<const char *>(b + at), (size_t)l);
        at += (size_t)l;
        return s;
    }
};

inline int scalar_size(uint32_t t)   // bytes of a fixed-size value type, 0 for string / array / unknown
{
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

inline void skip_value(Cursor &c, uint32_t t, int depth = 0)
{
    if (const int s = scalar_size(t)) return c.skip((uint64_t)s);
    if (t == 8) {
        c.skip(c.get<uint64_t>());
        return;
    }
    if (t != 9 || depth > 2) {
        c.ok = false;
        return;
    }
    const uint32_t et = c.get<uint32_t>();
    const uint64_t count = c.get<uint64_t>();
    if (const int s = scalar_size(et)) {
        if (count > (c.n - c.at) / (uint64_t)s) c.ok = false;
        else c.skip(count * (uint64_t)s);
        return;
    }
    for (uint64_t i = 0; i < count && c.ok; ++i) skip_value(c, et, depth + 1);
}

struct Tensor {
    uint32_t type = 0, n_dims = 0;
    uint64_t ne[4] = {1, 1, 1, 1}, offset = 0;
};

// bytes and values of one block of a row-blocked type (values 1 for the element types), 0 bytes when unknown
inline void block_geom(int t, int &bytes, int &values)
{
    values = 1;
    switch (t) {
    case kF32: bytes = 4; break;
    case kF16: case kBF16: bytes = 2; break;
    case kQ4_0: bytes = 18, values = 32; break;
    case kQ4_1: bytes = 20, values = 32; break;
    case kQ8_0: bytes = 34, values = 32; break;
    case kQ4_K: bytes = 144, values = 256; break;
    case kQ5_K: bytes = 176, values = 256; break;
    case kQ6_K: bytes = 210, values = 256; break;
    default: bytes = 0;
    }
}

inline float half_at(const uint8_t *p)
{
    uint16_t h;
    std::memcpy(&h, p, 2);
    return half_to_float(h);
}

// One row of whole blocks (cols a multiple of the block) -> floats, ggml's published block layouts, as the
// reference's dequantisers compute them (src/eif_tinyllm.c:3166-3256, src/eif_qwen35_gguf.c:112-187). The block
// fields are fp16, so every product below is exact and each value takes one rounding whatever the order.
//   F32, F16 (exact), BF16 (the 16 high bits of a binary32)
//   Q8_0  34 bytes / 32 values: d, 32 int8; y = d * q
//   Q4_0  18 bytes / 32 values: d, then 16 bytes; value j = (low nibble of byte j) - 8, value 16 + j = (high) - 8;
//         y = q * d
//   Q4_1  20 bytes / 32 values: d, m, 16 bytes as Q4_0 without the -8; y = q * d + m
//   Q4_K  144 bytes / 256 values: d, dmin, 12 bytes of eight 6-bit (scale, min) pairs, 128 bytes of nibbles; per
//         64 values, 32 bytes: their low nibbles with pair 2i, then their high nibbles with pair 2i + 1;
//         y = (d * scale) * q - dmin * min. Pair j < 4: scale = b[j] & 63, min = b[j + 4] & 63; j >= 4: scale =
//         (b[j + 4] & 15) | (b[j - 4] >> 6) << 4, min = (b[j + 4] >> 4) | (b[j] >> 6) << 4
//   Q5_K  176 bytes / 256 values: d, dmin, 12 bytes of pairs as Q4_K, 32 bytes of fifth bits (qh), 128 bytes of
//         nibbles; per 64 values i (0..3) as Q4_K, the low-nibble half adding 16 where qh[l] has bit 2i, the high
//         half where it has bit 2i + 1
//   Q6_K  210 bytes / 256 values: 128 bytes low nibbles (ql), 64 bytes of 2-bit pairs (qh), 16 int8 scales, d;
//         per 128 values (ql 64 bytes, qh 32, scales 8), for l < 32 with s = l / 16:
//         value l      = (ql[l] & 15 | (qh[l] & 3) << 4) - 32,           scale s
//         value l + 32 = (ql[l + 32] & 15 | (qh[l] >> 2 & 3) << 4) - 32, scale s + 2
//         value l + 64 = (ql[l] >> 4 | (qh[l] >> 4 & 3) << 4) - 32,      scale s + 4
//         value l + 96 = (ql[l + 32] >> 4 | (qh[l] >> 6) << 4) - 32,     scale s + 6;   y = (d * scale) * q
inline void dequant_row(int type, const uint8_t *b, int cols, float *y)
{
    switch (type) {
    case kF32:
        std::memcpy(y, b, (size_t)cols * 4);
        return;
    case kF16:
        for (int i = 0; i < cols; ++i) y[i] = half_at(b + 2 * (size_t)i);
        return;
    case kBF16:
        for (int i = 0; i < cols; ++i) {
            uint16_t h;
            std::memcpy(&h, b + 2 * (size_t)i, 2);
            const uint32_t u = (uint32_t)h << 16;
            std::memcpy(&y[i], &u, 4);
        }
        return;
    case kQ8_0:
        for (int i = 0; i < cols / 32; ++i, b += 34) {
            const float d = half_at(b);
            for (int j = 0; j < 32; ++j) y[32 * i + j] = d * (float)(int8_t)b[2 + j];
        }
        return;
    case kQ4_0:
    case kQ4_1: {
        const int bb = type == kQ4_0 ? 18 : 20;
        for (int i = 0; i < cols / 32; ++i, b += bb) {
            const float d = half_at(b), m = type == kQ4_1 ? half_at(b + 2) : 0.0f;
            const uint8_t *qs = b + bb - 16;
            for (int j = 0; j < 16; ++j) {
                const int lo = qs[j] & 15, hi = qs[j] >> 4;
                if (type == kQ4_0) {
                    y[32 * i + j] = (float)(lo - 8) * d;
                    y[32 * i + j + 16] = (float)(hi - 8) * d;
                } else {
                    y[32 * i + j] = (float)lo * d + m;
                    y[32 * i + j + 16] = (float)hi * d + m;
                }
            }
        }
        return;
    }
    case kQ4_K:
    case kQ5_K: {
        const int bb = type == kQ4_K ? 144 : 176;
        for (int i = 0; i < cols / 256; ++i, b += bb) {
            const float d = half_at(b), dmin = half_at(b + 2);
            const uint8_t *sm = b + 4, *qh = b + 16, *qs = b + bb - 128;
            float *o = y + 256 * i;
            for (int j = 0; j < 8; ++j) {
                int sc, mn;
                if (j < 4) {
                    sc = sm[j] & 63, mn = sm[j + 4] & 63;
                } else {
                    sc = (sm[j + 4] & 15) | ((sm[j - 4] >> 6) << 4);
                    mn = (sm[j + 4] >> 4) | ((sm[j] >> 6) << 4);
                }
                const float ds = d * (float)sc, dm = dmin * (float)mn;
                const uint8_t *q = qs + 32 * (j / 2);
                for (int l = 0; l < 32; ++l) {
                    int v = (j & 1) ? q[l] >> 4 : q[l] & 15;
                    if (type == kQ5_K && (qh[l] >> j) & 1) v += 16;
                    o[32 * j + l] = ds * (float)v - dm;
                }
            }
        }
        return;
    }
    case kQ6_K:
        for (int i = 0; i < cols / 256; ++i, b += 210) {
            const float d = half_at(b + 208);
            for (int n = 0; n < 2; ++n) {
                const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n;
                const int8_t *sc = reinterpret_cast<const int8_t *>(b + 192) + 8 * n;
                float *o = y + 256 * i + 128 * n;
                for (int l = 0; l < 32; ++l) {
                    const int s = l / 16;
                    const int q[4] = {((ql[l] & 15) | ((qh[l] & 3) << 4)) - 32,
                                      ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32,
                                      ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32,
                                      ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32};
                    for (int k = 0; k < 4; ++k) o[32 * k + l] = d * (float)sc[s + 2 * k] * (float)q[k];
                }
            }
        }
        return;
    default:
        return;
    }
}

}  // namespace gguf
}  // namespace eif

// f32linear.hip -- GEMVs with FP32 activations (what the reference engines run on x86), plus the INT8-in/INT8-out
// ternary GEMV.
//
// The main path reads a resident repacked copy of the weights ("row tiles"): tiles of 4 rows, each cut into
// chunks of one 32-bit word per row (16 ternary, 8 INT4 or 4 INT8 columns), a chunk being one 16-byte load for
// a lane. Tile t's chunks are contiguous. Column j of a chunk sits at bits 8 (j % 4) + B (j / 4) of its row's
// word (B bits per weight), so one shift and one mask bring four columns into the four bytes of a register,
// where the byte-to-float conversions read them. Codes are unsigned with an offset OFF: ternary t + 1, INT4
// the reference's nibble (value nibble - 8), INT8 w + 128; a row's sum is sum(v x) - OFF sum(x). A wave keeps
// its columns of x in registers and streams row tiles; lane l owns chunks l, l + 64, ... of every tile.
//
// The row-major kernels after it read the reference layouts in place, one wave per output row: the path for
// K > 8192 and for block scales whose block is not a multiple of 16 columns. FP32 sums are within the reference
// tests' normalised bounds (summation order differs).
#include <algorithm>

#include "hip_common.h"

namespace {

using namespace eif;

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

// ---- row tiles ----

constexpr int kF32MaxCols = 8192;   // x stays in registers: at most 128 floats per lane
constexpr int kF32Threads = 256;

template <int FMT>
struct F32Fmt {
    static constexpr int B = FMT == kF32Tern ? 2 : (FMT == kF32Int4 ? 4 : 8);   // bits per weight
    static constexpr int CPC = 32 / B;                                           // columns per chunk
    static constexpr float OFF = FMT == kF32Tern ? 1.0f : (FMT == kF32Int4 ? 8.0f : 128.0f);
    static constexpr uint32_t MASK = B == 2 ? 0x03030303u : (B == 4 ? 0x0F0F0F0Fu : 0xFFFFFFFFu);
};

// The stored code of column c of row r (the offset code of a zero for padding).
EIF_DEV uint32_t src_code(const uint8_t *__restrict__ src, int sf, int rows, int cols, int r, int c)
{
    if (r >= rows || c >= cols) return sf == kSrcInt4 ? 8u : (sf == kSrcInt8 ? 128u : 1u);
    if (sf == kSrcTernRow || sf == kSrcTernIl) {
        const int rb = (cols + 3) / 4, j = c >> 2;
        const uint8_t *p = (sf == kSrcTernIl && r < (rows & ~3)) ? src + (size_t)(r & ~3) * rb + 4 * (size_t)j + (r & 3)
                                                                 : src + (size_t)r * rb + j;
        const uint32_t code = (*p >> (2 * (c & 3))) & 3u;
        return code == 1u ? 2u : (code == 2u ? 0u : 1u);
    }
    if (sf == kSrcDense) {
        uint32_t t = src[(size_t)r * ((cols + 4) / 5) + c / 5];
        for (int i = c % 5; i > 0; --i) t /= 3u;
        const uint32_t d = t % 3u;
        return d == 1u ? 2u : (d == 2u ? 0u : 1u);
    }
    if (sf == kSrcInt4) {
        const uint32_t b = src[(size_t)r * ((cols + 1) / 2) + (c >> 1)];
        return (c & 1) ? (b & 15u) : (b >> 4);
    }
    return (uint32_t)((int)(int8_t)src[(size_t)r * cols + c] + 128);
}

// One thread per (tile, chunk, row of the tile): that row's word of the chunk.
__global__ __launch_bounds__(256) void f32_repack_kernel(const uint8_t *__restrict__ src, int sf, int B,
                                                         uint32_t *__restrict__ dst, int rows, int cols, int S,
                                                         size_t nwords)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nwords) return;
    const int i = (int)(idx & 3);
    const size_t tc = idx >> 2;
    const int t = (int)(tc / (size_t)S), c = (int)(tc % (size_t)S);
    const int cpc = 32 / B;
    uint32_t w = 0;
    for (int j = 0; j < cpc; ++j)
        w |= src_code(src, sf, rows, cols, 4 * t + i, cpc * c + j) << (8 * (j & 3) + B * (j >> 2));
    dst[idx] = w;
}

// w & m, opaque to the compiler: seeing the mask, it would extract every field of the word with its own bit-field
// extract before converting it, where one AND and the byte-to-float conversions do.
EIF_DEV uint32_t and_opaque(uint32_t w, uint32_t m)
{
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(w), "s"(m));
    return r;
}

// Sum over 64 lanes of four values at once: lanes 16 q .. 16 q + 15 return the sum of v_q.
EIF_DEV float wave_sum4(float v0, float v1, float v2, float v3, int lane)
{
    const bool h32 = lane & 32, h16 = lane & 16;
    float k0 = h32 ? v2 : v0, k1 = h32 ? v3 : v1;
    k0 += __shfl_xor(h32 ? v0 : v2, 32, 64);
    k1 += __shfl_xor(h32 ? v1 : v3, 32, 64);
    float k = h16 ? k1 : k0;
    k += __shfl_xor(h16 ? k0 : k1, 16, 64);
    k += xlane<8>(k);
    k += xlane<4>(k);
    k += xlane<2>(k);
    k += xlane<1>(k);
    return k;
}

// y[r] = scale * sum_c w[r][c] x[c] + bias[r] over row tiles. A workgroup holds NG groups of KS waves; the KS
// waves of a group take the same TW row tiles and split the passes of 64 chunks between them (wave k: passes k,
// k + KS, ...; P at least the passes one wave needs, those past them skipped wave-uniformly), their sums combined
// through LDS. Groups stride over the matrix's groups of TW tiles (the latency of one group's loads hidden by
// the other waves of the SIMD, up to eight). GRP: block scales in the [tile][block][4 rows] copy S4, each chunk inside
// one block (cpb chunks a block); else one scale a row, rscale (NULL = 1).
template <int FMT, int P, int TW, int KS, bool GRP>
__global__ __launch_bounds__(KS > 4 ? 64 * KS : kF32Threads) void f32_tiles_kernel(const uint4 *__restrict__ W,
                                                                const float4 *__restrict__ S4,
                                                                const float *__restrict__ rscale, int nb, int cpb,
                                                                const float *__restrict__ x,
                                                                const float *__restrict__ bias,
                                                                float *__restrict__ y, int rows, int cols, int S,
                                                                int ntiles)
{
    using F = F32Fmt<FMT>;
    constexpr int CPC = F::CPC, NG = KS >= 4 ? 1 : 4 / KS;
    __shared__ float red[2][NG][KS][TW * 4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ks = wave % KS, tg = wave / KS;
    const int np = (S + 63) >> 6, ngroups = (ntiles + TW - 1) / TW, gstride = gridDim.x * NG;

    // this wave's columns of x (raw; scaled below, after the first group's loads are on their way)
    float xr[P][CPC], xsum[P];
    int blk[P];
    bool live[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int q = ks + KS * p, c = lane + 64 * q;
        live[p] = q < np;
        xsum[p] = 0.0f;
        blk[p] = 0;
#pragma unroll
        for (int j = 0; j < CPC; ++j) xr[p][j] = 0.0f;
        if (live[p] && c < S) {
            const int c0 = CPC * c;
            if (c0 + CPC <= cols) {
#pragma unroll
                for (int j = 0; j < CPC; j += 4) {
                    const float4 v = *reinterpret_cast<const float4 *>(x + c0 + j);
                    xr[p][j] = v.x;
                    xr[p][j + 1] = v.y;
                    xr[p][j + 2] = v.z;
                    xr[p][j + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < CPC; ++j)
                    if (c0 + j < cols) xr[p][j] = x[c0 + j];
            }
            if constexpr (GRP) blk[p] = c / cpb;
        }
    }

    // A group's loads: its codes (and block scales), and the scale and bias of the rows this lane writes. Indices
    // past the matrix are clamped to its last tile and chunk, so every load is in bounds and unconditional: a
    // chunk past the columns meets x = 0, a tile past the rows is never written.
    struct Grp {
        uint4 w[TW][P];
        float4 s[TW][P];
        float rs[TW], bi[TW];
    };
    auto out_row = [&](int g, int tt) {
        return KS == 1 ? 4 * (g * TW + tt) + (lane >> 4) : 4 * (g * TW + ((lane >> 2) % TW)) + (lane & 3);
    };
    // No branch among the code loads (a pass past the columns loads the last chunk again): the loads of a group are
    // issued back to back, without waits between them.
    auto load = [&](Grp &G, int g) {
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) {
            const int t = min(g * TW + tt, ntiles - 1);
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const int c = min(lane + 64 * (ks + KS * p), S - 1);
                G.w[tt][p] = W[(size_t)t * S + c];
                if constexpr (GRP) G.s[tt][p] = S4[(size_t)t * nb + blk[p]];
            }
        }
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) {
            const int r = min(out_row(g, tt), rows - 1);
            G.rs[tt] = 1.0f;
            G.bi[tt] = 0.0f;
            if constexpr (!GRP) {
                if (rscale) G.rs[tt] = rscale[r];
            }
            if (bias) G.bi[tt] = bias[r];
        }
    };
    float xoff = 0.0f;   // OFF times this wave's share of sum(x), taken off once (no block scales)
    auto work = [&](const Grp &G, int g, int it) {
        float v[TW];
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) {
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int p = 0; p < P; ++p) {
                if (!live[p]) continue;
                const uint32_t wd[4] = {G.w[tt][p].x, G.w[tt][p].y, G.w[tt][p].z, G.w[tt][p].w};
                float sc[4];
                if constexpr (GRP) {
                    sc[0] = G.s[tt][p].x;
                    sc[1] = G.s[tt][p].y;
                    sc[2] = G.s[tt][p].z;
                    sc[3] = G.s[tt][p].w;
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                    for (int k = 0; k < CPC / 4; ++k) {
                        const uint32_t u = F::B == 8 ? wd[i] : and_opaque(wd[i], F::MASK << (F::B * k));
                        float &s = (k & 1) ? s1 : s0;
                        s = fmaf((float)(u & 255u), xr[p][4 * k], s);
                        s = fmaf((float)((u >> 8) & 255u), xr[p][4 * k + 1], s);
                        s = fmaf((float)((u >> 16) & 255u), xr[p][4 * k + 2], s);
                        s = fmaf((float)(u >> 24), xr[p][4 * k + 3], s);
                    }
                    if constexpr (GRP)
                        acc[i] = fmaf(fmaf(-F::OFF, xsum[p], s0 + s1), sc[i], acc[i]);
                    else
                        acc[i] += s0 + s1;
                }
            }
            if constexpr (!GRP) {
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] -= xoff;
            }
            v[tt] = wave_sum4(acc[0], acc[1], acc[2], acc[3], lane);
        }
        // lanes 16 i hold row i of each tile; KS > 1: the group's waves add theirs through LDS
        if constexpr (KS == 1) {
#pragma unroll
            for (int tt = 0; tt < TW; ++tt) {
                const int r = out_row(g, tt);
                if ((lane & 15) == 0 && g < ngroups && r < rows) y[r] = v[tt] * G.rs[tt] + G.bi[tt];
            }
        } else {
            if ((lane & 15) == 0) {
#pragma unroll
                for (int tt = 0; tt < TW; ++tt) red[it & 1][tg][ks][tt * 4 + (lane >> 4)] = v[tt];
            }
            // every wave of the workgroup makes the same trips (the loop below), so all reach this barrier; a
            // buffer is written again two trips later, after the next barrier, which its readers have passed
            __syncthreads();
            if (ks == 0 && lane < TW * 4) {
                float sum = 0.0f;
#pragma unroll
                for (int k = 0; k < KS; ++k) sum += red[it & 1][tg][k][lane];
                const int r = out_row(g, 0);
                if (g < ngroups && r < rows) y[r] = sum * G.rs[0] + G.bi[0];
            }
        }
    };

    int gb = blockIdx.x * NG;   // the workgroup's first group: trips are the same for all its waves
    Grp G;
    load(G, gb + tg);   // on its way while x is summed and scaled
#pragma unroll
    for (int p = 0; p < P; ++p) {
#pragma unroll
        for (int j = 0; j < CPC; ++j) {
            xsum[p] += xr[p][j];
            // column j's code is read as code * 2^(B (j / 4)) from its masked word: scale x by the inverse
            // power of two (exact)
            xr[p][j] *= 1.0f / (float)(1u << (F::B * (j / 4)));
        }
    }
    if constexpr (!GRP) {
#pragma unroll
        for (int p = 0; p < P; ++p) xoff += xsum[p];
        xoff *= F::OFF;
    }
    for (int it = 0; gb < ngroups; gb += gstride, ++it) {
        if (it) load(G, gb + tg);
        work(G, gb + tg, it);
    }
}

int g_f32_tiles_per_wave = 0;   // 0: from the shape
int g_f32_ksplit = 0;           // 0: from the shape

template <int FMT, int P, int TW, int KS, bool GRP>
int launch_tiles_t(const uint4 *W, const float4 *S4, const float *rscale, int nb, int cpb, const float *x,
                   const float *bias, float *y, int rows, int cols, int S, int ntiles, hipStream_t st)
{
    static int cap = 0;
    if (!cap) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cap = cus * 32;   // waves: eight a SIMD
    }
    constexpr int NG = KS >= 4 ? 1 : 4 / KS;
    const int blocks = std::min(eif_ceil_div(eif_ceil_div(ntiles, TW), NG), std::max(1, cap / (KS * NG)));
    f32_tiles_kernel<FMT, P, TW, KS, GRP><<<blocks, 64 * KS * NG, 0, st>>>(W, S4, rscale, nb, cpb, x, bias, y, rows,
                                                                          cols, S, ntiles);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

// Passes a wave takes (P >= ceil(np / KS)): the smallest compiled count that holds them.
template <int FMT, int TW, int KS, bool GRP>
int launch_tiles_p(const uint4 *W, const float4 *S4, const float *rscale, int nb, int cpb, const float *x,
                   const float *bias, float *y, int rows, int cols, int S, int ntiles, hipStream_t st)
{
    const int need = eif_ceil_div(eif_ceil_div(S, 64), KS);
#define EIF_F32_P(PP)                                                                                           \
    if (need <= PP)                                                                                             \
        return launch_tiles_t<FMT, PP, TW, KS, GRP>(W, S4, rscale, nb, cpb, x, bias, y, rows, cols, S, ntiles, st);
    EIF_F32_P(1)
    EIF_F32_P(2)
    EIF_F32_P(3)
    EIF_F32_P(4)
    if constexpr (FMT != kF32Tern) {
        EIF_F32_P(6)
        EIF_F32_P(8)
    }
    if constexpr (FMT == kF32Int8) {
        EIF_F32_P(12)
        EIF_F32_P(16)
    }
#undef EIF_F32_P
    return EIF_HIP_E_LIMIT;
}

// Tiles per wave and waves per tile from the shape (or the knobs): one tile; K split over waves (1, 2, 3, 4 or 8
// ways, at most one a pass) until the launch has 4096 waves and each wave at most 4 (ternary), 8 (INT4) or 12
// (INT8) passes.
template <int FMT, bool GRP>
int launch_tiles(const uint4 *W, const float4 *S4, const float *rscale, int nb, int cpb, const float *x,
                 const float *bias, float *y, int rows, int cols, hipStream_t st)
{
    constexpr int CPC = F32Fmt<FMT>::CPC;
    const int S = eif_ceil_div(cols, CPC), ntiles = eif_ceil_div(rows, 4), np = eif_ceil_div(S, 64);
    const int tw = g_f32_tiles_per_wave ? g_f32_tiles_per_wave : 1;
    int ks = g_f32_ksplit;
    if (!ks) {
        ks = 1;
        const int most = FMT == kF32Tern ? 4 : (FMT == kF32Int4 ? 8 : 12);   // passes a wave takes at most
        while (ks < std::min(8, np) && (eif_ceil_div(ntiles, tw) * ks < 4096 || eif_ceil_div(np, ks) > most))
            ks = ks < 4 ? ks + 1 : 8;
    }
    if (ks > 4) ks = 8;
    const int need = eif_ceil_div(np, ks);
    if (need > (FMT == kF32Tern ? 4 : (FMT == kF32Int4 ? 8 : 16))) ks = 8;   // keep x within the compiled passes
#define EIF_F32_KS(TWV, KSV)                                                                                    \
    if (tw == TWV && ks == KSV)                                                                                 \
        return launch_tiles_p<FMT, TWV, KSV, GRP>(W, S4, rscale, nb, cpb, x, bias, y, rows, cols, S, ntiles, st);
    EIF_F32_KS(1, 1)
    EIF_F32_KS(1, 2)
    EIF_F32_KS(1, 3)
    EIF_F32_KS(1, 4)
    EIF_F32_KS(2, 1)
    EIF_F32_KS(2, 2)
    EIF_F32_KS(2, 3)
    EIF_F32_KS(2, 4)
    EIF_F32_KS(1, 8)
    EIF_F32_KS(2, 8)
#undef EIF_F32_KS
    return EIF_HIP_E_LIMIT;
}

// One thread per (tile, block): the four rows' scales of a block, [rows, nb] -> [tile][block][4].
__global__ __launch_bounds__(256) void f32_scales_kernel(const float *__restrict__ sc, float4 *__restrict__ dst,
                                                         int rows, int nb, size_t n)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const int t = (int)(idx / (size_t)nb), b = (int)(idx % (size_t)nb);
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = 4 * t + i < rows ? sc[(size_t)(4 * t + i) * nb + b] : 0.0f;
    dst[idx] = make_float4(v[0], v[1], v[2], v[3]);
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


size_t f32_tiles_bytes(int fmt, int rows, int cols)
{
    const int cpc = fmt == kF32Tern ? 16 : (fmt == kF32Int4 ? 8 : 4);
    return (size_t)eif_ceil_div(rows, 4) * (size_t)eif_ceil_div(cols, cpc) * 16;
}

size_t f32_scales_bytes(int rows, int cols, int block)
{
    return (size_t)eif_ceil_div(rows, 4) * (size_t)eif_ceil_div(cols, block) * 16;
}

bool f32_tiles_fit(int cols, int block)
{
    return cols > 0 && cols <= kF32MaxCols && (block == 0 || block % 16 == 0);
}

int launch_f32_repack(int src_fmt, const uint8_t *src, void *dst, int rows, int cols, hipStream_t st)
{
    if (rows <= 0 || cols <= 0) return EIF_HIP_OK;
    const int B = src_fmt == kSrcInt4 ? 4 : (src_fmt == kSrcInt8 ? 8 : 2);
    const int S = eif_ceil_div(cols, 32 / B);
    const size_t nwords = (size_t)eif_ceil_div(rows, 4) * (size_t)S * 4;
    f32_repack_kernel<<<(unsigned)((nwords + 255) / 256), 256, 0, st>>>(src, src_fmt, B, (uint32_t *)dst, rows,
                                                                          cols, S, nwords);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

int launch_f32_scales(const float *scales, void *dst, int rows, int cols, int block, hipStream_t st)
{
    if (rows <= 0 || cols <= 0 || block <= 0) return EIF_HIP_OK;
    const int nb = eif_ceil_div(cols, block);
    const size_t n = (size_t)eif_ceil_div(rows, 4) * (size_t)nb;
    f32_scales_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(scales, (float4 *)dst, rows, nb, n);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

int launch_f32_tiles(int fmt, const void *Wt, const float *scales, int block, const float *x, const float *bias,
                     float *y, int rows, int cols, hipStream_t st)
{
    if (rows <= 0 || cols <= 0) return EIF_HIP_OK;
    if (!f32_tiles_fit(cols, block) || ((uintptr_t)x & 15) || (block && fmt != kF32Tern)) return EIF_HIP_E_LIMIT;
    const uint4 *W = static_cast<const uint4 *>(Wt);
    if (fmt == kF32Tern) {
        if (block && scales)
            return launch_tiles<kF32Tern, true>(W, reinterpret_cast<const float4 *>(scales), nullptr,
                                                eif_ceil_div(cols, block), block / 16, x, bias, y, rows, cols, st);
        return launch_tiles<kF32Tern, false>(W, nullptr, block ? nullptr : scales, 0, 1, x, bias, y, rows, cols, st);
    }
    if (fmt == kF32Int4) return launch_tiles<kF32Int4, false>(W, nullptr, scales, 0, 1, x, bias, y, rows, cols, st);
    return launch_tiles<kF32Int8, false>(W, nullptr, scales, 0, 1, x, bias, y, rows, cols, st);
}

}  // namespace eif

extern "C" int eif_hip_set_f32_tiles_per_wave(int tw)
{
    const int old = g_f32_tiles_per_wave;
    if (tw >= 0 && tw <= 2) g_f32_tiles_per_wave = tw;
    return old;
}

extern "C" int eif_hip_set_f32_ksplit(int ks)
{
    const int old = g_f32_ksplit;
    if ((ks >= 0 && ks <= 4) || ks == 8) g_f32_ksplit = ks;
    return old;
}

// qlinear.hip -- INT8-activation linears on int8 MFMA: ternary (group or row scales), INT8 and INT4 (row scales).
//
// One kernel template serves the GEMV (token counts below the GEMM threshold) and the prefill GEMM:
//
//   v_mfma_i32_16x16x32_i8, operand A = activations (16 tokens x 32 k), operand B = weights (32 k x 16 rows).
//   Lane l supplies 8 k-bytes of token / weight row (l & 15) for k-slot (l >> 4); the accumulator lane l holds
//   C[token 4*(l>>4)+v][row l&15], v = 0..3. Because A and B use the same (slot, byte) -> k mapping, any column
//   permutation applied to both is free: the GPU weight layouts below are such permutations, chosen so that
//   one 4..16-byte coalesced load per lane feeds several MFMAs and decoding is 1-2 VALU ops per 4 weights.
//
// GPU weight layouts (written once by the repack kernels; same bytes per weight as the reference formats):
//   ternary, group g = 32*UD: a row is a sequence of steps of 2g columns; a step is 4 slots x UD dwords;
//     dword u of slot s, bit pair p of byte b holds column  2g*step + g*grp + 8*UD*s + 8*(t % UD) + q  with
//     t = 2u + (p >> 1), q = 4*(p & 1) + b, grp = t / UD, as a 2-bit two's-complement value (+1 = 01, -1 = 11).
//     Decoding plane p is ((dword << (6 - 2p)) & 0xC0C0C0C0): int8 bytes equal to 64*w, so the MFMA sums are
//     64x the integer sums and each group's sum is recovered exactly by an arithmetic shift.
//     MFMA t covers one group only (grp = t / UD), so the int32 sum of every (row, group) is produced intact.
//   int4: steps of 128 columns, 4 slots x 4 dwords; dword t of slot s, byte b: high nibble = column
//     128*step + 32*s + 8*t + b, low nibble = that column + 4; nibbles hold v & 15 (two's complement), decoded
//     as (dword & 0xF0F0F0F0) and ((dword << 4) & 0xF0F0F0F0) = 16*v.
//   int8: the reference row-major layout, rows padded; steps of 64 columns, slot s owns bytes 16s..16s+15.
//   Every layout pads rows to a multiple of 64 and columns to a whole number of steps with zero weights.
//
// Accumulation contract (reference: src/eif_quantize_bitnet.c:1143-1203 for the row-scaled epilogue,
// src/eif_quantize_bitnet.c:1227-1296 and src/eif_qwen35.c:228-290 for group-scaled combination):
//   grouped ternary:  acc_g exact int32 per (token, row, group); F = sum_g fmaf((float)acc_g, s[r,g], F) within a
//                     wave, partial F of the K-split waves added in wave order; y = F * xs[m] (+ bias).
//   row-scaled:       isum = exact int32 over all K (K-split partials added as integers);
//                     y = ((float)isum * xs[m]) * s[r] (+ bias).
#include <mutex>
#include <new>

#include "hip_common.h"

namespace {

enum { kTern = EIF_HIP_W_TERNARY, kI8 = EIF_HIP_W_INT8, kI4 = EIF_HIP_W_INT4 };
constexpr int kRowPad = 64;

// Per-format step geometry: SB bytes per lane per step, SC columns per row per step, NMF MFMAs per step,
// SHIFT = log2 of the factor the decoded operand carries.
template <int FMT, int UD>
struct Geo;
template <int UD>
struct Geo<kTern, UD> {
    static constexpr int SB = 4 * UD, SC = 64 * UD, NMF = 2 * UD, SHIFT = 6;
};
template <int UD>
struct Geo<kI4, UD> {
    static constexpr int SB = 16, SC = 128, NMF = 4, SHIFT = 4;
};
template <int UD>
struct Geo<kI8, UD> {
    static constexpr int SB = 16, SC = 64, NMF = 2, SHIFT = 0;
};

template <int N>
EIF_DEV void load_words(const uint8_t *p, uint32_t (&w)[N])
{
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            uint4 v = *reinterpret_cast<const uint4 *>(p + 16 * i);
            w[4 * i] = v.x, w[4 * i + 1] = v.y, w[4 * i + 2] = v.z, w[4 * i + 3] = v.w;
        }
    } else if constexpr (N == 3) {
        uint3 v = *reinterpret_cast<const uint3 *>(p);
        w[0] = v.x, w[1] = v.y, w[2] = v.z;
    } else if constexpr (N == 2) {
        uint2 v = *reinterpret_cast<const uint2 *>(p);
        w[0] = v.x, w[1] = v.y;
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) w[i] = reinterpret_cast<const uint32_t *>(p)[i];
    }
}

// n consecutive 8-byte MFMA operands from an 8-byte aligned address (16-byte loads when aligned to 16).
template <int N, bool A16>
EIF_DEV void load_ops(const int8_t *p, long (&a)[N])
{
    if constexpr (A16 && N % 2 == 0) {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) {
            int4 v = *reinterpret_cast<const int4 *>(p + 16 * i);
            a[2 * i] = (long)(uint32_t)v.x | ((long)(uint32_t)v.y << 32);
            a[2 * i + 1] = (long)(uint32_t)v.z | ((long)(uint32_t)v.w << 32);
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) a[i] = reinterpret_cast<const long *>(p)[i];
    }
}

EIF_DEV long pack2(uint32_t lo, uint32_t hi) { return (long)lo | ((long)hi << 32); }

template <int FMT, int UD>
EIF_DEV void decode(const uint32_t (&w)[Geo<FMT, UD>::SB / 4], long (&b)[Geo<FMT, UD>::NMF])
{
    if constexpr (FMT == kTern) {
#pragma unroll
        for (int u = 0; u < UD; ++u) {
            const uint32_t m = 0xC0C0C0C0u, x = w[u];
            b[2 * u] = pack2((x << 6) & m, (x << 4) & m);
            b[2 * u + 1] = pack2((x << 2) & m, x & m);
        }
    } else if constexpr (FMT == kI4) {
#pragma unroll
        for (int t = 0; t < 4; ++t) b[t] = pack2(w[t] & 0xF0F0F0F0u, (w[t] << 4) & 0xF0F0F0F0u);
    } else {
        b[0] = pack2(w[0], w[1]);
        b[1] = pack2(w[2], w[3]);
    }
}

EIF_DEV v4i mfma(long a, long b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0); }

// Kernel parameters.
struct QArgs {
    const uint8_t *W;      // GPU layout, rows padded to kRowPad
    int wld;               // bytes per padded row
    const float *scales;   // grouped: [N, G]; row-scaled: [N] or NULL
    int G;                 // groups per row (grouped)
    const int8_t *xq;      // [M, ldq]
    int ldq;
    const float *xs;       // [M]
    const float *bias;     // [N] or NULL
    float *y;              // [M, ldy]
    int ldy;
    int32_t *acc;          // parity output or NULL
    int M, N, nsteps;
};

// RT row tiles x TT token tiles per workgroup, KSPLIT waves share a row tile and split its steps.
// V1: only token 0 is live (M == 1), so only accumulator register 0 is converted.
template <int FMT, int UD, bool GROUPED, bool ACC, int RT, int TT, int KSPLIT, bool V1>
__global__ __launch_bounds__(64 * RT * KSPLIT) void qlinear_kernel(QArgs a)
{
    using GE = Geo<FMT, UD>;
    constexpr int NV = V1 ? 1 : 4;
    constexpr int NW = GE::SB / 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kw = wave % KSPLIT, rw = wave / KSPLIT;
    const int r16 = lane & 15, s = lane >> 4;
    const int row = (blockIdx.x * RT + rw) * 16 + r16;
    const int m0 = blockIdx.y * (16 * TT);
    const bool row_ok = row < a.N;

    const uint8_t *wp = a.W + (size_t)row * a.wld + s * GE::SB;
    const int8_t *xp[TT];
    bool tok_ok[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        const int tok = m0 + 16 * tt + r16;
        tok_ok[tt] = tok < a.M;
        xp[tt] = a.xq + (size_t)(tok_ok[tt] ? tok : 0) * a.ldq;
    }

    float F[TT][4];
    v4i C[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        C[tt] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int v = 0; v < 4; ++v) F[tt][v] = 0.0f;
    }

#pragma unroll 2
    for (int st = kw; st < a.nsteps; st += KSPLIT) {
        uint32_t wv[NW];
        load_words<NW>(wp + (size_t)st * 4 * GE::SB, wv);
        long bop[GE::NMF];
        decode<FMT, UD>(wv, bop);
        if constexpr (FMT == kTern) {
#pragma unroll
            for (int grp = 0; grp < 2; ++grp) {
                const int gi = 2 * st + grp;
                float sc = 0.0f;
                if constexpr (GROUPED) {
                    if (row_ok && gi < a.G) sc = a.scales[(size_t)row * a.G + gi];
                }
                const int col = st * GE::SC + 32 * UD * grp + 8 * UD * s;
#pragma unroll
                for (int tt = 0; tt < TT; ++tt) {
                    long aop[UD];
                    if (tok_ok[tt]) {
                        load_ops<UD, (UD % 2 == 0)>(xp[tt] + col, aop);
                    } else {
#pragma unroll
                        for (int i = 0; i < UD; ++i) aop[i] = 0;
                    }
                    v4i c = GROUPED ? v4i{0, 0, 0, 0} : C[tt];
#pragma unroll
                    for (int i = 0; i < UD; ++i) c = mfma(aop[i], bop[grp * UD + i], c);
                    if constexpr (GROUPED) {
#pragma unroll
                        for (int v = 0; v < NV; ++v) {
                            const int g_acc = c[v] >> GE::SHIFT;
                            if constexpr (ACC) {
                                const int tok = m0 + 16 * tt + 4 * s + v;
                                if (row_ok && tok < a.M && gi < a.G)
                                    a.acc[((size_t)tok * a.N + row) * a.G + gi] = g_acc;
                            } else {
                                F[tt][v] = fmaf((float)g_acc, sc, F[tt][v]);
                            }
                        }
                    } else {
                        C[tt] = c;
                    }
                }
            }
        } else {
            const int col = st * GE::SC + (GE::SC / 4) * s;
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) {
                long aop[GE::NMF];
                if (tok_ok[tt]) {
                    load_ops<GE::NMF, true>(xp[tt] + col, aop);
                } else {
#pragma unroll
                    for (int i = 0; i < GE::NMF; ++i) aop[i] = 0;
                }
#pragma unroll
                for (int i = 0; i < GE::NMF; ++i) C[tt] = mfma(aop[i], bop[i], C[tt]);
            }
        }
    }

    if constexpr (GROUPED && ACC) return;

    // K-split reduction through LDS (waves kw > 0 hand their partials to wave kw == 0 of the same row tile).
    if constexpr (KSPLIT > 1) {
        __shared__ float red[RT][KSPLIT - 1][TT][NV][64];
        if (kw > 0) {
#pragma unroll
            for (int tt = 0; tt < TT; ++tt)
#pragma unroll
                for (int v = 0; v < NV; ++v)
                    red[rw][kw - 1][tt][v][lane] = GROUPED ? F[tt][v] : __int_as_float(C[tt][v]);
        }
        __syncthreads();
        if (kw > 0) return;
#pragma unroll
        for (int k = 0; k < KSPLIT - 1; ++k)
#pragma unroll
            for (int tt = 0; tt < TT; ++tt)
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    if constexpr (GROUPED)
                        F[tt][v] += red[rw][k][tt][v][lane];
                    else
                        C[tt][v] += __float_as_int(red[rw][k][tt][v][lane]);
                }
    }

    if (!row_ok) return;
    const float rs = (!GROUPED && a.scales) ? a.scales[row] : 1.0f;
    const float bb = a.bias ? a.bias[row] : 0.0f;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int tok = m0 + 16 * tt + 4 * s + v;
            if (tok >= a.M) continue;
            float out;
            if constexpr (GROUPED) {
                out = F[tt][v] * a.xs[tok];
            } else {
                const int isum = C[tt][v] >> GE::SHIFT;
                if constexpr (ACC) {
                    a.acc[(size_t)tok * a.N + row] = isum;
                    continue;
                }
                out = ((float)isum * a.xs[tok]) * rs;
            }
            if (a.bias) out = out + bb;
            a.y[(size_t)tok * a.ldy + row] = out;
        }
}

// ---- repack kernels: reference formats -> GPU layouts (one thread per destination dword) ----

EIF_DEV int tern_code(const uint8_t *src, int sld, int rows, int cols, int r, int c)
{
    if (r >= rows || c >= cols) return 0;
    unsigned code = (src[(size_t)r * sld + (c >> 2)] >> (2 * (c & 3))) & 3u;
    return code == 1u ? 1 : (code == 2u ? -1 : 0);
}

__global__ void repack_ternary_kernel(const uint8_t *__restrict__ src, int rows, int cols, int ud,
                                      uint32_t *__restrict__ dst, int rows_pad, int dw_per_row)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)rows_pad * dw_per_row) return;
    const int r = (int)(idx / dw_per_row), d = (int)(idx % dw_per_row);
    const int g = 32 * ud, step = d / (4 * ud), rem = d % (4 * ud), s = rem / ud, u = rem % ud;
    const int sld = (cols + 3) / 4;
    uint32_t out = 0;
    for (int p = 0; p < 4; ++p)
        for (int b = 0; b < 4; ++b) {
            const int t = 2 * u + (p >> 1), q = 4 * (p & 1) + b, grp = t / ud;
            const int c = 2 * g * step + g * grp + 8 * ud * s + 8 * (t % ud) + q;
            const unsigned code = (unsigned)tern_code(src, sld, rows, cols, r, c) & 3u;
            out |= code << (8 * b + 2 * p);
        }
    dst[idx] = out;
}

__global__ void repack_int4_kernel(const uint8_t *__restrict__ src, int rows, int cols, uint32_t *__restrict__ dst,
                                   int rows_pad, int dw_per_row)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)rows_pad * dw_per_row) return;
    const int r = (int)(idx / dw_per_row), d = (int)(idx % dw_per_row);
    const int step = d / 16, s = (d % 16) / 4, t = d % 4;
    const int sld = (cols + 1) / 2;
    uint32_t out = 0;
    for (int b = 0; b < 4; ++b) {
        const int c_hi = 128 * step + 32 * s + 8 * t + b, c_lo = c_hi + 4;
        unsigned v_hi = 0, v_lo = 0;
        if (r < rows && c_hi < cols) {
            const uint8_t byte = src[(size_t)r * sld + (c_hi >> 1)];
            v_hi = ((c_hi & 1) ? (byte & 0xFu) : (byte >> 4)) ^ 8u;
        }
        if (r < rows && c_lo < cols) {
            const uint8_t byte = src[(size_t)r * sld + (c_lo >> 1)];
            v_lo = ((c_lo & 1) ? (byte & 0xFu) : (byte >> 4)) ^ 8u;
        }
        out |= ((v_hi << 4) | v_lo) << (8 * b);
    }
    dst[idx] = out;
}

__global__ void repack_int8_kernel(const int8_t *__restrict__ src, int rows, int cols, int8_t *__restrict__ dst,
                                   int rows_pad, int kpad)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)rows_pad * kpad) return;
    const int r = (int)(idx / kpad), c = (int)(idx % kpad);
    dst[idx] = (r < rows && c < cols) ? src[(size_t)r * cols + c] : (int8_t)0;
}

}  // namespace

// ---- resident weight object ----

struct eif_hip_qweight {
    int fmt, rows, cols, group, ud, kpad, rows_pad, nsteps, wld, ngroups;
    uint8_t *w;       // GPU layout
    float *scales;    // grouped [rows, ngroups] or row [rows]; NULL = 1
    size_t bytes;
};

namespace {

int g_gemm_min_tokens = 16;

int ud_supported(int ud) { return ud == 1 || ud == 2 || ud == 3 || ud == 4 || ud == 8; }

template <int FMT, int UD, bool GROUPED, bool ACC, int RT, int TT, int KSPLIT, bool V1>
int launch_one(const QArgs &a, int rows_pad, hipStream_t st)
{
    dim3 grid(rows_pad / (16 * RT), eif_ceil_div(a.M, 16 * TT));
    qlinear_kernel<FMT, UD, GROUPED, ACC, RT, TT, KSPLIT, V1><<<grid, 64 * RT * KSPLIT, 0, st>>>(a);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

// K-split factor for the GEMV: enough waves to cover the chip, never more than the steps of a row.
int pick_ksplit(int row_tiles, int nsteps)
{
    int k = 1;
    while (k < 8 && row_tiles * k < 2048 && 2 * k <= nsteps) k *= 2;
    return k;
}

template <int FMT, int UD, bool GROUPED, bool ACC>
int launch_shape(const QArgs &a, int rows_pad, int path, hipStream_t st)
{
    if (path == EIF_HIP_PATH_GEMM) return launch_one<FMT, UD, GROUPED, ACC, 4, 4, 1, false>(a, rows_pad, st);
    const int ks = pick_ksplit(rows_pad / 16, a.nsteps);
    if constexpr (ACC) {
        return launch_one<FMT, UD, GROUPED, ACC, 1, 1, 4, false>(a, rows_pad, st);
    } else {
        if (a.M == 1) {
            switch (ks) {
            case 1: return launch_one<FMT, UD, GROUPED, ACC, 1, 1, 1, true>(a, rows_pad, st);
            case 2: return launch_one<FMT, UD, GROUPED, ACC, 1, 1, 2, true>(a, rows_pad, st);
            case 4: return launch_one<FMT, UD, GROUPED, ACC, 1, 1, 4, true>(a, rows_pad, st);
            default: return launch_one<FMT, UD, GROUPED, ACC, 1, 1, 8, true>(a, rows_pad, st);
            }
        }
        switch (ks) {
        case 1: return launch_one<FMT, UD, GROUPED, ACC, 1, 1, 1, false>(a, rows_pad, st);
        case 2: return launch_one<FMT, UD, GROUPED, ACC, 1, 1, 2, false>(a, rows_pad, st);
        case 4: return launch_one<FMT, UD, GROUPED, ACC, 1, 1, 4, false>(a, rows_pad, st);
        default: return launch_one<FMT, UD, GROUPED, ACC, 1, 1, 8, false>(a, rows_pad, st);
        }
    }
}

template <bool ACC>
int dispatch(const eif_hip_qweight *w, const QArgs &a, int path, hipStream_t st)
{
    const bool grouped = w->fmt == kTern && w->group > 0;
    if (w->fmt == kI8) return launch_shape<kI8, 0, false, ACC>(a, w->rows_pad, path, st);
    if (w->fmt == kI4) return launch_shape<kI4, 0, false, ACC>(a, w->rows_pad, path, st);
    if (!grouped) return launch_shape<kTern, 4, false, ACC>(a, w->rows_pad, path, st);
    switch (w->ud) {
    case 1: return launch_shape<kTern, 1, true, ACC>(a, w->rows_pad, path, st);
    case 2: return launch_shape<kTern, 2, true, ACC>(a, w->rows_pad, path, st);
    case 3: return launch_shape<kTern, 3, true, ACC>(a, w->rows_pad, path, st);
    case 4: return launch_shape<kTern, 4, true, ACC>(a, w->rows_pad, path, st);
    case 8: return launch_shape<kTern, 8, true, ACC>(a, w->rows_pad, path, st);
    default: return EIF_HIP_E_ARG;
    }
}

int check_linear_args(const eif_hip_qweight *w, const int8_t *xq, int ldq, int M)
{
    if (!w || M < 0) return EIF_HIP_E_ARG;
    if (M > 0 && (!xq || ldq < w->kpad || ldq % 16 != 0 || ((uintptr_t)xq & 15))) return EIF_HIP_E_ARG;
    return EIF_HIP_OK;
}

int resolve_path(int path, int M)
{
    if (path == EIF_HIP_PATH_AUTO) return M >= g_gemm_min_tokens ? EIF_HIP_PATH_GEMM : EIF_HIP_PATH_GEMV;
    return path;
}

QArgs make_args(const eif_hip_qweight *w, const int8_t *xq, int ldq, int M)
{
    QArgs a{};
    a.W = w->w;
    a.wld = w->wld;
    a.scales = w->scales;
    a.G = w->ngroups;
    a.xq = xq;
    a.ldq = ldq;
    a.M = M;
    a.N = w->rows;
    a.nsteps = w->nsteps;
    return a;
}

}  // namespace

namespace eif {

// The linear with an explicit scale array (the host drop-in passes per-call row scales for resident codes).
int qlinear_scaled(const eif_hip_qweight *w, const float *scales, const int8_t *xq, int ldq, const float *xs,
                   const float *bias, float *y, int ldy, int M, int path, hipStream_t st)
{
    int rc = check_linear_args(w, xq, ldq, M);
    if (rc) return rc;
    if (M == 0) return EIF_HIP_OK;
    if (!xs || !y || ldy < w->rows) return EIF_HIP_E_ARG;
    if (w->fmt == kTern && w->group > 0 && !scales) return EIF_HIP_E_ARG;
    QArgs a = make_args(w, xq, ldq, M);
    a.scales = scales;
    a.xs = xs;
    a.bias = bias;
    a.y = y;
    a.ldy = ldy;
    return dispatch<false>(w, a, resolve_path(path, M), st);
}

}  // namespace eif

extern "C" {

int eif_hip_set_gemm_min_tokens(int m)
{
    int old = g_gemm_min_tokens;
    if (m >= 1) g_gemm_min_tokens = m;
    return old;
}

int eif_hip_gemm_min_tokens(void) { return g_gemm_min_tokens; }

int eif_hip_qweight_create(eif_hip_qweight **out, int fmt, int rows, int cols, int group, const void *codes,
                           const float *scales, int src_on_device, void *stream)
{
    if (!out || !codes || rows <= 0 || cols <= 0) return EIF_HIP_E_ARG;
    *out = nullptr;
    hipStream_t st = (hipStream_t)stream;
    eif_hip_qweight q{};
    q.fmt = fmt;
    q.rows = rows;
    q.cols = cols;
    q.group = group;
    q.rows_pad = eif_round_up(rows, kRowPad);
    size_t src_bytes;
    int sc_count;
    if (fmt == kTern) {
        if (group < 0 || group % 32 != 0) return EIF_HIP_E_ARG;
        q.ud = group > 0 ? group / 32 : 4;
        if (!ud_supported(q.ud)) return EIF_HIP_E_ARG;
        q.kpad = eif_round_up(cols, 64 * q.ud);
        q.wld = q.kpad / 4;
        q.ngroups = group > 0 ? eif_ceil_div(cols, group) : 0;
        src_bytes = (size_t)rows * ((cols + 3) / 4);
        sc_count = group > 0 ? rows * q.ngroups : rows;
    } else if (fmt == kI4 || fmt == kI8) {
        if (group != 0) return EIF_HIP_E_ARG;
        q.kpad = eif_round_up(cols, fmt == kI4 ? 128 : 64);
        q.wld = fmt == kI4 ? q.kpad / 2 : q.kpad;
        src_bytes = fmt == kI4 ? (size_t)rows * ((cols + 1) / 2) : (size_t)rows * cols;
        sc_count = rows;
    } else {
        return EIF_HIP_E_ARG;
    }
    if (fmt == kTern && group > 0 && !scales) return EIF_HIP_E_ARG;
    q.nsteps = q.kpad / (fmt == kTern ? 64 * q.ud : (fmt == kI4 ? 128 : 64));
    const size_t wbytes = (size_t)q.rows_pad * q.wld;

    void *src_dev = nullptr;
    if (!src_on_device) {
        if (hipMalloc(&src_dev, src_bytes) != hipSuccess) return EIF_HIP_E_NOMEM;
        if (hipMemcpyAsync(src_dev, codes, src_bytes, hipMemcpyHostToDevice, st) != hipSuccess) {
            hipFree(src_dev);
            return EIF_HIP_E_DEVICE;
        }
    }
    const void *src = src_on_device ? codes : src_dev;
    int rc = EIF_HIP_OK;
    if (hipMalloc(&q.w, wbytes) != hipSuccess) rc = EIF_HIP_E_NOMEM;
    if (rc == EIF_HIP_OK && scales) {
        if (hipMalloc(&q.scales, sizeof(float) * sc_count) != hipSuccess)
            rc = EIF_HIP_E_NOMEM;
        else if (hipMemcpyAsync(q.scales, scales, sizeof(float) * sc_count,
                                src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st) != hipSuccess)
            rc = EIF_HIP_E_DEVICE;
    }
    if (rc == EIF_HIP_OK) {
        const int threads = 256;
        if (fmt == kTern) {
            const int dpr = q.wld / 4;
            const size_t n = (size_t)q.rows_pad * dpr;
            repack_ternary_kernel<<<(unsigned)((n + threads - 1) / threads), threads, 0, st>>>(
                (const uint8_t *)src, rows, cols, q.ud, (uint32_t *)q.w, q.rows_pad, dpr);
        } else if (fmt == kI4) {
            const int dpr = q.wld / 4;
            const size_t n = (size_t)q.rows_pad * dpr;
            repack_int4_kernel<<<(unsigned)((n + threads - 1) / threads), threads, 0, st>>>(
                (const uint8_t *)src, rows, cols, (uint32_t *)q.w, q.rows_pad, dpr);
        } else {
            const size_t n = (size_t)q.rows_pad * q.kpad;
            repack_int8_kernel<<<(unsigned)((n + threads - 1) / threads), threads, 0, st>>>(
                (const int8_t *)src, rows, cols, (int8_t *)q.w, q.rows_pad, q.kpad);
        }
        if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) rc = EIF_HIP_E_DEVICE;
    }
    if (src_dev) hipFree(src_dev);
    if (rc != EIF_HIP_OK) {
        if (q.w) hipFree(q.w);
        if (q.scales) hipFree(q.scales);
        return rc;
    }
    q.bytes = wbytes + (scales ? sizeof(float) * sc_count : 0);
    eif_hip_qweight *h = new (std::nothrow) eif_hip_qweight(q);
    if (!h) {
        hipFree(q.w);
        if (q.scales) hipFree(q.scales);
        return EIF_HIP_E_NOMEM;
    }
    *out = h;
    return EIF_HIP_OK;
}

void eif_hip_qweight_destroy(eif_hip_qweight *w)
{
    if (!w) return;
    if (w->w) hipFree(w->w);
    if (w->scales) hipFree(w->scales);
    delete w;
}

int eif_hip_qweight_info(const eif_hip_qweight *w, int *rows, int *cols, int *kpad, int *group, size_t *bytes)
{
    if (!w) return EIF_HIP_E_ARG;
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    if (kpad) *kpad = w->kpad;
    if (group) *group = w->group;
    if (bytes) *bytes = w->bytes;
    return EIF_HIP_OK;
}

int eif_hip_qlinear_ex(const eif_hip_qweight *w, const int8_t *xq, int ldq, const float *xs, const float *bias,
                       float *y, int ldy, int M, int path, void *stream)
{
    if (!w) return EIF_HIP_E_ARG;
    return eif::qlinear_scaled(w, w->scales, xq, ldq, xs, bias, y, ldy, M, path, (hipStream_t)stream);
}

int eif_hip_qlinear(const eif_hip_qweight *w, const int8_t *xq, int ldq, const float *xs, const float *bias,
                    float *y, int ldy, int M, void *stream)
{
    return eif_hip_qlinear_ex(w, xq, ldq, xs, bias, y, ldy, M, EIF_HIP_PATH_AUTO, stream);
}

int eif_hip_qlinear_acc(const eif_hip_qweight *w, const int8_t *xq, int ldq, int32_t *acc, int M, int path,
                        void *stream)
{
    int rc = check_linear_args(w, xq, ldq, M);
    if (rc) return rc;
    if (M == 0) return EIF_HIP_OK;
    if (!acc) return EIF_HIP_E_ARG;
    QArgs a = make_args(w, xq, ldq, M);
    a.acc = acc;
    return dispatch<true>(w, a, resolve_path(path, M), (hipStream_t)stream);
}

}  // extern "C"

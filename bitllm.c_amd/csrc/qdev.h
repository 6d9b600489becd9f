// qdev.h -- device code shared by the linear kernels (qlinear.hip) and the persistent decode step (persist.hip):
// the GPU weight layouts' step geometry and decoding, the int8 MFMA helpers, and the fused activation prep
// (pre-op, sign flip, blockwise WHT, absmax INT8 into LDS). Both users compile the same arithmetic, so a row
// prepped or a tile multiplied by either gives the same bits.
//
// Template knobs of the prep (defaults: the standalone kernels' forms):
//   COH  the activation rows are read with device-coherent loads (written earlier in the same launch by other
//        workgroups, possibly on another XCD): agent-scope relaxed atomic loads, which bypass the non-coherent
//        L2 lines; false: plain loads (rows written before the launch).
//   BAR  the workgroup barrier: 0 = __syncthreads(); 1 = an LDS-only barrier (s_waitcnt lgkmcnt(0); s_barrier),
//        which does not wait for outstanding global loads of other waves (the persistent step's weight
//        prefetches into LDS) -- only for LDS traffic, which is all these barriers order.
#pragma once

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
    static constexpr int SB = 32, SC = 128, NMF = 4, SHIFT = 0;
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
#pragma unroll
        for (int i = 0; i < Geo<FMT, UD>::NMF; ++i) b[i] = pack2(w[2 * i], w[2 * i + 1]);
    }
}

EIF_DEV v4i mfma(long a, long b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0); }

// Two 8-byte operands of the same lane concatenated into one 16-byte operand of v_mfma_i32_16x16x64_i8: A and
// B are concatenated alike, so the product is the sum of the two 16x16x32 products (the gfx950 double-rate
// form; a pair never spans two groups because it is formed inside one group's operands).
EIF_DEV v4i mfma64(long a0, long a1, long b0, long b1, v4i c)
{
    const v4i a = {(int)a0, (int)(a0 >> 32), (int)a1, (int)(a1 >> 32)};
    const v4i b = {(int)b0, (int)(b0 >> 32), (int)b1, (int)(b1 >> 32)};
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// c += sum_i a[i] * b[OFF + i] over the N operands of a, in pairs on the 64-deep form; an odd last operand is
// paired with zero operands on the same form (a g96 group's three operands take two MFMAs, not three 32-deep
// ones at the same issue cost each). An accumulation chain never mixes the two forms: a 64-deep result fed
// straight into a dependent 32-deep MFMA gave wrong sums on gfx950. Array references with a compile-time offset
// keep both operand arrays in registers.
template <int OFF, int N, int NB>
EIF_DEV v4i mfma_ops(const long (&a)[N], const long (&b)[NB], v4i c)
{
#pragma unroll
    for (int i = 0; i + 1 < N; i += 2) c = mfma64(a[i], a[i + 1], b[OFF + i], b[OFF + i + 1], c);
    if constexpr (N % 2 == 1) c = mfma64(a[N - 1], 0, b[OFF + N - 1], 0, c);
    return c;
}


// Workgroup barrier of policy BAR (see the header comment). The empty asm statements keep the compiler from
// moving memory accesses across the LDS-only barrier.
template <int BAR>
EIF_DEV void wg_sync()
{
    if constexpr (BAR == 0) {
        __syncthreads();
    } else {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt and expcnt not waited for
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }
}

// Device-coherent 4-byte load / store (agent-scope relaxed atomics: global_load/store ... sc1 on gfx950).
EIF_DEV float ld_coh(const float *p) { return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
EIF_DEV void st_coh(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
EIF_DEV int ld_coh_i(const int *p) { return __hip_atomic_load(const_cast<int *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
EIF_DEV void st_coh_i(int *p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
EIF_DEV uint64_t ld_coh_u64(const uint64_t *p)
{
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct PrepArgs {
    const float *x;       // [M, ldx] FP32 rows to prep in the kernel, or NULL (xq/xs of QArgs are staged)
    int ldx;
    const float *signs;   // [K] or NULL
    int K, block;         // block 0: no rotation
    float norm;
    int ldl;              // LDS row stride of the staged activations (bytes)
    int pre;              // EIF_HIP_PRE_*: what the rows are before the rotation (see eif_hip.h)
    const float *x2;      // EIF_HIP_PRE_SWIGLU_RMS: the up-projection rows [M, ldx] (x holds the gate)
    const float *nw;      // RMSNorm weight [K], NULL = 1
    float eps;            // RMSNorm epsilon
    const float *sh_o;    // attention shares in place of x (one row): [K / sh_hd][kAttnShares][sh_hd] outputs,
    const float *sh_ml;   // [K / sh_hd][2 kAttnShares] maxima then sums; NULL: x holds the rows
    int sh_hd;
};

// One WHT butterfly stage across threads t and t ^ LX: the lower thread keeps a + b, the upper one a - b (a the
// lower thread's value, b the upper one's). Written as partner + (upper ? -v : v): the same single rounding as
// the reference's a + b and a - b, in one negate-select and one DPP-sourced add per element.
template <int LX, int E>
EIF_DEV void wht_cross(float (&v)[E], int t)
{
    const bool upper = (t & LX) != 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float own = upper ? -v[e] : v[e];
        v[e] = xlane<LX>(v[e]) + own;
    }
}

// q = trunc(t +- 0.5) clamped, t = v*inv. copysign(0.5, t) + t equals the reference's branch for every t
// (t = -0 gives -0.5 -> 0 where the branch gives 0.5 -> 0).
EIF_DEV int quant1(float v, float inv)
{
    const float t = v * inv;
    const float r = t + __builtin_copysignf(0.5f, t);
    const int q = (int)r;
    return min(max(q, -128), 127);
}

// max over the 64 lanes: DPP butterflies inside each 16-lane row, then the four row maxima via readlane.
EIF_DEV float wave_max_dpp(float v)
{
    v = fmaxf(v, xlane<1>(v));
    v = fmaxf(v, xlane<2>(v));
    v = fmaxf(v, xlane<4>(v));
    v = fmaxf(v, xlane<8>(v));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// sum over the 64 lanes: DPP butterflies inside each 16-lane row, then the four row sums via readlane
EIF_DEV float wave_sum_dpp(float v)
{
    v = v + xlane<1>(v);
    v = v + xlane<2>(v);
    v = v + xlane<4>(v);
    v = v + xlane<8>(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return ((a + b) + c) + d;
}

// base[idx .. idx + E) (base uniform over the wave, idx a multiple of 4): 16-byte loads; COH: device-coherent
// 16-byte loads (a buffer load with the sc1 policy, the agent-scope coherence of the relaxed atomics above).
template <int E, bool COH = false>
EIF_DEV void load4(const float *base, int idx, float (&v)[E])
{
    if constexpr (COH) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), 0, 0x7fffffff,
                                                                            0x00020000);
#pragma unroll
        for (int q = 0; q < E / 4; ++q) {
            const auto r = __builtin_amdgcn_raw_buffer_load_b128(rs, 4 * (idx + 4 * q), 0, 16);   // sc1
            v[4 * q] = __uint_as_float(r[0]), v[4 * q + 1] = __uint_as_float(r[1]);
            v[4 * q + 2] = __uint_as_float(r[2]), v[4 * q + 3] = __uint_as_float(r[3]);
        }
        return;
    }
    const float *p = base + idx;
#pragma unroll
    for (int q = 0; q < E / 4; ++q) {
        const float4 a4 = *reinterpret_cast<const float4 *>(p + 4 * q);
        v[4 * q] = a4.x, v[4 * q + 1] = a4.y, v[4 * q + 2] = a4.z, v[4 * q + 3] = a4.w;
    }
}

// Thread t holds columns [E*t, E*t + E) of token row m (zeros past K); tid is the thread's index in the workgroup.
// The loads are clamped to the row and nothing consumes them here, so the weight loads a GEMV issues next are not
// held behind them; the pre-op, the sign flip and the zeroing past K happen in prep_finish.
//   v: x; sg: signs; v2: x2 (SwiGLU); nw: the RMSNorm weight. An absent operand (a null row) is not loaded: its
//   registers hold 1 (signs, weight) or 0 (x2). Each activation load costs address-unit time that the weight
//   loads issued after it wait for, so only the operands present are read (uniform branches, all of them before
//   the caller's weight loads; prep_finish holds every operand on every path, so none is sunk behind those).
// The per-column operands a fused prep reads, a compile-time choice of the launch:
//   kOpsX    x alone (no signs, no norm weight, no x2);
//   kOpsMul  x and one column multiplier, applied after the pre-op's sum of squares and before the rotation: the
//            norm weight, the signs, or their product (exact for +-1 signs: (v w) s = v (w s));
//   kOpsAny  every operand the rows name (signs, x2, norm weight), each read where present.
enum { kOpsX = 0, kOpsMul = 1, kOpsAny = 2 };

template <int E>
EIF_DEV void fill(float (&v)[E], float c)
{
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = c;
}

// OPS (kOpsX ...): kOpsAny reads what is present (uniform branches); kOpsMul reads x and the multiplier at nwr
// into nw; kOpsX reads x alone. Every load count is then fixed, and the code before the caller's weight loads
// has no branch.
template <int E, bool COH = false, int OPS = kOpsAny>
EIF_DEV void prep_load_rows(const float *xr, const float *sgr, const float *x2r, const float *nwr, int K,
                            float (&v)[E], float (&sg)[E], float (&v2)[E], float (&nw)[E], int tid = threadIdx.x)
{
    const int i0 = E * tid;
    const int ic = i0 < K ? i0 : 0;
    load4<E, COH>(xr, ic, v);
    if constexpr (OPS == kOpsAny) {
        if (sgr) load4<E>(sgr, ic, sg); else fill(sg, 1.0f);
        if (x2r) load4<E, COH>(x2r, ic, v2); else fill(v2, 0.0f);
        if (nwr) load4<E>(nwr, ic, nw); else fill(nw, 1.0f);
    } else {
        fill(sg, 1.0f);
        fill(v2, 0.0f);
        if constexpr (OPS == kOpsMul) load4<E>(nwr, ic, nw); else fill(nw, 1.0f);
    }
}

// prep_load_rows on the rows PrepArgs names (prep_load_rows itself takes them as given: a kernel's preloaded
// arguments).
template <int E, bool COH = false>
EIF_DEV void prep_load(const PrepArgs &p, int m, float (&v)[E], float (&sg)[E], float (&v2)[E], float (&nw)[E],
                       int tid = threadIdx.x)
{
    prep_load_rows<E, COH>(p.x + (size_t)m * p.ldx, p.signs,
                           p.pre == EIF_HIP_PRE_SWIGLU_RMS ? p.x2 + (size_t)m * p.ldx : nullptr,
                           p.pre != EIF_HIP_PRE_NONE ? p.nw : nullptr, p.K, v, sg, v2, nw, tid);
}

// The attention shares of thread t's columns [E t, E t + E) (head h = E t / sh_hd, dims from E t % sh_hd): every
// share's outputs and the head's maxima and sums, loaded unconditionally; the signs and the norm weight as in
// prep_load_rows (null: not loaded).
template <int E>
struct Shares {
    float o[kAttnShares][E];
    float ml[2 * kAttnShares];
};

template <int E, bool COH = false, int OPS = kOpsAny>
EIF_DEV void prep_load_sh_rows(const float *sh_o, const float *sh_ml, const float *sgr, const float *nwr, int K,
                               int sh_hd, Shares<E> &sh, float (&sg)[E], float (&nw)[E], int tid = threadIdx.x)
{
    const int i0 = E * tid;
    const int ic = i0 < K ? i0 : 0;
    const int h = ic / sh_hd, d = ic - h * sh_hd;
    load4<2 * kAttnShares, COH>(sh_ml, h * 2 * kAttnShares, sh.ml);
    const int o = h * kAttnShares * sh_hd + d;
#pragma unroll
    for (int s = 0; s < kAttnShares; ++s) load4<E, COH>(sh_o, o + s * sh_hd, sh.o[s]);
    if constexpr (OPS == kOpsAny) {
        if (sgr) load4<E>(sgr, ic, sg); else fill(sg, 1.0f);
        if (nwr) load4<E>(nwr, ic, nw); else fill(nw, 1.0f);
    } else {
        fill(sg, 1.0f);
        if constexpr (OPS == kOpsMul) load4<E>(nwr, ic, nw); else fill(nw, 1.0f);
    }
}

template <int E, bool COH = false>
EIF_DEV void prep_load_sh(const PrepArgs &p, Shares<E> &sh, float (&sg)[E], float (&nw)[E], int tid = threadIdx.x)
{
    prep_load_sh_rows<E, COH>(p.sh_o, p.sh_ml, p.signs, p.pre != EIF_HIP_PRE_NONE ? p.nw : nullptr, p.K, p.sh_hd,
                              sh, sg, nw, tid);
}

// v = sum_s e^(M_s - M) O_s / sum_s e^(M_s - M) L_s, M = max_s M_s (share 0 always holds rows, so M is finite).
template <int E>
EIF_DEV void sh_combine(const Shares<E> &sh, float (&v)[E])
{
    float mx = sh.ml[0];
#pragma unroll
    for (int s = 1; s < kAttnShares; ++s) mx = fmaxf(mx, sh.ml[s]);
    float ls = 0.0f, o[E];
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = 0.0f;
#pragma unroll
    for (int s = 0; s < kAttnShares; ++s) {
        const float w = expf(sh.ml[s] - mx);
        ls = fmaf(w, sh.ml[kAttnShares + s], ls);
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = fmaf(w, sh.o[s][e], o[e]);
    }
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = o[e] / ls;
}

// Rotation, absmax over the workgroup, INT8 codes of token m into LDS (row m, columns [0, kpad)).
// LB = log2 of the WHT block when it is fixed at compile time (0: no rotation), -1: block read from p.block.
struct NoHook {
    EIF_DEV void operator()() const {}
};

// OPS: the operands loaded (kOpsX ...); kOpsMul holds its multiplier in nwv. mid(): called once the row's
// maxima are reduced within each wave, before the workgroup barrier (a caller's loads that may wait for the
// struct arguments, issued where that wait costs nothing).
template <int E, int LB, int BAR = 0, int OPS = kOpsAny, class Mid = NoHook>
EIF_DEV void prep_finish(const PrepArgs &p, int m, int kpad, float (&v)[E], const float (&sg)[E],
                         const float (&v2)[E], const float (&nwv)[E], int8_t *lds_x, float *xs_l, float *red,
                         float *red_ss, int tid = threadIdx.x, Mid &&mid = Mid{})
{
    const int t = tid, i0 = E * t, nw = blockDim.x >> 6;
    const int block = LB >= 0 ? (LB > 0 ? 1 << LB : 0) : p.block;
    const bool live = i0 < p.K, flip = OPS == kOpsAny && block > 0 && p.signs;
    // Every operand is held here, on every path. An operand that only a branch below reads (the norm weight, x2,
    // the signs) would otherwise have its load sunk into that branch, issued after a GEMV's weight loads and
    // waited for together with them (vmcnt counts in issue order): the prep would start when the weights land.
    if constexpr (OPS == kOpsAny) {
#pragma unroll
        for (int e = 0; e < E; ++e) asm volatile("" ::"v"(sg[e]), "v"(v2[e]), "v"(nwv[e]));
    } else if constexpr (OPS == kOpsMul) {
#pragma unroll
        for (int e = 0; e < E; ++e) asm volatile("" ::"v"(nwv[e]));
    }
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = live ? v[e] : 0.0f;
    // RMSNorm over the K columns, (v * r) * weight with r = 1 / sqrtf(sum(v^2) / K + eps): r > 0 is one factor of
    // the whole row, and the absmax codes of a row do not change when the row is scaled, so the rotation and the
    // codes take v * weight and r enters the row's scale only; its sum of squares is reduced with the absmax
    // (one barrier). Codes equal those of the normalized row up to the rounding of values on a code boundary.
    const bool rms = p.pre != EIF_HIP_PRE_NONE;
    float ss = 0.0f;
    if (rms) {   // uniform
        if (OPS == kOpsAny && p.pre == EIF_HIP_PRE_SWIGLU_RMS) {
#pragma unroll
            for (int e = 0; e < E; ++e) v[e] = (v[e] * (1.0f / (1.0f + expf(-v[e])))) * (live ? v2[e] : 0.0f);
        }
#pragma unroll
        for (int e = 0; e < E; ++e) ss = fmaf(v[e], v[e], ss);
        if (OPS == kOpsAny && p.nw) {
#pragma unroll
            for (int e = 0; e < E; ++e) v[e] = v[e] * nwv[e];
        }
    }
    if constexpr (OPS == kOpsMul) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = v[e] * nwv[e];
    }
    if (flip) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = v[e] * sg[e];
    }
#pragma unroll
    for (int h = 1; h < E; h <<= 1) {
        if (h >= block) break;
#pragma unroll
        for (int e = 0; e < E; ++e)
            if ((e & h) == 0) {
                const float a = v[e], b = v[e + h];
                v[e] = a + b;
                v[e + h] = a - b;
            }
    }
    if (block > E) wht_cross<1>(v, t);
    if (block > 2 * E) wht_cross<2>(v, t);
    if (block > 4 * E) wht_cross<4>(v, t);
    if (block > 8 * E) wht_cross<8>(v, t);
    if (block > 16 * E) wht_cross<16>(v, t);
    if (block > 32 * E) wht_cross<32>(v, t);
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        if (block > 0) v[e] = v[e] * p.norm;
        amax = fmaxf(amax, fabsf(v[e]));
    }
    amax = wave_max_dpp(amax);
    if (rms) ss = wave_sum_dpp(ss);
    mid();
    if ((t & 63) == 0) red[t >> 6] = amax, red_ss[t >> 6] = ss;
    wg_sync<BAR>();
    // the per-wave maxima (and sums), one per lane, reduced again across the wave
    const int ln = t & 63;
    amax = wave_max_dpp(red[ln < nw ? ln : 0]);
    float r = 1.0f;
    if (rms) {
        ss = wave_sum_dpp(ln < nw ? red_ss[ln] : 0.0f);
        r = 1.0f / sqrtf(ss / (float)p.K + p.eps);
    }
    const float amax_n = amax * r;   // the absmax of the normalized row (amax itself without a pre-op)
    const bool zero = amax_n < 1e-12f;
    const float inv = zero ? 0.0f : 127.0f / amax;
    if (t == 0) xs_l[m] = zero ? 1.0f : amax_n * (1.0f / 127.0f);
    if (i0 < kpad) {
        uint32_t d[E / 4];
#pragma unroll
        for (int q = 0; q < E / 4; ++q) {
            uint32_t u = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b)
                u |= ((uint32_t)quant1(v[4 * q + b], inv) & 0xFFu) << (8 * b);
            d[q] = u;
        }
        int8_t *o = lds_x + m * p.ldl + i0;
        if constexpr (E % 16 == 0) {
#pragma unroll
            for (int q = 0; q < E / 16; ++q)
                *reinterpret_cast<uint4 *>(o + 16 * q) = make_uint4(d[4 * q], d[4 * q + 1], d[4 * q + 2], d[4 * q + 3]);
        } else if constexpr (E == 8) {
            *reinterpret_cast<uint2 *>(o) = make_uint2(d[0], d[1]);
        } else {
            *reinterpret_cast<uint32_t *>(o) = d[0];
        }
    }
    wg_sync<BAR>();   // red[] is reused by the next row; lds_x complete
}

}  // namespace

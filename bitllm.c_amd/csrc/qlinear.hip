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
//   int8: the reference row-major layout, rows padded; steps of 128 columns, slot s owns bytes 32s..32s+31 (two
//     64-deep MFMA operands per lane and step, so a K step of the GEMM carries as many MFMAs as INT4's).
//   Every layout pads rows to a multiple of 64 and columns to a whole number of steps with zero weights.
//
// Accumulation contract (reference: src/eif_quantize_bitnet.c:1143-1203 for the row-scaled epilogue,
// src/eif_quantize_bitnet.c:1227-1296 and src/eif_qwen35.c:228-290 for group-scaled combination):
//   grouped ternary:  acc_g exact int32 per (token, row, group); F = sum_g fmaf((float)acc_g, s[r,g], F) within a
//                     wave, partial F of the K-split waves added in wave order; y = F * xs[m] (+ bias).
//   row-scaled:       isum = exact int32 over all K (K-split partials added as integers);
//                     y = ((float)isum * xs[m]) * s[r] (+ bias).
#include <algorithm>
#include <mutex>
#include <new>
#include <thread>
#include <type_traits>
#include <unordered_map>

#include "hip_common.h"
#include "qdev.h"

namespace {

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
    float *part;           // GEMM split along K: partial sums [split][tile][thread][4 TT]
    int *cnt;              // GEMM split along K: one arrival counter per output tile, zero between launches
    unsigned long long *amax_key;   // row-scaled GEMV, M = 1: the largest output and its first row, atomic max of
                                    // eif_argmax_key over the 16-row tiles into kArgmaxSlots slots, or NULL
    int mw;                // GEMV: token rows per workgroup (0: all M in one workgroup)
    int nrb;               // GEMV with token chunks: row blocks (workgroups along the rows per chunk)
};

// ---- tiled GEMM (token batches above the small-batch GEMV) ----
//
// Workgroup: 4 waves, 64 rows x 16*TT tokens; wave w owns rows 16w..16w+15 for all TT token tiles and walks
// every step of K in order. Per step the workgroup stages the activation block [16*TT tokens x SC columns] in
// LDS (double-buffered), each wave loads its own weight codes and scales, decodes them once and reuses them for
// the TT token tiles. The loads of a step are issued PF - 1 steps before it is staged (a ring of PF register
// buffers): a workgroup's steps form a dependent chain, and with one step of loads in flight each step waits
// out a whole memory latency. Grouped ternary: each group's exact int32 sum is combined at once, in group
// order, into FP32 accumulators (the same sequence as the oracle); row-scaled: one int32 sum over K.
constexpr int kGemmThreads = 256;

// Waves per SIMD the register budget is cut for: four for the g128 ternary and INT formats (their MFMA sums
// would otherwise sit in accumulation registers, at three waves), two with a deeper prefetch ring (launched
// when the workgroups are few), the compiler's choice for the other group sizes (g32 at four waves spilled).
template <int FMT, int UD, int PF>
constexpr int gemm_waves() { return FMT == kTern && UD != 4 ? 1 : (PF > 2 ? 2 : 4); }

// The GEMM's epilogue for one thread's outputs (rows `row`, tokens m0 + 16 tt + 4 s + v): xs_l holds the
// workgroup's token scales (index tok - m0); rs and bb the row's scale (row-scaled) and bias, loaded at the
// kernel's start so that the epilogue waits for no load. Unsplit: the outputs. Split along K (gridDim.z > 1):
// each split stores its partial sums (the FP32 group combines, or the exact int32 sums) for this thread's
// outputs, value-major (part[split][tile][4 TT values][256 threads]: every store and load instruction covers
// 256 contiguous bytes), with device-coherent stores (sc1: past the XCDs' non-coherent L2s), waits for them, and
// counts the workgroup's arrival on the tile's counter. The last split to arrive reads every split's partials
// back with device-coherent loads, adds them in split order, writes the epilogue and resets the counter for the
// next launch.
template <int FMT, int UD, bool GROUPED, bool ACC, int TT>
__device__ __forceinline__ void gemm_finish(const QArgs &a, const float (&F)[TT][4], const v4i (&C)[TT], int row,
                                            bool row_ok, int m0, int s, const float *xs_l, float rs, float bb)
{
    using GE = Geo<FMT, UD>;
    if (gridDim.z > 1) {
        const int ntile = gridDim.x * gridDim.y, tile = blockIdx.y * gridDim.x + blockIdx.x, nz = gridDim.z;
        auto pz = [&](int z) { return a.part + ((size_t)z * ntile + tile) * (4 * TT * kGemmThreads) + threadIdx.x; };
        float *own = pz(blockIdx.z);
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                st_coh(own + (4 * tt + v) * kGemmThreads, GROUPED ? F[tt][v] : __int_as_float(C[tt][v] >> GE::SHIFT));
        __builtin_amdgcn_s_waitcnt(0);
        __shared__ int last_l;
        __syncthreads();
        if (threadIdx.x == 0)
            last_l = __hip_atomic_fetch_add(a.cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nz - 1;
        __syncthreads();
        if (!last_l) return;
        if (threadIdx.x == 0) st_coh_i(a.cnt + tile, 0);
        // split order, the loads of four splits in flight at once (indices past the last split read it again)
        float fs[TT][4];
        int is[TT][4];
        for (int z0 = 0; z0 < nz; z0 += 4) {
            float q[4][4 * TT];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float *p = pz(min(z0 + j, nz - 1));
#pragma unroll
                for (int i = 0; i < 4 * TT; ++i) q[j][i] = ld_coh(p + i * kGemmThreads);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (z0 + j >= nz) break;
#pragma unroll
                for (int tt = 0; tt < TT; ++tt)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float f = q[j][4 * tt + v];
                        if constexpr (GROUPED)
                            fs[tt][v] = z0 + j == 0 ? f : fs[tt][v] + f;
                        else
                            is[tt][v] = (z0 + j == 0 ? 0 : is[tt][v]) + __float_as_int(f);
                    }
            }
        }
        if (!row_ok) return;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int lt = 16 * tt + 4 * s + v, tok = m0 + lt;
                if (tok >= a.M) continue;
                float out = GROUPED ? fs[tt][v] * xs_l[lt] : ((float)is[tt][v] * xs_l[lt]) * rs;
                if (a.bias) out = out + bb;
                a.y[(size_t)tok * a.ldy + row] = out;
            }
        return;
    }

    if (!row_ok) return;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int lt = 16 * tt + 4 * s + v, tok = m0 + lt;
            if (tok >= a.M) continue;
            float out;
            if constexpr (GROUPED) {
                out = F[tt][v] * xs_l[lt];
            } else {
                const int isum = C[tt][v] >> GE::SHIFT;
                if constexpr (ACC) {
                    a.acc[(size_t)tok * a.N + row] = isum;
                    continue;
                }
                out = ((float)isum * xs_l[lt]) * rs;
            }
            if (a.bias) out = out + bb;
            a.y[(size_t)tok * a.ldy + row] = out;
        }
}

// The epilogue's operands of a GEMM thread, loaded at the kernel's start: the row's scale (row-scaled, else 1)
// and bias (else 0), rows past N clamped to the last; and one token scale of the workgroup's batch (token
// m0 + tid mod TM, clamped into the batch), which threads 0 .. TM - 1 stage in LDS.
template <bool GROUPED, int TM>
__device__ __forceinline__ void gemm_epilogue_loads(const QArgs &a, int row, int m0, float &rs, float &bb, float &xsv)
{
    const int rc = row < a.N ? row : a.N - 1;
    rs = (!GROUPED && a.scales) ? a.scales[rc] : 1.0f;
    bb = a.bias ? a.bias[rc] : 0.0f;
    const int xt = m0 + (int)(threadIdx.x & (TM - 1));
    xsv = a.xs ? a.xs[xt < a.M ? xt : a.M - 1] : 0.0f;
}

template <int FMT, int UD, bool GROUPED, bool ACC, int TT, int PF>
// The leading arguments (preloaded into SGPRs at wave launch, as qgemv_kernel's) duplicate the QArgs fields the
// first loads need.
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(gemm_waves<FMT, UD, PF>())))
void qgemm_kernel(const int8_t *__restrict__ xq, const uint8_t *__restrict__ W, const float *__restrict__ scales,
                  int wld, int ldq, int M, int nsteps, int G, int N, QArgs a)
{
    a.xq = xq, a.W = W, a.scales = scales, a.wld = wld, a.ldq = ldq, a.M = M, a.nsteps = nsteps, a.G = G, a.N = N;
    using GE = Geo<FMT, UD>;
    constexpr int NW = GE::SB / 4;
    constexpr int TM = 16 * TT;                    // tokens per workgroup
    constexpr int PR = GE::SC / 16;                // 16-byte pieces per token per step
    constexpr int PPT = (TM * PR + kGemmThreads - 1) / kGemmThreads;
    constexpr int LDA = GE::SC + 16;               // LDS row stride of the staged block
    __shared__ __align__(16) int8_t xa[2][TM * LDA];
    __shared__ float scl[2][GROUPED ? 256 : 1];    // grouped: the step's two group scales of the 64 rows, [grp][row]
    __shared__ float xs_l[TM];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, s = lane >> 4;
    const int row = blockIdx.x * 64 + wave * 16 + r16;   // < rows_pad
    const bool row_ok = row < a.N;
    const int m0 = blockIdx.y * TM;
    // split along K (gridDim.z > 1): this workgroup's steps [s0, s0 + ns)
    const int s0 = (int)(blockIdx.z * a.nsteps / gridDim.z);
    const int ns = (int)((blockIdx.z + 1) * a.nsteps / gridDim.z) - s0;
    // the epilogue's operands, loaded first (the first step's wait covers them)
    float rs, bb, xsv;
    gemm_epilogue_loads<GROUPED, TM>(a, row, m0, rs, bb, xsv);
    __builtin_amdgcn_sched_barrier(0);

    static_assert(PF >= 2 && PF % 2 == 0, "register buffers in pairs: a step's LDS buffer is its parity");
    v4i ra[PF][PPT];   // a clang vector type: an array of HIP's int4 structs would live in scratch
    uint32_t wb[PF][NW];
    float sc[PF];      // grouped: the scale this thread stages, of row (tid & 63) and group (tid >> 6) of the step
    // 32-bit byte offsets from the uniform bases (the launcher keeps the batch's int8 rows and the weights below
    // 4 GiB): the loads take the scalar-base form and a step adds st * SC (st * 4 * SB) to them.
    const uint32_t wo = (uint32_t)row * (uint32_t)a.wld + (uint32_t)(s * GE::SB);
    uint32_t xo[PPT];   // the thread's activation pieces at step 0, token rows clamped into the batch
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
        const int pc = threadIdx.x + i * kGemmThreads;
        const int t = pc / PR, q = pc - t * PR;
        const int tok = m0 + (t < TM ? t : TM - 1);
        xo[i] = (uint32_t)(tok < a.M ? tok : a.M - 1) * (uint32_t)a.ldq + (uint32_t)(16 * q);
    }
    // Grouped: threads 0..127 stage the step's scales (threads 128..255 the same ones again, into an unread half),
    // so they travel with the activation block through LDS. A loaded value that the loop carried in registers to
    // the next step was copied at the loop's end, and the copy waited for every load in flight.
    const int sc_row = blockIdx.x * 64 + (threadIdx.x & 63), sc_grp = (threadIdx.x >> 6) & 1;
    const uint32_t so = GROUPED ? (uint32_t)(sc_row < a.N ? sc_row : a.N - 1) * (uint32_t)a.G : 0u;
    auto load_step = [&](int st, v4i (&r)[PPT], uint32_t (&w)[NW], float &c) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) r[i] = *reinterpret_cast<const v4i *>(a.xq + (xo[i] + (uint32_t)(st * GE::SC)));
        load_words<NW>(a.W + (wo + (uint32_t)(st * 4 * GE::SB)), w);
        if constexpr (GROUPED) {
            const int gi = 2 * st + sc_grp;
            c = a.scales[so + (uint32_t)(gi < a.G ? gi : a.G - 1)];
        }
    };
    // The MFMA sums carry the weight codes' 2^SHIFT; the combine takes them unshifted against the group scale
    // times 2^-SHIFT: fmaf((float)sum, s * 2^-SHIFT, F) == fmaf((float)(sum >> SHIFT), s, F) bit for bit, since both
    // products are exact (|sum| < 2^24 and a power-of-two factor is exact for a normal scale). The staged scale is
    // s * 2^-SHIFT, and 0 for a group past the row's last one (a ragged final step), which then adds nothing:
    // F + 0 * x == F.
    constexpr float kUnshift = 1.0f / (float)(1 << GE::SHIFT);
    auto store_step = [&](int b, int st, const v4i (&r)[PPT], float c) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = threadIdx.x + i * kGemmThreads;
            if (PPT * kGemmThreads == TM * PR || pc < TM * PR) {
                const int t = pc / PR, q = pc - t * PR;
                *reinterpret_cast<v4i *>(&xa[b][t * LDA + 16 * q]) = r[i];
            }
        }
        if constexpr (GROUPED) scl[b][threadIdx.x] = 2 * st + sc_grp < a.G ? c * kUnshift : 0.0f;
    };

    float F[TT][4];
    v4i C[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        C[tt] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int v = 0; v < 4; ++v) F[tt][v] = 0.0f;
    }

    auto compute = [&](int b, int st, const uint32_t (&w)[NW]) __attribute__((always_inline)) {
        long bop[GE::NMF];
        decode<FMT, UD>(w, bop);
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
            const int8_t *xl = &xa[b][(16 * tt + r16) * LDA];
            if constexpr (FMT == kTern) {
                auto group = [&](auto grp_c) __attribute__((always_inline)) {
                    constexpr int grp = decltype(grp_c)::value;
                    long aop[UD];
                    load_ops<UD, (UD % 2 == 0)>(xl + 32 * UD * grp + 8 * UD * s, aop);
                    v4i cc = mfma_ops<grp * UD>(aop, bop, GROUPED ? v4i{0, 0, 0, 0} : C[tt]);
                    if constexpr (GROUPED) {
                        const int gi = 2 * st + grp;
                        if constexpr (ACC) {
                            if (gi < a.G) {
#pragma unroll
                                for (int v = 0; v < 4; ++v) {
                                    const int tok = m0 + 16 * tt + 4 * s + v;
                                    if (row_ok && tok < a.M)
                                        a.acc[((size_t)tok * a.N + row) * a.G + gi] = cc[v] >> GE::SHIFT;
                                }
                            }
                        } else {
                            const float cu = scl[b][64 * grp + 16 * wave + r16];
#pragma unroll
                            for (int v = 0; v < 4; ++v) F[tt][v] = fmaf((float)cc[v], cu, F[tt][v]);
                        }
                    } else {
                        C[tt] = cc;
                    }
                };
                group(std::integral_constant<int, 0>{});
                group(std::integral_constant<int, 1>{});
            } else {
                long aop[GE::NMF];
                load_ops<GE::NMF, true>(xl + (GE::SC / 4) * s, aop);
                C[tt] = mfma_ops<0>(aop, bop, C[tt]);
            }
        }
    };

    // The loop runs whole rounds of PF steps (register buffer k holds step PF * p + k; LDS buffer k & 1) and has
    // one exit, at its head; the last ns % PF steps follow it from buffers 0, 1, ... Every prefetch is issued, past
    // the split's last step as a reload of that step, and every staging store is made (past the last step into a
    // buffer no later step reads). A load or store skipped on some path, or an exit in the middle of the loop,
    // gives the loop head an entry with other loads in flight, and the compiler then waits there for nearly all
    // of them.
    const int s_last = s0 + ns - 1;
    auto clamp_step = [&](int st) { return st < s_last ? st : s_last; };
#pragma unroll
    for (int k = 0; k < PF; ++k) load_step(clamp_step(s0 + k), ra[k], wb[k], sc[k]);
    store_step(0, s0, ra[0], sc[0]);
    if ((int)threadIdx.x < TM) xs_l[threadIdx.x] = xsv;
    asm volatile("" :: "v"(rs), "v"(bb));   // keeps the loads here: the compiler sinks them to their use
    __syncthreads();
    const int nrounds = ns / PF;
    for (int p = 0; p < nrounds; ++p) {
        const int st = s0 + PF * p;
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            compute(k & 1, st + k, wb[k]);
            load_step(clamp_step(st + k + PF), ra[k], wb[k], sc[k]);
            store_step((k + 1) & 1, clamp_step(st + k + 1), ra[(k + 1) % PF], sc[(k + 1) % PF]);
            __syncthreads();
        }
    }
    {
        // buffer k holds step st + k; the first is staged in LDS buffer 0
        const int rem = ns - PF * nrounds, st = s0 + PF * nrounds;
#pragma unroll
        for (int k = 0; k + 1 < PF; ++k) {
            if (k < rem) {
                compute(k & 1, st + k, wb[k]);
                if (k + 1 < rem) {
                    store_step((k + 1) & 1, st + k + 1, ra[k + 1], sc[k + 1]);
                    __syncthreads();
                }
            }
        }
    }
    if constexpr (GROUPED && ACC) return;
    gemm_finish<FMT, UD, GROUPED, ACC, TT>(a, F, C, row, row_ok, m0, s, xs_l, rs, bb);
}

// ---- token-batch GEMM with the activation panel resident in LDS (launches of few workgroups) ----
//
// In qgemm_kernel each step of K is a chain: the activation block's loads, its LDS stores, a barrier, the LDS
// reads, the MFMAs. With one or two workgroups per CU nothing hides that chain (a step of 256 columns took about
// 350 ns at one workgroup per CU). This form stages the workgroup's whole activation panel [16*TT tokens x the
// split's columns] and, grouped, the 64 rows' group scales of those columns in LDS once, then each wave streams
// its weight codes through a ring of PF steps of loads in flight and reads its operands from LDS, with no barrier
// in the K loop. Tiles, MFMAs, the order of the group combine and the epilogue are qgemm_kernel's: the same bits.
constexpr int kPanelBatch = 8;   // group scales a thread has in flight at once

template <int FMT, int UD, bool GROUPED, int TT>
size_t panel_lds_bytes(int ns)
{
    return (size_t)16 * TT * (ns * Geo<FMT, UD>::SC + 16) + (GROUPED ? (size_t)2 * ns * 64 * sizeof(float) : 0);
}

template <int FMT, int UD, bool GROUPED, bool ACC, int TT, int PF>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2)))
void qgemm_panel_kernel(const int8_t *__restrict__ xq, const uint8_t *__restrict__ W,
                        const float *__restrict__ scales, int wld, int ldq, int M, int nsteps, int G, int N, QArgs a)
{
    a.xq = xq, a.W = W, a.scales = scales, a.wld = wld, a.ldq = ldq, a.M = M, a.nsteps = nsteps, a.G = G, a.N = N;
    using GE = Geo<FMT, UD>;
    constexpr int NW = GE::SB / 4;
    constexpr int TM = 16 * TT;
    constexpr int PR = GE::SC / 16;                // 16-byte pieces per token per step
    extern __shared__ __align__(16) int8_t pan[];  // [TM][ldp] int8 activations, then grouped [2 ns][64] scales
    __shared__ float xs_l[TM];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, s = lane >> 4;
    const int row = blockIdx.x * 64 + wave * 16 + r16;   // < rows_pad
    const bool row_ok = row < a.N;
    const int m0 = blockIdx.y * TM;
    const int s0 = (int)(blockIdx.z * a.nsteps / gridDim.z);
    const int ns = (int)((blockIdx.z + 1) * a.nsteps / gridDim.z) - s0;
    const int ldp = ns * GE::SC + 16;              // panel row stride: 16-byte aligned rows, 16 bytes apart in bank
    float *spn = reinterpret_cast<float *>(pan + TM * ldp);

    float rs, bb, xsv;
    gemm_epilogue_loads<GROUPED, TM>(a, row, m0, rs, bb, xsv);
    __builtin_amdgcn_sched_barrier(0);

    // the weight codes of the first PF steps (32-bit offsets from the uniform base, as qgemm_kernel)
    const uint32_t wo = (uint32_t)row * (uint32_t)a.wld + (uint32_t)(s * GE::SB);
    const int s_last = s0 + ns - 1;
    auto clamp_step = [&](int st) { return st < s_last ? st : s_last; };
    uint32_t wb[PF][NW];
    auto load_w = [&](int st, uint32_t (&w)[NW]) __attribute__((always_inline)) {
        load_words<NW>(a.W + (wo + (uint32_t)(st * 4 * GE::SB)), w);
    };
#pragma unroll
    for (int k = 0; k < PF; ++k) load_w(clamp_step(s0 + k), wb[k]);

    // the panel: thread t takes pieces t, t + 256, ... of every token row, the TM rows' loads in flight at once
    // (pieces past the row re-read its last one and are not stored; token rows past the batch repeat its last)
    constexpr int TR = TM < 32 ? TM : 32;   // token rows per pass (a 64-token panel takes two)
    const int prow = ns * PR;
    for (int q0 = 0; q0 < prow; q0 += kGemmThreads) {
        const int q = q0 + (int)threadIdx.x, qc = q < prow ? q : prow - 1;
#pragma unroll
        for (int t0 = 0; t0 < TM; t0 += TR) {
            v4i v[TR];
#pragma unroll
            for (int t = 0; t < TR; ++t) {
                const int tok = m0 + t0 + t < a.M ? m0 + t0 + t : a.M - 1;
                v[t] = *reinterpret_cast<const v4i *>(a.xq + ((uint32_t)tok * (uint32_t)a.ldq +
                                                              (uint32_t)(s0 * GE::SC + 16 * qc)));
            }
            if (q < prow) {
#pragma unroll
                for (int t = 0; t < TR; ++t) *reinterpret_cast<v4i *>(pan + (t0 + t) * ldp + 16 * q) = v[t];
            }
        }
    }
    // grouped: spn[lg][r] = scale of row 64 blockIdx.x + r, group 2 s0 + lg, times 2^-SHIFT (0 past the row's
    // last group, which then adds nothing: F + 0 * x == F). Thread t reads row t / 4, groups t % 4 + 4 i.
    constexpr float kUnshift = 1.0f / (float)(1 << GE::SHIFT);
    if constexpr (GROUPED) {
        const int ng = 2 * ns, r = (int)threadIdx.x >> 2, sr = blockIdx.x * 64 + r;
        const uint32_t so = (uint32_t)(sr < a.N ? sr : a.N - 1) * (uint32_t)a.G;
        for (int l0 = (int)threadIdx.x & 3; l0 < ng; l0 += 4 * kPanelBatch) {
            float c[kPanelBatch];
#pragma unroll
            for (int i = 0; i < kPanelBatch; ++i) {
                const int gi = 2 * s0 + l0 + 4 * i;
                c[i] = a.scales[so + (uint32_t)(gi < a.G ? gi : a.G - 1)];
            }
#pragma unroll
            for (int i = 0; i < kPanelBatch; ++i) {
                const int lg = l0 + 4 * i;
                if (lg < ng) spn[lg * 64 + r] = 2 * s0 + lg < a.G ? c[i] * kUnshift : 0.0f;
            }
        }
    }
    if ((int)threadIdx.x < TM) xs_l[threadIdx.x] = xsv;
    asm volatile("" :: "v"(rs), "v"(bb));   // keeps the loads here: the compiler sinks them to their use
    __syncthreads();

    float F[TT][4];
    v4i C[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        C[tt] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int v = 0; v < 4; ++v) F[tt][v] = 0.0f;
    }
    // The K loop is pipelined by hand: a step's LDS operands (and group scales) are read one step ahead, and a
    // scheduling barrier closes every step, so that the compiler does not hoist the next steps' code decodes
    // above this step's MFMAs (it did, and then waited for every weight load in flight at each round's start).
    constexpr int NG = FMT == kTern ? 2 : 1;          // operand groups of a step
    constexpr int NO = FMT == kTern ? UD : GE::NMF;   // 8-byte operands of a group
    long A[2][TT][NG][NO];
    float cu[2][NG];
    auto read_ops = [&](int st, long (&o)[TT][NG][NO], float (&c)[NG]) __attribute__((always_inline)) {
        const int ls = st - s0;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
            const int8_t *xl = pan + (16 * tt + r16) * ldp + ls * GE::SC;
            if constexpr (FMT == kTern) {
                load_ops<UD, (UD % 2 == 0)>(xl + 8 * UD * s, o[tt][0]);
                load_ops<UD, (UD % 2 == 0)>(xl + 32 * UD + 8 * UD * s, o[tt][1]);
            } else {
                load_ops<GE::NMF, true>(xl + (GE::SC / 4) * s, o[tt][0]);
            }
        }
        if constexpr (GROUPED && !ACC) {
            c[0] = spn[(2 * ls) * 64 + 16 * wave + r16];
            c[1] = spn[(2 * ls + 1) * 64 + 16 * wave + r16];
        }
    };
    auto compute = [&](int st, const uint32_t (&w)[NW], const long (&o)[TT][NG][NO], const float (&c)[NG])
        __attribute__((always_inline)) {
        long bop[GE::NMF];
        decode<FMT, UD>(w, bop);
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
            if constexpr (FMT == kTern) {
                auto group = [&](auto grp_c) __attribute__((always_inline)) {
                    constexpr int grp = decltype(grp_c)::value;
                    v4i cc = mfma_ops<grp * UD>(o[tt][grp], bop, GROUPED ? v4i{0, 0, 0, 0} : C[tt]);
                    if constexpr (GROUPED) {
                        const int gi = 2 * st + grp;
                        if constexpr (ACC) {
                            if (gi < a.G) {
#pragma unroll
                                for (int v = 0; v < 4; ++v) {
                                    const int tok = m0 + 16 * tt + 4 * s + v;
                                    if (row_ok && tok < a.M)
                                        a.acc[((size_t)tok * a.N + row) * a.G + gi] = cc[v] >> GE::SHIFT;
                                }
                            }
                        } else {
#pragma unroll
                            for (int v = 0; v < 4; ++v) F[tt][v] = fmaf((float)cc[v], c[grp], F[tt][v]);
                        }
                    } else {
                        C[tt] = cc;
                    }
                };
                group(std::integral_constant<int, 0>{});
                group(std::integral_constant<int, 1>{});
            } else {
                C[tt] = mfma_ops<0>(o[tt][0], bop, C[tt]);
            }
        }
    };
    // whole rounds of PF steps (register buffer k holds step PF * p + k; operand buffer k & 1), then the last
    // ns % PF steps; every prefetch is issued (past the split's last step a reload of it), so the loop head has
    // one set of loads in flight
    read_ops(s0, A[0], cu[0]);
    const int nrounds = ns / PF;
    for (int p = 0; p < nrounds; ++p) {
        const int st = s0 + PF * p;
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            read_ops(clamp_step(st + k + 1), A[(k + 1) & 1], cu[(k + 1) & 1]);
            compute(st + k, wb[k], A[k & 1], cu[k & 1]);
            load_w(clamp_step(st + k + PF), wb[k]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    {
        const int rem = ns - PF * nrounds, st = s0 + PF * nrounds;
#pragma unroll
        for (int k = 0; k + 1 < PF; ++k)
            if (k < rem) {
                read_ops(clamp_step(st + k + 1), A[(k + 1) & 1], cu[(k + 1) & 1]);
                compute(st + k, wb[k], A[k & 1], cu[k & 1]);
            }
    }
    if constexpr (GROUPED && ACC) return;
    gemm_finish<FMT, UD, GROUPED, ACC, TT>(a, F, C, row, row_ok, m0, s, xs_l, rs, bb);
}

// ---- small-batch GEMV (M <= kGemvMaxM): RT 16-row tiles per workgroup, ks waves per tile ----
//
// One MFMA covers 16 token rows (a token tile); a workgroup takes TT token tiles, each decoded weight step
// feeding TT MFMAs. A batch larger than the workgroup's rows (mw) is cut into token chunks, one workgroup per
// (row block, chunk). The workgroups of one row block are given ids 8 apart, which the dispatcher places on
// the same XCD one after another, so they read the same weight tile at about the same time through that XCD's
// L2. Each chunk's outputs are those of the whole batch (every token row is computed on its own).
//
// Each wave owns some steps of one tile. Order of work, chosen so no load waits on another:
//   1. the activation loads (the FP32 row slice of the fused prep, or the int8 row pieces to stage) and the
//      workgroup's group scales (one contiguous block of the scale array),
//   2. every weight load of the wave's steps (up to SPW steps in registers),
//   3. the prep (sign flip + blockwise WHT + absmax INT8 -- the operations of prep.hip, bit-identical) or the
//      copy, writing the int8 activations to LDS, while the weight loads are in flight,
//   4. the MFMAs, reading activations from LDS,
//   5. grouped: every exact per-group int32 sum goes to LDS and one thread per (token, row) combines them with
//      the scales in group order; row-scaled: the int32 partial sums of the K-split are added through LDS.
// Memory-level parallelism comes from the number of waves (up to 16 per workgroup, one to four steps each)
// rather than from long per-thread loops: for matrices of a few MB that is what keeps HBM busy. Every
// instruction of a wave is on its critical path (one or two waves per SIMD), so the prep is written for a
// short per-thread chain: few columns per thread, the WHT block fixed at compile time, DPP butterflies.

constexpr int kGemvMaxM = 63;    // token rows of the GEMV path (the GEMM takes 64 and more)
constexpr int kGemvTileM = 16;   // token rows of one MFMA (a token tile)
constexpr int kGemvMaxTT = 4;    // token tiles per workgroup
// Default token rows per workgroup above kFusedMaxM: two tiles. Four tiles staged at once (up to 64 rows of
// activations and their sums) hold a workgroup to one per CU with nothing to overlap its staging; measured
// slower than 32-row chunks on every shape tried.
constexpr int kGemvDefaultWgM = 32;
constexpr int kFusedMaxM = 8;    // token rows of the fused-prep GEMV (each workgroup preps them one by one)
constexpr int kMaxPieces = 8;   // 16-byte pieces of the staged int8 rows per thread (a count read at run time)
constexpr int kMaxScLoads = 8;

// Group sums staged in LDS as int16 where they fit: |sum| <= 128 * group <= 16384 for groups up to 128 columns
// (UD <= 4). That halves their LDS and lets 16 token rows of the g96 2560x6912 down projection fit one workgroup.
template <int FMT, int UD>
constexpr bool gemv_gs16() { return FMT == kTern && UD <= 4; }

// Scale loads per thread of the GEMV's group scales (a fixed count, so the waits count loads exactly): two for the
// BitNet layouts (g96, g128: up to 8 x the waves' groups per row), kMaxScLoads for the other group sizes.
template <int FMT, int UD, bool GROUPED>
constexpr int gemv_scl() { return FMT == kTern && GROUPED && (UD == 3 || UD == 4) ? 2 : kMaxScLoads; }

// E = 0: activations come prepped (xq/xs); E = 4/8/16: prep fused, E columns per thread, LB as in prep_finish.
// RT row tiles of 16 rows per workgroup; wave w works on tile w % RT and on steps w / RT, w / RT + ks, ... of
// it (ks = waves / RT). SPW: steps per wave held in registers at once; the first SPW are loaded unconditionally
// (a wave with fewer steps loads its last step again and skips the copies), later chunks only when a row has
// more steps. TT: token tiles (E = 0 only). SH: one token row combined from attention shares (PrepArgs::sh_o)
// in the prep.
//
// The leading arguments are what the first loads need, so they are preloaded into SGPRs at wave launch
// (-amdgpu-kernarg-preload-count, qlinear.hip's build line; struct arguments are not preloaded) and the
// activation and weight loads issue before any kernel-argument fetch returns (gemv_hot() builds them):
//   E > 0:  r0 = x row 0, r1 = signs, r2 = x2 (SwiGLU up rows), r3 = the norm weight (each null where absent:
//           not loaded), i0 = K;
//   SH:     r0 = shares' outputs, r1 = shares' maxima and sums, r2 = signs, r3 = norm weight (null where absent),
//           i0 = K, i1 bits 0..26 = the shares' head dim;
//   E = 0:  r0 = xq, r1 = xs, r2 = r3 unused, i0 = M, i1 bits 0..19 = ldq, bits 20..26 = token rows per workgroup;
//   every form: i1 bits 27..31 = ks, the waves per row tile (blockDim.x / 64 / RT: the workgroup size is itself
//           a kernel-argument fetch, and the weight steps of a wave depend on it).
// Loads are issued in the order activations, weights, scales, the weights and scales with a count known at
// compile time, so the prep waits for the activations alone.
//
// GLU (gated form, grouped FP32 outputs): the matrix stacks a gate half (rows 0 .. h - 1) over an up half (rows
// h .. 2h - 1), h = 16 * (i1 bits 0..26); a workgroup's first RT / 2 row tiles are gate tiles and its last RT / 2
// the matching up tiles, and it writes h rows y[r] = SiLU(gate_r) * up_r = (g * (1 / (1 + expf(-g)))) * u, the
// SwiGLU of the reference's FFN (src/eif_tinyllm.c:774-780) and the same expression as the SwiGLU pre-op of
// prep_finish, so a down projection fed with these rows and the RMSNorm pre-op gives the bits of one fed with
// the two halves and the SwiGLU pre-op.
template <int FMT, int UD, bool GROUPED, bool ACC, int E, int SPW, int LB, int RT, int TT = 1, bool SH = false,
          bool GLU = false, int OPS = kOpsAny>
__global__ __launch_bounds__(1024) void qgemv_kernel(const void *__restrict__ r0, const void *__restrict__ r1,
                                                     const void *__restrict__ r2, const void *__restrict__ r3,
                                                     const uint8_t *__restrict__ W, int wld, int nsteps, int i0,
                                                     int i1, QArgs a, PrepArgs p)
{
    static_assert(TT == 1 || E == 0, "token tiles with staged activations only");
    static_assert(!GLU || (GROUPED && !ACC && !SH && RT % 2 == 0), "the gated form: grouped FP32 outputs, paired tiles");
    using GE = Geo<FMT, UD>;
    constexpr int NW = GE::SB / 4;
    constexpr int EV = E > 0 ? E : 4;
    constexpr int MS = SPW;
    constexpr int TR = 16 * RT;   // rows per workgroup
    extern __shared__ __align__(16) int8_t smem[];
    __shared__ float xs_l[kGemvTileM * TT];
    __shared__ float red_max[16], red_ss[16];
    a.W = W, a.wld = wld, a.nsteps = nsteps;
    const int ks = (int)((unsigned)i1 >> 27), nthr = 64 * RT * ks;   // nthr == blockDim.x
    if constexpr (E == 0) {
        a.xq = static_cast<const int8_t *>(r0), a.xs = static_cast<const float *>(r1), a.M = i0;
        a.ldq = i1 & 0xFFFFF, a.mw = (i1 >> 20) & 0x7F;
    }
    // token chunks (E = 0 only): workgroup id -> (row block, chunk); ids 8 apart share the XCD (see above)
    int rb = blockIdx.x;
    if constexpr (E == 0) {
        if (a.mw > 0 && a.mw < a.M) {   // uniform
            const int nch = (a.M + a.mw - 1) / a.mw;
            const int xcd = blockIdx.x & 7, k = blockIdx.x >> 3;
            const int ch = k % nch;
            rb = (k / nch) * 8 + xcd;
            if (rb >= a.nrb) return;   // the grid is rounded up to whole XCD rounds
            const int m0 = ch * a.mw;
            a.M = min(a.mw, a.M - m0);
            a.xq += (size_t)m0 * a.ldq;
            a.xs += m0;
            a.y += (size_t)m0 * a.ldy;
            if (a.acc) a.acc += (size_t)m0 * a.N * (GROUPED ? a.G : 1);
        }
    }
    // the wave index through readfirstlane: a scalar, so the per-wave step bounds below are scalar branches
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rt = wv % RT, kw = wv / RT;
    const int r16 = lane & 15, s = lane >> 4;
    const int row0 = rb * TR;
    constexpr int RH = RT / 2;   // GLU: gate tiles per workgroup
    const int glu_t = GLU ? (i1 & 0x7FFFFFF) : 0;   // GLU: tiles of one half
    const int row = GLU ? (rt < RH ? rb * RH + rt : glu_t + rb * RH + rt - RH) * 16 + r16 : row0 + 16 * rt + r16;
    const int kpad = nsteps * GE::SC;
    const int nj = (nsteps - kw + ks - 1) / ks;
    int8_t *lds_x = smem;

    // 1. activation loads (preloaded pointers only)
    float v[EV], sg[EV], v2[EV], nwv[EV];
    v4i pc[kMaxPieces];   // the thread's 16-byte pieces of the int8 rows (np of them; a native vector type: an
                          // array of it stays in registers)
    const int pieces = kpad / 16;
    const int np = E == 0 ? (a.M * pieces + nthr - 1) / nthr : 0;
    auto piece_at = [&](int i) -> const v4i * {
        const int idx = threadIdx.x + i * nthr;
        const int ic = idx < a.M * pieces ? idx : a.M * pieces - 1;
        const int m = ic / pieces, c = ic - m * pieces;
        return reinterpret_cast<const v4i *>(a.xq + (size_t)m * a.ldq + 16 * c);
    };
    auto piece_store = [&](int i, const v4i &val) {
        const int idx = threadIdx.x + i * nthr;
        if (idx < a.M * pieces) {
            const int m = idx / pieces, c = idx - m * pieces;
            *reinterpret_cast<v4i *>(lds_x + m * p.ldl + 16 * c) = val;
        }
    };
    float xs_v = 0.0f;
    [[maybe_unused]] Shares<SH ? EV : 1> shv;
    if constexpr (SH) {
        prep_load_sh_rows<E, false, OPS>(static_cast<const float *>(r0), static_cast<const float *>(r1),
                                         static_cast<const float *>(r2), static_cast<const float *>(r3), i0,
                                         i1 & 0x7FFFFFF, shv, sg, nwv);
    } else if constexpr (E > 0) {
        prep_load_rows<E, false, OPS>(static_cast<const float *>(r0), static_cast<const float *>(r1),
                                      static_cast<const float *>(r2), static_cast<const float *>(r3), i0, v, sg, v2,
                                      nwv);
    } else {
#pragma unroll
        for (int i = 0; i < kMaxPieces; ++i)
            if (i < np) pc[i] = *piece_at(i);   // a uniform count: the loads after these stay fixed in number
        xs_v = a.xs[(int)threadIdx.x < a.M ? threadIdx.x : 0];
    }

    // Keep the activation loads ahead of the weight loads: loads complete in issue order, so staging them waits
    // for them alone.
    __builtin_amdgcn_sched_barrier(0);

    // 2. weight loads: unconditional, with the step clamped into the row (steps past nj are loaded from the
    // last step and never used); no branch, no wait.
    const uint8_t *wp = W + (size_t)row * wld + s * GE::SB;
    uint32_t wq[MS][NW];
    auto load_chunk = [&](int j0) {
#pragma unroll
        for (int j = 0; j < MS; ++j) {
            if (j0 > 0 && j0 + j >= nj) break;   // later chunks: wave-uniform bound
            const int stj = kw + (j0 + j) * ks;
            const int st = stj < nsteps ? stj : nsteps - 1;
            load_words<NW>(wp + (size_t)st * 4 * GE::SB, wq[j]);
        }
    };
    load_chunk(0);

    // 3. the workgroup's group scales, rows row0 .. row0 + TR - 1: one contiguous block of the [N, G] array,
    // loaded flat (gemv_scl() per thread, a fixed count) and staged in LDS after the prep. Row-scaled: the
    // row's scale and bias. A load with nothing to fetch reads an address the workgroup reads anyway (its first
    // scale, or the lane's own weight word), never one address shared by every workgroup: thousands of waves on
    // one cache line serialise on one L2 channel. The kernel arguments these need are read while the
    // activation and weight loads are in flight.
    __builtin_amdgcn_sched_barrier(0);
    const bool row_ok = row < a.N;
    using GS = std::conditional_t<gemv_gs16<FMT, UD>(), int16_t, int32_t>;   // staged group sums
    const int gld = gemv_gs16<FMT, UD>() ? (a.G + 7) & ~7 : (a.G + 3) & ~3;   // 16-byte rows of sums
    int32_t *red = reinterpret_cast<int32_t *>(smem + a.M * p.ldl);
    GS *acc_l = reinterpret_cast<GS *>(red);
    float *sc_l = reinterpret_cast<float *>(acc_l + a.M * TR * gld);
    constexpr int SCL = gemv_scl<FMT, UD, GROUPED>();
    float scv[SCL];
    // GLU: the gate tiles' block, then the up tiles' block (each RH * 16 rows, contiguous in [N, G])
    const int sbase = GLU ? rb * RH * 16 * a.G : row0 * a.G, shalf = RH * 16 * a.G, sup = glu_t * 16 * a.G;
    const int nsc = TR * a.G, last_sc = a.N * a.G - 1, sc0 = min(sbase, last_sc);
    float rs_raw = 0.0f, bb_raw = 0.0f, gb_raw = 0.0f;
    // The scale and bias loads address the matrix through the struct arguments (not preloaded), so issuing them
    // waits for the argument fetch. They are needed only by the epilogue: a fused prep issues them from its
    // middle (prep_finish's hook, by then the fetch has returned) rather than letting the fetch hold back its
    // start; the prepped form issues them here.
    auto issue_scales = [&]() __attribute__((always_inline)) {
        if constexpr (GROUPED && !ACC) {
#pragma unroll
            for (int i = 0; i < SCL; ++i) {
                const int l = (int)threadIdx.x + i * nthr;
                const int idx = sbase + l + (GLU && l >= shalf ? sup - shalf : 0);
                scv[i] = a.scales[idx <= last_sc && l < nsc ? idx : sc0];
            }
            // the bias of the row this thread combines (row0 + threadIdx % TR for every token)
            const int br = min(row0 + (int)threadIdx.x % TR, a.N - 1);
            gb_raw = *(a.bias ? a.bias + br : a.scales + sc0);
        }
        if constexpr (!GROUPED && !ACC) {
            const int rc = row_ok ? row : a.N - 1;
            const float *sp0 = a.scales ? a.scales + rc : reinterpret_cast<const float *>(wp);
            rs_raw = *sp0;
            bb_raw = *(a.bias ? a.bias + rc : sp0);
        }
    };
    if constexpr (E == 0) issue_scales();

    // 3. activations -> LDS
    if constexpr (SH) {
        sh_combine<E>(shv, v);
#pragma unroll
        for (int e = 0; e < E; ++e) v2[e] = 0.0f;
        prep_finish<E, LB, 0, OPS>(p, 0, kpad, v, sg, v2, nwv, lds_x, xs_l, red_max, red_ss, (int)threadIdx.x,
                                   issue_scales);
    } else if constexpr (E > 0) {
        prep_finish<E, LB, 0, OPS>(p, 0, kpad, v, sg, v2, nwv, lds_x, xs_l, red_max, red_ss, (int)threadIdx.x,
                                   issue_scales);
        for (int m = 1; m < a.M; ++m) {
            if constexpr (OPS == kOpsAny)
                prep_load<E>(p, m, v, sg, v2, nwv);
            else
                prep_load_rows<E, false, OPS>(p.x + (size_t)m * p.ldx, nullptr, nullptr,
                                              static_cast<const float *>(r3), p.K, v, sg, v2, nwv);
            prep_finish<E, LB, 0, OPS>(p, m, kpad, v, sg, v2, nwv, lds_x, xs_l, red_max, red_ss);
        }
    } else {
#pragma unroll
        for (int i = 0; i < kMaxPieces; ++i)
            if (i < np) piece_store(i, pc[i]);
        if ((int)threadIdx.x < a.M) xs_l[threadIdx.x] = xs_v;
        __syncthreads();
    }

    // 4. MFMAs. Token tile t: a lane's accumulator C[t] holds tokens 16t + 4s .. 16t + 4s + 3 (ntok of them live)
    // of row r16; tiles past the batch are skipped (a uniform bound).
    v4i C[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) C[t] = v4i{0, 0, 0, 0};
    for (int j0 = 0; j0 < nj; j0 += MS) {
        if (j0 > 0) load_chunk(j0);
#pragma unroll
        for (int j = 0; j < MS; ++j) {
            if (j0 + j >= nj) break;
            const int st = kw + (j0 + j) * ks;
            long bop[GE::NMF];
            decode<FMT, UD>(wq[j], bop);
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                if (t > 0 && 16 * t >= a.M) break;
                const int tb = 16 * t;
                const bool tok_ok = tb + r16 < a.M;
                const int8_t *xl = lds_x + (tok_ok ? tb + r16 : 0) * p.ldl;
                if constexpr (FMT == kTern) {
                    const int ntok = min(4, a.M - tb - 4 * s);
                    GS *accp = acc_l + ((tb + 4 * s) * TR + 16 * rt + r16) * gld;
                    auto group = [&](auto grp_c) __attribute__((always_inline)) {
                        constexpr int grp = decltype(grp_c)::value;
                        long aop[UD];
                        if (tok_ok) {
                            load_ops<UD, (UD % 2 == 0)>(xl + st * GE::SC + 32 * UD * grp + 8 * UD * s, aop);
                        } else {
#pragma unroll
                            for (int i = 0; i < UD; ++i) aop[i] = 0;
                        }
                        const v4i c = mfma_ops<grp * UD>(aop, bop, GROUPED ? v4i{0, 0, 0, 0} : C[t]);
                        if constexpr (GROUPED) {
                            const int gi = 2 * st + grp;
                            if (gi < a.G && ntok > 0) {
                                if constexpr (ACC) {
                                    if (row_ok) {
#pragma unroll
                                        for (int vv = 0; vv < 4; ++vv)
                                            if (vv < ntok)
                                                a.acc[((size_t)(tb + 4 * s + vv) * a.N + row) * a.G + gi] = c[vv] >> GE::SHIFT;
                                    }
                                } else {
                                    accp[gi] = (GS)(c[0] >> GE::SHIFT);
#pragma unroll
                                    for (int vv = 1; vv < 4; ++vv)
                                        if (vv < ntok) accp[vv * TR * gld + gi] = (GS)(c[vv] >> GE::SHIFT);
                                }
                            }
                        } else {
                            C[t] = c;
                        }
                    };
                    group(std::integral_constant<int, 0>{});
                    group(std::integral_constant<int, 1>{});
                } else {
                    long aop[GE::NMF];
                    if (tok_ok) {
                        load_ops<GE::NMF, true>(xl + st * GE::SC + (GE::SC / 4) * s, aop);
                    } else {
#pragma unroll
                        for (int i = 0; i < GE::NMF; ++i) aop[i] = 0;
                    }
                    C[t] = mfma_ops<0>(aop, bop, C[t]);
                }
            }
        }
    }
    if constexpr (GROUPED && ACC) return;

    if constexpr (GROUPED) {
        // 5. group combine, in group order for every (token, row): t = fmaf((float)acc_g, s[r,g], t); the
        // result does not depend on how the steps were split over waves. The scales are staged now, the
        // MFMAs above having waited for the weights alone.
#pragma unroll
        for (int i = 0; i < SCL; ++i) {
            const int idx = (int)threadIdx.x + i * nthr;
            if (idx < nsc) sc_l[idx] = scv[i];
        }
        __syncthreads();
        // the group sums of (token, local row r) combined with the row's scales
        auto combine = [&](int tok, int r) -> float {
            const GS *ap = acc_l + (tok * TR + r) * gld;
            const float *sp = sc_l + r * a.G;
            // four groups' sums as one 8-byte (int16) or 16-byte (int32) LDS load
            auto sums4 = [&](int g) {
                if constexpr (gemv_gs16<FMT, UD>()) {
                    const int2 h = *reinterpret_cast<const int2 *>(ap + g);
                    return int4{(int)(int16_t)(h.x & 0xFFFF), h.x >> 16, (int)(int16_t)(h.y & 0xFFFF), h.y >> 16};
                } else {
                    return *reinterpret_cast<const int4 *>(ap + g);
                }
            };
            float t = 0.0f;
            int g = 0;
            if ((a.G & 3) == 0) {   // the row's scales 16-byte aligned: 16 groups' sums and scales per LDS round trip
                for (; g + 16 <= a.G; g += 16) {
                    int4 av[4];
                    float4 sv[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        av[q] = sums4(g + 4 * q);
                        sv[q] = *reinterpret_cast<const float4 *>(sp + g + 4 * q);
                    }
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        t = fmaf((float)av[q].x, sv[q].x, t);
                        t = fmaf((float)av[q].y, sv[q].y, t);
                        t = fmaf((float)av[q].z, sv[q].z, t);
                        t = fmaf((float)av[q].w, sv[q].w, t);
                    }
                }
                for (; g + 4 <= a.G; g += 4) {
                    const int4 a4 = sums4(g);
                    const float4 s4 = *reinterpret_cast<const float4 *>(sp + g);
                    t = fmaf((float)a4.x, s4.x, t);
                    t = fmaf((float)a4.y, s4.y, t);
                    t = fmaf((float)a4.z, s4.z, t);
                    t = fmaf((float)a4.w, s4.w, t);
                }
            }
            for (; g + 4 <= a.G; g += 4) {
                const int4 a4 = sums4(g);
                t = fmaf((float)a4.x, sp[g], t);
                t = fmaf((float)a4.y, sp[g + 1], t);
                t = fmaf((float)a4.z, sp[g + 2], t);
                t = fmaf((float)a4.w, sp[g + 3], t);
            }
            for (; g < a.G; ++g) t = fmaf((float)ap[g], sp[g], t);
            return t;
        };
        if constexpr (GLU) {
            constexpr int TH = TR / 2;
            for (int c = threadIdx.x; c < TH * a.M; c += nthr) {
                const int tok = c / TH, r = c % TH, orow = rb * RH * 16 + r;
                if (orow >= 16 * glu_t) continue;
                const float g = combine(tok, r) * xs_l[tok], u = combine(tok, r + TH) * xs_l[tok];
                a.y[(size_t)tok * a.ldy + orow] = (g * (1.0f / (1.0f + expf(-g)))) * u;
            }
            return;
        }
        for (int c = threadIdx.x; c < TR * a.M; c += nthr) {
            const int tok = c / TR, r = c % TR, orow = row0 + r;
            if (orow >= a.N) continue;
            float out = combine(tok, r) * xs_l[tok];
            if (a.bias) out = out + gb_raw;
            a.y[(size_t)tok * a.ldy + orow] = out;
        }
        return;
    } else {
        // 5. K-split reduction of the exact int32 sums (waves with kw > 0 -> the kw == 0 wave of the tile)
        if (ks > 1) {
            if (kw > 0) {
#pragma unroll
                for (int t = 0; t < TT; ++t)
#pragma unroll
                    for (int vv = 0; vv < 4; ++vv) red[((((kw - 1) * RT + rt) * TT + t) * 4 + vv) * 64 + lane] = C[t][vv];
            }
            __syncthreads();
            if (kw > 0) return;
            for (int k = 0; k < ks - 1; ++k)
#pragma unroll
                for (int t = 0; t < TT; ++t)
#pragma unroll
                    for (int vv = 0; vv < 4; ++vv) C[t][vv] += red[(((k * RT + rt) * TT + t) * 4 + vv) * 64 + lane];
        }
        const float rs = a.scales ? rs_raw : 1.0f;
        float out0 = -INFINITY;
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) {
                const int tok = 16 * t + 4 * s + vv;
                if (tok >= a.M || !row_ok) continue;
                const int isum = C[t][vv] >> GE::SHIFT;
                if constexpr (ACC) {
                    a.acc[(size_t)tok * a.N + row] = isum;
                    continue;
                }
                float out = ((float)isum * xs_l[tok]) * rs;
                if (a.bias) out = out + bb_raw;
                a.y[(size_t)tok * a.ldy + row] = out;
                if (t == 0 && vv == 0) out0 = out;
            }
        }
        if constexpr (!ACC) {
            if (a.amax_key) {   // M = 1: lanes 0..15 (s = 0) hold the tile's rows; the tile's first largest
                unsigned long long key = eif_argmax_key(s == 0 ? out0 : -INFINITY, s == 0 && row_ok ? row : 0x7fffffff);
#pragma unroll
                for (int off = 1; off < 16; off <<= 1) {
                    const unsigned long long ok = __shfl_xor(key, off, 64);
                    key = ok > key ? ok : key;
                }
                if (lane == 0)
                    __hip_atomic_fetch_max(a.amax_key + (size_t)kArgmaxStride * ((rb * RT + rt) % kArgmaxSlots), key,
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}


// ---- streaming GEMV for vocabulary-sized row-scaled matrices (INT4, INT8) ----
//
// A workgroup of four waves stages the batch's int8 rows (M <= 16 TT) in LDS once, and each wave copies the MFMA
// activation operands of every step into registers. Waves then stride over the matrix's 16-row tiles, one tile
// per wave at a time, the next tile's codes (and the rows' scale and bias) loaded while the current one is
// multiplied. A tile's steps, MFMAs and epilogue are those of qgemv_kernel with one wave per tile, so the
// output bits are the same.
constexpr int kStreamThreads = 256;

template <int FMT, int UD, bool ACC, int NS, int TT, bool TMJ>
__global__ __launch_bounds__(kStreamThreads) void qstream_kernel(const int8_t *__restrict__ xq, const uint8_t *__restrict__ W,
                                                                  const float *__restrict__ scales, int wld, int ldq,
                                                                  int M, int N, int ntiles, QArgs a)
{
    a.xq = xq, a.W = W, a.scales = scales, a.wld = wld, a.ldq = ldq, a.M = M, a.N = N;   // preloaded (see qgemm_kernel)
    static_assert(FMT != kTern, "row-scaled INT4 / INT8 layouts");
    using GE = Geo<FMT, UD>;
    constexpr int NW = GE::SB / 4, NMF = GE::NMF;
    constexpr int ldl = NS * GE::SC + 16;   // LDS row stride: 16-byte aligned rows, 16 bytes apart in bank
    constexpr int PIECES = NS * GE::SC / 16;                                     // 16-byte pieces of a row
    constexpr int MAXP = (16 * TT * PIECES + kStreamThreads - 1) / kStreamThreads;   // pieces per thread
    extern __shared__ __align__(16) int8_t smem[];
    __shared__ float xs_l[16 * TT];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, s = lane >> 4;
    const int nw = gridDim.x * (kStreamThreads / 64);
    int t = blockIdx.x * (kStreamThreads / 64) + wave;

    // 1. the batch's int8 rows: loads first (they complete first), then the first tile's codes
    v4i pc[MAXP];   // a native vector type: an array of it stays in registers
    const int npc = a.M * PIECES;
#pragma unroll
    for (int i = 0; i < MAXP; ++i) {
        const int idx = min((int)threadIdx.x + i * kStreamThreads, npc - 1);
        const int m = idx / PIECES, c = idx - m * PIECES;
        pc[i] = *reinterpret_cast<const v4i *>(a.xq + (size_t)m * a.ldq + 16 * c);
    }
    const float xs_v = a.xs[(int)threadIdx.x < a.M ? threadIdx.x : 0];
    __builtin_amdgcn_sched_barrier(0);

    // a tile's loads: unconditional, the tile clamped into the matrix (rows are padded to whole tiles); an absent
    // scale or bias reads an address the lane reads anyway (its row's scale, else its first code word; selected at
    // use), so absent operands do not send every wave to one cache line
    auto load = [&](uint32_t (&w)[NS][NW], float &rs, float &bb, int tile) {
        const int row = min(tile, ntiles - 1) * 16 + r16;
        const uint8_t *wp = a.W + (size_t)row * a.wld + s * GE::SB;
        if constexpr (TMJ) {   // W is the tile-major copy: 1 KB of whole lines a load instruction
            const uint8_t *tp = a.W + (size_t)min(tile, ntiles - 1) * NS * 64 * GE::SB + 16 * lane;
#pragma unroll
            for (int st = 0; st < NS; ++st)
#pragma unroll
                for (int j = 0; j < NW / 4; ++j) {
                    const v4i v = __builtin_nontemporal_load(
                        reinterpret_cast<const v4i *>(tp + ((size_t)st * (NW / 4) + j) * 1024));
                    w[st][4 * j] = v[0], w[st][4 * j + 1] = v[1], w[st][4 * j + 2] = v[2], w[st][4 * j + 3] = v[3];
                }
        } else {
#pragma unroll
            for (int st = 0; st < NS; ++st) load_words<NW>(wp + (size_t)st * 4 * GE::SB, w[st]);
        }
        const int rc = min(row, a.N - 1);
        const float *sp0 = a.scales ? a.scales + rc : reinterpret_cast<const float *>(wp);
        rs = *sp0;
        bb = *(a.bias ? a.bias + rc : sp0);
    };
    uint32_t wA[NS][NW], wB[NS][NW];
    float rsA, bbA, rsB, bbB;
    load(wA, rsA, bbA, t);

    // indices past the batch were clamped to its last piece: those threads store the same bytes to the same place
#pragma unroll
    for (int i = 0; i < MAXP; ++i) {
        const int idx = min((int)threadIdx.x + i * kStreamThreads, npc - 1);
        const int m = idx / PIECES, c = idx - m * PIECES;
        *reinterpret_cast<v4i *>(smem + m * ldl + 16 * c) = pc[i];
    }
    if ((int)threadIdx.x < a.M) xs_l[threadIdx.x] = xs_v;
    __syncthreads();

    // 2. this lane's activation operands of every step and token tile, held in registers from here on (zeros
    // past the batch)
    long aop[TT][NS][NMF];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        const int tok = 16 * tt + r16;
        const int8_t *xl = smem + (tok < a.M ? tok : 0) * ldl + (GE::SC / 4) * s;
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            load_ops<NMF, true>(xl + st * GE::SC, aop[tt][st]);
            if (tok >= a.M) {
#pragma unroll
                for (int i = 0; i < NMF; ++i) aop[tt][st][i] = 0;
            }
        }
    }

    // 3. tiles
    auto work = [&](const uint32_t (&w)[NS][NW], float rs_raw, float bb_raw, int tile) {
        v4i C[TT];
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) C[tt] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            long bop[NMF];
            decode<FMT, UD>(w[st], bop);
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) C[tt] = mfma_ops<0>(aop[tt][st], bop, C[tt]);
        }
        const int row = tile * 16 + r16;
        if (tile >= ntiles || row >= a.N) return;
        const float rs = a.scales ? rs_raw : 1.0f;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) {
                const int tok = 16 * tt + 4 * s + vv;
                if (tok >= a.M) continue;
                const int isum = C[tt][vv] >> GE::SHIFT;
                if constexpr (ACC) {
                    a.acc[(size_t)tok * a.N + row] = isum;
                } else {
                    float out = ((float)isum * xs_l[tok]) * rs;
                    if (a.bias) out = out + bb_raw;
                    a.y[(size_t)tok * a.ldy + row] = out;
                }
            }
        }
    };
    while (t < ntiles) {   // the bound is the same for every lane of a wave
        load(wB, rsB, bbB, t + nw);
        work(wA, rsA, bbA, t);
        t += nw;
        if (t >= ntiles) break;
        load(wA, rsA, bbA, t + nw);
        work(wB, rsB, bbB, t);
        t += nw;
    }
}

// ---- row-pair GEMV for vocabulary-sized row-scaled matrices at one token row (INT4, INT8) ----
//
// The MFMA GEMV's load instructions each cover 64 bytes of 16 rows 512 bytes or more apart. Here each half-wave
// reads 512 contiguous bytes of one row, so a load instruction is two 512-byte runs of whole cache lines, and
// the products are taken with v_dot4_i32_i8 on the resident layouts as they are:
//   INT8: a row is in column order, so the 16-byte chunk k holds columns 16k .. 16k + 15;
//   INT4: the 16-byte chunk k of a row (step k / 4, slot k % 4) holds columns 32k .. 32k + 31: dword t's high
//         nibbles columns 32k + 8t + b, its low nibbles 32k + 8t + 4 + b (b = byte), each 16 v after masking.
// Lane h of a half reads chunks h, h + 32, .. (pass p = 0 .. P-1) of its row, so the activation bytes it needs
// are the same for every row: they are loaded once into registers. A wave takes one 16-row tile, 8 row pairs
// (half 0 the even row) x P passes, all its loads issued first. Each lane's sums of its 8 row pairs are summed
// over the half-wave by a transposed reduction (xor 16, 8, 4 exchanging half the values each time, then xor
// 2, 1), which leaves the sum of row pair (h >> 2) on the four lanes of each quad. The int32 sums are exact, so
// y has the MFMA GEMV's bits: ((float)isum * xs) * s[r] (+ bias); the per-tile maxima too. The codes are read
// once each, in whole-line runs, with non-temporal loads: the INT4 151936x1024 head 15.3 -> 13.4 us, the INT8
// 128256x2560 head 54.8 -> 48.0 us against plain loads (the streaming GEMV's 16-row pattern lost with them).
constexpr int kRowPairThreads = 256;
// Passes of 512 bytes per row it is compiled for (32 registers of codes per pass, plus 8 (INT4) or 4 (INT8) of
// activations): INT4 K up to 4096, INT8 K up to 2560.
template <int FMT>
constexpr int rowpair_max_p() { return FMT == kI4 ? 4 : 5; }

template <int FMT, int P, bool ACC>
__global__ __launch_bounds__(kRowPairThreads) void qrowpair_kernel(const int8_t *__restrict__ xq, const uint8_t *__restrict__ W,
                                                                    const float *__restrict__ scales, int wld, int N,
                                                                    int ntiles, QArgs a)
{
    a.xq = xq, a.W = W, a.scales = scales, a.wld = wld, a.N = N;   // preloaded (see qgemm_kernel)
    static_assert(FMT == kI4 || FMT == kI8, "row-scaled INT4 / INT8 layouts");
    constexpr int SHIFT = Geo<FMT, 0>::SHIFT;
    constexpr int CB = FMT == kI4 ? 32 : 16;   // activation bytes (columns) of a 16-byte chunk
    const int lane = threadIdx.x & 63, h = lane & 31, half = lane >> 5;
    const int tile = blockIdx.x * (kRowPairThreads / 64) + (int)(threadIdx.x >> 6);
    if (tile >= ntiles) return;   // the last workgroup's spare waves (no barrier in this kernel)

    // 1. weight loads (rows are padded to whole tiles), then the activation chunks, the row's scale and bias
    uint4 wv[8][P];
    const uint8_t *wp = a.W + (size_t)(tile * 16 + half) * a.wld + 16 * h;
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int q = 0; q < P; ++q) {
            const v4i t = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(wp + (size_t)(2 * c) * a.wld + 512 * q));
            wv[c][q] = make_uint4((uint32_t)t.x, (uint32_t)t.y, (uint32_t)t.z, (uint32_t)t.w);
        }
    uint4 xv[P][CB / 16];
#pragma unroll
    for (int q = 0; q < P; ++q)
#pragma unroll
        for (int i = 0; i < CB / 16; ++i)
            xv[q][i] = *reinterpret_cast<const uint4 *>(a.xq + CB * (32 * q + h) + 16 * i);
    const int orow = tile * 16 + 2 * (h >> 2) + half;   // the row whose sum this lane's quad ends with
    const bool row_ok = orow < a.N;
    const int rc = row_ok ? orow : a.N - 1;
    // an absent scale or bias reads an address the lane reads anyway (its row's scale, else its first code word)
    const float *sp0 = a.scales ? a.scales + rc : reinterpret_cast<const float *>(wp);
    const float rs_raw = *sp0;
    const float bb_raw = *(a.bias ? a.bias + rc : sp0);
    const float xs = a.xs[0];
    const bool b4 = h & 16, b3 = h & 8, b2 = h & 4;
    // 2. dot products, row pair by row pair in load order
    int acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        int sum = 0;
#pragma unroll
        for (int q = 0; q < P; ++q) {
            const uint32_t d[4] = {wv[c][q].x, wv[c][q].y, wv[c][q].z, wv[c][q].w};
            if constexpr (FMT == kI4) {
                const uint32_t x8[8] = {xv[q][0].x, xv[q][0].y, xv[q][0].z, xv[q][0].w,
                                        xv[q][1].x, xv[q][1].y, xv[q][1].z, xv[q][1].w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    sum = __builtin_amdgcn_sdot4((int)(d[t] & 0xF0F0F0F0u), (int)x8[2 * t], sum, false);
                    sum = __builtin_amdgcn_sdot4((int)((d[t] << 4) & 0xF0F0F0F0u), (int)x8[2 * t + 1], sum, false);
                }
            } else {
                const uint32_t x4[4] = {xv[q][0].x, xv[q][0].y, xv[q][0].z, xv[q][0].w};
#pragma unroll
                for (int t = 0; t < 4; ++t) sum = __builtin_amdgcn_sdot4((int)d[t], (int)x4[t], sum, false);
            }
        }
        acc[c] = sum;
    }

    // 3. transposed reduction over the 32 lanes of the half
    int w4[4], w2[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int keep = b4 ? acc[4 + i] : acc[i], give = b4 ? acc[i] : acc[4 + i];
        w4[i] = keep + __shfl_xor(give, 16, 64);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int keep = b3 ? w4[2 + i] : w4[i], give = b3 ? w4[i] : w4[2 + i];
        w2[i] = keep + __shfl_xor(give, 8, 64);
    }
    int z = (b2 ? w2[1] : w2[0]) + __shfl_xor(b2 ? w2[0] : w2[1], 4, 64);
    z += __shfl_xor(z, 2, 64);
    z += __shfl_xor(z, 1, 64);

    // 4. epilogue: one lane per quad writes; the tile's largest output and its first row over all 16 rows
    const int isum = z >> SHIFT;
    float out = -INFINITY;
    if (row_ok) {
        if constexpr (ACC) {
            if ((h & 3) == 0) a.acc[orow] = isum;
        } else {
            out = ((float)isum * xs) * (a.scales ? rs_raw : 1.0f);
            if (a.bias) out = out + bb_raw;
            if ((h & 3) == 0) a.y[orow] = out;
        }
    }
    if constexpr (!ACC) {
        if (a.amax_key) {
            unsigned long long key = eif_argmax_key(out, row_ok ? orow : 0x7fffffff);
#pragma unroll
            for (int off = 4; off < 64; off <<= 1) {
                const unsigned long long ok = __shfl_xor(key, off, 64);
                key = ok > key ? ok : key;
            }
            if (lane == 0)
                __hip_atomic_fetch_max(a.amax_key + (size_t)kArgmaxStride * (tile % kArgmaxSlots), key, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// The fused prep on its own: token row m = blockIdx.x -> int8 codes xq[m, 0 .. ldq) (zeros past K) and xs[m].
// E columns per thread, the threads covering ldq; LB as in prep_finish.
template <int E, int LB>
__global__ __launch_bounds__(1024) void prep_spec_kernel(PrepArgs p, int8_t *xq, float *xs)
{
    __shared__ float red_max[16], red_ss[16];
    float v[E], sg[E], v2[E], nwv[E];
    const int m = blockIdx.x;
    prep_load<E>(p, m, v, sg, v2, nwv);
    prep_finish<E, LB>(p, m, p.ldl, v, sg, v2, nwv, xq, xs, red_max, red_ss);
}

// ---- repack kernels: reference formats -> GPU layouts (one thread per destination dword) ----

EIF_DEV int tern_code(const uint8_t *src, int sld, int rows, int cols, int r, int c)
{
    if (r >= rows || c >= cols) return 0;
    unsigned code = (src[(size_t)r * sld + (c >> 2)] >> (2 * (c & 3))) & 3u;
    return code == 1u ? 1 : (code == 2u ? -1 : 0);
}

// The tile-major copy of a row-scaled INT4 / INT8 matrix for the streaming GEMV: block (tile, step) holds the 64
// lanes' code bytes of that step in SB / 16 sub-blocks of 1 KB, sub-block j holding lane L's j-th 16-byte piece at
// L * 16, where lane L = 16 s + r reads row 16 tile + r, bytes 4 SB step + SB s + 16 j of the row-tile layout.
// One load instruction of a wave then covers 1 KB of whole cache lines. Thread i copies 16-byte piece i.
__global__ void tile_major_kernel(const uint4 *__restrict__ src, int wld, int nsteps, int sb, uint4 *__restrict__ dst,
                                  size_t n)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int L = (int)(i & 63), nj = sb / 16;
    const size_t blk = i >> 6;                       // (tile, step, j)
    const int j = (int)(blk % nj);
    const size_t ts = blk / nj;
    const int step = (int)(ts % nsteps);
    const size_t tile = ts / nsteps;
    const size_t off = (tile * 16 + (L & 15)) * (size_t)wld + (size_t)4 * sb * step + (size_t)sb * (L >> 4) + 16 * j;
    dst[i] = src[off / 16];
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
    uint8_t *tm;      // vocabulary-sized row-scaled INT4 / INT8 of 8 or 16 steps: the tile-major copy, else NULL
    size_t bytes;
};

namespace {

int g_gemm_min_tokens = 64;
int g_gemv_ksplit = 0;   // waves per row tile of the GEMV, 0 = pick_ks_gemv()
int g_gemv_rt = 0;       // row tiles per workgroup of the GEMV, 0 = chosen from the shape
int g_gemv_chunk = 0;    // token rows per GEMV workgroup above kFusedMaxM (1 .. 64, powers of 2), 0 = what fits
int g_gemv_prep_cols = 0;   // fewest columns per thread of the fused prep (4, 8, 16), 0 = chosen from the shape

int ud_supported(int ud) { return ud == 1 || ud == 2 || ud == 3 || ud == 4 || ud == 8; }

// Workspaces per (stream, issuing thread): launches that one thread issues on one stream run in order, so one
// buffer per such pair and purpose suffices, and two threads issuing on the same stream (e.g. the null stream)
// never share one. Slot 0 the GEMM's split along K, slot 1 the int8 rows of a separate prep. Grown outside graph
// capture (inside a capture a missing buffer returns NULL and the caller takes another path). Buffers are never
// freed before the process ends, also when replaced by larger ones: a graph captured on the stream keeps using
// the buffers it was captured with.
struct WsKey {
    hipStream_t st;
    std::thread::id tid;
    bool operator==(const WsKey &o) const { return st == o.st && tid == o.tid; }
};
struct WsKeyHash {
    size_t operator()(const WsKey &k) const
    {
        return std::hash<const void *>()((const void *)k.st) * 31u + std::hash<std::thread::id>()(k.tid);
    }
};
std::mutex g_ws_mu;
std::unordered_map<WsKey, std::pair<float *, size_t>, WsKeyHash> g_ws[2];

float *split_ws(hipStream_t st, size_t bytes, int slot = 0, bool *fresh = nullptr)
{
    std::lock_guard<std::mutex> lk(g_ws_mu);
    auto &w = g_ws[slot][WsKey{st, std::this_thread::get_id()}];
    if (fresh) *fresh = false;
    if (w.second < bytes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
        float *p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
        w = {p, bytes};   // the old buffer stays allocated
        if (fresh) *fresh = true;
    }
    return w.first;
}

int device_cus()
{
    static const int n = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            return 256;
        return v;
    }();
    return n;
}

int g_gemm_split = 0;   // splits along K of the GEMM, 0 = chosen from the shape

// Splits along K (at most 16, at least three steps per split). Fewer tiles than CUs: none for a short K loop
// (under 24 steps, where a split's coherent round trip costs more than the steps it takes off), else about two
// workgroups per CU for grouped ternary, floor(2 CUs / tiles), and one for the row-scaled formats, floor(CUs /
// tiles), keeping six steps or more per split. One round or more: 3 (grouped) or 2 when a long K (24 steps or
// more) leaves the last round under 70% full (e.g. 320 tiles on 256 CUs). 1 for the parity outputs and when no
// workspace can be had (first use of a stream inside a graph capture). Measured per shape (µs): g96 2560x6912 at
// 64 and 128 tokens 9.1 and 12.0 at 3 splits, 11.1 and 19.9 unsplit, at 512 tokens 31.6 at 3, 33.6 at 2; INT8
// 896x4864 at 64, 128 and 256 tokens 8.0 at 4, 9.6 at 2, 12.7 unsplit, against 9.1, 10.2 and 14.3 at 6, 4, 2;
// INT4 1024x3584 at 128 tokens 6.7 at 2, 7.1 at 4.
int choose_split(int nsteps, int tiles, bool grouped)
{
    int ks = g_gemm_split;
    if (ks == 0) {
        const int C = device_cus();
        if (tiles < C)
            ks = nsteps < 24 ? 1 : std::max(1, std::min((grouped ? 2 : 1) * C / std::max(1, tiles), nsteps / 6));
        else
            ks = nsteps >= 24 && (double)tiles < 0.7 * eif_ceil_div(tiles, C) * C ? (grouped ? 3 : 2) : 1;
    }
    return std::min(ks, std::min(16, std::max(1, nsteps / 3)));
}

// The fixed scratch of eif_hip_qlinear_ex_noalloc: the GEMM's split-along-K partials, kScratchFloats floats in the
// code object's device memory (every device the library runs on holds one until the process ends). Host code
// uses its address per device from hipGetSymbolAddress (g_scratch_dev), never the array's name.
constexpr size_t kScratchFloats = (size_t)8 << 20;   // 32 MiB
static __device__ __align__(256) float scratch[kScratchFloats];
// The split GEMM's arrival counters: one per output tile, zero between launches (each tile's last arrival resets
// its own). The fixed scratch has its own (zero when the code object is loaded); a per-stream workspace starts
// with them, zeroed when it is allocated.
constexpr int kMaxSplitTiles = 65536;
static __device__ __align__(256) int scratch_cnt[kMaxSplitTiles] = {};
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch_dev[kMaxDevices];
int *g_scratch_cnt_dev[kMaxDevices];

int g_gemm_tt = 0;   // token tiles of a GEMM workgroup (1, 2, 4), 0 = chosen from the batch

// Token tiles of the GEMM (16 x TT tokens per workgroup) for M tokens on rt64 tiles of 64 rows and nsteps steps
// of K. The largest tile that holds the batch (64 tokens above 32), made smaller while the workgroups do not
// fill the CUs once, since a workgroup's time is a chain of dependent steps and more, shorter chains finish
// sooner; each extra token tile re-reads the weight tile, mostly from L2, so a long K loop stops at four token
// tiles. Measured: INT8 896x896 at 128 tokens 7.7 us with 64-token tiles, 5.4 with 16; ternary 13824x2560 at 64
// tokens 13.7 / 10.5 (32-token tiles) / 13.9 (16); ternary 2560x2560 at 512 tokens 16.0 / 12.2 (32).
int gemm_tt(int M, int rt64, int nsteps, bool grouped)
{
    if (g_gemm_tt > 0) return g_gemm_tt;
    int tt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
    const int C = device_cus();
    auto wgs = [&](int t) { return rt64 * eif_ceil_div(M, 16 * t); };
    // a short K loop takes 32-token tiles below 1.5 workgroups per CU at 64 (ternary 2560x2560 at 512 tokens, 320
    // workgroups: 12.1 us with 32-token tiles, 13.9 with 64; 3840x2560, 480: 15.5 against 14.8; 13824x2560 at 128
    // tokens, 432: 16.6 against 14.9)
    if (tt == 4 && nsteps < 24 && 2 * wgs(4) < 3 * C) tt = 2;
    // grouped ternary with a long K loop keeps the weight tile's re-reads to four token tiles (g96 2560x6912 at
    // 128 tokens: 12.0 us with 32-token tiles, 18.7 with 16 and two splits)
    const int min_tt = grouped && nsteps >= 24 ? std::max(1, std::min(4, M / 64)) : 1;
    while (tt > min_tt && wgs(tt) < C) tt /= 2;
    return tt;
}

// A caller-provided split workspace (eif_hip_qlinear_ex_noalloc): while set on this thread, the GEMM takes its
// split partials from it instead of the per-stream workspace.
struct FixedWs {
    float *ptr = nullptr;
    size_t bytes = 0;
    int *cnt = nullptr;
};
thread_local FixedWs tl_fixed_ws;

// Splits along K for `tiles` output tiles of nv values per thread, with the partials' space (ks x tiles x 256
// threads x nv floats) and the tiles' counters; 1 when the launch is not split.
template <bool ACC>
int pick_split(QArgs &a, int tiles, int nv, bool grouped, hipStream_t st)
{
    if (ACC) return 1;
    const int ks = choose_split(a.nsteps, tiles, grouped);
    if (ks <= 1 || tiles > kMaxSplitTiles) return 1;
    const size_t bytes = (size_t)ks * tiles * kGemmThreads * nv * sizeof(float);
    if (tl_fixed_ws.ptr) {   // a fixed workspace too small for this split: -1, nothing is launched
        if (bytes > tl_fixed_ws.bytes) return -1;
        a.part = tl_fixed_ws.ptr;
        a.cnt = tl_fixed_ws.cnt;
        return ks;
    }
    constexpr size_t cnt_bytes = (size_t)kMaxSplitTiles * sizeof(int);
    bool fresh = false;
    float *ws = split_ws(st, cnt_bytes + bytes, 0, &fresh);
    if (!ws) return 1;
    a.cnt = reinterpret_cast<int *>(ws);
    a.part = ws + kMaxSplitTiles;
    if (fresh && hipMemsetAsync(a.cnt, 0, cnt_bytes, st) != hipSuccess) return -2;
    return ks;
}

int g_gemm_pf = 0;   // register buffers of the GEMM's prefetch ring (2, 4, 8), 0 = chosen from the launch
int g_gemm_panel = 0;   // the GEMM's panel form: 0 = for few workgroups, 1 = wherever its LDS fits, -1 = off

// LDS a workgroup may allocate on the current device (160 KiB on gfx950), read once per process.
size_t gemm_max_lds()
{
    static const size_t bytes = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            return (size_t)65536;
        return (size_t)v;
    }();
    return bytes;
}

// Form and prefetch ring of a GEMM launch of `wgs` workgroups (tiles x splits ks) whose K loops take up to ns
// steps, with `wpc` panel workgroups fitting a CU's LDS (pf > 0: the tiled form with that ring; pf < 0: the
// panel form with ring -pf). Measured per linear (µs, a launch in a graph of launches, weights rotated past the
// Infinity Cache):
// - row-scaled INT8 / INT4, an unsplit launch of one to four workgroups per CU that all fit at once: panel,
//   ring 8, when the split's steps all fit the first ring (INT8 9728x896, 7 steps, at 128 tokens 10.2 against 11.6
//   tiled with ring 4); with more steps the tiled form with ring 2 (INT8 at 128 tokens: 9728x1024, 8 steps, 13.8
//   against 17.7 as a panel; 9728x1152 14.1 against 18.4; 4864x1024 at 64 tokens 7.6 against 11.7);
// - more than two workgroups per CU otherwise: tiled, ring 2 (four waves per SIMD hide each other's latency);
// - grouped ternary, every panel workgroup resident at once, and split along K, or a K loop of 20 steps or
//   more, or more workgroups than CUs: panel, ring 4 (down 2560x6912 g96 at 64 tokens, three splits: 8.5
//   against 10.6 tiled; gate+up 13824x2560 at 32 tokens 8.1 against 8.7);
// - else tiled, ring 4 with at most one workgroup per CU (QKV 3840x2560 at 64 tokens 5.6 against 6.2 with
//   ring 2), ring 2 above (gate+up at 64 tokens, whose 87 KB panels fit one a CU: 10.0 against 11.1 with ring
//   4, 12.7 as a panel).
int gemm_form(bool grouped, int wgs, int ks, int ns, int wpc)
{
    const int C = device_cus();
    const bool resident = wgs <= C * wpc;
    if (!grouped && ks == 1 && wgs > C && wgs <= 4 * C && resident && ns < 8) return -8;
    if (wgs > 2 * C) return 2;
    if (grouped && resident && (ks > 1 || ns >= 20 || wgs > C)) return -4;
    return wgs <= C ? 4 : 2;
}

template <int FMT, int UD, bool GROUPED, bool ACC, int TT>
int launch_gemm_t(QArgs a, int rows_pad, hipStream_t st)
{
    // the kernel addresses the batch rows and the weights with 32-bit offsets
    if ((size_t)a.M * a.ldq >= ((size_t)1 << 32) || (size_t)rows_pad * a.wld >= ((size_t)1 << 32)) return EIF_HIP_E_LIMIT;
    const int tm = eif_ceil_div(a.M, 16 * TT), tiles = rows_pad / 64 * tm;
    static_assert(TT == 1 || TT == 2 || TT == 4, "token tiles of gemm_tt");
    const int ks = pick_split<ACC>(a, tiles, 4 * TT, GROUPED, st);
    if (ks == -2) return EIF_HIP_E_DEVICE;
    if (ks < 0) return EIF_HIP_E_LIMIT;
    dim3 grid(rows_pad / 64, tm, ks);
    const int ns = eif_ceil_div(a.nsteps, ks);
    // panel workgroups a CU holds: by LDS, at most three (their registers)
    const size_t plds = panel_lds_bytes<FMT, UD, GROUPED, TT>(ns), pfoot = plds + 4 * 16 * TT + 64;
    const int wpc = (int)std::min<size_t>(3, gemm_max_lds() / pfoot);
    int form = ACC ? 2 : gemm_form(GROUPED, tiles * ks, ks, ns, wpc);
    if (g_gemm_panel != 0 && !ACC) form = g_gemm_panel > 0 ? -std::abs(form) : std::abs(form);
    if (g_gemm_pf > 0 && !ACC) form = form < 0 ? -std::max(g_gemm_pf, 4) : g_gemm_pf;
    if constexpr (!ACC) {
        // the panel form where its LDS fits
        if (form < 0 && wpc >= 1) {
            auto go_p = [&](auto pf_c) -> int {
                qgemm_panel_kernel<FMT, UD, GROUPED, ACC, TT, decltype(pf_c)::value><<<grid, kGemmThreads, plds, st>>>(
                    a.xq, a.W, a.scales, a.wld, a.ldq, a.M, a.nsteps, a.G, a.N, a);
                EIF_HIP_LAUNCHED();
                return EIF_HIP_OK;
            };
            if constexpr (TT < 4)
                if (form == -8) return go_p(std::integral_constant<int, 8>{});
            return go_p(std::integral_constant<int, 4>{});
        }
    }
    // a ring of 8 with 64-token tiles would spill (its activation pieces take 8 registers a step): 4 there
    const int pf = std::abs(form) > 4 && TT == 4 ? 4 : std::abs(form);
    auto go = [&](auto pf_c) -> int {
        qgemm_kernel<FMT, UD, GROUPED, ACC, TT, decltype(pf_c)::value><<<grid, kGemmThreads, 0, st>>>(
            a.xq, a.W, a.scales, a.wld, a.ldq, a.M, a.nsteps, a.G, a.N, a);
        EIF_HIP_LAUNCHED();
        return EIF_HIP_OK;
    };
    if constexpr (!ACC) {
        if (pf == 4) return go(std::integral_constant<int, 4>{});
        if constexpr (TT < 4)
            if (pf == 8) return go(std::integral_constant<int, 8>{});
    }
    return go(std::integral_constant<int, 2>{});
}

// Token tile of the GEMM: 16, 32 or 64 tokens (gemm_tt).
template <int FMT, int UD, bool GROUPED, bool ACC>
int launch_gemm(const QArgs &a, int rows_pad, hipStream_t st)
{
    switch (gemm_tt(a.M, rows_pad / 64, a.nsteps, GROUPED)) {
    case 1: return launch_gemm_t<FMT, UD, GROUPED, ACC, 1>(a, rows_pad, st);
    case 2: return launch_gemm_t<FMT, UD, GROUPED, ACC, 2>(a, rows_pad, st);
    default: return launch_gemm_t<FMT, UD, GROUPED, ACC, 4>(a, rows_pad, st);
    }
}

// Waves per tile of the small-batch GEMV (measured on MI355X with graph-chained launches): two steps per wave
// for the 1-9 MB matrices of a layer, four for long rows (>= 24 steps), eight for very long ones (>= 64 steps:
// INT8 896x4864 at one token 6.4 us with 10 waves, 7.6 with 16) and when the tiles alone fill the chip
// (vocabulary heads), at most 16 waves.
// Row tiles from which a row-scaled GEMV of prepped activations is shaped for streaming (one tile per
// workgroup, about 10 KiB of weights per wave) and from which eif_hip_qlinear_prep runs its prep separately once
// instead of in every workgroup (the vocabulary heads).
constexpr int kBigTiles = 4096;

int pick_ks_gemv(int row_tiles, int nsteps)
{
    const int spw = row_tiles >= 4096 || nsteps >= 64 ? 8 : (nsteps >= 24 ? 4 : 2);
    int ks = eif_ceil_div(nsteps, spw);
    return ks > 16 ? 16 : (ks < 1 ? 1 : ks);
}

// Token rows one GEMV workgroup takes: the chunk size, or the whole batch.
int gemv_wg_m(const QArgs &a) { return a.mw > 0 && a.mw < a.M ? a.mw : a.M; }
// Token tiles of a GEMV workgroup (the kernel's TT): 1, 2 or 4.
int gemv_tt(const QArgs &a)
{
    const int t = eif_ceil_div(gemv_wg_m(a), kGemvTileM);
    return t <= 1 ? 1 : (t == 2 ? 2 : 4);
}

// Dynamic LDS of qgemv_kernel: the staged int8 rows, then the group sums and scales (grouped) or the K-split
// partials (row-scaled).
size_t gemv_lds_bytes(bool grouped, bool gs16, const QArgs &a, int ldl, int rt, int ks)
{
    const size_t tr = 16 * (size_t)rt, m = (size_t)gemv_wg_m(a);
    const size_t gld = (size_t)(gs16 ? (a.G + 7) & ~7 : (a.G + 3) & ~3), gsb = gs16 ? 2 : 4;
    const size_t tail = grouped ? m * tr * gld * gsb + tr * (size_t)a.G * 4
                                : (size_t)(ks - 1) * rt * gemv_tt(a) * 4 * 64 * 4;
    return m * ldl + tail;
}

// Grid of a GEMV launch with nrb row blocks: one workgroup per row block, or with token chunks one per
// (row block, chunk) over whole rounds of the 8 XCDs (the kernel's id mapping; surplus ids return at once).
int gemv_grid(QArgs &a, int nrb)
{
    a.nrb = nrb;
    if (!(a.mw > 0 && a.mw < a.M)) return nrb;
    const int nch = eif_ceil_div(a.M, a.mw);
    return eif_ceil_div(nrb, 8) * 8 * nch;
}
// LDS a workgroup may allocate on the current device (160 KiB on gfx950), read once per process.
size_t gemv_max_lds()
{
    static const size_t bytes = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            return (size_t)65536;
        return (size_t)v;
    }();
    return bytes - 256;   // the kernel's static LDS (xs_l, red_max)
}

// Launch shapes compiled for every step count and tile count: the BitNet group layouts (g96, g128), ternary with
// one scale per row (the TTML / TLLM files), INT4 and INT8. The other ternary layouts get one shape (one tile per
// workgroup, SMAX steps per wave, block at run time).
template <int FMT, int UD, bool GROUPED>
constexpr bool gemv_tuned() { return FMT != kTern || UD == 4 || (GROUPED && UD == 3); }

// The preloaded leading arguments of qgemv_kernel (its header comment gives their meaning per form).
struct GemvHot {
    const void *r0, *r1, *r2, *r3;
    int i0, i1;
};

// The operand set of a fused prep (kOpsX ...) and, for kOpsMul, its multiplier: the signs count where the rows
// are rotated, the norm weight where a pre-op reads it.
int gemv_ops(const PrepArgs &p, const float **mul)
{
    const float *sg = p.block > 0 ? p.signs : nullptr, *nw = p.pre != EIF_HIP_PRE_NONE ? p.nw : nullptr;
    if (p.pre == EIF_HIP_PRE_SWIGLU_RMS || (sg && nw)) return kOpsAny;
    *mul = sg ? sg : nw;
    return *mul ? kOpsMul : kOpsX;
}

// ks: waves per row tile (1..16); ops: the kernel's operand set. Returns false when a field does not fit its
// bits (the launch is refused).
bool gemv_hot(const QArgs &a, const PrepArgs &p, bool fused, bool shares, int ks, GemvHot *h, int ops = kOpsAny)
{
    if (ks < 1 || ks > 16) return false;
    const unsigned kb = (unsigned)ks << 27;
    const float *mul = nullptr;
    if (ops != kOpsAny && gemv_ops(p, &mul) != ops) return false;
    if (shares) {
        const float *o = p.sh_o;
        if (p.sh_hd < 0 || p.sh_hd >= (1 << 27)) return false;
        if (ops == kOpsAny)
            *h = {o, p.sh_ml, p.signs, p.pre != EIF_HIP_PRE_NONE ? p.nw : nullptr, p.K, (int)((unsigned)p.sh_hd | kb)};
        else
            *h = {o, p.sh_ml, nullptr, mul, p.K, (int)((unsigned)p.sh_hd | kb)};
    } else if (fused) {
        if (ops == kOpsAny)
            *h = {p.x, p.signs, p.pre == EIF_HIP_PRE_SWIGLU_RMS ? p.x2 : nullptr,
                  p.pre != EIF_HIP_PRE_NONE ? p.nw : nullptr, p.K, (int)kb};
        else
            *h = {p.x, nullptr, nullptr, mul, p.K, (int)kb};
    } else {
        if (a.ldq < 0 || a.ldq >= (1 << 20) || a.mw < 0 || a.mw > 127) return false;
        *h = {a.xq, a.xs, a.xq, a.xq, a.M, (int)((unsigned)a.ldq | ((unsigned)a.mw << 20) | kb)};
    }
    return true;
}

template <int FMT, int UD, bool GROUPED, bool ACC, int E, int SPW, int LB, int RT, int TT, int OPS = kOpsAny>
int launch_gemv_s(const QArgs &a, const PrepArgs &p, int rows_pad, int ks, hipStream_t st)
{
    const size_t lds = gemv_lds_bytes(GROUPED, gemv_gs16<FMT, UD>(), a, p.ldl, RT, ks);
    QArgs ag = a;
    const int grid = gemv_grid(ag, rows_pad / (16 * RT));
    GemvHot h;
    if (!gemv_hot(ag, p, E > 0, false, ks, &h, OPS)) return EIF_HIP_E_LIMIT;   // a field beyond its packed bits
    qgemv_kernel<FMT, UD, GROUPED, ACC, E, SPW, LB, RT, TT, false, false, OPS><<<grid, 64 * RT * ks, lds, st>>>(
        h.r0, h.r1, h.r2, h.r3, ag.W, ag.wld, ag.nsteps, h.i0, h.i1, ag, p);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

// The gated form (qgemv_kernel's GLU): fused prep, ternary g128 layout, four row tiles per workgroup (two gate,
// two up), `half` output rows. E and the waves per tile follow launch_gemv_tiles' rules.
constexpr int kGluRT = 4;

template <int E, int SPW, int LB, int OPS>
int launch_glu_s(const QArgs &a, const PrepArgs &p, int half, int ks, hipStream_t st)
{
    const size_t lds = gemv_lds_bytes(true, true, a, p.ldl, kGluRT, ks);
    GemvHot h;
    if (!gemv_hot(a, p, true, false, ks, &h, OPS)) return EIF_HIP_E_LIMIT;
    h.i1 |= half / 16;   // bits 0..26: the tiles of one half
    qgemv_kernel<kTern, 4, true, false, E, SPW, LB, kGluRT, 1, false, true, OPS>
        <<<half / (16 * kGluRT / 2), 64 * kGluRT * ks, lds, st>>>(
        h.r0, h.r1, h.r2, h.r3, a.W, a.wld, a.nsteps, h.i0, h.i1, a, p);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

template <int E, int LB, int OPS = kOpsAny>
int launch_glu_e(const QArgs &a, const PrepArgs &p, int half, int ks, hipStream_t st)
{
    if constexpr (LB == 7 && OPS == kOpsAny) {   // the BitNet rotation: the operand set compiled in
        const float *mul = nullptr;
        const int ops = gemv_ops(p, &mul);
        if (ops == kOpsX) return launch_glu_e<E, LB, kOpsX>(a, p, half, ks, st);
        if (ops == kOpsMul) return launch_glu_e<E, LB, kOpsMul>(a, p, half, ks, st);
    }
    const int steps = eif_ceil_div(a.nsteps, ks);
    if (steps <= 1) return launch_glu_s<E, 1, LB, OPS>(a, p, half, ks, st);
    if (steps <= 2) return launch_glu_s<E, 2, LB, OPS>(a, p, half, ks, st);
    if (steps <= 4) return launch_glu_s<E, 4, LB, OPS>(a, p, half, ks, st);
    return launch_glu_s<E, 8, LB, OPS>(a, p, half, ks, st);
}

// The shares-combining form (one row, ternary weights, E = 4 or 8, one row tile per workgroup, one step per
// wave held at once).
template <int FMT, int UD, bool GROUPED, bool ACC, int E, int LB, int RT, int OPS = kOpsAny>
int launch_gemv_sh(const QArgs &a, const PrepArgs &p, int rows_pad, int ks, hipStream_t st)
{
    if constexpr (FMT == kTern && !ACC && (E == 4 || E == 8) && RT == 1) {
        const size_t lds = gemv_lds_bytes(GROUPED, gemv_gs16<FMT, UD>(), a, p.ldl, RT, ks);
        GemvHot h;
        if (!gemv_hot(a, p, true, true, ks, &h, OPS)) return EIF_HIP_E_LIMIT;
        qgemv_kernel<FMT, UD, GROUPED, ACC, E, 1, LB, RT, 1, true, false, OPS><<<rows_pad / 16, 64 * ks, lds, st>>>(
            h.r0, h.r1, h.r2, h.r3, a.W, a.wld, a.nsteps, h.i0, h.i1, a, p);
        EIF_HIP_LAUNCHED();
        return EIF_HIP_OK;
    } else {
        return EIF_HIP_E_ARG;
    }
}

template <int FMT, int UD, bool GROUPED, bool ACC, int E, int LB, int RT, int TT = 1, int OPS = kOpsAny>
int launch_gemv_e(const QArgs &a, const PrepArgs &p, int rows_pad, int ks, hipStream_t st)
{
    if (p.sh_ml) return launch_gemv_sh<FMT, UD, GROUPED, ACC, E, LB, RT, OPS>(a, p, rows_pad, ks, st);
    constexpr int SMAX = Geo<FMT, UD>::SB >= 32 ? 4 : 8;   // 8-dword steps: half the registers per chunk
    const int steps = eif_ceil_div(a.nsteps, ks);
    if constexpr (ACC || !gemv_tuned<FMT, UD, GROUPED>()) {
        return launch_gemv_s<FMT, UD, GROUPED, ACC, E, SMAX, LB, RT, TT, OPS>(a, p, rows_pad, ks, st);
    } else {
        if (steps <= 1) return launch_gemv_s<FMT, UD, GROUPED, ACC, E, 1, LB, RT, TT, OPS>(a, p, rows_pad, ks, st);
        if (steps <= 2) return launch_gemv_s<FMT, UD, GROUPED, ACC, E, 2, LB, RT, TT, OPS>(a, p, rows_pad, ks, st);
        if (steps <= 4 || SMAX == 4)
            return launch_gemv_s<FMT, UD, GROUPED, ACC, E, 4, LB, RT, TT, OPS>(a, p, rows_pad, ks, st);
        return launch_gemv_s<FMT, UD, GROUPED, ACC, E, SMAX, LB, RT, TT, OPS>(a, p, rows_pad, ks, st);
    }
}

template <int FMT, int UD, bool GROUPED, bool ACC, int E, int LB, int TT = 1, int OPS = kOpsAny>
int launch_gemv_rt(const QArgs &a, const PrepArgs &p, int rows_pad, int rt, int ks, hipStream_t st)
{
    if constexpr (gemv_tuned<FMT, UD, GROUPED>())
        if (rt == 4) return launch_gemv_e<FMT, UD, GROUPED, ACC, E, LB, 4, TT, OPS>(a, p, rows_pad, ks, st);
    return launch_gemv_e<FMT, UD, GROUPED, ACC, E, LB, 1, TT, OPS>(a, p, rows_pad, ks, st);
}

// Fused prep: E columns per thread. The WHT-128 of the BitNet configurations and no rotation (the INT8 head)
// are compiled with the block fixed; other blocks read it at run time.
template <int FMT, int UD, bool GROUPED, bool ACC, int E>
int launch_gemv_fused(const QArgs &a, const PrepArgs &p, int rows_pad, int rt, int ks, hipStream_t st)
{
    if constexpr (E <= 8 && gemv_tuned<FMT, UD, GROUPED>()) {
        if (p.block == 128) {
            // the BitNet rotation, the configurations that run it: the operand set compiled in, so the prep
            // reads only the columns it needs and the code before the weight loads has no branch
            if constexpr (!ACC && FMT == kTern) {
                const float *mul = nullptr;
                const int ops = gemv_ops(p, &mul);
                if (ops == kOpsX) return launch_gemv_rt<FMT, UD, GROUPED, ACC, E, 7, 1, kOpsX>(a, p, rows_pad, rt, ks, st);
                if (ops == kOpsMul)
                    return launch_gemv_rt<FMT, UD, GROUPED, ACC, E, 7, 1, kOpsMul>(a, p, rows_pad, rt, ks, st);
            }
            return launch_gemv_rt<FMT, UD, GROUPED, ACC, E, 7>(a, p, rows_pad, rt, ks, st);
        }
        if (p.block == 0 && !ACC) return launch_gemv_rt<FMT, UD, GROUPED, ACC, E, 0>(a, p, rows_pad, rt, ks, st);
    }
    return launch_gemv_rt<FMT, UD, GROUPED, ACC, E, -1>(a, p, rows_pad, rt, ks, st);
}

// Returns 1 when the shape is outside what the small-batch kernel stages (the caller uses the GEMM).
// Shape: four row tiles per workgroup for matrices of 768 tiles or more (fewer workgroups repeat the
// activation prep and staging), ks waves per tile from pick_ks_gemv, raised until the threads cover the row
// (fused prep), the int8 pieces fit (kMaxPieces per thread) and the scale block fits (gemv_scl()).
template <int FMT, int UD, bool GROUPED, bool ACC>
int launch_gemv_tiles(const QArgs &a, const PrepArgs &p, int rows_pad, int rt, hipStream_t st)
{
    const int kpad = a.nsteps * Geo<FMT, UD>::SC;
    const int maxks = 16 / rt;
    // fused prep over four row tiles: four steps per wave (the row's coverage by the prep raises it as needed);
    // fewer waves measured faster there (gate+up 13824x2560 at one token 6.70 us with 12 waves, 6.96 with 16)
    int ks = g_gemv_ksplit > 0 ? g_gemv_ksplit
                               : (p.x && rt == 4 ? eif_ceil_div(a.nsteps, 4) : pick_ks_gemv(rows_pad / 16, a.nsteps));
    // row-scaled INT8 / INT4 at one token row, under 24 steps: 4 (INT8) or 8 (INT4) steps per wave, the waves'
    // combine costing more than the steps it takes off (INT8 9728x896 4.07 us against 4.29 with 2 steps a wave,
    // 896x896 2.53 against 2.72; INT4 7168x1024 3.10 against 3.25)
    if (FMT != kTern && !p.x && a.M == 1 && a.nsteps < 24 && g_gemv_ksplit <= 0)
        ks = eif_ceil_div(a.nsteps, FMT == kI8 ? 4 : 8);
    // grouped ternary on prepped activations: 10 waves for 24 steps or more (down 2560x6912 g96 at one row 5.4 us
    // against 5.6 with 9, at 8 rows 7.1 against 7.4); with 8 or more token rows a step per wave under 24 steps
    // (each step combines 8-16 rows' groups; at 8 rows QKV 3840x2560 4.1 us against 4.5 with 2 steps a wave,
    // O 3.9 against 4.2)
    if (GROUPED && !p.x && g_gemv_ksplit <= 0 && (a.nsteps >= 24 || a.M >= 8)) ks = a.nsteps < 24 ? a.nsteps : 10;
    // the one-shape group layouts (g32, g64, g256) on prepped rows, one token tile: SMAX - 2 steps a wave. Their
    // single launch shape holds SMAX steps in registers and loads all of them, a wave's last step again past its
    // own, so fewer waves with fuller registers load less (6912x2560 g64 at 1 / 8 rows 5.7 / 7.0 us against 9.3 /
    // 12.3, g32 8.0 / 9.7 against 8.9 / 10.5; 2560x6912 g32 at 16 rows 21.7 against 23.9, g256 at 8 rows 6.9
    // against 7.8; g64 there and g256 at 6912x2560 within 0.1 us either way)
    if constexpr (GROUPED && !gemv_tuned<FMT, UD, GROUPED>()) {
        constexpr int SMAX = Geo<FMT, UD>::SB >= 32 ? 4 : 8;   // launch_gemv_e's steps per wave
        if (!p.x && a.M <= kGemvTileM && g_gemv_ksplit <= 0) ks = eif_ceil_div(a.nsteps, std::max(2, SMAX - 2));
    }
    if (!GROUPED && !p.x && rows_pad / 16 >= kBigTiles && g_gemv_ksplit <= 0) {
        // row-scaled, many tiles, prepped activations: about 10 KiB of weights per wave
        const int row_bytes = a.nsteps * 4 * Geo<FMT, UD>::SB;
        ks = (16 * row_bytes + 5120) / 10240;
        ks = ks < 1 ? 1 : ks;
    }
    if (ks > maxks) ks = maxks;
    auto scales_fit = [&](int k) { return !GROUPED || ACC || a.G <= gemv_scl<FMT, UD, GROUPED>() * 4 * k; };
    auto lds_fit = [&](int k) { return gemv_lds_bytes(GROUPED, gemv_gs16<FMT, UD>(), a, p.ldl, rt, k) <= gemv_max_lds(); };
    if (p.x) {
        // E columns per thread: the fewest that let at most 16 waves cover the padded row, and a WHT block within
        // one wave. The prep is a chain of dependent steps per wave (cross-lane butterflies, reductions), so the
        // shortest chains win: E = 16 on 3 waves measured slower than E = 4 on 10 for K = 2560 (QKV 4.8 against
        // 4.1 us), E = 16 slower than E = 8 for K = 6912 (down 7.2 against 6.6 us). The standalone prep kernel
        // and the persistent decode step take the same E, so a pre-op's sum of squares has the same order there.
        // The one-shape group layouts at one token row with no pre-op (E does not change the prep's bits then):
        // 8 columns a thread on the fewest waves that cover the row (K = 2560: g64 8.4 us against 10.0 with 4
        // columns on 10 waves, g32 9.7 against 10.3, g256 7.6 against 9.4; K = 6912 takes 8 columns anyway).
        int e0 = 4;
        if constexpr (GROUPED && !gemv_tuned<FMT, UD, GROUPED>()) {
            if (a.M == 1 && p.pre == EIF_HIP_PRE_NONE && !p.sh_ml && g_gemv_prep_cols <= 0 && g_gemv_ksplit <= 0) {
                e0 = 8;
                ks = 1;
            }
        }
        for (int e = e0; e <= 16; e *= 2) {
            if (64 * e < p.block || e < g_gemv_prep_cols) continue;
            if (p.sh_ml && (e > 8 || p.sh_hd % e != 0)) continue;
            int k = ks;
            while (k < maxks && (64 * rt * k * e < kpad || !scales_fit(k))) ++k;
            if (64 * rt * k * e < kpad || !scales_fit(k)) continue;
            if (!lds_fit(k)) return EIF_HIP_E_LIMIT;
            if (e == 4) return launch_gemv_fused<FMT, UD, GROUPED, ACC, 4>(a, p, rows_pad, rt, k, st);
            if (e == 8) return launch_gemv_fused<FMT, UD, GROUPED, ACC, 8>(a, p, rows_pad, rt, k, st);
            return launch_gemv_fused<FMT, UD, GROUPED, ACC, 16>(a, p, rows_pad, rt, k, st);
        }
        return EIF_HIP_E_LIMIT;
    }
    const int wm = gemv_wg_m(a);
    if (wm > kGemvTileM * kGemvMaxTT) return 1;
    // pieces per thread: kMaxPieces for one token tile (16 rows of the long down projections fit), 4 for more
    // rows, so that a 32-row batch of the layer shapes runs as two 16-row chunks (two workgroups a row block):
    // ternary 6912x2560 at 32 tokens 12.7 us as one 32-row chunk, 8.9 as two
    const int maxp = wm <= kGemvTileM ? kMaxPieces : 4;
    while (ks < maxks && (wm * (kpad / 16) > maxp * 64 * rt * ks || !scales_fit(ks))) ++ks;
    if (wm * (kpad / 16) > maxp * 64 * rt * ks || !scales_fit(ks) || !lds_fit(ks)) return 1;
    switch (gemv_tt(a)) {
    case 1: return launch_gemv_rt<FMT, UD, GROUPED, ACC, 0, 0, 1>(a, p, rows_pad, rt, ks, st);
    case 2: return launch_gemv_rt<FMT, UD, GROUPED, ACC, 0, 0, 2>(a, p, rows_pad, rt, ks, st);
    default: return launch_gemv_rt<FMT, UD, GROUPED, ACC, 0, 0, 4>(a, p, rows_pad, rt, ks, st);
    }
}

// Returns 1 when the shape is outside what the small-batch kernel stages (the caller uses the GEMM).
// Shape: four row tiles per workgroup for matrices of 768 tiles or more (fewer workgroups repeat the
// activation prep and staging), else one; ks waves per tile from pick_ks_gemv, raised until the threads cover
// the row (fused prep), the int8 pieces fit (kMaxPieces per thread) and the scale block fits (gemv_scl()).
// A shape that does not fit with four tiles is launched with one.
template <int FMT, int UD, bool GROUPED, bool ACC>
int launch_gemv_m(const QArgs &a, PrepArgs p, int rows_pad, hipStream_t st)
{
    p.ldl = a.nsteps * Geo<FMT, UD>::SC + 16;
    int rt = 1;
    if constexpr (gemv_tuned<FMT, UD, GROUPED>())
        if (!p.sh_ml) {
            const int tiles = rows_pad / 16;
            const bool chunked = a.M > kFusedMaxM && !p.x;
            // more than kFusedMaxM tokens: four tiles once the workgroups (row tiles x token chunks) reach 768
            // one token row of prepped activations: one tile (ternary 13824x2560 5.0 us against 6.3 with four)
            const bool four = chunked ? tiles * eif_ceil_div(a.M, gemv_wg_m(a)) >= 768
                                      : tiles >= 768 && (GROUPED || p.x || tiles < kBigTiles) && (p.x || a.M > 1);
            rt = g_gemv_rt > 0 ? g_gemv_rt : (four ? 4 : 1);
        }
    if (rt > 1) {
        const int rc = launch_gemv_tiles<FMT, UD, GROUPED, ACC>(a, p, rows_pad, rt, st);
        if (rc == EIF_HIP_OK || rc == EIF_HIP_E_DEVICE) return rc;
    }
    return launch_gemv_tiles<FMT, UD, GROUPED, ACC>(a, p, rows_pad, 1, st);
}

int g_gemv_rowpair = 0;   // 0 = vocabulary-sized matrices, 1 = every shape it takes, -1 = off
int g_gemv_stream = 0;   // streaming GEMV: waves per CU (0 = the default, -1 = off)
int g_gemv_stream_tm = 0;   // streaming GEMV: the tile-major copy where there is one (0), the row-tile layout (-1)
constexpr int kStreamWavesPerCU = 8;

template <int FMT, int UD, bool ACC, int NS, int TT>
int launch_stream_t(const QArgs &a, int rows_pad, const uint8_t *wt, hipStream_t st)
{
    const int ldl = NS * Geo<FMT, UD>::SC + 16, ntiles = rows_pad / 16;
    const int wpc = g_gemv_stream > 0 ? g_gemv_stream : kStreamWavesPerCU;
    const int waves = std::min(ntiles, device_cus() * wpc);
    const int grid = eif_ceil_div(waves, kStreamThreads / 64);
    if (wt)   // the tile-major copy
        qstream_kernel<FMT, UD, ACC, NS, TT, true><<<grid, kStreamThreads, (size_t)a.M * ldl, st>>>(
            a.xq, wt, a.scales, a.wld, a.ldq, a.M, a.N, ntiles, a);
    else
        qstream_kernel<FMT, UD, ACC, NS, TT, false><<<grid, kStreamThreads, (size_t)a.M * ldl, st>>>(
            a.xq, a.W, a.scales, a.wld, a.ldq, a.M, a.N, ntiles, a);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

template <int FMT, int UD, bool GROUPED, bool ACC>
int launch_stream(const QArgs &a, const PrepArgs &p, int rows_pad, const uint8_t *wt, hipStream_t st)
{
    if constexpr (FMT == kTern || GROUPED) {
        return 1;
    } else {
        if (g_gemv_stream < 0 || p.x || p.sh_ml || a.amax_key || a.M > 32 || rows_pad / 16 < kBigTiles) return 1;
        if (a.M < 4 && g_gemv_stream == 0) return 1;   // up to 3 token rows: the tiled GEMV measured as fast or faster
        if (g_gemv_stream_tm < 0) wt = nullptr;
        if (a.M <= 16) {
            if (a.nsteps == 8) return launch_stream_t<FMT, UD, ACC, 8, 1>(a, rows_pad, wt, st);
            if (a.nsteps == 16) return launch_stream_t<FMT, UD, ACC, 16, 1>(a, rows_pad, wt, st);
        } else {
            if (a.nsteps == 8) return launch_stream_t<FMT, UD, ACC, 8, 2>(a, rows_pad, wt, st);
        }
        return 1;
    }
}

// The row-pair GEMV: row-scaled INT4 / INT8 matrices at one prepped token row whose rows are whole 512-byte runs
// (at most rowpair_max_p of them); by default those of 1024 tiles (16,384 rows) or 20 MB of codes or more, where
// bandwidth decides. Returns 1 for other shapes. Measured at one token row (µs, tiled GEMV / row-pair, weights
// rotated past the Infinity Cache): INT8 9728x2560 6.86 / 6.61, 13824x2048 7.01 / 6.42, 27648x2560 14.1 / 12.2;
// INT4 16384x2048 5.51 / 4.99, 32768x2048 8.37 / 7.33, 32768x1024 4.96 / 4.74; below, the tiled GEMV: INT8
// 6912x2560 5.53 / 6.32, 4096x2560 4.34 / 6.01; INT4 8192x4096 5.59 / 5.98, 7168x1024 2.87 / 3.19.
constexpr int kRowPairTiles = 1024;
constexpr size_t kRowPairBytes = 20000000;

template <int FMT, int UD, bool GROUPED, bool ACC>
int launch_rowpair(const QArgs &a, const PrepArgs &p, int rows_pad, hipStream_t st)
{
    if constexpr (FMT == kTern || GROUPED) {
        return 1;
    } else {
        if (g_gemv_rowpair < 0 || p.x || p.sh_ml || a.M != 1 || a.wld % 512 != 0) return 1;
        const int ntiles = rows_pad / 16;
        if (g_gemv_rowpair == 0 && ntiles < kRowPairTiles && (size_t)rows_pad * a.wld < kRowPairBytes) return 1;
        const int grid = eif_ceil_div(ntiles, kRowPairThreads / 64);
        constexpr int PM = rowpair_max_p<FMT>();
        static_assert(PM <= 5, "one case per pass count");
#define EIF_RP(PP) qrowpair_kernel<FMT, PP, ACC><<<grid, kRowPairThreads, 0, st>>>(a.xq, a.W, a.scales, a.wld, a.N, ntiles, a)
        switch (a.wld / 512) {
        case 1: EIF_RP(1); break;
        case 2: EIF_RP(2); break;
        case 3: EIF_RP(3); break;
        case 4: EIF_RP(4); break;
        case 5:
            if constexpr (PM >= 5) {
                EIF_RP(PM >= 5 ? 5 : 1);
                break;
            }
            return 1;
        default: return 1;
        }
#undef EIF_RP
        EIF_HIP_LAUNCHED();
        return EIF_HIP_OK;
    }
}

// The batch in one workgroup when the fused prep or the shares are in (at most kFusedMaxM rows) or it is at
// most kFusedMaxM rows; else workgroups of mw token rows (token tiles, then chunks), mw from kGemvDefaultWgM
// (or the knob) halved until the staged rows and sums fit.
template <int FMT, int UD, bool GROUPED, bool ACC>
int launch_gemv(const QArgs &a, const PrepArgs &p, int rows_pad, const uint8_t *wt, hipStream_t st)
{
    const int rp = launch_rowpair<FMT, UD, GROUPED, ACC>(a, p, rows_pad, st);
    if (rp != 1) return rp;
    const int rs = launch_stream<FMT, UD, GROUPED, ACC>(a, p, rows_pad, wt, st);
    if (rs != 1) return rs;
    if (p.x || p.sh_ml || a.M <= kFusedMaxM) {
        if (a.M > (p.x ? kFusedMaxM : kGemvTileM)) return 1;
        QArgs a1 = a;
        a1.mw = 0;
        return launch_gemv_m<FMT, UD, GROUPED, ACC>(a1, p, rows_pad, st);
    }
    for (int mw = g_gemv_chunk > 0 ? g_gemv_chunk : kGemvDefaultWgM; mw >= 1; mw /= 2) {
        QArgs a1 = a;
        a1.mw = mw;
        const int rc = launch_gemv_m<FMT, UD, GROUPED, ACC>(a1, p, rows_pad, st);
        if (rc != 1) return rc;
    }
    return 1;
}

template <int FMT, int UD, bool GROUPED, bool ACC>
int launch_shape(const QArgs &a, const PrepArgs &p, int rows_pad, int path, hipStream_t st, const uint8_t *wt = nullptr)
{
    if (p.x || (path == EIF_HIP_PATH_GEMV && a.M <= kGemvMaxM)) {
        const int rc = launch_gemv<FMT, UD, GROUPED, ACC>(a, p, rows_pad, wt, st);
        if (rc != 1) return rc;
    }
    return launch_gemm<FMT, UD, GROUPED, ACC>(a, rows_pad, st);
}

template <bool ACC>
int dispatch(const eif_hip_qweight *w, const QArgs &a, const PrepArgs &p, int path, hipStream_t st)
{
    const bool grouped = w->fmt == kTern && w->group > 0;
    if (w->fmt == kI8) return launch_shape<kI8, 0, false, ACC>(a, p, w->rows_pad, path, st, w->tm);
    if (w->fmt == kI4) return launch_shape<kI4, 0, false, ACC>(a, p, w->rows_pad, path, st, w->tm);
    if (!grouped) return launch_shape<kTern, 4, false, ACC>(a, p, w->rows_pad, path, st);
    switch (w->ud) {
    case 1: return launch_shape<kTern, 1, true, ACC>(a, p, w->rows_pad, path, st);
    case 2: return launch_shape<kTern, 2, true, ACC>(a, p, w->rows_pad, path, st);
    case 3: return launch_shape<kTern, 3, true, ACC>(a, p, w->rows_pad, path, st);
    case 4: return launch_shape<kTern, 4, true, ACC>(a, p, w->rows_pad, path, st);
    case 8: return launch_shape<kTern, 8, true, ACC>(a, p, w->rows_pad, path, st);
    default: return EIF_HIP_E_ARG;
    }
}

// Prep arguments: x [M, ldx] FP32 with K columns, K % 32 == 0, 16-byte aligned rows and signs.
int make_prep_cols(int K, const float *x, int ldx, const float *signs, int block, float norm, PrepArgs *p)
{
    *p = PrepArgs{};
    if (!x || K < 32) return EIF_HIP_E_ARG;
    if (K % 32 != 0 || ldx < K || ldx % 4 != 0 || ((uintptr_t)x & 15) || ((uintptr_t)signs & 15))
        return EIF_HIP_E_ARG;
    if (block < 0 || block > 1024 || (block > 0 && ((block & (block - 1)) || K % block != 0))) return EIF_HIP_E_ARG;
    p->x = x;
    p->ldx = ldx;
    p->signs = signs;
    p->K = K;
    p->block = block;
    p->norm = norm;
    p->pre = EIF_HIP_PRE_NONE;
    return EIF_HIP_OK;
}

// Fused-prep arguments of a linear: K == cols, at most kFusedMaxM token rows.
int make_prep(const eif_hip_qweight *w, const float *x, int ldx, const float *signs, int block, float norm, int M,
              PrepArgs *p)
{
    *p = PrepArgs{};
    if (!w || !x || M < 1 || M > kFusedMaxM) return M > kFusedMaxM ? EIF_HIP_E_LIMIT : EIF_HIP_E_ARG;
    return make_prep_cols(w->cols, x, ldx, signs, block, norm, p);
}

// The pre-op fields of a prep spec (p already holds the rotation arguments).
int apply_pre(const eif_hip_prep_spec *sp, PrepArgs *p)
{
    if (sp->pre != EIF_HIP_PRE_NONE && sp->pre != EIF_HIP_PRE_RMS && sp->pre != EIF_HIP_PRE_SWIGLU_RMS)
        return EIF_HIP_E_ARG;
    if (sp->pre == EIF_HIP_PRE_SWIGLU_RMS && (!sp->x2 || ((uintptr_t)sp->x2 & 15))) return EIF_HIP_E_ARG;
    if (((uintptr_t)sp->norm_w & 15) || !(sp->eps >= 0.0f)) return EIF_HIP_E_ARG;
    p->pre = sp->pre;
    p->x2 = sp->x2;
    p->nw = sp->norm_w;
    p->eps = sp->eps;
    return EIF_HIP_OK;
}

// The prep kernel on its own, M token rows into xq [M, ldq] (ldq >= K, a multiple of 16) and xs [M]: E columns
// per thread, the fewest that cover ldq with at most 1024 threads and hold a WHT block within one wave.
template <int E>
int launch_prep_spec_e(PrepArgs p, int8_t *xq, float *xs, int M, hipStream_t st)
{
    const int threads = eif_ceil_div(eif_ceil_div(p.ldl, E), 64) * 64;
    if (p.block == 128) prep_spec_kernel<E, 7><<<M, threads, 0, st>>>(p, xq, xs);
    else if (p.block == 0) prep_spec_kernel<E, 0><<<M, threads, 0, st>>>(p, xq, xs);
    else prep_spec_kernel<E, -1><<<M, threads, 0, st>>>(p, xq, xs);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

int launch_prep_spec(PrepArgs p, int8_t *xq, int ldq, float *xs, int M, hipStream_t st)
{
    if (!xq || !xs || ldq < p.K || ldq % 16 != 0 || ((uintptr_t)xq & 15) || M < 1) return EIF_HIP_E_ARG;
    p.ldl = ldq;
    for (int e = 4; e <= 16; e *= 2) {
        if (64 * e < p.block || eif_ceil_div(ldq, e) > 1024) continue;
        if (e == 4) return launch_prep_spec_e<4>(p, xq, xs, M, st);
        if (e == 8) return launch_prep_spec_e<8>(p, xq, xs, M, st);
        return launch_prep_spec_e<16>(p, xq, xs, M, st);
    }
    return EIF_HIP_E_LIMIT;
}

int make_prep_spec(const eif_hip_qweight *w, const eif_hip_prep_spec *sp, int M, PrepArgs *p)
{
    if (!sp) return EIF_HIP_E_ARG;
    int rc = make_prep(w, sp->x, sp->ldx, sp->signs, sp->wht_block, sp->wht_norm, M, p);
    if (rc) return rc;
    return apply_pre(sp, p);
}

// A row-scaled GEMV launch only (no GEMM fallback): 1 when the shape does not fit the GEMV.
int gemv_rowscaled(const eif_hip_qweight *w, const QArgs &a, hipStream_t st)
{
    const PrepArgs p{};
    if (w->fmt == kI8) return launch_gemv<kI8, 0, false, false>(a, p, w->rows_pad, w->tm, st);
    if (w->fmt == kI4) return launch_gemv<kI4, 0, false, false>(a, p, w->rows_pad, w->tm, st);
    if (w->group == 0) return launch_gemv<kTern, 4, false, false>(a, p, w->rows_pad, nullptr, st);
    return EIF_HIP_E_ARG;
}

int check_linear_args(const eif_hip_qweight *w, const int8_t *xq, int ldq, int M)
{
    if (!w || M < 0) return EIF_HIP_E_ARG;
    if (M > 0 && (!xq || ldq < w->kpad || ldq % 16 != 0 || ((uintptr_t)xq & 15))) return EIF_HIP_E_ARG;
    return EIF_HIP_OK;
}

// Whether one GEMV workgroup can stage a full token tile (16 rows) of the weight's activations and sums.
bool gemv_fits_tile(const eif_hip_qweight *w)
{
    const bool grouped = w->fmt == kTern && w->group > 0, gs16 = w->fmt == kTern && w->ud <= 4;
    const size_t m = kGemvTileM, ldl = (size_t)w->kpad + 16;
    const size_t gld = (size_t)(gs16 ? (w->ngroups + 7) & ~7 : (w->ngroups + 3) & ~3), gsb = gs16 ? 2 : 4;
    const size_t lds = m * ldl + (grouped ? m * 16 * gld * gsb + 16 * (size_t)w->ngroups * 4 : 0);
    return m * (size_t)(w->kpad / 16) <= (size_t)kMaxPieces * 1024 && lds <= gemv_max_lds();
}

// Auto path (measured on MI355X, weights rotated past the Infinity Cache; us, GEMV / GEMM):
// * up to kFusedMaxM tokens: the GEMV;
// * group-scaled ternary, 9 .. 16 tokens: the GEMV for matrices of under 256 tiles of 16 rows and under 24 steps
//   of K, where a 16-row token tile fits one workgroup (GEMV / GEMM at 16 tokens, µs: 3840x2560 4.9 / 5.6,
//   2560x2560 4.7 / 5.5); the GEMM for the others (6912x2560 6.8 / 6.4, g96 2560x6912 9.1 / 8.2);
// * group-scaled ternary, 17 .. 63 tokens: the GEMM. The GEMV streams the weights once per 16- or 32-row token
//   chunk and stages every chunk's int8 rows and group sums in LDS, and at these batches it loses on every layer
//   shape (32 tokens: 3840x2560 7.3 / 5.7, 6912x2560 8.0 / 6.4, g96 2560x6912 17.2 / 9.0; 48 tokens:
//   9.7 / 5.7, 13.7 / 7.5, 17.6 / 8.7), so the dense contraction takes them below the 64-token line;
// * row-scaled matrices (INT8, INT4), 9 .. 63 tokens: the GEMV up to 16 tokens (INT8 4864x896 4.3 / 5.0, INT4
//   3584x1024 3.6 / 4.3), up to 32 for vocabulary-sized matrices (the streaming GEMV: INT4 151936x1024 at 32
//   tokens 19.2 / 27.1), and at any batch for matrices of fewer than 32 tiles of 64 rows (INT8 896x4864 at 48 /
//   63 tokens 7.6 / 7.6 against 8.1 / 9.3), and up to 32 tokens for INT8 matrices of 8192 rows or 16 steps of K
//   and more (17 / 32 tokens: 9728x896 5.5 / 6.8 against 6.8 / 7.0, 9728x1024 5.7 / 7.1 against 7.8 / 8.1,
//   4096x2048 5.3 / 6.3 against 7.8 / 7.9, 2560x2560 5.5 / 7.2 against 8.7 / 8.8) and INT4 ones of 2048 tiles
//   and more (32768x1024 7.0 / 7.8 against 7.1 / 7.8); the GEMM otherwise (INT8 4864x896 at 32 tokens 5.6
//   against 5.0, INT4 3584x1024 4.3 against 4.6, 7168x1024 5.8 against 4.3, 16384x2048 9.0 against 7.6).
constexpr int kGemvFewRows = 32 * 64;
constexpr int kGemvI8Rows = 8192;    // INT8 rows from which the GEMV takes up to 32 tokens
constexpr int kGemvI8Steps = 16;     // INT8 steps of K from which it does so too
constexpr int kGemvI4Tiles = 2048;   // INT4 tiles of 16 rows from which it does so

int resolve_path(const eif_hip_qweight *w, int path, int M)
{
    if (path != EIF_HIP_PATH_AUTO) return path;
    if (M >= g_gemm_min_tokens) return EIF_HIP_PATH_GEMM;
    if (M <= kFusedMaxM) return EIF_HIP_PATH_GEMV;
    if (!gemv_fits_tile(w)) return EIF_HIP_PATH_GEMM;
    const bool grouped = w->fmt == kTern && w->group > 0;
    const int tiles = w->rows_pad / 16;
    if (grouped) return M <= kGemvTileM && tiles < 256 && w->nsteps < 24 ? EIF_HIP_PATH_GEMV : EIF_HIP_PATH_GEMM;
    if (M <= kGemvTileM || w->rows_pad < kGemvFewRows) return EIF_HIP_PATH_GEMV;
    if (M > 2 * kGemvTileM) return EIF_HIP_PATH_GEMM;
    const bool big = tiles >= kBigTiles ||
                     (w->fmt == kI8 && (w->rows_pad >= kGemvI8Rows || w->nsteps >= kGemvI8Steps)) ||
                     (w->fmt == kI4 && tiles >= kGemvI4Tiles);
    return big ? EIF_HIP_PATH_GEMV : EIF_HIP_PATH_GEMM;
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

int qweight_row_tiles(const eif_hip_qweight *w) { return w ? w->rows_pad / 16 : 0; }

// The address of this device's scratch (device current), made once per device at eif_hip_init or at the first
// eif_hip_qlinear_ex_noalloc call on the device.
int scratch_init(int device, float **out, int **cnt)
{
    if (device < 0 || device >= kMaxDevices) return EIF_HIP_E_DEVICE;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_dev[device]) {
        void *ptr = nullptr, *cptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e == hipSuccess) e = hipGetSymbolAddress(&cptr, HIP_SYMBOL(scratch_cnt));
        if (e != hipSuccess || !ptr || !cptr) {
            fprintf(stderr, "libbitllm_hip: hipGetSymbolAddress(scratch) failed: %s\n", hipGetErrorString(e));
            return EIF_HIP_E_DEVICE;
        }
        g_scratch_dev[device] = static_cast<float *>(ptr);
        g_scratch_cnt_dev[device] = static_cast<int *>(cptr);
    }
    if (out) *out = g_scratch_dev[device];
    if (cnt) *cnt = g_scratch_cnt_dev[device];
    return EIF_HIP_OK;
}

int qweight_view(const eif_hip_qweight *w, QView *v)
{
    if (!w || !v) return EIF_HIP_E_ARG;
    *v = QView{w->w, w->scales, w->fmt, w->rows, w->cols, w->group, w->ud, w->kpad, w->rows_pad, w->nsteps, w->wld,
               w->ngroups};
    return EIF_HIP_OK;
}

// Row-scaled GEMV of one prepped token row that also folds the largest output and its first row into amax_key
// (atomic max of eif_argmax_key over the 16-row tiles into kArgmaxSlots slots, kArgmaxStride keys apart): the
// greedy argmax is the largest slot. The slots must hold 0 (or smaller keys) before the launch.
int qlinear_argmax(const eif_hip_qweight *w, const int8_t *xq, int ldq, const float *xs, float *y,
                   unsigned long long *amax_key, hipStream_t st)
{
    int rc = check_linear_args(w, xq, ldq, 1);
    if (rc) return rc;
    if (!xs || !y || !amax_key || (w->fmt == kTern && w->group > 0)) return EIF_HIP_E_ARG;
    QArgs a = make_args(w, xq, ldq, 1);
    a.xs = xs;
    a.y = y;
    a.ldy = w->rows;
    a.amax_key = amax_key;
    rc = gemv_rowscaled(w, a, st);
    return rc == 1 ? EIF_HIP_E_LIMIT : rc;
}

int qlinear_prep_shares(const eif_hip_qweight *w, const eif_hip_prep_spec *spec, const float *sh_o,
                        const float *sh_ml, int hd, const float *bias, float *y, int ldy, hipStream_t st)
{
    if (!w || !spec || !sh_o || !sh_ml || w->fmt != kTern || hd < 4 || w->cols % hd != 0 ||
        ((uintptr_t)sh_o & 15) || ((uintptr_t)sh_ml & 15) || spec->pre == EIF_HIP_PRE_SWIGLU_RMS)
        return EIF_HIP_E_ARG;
    eif_hip_prep_spec sp = *spec;
    sp.x = sh_o, sp.ldx = w->cols;   // the row's bounds checks (the kernel reads the shares instead)
    PrepArgs p;
    int rc = make_prep_spec(w, &sp, 1, &p);
    if (rc) return rc;
    if (!y || ldy < w->rows) return EIF_HIP_E_ARG;
    p.sh_o = sh_o, p.sh_ml = sh_ml, p.sh_hd = hd;
    QArgs a = make_args(w, nullptr, 0, 1);
    a.bias = bias;
    a.y = y;
    a.ldy = ldy;
    rc = dispatch<false>(w, a, p, EIF_HIP_PATH_GEMV, st);
    return rc == 1 ? EIF_HIP_E_LIMIT : rc;
}

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
    return dispatch<false>(w, a, PrepArgs{}, resolve_path(w, path, M), st);
}

}  // namespace eif

extern "C" int eif_hip_qlinear_f32(const eif_hip_qweight *w, const float *x, int ldx, const float *signs,
                                   int wht_block, float norm, const float *bias, float *y, int ldy, int M,
                                   void *stream)
{
    PrepArgs p;
    int rc = make_prep(w, x, ldx, signs, wht_block, norm, M, &p);
    if (rc) return rc;
    if (!y || ldy < w->rows) return EIF_HIP_E_ARG;
    QArgs a = make_args(w, nullptr, 0, M);
    a.bias = bias;
    a.y = y;
    a.ldy = ldy;
    return dispatch<false>(w, a, p, EIF_HIP_PATH_GEMV, (hipStream_t)stream);
}

// More than kFusedMaxM rows of a spec: the prep on its own into the stream's prep workspace (xq [M, kpad], then xs
// [M]), then the linear on the auto path. EIF_HIP_E_LIMIT when the workspace cannot be had (a stream's first such
// call inside a graph capture).
static int qlinear_prep_rows(const eif_hip_qweight *w, const eif_hip_prep_spec *spec, const float *bias, float *y,
                             int ldy, int32_t *acc, int M, hipStream_t st)
{
    PrepArgs p;
    int rc = make_prep_cols(w->cols, spec->x, spec->ldx, spec->signs, spec->wht_block, spec->wht_norm, &p);
    if (rc) return rc;
    if ((rc = apply_pre(spec, &p))) return rc;
    const size_t qb = (size_t)M * w->kpad, bytes = qb + 4 * (size_t)M + 16;
    int8_t *xq = reinterpret_cast<int8_t *>(split_ws(st, bytes, 1));
    if (!xq) return EIF_HIP_E_LIMIT;
    float *xs = reinterpret_cast<float *>(xq + ((qb + 15) & ~(size_t)15));
    if ((rc = launch_prep_spec(p, xq, w->kpad, xs, M, st))) return rc;
    if (acc) return eif_hip_qlinear_acc(w, xq, w->kpad, acc, M, EIF_HIP_PATH_AUTO, st);
    return eif::qlinear_scaled(w, w->scales, xq, w->kpad, xs, bias, y, ldy, M, EIF_HIP_PATH_AUTO, st);
}

extern "C" int eif_hip_qlinear_prep(const eif_hip_qweight *w, const eif_hip_prep_spec *spec, const float *bias,
                                    float *y, int ldy, int M, void *stream)
{
    if (w && spec && y && M > kFusedMaxM) {
        if (ldy < w->rows || (bias && bias + w->rows > y && bias < y + (size_t)M * ldy)) return EIF_HIP_E_ARG;
        return qlinear_prep_rows(w, spec, bias, y, ldy, nullptr, M, (hipStream_t)stream);
    }
    PrepArgs p;
    int rc = make_prep_spec(w, spec, M, &p);
    if (rc) return rc;
    if (!y || ldy < w->rows) return EIF_HIP_E_ARG;
    const hipStream_t st = (hipStream_t)stream;
    QArgs a = make_args(w, nullptr, 0, M);
    a.bias = bias;
    a.y = y;
    a.ldy = ldy;
    if (M == 1 && w->rows_pad / 16 >= kBigTiles && !(w->fmt == kTern && w->group > 0)) {
        // a vocabulary-sized row-scaled matrix: one prep, then the GEMV of the prepped row (the same codes
        // and scale as the fused prep, so the same output bits)
        int8_t *xq = reinterpret_cast<int8_t *>(split_ws(st, (size_t)w->kpad + 16, 1));
        if (xq) {
            float *xs = reinterpret_cast<float *>(xq + w->kpad);
            if ((rc = launch_prep_spec(p, xq, w->kpad, xs, 1, st))) return rc;
            a.xq = xq, a.ldq = w->kpad, a.xs = xs;
            rc = gemv_rowscaled(w, a, st);
            if (rc != 1) return rc;
        }
    }
    return dispatch<false>(w, a, p, EIF_HIP_PATH_GEMV, st);
}

// y[m, r] = SiLU(gate_r) * up_r for r < rows / 2 (gate = rows 0 .. rows/2 - 1 of w, up = the rest), one GEMV launch
// with the prep fused (qgemv_kernel's GLU form).
extern "C" int eif_hip_qlinear_prep_glu(const eif_hip_qweight *w, const eif_hip_prep_spec *spec, float *y, int ldy,
                                        int M, void *stream)
{
    PrepArgs p;
    int rc = make_prep_spec(w, spec, M, &p);
    if (rc) return rc;
    const int half = w->rows / 2;
    if (!y || ldy < half || w->rows % 2) return EIF_HIP_E_ARG;
    // the form's shapes: ternary g128, whole pairs of gate tiles per workgroup, the WHT-128 or none
    if (w->fmt != kTern || w->group != 128 || half % (16 * kGluRT / 2) || (p.block != 128 && p.block != 0))
        return EIF_HIP_E_LIMIT;
    QArgs a = make_args(w, nullptr, 0, M);
    a.y = y;
    a.ldy = ldy;
    p.ldl = a.nsteps * Geo<kTern, 4>::SC + 16;
    const int kpad = a.nsteps * Geo<kTern, 4>::SC, maxks = 16 / kGluRT;
    int ks = std::min(g_gemv_ksplit > 0 ? g_gemv_ksplit : eif_ceil_div(a.nsteps, 4), maxks);   // as launch_gemv_tiles
    const hipStream_t st = (hipStream_t)stream;
    for (int e = 4; e <= 8; e *= 2) {
        if (64 * e < p.block || e < g_gemv_prep_cols) continue;
        int k = ks;
        while (k < maxks && (64 * kGluRT * k * e < kpad || a.G > gemv_scl<kTern, 4, true>() * 4 * k)) ++k;
        if (64 * kGluRT * k * e < kpad || a.G > gemv_scl<kTern, 4, true>() * 4 * k) continue;
        if (gemv_lds_bytes(true, true, a, p.ldl, kGluRT, k) > gemv_max_lds()) return EIF_HIP_E_LIMIT;
        if (e == 4) return p.block == 128 ? launch_glu_e<4, 7>(a, p, half, k, st) : launch_glu_e<4, 0>(a, p, half, k, st);
        return p.block == 128 ? launch_glu_e<8, 7>(a, p, half, k, st) : launch_glu_e<8, 0>(a, p, half, k, st);
    }
    return EIF_HIP_E_LIMIT;
}

extern "C" int eif_hip_prep_spec_rows(const eif_hip_prep_spec *spec, int K, int8_t *xq, int ldq, float *xs, int M,
                                      void *stream)
{
    if (!spec || M < 0) return EIF_HIP_E_ARG;
    PrepArgs p;
    int rc = make_prep_cols(K, spec->x, spec->ldx, spec->signs, spec->wht_block, spec->wht_norm, &p);
    if (rc) return rc;
    if ((rc = apply_pre(spec, &p))) return rc;
    if (M == 0) return EIF_HIP_OK;
    return launch_prep_spec(p, xq, ldq, xs, M, (hipStream_t)stream);
}

extern "C" int eif_hip_qlinear_prep_acc(const eif_hip_qweight *w, const eif_hip_prep_spec *spec, int32_t *acc, int M,
                                        void *stream)
{
    if (w && spec && acc && M > kFusedMaxM) return qlinear_prep_rows(w, spec, nullptr, nullptr, 0, acc, M, (hipStream_t)stream);
    PrepArgs p;
    int rc = make_prep_spec(w, spec, M, &p);
    if (rc) return rc;
    if (!acc) return EIF_HIP_E_ARG;
    QArgs a = make_args(w, nullptr, 0, M);
    a.acc = acc;
    return dispatch<true>(w, a, p, EIF_HIP_PATH_GEMV, (hipStream_t)stream);
}

extern "C" int eif_hip_qlinear_f32_acc(const eif_hip_qweight *w, const float *x, int ldx, const float *signs,
                                       int wht_block, float norm, int32_t *acc, int M, void *stream)
{
    PrepArgs p;
    int rc = make_prep(w, x, ldx, signs, wht_block, norm, M, &p);
    if (rc) return rc;
    if (!acc) return EIF_HIP_E_ARG;
    QArgs a = make_args(w, nullptr, 0, M);
    a.acc = acc;
    return dispatch<true>(w, a, p, EIF_HIP_PATH_GEMV, (hipStream_t)stream);
}

extern "C" {

int eif_hip_set_gemm_min_tokens(int m)
{
    int old = g_gemm_min_tokens;
    if (m >= 1) g_gemm_min_tokens = m;
    return old;
}

int eif_hip_gemm_min_tokens(void) { return g_gemm_min_tokens; }

int eif_hip_set_gemv_ksplit(int k)
{
    int old = g_gemv_ksplit;
    if (k >= 0 && k <= 16) g_gemv_ksplit = k;
    return old;
}

int eif_hip_set_gemm_split(int k)
{
    int old = g_gemm_split;
    if (k >= 0 && k <= 16) g_gemm_split = k;
    return old;
}

int eif_hip_set_gemv_rowpair(int mode)
{
    const int old = g_gemv_rowpair;
    if (mode >= -1 && mode <= 1) g_gemv_rowpair = mode;
    return old;
}

int eif_hip_set_gemm_panel(int mode)
{
    const int old = g_gemm_panel;
    if (mode >= -1 && mode <= 1) g_gemm_panel = mode;
    return old;
}

int eif_hip_set_gemm_prefetch(int pf)
{
    const int old = g_gemm_pf;
    if (pf == 0 || pf == 2 || pf == 4 || pf == 8) g_gemm_pf = pf;
    return old;
}

int eif_hip_set_gemm_token_tiles(int tt)
{
    const int old = g_gemm_tt;
    if (tt == 0 || tt == 1 || tt == 2 || tt == 4) g_gemm_tt = tt;
    return old;
}

int eif_hip_set_gemv_prep_cols(int e)
{
    const int old = g_gemv_prep_cols;
    if (e == 0 || e == 4 || e == 8 || e == 16) g_gemv_prep_cols = e;
    return old;
}

int eif_hip_set_gemv_row_tiles(int rt)
{
    int old = g_gemv_rt;
    if (rt == 0 || rt == 1 || rt == 4) g_gemv_rt = rt;
    return old;
}

int eif_hip_set_gemv_stream(int wpc)
{
    const int old = g_gemv_stream_tm < 0 && g_gemv_stream >= 0 ? -2 - g_gemv_stream : g_gemv_stream;
    if (wpc >= -1 && wpc <= 32) {
        g_gemv_stream = wpc;
        g_gemv_stream_tm = 0;
    } else if (wpc <= -2 && wpc >= -34) {   // -2 - wpc: the same launch on the row-tile layout
        g_gemv_stream = -2 - wpc;
        g_gemv_stream_tm = -1;
    }
    return old;
}

int eif_hip_set_gemv_token_chunk(int m)
{
    const int old = g_gemv_chunk;
    if (m >= 0 && m <= 64 && (m & (m - 1)) == 0) g_gemv_chunk = m;
    return old;
}

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
        q.kpad = eif_round_up(cols, 128);
        q.wld = fmt == kI4 ? q.kpad / 2 : q.kpad;
        src_bytes = fmt == kI4 ? (size_t)rows * ((cols + 1) / 2) : (size_t)rows * cols;
        sc_count = rows;
    } else {
        return EIF_HIP_E_ARG;
    }
    if (fmt == kTern && group > 0 && !scales) return EIF_HIP_E_ARG;
    q.nsteps = q.kpad / (fmt == kTern ? 64 * q.ud : 128);
    const size_t wbytes = (size_t)q.rows_pad * q.wld;

    void *src_dev = nullptr;
    if (!src_on_device) {
        if (hipMalloc(&src_dev, src_bytes) != hipSuccess) return EIF_HIP_E_NOMEM;
        if (hipMemcpyAsync(src_dev, codes, src_bytes, hipMemcpyHostToDevice, st) != hipSuccess) {
            (void)hipFree(src_dev);
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
        if (hipGetLastError() != hipSuccess) rc = EIF_HIP_E_DEVICE;
    }
    // the streaming GEMV's tile-major copy (same bytes, another order)
    size_t tmbytes = 0;
    if (rc == EIF_HIP_OK && fmt != kTern && q.rows_pad / 16 >= kBigTiles && (q.nsteps == 8 || q.nsteps == 16)) {
        tmbytes = wbytes;
        if (hipMalloc(&q.tm, tmbytes) != hipSuccess) {
            rc = EIF_HIP_E_NOMEM;
        } else {
            const size_t n = tmbytes / 16;
            tile_major_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>((const uint4 *)q.w, q.wld, q.nsteps,
                                                                          fmt == kI4 ? 16 : 32, (uint4 *)q.tm, n);
            if (hipGetLastError() != hipSuccess) rc = EIF_HIP_E_DEVICE;
        }
    }
    if (rc == EIF_HIP_OK && hipStreamSynchronize(st) != hipSuccess) rc = EIF_HIP_E_DEVICE;
    if (src_dev) (void)hipFree(src_dev);
    if (rc != EIF_HIP_OK) {
        if (q.w) (void)hipFree(q.w);
        if (q.scales) (void)hipFree(q.scales);
        if (q.tm) (void)hipFree(q.tm);
        return rc;
    }
    q.bytes = wbytes + tmbytes + (scales ? sizeof(float) * sc_count : 0);
    eif_hip_qweight *h = new (std::nothrow) eif_hip_qweight(q);
    if (!h) {
        (void)hipFree(q.w);
        if (q.scales) (void)hipFree(q.scales);
        if (q.tm) (void)hipFree(q.tm);
        return EIF_HIP_E_NOMEM;
    }
    *out = h;
    return EIF_HIP_OK;
}

void eif_hip_qweight_destroy(eif_hip_qweight *w)
{
    if (!w) return;
    if (w->w) (void)hipFree(w->w);
    if (w->scales) (void)hipFree(w->scales);
    if (w->tm) (void)hipFree(w->tm);
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

int eif_hip_qlinear_ex_noalloc(const eif_hip_qweight *w, const int8_t *xq, int ldq, const float *xs,
                               const float *bias, float *y, int ldy, int M, int path, void *stream)
{
    if (!w) return EIF_HIP_E_ARG;
    int dev = 0;
    float *ws = nullptr;
    if (hipGetDevice(&dev) != hipSuccess) return EIF_HIP_E_DEVICE;
    int *cnt = nullptr;
    const int rc = eif::scratch_init(dev, &ws, &cnt);
    if (rc) return rc;
    tl_fixed_ws = FixedWs{ws, kScratchFloats * sizeof(float), cnt};
    const int r = eif::qlinear_scaled(w, w->scales, xq, ldq, xs, bias, y, ldy, M, path, (hipStream_t)stream);
    tl_fixed_ws = FixedWs{};
    return r;
}

size_t eif_hip_qlinear_noalloc_max_bytes(void) { return kScratchFloats * sizeof(float); }

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
    return dispatch<true>(w, a, PrepArgs{}, resolve_path(w, path, M), (hipStream_t)stream);
}

}  // extern "C"

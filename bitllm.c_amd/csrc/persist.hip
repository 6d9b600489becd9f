// persist.hip -- the BitNet decoder's token step (the layer stack of src/eif_tinyllm.c:371-857, BitNet path) as
// one persistent kernel: one 1024-thread workgroup per CU runs the five stages of every layer, the stages separated
// by grid barriers, and the next layer's weight tiles stream into LDS while the current layer computes.
//
// Per layer:   S1 RMSNorm + WHT + INT8 prep of x, QKV GEMV            -> qkv
//              S2 RoPE, fp16 KV append, attention per (head, chunk)   -> attention shares
//              S3 shares combined + sub-RMSNorm + prep, O GEMV        -> x += O out
//              S4 RMSNorm + prep of x, gate|up GEMV                   -> hb
//              S5 SiLU(gate) * up + sub-RMSNorm + prep, down GEMV     -> x += down out
// then the head's prep (RMSNorm + INT8 of x, no rotation) into hq / hs for the head GEMV that follows.
//
// Every stage computes what the decoder's separate launches compute, with the same code (qdev.h prep and MFMA
// helpers, attn_dev.h attention) and the same reduction trees: the workgroup's 16 waves hold the columns the
// separate launch's threads hold (threads past the row hold zeros, which leave every sum and maximum unchanged),
// each row tile's exact per-group int32 sums are combined in group order, and the attention runs per (head,
// chunk) on 512 threads as there. So the step gives the same bits as the separate launches.
//
// Work: the 16-row tiles of a linear go round-robin over the workgroups (tile j to workgroup j mod G); waves 0-13
// run the MFMAs of a workgroup's (tile, step) pairs. Waves 14 and 15 are loaders: wave 14 streams the QKV and
// gate|up tiles, wave 15 the O and down tiles, each as soon as the stage that used the previous layer's tiles has
// ended (global_load_lds, 12 or 16 bytes per lane straight into LDS: codes in the MFMA's lane order, then the
// tile's group scales). A loader waits for its own loads only (vmcnt counts per wave, loads complete in order),
// so the compute waves never wait behind the weight stream: their barriers wait for LDS traffic only (BAR = 1).
//
// Inter-workgroup data (x, qkv, hb, the shares) is written and read with device-coherent accesses (agent-scope
// relaxed atomics: sc1, past the XCDs' non-coherent L2 lines), each wave waiting for its stores before the
// barrier; the grid barrier is a two-level counter (eight groups of workgroups, then one top counter) whose last
// arrival publishes a generation flag per group. Spins are bounded: a wait that exceeds the bound sets a flag
// that every other workgroup sees at its next barrier, all workgroups leave, and the decoder reports the step as
// failed (persist_failed) instead of hanging.
#include <algorithm>
#include <new>
#include <vector>

#include "hip_common.h"
#include "qdev.h"
#include "attn_dev.h"
#include "persist.h"

namespace {

using eif::kPersistBarStride;
using eif::kPersistBarWords;

constexpr int kPT = 1024;          // threads per workgroup
constexpr int kLoadA = 14;         // loader wave of the QKV and gate|up tiles
constexpr int kLoadB = 15;         // loader wave of the O and down tiles
constexpr int kMW = 14;            // MFMA waves 0 .. kMW - 1
constexpr int kPrepMaxThreads = 64 * kMW;   // a prep's live columns must lie in the non-loader waves
constexpr int kAttnSubs = 1;       // attention items per workgroup, 512 threads each (waves 0-7)
constexpr int kAttnNT = 512;       // threads of an attention item (attn_split_kernel's)
constexpr int kBarGroups = 8;
constexpr long kSpinMax = 1L << 21;   // barrier polls before giving up (far beyond any stage's time)
constexpr int kLdsLane = 16;          // LDS bytes per lane of a weight step (12- and 16-byte loads alike)

enum { kQKV = 0, kO = 1, kGU = 2, kDN = 3 };

struct PLin {
    const uint8_t *W;        // GPU layout (qlinear.hip), rows padded
    const float *scales;     // [rows, G]
    int wld, G, nsteps, rows, tiles, kpad;
};

struct PLayer {
    PLin lin[4];
    const float *rms_att, *rms_ffn, *rms_sub_att, *rms_sub_ffn;
};

struct PArgs {
    const PLayer *layers;
    int n_layers, dim, hidden, q_dim, kv_dim, n_heads, n_kv, seq_len;
    float rms_eps, sub_eps, inv_sqrt_hd;
    const float *signs_dim, *signs_q, *signs_hidden;
    int blk_dim, blk_q, blk_hid;
    float norm_dim, norm_q, norm_hid;
    float *x, *qkv, *hb, *sh_o, *sh_ml;
    __half *kc, *vc;
    const float2 *rope;
    const int *state;
    const float *rms_final;
    int8_t *hq;
    float *hs;
    int head_kpad;
    int *bar, *err;
    // LDS (bytes from the dynamic base): the four weight regions, the staged int8 row, the group sums, the
    // attention items' LDS (over the row and sums: stages are apart)
    int reg_off[4], tile_bytes[4], codes_bytes[4];
    int x_off, acc_off, att_off, gld;
};

// The layer table is read through the constant address space: scalar loads (counted by lgkmcnt), so reading it
// never waits for a loader wave's outstanding weight loads (vmcnt), and its fields stay in scalar registers.
// (The host compilation pass, which only parses these device functions, has no constant address space.)
#if defined(__HIP_DEVICE_COMPILE__)
typedef const __attribute__((address_space(4))) PLayer *ConstLayers;
EIF_DEV PLin lin_at(const PArgs &a, int l, int k) { return ((ConstLayers)a.layers)[l].lin[k]; }
EIF_DEV PLayer layer_at(const PArgs &a, int l) { return ((ConstLayers)a.layers)[l]; }
#else
EIF_DEV PLin lin_at(const PArgs &a, int l, int k) { return a.layers[l].lin[k]; }
EIF_DEV PLayer layer_at(const PArgs &a, int l) { return a.layers[l]; }
#endif

// s_waitcnt vmcnt(n) for a wave-uniform n in 0..63 (the immediate must be a constant).
EIF_DEV void wait_vm(int n)
{
#define EIF_VM_CASE(k) \
    case k: __builtin_amdgcn_s_waitcnt(((k) & 15) | (((k) >> 4) << 14) | 0x70 | 0xF00); break;
#define EIF_VM_CASE8(b) EIF_VM_CASE(b) EIF_VM_CASE(b + 1) EIF_VM_CASE(b + 2) EIF_VM_CASE(b + 3) \
    EIF_VM_CASE(b + 4) EIF_VM_CASE(b + 5) EIF_VM_CASE(b + 6) EIF_VM_CASE(b + 7)
    switch (n) {
        EIF_VM_CASE8(0) EIF_VM_CASE8(8) EIF_VM_CASE8(16) EIF_VM_CASE8(24)
        EIF_VM_CASE8(32) EIF_VM_CASE8(40) EIF_VM_CASE8(48) EIF_VM_CASE8(56)
        default: __builtin_amdgcn_s_waitcnt(0); break;
    }
#undef EIF_VM_CASE8
#undef EIF_VM_CASE
}

// Tiles of a linear this workgroup owns (round-robin over the grid).
EIF_DEV int n_tiles(int tiles) { return tiles > (int)blockIdx.x ? (tiles - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0; }

// Loader wave: the workgroup's tiles of linear L into its LDS region. Per tile and step one load instruction of SB
// bytes per lane, laid out as the MFMA lanes read them (lane l: row l & 15, slot l >> 4) at kLdsLane bytes per lane
// (global_load_lds writes a lane's 12 bytes at a 16-byte lane stride too), then the tile's group scales [16][G] in
// 16-byte pieces. Returns the number of load instructions issued.
template <int SB>
EIF_DEV int issue_tiles(const PLin L, uint8_t *region, int tile_bytes, int codes_bytes, int tid)
{
    static_assert(SB == 16 || SB == 12, "global_load_lds moves 12 or 16 bytes per lane");
    const int lane = tid & 63, nt = n_tiles(L.tiles);
    int n = 0;
    for (int i = 0; i < nt; ++i) {
        const int tile = (int)blockIdx.x + i * (int)gridDim.x;
        uint8_t *dst = region + i * tile_bytes;
        const uint8_t *src = L.W + (size_t)(16 * tile + (lane & 15)) * L.wld + (lane >> 4) * SB;
        for (int st = 0; st < L.nsteps; ++st, ++n) {
            if constexpr (SB == 16) __builtin_amdgcn_global_load_lds(src + st * 64, dst + st * 64 * kLdsLane, 16, 0, 0);
            else __builtin_amdgcn_global_load_lds(src + st * 48, dst + st * 64 * kLdsLane, 12, 0, 0);
        }
        const int pieces = 4 * L.G;   // 16 rows x G floats = 4 G pieces of 16 bytes
        const uint8_t *ssrc = reinterpret_cast<const uint8_t *>(L.scales + (size_t)16 * tile * L.G);
        for (int p0 = 0; p0 < pieces; p0 += 64, ++n)
            if (p0 + lane < pieces)
                __builtin_amdgcn_global_load_lds(ssrc + 16 * (p0 + lane), dst + codes_bytes + 16 * p0, 16, 0, 0);
    }
    return n;
}

// Grid barrier idx (0, 1, ... within the launch). Compute waves first wait for their own coherent stores; between
// the two workgroup barriers the loader waves issue the next loads (issue()) into regions the stage has freed.
// Returns false when the step gives up (this or another workgroup exceeded the spin bound).
template <class Issue>
EIF_DEV bool grid_sync(const PArgs &a, int idx, bool loader, int &go_l, Issue &&issue)
{
    if (!loader) __builtin_amdgcn_s_waitcnt(0);
    wg_sync<1>();
    issue();
    if (threadIdx.x == 0) {
        const int G = gridDim.x, grp = blockIdx.x % kBarGroups;
        const int ng = G < kBarGroups ? G : kBarGroups;
        const int members = (G - grp + kBarGroups - 1) / kBarGroups;
        const int target = idx + 1;
        int *cnt = a.bar + kPersistBarStride * (1 + grp);
        const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == target * members - 1) {
            const int o2 = __hip_atomic_fetch_add(a.bar, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (o2 == target * ng - 1)
                for (int q = 0; q < ng; ++q) st_coh_i(a.bar + kPersistBarStride * (1 + kBarGroups + q), target);
        }
        const int *flag = a.bar + kPersistBarStride * (1 + kBarGroups + grp);
        long i = 0;
        int ok = 1;
        while (ld_coh_i(flag) < target) {
            if ((++i & 255) == 0 && ld_coh_i(a.err)) {
                ok = 0;
                break;
            }
            if (i > kSpinMax) {
                st_coh_i(a.err, 1);
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        go_l = ok;
    }
    wg_sync<1>();
    return go_l != 0;
}

// The MFMAs of the workgroup's tiles of one linear (waves 0 .. kMW - 1): (tile, step) pairs round-robin over the
// waves; per pair the two groups' exact int32 sums of the prepped row (token 0, lanes 0-15 hold the rows) go to
// acc_l [tile][row][gld] (the same decode and MFMA sequence as qgemv_kernel at M = 1).
template <int UD>
EIF_DEV void mfma_tiles(const PLin L, int nt, const uint8_t *region, int tile_bytes, const int8_t *lds_x,
                        int32_t *acc_l, int gld, int tid)
{
    using GE = Geo<kTern, UD>;
    constexpr int NW = GE::SB / 4;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, s = lane >> 4;
    const int npairs = nt * L.nsteps;
    for (int pr = wave; pr < npairs; pr += kMW) {
        const int tt = pr / L.nsteps, st = pr - tt * L.nsteps;
        const uint8_t *wb = region + tt * tile_bytes + (st * 64 + lane) * kLdsLane;
        uint32_t wq[NW];
        if constexpr (NW == 4) {
            const uint4 q4 = *reinterpret_cast<const uint4 *>(wb);
            wq[0] = q4.x, wq[1] = q4.y, wq[2] = q4.z, wq[3] = q4.w;
        } else {
#pragma unroll
            for (int i = 0; i < NW; ++i) wq[i] = reinterpret_cast<const uint32_t *>(wb)[i];
        }
        long bop[GE::NMF];
        decode<kTern, UD>(wq, bop);
        auto group = [&](auto grp_c) __attribute__((always_inline)) {
            constexpr int grp = decltype(grp_c)::value;
            long aop[UD];
            if (r16 == 0) {
                load_ops<UD, (UD % 2 == 0)>(lds_x + st * GE::SC + 32 * UD * grp + 8 * UD * s, aop);
            } else {
#pragma unroll
                for (int i = 0; i < UD; ++i) aop[i] = 0;
            }
            const v4i c = mfma_ops<grp * UD>(aop, bop, v4i{0, 0, 0, 0});
            const int gi = 2 * st + grp;
            if (gi < L.G && s == 0) acc_l[(tt * 16 + r16) * gld + gi] = c[0] >> GE::SHIFT;
        };
        group(std::integral_constant<int, 0>{});
        group(std::integral_constant<int, 1>{});
    }
}

// One row's group combine in group order (qgemv_kernel's step 5): t = fmaf((float)acc_g, s_g, t), y = t * xs.
EIF_DEV float combine_row(const int32_t *ap, const float *sp, int G, float xs)
{
    float t = 0.0f;
    int g = 0;
    for (; g + 4 <= G; g += 4) {
        const int4 a4 = *reinterpret_cast<const int4 *>(ap + g);
        t = fmaf((float)a4.x, sp[g], t);
        t = fmaf((float)a4.y, sp[g + 1], t);
        t = fmaf((float)a4.z, sp[g + 2], t);
        t = fmaf((float)a4.w, sp[g + 3], t);
    }
    for (; g < G; ++g) t = fmaf((float)ap[g], sp[g], t);
    return t * xs;
}

// Per-stage LDS scratch that is not a weight region.
struct PScratch {
    float xs_l[1];
    float red_max[16], red_ss[16];
};

// A linear stage LI of layer l: the prep of its input row into LDS (QKV: RMSNorm of x; O: the attention shares
// combined, then the sub-RMSNorm; gate|up: RMSNorm of x; down: SiLU(gate) * up of hb, then the sub-RMSNorm; each
// followed by the sign flip, the WHT and the absmax INT8), the MFMAs against the region's tiles and the combine;
// outputs coherent: QKV -> qkv, gate|up -> hb, O and down -> x += out. The caller's loader wave has waited for the
// region.
template <int LI, int UD, int E>
EIF_DEV void linear_stage(const PArgs &a, int l, uint8_t *smem, PScratch &ps, bool loader, int tid)
{
    const PLayer Ly = layer_at(a, l);
    const PLin &L = Ly.lin[LI];
    PrepArgs p{};
    float *y;
    if constexpr (LI == kQKV || LI == kGU) {
        p.x = a.x, p.ldx = a.dim, p.K = a.dim, p.signs = a.signs_dim, p.block = a.blk_dim, p.norm = a.norm_dim;
        p.pre = EIF_HIP_PRE_RMS, p.nw = LI == kQKV ? Ly.rms_att : Ly.rms_ffn, p.eps = a.rms_eps;
        y = LI == kQKV ? a.qkv : a.hb;
    } else if constexpr (LI == kO) {
        p.x = a.sh_o, p.ldx = a.q_dim, p.K = a.q_dim, p.signs = a.signs_q, p.block = a.blk_q, p.norm = a.norm_q;
        p.pre = EIF_HIP_PRE_RMS, p.nw = Ly.rms_sub_att, p.eps = a.sub_eps;
        p.sh_o = a.sh_o, p.sh_ml = a.sh_ml, p.sh_hd = a.q_dim / a.n_heads;
        y = a.x;
    } else {
        p.x = a.hb, p.x2 = a.hb + a.hidden, p.ldx = a.hidden, p.K = a.hidden, p.signs = a.signs_hidden;
        p.block = a.blk_hid, p.norm = a.norm_hid;
        p.pre = EIF_HIP_PRE_SWIGLU_RMS, p.nw = Ly.rms_sub_ffn, p.eps = a.sub_eps;
        y = a.x;
    }
    const int nt = n_tiles(L.tiles);
    int8_t *lds_x = reinterpret_cast<int8_t *>(smem + a.x_off);
    int32_t *acc_l = reinterpret_cast<int32_t *>(smem + a.acc_off);
    const uint8_t *region = smem + a.reg_off[LI];
    float v[E], sg[E], v2[E], nwv[E];
    if (loader) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = sg[e] = v2[e] = nwv[e] = 0.0f;
    } else if constexpr (LI == kO) {
        Shares<E> shv;
        prep_load_sh<E, true>(p, shv, sg, nwv, tid);
        sh_combine<E>(shv, v);
#pragma unroll
        for (int e = 0; e < E; ++e) v2[e] = 0.0f;
    } else {
        prep_load<E, true>(p, 0, v, sg, v2, nwv, tid);
    }
    prep_finish<E, -1, 1>(p, 0, L.kpad, v, sg, v2, nwv, lds_x, ps.xs_l, ps.red_max, ps.red_ss, tid);
    if (__builtin_amdgcn_readfirstlane(tid >> 6) < kMW) mfma_tiles<UD>(L, nt, region, a.tile_bytes[LI], lds_x, acc_l, a.gld, tid);
    wg_sync<1>();
    const int j = tid;
    if (j < 16 * nt) {
        const int tt = j >> 4, r = j & 15;
        const int orow = 16 * ((int)blockIdx.x + tt * (int)gridDim.x) + r;
        if (orow < L.rows) {
            const float *sp = reinterpret_cast<const float *>(region + tt * a.tile_bytes[LI] + a.codes_bytes[LI]) + r * L.G;
            float out = combine_row(acc_l + (tt * 16 + r) * a.gld, sp, L.G, ps.xs_l[0]);
            if constexpr (LI == kO || LI == kDN) out = out + ld_coh(y + orow);
            st_coh(y + orow, out);
        }
    }
}

// The head's input after the last layer: RMSNorm + INT8 of x (no rotation) into hq / hs, as the decoder's separate
// prep launch (prep_spec_kernel, E columns per thread) makes it.
template <int E>
EIF_DEV void head_prep(const PArgs &a, PScratch &ps, bool loader, int tid)
{
    PrepArgs p{};
    p.x = a.x, p.ldx = a.dim, p.K = a.dim, p.block = 0, p.norm = 1.0f, p.ldl = a.head_kpad;
    p.pre = EIF_HIP_PRE_RMS, p.nw = a.rms_final, p.eps = a.rms_eps;
    float v[E], sg[E], v2[E], nwv[E];
    if (loader) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = sg[e] = v2[e] = nwv[e] = 0.0f;
    } else {
        prep_load<E, true>(p, 0, v, sg, v2, nwv, tid);
    }
    prep_finish<E, 0, 1>(p, 0, a.head_kpad, v, sg, v2, nwv, a.hq, a.hs, ps.red_max, ps.red_ss, tid);
}

// The attention items' LDS: the query and the new key / value row, and attend()'s own.
template <int HD>
struct PAttn {
    float q_l[HD], k_l[HD], v_l[HD];
    AttnLds<HD, kAttnNT> att;
};

template <int HD>
constexpr int attn_unit() { return 2048 / (HD / 8); }

// S2: items (h, chunk) = kAttnSubs b + sub for sub < kAttnSubs (threads kAttnNT sub .. kAttnNT (sub + 1) - 1); the
// decode attention of attn_split_kernel (decode.hip) on each: RoPE of q (and of k in the chunk holding pos), fp16
// KV append by the kv head's first query head, attention over the chunk, the chunk's share. The other non-loader
// waves take part in the items' barriers without work.
template <int HD>
EIF_DEV void attn_stage(const PArgs &a, int l, int pos, uint8_t *smem, int tid)
{
    constexpr int HALF = HD / 2, UNIT = attn_unit<HD>();
    const int sub = __builtin_amdgcn_readfirstlane(tid / kAttnNT), t = tid % kAttnNT;
    const int it = kAttnSubs * (int)blockIdx.x + sub;
    const bool valid = sub < kAttnSubs && it < a.n_heads * kAttnShares;
    const int h = valid ? it / kAttnShares : 0, sc = valid ? it % kAttnShares : 0;
    const int kv_mul = a.n_heads / a.n_kv, g = h / kv_mul;
    const int ch = UNIT * ((pos + UNIT * kAttnShares) / (UNIT * kAttnShares));
    const int c0 = sc * ch;
    float *ml = a.sh_ml + (size_t)h * 2 * kAttnShares + sc;
    const bool live = valid && c0 <= pos;
    if (valid && !live && t == 0) st_coh(ml, -INFINITY);
    const bool last = pos < c0 + ch;
    PAttn<HD> &S = reinterpret_cast<PAttn<HD> *>(smem + a.att_off)[sub < kAttnSubs ? sub : 0];
    const size_t cache_l = (size_t)l * a.n_kv * a.seq_len * HD;
    auto rotate = [&]() {
        if (live && t < HALF) {
            const float2 cs = a.rope[(size_t)pos * HALF + t];
            const float c = cs.x, sn = cs.y;
            const float *qh = a.qkv + h * HD;
            const float qa = ld_coh(qh + t), qb = ld_coh(qh + t + HALF);
            S.q_l[t] = qa * c - qb * sn;
            S.q_l[t + HALF] = qb * c + qa * sn;
            if (last) {
                const float *kh = a.qkv + a.q_dim + g * HD, *vh = a.qkv + a.q_dim + a.kv_dim + g * HD;
                const float ka = ld_coh(kh + t), kb = ld_coh(kh + t + HALF);
                const __half k0 = __float2half(ka * c - kb * sn), k1 = __float2half(kb * c + ka * sn);
                const __half v0 = __float2half(ld_coh(vh + t)), v1 = __float2half(ld_coh(vh + t + HALF));
                S.k_l[t] = __half2float(k0), S.k_l[t + HALF] = __half2float(k1);
                S.v_l[t] = __half2float(v0), S.v_l[t + HALF] = __half2float(v1);
                if (h % kv_mul == 0) {
                    __half *kw = a.kc + cache_l + ((size_t)g * a.seq_len + pos) * HD;
                    __half *vw = a.vc + cache_l + ((size_t)g * a.seq_len + pos) * HD;
                    kw[t] = k0, kw[t + HALF] = k1;
                    vw[t] = v0, vw[t + HALF] = v1;
                }
            }
        }
        wg_sync<1>();
    };
    const size_t base = cache_l + ((size_t)g * a.seq_len + c0) * HD;
    const int rows = (last ? pos : c0 + ch) - c0;
    attend<HD, kAttnNT, 1, true>(S.att, t, live, S.q_l, a.kc + base, a.vc + base, rows, last ? S.k_l : nullptr,
                             last ? S.v_l : nullptr, a.inv_sqrt_hd, a.sh_o + ((size_t)h * kAttnShares + sc) * HD, ml,
                             rotate);
}

template <int HD, int UDI, int UDD, int EI, int EH>
__global__ __launch_bounds__(kPT) void persist_step_kernel(PArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ PScratch ps;
    __shared__ int go_l;
    constexpr int SBI = Geo<kTern, UDI>::SB, SBD = Geo<kTern, UDD>::SB;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar branches by role
    const bool loader = wave >= kLoadA, la = wave == kLoadA, lb = wave == kLoadB;
    const int pos = a.state[0];
    const int L = a.n_layers;
    // load instructions this workgroup's loaders issue per region (issue_tiles; the same for every layer)
    int n_load[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const PLin lin = lin_at(a, 0, k);
        n_load[k] = n_tiles(lin.tiles) * (lin.nsteps + (4 * lin.G + 63) / 64);
    }
    // the thread index passed through an empty asm at each use: what a stage derives from it is computed in the
    // stage, not hoisted out of the layer loop into registers held across all stages
    auto fresh_tid = []() {
        int t = threadIdx.x;
        asm volatile("" : "+v"(t));
        return t;
    };
    auto issue = [&](int li, int layer) {
        const PLin lin = lin_at(a, layer, li);
        uint8_t *reg = smem + a.reg_off[li];
        return li == kDN ? issue_tiles<SBD>(lin, reg, a.tile_bytes[li], a.codes_bytes[li], fresh_tid())
                         : issue_tiles<SBI>(lin, reg, a.tile_bytes[li], a.codes_bytes[li], fresh_tid());
    };
    // layer 0's tiles, in the order the waits below assume: A: QKV, gate|up; B: O, down
    if (la) issue(kQKV, 0), issue(kGU, 0);
    if (lb) issue(kO, 0), issue(kDN, 0);
    int bi = 0;
    for (int l = 0; l < L; ++l) {
        int tiles[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) tiles[k] = lin_at(a, l, k).tiles;
        const bool more = l + 1 < L;
        // S1: x -> RMSNorm -> WHT -> INT8 -> QKV
        if (n_tiles(tiles[kQKV]) > 0) {
            if (la) wait_vm(n_load[kGU]);   // QKV(l); gate|up(l) issued after it
            linear_stage<kQKV, UDI, EI>(a, l, smem, ps, loader, fresh_tid());
        }
        if (!grid_sync(a, bi++, loader, go_l, [&] { if (la && more) issue(kQKV, l + 1); })) return;
        // S2: attention
        if (kAttnSubs * (int)blockIdx.x < a.n_heads * kAttnShares) {
            // pos passed through an empty asm per layer: what the attention derives from it is computed here, not
            // hoisted out of the layer loop into registers held across every stage
            int pos_l = pos;
            asm volatile("" : "+s"(pos_l));
            if (!loader) attn_stage<HD>(a, l, pos_l, smem, fresh_tid());
            else wg_sync<1>(), wg_sync<1>(), wg_sync<1>();   // the items' three workgroup barriers
        }
        if (!grid_sync(a, bi++, loader, go_l, [] {})) return;
        // S3: shares -> combine -> sub-RMSNorm -> WHT -> INT8 -> O, x += out
        if (n_tiles(tiles[kO]) > 0) {
            if (lb) wait_vm(n_load[kDN]);   // O(l); down(l) issued after it
            linear_stage<kO, UDI, EI>(a, l, smem, ps, loader, fresh_tid());
        }
        if (!grid_sync(a, bi++, loader, go_l, [&] { if (lb && more) issue(kO, l + 1); })) return;
        // S4: x -> RMSNorm -> WHT -> INT8 -> gate|up
        if (n_tiles(tiles[kGU]) > 0) {
            if (la) wait_vm(more ? n_load[kQKV] : 0);   // gate|up(l); QKV(l + 1) issued after it
            linear_stage<kGU, UDI, EI>(a, l, smem, ps, loader, fresh_tid());
        }
        if (!grid_sync(a, bi++, loader, go_l, [&] { if (la && more) issue(kGU, l + 1); })) return;
        // S5: SiLU(gate) * up -> sub-RMSNorm -> WHT -> INT8 -> down, x += out
        if (n_tiles(tiles[kDN]) > 0) {
            if (lb) wait_vm(more ? n_load[kO] : 0);   // down(l); O(l + 1) issued after it
            linear_stage<kDN, UDD, EH>(a, l, smem, ps, loader, fresh_tid());
        }
        if (!grid_sync(a, bi++, loader, go_l, [&] { if (lb && more) issue(kDN, l + 1); })) return;
    }
    if (blockIdx.x == 0) head_prep<EI>(a, ps, loader, fresh_tid());
}

typedef void (*PKernel)(PArgs);

// The instantiated configurations: head_dim 128 with g128 input matrices and a g96 or g128 down projection, the
// down projection's prep at 4 or 8 columns per thread (hidden up to 3584 or 7168).
template <int HD, int UDI, int UDD, int EI, int EH>
PKernel kernel_of() { return persist_step_kernel<HD, UDI, UDD, EI, EH>; }

PKernel pick_kernel(int hd, int udi, int udd, int ei, int eh)
{
    if (hd != 128 || udi != 4 || ei != 4) return nullptr;
    if (udd == 3 && eh == 8) return kernel_of<128, 4, 3, 4, 8>();
    if (udd == 3 && eh == 4) return kernel_of<128, 4, 3, 4, 4>();
    if (udd == 4 && eh == 8) return kernel_of<128, 4, 4, 4, 8>();
    if (udd == 4 && eh == 4) return kernel_of<128, 4, 4, 4, 4>();
    return nullptr;
}

// Columns per thread of the separate launch's fused prep for a row of kpad columns: the fewest of 4, 8, 16 whose
// 16 waves cover it (launch_gemv_tiles); the persistent step needs those columns within waves 0-13.
int prep_cols(int kpad)
{
    for (int e = 4; e <= 16; e *= 2)
        if (64 * 16 * e >= kpad) return e;
    return 0;
}

}  // namespace

namespace eif {

struct PersistPlan {
    PArgs args{};
    PLayer *layers = nullptr;   // device
    int *bar = nullptr;         // barrier words + give-up flag (device)
    PKernel kernel = nullptr;
    int grid = 0;
    size_t lds = 0;
};

int persist_create(PersistPlan **out, const PersistModel &pm)
{
    *out = nullptr;
    if (pm.head_dim != 128 || pm.n_heads % pm.n_kv || pm.seq_len > 4096) return EIF_HIP_E_LIMIT;
    std::vector<PLayer> host(pm.n_layers);
    int udi = -1, udd = -1;
    int tiles_max[4] = {0, 0, 0, 0};
    int geo[4][4];   // per linear kind: G, nsteps, wld, kpad (equal over layers)
    for (int l = 0; l < pm.n_layers; ++l) {
        const eif_hip_qweight *ws[4] = {pm.wqkv[l], pm.wo[l], pm.w13[l], pm.w2[l]};
        for (int k = 0; k < 4; ++k) {
            QView v;
            if (!ws[k] || qweight_view(ws[k], &v) || v.fmt != EIF_HIP_W_TERNARY || v.group <= 0 || !v.scales ||
                v.rows % 16 != 0)
                return EIF_HIP_E_LIMIT;
            if (k == kDN) {
                if (udd >= 0 && v.ud != udd) return EIF_HIP_E_LIMIT;
                udd = v.ud;
            } else {
                if (udi >= 0 && v.ud != udi) return EIF_HIP_E_LIMIT;
                udi = v.ud;
            }
            if (l == 0) {
                geo[k][0] = v.G, geo[k][1] = v.nsteps, geo[k][2] = v.wld, geo[k][3] = v.kpad;
            } else if (geo[k][0] != v.G || geo[k][1] != v.nsteps || geo[k][2] != v.wld || geo[k][3] != v.kpad) {
                return EIF_HIP_E_LIMIT;
            }
            PLin &pl = host[l].lin[k];
            pl.W = v.W, pl.scales = v.scales, pl.wld = v.wld, pl.G = v.G, pl.nsteps = v.nsteps, pl.rows = v.rows;
            pl.tiles = v.rows / 16, pl.kpad = v.kpad;
            tiles_max[k] = std::max(tiles_max[k], pl.tiles);
        }
        host[l].rms_att = pm.rms_att[l], host[l].rms_ffn = pm.rms_ffn[l];
        host[l].rms_sub_att = pm.rms_sub_att[l], host[l].rms_sub_ffn = pm.rms_sub_ffn[l];
    }
    // every prep's columns in waves 0-13 (same columns per thread as the separate launch)
    const int ei = prep_cols(geo[kQKV][3]), eq = prep_cols(geo[kO][3]), eh = prep_cols(geo[kDN][3]);
    if (ei != 4 || eq != 4 || prep_cols(geo[kGU][3]) != 4 || prep_cols(pm.head_kpad) != 4 || !eh) return EIF_HIP_E_LIMIT;
    if (eif_ceil_div(geo[kQKV][3], ei) > kPrepMaxThreads || eif_ceil_div(geo[kO][3], eq) > kPrepMaxThreads ||
        eif_ceil_div(geo[kGU][3], ei) > kPrepMaxThreads || eif_ceil_div(geo[kDN][3], eh) > kPrepMaxThreads ||
        eif_ceil_div(pm.head_kpad, 4) > kPrepMaxThreads)
        return EIF_HIP_E_LIMIT;
    const PKernel kern = pick_kernel(pm.head_dim, udi, udd, ei, eh);
    if (!kern) return EIF_HIP_E_LIMIT;

    int dev = 0, cus = 0, max_lds = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || cus <= 0)
        return EIF_HIP_E_DEVICE;
    const int G = cus;
    if (pm.n_heads * kAttnShares > kAttnSubs * G) return EIF_HIP_E_LIMIT;   // one round of attention items
    PArgs a{};
    int off = 0;
    int n_load[4];
    for (int k = 0; k < 4; ++k) {
        const int nt = eif_ceil_div(tiles_max[k], G);   // tiles per workgroup at most
        a.codes_bytes[k] = geo[k][1] * 64 * kLdsLane;   // nsteps x 64 lanes x 16 bytes
        a.tile_bytes[k] = a.codes_bytes[k] + 16 * geo[k][0] * 4;
        a.reg_off[k] = off;
        off += nt * a.tile_bytes[k];
        // load instructions of the most loaded workgroup's loader for this region
        n_load[k] = nt * (geo[k][1] + eif_ceil_div(4 * geo[k][0], 64));
    }
    // a loader's outstanding loads (its two regions) must stay within what vmcnt counts
    if (n_load[kQKV] + n_load[kGU] > 63 || n_load[kO] + n_load[kDN] > 63) return EIF_HIP_E_LIMIT;
    off = eif_round_up(off, 16);
    const int kmax = std::max(std::max(geo[kQKV][3], geo[kO][3]), std::max(geo[kDN][3], pm.head_kpad));
    int gmax = 0, acc_tiles = 0;
    for (int k = 0; k < 4; ++k) {
        gmax = std::max(gmax, geo[k][0]);
        acc_tiles = std::max(acc_tiles, eif_ceil_div(tiles_max[k], G));
    }
    a.gld = (gmax + 3) & ~3;
    a.x_off = off;
    a.acc_off = eif_round_up(a.x_off + kmax + 16, 16);
    const int scratch_end = a.acc_off + acc_tiles * 16 * a.gld * 4;
    a.att_off = off;   // the attention items' LDS overlays the row and the sums (other stages)
    const int att_end = a.att_off + kAttnSubs * (int)sizeof(PAttn<128>);
    const int lds = eif_round_up(std::max(scratch_end, att_end), 16);
    if (lds + (int)sizeof(PScratch) + 64 > max_lds) return EIF_HIP_E_LIMIT;

    PersistPlan *p = new (std::nothrow) PersistPlan;
    if (!p) return EIF_HIP_E_NOMEM;
    const size_t bar_ints = (size_t)kPersistBarStride * kPersistBarWords + 64;
    if (hipMalloc(&p->layers, sizeof(PLayer) * pm.n_layers) != hipSuccess ||
        hipMalloc(&p->bar, sizeof(int) * bar_ints) != hipSuccess ||
        hipMemcpy(p->layers, host.data(), sizeof(PLayer) * pm.n_layers, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(p->bar, 0, sizeof(int) * bar_ints) != hipSuccess ||
        hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess) {
        persist_destroy(p);
        return EIF_HIP_E_DEVICE;
    }
    // the grid barriers need every workgroup resident at once: one 1024-thread workgroup with this LDS must fit
    // on a CU (what other streams hold at run time is caught by the barriers' bounded spin instead)
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kPT, (size_t)lds) != hipSuccess) {
        persist_destroy(p);
        return EIF_HIP_E_DEVICE;
    }
    if (per_cu < 1) {
        persist_destroy(p);
        return EIF_HIP_E_LIMIT;
    }
    a.layers = p->layers;
    a.n_layers = pm.n_layers, a.dim = pm.dim, a.hidden = pm.hidden, a.q_dim = pm.q_dim, a.kv_dim = pm.kv_dim;
    a.n_heads = pm.n_heads, a.n_kv = pm.n_kv, a.seq_len = pm.seq_len;
    a.rms_eps = pm.rms_eps, a.sub_eps = pm.sub_eps, a.inv_sqrt_hd = 1.0f / sqrtf((float)pm.head_dim);
    a.signs_dim = pm.signs_dim, a.signs_q = pm.signs_q, a.signs_hidden = pm.signs_hidden;
    a.blk_dim = pm.wht_dim, a.blk_q = pm.wht_q, a.blk_hid = pm.wht_hidden;
    a.norm_dim = pm.norm_dim, a.norm_q = pm.norm_q, a.norm_hid = pm.norm_hidden;
    a.x = pm.x, a.qkv = pm.qkv, a.hb = pm.hb, a.sh_o = pm.sh_o, a.sh_ml = pm.sh_ml;
    a.kc = pm.kc, a.vc = pm.vc, a.rope = pm.rope, a.state = pm.state;
    a.rms_final = pm.rms_final, a.hq = pm.hq, a.hs = pm.hs, a.head_kpad = pm.head_kpad;
    a.bar = p->bar;
    a.err = p->bar + (size_t)kPersistBarStride * kPersistBarWords;
    p->args = a;
    p->kernel = kern;
    p->grid = G;
    p->lds = (size_t)lds;
    *out = p;
    return EIF_HIP_OK;
}

void persist_destroy(PersistPlan *p)
{
    if (!p) return;
    if (p->layers) (void)hipFree(p->layers);
    if (p->bar) (void)hipFree(p->bar);
    delete p;
}

int persist_enqueue(PersistPlan *p, hipStream_t st)
{
    if (!p) return EIF_HIP_E_ARG;
    hipLaunchKernelGGL(p->kernel, dim3(p->grid), dim3(kPT), p->lds, st, p->args);
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

int *persist_bar(PersistPlan *p) { return p ? p->bar : nullptr; }

int persist_reset(PersistPlan *p, hipStream_t st)
{
    if (!p) return EIF_HIP_OK;
    const size_t bar_ints = (size_t)kPersistBarStride * kPersistBarWords + 64;
    EIF_HIP_TRY(hipMemsetAsync(p->bar, 0, sizeof(int) * bar_ints, st));
    return EIF_HIP_OK;
}

int persist_failed(PersistPlan *p, hipStream_t st)
{
    if (!p) return 0;
    int e = 0;
    if (hipMemcpyAsync(&e, p->args.err, sizeof(int), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return 1;
    return e != 0;
}

}  // namespace eif

// attn_dev.h -- the decode attention of one query head over one chunk of cached positions, shared by the
// standalone decode kernel (decode.hip attn_split_kernel) and the persistent decode step (persist.hip), which
// therefore compute the same bits.
#pragma once

#include <hip/hip_fp16.h>

#include "qdev.h"

namespace {

// 8 consecutive fp16 values -> float.
EIF_DEV void half8_to_float(const uint4 &raw, float (&f)[8])
{
    const __half2 *hp = reinterpret_cast<const __half2 *>(&raw);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float2 v = __half22float2(hp[i]);
        f[2 * i] = v.x, f[2 * i + 1] = v.y;
    }
}

// The LDS of one attend() call: per row group its maximum, sum and value sums, and the combine's partial sums.
template <int HD, int NT>
struct AttnLds {
    static constexpr int DPR = HD / 8, RG = NT / DPR, PARTS = NT / HD;
    __align__(16) float m_l[RG];
    float l_l[RG];
    float o_l[RG][HD + 4];
    float po_l[PARTS][HD], pl_l[PARTS];
};

// Softmax attention of one query (q_l, HD floats in LDS) over cache rows 0 .. n_cache - 1 (fp16 [HD] rows at
// kcg / vcg) and, when k_x is not NULL, one more row (k_x, v_x in LDS) after them, as a share of the query's
// attention (below). NT threads, t = 0 .. NT - 1 this thread's index among them; L the call's LDS. A thread holds
// 8 of the HD dimensions of a key / value row: DPR = HD / 8 threads per row and RG row groups; row group r takes
// rows r, r + RG, r + 2 RG, ... in batches of UNR = 2048 / NT rows whose keys and values are loaded together
// (a batch covers 2048 / DPR rows whatever NT: more threads hold fewer rows each), and keeps a
// running softmax over them (max m, sum l, the weighted value sums o of its dims):
//   s_t = (q . k_t) / sqrt(HD), m' = max(m, s_t), l = l e^(m - m') + sum e^(s_t - m'),
//   o = o e^(m - m') + sum e^(s_t - m') v_t;
// the row groups are then combined, M = max_r m_r: out[0 .. HD) = sum_r e^(m_r - M) o_r unnormalized,
// out_ml[0] = M, out_ml[kAttnShares] = sum_r e^(m_r - M) l_r (a chunk's share, combined by the next linear's prep
// into out / l: the softmax of the scores followed by the weighted sum of the values, the sums in another order).
// pro(): called once the first batch's loads are issued, before q_l is read (the caller fills q_l, k_x and v_x
// there and synchronizes the workgroup), so those loads overlap the caller's set-up.
// live = false: the call does no work and touches no memory, but takes part in the workgroup barriers (policy
// BAR, see qdev.h) like a live call, so that calls of other thread groups of the workgroup can run beside it.
// COH: the share is written with device-coherent stores.
template <int HD, int NT, int BAR = 0, bool COH = false, class Pro>
EIF_DEV void attend(AttnLds<HD, NT> &L, int t, bool live, const float *q_l, const __half *kcg, const __half *vcg,
                    int n_cache, const float *k_x, const float *v_x, float inv_sqrt_hd, float *out, float *out_ml,
                    Pro &&pro)
{
    using A = AttnLds<HD, NT>;
    constexpr int DPR = A::DPR, RG = A::RG, UNR = 2048 / NT, PARTS = A::PARTS;
    static_assert(UNR >= 1 && RG * UNR == 2048 / DPR, "a batch of 2048 / DPR rows");
    const int sub = t % DPR, r0 = t / DPR;
    uint4 kr[UNR], vr[UNR];
    auto load_batch = [&](int base) {
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int tt = base + u * RG + r0;
            const size_t off = (size_t)(tt < n_cache ? tt : 0) * HD + 8 * sub;
            kr[u] = *reinterpret_cast<const uint4 *>(kcg + off);
            vr[u] = *reinterpret_cast<const uint4 *>(vcg + off);
        }
    };
    if (live) load_batch(0);
    pro();
    float qv[8], o[8];
    float m = -INFINITY, l = 0.0f;
    if (live) {
#pragma unroll
        for (int i = 0; i < 8; ++i) qv[i] = q_l[8 * sub + i], o[i] = 0.0f;
        auto score = [&](const float (&k8)[8]) {
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) d = fmaf(qv[i], k8[i], d);
            // the row's DPR lanes summed by DPP butterflies (lane exchanges inside 16-lane rows; DPR <= 16)
            static_assert(DPR <= 16, "a key row within one 16-lane row");
            if constexpr (DPR > 1) d += xlane<1>(d);
            if constexpr (DPR > 2) d += xlane<2>(d);
            if constexpr (DPR > 4) d += xlane<4>(d);
            if constexpr (DPR > 8) d += xlane<8>(d);
            return d * inv_sqrt_hd;
        };
        for (int base = 0; base < n_cache; base += RG * UNR) {
            if (base > 0) load_batch(base);
            float sv[UNR];
            float bm = -INFINITY;
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
                float k8[8];
                half8_to_float(kr[u], k8);
                const float d = score(k8);
                sv[u] = base + u * RG + r0 < n_cache ? d : -INFINITY;
                bm = fmaxf(bm, sv[u]);
            }
            const float mn = fmaxf(m, bm);
            if (mn != -INFINITY) {   // the row group has rows in this batch or before
                const float sc = expf(m - mn);
                l = l * sc;
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = o[i] * sc;
#pragma unroll
                for (int u = 0; u < UNR; ++u) {
                    const float pw = expf(sv[u] - mn);
                    const bool ok = base + u * RG + r0 < n_cache;   // a row past the end holds a stand-in row
                    float v8[8];
                    half8_to_float(vr[u], v8);
                    l = l + pw;
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = fmaf(pw, ok ? v8[i] : 0.0f, o[i]);
                }
                m = mn;
            }
        }
        if (k_x) {   // uniform
            float k8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) k8[i] = k_x[8 * sub + i];
            const float d = score(k8);   // every row group computes it (uniform shuffles); row group 0 keeps it
            if (r0 == 0) {
                const float mn = fmaxf(m, d);
                const float sc = expf(m - mn), pw = expf(d - mn);
                l = l * sc + pw;
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = fmaf(pw, v_x[8 * sub + i], o[i] * sc);
                m = mn;
            }
        }

        // combine the row groups
        if (sub == 0) L.m_l[r0] = m, L.l_l[r0] = l;
#pragma unroll
        for (int i = 0; i < 8; ++i) L.o_l[r0][8 * sub + i] = o[i];
    }
    wg_sync<BAR>();
    if (live) {
        float mx = -INFINITY;
#pragma unroll 4
        for (int r = 0; r < RG; r += 4) {
            const float4 m4 = *reinterpret_cast<const float4 *>(&L.m_l[r]);
            mx = fmaxf(mx, fmaxf(fmaxf(m4.x, m4.y), fmaxf(m4.z, m4.w)));
        }
        const int d = t % HD, part = t / HD;
        float os = 0.0f, ls = 0.0f;
        for (int r = part; r < RG; r += PARTS) {
            const float w = expf(L.m_l[r] - mx);   // 0 for a row group without rows
            os = fmaf(w, L.o_l[r][d], os);
            ls = fmaf(w, L.l_l[r], ls);
        }
        L.po_l[part][d] = os;
        if (d == 0) L.pl_l[part] = ls;
        if (t < HD) m = mx;
    }
    wg_sync<BAR>();
    if (live && t < HD) {
        float os = L.po_l[0][t], ls = L.pl_l[0];
#pragma unroll
        for (int q = 1; q < PARTS; ++q) os += L.po_l[q][t], ls += L.pl_l[q];
        if constexpr (COH) {
            st_coh(out + t, os);
            if (t == 0) st_coh(out_ml, m), st_coh(out_ml + kAttnShares, ls);
        } else {
            out[t] = os;
            if (t == 0) out_ml[0] = m, out_ml[kAttnShares] = ls;
        }
    }
}

}  // namespace

// qwen35_file.cpp -- QWN5 model images (include/eif_hip_qwen35.h) into resident GPU weights.
//
// eif_qwen35_parse restates the layout walk of the reference's qwen35_load (src/eif_qwen35.c:1223-1430): header
// and config checks (:1250-1307), the weights region in the order embedding, DeltaNet qkv / z / out / proj_b /
// proj_a, attention q(+gate) / k / v / o, FFN gate / up / down for 24 layer slots, then the DeltaNet conv, dt_bias
// and A_log arrays (:1321-1343); the per-layer assignment (:1346-1372); the scales region (:1374-1394) with its
// grouped counts (scale_count :103-106, small_qtype :108); the norms region (:1396-1430), whose SubLN vectors are
// present when they fit in norms_size. Row sizes: row_bytes / embed_row_bytes (:110-125).
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <new>
#include <memory>
#include <vector>

#include <hip/hip_runtime.h>

#include "../../include/eif_hip.h"
#include "../../include/eif_hip_qwen35.h"

namespace {

constexpr uint32_t kMagic = 0x51574E35u, kVersion = 1u;
enum { kEmbInt8 = 0, kEmbInt4 = 1, kEmb2bit = 2, kEmbDense = 3, kEmbFp32 = 4 };
// config block words (qwen35_config_t, include/eif_qwen35.h:56-110)
enum {
    cDim = 0, cHidden, cLayers, cHeads, cKv, cHeadDim, cVocab, cSeq, cDelta, cFull, cLinK, cLinKd, cLinV, cLinVd,
    cConvK, cLmTied = 22, cQuantLm = 23, cQuantEmbed = 25, cPlain = 26, cGroup = 27, cHadamard = 28
};

size_t row_bytes(int cols, int qt)
{
    if (qt == EIF_Q35_TERN3) return (size_t)(cols + 4) / 5;
    if (qt == EIF_Q35_INT4) return (size_t)(cols + 1) / 2;
    if (qt == EIF_Q35_FP32) return (size_t)cols * 4;
    return (size_t)(cols + 3) / 4;
}

size_t embed_row_bytes(int cols, int eq)
{
    if (eq == kEmbInt8) return (size_t)cols;
    if (eq == kEmbInt4) return (size_t)(cols + 1) / 2;
    if (eq == kEmb2bit) return (size_t)(cols + 3) / 4;
    if (eq == kEmbDense) return (size_t)(cols + 4) / 5;
    return (size_t)cols * 4;
}

// A region walk: each take() hands out the next n bytes, failing (ok = false) past the file's end.
struct Walk {
    size_t off, limit;
    bool ok = true;
    size_t take(size_t n)
    {
        if (!ok || off > limit || n > limit - off) {
            ok = false;
            return 0;
        }
        const size_t o = off;
        off += n;
        return o;
    }
};

eif_qwen35_tensor tensor(size_t codes, int rows, int cols, int qtype, int group)
{
    eif_qwen35_tensor t{};
    t.codes = codes, t.rows = rows, t.cols = cols, t.qtype = qtype, t.group = qtype == EIF_Q35_TERN2 ? group : 0;
    return t;
}

}  // namespace

extern "C" int eif_qwen35_parse(const void *image, size_t bytes, eif_qwen35_layout *out)
{
    if (!image || !out || bytes < 48) return EIF_HIP_E_ARG;
    *out = eif_qwen35_layout{};
    const uint8_t *base = static_cast<const uint8_t *>(image);
    uint32_t hdr[12];
    std::memcpy(hdr, base, sizeof(hdr));
    if (hdr[0] != kMagic || hdr[1] != kVersion) return EIF_HIP_E_ARG;
    const size_t cfg_off = hdr[2], w_off = hdr[3], s_off = hdr[4], n_off = hdr[5], n_size = hdr[9];
    if (cfg_off + 128 > bytes) return EIF_HIP_E_ARG;
    int32_t *c = out->config;
    std::memcpy(c, base + cfg_off, 128);
    const int n_layers = c[cLayers];
    if (n_layers <= 0 || n_layers > 24 || cfg_off + 128 + (size_t)n_layers > bytes || w_off > bytes ||
        s_off > bytes || n_off > bytes || n_off + n_size > bytes)
        return EIF_HIP_E_ARG;
    std::memcpy(out->layer_types, base + cfg_off + 128, (size_t)n_layers);
    out->n_layers = n_layers;

    const int dim = c[cDim], hidden = c[cHidden], nh = c[cHeads], nkv = c[cKv], hd = c[cHeadDim];
    const int vocab = c[cVocab], n_dn = c[cDelta], n_fa = c[cFull];
    const int nk = c[cLinK], kd = c[cLinKd], nv = c[cLinV], vd = c[cLinVd], ck = c[cConvK];
    const int qlm = c[cQuantLm], qemb = c[cQuantEmbed], g = c[cGroup], had = c[cHadamard];
    if (dim <= 0 || vocab <= 0 || hidden <= 0 || nh <= 0 || hd <= 0 || nkv <= 0 || n_dn < 0 || n_dn > 18 ||
        n_fa < 0 || n_fa > 6 || n_dn + n_fa != n_layers || nk <= 0 || nv <= 0 || kd <= 0 || vd <= 0 ||
        c[cSeq] <= 0 || ck <= 0 || qlm < EIF_Q35_FP32 || qlm > EIF_Q35_TERN3 || qemb < kEmbInt8 || qemb > kEmbFp32)
        return EIF_HIP_E_ARG;
    int seen_dn = 0, seen_fa = 0;
    for (int l = 0; l < n_layers; ++l) {
        if (out->layer_types[l] > 1) return EIF_HIP_E_ARG;
        (out->layer_types[l] ? seen_fa : seen_dn)++;
    }
    if (seen_dn != n_dn || seen_fa != n_fa) return EIF_HIP_E_ARG;
    const int64_t cap = (int64_t)1 << 26;   // the products below stay far inside int
    if (dim > cap || hidden > cap || ck > cap || (int64_t)nk * kd > cap || (int64_t)nv * vd > cap ||
        (int64_t)nh * hd > cap || (int64_t)nkv * hd > cap)
        return EIF_HIP_E_ARG;
    const int key_dim = nk * kd, val_dim = nv * vd, conv_dim = 2 * key_dim + val_dim;
    const int q_dim = nh * hd, kv_dim = nkv * hd, qg_dim = 2 * q_dim;
    if (g != 0 && (g < 32 || g > 4096 || g % 32 != 0 || qlm != EIF_Q35_TERN2 ||
                   (qemb != kEmb2bit && qemb != kEmbInt8) || dim % g || hidden % g || q_dim % g || val_dim % g))
        return EIF_HIP_E_ARG;
    if (had != 0 && (g <= 0 || had < 2 || (had & (had - 1)) || dim % had || hidden % had || q_dim != dim ||
                     val_dim != dim || qemb != kEmb2bit))
        return EIF_HIP_E_ARG;
    out->hadamard_block = had;
    const int small = g > 0 ? EIF_Q35_FP32 : qlm;   // proj_b / proj_a

    // weights
    Walk w{w_off, bytes};
    const size_t emb = w.take((size_t)vocab * embed_row_bytes(dim, qemb));
    auto psz = [&](int r, int cols) { return row_bytes(cols, qlm) * (size_t)r; };
    const size_t dn_qkv = w.take((size_t)n_dn * psz(conv_dim, dim)), dn_z = w.take((size_t)n_dn * psz(val_dim, dim));
    const size_t dn_out = w.take((size_t)n_dn * psz(dim, val_dim));
    const size_t dn_pb = w.take((size_t)n_dn * row_bytes(dim, small) * nv);
    const size_t dn_pa = w.take((size_t)n_dn * row_bytes(dim, small) * nv);
    const size_t fa_q = w.take((size_t)n_fa * psz(qg_dim, dim)), fa_k = w.take((size_t)n_fa * psz(kv_dim, dim));
    const size_t fa_v = w.take((size_t)n_fa * psz(kv_dim, dim)), fa_o = w.take((size_t)n_fa * psz(dim, q_dim));
    const size_t ff_g = w.take(24 * psz(hidden, dim)), ff_u = w.take(24 * psz(hidden, dim));
    const size_t ff_d = w.take(24 * psz(dim, hidden));
    const size_t dn_cv = w.take((size_t)n_dn * conv_dim * ck * 4), dn_dt = w.take((size_t)n_dn * nv * 4);
    const size_t dn_al = w.take((size_t)n_dn * nv * 4);
    if (!w.ok) return EIF_HIP_E_ARG;
    out->weights_end = w.off;

    const int emb_qt = qemb == kEmbInt8 ? EIF_Q35_INT8
                       : qemb == kEmbInt4 ? EIF_Q35_INT4
                       : qemb == kEmb2bit ? EIF_Q35_TERN2
                       : qemb == kEmbDense ? EIF_Q35_TERN3 : EIF_Q35_FP32;
    out->embed = tensor(emb, vocab, dim, emb_qt, g);
    int di = 0, fi = 0;
    for (int l = 0; l < n_layers; ++l) {
        eif_qwen35_tensor *t = out->lin[l];
        t[EIF_Q35_FF_GATE] = tensor(ff_g + (size_t)l * psz(hidden, dim), hidden, dim, qlm, g);
        t[EIF_Q35_FF_UP] = tensor(ff_u + (size_t)l * psz(hidden, dim), hidden, dim, qlm, g);
        t[EIF_Q35_FF_DOWN] = tensor(ff_d + (size_t)l * psz(dim, hidden), dim, hidden, qlm, g);
        if (out->layer_types[l] == 0) {
            t[EIF_Q35_DN_QKV] = tensor(dn_qkv + (size_t)di * psz(conv_dim, dim), conv_dim, dim, qlm, g);
            t[EIF_Q35_DN_Z] = tensor(dn_z + (size_t)di * psz(val_dim, dim), val_dim, dim, qlm, g);
            t[EIF_Q35_DN_OUT] = tensor(dn_out + (size_t)di * psz(dim, val_dim), dim, val_dim, qlm, g);
            t[EIF_Q35_DN_B] = tensor(dn_pb + (size_t)di * row_bytes(dim, small) * nv, nv, dim, small, 0);
            t[EIF_Q35_DN_A] = tensor(dn_pa + (size_t)di * row_bytes(dim, small) * nv, nv, dim, small, 0);
            out->conv[l] = dn_cv + (size_t)di * conv_dim * ck * 4;
            out->dt_bias[l] = dn_dt + (size_t)di * nv * 4;
            out->a_log[l] = dn_al + (size_t)di * nv * 4;
            ++di;
        } else {
            t[EIF_Q35_FA_Q] = tensor(fa_q + (size_t)fi * psz(qg_dim, dim), qg_dim, dim, qlm, g);
            t[EIF_Q35_FA_K] = tensor(fa_k + (size_t)fi * psz(kv_dim, dim), kv_dim, dim, qlm, g);
            t[EIF_Q35_FA_V] = tensor(fa_v + (size_t)fi * psz(kv_dim, dim), kv_dim, dim, qlm, g);
            t[EIF_Q35_FA_O] = tensor(fa_o + (size_t)fi * psz(dim, q_dim), dim, q_dim, qlm, g);
            ++fi;
        }
    }

    // scales, in the order of the walk: per DeltaNet layer, per attention layer, then 24 FFN slots
    auto sc_count = [&](int rows, int cols) { return (size_t)rows * (g > 0 ? (size_t)(cols / g) : 1u); };
    Walk s{s_off, bytes};
    out->embed.scales = s.take(4 * (qemb == kEmb2bit && g > 0 ? (size_t)vocab * (dim / g) : (size_t)vocab));
    std::vector<int> dn_layer, fa_layer;
    for (int l = 0; l < n_layers; ++l) (out->layer_types[l] ? fa_layer : dn_layer).push_back(l);
    for (int l : dn_layer) {
        eif_qwen35_tensor *t = out->lin[l];
        t[EIF_Q35_DN_QKV].scales = s.take(4 * sc_count(conv_dim, dim));
        t[EIF_Q35_DN_Z].scales = s.take(4 * sc_count(val_dim, dim));
        t[EIF_Q35_DN_OUT].scales = s.take(4 * sc_count(dim, val_dim));
        if (g == 0) {
            t[EIF_Q35_DN_B].scales = s.take(4 * (size_t)nv);
            t[EIF_Q35_DN_A].scales = s.take(4 * (size_t)nv);
        }
    }
    for (int l : fa_layer) {
        eif_qwen35_tensor *t = out->lin[l];
        t[EIF_Q35_FA_Q].scales = s.take(4 * sc_count(qg_dim, dim));
        t[EIF_Q35_FA_K].scales = s.take(4 * sc_count(kv_dim, dim));
        t[EIF_Q35_FA_V].scales = s.take(4 * sc_count(kv_dim, dim));
        t[EIF_Q35_FA_O].scales = s.take(4 * sc_count(dim, q_dim));
    }
    for (int l = 0; l < 24; ++l) {
        const size_t gs = s.take(4 * sc_count(hidden, dim)), us = s.take(4 * sc_count(hidden, dim));
        const size_t ds = s.take(4 * sc_count(dim, hidden));
        if (l < n_layers) {
            out->lin[l][EIF_Q35_FF_GATE].scales = gs;
            out->lin[l][EIF_Q35_FF_UP].scales = us;
            out->lin[l][EIF_Q35_FF_DOWN].scales = ds;
        }
    }
    if (!s.ok) return EIF_HIP_E_ARG;
    out->scales_end = s.off;

    // norms: 24 input norms, 24 post-attention norms, the final norm, then per layer the DeltaNet norm or the
    // QK norms, the Hadamard signs, the SubLN vectors that fit in norms_size
    const size_t nend = n_off + n_size;
    Walk n{n_off, nend};
    for (int l = 0; l < 24; ++l) {
        const size_t o = n.take(4 * (size_t)dim);
        if (l < n_layers) out->rms_att[l] = o;
    }
    for (int l = 0; l < 24; ++l) {
        const size_t o = n.take(4 * (size_t)dim);
        if (l < n_layers) out->rms_ffn[l] = o;
    }
    out->rms_final = n.take(4 * (size_t)dim);
    for (int l = 0; l < n_layers; ++l) {
        if (out->layer_types[l] == 0) {
            out->delta_norm[l] = n.take(4 * (size_t)vd);
        } else {
            out->q_norm[l] = n.take(4 * (size_t)hd);
            out->k_norm[l] = n.take(4 * (size_t)hd);
        }
    }
    if (!n.ok) return EIF_HIP_E_ARG;
    if (had > 0) {
        out->signs_dim = n.take(4 * (size_t)dim);
        out->signs_hid = n.take(4 * (size_t)hidden);
        if (!n.ok) return EIF_HIP_E_ARG;   // the reference: "Hadamard signs missing"
    }
    for (int l = 0; l < n_layers && !c[cPlain]; ++l) {
        if (out->layer_types[l] == 1 && n.off + 4 * (size_t)q_dim <= nend) out->sub_att[l] = n.take(4 * (size_t)q_dim);
        if (n.off + 4 * (size_t)hidden <= nend) out->sub_ffn[l] = n.take(4 * (size_t)hidden);
    }
    out->norms_end = n.off;
    return EIF_HIP_OK;
}

struct eif_hip_qwen35 {
    eif_qwen35_layout layout{};
    eif_hip_qweight *lin[24][EIF_Q35_KINDS] = {};
    eif_hip_qweight *head = nullptr;
    float *vec = nullptr;                              // the FP32 vectors, each 16-byte aligned
    std::vector<std::pair<size_t, size_t>> vec_at;     // (layout offset, float index into vec), sorted
};

namespace {

// Base-3 rows (five digits per byte, least significant first; 1 = +1, 2 = -1; the reference's LUT,
// src/eif_qwen35.c:78-92) -> 2-bit rows (code 1 = +1, 2 = -1, four per byte from the low bits).
void tern3_to_2bit(const uint8_t *src, int rows, int cols, std::vector<uint8_t> &dst)
{
    const size_t sb = (size_t)(cols + 4) / 5, db = (size_t)(cols + 3) / 4;
    dst.assign((size_t)rows * db, 0);
    for (int r = 0; r < rows; ++r) {
        const uint8_t *s = src + (size_t)r * sb;
        uint8_t *d = dst.data() + (size_t)r * db;
        for (int c = 0; c < cols; ++c) {
            int v = s[c / 5];
            for (int k = 0; k < c % 5; ++k) v /= 3;
            const int digit = v % 3;   // 0, 1 (+1) or 2 (-1): the 2-bit code of the same value
            d[c / 4] |= (uint8_t)(digit << (2 * (c % 4)));
        }
    }
}

std::vector<float> floats_at(const uint8_t *base, size_t off, size_t n)
{
    std::vector<float> v(n);
    std::memcpy(v.data(), base + off, n * sizeof(float));
    return v;
}

int upload(eif_hip_qweight **out, const uint8_t *base, const eif_qwen35_tensor &t, hipStream_t st)
{
    *out = nullptr;
    if (!t.codes || t.qtype == EIF_Q35_FP32) return EIF_HIP_OK;
    const size_t n_sc = (size_t)t.rows * (t.group > 0 ? (size_t)(t.cols / t.group) : 1u);
    const std::vector<float> sc = floats_at(base, t.scales, n_sc);
    if (t.qtype == EIF_Q35_TERN3) {
        std::vector<uint8_t> codes;
        tern3_to_2bit(base + t.codes, t.rows, t.cols, codes);
        return eif_hip_qweight_create(out, EIF_HIP_W_TERNARY, t.rows, t.cols, 0, codes.data(), sc.data(), 0, st);
    }
    const int fmt = t.qtype == EIF_Q35_TERN2 ? EIF_HIP_W_TERNARY
                    : t.qtype == EIF_Q35_INT4 ? EIF_HIP_W_INT4 : EIF_HIP_W_INT8;
    return eif_hip_qweight_create(out, fmt, t.rows, t.cols, t.group, base + t.codes, sc.data(), 0, st);
}

}  // namespace

extern "C" void eif_hip_qwen35_destroy(eif_hip_qwen35 *m)
{
    if (!m) return;
    for (auto &row : m->lin)
        for (eif_hip_qweight *w : row) eif_hip_qweight_destroy(w);
    eif_hip_qweight_destroy(m->head);
    if (m->vec) (void)hipFree(m->vec);
    delete m;
}

namespace {

int load_model(eif_hip_qwen35 **out, const char *path, void *stream)
{
    std::FILE *f = std::fopen(path, "rb");
    if (!f) return EIF_HIP_E_ARG;
    std::vector<uint8_t> img;
    bool ok = std::fseek(f, 0, SEEK_END) == 0;
    const long size = ok ? std::ftell(f) : -1;
    ok = ok && size > 0 && std::fseek(f, 0, SEEK_SET) == 0;
    if (ok) {
        try {
            img.resize((size_t)size);
        } catch (...) {
            std::fclose(f);
            return EIF_HIP_E_NOMEM;
        }
        ok = std::fread(img.data(), 1, img.size(), f) == img.size();
    }
    std::fclose(f);
    if (!ok) return EIF_HIP_E_ARG;
    if (img.size() >= 4 && img[0] == 'G' && img[1] == 'G' && img[2] == 'U' && img[3] == 'F') {
        // a Qwen3.5 GGUF file: its QWN5 image, as the reference's qwen35_load builds it (src/eif_qwen35.c:1236-1246)
        void *built = nullptr;
        size_t n = 0;
        const int rc = eif_qwen35_gguf_image(img.data(), img.size(), &built, &n);
        if (rc) return rc;
        try {
            img.assign(static_cast<uint8_t *>(built), static_cast<uint8_t *>(built) + n);
        } catch (...) {
            eif_qwen35_image_free(built);
            return EIF_HIP_E_NOMEM;
        }
        eif_qwen35_image_free(built);
    }

    // Owned until the end: an exception (host allocation) or an error after this point frees every uploaded weight.
    std::unique_ptr<eif_hip_qwen35, void (*)(eif_hip_qwen35 *)> owner(new (std::nothrow) eif_hip_qwen35,
                                                                       eif_hip_qwen35_destroy);
    eif_hip_qwen35 *m = owner.get();
    if (!m) return EIF_HIP_E_NOMEM;
    int rc = eif_qwen35_parse(img.data(), img.size(), &m->layout);
    const hipStream_t st = (hipStream_t)stream;
    const eif_qwen35_layout &L = m->layout;
    for (int l = 0; l < L.n_layers && rc == EIF_HIP_OK; ++l)
        for (int k = 0; k < EIF_Q35_KINDS && rc == EIF_HIP_OK; ++k) rc = upload(&m->lin[l][k], img.data(), L.lin[l][k], st);
    if (rc == EIF_HIP_OK) rc = upload(&m->head, img.data(), L.embed, st);
    if (rc == EIF_HIP_OK) {
        // the FP32 vectors of the norms region and the DeltaNet parameters, each at a 16-byte aligned slot
        const int32_t *c = L.config;
        const int dim = c[cDim], hidden = c[cHidden], hd = c[cHeadDim], nv = c[cLinV], vd = c[cLinVd];
        const int conv_dim = 2 * c[cLinK] * c[cLinKd] + nv * vd, q_dim = c[cHeads] * hd;
        std::vector<std::pair<size_t, size_t>> items;   // (offset, floats)
        auto add = [&](size_t off, int n) {
            if (off) items.emplace_back(off, (size_t)n);
        };
        for (int l = 0; l < L.n_layers; ++l) {
            add(L.rms_att[l], dim), add(L.rms_ffn[l], dim), add(L.sub_att[l], q_dim), add(L.sub_ffn[l], hidden);
            add(L.conv[l], conv_dim * c[cConvK]), add(L.dt_bias[l], nv), add(L.a_log[l], nv);
            add(L.delta_norm[l], vd), add(L.q_norm[l], hd), add(L.k_norm[l], hd);
        }
        add(L.rms_final, dim), add(L.signs_dim, dim), add(L.signs_hid, hidden);
        std::sort(items.begin(), items.end());
        std::vector<float> host;
        for (const auto &it : items) {
            m->vec_at.emplace_back(it.first, host.size());
            const std::vector<float> v = floats_at(img.data(), it.first, it.second);
            host.insert(host.end(), v.begin(), v.end());
            host.resize((host.size() + 3) & ~(size_t)3, 0.0f);
        }
        if (!host.empty()) {
            if (hipMalloc(&m->vec, host.size() * sizeof(float)) != hipSuccess) rc = EIF_HIP_E_NOMEM;
            else if (hipMemcpy(m->vec, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
                rc = EIF_HIP_E_DEVICE;
        }
    }
    if (rc) return rc;   // owner frees m
    *out = owner.release();
    return EIF_HIP_OK;
}

}  // namespace

extern "C" int eif_hip_qwen35_load(eif_hip_qwen35 **out, const char *path, void *stream)
{
    if (!out || !path) return EIF_HIP_E_ARG;
    *out = nullptr;
    try {
        return load_model(out, path, stream);
    } catch (...) {   // allocation failures of the host-side bookkeeping
        return EIF_HIP_E_NOMEM;
    }
}

extern "C" const eif_qwen35_layout *eif_hip_qwen35_get_layout(const eif_hip_qwen35 *m)
{
    return m ? &m->layout : nullptr;
}

extern "C" const eif_hip_qweight *eif_hip_qwen35_linear(const eif_hip_qwen35 *m, int layer, int kind)
{
    if (!m || layer < 0 || layer >= m->layout.n_layers || kind < 0 || kind >= EIF_Q35_KINDS) return nullptr;
    return m->lin[layer][kind];
}

extern "C" const eif_hip_qweight *eif_hip_qwen35_head(const eif_hip_qwen35 *m)
{
    return m ? m->head : nullptr;
}

// The batched linear of the engine's prefill (linear_gemm, src/eif_qwen35.c:1034-1065, as prefill_chunk calls it,
// :1067-1153) on a resident matrix: eif_hip_qlinear_prep over the batch's rows.
extern "C" int eif_hip_qwen35_linear_batch(const eif_hip_qwen35 *m, int layer, int kind, const eif_hip_prep_spec *spec,
                                           const float *bias, float *y, int ldy, int M, void *stream)
{
    const eif_hip_qweight *w = kind == EIF_Q35_HEAD ? eif_hip_qwen35_head(m) : eif_hip_qwen35_linear(m, layer, kind);
    if (!w || !spec || M < 1) return EIF_HIP_E_ARG;
    return eif_hip_qlinear_prep(w, spec, bias, y, ldy, M, stream);
}

extern "C" const float *eif_hip_qwen35_vector(const eif_hip_qwen35 *m, size_t offset)
{
    if (!m || !offset || !m->vec) return nullptr;
    const auto it = std::lower_bound(m->vec_at.begin(), m->vec_at.end(), std::make_pair(offset, (size_t)0));
    if (it == m->vec_at.end() || it->first != offset) return nullptr;
    return m->vec + it->second;
}

// qwen35_gguf.cpp -- a llama.cpp-style Qwen3.5 text GGUF -> the QWN5 image the Qwen3.5 loader reads
// (eif_hip_qwen35.h), as the reference's qwen35_gguf_build_image builds it (src/eif_qwen35_gguf.c:262-454).
//
// Every linear is dequantised row by row (F32, F16, BF16, Q8_0, Q4_0, Q4_K, Q5_K, Q6_K; gguf_container.h) and
// requantised to INT4 rows, the tied embedding to INT8 rows, with quant_rows (:225-258) as the reference's
// -ffast-math build computes it: amax = max(1e-8, max |x|), s = amax * (1 / qmax), inv = 1 / s,
// q = round-half-even(x * inv) clamped, INT4 columns (2i, 2i + 1) in byte i high nibble first. Norms, the conv
// kernel and dt bias are copied as FP32, ssm_a becomes A_log = logf(-ssm_a). The image: a 48-byte header, the
// 128-byte configuration (INT4 linears, INT8 tied embedding, plain linears), 24 layer types, then the weights,
// scales and norms regions in the loader's order. Limits of the reference's builder, kept: 24 layers, a tied head,
// as many key heads as value heads, RMSNorm epsilon 1e-6, no vision tower.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/eif_hip.h"
#include "../../include/eif_hip_qwen35.h"
#include "gguf_container.h"

namespace {

using namespace eif::gguf;

constexpr uint32_t kQwn5Magic = 0x51574E35u, kQwn5Version = 1u;
constexpr int kLayers = 24;

double read_number(Cursor &c, uint32_t t)   // a scalar value as a double (bool reads as 0, as the reference's)
{
    switch (t) {
    case 0: return c.get<uint8_t>();
    case 1: return c.get<int8_t>();
    case 2: return c.get<uint16_t>();
    case 3: return c.get<int16_t>();
    case 4: return c.get<uint32_t>();
    case 5: return c.get<int32_t>();
    case 6: return c.get<float>();
    case 7: c.get<uint8_t>(); return 0.0;
    case 10: return (double)c.get<uint64_t>();
    case 11: return (double)c.get<int64_t>();
    case 12: return c.get<double>();
    default: c.ok = false; return 0.0;
    }
}

bool readable(int t)   // the types the builder dequantises
{
    return t == kF32 || t == kF16 || t == kBF16 || t == kQ8_0 || t == kQ4_0 || t == kQ4_K || t == kQ5_K ||
           t == kQ6_K;
}

struct Model {
    const uint8_t *file = nullptr, *data = nullptr;
    size_t n = 0;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> index;   // the first tensor of a name
    bool bad = false;

    const Tensor *find(const std::string &name) const
    {
        const auto it = index.find(name);
        return it == index.end() ? nullptr : &tensors[it->second];
    }
    // the tensor as [rows, cols] of a readable type, whole blocks per row, inside the file (else bad)
    const Tensor *need(const std::string &name, int rows, int cols)
    {
        const Tensor *t = find(name);
        int bytes = 0, values = 1;
        if (t) block_geom((int)t->type, bytes, values);
        const uint64_t r = t && t->n_dims >= 2 ? t->ne[1] : 1;
        if (!t || !readable((int)t->type) || t->ne[0] != (uint64_t)cols || r != (uint64_t)rows || cols % values) {
            bad = true;
            return nullptr;
        }
        const uint64_t sz = (uint64_t)rows * (uint64_t)(cols / values) * (uint64_t)bytes;
        const uint64_t start = (uint64_t)(data - file);
        if (t->offset > n - start || sz > n - start - t->offset) {
            bad = true;
            return nullptr;
        }
        return t;
    }
    const uint8_t *row(const Tensor *t, int r, int cols) const
    {
        int bytes = 0, values = 1;
        block_geom((int)t->type, bytes, values);
        return data + t->offset + (size_t)r * (size_t)(cols / values) * (size_t)bytes;
    }
    void copy_f32(const std::string &name, int rows, int cols, float *dst)
    {
        const Tensor *t = need(name, rows, cols);
        if (!t) return;
        for (int r = 0; r < rows; ++r) dequant_row((int)t->type, row(t, r, cols), cols, dst + (size_t)r * cols);
    }
    // rows of the tensor -> INT8 (bits 8) or INT4 (bits 4) rows and one scale each, over a few host threads
    void quant_rows(const std::string &name, int rows, int cols, int bits, uint8_t *dst, float *scales)
    {
        const Tensor *t = need(name, rows, cols);
        if (!t) return;
        const size_t rb = bits == 8 ? (size_t)cols : (size_t)(cols + 1) / 2;
        const float rq = bits == 8 ? 1.0f / 127.0f : 1.0f / 7.0f;
        const int lo = bits == 8 ? -128 : -8, hi = bits == 8 ? 127 : 7;
        auto work = [&](int r0, int r1) {
            std::vector<float> x((size_t)cols + 1);
            for (int r = r0; r < r1; ++r) {
                dequant_row((int)t->type, row(t, r, cols), cols, x.data());
                x[cols] = 0.0f;
                float amax = 1e-8f;
                for (int c = 0; c < cols; ++c) amax = std::fabs(x[c]) > amax ? std::fabs(x[c]) : amax;
                const float s = amax * rq, inv = 1.0f / s;
                scales[r] = s;
                auto code = [&](float v) {   // a NaN takes the lowest code, as the reference's x86 conversion
                    const float q = std::nearbyint(v * inv);
                    if (!(q >= (float)lo)) return lo;
                    return q > (float)hi ? hi : (int)q;
                };
                uint8_t *o = dst + (size_t)r * rb;
                if (bits == 8) {
                    for (int c = 0; c < cols; ++c) o[c] = (uint8_t)(int8_t)code(x[c]);
                } else {
                    for (int c = 0; c < cols; c += 2)
                        o[c / 2] = (uint8_t)(((code(x[c]) + 8) << 4) | ((code(x[c + 1]) + 8) & 15));
                }
            }
        };
        const int nt = std::max(1, std::min<int>({16, (int)std::thread::hardware_concurrency(), rows / 256}));
        if (nt == 1) {
            work(0, rows);
            return;
        }
        auto lo_of = [&](int i) { return (int)((int64_t)rows * i / nt); };
        std::vector<std::thread> pool;
        int started = 0;
        try {
            for (; started < nt; ++started) pool.emplace_back(work, lo_of(started), lo_of(started + 1));
        } catch (...) {   // no more threads: the caller takes the rest
        }
        for (int i = started; i < nt; ++i) work(lo_of(i), lo_of(i + 1));
        for (auto &th : pool) th.join();
    }
};

}  // namespace

namespace {

int build_image(const void *file, size_t bytes, void **image, size_t *image_bytes)
{
    *image = nullptr, *image_bytes = 0;
    Cursor c{static_cast<const uint8_t *>(file), bytes};
    if (c.get<uint32_t>() != kMagic) return EIF_HIP_E_ARG;
    c.get<uint32_t>();
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    std::string arch;
    uint64_t alignment = 32;
    double v_block = 0, v_dim = 0, v_ff = 0, v_heads = 0, v_kv = 0, v_keylen = 0, v_ctx = 0, v_interval = 4,
           v_eps = 1e-6, s_conv = 0, s_state = 0, s_group = 0, s_rank = 0, s_inner = 0;
    for (uint64_t i = 0; i < n_kv && c.ok; ++i) {
        const std::string key = c.str();
        if (key.size() >= 160) return EIF_HIP_E_ARG;
        const uint32_t t = c.get<uint32_t>();
        if (!c.ok) break;
        if (key == "general.architecture" && t == 8) {
            arch = c.str().substr(0, 63);
        } else if (key == "general.alignment" && scalar_size(t)) {
            const double a = read_number(c, t);
            alignment = a >= 1.0 && a <= 65536.0 ? (uint64_t)a : 0;   // 0: the default below
        } else if (scalar_size(t) && key.compare(0, 7, "qwen35.") == 0) {
            const double v = read_number(c, t);
            const std::string k = key.substr(7);
            if (k == "block_count") v_block = v;
            else if (k == "embedding_length") v_dim = v;
            else if (k == "feed_forward_length") v_ff = v;
            else if (k == "attention.head_count") v_heads = v;
            else if (k == "attention.head_count_kv") v_kv = v;
            else if (k == "attention.key_length") v_keylen = v;
            else if (k == "context_length") v_ctx = v;
            else if (k == "full_attention_interval") v_interval = v;
            else if (k == "attention.layer_norm_rms_epsilon") v_eps = v;
            else if (k == "ssm.conv_kernel") s_conv = v;
            else if (k == "ssm.state_size") s_state = v;
            else if (k == "ssm.group_count") s_group = v;
            else if (k == "ssm.time_step_rank") s_rank = v;
            else if (k == "ssm.inner_size") s_inner = v;
        } else {
            skip_value(c, t);
        }
    }
    if (!c.ok || arch != "qwen35" || n_tensors == 0 || n_tensors > 100000) return EIF_HIP_E_ARG;
    Model m;
    m.file = static_cast<const uint8_t *>(file), m.n = bytes;
    try {
        m.tensors.reserve((size_t)n_tensors);
        for (uint64_t i = 0; i < n_tensors && c.ok; ++i) {
            const std::string name = c.str();
            Tensor t;
            t.n_dims = c.get<uint32_t>();
            if (!c.ok || name.size() >= 128 || t.n_dims > (c.n - c.at) / 8) return EIF_HIP_E_ARG;
            for (uint32_t d = 0; d < t.n_dims; ++d) {
                const uint64_t v = c.get<uint64_t>();
                if (d < 4) t.ne[d] = v;
            }
            t.type = c.get<uint32_t>();
            t.offset = c.get<uint64_t>();
            m.tensors.push_back(t);
            m.index.emplace(name, m.tensors.size() - 1);
        }
    } catch (...) {
        return EIF_HIP_E_NOMEM;
    }
    if (!c.ok) return EIF_HIP_E_ARG;
    if (alignment == 0) alignment = 32;
    const uint64_t start = (c.at + alignment - 1) / alignment * alignment;
    if (start > bytes) return EIF_HIP_E_ARG;
    m.data = m.file + start;

    auto iv = [](double v) { return v >= -1e9 && v <= 1e9 ? (int)v : -1; };   // out of range: refused below
    const int dim = iv(v_dim), hidden = iv(v_ff), L = iv(v_block), nh = iv(v_heads), nkv = iv(v_kv);
    const int hd = iv(v_keylen), ck = iv(s_conv), kd = iv(s_state), nk = iv(s_group), nv = iv(s_rank);
    const int interval = iv(v_interval), vd = nv > 0 ? iv(s_inner) / nv : 0;
    if (L != kLayers || nk != nv || std::fabs(v_eps - 1e-6) > 1e-8 || m.find("output.weight") || dim <= 0 ||
        hidden <= 0 || nh <= 0 || nkv <= 0 || hd <= 0 || ck <= 0 || kd <= 0 || vd <= 0 || interval <= 0)
        return EIF_HIP_E_ARG;
    const int64_t cap = (int64_t)1 << 26;   // products below stay far inside int
    if (dim > cap || hidden > cap || ck > cap || (int64_t)nk * kd > cap || (int64_t)nv * vd > cap ||
        (int64_t)nh * hd > cap || (int64_t)nkv * hd > cap)
        return EIF_HIP_E_ARG;
    const Tensor *te = m.find("token_embd.weight");
    if (!te || te->n_dims < 2 || te->ne[1] == 0 || te->ne[1] > 0x7fffffff) return EIF_HIP_E_ARG;
    const int vocab = (int)te->ne[1];

    uint8_t full[kLayers];
    int n_fa = 0, n_dn = 0;
    for (int l = 0; l < L; ++l) {
        full[l] = (l + 1) % interval == 0;
        full[l] ? ++n_fa : ++n_dn;
    }
    const int key_dim = nk * kd, val_dim = nv * vd, conv_dim = 2 * key_dim + val_dim, q_dim = nh * hd;
    const int kv_dim = nkv * hd, qg_dim = 2 * q_dim;
    const size_t rbd = (size_t)(dim + 1) / 2, rbh = (size_t)(hidden + 1) / 2, rbv = (size_t)(val_dim + 1) / 2;
    const size_t rbq = (size_t)(q_dim + 1) / 2;
    const size_t w_embed = (size_t)vocab * dim;
    const size_t w_total = w_embed + (size_t)n_dn * (rbd * conv_dim + rbd * val_dim + rbv * dim + 2 * rbd * nv) +
                           (size_t)n_fa * (rbd * qg_dim + rbd * kv_dim * 2 + rbq * dim) +
                           (size_t)L * (rbd * hidden * 2 + rbh * dim) + (size_t)n_dn * ((size_t)conv_dim * ck + 2 * nv) * 4;
    const size_t s_total = ((size_t)vocab + (size_t)n_dn * (conv_dim + val_dim + dim + 2 * nv) +
                            (size_t)n_fa * (qg_dim + 2 * kv_dim + dim) + (size_t)L * (hidden * 2 + dim)) * 4;
    const size_t n_total = ((size_t)(2 * L + 1) * dim + (size_t)n_dn * vd + (size_t)n_fa * 2 * hd) * 4;
    const size_t kHdr = 48, kCfg = 128, kLt = 24, total = kHdr + kCfg + kLt + w_total + s_total + n_total;
    if (total > 0xFFFFFFFFu) return EIF_HIP_E_LIMIT;
    uint8_t *img = static_cast<uint8_t *>(std::calloc(1, total + 64));
    if (!img) return EIF_HIP_E_NOMEM;
    *image = img;   // released by the caller's error path from here on

    uint32_t hdr[12] = {kQwn5Magic, kQwn5Version, (uint32_t)kHdr, (uint32_t)(kHdr + kCfg + kLt)};
    hdr[4] = hdr[3] + (uint32_t)w_total, hdr[5] = hdr[4] + (uint32_t)s_total, hdr[6] = hdr[5] + (uint32_t)n_total;
    hdr[7] = (uint32_t)w_total, hdr[8] = (uint32_t)s_total, hdr[9] = (uint32_t)n_total;
    std::memcpy(img, hdr, sizeof(hdr));
    int32_t cfg[32] = {dim, hidden, L, nh, nkv, hd, vocab, v_ctx > 0 && v_ctx < 4096 ? (int)v_ctx : 4096, n_dn, n_fa,
                       nk, kd, nv, vd, ck};
    cfg[22] = 1;   // tied head
    cfg[23] = 1;   // INT4 linears
    cfg[25] = 0;   // INT8 embedding
    cfg[26] = 1;   // plain linears
    std::memcpy(img + kHdr, cfg, sizeof(cfg));
    std::memcpy(img + kHdr + kCfg, full, (size_t)L);

    uint8_t *wp = img + hdr[3];
    float *sc = reinterpret_cast<float *>(img + hdr[4]);
    float *np = reinterpret_cast<float *>(img + hdr[5]);
    // weights in the loader's order: embed, DeltaNet qkv / z / out / beta / alpha, attention q / k / v / o,
    // FFN gate / up / down, conv, dt, A_log
    uint8_t *w_emb = wp;
    wp += w_embed;
    auto take = [&](size_t n) {
        uint8_t *p = wp;
        wp += n;
        return p;
    };
    uint8_t *w_qkv = take((size_t)n_dn * rbd * conv_dim), *w_z = take((size_t)n_dn * rbd * val_dim);
    uint8_t *w_out = take((size_t)n_dn * rbv * dim), *w_pb = take((size_t)n_dn * rbd * nv);
    uint8_t *w_pa = take((size_t)n_dn * rbd * nv), *w_q = take((size_t)n_fa * rbd * qg_dim);
    uint8_t *w_k = take((size_t)n_fa * rbd * kv_dim), *w_v = take((size_t)n_fa * rbd * kv_dim);
    uint8_t *w_o = take((size_t)n_fa * rbq * dim), *w_g = take((size_t)L * rbd * hidden);
    uint8_t *w_u = take((size_t)L * rbd * hidden), *w_d = take((size_t)L * rbh * dim);
    float *w_conv = reinterpret_cast<float *>(take((size_t)n_dn * conv_dim * ck * 4));
    float *w_dt = reinterpret_cast<float *>(take((size_t)n_dn * nv * 4));
    float *w_al = reinterpret_cast<float *>(wp);

    // scales: the embedding's, then every DeltaNet layer's, every attention layer's, every FFN's
    float *s_emb = sc;
    sc += vocab;
    m.quant_rows("token_embd.weight", vocab, dim, 8, w_emb, s_emb);
    float *sc_dn = sc, *sc_fa = sc_dn + (size_t)n_dn * (conv_dim + val_dim + dim + 2 * nv);
    float *sc_ffn = sc_fa + (size_t)n_fa * (qg_dim + 2 * kv_dim + dim);
    auto next = [](float *&p, int n) {
        float *q = p;
        p += n;
        return q;
    };
    const std::string b = "blk.";
    for (int l = 0, di = 0, fi = 0; l < L && !m.bad; ++l) {
        const std::string p = b + std::to_string(l) + ".";
        if (!full[l]) {
            m.quant_rows(p + "attn_qkv.weight", conv_dim, dim, 4, w_qkv + (size_t)di * rbd * conv_dim, next(sc_dn, conv_dim));
            m.quant_rows(p + "attn_gate.weight", val_dim, dim, 4, w_z + (size_t)di * rbd * val_dim, next(sc_dn, val_dim));
            m.quant_rows(p + "ssm_out.weight", dim, val_dim, 4, w_out + (size_t)di * rbv * dim, next(sc_dn, dim));
            m.quant_rows(p + "ssm_beta.weight", nv, dim, 4, w_pb + (size_t)di * rbd * nv, next(sc_dn, nv));
            m.quant_rows(p + "ssm_alpha.weight", nv, dim, 4, w_pa + (size_t)di * rbd * nv, next(sc_dn, nv));
            m.copy_f32(p + "ssm_conv1d.weight", conv_dim, ck, w_conv + (size_t)di * conv_dim * ck);
            m.copy_f32(p + "ssm_dt.bias", 1, nv, w_dt + (size_t)di * nv);
            m.copy_f32(p + "ssm_a", 1, nv, w_al + (size_t)di * nv);
            if (!m.bad)
                for (int i = 0; i < nv; ++i) w_al[(size_t)di * nv + i] = std::log(-w_al[(size_t)di * nv + i]);
            ++di;
        } else {
            m.quant_rows(p + "attn_q.weight", qg_dim, dim, 4, w_q + (size_t)fi * rbd * qg_dim, next(sc_fa, qg_dim));
            m.quant_rows(p + "attn_k.weight", kv_dim, dim, 4, w_k + (size_t)fi * rbd * kv_dim, next(sc_fa, kv_dim));
            m.quant_rows(p + "attn_v.weight", kv_dim, dim, 4, w_v + (size_t)fi * rbd * kv_dim, next(sc_fa, kv_dim));
            m.quant_rows(p + "attn_output.weight", dim, q_dim, 4, w_o + (size_t)fi * rbq * dim, next(sc_fa, dim));
            ++fi;
        }
    }
    for (int l = 0; l < L && !m.bad; ++l) {
        const std::string p = b + std::to_string(l) + ".";
        m.quant_rows(p + "ffn_gate.weight", hidden, dim, 4, w_g + (size_t)l * rbd * hidden, next(sc_ffn, hidden));
        m.quant_rows(p + "ffn_up.weight", hidden, dim, 4, w_u + (size_t)l * rbd * hidden, next(sc_ffn, hidden));
        m.quant_rows(p + "ffn_down.weight", dim, hidden, 4, w_d + (size_t)l * rbh * dim, next(sc_ffn, dim));
    }
    // norms (GGUF holds the +1 form the loader expects): attention, post-attention, final, then per layer the
    // DeltaNet output norm or the attention q / k norms
    for (int l = 0; l < L && !m.bad; ++l) m.copy_f32(b + std::to_string(l) + ".attn_norm.weight", 1, dim, next(np, dim));
    for (int l = 0; l < L && !m.bad; ++l)
        m.copy_f32(b + std::to_string(l) + ".post_attention_norm.weight", 1, dim, next(np, dim));
    if (!m.bad) m.copy_f32("output_norm.weight", 1, dim, next(np, dim));
    for (int l = 0; l < L && !m.bad; ++l) {
        const std::string p = b + std::to_string(l) + ".";
        if (!full[l]) {
            m.copy_f32(p + "ssm_norm.weight", 1, vd, next(np, vd));
        } else {
            m.copy_f32(p + "attn_q_norm.weight", 1, hd, next(np, hd));
            m.copy_f32(p + "attn_k_norm.weight", 1, hd, next(np, hd));
        }
    }
    if (m.bad) return EIF_HIP_E_ARG;
    *image_bytes = total;
    return EIF_HIP_OK;
}

}  // namespace

extern "C" int eif_qwen35_gguf_image(const void *file, size_t bytes, void **image, size_t *image_bytes)
{
    if (!file || !image || !image_bytes) return EIF_HIP_E_ARG;
    *image = nullptr, *image_bytes = 0;
    int rc;
    try {
        rc = build_image(file, bytes, image, image_bytes);
    } catch (...) {   // allocation failures of the host-side bookkeeping
        rc = EIF_HIP_E_NOMEM;
    }
    if (rc) {
        std::free(*image);
        *image = nullptr, *image_bytes = 0;
    }
    return rc;
}

extern "C" void eif_qwen35_image_free(void *image) { std::free(image); }

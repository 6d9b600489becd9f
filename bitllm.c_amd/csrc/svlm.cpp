// svlm.cpp -- a BitNet-b1.58 model file in the reference's SVLM or TTML layout -> the GPU decoder (eif_hip_decode.h).
//
// The file is what tinyllm_load_quantized_model reads (src/eif_tinyllm.c:2442-2556) with the pointer layout of
// tinyllm_setup_quantized_pointers for BitNet (:2663-2731) and the configuration that the reference's engine
// reads from it (src/eif_llm.c:321-351). SVLM:
//   header   12 x u32: [0] 'SVLM', [3] weights offset, [4] scales offset, [5] norms offset, [7] weights bytes,
//            [8] scales bytes, [9] norms bytes (the other words: version and the vision encoder, unused here)
//   config   32 x i32 at byte 48: dim, hidden, layers, heads, kv heads, head_dim (0: dim / heads), vocab,
//            seq_len (0: 512); [12] qtype (3 = BitNet b1.58), [14] group bound (0: one scale per row),
//            [15] Hadamard-rotated weights; RoPE theta 100000
//   weights  INT8 embedding [vocab][dim]; per kind q, k, v, o, w1, w2, w3 the 2-bit rows of every layer
//            [layers][rows][(in + 3) / 4]; INT8 head [vocab][dim]
//   scales   embedding scales [vocab]; per kind q, k, v, o, w1, w3, w2 the group scales [layers][rows][in / g]
//            with g = eif_bitnet_group_size(in, bound) (the input width itself when 0); head scales [vocab];
//            with the Hadamard flag, the signs of the dim, q_dim and hidden inputs
//   norms    attention [layers][dim], FFN [layers][dim], final [dim], then the sub-norms [layers][q_dim] and
//            [layers][hidden] (absent: weight 1)
// TTML / TLLM (tinyllm_save_quantized_model, src/eif_tinyllm.c:2305-2400): a 36-byte header (magic, version,
// config, weights, scales and norms sizes) and tinyllm_config_t (dim, hidden, layers, heads, kv heads, vocab,
// seq_len, qtype, head_dim, rope_interleaved, rope_theta (0: 5e6 above 120000 tokens of vocabulary, 1e5 above
// 60000, else 1e4, src/eif_tinyllm.c:399), kv_type; the BitNet group fields are not read), then the regions in
// that order; one scale per row, no rotation. With rope_interleaved set the rows of wq and wk are reordered
// within each head for the decoder's half-split pairs (eif::rope_rows_to_half_split).
// One scale per row without rotation (every TTML file, SVLM with bound 0 and no flag): scales are the embedding's
// [vocab]; per layer the attention rows' at q 0, k wk, v wv, o wo within a stride of 4 dim + 2 kv_dim (k at
// dim, v at 2 dim, o at 2 dim + kv_dim), or of q_dim + 2 kv_dim + dim packed when head_dim is set apart from
// dim / heads (src/eif_tinyllm.c:383-385, :420-422); per layer w1, w3, w2 (:713-787); the head's [vocab].
// The model's other choices are tinyllm's: rotation blocks eif_hadamard_block_size(width) with the reference
// build's 1/sqrt(block) (eif_hip_wht_norm), RMSNorm epsilon 1e-6 above 120000 tokens of vocabulary else 1e-5,
// sub-norm epsilon 1e-5 (src/eif_tinyllm.c:395-410, :660-670, :790-795).
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/eif_hip.h"
#include "../../include/eif_hip_decode.h"
#include "host_formats.h"
#include "../../include/eif_quantize_bitnet.h"

namespace {

constexpr uint32_t kSvlmMagic = 0x53564C4Du, kTtmlMagic = 0x54544D4Cu, kTllmMagic = 0x544C4C4Du;

struct File {
    FILE *f = nullptr;
    ~File()
    {
        if (f) std::fclose(f);
    }
};

bool read_at(FILE *f, long off, void *dst, size_t bytes)
{
    return std::fseek(f, off, SEEK_SET) == 0 && std::fread(dst, 1, bytes, f) == bytes;
}

}  // namespace

extern "C" int eif_hip_bitnet_load_svlm(eif_hip_bitnet **out, const char *path, int seq_len)
{
    if (!out || !path) return EIF_HIP_E_ARG;
    *out = nullptr;
    File file;
    file.f = std::fopen(path, "rb");
    if (!file.f) return EIF_HIP_E_ARG;
    uint32_t magic = 0;
    if (!read_at(file.f, 0, &magic, 4)) return EIF_HIP_E_ARG;
    int dim, hidden, L, nh, nkv, hd, vocab, file_seq, bound, had;
    bool interleaved = false;   // RoPE on interleaved pairs (TTML's rope_interleaved)
    float theta;
    long w_off, s_off, n_off;
    size_t w_size, s_size, n_size;
    if (magic == kSvlmMagic) {
        uint32_t hdr[12];
        int32_t ci[32];
        if (!read_at(file.f, 0, hdr, sizeof(hdr)) || !read_at(file.f, 48, ci, sizeof(ci))) return EIF_HIP_E_ARG;
        dim = ci[0], hidden = ci[1], L = ci[2], nh = ci[3], nkv = ci[4], vocab = ci[6];
        hd = ci[5] > 0 ? ci[5] : (nh > 0 ? dim / nh : 0);
        file_seq = ci[7] > 0 ? ci[7] : 512;
        bound = ci[14], had = ci[15];
        theta = 100000.0f;
        if (ci[12] != 3) return EIF_HIP_E_ARG;
        w_off = hdr[3], s_off = hdr[4], n_off = hdr[5], w_size = hdr[7], s_size = hdr[8], n_size = hdr[9];
    } else if (magic == kTtmlMagic || magic == kTllmMagic) {
        uint32_t hdr[9];
        int32_t ci[12];
        if (!read_at(file.f, 0, hdr, sizeof(hdr)) || hdr[2] < sizeof(ci) || !read_at(file.f, 36, ci, sizeof(ci)))
            return EIF_HIP_E_ARG;
        dim = ci[0], hidden = ci[1], L = ci[2], nh = ci[3], nkv = ci[4], vocab = ci[5];
        file_seq = ci[6];
        hd = ci[8] > 0 ? ci[8] : (nh > 0 ? dim / nh : 0);
        std::memcpy(&theta, &ci[10], 4);
        if (!(theta > 0.0f)) theta = vocab > 120000 ? 5000000.0f : (vocab > 60000 ? 100000.0f : 10000.0f);
        bound = 0, had = 0, interleaved = ci[9] != 0;
        if (ci[7] != 3) return EIF_HIP_E_ARG;   // BitNet only
        w_off = 36 + (long)hdr[2], w_size = hdr[3];
        s_off = w_off + (long)hdr[3], s_size = hdr[4];
        n_off = s_off + (long)hdr[4], n_size = hdr[5];
    } else {
        return EIF_HIP_E_ARG;
    }
    if (dim <= 0 || hidden <= 0 || L <= 0 || nh <= 0 || nkv <= 0 || vocab <= 0 || hd <= 0 || bound < 0 ||
        file_seq <= 0 || (interleaved && hd % 2))
        return EIF_HIP_E_ARG;
    const int64_t cap = (int64_t)1 << 26;   // the sizes below stay far inside int
    if (dim > cap || hidden > cap || vocab > cap || L > 4096 || (int64_t)nh * hd > cap || (int64_t)nkv * hd > cap)
        return EIF_HIP_E_ARG;
    const bool rowwise = bound == 0 && !had;   // the per-row scale layout
    const int q_dim = nh * hd, kv_dim = nkv * hd;
    const bool explicit_hd = hd != dim / nh;
    const size_t att_stride = explicit_hd ? (size_t)q_dim + 2 * kv_dim + dim : (size_t)4 * dim + 2 * kv_dim;
    const size_t att_off[4] = {0, explicit_hd ? (size_t)q_dim : (size_t)dim,
                               explicit_hd ? (size_t)q_dim + kv_dim : (size_t)2 * dim,
                               explicit_hd ? (size_t)q_dim + 2 * kv_dim : (size_t)2 * dim + kv_dim};
    const size_t ffn_stride = (size_t)2 * hidden + dim;
    // group of a kind with input width `in` (0 = one scale per row, as the file stores g = in)
    auto group_of = [&](int in) {
        const int g = bound > 0 ? eif_bitnet_group_size(in, bound) : 0;
        return g <= 0 || g >= in ? 0 : g;
    };
    auto ngroups = [&](int in) {
        const int g = group_of(in);
        return g > 0 ? (size_t)(in / g) : (size_t)1;
    };
    const size_t dp = (size_t)(dim + 3) / 4, qp = (size_t)(q_dim + 3) / 4, hp = (size_t)(hidden + 3) / 4;
    const size_t w_bytes = (size_t)vocab * dim * 2 +
                           (size_t)L * ((size_t)q_dim * dp + 2 * (size_t)kv_dim * dp + (size_t)dim * qp +
                                        2 * (size_t)hidden * dp + (size_t)dim * hp);
    const size_t rows_in[7][2] = {{(size_t)q_dim, (size_t)dim}, {(size_t)kv_dim, (size_t)dim},
                                  {(size_t)kv_dim, (size_t)dim}, {(size_t)dim, (size_t)q_dim},
                                  {(size_t)hidden, (size_t)dim}, {(size_t)hidden, (size_t)dim},
                                  {(size_t)dim, (size_t)hidden}};   // q, k, v, o, w1, w3, w2 (the scales' order)
    size_t s_count = 2 * (size_t)vocab;
    if (rowwise) {
        s_count += (size_t)L * (att_stride + ffn_stride);
    } else {
        for (const auto &ri : rows_in) s_count += (size_t)L * ri[0] * ngroups((int)ri[1]);
        if (had) s_count += (size_t)dim + q_dim + hidden;
    }
    const size_t n_std = (size_t)L * dim * 2 + dim, n_sub = (size_t)L * (q_dim + hidden);
    if (w_size < w_bytes || s_size < s_count * sizeof(float) || n_size < n_std * sizeof(float)) return EIF_HIP_E_ARG;
    const bool subs = n_size >= (n_std + n_sub) * sizeof(float);
    std::vector<uint8_t> wb;
    std::vector<float> sb, nb;
    try {
        wb.resize(w_bytes);
        sb.resize(s_count);
        nb.resize(subs ? n_std + n_sub : n_std);
    } catch (...) {
        return EIF_HIP_E_NOMEM;
    }
    if (!read_at(file.f, w_off, wb.data(), wb.size()) || !read_at(file.f, s_off, sb.data(), sb.size() * sizeof(float)) ||
        !read_at(file.f, n_off, nb.data(), nb.size() * sizeof(float)))
        return EIF_HIP_E_ARG;

    eif_hip_bitnet_config c{};
    c.dim = dim, c.hidden = hidden, c.n_layers = L, c.n_heads = nh, c.n_kv_heads = nkv, c.head_dim = hd;
    c.vocab = vocab, c.seq_len = seq_len > 0 ? seq_len : file_seq;
    c.rope_theta = theta;
    c.rms_eps = vocab > 120000 ? 1e-6f : 1e-5f;
    c.sub_eps = 1e-5f;
    if (had) {
        c.wht_dim = eif_hadamard_block_size(dim), c.wht_q = eif_hadamard_block_size(q_dim);
        c.wht_hidden = eif_hadamard_block_size(hidden);
        c.wht_norm_dim = eif_hip_wht_norm(c.wht_dim), c.wht_norm_q = eif_hip_wht_norm(c.wht_q);
        c.wht_norm_hidden = eif_hip_wht_norm(c.wht_hidden);
    }
    c.g_q = group_of(dim), c.g_o = group_of(q_dim), c.g_13 = group_of(dim), c.g_2 = group_of(hidden);

    // weights: embedding, then per kind all layers
    const uint8_t *p = wb.data();
    const int8_t *emb = reinterpret_cast<const int8_t *>(p);
    p += (size_t)vocab * dim;
    const uint8_t *wq = p;
    p += (size_t)L * q_dim * dp;
    const uint8_t *wk = p;
    p += (size_t)L * kv_dim * dp;
    const uint8_t *wv = p;
    p += (size_t)L * kv_dim * dp;
    const uint8_t *wo = p;
    p += (size_t)L * dim * qp;
    const uint8_t *w1 = p;
    p += (size_t)L * hidden * dp;
    const uint8_t *w2 = p;
    p += (size_t)L * dim * hp;
    const uint8_t *w3 = p;
    p += (size_t)L * hidden * dp;
    const int8_t *wcls = reinterpret_cast<const int8_t *>(p);
    // scales
    const float *sp = sb.data();
    const float *emb_scale = sp;
    sp += vocab;
    const float *gs[7];   // q, k, v, o, w1, w3, w2: grouped, the kind's first layer; per-row, the layer strides'
    if (rowwise) {
        for (int k = 0; k < 4; ++k) gs[k] = sp + att_off[k];
        sp += (size_t)L * att_stride;
        gs[4] = sp, gs[5] = sp + hidden, gs[6] = sp + 2 * (size_t)hidden;
        sp += (size_t)L * ffn_stride;
    } else {
        for (int k = 0; k < 7; ++k) {
            gs[k] = sp;
            sp += (size_t)L * rows_in[k][0] * ngroups((int)rows_in[k][1]);
        }
    }
    const float *wcls_scale = sp;
    sp += vocab;
    if (interleaved) {   // the decoder rotates half-split pairs: reorder the rows of wq and wk (one scale per row)
        for (int l = 0; l < L; ++l) {
            eif::rope_rows_to_half_split(wb.data() + (wq - wb.data()) + (size_t)l * q_dim * dp, dp,
                                         sb.data() + (gs[0] - sb.data()) + (size_t)l * att_stride, nh, hd);
            eif::rope_rows_to_half_split(wb.data() + (wk - wb.data()) + (size_t)l * kv_dim * dp, dp,
                                         sb.data() + (gs[1] - sb.data()) + (size_t)l * att_stride, nkv, hd);
        }
    }
    const float *sg_dim = had ? sp : nullptr;
    const float *sg_q = had ? sp + dim : nullptr;
    const float *sg_hidden = had ? sp + dim + q_dim : nullptr;
    // norms
    const float *rms_att = nb.data(), *rms_ffn = rms_att + (size_t)L * dim, *rms_final = rms_ffn + (size_t)L * dim;
    const float *sub_att = subs ? rms_final + dim : nullptr;
    const float *sub_ffn = subs ? sub_att + (size_t)L * q_dim : nullptr;

    eif_hip_bitnet *m = nullptr;
    int rc = eif_hip_bitnet_create(&m, &c);
    if (rc) return rc;
    for (int l = 0; l < L && rc == EIF_HIP_OK; ++l) {
        eif_hip_bitnet_layer lw{};
        lw.wq = wq + (size_t)l * q_dim * dp, lw.wk = wk + (size_t)l * kv_dim * dp, lw.wv = wv + (size_t)l * kv_dim * dp;
        lw.wo = wo + (size_t)l * dim * qp, lw.w1 = w1 + (size_t)l * hidden * dp, lw.w3 = w3 + (size_t)l * hidden * dp;
        lw.w2 = w2 + (size_t)l * dim * hp;
        const float **g[7] = {&lw.gq, &lw.gk, &lw.gv, &lw.go, &lw.g1, &lw.g3, &lw.g2};
        for (int k = 0; k < 7; ++k)
            *g[k] = gs[k] + (size_t)l * (rowwise ? (k < 4 ? att_stride : ffn_stride)
                                                 : rows_in[k][0] * ngroups((int)rows_in[k][1]));
        lw.rms_att = rms_att + (size_t)l * dim, lw.rms_ffn = rms_ffn + (size_t)l * dim;
        lw.rms_sub_att = sub_att ? sub_att + (size_t)l * q_dim : nullptr;
        lw.rms_sub_ffn = sub_ffn ? sub_ffn + (size_t)l * hidden : nullptr;
        rc = eif_hip_bitnet_set_layer(m, l, &lw);
    }
    if (rc == EIF_HIP_OK) {
        eif_hip_bitnet_globals gl{};
        gl.emb = emb, gl.emb_scale = emb_scale, gl.rms_final = rms_final;
        gl.signs_dim = sg_dim, gl.signs_q = sg_q, gl.signs_hidden = sg_hidden;
        gl.wcls = wcls, gl.wcls_scale = wcls_scale;
        rc = eif_hip_bitnet_set_globals(m, &gl);
    }
    if (rc) {
        eif_hip_bitnet_destroy(m);
        return rc;
    }
    *out = m;
    return EIF_HIP_OK;
}

// gguf_model.cpp -- BitNet-b1.58 models in GGUF files -> the reference's weight formats in host memory, and from
// there the GPU decoder (eif_hip_gguf.h).
//
// The container is described in gguf_container.h. What is read follows the reference's two passes
// (tinyllm_read_gguf_config, src/eif_tinyllm.c:2843-3009; tinyllm_load_gguf, :3529-3838), with every read
// bounds-checked against the file.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/eif_hip.h"
#include "../../include/eif_hip_gguf.h"
#include "gguf_container.h"

namespace {

using namespace eif::gguf;

// an integer configuration value: u32 / i32 or u64 / i64, as the reference reads them (src/eif_tinyllm.c:2899-2943)
bool read_int(Cursor &c, uint32_t t, int &out)
{
    if (t == 4 || t == 5) out = (int)c.get<uint32_t>();
    else if (t == 10 || t == 11) out = (int)c.get<uint64_t>();
    else return false;
    return c.ok;
}

// bytes of a [rows, cols] tensor of ggml type t as the reference strides it (0: a type it is not read as, or a
// row that is not whole blocks of a type whose rows the reference strides by cols / block)
uint64_t tensor_bytes(int t, uint64_t rows, uint64_t cols)
{
    const uint64_t blocks = (cols + 31) / 32;
    switch (t) {
    case kF32: return rows * cols * 4;
    case kF16: return rows * cols * 2;
    case kQ8_0: return rows * blocks * 34;
    case kTL1: case kTL2: return rows * blocks * 10;
    case kQ4_0: return cols % 32 ? 0 : rows * (cols / 32) * 18;
    case kQ4_1: return cols % 32 ? 0 : rows * (cols / 32) * 20;
    case kQ4_K: return cols % 256 ? 0 : rows * (cols / 256) * 144;
    case kQ6_K: return cols % 256 ? 0 : rows * (cols / 256) * 210;
    default: return 0;
    }
}

// per row: s = max|x| * (1 / 127), q = round-half-away(x * (127 / max|x|)) clamped; s = 1 and q = round(x) when s is
// below 1e-12 (load_embedding_tensor, quantize_row_f32_to_int8, src/eif_tinyllm.c:3258-3349, as the reference's
// -ffast-math build computes the source's s = max / 127 and inv = 1 / s); rows of F32, F16 or Q8_0 / Q4_0 / Q4_1 /
// Q4_K / Q6_K blocks dequantised first
void int8_rows(int type, const uint8_t *src, int rows, int cols, int8_t *q, float *scale)
{
    std::vector<float> x((size_t)cols);
    const size_t blocks = (size_t)(cols + 31) / 32;
    for (int r = 0; r < rows; ++r) {
        if (type == kF32) {
            std::memcpy(x.data(), src + (size_t)r * cols * 4, (size_t)cols * 4);
        } else if (type == kF16) {
            const uint8_t *rs = src + (size_t)r * cols * 2;
            for (int c = 0; c < cols; ++c) {
                uint16_t h;
                std::memcpy(&h, rs + 2 * (size_t)c, 2);
                x[c] = eif::half_to_float(h);
            }
        } else if (type != kQ8_0) {   // Q4_0, Q4_1, Q4_K, Q6_K: rows of whole blocks
            dequant_row(type, src + (size_t)r * tensor_bytes(type, 1, (uint64_t)cols), cols, x.data());
        } else {   // Q8_0: 32-value blocks of an fp16 scale then 32 int8
            const uint8_t *rs = src + (size_t)r * blocks * 34;
            for (size_t b = 0; b < blocks; ++b) {
                uint16_t h;
                std::memcpy(&h, rs + b * 34, 2);
                const float sc = eif::half_to_float(h);
                const int8_t *v = reinterpret_cast<const int8_t *>(rs + b * 34 + 2);
                for (int i = 0; i < 32 && b * 32 + i < (size_t)cols; ++i) x[b * 32 + i] = sc * (float)v[i];
            }
        }
        float amax = 0.0f;
        for (int c = 0; c < cols; ++c) {
            const float a = std::fabs(x[c]);
            if (a > amax) amax = a;
        }
        float s = amax * (1.0f / 127.0f), inv = 1.0f;
        if (s < 1e-12f) s = 1.0f;
        else inv = 127.0f / amax;
        scale[r] = s;
        int8_t *qr = q + (size_t)r * cols;
        for (int c = 0; c < cols; ++c) {
            int v = (int)std::round(x[c] * inv);
            qr[c] = (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v));
        }
    }
}

// Projections of other types ternarized by their absolute mean (load_projection_tensor's BitNet branch,
// src/eif_tinyllm.c:3403-3461): per row gamma = sum |x| * (1 / cols) (1 below 1e-12), code +1 where
// x * (1 / gamma) > 0.5, -1 where < -0.5, else 0. The sum is the one the reference's -ffast-math build forms:
// in column order for F32 / F16 rows, and for rows dequantised from blocks (Q4_0, Q4_1, Q4_K, Q6_K) as eight
// lane sums over columns c = l (mod 8), added pairwise (lanes l and l + 4, then l and l + 2, then 0 and 1).
void absmean_rows(int type, const uint8_t *src, int rows, int cols, uint8_t *codes, float *scales)
{
    std::vector<float> x((size_t)cols);
    const size_t rb = (size_t)(cols + 3) / 4;
    for (int r = 0; r < rows; ++r) {
        dequant_row(type, src + (size_t)r * tensor_bytes(type, 1, (uint64_t)cols), cols, x.data());
        float sum = 0.0f;
        if (type == kF32 || type == kF16) {
            for (int c = 0; c < cols; ++c) sum += std::fabs(x[c]);
        } else {   // cols is a multiple of 32
            float lane[8] = {};
            for (int c = 0; c < cols; c += 8)
                for (int l = 0; l < 8; ++l) lane[l] += std::fabs(x[c + l]);
            for (int w = 4; w >= 1; w >>= 1)
                for (int l = 0; l < w; ++l) lane[l] += lane[l + w];
            sum = lane[0];
        }
        float gamma = sum * (1.0f / (float)cols);
        if (gamma < 1e-12f) gamma = 1.0f;
        scales[r] = gamma;
        const float inv = 1.0f / gamma;
        uint8_t *o = codes + (size_t)r * rb;
        std::memset(o, 0, rb);
        for (int c = 0; c < cols; ++c) {
            const float v = x[c] * inv;
            const uint8_t code = v > 0.5f ? 1 : (v < -0.5f ? 2 : 0);
            o[c / 4] |= (uint8_t)(code << ((c % 4) * 2));
        }
    }
}

}  // namespace

// kinds in the order of eif_hip_bitnet_layer: q, k, v, o, w1 (gate), w3 (up), w2 (down)
struct eif_gguf_bitnet {
    eif_gguf_bitnet_info info{};
    std::vector<uint8_t> codes[7];
    std::vector<float> scales[7];
    std::vector<int8_t> emb, head;
    std::vector<float> emb_scale, head_scale, rms_att, rms_ffn, rms_final;
    size_t rows[7] = {}, row_bytes[7] = {};
};

namespace {

int open_model(eif_gguf_bitnet &m, const char *path)
{
    Mapped f;
    if (!f.open(path)) return EIF_HIP_E_ARG;
    Cursor c{f.p, f.n};
    const uint32_t magic = c.get<uint32_t>(), version = c.get<uint32_t>();
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (!c.ok || magic != kMagic || n_tensors == 0 || n_tensors > f.n / 24 || n_kv > f.n / 12)
        return EIF_HIP_E_ARG;
    eif_gguf_bitnet_info &in = m.info;
    in.version = version;
    in.alignment = 32;
    std::string key_arch = "llama", arch;   // the key prefix: the architecture read so far
    bool has_arch = false;
    float theta = 0.0f;
    int dim = 0, hidden = 0, L = 0, nh = 0, nkv = 0, hd = 0, seq = 0, vocab = 0;
    for (uint64_t i = 0; i < n_kv && c.ok; ++i) {
        const std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        if (!c.ok) break;
        const std::string pre = key_arch + ".";
        if (key == "general.architecture" && t == 8) {
            arch = c.str().substr(0, 63);
            key_arch = arch, has_arch = true;
        } else if (key == "general.alignment") {
            int a = 0;
            if (!(t == 4 || t == 5) || !read_int(c, t, a) || a <= 0 || (a & (a - 1))) return EIF_HIP_E_ARG;
            in.alignment = (uint32_t)a;
        } else if (key == pre + "embedding_length") {
            if (!read_int(c, t, dim)) return EIF_HIP_E_ARG;
        } else if (key == pre + "feed_forward_length") {
            if (!read_int(c, t, hidden)) return EIF_HIP_E_ARG;
        } else if (key == pre + "block_count") {
            if (!read_int(c, t, L)) return EIF_HIP_E_ARG;
        } else if (key == pre + "attention.head_count") {
            if (!read_int(c, t, nh)) return EIF_HIP_E_ARG;
        } else if (key == pre + "attention.head_count_kv") {
            if (!read_int(c, t, nkv)) return EIF_HIP_E_ARG;
        } else if (key == pre + "context_length") {
            if (!read_int(c, t, seq)) return EIF_HIP_E_ARG;
        } else if (key.find("rope.freq_base") != std::string::npos ||
                   key.find("rope_freq_base") != std::string::npos) {
            if (t == 6) theta = c.get<float>();
            else if (t == 12) theta = (float)c.get<double>();
            else if (t == 4 || t == 5) theta = (float)c.get<uint32_t>();
            else if (t == 10 || t == 11) theta = (float)c.get<uint64_t>();
            else return EIF_HIP_E_ARG;
        } else if (key == pre + "attention.key_length") {
            if (!read_int(c, t, hd)) return EIF_HIP_E_ARG;
        } else if (key == "tokenizer.ggml.tokens" && t == 9) {
            const uint32_t et = c.get<uint32_t>();
            const uint64_t count = c.get<uint64_t>();
            if (!c.ok || count > (uint64_t)0x7fffffff) return EIF_HIP_E_ARG;
            vocab = (int)count;
            if (const int s = scalar_size(et)) {
                if (count > (c.n - c.at) / (uint64_t)s) return EIF_HIP_E_ARG;
                c.skip(count * (uint64_t)s);
            } else {
                for (uint64_t k = 0; k < count && c.ok; ++k) skip_value(c, et, 1);
            }
        } else {
            skip_value(c, t);
        }
    }
    // the tensor table
    std::vector<std::string> names;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> index;   // the first tensor of a name, as the reference's search
    try {
        const size_t hint = n_tensors < 4096 ? (size_t)n_tensors : 4096;   // the table itself bounds the rest
        names.reserve(hint), tensors.reserve(hint);
        for (uint64_t i = 0; i < n_tensors && c.ok; ++i) {
            Tensor t;
            names.push_back(c.str());
            t.n_dims = c.get<uint32_t>();
            if (!c.ok || t.n_dims == 0 || t.n_dims > 4) return EIF_HIP_E_ARG;
            for (uint32_t d = 0; d < t.n_dims; ++d) t.ne[d] = c.get<uint64_t>();
            t.type = c.get<uint32_t>();
            t.offset = c.get<uint64_t>();
            tensors.push_back(t);
            index.emplace(names.back(), tensors.size() - 1);
        }
    } catch (...) {
        return EIF_HIP_E_NOMEM;
    }
    if (!c.ok) return EIF_HIP_E_ARG;
    const size_t data = (c.at + in.alignment - 1) & ~(size_t)(in.alignment - 1);
    if (data > f.n) return EIF_HIP_E_ARG;

    // configuration (src/eif_tinyllm.c:2984-3007)
    if (nkv == 0) nkv = nh;
    if (hd == 0 && nh > 0) hd = dim / nh;
    if (seq <= 0) seq = 2048;
    if (seq > 4096) seq = 4096;
    if (theta <= 0.0f)
        theta = (key_arch.find("qwen") != std::string::npos || std::strstr(path, "qwen")) ? 1000000.0f : 10000.0f;
    if (dim <= 0 || hidden <= 0 || L <= 0 || nh <= 0 || nkv <= 0 || hd <= 0 || vocab <= 0 || hd % 2 || L > 4096 ||
        (int64_t)nh * hd > (1 << 30) || (int64_t)nkv * hd > (1 << 30) || dim > (1 << 30) || hidden > (1 << 30))
        return EIF_HIP_E_ARG;
    std::snprintf(in.arch, sizeof(in.arch), "%s", has_arch ? arch.c_str() : "");
    in.dim = dim, in.hidden = hidden, in.n_layers = L, in.n_heads = nh, in.n_kv_heads = nkv, in.head_dim = hd;
    in.vocab = vocab, in.seq_len = seq, in.rope_theta = theta;
    in.rope_interleaved = has_arch && (arch == "llama" || arch == "granite" || arch == "minicpm" || arch == "smollm");

    auto find = [&](const std::string &name) -> const Tensor * {
        const auto it = index.find(name);
        return it == index.end() ? nullptr : &tensors[it->second];
    };
    // the tensor's bytes, when it is [rows, cols] of a type the reference reads and lies inside the file
    auto bytes_of = [&](const Tensor *t, uint64_t rows, uint64_t cols) -> const uint8_t * {
        uint64_t outer = 1;
        for (uint32_t d = 1; d < t->n_dims; ++d) outer *= t->ne[d];
        const uint64_t sz = tensor_bytes((int)t->type, rows, cols);
        if (t->ne[0] != cols || outer != rows || sz == 0 || t->offset > f.n - data || sz > f.n - data - t->offset)
            return nullptr;
        return f.p + data + t->offset;
    };
    // the probe projection decides BitNet (src/eif_tinyllm.c:3637-3662)
    const Tensor *probe = find("blk.0.attn_q.weight");
    if (!probe) probe = find("blk.0.ffn_down.weight");
    uint32_t ptype = 0;
    if (probe) {
        ptype = probe->type;
    } else {
        for (size_t i = 0; i < tensors.size(); ++i)
            if (names[i].find("blk.0.") != std::string::npos && names[i].find(".weight") != std::string::npos) {
                ptype = tensors[i].type;
                if (ptype != kF32 && ptype != kF16) break;
            }
    }
    if (ptype != kTL1 && ptype != kTL2) return EIF_HIP_E_ARG;
    in.proj_type = (int)ptype;
    if (find("blk.0.attn_q.bias")) return EIF_HIP_E_ARG;   // the decoder has no Q/K/V biases

    const int q_dim = nh * hd, kv_dim = nkv * hd;
    const size_t shape[7][2] = {{(size_t)q_dim, (size_t)dim}, {(size_t)kv_dim, (size_t)dim},
                                {(size_t)kv_dim, (size_t)dim}, {(size_t)dim, (size_t)q_dim},
                                {(size_t)hidden, (size_t)dim}, {(size_t)hidden, (size_t)dim},
                                {(size_t)dim, (size_t)hidden}};
    const char *kind_name[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
    // every tensor is found and lies inside the file before anything is allocated, so the arrays below stay
    // within a small multiple of the file's size whatever the metadata says
    char name[160];
    std::vector<std::pair<const Tensor *, const uint8_t *>> proj((size_t)L * 7);
    for (int l = 0; l < L; ++l) {
        for (int k = 0; k < 7; ++k) {
            std::snprintf(name, sizeof(name), "blk.%d.%s.weight", l, kind_name[k]);
            const Tensor *t = find(name);
            if (!t && k == 3) {
                std::snprintf(name, sizeof(name), "blk.%d.attn_out.weight", l);
                t = find(name);
            }
            const uint8_t *src = t ? bytes_of(t, shape[k][0], shape[k][1]) : nullptr;
            if (!src) return EIF_HIP_E_ARG;
            proj[(size_t)l * 7 + k] = {t, src};
        }
    }
    const Tensor *te = find("token_embd.weight"), *th = find("output.weight");
    if (!th) th = find("lm_head.weight");
    if (!te || !bytes_of(te, (uint64_t)vocab, (uint64_t)dim) || (th && !bytes_of(th, (uint64_t)vocab, (uint64_t)dim)))
        return EIF_HIP_E_ARG;
    try {
        for (int k = 0; k < 7; ++k) {
            m.rows[k] = shape[k][0], m.row_bytes[k] = (shape[k][1] + 3) / 4;
            m.codes[k].assign((size_t)L * m.rows[k] * m.row_bytes[k], 0);
            m.scales[k].assign((size_t)L * m.rows[k], 0.0f);
        }
        m.rms_att.assign((size_t)L * dim, 1.0f), m.rms_ffn.assign((size_t)L * dim, 1.0f);
        m.rms_final.assign((size_t)dim, 1.0f);
        m.emb.resize((size_t)vocab * dim), m.emb_scale.resize(vocab);
    } catch (...) {
        return EIF_HIP_E_NOMEM;
    }
    for (int l = 0; l < L; ++l) {
        for (int k = 0; k < 7; ++k) {
            const Tensor *t = proj[(size_t)l * 7 + k].first;
            const uint8_t *src = proj[(size_t)l * 7 + k].second;
            uint8_t *codes = m.codes[k].data() + (size_t)l * m.rows[k] * m.row_bytes[k];
            float *scales = m.scales[k].data() + (size_t)l * m.rows[k];
            if (t->type == kTL1 || t->type == kTL2 || t->type == kQ8_0) {
                const int rc = eif_gguf_ternary_rows((int)t->type, src, (int)shape[k][0], (int)shape[k][1], codes,
                                                     scales);
                if (rc) return rc;
            } else {   // F32, F16, Q4_0, Q4_1, Q4_K, Q6_K (bytes_of has taken only these, in whole blocks)
                absmean_rows((int)t->type, src, (int)shape[k][0], (int)shape[k][1], codes, scales);
            }
        }
    }
    // norms (load_rmsnorm, src/eif_tinyllm.c:3112-3130): F32 / F16; absent or another type -> 1
    auto norm = [&](const char *nm, float *dst) -> bool {
        const Tensor *t = find(nm);
        if (!t || (t->type != kF32 && t->type != kF16)) return true;
        const uint8_t *src = bytes_of(t, 1, (uint64_t)dim);
        if (!src) return false;
        for (int i = 0; i < dim; ++i) {
            if (t->type == kF32) {
                std::memcpy(&dst[i], src + 4 * (size_t)i, 4);
            } else {
                uint16_t h;
                std::memcpy(&h, src + 2 * (size_t)i, 2);
                dst[i] = eif::half_to_float(h);
            }
        }
        return true;
    };
    for (int l = 0; l < L; ++l) {
        std::snprintf(name, sizeof(name), "blk.%d.attn_norm.weight", l);
        if (!norm(name, &m.rms_att[(size_t)l * dim])) return EIF_HIP_E_ARG;
        std::snprintf(name, sizeof(name), "blk.%d.ffn_norm.weight", l);
        if (!norm(name, &m.rms_ffn[(size_t)l * dim])) return EIF_HIP_E_ARG;
    }
    if (!norm(find("output_norm.weight") ? "output_norm.weight" : "norm.weight", m.rms_final.data()))
        return EIF_HIP_E_ARG;
    // embedding and head
    auto int8_tensor = [&](const Tensor *t, std::vector<int8_t> &q, std::vector<float> &s) -> int {
        const uint8_t *src = t ? bytes_of(t, (uint64_t)vocab, (uint64_t)dim) : nullptr;
        const bool ok = t && (t->type == kF32 || t->type == kF16 || t->type == kQ8_0 || t->type == kQ4_0 ||
                              t->type == kQ4_1 || t->type == kQ4_K || t->type == kQ6_K);
        if (!src || !ok) return EIF_HIP_E_ARG;
        try {
            q.resize((size_t)vocab * dim), s.resize(vocab);
        } catch (...) {
            return EIF_HIP_E_NOMEM;
        }
        int8_rows((int)t->type, src, vocab, dim, q.data(), s.data());
        return EIF_HIP_OK;
    };
    int rc = int8_tensor(te, m.emb, m.emb_scale);
    if (rc) return rc;
    in.emb_type = (int)te->type;
    in.head_type = th ? (int)th->type : -1;
    if (th && (rc = int8_tensor(th, m.head, m.head_scale))) return rc;
    return EIF_HIP_OK;
}

}  // namespace

extern "C" int eif_gguf_bitnet_open(eif_gguf_bitnet **out, const char *path)
{
    if (!out || !path) return EIF_HIP_E_ARG;
    *out = nullptr;
    eif_gguf_bitnet *m = new (std::nothrow) eif_gguf_bitnet;
    if (!m) return EIF_HIP_E_NOMEM;
    int rc;
    try {
        rc = open_model(*m, path);
    } catch (...) {   // allocation failures of the host-side bookkeeping
        rc = EIF_HIP_E_NOMEM;
    }
    if (rc) {
        delete m;
        return rc;
    }
    *out = m;
    return EIF_HIP_OK;
}

extern "C" void eif_gguf_bitnet_close(eif_gguf_bitnet *m) { delete m; }

extern "C" int eif_gguf_bitnet_get_info(const eif_gguf_bitnet *m, eif_gguf_bitnet_info *info)
{
    if (!m || !info) return EIF_HIP_E_ARG;
    *info = m->info;
    return EIF_HIP_OK;
}

extern "C" int eif_gguf_bitnet_get_layer(const eif_gguf_bitnet *m, int l, eif_hip_bitnet_layer *lw)
{
    if (!m || !lw || l < 0 || l >= m->info.n_layers) return EIF_HIP_E_ARG;
    *lw = eif_hip_bitnet_layer{};
    const uint8_t **w[7] = {&lw->wq, &lw->wk, &lw->wv, &lw->wo, &lw->w1, &lw->w3, &lw->w2};
    const float **g[7] = {&lw->gq, &lw->gk, &lw->gv, &lw->go, &lw->g1, &lw->g3, &lw->g2};
    for (int k = 0; k < 7; ++k) {
        *w[k] = m->codes[k].data() + (size_t)l * m->rows[k] * m->row_bytes[k];
        *g[k] = m->scales[k].data() + (size_t)l * m->rows[k];
    }
    lw->rms_att = m->rms_att.data() + (size_t)l * m->info.dim;
    lw->rms_ffn = m->rms_ffn.data() + (size_t)l * m->info.dim;
    return EIF_HIP_OK;
}

extern "C" int eif_gguf_bitnet_get_globals(const eif_gguf_bitnet *m, eif_hip_bitnet_globals *g)
{
    if (!m || !g) return EIF_HIP_E_ARG;
    *g = eif_hip_bitnet_globals{};
    g->emb = m->emb.data(), g->emb_scale = m->emb_scale.data(), g->rms_final = m->rms_final.data();
    const bool tied = m->head.empty();
    g->wcls = tied ? m->emb.data() : m->head.data();
    g->wcls_scale = tied ? m->emb_scale.data() : m->head_scale.data();
    return EIF_HIP_OK;
}

extern "C" int eif_hip_bitnet_load_gguf(eif_hip_bitnet **out, const char *path, int seq_len)
{
    if (!out || !path) return EIF_HIP_E_ARG;
    *out = nullptr;
    eif_gguf_bitnet *m = nullptr;
    int rc = eif_gguf_bitnet_open(&m, path);
    if (rc) return rc;
    const eif_gguf_bitnet_info &in = m->info;
    if (in.rope_interleaved) {
        for (int l = 0; l < in.n_layers; ++l)
            for (int k = 0; k < 2; ++k)   // q (n_heads heads), k (n_kv_heads heads)
                eif::rope_rows_to_half_split(m->codes[k].data() + (size_t)l * m->rows[k] * m->row_bytes[k],
                                             m->row_bytes[k], m->scales[k].data() + (size_t)l * m->rows[k],
                                             k == 0 ? in.n_heads : in.n_kv_heads, in.head_dim);
    }
    eif_hip_bitnet_config c{};
    c.dim = in.dim, c.hidden = in.hidden, c.n_layers = in.n_layers, c.n_heads = in.n_heads;
    c.n_kv_heads = in.n_kv_heads, c.head_dim = in.head_dim, c.vocab = in.vocab;
    c.seq_len = seq_len > 0 ? seq_len : in.seq_len;
    c.rope_theta = in.rope_theta;
    c.rms_eps = in.vocab > 120000 ? 1e-6f : 1e-5f;
    c.sub_eps = 1e-5f;
    eif_hip_bitnet *gm = nullptr;
    rc = eif_hip_bitnet_create(&gm, &c);
    for (int l = 0; l < in.n_layers && rc == EIF_HIP_OK; ++l) {
        eif_hip_bitnet_layer lw;
        eif_gguf_bitnet_get_layer(m, l, &lw);
        rc = eif_hip_bitnet_set_layer(gm, l, &lw);
    }
    if (rc == EIF_HIP_OK) {
        eif_hip_bitnet_globals g;
        eif_gguf_bitnet_get_globals(m, &g);
        rc = eif_hip_bitnet_set_globals(gm, &g);
    }
    eif_gguf_bitnet_close(m);
    if (rc) {
        eif_hip_bitnet_destroy(gm);
        return rc;
    }
    *out = gm;
    return EIF_HIP_OK;
}

/*
 * ref_tinyllm_wrap.c -- TEST INFRASTRUCTURE. Builds the reference's own BitNet tinyllm model (include/eif_tinyllm.h,
 * the in-memory construction of tests/test_seq_bounds.c:11-26) from the oracle's weight arrays and runs its decode
 * (tinyllm_forward, src/eif_tinyllm.c:1502-1506). Compiled together with the reference sources into oracle/_ref/.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "eif_tinyllm.h"
#include "oracle.h"

typedef struct {
    tinyllm_t llm;
    void *pool;
    float *ones;
    void *wbuf;
} ref_bitnet;

/* bitnet_group: the reference's one group bound for all matrices (eif_bitnet_group_size per input width). */
void *ref_bitnet_create(const orc_bitnet_cfg *c, const orc_bitnet_weights *w, int bitnet_group)
{
    ref_bitnet *r = (ref_bitnet *)calloc(1, sizeof(ref_bitnet));
    if (!r) return NULL;
    tinyllm_config_t cfg;
    memset(&cfg, 0, sizeof(cfg));
    cfg.dim = c->dim;
    cfg.hidden_dim = c->hidden;
    cfg.n_layers = c->n_layers;
    cfg.n_heads = c->n_heads;
    cfg.n_kv_heads = c->n_kv_heads;
    cfg.vocab_size = c->vocab;
    cfg.seq_len = c->seq_len;
    cfg.qtype = TINYLLM_QTYPE_BITNET_158;
    cfg.head_dim = c->head_dim;
    cfg.rope_theta = c->rope_theta;
    cfg.bitnet_group = bitnet_group;
    cfg.bitnet_hadamard = 1;
    const size_t sz = tinyllm_memory_size(&cfg);
    r->pool = malloc(sz);
    const int big = c->dim * 4 + c->hidden * 3 + c->n_heads * c->head_dim * 4;
    r->ones = (float *)malloc(sizeof(float) * (size_t)big * c->n_layers);
    if (!r->pool || !r->ones || tinyllm_init(&r->llm, &cfg, r->pool, sz) != 0) {
        free(r->pool), free(r->ones), free(r);
        return NULL;
    }
    for (int i = 0; i < big * c->n_layers; i++) r->ones[i] = 1.0f;
    tinyllm_weights_t *tw = &r->llm.weights;
    tw->token_embedding = (void *)w->emb;
    tw->token_embedding_scale = (float *)w->emb_scale;
    tw->rms_att_weight = (float *)w->rms_att;
    tw->rms_ffn_weight = (float *)w->rms_ffn;
    tw->rms_sub_att_weight = (float *)w->rms_sub_att;
    tw->rms_sub_ffn_weight = (float *)w->rms_sub_ffn;
    tw->rms_final_weight = (float *)w->rms_final;
    tw->wq = (void *)w->wq, tw->wk = (void *)w->wk, tw->wv = (void *)w->wv, tw->wo = (void *)w->wo;
    tw->w1 = (void *)w->w1, tw->w2 = (void *)w->w2, tw->w3 = (void *)w->w3;
    tw->attn_scale = r->ones;   /* row scales: unused with grouped scales */
    tw->ffn_scale = r->ones;
    tw->bitnet_gscale[TL_BN_WQ] = w->gq, tw->bitnet_gscale[TL_BN_WK] = w->gk, tw->bitnet_gscale[TL_BN_WV] = w->gv;
    tw->bitnet_gscale[TL_BN_WO] = w->go, tw->bitnet_gscale[TL_BN_W1] = w->g1, tw->bitnet_gscale[TL_BN_W3] = w->g3;
    tw->bitnet_gscale[TL_BN_W2] = w->g2;
    tw->had_signs_dim = w->signs_dim, tw->had_signs_q = w->signs_q, tw->had_signs_hidden = w->signs_hidden;
    tw->wcls = (void *)w->wcls;
    tw->wcls_scale = (float *)w->wcls_scale;
    return r;
}

float *ref_bitnet_forward(void *h, int token, int pos) { return tinyllm_forward(&((ref_bitnet *)h)->llm, token, pos); }

/* Fills the FP32 KV cache of positions 0 .. npos - 1 of every layer with synthetic values (a fixed 32-bit LCG
 * mapped to [-1, 1)), so that tinyllm_forward at position npos reads a full cache of that length without the
 * npos steps before it. For timing only: the values are not those of a prompt. The cache layout is the one
 * tinyllm_forward indexes, [layer][seq_len][n_kv_heads * head_dim] (src/eif_tinyllm.c:415-418). Returns 0, or
 * -1 when npos is outside 0 .. seq_len or the model keeps an INT8 cache. */
int ref_bitnet_fill_cache(void *h, int npos)
{
    ref_bitnet *r = (ref_bitnet *)h;
    const tinyllm_config_t *p = &r->llm.config;
    tinyllm_state_t *s = &r->llm.state;
    if (npos < 0 || npos > p->seq_len || p->kv_type != 0 || !s->key_cache || !s->value_cache) return -1;
    const size_t kv_dim = (size_t)p->n_kv_heads * (size_t)(p->head_dim > 0 ? p->head_dim : p->dim / p->n_heads);
    uint32_t st = 12345u;
    for (int l = 0; l < p->n_layers; l++) {
        const size_t loff = (size_t)l * p->seq_len * kv_dim;
        for (size_t i = 0; i < (size_t)npos * kv_dim; i++) {
            st = st * 1664525u + 1013904223u;
            s->key_cache[loff + i] = (float)(st >> 8) * (2.0f / 16777216.0f) - 1.0f;
            st = st * 1664525u + 1013904223u;
            s->value_cache[loff + i] = (float)(st >> 8) * (2.0f / 16777216.0f) - 1.0f;
        }
    }
    return 0;
}

void ref_bitnet_destroy(void *h)
{
    ref_bitnet *r = (ref_bitnet *)h;
    if (!r) return;
    free(r->pool), free(r->ones), free(r->wbuf), free(r);
}

/* A BitNet model file in the SVLM layout read by the reference itself: the configuration words as its engine
 * reads them (src/eif_llm.c:321-342), tinyllm_init, then tinyllm_load_quantized_model (src/eif_tinyllm.c:2442)
 * into a weight buffer, as src/eif_llm.c:343-395 does. Returns a handle for ref_bitnet_forward / _destroy. */
void *ref_svlm_create(const char *path)
{
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    uint32_t hdr[12];
    int32_t ci[32];
    const int ok = fread(hdr, 4, 12, f) == 12 && fseek(f, 48, SEEK_SET) == 0 && fread(ci, 4, 32, f) == 32;
    fclose(f);
    if (!ok || hdr[0] != 0x53564C4Du) return NULL;
    tinyllm_config_t cfg;
    memset(&cfg, 0, sizeof(cfg));
    cfg.dim = ci[0], cfg.hidden_dim = ci[1], cfg.n_layers = ci[2], cfg.n_heads = ci[3], cfg.n_kv_heads = ci[4];
    cfg.head_dim = ci[5], cfg.vocab_size = ci[6], cfg.seq_len = ci[7] > 0 ? ci[7] : 512;
    cfg.rope_theta = 100000.0f;
    cfg.qtype = ci[12] == 3 ? TINYLLM_QTYPE_BITNET_158 : (tinyllm_qtype_t)ci[12];
    cfg.bitnet_group = ci[14];
    cfg.bitnet_hadamard = ci[15];
    ref_bitnet *r = (ref_bitnet *)calloc(1, sizeof(ref_bitnet));
    if (!r) return NULL;
    const size_t sz = tinyllm_memory_size(&cfg), wsz = (size_t)hdr[7] + hdr[8] + hdr[9];
    r->pool = malloc(sz);
    r->wbuf = malloc(wsz);
    if (!r->pool || !r->wbuf || tinyllm_init(&r->llm, &cfg, r->pool, sz) != 0 ||
        tinyllm_load_quantized_model(&r->llm, path, r->wbuf, wsz) != 0) {
        free(r->pool), free(r->wbuf), free(r);
        return NULL;
    }
    return r;
}

/* A BitNet model from a TTML / TLLM file, configured as the reference's engine reads that format
 * (src/eif_llm.c:341-351: tinyllm_config_t after the 36-byte header, up to the BitNet group fields) and loaded by
 * its own tinyllm_load_quantized_model. */
void *ref_ttml_create(const char *path)
{
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    uint32_t magic = 0;
    tinyllm_config_t cfg;
    memset(&cfg, 0, sizeof(cfg));
    const int ok = fread(&magic, 4, 1, f) == 1 && fseek(f, 36, SEEK_SET) == 0 &&
                   fread(&cfg, offsetof(tinyllm_config_t, bitnet_group), 1, f) == 1;
    if (!ok || (magic != 0x54544D4Cu && magic != 0x544C4C4Du)) {
        fclose(f);
        return NULL;
    }
    uint32_t hdr[9];
    fseek(f, 0, SEEK_SET);
    const int ok2 = fread(hdr, 4, 9, f) == 9;
    fclose(f);
    if (!ok2) return NULL;
    ref_bitnet *r = (ref_bitnet *)calloc(1, sizeof(ref_bitnet));
    if (!r) return NULL;
    const size_t sz = tinyllm_memory_size(&cfg), wsz = (size_t)hdr[3] + hdr[4] + hdr[5];
    r->pool = malloc(sz);
    r->wbuf = malloc(wsz);
    if (!r->pool || !r->wbuf || tinyllm_init(&r->llm, &cfg, r->pool, sz) != 0 ||
        tinyllm_load_quantized_model(&r->llm, path, r->wbuf, wsz) != 0) {
        free(r->pool), free(r->wbuf), free(r);
        return NULL;
    }
    return r;
}

/* A GGUF causal model read by the reference itself, as its engine does (src/eif_llm.c:312-319, :370-389):
 * tinyllm_read_gguf_config, tinyllm_init, then tinyllm_load_gguf (src/eif_tinyllm.c:3529) into a zeroed weight
 * buffer (so regions the loader leaves unwritten compare as zeros). */
void *ref_gguf_create(const char *path)
{
    tinyllm_config_t cfg;
    char arch[64] = {0};
    if (tinyllm_read_gguf_config(path, &cfg, arch, sizeof(arch)) != 0) return NULL;
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    const long fsize = ftell(f);
    fclose(f);
    ref_bitnet *r = (ref_bitnet *)calloc(1, sizeof(ref_bitnet));
    if (!r) return NULL;
    const size_t sz = tinyllm_memory_size(&cfg);
    const size_t wsz = (size_t)fsize * 8 + (size_t)cfg.vocab_size * cfg.dim * 2 + ((size_t)16 << 20);
    r->pool = malloc(sz);
    r->wbuf = calloc(1, wsz);
    if (!r->pool || !r->wbuf || tinyllm_init(&r->llm, &cfg, r->pool, sz) != 0 ||
        tinyllm_load_gguf(&r->llm, path, r->wbuf, wsz) != 0) {
        free(r->pool), free(r->wbuf), free(r);
        return NULL;
    }
    return r;
}

/* A loaded model's configuration (cfg[0..9]: dim, hidden, layers, heads, kv heads, head_dim, vocab, seq_len,
 * qtype, rope_interleaved; *theta) and weight pointers (ptrs[0..18]: token_embedding, its scale, wq, wk, wv, wo,
 * w1, w2, w3, attn_scale, ffn_scale, rms_att, rms_ffn, rms_final, wcls, wcls_scale, rms_sub_att, rms_sub_ffn,
 * bq), as the decode reads them. */
int ref_tinyllm_view(void *h, int *cfg, float *theta, const void **ptrs)
{
    const tinyllm_t *t = &((ref_bitnet *)h)->llm;
    const tinyllm_config_t *c = &t->config;
    const tinyllm_weights_t *w = &t->weights;
    const int v[10] = {c->dim, c->hidden_dim, c->n_layers, c->n_heads, c->n_kv_heads, c->head_dim, c->vocab_size,
                       c->seq_len, (int)c->qtype, c->rope_interleaved};
    memcpy(cfg, v, sizeof(v));
    *theta = c->rope_theta;
    const void *p[19] = {w->token_embedding, w->token_embedding_scale, w->wq, w->wk, w->wv, w->wo, w->w1, w->w2,
                         w->w3, w->attn_scale, w->ffn_scale, w->rms_att_weight, w->rms_ffn_weight,
                         w->rms_final_weight, w->wcls, w->wcls_scale, w->rms_sub_att_weight, w->rms_sub_ffn_weight,
                         w->bq};
    memcpy(ptrs, p, sizeof(p));
    return 0;
}

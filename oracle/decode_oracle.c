/*
 * decode_oracle.c -- CPU restatement of one BitNet-b1.58 decoder step. TEST INFRASTRUCTURE ONLY: used by
 * tests/, smoke() and bench.py's CPU leg as the checker of the GPU decode, never by the product library.
 *
 * Follows tinyllm_forward_embedding_ex, BitNet path (src/eif_tinyllm.c:371-857):
 *   x = embedding[token] * scale[token]                   (src/eif_tinyllm.c:902-916, INT8 table)
 *   per layer l:
 *     xb = rmsnorm(x, rms_att[l], eps)                    (:410-411; rmsnorm :319-330: (x * (1/sqrtf(ss/n + eps))) * w)
 *     q, k, v = linear(xb, signs_dim)                     (:450-459, tl_bitnet_rotate + tl_bitnet_mm :66-86)
 *     RoPE, half-split pairs (j, j + head_dim/2)          (:396-405 tables, :476-507)
 *     k, v appended to the cache at pos
 *     per head: att = softmax(q . k_t / sqrtf(head_dim)), out = sum_t att_t v_t   (:555-650, softmax :334-352)
 *     xb = rmsnorm(out, rms_sub_att[l], 1e-5); x += linear(xb, signs_q)          (:659-668, :680-701)
 *     xb = rmsnorm(x, rms_ffn[l], eps); h1, h3 = linear(xb, signs_dim)           (:703, :724-733)
 *     h = (h1 * (1 / (1 + expf(-h1)))) * h3                                      (:774-780, the scalar form)
 *     h = rmsnorm(h, rms_sub_ffn[l], 1e-5); x += linear(h, signs_hidden)         (:792-800, :805-825)
 *   logits = head(rmsnorm(x, rms_final, eps))            (:827-848)
 *
 * Two forms of the linears:
 *   ORC_LIN_INT8 (the GPU contract): prep = signs, blockwise WHT, per-row absmax INT8 (orc_prep_rows); ternary
 *     grouped GEMV on the int8 row (orc_ternary_gemv_grouped); INT8 head on the int8 row
 *     (orc_int8_gemv_i8act); KV cache values rounded to fp16.
 *   ORC_LIN_F32 (the reference's x86 engine): in-place rotation (orc_hadamard_rotate) and the FP32-activation
 *     grouped GEMV (orc_matmul_bitnet_block_f32, src/eif_quantize_bitnet.c:1227-1420); FP32 head
 *     (orc_int8_rowscale_f32, src/eif_tinyllm.c:1863-1874); FP32 KV cache.
 * Pinned in tests against the reference's own tinyllm decode compiled from its sources (ORC_LIN_F32).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static void orc_rmsnorm(float *out, const float *x, const float *w, int n, float eps)
{
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    ss = ss / (float)n + eps;
    ss = 1.0f / sqrtf(ss);
    for (int i = 0; i < n; i++) out[i] = x[i] * ss * (w ? w[i] : 1.0f);
}

/* v rounded to the nearest IEEE binary16 value, ties to even (the GPU's fp32 -> fp16 conversion), as a float:
 * the spacing at v is 2^(e - 10) for normal binary16 values (e = the binary exponent of v) and 2^-24 below
 * 2^-14; magnitudes from 65520 round to infinity. */
float orc_round_f16(float v)
{
    if (!isfinite(v)) return v;
    const float av = fabsf(v);
    if (av >= 65520.0f) return copysignf(INFINITY, v);
    if (av == 0.0f) return v;
    int e;
    (void)frexpf(av, &e);   /* av = m * 2^e, m in [0.5, 1): binary exponent e - 1 */
    const int qe = (e - 1) < -14 ? -24 : (e - 1) - 10;
    const float r = ldexpf(rintf(ldexpf(av, -qe)), qe);
    return copysignf(r, v);
}

/* y[rows] = linear(x[cols]); x is not modified. */
static int orc_linear(int mode, const uint8_t *w, const float *gs, int group, const float *x, const float *signs,
                      int block, float norm, float *y, int rows, int cols)
{
    if (mode == ORC_LIN_INT8) {
        const int kpad = cols;
        int8_t *xq = (int8_t *)malloc((size_t)kpad);
        float xs = 0.0f;
        if (!xq) return -1;
        if (orc_prep_rows(x, cols, signs, 1, cols, block, norm, xq, kpad, &xs, NULL, 0) != 0) {
            free(xq);
            return -1;
        }
        orc_ternary_gemv_grouped(w, gs, group, xq, kpad, &xs, NULL, y, rows, 1, rows, cols);
        free(xq);
        return 0;
    }
    float *t = (float *)malloc(sizeof(float) * (size_t)cols);
    if (!t) return -1;
    memcpy(t, x, sizeof(float) * (size_t)cols);
    if (block > 0 && orc_hadamard_rotate(t, signs, cols, block, norm) != 0) {
        free(t);
        return -1;
    }
    orc_matmul_bitnet_block_f32(w, gs, group, t, NULL, y, rows, cols);
    free(t);
    return 0;
}

int orc_bitnet_forward(const orc_bitnet_cfg *c, const orc_bitnet_weights *w, float *kcache, float *vcache,
                       int token, int pos, int mode, float *logits)
{
    if (!c || !w || token < 0 || token >= c->vocab || pos < 0 || pos >= c->seq_len) return -1;
    const int dim = c->dim, hid = c->hidden, hd = c->head_dim, half = hd / 2;
    const int q_dim = c->n_heads * hd, kv_dim = c->n_kv_heads * hd, kv_mul = c->n_heads / c->n_kv_heads;
    const int dp = (dim + 3) / 4, qp = (q_dim + 3) / 4, hp = (hid + 3) / 4;
    const int gq = (dim + c->g_q - 1) / c->g_q, go = (q_dim + c->g_o - 1) / c->g_o;
    const int g13 = (dim + c->g_13 - 1) / c->g_13, g2 = (hid + c->g_2 - 1) / c->g_2;
    float *x = (float *)malloc(sizeof(float) * dim), *xb = (float *)malloc(sizeof(float) * (q_dim > dim ? q_dim : dim));
    float *q = (float *)malloc(sizeof(float) * q_dim), *kv = (float *)malloc(sizeof(float) * 2 * kv_dim);
    float *att = (float *)malloc(sizeof(float) * (pos + 1)), *o = (float *)malloc(sizeof(float) * q_dim);
    float *h1 = (float *)malloc(sizeof(float) * hid), *h3 = (float *)malloc(sizeof(float) * hid);
    float *rc = (float *)malloc(sizeof(float) * half), *rs = (float *)malloc(sizeof(float) * half);
    int rcode = -1;
    if (!x || !xb || !q || !kv || !att || !o || !h1 || !h3 || !rc || !rs) goto done;

    {
        const int8_t *row = w->emb + (size_t)token * dim;
        const float sc = w->emb_scale ? w->emb_scale[token] : 1.0f;
        for (int i = 0; i < dim; i++) x[i] = (float)row[i] * sc;
    }
    for (int j = 0; j < half; j++) {
        const float freq = 1.0f / powf(c->rope_theta, (float)(2 * j) / (float)hd);
        const float val = (float)pos * freq;
        rc[j] = cosf(val);
        rs[j] = sinf(val);
    }
    const float inv_sqrt_hd = 1.0f / sqrtf((float)hd);

    for (int l = 0; l < c->n_layers; l++) {
        orc_rmsnorm(xb, x, w->rms_att ? w->rms_att + (size_t)l * dim : NULL, dim, c->rms_eps);
        if (orc_linear(mode, w->wq + (size_t)l * q_dim * dp, w->gq + (size_t)l * q_dim * gq, c->g_q, xb, w->signs_dim,
                       c->wht_dim, c->wht_norm_dim, q, q_dim, dim) ||
            orc_linear(mode, w->wk + (size_t)l * kv_dim * dp, w->gk + (size_t)l * kv_dim * gq, c->g_q, xb, w->signs_dim,
                       c->wht_dim, c->wht_norm_dim, kv, kv_dim, dim) ||
            orc_linear(mode, w->wv + (size_t)l * kv_dim * dp, w->gv + (size_t)l * kv_dim * gq, c->g_q, xb, w->signs_dim,
                       c->wht_dim, c->wht_norm_dim, kv + kv_dim, kv_dim, dim))
            goto done;
        for (int h = 0; h < c->n_heads + c->n_kv_heads; h++) {
            float *v = h < c->n_heads ? q + h * hd : kv + (h - c->n_heads) * hd;
            for (int j = 0; j < half; j++) {
                const float a = v[j], b = v[j + half];
                v[j] = a * rc[j] - b * rs[j];
                v[j + half] = b * rc[j] + a * rs[j];
            }
        }
        float *kc = kcache + ((size_t)l * c->seq_len + pos) * kv_dim, *vc = vcache + ((size_t)l * c->seq_len + pos) * kv_dim;
        for (int i = 0; i < kv_dim; i++) {
            kc[i] = mode == ORC_LIN_INT8 ? orc_round_f16(kv[i]) : kv[i];
            vc[i] = mode == ORC_LIN_INT8 ? orc_round_f16(kv[kv_dim + i]) : kv[kv_dim + i];
        }
        for (int h = 0; h < c->n_heads; h++) {
            const float *qh = q + h * hd;
            const int g = h / kv_mul;
            for (int t = 0; t <= pos; t++) {
                const float *kt = kcache + ((size_t)l * c->seq_len + t) * kv_dim + g * hd;
                float s = 0.0f;
                for (int i = 0; i < hd; i++) s += qh[i] * kt[i];
                att[t] = s * inv_sqrt_hd;
            }
            float mx = att[0];
            for (int t = 1; t <= pos; t++) mx = att[t] > mx ? att[t] : mx;
            float sum = 0.0f;
            for (int t = 0; t <= pos; t++) {
                att[t] = expf(att[t] - mx);
                sum += att[t];
            }
            const float inv = 1.0f / sum;
            for (int t = 0; t <= pos; t++) att[t] *= inv;
            float *oh = o + h * hd;
            for (int i = 0; i < hd; i++) oh[i] = 0.0f;
            for (int t = 0; t <= pos; t++) {
                const float *vt = vcache + ((size_t)l * c->seq_len + t) * kv_dim + g * hd;
                for (int i = 0; i < hd; i++) oh[i] += att[t] * vt[i];
            }
        }
        orc_rmsnorm(xb, o, w->rms_sub_att ? w->rms_sub_att + (size_t)l * q_dim : NULL, q_dim, c->sub_eps);
        if (orc_linear(mode, w->wo + (size_t)l * dim * qp, w->go + (size_t)l * dim * go, c->g_o, xb, w->signs_q,
                       c->wht_q, c->wht_norm_q, o, dim, q_dim))
            goto done;
        for (int i = 0; i < dim; i++) x[i] = x[i] + o[i];
        orc_rmsnorm(xb, x, w->rms_ffn ? w->rms_ffn + (size_t)l * dim : NULL, dim, c->rms_eps);
        if (orc_linear(mode, w->w1 + (size_t)l * hid * dp, w->g1 + (size_t)l * hid * g13, c->g_13, xb, w->signs_dim,
                       c->wht_dim, c->wht_norm_dim, h1, hid, dim) ||
            orc_linear(mode, w->w3 + (size_t)l * hid * dp, w->g3 + (size_t)l * hid * g13, c->g_13, xb, w->signs_dim,
                       c->wht_dim, c->wht_norm_dim, h3, hid, dim))
            goto done;
        for (int i = 0; i < hid; i++) {
            float val = h1[i];
            val *= (1.0f / (1.0f + expf(-val)));
            val *= h3[i];
            h1[i] = val;
        }
        orc_rmsnorm(h1, h1, w->rms_sub_ffn ? w->rms_sub_ffn + (size_t)l * hid : NULL, hid, c->sub_eps);
        if (orc_linear(mode, w->w2 + (size_t)l * dim * hp, w->g2 + (size_t)l * dim * g2, c->g_2, h1, w->signs_hidden,
                       c->wht_hidden, c->wht_norm_hidden, o, dim, hid))
            goto done;
        for (int i = 0; i < dim; i++) x[i] = x[i] + o[i];
    }
    orc_rmsnorm(x, x, w->rms_final, dim, c->rms_eps);
    if (mode == ORC_LIN_INT8) {
        int8_t *xq = (int8_t *)malloc((size_t)dim);
        float xs = 0.0f;
        if (!xq) goto done;
        orc_prep_rows(x, dim, NULL, 1, dim, 0, 1.0f, xq, dim, &xs, NULL, 0);
        orc_int8_gemv_i8act(w->wcls, w->wcls_scale, xq, dim, &xs, NULL, logits, c->vocab, 1, c->vocab, dim);
        free(xq);
    } else {
        orc_int8_rowscale_f32(logits, w->wcls, x, dim, c->vocab, w->wcls_scale);
    }
    rcode = 0;
done:
    free(x), free(xb), free(q), free(kv), free(att), free(o), free(h1), free(h3), free(rc), free(rs);
    return rcode;
}

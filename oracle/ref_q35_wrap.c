/*
 * ref_q35_wrap.c -- exposes the file-static INT4/INT8/base-3 GEMVs of the reference's src/eif_qwen35.c
 * (int4_gemv :293-352, int8_gemv :384-419, bitnet_gemv_dense :148-181) and where its loader places a QWN5 file's
 * arrays, by compiling that file where it lies, the way the reference's own
 * tests/test_q35_int4.c:3 reaches them. Built only into oracle/_ref/libref.so (test infrastructure); the path
 * of the reference tree comes from the Makefile's -DREF_QWEN35_C.
 */
#include REF_QWEN35_C

void ref_q35_int4_gemv(float *out, const uint8_t *W, const float *sc, const float *x, int rows, int cols)
{
    int4_gemv(out, W, sc, x, rows, cols);
}

void ref_q35_int8_gemv(float *out, const int8_t *W, const float *sc, const float *x, int rows, int cols)
{
    int8_gemv(out, W, sc, x, rows, cols);
}

/* The base-3 ternary GEMV of the qwen35 engine (bitnet_gemv_dense, src/eif_qwen35.c:148-181). */
void ref_q35_dense_gemv(float *out, const uint8_t *W, const float *sc, const float *x, int rows, int cols)
{
    bitnet_gemv_dense(out, W, sc, x, rows, cols);
}

/* Where the reference's own loader, qwen35_load (src/eif_qwen35.c:1223-1481), places every array of a QWN5 file:
 * byte offsets from the file's start (-1 for NULL) into offs, in the order of its structures:
 *   embed, embed_s;
 *   per DeltaNet layer: qkv, z, out, proj_b, proj_a, conv, dt_bias, A_log, qkv_s, z_s, out_s, b_s, a_s, norm_w;
 *   per attention layer: q, k, v, o, q_s, k_s, v_s, o_s, q_norm, k_norm, sub_norm;
 *   per layer: gate, up, down, gate_s, up_s, down_s, sub_norm, rms_att, rms_ffn;
 *   rms_final, had.s_dim, had.s_hid.
 * Returns qwen35_load's code (offs filled only on 0) or < -99 when the file cannot be read; *count = entries. */
int ref_q35_layout(const char *path, long long *offs, int cap, int *count)
{
    FILE *f = fopen(path, "rb");
    if (!f) return -100;
    qwen35_file_header_t h;
    qwen35_config_t c;
    int ok = fread(&h, sizeof h, 1, f) == 1 && fseek(f, (long)h.config_offset, SEEK_SET) == 0 &&
             fread(&c, sizeof c, 1, f) == 1;
    fclose(f);
    if (!ok) return -101;
    const size_t ss = qwen35_state_size(&c) + 64;
    void *state = malloc(ss);
    qwen35_t *m = (qwen35_t *)calloc(1, sizeof *m);
    if (!state || !m) return -102;
    int rc = qwen35_load(m, path, state, ss);
    int n = 0;
    if (rc == 0) {
        const uint8_t *b = (const uint8_t *)m->file_data;
        const qwen35_weights_t *W = &m->weights;
#define PUT(p) do { if (n < cap) offs[n] = (p) ? (long long)((const uint8_t *)(p) - b) : -1; n++; } while (0)
        PUT(W->embed); PUT(W->embed_s);
        for (int i = 0; i < m->config.n_delta; i++) {
            const qwen35_delta_weights_t *d = &W->delta[i];
            PUT(d->qkv); PUT(d->z); PUT(d->out); PUT(d->proj_b); PUT(d->proj_a); PUT(d->conv); PUT(d->dt_bias);
            PUT(d->A_log); PUT(d->qkv_s); PUT(d->z_s); PUT(d->out_s); PUT(d->b_s); PUT(d->a_s); PUT(d->norm_w);
        }
        for (int i = 0; i < m->config.n_full; i++) {
            const qwen35_attn_weights_t *a = &W->full[i];
            PUT(a->q); PUT(a->k); PUT(a->v); PUT(a->o); PUT(a->q_s); PUT(a->k_s); PUT(a->v_s); PUT(a->o_s);
            PUT(a->q_norm); PUT(a->k_norm); PUT(a->sub_norm);
        }
        for (int l = 0; l < m->config.n_layers; l++) {
            const qwen35_ffn_weights_t *q = &W->ffn[l];
            PUT(q->gate); PUT(q->up); PUT(q->down); PUT(q->gate_s); PUT(q->up_s); PUT(q->down_s); PUT(q->sub_norm);
            PUT(W->rms_att[l]); PUT(W->rms_ffn[l]);
        }
        PUT(W->rms_final); PUT(W->had.s_dim); PUT(W->had.s_hid);
#undef PUT
        qwen35_free(m);
    }
    *count = n;
    free(m);
    free(state);
    return rc;
}

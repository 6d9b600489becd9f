// persist.h -- internal interface of the persistent decode step (persist.hip) for the decoder (decode.hip).
#pragma once

#include <hip/hip_fp16.h>

#include "hip_common.h"

namespace eif {

// Barrier words of the persistent step: kPersistBarWords ints, kPersistBarStride apart; all zero before every
// launch (made zero at creation and by the sampler, which runs after each step).
constexpr int kPersistBarStride = 4096;
constexpr int kPersistBarWords = 17;

// What the persistent step reads and writes: the decoder's resident weights, its buffers and configuration.
struct PersistModel {
    int n_layers, dim, hidden, q_dim, kv_dim, n_heads, n_kv, head_dim, seq_len;
    float rms_eps, sub_eps;
    int wht_dim, wht_q, wht_hidden;
    float norm_dim, norm_q, norm_hidden;
    const float *signs_dim, *signs_q, *signs_hidden;
    const eif_hip_qweight *const *wqkv, *const *wo, *const *w13, *const *w2;   // [n_layers] each
    const float *const *rms_att, *const *rms_ffn, *const *rms_sub_att, *const *rms_sub_ffn;
    float *x, *qkv, *hb, *sh_o, *sh_ml;
    __half *kc, *vc;
    const float2 *rope;
    const int *state;
    const float *rms_final;
    int8_t *hq;
    float *hs;
    int head_kpad;
};

struct PersistPlan;

// The plan of the persistent step for a model, or EIF_HIP_E_LIMIT when its shapes are outside what the step
// supports (the caller keeps the step of separate launches; both give the same bits).
int persist_create(PersistPlan **out, const PersistModel &pm);
void persist_destroy(PersistPlan *p);
// One token step's 30-layer stack and the head's prep (hq, hs) as one launch on st.
int persist_enqueue(PersistPlan *p, hipStream_t st);
// The barrier words (for the sampler to clear) and the give-up flag (non-zero after a step that timed out).
int *persist_bar(PersistPlan *p);
int persist_failed(PersistPlan *p, hipStream_t st);
// Barrier words and the give-up flag back to zero (outside graph capture).
int persist_reset(PersistPlan *p, hipStream_t st);

}  // namespace eif

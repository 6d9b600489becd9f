// decode.hip -- BitNet-b1.58 decoder step on one MI355X (include/eif_hip_decode.h).
//
// The step follows tinyllm_forward_embedding_ex's BitNet path (src/eif_tinyllm.c:371-857) with every linear on
// the fused prep + int8-MFMA GEMV of qlinear.hip (eif_hip_qlinear_prep: RMSNorm / SiLU-gate + RMSNorm, WHT,
// absmax INT8, group-scaled ternary GEMV, residual as the epilogue bias), the INT8 head as a prep launch plus
// the GEMV with per-tile maxima (the argmax's first stage), and kernels of its own:
//   attn_split_kernel   RoPE of q and k (:396-405, :476-507; angles from a table made once), fp16 KV append,
//                       softmax attention (:555-650) of each query head over one chunk of the positions per
//                       workgroup, one pass over the chunk, leaving the chunk's share; the O projection's
//                       fused prep combines a head's shares (qlinear_prep_shares)
//   sample_kernel       greedy argmax over the head's tile maxima (first maximum, src/eif_tinyllm.c:1519-1530)
//                       or the next prompt token, stored in the sequence; position + 1; x = the next token's
//                       INT8 embedding row * its scale (src/eif_tinyllm.c:902-916)
//   embed_kernel        the same embedding for the first token, at reset
// Device state (position, current token, prompt, sequence) lets one captured HIP graph serve every step.
#include <hip/hip_fp16.h>

#include <algorithm>
#include <new>
#include <vector>

#include "hip_common.h"
#include "attn_dev.h"
#include "persist.h"
#include "../../include/eif_hip_decode.h"

namespace {

constexpr int kMaxSeq = 4096;

// state[0] = position of the step about to run, state[1] = its token, state[2] = prompt length
__global__ __launch_bounds__(256) void embed_kernel(const int8_t *emb, const float *emb_scale, const int *state,
                                                    float *x, int dim, int vocab)
{
    int tok = state[1];
    tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);
    const float sc = emb_scale ? emb_scale[tok] : 1.0f;
    const int8_t *row = emb + (size_t)tok * dim;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) x[i] = (float)row[i] * sc;
}

// RoPE angle of pair j (dims j, j + HD/2) at position pos: freq = 1 / powf(theta, 2j / HD), val = pos * freq;
// rope_table_kernel stores (cos, sin) of every (pos, j) once per model.
EIF_DEV void rope_cs(int pos, int j, int hd, float theta, float &c, float &sn)
{
    const float freq = 1.0f / powf(theta, (float)(2 * j) / (float)hd);
    const float val = (float)pos * freq;
    c = cosf(val), sn = sinf(val);
}

__global__ void rope_table_kernel(float2 *tab, int seq_len, int hd, float theta)
{
    const int half = hd / 2;
    const size_t n = (size_t)seq_len * half;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float c, sn;
        rope_cs((int)(i / half), (int)(i % half), hd, theta, c, sn);
        tab[i] = make_float2(c, sn);
    }
}

// Decode, split over the positions: workgroup (h, s) takes query head h (kv head g = h / kv_mul) over the
// positions of chunk s, [s CH, (s + 1) CH), CH = the fewest whole UNITs (the rows one batch of attend<HD, 512>
// covers) that cover positions 0 .. pos in kAttnShares chunks; cache rows below pos, and row pos itself in the
// chunk holding it. A chunk past pos sets its share's maximum to -inf and exits. Every workgroup rotates q_h (RoPE
// from the table); the workgroup of the chunk holding pos also rotates k_g, rounds k and v to fp16 and, for the
// first query head of the kv head, appends them to the cache. Each writes its share (attend's partial form):
// outputs sh_o[h][s][HD], maximum sh_ml[h][s], sum sh_ml[h][kAttnShares + s]; the O projection combines them,
//   M = max_s M_s, out = sum_s e^(M_s - M) O_s / sum_s e^(M_s - M) L_s.
// Cache layout: [kv_head][seq_len][HD] fp16 per layer. Grid (kAttnShares, heads): workgroup ids run over the
// chunks of a head first, so the dispatcher, which deals ids round-robin over the eight XCDs, puts chunk s of
// every head on one XCD, and the query heads of a kv head read that chunk's keys and values through one L2.
template <int HD>
constexpr int attn_chunk() { return 2048 / (HD / 8); }
constexpr int kAttnThreads = 512;   // two waves per SIMD: each thread holds 4 rows of a batch

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attn_split_kernel(const float *qkv, __half *kc, __half *vc, const int *state,
                                                         const float2 *rope, float *sh_o, float *sh_ml, int n_heads,
                                                         int n_kv, int seq_len, float inv_sqrt_hd)
{
    constexpr int HALF = HD / 2, UNIT = attn_chunk<HD>();
    __shared__ float q_l[HD], k_l[HD], v_l[HD];
    __shared__ AttnLds<HD, kAttnThreads> att_l;
    const int h = blockIdx.y, sc = blockIdx.x, kv_mul = n_heads / n_kv, g = h / kv_mul;
    const int q_dim = n_heads * HD, kv_dim = n_kv * HD;
    const int t = threadIdx.x;
    const int pos = state[0];
    const int ch = UNIT * ((pos + UNIT * kAttnShares) / (UNIT * kAttnShares));
    const int c0 = sc * ch;
    float *ml = sh_ml + (size_t)h * 2 * kAttnShares + sc;
    if (c0 > pos) {   // uniform over the workgroup
        if (t == 0) ml[0] = -INFINITY;
        return;
    }
    const bool last = pos < c0 + ch;
    auto rotate = [&]() {
        if (t < HALF) {
            const float2 cs = rope[(size_t)pos * HALF + t];
            const float c = cs.x, sn = cs.y;
            const float *qh = qkv + h * HD;
            const float a = qh[t], b = qh[t + HALF];
            q_l[t] = a * c - b * sn;
            q_l[t + HALF] = b * c + a * sn;
            if (last) {
                const float *kh = qkv + q_dim + g * HD, *vh = qkv + q_dim + kv_dim + g * HD;
                const float ka = kh[t], kb = kh[t + HALF];
                const __half k0 = __float2half(ka * c - kb * sn), k1 = __float2half(kb * c + ka * sn);
                const __half v0 = __float2half(vh[t]), v1 = __float2half(vh[t + HALF]);
                k_l[t] = __half2float(k0), k_l[t + HALF] = __half2float(k1);
                v_l[t] = __half2float(v0), v_l[t + HALF] = __half2float(v1);
                if (h % kv_mul == 0) {
                    __half *kw = kc + ((size_t)g * seq_len + pos) * HD, *vw = vc + ((size_t)g * seq_len + pos) * HD;
                    kw[t] = k0, kw[t + HALF] = k1;
                    vw[t] = v0, vw[t + HALF] = v1;
                }
            }
        }
        __syncthreads();
    };
    const size_t base = ((size_t)g * seq_len + c0) * HD;
    const int rows = (last ? pos : c0 + ch) - c0;
    attend<HD, kAttnThreads>(att_l, t, true, q_l, kc + base, vc + base, rows, last ? k_l : nullptr, last ? v_l : nullptr,
                    inv_sqrt_hd, sh_o + ((size_t)h * kAttnShares + sc) * HD, ml, rotate);
}

// Prefill, step 1: token i of a batch at position pos0 + i (one workgroup per token). RoPE of every query head
// in place in its qkv row, RoPE of every key head, the keys and values rounded to fp16 into the cache.
template <int HD>
__global__ __launch_bounds__(256) void rope_append_kernel(float *qkv, int ldqkv, __half *kc, __half *vc, int pos0,
                                                          int n_heads, int n_kv, int seq_len, const float2 *rope)
{
    constexpr int HALF = HD / 2;
    const int i = blockIdx.x, pos = pos0 + i;
    const int q_dim = n_heads * HD, kv_dim = n_kv * HD;
    float *row = qkv + (size_t)i * ldqkv;
    for (int idx = threadIdx.x; idx < (n_heads + n_kv) * HALF; idx += blockDim.x) {
        const int hh = idx / HALF, j = idx % HALF;
        const float2 cs = rope[(size_t)pos * HALF + j];
        const float c = cs.x, sn = cs.y;
        if (hh < n_heads) {
            float *qh = row + hh * HD;
            const float a = qh[j], b = qh[j + HALF];
            qh[j] = a * c - b * sn;
            qh[j + HALF] = b * c + a * sn;
        } else {
            const int g = hh - n_heads;
            const float *kh = row + q_dim + g * HD, *vh = row + q_dim + kv_dim + g * HD;
            const float a = kh[j], b = kh[j + HALF];
            __half *kw = kc + ((size_t)g * seq_len + pos) * HD, *vw = vc + ((size_t)g * seq_len + pos) * HD;
            kw[j] = __float2half(a * c - b * sn), kw[j + HALF] = __float2half(b * c + a * sn);
            vw[j] = __float2half(vh[j]), vw[j + HALF] = __float2half(vh[j + HALF]);
        }
    }
}

// Prefill, step 2: causal attention of the batch on fp32 MFMAs (v_mfma_f32_16x16x4f32: lane l supplies A[l % 16][l / 16]
// and B[l / 16][l % 16], and holds D[4 (l / 16) + i][l % 16] in register i). Workgroup (x, y) takes batch tokens
// [16 b, 16 b + 16) (b = y / s_call) and up to four query heads of kv head g = x / P (P = ceil(kv_mul / 4)), one
// wave per head, over key tiles [kPrefillTiles s, kPrefillTiles (s + 1)) (s = y % s_call) of the block's causal
// range. Per 16-key tile: S = Q K^T over the head's dims (lane group q holds dims [q HD/4, (q + 1) HD/4), the same
// order for Q and K), s = S / sqrt(HD) with keys past the query's position at -inf; per query row the online
// softmax of the decode (max m, sum l, the outputs rescaled by e^(m - m')); then O += P V with P passed through LDS
// and the tile's values staged in LDS once for the workgroup (dims x keys, zero past the batch's last key). A block
// whose range is one workgroup's writes out = O / l; a longer one writes each workgroup's share (O, m, l) to
// po / pml for attn_prefill_combine_kernel.
constexpr int kPrefillTiles = 8;

template <int HD>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const float *qkv, int ldqkv, const __half *kc,
                                                           const __half *vc, float *out, int ldo, float *po,
                                                           float *pml, int s_call, int s_cap, int pos0, int n,
                                                           int n_heads, int n_kv, int seq_len, float inv_sqrt_hd)
{
    typedef float v4f __attribute__((ext_vector_type(4)));
    constexpr int DQ = HD / 4, NT = HD / 16, VP = 20;
    __shared__ __align__(16) float v_l[2][HD][VP];
    __shared__ __align__(16) float p_l[4][16][VP];
    const int kv_mul = n_heads / n_kv, parts = (kv_mul + 3) / 4;
    const int g = blockIdx.x / parts, part = blockIdx.x - g * parts;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const bool active = part * 4 + w < kv_mul;   // uniform over the wave
    const int h = g * kv_mul + (active ? part * 4 + w : 0);
    const int b = blockIdx.y / s_call, sp = blockIdx.y - b * s_call;
    const int i0 = b * 16, r = lane & 15, q = lane >> 4;
    const __half *kg = kc + (size_t)g * seq_len * HD, *vg = vc + (size_t)g * seq_len * HD;
    const int n_keys = pos0 + min(i0 + 16, n);   // keys the block's queries may see
    const int all_tiles = (n_keys + 15) / 16;
    const int t_begin = sp * kPrefillTiles, n_tiles = min(t_begin + kPrefillTiles, all_tiles);
    if (t_begin >= n_tiles) return;   // uniform over the workgroup
    const bool split = all_tiles > kPrefillTiles;

    float qv[DQ];   // query row r (batch token i0 + r), dims [DQ q, DQ q + DQ)
    {
        const float *qp = qkv + (size_t)min(i0 + r, n - 1) * ldqkv + h * HD + DQ * q;
#pragma unroll
        for (int j = 0; j < DQ; j += 4) {
            const float4 f = *reinterpret_cast<const float4 *>(qp + j);
            qv[j] = f.x, qv[j + 1] = f.y, qv[j + 2] = f.z, qv[j + 3] = f.w;
        }
    }
    v4f O[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) O[tt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float m_r[4], l_r[4];   // rows 4 q + i
#pragma unroll
    for (int i = 0; i < 4; ++i) m_r[i] = -INFINITY, l_r[i] = 0.0f;

    // Tile kt + 1's keys and values are loaded into registers while tile kt computes (the last tile loads
    // itself again); the values go to LDS at the top of the next iteration.
    constexpr int VI = 2 * HD / 64;   // staging pieces per thread at most (8 values each, 64-thread workgroups)
    uint4 vraw[VI], kraw[DQ / 8];
    auto fetch = [&](int kt) {
        const int k0 = 16 * kt;
#pragma unroll
        for (int u = 0; u < VI; ++u) {
            const int idx = t + u * (int)blockDim.x;
            const int key = min(idx, 2 * HD - 1) & 15, d0 = (min(idx, 2 * HD - 1) >> 4) * 8;
            vraw[u] = *reinterpret_cast<const uint4 *>(vg + (size_t)min(k0 + key, n_keys - 1) * HD + d0);
        }
        const __half *kp = kg + (size_t)min(k0 + r, n_keys - 1) * HD + DQ * q;
#pragma unroll
        for (int j = 0; j < DQ / 8; ++j) kraw[j] = *reinterpret_cast<const uint4 *>(kp + 8 * j);
    };
    fetch(t_begin);
    for (int kt = t_begin; kt < n_tiles; ++kt) {
        const int k0 = 16 * kt;
        float(*vb)[VP] = v_l[kt & 1];
#pragma unroll
        for (int u = 0; u < VI; ++u) {   // 8 values of one key per piece, zero past the batch's last key
            const int idx = t + u * (int)blockDim.x;
            if (idx < 2 * HD) {
                const int key = idx & 15, d0 = (idx >> 4) * 8;
                float vv[8];
                half8_to_float(vraw[u], vv);
                const bool ok = k0 + key < n_keys;
#pragma unroll
                for (int e = 0; e < 8; ++e) vb[d0 + e][key] = ok ? vv[e] : 0.0f;
            }
        }
        float kv[DQ];   // key row k0 + r (clamped; keys past n_keys are masked), dims [DQ q, DQ q + DQ)
#pragma unroll
        for (int j = 0; j < DQ / 8; ++j) {
            float f8[8];
            half8_to_float(kraw[j], f8);
#pragma unroll
            for (int e = 0; e < 8; ++e) kv[8 * j + e] = f8[e];
        }
        fetch(min(kt + 1, n_tiles - 1));
        __syncthreads();   // the tile's values staged; the other buffer's readers (tile kt - 1) are done
        if (active) {
            v4f S = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < DQ; ++j) S = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[j], kv[j], S, 0, 0, 0);
            const int kpos = k0 + r;
#pragma unroll
            for (int i = 0; i < 4; ++i) {   // S[i] = score of query row 4 q + i and key k0 + r
                const int qpos = pos0 + i0 + 4 * q + i;
                const float sv = kpos <= qpos && kpos < n_keys ? S[i] * inv_sqrt_hd : -INFINITY;
                float mx = fmaxf(sv, xlane<1>(sv));   // the row's 16 keys: DPP butterflies inside the lane row
                mx = fmaxf(mx, xlane<2>(mx));
                mx = fmaxf(mx, xlane<4>(mx));
                mx = fmaxf(mx, xlane<8>(mx));
                // mn = -inf only while a share's keys all lie past the query (a split range); the row then
                // keeps m = -inf, l = 0, O = 0, which weighs 0 in the combine
                const float mn = fmaxf(m_r[i], mx);
                const bool none = mn == -INFINITY;
                const float sc = none ? 1.0f : expf(m_r[i] - mn), pw = none ? 0.0f : expf(sv - mn);
                float ps = pw + xlane<1>(pw);
                ps = ps + xlane<2>(ps);
                ps = ps + xlane<4>(ps);
                ps = ps + xlane<8>(ps);
                l_r[i] = l_r[i] * sc + ps;
                m_r[i] = mn;
                p_l[w][4 * q + i][r] = pw;
#pragma unroll
                for (int tt = 0; tt < NT; ++tt) O[tt][i] *= sc;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const float4 pa = *reinterpret_cast<const float4 *>(&p_l[w][r][4 * q]);   // P[r][4 q .. 4 q + 3]
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) {
                const float4 vv = *reinterpret_cast<const float4 *>(&vb[16 * tt + r][4 * q]);   // V[4 q + j][16 tt + r]
                O[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.x, vv.x, O[tt], 0, 0, 0);
                O[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.y, vv.y, O[tt], 0, 0, 0);
                O[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.z, vv.z, O[tt], 0, 0, 0);
                O[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.w, vv.w, O[tt], 0, 0, 0);
            }
        }
    }
    if (!active) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int qi = i0 + 4 * q + i;
        if (qi >= n) continue;
        if (split) {   // share (b, sp) of query row 4 q + i: [b][s][head][row]
            const size_t e = (((size_t)b * s_cap + sp) * n_heads + h) * 16 + 4 * q + i;
            float *op = po + e * HD + r;
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) op[16 * tt] = O[tt][i];
            if (r == 0) pml[2 * e] = m_r[i], pml[2 * e + 1] = l_r[i];
        } else {
            float *op = out + (size_t)qi * ldo + h * HD + r;
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) op[16 * tt] = O[tt][i] / l_r[i];
        }
    }
}

// Prefill, step 3 (blocks whose causal range was split): out = sum_s e^(m_s - M) O_s / sum_s e^(m_s - M) l_s over the
// block's shares, M = max_s m_s (a share with m_s = -inf weighs 0). Workgroup (token i, head h), HD threads.
template <int HD>
__global__ __launch_bounds__(128) void attn_prefill_combine_kernel(const float *po, const float *pml, float *out,
                                                                   int ldo, int s_cap, int pos0, int n, int n_heads)
{
    const int i = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
    const int b = i / 16, row = i - 16 * b;
    const int all_tiles = (pos0 + min(16 * b + 16, n) + 15) / 16;
    if (all_tiles <= kPrefillTiles) return;   // written by the attention kernel
    const int ns = (all_tiles + kPrefillTiles - 1) / kPrefillTiles;
    const size_t e0 = ((size_t)b * s_cap * n_heads + h) * 16 + row, es = (size_t)n_heads * 16;
    float mx = -INFINITY;
    for (int s2 = 0; s2 < ns; ++s2) mx = fmaxf(mx, pml[2 * (e0 + s2 * es)]);
    float os = 0.0f, ls = 0.0f;
    for (int s2 = 0; s2 < ns; ++s2) {
        const size_t e = e0 + s2 * es;
        const float ms = pml[2 * e];
        const float wgt = ms == -INFINITY ? 0.0f : expf(ms - mx);
        os = fmaf(wgt, po[e * HD + d], os);
        ls = fmaf(wgt, pml[2 * e + 1], ls);
    }
    out[(size_t)i * ldo + h * HD + d] = os / ls;
}

// Prefill: the embedding rows of prompt tokens pos0 .. pos0 + n - 1 (one workgroup per token).
__global__ __launch_bounds__(256) void embed_rows_kernel(const int8_t *emb, const float *emb_scale, const int *prompt,
                                                         int pos0, float *x, int dim)
{
    const int i = blockIdx.x, tok = prompt[pos0 + i];
    const float sc = emb_scale ? emb_scale[tok] : 1.0f;
    const int8_t *row = emb + (size_t)tok * dim;
    for (int c = threadIdx.x; c < dim; c += blockDim.x) x[(size_t)i * dim + c] = (float)row[c] * sc;
}

// out = a * b over n floats (an RMSNorm weight times +-1 rotation signs: exact).
__global__ void mul_rows_kernel(float *out, const float *a, const float *b, int n)
{
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) out[i] = a[i] * b[i];
}

// Prefill: the residual stream x += y over n floats.
__global__ void add_rows_kernel(float *x, const float *y, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        x[i] = y[i] + x[i];
}

// Prefill: the sequence entries of a batch's prompt tokens and the position of its last token (the sampler then
// makes the step of that token as a decode step would).
__global__ void prefill_state_kernel(int *state, int *seq, const int *prompt, int pos0, int n)
{
    for (int i = threadIdx.x; i + 1 < n; i += blockDim.x) seq[pos0 + 1 + i] = prompt[pos0 + 1 + i];
    if (threadIdx.x == 0) state[0] = pos0 + n - 1;
}

// Greedy token: first index of the largest logit (NaN never wins), from the head GEMV's argmax slots (atomic max of
// eif_argmax_key over its tiles; folded here by the first wave and reset to 0 for the next step); while the prompt
// lasts the next token is the prompt's. The made token is stored at position pos + 1 of the sequence, the position advances, and x becomes
// the next token's embedding row.
__global__ __launch_bounds__(1024) void sample_kernel(unsigned long long *amax_key, int *state, const int *prompt,
                                                      int *seq, int seq_len, const int8_t *emb,
                                                      const float *emb_scale, float *x, int dim, int vocab, int *bar)
{
    // the persistent step's barrier words back to zero for the next step (that step ended before this launch)
    if (bar && (int)threadIdx.x < eif::kPersistBarWords) bar[(size_t)eif::kPersistBarStride * threadIdx.x] = 0;
    __shared__ int next_l;
    const int t = threadIdx.x, nt = blockDim.x;
    static_assert(kArgmaxSlots == 64, "one slot per lane of the first wave");
    unsigned long long key = 0;
    if (t < 64) {
        key = amax_key[(size_t)kArgmaxStride * t];
        amax_key[(size_t)kArgmaxStride * t] = 0ull;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const unsigned long long o = __shfl_xor(key, off, 64);
            key = o > key ? o : key;
        }
    }
    if (t == 0) {
        int idx = eif_argmax_key_row(key);
        if (idx < 0 || idx >= vocab) idx = 0;   // every logit NaN or -inf
        const int pos = state[0], np = state[2];
        const int next = pos + 1 < np ? prompt[pos + 1] : idx;
        if (pos + 1 < seq_len) seq[pos + 1] = next;
        state[1] = next;
        state[0] = pos + 1;
        next_l = next;
    }
    __syncthreads();
    const int tok = next_l;
    const float sc = emb_scale ? emb_scale[tok] : 1.0f;
    const int8_t *row = emb + (size_t)tok * dim;
    for (int i = t; i < dim; i += nt) x[i] = (float)row[i] * sc;
}

__global__ void fill_half_kernel(__half *p, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = __float2half(0.0f);
}

__global__ void start_kernel(int *state, int *seq, const int *prompt, int n_prompt)
{
    state[0] = 0;
    state[1] = prompt[0];
    state[2] = n_prompt;
    seq[0] = prompt[0];
}

template <typename T>
int dev_upload(T **dst, const T *src, size_t n)
{
    *dst = nullptr;
    if (!src) return EIF_HIP_OK;
    T *p = nullptr;
    if (hipMalloc(&p, n * sizeof(T)) != hipSuccess) return EIF_HIP_E_NOMEM;
    if (hipMemcpy(p, src, n * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(p);
        return EIF_HIP_E_DEVICE;
    }
    *dst = p;
    return EIF_HIP_OK;
}

}  // namespace

struct eif_hip_bitnet {
    eif_hip_bitnet_config c{};
    int q_dim = 0, kv_dim = 0;
    std::vector<eif_hip_qweight *> wqkv, wo, w13, w2;
    eif_hip_qweight *head = nullptr;
    std::vector<float *> rms_att, rms_ffn, rms_sub_att, rms_sub_ffn;
    float *rms_final = nullptr, *signs_dim = nullptr, *signs_q = nullptr, *signs_hidden = nullptr;
    // Each RMSNorm weight times its input's rotation signs ((v w) s = v (w s) exactly for +-1 signs), so the
    // fused prep of a token step reads one column multiplier instead of two; null where nothing is folded.
    std::vector<float *> mul_att, mul_ffn, mul_sub_att, mul_sub_ffn;
    bool fold_dim = false, fold_q = false, fold_hidden = false;   // signs present, all +-1, inputs rotated
    int8_t *emb = nullptr;
    float *emb_scale = nullptr;
    float *x = nullptr, *qkv = nullptr, *hb = nullptr, *logits = nullptr;
    __half *kc = nullptr, *vc = nullptr;
    int *state = nullptr, *prompt = nullptr, *seq = nullptr;
    float2 *rope = nullptr;          // RoPE (cos, sin) [seq_len][head_dim / 2]
    float *sh_o = nullptr;           // attention shares: outputs [n_heads][kAttnShares][head_dim]
    float *sh_ml = nullptr;          // and their maxima, then sums [n_heads][2 kAttnShares]
    int8_t *hq = nullptr;            // the head's prepped input row [head_kpad] and its scale
    float *hs = nullptr;
    unsigned long long *amax_key = nullptr;   // the head's greedy argmax slots (eif_argmax_key), 0 between steps
    int head_kpad = 0, head_tiles = 0;
    int hpos = 0;                    // host copy of the position (steps are deterministic)
    int n_prompt = 0;                // host copy of the prompt length
    // prefill batch buffers for up to pf_cap tokens (allocated by the first eif_hip_bitnet_prefill):
    // residual x, attention output, qkv, gate|up, a linear's output, int8 rows and their scales
    int pf_cap = 0;
    float *p_x = nullptr, *p_xb = nullptr, *p_qkv = nullptr, *p_h = nullptr, *p_y = nullptr, *p_xs = nullptr;
    float *p_po = nullptr, *p_pml = nullptr;   // attention shares of split blocks [block][share][head][16][HD | 2]
    int pf_scap = 0;                           // shares per block the buffers hold
    int8_t *p_xq = nullptr;
    size_t weight_bytes = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipStream_t cap = nullptr;       // the stream the step is captured on (the legacy stream cannot capture)
    // the persistent step (persist.hip): made at the first step when the shapes allow it
    eif::PersistPlan *plan = nullptr;
    int plan_state = 0;              // 0 not tried, 1 made, -1 shapes outside the persistent step
    int use_persist = 0;             // requested (eif_hip_bitnet_set_persistent); separate launches by default
};

namespace {

int enqueue_head(eif_hip_bitnet *m, hipStream_t st);

int enqueue_head_gemv(eif_hip_bitnet *m, hipStream_t st);

// The folded multipliers of layer l (eif_hip_bitnet::mul_att ...), made once its norm weights and the signs are
// both set.
int fold_signs(eif_hip_bitnet *m, int l)
{
    const eif_hip_bitnet_config &c = m->c;
    struct Fold {
        std::vector<float *> *dst;
        const float *nw, *sg;
        bool ok;
        int n;
    } const f[4] = {{&m->mul_att, m->rms_att[l], m->signs_dim, m->fold_dim, c.dim},
                    {&m->mul_ffn, m->rms_ffn[l], m->signs_dim, m->fold_dim, c.dim},
                    {&m->mul_sub_att, m->rms_sub_att[l], m->signs_q, m->fold_q, m->q_dim},
                    {&m->mul_sub_ffn, m->rms_sub_ffn[l], m->signs_hidden, m->fold_hidden, c.hidden}};
    for (const Fold &d : f) {
        if (!d.ok || !d.nw || !d.sg || (*d.dst)[l]) continue;
        float *out = nullptr;
        if (hipMalloc(&out, sizeof(float) * d.n) != hipSuccess) return EIF_HIP_E_NOMEM;
        mul_rows_kernel<<<(d.n + 255) / 256, 256>>>(out, d.nw, d.sg, d.n);
        if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
            (void)hipFree(out);
            return EIF_HIP_E_DEVICE;
        }
        (*d.dst)[l] = out;
    }
    return EIF_HIP_OK;
}

// A prep spec's norm weight and signs: the folded multiplier where there is one.
void spec_norm(eif_hip_prep_spec &sp, const float *mul, const float *nw, const float *signs)
{
    sp.norm_w = mul ? mul : nw;
    sp.signs = mul ? nullptr : signs;
}

int enqueue_step(eif_hip_bitnet *m, hipStream_t st)
{
    if (m->plan && m->use_persist) {   // the layer stack and the head's prep as one launch, then head and sampler
        const int rc = eif::persist_enqueue(m->plan, st);
        if (rc) return rc;
        return enqueue_head_gemv(m, st);
    }
    const eif_hip_bitnet_config &c = m->c;
    const float inv_sqrt_hd = 1.0f / sqrtf((float)c.head_dim);
    for (int l = 0; l < c.n_layers; ++l) {
        eif_hip_prep_spec sp{};
        sp.x = m->x, sp.ldx = c.dim, sp.pre = EIF_HIP_PRE_RMS, sp.eps = c.rms_eps;
        spec_norm(sp, m->mul_att[l], m->rms_att[l], m->signs_dim);
        sp.wht_block = c.wht_dim, sp.wht_norm = c.wht_norm_dim;
        int rc = eif_hip_qlinear_prep(m->wqkv[l], &sp, nullptr, m->qkv, m->q_dim + 2 * m->kv_dim, 1, st);
        if (rc) return rc;
        const size_t cache_l = (size_t)l * c.n_kv_heads * c.seq_len * c.head_dim;
        auto attn = c.head_dim == 128 ? attn_split_kernel<128>
                    : (c.head_dim == 64 ? attn_split_kernel<64> : attn_split_kernel<32>);
        attn<<<dim3(kAttnShares, c.n_heads), kAttnThreads, 0, st>>>(m->qkv, m->kc + cache_l, m->vc + cache_l, m->state,
                                                           m->rope, m->sh_o, m->sh_ml, c.n_heads, c.n_kv_heads,
                                                           c.seq_len, inv_sqrt_hd);
        EIF_HIP_LAUNCHED();
        sp = eif_hip_prep_spec{};
        sp.pre = EIF_HIP_PRE_RMS, sp.eps = c.sub_eps;
        spec_norm(sp, m->mul_sub_att[l], m->rms_sub_att[l], m->signs_q);
        sp.wht_block = c.wht_q, sp.wht_norm = c.wht_norm_q;
        // x += O attention (the shares combined in the prep)
        if ((rc = eif::qlinear_prep_shares(m->wo[l], &sp, m->sh_o, m->sh_ml, c.head_dim, m->x, m->x, c.dim, st)))
            return rc;
        sp = eif_hip_prep_spec{};
        sp.x = m->x, sp.ldx = c.dim, sp.pre = EIF_HIP_PRE_RMS, sp.eps = c.rms_eps;
        spec_norm(sp, m->mul_ffn[l], m->rms_ffn[l], m->signs_dim);
        sp.wht_block = c.wht_dim, sp.wht_norm = c.wht_norm_dim;
        // h = SiLU(gate) * up in the gate|up launch (its GLU form) where the shape allows, then the down projection
        // with the sub-RMSNorm alone: the same bits as both halves and the SwiGLU pre-op
        rc = eif_hip_qlinear_prep_glu(m->w13[l], &sp, m->hb, c.hidden, 1, st);
        const bool glu = rc == EIF_HIP_OK;
        if (!glu && (rc != EIF_HIP_E_LIMIT || (rc = eif_hip_qlinear_prep(m->w13[l], &sp, nullptr, m->hb, 2 * c.hidden, 1, st))))
            return rc;
        sp = eif_hip_prep_spec{};
        sp.x = m->hb, sp.x2 = m->hb + c.hidden, sp.ldx = c.hidden;
        sp.pre = glu ? EIF_HIP_PRE_RMS : EIF_HIP_PRE_SWIGLU_RMS;
        sp.eps = c.sub_eps;
        spec_norm(sp, m->mul_sub_ffn[l], m->rms_sub_ffn[l], m->signs_hidden);
        sp.wht_block = c.wht_hidden, sp.wht_norm = c.wht_norm_hidden;
        if ((rc = eif_hip_qlinear_prep(m->w2[l], &sp, m->x, m->x, c.dim, 1, st))) return rc;   // x += W2 h
    }
    return enqueue_head(m, st);
}

// The head and the sampler on x: RMSNorm + INT8 prep once, the INT8 GEMV with per-tile maxima, then the argmax
// over the tiles (or the next prompt token), position + 1, x = the next token's embedding row.
int enqueue_head(eif_hip_bitnet *m, hipStream_t st)
{
    const eif_hip_bitnet_config &c = m->c;
    eif_hip_prep_spec sp{};
    sp.x = m->x, sp.ldx = c.dim, sp.pre = EIF_HIP_PRE_RMS, sp.norm_w = m->rms_final, sp.eps = c.rms_eps;
    const int rc = eif_hip_prep_spec_rows(&sp, c.dim, m->hq, m->head_kpad, m->hs, 1, st);
    if (rc) return rc;
    return enqueue_head_gemv(m, st);
}

// The head GEMV on the prepped row (hq, hs) with per-tile maxima, then the sampler.
int enqueue_head_gemv(eif_hip_bitnet *m, hipStream_t st)
{
    const eif_hip_bitnet_config &c = m->c;
    int rc;
    if ((rc = eif::qlinear_argmax(m->head, m->hq, m->head_kpad, m->hs, m->logits, m->amax_key, st))) return rc;
    sample_kernel<<<1, 1024, 0, st>>>(m->amax_key, m->state, m->prompt, m->seq, c.seq_len,
                                      m->emb, m->emb_scale, m->x, c.dim, c.vocab, eif::persist_bar(m->plan));
    EIF_HIP_LAUNCHED();
    return EIF_HIP_OK;
}

// The persistent step's plan, made once all weights are set (or left unmade when the shapes are outside it).
void ensure_plan(eif_hip_bitnet *m)
{
    if (m->plan_state != 0) return;
    const eif_hip_bitnet_config &c = m->c;
    eif::PersistModel pm{};
    pm.n_layers = c.n_layers, pm.dim = c.dim, pm.hidden = c.hidden, pm.q_dim = m->q_dim, pm.kv_dim = m->kv_dim;
    pm.n_heads = c.n_heads, pm.n_kv = c.n_kv_heads, pm.head_dim = c.head_dim, pm.seq_len = c.seq_len;
    pm.rms_eps = c.rms_eps, pm.sub_eps = c.sub_eps;
    pm.wht_dim = c.wht_dim, pm.wht_q = c.wht_q, pm.wht_hidden = c.wht_hidden;
    pm.norm_dim = c.wht_norm_dim, pm.norm_q = c.wht_norm_q, pm.norm_hidden = c.wht_norm_hidden;
    pm.signs_dim = m->signs_dim, pm.signs_q = m->signs_q, pm.signs_hidden = m->signs_hidden;
    pm.wqkv = m->wqkv.data(), pm.wo = m->wo.data(), pm.w13 = m->w13.data(), pm.w2 = m->w2.data();
    pm.rms_att = m->rms_att.data(), pm.rms_ffn = m->rms_ffn.data();
    pm.rms_sub_att = m->rms_sub_att.data(), pm.rms_sub_ffn = m->rms_sub_ffn.data();
    pm.x = m->x, pm.qkv = m->qkv, pm.hb = m->hb, pm.sh_o = m->sh_o, pm.sh_ml = m->sh_ml;
    pm.kc = m->kc, pm.vc = m->vc, pm.rope = m->rope, pm.state = m->state;
    pm.rms_final = m->rms_final, pm.hq = m->hq, pm.hs = m->hs, pm.head_kpad = m->head_kpad;
    eif::PersistPlan *p = nullptr;
    if (eif::persist_create(&p, pm) == EIF_HIP_OK) {
        m->plan = p;
        m->plan_state = 1;
    } else {
        m->plan_state = -1;
    }
}

// EIF_HIP_E_DEVICE when a persistent step gave up at a barrier (synchronous; clears nothing).
int check_plan(eif_hip_bitnet *m, hipStream_t st)
{
    if (m->plan && eif::persist_failed(m->plan, st)) {
        fprintf(stderr, "libbitllm_hip: a persistent decode step gave up waiting at a grid barrier\n");
        return EIF_HIP_E_DEVICE;
    }
    return EIF_HIP_OK;
}

int kpad_of(const eif_hip_qweight *w)
{
    int kp = 0;
    eif_hip_qweight_info(w, nullptr, nullptr, &kp, nullptr, nullptr);
    return kp;
}

void free_prefill(eif_hip_bitnet *m)
{
    for (void *p : {(void *)m->p_po, (void *)m->p_pml, (void *)m->p_x, (void *)m->p_xb, (void *)m->p_qkv, (void *)m->p_h, (void *)m->p_y,
                    (void *)m->p_xs, (void *)m->p_xq})
        if (p) (void)hipFree(p);
    m->p_x = m->p_xb = m->p_qkv = m->p_h = m->p_y = m->p_xs = m->p_po = m->p_pml = nullptr;
    m->pf_scap = 0;
    m->p_xq = nullptr;
    m->pf_cap = 0;
}

int ensure_prefill(eif_hip_bitnet *m, int n)
{
    if (n <= m->pf_cap) return EIF_HIP_OK;
    const eif_hip_bitnet_config &c = m->c;
    int kmax = kpad_of(m->head);
    for (int l = 0; l < c.n_layers; ++l)
        for (const eif_hip_qweight *w : {m->wqkv[l], m->wo[l], m->w13[l], m->w2[l]}) kmax = std::max(kmax, kpad_of(w));
    free_prefill(m);   // synchronizes with work that used the old buffers
    const size_t N = (size_t)n;
    if (hipMalloc(&m->p_x, sizeof(float) * N * c.dim) != hipSuccess ||
        hipMalloc(&m->p_xb, sizeof(float) * N * m->q_dim) != hipSuccess ||
        hipMalloc(&m->p_qkv, sizeof(float) * N * (m->q_dim + 2 * m->kv_dim)) != hipSuccess ||
        hipMalloc(&m->p_h, sizeof(float) * N * 2 * c.hidden) != hipSuccess ||
        hipMalloc(&m->p_y, sizeof(float) * N * std::max(c.dim, m->q_dim)) != hipSuccess ||
        hipMalloc(&m->p_xs, sizeof(float) * N) != hipSuccess || hipMalloc(&m->p_xq, N * kmax) != hipSuccess) {
        free_prefill(m);
        return EIF_HIP_E_NOMEM;
    }
    // attention shares: up to ceil(ceil(seq_len / 16) / kPrefillTiles) per 16-token block
    const int scap = ((c.seq_len + 15) / 16 + kPrefillTiles - 1) / kPrefillTiles;
    const size_t ne = (size_t)((n + 15) / 16) * scap * c.n_heads * 16;
    if (scap > 1 && (hipMalloc(&m->p_po, sizeof(float) * ne * c.head_dim) != hipSuccess ||
                     hipMalloc(&m->p_pml, sizeof(float) * ne * 2) != hipSuccess)) {
        free_prefill(m);
        return EIF_HIP_E_NOMEM;
    }
    m->pf_scap = scap;
    m->pf_cap = n;
    return EIF_HIP_OK;
}

// The prompt tokens at positions pos0 .. pos0 + n - 1 as one batch: every linear as prep + MFMA GEMM over the
// n rows, RoPE + KV append for the batch, causal attention per 16-token block (shares of long ranges combined),
// the residual adds; then the head and the sampler for the last token, as its decode step would run them.
int enqueue_prefill(eif_hip_bitnet *m, int pos0, int n, hipStream_t st)
{
    const eif_hip_bitnet_config &c = m->c;
    const float inv_sqrt_hd = 1.0f / sqrtf((float)c.head_dim);
    const int ldqkv = m->q_dim + 2 * m->kv_dim;
    const unsigned add_blocks = (unsigned)std::min<size_t>(1024, ((size_t)n * c.dim + 255) / 256);
    auto prep_linear = [&](const eif_hip_qweight *w, const eif_hip_prep_spec &sp, int K, float *y, int ldy) {
        const int kp = kpad_of(w);
        int rc = eif_hip_prep_spec_rows(&sp, K, m->p_xq, kp, m->p_xs, n, st);
        if (rc) return rc;
        return eif_hip_qlinear_ex(w, m->p_xq, kp, m->p_xs, nullptr, y, ldy, n, EIF_HIP_PATH_AUTO, st);
    };
    embed_rows_kernel<<<n, 256, 0, st>>>(m->emb, m->emb_scale, m->prompt, pos0, m->p_x, c.dim);
    EIF_HIP_LAUNCHED();
    for (int l = 0; l < c.n_layers; ++l) {
        eif_hip_prep_spec sp{};
        sp.x = m->p_x, sp.ldx = c.dim, sp.pre = EIF_HIP_PRE_RMS, sp.norm_w = m->rms_att[l], sp.eps = c.rms_eps;
        sp.signs = m->signs_dim, sp.wht_block = c.wht_dim, sp.wht_norm = c.wht_norm_dim;
        int rc = prep_linear(m->wqkv[l], sp, c.dim, m->p_qkv, ldqkv);
        if (rc) return rc;
        const size_t cache_l = (size_t)l * c.n_kv_heads * c.seq_len * c.head_dim;
        auto rope = c.head_dim == 128 ? rope_append_kernel<128>
                    : (c.head_dim == 64 ? rope_append_kernel<64> : rope_append_kernel<32>);
        rope<<<n, 256, 0, st>>>(m->p_qkv, ldqkv, m->kc + cache_l, m->vc + cache_l, pos0, c.n_heads, c.n_kv_heads,
                                c.seq_len, m->rope);
        EIF_HIP_LAUNCHED();
        auto attn = c.head_dim == 128 ? attn_prefill_kernel<128>
                    : (c.head_dim == 64 ? attn_prefill_kernel<64> : attn_prefill_kernel<32>);
        const int kv_mul = c.n_heads / c.n_kv_heads, parts = (kv_mul + 3) / 4;
        const int s_call = ((pos0 + n + 15) / 16 + kPrefillTiles - 1) / kPrefillTiles;   // shares of the longest block
        attn<<<dim3(c.n_kv_heads * parts, (n + 15) / 16 * s_call), 64 * std::min(kv_mul, 4), 0, st>>>(
            m->p_qkv, ldqkv, m->kc + cache_l, m->vc + cache_l, m->p_xb, m->q_dim, m->p_po, m->p_pml, s_call,
            m->pf_scap, pos0, n, c.n_heads, c.n_kv_heads, c.seq_len, inv_sqrt_hd);
        EIF_HIP_LAUNCHED();
        if (s_call > 1) {
            auto comb = c.head_dim == 128 ? attn_prefill_combine_kernel<128>
                        : (c.head_dim == 64 ? attn_prefill_combine_kernel<64> : attn_prefill_combine_kernel<32>);
            comb<<<dim3(n, c.n_heads), c.head_dim, 0, st>>>(m->p_po, m->p_pml, m->p_xb, m->q_dim, m->pf_scap, pos0, n,
                                                            c.n_heads);
        }
        EIF_HIP_LAUNCHED();
        sp = eif_hip_prep_spec{};
        sp.x = m->p_xb, sp.ldx = m->q_dim, sp.pre = EIF_HIP_PRE_RMS, sp.norm_w = m->rms_sub_att[l];
        sp.eps = c.sub_eps, sp.signs = m->signs_q, sp.wht_block = c.wht_q, sp.wht_norm = c.wht_norm_q;
        if ((rc = prep_linear(m->wo[l], sp, m->q_dim, m->p_y, c.dim))) return rc;
        add_rows_kernel<<<add_blocks, 256, 0, st>>>(m->p_x, m->p_y, (size_t)n * c.dim);   // x += O xb
        EIF_HIP_LAUNCHED();
        sp = eif_hip_prep_spec{};
        sp.x = m->p_x, sp.ldx = c.dim, sp.pre = EIF_HIP_PRE_RMS, sp.norm_w = m->rms_ffn[l], sp.eps = c.rms_eps;
        sp.signs = m->signs_dim, sp.wht_block = c.wht_dim, sp.wht_norm = c.wht_norm_dim;
        if ((rc = prep_linear(m->w13[l], sp, c.dim, m->p_h, 2 * c.hidden))) return rc;
        sp = eif_hip_prep_spec{};
        sp.x = m->p_h, sp.x2 = m->p_h + c.hidden, sp.ldx = 2 * c.hidden, sp.pre = EIF_HIP_PRE_SWIGLU_RMS;
        sp.norm_w = m->rms_sub_ffn[l], sp.eps = c.sub_eps;
        sp.signs = m->signs_hidden, sp.wht_block = c.wht_hidden, sp.wht_norm = c.wht_norm_hidden;
        if ((rc = prep_linear(m->w2[l], sp, c.hidden, m->p_y, c.dim))) return rc;
        add_rows_kernel<<<add_blocks, 256, 0, st>>>(m->p_x, m->p_y, (size_t)n * c.dim);   // x += W2 h
        EIF_HIP_LAUNCHED();
    }
    EIF_HIP_TRY(hipMemcpyAsync(m->x, m->p_x + (size_t)(n - 1) * c.dim, sizeof(float) * c.dim,
                               hipMemcpyDeviceToDevice, st));
    prefill_state_kernel<<<1, 256, 0, st>>>(m->state, m->seq, m->prompt, pos0, n);
    EIF_HIP_LAUNCHED();
    return enqueue_head(m, st);
}

// Rows of two reference-format ternary matrices stacked (same columns): codes and grouped scales.
void stack_rows(std::vector<uint8_t> &codes, std::vector<float> &scales, const uint8_t *w, const float *s, int rows,
                int cols, int group)
{
    const size_t rb = (size_t)(cols + 3) / 4, ng = group > 0 ? (size_t)(cols + group - 1) / group : 1;
    codes.insert(codes.end(), w, w + rows * rb);
    scales.insert(scales.end(), s, s + rows * ng);
}

int make_tern(eif_hip_qweight **q, const std::vector<uint8_t> &codes, const std::vector<float> &scales, int rows,
              int cols, int group, size_t *bytes)
{
    const int rc = eif_hip_qweight_create(q, EIF_HIP_W_TERNARY, rows, cols, group, codes.data(), scales.data(), 0,
                                          nullptr);
    if (rc == EIF_HIP_OK) {
        size_t b = 0;
        eif_hip_qweight_info(*q, nullptr, nullptr, nullptr, nullptr, &b);
        *bytes += b;
    }
    return rc;
}

}  // namespace

extern "C" {

int eif_hip_bitnet_create(eif_hip_bitnet **out, const eif_hip_bitnet_config *cfg)
{
    if (!out || !cfg) return EIF_HIP_E_ARG;
    *out = nullptr;
    const eif_hip_bitnet_config &c = *cfg;
    if (c.dim <= 0 || c.hidden <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.vocab <= 0 ||
        c.n_heads % c.n_kv_heads || (c.head_dim != 32 && c.head_dim != 64 && c.head_dim != 128) || c.seq_len <= 0 ||
        c.seq_len > kMaxSeq || c.dim % 32 || c.hidden % 32 || (c.n_heads * c.head_dim) % 32)
        return EIF_HIP_E_ARG;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return EIF_HIP_E_DEVICE;
    int rc = eif_hip_init(dev);
    if (rc) return rc;
    eif_hip_bitnet *m = new (std::nothrow) eif_hip_bitnet;
    if (!m) return EIF_HIP_E_NOMEM;
    m->c = c;
    m->q_dim = c.n_heads * c.head_dim;
    m->kv_dim = c.n_kv_heads * c.head_dim;
    const size_t cache = (size_t)c.n_layers * c.n_kv_heads * c.seq_len * c.head_dim;
    m->wqkv.assign(c.n_layers, nullptr), m->wo.assign(c.n_layers, nullptr);
    m->w13.assign(c.n_layers, nullptr), m->w2.assign(c.n_layers, nullptr);
    m->rms_att.assign(c.n_layers, nullptr), m->rms_ffn.assign(c.n_layers, nullptr);
    m->rms_sub_att.assign(c.n_layers, nullptr), m->rms_sub_ffn.assign(c.n_layers, nullptr);
    m->mul_att.assign(c.n_layers, nullptr), m->mul_ffn.assign(c.n_layers, nullptr);
    m->mul_sub_att.assign(c.n_layers, nullptr), m->mul_sub_ffn.assign(c.n_layers, nullptr);
    if (hipMalloc(&m->x, sizeof(float) * c.dim) != hipSuccess ||
        hipMalloc(&m->qkv, sizeof(float) * (m->q_dim + 2 * m->kv_dim)) != hipSuccess ||
        hipMalloc(&m->hb, sizeof(float) * 2 * c.hidden) != hipSuccess ||
        hipMalloc(&m->logits, sizeof(float) * c.vocab) != hipSuccess ||
        hipMalloc(&m->kc, sizeof(__half) * cache) != hipSuccess ||
        hipMalloc(&m->vc, sizeof(__half) * cache) != hipSuccess ||
        hipMalloc(&m->state, sizeof(int) * 4) != hipSuccess ||
        hipMalloc(&m->prompt, sizeof(int) * c.seq_len) != hipSuccess ||
        hipMalloc(&m->seq, sizeof(int) * c.seq_len) != hipSuccess) {
        eif_hip_bitnet_destroy(m);
        return EIF_HIP_E_NOMEM;
    }
    // defined device state before the first reset (steps and prefill refuse to run until then)
    if (hipMemset(m->state, 0, sizeof(int) * 4) != hipSuccess ||
        hipMemset(m->prompt, 0, sizeof(int) * c.seq_len) != hipSuccess ||
        hipMemset(m->seq, 0, sizeof(int) * c.seq_len) != hipSuccess) {
        eif_hip_bitnet_destroy(m);
        return EIF_HIP_E_DEVICE;
    }
    // the shares start at zero: a share a step does not reach keeps finite values, weighed by 0
    const size_t n_sh_o = (size_t)c.n_heads * kAttnShares * c.head_dim, n_sh_ml = (size_t)c.n_heads * 2 * kAttnShares;
    if (hipMalloc(&m->rope, sizeof(float2) * c.seq_len * (c.head_dim / 2)) != hipSuccess ||
        hipMalloc(&m->sh_o, sizeof(float) * n_sh_o) != hipSuccess ||
        hipMalloc(&m->sh_ml, sizeof(float) * n_sh_ml) != hipSuccess ||
        hipMemset(m->sh_o, 0, sizeof(float) * n_sh_o) != hipSuccess ||
        hipMemset(m->sh_ml, 0, sizeof(float) * n_sh_ml) != hipSuccess) {
        eif_hip_bitnet_destroy(m);
        return EIF_HIP_E_NOMEM;
    }
    rope_table_kernel<<<256, 256, 0, nullptr>>>(m->rope, c.seq_len, c.head_dim, c.rope_theta);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(nullptr) != hipSuccess) {
        eif_hip_bitnet_destroy(m);
        return EIF_HIP_E_DEVICE;
    }
    *out = m;
    return EIF_HIP_OK;
}

int eif_hip_bitnet_set_layer(eif_hip_bitnet *m, int l, const eif_hip_bitnet_layer *w)
{
    if (!m || !w || l < 0 || l >= m->c.n_layers || !w->wq || !w->wk || !w->wv || !w->wo || !w->w1 || !w->w3 ||
        !w->w2 || !w->gq || !w->gk || !w->gv || !w->go || !w->g1 || !w->g3 || !w->g2)
        return EIF_HIP_E_ARG;
    const eif_hip_bitnet_config &c = m->c;
    if (m->exec) return EIF_HIP_E_ARG;   // weights are baked into the captured step
    if (m->wqkv[l]) return EIF_HIP_E_ARG;   // each layer is set once
    // All of the layer's device objects are made first and kept only when every one succeeded: a failed call
    // leaves the layer unset (and may be repeated).
    eif_hip_qweight *qkv = nullptr, *wo = nullptr, *w13 = nullptr, *w2 = nullptr;
    float *n_att = nullptr, *n_ffn = nullptr, *n_sa = nullptr, *n_sf = nullptr;
    size_t bytes = 0;
    std::vector<uint8_t> codes;
    std::vector<float> scales;
    int rc;
    do {
        try {
            stack_rows(codes, scales, w->wq, w->gq, m->q_dim, c.dim, c.g_q);
            stack_rows(codes, scales, w->wk, w->gk, m->kv_dim, c.dim, c.g_q);
            stack_rows(codes, scales, w->wv, w->gv, m->kv_dim, c.dim, c.g_q);
        } catch (const std::bad_alloc &) {
            rc = EIF_HIP_E_NOMEM;
            break;
        }
        if ((rc = make_tern(&qkv, codes, scales, m->q_dim + 2 * m->kv_dim, c.dim, c.g_q, &bytes))) break;
        codes.clear(), scales.clear();
        try {
            stack_rows(codes, scales, w->wo, w->go, c.dim, m->q_dim, c.g_o);
        } catch (const std::bad_alloc &) {
            rc = EIF_HIP_E_NOMEM;
            break;
        }
        if ((rc = make_tern(&wo, codes, scales, c.dim, m->q_dim, c.g_o, &bytes))) break;
        codes.clear(), scales.clear();
        try {
            stack_rows(codes, scales, w->w1, w->g1, c.hidden, c.dim, c.g_13);
            stack_rows(codes, scales, w->w3, w->g3, c.hidden, c.dim, c.g_13);
        } catch (const std::bad_alloc &) {
            rc = EIF_HIP_E_NOMEM;
            break;
        }
        if ((rc = make_tern(&w13, codes, scales, 2 * c.hidden, c.dim, c.g_13, &bytes))) break;
        codes.clear(), scales.clear();
        try {
            stack_rows(codes, scales, w->w2, w->g2, c.dim, c.hidden, c.g_2);
        } catch (const std::bad_alloc &) {
            rc = EIF_HIP_E_NOMEM;
            break;
        }
        if ((rc = make_tern(&w2, codes, scales, c.dim, c.hidden, c.g_2, &bytes))) break;
        if ((rc = dev_upload(&n_att, w->rms_att, c.dim)) || (rc = dev_upload(&n_ffn, w->rms_ffn, c.dim)) ||
            (rc = dev_upload(&n_sa, w->rms_sub_att, m->q_dim)) || (rc = dev_upload(&n_sf, w->rms_sub_ffn, c.hidden)))
            break;
    } while (false);
    if (rc) {
        for (eif_hip_qweight *q : {qkv, wo, w13, w2}) eif_hip_qweight_destroy(q);
        for (float *p : {n_att, n_ffn, n_sa, n_sf})
            if (p) (void)hipFree(p);
        return rc;
    }
    m->wqkv[l] = qkv, m->wo[l] = wo, m->w13[l] = w13, m->w2[l] = w2;
    m->rms_att[l] = n_att, m->rms_ffn[l] = n_ffn, m->rms_sub_att[l] = n_sa, m->rms_sub_ffn[l] = n_sf;
    m->weight_bytes += bytes + sizeof(float) * (2 * c.dim + m->q_dim + c.hidden);
    return m->head ? fold_signs(m, l) : EIF_HIP_OK;   // the signs are set (eif_hip_bitnet_set_globals)
}

int eif_hip_bitnet_set_globals(eif_hip_bitnet *m, const eif_hip_bitnet_globals *g)
{
    if (!m || !g || !g->emb || !g->wcls) return EIF_HIP_E_ARG;
    if (m->exec || m->head) return EIF_HIP_E_ARG;   // once, before the first captured step
    const eif_hip_bitnet_config &c = m->c;
    int rc;
    if ((rc = dev_upload(&m->emb, g->emb, (size_t)c.vocab * c.dim)) ||
        (rc = dev_upload(&m->emb_scale, g->emb_scale, (size_t)c.vocab)) ||
        (rc = dev_upload(&m->rms_final, g->rms_final, (size_t)c.dim)) ||
        (rc = dev_upload(&m->signs_dim, g->signs_dim, (size_t)c.dim)) ||
        (rc = dev_upload(&m->signs_q, g->signs_q, (size_t)m->q_dim)) ||
        (rc = dev_upload(&m->signs_hidden, g->signs_hidden, (size_t)c.hidden)))
        return rc;
    if ((rc = eif_hip_qweight_create(&m->head, EIF_HIP_W_INT8, c.vocab, c.dim, 0, g->wcls, g->wcls_scale, 0,
                                     nullptr)))
        return rc;
    size_t b = 0;
    int kp = 0;
    eif_hip_qweight_info(m->head, nullptr, nullptr, &kp, nullptr, &b);
    m->weight_bytes += b + sizeof(float) * c.dim;
    m->head_kpad = kp;
    m->head_tiles = eif::qweight_row_tiles(m->head);
    auto pm1 = [](const float *s, int n, int block) {
        if (!s || block <= 0) return false;
        for (int i = 0; i < n; ++i)
            if (s[i] != 1.0f && s[i] != -1.0f) return false;
        return true;
    };
    m->fold_dim = pm1(g->signs_dim, c.dim, c.wht_dim);
    m->fold_q = pm1(g->signs_q, m->q_dim, c.wht_q);
    m->fold_hidden = pm1(g->signs_hidden, c.hidden, c.wht_hidden);
    for (int l = 0; l < c.n_layers; ++l)
        if (m->rms_att[l] && (rc = fold_signs(m, l))) return rc;
    if (hipMalloc(&m->hq, (size_t)kp) != hipSuccess || hipMalloc(&m->hs, sizeof(float) * 4) != hipSuccess ||
        hipMalloc(&m->amax_key, sizeof(unsigned long long) * kArgmaxSlots * kArgmaxStride) != hipSuccess ||
        hipMemset(m->amax_key, 0, sizeof(unsigned long long) * kArgmaxSlots * kArgmaxStride) != hipSuccess)
        return EIF_HIP_E_NOMEM;
    return EIF_HIP_OK;
}

int eif_hip_bitnet_reset(eif_hip_bitnet *m, const int *prompt, int n_prompt, void *stream)
{
    if (!m || !prompt || n_prompt < 1 || n_prompt > m->c.seq_len || !m->emb || !m->head) return EIF_HIP_E_ARG;
    for (int i = 0; i < n_prompt; ++i)
        if (prompt[i] < 0 || prompt[i] >= m->c.vocab) return EIF_HIP_E_ARG;
    hipStream_t st = (hipStream_t)stream;
    const eif_hip_bitnet_config &c = m->c;
    const size_t cache = (size_t)c.n_layers * c.n_kv_heads * c.seq_len * c.head_dim;
    EIF_HIP_TRY(hipMemcpyAsync(m->prompt, prompt, sizeof(int) * n_prompt, hipMemcpyHostToDevice, st));
    fill_half_kernel<<<1024, 256, 0, st>>>(m->kc, cache);
    EIF_HIP_LAUNCHED();
    fill_half_kernel<<<1024, 256, 0, st>>>(m->vc, cache);
    EIF_HIP_LAUNCHED();
    if (m->plan && eif::persist_reset(m->plan, st)) return EIF_HIP_E_DEVICE;
    start_kernel<<<1, 1, 0, st>>>(m->state, m->seq, m->prompt, n_prompt);
    EIF_HIP_LAUNCHED();
    embed_kernel<<<1, 256, 0, st>>>(m->emb, m->emb_scale, m->state, m->x, c.dim, c.vocab);   // each step
    EIF_HIP_LAUNCHED();                                                                      // leaves the next
    EIF_HIP_TRY(hipStreamSynchronize(st));   // the prompt buffer is the caller's
    m->hpos = 0;
    m->n_prompt = n_prompt;
    return EIF_HIP_OK;
}

int eif_hip_bitnet_steps(eif_hip_bitnet *m, int n, int use_graph, void *stream)
{
    if (!m || n < 0 || !m->head || !m->emb) return EIF_HIP_E_ARG;
    if (m->n_prompt == 0) return EIF_HIP_E_ARG;   // no eif_hip_bitnet_reset yet: no position or token
    for (int l = 0; l < m->c.n_layers; ++l)
        if (!m->wqkv[l]) return EIF_HIP_E_ARG;
    if (m->hpos + n > m->c.seq_len) return EIF_HIP_E_LIMIT;
    hipStream_t st = (hipStream_t)stream;
    ensure_plan(m);
    if (use_graph && !m->exec) {   // capture once, on the model's own stream; replay on the caller's
        if (!m->cap) EIF_HIP_TRY(hipStreamCreateWithFlags(&m->cap, hipStreamNonBlocking));
        EIF_HIP_TRY(hipStreamBeginCapture(m->cap, hipStreamCaptureModeRelaxed));
        const int rc = enqueue_step(m, m->cap);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(m->cap, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        EIF_HIP_TRY(e);
        m->graph = g;
        EIF_HIP_TRY(hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0));
    }
    for (int i = 0; i < n; ++i) {
        if (use_graph) {
            EIF_HIP_TRY(hipGraphLaunch(m->exec, st));
        } else {
            const int rc = enqueue_step(m, st);
            if (rc) return rc;
        }
        ++m->hpos;
    }
    return EIF_HIP_OK;
}

int eif_hip_bitnet_prefill(eif_hip_bitnet *m, int n, void *stream)
{
    if (!m || n < 1 || !m->head || !m->emb) return EIF_HIP_E_ARG;
    for (int l = 0; l < m->c.n_layers; ++l)
        if (!m->wqkv[l]) return EIF_HIP_E_ARG;
    if (m->hpos + n > m->n_prompt) return EIF_HIP_E_ARG;   // prompt tokens only
    int rc = ensure_prefill(m, n);
    if (rc) return rc;
    if ((rc = enqueue_prefill(m, m->hpos, n, (hipStream_t)stream))) return rc;
    m->hpos += n;
    return EIF_HIP_OK;
}

int eif_hip_bitnet_tokens(eif_hip_bitnet *m, int *out, int n, void *stream)
{
    if (!m || !out || n < 0 || n > m->c.seq_len) return EIF_HIP_E_ARG;
    if (const int rc = check_plan(m, (hipStream_t)stream)) return rc;
    EIF_HIP_TRY(hipMemcpyAsync(out, m->seq, sizeof(int) * n, hipMemcpyDeviceToHost, (hipStream_t)stream));
    EIF_HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return EIF_HIP_OK;
}

int eif_hip_bitnet_logits(eif_hip_bitnet *m, float *out, void *stream)
{
    if (!m || !out) return EIF_HIP_E_ARG;
    if (const int rc = check_plan(m, (hipStream_t)stream)) return rc;
    EIF_HIP_TRY(hipMemcpyAsync(out, m->logits, sizeof(float) * m->c.vocab, hipMemcpyDeviceToHost, (hipStream_t)stream));
    EIF_HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return EIF_HIP_OK;
}

int eif_hip_bitnet_position(eif_hip_bitnet *m, void *stream)
{
    if (!m) return EIF_HIP_E_ARG;
    if (const int rc = check_plan(m, (hipStream_t)stream)) return rc;
    int s[4];
    EIF_HIP_TRY(hipMemcpyAsync(s, m->state, sizeof(s), hipMemcpyDeviceToHost, (hipStream_t)stream));
    EIF_HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return s[0];
}

int eif_hip_bitnet_kv_cache(eif_hip_bitnet *m, int layer, int pos0, int n, float *k, float *v, void *stream)
{
    if (!m || !k || !v || layer < 0 || layer >= m->c.n_layers || pos0 < 0 || n < 0 || pos0 + n > m->c.seq_len)
        return EIF_HIP_E_ARG;
    const eif_hip_bitnet_config &c = m->c;
    std::vector<__half> hk((size_t)c.n_kv_heads * n * c.head_dim), hv(hk.size());
    const size_t cache_l = (size_t)layer * c.n_kv_heads * c.seq_len * c.head_dim;
    hipStream_t st = (hipStream_t)stream;
    for (int g = 0; g < c.n_kv_heads; ++g) {
        const size_t src = cache_l + ((size_t)g * c.seq_len + pos0) * c.head_dim, cnt = (size_t)n * c.head_dim;
        EIF_HIP_TRY(hipMemcpyAsync(hk.data() + g * cnt, m->kc + src, cnt * sizeof(__half), hipMemcpyDeviceToHost, st));
        EIF_HIP_TRY(hipMemcpyAsync(hv.data() + g * cnt, m->vc + src, cnt * sizeof(__half), hipMemcpyDeviceToHost, st));
    }
    EIF_HIP_TRY(hipStreamSynchronize(st));
    for (int g = 0; g < c.n_kv_heads; ++g)
        for (int p = 0; p < n; ++p)
            for (int i = 0; i < c.head_dim; ++i) {
                const size_t s = ((size_t)g * n + p) * c.head_dim + i, d = (size_t)p * m->kv_dim + g * c.head_dim + i;
                k[d] = __half2float(hk[s]);
                v[d] = __half2float(hv[s]);
            }
    return EIF_HIP_OK;
}

int eif_hip_bitnet_set_persistent(eif_hip_bitnet *m, int on)
{
    if (!m || on < -1 || on > 1) return EIF_HIP_E_ARG;
    for (int l = 0; l < m->c.n_layers; ++l)
        if (!m->wqkv[l]) return EIF_HIP_E_ARG;
    if (!m->head) return EIF_HIP_E_ARG;
    ensure_plan(m);
    if (on >= 0 && on != m->use_persist) {
        m->use_persist = on;
        if (m->exec) {   // the captured step holds the other path: capture again at the next graph step
            (void)hipGraphExecDestroy(m->exec);
            (void)hipGraphDestroy(m->graph);
            m->exec = nullptr, m->graph = nullptr;
        }
    }
    return m->plan && m->use_persist ? 1 : 0;
}

int eif_hip_bitnet_get_config(const eif_hip_bitnet *m, eif_hip_bitnet_config *out)
{
    if (!m || !out) return EIF_HIP_E_ARG;
    *out = m->c;
    return EIF_HIP_OK;
}

size_t eif_hip_bitnet_weight_bytes(const eif_hip_bitnet *m) { return m ? m->weight_bytes : 0; }

size_t eif_hip_bitnet_kv_bytes(const eif_hip_bitnet *m, int p)
{
    if (!m) return 0;
    return (size_t)m->c.n_layers * m->c.n_kv_heads * (size_t)(p + 1) * m->c.head_dim * 2 * sizeof(__half);
}

void eif_hip_bitnet_destroy(eif_hip_bitnet *m)
{
    if (!m) return;
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    if (m->cap) (void)hipStreamDestroy(m->cap);
    eif::persist_destroy(m->plan);
    free_prefill(m);
    for (auto *v : {&m->wqkv, &m->wo, &m->w13, &m->w2})
        for (eif_hip_qweight *q : *v) eif_hip_qweight_destroy(q);
    eif_hip_qweight_destroy(m->head);
    for (auto *v : {&m->rms_att, &m->rms_ffn, &m->rms_sub_att, &m->rms_sub_ffn, &m->mul_att, &m->mul_ffn,
                    &m->mul_sub_att, &m->mul_sub_ffn})
        for (float *p : *v)
            if (p) (void)hipFree(p);
    for (void *p : {(void *)m->rms_final, (void *)m->signs_dim, (void *)m->signs_q, (void *)m->signs_hidden,
                    (void *)m->emb, (void *)m->emb_scale, (void *)m->x, (void *)m->qkv, (void *)m->hb,
                    (void *)m->logits, (void *)m->kc, (void *)m->vc, (void *)m->state, (void *)m->prompt,
                    (void *)m->seq, (void *)m->hq, (void *)m->hs, (void *)m->amax_key,
                    (void *)m->rope, (void *)m->sh_o, (void *)m->sh_ml})
        if (p) (void)hipFree(p);
    delete m;
}

}  // extern "C"

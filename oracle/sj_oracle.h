/*
 * sj_oracle.h -- CPU restatement of snapjudge's DecisionModel forward.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product (libsnapjudge_hip.so) never links,
 * loads or calls it.
 *
 * Every function restates one reference routine in plain C and cites the
 * reference file:line it follows (paths are relative to the reference tree).
 * The arithmetic types and operation order follow the reference so that, built
 * with -ffp-contract=off, results match the reference CPU build bit for bit
 * (the reference's no-BLAS GEMM, src/cblas_fallback.cpp:22-47, is a per-element
 * k-ordered float dot product, and that is what orc_gemm_nt does).
 *
 * Pinning (each function is checked by tests/test_oracle.py):
 *   - tensor ops against the reference's own golden vectors
 *     (tests/golden/tensor_ops.json, used by tests/test_tensor.cpp:58-100);
 *   - encode/forward against the compiled reference (oracle/_ref) on the
 *     reference's tiny checkpoint and on synthetic checkpoints;
 *   - closed forms: RoPE tables (cos^2+sin^2, pos 0), LayerNorm moments,
 *     attention with constant keys (uniform weights -> mean of V), window
 *     semantics |i-j| <= w, key padding invariance, softmax/entropy identities.
 */
#ifndef SJ_ORACLE_H
#define SJ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One encoder layer (reference LayerWeights, include/snapjudge/model.hpp:37-44). */
typedef struct {
  const float* attn_norm; /* [D] or NULL: layer 0 has none (src/model.cpp:112-117) */
  const float* wqkv;      /* [3D, D] */
  const float* wo;        /* [D, D] */
  const float* mlp_norm;  /* [D] */
  const float* wi;        /* [2F, D]: rows [0,F) input, [F,2F) gate */
  const float* wo2;       /* [D, F] */
  int32_t window;         /* 0 = full; else local_attention/2 (src/model.cpp:103,111) */
  int32_t sliding;        /* 1: sliding RoPE tables (src/model.cpp:257-263) */
} orc_layer;

/* One decision-head layer (src/model.cpp:107-111). */
typedef struct {
  const float *n1w, *n1b, *n2w, *n2b;
  const float *in_w, *in_b;   /* [3D, D], [3D] */
  const float *out_w, *out_b; /* [D, D], [D] */
  const float *l1w, *l1b;     /* [4D, D], [4D] */
  const float *l2w, *l2b;     /* [D, 4D], [D] */
} orc_head_layer;

/* All DecisionModel state the forward reads (src/model.cpp:89-126). */
typedef struct {
  int64_t D, H, F, V, n_layers, max_pos, n_act, head_layers, lora_r;
  float eps;
  const float* emb_w;      /* [V, D] */
  const float* emb_norm;   /* [D] */
  const float* final_norm; /* [D] */
  const float *rope_cos_full, *rope_sin_full;   /* [max_pos, Dh/2] */
  const float *rope_cos_slide, *rope_sin_slide; /* [max_pos, Dh/2] */
  const orc_layer* layers;
  const float* lora_a; /* [r, D] or NULL */
  const float* lora_b; /* [D, r] or NULL */
  const float* type_emb; /* [3, D] */
  const orc_head_layer* head;
  const float *sc_ln_w, *sc_ln_b; /* [D], [D] or NULL */
  const float *sc_w1, *sc_b1;     /* [D, D], [D] or NULL */
  const float *sc_w2, *sc_b2;     /* [1, D], [1] or NULL */
  const float *act_w1, *act_b1;   /* [256, D+4], [256] */
  const float *act_w2, *act_b2;   /* [n_act, 256], [n_act] */
} orc_model;

/* ---- tensor ops (src/tensor.cpp) ---- */
void orc_layer_norm(const float* x, int64_t rows, int64_t D, const float* w,
                    const float* b, float eps, float* out);
float orc_gelu_erf(float x);
void orc_softmax_rows(float* x, int64_t rows, int64_t K);
void orc_gemm_nt(const float* a, const float* w, const float* bias, int act, int64_t M,
                 int64_t N, int64_t K, float* out);
void orc_gemm_geglu(const float* a, const float* wi, int64_t M, int64_t F, int64_t K,
                    float* out);
void orc_attention(const float* q, const float* k, const float* v, const int64_t* lens,
                   int64_t B, int64_t H, int64_t L, int64_t Dh, int window, float* out);
void orc_embedding(const float* table, int64_t D, const int64_t* ids, int64_t n,
                   float* out);
void orc_rope_inplace(float* qkv, int64_t M, const float* cos_t, const float* sin_t,
                      int64_t L, int64_t H, int64_t Dh);

/* ---- model (src/model.cpp) ---- */
void orc_rope_table(double theta, int64_t max_pos, int64_t Dh, float* cos_t,
                    float* sin_t);
/* encode: hidden states [B, L, D] for every position (padding included). */
int orc_encode(const orc_model* m, const int64_t* ids, const int64_t* mask, int64_t B,
               int64_t L, float* out);
/* forward: logits [B, K] (masked = -1e4), act [B, n_act]; optionally the
 * post-head hidden states [B, L, D] (NULL to skip). */
int orc_forward(const orc_model* m, const int64_t* ids, const int64_t* mask,
                const int64_t* marker_pos, const uint8_t* marker_mask,
                const int64_t* qtype, int64_t B, int64_t L, int64_t K, float* logits,
                float* act, float* hidden_out);

/* ---- SjModel, snapjudge's own BERT-style model (src/sj_model.cpp) ---- */

/* One layer of the encoder or of the head (src/sj_model.cpp EncLayer /
 * HeadLayer, include/snapjudge/sj_model.hpp:79-101): pre-norm attention with
 * separate q/k/v/o projections and biases, then a pre-norm GELU FFN with
 * biases.  For a head layer n1 -> an_*, n2 -> fn_*. */
typedef struct {
  const float *an_w, *an_b;             /* [D] */
  const float *q_w, *q_b, *k_w, *k_b;   /* [D, D], [D] */
  const float *v_w, *v_b, *o_w, *o_b;   /* [D, D], [D] */
  const float *fn_w, *fn_b;             /* [D] */
  const float *w1_w, *w1_b;             /* [F, D], [F] */
  const float *w2_w, *w2_b;             /* [D, F], [D] */
} orc_sj_layer;

typedef struct {
  int64_t D, H, F, V, n_layers, max_pos, head_layers, head_ff;
  float eps;
  const float *word_emb, *pos_emb;      /* [V, D], [max_pos, D] */
  const float *emb_norm_w, *emb_norm_b; /* [D] */
  const orc_sj_layer* layers;           /* F = intermediate_size */
  const float *final_norm_w, *final_norm_b;
  const float* type_emb;                /* [n_types, D] */
  const orc_sj_layer* head;             /* F = head_intermediate */
  const float *sc_n_w, *sc_n_b, *sc_w1, *sc_b1, *sc_w2, *sc_b2;
} orc_sj_model;

/* SjModel::encode (src/sj_model.cpp:257-275): [B, L, D], padding included. */
int orc_sj_encode(const orc_sj_model* m, const int64_t* ids, const int64_t* mask, int64_t B,
                  int64_t L, float* out);
/* SjModel::forward (src/sj_model.cpp:277-368): logits [B, K] (masked -1e4),
 * act [B, 2] = {top1, 1 - top1}; optionally the post-head hidden [B, L, D]. */
int orc_sj_forward(const orc_sj_model* m, const int64_t* ids, const int64_t* mask,
                   const int64_t* marker_pos, const uint8_t* marker_mask, const int64_t* qtype,
                   int64_t B, int64_t L, int64_t K, float* logits, float* act, float* hidden_out);

/* ---- answer decoding (src/agent.cpp:256-266, src/common.cpp:199-237) ---- */
double orc_clamp_temperature(double t);
void orc_calibrated_probs(const float* logits, int k, double t_scale, double* p);
double orc_confidence_from_probs(const double* p, int k);
double orc_round4(double v);

#ifdef __cplusplus
}
#endif
#endif /* SJ_ORACLE_H */

/*
 * sj_oracle.c -- CPU restatement of snapjudge's DecisionModel forward.
 *
 * TEST INFRASTRUCTURE ONLY (see sj_oracle.h).  Build with -ffp-contract=off:
 * the reference's float expressions are evaluated one rounding at a time.
 */
#include "sj_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ORC_ALLOC(n, T) ((T*)malloc((size_t)(n) * sizeof(T)))

/* src/tensor.cpp:54-79 -- mean and population variance accumulated in double,
 * inverse std rounded to float, then (x - (float)mean) * inv * w (+ b) in float. */
void orc_layer_norm(const float* x, int64_t rows, int64_t D, const float* w,
                    const float* b, float eps, float* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * D;
    float* o = out + r * D;
    double mean = 0.0;
    for (int64_t j = 0; j < D; ++j) mean += xr[j];
    mean /= (double)D;
    double var = 0.0;
    for (int64_t j = 0; j < D; ++j) {
      double d = (double)xr[j] - mean;
      var += d * d;
    }
    var /= (double)D;
    float inv = (float)(1.0 / sqrt(var + (double)eps));
    float fmean = (float)mean;
    for (int64_t j = 0; j < D; ++j) {
      float v = (xr[j] - fmean) * inv;
      v = v * (w ? w[j] : 1.0f);
      o[j] = b ? v + b[j] : v;
    }
  }
}

/* src/tensor.cpp:96-98 -- exact erf GELU in float. */
float orc_gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654757f)); }

/* src/tensor.cpp:81-94 -- float max, float exp, double sum, float 1/sum. */
void orc_softmax_rows(float* x, int64_t rows, int64_t K) {
  for (int64_t r = 0; r < rows; ++r) {
    float* xr = x + r * K;
    float m = xr[0];
    for (int64_t j = 1; j < K; ++j) m = xr[j] > m ? xr[j] : m;
    double s = 0.0;
    for (int64_t j = 0; j < K; ++j) {
      xr[j] = expf(xr[j] - m);
      s += xr[j];
    }
    float inv = (float)(1.0 / s);
    for (int64_t j = 0; j < K; ++j) xr[j] *= inv;
  }
}

/* src/tensor.cpp:108-131 over src/cblas_fallback.cpp:22-47 (row-major, A
 * NoTrans, W Trans, alpha 1, beta 0): out[i][j] = sum_k a[i][k]*w[j][k] as a
 * float accumulation in k order; then bias add and activation (1 = erf-GELU,
 * 2 = ReLU) in a second pass. */
void orc_gemm_nt(const float* a, const float* w, const float* bias, int act, int64_t M,
                 int64_t N, int64_t K, float* out) {
  for (int64_t i = 0; i < M; ++i) {
    const float* ar = a + i * K;
    for (int64_t j = 0; j < N; ++j) {
      const float* wr = w + j * K;
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) acc += ar[k] * wr[k];
      float v = 1.0f * acc;
      if (bias) v += bias[j];
      if (act == 1) v = orc_gelu_erf(v);
      else if (act == 2) v = v > 0.0f ? v : 0.0f;
      out[i * N + j] = v;
    }
  }
}

/* src/tensor.cpp:133-151 -- tmp = a @ wi^T ([M, 2F]); out[:, j] =
 * gelu(tmp[:, j]) * tmp[:, F + j]: the first F rows of wi are the input half,
 * the last F rows the gate half. */
void orc_gemm_geglu(const float* a, const float* wi, int64_t M, int64_t F, int64_t K,
                    float* out) {
  float* tmp = ORC_ALLOC(M * 2 * F, float);
  orc_gemm_nt(a, wi, NULL, 0, M, 2 * F, K, tmp);
  for (int64_t r = 0; r < M; ++r)
    for (int64_t j = 0; j < F; ++j)
      out[r * F + j] = orc_gelu_erf(tmp[r * 2 * F + j]) * tmp[r * 2 * F + F + j];
  free(tmp);
}

/* src/tensor.cpp:156-228 -- q/k/v [B, H, L, Dh]; every query row i (padded ones
 * too) attends to keys j in [lo, hi) with hi = len (full) or
 * [max(0, i-w), min(len, i+w+1)) (window w > 0).  Scores are float dot
 * products times 1/sqrt(Dh); exp(s - max) in float; the normaliser summed in
 * double; output accumulated in float as sum_j (e_j * (float)(1/l)) * v_j.
 * The reference's thread team only splits (b, h) work items; each item's
 * arithmetic is sequential, so this single-threaded loop is identical. */
void orc_attention(const float* q, const float* k, const float* v, const int64_t* lens,
                   int64_t B, int64_t H, int64_t L, int64_t Dh, int window, float* out) {
  const float scale = 1.0f / sqrtf((float)Dh);
  float* scores = ORC_ALLOC(L > 0 ? L : 1, float);
  for (int64_t b = 0; b < B; ++b) {
    int64_t len = lens ? lens[b] : L;
    for (int64_t h = 0; h < H; ++h) {
      const float* qb = q + ((b * H + h) * L) * Dh;
      const float* kb = k + ((b * H + h) * L) * Dh;
      const float* vb = v + ((b * H + h) * L) * Dh;
      float* ob = out + ((b * H + h) * L) * Dh;
      for (int64_t i = 0; i < L; ++i) {
        const float* qi = qb + i * Dh;
        int64_t lo = 0, hi = len;
        if (window > 0) {
          lo = i - window > 0 ? i - window : 0;
          hi = i + window + 1 < len ? i + window + 1 : len;
        }
        float m = -INFINITY;
        for (int64_t j = lo; j < hi; ++j) {
          const float* kj = kb + j * Dh;
          float s = 0.0f;
          for (int64_t d = 0; d < Dh; ++d) s += qi[d] * kj[d];
          scores[j] = s * scale;
          m = scores[j] > m ? scores[j] : m;
        }
        double l = 0.0;
        for (int64_t j = lo; j < hi; ++j) {
          float e = expf(scores[j] - m);
          scores[j] = e;
          l += e;
        }
        float linv = (float)(1.0 / l);
        float* oi = ob + i * Dh;
        for (int64_t d = 0; d < Dh; ++d) oi[d] = 0.0f;
        for (int64_t j = lo; j < hi; ++j) {
          float wgt = scores[j] * linv;
          const float* vj = vb + j * Dh;
          for (int64_t d = 0; d < Dh; ++d) oi[d] += wgt * vj[d];
        }
      }
    }
  }
  free(scores);
}

/* src/tensor.cpp:247-255 -- row gather. */
void orc_embedding(const float* table, int64_t D, const int64_t* ids, int64_t n,
                   float* out) {
  for (int64_t r = 0; r < n; ++r)
    memcpy(out + r * D, table + ids[r] * D, sizeof(float) * (size_t)D);
}

/* src/tensor.cpp:257-279 -- rotate-half on the 2H q and k heads of each packed
 * (q|k|v)(head)(dim) row; pairs (d, d + Dh/2); row r is at position r % L. */
void orc_rope_inplace(float* qkv, int64_t M, const float* cos_t, const float* sin_t,
                      int64_t L, int64_t H, int64_t Dh) {
  const int64_t half = Dh / 2;
  for (int64_t r = 0; r < M; ++r) {
    const int64_t pos = r % L;
    const float* cr = cos_t + pos * half;
    const float* sr = sin_t + pos * half;
    float* row = qkv + r * 3 * H * Dh;
    for (int64_t hh = 0; hh < 2 * H; ++hh) {
      float* x = row + hh * Dh;
      for (int64_t d = 0; d < half; ++d) {
        float x0 = x[d], x1 = x[d + half];
        float c = cr[d], s = sr[d];
        float a0 = x0 * c, b0 = x1 * s;
        float a1 = x1 * c, b1 = x0 * s;
        x[d] = a0 - b0;
        x[d + half] = a1 + b1;
      }
    }
  }
}

/* src/model.cpp:173-190 -- inv = 1/theta^(2d/Dh) and cos/sin(pos*inv) in double,
 * rounded to float.  Tables are [max_pos, Dh/2]. */
void orc_rope_table(double theta, int64_t max_pos, int64_t Dh, float* cos_t,
                    float* sin_t) {
  const int64_t half = Dh / 2;
  for (int64_t pos = 0; pos < max_pos; ++pos)
    for (int64_t d = 0; d < half; ++d) {
      double inv = 1.0 / pow(theta, 2.0 * (double)d / (double)Dh);
      double fr = (double)pos * inv;
      cos_t[pos * half + d] = (float)cos(fr);
      sin_t[pos * half + d] = (float)sin(fr);
    }
}

/* [M, 3*H*Dh] packed rows -> three [B, H, L, Dh] blocks (src/model.cpp:368-380). */
static void split_heads(const float* qkv, int64_t B, int64_t L, int64_t H, int64_t Dh,
                        float* Q, float* K, float* V) {
  const int64_t HD = H * Dh;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t i = 0; i < L; ++i) {
      const float* row = qkv + (b * L + i) * 3 * HD;
      for (int64_t h = 0; h < H; ++h) {
        int64_t dst = ((b * H + h) * L + i) * Dh;
        memcpy(Q + dst, row + h * Dh, sizeof(float) * (size_t)Dh);
        memcpy(K + dst, row + HD + h * Dh, sizeof(float) * (size_t)Dh);
        memcpy(V + dst, row + 2 * HD + h * Dh, sizeof(float) * (size_t)Dh);
      }
    }
}

/* [B, H, L, Dh] -> [M, H*Dh] rows (src/model.cpp:382-387). */
static void merge_heads(const float* At, int64_t B, int64_t L, int64_t H, int64_t Dh,
                        float* O) {
  for (int64_t b = 0; b < B; ++b)
    for (int64_t i = 0; i < L; ++i)
      for (int64_t h = 0; h < H; ++h)
        memcpy(O + (b * L + i) * H * Dh + h * Dh, At + ((b * H + h) * L + i) * Dh,
               sizeof(float) * (size_t)Dh);
}

static void add_inplace(float* a, const float* b, int64_t n) {
  for (int64_t i = 0; i < n; ++i) a[i] += b[i];
}

/* Encoder half shared by encode (src/model.cpp:222-307) and forward
 * (src/model.cpp:309-407): embeddings + emb norm, the layer stack, the final
 * norm and the optional LoRA adapter.  Writes h [M, D]. */
static void encoder_stack(const orc_model* m, const int64_t* ids, const int64_t* lens,
                          int64_t B, int64_t L, float* h) {
  const int64_t D = m->D, H = m->H, Dh = D / H, F = m->F, M = B * L;
  float* X = ORC_ALLOC(M * D, float);
  float* Y = ORC_ALLOC(M * D, float);
  float* qkv = ORC_ALLOC(M * 3 * D, float);
  float* Q = ORC_ALLOC(M * D, float);
  float* Kt = ORC_ALLOC(M * D, float);
  float* V = ORC_ALLOC(M * D, float);
  float* At = ORC_ALLOC(M * D, float);
  float* O = ORC_ALLOC(M * D, float);
  float* G = ORC_ALLOC(M * F, float);

  /* src/model.cpp:333-340: X = LN(emb[ids]) */
  orc_embedding(m->emb_w, D, ids, M, Y);
  orc_layer_norm(Y, M, D, m->emb_norm, NULL, m->eps, X);

  for (int64_t li = 0; li < m->n_layers; ++li) {
    const orc_layer* ly = &m->layers[li];
    const float* Yin = X; /* layer 0: attn_norm is Identity (src/model.cpp:350-353) */
    if (ly->attn_norm) {
      orc_layer_norm(X, M, D, ly->attn_norm, NULL, m->eps, Y);
      Yin = Y;
    }
    orc_gemm_nt(Yin, ly->wqkv, NULL, 0, M, 3 * D, D, qkv);       /* :355 */
    orc_rope_inplace(qkv, M, ly->sliding ? m->rope_cos_slide : m->rope_cos_full,
                     ly->sliding ? m->rope_sin_slide : m->rope_sin_full, L, H, Dh); /* :357-365 */
    split_heads(qkv, B, L, H, Dh, Q, Kt, V);                    /* :368-380 */
    orc_attention(Q, Kt, V, lens, B, H, L, Dh, ly->window, At);  /* :381 */
    merge_heads(At, B, L, H, Dh, O);                             /* :382-387 */
    orc_gemm_nt(O, ly->wo, NULL, 0, M, D, D, Y);                 /* :389 */
    add_inplace(X, Y, M * D);                                    /* :391 */
    orc_layer_norm(X, M, D, ly->mlp_norm, NULL, m->eps, Y);      /* :392 */
    orc_gemm_geglu(Y, ly->wi, M, F, D, G);                       /* :394 */
    orc_gemm_nt(G, ly->wo2, NULL, 0, M, D, F, Y);                /* :395 */
    add_inplace(X, Y, M * D);                                    /* :397 */
  }
  orc_layer_norm(X, M, D, m->final_norm, NULL, m->eps, h);       /* :400 */
  if (m->lora_r > 0 && m->lora_a && m->lora_b) {                 /* :402-407 */
    float* z = ORC_ALLOC(M * m->lora_r, float);
    orc_gemm_nt(h, m->lora_a, NULL, 0, M, m->lora_r, D, z);
    orc_gemm_nt(z, m->lora_b, NULL, 0, M, D, m->lora_r, Y);
    add_inplace(h, Y, M * D);
    free(z);
  }
  free(X); free(Y); free(qkv); free(Q); free(Kt); free(V); free(At); free(O); free(G);
}

/* Valid length per row = sum of the 0/1 mask (src/model.cpp:324-330). */
static void lens_from_mask(const int64_t* mask, int64_t B, int64_t L, int64_t* lens) {
  for (int64_t b = 0; b < B; ++b) {
    int64_t s = 0;
    for (int64_t i = 0; i < L; ++i) s += mask[b * L + i];
    lens[b] = s;
  }
}

int orc_encode(const orc_model* m, const int64_t* ids, const int64_t* mask, int64_t B,
               int64_t L, float* out) {
  if (B <= 0) return 0;
  int64_t* lens = ORC_ALLOC(B, int64_t);
  lens_from_mask(mask, B, L, lens);
  encoder_stack(m, ids, lens, B, L, out);
  free(lens);
  return 0;
}

/* src/model.cpp:309-536 */
int orc_forward(const orc_model* m, const int64_t* ids, const int64_t* mask,
                const int64_t* marker_pos, const uint8_t* marker_mask,
                const int64_t* qtype, int64_t B, int64_t L, int64_t K, float* logits,
                float* act, float* hidden_out) {
  if (B <= 0) return 0;
  const int64_t D = m->D, H = m->H, Dh = D / H, M = B * L;
  int64_t* lens = ORC_ALLOC(B, int64_t);
  lens_from_mask(mask, B, L, lens);
  float* h = ORC_ALLOC(M * D, float);
  encoder_stack(m, ids, lens, B, L, h);

  /* :409-416 h += type_emb[qtype] on every position */
  for (int64_t b = 0; b < B; ++b) {
    const float* te = m->type_emb + qtype[b] * D;
    for (int64_t i = 0; i < L; ++i) {
      float* hr = h + (b * L + i) * D;
      for (int64_t j = 0; j < D; ++j) hr[j] += te[j];
    }
  }

  /* :418-459 head layers: pre-norm TransformerEncoderLayer, ReLU FFN, biases,
   * LN eps 1e-5, attention without RoPE and without a window. */
  {
    float* ln = ORC_ALLOC(M * D, float);
    float* qkv = ORC_ALLOC(M * 3 * D, float);
    float* Q = ORC_ALLOC(M * D, float);
    float* Kt = ORC_ALLOC(M * D, float);
    float* V = ORC_ALLOC(M * D, float);
    float* At = ORC_ALLOC(M * D, float);
    float* AO = ORC_ALLOC(M * D, float);
    float* proj = ORC_ALLOC(M * D, float);
    float* f1 = ORC_ALLOC(M * 4 * D, float);
    for (int64_t li = 0; li < m->head_layers; ++li) {
      const orc_head_layer* hl = &m->head[li];
      orc_layer_norm(h, M, D, hl->n1w, hl->n1b, 1e-5f, ln);
      orc_gemm_nt(ln, hl->in_w, hl->in_b, 0, M, 3 * D, D, qkv);
      split_heads(qkv, B, L, H, Dh, Q, Kt, V);
      orc_attention(Q, Kt, V, lens, B, H, L, Dh, 0, At);
      merge_heads(At, B, L, H, Dh, AO);
      orc_gemm_nt(AO, hl->out_w, hl->out_b, 0, M, D, D, proj);
      add_inplace(h, proj, M * D);
      orc_layer_norm(h, M, D, hl->n2w, hl->n2b, 1e-5f, ln);
      orc_gemm_nt(ln, hl->l1w, hl->l1b, 2, M, 4 * D, D, f1);
      orc_gemm_nt(f1, hl->l2w, hl->l2b, 0, M, D, 4 * D, proj);
      add_inplace(h, proj, M * D);
    }
    free(ln); free(qkv); free(Q); free(Kt); free(V); free(At); free(AO); free(proj); free(f1);
  }
  if (hidden_out) memcpy(hidden_out, h, sizeof(float) * (size_t)(M * D));

  /* :461-487 scorer: gather marker rows (positions clamped to [0, L-1]),
   * LN(w, b; eps = norm_eps) -> Linear + GELU -> Linear(1); masked = -1e4. */
  {
    float* mk = ORC_ALLOC(B * K * D, float);
    float* s0 = ORC_ALLOC(B * K * D, float);
    float* s1 = ORC_ALLOC(B * K * D, float);
    float* s2 = ORC_ALLOC(B * K, float);
    for (int64_t b = 0; b < B; ++b)
      for (int64_t kk = 0; kk < K; ++kk) {
        int64_t p = marker_pos[b * K + kk];
        if (p < 0) p = 0;
        if (p >= L) p = L - 1;
        memcpy(mk + (b * K + kk) * D, h + (b * L + p) * D, sizeof(float) * (size_t)D);
      }
    orc_layer_norm(mk, B * K, D, m->sc_ln_w, m->sc_ln_b, m->eps, s0);
    orc_gemm_nt(s0, m->sc_w1, m->sc_b1, 1, B * K, D, D, s1);
    orc_gemm_nt(s1, m->sc_w2, m->sc_b2, 0, B * K, 1, D, s2);
    for (int64_t i = 0; i < B * K; ++i) logits[i] = marker_mask[i] ? s2[i] : -1e4f;
    free(mk); free(s0); free(s1); free(s2);
  }

  /* :489-535 act head on [CLS row, top1, top1 - top2, normalised entropy,
   * max(2, #markers)/255]: Linear(D+4, 256) + GELU -> Linear(256, n_act) ->
   * softmax (float exp, double sum). */
  {
    double* p = ORC_ALLOC(K, double);
    float* feats = ORC_ALLOC(D + 4, float);
    float* a1 = ORC_ALLOC(256, float);
    float* a2 = ORC_ALLOC(m->n_act, float);
    for (int64_t b = 0; b < B; ++b) {
      const float* lg = logits + b * K;
      float mx = lg[0];
      for (int64_t j = 1; j < K; ++j) mx = lg[j] > mx ? lg[j] : mx;
      double s = 0.0;
      for (int64_t j = 0; j < K; ++j) {
        p[j] = (double)expf(lg[j] - mx);
        s += p[j];
      }
      for (int64_t j = 0; j < K; ++j) p[j] /= s;
      double top1 = 0.0, top2 = 0.0;
      for (int64_t j = 0; j < K; ++j) {
        if (p[j] > top1) {
          top2 = top1;
          top1 = p[j];
        } else if (p[j] > top2) {
          top2 = p[j];
        }
      }
      double ksum = 0.0;
      for (int64_t kk = 0; kk < K; ++kk) ksum += marker_mask[b * K + kk];
      double kf = ksum > 2.0 ? ksum : 2.0;
      double ent = 0.0;
      for (int64_t j = 0; j < K; ++j) ent -= p[j] * log(p[j] > 1e-9 ? p[j] : 1e-9);
      ent /= log(kf);
      memcpy(feats, h + (b * L) * D, sizeof(float) * (size_t)D);
      feats[D + 0] = (float)top1;
      feats[D + 1] = (float)(top1 - top2);
      feats[D + 2] = (float)ent;
      feats[D + 3] = (float)(kf / 255.0);
      orc_gemm_nt(feats, m->act_w1, m->act_b1, 1, 1, 256, D + 4, a1);
      orc_gemm_nt(a1, m->act_w2, m->act_b2, 0, 1, m->n_act, 256, a2);
      float amx = a2[0];
      for (int64_t j = 1; j < m->n_act; ++j) amx = a2[j] > amx ? a2[j] : amx;
      double as = 0.0;
      for (int64_t j = 0; j < m->n_act; ++j) {
        a2[j] = expf(a2[j] - amx);
        as += a2[j];
      }
      for (int64_t j = 0; j < m->n_act; ++j) act[b * m->n_act + j] = (float)(a2[j] / as);
    }
    free(p); free(feats); free(a1); free(a2);
  }
  free(h);
  free(lens);
  return 0;
}

/* src/common.cpp:199-202 with TEMP_MIN 0.5, TEMP_MAX 5.0 (include/snapjudge/common.hpp:22). */
double orc_clamp_temperature(double t) {
  if (isnan(t) || isinf(t)) return 1.0;
  if (t < 0.5) return 0.5;
  if (t > 5.0) return 5.0;
  return t;
}

/* src/agent.cpp:256-266 -- z = logit / T in double, max-subtracted softmax. */
void orc_calibrated_probs(const float* logits, int k, double t_scale, double* p) {
  double mx = -INFINITY;
  for (int i = 0; i < k; ++i) {
    p[i] = (double)logits[i] / t_scale;
    if (p[i] > mx) mx = p[i];
  }
  double s = 0.0;
  for (int i = 0; i < k; ++i) {
    p[i] = exp(p[i] - mx);
    s += p[i];
  }
  for (int i = 0; i < k; ++i) p[i] /= s;
}

/* src/common.cpp:225-230 */
double orc_confidence_from_probs(const double* p, int k) {
  if (k < 2) return 1.0;
  double ent = 0.0;
  for (int i = 0; i < k; ++i) ent -= p[i] * log(p[i] > 1e-12 ? p[i] : 1e-12);
  double c = 1.0 - ent / log((double)k);
  return c < 0.0 ? 0.0 : (c > 1.0 ? 1.0 : c);
}

/* src/common.cpp:232-237 -- round half to even at 1e-4. */
double orc_round4(double v) { return nearbyint(v * 1e4) / 1e4; }

/* ------------------------------------------------------------------ SjModel */

/* src/sj_model.cpp:44-85 -- self_attention: q, k, v = three separate
 * projections with biases ([M, D] each), split into [B, H, L, Dh], full
 * attention over the first lens[b] keys (no window, no RoPE), merged back and
 * projected by o (+ bias).  Writes the projected output [M, D]. */
static void sj_self_attention(const float* Y, int64_t B, int64_t H, int64_t L, int64_t Dh,
                              const int64_t* lens, const orc_sj_layer* ly, float* out) {
  const int64_t D = H * Dh, M = B * L;
  float* q = ORC_ALLOC(M * D, float);
  float* k = ORC_ALLOC(M * D, float);
  float* v = ORC_ALLOC(M * D, float);
  float* qkv = ORC_ALLOC(M * 3 * D, float);
  float* Q = ORC_ALLOC(M * D, float);
  float* Kt = ORC_ALLOC(M * D, float);
  float* V = ORC_ALLOC(M * D, float);
  float* At = ORC_ALLOC(M * D, float);
  float* AO = ORC_ALLOC(M * D, float);
  orc_gemm_nt(Y, ly->q_w, ly->q_b, 0, M, D, D, q);
  orc_gemm_nt(Y, ly->k_w, ly->k_b, 0, M, D, D, k);
  orc_gemm_nt(Y, ly->v_w, ly->v_b, 0, M, D, D, v);
  /* packed (q|k|v) rows, then the same [B, H, L, Dh] split as the
   * DecisionModel path (pure copies: the permute of src/sj_model.cpp:57-71) */
  for (int64_t r = 0; r < M; ++r) {
    memcpy(qkv + r * 3 * D, q + r * D, sizeof(float) * (size_t)D);
    memcpy(qkv + r * 3 * D + D, k + r * D, sizeof(float) * (size_t)D);
    memcpy(qkv + r * 3 * D + 2 * D, v + r * D, sizeof(float) * (size_t)D);
  }
  split_heads(qkv, B, L, H, Dh, Q, Kt, V);
  orc_attention(Q, Kt, V, lens, B, H, L, Dh, 0, At);
  merge_heads(At, B, L, H, Dh, AO);
  orc_gemm_nt(AO, ly->o_w, ly->o_b, 0, M, D, D, out);
  free(q); free(k); free(v); free(qkv); free(Q); free(Kt); free(V); free(At); free(AO);
}

/* One pre-norm layer (src/sj_model.cpp:240-252 for the encoder, :308-318 for
 * the head): X += attn(LN(X)); X += W2 . gelu(W1 . LN(X) + b1) + b2. */
static void sj_layer(float* X, int64_t B, int64_t H, int64_t L, int64_t Dh, int64_t F,
                     const int64_t* lens, const orc_sj_layer* ly, float eps) {
  const int64_t D = H * Dh, M = B * L;
  float* Y = ORC_ALLOC(M * D, float);
  float* P = ORC_ALLOC(M * D, float);
  float* G = ORC_ALLOC(M * F, float);
  orc_layer_norm(X, M, D, ly->an_w, ly->an_b, eps, Y);
  sj_self_attention(Y, B, H, L, Dh, lens, ly, P);
  add_inplace(X, P, M * D);
  orc_layer_norm(X, M, D, ly->fn_w, ly->fn_b, eps, Y);
  orc_gemm_nt(Y, ly->w1_w, ly->w1_b, 1, M, F, D, G);
  orc_gemm_nt(G, ly->w2_w, ly->w2_b, 0, M, D, F, P);
  add_inplace(X, P, M * D);
  free(Y); free(P); free(G);
}

/* src/sj_model.cpp:206-255 -- run_encoder: word embedding + learned position
 * embedding of row r at position r % L clamped to max_pos - 1, summed in
 * float, LayerNorm with bias; the layers; the final LayerNorm with bias. */
static void sj_run_encoder(const orc_sj_model* m, const int64_t* ids, const int64_t* lens,
                           int64_t B, int64_t L, float* h) {
  const int64_t D = m->D, H = m->H, Dh = D / H, M = B * L;
  float* X = ORC_ALLOC(M * D, float);
  float* E = ORC_ALLOC(M * D, float);
  orc_embedding(m->word_emb, D, ids, M, E);
  for (int64_t r = 0; r < M; ++r) {
    int64_t pos = r % L;
    if (pos >= m->max_pos) pos = m->max_pos - 1;
    add_inplace(E + r * D, m->pos_emb + pos * D, D);
  }
  orc_layer_norm(E, M, D, m->emb_norm_w, m->emb_norm_b, m->eps, X);
  for (int64_t li = 0; li < m->n_layers; ++li)
    sj_layer(X, B, H, L, Dh, m->F, lens, &m->layers[li], m->eps);
  orc_layer_norm(X, M, D, m->final_norm_w, m->final_norm_b, m->eps, h);
  free(X); free(E);
}

int orc_sj_encode(const orc_sj_model* m, const int64_t* ids, const int64_t* mask, int64_t B,
                  int64_t L, float* out) {
  if (B <= 0) return 0;
  int64_t* lens = ORC_ALLOC(B, int64_t);
  lens_from_mask(mask, B, L, lens);
  sj_run_encoder(m, ids, lens, B, L, out);
  free(lens);
  return 0;
}

/* src/sj_model.cpp:277-368 */
int orc_sj_forward(const orc_sj_model* m, const int64_t* ids, const int64_t* mask,
                   const int64_t* marker_pos, const uint8_t* marker_mask, const int64_t* qtype,
                   int64_t B, int64_t L, int64_t K, float* logits, float* act, float* hidden_out) {
  if (B <= 0) return 0;
  const int64_t D = m->D, H = m->H, Dh = D / H, M = B * L;
  int64_t* lens = ORC_ALLOC(B, int64_t);
  lens_from_mask(mask, B, L, lens);
  float* h = ORC_ALLOC(M * D, float);
  sj_run_encoder(m, ids, lens, B, L, h);
  /* :291-298 h += type_emb[qtype] on every position */
  for (int64_t b = 0; b < B; ++b)
    for (int64_t i = 0; i < L; ++i)
      add_inplace(h + (b * L + i) * D, m->type_emb + qtype[b] * D, D);
  /* :300-321 head layers: the encoder's layer shape, GELU FFN of width
   * head_intermediate, LayerNorm eps = norm_eps */
  for (int64_t li = 0; li < m->head_layers; ++li)
    sj_layer(h, B, H, L, Dh, m->head_ff, lens, &m->head[li], m->eps);
  if (hidden_out) memcpy(hidden_out, h, sizeof(float) * (size_t)(M * D));
  /* :323-347 scorer on the marker rows (positions clamped to [0, L-1]) */
  {
    float* mk = ORC_ALLOC(B * K * D, float);
    float* s0 = ORC_ALLOC(B * K * D, float);
    float* s1 = ORC_ALLOC(B * K * D, float);
    float* s2 = ORC_ALLOC(B * K, float);
    for (int64_t b = 0; b < B; ++b)
      for (int64_t kk = 0; kk < K; ++kk) {
        int64_t p = marker_pos[b * K + kk];
        if (p < 0) p = 0;
        if (p >= L) p = L - 1;
        memcpy(mk + (b * K + kk) * D, h + (b * L + p) * D, sizeof(float) * (size_t)D);
      }
    orc_layer_norm(mk, B * K, D, m->sc_n_w, m->sc_n_b, m->eps, s0);
    orc_gemm_nt(s0, m->sc_w1, m->sc_b1, 1, B * K, D, D, s1);
    orc_gemm_nt(s1, m->sc_w2, m->sc_b2, 0, B * K, 1, D, s2);
    for (int64_t i = 0; i < B * K; ++i) logits[i] = marker_mask[i] ? s2[i] : -1e4f;
    free(mk); free(s0); free(s1); free(s2);
  }
  /* :349-367 act = {top1, 1 - top1} of softmax(logits): float exp of the
   * max-subtracted logit, double sum and division */
  {
    double* p = ORC_ALLOC(K, double);
    for (int64_t b = 0; b < B; ++b) {
      const float* lg = logits + b * K;
      float mx = lg[0];
      for (int64_t j = 1; j < K; ++j) mx = lg[j] > mx ? lg[j] : mx;
      double s = 0.0;
      for (int64_t j = 0; j < K; ++j) {
        p[j] = (double)expf(lg[j] - mx);
        s += p[j];
      }
      double top1 = 0.0;
      for (int64_t j = 0; j < K; ++j) {
        p[j] /= s;
        top1 = j == 0 || p[j] > top1 ? p[j] : top1;
      }
      act[b * 2 + 0] = (float)top1;
      act[b * 2 + 1] = (float)(1.0 - top1);
    }
    free(p);
  }
  free(h);
  free(lens);
  return 0;
}

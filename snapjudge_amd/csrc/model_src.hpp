// model_src.hpp -- where a model's weights come from, before staging.
//
// The engine stages every tensor from a Src: one or more host segments
// (concatenated, for a matrix stored as several row blocks, such as SjModel's
// separate q, k and v), each of an element type.  Segments point at the
// caller's fp32 arrays (sjh_model_create) or straight into a memory-mapped
// checkpoint (sjh_model_load), whose bf16 / f16 / f32 / e4m3 bytes are
// converted on the device while they are staged.
#pragma once

#include <cstdint>
#include <vector>

#include "sjh_kernels.hpp"
#include "snapjudge_hip.h"

namespace sjh {

struct Seg {
  int type = SRC_F32;  // SrcType
  const void* p = nullptr;
  int64_t n = 0;  // elements
};

struct Src {
  std::vector<Seg> segs;
  bool empty() const { return segs.empty(); }
  int64_t numel() const {
    int64_t n = 0;
    for (const Seg& s : segs) n += s.n;
    return n;
  }
  static Src host_f32(const float* p, int64_t n) {
    Src s;
    if (p) s.segs.push_back({SRC_F32, p, n});
    return s;
  }
};

// A projection matrix: its rows, and one fp32 scale per row when the rows
// hold e4m3 codes (SRC_F8).
struct Mat {
  Src w, scale;
};

// Model families: the DecisionModel's ModernBERT-style encoder
// (src/model.cpp) and snapjudge's own BERT-style SjModel (src/sj_model.cpp).
enum Arch : int { ARCH_MODERNBERT = 0, ARCH_BERT = 1 };
// Act heads: the DecisionModel's MLP over [CLS, decision statistics]
// (src/model.cpp:489-535) or SjModel's {top1, 1 - top1} (src/sj_model.cpp:349-367).
enum ActHead : int { ACT_MLP = 0, ACT_TOP1 = 1 };

// One encoder layer.  ModernBERT: attn_norm (absent in layer 0), fused Wqkv,
// Wo, mlp_norm, Wi [2F, D] (GEGLU), Wo2; no biases.  BERT: every norm with a
// bias, wqkv = q|k|v rows with their biases, wo, wi = w1 [F, D] (GELU), wo2 =
// w2, each with a bias.
struct LayerSrc {
  Src attn_norm, attn_norm_b;
  Mat wqkv;
  Src wqkv_b;
  Mat wo;
  Src wo_b;
  Src mlp_norm, mlp_norm_b;
  Mat wi;
  Src wi_b;
  Mat wo2;
  Src wo2_b;
  int window = 0, sliding = 0;
};

// One decision-head layer (both families: pre-norm, attention without RoPE,
// biased projections; FFN width head_ff, activation head_act).
struct HeadSrc {
  Src n1w, n1b, n2w, n2b, in_w, in_b, out_w, out_b, l1w, l1b, l2w, l2b;
};

struct ModelSource {
  int arch = ARCH_MODERNBERT;
  int D = 0, H = 0, F = 0, V = 0, n_layers = 0, max_pos = 0;
  int n_act = 0, head_layers = 0, head_ff = 0, lora_r = 0;
  float eps = 1e-5f;
  float head_eps = 1e-5f;  // DecisionModel head norms: 1e-5 (src/model.cpp:424,453)
  int head_act = 2;        // 2 ReLU (DecisionModel), 1 erf-GELU (SjModel)
  int act_head = ACT_MLP;
  double theta_full = 10000.0, theta_sliding = 10000.0;
  Src emb_w, pos_emb, emb_norm, emb_norm_b, final_norm, final_norm_b;
  const float *rope_cos_full = nullptr, *rope_sin_full = nullptr;  // [max_pos, Dh/2] or null
  const float *rope_cos_slide = nullptr, *rope_sin_slide = nullptr;
  std::vector<LayerSrc> layers;
  Src lora_a, lora_b, type_emb;
  std::vector<HeadSrc> head;
  Src sc_ln_w, sc_ln_b, sc_w1, sc_b1, sc_w2, sc_b2;
  Src act_w1, act_b1, act_w2, act_b2;
};

// The DecisionModel descriptor of sjh_model_create as a source (fp32 host arrays).
ModelSource source_from_desc(const sjh_model_desc& d);

}  // namespace sjh

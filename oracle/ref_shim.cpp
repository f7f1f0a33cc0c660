// ref_shim.cpp -- C entry points over the reference's own CPU forward.
//
// TEST INFRASTRUCTURE ONLY.  Compiled together with the reference's
// src/{tensor,model,safetensors,cblas_fallback}.cpp where they lie under the
// reference tree (see oracle/Makefile); the result, oracle/_ref/libsjref.so,
// is the compiled reference used to pin the C restatement in sj_oracle.c and
// as the CPU baseline in bench.py.  Nothing here re-implements the reference:
// every entry point forwards to the reference's own functions.
#include <cstdint>
#include <cstring>
#include <fstream>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "nlohmann/json.hpp"
#include "snapjudge/model.hpp"
#include "snapjudge/safetensors.hpp"
#include "snapjudge/sj_model.hpp"
#include "snapjudge/tensor.hpp"

using nlohmann::json;
using snapjudge::DecisionModel;
using snapjudge::SjModel;
using snapjudge::Tensor;

namespace {
thread_local std::string g_err;

Tensor copy_in(const float* p, std::vector<int64_t> shape) {
  Tensor t(std::move(shape));
  std::memcpy(t.mutable_data(), p, sizeof(float) * static_cast<size_t>(t.numel()));
  return t;
}

void copy_out(const Tensor& t, float* out) {
  std::memcpy(out, t.data_ptr(), sizeof(float) * static_cast<size_t>(t.numel()));
}

std::vector<std::vector<int64_t>> rows_i64(const int64_t* p, int64_t B, int64_t L) {
  std::vector<std::vector<int64_t>> v(static_cast<size_t>(B));
  for (int64_t b = 0; b < B; ++b) v[static_cast<size_t>(b)].assign(p + b * L, p + (b + 1) * L);
  return v;
}
}  // namespace

extern "C" {

const char* sjref_last_error() { return g_err.c_str(); }

// Loads <dir>/rl_agent_config.json, <dir>/encoder/config.json and
// <dir>/model.safetensors exactly as Agent::Agent does (src/agent.cpp:59-85).
void* sjref_load(const char* dir) {
  try {
    std::string d(dir);
    json rl, enc;
    std::ifstream(d + "/rl_agent_config.json") >> rl;
    std::ifstream(d + "/encoder/config.json") >> enc;
    auto w = snapjudge::SafeTensors::load(d + "/model.safetensors");
    return DecisionModel::load(rl, enc, w, d).release();
  } catch (const std::exception& e) {
    g_err = e.what();
    return nullptr;
  }
}

void sjref_free(void* m) { delete static_cast<DecisionModel*>(m); }

// D, H, Dh, F, n_layers, n_act, max_pos, head_layers
void sjref_dims(void* mp, int64_t* out) {
  auto* m = static_cast<DecisionModel*>(mp);
  const auto& c = m->cfg();
  out[0] = m->D(); out[1] = m->H(); out[2] = m->Dh(); out[3] = m->F();
  out[4] = c.num_hidden_layers; out[5] = c.n_act; out[6] = c.max_position_embeddings;
  out[7] = c.head_layers;
}

// The model's own RoPE tables (src/model.cpp:173-190), [max_pos, Dh/2] each.
void sjref_rope_tables(void* mp, float* cos_full, float* sin_full, float* cos_slide,
                       float* sin_slide) {
  auto* m = static_cast<DecisionModel*>(mp);
  size_t n = static_cast<size_t>(m->cfg().max_position_embeddings) * (m->Dh() / 2);
  std::memcpy(cos_full, m->rope_cos_full().get(), n * 4);
  std::memcpy(sin_full, m->rope_sin_full().get(), n * 4);
  std::memcpy(cos_slide, m->rope_cos_slide().get(), n * 4);
  std::memcpy(sin_slide, m->rope_sin_slide().get(), n * 4);
}

int sjref_encode(void* mp, const int64_t* ids, const int64_t* mask, int64_t B, int64_t L,
                 float* out) {
  try {
    auto* m = static_cast<DecisionModel*>(mp);
    auto h = m->encode(rows_i64(ids, B, L), rows_i64(mask, B, L));
    const int64_t D = m->D();
    for (int64_t b = 0; b < B; ++b)
      for (int64_t i = 0; i < L; ++i)
        std::memcpy(out + (b * L + i) * D, h[static_cast<size_t>(b)][static_cast<size_t>(i)].data(),
                    sizeof(float) * static_cast<size_t>(D));
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

int sjref_forward(void* mp, const int64_t* ids, const int64_t* mask, const int64_t* marker_pos,
                  const uint8_t* marker_mask, const int64_t* qtype, int64_t B, int64_t L,
                  int64_t K, float* logits, float* act) {
  try {
    auto* m = static_cast<DecisionModel*>(mp);
    std::vector<std::vector<uint8_t>> mm(static_cast<size_t>(B));
    for (int64_t b = 0; b < B; ++b) mm[static_cast<size_t>(b)].assign(marker_mask + b * K, marker_mask + (b + 1) * K);
    std::vector<int64_t> qt(qtype, qtype + B);
    std::vector<std::vector<float>> lg, ac;
    m->forward(rows_i64(ids, B, L), rows_i64(mask, B, L), rows_i64(marker_pos, B, K), mm, qt,
               lg, ac);
    const int64_t A = m->cfg().n_act;
    for (int64_t b = 0; b < B; ++b) {
      std::memcpy(logits + b * K, lg[static_cast<size_t>(b)].data(), sizeof(float) * static_cast<size_t>(K));
      std::memcpy(act + b * A, ac[static_cast<size_t>(b)].data(), sizeof(float) * static_cast<size_t>(A));
    }
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

// ---- SjModel (src/sj_model.cpp) ----
// Loads <dir>/sj_config.json and <dir>/model.safetensors, the layout
// SjTrainModel and SjPretrain read (src/sj_train.cpp:180-184).
void* sjref_sj_load(const char* dir) {
  try {
    std::string d(dir);
    json cfg;
    std::ifstream(d + "/sj_config.json") >> cfg;
    auto w = snapjudge::SafeTensors::load(d + "/model.safetensors");
    return SjModel::load(cfg, w, d).release();
  } catch (const std::exception& e) {
    g_err = e.what();
    return nullptr;
  }
}

void sjref_sj_free(void* m) { delete static_cast<SjModel*>(m); }

int sjref_sj_encode(void* mp, const int64_t* ids, const int64_t* mask, int64_t B, int64_t L,
                    float* out) {
  try {
    auto* m = static_cast<SjModel*>(mp);
    auto h = m->encode(rows_i64(ids, B, L), rows_i64(mask, B, L));
    const int64_t D = m->D();
    for (int64_t b = 0; b < B; ++b)
      for (int64_t i = 0; i < L; ++i)
        std::memcpy(out + (b * L + i) * D, h[static_cast<size_t>(b)][static_cast<size_t>(i)].data(),
                    sizeof(float) * static_cast<size_t>(D));
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

int sjref_sj_forward(void* mp, const int64_t* ids, const int64_t* mask, const int64_t* marker_pos,
                     const uint8_t* marker_mask, const int64_t* qtype, int64_t B, int64_t L,
                     int64_t K, float* logits, float* act) {
  try {
    auto* m = static_cast<SjModel*>(mp);
    std::vector<std::vector<uint8_t>> mm(static_cast<size_t>(B));
    for (int64_t b = 0; b < B; ++b) mm[static_cast<size_t>(b)].assign(marker_mask + b * K, marker_mask + (b + 1) * K);
    std::vector<int64_t> qt(qtype, qtype + B);
    std::vector<std::vector<float>> lg, ac;
    m->forward(rows_i64(ids, B, L), rows_i64(mask, B, L), rows_i64(marker_pos, B, K), mm, qt,
               lg, ac);
    for (int64_t b = 0; b < B; ++b) {
      std::memcpy(logits + b * K, lg[static_cast<size_t>(b)].data(), sizeof(float) * static_cast<size_t>(K));
      std::memcpy(act + b * 2, ac[static_cast<size_t>(b)].data(), sizeof(float) * 2);
    }
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

// ---- single ops (src/tensor.cpp) ----
void sjref_layer_norm(const float* x, int64_t rows, int64_t D, const float* w, const float* b,
                      float eps, float* out) {
  copy_out(snapjudge::layer_norm(copy_in(x, {rows, D}), w, b, eps), out);
}

void sjref_gemm_nt(const float* a, const float* w, const float* bias, int act, int64_t M,
                   int64_t N, int64_t K, float* out) {
  copy_out(snapjudge::gemm_nt(copy_in(a, {M, K}), copy_in(w, {N, K}), bias, act), out);
}

void sjref_gemm_geglu(const float* a, const float* wi, int64_t M, int64_t F, int64_t K,
                      float* out) {
  copy_out(snapjudge::gemm_geglu(copy_in(a, {M, K}), copy_in(wi, {2 * F, K})), out);
}

void sjref_attention(const float* q, const float* k, const float* v, const int64_t* lens,
                     int64_t B, int64_t H, int64_t L, int64_t Dh, int window, float* out) {
  std::vector<int64_t> ln(lens, lens + B);
  copy_out(snapjudge::attention(copy_in(q, {B, H, L, Dh}), copy_in(k, {B, H, L, Dh}),
                                copy_in(v, {B, H, L, Dh}), ln, window),
           out);
}

void sjref_rope_inplace(float* qkv, int64_t M, const float* cos_t, const float* sin_t,
                        int64_t L, int64_t H, int64_t Dh) {
  Tensor t = copy_in(qkv, {M, 3 * H * Dh});
  snapjudge::rope_inplace(t, cos_t, sin_t, L, H, Dh);
  copy_out(t, qkv);
}

void sjref_softmax_rows(float* x, int64_t rows, int64_t K) {
  Tensor t = copy_in(x, {rows, K});
  snapjudge::softmax_rows(t);
  copy_out(t, x);
}

}  // extern "C"

// fast_hip.cpp -- snapjudge::FastSnapjudge (include/snapjudge_fast_hip.hpp) over
// the MI355X C ABI (include/snapjudge_hip.h).
//
// Compiled against the reference's own headers (include/snapjudge/model.hpp,
// which names FastSnapjudge a friend of DecisionModel at model.hpp:128-129),
// so it reads the model's fp32 weights and RoPE tables directly, exactly as
// the reference's cuda/fast.cpp:272-352 does, and hands them to
// sjh_model_create.  The only code that runs on the GPU is
// libsnapjudge_hip.so; this file converts the reference's nested-vector
// arguments to flat arrays and back.
//
// Also exports a small C surface (sjfast_*) over the class, the binding a
// ctypes or cgo caller of the reference's engine would use for this object.
#include "snapjudge_fast_hip.hpp"

#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>

#include "snapjudge/model.hpp"
#include "snapjudge_hip.h"

namespace snapjudge {

namespace {

[[noreturn]] void fail(const std::string& what) {
  throw std::runtime_error("snapjudge HIP: " + what);
}

void check(int rc, const char* what) {
  if (rc != SJH_OK) fail(std::string(what) + ": " + sjh_last_error());
}

// Rows of a [N][L] argument, all of length L (the reference's collate pads
// every row to the batch maximum, src/agent.cpp:186-215).
template <typename T>
void flatten(const std::vector<std::vector<T>>& rows, size_t L, const char* what,
             std::vector<T>& out) {
  out.resize(rows.size() * L);
  for (size_t b = 0; b < rows.size(); ++b) {
    if (rows[b].size() != L) fail(std::string(what) + ": rows must all have the same length");
    if (L) std::memcpy(out.data() + b * L, rows[b].data(), L * sizeof(T));
  }
}

}  // namespace

struct FastSnapjudge::Impl {
  sjh_model* m = nullptr;
  int D = 0, n_act = 0;
  std::mutex mu;
  ~Impl() {
    if (m) sjh_model_destroy(m);
  }
};

FastSnapjudge::FastSnapjudge(DecisionModel* model, int max_len, bool use_graphs)
    : FastSnapjudge(model, max_len, use_graphs, SJH_PREC_BF16, 0) {}

FastSnapjudge::FastSnapjudge(DecisionModel* model, int max_len, bool use_graphs, int precision,
                             int pad_rows)
    : impl_(new Impl) {
  if (!model) fail("null DecisionModel");
  const DecisionModel& M = *model;
  const ModelConfig& c = M.cfg_;

  std::vector<sjh_layer_desc> layers(M.layers_.size());
  for (size_t i = 0; i < layers.size(); ++i) {
    const LayerWeights& ly = M.layers_[i];
    sjh_layer_desc& d = layers[i];
    d.attn_norm = ly.has_attn_norm ? ly.attn_norm.d.get() : nullptr;
    d.wqkv = ly.wqkv.d.get();
    d.wo = ly.wo.d.get();
    d.mlp_norm = ly.mlp_norm.d.get();
    d.wi = ly.wi.d.get();
    d.wo2 = ly.wo2.d.get();
    d.window = ly.window;
    d.sliding = ly.attention_type == "sliding_attention" ? 1 : 0;
  }
  std::vector<sjh_head_desc> head(M.head_.size());
  for (size_t i = 0; i < head.size(); ++i) {
    const auto& h = M.head_[i];
    head[i] = sjh_head_desc{h.n1w.get(),   h.n1b.get(),   h.n2w.get(), h.n2b.get(),
                            h.in_w.get(),  h.in_b.get(),  h.out_w.get(), h.out_b.get(),
                            h.l1w.get(),   h.l1b.get(),   h.l2w.get(), h.l2b.get()};
  }

  sjh_model_desc d;
  std::memset(&d, 0, sizeof(d));
  d.hidden_size = M.D_;
  d.num_heads = M.H_;
  d.intermediate_size = M.F_;
  d.vocab_size = c.vocab_size;
  d.num_layers = static_cast<int32_t>(layers.size());
  d.max_position = c.max_position_embeddings;  // rows of the RoPE tables (model.cpp:173-190)
  d.n_act = c.n_act;
  d.head_layers = static_cast<int32_t>(head.size());
  d.lora_r = M.lora_r_;
  d.norm_eps = c.norm_eps;
  d.rope_theta_full = c.rope_theta_full;
  d.rope_theta_sliding = c.rope_theta_sliding;
  d.emb_w = M.emb_w_.get();
  d.emb_norm = M.emb_norm_.get();
  d.final_norm = M.final_norm_.get();
  d.rope_cos_full = M.rope_cos_full_.get();
  d.rope_sin_full = M.rope_sin_full_.get();
  d.rope_cos_slide = M.rope_cos_slide_.get();
  d.rope_sin_slide = M.rope_sin_slide_.get();
  d.layers = layers.data();
  d.lora_a = M.lora_r_ > 0 ? M.lora_a_.get() : nullptr;
  d.lora_b = M.lora_r_ > 0 ? M.lora_b_.get() : nullptr;
  d.type_emb = M.type_emb_.get();
  d.head = head.empty() ? nullptr : head.data();
  d.sc_ln_w = M.scorer_ln_w_.get();
  d.sc_ln_b = M.scorer_ln_b_.get();
  d.sc_w1 = M.scorer_w1_.get();
  d.sc_b1 = M.scorer_b1_.get();
  d.sc_w2 = M.scorer_w2_.get();
  d.sc_b2 = M.scorer_b2_.get();
  d.act_w1 = M.act_w1_.get();
  d.act_b1 = M.act_b1_.get();
  d.act_w2 = M.act_w2_.get();
  d.act_b2 = M.act_b2_.get();

  sjh_options o;
  sjh_default_options(&o);
  o.precision = precision;
  o.max_len = max_len;
  o.use_graphs = use_graphs ? 1 : 0;
  o.pad_rows = pad_rows;
  check(sjh_model_create(&d, &o, &impl_->m), "model create");
  int32_t D = 0, H = 0, n_act = 0, prec = 0;
  check(sjh_model_info(impl_->m, &D, &H, &n_act, &prec), "model info");
  impl_->D = D;
  impl_->n_act = n_act;
}

FastSnapjudge::~FastSnapjudge() = default;

void FastSnapjudge::forward(const std::vector<std::vector<int64_t>>& input_ids,
                            const std::vector<std::vector<int64_t>>& attention_mask,
                            const std::vector<std::vector<int64_t>>& marker_pos,
                            const std::vector<std::vector<uint8_t>>& marker_mask,
                            const std::vector<int64_t>& qtype,
                            std::vector<std::vector<float>>& logits,
                            std::vector<std::vector<float>>& act) {
  std::lock_guard<std::mutex> lk(impl_->mu);
  const size_t N = input_ids.size();
  logits.clear();
  act.clear();
  if (N == 0) return;
  if (attention_mask.size() != N || marker_pos.size() != N || marker_mask.size() != N ||
      qtype.size() != N)
    fail("forward: argument batch sizes differ");
  const size_t L = input_ids[0].size(), K = marker_pos[0].size();
  std::vector<int64_t> ids, mask, mp;
  std::vector<uint8_t> mm;
  flatten(input_ids, L, "input_ids", ids);
  flatten(attention_mask, L, "attention_mask", mask);
  flatten(marker_pos, K, "marker_pos", mp);
  flatten(marker_mask, K, "marker_mask", mm);
  std::vector<float> lg(N * K), ac(N * static_cast<size_t>(impl_->n_act));
  check(sjh_model_forward(impl_->m, ids.data(), mask.data(), mp.data(), mm.data(), qtype.data(),
                          static_cast<int32_t>(N), static_cast<int32_t>(L),
                          static_cast<int32_t>(K), lg.data(), ac.data()),
        "forward");
  logits.resize(N);
  act.resize(N);
  for (size_t b = 0; b < N; ++b) {
    logits[b].assign(lg.begin() + static_cast<ptrdiff_t>(b * K),
                     lg.begin() + static_cast<ptrdiff_t>((b + 1) * K));
    act[b].assign(ac.begin() + static_cast<ptrdiff_t>(b * impl_->n_act),
                  ac.begin() + static_cast<ptrdiff_t>((b + 1) * impl_->n_act));
  }
}

std::vector<std::vector<std::vector<float>>> FastSnapjudge::encode(
    const std::vector<std::vector<int64_t>>& input_ids,
    const std::vector<std::vector<int64_t>>& attention_mask) {
  std::lock_guard<std::mutex> lk(impl_->mu);
  const size_t N = input_ids.size();
  std::vector<std::vector<std::vector<float>>> out(N);
  if (N == 0) return out;
  if (attention_mask.size() != N) fail("encode: argument batch sizes differ");
  const size_t L = input_ids[0].size(), D = static_cast<size_t>(impl_->D);
  std::vector<int64_t> ids, mask;
  flatten(input_ids, L, "input_ids", ids);
  flatten(attention_mask, L, "attention_mask", mask);
  std::vector<float> h(N * L * D);
  check(sjh_model_encode(impl_->m, ids.data(), mask.data(), static_cast<int32_t>(N),
                         static_cast<int32_t>(L), h.data()),
        "encode");
  for (size_t b = 0; b < N; ++b) {
    out[b].resize(L);
    for (size_t i = 0; i < L; ++i) {
      const float* src = h.data() + (b * L + i) * D;
      out[b][i].assign(src, src + D);
    }
  }
  return out;
}

}  // namespace snapjudge

// ---------------------------------------------------------------- C surface
namespace {
thread_local std::string g_err;

template <typename Fn>
int guarded(Fn&& fn) {
  try {
    fn();
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

std::vector<std::vector<int64_t>> rows64(const int64_t* p, int N, int L) {
  std::vector<std::vector<int64_t>> v(static_cast<size_t>(N));
  for (int b = 0; b < N; ++b) v[static_cast<size_t>(b)].assign(p + static_cast<size_t>(b) * L,
                                                              p + static_cast<size_t>(b + 1) * L);
  return v;
}
}  // namespace

extern "C" {

const char* sjfast_last_error(void) { return g_err.c_str(); }

// model: a snapjudge::DecisionModel* owned by the caller (it must outlive the result).
void* sjfast_create(void* model, int max_len, int use_graphs, int precision, int pad_rows) {
  snapjudge::FastSnapjudge* f = nullptr;
  const int rc = guarded([&] {
    f = new snapjudge::FastSnapjudge(static_cast<snapjudge::DecisionModel*>(model), max_len,
                                     use_graphs != 0, precision, pad_rows);
  });
  return rc == 0 ? f : nullptr;
}

void sjfast_destroy(void* f) { delete static_cast<snapjudge::FastSnapjudge*>(f); }

int sjfast_forward(void* f, const int64_t* ids, const int64_t* mask, const int64_t* marker_pos,
                   const uint8_t* marker_mask, const int64_t* qtype, int N, int L, int K,
                   float* logits, float* act) {
  return guarded([&] {
    if (!f || N < 0 || L <= 0 || K <= 0) throw std::runtime_error("sjfast_forward: bad arguments");
    std::vector<std::vector<uint8_t>> mm(static_cast<size_t>(N));
    for (int b = 0; b < N; ++b)
      mm[static_cast<size_t>(b)].assign(marker_mask + static_cast<size_t>(b) * K,
                                        marker_mask + static_cast<size_t>(b + 1) * K);
    std::vector<int64_t> qt(qtype, qtype + N);
    std::vector<std::vector<float>> lg, ac;
    static_cast<snapjudge::FastSnapjudge*>(f)->forward(rows64(ids, N, L), rows64(mask, N, L),
                                                        rows64(marker_pos, N, K), mm, qt, lg, ac);
    for (int b = 0; b < N; ++b) {
      std::memcpy(logits + static_cast<size_t>(b) * K, lg[static_cast<size_t>(b)].data(),
                  sizeof(float) * static_cast<size_t>(K));
      std::memcpy(act + static_cast<size_t>(b) * ac[0].size(), ac[static_cast<size_t>(b)].data(),
                  sizeof(float) * ac[0].size());
    }
  });
}

int sjfast_encode(void* f, const int64_t* ids, const int64_t* mask, int N, int L, float* hidden) {
  return guarded([&] {
    if (!f || N < 0 || L <= 0) throw std::runtime_error("sjfast_encode: bad arguments");
    auto h = static_cast<snapjudge::FastSnapjudge*>(f)->encode(rows64(ids, N, L),
                                                              rows64(mask, N, L));
    for (int b = 0; b < N; ++b)
      for (int i = 0; i < L; ++i) {
        const auto& v = h[static_cast<size_t>(b)][static_cast<size_t>(i)];
        std::memcpy(hidden + (static_cast<size_t>(b) * L + i) * v.size(), v.data(),
                    sizeof(float) * v.size());
      }
  });
}

}  // extern "C"

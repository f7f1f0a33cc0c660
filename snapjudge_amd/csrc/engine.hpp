// engine.hpp -- the device-resident DecisionModel (host orchestration).
//
// Owns the device copies of all weights, a grow-only workspace, one HIP stream
// (default priority) and a cache of captured hipGraphs keyed by a shape
// bucket: every kernel reads the real token count and the per-sequence
// lengths from a device table, so one graph serves all batches of a bucket.
// The forward follows src/model.cpp:309-536 op for op; the differences are in
// layout only:
//   * tokens are packed: sequence b occupies rows [seq_start[b],
//     seq_start[b] + n_b) of every [T, .] activation, T = sum of lengths, so
//     GEMMs and attention touch valid tokens only (pad_rows = 1 keeps the
//     reference's [B*L] layout and computes padded query rows as it does);
//   * RoPE is applied in the QKV GEMM epilogue, GEGLU in the Wi GEMM epilogue
//     and the residual adds in the Wo / Wo2 GEMM epilogues;
//   * q, k, v stay in the packed (q|k|v)(head)(dim) rows of one [T, 3D]
//     buffer; attention reads them with strides (no permute copies,
//     src/model.cpp:368-387).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "model_src.hpp"
#include "sjh_kernels.hpp"
#include "snapjudge_hip.h"

namespace sjh {

// Host-side fp8 quantizer of the SJH_PREC_FP8W mode (engine.cpp).
uint8_t fp8_e4m3_rne(float x);
void quantize_fp8_rows(const float* w, size_t rows, size_t cols, uint8_t* q, float* scale);

class DevBuf {
 public:
  DevBuf() = default;
  ~DevBuf();
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept : p_(o.p_), bytes_(o.bytes_) {
    o.p_ = nullptr;
    o.bytes_ = 0;
  }
  DevBuf& operator=(DevBuf&& o) noexcept;
  void alloc(size_t bytes);  // frees and reallocates
  void ensure(size_t bytes); // grows when smaller
  void* get() const { return p_; }
  template <typename T>
  T* as() const { return static_cast<T*>(p_); }
  size_t bytes() const { return bytes_; }

 private:
  void* p_ = nullptr;
  size_t bytes_ = 0;
};

class PinnedBuf {
 public:
  PinnedBuf() = default;
  ~PinnedBuf();
  PinnedBuf(const PinnedBuf&) = delete;
  PinnedBuf& operator=(const PinnedBuf&) = delete;
  void ensure(size_t bytes);
  template <typename T>
  T* as() const { return static_cast<T*>(p_); }

 private:
  void* p_ = nullptr;
  size_t bytes_ = 0;
};

// Device-side batch layout (see the file comment).  B, T and max_q are the
// batch's own; Bb, Tb and max_qb its bucket, which sizes the launches (and
// keys the graph cache): Bb the next power of two of B, Tb the token count
// rounded up (to 64 up to 1024 tokens, then to an eighth of its power of
// two), max_qb the longest row rounded up to the attention query block (128,
// or 1024 above 1024).
struct BatchPlan {
  int B = 0, L = 0, T = 0, max_q = 0;
  int Bb = 0, Tb = 0, max_qb = 0;
  std::vector<int32_t> seq_start, q_len, k_len;
  std::vector<int32_t> order;  // sequences by decreasing length (attention dispatch order)
};

// Device buffers one forward works in (the engine's grow-only workspace).
struct Ws {
  int32_t* seq = nullptr;  // sequence table (sjh_kernels.hpp, seq_table_ints(Bb) ints)
  int* tok_pos = nullptr;  // [Tb] position of each token in its sequence
  int* tok_seq = nullptr;  // [Tb] sequence of each token
  void *Y = nullptr, *QKV = nullptr, *O = nullptr, *G = nullptr;
  float* Z = nullptr;  // LoRA [Tb, r]
  float* partial = nullptr;  // split-K partial sums
  int64_t partial_cap = 0;   // floats
  int32_t* attn_items = nullptr;  // attention work list (AttnArgs::items)
  int attn_slots_cap = 0;         // its slots
  float* attn_part = nullptr;     // partials of key-split items (AttnArgs::part), or none
  int attn_pairs_cap = 0;         // split items they hold
  float* ln_stats = nullptr;      // row moments of a folded LayerNorm (GemmArgs::ln_stats_out), or none
  // the LayerNorm finished by the residual epilogue (GemmArgs::rln_y): row
  // moments [Tb][D / 256][4] and kRlnSyncInts zeroed ints per 256-row panel,
  // or none
  float* rln_mom = nullptr;
  int* rln_sync = nullptr;
};

class Engine {
 public:
  // Stages every weight of `src` on the device (its host memory may be
  // released after the constructor returns).
  Engine(const ModelSource& src, const sjh_options& o);
  ~Engine();

  int D() const { return D_; }
  int H() const { return H_; }
  int n_act() const { return n_act_; }
  int precision() const { return prec_; }

  void encode(const int64_t* ids, const int64_t* mask, int B, int L, float* hidden);
  void forward(const int64_t* ids, const int64_t* mask, const int64_t* marker_pos,
               const uint8_t* marker_mask, const int64_t* qtype, int B, int L, int K,
               float* logits, float* act);
  void encode_device(const int32_t* d_ids, const int32_t* h_lens, int B, float* d_hidden,
                     hipStream_t stream);
  // forward on B rows that share U token sequences: row b is sequence
  // row_seq[b] of ids/mask [U, L] with its own markers and qtype
  void forward_shared(const int64_t* ids, const int64_t* mask, int U, int L,
                      const int32_t* row_seq, const int64_t* marker_pos,
                      const uint8_t* marker_mask, const int64_t* qtype, int B, int K,
                      float* logits, float* act);
  // encode_device with every buffer carved out of the library's fixed
  // per-device scratch array: no device allocation, no graph, no pinned
  // staging.  Throws when the batch does not fit the array.
  void encode_device_noalloc(const int32_t* d_ids, const int32_t* h_lens, int B,
                             float* d_hidden, hipStream_t stream);

  void set_profile(bool on);
  void graph_stats(int32_t* cached, int64_t* captures, int64_t* replays);
  std::vector<std::tuple<const char*, double, int64_t>> profile_totals();

 private:
  struct LayerDev {
    DevBuf attn_norm, attn_norm_b, wqkv, wqkv_b, wo, wo_b, mlp_norm, mlp_norm_b, wi, wi_b, wo2,
        wo2_b;                         // the biases and norm biases of the BERT family
    DevBuf wqkv_s, wo_s, wi_s, wo2_s;  // per-row scales of fp8 projections
    // consumer constants of a folded LayerNorm (GemmArgs::ln_c1 / ln_c2):
    // attn_norm over Wqkv, mlp_norm over Wi
    DevBuf ln1_c1, ln1_c2, ln2_c1, ln2_c2;
    bool has_attn_norm = false;
    int window = 0, sliding = 0;
  };
  struct Fp8Dev {
    DevBuf q, scale;
  };
  struct HeadDev {
    DevBuf n1w, n1b, n2w, n2b, in_w, in_b, out_w, out_b, l1w, l1b, l2w, l2b;
  };
  struct Graph {
    hipGraphExec_t exec = nullptr;
    hipEvent_t done = nullptr;  // recorded after each launch: eviction waits on it
    uint64_t last_use = 0;      // LRU eviction
  };
  void drop_graph(Graph& g);
  static constexpr size_t kMaxGraphs = 32;

  void stage_weights(const ModelSource& s);
  // one tensor of a source to the device: fp32, the activation type, or
  // per-row e4m3 codes + scales (converted on the device when the source
  // holds another type)
  DevBuf put_f32(const Src& s, int64_t n, const char* what);
  DevBuf put_f32_opt(const Src& s, int64_t n, const char* what);
  DevBuf put_act(const Src& s, int64_t n, const char* what);
  Fp8Dev put_fp8(const Mat& m, int64_t rows, int64_t cols, const char* what);
  BatchPlan plan(const int64_t* ids, const int64_t* mask, int B, int L, int32_t* ids_out) const;
  BatchPlan plan_lens(const int32_t* h_lens, int B) const;
  void ensure_workspace(int Tb, int Bb);
  // the sequence table (and the token ids) through the pinned staging buffer
  void upload_batch(const BatchPlan& p, const int32_t* h_ids, const int32_t* h_qtype,
                    hipStream_t st);
  // the sequence table of a device-resident batch: built by a kernel from
  // the lengths in its arguments (up to kSeqTableMaxB sequences), else uploaded
  void set_seq_table(const BatchPlan& p, const int32_t* h_lens, int32_t* table, hipStream_t st);
  // device work from token ids to the final hidden states in X (and, with
  // `head`, through the decision-head layers)
  void run_device(const BatchPlan& p, const Ws& w, const int32_t* d_ids, float* X, bool head,
                  hipStream_t st);
  void run_device_maybe_graph(const BatchPlan& p, const int32_t* d_ids, float* X, bool head,
                              hipStream_t st);
  void enqueue_encoder(const BatchPlan& p, const Ws& w, const int32_t* d_ids, float* X,
                       hipStream_t st);
  void enqueue_head_layers(const BatchPlan& p, const Ws& w, float* X, hipStream_t st);
  // scorer and act head on the final hidden states X of plan p (src/model.cpp:461-535)
  void decision_tail(const BatchPlan& p, const float* X, const int64_t* marker_pos,
                     const uint8_t* marker_mask, int L, int K, float* logits, float* act,
                     hipStream_t st);
  // order this call's stream after the engine's previous call (any stream),
  // and mark the end of this call's work
  void begin_call(hipStream_t st);
  void end_call(hipStream_t st);

  // launch helpers (record profile events when enabled)
  void gemm(const char* name, const GemmArgs& g, const Ws& w, hipStream_t st);
  void ln(const char* name, const LnArgs& a, hipStream_t st);
  // X += A . W^T followed by the layer norm `a` that reads X: for short
  // batches the split-K residual epilogue is folded into that layer norm.
  void resid_gemm_ln(const char* gname, const GemmArgs& g, const char* lname, LnArgs a,
                     const Ws& w, hipStream_t st);
  // Sets g up to finish the LayerNorm a (of X's rows into bf16 Y) in its
  // residual epilogue (GemmArgs::rln_y) and returns true where that applies;
  // false leaves g as it was.
  bool rln_resid(GemmArgs& g, const LnArgs& a, const Ws& w) const;
  // polls of a panel's arrival count before a tile gives up waiting
  static constexpr int kRlnSpin = 20000;
  void attn(const char* name, const AttnArgs& a, hipStream_t st);
  void prof_begin(hipStream_t st);
  void prof_end(const char* name, hipStream_t st);
  void prof_collect();

  // Buffers of one forward carved out of the scratch array for plan p, or
  // the number of bytes that would take when it does not fit (ws.seq null).
  size_t scratch_layout(const BatchPlan& p, Ws& ws) const;

  int dev_ = 0;
  char* scratch_ = nullptr;  // this device's copy of the scratch array (engine.cpp)
  bool quiet_ = false;       // no per-launch profile events (the no-allocation path)
  int prec_ = SJH_PREC_BF16;
  int act_dt_ = DT_BF16;  // activation / GEMM operand type
  bool w8_ = false;       // encoder projections stored as fp8 e4m3 + per-row scales
  int D_ = 0, H_ = 0, Dh_ = 0, F_ = 0, V_ = 0, nlayers_ = 0, max_pos_ = 0;
  int n_act_ = 0, head_layers_ = 0, lora_r_ = 0, max_len_ = 0;
  float eps_ = 1e-5f;
  bool attn_split_ = false;  // every layer has full attention and sequences can reach kAttnSplitMinKeys
  // the encoder's LayerNorms after its residual GEMMs can fold into them and
  // the next GEMMs (GemmArgs::ln_y) on the persistent kernel's batches
  bool ln_fold_ = false;
  // the residual GEMMs' epilogues finish the LayerNorm that reads X next
  // where their tiles all run at once (sjh_options::fuse_ln)
  bool rln_ = false;
  int rln_spin_ = 0;  // GemmArgs::rln_spin
  // short batches: attention folds the output projection in (AttnArgs::wo;
  // sjh_options::fuse_attn_wo)
  bool attn_wo_ = false;
  int arch_ = ARCH_MODERNBERT;  // ModernBERT (DecisionModel) or BERT (SjModel)
  int act_head_ = ACT_MLP;
  int head_ff_ = 0, head_act_ = 2;
  float head_eps_ = 1e-5f;
  bool use_graphs_ = true, pad_rows_ = false;

  DevBuf emb_w_, emb_norm_, final_norm_, type_emb_;
  DevBuf pos_emb_, emb_norm_b_, final_norm_b_;  // BERT family
  DevBuf rope_cos_full_, rope_sin_full_, rope_cos_slide_, rope_sin_slide_;
  std::vector<LayerDev> layers_;
  std::vector<HeadDev> head_;
  DevBuf lora_a_, lora_b_;
  DevBuf sc_ln_w_, sc_ln_b_, sc_w1_, sc_b1_, sc_w2_, sc_b2_;
  DevBuf act_w1_, act_b1_, act_w2_, act_b2_;

  // workspace
  int cap_T_ = 0, cap_B_ = 0;
  DevBuf ids_, seqinfo_, tok_pos_, tok_seq_;
  DevBuf X_, Y_, QKV_, O_, G_, Z_;
  DevBuf X2_, expand_idx_;  // forward_shared: hidden states of the (sequence, qtype) pairs
  std::vector<int32_t> tail_hidx_;  // host copy of the head tail's row indices
  DevBuf splitk_;  // split-K partial sums for short batches (GemmArgs::partial)
  DevBuf attn_items_;  // attention work list (AttnArgs::items)
  DevBuf attn_part_;   // partials of key-split attention items (AttnArgs::part)
  DevBuf ln_stats_;    // folded LayerNorm row moments (Ws::ln_stats)
  DevBuf rln_mom_, rln_sync_;  // Ws::rln_mom, Ws::rln_sync
  Ws ws_;          // views of the buffers above
  DevBuf tail_idx_, tail_rows_, tail_s0_, tail_s1_, tail_s2_, tail_lg_, tail_ain_, tail_ah_,
      tail_ao_, tail_act_;
  PinnedBuf h_stage_, h_out_;
  uint64_t ws_gen_ = 0;

  hipStream_t stream_ = nullptr;
  hipEvent_t ev_null_ = nullptr;  // orders NULL-stream callers of encode_device
  // ev_done_: the end of the last call's device work, on whichever stream it
  // ran; every call waits for it first.  ev_upload_: the last copy out of
  // the pinned staging buffer, awaited before the buffer is rewritten.
  hipEvent_t ev_done_ = nullptr, ev_upload_ = nullptr;
  bool done_recorded_ = false, upload_recorded_ = false;
  std::map<std::vector<int64_t>, Graph> graphs_;
  uint64_t graph_clock_ = 0;
  int64_t n_captures_ = 0, n_replays_ = 0;
  std::mutex mu_;

  bool profile_ = false;
  struct ProfEv {
    const char* name;
    hipEvent_t a, b;
  };
  std::vector<ProfEv> prof_pending_;
  std::vector<hipEvent_t> ev_pool_;
  hipEvent_t ev_open_ = nullptr;
  std::map<std::string, std::tuple<const char*, double, int64_t>> prof_tot_;
};

}  // namespace sjh

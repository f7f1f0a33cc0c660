// snapjudge_fast_hip.hpp -- the reference's GPU fast-path class, backed by the
// MI355X C ABI (snapjudge_hip.h).
//
// Same class, constructor and forward() as the reference's
// include/snapjudge/fast.hpp:15-31 (FastSnapjudge, built there under
// SNAPJUDGE_CUDA), so Agent::accelerate (src/agent.cpp:363-386) constructs it
// unchanged; a SNAPJUDGE_HIP build includes this header where the CUDA build
// includes snapjudge/fast.hpp.  It adds encode(), the device twin of
// DecisionModel::encode (src/model.cpp:222-307), for Agent::embed
// (src/agent.cpp:348) and the trainer's frozen encoder.
//
// The class reads the model's fp32 weights through the friend declaration in
// include/snapjudge/model.hpp:128-129 and copies them to the GPU once.  Errors
// throw std::runtime_error("snapjudge HIP: ...") like the reference's
// cuda/fast.cpp:54-58.  Calls are serialised internally (one stream and one
// workspace per instance).
#pragma once

#include <cstdint>
#include <memory>
#include <vector>

namespace snapjudge {

class DecisionModel;

class FastSnapjudge {
 public:
  FastSnapjudge(DecisionModel* model, int max_len, bool use_graphs = true);
  // Numerics mode: precision 0 = fp32 parity path, 1 = bf16 MFMA path (the
  // three-argument constructor's choice), 2 = bf16 path with the encoder
  // projections quantized once to per-row fp8 e4m3 (SJH_PREC_FP8W in
  // snapjudge_hip.h); pad_rows 1 also computes the padded
  // query rows, as the reference does, so encode() returns them too.
  FastSnapjudge(DecisionModel* model, int max_len, bool use_graphs, int precision, int pad_rows);
  ~FastSnapjudge();
  FastSnapjudge(const FastSnapjudge&) = delete;
  FastSnapjudge& operator=(const FastSnapjudge&) = delete;

  // DecisionModel::forward (src/model.cpp:309-536): right-padded ids and mask
  // [N][L], marker positions/mask [N][K], qtype [N] -> logits [N][K] (masked
  // markers -1e4), act [N][n_act].
  void forward(const std::vector<std::vector<int64_t>>& input_ids,
               const std::vector<std::vector<int64_t>>& attention_mask,
               const std::vector<std::vector<int64_t>>& marker_pos,
               const std::vector<std::vector<uint8_t>>& marker_mask,
               const std::vector<int64_t>& qtype,
               std::vector<std::vector<float>>& logits,
               std::vector<std::vector<float>>& act);

  // DecisionModel::encode (src/model.cpp:222-307): hidden states [N][L][D]
  // after the final norm (and LoRA).  Padded positions hold zeros unless the
  // instance computes padded rows (pad_rows).
  std::vector<std::vector<std::vector<float>>> encode(
      const std::vector<std::vector<int64_t>>& input_ids,
      const std::vector<std::vector<int64_t>>& attention_mask);

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

}  // namespace snapjudge

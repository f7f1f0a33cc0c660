// ckpt.hpp -- checkpoint directories read straight into a ModelSource.
#pragma once

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "model_src.hpp"

namespace sjh {

// A memory-mapped .safetensors file (src/safetensors.cpp:16-61): an 8-byte
// little-endian header length, a JSON header of name -> {dtype, shape,
// data_offsets}, then the data.  Tensors are views into the mapping.
class StFile {
 public:
  struct Entry {
    std::string dtype;
    std::vector<int64_t> shape;
    size_t begin = 0, end = 0;  // absolute offsets into the mapping
    int64_t numel = 0;
  };
  explicit StFile(const std::string& path);
  ~StFile();
  StFile(const StFile&) = delete;
  StFile& operator=(const StFile&) = delete;
  bool has(const std::string& name) const { return entries_.count(name) > 0; }
  const Entry& entry(const std::string& name) const;
  const std::vector<std::string>& names() const { return names_; }
  const uint8_t* base() const { return static_cast<const uint8_t*>(map_); }

 private:
  std::string path_;
  void* map_ = nullptr;
  size_t size_ = 0;
  std::map<std::string, Entry> entries_;
  std::vector<std::string> names_;
};

// A checkpoint directory, mapped: either a DecisionModel
// (rl_agent_config.json, encoder/config.json, model.safetensors; the files
// src/agent.cpp:59-85 reads) or an SjModel (sj_config.json +
// model.safetensors).  `src` points into `file`, which stays mapped while the
// Checkpoint lives.
struct Checkpoint {
  std::unique_ptr<StFile> file;
  ModelSource src;
  int max_len = 0;  // the config's max_len
};
std::unique_ptr<Checkpoint> read_checkpoint(const std::string& dir);

}  // namespace sjh

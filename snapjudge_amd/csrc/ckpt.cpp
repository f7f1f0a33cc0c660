// ckpt.cpp -- checkpoint directories read straight into a ModelSource.
//
// Mirrors the reference's loaders: the safetensors reader
// (src/safetensors.cpp:16-61, with a size check for every dtype, not only
// F32), DecisionModel::load (src/model.cpp:35-205: configuration keys and
// defaults, required prefixes, strict shapes, optional scorer biases, optional
// LoRA) and SjModel::load (src/sj_model.cpp:87-204).  Tensors stay in the
// mapping; the engine converts them on the device while staging.  Beyond the
// reference, the four encoder projections of a DecisionModel may be stored
// as e4m3 codes ("F8_E4M3") with one fp32 scale per output row in
// "<name>_scale" (the SJH_PREC_FP8W format).
#include "ckpt.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>

#include "sjh_host.hpp"

namespace sjh {

// ------------------------------------------------------------------- json --
namespace {

// A parsed JSON value (objects keep their keys in order of appearance).
struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;

  const JVal* get(const std::string& k) const {
    if (kind != OBJ) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
  bool has(const std::string& k) const { return get(k) != nullptr; }
  const char* type_name() const {
    static const char* const names[] = {"null", "boolean", "number", "string", "array", "object"};
    return names[kind];
  }
  // the reference's json.value(key, default) for numbers: the default when the
  // key is absent; a present key must hold a number (a boolean reads as 0 or
  // 1), anything else fails as the reference's type error does
  double number(const std::string& k, double dflt) const {
    const JVal* v = get(k);
    if (!v) return dflt;
    if (v->kind == BOOL) return v->b ? 1.0 : 0.0;
    if (v->kind != NUM)
      fail_arg("config key '" + k + "': type must be number, but is " + v->type_name());
    return v->num;
  }
  int integer(const std::string& k, int dflt) const {
    return static_cast<int>(number(k, static_cast<double>(dflt)));
  }
};

class JParser {
 public:
  JParser(const char* b, const char* e, const std::string& what) : p_(b), e_(e), what_(what) {}
  JVal parse() {
    JVal v = value();
    ws();
    if (p_ != e_) bad("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void bad(const char* why) { fail_arg("bad JSON in " + what_ + ": " + why); }
  void ws() {
    while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if (static_cast<size_t>(e_ - p_) >= n && std::memcmp(p_, s, n) == 0) {
      p_ += n;
      return true;
    }
    return false;
  }
  JVal value() {
    if (++depth_ > 64) bad("nesting too deep");
    ws();
    if (p_ >= e_) bad("unexpected end");
    JVal v;
    const char c = *p_;
    if (c == '{') {
      v.kind = JVal::OBJ;
      ++p_;
      ws();
      if (p_ < e_ && *p_ == '}') {
        ++p_;
      } else {
        for (;;) {
          ws();
          if (p_ >= e_ || *p_ != '"') bad("expected a key");
          std::string k = string();
          ws();
          if (p_ >= e_ || *p_ != ':') bad("expected ':'");
          ++p_;
          v.obj.emplace_back(std::move(k), value());
          ws();
          if (p_ < e_ && *p_ == ',') { ++p_; continue; }
          if (p_ < e_ && *p_ == '}') { ++p_; break; }
          bad("expected ',' or '}'");
        }
      }
    } else if (c == '[') {
      v.kind = JVal::ARR;
      ++p_;
      ws();
      if (p_ < e_ && *p_ == ']') {
        ++p_;
      } else {
        for (;;) {
          v.arr.push_back(value());
          ws();
          if (p_ < e_ && *p_ == ',') { ++p_; continue; }
          if (p_ < e_ && *p_ == ']') { ++p_; break; }
          bad("expected ',' or ']'");
        }
      }
    } else if (c == '"') {
      v.kind = JVal::STR;
      v.str = string();
    } else if (lit("true")) {
      v.kind = JVal::BOOL;
      v.b = true;
    } else if (lit("false")) {
      v.kind = JVal::BOOL;
    } else if (lit("null")) {
      v.kind = JVal::NUL;
    } else {
      v.kind = JVal::NUM;
      std::string tok;
      while (p_ < e_ && (std::strchr("+-0123456789.eE", *p_) != nullptr)) tok.push_back(*p_++);
      if (tok.empty()) bad("unexpected character");
      char* end = nullptr;
      v.num = std::strtod(tok.c_str(), &end);
      if (!end || *end != '\0') bad("bad number");
    }
    --depth_;
    return v;
  }
  std::string string() {
    ++p_;  // opening quote
    std::string s;
    while (p_ < e_ && *p_ != '"') {
      char c = *p_++;
      if (c == '\\') {
        if (p_ >= e_) bad("bad escape");
        const char x = *p_++;
        switch (x) {
          case '"': case '\\': case '/': s.push_back(x); break;
          case 'b': s.push_back('\b'); break;
          case 'f': s.push_back('\f'); break;
          case 'n': s.push_back('\n'); break;
          case 'r': s.push_back('\r'); break;
          case 't': s.push_back('\t'); break;
          case 'u': {
            if (e_ - p_ < 4) bad("bad \\u escape");
            const unsigned cp = static_cast<unsigned>(std::strtoul(std::string(p_, 4).c_str(), nullptr, 16));
            p_ += 4;
            // names and config strings here are ASCII; other code points are
            // kept as UTF-8 of the BMP value
            if (cp < 0x80) {
              s.push_back(static_cast<char>(cp));
            } else if (cp < 0x800) {
              s.push_back(static_cast<char>(0xC0 | (cp >> 6)));
              s.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
            } else {
              s.push_back(static_cast<char>(0xE0 | (cp >> 12)));
              s.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
              s.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
            }
            break;
          }
          default: bad("bad escape");
        }
      } else {
        s.push_back(c);
      }
    }
    if (p_ >= e_) bad("unterminated string");
    ++p_;
    return s;
  }
  const char* p_;
  const char* e_;
  std::string what_;
  int depth_ = 0;
};

JVal read_json(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) fail_arg("cannot open " + path);
  std::stringstream ss;
  ss << f.rdbuf();
  const std::string t = ss.str();
  return JParser(t.data(), t.data() + t.size(), path).parse();
}

bool file_exists(const std::string& p) {
  struct stat st;
  return ::stat(p.c_str(), &st) == 0;
}
}  // namespace

// ---------------------------------------------------------------- StFile --
StFile::StFile(const std::string& path) : path_(path) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) fail_arg("cannot open " + path);
  struct stat st;
  if (::fstat(fd, &st) != 0) {
    ::close(fd);
    fail_arg("cannot stat " + path);
  }
  size_ = static_cast<size_t>(st.st_size);
  if (size_ < 8) {
    ::close(fd);
    fail_arg("not a safetensors file (too small): " + path);
  }
  map_ = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (map_ == MAP_FAILED) {
    map_ = nullptr;
    fail_arg("mmap failed for " + path);
  }
  uint64_t hlen = 0;
  std::memcpy(&hlen, map_, 8);
  if (hlen > size_ - 8) fail_arg("bad header length in " + path);
  const char* h = static_cast<const char*>(map_) + 8;
  const JVal hdr = JParser(h, h + hlen, path + " (safetensors header)").parse();
  if (hdr.kind != JVal::OBJ) fail_arg("safetensors header is not an object: " + path);
  const size_t base = 8 + hlen;
  for (const auto& kv : hdr.obj) {
    if (kv.first == "__metadata__") continue;
    const JVal& v = kv.second;
    Entry e;
    const JVal* dt = v.get("dtype");
    const JVal* sh = v.get("shape");
    const JVal* off = v.get("data_offsets");
    if (!dt || dt->kind != JVal::STR || !sh || sh->kind != JVal::ARR || !off ||
        off->kind != JVal::ARR || off->arr.size() != 2)
      fail_arg("bad header entry " + kv.first + " in " + path);
    e.dtype = dt->str;
    e.numel = 1;
    for (const JVal& d : sh->arr) {
      if (d.kind != JVal::NUM || d.num < 0) fail_arg("bad shape of " + kv.first + " in " + path);
      e.shape.push_back(static_cast<int64_t>(d.num));
      e.numel *= e.shape.back();
    }
    const double b0 = off->arr[0].num, b1 = off->arr[1].num;
    if (b0 < 0 || b1 < b0) fail_arg("bad data offsets of " + kv.first + " in " + path);
    e.begin = base + static_cast<size_t>(b0);
    e.end = base + static_cast<size_t>(b1);
    if (e.end > size_) fail_arg("tensor out of bounds in " + path);
    size_t es = 0;
    if (e.dtype == "F32") es = 4;
    else if (e.dtype == "F16" || e.dtype == "BF16") es = 2;
    else if (e.dtype == "F8_E4M3") es = 1;
    if (es && e.end - e.begin != static_cast<size_t>(e.numel) * es)
      fail_arg("size mismatch " + kv.first + " in " + path);
    names_.push_back(kv.first);
    entries_[kv.first] = std::move(e);
  }
}

StFile::~StFile() {
  if (map_) ::munmap(map_, size_);
}

const StFile::Entry& StFile::entry(const std::string& name) const {
  auto it = entries_.find(name);
  if (it == entries_.end()) fail_arg("no tensor named " + name + " in " + path_);
  return it->second;
}

// ------------------------------------------------------------- readers --
namespace {

std::string shape_str(const std::vector<int64_t>& s) {
  std::string o = "[";
  for (size_t i = 0; i < s.size(); ++i) o += (i ? "," : "") + std::to_string(s[i]);
  return o + "]";
}

// A tensor of the file as a staging source, with the reference's strict
// shape check (require_shape, src/model.cpp and src/sj_model.cpp).  F32,
// F16 and BF16 as in src/safetensors.cpp:109-135; "F8_E4M3" only where the
// caller allows codes (a projection with its row scales).
Src take(const StFile& f, const std::string& name, std::vector<int64_t> want,
         const std::string& id, bool allow_f8 = false) {
  if (!f.has(name)) fail_arg("model '" + id + "': missing tensor " + name);
  const StFile::Entry& e = f.entry(name);
  if (e.shape != want)
    fail_arg("model '" + id + "': tensor " + name + " expected " + shape_str(want) + " but has " +
             shape_str(e.shape));
  Seg s;
  s.p = f.base() + e.begin;
  s.n = e.numel;
  if (e.dtype == "F32") s.type = SRC_F32;
  else if (e.dtype == "F16") s.type = SRC_F16;
  else if (e.dtype == "BF16") s.type = SRC_BF16;
  else if (e.dtype == "F8_E4M3" && allow_f8) s.type = SRC_F8;
  else fail_arg("unsupported dtype " + e.dtype + " for " + name);
  Src out;
  out.segs.push_back(s);
  return out;
}

Src take_opt(const StFile& f, const std::string& name, std::vector<int64_t> want,
             const std::string& id) {
  return f.has(name) ? take(f, name, std::move(want), id) : Src();
}

// A projection: F32/F16/BF16 rows, or e4m3 codes with "<name>_scale" [rows] F32.
Mat take_mat(const StFile& f, const std::string& name, int64_t rows, int64_t cols,
             const std::string& id) {
  Mat m;
  m.w = take(f, name, {rows, cols}, id, true);
  if (m.w.segs[0].type == SRC_F8) {
    m.scale = take(f, name + "_scale", {rows}, id);
    if (m.scale.segs[0].type != SRC_F32) fail_arg("model '" + id + "': " + name + "_scale must be F32");
  }
  return m;
}

void cat(Src& a, const Src& b) { a.segs.insert(a.segs.end(), b.segs.begin(), b.segs.end()); }

// src/model.cpp:35-205
void read_decision(Checkpoint& ck, const std::string& dir) {
  const JVal rl = read_json(dir + "/rl_agent_config.json");
  const JVal enc = read_json(dir + "/encoder/config.json");
  const std::string id = dir;
  for (const char* k : {"encoder", "head_layers"})
    if (!rl.has(k))
      fail_arg("Incompatible model config for '" + id + "': missing configuration keys ['" + k +
               "']. Ensure this is a valid RL Agent decision model.");
  ck.file = std::make_unique<StFile>(dir + "/model.safetensors");
  const StFile& f = *ck.file;
  for (const char* p : {"encoder.", "type_emb.", "scorer.", "act_head."}) {
    bool any = false;
    for (const auto& n : f.names())
      if (n.rfind(p, 0) == 0) {
        any = true;
        break;
      }
    if (!any)
      fail_arg("Incompatible model weights for '" + id + "': checkpoint is missing '" + p +
               "' parameters.");
  }
  ModelSource& s = ck.src;
  s.arch = ARCH_MODERNBERT;
  s.act_head = ACT_MLP;
  s.head_layers = rl.integer("head_layers", 2);
  ck.max_len = rl.integer("max_len", 512);
  const JVal* costs = rl.get("act_costs");
  s.n_act = (costs && costs->kind == JVal::OBJ ? static_cast<int>(costs->obj.size()) : 0) + 1;
  s.D = enc.integer("hidden_size", 0);
  s.n_layers = enc.integer("num_hidden_layers", 0);
  s.H = enc.integer("num_attention_heads", 0);
  s.F = enc.integer("intermediate_size", 0);
  s.max_pos = enc.integer("max_position_embeddings", 8192);
  s.V = enc.integer("vocab_size", 0);
  s.eps = static_cast<float>(enc.number("norm_eps", 1e-5));
  const int local = enc.integer("local_attention", 0);
  std::vector<std::string> types;
  if (const JVal* lt = enc.get("layer_types"))
    for (const JVal& t : lt->arr) types.push_back(t.str);
  if (const JVal* rp = enc.get("rope_parameters")) {
    if (const JVal* fa = rp->get("full_attention")) s.theta_full = fa->number("rope_theta", s.theta_full);
    if (const JVal* sa = rp->get("sliding_attention"))
      s.theta_sliding = sa->number("rope_theta", s.theta_sliding);
  }
  if (s.D <= 0 || s.H <= 0 || s.D % s.H != 0) fail_arg("model '" + id + "': bad hidden_size / heads");
  const int64_t D = s.D, F = s.F, V = s.V;
  s.emb_w = take(f, "encoder.embeddings.tok_embeddings.weight", {V, D}, id);
  s.emb_norm = take(f, "encoder.embeddings.norm.weight", {D}, id);
  s.final_norm = take(f, "encoder.final_norm.weight", {D}, id);
  const int win = local > 0 ? local / 2 : 0;
  s.layers.resize(static_cast<size_t>(s.n_layers));
  for (int i = 0; i < s.n_layers; ++i) {
    LayerSrc& ly = s.layers[static_cast<size_t>(i)];
    const std::string p = "encoder.layers." + std::to_string(i) + ".";
    const std::string type = i < static_cast<int>(types.size()) ? types[static_cast<size_t>(i)]
                                                                : "full_attention";
    ly.sliding = type == "sliding_attention" ? 1 : 0;
    ly.window = ly.sliding ? win : 0;
    ly.attn_norm = take_opt(f, p + "attn_norm.weight", {D}, id);
    ly.wqkv = take_mat(f, p + "attn.Wqkv.weight", 3 * D, D, id);
    ly.wo = take_mat(f, p + "attn.Wo.weight", D, D, id);
    ly.mlp_norm = take(f, p + "mlp_norm.weight", {D}, id);
    ly.wi = take_mat(f, p + "mlp.Wi.weight", 2 * F, D, id);
    ly.wo2 = take_mat(f, p + "mlp.Wo.weight", D, F, id);
  }
  s.type_emb = take(f, "type_emb.weight", {3, D}, id);
  s.head_ff = 4 * s.D;
  s.head_eps = 1e-5f;
  s.head_act = 2;
  s.head.resize(static_cast<size_t>(s.head_layers));
  for (int i = 0; i < s.head_layers; ++i) {
    HeadSrc& h = s.head[static_cast<size_t>(i)];
    const std::string p = "head.layers." + std::to_string(i) + ".";
    h.n1w = take(f, p + "norm1.weight", {D}, id);
    h.n1b = take(f, p + "norm1.bias", {D}, id);
    h.n2w = take(f, p + "norm2.weight", {D}, id);
    h.n2b = take(f, p + "norm2.bias", {D}, id);
    h.in_w = take(f, p + "self_attn.in_proj_weight", {3 * D, D}, id);
    h.in_b = take(f, p + "self_attn.in_proj_bias", {3 * D}, id);
    h.out_w = take(f, p + "self_attn.out_proj.weight", {D, D}, id);
    h.out_b = take(f, p + "self_attn.out_proj.bias", {D}, id);
    h.l1w = take(f, p + "linear1.weight", {4 * D, D}, id);
    h.l1b = take(f, p + "linear1.bias", {4 * D}, id);
    h.l2w = take(f, p + "linear2.weight", {D, 4 * D}, id);
    h.l2b = take(f, p + "linear2.bias", {D}, id);
  }
  s.sc_ln_w = take(f, "scorer.0.weight", {D}, id);
  s.sc_ln_b = take_opt(f, "scorer.0.bias", {D}, id);
  s.sc_w1 = take(f, "scorer.1.weight", {D, D}, id);
  s.sc_b1 = take_opt(f, "scorer.1.bias", {D}, id);
  s.sc_w2 = take(f, "scorer.3.weight", {1, D}, id);
  s.sc_b2 = take_opt(f, "scorer.3.bias", {1}, id);
  s.act_w1 = take(f, "act_head.0.weight", {256, D + 4}, id);
  s.act_b1 = take(f, "act_head.0.bias", {256}, id);
  s.act_w2 = take(f, "act_head.2.weight", {s.n_act, 256}, id);
  s.act_b2 = take(f, "act_head.2.bias", {s.n_act}, id);
  if (f.has("lora_A.weight") && f.has("lora_B.weight")) {  // src/model.cpp:192-203
    const auto& a = f.entry("lora_A.weight").shape;
    const auto& b = f.entry("lora_B.weight").shape;
    if (a.size() != 2 || b.size() != 2 || a[0] != b[1] || a[1] != D || b[0] != D)
      fail_arg("Model 'lora_A.weight'/'lora_B.weight' must be [r,D] and [D,r]");
    s.lora_r = static_cast<int>(a[0]);
    s.lora_a = take(f, "lora_A.weight", {a[0], D}, id);
    s.lora_b = take(f, "lora_B.weight", {D, a[0]}, id);
  }
}

// src/sj_model.cpp:87-204
void read_sj(Checkpoint& ck, const std::string& dir) {
  const JVal c = read_json(dir + "/sj_config.json");
  const std::string id = dir;
  for (const char* k : {"vocab_size", "hidden_size", "num_layers", "num_heads"})
    if (!c.has(k))
      fail_arg("SjModel '" + id + "': config missing required keys (vocab_size/hidden_size/num_layers/num_heads)");
  ModelSource& s = ck.src;
  s.arch = ARCH_BERT;
  s.act_head = ACT_TOP1;
  s.n_act = 2;
  s.V = c.integer("vocab_size", 0);
  s.D = c.integer("hidden_size", 0);
  s.n_layers = c.integer("num_layers", 0);
  s.H = c.integer("num_heads", 0);
  s.F = c.integer("intermediate_size", 4 * s.D);
  s.max_pos = c.integer("max_positions", 512);
  s.eps = static_cast<float>(c.number("norm_eps", 1e-5));
  s.head_layers = c.integer("head_layers", 1);
  s.head_ff = c.integer("head_intermediate", 4 * s.D);
  s.head_eps = s.eps;
  s.head_act = 1;
  ck.max_len = c.integer("max_len", 512);
  const int n_types = c.integer("n_types", 3);
  if (s.D <= 0 || s.H <= 0 || s.D % s.H != 0)
    fail_arg("SjModel '" + id + "': hidden_size must be divisible by num_heads");
  if (n_types != 3) fail_arg("SjModel '" + id + "': only the three question types are supported");
  ck.file = std::make_unique<StFile>(dir + "/model.safetensors");
  const StFile& f = *ck.file;
  const int64_t D = s.D, F = s.F, HF = s.head_ff;
  s.emb_w = take(f, "sj.embeddings.word.weight", {s.V, D}, id);
  s.pos_emb = take(f, "sj.embeddings.position.weight", {s.max_pos, D}, id);
  s.emb_norm = take(f, "sj.embeddings.norm.weight", {D}, id);
  s.emb_norm_b = take(f, "sj.embeddings.norm.bias", {D}, id);
  s.layers.resize(static_cast<size_t>(s.n_layers));
  for (int i = 0; i < s.n_layers; ++i) {
    LayerSrc& ly = s.layers[static_cast<size_t>(i)];
    const std::string p = "sj.encoder.layers." + std::to_string(i) + ".";
    ly.attn_norm = take(f, p + "attn_norm.weight", {D}, id);
    ly.attn_norm_b = take(f, p + "attn_norm.bias", {D}, id);
    // q, k, v as the row blocks of one [3D, D] projection (the packed
    // (q|k|v)(head)(dim) rows the attention kernel reads)
    for (const char* x : {"q", "k", "v"}) {
      cat(ly.wqkv.w, take(f, p + "attn." + x + ".weight", {D, D}, id));
      cat(ly.wqkv_b, take(f, p + "attn." + x + ".bias", {D}, id));
    }
    ly.wo.w = take(f, p + "attn.o.weight", {D, D}, id);
    ly.wo_b = take(f, p + "attn.o.bias", {D}, id);
    ly.mlp_norm = take(f, p + "ffn_norm.weight", {D}, id);
    ly.mlp_norm_b = take(f, p + "ffn_norm.bias", {D}, id);
    ly.wi.w = take(f, p + "ffn.w1.weight", {F, D}, id);
    ly.wi_b = take(f, p + "ffn.w1.bias", {F}, id);
    ly.wo2.w = take(f, p + "ffn.w2.weight", {D, F}, id);
    ly.wo2_b = take(f, p + "ffn.w2.bias", {D}, id);
  }
  s.final_norm = take(f, "sj.encoder.final_norm.weight", {D}, id);
  s.final_norm_b = take(f, "sj.encoder.final_norm.bias", {D}, id);
  s.type_emb = take(f, "sj.type_emb.weight", {3, D}, id);
  s.head.resize(static_cast<size_t>(s.head_layers));
  for (int i = 0; i < s.head_layers; ++i) {
    HeadSrc& h = s.head[static_cast<size_t>(i)];
    const std::string p = "sj.head.layers." + std::to_string(i) + ".";
    h.n1w = take(f, p + "norm1.weight", {D}, id);
    h.n1b = take(f, p + "norm1.bias", {D}, id);
    h.n2w = take(f, p + "norm2.weight", {D}, id);
    h.n2b = take(f, p + "norm2.bias", {D}, id);
    for (const char* x : {"q", "k", "v"}) {
      cat(h.in_w, take(f, p + "attn." + x + ".weight", {D, D}, id));
      cat(h.in_b, take(f, p + "attn." + x + ".bias", {D}, id));
    }
    h.out_w = take(f, p + "attn.o.weight", {D, D}, id);
    h.out_b = take(f, p + "attn.o.bias", {D}, id);
    h.l1w = take(f, p + "ffn.w1.weight", {HF, D}, id);
    h.l1b = take(f, p + "ffn.w1.bias", {HF}, id);
    h.l2w = take(f, p + "ffn.w2.weight", {D, HF}, id);
    h.l2b = take(f, p + "ffn.w2.bias", {D}, id);
  }
  s.sc_ln_w = take(f, "sj.scorer.norm.weight", {D}, id);
  s.sc_ln_b = take(f, "sj.scorer.norm.bias", {D}, id);
  s.sc_w1 = take(f, "sj.scorer.w1.weight", {D, D}, id);
  s.sc_b1 = take(f, "sj.scorer.w1.bias", {D}, id);
  s.sc_w2 = take(f, "sj.scorer.w2.weight", {1, D}, id);
  s.sc_b2 = take(f, "sj.scorer.w2.bias", {1}, id);
}
}  // namespace

std::unique_ptr<Checkpoint> read_checkpoint(const std::string& dir) {
  auto ck = std::make_unique<Checkpoint>();
  if (file_exists(dir + "/sj_config.json"))
    read_sj(*ck, dir);
  else if (file_exists(dir + "/rl_agent_config.json") && file_exists(dir + "/encoder/config.json"))
    read_decision(*ck, dir);
  else
    fail_arg("no checkpoint in " + dir +
             ": expected sj_config.json, or rl_agent_config.json and encoder/config.json");
  return ck;
}

}  // namespace sjh

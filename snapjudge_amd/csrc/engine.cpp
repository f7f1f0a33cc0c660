// engine.cpp -- device-resident DecisionModel forward (host orchestration).
#include "engine.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

#include "sjh_fp8.hpp"
#include "sjh_host.hpp"

namespace sjh {

// ------------------------------------------------------------------ buffers --
DevBuf::~DevBuf() {
  if (p_) (void)hipFree(p_);
}

DevBuf& DevBuf::operator=(DevBuf&& o) noexcept {
  if (this != &o) {
    if (p_) (void)hipFree(p_);
    p_ = o.p_;
    bytes_ = o.bytes_;
    o.p_ = nullptr;
    o.bytes_ = 0;
  }
  return *this;
}

void DevBuf::alloc(size_t bytes) {
  if (p_) hip_check(hipFree(p_), "hipFree");
  p_ = nullptr;
  bytes_ = 0;
  if (bytes == 0) return;
  hipError_t e = hipMalloc(&p_, bytes);
  if (e != hipSuccess) {
    p_ = nullptr;
    (void)hipGetLastError();
    throw std::runtime_error("snapjudge HIP: out of device memory (" + std::to_string(bytes) +
                             " bytes)");
  }
  bytes_ = bytes;
}

void DevBuf::ensure(size_t bytes) {
  if (bytes > bytes_) alloc(bytes);
}

PinnedBuf::~PinnedBuf() {
  if (p_) (void)hipHostFree(p_);
}

void PinnedBuf::ensure(size_t bytes) {
  if (bytes <= bytes_) return;
  if (p_) hip_check(hipHostFree(p_), "hipHostFree");
  p_ = nullptr;
  bytes_ = 0;
  hip_check(hipHostMalloc(&p_, bytes, hipHostMallocDefault), "hipHostMalloc");
  bytes_ = bytes;
}

uint8_t fp8_e4m3_rne(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  return fp8_e4m3_rne_bits(u);
}

// Per-row symmetric quantization: scale[r] = max |w[r, :]| / 448 (1 for an
// all-zero row), q[r, c] = e4m3(w[r, c] / scale[r]).  Row r then stands for
// decode(q[r, :]) * scale[r].  convert.hip's device quantizer computes the
// same codes and scales.
void quantize_fp8_rows(const float* w, size_t rows, size_t cols, uint8_t* q, float* scale) {
  for (size_t r = 0; r < rows; ++r) {
    const float* row = w + r * cols;
    float amax = 0.f;
    for (size_t c = 0; c < cols; ++c) {
      const float v = std::fabs(row[c]);
      if (v > amax) amax = v;  // NaN compares false
    }
    const float sc = fp8_row_scale(amax);
    scale[r] = sc;
    for (size_t c = 0; c < cols; ++c) q[r * cols + c] = fp8_e4m3_rne(row[c] / sc);
  }
}

namespace {
// RoPE tables exactly as src/model.cpp:173-190: inverse frequency and angle in
// double, cos/sin rounded to float; [max_pos, Dh/2].
void rope_table(double theta, int max_pos, int Dh, std::vector<float>& c, std::vector<float>& s) {
  const int half = Dh / 2;
  c.resize(static_cast<size_t>(max_pos) * half);
  s.resize(c.size());
  for (int pos = 0; pos < max_pos; ++pos)
    for (int d = 0; d < half; ++d) {
      const double inv = 1.0 / std::pow(theta, 2.0 * static_cast<double>(d) / Dh);
      const double fr = static_cast<double>(pos) * inv;
      c[static_cast<size_t>(pos) * half + d] = static_cast<float>(std::cos(fr));
      s[static_cast<size_t>(pos) * half + d] = static_cast<float>(std::sin(fr));
    }
}

size_t dt_size(int dt) { return dt == DT_BF16 ? 2 : 4; }

template <typename T>
const T* off(const void* base, int64_t elems, int dt) {
  return reinterpret_cast<const T*>(static_cast<const char*>(base) + elems * dt_size(dt));
}

}  // namespace

// ------------------------------------------------------------------ scratch --
// The workspace of sjh_model_encode_device_noalloc: one array per device,
// shared by every model on that device, held until the process ends.  Host
// code never names it directly (its host-side symbol is a stand-in, not a
// device address); each device's address comes from hipGetSymbolAddress with
// that device current, once, and is kept here.
namespace {
constexpr size_t kScratchBytes = SJH_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_ptr[kMaxDevices] = {};

// The calling thread's current device must be `dev`.
char* scratch_for_device(int dev) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (dev < 0 || dev >= kMaxDevices) fail("device ordinal out of range for the scratch table");
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = static_cast<char*>(p);
  }
  return g_scratch_ptr[dev];
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }
}  // namespace

// ------------------------------------------------------------------ engine --
ModelSource source_from_desc(const sjh_model_desc& d) {
  ModelSource s;
  s.arch = ARCH_MODERNBERT;
  s.act_head = ACT_MLP;
  s.D = d.hidden_size;
  s.H = d.num_heads;
  s.F = d.intermediate_size;
  s.V = d.vocab_size;
  s.n_layers = d.num_layers;
  s.max_pos = d.max_position;
  s.n_act = d.n_act;
  s.head_layers = d.head_layers;
  s.lora_r = (d.lora_a && d.lora_b) ? d.lora_r : 0;
  s.eps = d.norm_eps;
  s.head_ff = 4 * d.hidden_size;
  s.head_eps = 1e-5f;
  s.head_act = 2;
  s.theta_full = d.rope_theta_full;
  s.theta_sliding = d.rope_theta_sliding;
  const int64_t D = d.hidden_size, F = d.intermediate_size, V = d.vocab_size;
  auto h = [](const float* p, int64_t n) { return Src::host_f32(p, n); };
  auto hm = [](const float* p, int64_t n) {
    Mat m;
    m.w = Src::host_f32(p, n);
    return m;
  };
  s.emb_w = h(d.emb_w, V * D);
  s.emb_norm = h(d.emb_norm, D);
  s.final_norm = h(d.final_norm, D);
  s.rope_cos_full = d.rope_cos_full;
  s.rope_sin_full = d.rope_sin_full;
  s.rope_cos_slide = d.rope_cos_slide;
  s.rope_sin_slide = d.rope_sin_slide;
  if (d.num_layers > 0 && !d.layers) fail("model descriptor: missing layers");
  for (int i = 0; i < d.num_layers; ++i) {
    const sjh_layer_desc& l = d.layers[i];
    LayerSrc ly;
    ly.attn_norm = h(l.attn_norm, D);
    ly.wqkv = hm(l.wqkv, 3 * D * D);
    ly.wo = hm(l.wo, D * D);
    ly.mlp_norm = h(l.mlp_norm, D);
    ly.wi = hm(l.wi, 2 * F * D);
    ly.wo2 = hm(l.wo2, D * F);
    ly.window = l.window;
    ly.sliding = l.sliding;
    s.layers.push_back(ly);
  }
  if (s.lora_r > 0) {
    s.lora_a = h(d.lora_a, s.lora_r * D);
    s.lora_b = h(d.lora_b, D * s.lora_r);
  }
  s.type_emb = h(d.type_emb, 3 * D);
  if (d.head_layers > 0 && !d.head) fail("model descriptor: missing head layers");
  for (int i = 0; i < d.head_layers; ++i) {
    const sjh_head_desc& hd = d.head[i];
    HeadSrc x;
    x.n1w = h(hd.n1w, D), x.n1b = h(hd.n1b, D), x.n2w = h(hd.n2w, D), x.n2b = h(hd.n2b, D);
    x.in_w = h(hd.in_w, 3 * D * D), x.in_b = h(hd.in_b, 3 * D);
    x.out_w = h(hd.out_w, D * D), x.out_b = h(hd.out_b, D);
    x.l1w = h(hd.l1w, 4 * D * D), x.l1b = h(hd.l1b, 4 * D);
    x.l2w = h(hd.l2w, D * 4 * D), x.l2b = h(hd.l2b, D);
    s.head.push_back(x);
  }
  s.sc_ln_w = h(d.sc_ln_w, D);
  s.sc_ln_b = h(d.sc_ln_b, D);
  s.sc_w1 = h(d.sc_w1, D * D);
  s.sc_b1 = h(d.sc_b1, D);
  s.sc_w2 = h(d.sc_w2, D);
  s.sc_b2 = h(d.sc_b2, 1);
  s.act_w1 = h(d.act_w1, 256 * (D + 4));
  s.act_b1 = h(d.act_b1, 256);
  s.act_w2 = h(d.act_w2, static_cast<int64_t>(d.n_act) * 256);
  s.act_b2 = h(d.act_b2, d.n_act);
  return s;
}

Engine::Engine(const ModelSource& src, const sjh_options& o) {
  dev_ = o.device;
  int ndev = 0;
  hip_check(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
  if (dev_ < 0 || dev_ >= ndev) fail("device ordinal " + std::to_string(dev_) + " not present");
  hip_check(hipSetDevice(dev_), "hipSetDevice");
  hipDeviceProp_t prop;
  hip_check(hipGetDeviceProperties(&prop, dev_), "hipGetDeviceProperties");
  if (std::string(prop.gcnArchName).find("gfx950") == std::string::npos)
    fail(std::string("device is ") + prop.gcnArchName + "; this library is built for gfx950");

  require(o.precision == SJH_PREC_FP32 || o.precision == SJH_PREC_BF16 ||
              o.precision == SJH_PREC_FP8W,
          "unknown precision");
  prec_ = o.precision;
  act_dt_ = prec_ == SJH_PREC_FP32 ? DT_F32 : DT_BF16;
  w8_ = prec_ == SJH_PREC_FP8W;
  use_graphs_ = o.use_graphs != 0;
  pad_rows_ = o.pad_rows != 0;
  rln_ = o.fuse_ln != 0;
  rln_spin_ = o.fuse_ln == 2 ? 1 : kRlnSpin;
  attn_wo_ = o.fuse_attn_wo != 0;

  arch_ = src.arch;
  act_head_ = src.act_head;
  D_ = src.D;
  H_ = src.H;
  F_ = src.F;
  V_ = src.V;
  nlayers_ = src.n_layers;
  max_pos_ = src.max_pos;
  n_act_ = src.n_act;
  head_layers_ = src.head_layers;
  head_ff_ = src.head_ff;
  head_eps_ = src.head_eps;
  head_act_ = src.head_act;
  lora_r_ = src.lora_r;
  eps_ = src.eps;
  require(arch_ == ARCH_MODERNBERT || arch_ == ARCH_BERT, "unknown model family");
  require(D_ > 0 && H_ > 0 && D_ % H_ == 0, "hidden_size must be a positive multiple of num_heads");
  Dh_ = D_ / H_;
  require(Dh_ % 2 == 0, "head_dim must be even");
  require(F_ > 0 && V_ > 0 && nlayers_ > 0 && max_pos_ > 0, "bad model dimensions");
  require(!w8_ || (D_ % 64 == 0 && F_ % 64 == 0),
          "fp8 weights need hidden_size and intermediate_size multiples of 64");
  require(n_act_ > 0 && head_layers_ >= 0 && lora_r_ >= 0 && (head_layers_ == 0 || head_ff_ > 0),
          "bad head dimensions");
  require(act_head_ != ACT_TOP1 || n_act_ == 2, "the top-1 act head has two outputs");
  require(static_cast<int>(src.layers.size()) == nlayers_ &&
              static_cast<int>(src.head.size()) == head_layers_,
          "model source: layer count mismatch");
  // ModernBERT rows are bounded by the RoPE tables; the BERT family clamps
  // positions past its table to the last row (src/sj_model.cpp:229-236), so
  // its rows are bounded only by the caller's max_len
  if (arch_ == ARCH_BERT)
    max_len_ = o.max_len > 0 ? o.max_len : (1 << 24);
  else
    max_len_ = o.max_len > 0 ? std::min(o.max_len, max_pos_) : max_pos_;

  hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
  hip_check(hipEventCreateWithFlags(&ev_done_, hipEventDisableTiming), "hipEventCreate");
  hip_check(hipEventCreateWithFlags(&ev_upload_, hipEventDisableTiming), "hipEventCreate");
  hip_check(hipEventCreateWithFlags(&ev_null_, hipEventDisableTiming), "hipEventCreate");
  try {
    scratch_ = scratch_for_device(dev_);
    stage_weights(src);
    hip_check(hipStreamSynchronize(stream_), "weight staging");
  } catch (...) {  // the destructor does not run for a constructor that throws
    (void)hipStreamSynchronize(stream_);
    (void)hipEventDestroy(ev_null_);
    (void)hipEventDestroy(ev_done_);
    (void)hipEventDestroy(ev_upload_);
    (void)hipStreamDestroy(stream_);
    throw;
  }
}

Engine::~Engine() {
  (void)hipSetDevice(dev_);
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (auto& kv : graphs_) {
    if (kv.second.done) (void)hipEventSynchronize(kv.second.done);
    drop_graph(kv.second);
  }
  for (auto& p : prof_pending_) {
    (void)hipEventDestroy(p.a);
    (void)hipEventDestroy(p.b);
  }
  for (hipEvent_t e : ev_pool_) (void)hipEventDestroy(e);
  if (done_recorded_) (void)hipEventSynchronize(ev_done_);
  if (ev_null_) (void)hipEventDestroy(ev_null_);
  if (ev_done_) (void)hipEventDestroy(ev_done_);
  if (ev_upload_) (void)hipEventDestroy(ev_upload_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

// ---- staging: every segment of a source goes to consecutive elements of one
// device buffer.  fp32 and bf16 segments that already have the target type
// are copied as they are; others are converted on the device (convert.hip)
// from a temporary copy of their bytes, which is released once the
// conversion has run.
DevBuf Engine::put_f32(const Src& s, int64_t n, const char* what) {
  if (s.empty()) fail(std::string("model: missing ") + what);
  if (s.numel() != n) fail(std::string("model: wrong size of ") + what);
  DevBuf d;
  d.alloc(static_cast<size_t>(n) * 4);
  int64_t off = 0;
  for (const Seg& g : s.segs) {
    float* dst = d.as<float>() + off;
    if (g.type == SRC_F32) {
      hip_check(hipMemcpy(dst, g.p, static_cast<size_t>(g.n) * 4, hipMemcpyHostToDevice), what);
    } else if (g.type == SRC_BF16 || g.type == SRC_F16) {
      DevBuf tmp;
      tmp.alloc(static_cast<size_t>(g.n) * 2);
      hip_check(hipMemcpy(tmp.get(), g.p, static_cast<size_t>(g.n) * 2, hipMemcpyHostToDevice), what);
      launch_widen_f32(tmp.get(), g.type, dst, g.n, stream_);
      hip_check(hipStreamSynchronize(stream_), what);
    } else {
      fail(std::string("model: ") + what + " cannot be stored as e4m3 codes");
    }
    off += g.n;
  }
  return d;
}

DevBuf Engine::put_f32_opt(const Src& s, int64_t n, const char* what) {
  return s.empty() ? DevBuf() : put_f32(s, n, what);
}

DevBuf Engine::put_act(const Src& s, int64_t n, const char* what) {
  if (act_dt_ == DT_F32) return put_f32(s, n, what);
  if (s.empty()) fail(std::string("model: missing ") + what);
  if (s.numel() != n) fail(std::string("model: wrong size of ") + what);
  DevBuf d;
  d.alloc(static_cast<size_t>(n) * 2);
  int64_t off = 0;
  for (const Seg& g : s.segs) {
    uint16_t* dst = d.as<uint16_t>() + off;
    if (g.type == SRC_BF16) {
      hip_check(hipMemcpy(dst, g.p, static_cast<size_t>(g.n) * 2, hipMemcpyHostToDevice), what);
    } else if (g.type == SRC_F32 || g.type == SRC_F16) {
      const size_t es = g.type == SRC_F32 ? 4 : 2;
      DevBuf tmp;
      tmp.alloc(static_cast<size_t>(g.n) * es);
      hip_check(hipMemcpy(tmp.get(), g.p, static_cast<size_t>(g.n) * es, hipMemcpyHostToDevice), what);
      launch_narrow_bf16(tmp.get(), g.type, dst, g.n, stream_);
      hip_check(hipStreamSynchronize(stream_), what);
    } else {
      fail(std::string("model: ") + what + " holds e4m3 codes; load it with SJH_PREC_FP8W");
    }
    off += g.n;
  }
  return d;
}

Engine::Fp8Dev Engine::put_fp8(const Mat& m, int64_t rows, int64_t cols, const char* what) {
  if (m.w.empty()) fail(std::string("model: missing ") + what);
  if (m.w.numel() != rows * cols) fail(std::string("model: wrong size of ") + what);
  Fp8Dev d;
  d.q.alloc(static_cast<size_t>(rows * cols));
  d.scale.alloc(static_cast<size_t>(rows) * 4);
  bool codes = true, values = true;
  for (const Seg& g : m.w.segs) (g.type == SRC_F8 ? values : codes) = false;
  if (codes) {  // stored e4m3 rows and their scales: copied as they are
    if (m.scale.numel() != rows) fail(std::string("model: ") + what + " needs one scale per row");
    int64_t off = 0;
    for (const Seg& g : m.w.segs) {
      hip_check(hipMemcpy(d.q.as<uint8_t>() + off, g.p, static_cast<size_t>(g.n), hipMemcpyHostToDevice), what);
      off += g.n;
    }
    off = 0;
    for (const Seg& g : m.scale.segs) {
      if (g.type != SRC_F32) fail(std::string("model: scales of ") + what + " must be fp32");
      hip_check(hipMemcpy(d.scale.as<float>() + off, g.p, static_cast<size_t>(g.n) * 4, hipMemcpyHostToDevice), what);
      off += g.n;
    }
  } else if (values) {  // quantized here, with the host quantizer's arithmetic
    DevBuf w = put_f32(m.w, rows * cols, what);
    launch_quantize_fp8_rows(w.as<float>(), rows, cols, d.q.as<uint8_t>(), d.scale.as<float>(), stream_);
    hip_check(hipStreamSynchronize(stream_), what);
  } else {
    fail(std::string("model: ") + what + " mixes e4m3 codes and other types");
  }
  return d;
}

void Engine::stage_weights(const ModelSource& s) {
  const int64_t D = D_, F = F_;
  const bool bert = arch_ == ARCH_BERT;
  emb_w_ = put_act(s.emb_w, static_cast<int64_t>(V_) * D, "emb_w");
  emb_norm_ = put_f32(s.emb_norm, D, "emb_norm");
  final_norm_ = put_f32(s.final_norm, D, "final_norm");
  if (bert) {
    pos_emb_ = put_f32(s.pos_emb, static_cast<int64_t>(max_pos_) * D, "position embedding");
    emb_norm_b_ = put_f32(s.emb_norm_b, D, "emb_norm bias");
    final_norm_b_ = put_f32(s.final_norm_b, D, "final_norm bias");
  } else {
    const int64_t nt = static_cast<int64_t>(max_pos_) * (Dh_ / 2);
    std::vector<float> c, sn;
    auto table = [&](const float* hc, const float* hs, double theta, DevBuf& dc, DevBuf& ds,
                     const char* what) {
      if (hc && hs) {
        dc = put_f32(Src::host_f32(hc, nt), nt, what);
        ds = put_f32(Src::host_f32(hs, nt), nt, what);
      } else {
        rope_table(theta, max_pos_, Dh_, c, sn);
        dc = put_f32(Src::host_f32(c.data(), nt), nt, what);
        ds = put_f32(Src::host_f32(sn.data(), nt), nt, what);
      }
    };
    table(s.rope_cos_full, s.rope_sin_full, s.theta_full, rope_cos_full_, rope_sin_full_,
          "rope tables (full)");
    table(s.rope_cos_slide, s.rope_sin_slide, s.theta_sliding, rope_cos_slide_, rope_sin_slide_,
          "rope tables (sliding)");
  }

  // ModernBERT: Wi [2F, D] feeds GEGLU; BERT: w1 [F, D] feeds GELU
  const int64_t wi_rows = bert ? F : 2 * F;
  layers_.resize(static_cast<size_t>(nlayers_));
  for (int i = 0; i < nlayers_; ++i) {
    const LayerSrc& s0 = s.layers[static_cast<size_t>(i)];
    LayerDev& L = layers_[static_cast<size_t>(i)];
    L.has_attn_norm = !s0.attn_norm.empty();
    require(!bert || L.has_attn_norm, "model: every BERT layer has an attention norm");
    if (L.has_attn_norm) L.attn_norm = put_f32(s0.attn_norm, D, "attn_norm");
    L.attn_norm_b = put_f32_opt(s0.attn_norm_b, D, "attn_norm bias");
    L.mlp_norm = put_f32(s0.mlp_norm, D, "mlp_norm");
    L.mlp_norm_b = put_f32_opt(s0.mlp_norm_b, D, "mlp_norm bias");
    if (w8_) {  // the four projections as per-row fp8 (src/model.cpp:96-128 shapes)
      Fp8Dev a = put_fp8(s0.wqkv, 3 * D, D, "wqkv"), b = put_fp8(s0.wo, D, D, "wo"),
             c2 = put_fp8(s0.wi, wi_rows, D, "wi"), e = put_fp8(s0.wo2, D, F, "wo2");
      L.wqkv = std::move(a.q), L.wqkv_s = std::move(a.scale);
      L.wo = std::move(b.q), L.wo_s = std::move(b.scale);
      L.wi = std::move(c2.q), L.wi_s = std::move(c2.scale);
      L.wo2 = std::move(e.q), L.wo2_s = std::move(e.scale);
    } else {
      L.wqkv = put_act(s0.wqkv.w, 3 * D * D, "wqkv");
      L.wo = put_act(s0.wo.w, D * D, "wo");
      L.wi = put_act(s0.wi.w, wi_rows * D, "wi");
      L.wo2 = put_act(s0.wo2.w, D * F, "wo2");
    }
    L.wqkv_b = put_f32_opt(s0.wqkv_b, 3 * D, "wqkv bias");
    L.wo_b = put_f32_opt(s0.wo_b, D, "wo bias");
    L.wi_b = put_f32_opt(s0.wi_b, wi_rows, "wi bias");
    L.wo2_b = put_f32_opt(s0.wo2_b, D, "wo2 bias");
    require(s0.window >= 0, "negative attention window");
    require(!bert || (s0.window == 0 && L.attn_norm_b.get() && L.wqkv_b.get() && L.wo_b.get() &&
                      L.mlp_norm_b.get() && L.wi_b.get() && L.wo2_b.get()),
            "model: a BERT-family layer has full attention and a bias on every norm and projection");
    L.window = s0.window;
    L.sliding = s0.sliding;
  }
  attn_split_ = max_len_ >= kAttnSplitMinKeys;
  for (const auto& L : layers_) attn_split_ = attn_split_ && L.window == 0;
  // LayerNorms folded across the residual GEMMs: the consumer constants of
  // attn_norm over Wqkv and of mlp_norm over Wi (the persistent kernel's
  // bf16-activation epilogues, D a multiple of 256 up to 1024, head_dim 64)
  // Switched off: the first GPU run of this path faulted the device, and
  // its cause has not been found (the kernels' global addresses check out
  // on the CPU).  The standalone LayerNorms run instead.
  ln_fold_ = kLnFoldEnabled && act_dt_ == DT_BF16 && !bert && D % kLnBlock == 0 &&
             D / kLnBlock <= kLnMaxBlocks && Dh_ == 64 && F % 128 == 0;
  // The residual GEMMs' epilogues finish the next LayerNorm (GemmArgs::rln_y)
  // on the bf16-weight persistent path, for D a multiple of 256 up to 1024.
  rln_ = rln_ && act_dt_ == DT_BF16 && !w8_ && !bert && D % kLnBlock == 0 && D / kLnBlock <= kLnMaxBlocks;
  if (ln_fold_) {
    for (auto& L : layers_) {
      const int wdt = w8_ ? DT_FP8 : DT_BF16;
      if (L.has_attn_norm) {
        L.ln1_c1.alloc(static_cast<size_t>(3 * D) * 16);
        if (L.attn_norm_b.get()) L.ln1_c2.alloc(static_cast<size_t>(3 * D) * 4);
        launch_ln_fold_consts(L.wqkv.get(), wdt, L.wqkv_s.as<float>(), static_cast<int>(3 * D), static_cast<int>(D),
                              L.attn_norm.as<float>(), L.attn_norm_b.as<float>(), L.ln1_c1.as<uint16_t>(),
                              L.ln1_c2.as<float>(), stream_);
      }
      L.ln2_c1.alloc(static_cast<size_t>(wi_rows) * 16);
      if (L.mlp_norm_b.get()) L.ln2_c2.alloc(static_cast<size_t>(wi_rows) * 4);
      launch_ln_fold_consts(L.wi.get(), wdt, L.wi_s.as<float>(), static_cast<int>(wi_rows), static_cast<int>(D),
                            L.mlp_norm.as<float>(), L.mlp_norm_b.as<float>(), L.ln2_c1.as<uint16_t>(),
                            L.ln2_c2.as<float>(), stream_);
    }
  }

  if (lora_r_ > 0) {
    lora_a_ = put_f32(s.lora_a, static_cast<int64_t>(lora_r_) * D, "lora_a");
    lora_b_ = put_f32(s.lora_b, D * lora_r_, "lora_b");
  }
  type_emb_ = put_f32(s.type_emb, 3 * D, "type_emb");
  const int64_t HF = head_ff_;
  head_.resize(static_cast<size_t>(head_layers_));
  for (int i = 0; i < head_layers_; ++i) {
    const HeadSrc& h = s.head[static_cast<size_t>(i)];
    HeadDev& hd = head_[static_cast<size_t>(i)];
    hd.n1w = put_f32(h.n1w, D, "head n1w");
    hd.n1b = put_f32(h.n1b, D, "head n1b");
    hd.n2w = put_f32(h.n2w, D, "head n2w");
    hd.n2b = put_f32(h.n2b, D, "head n2b");
    hd.in_w = put_act(h.in_w, 3 * D * D, "head in_w");
    hd.in_b = put_f32(h.in_b, 3 * D, "head in_b");
    hd.out_w = put_act(h.out_w, D * D, "head out_w");
    hd.out_b = put_f32(h.out_b, D, "head out_b");
    hd.l1w = put_act(h.l1w, HF * D, "head l1w");
    hd.l1b = put_f32(h.l1b, HF, "head l1b");
    hd.l2w = put_act(h.l2w, D * HF, "head l2w");
    hd.l2b = put_f32(h.l2b, D, "head l2b");
  }
  sc_ln_w_ = put_f32(s.sc_ln_w, D, "scorer ln weight");
  sc_ln_b_ = put_f32_opt(s.sc_ln_b, D, "scorer ln bias");
  sc_w1_ = put_f32(s.sc_w1, D * D, "scorer w1");
  sc_b1_ = put_f32_opt(s.sc_b1, D, "scorer b1");
  sc_w2_ = put_f32(s.sc_w2, D, "scorer w2");
  sc_b2_ = put_f32_opt(s.sc_b2, 1, "scorer b2");
  if (act_head_ == ACT_MLP) {
    act_w1_ = put_f32(s.act_w1, 256 * (D + 4), "act w1");
    act_b1_ = put_f32(s.act_b1, 256, "act b1");
    act_w2_ = put_f32(s.act_w2, static_cast<int64_t>(n_act_) * 256, "act w2");
    act_b2_ = put_f32(s.act_b2, n_act_, "act b2");
  }
}

// ------------------------------------------------------------------ batches --
namespace {
// Longest sequences first: attention workgroups of a long sequence run
// longest, so dispatching them first keeps the tail of the launch short.
void set_order(BatchPlan& p) {
  p.order.resize(static_cast<size_t>(p.B));
  for (int b = 0; b < p.B; ++b) p.order[static_cast<size_t>(b)] = b;
  std::stable_sort(p.order.begin(), p.order.end(), [&](int32_t x, int32_t y) {
    return p.q_len[static_cast<size_t>(x)] > p.q_len[static_cast<size_t>(y)];
  });
}

int round_up(int x, int g) { return (x + g - 1) / g * g; }

// The launch bucket of a batch (see BatchPlan).  Launches are sized for the
// bucket and every kernel stops at the batch's own token count, read from the
// device table, so the results depend on the bucket only through the choice
// of GEMM tiling; graph replay and direct launches share the same plan.
void set_bucket(BatchPlan& p) {
  int bb = 1;
  while (bb < p.B) bb <<= 1;
  p.Bb = bb;
  if (p.T <= 1024) {
    p.Tb = round_up(std::max(p.T, 1), 64);
  } else {
    int lg = 0;
    while ((2 << lg) <= p.T) ++lg;  // 2^lg <= T < 2^(lg+1)
    p.Tb = round_up(p.T, 1 << (lg - 3));
  }
  p.max_qb = p.max_q <= 1024 ? round_up(std::max(p.max_q, 1), 128) : round_up(p.max_q, 1024);
}

// The sequence table (layout in sjh_kernels.hpp) of a plan, on the host.
void fill_seq_table(const BatchPlan& p, const int32_t* qtype, int32_t* t) {
  const int Bb = p.Bb;
  t[0] = p.T;
  t[1] = p.B;
  t[2] = t[3] = 0;
  int32_t* seq_start = t + kSeqHdr;
  for (int b = 0; b < Bb; ++b) {
    const bool real = b < p.B;
    const size_t u = static_cast<size_t>(b);
    seq_start[b] = real ? p.seq_start[u] : p.T;
    seq_start[Bb + b] = real ? p.q_len[u] : 0;
    seq_start[2 * Bb + b] = real ? p.k_len[u] : 0;
    seq_start[3 * Bb + b] = real && qtype ? qtype[b] : 0;
    seq_start[4 * Bb + b] = real ? p.order[u] : b;
  }
  int32_t* meta = t + seq_table_meta(Bb);
  int32_t* qbp = t + seq_table_qbp(Bb);
  int nqb = 0;
  for (int z = 0; z < Bb; ++z) {
    const int b = seq_start[4 * Bb + z];
    meta[4 * z + 0] = seq_start[b];
    meta[4 * z + 1] = seq_start[Bb + b];
    meta[4 * z + 2] = seq_start[2 * Bb + b];
    meta[4 * z + 3] = 0;
    qbp[z] = nqb;
    nqb += (meta[4 * z + 1] + kAttnQ - 1) / kAttnQ;
  }
  qbp[Bb] = nqb;
}
}  // namespace

BatchPlan Engine::plan(const int64_t* ids, const int64_t* mask, int B, int L,
                       int32_t* ids_out) const {
  BatchPlan p;
  p.B = B;
  p.L = L;
  require(L > 0, "sequence length must be positive");
  if (L > max_len_)
    fail("sequence length " + std::to_string(L) + " exceeds max_len " + std::to_string(max_len_));
  p.seq_start.resize(static_cast<size_t>(B));
  p.q_len.resize(static_cast<size_t>(B));
  p.k_len.resize(static_cast<size_t>(B));
  int64_t T = 0;
  for (int b = 0; b < B; ++b) {
    int64_t n = 0;
    for (int i = 0; i < L; ++i) n += mask[static_cast<int64_t>(b) * L + i];
    if (n < 0 || n > L) fail("attention_mask row " + std::to_string(b) + " is not 0/1");
    p.k_len[static_cast<size_t>(b)] = static_cast<int32_t>(n);
    const int rows = pad_rows_ ? L : static_cast<int>(n);
    p.q_len[static_cast<size_t>(b)] = rows;
    p.seq_start[static_cast<size_t>(b)] = static_cast<int32_t>(T);
    T += rows;
  }
  if (T > (int64_t{1} << 30)) fail("batch too large");
  p.T = static_cast<int>(T);
  p.max_q = 0;
  for (int b = 0; b < B; ++b) p.max_q = std::max(p.max_q, p.q_len[static_cast<size_t>(b)]);
  set_order(p);
  set_bucket(p);
  if (ids_out) {
    for (int b = 0; b < B; ++b) {
      const int rows = p.q_len[static_cast<size_t>(b)];
      for (int i = 0; i < rows; ++i) {
        const int64_t id = ids[static_cast<int64_t>(b) * L + i];
        if (id < 0 || id >= V_) fail("token id " + std::to_string(id) + " outside the vocabulary");
        ids_out[p.seq_start[static_cast<size_t>(b)] + i] = static_cast<int32_t>(id);
      }
    }
  }
  return p;
}

BatchPlan Engine::plan_lens(const int32_t* h_lens, int B) const {
  BatchPlan p;
  p.B = B;
  p.seq_start.resize(static_cast<size_t>(B));
  p.q_len.resize(static_cast<size_t>(B));
  p.k_len.resize(static_cast<size_t>(B));
  int64_t T = 0;
  for (int b = 0; b < B; ++b) {
    const int n = h_lens[b];
    if (n < 0 || n > max_len_) fail("sequence length outside [0, max_len]");
    p.seq_start[static_cast<size_t>(b)] = static_cast<int32_t>(T);
    p.q_len[static_cast<size_t>(b)] = n;
    p.k_len[static_cast<size_t>(b)] = n;
    p.max_q = std::max(p.max_q, n);
    T += n;
  }
  if (T > (int64_t{1} << 30)) fail("batch too large");
  p.T = static_cast<int>(T);
  p.L = p.max_q;
  set_order(p);
  set_bucket(p);
  return p;
}

void Engine::ensure_workspace(int Tb, int Bb) {
  if (Tb <= cap_T_ && Bb <= cap_B_) return;
  // every earlier call's work (on any stream) has finished with the old buffers
  if (done_recorded_) hip_check(hipEventSynchronize(ev_done_), "sync before workspace growth");
  const int nT = std::max(Tb, cap_T_ + cap_T_ / 4);
  const int nB = std::max(Bb, cap_B_);
  const size_t t = static_cast<size_t>(std::max(nT, 1));
  const size_t D = D_, as = dt_size(act_dt_);
  ids_.ensure(t * 4);
  tok_pos_.ensure(t * 4);
  tok_seq_.ensure(t * 4);
  seqinfo_.ensure(seq_table_ints(std::max(nB, 1)) * 4);
  const int n_items = attn_item_slots(nT, nB, H_, attn_split_);
  attn_items_.ensure(attn_items_ints(n_items) * 4);
  const int n_pairs = attn_split_ ? attn_split_pairs(nT, nB, H_) : 0;
  if (n_pairs > 0) attn_part_.ensure(static_cast<size_t>(n_pairs) * 2 * kAttnPartFloats * 4);
  // moments of every 256-row tile the persistent kernel reads, one tile past the last
  if (ln_fold_) ln_stats_.ensure(((t + 255) / 256 * 256 + 256) * static_cast<size_t>(D / kLnBlock) * 8);
  if (rln_) {
    // the sync ints start at zero and every launch leaves them at zero
    rln_mom_.ensure(t * static_cast<size_t>(D / kLnBlock) * 16);
    const size_t sync_bytes = (t + 255) / 256 * kRlnSyncInts * 4;
    rln_sync_.ensure(sync_bytes);
    hip_check(hipMemsetAsync(rln_sync_.get(), 0, rln_sync_.bytes(), stream_), "clear LayerNorm sync ints");
    hip_check(hipStreamSynchronize(stream_), "clear LayerNorm sync ints");
  }
  X_.ensure(t * D * 4);
  Y_.ensure(t * D * as);
  QKV_.ensure(t * 3 * D * as);
  O_.ensure(t * D * as);
  const size_t hff = head_layers_ > 0 ? static_cast<size_t>(head_ff_) : 0;
  G_.ensure(t * std::max<size_t>(F_, hff) * as);
  if (lora_r_ > 0) Z_.ensure(t * static_cast<size_t>(lora_r_) * 4);
  {  // up to 16 K splits of a 256-row batch over the widest weight matrix
    const size_t nw = std::max<size_t>({3 * D, 2 * static_cast<size_t>(F_), hff});
    splitk_.ensure(16 * std::min<size_t>(t, 256) * nw * 4);
  }
  cap_T_ = nT;
  cap_B_ = nB;
  ws_.seq = seqinfo_.as<int32_t>();
  ws_.tok_pos = tok_pos_.as<int>();
  ws_.tok_seq = tok_seq_.as<int>();
  ws_.Y = Y_.get();
  ws_.QKV = QKV_.get();
  ws_.O = O_.get();
  ws_.G = G_.get();
  ws_.Z = Z_.as<float>();
  ws_.partial = splitk_.as<float>();
  ws_.partial_cap = static_cast<int64_t>(splitk_.bytes() / 4);
  ws_.attn_items = attn_items_.as<int32_t>();
  ws_.attn_slots_cap = n_items;
  ws_.attn_part = n_pairs > 0 ? attn_part_.as<float>() : nullptr;
  ws_.attn_pairs_cap = n_pairs;
  ws_.ln_stats = ln_fold_ ? ln_stats_.as<float>() : nullptr;
  ws_.rln_mom = rln_ ? rln_mom_.as<float>() : nullptr;
  ws_.rln_sync = rln_ ? rln_sync_.as<int>() : nullptr;
  ++ws_gen_;
  for (auto& kv : graphs_) drop_graph(kv.second);  // every launch ended (above)
  graphs_.clear();
}

void Engine::upload_batch(const BatchPlan& p, const int32_t* h_ids, const int32_t* h_qtype,
                          hipStream_t st) {
  // pinned staging: the sequence table, then the token ids.  The previous
  // copy out of the buffer (possibly on another stream) must be done first.
  const size_t nsi = seq_table_ints(p.Bb);
  if (upload_recorded_) hip_check(hipEventSynchronize(ev_upload_), "staging buffer reuse");
  h_stage_.ensure((nsi + (h_ids ? p.T : 0)) * 4);
  int32_t* s = h_stage_.as<int32_t>();
  fill_seq_table(p, h_qtype, s);
  hip_check(hipMemcpyAsync(seqinfo_.get(), s, nsi * 4, hipMemcpyHostToDevice, st), "upload seqinfo");
  if (h_ids) {
    std::memcpy(s + nsi, h_ids, static_cast<size_t>(p.T) * 4);
    hip_check(hipMemcpyAsync(ids_.get(), s + nsi, static_cast<size_t>(p.T) * 4,
                             hipMemcpyHostToDevice, st),
              "upload ids");
  }
  hip_check(hipEventRecord(ev_upload_, st), "record upload");
  upload_recorded_ = true;
}

void Engine::set_seq_table(const BatchPlan& p, const int32_t* h_lens, int32_t* table,
                           hipStream_t st) {
  if (p.Bb <= kSeqTableMaxB) {
    launch_seq_table(h_lens, p.B, p.Bb, table, st);
  } else {
    require(table == seqinfo_.as<int32_t>(), "sequence table: more than 256 sequences need the workspace");
    upload_batch(p, nullptr, nullptr, st);
  }
}

void Engine::begin_call(hipStream_t st) {
  if (done_recorded_) hip_check(hipStreamWaitEvent(st, ev_done_, 0), "order after the previous call");
}

void Engine::end_call(hipStream_t st) {
  hip_check(hipEventRecord(ev_done_, st), "record call end");
  done_recorded_ = true;
}

// ------------------------------------------------------------------ launches --
void Engine::prof_begin(hipStream_t st) {
  if (!profile_ || quiet_) return;
  hipEvent_t e;
  if (!ev_pool_.empty()) {
    e = ev_pool_.back();
    ev_pool_.pop_back();
  } else {
    hip_check(hipEventCreate(&e), "hipEventCreate");
  }
  hip_check(hipEventRecord(e, st), "hipEventRecord");
  ev_open_ = e;
}

void Engine::prof_end(const char* name, hipStream_t st) {
  if (!profile_ || quiet_) return;
  hipEvent_t e;
  if (!ev_pool_.empty()) {
    e = ev_pool_.back();
    ev_pool_.pop_back();
  } else {
    hip_check(hipEventCreate(&e), "hipEventCreate");
  }
  hip_check(hipEventRecord(e, st), "hipEventRecord");
  prof_pending_.push_back({name, ev_open_, e});
  ev_open_ = nullptr;
}

void Engine::prof_collect() {
  for (auto& p : prof_pending_) {
    hip_check(hipEventSynchronize(p.b), "hipEventSynchronize");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, p.a, p.b), "hipEventElapsedTime");
    auto& t = prof_tot_[p.name];
    std::get<0>(t) = p.name;
    std::get<1>(t) += ms;
    std::get<2>(t) += 1;
    ev_pool_.push_back(p.a);
    ev_pool_.push_back(p.b);
  }
  prof_pending_.clear();
}

void Engine::set_profile(bool on) {
  std::lock_guard<std::mutex> lk(mu_);
  hip_check(hipSetDevice(dev_), "hipSetDevice");
  if (!on) prof_collect();
  profile_ = on;
  if (on) prof_tot_.clear();
}

void Engine::graph_stats(int32_t* cached, int64_t* captures, int64_t* replays) {
  std::lock_guard<std::mutex> lk(mu_);
  if (cached) *cached = static_cast<int32_t>(graphs_.size());
  if (captures) *captures = n_captures_;
  if (replays) *replays = n_replays_;
}

std::vector<std::tuple<const char*, double, int64_t>> Engine::profile_totals() {
  std::lock_guard<std::mutex> lk(mu_);
  hip_check(hipSetDevice(dev_), "hipSetDevice");
  prof_collect();
  std::vector<std::tuple<const char*, double, int64_t>> v;
  for (auto& kv : prof_tot_) v.push_back(kv.second);
  return v;
}

void Engine::gemm(const char* name, const GemmArgs& g0, const Ws& w, hipStream_t st) {
  GemmArgs g = g0;
  g.partial = w.partial;
  g.partial_cap = w.partial_cap;
  prof_begin(st);
  launch_gemm(g, st);
  prof_end(name, st);
}

void Engine::resid_gemm_ln(const char* gname, const GemmArgs& g0, const char* lname, LnArgs a,
                           const Ws& w, hipStream_t st) {
  GemmArgs g = g0;
  g.partial = w.partial;
  g.partial_cap = w.partial_cap;
  // the layer norm that would add the splits: X rows written back in place
  LnArgs folded = a;
  folded.parts = g.partial;
  folded.part_stride = static_cast<int64_t>(g.M) * g.N;
  folded.ld_part = g.N;
  folded.part_bias = g.bias;
  folded.xio = g.X;
  folded.n_parts = 1;
  prof_begin(st);
  const int S = g.M <= 256 && ln_takes_parts(folded) ? launch_gemm_resid_partials(g, st) : 0;
  if (S == 0) launch_gemm(g, st);
  prof_end(gname, st);
  if (S > 0) {  // X is updated by the layer norm: X += sum of the splits (+ bias)
    folded.n_parts = S;
    a = folded;
  }
  ln(lname, a, st);
}

bool Engine::rln_resid(GemmArgs& g, const LnArgs& a, const Ws& w) const {
  // a plain LayerNorm of X's rows into bf16 Y (the attn_norm and mlp_norm
  // steps), on a launch whose tiles all run at once
  if (!rln_ || !w.rln_mom || !w.rln_sync || !a.normalize || !a.w || a.in != g.X || a.ld_in != g.ldx ||
      a.in_dtype != DT_F32 || a.y_dtype != DT_BF16 || !a.y_out || a.x_out || a.xio || a.resid || a.ids ||
      a.add || a.M != g.M || a.D != g.N)
    return false;
  if (!gemm_takes_rln(g)) return false;
  g.rln_y = a.y_out;
  g.rln_ldy = a.ld_y;
  g.rln_w = a.w;
  g.rln_b = a.b;
  g.rln_eps = a.eps;
  g.rln_mom = w.rln_mom;
  g.rln_sync = w.rln_sync;
  g.rln_spin = rln_spin_;
  return true;
}

void Engine::ln(const char* name, const LnArgs& a, hipStream_t st) {
  prof_begin(st);
  launch_ln(a, st);
  prof_end(name, st);
}

void Engine::attn(const char* name, const AttnArgs& a, hipStream_t st) {
  prof_begin(st);
  launch_attn(a, st);
  prof_end(name, st);
}

// ------------------------------------------------------------------ encoder --
// Launch sizes come from the plan's bucket (Tb rows, Bb table entries, max_qb
// queries); every kernel reads the real token count from the table's header.
void Engine::enqueue_encoder(const BatchPlan& p, const Ws& w, const int32_t* d_ids, float* X,
                             hipStream_t st) {
  const int T = p.Tb, D = D_, F = F_, Bb = p.Bb;
  const int32_t* si = w.seq;
  const int* T_dev = si;  // header[0]
  const int32_t* seq_start = si + kSeqHdr;
  const int32_t* q_len = seq_start + Bb;
  const int32_t* k_len = seq_start + 2 * Bb;
  const int adt = act_dt_;
  void* Y = w.Y;
  void* QKV = w.QKV;
  void* O = w.O;
  void* G = w.G;

  launch_token_index(seq_start, q_len, Bb, w.tok_pos, w.tok_seq, st);
  // the attention work list of the batch, when the bf16 head_dim-64 kernel runs
  // (the list holds a query block's index in 16 bits); the shortest
  // sequences' items split by keys when the batch may hold such (launch_attn_items)
  const bool attn_list = adt == DT_BF16 && Dh_ == 64 && w.attn_items && p.max_qb <= 65536 * kAttnQ;
  const bool attn_split = attn_list && w.attn_part && p.max_qb >= kAttnSplitMinKeys;
  const int attn_slots = attn_list ? attn_item_slots(T, Bb, H_, attn_split) : 0;
  const int attn_pairs = attn_split ? attn_split_pairs(T, Bb, H_) : 0;
  if (attn_list) {
    require(attn_slots <= w.attn_slots_cap && attn_pairs <= w.attn_pairs_cap,
            "attention work list: workspace too small");
    launch_attn_items(si, Bb, H_, attn_slots, attn_split, w.attn_items, st);
  }
  // short batches: attention folds the output projection in (AttnArgs::wo),
  // each head's partial product going to the split-K workspace, and the
  // LayerNorm that reads X next adds the H partials (LnArgs::parts), so no
  // Wo launch runs
  const bool attn_wo = attn_wo_ && attn_list && !attn_split && !w8_ && T <= 256 && D == 64 * H_ &&
                       D % kAttnWoCols == 0 && D <= 1024 && w.partial &&
                       static_cast<int64_t>(H_) * T * D <= w.partial_cap;

  // src/model.cpp:332-340: X = LN(emb[ids]); layer 0 reads X itself.  BERT
  // family (src/sj_model.cpp:220-237): X = LN(word[ids] + pos[position] ; w, b)
  const bool bert = arch_ == ARCH_BERT;
  {
    LnArgs e;
    e.in = emb_w_.get();
    e.in_dtype = adt;
    e.ld_in = D;
    e.ids = d_ids;
    e.w = emb_norm_.as<float>();
    e.b = emb_norm_b_.as<float>();
    if (bert) {
      e.add = pos_emb_.as<float>();
      e.add_ids = w.tok_pos;
      e.add_rows = max_pos_;
      e.ld_add = D;
    }
    e.eps = eps_;
    e.x_out = X;
    e.ld_x = D;
    if (!layers_[0].has_attn_norm) {
      e.y_out = Y;
      e.y_dtype = adt;
      e.ld_y = D;
    }
    e.M = T;
    e.M_dev = T_dev;
    e.D = D;
    ln("emb_ln", e, st);
  }

  const float scale = 1.0f / std::sqrt(static_cast<float>(Dh_));
  // bf16 with head_dim 64: the QKV projection writes q * scale * log2(e), so
  // attention's QK^T product yields log2-domain logits (no per-logit scaling
  // in its softmax); the rounding to bf16 then applies to the scaled q
  const bool q_pre = !bert && adt == DT_BF16 && Dh_ == 64;
  // Y = attn_norm(X) of layer li (src/model.cpp:347-353; identity copy when
  // the layer has none)
  auto attn_norm_args = [&](int li) {
    const LayerDev& ly = layers_[static_cast<size_t>(li)];
    LnArgs a;
    a.in = X;
    a.in_dtype = DT_F32;
    a.ld_in = D;
    a.normalize = ly.has_attn_norm;
    a.w = ly.has_attn_norm ? ly.attn_norm.as<float>() : nullptr;
    a.b = ly.attn_norm_b.as<float>();
    a.eps = eps_;
    a.y_out = Y;
    a.y_dtype = adt;
    a.ld_y = D;
    a.M = T;
    a.M_dev = T_dev;
    a.D = D;
    return a;
  };
  // final norm, in place (src/model.cpp:400)
  LnArgs final_args;
  final_args.in = X;
  final_args.in_dtype = DT_F32;
  final_args.ld_in = D;
  final_args.w = final_norm_.as<float>();
  final_args.b = final_norm_b_.as<float>();
  final_args.eps = eps_;
  final_args.x_out = X;
  final_args.ld_x = D;
  final_args.M = T;
  final_args.M_dev = T_dev;
  final_args.D = D;
  // LayerNorms folded across the residual GEMMs (GemmArgs::ln_y): on the
  // persistent kernel's batches the Wo and Wo2 epilogues write the next
  // LayerNorm's bf16 input rows (centred on each 256-column block's mean,
  // times the norm weight) and the row moments, and the QKV and Wi products
  // that read them finish the normalisation in their epilogues: no LayerNorm
  // launch between the residual GEMMs.  The probe arguments stand for every
  // layer (same shapes, 256-byte aligned buffers).
  bool fold = false;
  if (ln_fold_ && w.ln_stats) {
    GemmArgs q;
    q.A = Y, q.lda = D, q.W = layers_[0].wqkv.get(), q.ldw = D, q.M = T, q.N = 3 * D, q.K = D;
    if (w8_) q.w_dtype = DT_FP8, q.w_scale = layers_[0].wqkv_s.as<float>();
    q.epi = EPI_ROPE, q.out = QKV, q.ldo = 3 * D, q.head_dim = Dh_, q.rope_dim = D, q.rope_rows = max_pos_;
    q.rope_cos = rope_cos_full_.as<float>(), q.rope_sin = rope_sin_full_.as<float>();
    GemmArgs o = q;
    o.A = O, o.W = layers_[0].wo.get(), o.w_scale = layers_[0].wo_s.as<float>(), o.N = D, o.epi = EPI_RESID;
    o.out = nullptr, o.ldo = 0, o.X = X, o.ldx = D;
    GemmArgs i2 = q;
    i2.W = layers_[0].wi.get(), i2.w_scale = layers_[0].wi_s.as<float>(), i2.N = F, i2.epi = EPI_GEGLU, i2.out = G,
    i2.ldo = F;
    GemmArgs o2 = o;
    o2.A = G, o2.lda = F, o2.W = layers_[0].wo2.get(), o2.w_scale = layers_[0].wo2_s.as<float>(), o2.ldw = F,
    o2.K = F;
    fold = gemm_takes_ln_fold(q) && gemm_takes_ln_fold(o) && gemm_takes_ln_fold(i2) && gemm_takes_ln_fold(o2);
  }
  for (int li = 0; li < nlayers_; ++li) {
    const LayerDev& ly = layers_[static_cast<size_t>(li)];
    // layers after the first get their attn_norm from the previous layer's
    // Wo2 step (resid_gemm_ln, or folded)
    if (li == 0 && ly.has_attn_norm) ln("attn_norm", attn_norm_args(0), st);
    // this layer's QKV product reads the previous Wo2's folded rows
    const bool fold_in = fold && li > 0 && ly.has_attn_norm;
    {  // qkv = Y . Wqkv^T with RoPE on q, k (src/model.cpp:355-365); BERT:
       // q|k|v rows with their biases, no RoPE (src/sj_model.cpp:44-52)
      GemmArgs g;
      g.A = Y;
      g.lda = D;
      g.W = ly.wqkv.get();
      if (w8_) g.w_dtype = DT_FP8, g.w_scale = ly.wqkv_s.as<float>();
      g.ldw = D;
      g.M = T;
      g.M_dev = T_dev;
      g.N = 3 * D;
      g.K = D;
      g.in_dtype = adt;
      g.out = QKV;
      g.ldo = 3 * D;
      g.out_dtype = adt;
      if (bert) {
        g.epi = EPI_STORE;
        g.bias = ly.wqkv_b.as<float>();
        gemm("gemm_qkv_bias", g, w, st);
      } else {
        g.epi = EPI_ROPE;
        g.pos = w.tok_pos;
        g.rope_cos = (ly.sliding ? rope_cos_slide_ : rope_cos_full_).as<float>();
        g.rope_sin = (ly.sliding ? rope_sin_slide_ : rope_sin_full_).as<float>();
        g.rope_rows = max_pos_;
        g.rope_dim = D;
        g.head_dim = Dh_;
        if (q_pre) g.q_scale = scale * 1.4426950408889634f;
        if (fold_in) {
          g.ln_stats_in = w.ln_stats;
          g.ln_c1 = ly.ln1_c1.as<uint16_t>();
          g.ln_c2 = ly.ln1_c2.as<float>();
          g.ln_eps = eps_;
        }
        gemm("gemm_qkv_rope", g, w, st);
      }
    }
    {  // attention (src/model.cpp:381)
      AttnArgs a;
      a.q = QKV;
      a.k = off<char>(QKV, D, adt);
      a.v = off<char>(QKV, 2 * D, adt);
      a.ld_q = a.ld_k = a.ld_v = 3 * D;
      a.o = O;
      a.ld_o = D;
      a.dtype = adt;
      a.seq_start = seq_start;
      a.q_len = q_len;
      a.k_len = k_len;
      a.seq_order = seq_start + 4 * Bb;
      a.seq_meta = si + seq_table_meta(Bb);
      a.B = Bb;
      a.H = H_;
      a.Dh = Dh_;
      a.max_q = p.max_qb;
      a.window = ly.window;
      a.scale = scale;
      a.q_log2_scaled = q_pre;
      if (attn_list) {
        a.items = w.attn_items;
        a.n_slots = attn_slots;
        if (attn_split) a.part = w.attn_part;
      }
      if (attn_wo) {
        a.wo = ly.wo.get();
        a.ld_wo = D;
        a.wo_n = D;
        a.wo_part = w.partial;
        a.wo_part_stride = static_cast<int64_t>(T) * D;
        a.wo_ld_part = D;
      }
      prof_begin(st);
      launch_attn(a, st);
      if (attn_split) launch_attn_merge(si, Bb, H_, attn_pairs, w.attn_part, O, D, st);
      prof_end(attn_wo ? "attention_wo" : "attention", st);
    }
    {  // X += O . Wo^T (src/model.cpp:389-391)
      GemmArgs g;
      g.A = O;
      g.lda = D;
      g.W = ly.wo.get();
      if (w8_) g.w_dtype = DT_FP8, g.w_scale = ly.wo_s.as<float>();
      g.ldw = D;
      g.M = T;
      g.M_dev = T_dev;
      g.N = D;
      g.K = D;
      g.in_dtype = adt;
      g.epi = EPI_RESID;
      g.X = X;
      g.ldx = D;
      g.bias = ly.wo_b.as<float>();
      // Y = mlp_norm(X) (src/model.cpp:392)
      LnArgs a;
      a.in = X;
      a.in_dtype = DT_F32;
      a.ld_in = D;
      a.w = ly.mlp_norm.as<float>();
      a.b = ly.mlp_norm_b.as<float>();
      a.eps = eps_;
      a.y_out = Y;
      a.y_dtype = adt;
      a.ld_y = D;
      a.M = T;
      a.M_dev = T_dev;
      a.D = D;
      if (attn_wo) {  // attention wrote the heads' partials of O . Wo^T
        LnArgs f = a;
        f.parts = w.partial;
        f.n_parts = H_;
        f.part_stride = static_cast<int64_t>(T) * D;
        f.ld_part = D;
        f.part_bias = g.bias;
        f.xio = X;
        require(ln_takes_parts(f), "the layer norm after the folded output projection takes no partials");
        ln("mlp_norm", f, st);
      } else if (fold) {
        g.ln_y = Y;
        g.ln_w = ly.mlp_norm.as<float>();
        g.ln_stats_out = w.ln_stats;
        gemm("gemm_wo_resid", g, w, st);
      } else if (rln_resid(g, a, w)) {
        gemm("gemm_wo_resid_ln", g, w, st);
      } else {
        resid_gemm_ln("gemm_wo_resid", g, "mlp_norm", a, w, st);
      }
    }
    {  // G = geglu(Y . Wi^T) (src/model.cpp:394); BERT: G = gelu(Y . W1^T + b1)
       // (src/sj_model.cpp:249)
      GemmArgs g;
      g.A = Y;
      g.lda = D;
      g.W = ly.wi.get();
      if (w8_) g.w_dtype = DT_FP8, g.w_scale = ly.wi_s.as<float>();
      g.ldw = D;
      g.M = T;
      g.M_dev = T_dev;
      g.N = F;
      g.K = D;
      g.in_dtype = adt;
      g.out = G;
      g.ldo = F;
      g.out_dtype = adt;
      if (bert) {
        g.epi = EPI_STORE;
        g.bias = ly.wi_b.as<float>();
        g.act = 1;
        gemm("gemm_w1_gelu", g, w, st);
      } else {
        g.epi = EPI_GEGLU;
        if (fold) {
          g.ln_stats_in = w.ln_stats;
          g.ln_c1 = ly.ln2_c1.as<uint16_t>();
          g.ln_c2 = ly.ln2_c2.as<float>();
          g.ln_eps = eps_;
        }
        gemm("gemm_wi_geglu", g, w, st);
      }
    }
    {  // X += G . Wo2^T (src/model.cpp:395-397)
      GemmArgs g;
      g.A = G;
      g.lda = F;
      g.W = ly.wo2.get();
      if (w8_) g.w_dtype = DT_FP8, g.w_scale = ly.wo2_s.as<float>();
      g.ldw = F;
      g.M = T;
      g.M_dev = T_dev;
      g.N = D;
      g.K = F;
      g.in_dtype = adt;
      g.epi = EPI_RESID;
      g.X = X;
      g.ldx = D;
      g.bias = ly.wo2_b.as<float>();
      // then the next layer's attn_norm (folded into its QKV product), or
      // the final norm
      if (li + 1 < nlayers_ && fold && layers_[static_cast<size_t>(li + 1)].has_attn_norm) {
        g.ln_y = Y;
        g.ln_w = layers_[static_cast<size_t>(li + 1)].attn_norm.as<float>();
        g.ln_stats_out = w.ln_stats;
        gemm("gemm_wo2_resid", g, w, st);
      } else if (li + 1 < nlayers_) {
        const LnArgs a = attn_norm_args(li + 1);
        if (rln_resid(g, a, w))
          gemm("gemm_wo2_resid_ln", g, w, st);
        else
          resid_gemm_ln("gemm_wo2_resid", g, "attn_norm", a, w, st);
      } else {
        resid_gemm_ln("gemm_wo2_resid", g, "final_norm", final_args, w, st);
      }
    }
  }
  if (lora_r_ > 0) {  // h += (h . A^T) . B^T (src/model.cpp:402-407)
    GemmArgs g;
    g.A = X;
    g.lda = D;
    g.W = lora_a_.get();
    g.ldw = D;
    g.M = T;
    g.M_dev = T_dev;
    g.N = lora_r_;
    g.K = D;
    g.in_dtype = DT_F32;
    g.epi = EPI_STORE;
    g.out = w.Z;
    g.ldo = lora_r_;
    g.out_dtype = DT_F32;
    gemm("gemm_lora_a", g, w, st);
    GemmArgs g2;
    g2.A = w.Z;
    g2.lda = lora_r_;
    g2.W = lora_b_.get();
    g2.ldw = lora_r_;
    g2.M = T;
    g2.M_dev = T_dev;
    g2.N = D;
    g2.K = lora_r_;
    g2.in_dtype = DT_F32;
    g2.epi = EPI_RESID;
    g2.X = X;
    g2.ldx = D;
    gemm("gemm_lora_b", g2, w, st);
  }
}

// src/model.cpp:409-459: type embedding, then N pre-norm TransformerEncoderLayers
// (ReLU FFN of width 4D, norms eps 1e-5).  BERT family, src/sj_model.cpp:291-321:
// the same layer with a GELU FFN of width head_intermediate and eps norm_eps.
void Engine::enqueue_head_layers(const BatchPlan& p, const Ws& w, float* X, hipStream_t st) {
  const int T = p.Tb, D = D_, Bb = p.Bb;
  const int32_t* si = w.seq;
  const int* T_dev = si;
  const int32_t* seq_start = si + kSeqHdr;
  const int adt = act_dt_;
  launch_add_row_embedding(X, D, type_emb_.as<float>(), seq_start + 3 * Bb, w.tok_seq, T, T_dev,
                           D, st);
  const float scale = 1.0f / std::sqrt(static_cast<float>(Dh_));
  for (const HeadDev& hd : head_) {
    LnArgs a;
    a.in = X;
    a.in_dtype = DT_F32;
    a.ld_in = D;
    a.w = hd.n1w.as<float>();
    a.b = hd.n1b.as<float>();
    a.eps = head_eps_;
    a.y_out = w.Y;
    a.y_dtype = adt;
    a.ld_y = D;
    a.M = T;
    a.M_dev = T_dev;
    a.D = D;
    ln("head_norm1", a, st);

    GemmArgs g;
    g.A = w.Y;
    g.lda = D;
    g.W = hd.in_w.get();
    g.ldw = D;
    g.M = T;
    g.M_dev = T_dev;
    g.N = 3 * D;
    g.K = D;
    g.in_dtype = adt;
    g.epi = EPI_STORE;
    g.out = w.QKV;
    g.ldo = 3 * D;
    g.out_dtype = adt;
    g.bias = hd.in_b.as<float>();
    gemm("head_in_proj", g, w, st);

    AttnArgs at;
    at.q = w.QKV;
    at.k = off<char>(w.QKV, D, adt);
    at.v = off<char>(w.QKV, 2 * D, adt);
    at.ld_q = at.ld_k = at.ld_v = 3 * D;
    at.o = w.O;
    at.ld_o = D;
    at.dtype = adt;
    at.seq_start = seq_start;
    at.q_len = seq_start + Bb;
    at.k_len = seq_start + 2 * Bb;
    at.seq_order = seq_start + 4 * Bb;
    at.seq_meta = si + seq_table_meta(Bb);
    at.B = Bb;
    at.H = H_;
    at.Dh = Dh_;
    at.max_q = p.max_qb;
    at.window = 0;
    at.scale = scale;
    attn("head_attention", at, st);

    GemmArgs go;
    go.A = w.O;
    go.lda = D;
    go.W = hd.out_w.get();
    go.ldw = D;
    go.M = T;
    go.M_dev = T_dev;
    go.N = D;
    go.K = D;
    go.in_dtype = adt;
    go.epi = EPI_RESID;
    go.X = X;
    go.ldx = D;
    go.bias = hd.out_b.as<float>();
    gemm("head_out_proj", go, w, st);

    LnArgs a2 = a;
    a2.w = hd.n2w.as<float>();
    a2.b = hd.n2b.as<float>();
    ln("head_norm2", a2, st);

    GemmArgs g1;
    g1.A = w.Y;
    g1.lda = D;
    g1.W = hd.l1w.get();
    g1.ldw = D;
    g1.M = T;
    g1.M_dev = T_dev;
    g1.N = head_ff_;
    g1.K = D;
    g1.in_dtype = adt;
    g1.epi = EPI_STORE;
    g1.out = w.G;
    g1.ldo = head_ff_;
    g1.out_dtype = adt;
    g1.bias = hd.l1b.as<float>();
    g1.act = head_act_;
    gemm("head_linear1", g1, w, st);

    GemmArgs g2;
    g2.A = w.G;
    g2.lda = head_ff_;
    g2.W = hd.l2w.get();
    g2.ldw = head_ff_;
    g2.M = T;
    g2.M_dev = T_dev;
    g2.N = D;
    g2.K = head_ff_;
    g2.in_dtype = adt;
    g2.epi = EPI_RESID;
    g2.X = X;
    g2.ldx = D;
    g2.bias = hd.l2b.as<float>();
    gemm("head_linear2", g2, w, st);
  }
}

void Engine::run_device(const BatchPlan& p, const Ws& w, const int32_t* d_ids, float* X,
                        bool head, hipStream_t st) {
  enqueue_encoder(p, w, d_ids, X, st);
  if (head) enqueue_head_layers(p, w, X, st);
}

void Engine::run_device_maybe_graph(const BatchPlan& p, const int32_t* d_ids, float* X,
                                    bool head, hipStream_t st) {
  if (!use_graphs_ || profile_) {
    run_device(p, ws_, d_ids, X, head, st);
    return;
  }
  // one graph per bucket and buffer set: the batch's own sizes and lengths
  // reach the kernels through the sequence table, written before the launch
  const std::vector<int64_t> key = {p.Bb,
                                    p.Tb,
                                    p.max_qb,
                                    head ? 1 : 0,
                                    static_cast<int64_t>(ws_gen_),
                                    reinterpret_cast<int64_t>(d_ids),
                                    reinterpret_cast<int64_t>(X),
                                    reinterpret_cast<int64_t>(st)};
  auto it = graphs_.find(key);
  if (it == graphs_.end()) {
    if (graphs_.size() >= kMaxGraphs) {  // evict the least recently used graph
      auto lru = graphs_.begin();
      for (auto jt = graphs_.begin(); jt != graphs_.end(); ++jt)
        if (jt->second.last_use < lru->second.last_use) lru = jt;
      // its last launch may still be queued (calls return before their work
      // ends): the executable graph is destroyed only after that launch
      if (lru->second.done) hip_check(hipEventSynchronize(lru->second.done), "wait for an evicted graph");
      drop_graph(lru->second);
      graphs_.erase(lru);
    }
    hipGraph_t graph = nullptr;
    hip_check(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "begin capture");
    try {
      run_device(p, ws_, d_ids, X, head, st);
    } catch (...) {
      (void)hipStreamEndCapture(st, &graph);
      if (graph) (void)hipGraphDestroy(graph);
      throw;
    }
    hip_check(hipStreamEndCapture(st, &graph), "end capture");
    Graph g;
    hipError_t e = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    hip_check(e, "graph instantiate");
    e = hipEventCreateWithFlags(&g.done, hipEventDisableTiming);
    if (e != hipSuccess) {
      drop_graph(g);
      hip_check(e, "graph event");
    }
    it = graphs_.emplace(key, g).first;
    ++n_captures_;
  } else {
    ++n_replays_;
  }
  it->second.last_use = ++graph_clock_;
  hip_check(hipGraphLaunch(it->second.exec, st), "graph launch");
  hip_check(hipEventRecord(it->second.done, st), "record graph launch");
}

void Engine::drop_graph(Graph& g) {
  if (g.exec) (void)hipGraphExecDestroy(g.exec);
  if (g.done) (void)hipEventDestroy(g.done);
  g.exec = nullptr;
  g.done = nullptr;
}

// ------------------------------------------------------------------ entries --
void Engine::encode(const int64_t* ids, const int64_t* mask, int B, int L, float* hidden) {
  std::lock_guard<std::mutex> lk(mu_);
  hip_check(hipSetDevice(dev_), "hipSetDevice");
  if (B <= 0) return;
  require(ids && mask && hidden, "encode: null argument");
  std::vector<int32_t> packed;
  BatchPlan p0 = plan(ids, mask, B, L, nullptr);
  packed.resize(static_cast<size_t>(p0.T));
  BatchPlan p = plan(ids, mask, B, L, packed.data());
  ensure_workspace(p.Tb, p.Bb);
  const size_t D = D_;
  hipStream_t st = stream_;
  begin_call(st);
  if (p.T > 0) {
    upload_batch(p, packed.data(), nullptr, st);
    run_device_maybe_graph(p, ids_.as<int32_t>(), X_.as<float>(), false, st);
  }
  if (pad_rows_) {
    if (p.T > 0)
      hip_check(hipMemcpyAsync(hidden, X_.get(), static_cast<size_t>(p.T) * D * 4,
                               hipMemcpyDeviceToHost, st),
                "download hidden");
    end_call(st);
    hip_check(hipStreamSynchronize(st), "encode");
  } else {
    h_out_.ensure(std::max<size_t>(static_cast<size_t>(p.T) * D * 4, 4));
    if (p.T > 0)
      hip_check(hipMemcpyAsync(h_out_.as<float>(), X_.get(), static_cast<size_t>(p.T) * D * 4,
                               hipMemcpyDeviceToHost, st),
                "download hidden");
    end_call(st);
    hip_check(hipStreamSynchronize(st), "encode");
    std::memset(hidden, 0, static_cast<size_t>(B) * L * D * 4);
    const float* src = h_out_.as<float>();
    for (int b = 0; b < B; ++b)
      std::memcpy(hidden + static_cast<size_t>(b) * L * D,
                  src + static_cast<size_t>(p.seq_start[static_cast<size_t>(b)]) * D,
                  static_cast<size_t>(p.q_len[static_cast<size_t>(b)]) * D * 4);
  }
  if (profile_) prof_collect();
}

void Engine::encode_device(const int32_t* d_ids, const int32_t* h_lens, int B, float* d_hidden,
                           hipStream_t stream) {
  std::lock_guard<std::mutex> lk(mu_);
  hip_check(hipSetDevice(dev_), "hipSetDevice");
  if (B <= 0) return;
  require(d_ids && h_lens && d_hidden, "encode_device: null argument");
  // NULL selects the model's own stream, ordered after and before the legacy
  // null stream so that NULL behaves like the default stream for the caller.
  hipStream_t st = stream ? stream : stream_;
  BatchPlan p = plan_lens(h_lens, B);
  if (p.T == 0) return;
  ensure_workspace(p.Tb, p.Bb);
  begin_call(st);
  if (!stream) {
    hip_check(hipEventRecord(ev_null_, nullptr), "record null stream");
    hip_check(hipStreamWaitEvent(st, ev_null_, 0), "wait null stream");
  }
  set_seq_table(p, h_lens, ws_.seq, st);
  run_device_maybe_graph(p, d_ids, d_hidden, false, st);
  end_call(st);
  if (!stream) {
    hip_check(hipEventRecord(ev_null_, st), "record model stream");
    hip_check(hipStreamWaitEvent(nullptr, ev_null_, 0), "null stream waits");
  }
}

size_t Engine::scratch_layout(const BatchPlan& p, Ws& ws) const {
  // the regions of ensure_workspace, for the plan's bucket, 256-byte aligned;
  // split-K partials (residual GEMMs of at most 256 rows: up to 16 slices of
  // [Tb, D]) only where the bucket takes that path
  const size_t t = static_cast<size_t>(p.Tb), D = D_, as = dt_size(act_dt_);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += align256(bytes);
    return o;
  };
  const size_t seq = take(seq_table_ints(p.Bb) * 4);
  const size_t tok_pos = take(t * 4), tok_seq = take(t * 4);
  const size_t Y = take(t * D * as), QKV = take(t * 3 * D * as), O = take(t * D * as);
  const size_t G = take(t * static_cast<size_t>(F_) * as);
  const size_t Z = lora_r_ > 0 ? take(t * static_cast<size_t>(lora_r_) * 4) : 0;
  const size_t part_floats = p.Tb <= 256 ? 16 * t * D : 0;
  const size_t part = take(part_floats * 4);
  const int n_items = attn_item_slots(p.Tb, p.Bb, H_);
  const size_t items = take(static_cast<size_t>(n_items) * 16);
  ws = Ws();
  if (off > kScratchBytes) return off;
  ws.seq = reinterpret_cast<int32_t*>(scratch_ + seq);
  ws.tok_pos = reinterpret_cast<int*>(scratch_ + tok_pos);
  ws.tok_seq = reinterpret_cast<int*>(scratch_ + tok_seq);
  ws.Y = scratch_ + Y;
  ws.QKV = scratch_ + QKV;
  ws.O = scratch_ + O;
  ws.G = scratch_ + G;
  ws.Z = lora_r_ > 0 ? reinterpret_cast<float*>(scratch_ + Z) : nullptr;
  ws.partial = part_floats ? reinterpret_cast<float*>(scratch_ + part) : nullptr;
  ws.partial_cap = static_cast<int64_t>(part_floats);
  ws.attn_items = reinterpret_cast<int32_t*>(scratch_ + items);
  ws.attn_slots_cap = n_items;
  return off;
}

void Engine::encode_device_noalloc(const int32_t* d_ids, const int32_t* h_lens, int B,
                                   float* d_hidden, hipStream_t stream) {
  std::lock_guard<std::mutex> lk(mu_);
  hip_check(hipSetDevice(dev_), "hipSetDevice");
  if (B <= 0) return;
  require(d_ids && h_lens && d_hidden, "encode_device_noalloc: null argument");
  if (B > kSeqTableMaxB)
    fail_arg("encode_device_noalloc: at most " + std::to_string(kSeqTableMaxB) + " sequences per call");
  BatchPlan p = plan_lens(h_lens, B);
  if (p.T == 0) return;
  Ws w;
  const size_t need = scratch_layout(p, w);
  if (!w.seq) {
    const size_t D = D_, as = dt_size(act_dt_);
    const size_t per_tok = 8 + (5 * D + static_cast<size_t>(F_)) * as + static_cast<size_t>(lora_r_) * 4;
    fail_arg("encode_device_noalloc: this batch (" + std::to_string(p.T) + " tokens, launched as " +
         std::to_string(p.Tb) + ") needs " + std::to_string(need) +
         " bytes of scratch; the fixed scratch array holds " + std::to_string(kScratchBytes) +
         " bytes, about " + std::to_string(kScratchBytes / per_tok) + " tokens of this model");
  }
  hipStream_t st = stream ? stream : stream_;
  begin_call(st);
  if (!stream) {
    hip_check(hipEventRecord(ev_null_, nullptr), "record null stream");
    hip_check(hipStreamWaitEvent(st, ev_null_, 0), "wait null stream");
  }
  quiet_ = true;
  try {
    launch_seq_table(h_lens, p.B, p.Bb, w.seq, st);
    run_device(p, w, d_ids, d_hidden, false, st);
  } catch (...) {
    quiet_ = false;
    throw;
  }
  quiet_ = false;
  end_call(st);
  if (!stream) {
    hip_check(hipEventRecord(ev_null_, st), "record model stream");
    hip_check(hipStreamWaitEvent(nullptr, ev_null_, 0), "null stream waits");
  }
}

void Engine::forward(const int64_t* ids, const int64_t* mask, const int64_t* marker_pos,
                     const uint8_t* marker_mask, const int64_t* qtype, int B, int L, int K,
                     float* logits, float* act) {
  std::lock_guard<std::mutex> lk(mu_);
  hip_check(hipSetDevice(dev_), "hipSetDevice");
  if (B <= 0) return;
  require(ids && mask && marker_pos && marker_mask && qtype && logits && act,
          "forward: null argument");
  require(K > 0, "forward: need at least one marker column");
  BatchPlan p0 = plan(ids, mask, B, L, nullptr);
  std::vector<int32_t> packed(static_cast<size_t>(p0.T));
  BatchPlan p = plan(ids, mask, B, L, packed.data());
  std::vector<int32_t> qt(static_cast<size_t>(B));
  for (int b = 0; b < B; ++b) {
    if (qtype[b] < 0 || qtype[b] > 2) fail("qtype must be 0, 1 or 2");
    qt[static_cast<size_t>(b)] = static_cast<int32_t>(qtype[b]);
  }
  ensure_workspace(p.Tb, p.Bb);
  hipStream_t st = stream_;
  begin_call(st);
  if (p.T > 0) {
    upload_batch(p, packed.data(), qt.data(), st);
    run_device_maybe_graph(p, ids_.as<int32_t>(), X_.as<float>(), true, st);
  }
  decision_tail(p, X_.as<float>(), marker_pos, marker_mask, L, K, logits, act, st);
  end_call(st);
  hip_check(hipStreamSynchronize(st), "forward: decision head");
  if (profile_) prof_collect();
}

void Engine::forward_shared(const int64_t* ids, const int64_t* mask, int U, int L,
                            const int32_t* row_seq, const int64_t* marker_pos,
                            const uint8_t* marker_mask, const int64_t* qtype, int B, int K,
                            float* logits, float* act) {
  std::lock_guard<std::mutex> lk(mu_);
  hip_check(hipSetDevice(dev_), "hipSetDevice");
  if (B <= 0) return;
  require(U > 0, "forward_shared: need at least one sequence");
  require(ids && mask && row_seq && marker_pos && marker_mask && qtype && logits && act,
          "forward_shared: null argument");
  require(K > 0, "forward_shared: need at least one marker column");
  // the U sequences, encoded once
  BatchPlan p0 = plan(ids, mask, U, L, nullptr);
  std::vector<int32_t> packed(static_cast<size_t>(p0.T));
  BatchPlan pu = plan(ids, mask, U, L, packed.data());
  // The head's input for row b is sequence row_seq[b]'s hidden states plus
  // the type embedding of qtype[b] (src/model.cpp:409-459); the markers enter
  // only in the tail.  Rows that share (sequence, qtype) are therefore
  // identical through the head layers, which run once per distinct pair: pe
  // holds the pairs, pt the B rows, each pointing at its pair's rows.
  BatchPlan pe, pt;
  pe.L = pt.L = L;
  pt.B = B;
  pt.seq_start.resize(static_cast<size_t>(B));
  pt.q_len.resize(static_cast<size_t>(B));
  std::vector<int32_t> qt, pair_seq;
  std::vector<int32_t> pair_of(static_cast<size_t>(U) * 3, -1);
  int64_t T = 0;
  for (int b = 0; b < B; ++b) {
    const int u = row_seq[b];
    if (u < 0 || u >= U) fail("forward_shared: row_seq outside [0, U)");
    if (qtype[b] < 0 || qtype[b] > 2) fail("qtype must be 0, 1 or 2");
    int32_t& j = pair_of[static_cast<size_t>(u) * 3 + static_cast<size_t>(qtype[b])];
    if (j < 0) {
      j = static_cast<int32_t>(qt.size());
      qt.push_back(static_cast<int32_t>(qtype[b]));
      pair_seq.push_back(u);
      const int n = pu.q_len[static_cast<size_t>(u)];
      pe.seq_start.push_back(static_cast<int32_t>(T));
      pe.q_len.push_back(n);
      pe.k_len.push_back(pu.k_len[static_cast<size_t>(u)]);
      pe.max_q = std::max(pe.max_q, n);
      T += n;
    }
    pt.seq_start[static_cast<size_t>(b)] = pe.seq_start[static_cast<size_t>(j)];
    pt.q_len[static_cast<size_t>(b)] = pe.q_len[static_cast<size_t>(j)];
  }
  if (T > (int64_t{1} << 30)) fail("batch too large");
  pe.B = static_cast<int>(qt.size());
  pe.T = static_cast<int>(T);
  set_order(pe);
  set_bucket(pe);
  // the source row of every head token
  std::vector<int32_t> src(static_cast<size_t>(pe.T));
  for (int j = 0; j < pe.B; ++j) {
    const int u = pair_seq[static_cast<size_t>(j)];
    for (int i = 0; i < pe.q_len[static_cast<size_t>(j)]; ++i)
      src[static_cast<size_t>(pe.seq_start[static_cast<size_t>(j)] + i)] =
          pu.seq_start[static_cast<size_t>(u)] + i;
  }
  ensure_workspace(std::max(pu.Tb, pe.Tb), std::max(pu.Bb, pe.Bb));
  const size_t D = D_;
  X2_.ensure(std::max<size_t>(static_cast<size_t>(pe.Tb) * D * 4, 4));
  expand_idx_.ensure(std::max<size_t>(src.size() * 4, 4));
  hipStream_t st = stream_;
  begin_call(st);
  if (pu.T > 0) {
    upload_batch(pu, packed.data(), nullptr, st);
    run_device_maybe_graph(pu, ids_.as<int32_t>(), X_.as<float>(), false, st);
  }
  if (pe.T > 0) {
    // after the encoder (same stream): the pairs' table, their hidden states
    // gathered from the encoded sequences, then the head layers
    upload_batch(pe, nullptr, qt.data(), st);
    hip_check(hipMemcpyAsync(expand_idx_.get(), src.data(), src.size() * 4, hipMemcpyHostToDevice, st),
              "upload expanded rows");
    launch_gather_rows(X_.as<float>(), D_, expand_idx_.as<int32_t>(), pe.T, D_, X2_.as<float>(), D_,
                       st);
    launch_token_index(ws_.seq + kSeqHdr, ws_.seq + kSeqHdr + pe.Bb, pe.Bb, ws_.tok_pos, ws_.tok_seq,
                       st);
    enqueue_head_layers(pe, ws_, X2_.as<float>(), st);
  }
  decision_tail(pt, X2_.as<float>(), marker_pos, marker_mask, L, K, logits, act, st);
  end_call(st);
  hip_check(hipStreamSynchronize(st), "forward_shared: decision head");
  if (profile_) prof_collect();
}

void Engine::decision_tail(const BatchPlan& p, const float* X, const int64_t* marker_pos,
                           const uint8_t* marker_mask, int L, int K, float* logits, float* act,
                           hipStream_t st) {
  const int B = p.B, D = D_;
  // ---- scorer (src/model.cpp:461-487) and act head (:489-535), all on the
  // device: gather the marker rows and the [CLS] rows, then only the logits
  // and the act probabilities come back
  const int nmk = B * K, nrow = nmk + B;
  // row indices, then the marker mask; a member, so that it outlives the
  // copy below until the caller synchronizes
  std::vector<int32_t>& idx = tail_hidx_;
  idx.assign(static_cast<size_t>(nrow + nmk), 0);
  for (int b = 0; b < B; ++b) {
    for (int k = 0; k < K; ++k) {
      int64_t pp = marker_pos[static_cast<int64_t>(b) * K + k];
      if (pp < 0) pp = 0;
      if (pp >= L) pp = L - 1;
      idx[static_cast<size_t>(b) * K + k] =
          pp < p.q_len[static_cast<size_t>(b)] ? p.seq_start[static_cast<size_t>(b)] +
                                                     static_cast<int32_t>(pp)
                                               : -1;
    }
    idx[static_cast<size_t>(nmk + b)] =
        p.q_len[static_cast<size_t>(b)] > 0 ? p.seq_start[static_cast<size_t>(b)] : -1;
  }
  for (int i = 0; i < nmk; ++i) idx[static_cast<size_t>(nrow + i)] = marker_mask[i] ? 1 : 0;
  tail_idx_.ensure(idx.size() * 4);
  tail_rows_.ensure(static_cast<size_t>(nrow) * D * 4);
  tail_s0_.ensure(static_cast<size_t>(nmk) * D * 4);
  tail_s1_.ensure(static_cast<size_t>(nmk) * D * 4);
  tail_s2_.ensure(static_cast<size_t>(nmk) * 4);
  tail_lg_.ensure(static_cast<size_t>(nmk) * 4);
  tail_ain_.ensure(static_cast<size_t>(B) * (D + 4) * 4);
  tail_ah_.ensure(static_cast<size_t>(B) * 256 * 4);
  tail_ao_.ensure(static_cast<size_t>(B) * n_act_ * 4);
  tail_act_.ensure(static_cast<size_t>(B) * n_act_ * 4);
  hip_check(hipMemcpyAsync(tail_idx_.get(), idx.data(), idx.size() * 4, hipMemcpyHostToDevice, st),
            "upload marker rows");
  launch_gather_rows(X, D, tail_idx_.as<int32_t>(), nrow, D, tail_rows_.as<float>(),
                     D, st);
  {
    LnArgs a;
    a.in = tail_rows_.get();
    a.in_dtype = DT_F32;
    a.ld_in = D;
    a.w = sc_ln_w_.as<float>();
    a.b = sc_ln_b_.as<float>();
    a.eps = eps_;
    a.x_out = tail_s0_.as<float>();
    a.ld_x = D;
    a.M = nmk;
    a.D = D;
    ln("scorer_norm", a, st);
    GemmArgs g;
    g.A = tail_s0_.get();
    g.lda = D;
    g.W = sc_w1_.get();
    g.ldw = D;
    g.M = nmk;
    g.N = D;
    g.K = D;
    g.in_dtype = DT_F32;
    g.epi = EPI_STORE;
    g.out = tail_s1_.get();
    g.ldo = D;
    g.out_dtype = DT_F32;
    g.bias = sc_b1_.as<float>();
    g.act = 1;
    gemm("scorer_linear1", g, ws_, st);
    GemmArgs g2 = g;
    g2.A = tail_s1_.get();
    g2.W = sc_w2_.get();
    g2.N = 1;
    g2.out = tail_s2_.get();
    g2.ldo = 1;
    g2.bias = sc_b2_.as<float>();
    g2.act = 0;
    gemm("scorer_linear2", g2, ws_, st);
  }
  if (act_head_ == ACT_TOP1) {
    launch_act_top1(tail_s2_.as<float>(), tail_idx_.as<int32_t>() + nrow, B, K, tail_lg_.as<float>(),
                    tail_act_.as<float>(), st);
  } else {
  launch_act_features(tail_s2_.as<float>(), tail_idx_.as<int32_t>() + nrow, B, K,
                      tail_rows_.as<float>() + static_cast<size_t>(nmk) * D, D, D,
                      tail_lg_.as<float>(), tail_ain_.as<float>(), D + 4, st);
  {
    GemmArgs g;
    g.A = tail_ain_.get();
    g.lda = D + 4;
    g.W = act_w1_.get();
    g.ldw = D + 4;
    g.M = B;
    g.N = 256;
    g.K = D + 4;
    g.in_dtype = DT_F32;
    g.epi = EPI_STORE;
    g.out = tail_ah_.get();
    g.ldo = 256;
    g.out_dtype = DT_F32;
    g.bias = act_b1_.as<float>();
    g.act = 1;
    gemm("act_linear1", g, ws_, st);
    GemmArgs g2 = g;
    g2.A = tail_ah_.get();
    g2.lda = 256;
    g2.W = act_w2_.get();
    g2.ldw = 256;
    g2.N = n_act_;
    g2.K = 256;
    g2.out = tail_ao_.get();
    g2.ldo = n_act_;
    g2.bias = act_b2_.as<float>();
    g2.act = 0;
    gemm("act_linear2", g2, ws_, st);
  }
  launch_act_softmax(tail_ao_.as<float>(), B, n_act_, tail_act_.as<float>(), st);
  }
  hip_check(hipMemcpyAsync(logits, tail_lg_.get(), static_cast<size_t>(nmk) * 4, hipMemcpyDeviceToHost, st),
            "download logits");
  hip_check(hipMemcpyAsync(act, tail_act_.get(), static_cast<size_t>(B) * n_act_ * 4,
                           hipMemcpyDeviceToHost, st),
            "download act");
}

}  // namespace sjh

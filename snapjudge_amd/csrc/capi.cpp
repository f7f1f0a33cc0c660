// capi.cpp -- extern "C" surface of libsnapjudge_hip.so (include/snapjudge_hip.h).
//
// Exceptions never cross the boundary: each entry point catches, stores the
// message in a thread-local slot readable through sjh_last_error(), and
// returns a negative status, the convention of the reference's engine ABI
// (include/snapjudge/capi.h).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <memory>
#include <new>
#include <stdexcept>
#include <string>

#include "ckpt.hpp"
#include "engine.hpp"
#include "sjh_host.hpp"
#include "sjh_kernels.hpp"
#include "snapjudge_hip.h"

struct sjh_model {
  sjh::Engine* eng;
};

namespace {

thread_local std::string g_last_error;

template <typename Fn>
int guarded(Fn&& fn) {
  try {
    fn();
    return SJH_OK;
  } catch (const std::bad_alloc&) {
    g_last_error = "snapjudge HIP: host allocation failed";
    return SJH_E_OOM;
  } catch (const sjh::ArgError& e) {
    g_last_error = e.what();
    return SJH_E_INVALID;
  } catch (const std::runtime_error& e) {
    g_last_error = e.what();
    const std::string s = e.what();
    if (s.find("out of device memory") != std::string::npos) return SJH_E_OOM;
    if (s.find("hip") != std::string::npos || s.find("device") != std::string::npos ||
        s.find("launch") != std::string::npos)
      return SJH_E_DEVICE;
    return SJH_E_INVALID;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return SJH_E_INVALID;
  }
}

hipStream_t as_stream(sjh_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

size_t esize(int32_t dt) { return dt == SJH_BF16 ? 2 : 4; }

void check_dtype(int32_t dt) {
  if (dt != SJH_F32 && dt != SJH_BF16) sjh::fail("dtype must be SJH_F32 or SJH_BF16");
}

}  // namespace

extern "C" {

const char* sjh_last_error(void) { return g_last_error.c_str(); }

int sjh_version(void) { return 1; }

void sjh_default_options(sjh_options* opt) {
  if (!opt) return;
  opt->precision = SJH_PREC_BF16;
  opt->max_len = 0;
  opt->use_graphs = 1;
  opt->pad_rows = 0;
  opt->device = 0;
  opt->fuse_ln = 1;
  opt->fuse_attn_wo = 1;
}

int sjh_model_create(const sjh_model_desc* desc, const sjh_options* opt, sjh_model** out) {
  return guarded([&] {
    if (!desc || !out) sjh::fail("sjh_model_create: null argument");
    *out = nullptr;
    sjh_options o;
    sjh_default_options(&o);
    if (opt) o = *opt;
    auto* m = new sjh_model{nullptr};
    try {
      m->eng = new sjh::Engine(sjh::source_from_desc(*desc), o);
    } catch (...) {
      delete m;
      throw;
    }
    *out = m;
  });
}

int sjh_model_load(const char* dir, const sjh_options* opt, sjh_model** out) {
  return guarded([&] {
    if (!dir || !out) sjh::fail_arg("sjh_model_load: null argument");
    *out = nullptr;
    sjh_options o;
    sjh_default_options(&o);
    if (opt) o = *opt;
    // the mapping stays open until every tensor is on the device
    std::unique_ptr<sjh::Checkpoint> ck = sjh::read_checkpoint(dir);
    auto* m = new sjh_model{nullptr};
    try {
      m->eng = new sjh::Engine(ck->src, o);
    } catch (...) {
      delete m;
      throw;
    }
    *out = m;
  });
}

void sjh_model_destroy(sjh_model* m) {
  if (!m) return;
  delete m->eng;
  delete m;
}

int sjh_model_encode(sjh_model* m, const int64_t* ids, const int64_t* mask, int32_t B, int32_t L,
                     float* hidden) {
  return guarded([&] {
    if (!m) sjh::fail("null model");
    if (B < 0) sjh::fail("negative batch");
    m->eng->encode(ids, mask, B, L, hidden);
  });
}

int sjh_model_forward(sjh_model* m, const int64_t* ids, const int64_t* mask,
                      const int64_t* marker_pos, const uint8_t* marker_mask, const int64_t* qtype,
                      int32_t B, int32_t L, int32_t K, float* logits, float* act) {
  return guarded([&] {
    if (!m) sjh::fail("null model");
    if (B < 0) sjh::fail("negative batch");
    m->eng->forward(ids, mask, marker_pos, marker_mask, qtype, B, L, K, logits, act);
  });
}

int sjh_model_forward_shared(sjh_model* m, const int64_t* ids, const int64_t* mask, int32_t U,
                             int32_t L, const int32_t* row_seq, const int64_t* marker_pos,
                             const uint8_t* marker_mask, const int64_t* qtype, int32_t B,
                             int32_t K, float* logits, float* act) {
  return guarded([&] {
    if (!m) sjh::fail("null model");
    if (B < 0 || U < 0) sjh::fail("negative batch");
    m->eng->forward_shared(ids, mask, U, L, row_seq, marker_pos, marker_mask, qtype, B, K, logits,
                           act);
  });
}

int sjh_model_encode_device(sjh_model* m, const int32_t* d_ids, const int32_t* h_lens, int32_t B,
                            float* d_hidden, sjh_stream_t stream) {
  return guarded([&] {
    if (!m) sjh::fail("null model");
    if (B < 0) sjh::fail("negative batch");
    m->eng->encode_device(d_ids, h_lens, B, d_hidden, as_stream(stream));
  });
}

int sjh_model_encode_device_noalloc(sjh_model* m, const int32_t* d_ids, const int32_t* h_lens,
                                    int32_t B, float* d_hidden, sjh_stream_t stream) {
  return guarded([&] {
    if (!m) sjh::fail("null model");
    if (B < 0) sjh::fail("negative batch");
    m->eng->encode_device_noalloc(d_ids, h_lens, B, d_hidden, as_stream(stream));
  });
}

int sjh_model_info(const sjh_model* m, int32_t* D, int32_t* H, int32_t* n_act,
                   int32_t* precision) {
  return guarded([&] {
    if (!m) sjh::fail("null model");
    if (D) *D = m->eng->D();
    if (H) *H = m->eng->H();
    if (n_act) *n_act = m->eng->n_act();
    if (precision) *precision = m->eng->precision();
  });
}

int sjh_model_graph_stats(const sjh_model* m, int32_t* cached, int64_t* captures,
                          int64_t* replays) {
  return guarded([&] {
    if (!m) sjh::fail("null model");
    m->eng->graph_stats(cached, captures, replays);
  });
}

int sjh_model_profile(sjh_model* m, int32_t enable) {
  return guarded([&] {
    if (!m) sjh::fail("null model");
    m->eng->set_profile(enable != 0);
  });
}

int sjh_model_profile_read(sjh_model* m, int32_t max_entries, const char** names,
                           double* total_ms, int64_t* launches, int32_t* n_entries) {
  return guarded([&] {
    if (!m || !n_entries) sjh::fail("null argument");
    auto v = m->eng->profile_totals();
    int n = 0;
    for (auto& t : v) {
      if (n >= max_entries) break;
      if (names) names[n] = std::get<0>(t);
      if (total_ms) total_ms[n] = std::get<1>(t);
      if (launches) launches[n] = std::get<2>(t);
      ++n;
    }
    *n_entries = n;
  });
}

// ---------------------------------------------------------------- kernels --
int sjh_gemm(const void* A, const void* W, const float* bias, void* C, int32_t M, int32_t N,
             int32_t K, int32_t act, int32_t dtype, sjh_stream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    if (act < 0 || act > 2) sjh::fail("act must be 0, 1 or 2");
    sjh::GemmArgs g;
    g.A = A;
    g.lda = K;
    g.W = W;
    g.ldw = K;
    g.M = M;
    g.N = N;
    g.K = K;
    g.in_dtype = dtype;
    g.epi = sjh::EPI_STORE;
    g.out = C;
    g.ldo = N;
    g.out_dtype = dtype;
    g.bias = bias;
    g.act = act;
    sjh::launch_gemm(g, as_stream(stream));
  });
}

int sjh_quantize_fp8(const float* w, int64_t rows, int64_t cols, uint8_t* q, float* scale) {
  return guarded([&] {
    if (rows < 0 || cols < 0) sjh::fail("quantize_fp8: negative shape");
    if (rows > 0 && cols > 0 && (!w || !q || !scale)) sjh::fail("quantize_fp8: null argument");
    sjh::quantize_fp8_rows(w, static_cast<size_t>(rows), static_cast<size_t>(cols), q, scale);
  });
}

int sjh_gemm_fp8w(const void* A, const uint8_t* Wq, const float* w_scale, const float* bias,
                  void* C, int32_t M, int32_t N, int32_t K, int32_t act, sjh_stream_t stream) {
  return guarded([&] {
    if (act < 0 || act > 2) sjh::fail("act must be 0, 1 or 2");
    sjh::GemmArgs g;
    g.A = A;
    g.lda = K;
    g.W = Wq;
    g.ldw = K;
    g.M = M;
    g.N = N;
    g.K = K;
    g.in_dtype = SJH_BF16;
    g.w_dtype = sjh::DT_FP8;
    g.w_scale = w_scale;
    g.epi = sjh::EPI_STORE;
    g.out = C;
    g.ldo = N;
    g.out_dtype = SJH_BF16;
    g.bias = bias;
    g.act = act;
    sjh::launch_gemm(g, as_stream(stream));
  });
}

int sjh_gemm_geglu(const void* A, const void* Wi, void* C, int32_t M, int32_t F, int32_t K,
                   int32_t dtype, sjh_stream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    sjh::GemmArgs g;
    g.A = A;
    g.lda = K;
    g.W = Wi;
    g.ldw = K;
    g.M = M;
    g.N = F;
    g.K = K;
    g.in_dtype = dtype;
    g.epi = sjh::EPI_GEGLU;
    g.out = C;
    g.ldo = F;
    g.out_dtype = dtype;
    sjh::launch_gemm(g, as_stream(stream));
  });
}

int sjh_gemm_residual(const void* A, const void* W, float* X, int32_t M, int32_t D, int32_t K,
                      int32_t dtype, sjh_stream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    sjh::GemmArgs g;
    g.A = A;
    g.lda = K;
    g.W = W;
    g.ldw = K;
    g.M = M;
    g.N = D;
    g.K = K;
    g.in_dtype = dtype;
    g.epi = sjh::EPI_RESID;
    g.X = X;
    g.ldx = D;
    sjh::launch_gemm(g, as_stream(stream));
  });
}

int sjh_gemm_qkv_rope(const void* A, const void* Wqkv, void* qkv, const int32_t* pos,
                      const float* cos_t, const float* sin_t, int32_t max_pos, int32_t M,
                      int32_t H, int32_t Dh, int32_t K, int32_t dtype, sjh_stream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    if (H <= 0 || Dh <= 0 || Dh % 2 != 0) sjh::fail("gemm_qkv_rope: bad head shape");
    if (!pos || !cos_t || !sin_t) sjh::fail("gemm_qkv_rope: null positions or tables");
    if (max_pos <= 0) sjh::fail("gemm_qkv_rope: max_pos must be positive");
    sjh::GemmArgs g;
    g.A = A;
    g.lda = K;
    g.W = Wqkv;
    g.ldw = K;
    g.M = M;
    g.N = 3 * H * Dh;
    g.K = K;
    g.in_dtype = dtype;
    g.epi = sjh::EPI_ROPE;
    g.out = qkv;
    g.ldo = 3 * H * Dh;
    g.out_dtype = dtype;
    g.pos = pos;
    g.rope_cos = cos_t;
    g.rope_sin = sin_t;
    g.rope_rows = max_pos;
    g.rope_dim = H * Dh;
    g.head_dim = Dh;
    sjh::launch_gemm(g, as_stream(stream));
  });
}

int sjh_add_ln(float* X, const void* R, const float* W, const float* B, void* Y, int32_t M,
               int32_t D, float eps, int32_t residual, int32_t bias, int32_t dtype,
               sjh_stream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    sjh::LnArgs a;
    a.in = X;
    a.in_dtype = sjh::DT_F32;
    a.ld_in = D;
    if (residual) {
      if (!R) sjh::fail("add_ln: residual requested without R");
      a.resid = R;
      a.resid_dtype = dtype;
      a.xio = X;
    }
    a.w = W;
    a.b = bias ? B : nullptr;
    a.eps = eps;
    a.y_out = Y;
    a.y_dtype = dtype;
    a.ld_y = D;
    a.M = M;
    a.D = D;
    sjh::launch_ln(a, as_stream(stream));
  });
}

int sjh_rope(void* qkv, const float* cos_t, const float* sin_t, int64_t M, int32_t L, int32_t H,
             int32_t Dh, int32_t dtype, sjh_stream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    if (L <= 0) sjh::fail("rope: L must be positive");
    sjh::launch_rope(qkv, dtype, M, static_cast<int64_t>(3) * H * Dh, nullptr, L, H, Dh, cos_t,
                     sin_t, as_stream(stream));
  });
}

int sjh_attn(const void* qkv, const int32_t* lens, void* O, int32_t B, int32_t L, int32_t H,
             int32_t Dh, int32_t window, int32_t dtype, sjh_stream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    if (L <= 0 || H <= 0 || Dh <= 0) sjh::fail("attn: bad shape");
    const size_t es = esize(dtype);
    const int64_t HD = static_cast<int64_t>(H) * Dh;
    sjh::AttnArgs a;
    a.q = qkv;
    a.k = static_cast<const char*>(qkv) + HD * es;
    a.v = static_cast<const char*>(qkv) + 2 * HD * es;
    a.ld_q = a.ld_k = a.ld_v = 3 * HD;
    a.o = O;
    a.ld_o = HD;
    a.dtype = dtype;
    a.k_len = lens;
    a.uniform_L = L;
    a.B = B;
    a.H = H;
    a.Dh = Dh;
    a.max_q = L;
    a.window = window;
    a.scale = 1.0f / std::sqrt(static_cast<float>(Dh));
    sjh::launch_attn(a, as_stream(stream));
  });
}

int sjh_attn_log2(const void* qkv, const int32_t* lens, void* O, int32_t B, int32_t L, int32_t H,
                  int32_t window, sjh_stream_t stream) {
  return guarded([&] {
    if (L <= 0 || H <= 0) sjh::fail("attn_log2: bad shape");
    const int64_t HD = static_cast<int64_t>(H) * 64;
    sjh::AttnArgs a;
    a.q = qkv;
    a.k = static_cast<const char*>(qkv) + HD * 2;
    a.v = static_cast<const char*>(qkv) + 2 * HD * 2;
    a.ld_q = a.ld_k = a.ld_v = 3 * HD;
    a.o = O;
    a.ld_o = HD;
    a.dtype = sjh::DT_BF16;
    a.k_len = lens;
    a.uniform_L = L;
    a.B = B;
    a.H = H;
    a.Dh = 64;
    a.max_q = L;
    a.window = window;
    a.scale = 0.125f;
    a.q_log2_scaled = true;
    sjh::launch_attn(a, as_stream(stream));
  });
}

int sjh_embed_ln(const void* table, const int32_t* ids, const float* w, float* X, int32_t M,
                 int32_t D, float eps, int32_t dtype, sjh_stream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    sjh::LnArgs a;
    a.in = table;
    a.in_dtype = dtype;
    a.ld_in = D;
    a.ids = ids;
    a.w = w;
    a.eps = eps;
    a.x_out = X;
    a.ld_x = D;
    a.M = M;
    a.D = D;
    sjh::launch_ln(a, as_stream(stream));
  });
}

}  // extern "C"

// attn.hip -- non-causal varlen flash attention for gfx950.
//
// Fast path (bf16, head_dim 64): one workgroup = (sequence, head, 128
// queries); 4 waves own 32 queries each.  Key/value tiles of 64 rows are
// staged in LDS (K row-major, V transposed to [dim][key]).  Per tile a wave
// computes S^T = K . Q^T with v_mfma_f32_32x32x16_bf16 (the query is the MFMA
// column, so each lane owns one query and 32 of the tile's keys), does the
// online-softmax update in registers (row max over its own values plus one
// cross-half exchange; exp2 with the 1/sqrt(Dh)*log2(e) scale folded in), and
// accumulates O^T += V^T . P^T.  The accumulator of S^T is already laid out
// as the B operand of the second MFMA once the key order inside a 16-key
// step is taken as the MFMA's k order, so P never leaves registers.
//
// Generic path (fp32 or bf16, head_dim 8/16/32/64/128): one thread per query,
// K/V tiles of 32 keys in LDS (broadcast reads), blocked online softmax with
// expf.  It serves the fp32 parity mode.
//
// Masking follows src/tensor.cpp:186-192: query i sees keys
// [0, k_len) (full) or [max(0, i-w), min(k_len, i+w+1)) (window w).  A query
// with no visible key yields zeros, as the reference does for len = 0.
#include "sjh_common.hpp"
#include "sjh_host.hpp"
#include "sjh_kernels.hpp"

namespace sjh {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kQ = 128;   // queries per workgroup
constexpr int kKey = 64;  // keys per tile
constexpr int kLdK = 64 + 8;  // padded K row (elements): 144 B
constexpr int kLdV = 64 + 8;  // padded V^T row (elements)

__device__ __forceinline__ float wave_max32(float v) {
  // lanes l and l^32 hold the two halves of one query's keys
  return fmaxf(v, __shfl_xor(v, 32, 64));
}

__global__ __launch_bounds__(256) void attn_bf16_mfma_kernel(AttnArgs a) {
  const int b = blockIdx.z, h = blockIdx.y;
  const int qlen = a.q_len ? a.q_len[b] : a.uniform_L;
  const int q0 = blockIdx.x * kQ;
  if (q0 >= qlen) return;
  // keys never extend past the rows a sequence owns (a caller's k_len > L in
  // the padded layout is clamped rather than read out of bounds)
  const int klen = a.seq_start ? a.k_len[b] : max(0, min(a.k_len[b], a.uniform_L));
  const int64_t row0 = a.seq_start ? a.seq_start[b] : static_cast<int64_t>(b) * a.uniform_L;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hb = lane >> 5;

  const bf16_t* Q = static_cast<const bf16_t*>(a.q) + h * 64;
  const bf16_t* K = static_cast<const bf16_t*>(a.k) + h * 64;
  const bf16_t* V = static_cast<const bf16_t*>(a.v) + h * 64;

  __shared__ __attribute__((aligned(16))) bf16_t Ks[kKey * kLdK];
  __shared__ __attribute__((aligned(16))) bf16_t Vt[64 * kLdV];

  // this lane's query (clamped for the load; rows past q_len are not stored)
  const int qi = q0 + wave * 32 + l32;
  const int64_t qrow = row0 + min(qi, qlen - 1);
  bf16x8_t qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    qf[s] = *reinterpret_cast<const bf16x8_t*>(Q + qrow * a.ld_q + 16 * s + 8 * hb);

  int klo = 0, khi = klen;
  if (a.window > 0) {
    klo = max(0, q0 - a.window);
    khi = min(klen, q0 + kQ - 1 + a.window + 1);
  }
  const int qlo = a.window > 0 ? max(0, qi - a.window) : 0;
  const int qhi = a.window > 0 ? min(klen, qi + a.window + 1) : klen;

  f32x16_t o[2];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    o[0][e] = 0.f;
    o[1][e] = 0.f;
  }
  float m_i = -INFINITY, l_i = 0.f;
  const float c = a.scale * kLog2e;

  for (int kt = klo; kt < khi; kt += kKey) {
    // K tile: 64 keys x 64 dims, 16-byte chunks, 2 per thread.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ch = tid + 256 * i, r = ch >> 3, dc = ch & 7;
      const int key = min(kt + r, klen - 1);
      *reinterpret_cast<u32x4_t*>(Ks + r * kLdK + dc * 8) =
          *reinterpret_cast<const u32x4_t*>(K + (row0 + key) * a.ld_k + dc * 8);
    }
    // V tile transposed: a thread takes two keys x 8 dims and writes 8 key pairs.
    {
      const int kp = tid >> 3, dc = tid & 7;
      const int k0 = min(kt + 2 * kp, klen - 1), k1 = min(kt + 2 * kp + 1, klen - 1);
      const u32x4_t w0 = *reinterpret_cast<const u32x4_t*>(V + (row0 + k0) * a.ld_v + dc * 8);
      const u32x4_t w1 = *reinterpret_cast<const u32x4_t*>(V + (row0 + k1) * a.ld_v + dc * 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        *reinterpret_cast<uint32_t*>(Vt + (dc * 8 + 2 * e) * kLdV + 2 * kp) =
            (w0[e] & 0xffffu) | (w1[e] << 16);
        *reinterpret_cast<uint32_t*>(Vt + (dc * 8 + 2 * e + 1) * kLdV + 2 * kp) =
            (w0[e] >> 16) | (w1[e] & 0xffff0000u);
      }
    }
    __syncthreads();

    // S^T[key][query] for keys kt + [0, 32) and kt + [32, 64)
    f32x16_t s[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[jb][e] = 0.f;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const bf16x8_t kf =
            *reinterpret_cast<const bf16x8_t*>(Ks + (jb * 32 + l32) * kLdK + 16 * st + 8 * hb);
        s[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], s[jb], 0, 0, 0);
      }
    }
    // scale into the log2 domain, mask, tile max
    const bool need_mask = (kt + kKey > klen) || a.window > 0;
    float tmax = -INFINITY;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float v = s[jb][e] * c;
        if (need_mask) {
          const int key = kt + jb * 32 + 8 * (e >> 2) + 4 * hb + (e & 3);
          if (key < qlo || key >= qhi) v = -INFINITY;
        }
        s[jb][e] = v;
        tmax = fmaxf(tmax, v);
      }
    tmax = wave_max32(tmax);
    const float m_new = fmaxf(m_i, tmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_i - m_use);
    m_i = m_new;
    l_i *= alpha;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      o[0][e] *= alpha;
      o[1][e] *= alpha;
    }
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = exp2f(s[jb][e] - m_use);
        s[jb][e] = p;
        l_i += p;
      }
    // O^T[dim][query] += V^T[dim][key] . P^T[key][query]
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        bf16x8_t pf;
#pragma unroll
        for (int e = 0; e < 8; ++e) pf[e] = static_cast<__bf16>(s[jb][8 * u + e]);
        const int kb = jb * 32 + 16 * u + 4 * hb;
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const bf16_t* vr = Vt + (db * 32 + l32) * kLdV + kb;
          const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(vr);
          const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(vr + 8);
          const u32x4_t vv = {lo[0], lo[1], hi[0], hi[1]};
          const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, vv);
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[db], 0, 0, 0);
        }
      }
    __syncthreads();
  }

  const float l_tot = l_i + __shfl_xor(l_i, 32, 64);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (qi < qlen) {
    bf16_t* O = static_cast<bf16_t*>(a.o) + (row0 + qi) * a.ld_o + h * 64;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d = db * 32 + 8 * gq + 4 * hb;
        u32x2_t w;
        w[0] = pack_bf16x2(o[db][4 * gq + 0] * inv, o[db][4 * gq + 1] * inv);
        w[1] = pack_bf16x2(o[db][4 * gq + 2] * inv, o[db][4 * gq + 3] * inv);
        *reinterpret_cast<u32x2_t*>(O + d) = w;
      }
  }
}

// ------------------------------------------------------------------ generic
constexpr int gQ = 128;   // queries per workgroup (one per thread)
constexpr int gKey = 32;  // keys per LDS tile

template <typename T, int DH>
__global__ __launch_bounds__(gQ) void attn_generic_kernel(AttnArgs a) {
  const int b = blockIdx.z, h = blockIdx.y;
  const int qlen = a.q_len ? a.q_len[b] : a.uniform_L;
  const int q0 = blockIdx.x * gQ;
  if (q0 >= qlen) return;
  // keys never extend past the rows a sequence owns (a caller's k_len > L in
  // the padded layout is clamped rather than read out of bounds)
  const int klen = a.seq_start ? a.k_len[b] : max(0, min(a.k_len[b], a.uniform_L));
  const int64_t row0 = a.seq_start ? a.seq_start[b] : static_cast<int64_t>(b) * a.uniform_L;
  const int tid = threadIdx.x;
  const int qi = q0 + tid;
  const bool active = qi < qlen;

  const T* Q = static_cast<const T*>(a.q) + h * DH;
  const T* K = static_cast<const T*>(a.k) + h * DH;
  const T* V = static_cast<const T*>(a.v) + h * DH;
  __shared__ float Ks[gKey][DH];
  __shared__ float Vs[gKey][DH];

  float q[DH], o[DH];
  const int64_t qrow = row0 + min(qi, qlen - 1);
#pragma unroll
  for (int d = 0; d < DH; ++d) {
    q[d] = load_f32(Q + qrow * a.ld_q + d);
    o[d] = 0.f;
  }
  int klo = 0, khi = klen;
  if (a.window > 0) {
    klo = max(0, q0 - a.window);
    khi = min(klen, q0 + gQ - 1 + a.window + 1);
  }
  const int qlo = a.window > 0 ? max(0, qi - a.window) : 0;
  const int qhi = a.window > 0 ? min(klen, qi + a.window + 1) : klen;
  float m_i = -INFINITY, l_i = 0.f;

  for (int kt = klo; kt < khi; kt += gKey) {
    for (int idx = tid; idx < gKey * DH; idx += gQ) {
      const int r = idx / DH, d = idx - r * DH;
      const int key = min(kt + r, klen - 1);
      Ks[r][d] = load_f32(K + (row0 + key) * a.ld_k + d);
      Vs[r][d] = load_f32(V + (row0 + key) * a.ld_v + d);
    }
    __syncthreads();
    float sc[gKey];
    float tmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < gKey; ++j) {
      const int key = kt + j;
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < DH; ++d) s += q[d] * Ks[j][d];
      s *= a.scale;
      if (key < qlo || key >= qhi) s = -INFINITY;
      sc[j] = s;
      tmax = fmaxf(tmax, s);
    }
    const float m_new = fmaxf(m_i, tmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = expf(m_i - m_use);
    m_i = m_new;
    l_i *= alpha;
#pragma unroll
    for (int d = 0; d < DH; ++d) o[d] *= alpha;
#pragma unroll
    for (int j = 0; j < gKey; ++j) {
      const float p = expf(sc[j] - m_use);
      l_i += p;
#pragma unroll
      for (int d = 0; d < DH; ++d) o[d] += p * Vs[j][d];
    }
    __syncthreads();
  }
  if (active) {
    const float inv = l_i > 0.f ? 1.f / l_i : 0.f;
    T* O = static_cast<T*>(a.o) + (row0 + qi) * a.ld_o + h * DH;
#pragma unroll
    for (int d = 0; d < DH; ++d) store_f32(O + d, o[d] * inv);
  }
}

template <typename T>
void launch_generic(const AttnArgs& a, hipStream_t st) {
  dim3 grid((a.max_q + gQ - 1) / gQ, a.H, a.B), block(gQ);
  switch (a.Dh) {
    case 8: attn_generic_kernel<T, 8><<<grid, block, 0, st>>>(a); break;
    case 16: attn_generic_kernel<T, 16><<<grid, block, 0, st>>>(a); break;
    case 32: attn_generic_kernel<T, 32><<<grid, block, 0, st>>>(a); break;
    case 64: attn_generic_kernel<T, 64><<<grid, block, 0, st>>>(a); break;
    case 128: attn_generic_kernel<T, 128><<<grid, block, 0, st>>>(a); break;
    default: fail("attention: head_dim must be 8, 16, 32, 64 or 128");
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

void launch_attn(const AttnArgs& a, hipStream_t st) {
  if (a.B <= 0 || a.max_q <= 0) return;
  require(a.q && a.k && a.v && a.o, "attention: null pointer");
  require(a.k_len != nullptr, "attention: null key lengths");
  require((a.seq_start && a.q_len) || a.uniform_L > 0,
          "attention: need seq_start/q_len or a uniform row count");
  require(a.H > 0 && a.Dh > 0, "attention: bad head shape");
  require(a.ld_q >= a.H * a.Dh && a.ld_k >= a.H * a.Dh && a.ld_v >= a.H * a.Dh &&
              a.ld_o >= a.H * a.Dh,
          "attention: row stride < H*Dh");
  require(a.window >= 0, "attention: negative window");
  const bool mfma = a.dtype == DT_BF16 && a.Dh == 64 && a.ld_q % 8 == 0 && a.ld_k % 8 == 0 &&
                    a.ld_v % 8 == 0 && a.ld_o % 4 == 0 && aligned16(a.q) && aligned16(a.k) &&
                    aligned16(a.v) && (reinterpret_cast<uintptr_t>(a.o) & 7u) == 0;
  if (mfma) {
    dim3 grid((a.max_q + kQ - 1) / kQ, a.H, a.B), block(256);
    attn_bf16_mfma_kernel<<<grid, block, 0, st>>>(a);
    check_launch("attn_bf16_mfma");
    return;
  }
  if (a.dtype == DT_BF16)
    launch_generic<bf16_t>(a, st);
  else
    launch_generic<float>(a, st);
  check_launch("attn_generic");
}

}  // namespace sjh

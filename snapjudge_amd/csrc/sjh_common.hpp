// sjh_common.hpp -- device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>

namespace sjh {

// bf16 travels as raw uint16_t storage everywhere (the C ABI has no bf16 type).
typedef uint16_t bf16_t;

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;  // MFMA bf16 operand
typedef __attribute__((ext_vector_type(16))) float f32x16_t;  // 32x32 MFMA accumulator
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;  // 16-byte copies
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2_t;  // 8-byte copies

__device__ __forceinline__ float bf16_to_f32(bf16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet): the hardware
// conversion (v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) float f2_t;
  typedef __attribute__((ext_vector_type(2))) __bf16 bf2_t;
  const bf2_t v = __builtin_convertvector((f2_t){lo, hi}, bf2_t);
  return __builtin_bit_cast(uint32_t, v);
}

// Eight OCP e4m3fn codes (bytes of lo then hi, lowest byte first) as bf16.
// Every e4m3 value is exactly representable in bf16.  One
// v_cvt_scalef32_pk_bf16_fp8 (scale 1) turns two codes into two bf16; on the
// device it gave the same bits for all 256 codes in every byte position as
// the two-step decode through fp32 (v_cvt_pk_f32_fp8, itself checked against
// the e4m3fn table, then a round-to-nearest pack), at half the instructions.
__device__ __forceinline__ bf16x8_t fp8x8_to_bf16(uint32_t lo, uint32_t hi) {
  typedef __attribute__((ext_vector_type(2))) __bf16 bf2_t;
  const bf2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
  const bf2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
  const bf2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
  const bf2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
  const u32x4_t v = {__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                     __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d)};
  return __builtin_bit_cast(bf16x8_t, v);
}

// Exact erf GELU, the reference's activation (src/tensor.cpp:96-98).
__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654757f));
}

// GELU for outputs rounded to bf16, with the erf of Abramowitz & Stegun
// 7.1.26 (|erf error| <= 1.5e-7): 1 + erf(z) = 2 - q for z >= 0 and q for
// z < 0, q = erfc(|z|) = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-z^2),
// t = 1 / (1 + p |z|).  No branches (erff branches per element) and no
// cancellation for negative inputs; within 4.3e-7 of the exact GELU.
__device__ __forceinline__ float gelu_as(float x) {
  constexpr float kP = 0.3275911f, kA1 = 0.254829592f, kA2 = -0.284496736f, kA3 = 1.421413741f,
                  kA4 = -1.453152027f, kA5 = 1.061405429f;
  const float z = fabsf(x) * 0.70710678118654757f;
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(kP, z, 1.f));
  const float poly = t * __builtin_fmaf(t, __builtin_fmaf(t, __builtin_fmaf(t, __builtin_fmaf(t, kA5, kA4), kA3), kA2), kA1);
  const float q = poly * __builtin_amdgcn_exp2f(-1.4426950408889634f * z * z);
  return 0.5f * x * (x >= 0.f ? 2.f - q : q);
}

// GELU of a GEMM epilogue: the branch-free form where the output is rounded
// to bf16, erff (the reference's function) for fp32 outputs.
template <typename OutT>
__device__ __forceinline__ float gelu_out(float x) {
  if constexpr (std::is_same<OutT, bf16_t>::value)
    return gelu_as(x);
  else
    return gelu_erf(x);
}

// Rotate-half RoPE on one pair (x0 = dim d, x1 = dim d + Dh/2), as
// src/tensor.cpp:257-279: each product rounded to float, then the sum.
// Contraction into a fused multiply-add is switched off here so that every
// kernel that inlines these (whatever its register schedule) rounds the same
// way.
__device__ __forceinline__ float rope_lo(float x0, float x1, float c, float s) {
#pragma clang fp contract(off)
  return x0 * c - x1 * s;
}
__device__ __forceinline__ float rope_hi(float x0, float x1, float c, float s) {
#pragma clang fp contract(off)
  return x1 * c + x0 * s;
}

template <typename T>
__device__ __forceinline__ float load_f32(const T* p);
template <>
__device__ __forceinline__ float load_f32<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_f32<bf16_t>(const bf16_t* p) { return bf16_to_f32(*p); }

template <typename T>
__device__ __forceinline__ void store_f32(T* p, float v);
template <>
__device__ __forceinline__ void store_f32<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_f32<bf16_t>(bf16_t* p, float v) { *p = f32_to_bf16(v); }

// Wait until at most N vector-memory operations of this wave are
// outstanding.  Direct-to-LDS loads complete in issue order, so this is how a
// kernel knows that the oldest stages of its LDS ring have landed.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt immediate");
  if constexpr (N == 0) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
  }
}

// Every LDS read of this wave has returned (lgkmcnt(0)).  A wave that still
// has operand reads of a ring slot in flight must not pass the barrier after
// which other waves refill that slot.  Issued through the builtin (not inline
// asm) so that the compiler's own wait insertion knows that nothing of LGKM
// is outstanding afterwards.  gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt[5:4] at [15:14]; vmcnt 63 and expcnt 7 wait for nothing.
__device__ __forceinline__ void wait_lgkm0() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
}

// The lane's index in its wavefront, computed where it is used: the asm
// cannot be hoisted or merged with an earlier copy, so a kernel near its
// register limit recomputes the value (two VALU ops) instead of keeping it
// live, or spilling it, across a long loop.
__device__ __forceinline__ int lane_id_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Direct-to-LDS 16-byte load: lane l's 16 bytes from src land at
// lds_base + 16 * l (lds_base must be the same for the whole wave).
__device__ __forceinline__ void load_lds16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(lds_base), 16,
                                   0, 0);
}

// ---- LayerNorm statistics (src/tensor.cpp:54-79) -------------------------
// Shared by the standalone LayerNorm and the residual GEMM epilogue that
// finishes one, so that both give the same bits.  A row of D = 256 nb
// columns is taken in 256-column blocks.  Per block, d = x - x0 (x0 the
// block's first value) is summed over a fixed pairwise tree -- columns k and
// k + 32 of each 64-column group first, then the partial sums at column
// distance 16, 8, 4, 2 and 1, then the four groups as (g0 + g1) + (g2 + g3)
// -- and s = sum /
// 256; the squares of e = d - s go through the same tree, its first level as
// fma(e[k + 32], e[k + 32], e[k] * e[k]).  The blocks combine in double: the
// block means x0 + s, the row mean, and the pooled sum of squared deviations
// (Chan et al.), giving the population variance; the mean and the inverse
// std are then rounded to float and y = (x - mean) * inv * w (+ b) in float,
// as the reference computes them.  The shift keeps the fp32 sums exact to
// the rows' spread however large their offset.
constexpr int kLnStatBlock = 256;
constexpr int kLnStatMaxBlocks = 4;

// First level of the squares' tree: e_lo = e[k], e_hi = e[k + 32].
__device__ __forceinline__ float ln_pair_sq(float e_lo, float e_hi) {
#pragma clang fp contract(off)
  return __builtin_fmaf(e_hi, e_hi, e_lo * e_lo);
}

// Row statistics from the nb blocks' (x0, s, q): mean and inverse std.
__device__ __forceinline__ void ln_block_combine(const float (&x0)[kLnStatMaxBlocks], const float (&s)[kLnStatMaxBlocks],
                                                 const float (&q)[kLnStatMaxBlocks], int nb, float eps,
                                                 float& fmean, float& finv) {
  double mb[kLnStatMaxBlocks], sum = 0.0;
#pragma unroll
  for (int b = 0; b < kLnStatMaxBlocks; ++b)
    if (b < nb) {
      mb[b] = static_cast<double>(x0[b]) + static_cast<double>(s[b]);
      sum += mb[b];
    }
  const double mean = sum / nb;
  double m2 = 0.0;
#pragma unroll
  for (int b = 0; b < kLnStatMaxBlocks; ++b)
    if (b < nb) {
      const double dm = mb[b] - mean;
      m2 += static_cast<double>(q[b]) + static_cast<double>(kLnStatBlock) * dm * dm;
    }
  const double var = m2 / (static_cast<double>(kLnStatBlock) * nb);
  fmean = static_cast<float>(mean);
  finv = static_cast<float>(1.0 / sqrt(var + static_cast<double>(eps)));
}

// y = (x - mean) * inv * w (+ b), in this order and unfused.
__device__ __forceinline__ float ln_apply(float x, float fmean, float finv, float w, float b, bool has_b) {
#pragma clang fp contract(off)
  float y = (x - fmean) * finv;
  y = y * w;
  if (has_b) y = y + b;
  return y;
}

// 64-lane wavefront reductions via DPP-backed shuffles.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace sjh

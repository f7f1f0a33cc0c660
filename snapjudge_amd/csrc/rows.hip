// rows.hip -- row-wise HBM-bound kernels for gfx950: LayerNorm (with the
// embedding gather and the residual add fused in), RoPE, token indexing,
// row gathers.
//
// One 64-lane wavefront owns one row: the row is read once into registers
// (coalesced, one float per lane per 64 columns), reduced with cross-lane
// shuffles, normalised and written once.
#include <type_traits>

#include "sjh_common.hpp"
#include "sjh_host.hpp"
#include "sjh_kernels.hpp"

namespace sjh {

namespace {

constexpr int kLnWaves = 4;        // rows per workgroup
#ifndef SJH_LN_PARTS_WAVES
#define SJH_LN_PARTS_WAVES 1
#endif
constexpr int kLnPartsWaves = SJH_LN_PARTS_WAVES;  // rows per workgroup of the split-K sums
constexpr int kLnMaxPerLane = 64;  // D <= 4096 (64 lanes x 64 values)

// LayerNorm as src/tensor.cpp:54-79: mean and population variance
// accumulated in double, inverse std rounded to float, then
// (x - (float)mean) * inv * w (+ b) in float.
template <int NPL, typename InT, typename ResT, typename OutT>
__global__ __launch_bounds__(64 * kLnWaves) void ln_rows_kernel(LnArgs a) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * kLnWaves + (threadIdx.x >> 6);
  if (r >= (a.M_dev ? *a.M_dev : a.M)) return;
  const int D = a.D;
  const int64_t src_row = a.ids ? static_cast<int64_t>(a.ids[r]) : static_cast<int64_t>(r);
  const InT* in = static_cast<const InT*>(a.in) + src_row * a.ld_in;
  const ResT* res = a.resid ? static_cast<const ResT*>(a.resid) + static_cast<int64_t>(r) * a.ld_in
                            : nullptr;
  const float* add = a.add ? a.add + static_cast<int64_t>(min(max(a.add_ids[r], 0), a.add_rows - 1)) * a.ld_add
                           : nullptr;
  float v[NPL];
  const int npl = (D + 63) >> 6;
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    if (i < npl) {
      const int j = i * 64 + lane;
      float x = 0.f;
      if (j < D) {
        x = load_f32(in + j);
        if (add) x += add[j];
        if (res) x += load_f32(res + j);
      }
      v[i] = x;
      s += static_cast<double>(x);
    }
  }
  if (a.xio) {
    float* xo = a.xio + static_cast<int64_t>(r) * a.ld_in;
#pragma unroll
    for (int i = 0; i < NPL; ++i)
      if (i < npl && i * 64 + lane < D) xo[i * 64 + lane] = v[i];
  }
  float inv = 1.f, fmean = 0.f;
  if (a.normalize) {
    const double mean = wave_sum(s) / static_cast<double>(D);
    double q = 0.0;
#pragma unroll
    for (int i = 0; i < NPL; ++i)
      if (i < npl && i * 64 + lane < D) {
        const double d = static_cast<double>(v[i]) - mean;
        q += d * d;
      }
    const double var = wave_sum(q) / static_cast<double>(D);
    inv = static_cast<float>(1.0 / sqrt(var + static_cast<double>(a.eps)));
    fmean = static_cast<float>(mean);
  }
  float* xo = a.x_out ? a.x_out + static_cast<int64_t>(r) * a.ld_x : nullptr;
  OutT* yo = a.y_out ? static_cast<OutT*>(a.y_out) + static_cast<int64_t>(r) * a.ld_y : nullptr;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int j = i * 64 + lane;
    if (i < npl && j < D) {
      float y = v[i];
      if (a.normalize) {
        y = (y - fmean) * inv;
        if (a.w) y = y * a.w[j];
        if (a.b) y = y + a.b[j];
      }
      if (xo) xo[j] = y;
      if (yo) store_f32(yo + j, y);
    }
  }
}

// Vector variant for D % 4 == 0 and D <= 1024: lane l owns the 4-column
// chunks l, l + 64, ..., so every row moves with 16-byte (fp32) or 8-byte
// (bf16) accesses.  Same arithmetic as ln_rows_kernel.
template <typename T>
struct Vec4;
template <>
struct Vec4<float> {
  using Raw = f32x4_t;
  static __device__ __forceinline__ Raw raw(const float* p) { return *reinterpret_cast<const Raw*>(p); }
  static __device__ __forceinline__ void cvt(const Raw& v, float (&o)[4]) {
    o[0] = v[0], o[1] = v[1], o[2] = v[2], o[3] = v[3];
  }
  static __device__ __forceinline__ void load(const float* p, float (&o)[4]) {
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(p);
    o[0] = v[0], o[1] = v[1], o[2] = v[2], o[3] = v[3];
  }
  static __device__ __forceinline__ void store(float* p, const float (&o)[4]) {
    *reinterpret_cast<f32x4_t*>(p) = f32x4_t{o[0], o[1], o[2], o[3]};
  }
};
template <>
struct Vec4<bf16_t> {
  using Raw = u32x2_t;
  static __device__ __forceinline__ Raw raw(const bf16_t* p) { return *reinterpret_cast<const Raw*>(p); }
  static __device__ __forceinline__ void cvt(const Raw& v, float (&o)[4]) {
    o[0] = __uint_as_float(v[0] << 16), o[1] = __uint_as_float(v[0] & 0xffff0000u);
    o[2] = __uint_as_float(v[1] << 16), o[3] = __uint_as_float(v[1] & 0xffff0000u);
  }
  static __device__ __forceinline__ void load(const bf16_t* p, float (&o)[4]) {
    const u32x2_t v = *reinterpret_cast<const u32x2_t*>(p);
    o[0] = __uint_as_float(v[0] << 16), o[1] = __uint_as_float(v[0] & 0xffff0000u);
    o[2] = __uint_as_float(v[1] << 16), o[3] = __uint_as_float(v[1] & 0xffff0000u);
  }
  static __device__ __forceinline__ void store(bf16_t* p, const float (&o)[4]) {
    *reinterpret_cast<u32x2_t*>(p) = u32x2_t{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
  }
};

// Residual types of a vector layer norm: none, or the split-K partials of the
// residual GEMM that produced the input (LnArgs::parts).
struct NoRes {};
template <>
struct Vec4<NoRes> {
  using Raw = int;
};
struct PartsRes {};
template <>
struct Vec4<PartsRes> {
  using Raw = int;
};

// Sum of a double over the 64 lanes, every lane receiving the total: DPP
// exchanges inside each row of 16 lanes (pairs, quads, mirrored halves,
// mirrored rows), then two shuffles across the rows.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(u), CTRL, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(u >> 32), CTRL, 0xf, 0xf, false);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                        static_cast<uint32_t>(lo));
}
__device__ __forceinline__ void wave_sum2(double& a, double& b) {
  a += dpp_f64<0xB1>(a), b += dpp_f64<0xB1>(b);    // quad_perm [1,0,3,2]
  a += dpp_f64<0x4E>(a), b += dpp_f64<0x4E>(b);    // quad_perm [2,3,0,1]
  a += dpp_f64<0x141>(a), b += dpp_f64<0x141>(b);  // row_half_mirror
  a += dpp_f64<0x140>(a), b += dpp_f64<0x140>(b);  // row_mirror
  a += __shfl_xor(a, 16, 64), b += __shfl_xor(b, 16, 64);
  a += __shfl_xor(a, 32, 64), b += __shfl_xor(b, 32, 64);
}

// Vector variant for D % 4 == 0 and D <= 1024: lane l owns the 4-column
// chunks l, l + 64, ..., so every row moves with 16-byte (fp32) or 8-byte
// (bf16) accesses.  FULL: D == 256 * NV, so every chunk exists and a row's
// loads all go out before the first use.  The statistics are those of
// src/tensor.cpp:63-71 (mean and population variance in double, inverse std
// rounded to float), gathered in one pass as the moments of x - x0 (x0 =
// the row's first value, which keeps E[d^2] - E[d]^2 well conditioned).
template <int NV, bool FULL, typename InT, typename ResT, typename OutT, int WPB>
__global__ __launch_bounds__(64 * WPB) void ln_vec_kernel(LnArgs a) {
  const int lane = threadIdx.x & 63;
  // The row is uniform over the wave: scalar row addresses and gather index.
  const int r = __builtin_amdgcn_readfirstlane(blockIdx.x * WPB + (threadIdx.x >> 6));
  if (r >= (a.M_dev ? *a.M_dev : a.M)) return;
  const int D = a.D, nch = D >> 2;
  const int64_t src_row = a.ids ? static_cast<int64_t>(a.ids[r]) : static_cast<int64_t>(r);
  const InT* in = static_cast<const InT*>(a.in) + src_row * a.ld_in;
  constexpr bool kParts = std::is_same<ResT, PartsRes>::value;
  constexpr bool kRes = !std::is_same<ResT, NoRes>::value && !kParts;
  // Every load of the row (residual, input, gain, bias) is issued before the
  // first use; raw registers are converted afterwards.
  float w[NV][4], b[NV][4];
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k) w[i][k] = 1.f, b[i][k] = 0.f;
  if (a.normalize && a.w) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (FULL || lane + 64 * i < nch) Vec4<float>::load(a.w + 4 * (lane + 64 * i), w[i]);
  }
  if (a.normalize && a.b) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (FULL || lane + 64 * i < nch) Vec4<float>::load(a.b + 4 * (lane + 64 * i), b[i]);
  }
  typename Vec4<InT>::Raw vr[NV] = {};
  typename Vec4<ResT>::Raw tr[NV] = {};
  if constexpr (kRes) {
    const ResT* res = static_cast<const ResT*>(a.resid) + static_cast<int64_t>(r) * a.ld_in;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (FULL || lane + 64 * i < nch) tr[i] = Vec4<ResT>::raw(res + 4 * (lane + 64 * i));
  }
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (FULL || lane + 64 * i < nch) vr[i] = Vec4<InT>::raw(in + 4 * (lane + 64 * i));
  // the added row (a learned position embedding), when given
  f32x4_t ar[NV] = {};
  if (a.add) {
    const float* add = a.add + static_cast<int64_t>(min(max(a.add_ids[r], 0), a.add_rows - 1)) * a.ld_add;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (FULL || lane + 64 * i < nch) ar[i] = *reinterpret_cast<const f32x4_t*>(add + 4 * (lane + 64 * i));
  }
  float v[NV][4];
#pragma unroll
  for (int i = 0; i < NV; ++i) Vec4<InT>::cvt(vr[i], v[i]);
  if (a.add) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) v[i][k] += ar[i][k];
  }
  if constexpr (kParts) {
    // x = in + (p_0 + p_1 + ... + p_{S-1} + bias), summed from 0 in split
    // order: the split-K residual epilogue's arithmetic
    // (splits are loaded PG at a time, every load of a group issued before
    // the first add)
    constexpr int PG = 8;
    const float* pr = a.parts + static_cast<int64_t>(r) * a.ld_part;
    float t[NV][4] = {};
    for (int s0 = 0; s0 < a.n_parts; s0 += PG) {
      f32x4_t p[PG][NV];
#pragma unroll
      for (int u = 0; u < PG; ++u)
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int c = lane + 64 * i;
          p[u][i] = (s0 + u < a.n_parts && (FULL || c < nch))
                        ? *reinterpret_cast<const f32x4_t*>(pr + (s0 + u) * a.part_stride + 4 * c)
                        : (f32x4_t){0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
      for (int u = 0; u < PG; ++u)
        if (s0 + u < a.n_parts)
#pragma unroll
          for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k) t[i][k] += p[u][i][k];
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i;
      if (!FULL && c >= nch) continue;
      if (a.part_bias) {
        const f32x4_t b = *reinterpret_cast<const f32x4_t*>(a.part_bias + 4 * c);
#pragma unroll
        for (int k = 0; k < 4; ++k) t[i][k] += b[k];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) v[i][k] += t[i][k];
    }
  }
  if constexpr (kRes) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (FULL || lane + 64 * i < nch) {
        float t[4];
        Vec4<ResT>::cvt(tr[i], t);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[i][k] += t[k];
      }
  }
  if (a.xio) {
    float* xo = a.xio + static_cast<int64_t>(r) * a.ld_in;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (FULL || lane + 64 * i < nch) Vec4<float>::store(xo + 4 * (lane + 64 * i), v[i]);
  }
  float inv = 1.f, fmean = 0.f;
  if (a.normalize) {
    if constexpr (FULL) {
      // D = 256 NV: the 256-column block statistics of sjh_common.hpp
      // (ln_block_combine), the residual epilogue's arithmetic bit for bit.
      // Block b is chunk 64 b + lane: columns 256 b + 4 lane + [0, 4), so the
      // tree's column distances 32, 16, 8, 4 are lane distances 8, 4, 2, 1
      // inside each 16-lane DPP row (one row per 64-column group) and 2, 1
      // are inside the lane.  Each level's sums gather in the upper lane of
      // its pairs (row_shr), so lane 15 of row g ends with group g's sum; the
      // groups combine as (g0 + g1) + (g2 + g3) through row broadcasts into
      // lane 63.
      float x0b[kLnStatMaxBlocks] = {}, sb[kLnStatMaxBlocks] = {}, qb[kLnStatMaxBlocks] = {};
      auto shr = [](float x, auto ctrl_tag) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                    decltype(ctrl_tag)::value, 0xf, 0xf, false));
      };
      using Shr4 = std::integral_constant<int, 0x114>;
      using Shr2 = std::integral_constant<int, 0x112>;
      using Shr1 = std::integral_constant<int, 0x111>;
      auto tree = [&](float (&t4)[4]) {  // t4: level 1 done (lane distance 8)
#pragma unroll
        for (int k = 0; k < 4; ++k) t4[k] = t4[k] + shr(t4[k], Shr4{});
#pragma unroll
        for (int k = 0; k < 4; ++k) t4[k] = t4[k] + shr(t4[k], Shr2{});
#pragma unroll
        for (int k = 0; k < 4; ++k) t4[k] = t4[k] + shr(t4[k], Shr1{});
        float g = (t4[0] + t4[2]) + (t4[1] + t4[3]);
        g = g + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, g), 0x142, 0xa,
                                                                        0xf, false));  // row_bcast:15
        g = g + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, g), 0x143, 0xc,
                                                                        0xf, false));  // row_bcast:31
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, g), 63));
      };
      using Shr8 = std::integral_constant<int, 0x118>;
#pragma unroll
      for (int b = 0; b < NV; ++b) {
        const float x0 = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v[b][0])));
        float d[4], t4[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) d[k] = v[b][k] - x0;
#pragma unroll
        for (int k = 0; k < 4; ++k) t4[k] = d[k] + shr(d[k], Shr8{});  // columns k + 32 (own), k (shifted)
        const float sm = tree(t4) * (1.0f / kLnStatBlock);
        float e[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) e[k] = d[k] - sm;
#pragma unroll
        for (int k = 0; k < 4; ++k) t4[k] = ln_pair_sq(shr(e[k], Shr8{}), e[k]);
        x0b[b] = x0;
        sb[b] = sm;
        qb[b] = tree(t4);
      }
      ln_block_combine(x0b, sb, qb, NV, a.eps, fmean, inv);
    } else {
      const double x0 = static_cast<double>(__builtin_bit_cast(
          float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v[0][0]))));
      double s1 = 0.0, s2 = 0.0;
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (FULL || lane + 64 * i < nch)
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const double d = static_cast<double>(v[i][k]) - x0;
            s1 += d;
            s2 += d * d;
          }
      wave_sum2(s1, s2);
      const double dm = s1 / static_cast<double>(D);
      const double mean = x0 + dm;
      const double var = fmax(s2 / static_cast<double>(D) - dm * dm, 0.0);
      inv = static_cast<float>(1.0 / sqrt(var + static_cast<double>(a.eps)));
      fmean = static_cast<float>(mean);
    }
  }
  float* xo = a.x_out ? a.x_out + static_cast<int64_t>(r) * a.ld_x : nullptr;
  OutT* yo = a.y_out ? static_cast<OutT*>(a.y_out) + static_cast<int64_t>(r) * a.ld_y : nullptr;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    if (!FULL && c >= nch) continue;
    float y[4] = {v[i][0], v[i][1], v[i][2], v[i][3]};
    if (a.normalize) {
#pragma unroll
      for (int k = 0; k < 4; ++k) y[k] = ln_apply(y[k], fmean, inv, w[i][k], b[i][k], a.b != nullptr);
    }
    if (xo) Vec4<float>::store(xo + 4 * c, y);
    if (yo) Vec4<OutT>::store(yo + 4 * c, y);
  }
}

template <int NV, typename InT, typename ResT>
void ln_vec_dispatch_out(const LnArgs& a, hipStream_t st) {
  // Rows (waves) per workgroup.  The split-K partial sums run on short
  // batches only (M <= 256): each row there streams its partial rows, so
  // the rows are spread over kLnPartsWaves-wave workgroups.
  constexpr int WPB = std::is_same<ResT, PartsRes>::value ? kLnPartsWaves : kLnWaves;
  dim3 grid((a.M + WPB - 1) / WPB), block(64 * WPB);
  const bool full = a.D == 256 * NV;
  if (a.y_dtype == DT_BF16)
    full ? ln_vec_kernel<NV, true, InT, ResT, bf16_t, WPB><<<grid, block, 0, st>>>(a)
         : ln_vec_kernel<NV, false, InT, ResT, bf16_t, WPB><<<grid, block, 0, st>>>(a);
  else
    full ? ln_vec_kernel<NV, true, InT, ResT, float, WPB><<<grid, block, 0, st>>>(a)
         : ln_vec_kernel<NV, false, InT, ResT, float, WPB><<<grid, block, 0, st>>>(a);
}

template <typename InT, typename ResT>
void ln_vec_dispatch(const LnArgs& a, hipStream_t st) {
  switch ((a.D + 255) / 256) {
    case 1: ln_vec_dispatch_out<1, InT, ResT>(a, st); break;
    case 2: ln_vec_dispatch_out<2, InT, ResT>(a, st); break;
    case 3: ln_vec_dispatch_out<3, InT, ResT>(a, st); break;
    default: ln_vec_dispatch_out<4, InT, ResT>(a, st); break;
  }
}

template <int NPL, typename InT, typename ResT>
void ln_dispatch_out(const LnArgs& a, hipStream_t st) {
  dim3 grid((a.M + kLnWaves - 1) / kLnWaves), block(64 * kLnWaves);
  if (a.y_dtype == DT_BF16)
    ln_rows_kernel<NPL, InT, ResT, bf16_t><<<grid, block, 0, st>>>(a);
  else
    ln_rows_kernel<NPL, InT, ResT, float><<<grid, block, 0, st>>>(a);
}

// Per-lane register budget: the smallest of 4 / 16 / 64 values that holds D.
template <typename InT, typename ResT>
void ln_dispatch_npl(const LnArgs& a, hipStream_t st) {
  const int npl = (a.D + 63) / 64;
  if (npl <= 4)
    ln_dispatch_out<4, InT, ResT>(a, st);
  else if (npl <= 16)
    ln_dispatch_out<16, InT, ResT>(a, st);
  else
    ln_dispatch_out<kLnMaxPerLane, InT, ResT>(a, st);
}

template <typename InT>
void ln_dispatch_res(const LnArgs& a, hipStream_t st) {
  if (a.resid_dtype == DT_BF16)
    ln_dispatch_npl<InT, bf16_t>(a, st);
  else
    ln_dispatch_npl<InT, float>(a, st);
}

// Rotate-half RoPE on packed rows (src/tensor.cpp:257-279); one thread per
// (row, q/k head, pair).
template <typename T>
__global__ void rope_kernel(T* qkv, int64_t M, int64_t ld, const int* pos, int L, int H, int Dh,
                            const float* cos_t, const float* sin_t) {
  const int half = Dh / 2;
  const int64_t per_row = static_cast<int64_t>(2) * H * half;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= M * per_row) return;
  const int64_t r = idx / per_row;
  const int rem = static_cast<int>(idx - r * per_row);
  const int hh = rem / half, d = rem - hh * half;
  const int p = pos ? pos[r] : static_cast<int>(r % L);
  T* x = qkv + r * ld + static_cast<int64_t>(hh) * Dh;
  const float x0 = load_f32(x + d), x1 = load_f32(x + d + half);
  const float c = cos_t[static_cast<int64_t>(p) * half + d];
  const float s = sin_t[static_cast<int64_t>(p) * half + d];
  store_f32(x + d, rope_lo(x0, x1, c, s));
  store_f32(x + d + half, rope_hi(x0, x1, c, s));
}

__global__ void token_index_kernel(const int* seq_start, const int* rows, int* tok_pos,
                                   int* tok_seq) {
  const int b = blockIdx.x;
  const int s0 = seq_start[b], n = rows[b];
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    tok_pos[s0 + i] = i;
    tok_seq[s0 + i] = b;
  }
}

__global__ void add_row_embedding_kernel(float* X, int64_t ldx, const float* table,
                                         const int* sel, const int* tok_seq, int T,
                                         const int* T_dev, int D) {
  const int t = blockIdx.x;
  if (t >= (T_dev ? *T_dev : T)) return;
  const float* te = table + static_cast<int64_t>(sel[tok_seq[t]]) * D;
  float* x = X + static_cast<int64_t>(t) * ldx;
  for (int j = threadIdx.x; j < D; j += blockDim.x) x[j] += te[j];
}

__global__ void gather_rows_kernel(const float* src, int64_t ld_src, const int* idx, int n, int D,
                                   float* dst, int64_t ld_dst) {
  const int i = blockIdx.x;
  if (i >= n) return;
  const int s = idx[i];
  float* d = dst + static_cast<int64_t>(i) * ld_dst;
  for (int j = threadIdx.x; j < D; j += blockDim.x)
    d[j] = s >= 0 ? src[static_cast<int64_t>(s) * ld_src + j] : 0.f;
}

// Act-head inputs of row b (src/model.cpp:484, 489-517): the masked logits
// (-1e4 where the marker is padding), their softmax (exp in float, sums in
// double, as the reference), top1, top1 - top2, the entropy over log(max(2,
// live markers)) and kf / 255, written after the row's [CLS] hidden state.
// One workgroup per row; the short serial part runs on one lane.
__global__ void act_features_kernel(const float* s2, const int* mmask, int K, const float* cls,
                                    int64_t ld_cls, int D, float* logits, float* ain,
                                    int64_t ld_ain) {
  const int b = blockIdx.x;
  const float* sb = s2 + static_cast<int64_t>(b) * K;
  const int* mb = mmask + static_cast<int64_t>(b) * K;
  float* lg = logits + static_cast<int64_t>(b) * K;
  float* f = ain + static_cast<int64_t>(b) * ld_ain;
  for (int k = threadIdx.x; k < K; k += blockDim.x) lg[k] = mb[k] ? sb[k] : -1e4f;
  for (int j = threadIdx.x; j < D; j += blockDim.x) f[j] = cls[static_cast<int64_t>(b) * ld_cls + j];
  __syncthreads();
  if (threadIdx.x != 0) return;
  float mx = lg[0];
  for (int j = 1; j < K; ++j) mx = fmaxf(mx, lg[j]);
  double s = 0.0;
  for (int j = 0; j < K; ++j) s += static_cast<double>(expf(lg[j] - mx));
  double top1 = 0.0, top2 = 0.0, ent = 0.0, ksum = 0.0;
  for (int j = 0; j < K; ++j) {
    const double v = static_cast<double>(expf(lg[j] - mx)) / s;
    if (v > top1) {
      top2 = top1;
      top1 = v;
    } else if (v > top2) {
      top2 = v;
    }
    ent -= v * log(fmax(v, 1e-9));
    ksum += mb[j];
  }
  const double kf = fmax(2.0, ksum);
  ent /= log(kf);
  f[D + 0] = static_cast<float>(top1);
  f[D + 1] = static_cast<float>(top1 - top2);
  f[D + 2] = static_cast<float>(ent);
  f[D + 3] = static_cast<float>(kf / 255.0);
}

// act = softmax(a) per row (src/model.cpp:523-534): exp in float, the sum in
// double, each probability divided in double.  One thread per row.
__global__ void act_softmax_kernel(const float* a, int B, int n, float* act) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const float* ab = a + static_cast<int64_t>(b) * n;
  float amx = ab[0];
  for (int j = 1; j < n; ++j) amx = fmaxf(amx, ab[j]);
  double as = 0.0;
  for (int j = 0; j < n; ++j) as += static_cast<double>(expf(ab[j] - amx));
  for (int j = 0; j < n; ++j)
    act[static_cast<int64_t>(b) * n + j] = static_cast<float>(static_cast<double>(expf(ab[j] - amx)) / as);
}

// SjModel's act head (src/sj_model.cpp:336-367), one thread per row:
// logits[b, k] = mmask[b, k] ? s2[b, k] : -1e4; p = softmax over the row's K
// logits (float exp of the max-subtracted logit, double sum and division);
// act[b] = {top1, 1 - top1}.
__global__ void act_top1_kernel(const float* s2, const int* mmask, int B, int K, float* logits,
                                float* act) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const float* sb = s2 + static_cast<int64_t>(b) * K;
  const int* mb = mmask + static_cast<int64_t>(b) * K;
  float* lg = logits + static_cast<int64_t>(b) * K;
  float mx = 0.f;
  for (int k = 0; k < K; ++k) {
    const float v = mb[k] ? sb[k] : -1e4f;
    lg[k] = v;
    mx = (k == 0 || v > mx) ? v : mx;
  }
  double s = 0.0;
  for (int k = 0; k < K; ++k) s += static_cast<double>(expf(lg[k] - mx));
  double top1 = 0.0;
  for (int k = 0; k < K; ++k) {
    const double p = static_cast<double>(expf(lg[k] - mx)) / s;
    top1 = (k == 0 || p > top1) ? p : top1;
  }
  act[2 * b] = static_cast<float>(top1);
  act[2 * b + 1] = static_cast<float>(1.0 - top1);
}

// Lengths of a batch, passed by value (no host staging buffer).
struct SeqTableArgs {
  int B, Bb;
  int32_t lens[kSeqTableMaxB];
};

// The per-batch sequence table (layout in sjh_kernels.hpp) from the lengths,
// one workgroup of kSeqTableMaxB threads, thread b = table entry b.  The
// order is the stable sort by decreasing length: entry b's rank counts the
// longer entries and the equal ones before it.
__global__ __launch_bounds__(kSeqTableMaxB) void seq_table_kernel(SeqTableArgs a, int32_t* t) {
  __shared__ int32_t len_s[kSeqTableMaxB], start_s[kSeqTableMaxB];
  const int b = threadIdx.x;
  const int32_t* lens = a.lens;
  const int n = b < a.B ? lens[b] : 0;
  len_s[b] = n;
  __syncthreads();
  // exclusive prefix sum of the lengths (Hillis-Steele over the workgroup)
  int incl = n;
  start_s[b] = incl;
  __syncthreads();
  for (int off = 1; off < kSeqTableMaxB; off <<= 1) {
    const int add = b >= off ? start_s[b - off] : 0;
    __syncthreads();
    incl += add;
    start_s[b] = incl;
    __syncthreads();
  }
  const int total = start_s[kSeqTableMaxB - 1];
  const int start = b < a.B ? incl - n : total;
  if (b == 0) {
    t[0] = total;
    t[1] = a.B;
    t[2] = 0;
    t[3] = 0;
  }
  int rank = b;  // empty entries keep their place after the real sequences
  if (b < a.B) {
    rank = 0;
    for (int c = 0; c < a.B; ++c) {
      const int m = len_s[c];
      rank += (m > n || (m == n && c < b)) ? 1 : 0;
    }
  }
  // attention query blocks per entry, in table order, and their prefix
  // (ranks are a permutation of [0, Bb); entries past Bb have none)
  __syncthreads();  // every thread is done with start_s
  start_s[b] = 0;
  __syncthreads();
  if (b < a.Bb) start_s[rank] = (n + kAttnQ - 1) / kAttnQ;
  __syncthreads();
  int qb_incl = start_s[b];
  const int qb_own = qb_incl;
  for (int off = 1; off < kSeqTableMaxB; off <<= 1) {
    const int add = b >= off ? start_s[b - off] : 0;
    __syncthreads();
    qb_incl += add;
    start_s[b] = qb_incl;
    __syncthreads();
  }
  int32_t* qbp = t + seq_table_qbp(a.Bb);
  if (b == 0) qbp[a.Bb] = start_s[kSeqTableMaxB - 1];  // the total
  if (b >= a.Bb) return;
  qbp[b] = qb_incl - qb_own;  // exclusive prefix
  int32_t* seq_start = t + kSeqHdr;
  seq_start[b] = start;
  seq_start[a.Bb + b] = n;       // q_len
  seq_start[2 * a.Bb + b] = n;   // k_len
  seq_start[3 * a.Bb + b] = 0;   // qtype
  seq_start[4 * a.Bb + rank] = b;  // order
  int32_t* meta = t + (kSeqHdr + 5 * a.Bb + 3) / 4 * 4 + 4 * rank;
  meta[0] = start;
  meta[1] = n;
  meta[2] = n;
  meta[3] = 0;
}

}  // namespace

void launch_seq_table(const int32_t* h_lens, int B, int Bb, int32_t* table, hipStream_t st) {
  require(B >= 0 && B <= Bb && Bb <= kSeqTableMaxB, "seq_table: need 0 <= B <= Bb <= 256");
  require(B == 0 || h_lens != nullptr, "seq_table: null lengths");
  SeqTableArgs a;
  a.B = B;
  a.Bb = Bb;
  for (int b = 0; b < kSeqTableMaxB; ++b) a.lens[b] = b < B ? h_lens[b] : 0;
  seq_table_kernel<<<1, kSeqTableMaxB, 0, st>>>(a, table);
  check_launch("seq_table");
}

void launch_act_features(const float* s2, const int* mmask, int B, int K, const float* cls,
                         int64_t ld_cls, int D, float* logits, float* ain, int64_t ld_ain,
                         hipStream_t st) {
  if (B <= 0 || K <= 0) return;
  act_features_kernel<<<B, 256, 0, st>>>(s2, mmask, K, cls, ld_cls, D, logits, ain, ld_ain);
  check_launch("act_features");
}

void launch_act_top1(const float* s2, const int* mmask, int B, int K, float* logits, float* act,
                     hipStream_t st) {
  if (B <= 0 || K <= 0) return;
  act_top1_kernel<<<(B + 63) / 64, 64, 0, st>>>(s2, mmask, B, K, logits, act);
  check_launch("act_top1");
}

void launch_act_softmax(const float* a, int B, int n, float* act, hipStream_t st) {
  if (B <= 0 || n <= 0) return;
  act_softmax_kernel<<<(B + 63) / 64, 64, 0, st>>>(a, B, n, act);
  check_launch("act_softmax");
}

namespace {
bool ln_aligned(const void* p, int dt) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) & (dt == DT_BF16 ? 7u : 15u)) == 0;
}

// The vector kernel's shape: 4-column chunks, every row start 16-byte (fp32)
// or 8-byte (bf16) aligned, at most 1024 columns.
bool ln_vec_ok(const LnArgs& a) {
  return a.D % 4 == 0 && a.D <= 1024 && a.ld_in % 4 == 0 && a.ld_x % 4 == 0 &&
         a.ld_y % 4 == 0 && a.ld_add % 4 == 0 && ln_aligned(a.in, a.in_dtype) &&
         ln_aligned(a.resid, a.resid_dtype) && ln_aligned(a.xio, DT_F32) &&
         ln_aligned(a.x_out, DT_F32) && ln_aligned(a.y_out, a.y_dtype) &&
         ln_aligned(a.w, DT_F32) && ln_aligned(a.b, DT_F32) && ln_aligned(a.add, DT_F32);
}
}  // namespace

bool ln_takes_parts(const LnArgs& a) {
  return ln_vec_ok(a) && a.resid == nullptr && a.add == nullptr && a.in_dtype == DT_F32 &&
         a.ids == nullptr && a.xio != nullptr && ln_aligned(a.parts, DT_F32) &&
         a.part_stride % 4 == 0 && a.ld_part % 4 == 0 && ln_aligned(a.part_bias, DT_F32);
}

void launch_ln(const LnArgs& a, hipStream_t st) {
  if (a.M <= 0) return;
  require(a.D > 0 && a.D <= 64 * kLnMaxPerLane, "layer_norm: D must be in [1, 4096]");
  require(a.in != nullptr, "layer_norm: null input");
  require(a.ld_in >= a.D, "layer_norm: ld_in < D");
  require(!a.xio || (a.in_dtype == DT_F32 && a.ids == nullptr),
        "layer_norm: residual write-back needs fp32 rows without a gather");
  require(!a.x_out || a.ld_x >= a.D, "layer_norm: ld_x < D");
  require(!a.y_out || a.ld_y >= a.D, "layer_norm: ld_y < D");
  require(!a.add || (a.add_ids && a.add_rows > 0 && a.ld_add >= a.D),
          "layer_norm: an added row needs its row indices, a row count and ld_add >= D");
  const bool vec = ln_vec_ok(a);
  if (a.n_parts > 0) {
    require(a.parts && ln_takes_parts(a),
            "layer_norm: split-K partials need fp32 vector rows written back to xio");
    ln_vec_dispatch<float, PartsRes>(a, st);
  } else if (vec && a.resid == nullptr) {
    a.in_dtype == DT_BF16 ? ln_vec_dispatch<bf16_t, NoRes>(a, st)
                          : ln_vec_dispatch<float, NoRes>(a, st);
  } else if (vec && a.in_dtype == DT_F32) {
    a.resid_dtype == DT_BF16 ? ln_vec_dispatch<float, bf16_t>(a, st)
                             : ln_vec_dispatch<float, float>(a, st);
  } else if (a.in_dtype == DT_BF16) {
    ln_dispatch_res<bf16_t>(a, st);
  } else {
    ln_dispatch_res<float>(a, st);
  }
  check_launch("layer_norm");
}

void launch_rope(void* qkv, int dtype, int64_t M, int64_t ld, const int* pos, int L, int H,
                 int Dh, const float* cos_t, const float* sin_t, hipStream_t st) {
  if (M <= 0) return;
  require(Dh > 0 && Dh % 2 == 0, "rope: head_dim must be even");
  require(ld >= static_cast<int64_t>(3) * H * Dh, "rope: row stride < 3*H*Dh");
  require(pos != nullptr || L > 0, "rope: need positions or L > 0");
  const int64_t total = M * 2 * H * (Dh / 2);
  dim3 block(256), grid(static_cast<unsigned>((total + 255) / 256));
  if (dtype == DT_BF16)
    rope_kernel<bf16_t><<<grid, block, 0, st>>>(static_cast<bf16_t*>(qkv), M, ld, pos, L, H, Dh,
                                                 cos_t, sin_t);
  else
    rope_kernel<float><<<grid, block, 0, st>>>(static_cast<float*>(qkv), M, ld, pos, L, H, Dh,
                                               cos_t, sin_t);
  check_launch("rope");
}

void launch_token_index(const int* seq_start, const int* rows, int B, int* tok_pos, int* tok_seq,
                        hipStream_t st) {
  if (B <= 0) return;
  token_index_kernel<<<B, 256, 0, st>>>(seq_start, rows, tok_pos, tok_seq);
  check_launch("token_index");
}

void launch_add_row_embedding(float* X, int64_t ldx, const float* table, const int* sel,
                              const int* tok_seq, int T, const int* T_dev, int D, hipStream_t st) {
  if (T <= 0) return;
  add_row_embedding_kernel<<<T, 256, 0, st>>>(X, ldx, table, sel, tok_seq, T, T_dev, D);
  check_launch("add_row_embedding");
}

void launch_gather_rows(const float* src, int64_t ld_src, const int* idx, int n, int D,
                        float* dst, int64_t ld_dst, hipStream_t st) {
  if (n <= 0) return;
  gather_rows_kernel<<<n, 256, 0, st>>>(src, ld_src, idx, n, D, dst, ld_dst);
  check_launch("gather_rows");
}

}  // namespace sjh

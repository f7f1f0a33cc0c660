// convert.hip -- device-side conversions of checkpoint tensors while they are
// staged (the checkpoint loader, ckpt.cpp): no fp32 copy of a model is ever
// built on the host.
//
//   widen    bf16 / f16 -> fp32, exact (src/safetensors.cpp:78-107 widens the
//            same way on the host)
//   narrow   fp32 / f16 -> bf16, round to nearest even (the rounding the
//            host path applies to fp32 weights)
//   fp8      per-row e4m3 quantization with the host quantizer's arithmetic
//            (sjh_fp8.hpp): the same codes and scales bit for bit
#include "sjh_common.hpp"
#include "sjh_fp8.hpp"
#include "sjh_host.hpp"
#include "sjh_kernels.hpp"

namespace sjh {

namespace {

__device__ __forceinline__ float half_bits_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Grid-stride loops: the grid is capped (blocks() below), so any element
// count the launchers accept is covered.
__global__ void widen_kernel(const uint16_t* src, int src_dtype, float* dst, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint16_t h = src[i];
    dst[i] = src_dtype == SRC_BF16 ? bf16_to_f32(h) : half_bits_to_f32(h);
  }
}

__global__ void narrow_kernel(const void* src, int src_dtype, bf16_t* dst, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float v = src_dtype == SRC_F32 ? static_cast<const float*>(src)[i]
                                         : half_bits_to_f32(static_cast<const uint16_t*>(src)[i]);
    dst[i] = f32_to_bf16(v);
  }
}

// One workgroup per row: the row's largest magnitude (max is exact in any
// order; NaN never raises it), the scale, then the codes.
constexpr int kQT = 256;
__global__ __launch_bounds__(kQT) void quantize_fp8_kernel(const float* w, int64_t cols,
                                                           uint8_t* q, float* scale) {
  __shared__ float red[kQT / 64];
  const int64_t r = blockIdx.x;
  const float* row = w + r * cols;
  float amax = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kQT) {
    const float v = fabsf(row[c]);
    amax = v > amax ? v : amax;  // a NaN v compares false
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(amax, off, 64);
    amax = o > amax ? o : amax;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = red[0];
  for (int i = 1; i < kQT / 64; ++i) amax = red[i] > amax ? red[i] : amax;
  const float sc = fp8_row_scale(amax);
  if (threadIdx.x == 0) scale[r] = sc;
  uint8_t* qr = q + r * cols;
  for (int64_t c = threadIdx.x; c < cols; c += kQT)
    qr[c] = fp8_e4m3_rne_bits(__float_as_uint(row[c] / sc));
}

// The consumer constants of a folded LayerNorm (launch_ln_fold_consts): one
// wave per W row, sums in double over the row's effective values (bf16, or
// e4m3 code * row scale), then a fixed-order reduction over the lanes.
__device__ __forceinline__ float fp8_e4m3_value(uint8_t c) {
  const int e = (c >> 3) & 15, m = c & 7;
  const float v = e == 0 ? static_cast<float>(m) * 0x1p-9f : (1.0f + static_cast<float>(m) * 0.125f) * __builtin_ldexpf(1.0f, e - 7);
  return (c & 0x80) ? -v : v;
}

__global__ __launch_bounds__(256) void ln_fold_consts_kernel(const void* W, int w_dtype, const float* w_scale,
                                                             int n_w, int K, const float* ln_w,
                                                             const float* ln_b, uint16_t* c1, float* c2) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= n_w) return;  // uniform per wave
  const int nb = K / kLnBlock;
  const double sc = w_dtype == DT_FP8 ? static_cast<double>(w_scale[row]) : 1.0;
  auto wv = [&](int k) -> double {
    const int64_t i = static_cast<int64_t>(row) * K + k;
    return w_dtype == DT_FP8 ? sc * fp8_e4m3_value(static_cast<const uint8_t*>(W)[i])
                             : static_cast<double>(bf16_to_f32(static_cast<const bf16_t*>(W)[i]));
  };
  double cb = 0.0;
  for (int b = 0; b < 8; ++b) {  // a c1 row is one 16-byte MFMA operand row: blocks past nb are zero
    double s = 0.0;
    if (b < nb)
      for (int k = b * kLnBlock + lane; k < (b + 1) * kLnBlock; k += 64) {
        const double w = wv(k);
        s += static_cast<double>(ln_w[k]) * w;
        if (ln_b) cb += static_cast<double>(ln_b[k]) * w;
      }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) c1[static_cast<int64_t>(row) * 8 + b] = f32_to_bf16(static_cast<float>(s));
  }
  if (c2) {
    for (int off = 32; off > 0; off >>= 1) cb += __shfl_xor(cb, off, 64);
    if (lane == 0) c2[row] = static_cast<float>(cb);
  }
}

// 256-thread workgroups for n elements, at most 2^16 of them (the kernels
// loop over the rest)
unsigned blocks(int64_t n) { return static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 65536)); }

}  // namespace

void launch_widen_f32(const void* src, int src_dtype, float* dst, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  require(src_dtype == SRC_BF16 || src_dtype == SRC_F16, "widen: source must be bf16 or f16");
  require(n < (int64_t{1} << 40), "widen: too many elements");
  widen_kernel<<<blocks(n), 256, 0, st>>>(static_cast<const uint16_t*>(src), src_dtype, dst, n);
  check_launch("widen_f32");
}

void launch_narrow_bf16(const void* src, int src_dtype, uint16_t* dst, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  require(src_dtype == SRC_F32 || src_dtype == SRC_F16, "narrow: source must be f32 or f16");
  require(n < (int64_t{1} << 40), "narrow: too many elements");
  narrow_kernel<<<blocks(n), 256, 0, st>>>(src, src_dtype, dst, n);
  check_launch("narrow_bf16");
}

void launch_ln_fold_consts(const void* W, int w_dtype, const float* w_scale, int n_w, int K,
                           const float* ln_w, const float* ln_b, uint16_t* c1, float* c2,
                           hipStream_t st) {
  if (n_w <= 0) return;
  require(W && ln_w && c1, "ln_fold_consts: null argument");
  require(w_dtype == DT_BF16 || (w_dtype == DT_FP8 && w_scale), "ln_fold_consts: bf16 or fp8 weights");
  require(K > 0 && K % kLnBlock == 0 && K / kLnBlock <= kLnMaxBlocks, "ln_fold_consts: K % 256 == 0, K <= 1024");
  require(!ln_b || c2, "ln_fold_consts: a norm bias needs c2");
  ln_fold_consts_kernel<<<static_cast<unsigned>((n_w + 3) / 4), 256, 0, st>>>(W, w_dtype, w_scale, n_w, K, ln_w,
                                                                               ln_b, c1, ln_b ? c2 : nullptr);
  check_launch("ln_fold_consts");
}

void launch_quantize_fp8_rows(const float* w, int64_t rows, int64_t cols, uint8_t* q,
                              float* scale, hipStream_t st) {
  if (rows <= 0 || cols <= 0) return;
  require(rows < (int64_t{1} << 31), "quantize_fp8: too many rows");
  quantize_fp8_kernel<<<static_cast<unsigned>(rows), kQT, 0, st>>>(w, cols, q, scale);
  check_launch("quantize_fp8_rows");
}

}  // namespace sjh

// gemm.hip -- projection GEMMs for gfx950: out[M, N] = epi(A[M, K] . W[N, K]^T).
//
// Fast path (bf16 in, fp32 accumulate): v_mfma_f32_32x32x16_bf16 on
// 128x128x64 workgroup tiles.  256 threads = 4 waves in a 2x2 grid, each wave
// owning a 64x64 sub-tile (2x2 MFMA blocks).  A and W tiles are staged in LDS
// with a 16-byte row pad (double buffered; the next tile's global loads are in
// flight while the current one feeds the MFMAs).  After the K loop the fp32
// accumulators are staged in LDS once more so that the epilogue -- bias,
// GELU/ReLU, residual add into the fp32 stream, RoPE on q/k, GEGLU -- works
// on whole rows with coalesced stores.
//
// Generic path (any shape, fp32 or bf16): 64x64x16 LDS tiles with 4x4 FMA
// micro-tiles per thread and the same LDS-staged epilogue.  It serves the fp32
// parity mode and the shapes the MFMA tiling does not cover (tiny models, the
// scorer's N = 1 projection, LoRA ranks).
#include "sjh_common.hpp"
#include "sjh_host.hpp"
#include "sjh_kernels.hpp"

namespace sjh {

namespace {

// ---- epilogue over an fp32 BMxBN tile staged in LDS (row stride ldcs) ----
template <int BM, int BN, int NT, typename OutT>
__device__ __forceinline__ void tile_epilogue(const float* Cs, int ldcs, int m0, int tile_n,
                                              const GemmArgs g) {
  const int tid = threadIdx.x;
  if (g.epi == EPI_GEGLU) {
    constexpr int HB = BN / 2;
    const int j0 = tile_n * HB;
    OutT* out = static_cast<OutT*>(g.out);
    for (int idx = tid; idx < BM * HB; idx += NT) {
      const int r = idx / HB, c = idx - r * HB;
      const int m = m0 + r, j = j0 + c;
      if (m < g.M && j < g.N) {
        const float in = Cs[r * ldcs + c], gate = Cs[r * ldcs + HB + c];
        store_f32(out + static_cast<int64_t>(m) * g.ldo + j, gelu_erf(in) * gate);
      }
    }
    return;
  }
  const int n0 = tile_n * BN;
  for (int idx = tid; idx < BM * BN; idx += NT) {
    const int r = idx / BN, c = idx - r * BN;
    const int m = m0 + r, n = n0 + c;
    if (m >= g.M || n >= g.N) continue;
    float v = Cs[r * ldcs + c];
    if (g.epi == EPI_RESID) {
      if (g.bias) v += g.bias[n];
      g.X[static_cast<int64_t>(m) * g.ldx + n] += v;
      continue;
    }
    if (g.epi == EPI_ROPE) {
      if (n < 2 * g.rope_dim) {
        const int hd = g.head_dim, half = hd >> 1;
        const int dd = n % hd;
        const int64_t p = g.pos[m];
        if (dd < half) {
          const float x1 = Cs[r * ldcs + c + half];
          const float cs = g.rope_cos[p * half + dd], sn = g.rope_sin[p * half + dd];
          v = v * cs - x1 * sn;
        } else {
          const int d2 = dd - half;
          const float x0 = Cs[r * ldcs + c - half];
          const float cs = g.rope_cos[p * half + d2], sn = g.rope_sin[p * half + d2];
          v = v * cs + x0 * sn;
        }
      }
    } else {
      if (g.bias) v += g.bias[n];
      if (g.act == 1)
        v = gelu_erf(v);
      else if (g.act == 2)
        v = fmaxf(v, 0.f);
    }
    store_f32(static_cast<OutT*>(g.out) + static_cast<int64_t>(m) * g.ldo + n, v);
  }
}

// W row feeding tile row i of column tile tile_n (GEGLU: first half of the
// tile = input rows, second half = gate rows of the reference's [2F, K] Wi).
template <int BN>
__device__ __forceinline__ int64_t w_row(const GemmArgs g, int tile_n, int i) {
  if (g.epi == EPI_GEGLU) {
    constexpr int HB = BN / 2;
    const int j = tile_n * HB + (i < HB ? i : i - HB);
    const int jc = j < g.N ? j : g.N - 1;
    return i < HB ? jc : static_cast<int64_t>(g.N) + jc;
  }
  const int n = tile_n * BN + i;
  return n < g.N ? n : g.N - 1;
}

// ------------------------------------------------------------------ MFMA bf16
constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kLdsK = kBK + 8;  // padded LDS row (elements): 144 B
constexpr int kStageElems = (kBM + kBN) * kLdsK;
constexpr int kLdsBytes = 2 * kStageElems * 2;  // two stages of bf16
constexpr int kLdc = kBN + 4;
static_assert(kBM * kLdc * 4 <= kLdsBytes, "epilogue tile must fit the staging LDS");

template <typename OutT>
__global__ __launch_bounds__(256) void gemm_bf16_mfma_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) char smem[kLdsBytes];
  bf16_t* stage = reinterpret_cast<bf16_t*>(smem);

  const int tile_n = blockIdx.x, tile_m = blockIdx.y;
  const int m0 = tile_m * kBM;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hb = lane >> 5;

  const bf16_t* A = static_cast<const bf16_t*>(g.A);
  const bf16_t* W = static_cast<const bf16_t*>(g.W);

  // global -> register assignment: 16-byte chunks, 8 per 64-element row; a
  // thread moves rows r0 + 32*i (i < 4) at k-chunk kc of both operands.
  constexpr int kChunks = kBM * kBK / 8 / 256;  // 4 (A) and 4 (W)
  static_assert(kBM == kBN, "A and W tiles share the chunk assignment");
  const int r0 = tid >> 3, kc = tid & 7;
  int64_t a_off[kChunks], w_off[kChunks];
#pragma unroll
  for (int i = 0; i < kChunks; ++i) {
    const int row = r0 + 32 * i;
    a_off[i] = static_cast<int64_t>(min(m0 + row, g.M - 1)) * g.lda + kc * 8;
    w_off[i] = w_row<kBN>(g, tile_n, row) * g.ldw + kc * 8;
  }
  const int lds_off = r0 * kLdsK + kc * 8;  // + 32*i rows

  u32x4_t ra[kChunks], rw[kChunks];
  static_assert(kChunks == 4, "the load/store macros below move 4 chunks per operand");
#define SJH_LD1(i, k0)                                                   \
  ra[i] = *reinterpret_cast<const u32x4_t*>(A + a_off[i] + (k0));          \
  rw[i] = *reinterpret_cast<const u32x4_t*>(W + w_off[i] + (k0));
#define SJH_GEMM_LOAD(k0) \
  SJH_LD1(0, k0) SJH_LD1(1, k0) SJH_LD1(2, k0) SJH_LD1(3, k0)
#define SJH_ST1(i, buf)                                                                     \
  *reinterpret_cast<u32x4_t*>(stage + (buf) * kStageElems + lds_off + 32 * (i) * kLdsK) = ra[i]; \
  *reinterpret_cast<u32x4_t*>(stage + (buf) * kStageElems + kBM * kLdsK + lds_off +             \
                            32 * (i) * kLdsK) = rw[i];
#define SJH_GEMM_STORE(buf) \
  SJH_ST1(0, buf) SJH_ST1(1, buf) SJH_ST1(2, buf) SJH_ST1(3, buf)

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  SJH_GEMM_LOAD(0)
  SJH_GEMM_STORE(0)
  __syncthreads();
  const int nk = g.K / kBK;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      const int kn = (kt + 1) * kBK;
      SJH_GEMM_LOAD(kn)
    }
    const bf16_t* As = stage + cur * kStageElems + (wm * 64 + l32) * kLdsK + hb * 8;
    const bf16_t* Ws = stage + cur * kStageElems + kBM * kLdsK + (wn * 64 + l32) * kLdsK + hb * 8;
#pragma unroll
    for (int s = 0; s < kBK / 16; ++s) {
      bf16x8_t af[2], bw[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const bf16x8_t*>(As + i * 32 * kLdsK + s * 16);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bw[j] = *reinterpret_cast<const bf16x8_t*>(Ws + j * 32 * kLdsK + s * 16);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bw[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) {
      SJH_GEMM_STORE(cur ^ 1)
    }
    __syncthreads();
  }
#undef SJH_LD1
#undef SJH_ST1
#undef SJH_GEMM_LOAD
#undef SJH_GEMM_STORE

  // accumulator layout of a 32x32 block: lane l holds column l%32 and rows
  // 8*(e/4) + 4*(l/32) + e%4 for e = 0..15.
  float* Cs = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wm * 64 + i * 32 + 8 * (e >> 2) + 4 * hb + (e & 3);
        const int col = wn * 64 + j * 32 + l32;
        Cs[row * kLdc + col] = acc[i][j][e];
      }
  __syncthreads();
  tile_epilogue<kBM, kBN, 256, OutT>(Cs, kLdc, m0, tile_n, g);
}

// ------------------------------------------------------------------ generic
constexpr int gBM = 64, gBN = 64, gBK = 16;
constexpr int gLdc = gBN + 4;

template <typename InT, typename OutT>
__global__ __launch_bounds__(256) void gemm_generic_kernel(GemmArgs g) {
  constexpr int kStage = 2 * gBK * (gBM + 1);  // As[k][m] and Ws[k][n]
  constexpr int kFloats = kStage > gBM * gLdc ? kStage : gBM * gLdc;
  __shared__ float smem[kFloats];
  float* As = smem;
  float* Ws = smem + gBK * (gBM + 1);

  const int tile_n = blockIdx.x, tile_m = blockIdx.y;
  const int m0 = tile_m * gBM;
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const InT* A = static_cast<const InT*>(g.A);
  const InT* W = static_cast<const InT*>(g.W);

  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;

  for (int k0 = 0; k0 < g.K; k0 += gBK) {
    // 64 rows x 16 k per operand: 1024 elements, 4 per thread
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, row = c >> 4, kk = c & 15;
      const int k = k0 + kk;
      const int m = m0 + row;
      float av = 0.f, wv = 0.f;
      if (k < g.K) {
        if (m < g.M) av = load_f32(A + static_cast<int64_t>(m) * g.lda + k);
        wv = load_f32(W + w_row<gBN>(g, tile_n, row) * g.ldw + k);
      }
      As[kk * (gBM + 1) + row] = av;
      Ws[kk * (gBN + 1) + row] = wv;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < gBK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk * (gBM + 1) + ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Ws[kk * (gBN + 1) + tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
    }
    __syncthreads();
  }
  float* Cs = smem;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) Cs[(ty * 4 + i) * gLdc + tx * 4 + j] = acc[i][j];
  __syncthreads();
  tile_epilogue<gBM, gBN, 256, OutT>(Cs, gLdc, m0, tile_n, g);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename InT>
void launch_generic(const GemmArgs& g, hipStream_t st) {
  const int ntiles = g.epi == EPI_GEGLU ? (g.N + gBN / 2 - 1) / (gBN / 2) : (g.N + gBN - 1) / gBN;
  dim3 grid(ntiles, (g.M + gBM - 1) / gBM), block(256);
  if (g.out_dtype == DT_BF16)
    gemm_generic_kernel<InT, bf16_t><<<grid, block, 0, st>>>(g);
  else
    gemm_generic_kernel<InT, float><<<grid, block, 0, st>>>(g);
}

}  // namespace

void launch_gemm(const GemmArgs& g, hipStream_t st) {
  if (g.M <= 0 || g.N <= 0) return;
  require(g.K > 0, "gemm: K must be positive");
  require(g.A && g.W, "gemm: null operand");
  require(g.lda >= g.K && g.ldw >= g.K, "gemm: leading dimension < K");
  switch (g.epi) {
    case EPI_STORE:
      require(g.out && g.ldo >= g.N, "gemm: STORE needs out with ldo >= N");
      break;
    case EPI_RESID:
      require(g.X && g.ldx >= g.N, "gemm: RESID needs X with ldx >= N");
      break;
    case EPI_ROPE:
      require(g.out && g.ldo >= g.N, "gemm: ROPE needs out with ldo >= N");
      require(g.pos && g.rope_cos && g.rope_sin, "gemm: ROPE needs positions and tables");
      require(g.head_dim > 0 && g.head_dim % 2 == 0 && g.rope_dim % g.head_dim == 0 &&
                  2 * g.rope_dim <= g.N,
              "gemm: ROPE head layout");
      break;
    case EPI_GEGLU:
      require(g.out && g.ldo >= g.N, "gemm: GEGLU needs out with ldo >= N (= F)");
      break;
    default:
      fail("gemm: unknown epilogue");
  }
  const bool mfma = g.in_dtype == DT_BF16 && g.K % kBK == 0 && g.lda % 8 == 0 &&
                    g.ldw % 8 == 0 && aligned16(g.A) && aligned16(g.W) &&
                    (g.epi != EPI_ROPE || kBN % g.head_dim == 0) &&
                    (g.epi != EPI_GEGLU || g.N % (kBN / 2) == 0);
  if (g.epi == EPI_ROPE && !mfma)
    require(gBN % g.head_dim == 0, "gemm: ROPE epilogue needs head_dim dividing 64");
  if (mfma) {
    const int ntiles =
        g.epi == EPI_GEGLU ? g.N / (kBN / 2) : (g.N + kBN - 1) / kBN;
    dim3 grid(ntiles, (g.M + kBM - 1) / kBM), block(256);
    if (g.out_dtype == DT_BF16)
      gemm_bf16_mfma_kernel<bf16_t><<<grid, block, 0, st>>>(g);
    else
      gemm_bf16_mfma_kernel<float><<<grid, block, 0, st>>>(g);
    check_launch("gemm_bf16_mfma");
    return;
  }
  if (g.in_dtype == DT_BF16)
    launch_generic<bf16_t>(g, st);
  else
    launch_generic<float>(g, st);
  check_launch("gemm_generic");
}

}  // namespace sjh

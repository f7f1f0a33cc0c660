// gemm.hip -- projection GEMMs for gfx950: out[M, N] = epi(A[M, K] . W[N, K]^T).
//
// Fast path (bf16 in, fp32 accumulate): v_mfma_f32_32x32x16_bf16 on block
// tiles of up to 256x256 (16 waves of 64x64 for the throughput shapes).  A
// and W tiles move from HBM into an LDS ring with direct-to-LDS loads
// (global_load_lds_dwordx4, no register staging), XOR-swizzled so that the
// MFMA operand reads are free of bank conflicts.  The epilogue -- bias,
// GELU/ReLU, residual add into the fp32 stream, RoPE on q/k, GEGLU -- works on
// the accumulators in registers, and the tile order is XCD-aware.
//
// Generic path (any shape, fp32 or bf16): 64x64x16 LDS tiles with 4x4 FMA
// micro-tiles per thread and the same LDS-staged epilogue.  It serves the fp32
// parity mode and the shapes the MFMA tiling does not cover (tiny models, the
// scorer's N = 1 projection, LoRA ranks).
#include <algorithm>
#include <type_traits>

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
        store_f32(out + static_cast<int64_t>(m) * g.ldo + j, gelu_out<OutT>(in) * gate);
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
        const int64_t p = min(max(g.pos[m], 0), g.rope_rows - 1);
        if (dd < half) {
          const float x1 = Cs[r * ldcs + c + half];
          const float cs = g.rope_cos[p * half + dd], sn = g.rope_sin[p * half + dd];
          v = rope_lo(v, x1, cs, sn);
        } else {
          const int d2 = dd - half;
          const float x0 = Cs[r * ldcs + c - half];
          const float cs = g.rope_cos[p * half + d2], sn = g.rope_sin[p * half + d2];
          v = rope_hi(x0, v, cs, sn);
        }
        if (n < g.rope_dim) v *= g.q_scale;
      }
    } else {
      if (g.bias) v += g.bias[n];
      if (g.act == 1)
        v = gelu_out<OutT>(v);
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
//
// Block tile BM x BN x 64 with WGM x WGN waves; each wave owns a
// (BM/WGM) x (BN/WGN) sub-tile made of TI x TJ blocks of
// v_mfma_f32_32x32x16_bf16.  Accumulator layout of one 32x32 block: lane l
// holds column l % 32 and rows 8*(e/4) + 4*(l/32) + e%4, e = 0..15.
//
// The epilogue runs on the accumulators in registers:
//   STORE  bias + GELU/ReLU, one element per (lane, e);
//   RESID  X += acc (+ bias) on the fp32 residual stream;
//   ROPE   head_dim 64: the two halves of a head (columns d and d + 32) are
//          the same lane and register in blocks j and j + 1, so rotate-half
//          needs no data movement;
//   GEGLU  the block's W rows are arranged so that wave column wn's first
//          TJ/2 blocks are input rows and its last TJ/2 blocks the gate rows
//          of the same outputs: out = gelu(acc[j]) * acc[j + TJ/2].
constexpr int kBK = 64;  // K must be a multiple of this for the MFMA path

// Workgroups are handed to the 8 XCDs round-robin (id % 8).  Renumber them
// so that each XCD receives a contiguous run of tiles, N fastest: the tiles
// of one A row panel then share that XCD's L2.
__device__ __forceinline__ int xcd_tile(int bid, int nblocks) {
  const int xcd = bid & 7, local = bid >> 3;
  const int per = nblocks >> 3, rem = nblocks & 7;
  return xcd * per + min(xcd, rem) + local;
}

// W row staged at tile row i (0 <= i < BN) of column tile tile_n.
template <int BN, int WN, int EPI>
__device__ __forceinline__ int64_t mfma_w_row(const GemmArgs& g, int tile_n, int i) {
  if constexpr (EPI == EPI_GEGLU) {
    constexpr int half = WN / 2;
    const int wn = i / WN, within = i - wn * WN;
    int o = tile_n * (BN / 2) + wn * half + (within < half ? within : within - half);
    o = o < g.N ? o : g.N - 1;
    return within < half ? o : static_cast<int64_t>(g.N) + o;
  } else if constexpr (EPI == EPI_ROPE && BN == 32) {
    // 32-column RoPE tiles (head_dim 64): tile_n = 2 h + c takes dims
    // 16 c + [0, 16) of head h (rows i < 16) and their rotation partners 32
    // higher (rows i >= 16), so each pair meets in one tile
    const int n = (tile_n >> 1) * 64 + (tile_n & 1) * 16 + (i & 15) + (i & 16) * 2;
    return n < g.N ? n : g.N - 1;
  } else {
    const int n = tile_n * BN + i;
    return n < g.N ? n : g.N - 1;
  }
}

// Marks a loaded value as used on every path.  A load whose result some path
// never reads (rows past M skip their stores) stays pending in the compiler's
// bookkeeping, which then drains the whole load ring (vmcnt(0)) before the
// next reuse of its register in the main loop.
template <typename T>
__device__ __forceinline__ void consume(const T& v) {
  asm volatile("" ::"v"(v));
}

// The arguments a kernel works with: M becomes the device row count when
// the launch carries one (GemmArgs::M_dev).
__device__ __forceinline__ GemmArgs resolve_rows(const GemmArgs& g0) {
  GemmArgs g = g0;
  if (g.M_dev) g.M = *g.M_dev;
  return g;
}

// The value lane l ^ 16 holds (v_permlane16_swap of v with itself hands
// rows 0 and 2 of 16 lanes to rows 1 and 3 in its first result and rows 1
// and 3 to rows 0 and 2 in its second).  hi_row: lane & 16.
__device__ __forceinline__ float swap16(float v, bool hi_row) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(hi_row ? r[0] : r[1]);
}

// Epilogue on the accumulators in registers (see the comment above).
// TAB_LDS: the RoPE table rows of the tile are staged in LDS at rope_tab
// (given whenever the tile has rotated columns).
template <int BM, int BN, int WM, int WN, int TI, int TJ, int EPI, typename OutT, bool TAB_LDS = false>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& g, f32x16_t (&acc)[TI][TJ], int m0,
                                              int tile_n, int wm, int wn, int l32, int hb,
                                              const char* rope_tab = nullptr) {
  const int row_base = m0 + wm * WM + 4 * hb;
  if constexpr (EPI == EPI_GEGLU && TJ == 1) {
    // one 32-column block (see mfma_w_row): lane c < 16 holds the input of
    // output tile_n * BN / 2 + wn * WN / 2 + c, lane c + 16 its gate
    static_assert(WN == 32, "GEGLU with one column block per wave");
    OutT* out = static_cast<OutT*>(g.out);
    const bool hi = l32 >= 16;
    const int col = tile_n * (BN / 2) + wn * (WN / 2) + (l32 & 15);
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float own = acc[i][0][e];
        const float gate = swap16(own, hi);  // every lane takes part
        const int m = row_base + i * 32 + 8 * (e >> 2) + (e & 3);
        if (!hi && m < g.M && col < g.N)
          store_f32(out + static_cast<int64_t>(m) * g.ldo + col, gelu_out<OutT>(own) * gate);
      }
  } else if constexpr (EPI == EPI_GEGLU) {
    OutT* out = static_cast<OutT*>(g.out);
    const int c0 = tile_n * (BN / 2) + wn * (WN / 2) + l32;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = row_base + i * 32 + 8 * (e >> 2) + (e & 3);
        if (m >= g.M) continue;
        OutT* orow = out + static_cast<int64_t>(m) * g.ldo;
#pragma unroll
        for (int j = 0; j < TJ / 2; ++j) {
          const int col = c0 + j * 32;
          if (col < g.N) store_f32(orow + col, gelu_out<OutT>(acc[i][j][e]) * acc[i][j + TJ / 2][e]);
        }
      }
  } else if constexpr (EPI == EPI_RESID) {
    // X += acc (+ bias).  The X reads of a group of RG rows are all issued
    // before the first add, so a group costs one memory round trip rather
    // than one per element.  Addresses are the wave's uniform corner plus one
    // 32-bit byte offset per access; elements past M or N are skipped.
    constexpr int RG = 8;
    const int c0 = tile_n * BN + wn * WN;
    const int rw = m0 + wm * WM;  // the wave's first row
    const char* xw = reinterpret_cast<const char*>(g.X + static_cast<int64_t>(rw) * g.ldx + c0);
    const uint32_t ld4 = static_cast<uint32_t>(g.ldx) * 4u;
    const uint32_t lo = 4 * hb * ld4 + l32 * 4;
    const bool rfull = rw + WM <= g.M, cfull = c0 + WN <= g.N;  // uniform
    float bv[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) bv[j] = g.bias ? g.bias[min(c0 + j * 32 + l32, g.N - 1)] : 0.f;
    auto body = [&](auto checked) {  // checked: the wave's rows or columns run past M or N
      auto in = [&](int r, int j) {
        if constexpr (decltype(checked)::value)
          return rw + r + 4 * hb < g.M && c0 + j * 32 + l32 < g.N;
        return true;
      };
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int e0 = 0; e0 < 16; e0 += RG) {
          float xv[RG][TJ];
#pragma unroll
          for (int e = 0; e < RG; ++e) {
            const int r = i * 32 + 8 * ((e0 + e) >> 2) + ((e0 + e) & 3);
            const char* xr = xw + static_cast<uint32_t>(r * ld4 + lo);
#pragma unroll
            for (int j = 0; j < TJ; ++j)
              xv[e][j] = in(r, j) ? *reinterpret_cast<const float*>(xr + j * 128) : 0.f;
          }
#pragma unroll
          for (int e = 0; e < RG; ++e) {
            const int r = i * 32 + 8 * ((e0 + e) >> 2) + ((e0 + e) & 3);
            char* xr = const_cast<char*>(xw) + static_cast<uint32_t>(r * ld4 + lo);
#pragma unroll
            for (int j = 0; j < TJ; ++j)
              if (in(r, j)) *reinterpret_cast<float*>(xr + j * 128) = xv[e][j] + (acc[i][j][e0 + e] + bv[j]);
          }
        }
    };
    if (rfull && cfull)
      body(std::false_type{});
    else
      body(std::true_type{});
  } else if constexpr (EPI == EPI_ROPE && BN == 32) {
    // 32-column tiles (see mfma_w_row): lane c < 16 holds dim d = 16 (tile_n
    // & 1) + c of head tile_n >> 1, lane c + 16 dim d + 32; each takes its
    // partner by a lane swap and writes its own output column.  A group of
    // 16 rows per lane gathers its positions, then its table entries.
    static_assert(WN == 32 && TJ == 1 && TI == 1, "one 32 x 32 block per wave");
    const bool hi = l32 >= 16;
    const int col = (tile_n >> 1) * 64 + (tile_n & 1) * 16 + (l32 & 15) + (hi ? 32 : 0);
    const int d = (tile_n & 1) * 16 + (l32 & 15);
    const bool rot = (tile_n >> 1) * 64 < 2 * g.rope_dim, qh = (tile_n >> 1) * 64 < g.rope_dim;  // uniform
    OutT* out = static_cast<OutT*>(g.out);
    float cs[16], sn[16];
    if (rot) {
      int p[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) p[e] = g.pos[min(row_base + 8 * (e >> 2) + (e & 3), g.M - 1)];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t tb = static_cast<int64_t>(min(max(p[e], 0), g.rope_rows - 1)) * 32 + d;
        cs[e] = g.rope_cos[tb];
        sn[e] = g.rope_sin[tb];
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        consume(cs[e]);
        consume(sn[e]);
      }
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float own = acc[0][0][e];
      const float partner = swap16(own, hi);  // every lane takes part
      const int m = row_base + 8 * (e >> 2) + (e & 3);
      float v = own;
      if (rot) {
        v = hi ? rope_hi(partner, own, cs[e], sn[e]) : rope_lo(own, partner, cs[e], sn[e]);
        if (qh) v *= g.q_scale;
      }
      if (m < g.M && col < g.N) store_f32(out + static_cast<int64_t>(m) * g.ldo + col, v);
    }
  } else if constexpr (EPI == EPI_ROPE) {
    // head_dim 64 (checked by the launcher): block j holds dims [0, 32) of a
    // head when j is even and dims [32, 64) when odd; its partner is j ^ 1.
    // Table entries of a group of RG rows are fetched together: from the
    // unit's table rows in LDS (rope_tab) or, without them, gathered through
    // the positions (two memory round trips per group, not two per row; a
    // wave with one 32-row block takes its 16 rows per lane in one group).
    // Addresses are the wave's uniform corner plus one 32-bit byte offset per
    // access; elements past M or N are skipped.
    static_assert(TJ % 2 == 0, "RoPE pairs need an even number of column blocks");
    constexpr int RG = (!TAB_LDS && TI == 1) ? 16 : 8;
    constexpr int EB = sizeof(OutT);
    const int c0 = tile_n * BN + wn * WN;
    const int rw = m0 + wm * WM;  // the wave's first row
    const char* ow = reinterpret_cast<const char*>(static_cast<OutT*>(g.out) + static_cast<int64_t>(rw) * g.ldo + c0);
    const uint32_t ldb = static_cast<uint32_t>(g.ldo) * EB;
    const uint32_t lo = 4 * hb * ldb + l32 * EB;
    const bool rfull = rw + WM <= g.M, cfull = c0 + WN <= g.N;  // uniform
    const bool wave_rot = c0 < 2 * g.rope_dim;  // rotated blocks come first in a row
    auto body = [&](auto checked) {  // checked: the wave's rows or columns run past M or N
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int e0 = 0; e0 < 16; e0 += RG) {
          float cs[RG], sn[RG];
          if (wave_rot) {
            if constexpr (TAB_LDS) {
              // the unit's table rows: cos at row * 128, sin 32 KB on
              typedef __attribute__((address_space(3))) const float lds_f32;
              lds_f32* t = (lds_f32*)(rope_tab + (rw - m0 + 4 * hb + i * 32) * 128 + l32 * 4);
#pragma unroll
              for (int e = 0; e < RG; ++e) {
                const int r = 8 * ((e0 + e) >> 2) + ((e0 + e) & 3);
                cs[e] = t[r * 32];
                sn[e] = t[r * 32 + 8192];
              }
            } else {
              int p[RG];
#pragma unroll
              for (int e = 0; e < RG; ++e) {
                const int m = min(rw + 4 * hb + i * 32 + 8 * ((e0 + e) >> 2) + ((e0 + e) & 3), g.M - 1);
                p[e] = g.pos[m];
              }
#pragma unroll
              for (int e = 0; e < RG; ++e) {
                const int64_t tb = static_cast<int64_t>(min(max(p[e], 0), g.rope_rows - 1)) * 32 + l32;
                cs[e] = g.rope_cos[tb];
                sn[e] = g.rope_sin[tb];
              }
            }
#pragma unroll
            for (int e = 0; e < RG; ++e) {
              consume(cs[e]);
              consume(sn[e]);
            }
          }
#pragma unroll
          for (int e = 0; e < RG; ++e) {
            const int r = i * 32 + 8 * ((e0 + e) >> 2) + ((e0 + e) & 3);
            if (decltype(checked)::value && rw + r + 4 * hb >= g.M) continue;
            char* orow = const_cast<char*>(ow) + static_cast<uint32_t>(r * ldb + lo);
#pragma unroll
            for (int j = 0; j < TJ; j += 2) {
              const int col = c0 + j * 32 + l32;
              if (decltype(checked)::value && col >= g.N) continue;
              float x0 = acc[i][j][e0 + e], x1 = acc[i][j + 1][e0 + e];
              if (wave_rot && c0 + j * 32 < 2 * g.rope_dim) {
                const float r0 = rope_lo(x0, x1, cs[e], sn[e]);
                const float r1 = rope_hi(x0, x1, cs[e], sn[e]);
                x0 = r0;
                x1 = r1;
                if (c0 + j * 32 < g.rope_dim) {  // a q head: attention's scale folded in
                  x0 *= g.q_scale;
                  x1 *= g.q_scale;
                }
              }
              store_f32(reinterpret_cast<OutT*>(orow + j * 32 * EB), x0);
              if (!decltype(checked)::value || col + 32 < g.N) store_f32(reinterpret_cast<OutT*>(orow + (j + 1) * 32 * EB), x1);
            }
          }
        }
    };
    if (rfull && cfull)
      body(std::false_type{});
    else
      body(std::true_type{});
  } else {
    // out = act(acc + bias).  Addresses are the wave's uniform corner plus
    // one 32-bit byte offset per access; the activation and the bounds checks
    // (rows or columns of the wave past M or N) are chosen once per wave.
    constexpr int EB = sizeof(OutT);
    const int c0 = tile_n * BN + wn * WN;
    const int rw = m0 + wm * WM;  // the wave's first row
    const char* ow = reinterpret_cast<const char*>(static_cast<OutT*>(g.out) + static_cast<int64_t>(rw) * g.ldo + c0);
    const uint32_t ldb = static_cast<uint32_t>(g.ldo) * EB;
    const uint32_t lo = 4 * hb * ldb + l32 * EB;
    const bool rfull = rw + WM <= g.M, cfull = c0 + WN <= g.N;  // uniform
    float bv[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) bv[j] = g.bias ? g.bias[min(c0 + j * 32 + l32, g.N - 1)] : 0.f;
    auto body = [&](auto checked, auto act_tag) {
      constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = i * 32 + 8 * (e >> 2) + (e & 3);
          if (decltype(checked)::value && rw + r + 4 * hb >= g.M) continue;
          char* orow = const_cast<char*>(ow) + static_cast<uint32_t>(r * ldb + lo);
#pragma unroll
          for (int j = 0; j < TJ; ++j) {
            if (decltype(checked)::value && c0 + j * 32 + l32 >= g.N) continue;
            float v = acc[i][j][e] + bv[j];
            if constexpr (ACT == 1)
              v = gelu_out<OutT>(v);
            else if constexpr (ACT == 2)
              v = fmaxf(v, 0.f);
            store_f32(reinterpret_cast<OutT*>(orow + j * 32 * EB), v);
          }
        }
    };
    auto by_act = [&](auto checked) {
      if (g.act == 1)
        body(checked, std::integral_constant<int, 1>{});
      else if (g.act == 2)
        body(checked, std::integral_constant<int, 2>{});
      else
        body(checked, std::integral_constant<int, 0>{});
    };
    if (rfull && cfull)
      by_act(std::false_type{});
    else
      by_act(std::true_type{});
  }
}

// ---- LayerNorm folded across a residual GEMM and the next GEMM -------------
// (GemmArgs::ln_y / ln_stats_in).  Both sides run in the persistent kernel's
// direct accumulator layout (lane l holds column l % 32 of each 32x32 block
// and rows 8 (e / 4) + 4 (l / 32) + e % 4) or, for the consumer, the
// transposed one (lane l holds row l % 32).

// Reduce-scatter of 16 row sums over the 32 lanes of a wave half (one
// column each): every stage pairs the lanes that differ in one bit (16, 8, 4,
// 2), each keeps half of the slots and adds its partner's value for them.
// Then lanes 2k and 2k + 1 hold the whole sum of slot k (in both).  Float
// addition is commutative, so every slot's sum is the same function of its
// 32 values, whichever slot (row) it is.
__device__ __forceinline__ float rows16_sum(float (&v)[16], int l32) {
#pragma unroll
  for (int p = 0; p < 8; ++p) {  // lanes l and l ^ 16: one swap moves both halves
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[p]), __float_as_uint(v[p + 8]), false, false);
    v[p] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  auto stage = [&](auto c_tag, auto s_tag) {
    constexpr int C = decltype(c_tag)::value, S = decltype(s_tag)::value;
    const bool up = (l32 & S) != 0;
#pragma unroll
    for (int p = 0; p < C / 2; ++p) {
      const float lo = v[p], hi = v[p + C / 2];
      const float keep = up ? hi : lo, send = up ? lo : hi;
      v[p] = keep + __shfl_xor(send, S, 64);
    }
  };
  stage(std::integral_constant<int, 8>{}, std::integral_constant<int, 8>{});
  stage(std::integral_constant<int, 4>{}, std::integral_constant<int, 4>{});
  stage(std::integral_constant<int, 2>{}, std::integral_constant<int, 2>{});
  return v[0] + __shfl_xor(v[0], 1, 64);
}
// The row (within a 32-row block) of the slot that lane l32 of half hb holds
// after rows16_sum: slot k = l32 / 2 is row 8 (k / 4) + 4 hb + k % 4.
__device__ __forceinline__ int rows16_row(int l32, int hb) {
  const int k = l32 >> 1;
  return 8 * (k >> 2) + 4 * hb + (k & 3);
}

// Producer: the residual epilogue (X += acc + bias, the same arithmetic as
// gemm_epilogue's) that also writes the next LayerNorm's input rows and the
// row moments of this tile's 256 columns.  Two passes over the registers:
// block means, then squared deviations from them; each reduces over the 64
// columns of a wave (rows16_sum) and over the WGN waves of the tile through
// LDS in a fixed order.  Every wave of the workgroup calls it (waves with no
// rows in a half unit with busy = false): it holds three barriers.
// red: WGN * BM floats, mu: BM floats of LDS; tid: the thread's index in the
// workgroup (passed in, so that the kernel need not keep threadIdx.x live
// through its K loop).
template <int BM, int BN, int WM, int WN, int TI, int TJ, int WGN>
__device__ __forceinline__ void resid_ln_epilogue(const GemmArgs& g, f32x16_t (&acc)[TI][TJ], int m0,
                                                  int unit_rows, int tile_n, int wm, int wn, int l32,
                                                  int hb, int tid, bool busy, float* red, float* mu) {
  static_assert(BN == kLnBlock, "one LayerNorm block per column tile");
  const int c0 = tile_n * BN + wn * WN;
  const int rw = m0 + wm * WM;  // the wave's first row
  const uint32_t ld4 = static_cast<uint32_t>(g.ldx) * 4u, ld2 = static_cast<uint32_t>(g.ldx) * 2u;
  char* xw = reinterpret_cast<char*>(g.X + static_cast<int64_t>(rw) * g.ldx + c0);
  char* yw = reinterpret_cast<char*>(static_cast<bf16_t*>(g.ln_y) + static_cast<int64_t>(rw) * g.ldx + c0);
  const uint32_t lo4 = 4 * hb * ld4 + l32 * 4, lo2 = 4 * hb * ld2 + l32 * 2;
  const int rows_in = min(g.M - rw, WM);  // the wave's rows below M (may be <= 0)
  if (busy) {
    float bv[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) bv[j] = g.bias ? g.bias[c0 + j * 32 + l32] : 0.f;
    constexpr int RG = 4;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int e0 = 0; e0 < 16; e0 += RG) {
        float xv[RG][TJ];
#pragma unroll
        for (int e = 0; e < RG; ++e) {
          const int r = i * 32 + 8 * ((e0 + e) >> 2) + ((e0 + e) & 3) + 4 * hb;
#pragma unroll
          for (int j = 0; j < TJ; ++j)
            xv[e][j] = r < rows_in ? *reinterpret_cast<const float*>(xw + static_cast<uint32_t>((r - 4 * hb) * ld4 + lo4) + j * 128) : 0.f;
        }
#pragma unroll
        for (int e = 0; e < RG; ++e) {
          const int r = i * 32 + 8 * ((e0 + e) >> 2) + ((e0 + e) & 3) + 4 * hb;
#pragma unroll
          for (int j = 0; j < TJ; ++j) {
            acc[i][j][e0 + e] = xv[e][j] + (acc[i][j][e0 + e] + bv[j]);
            if (r < rows_in)
              *reinterpret_cast<float*>(xw + static_cast<uint32_t>((r - 4 * hb) * ld4 + lo4) + j * 128) = acc[i][j][e0 + e];
          }
        }
      }
    // pass 1: row sums over the wave's columns
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      float v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        v[e] = acc[i][0][e];
#pragma unroll
        for (int j = 1; j < TJ; ++j) v[e] += acc[i][j][e];
      }
      const float sum = rows16_sum(v, l32);
      if ((l32 & 1) == 0) red[wn * BM + wm * WM + i * 32 + rows16_row(l32, hb)] = sum;
    }
  }
  __syncthreads();
  if (tid < BM) {
    float s = red[tid];
#pragma unroll
    for (int w = 1; w < WGN; ++w) s += red[w * BM + tid];
    mu[tid] = s * (1.0f / BN);
  }
  __syncthreads();
  if (busy) {
    float lw[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) lw[j] = g.ln_w[c0 + j * 32 + l32];
#pragma unroll
    for (int i = 0; i < TI; ++i) {
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const f32x4_t m4 = *reinterpret_cast<const f32x4_t*>(mu + wm * WM + i * 32 + 8 * e4 + 4 * hb);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int e = 4 * e4 + t;
          const int r = i * 32 + 8 * e4 + t + 4 * hb;
#pragma unroll
          for (int j = 0; j < TJ; ++j) {
            acc[i][j][e] -= m4[t];
            if (r < rows_in)
              *reinterpret_cast<bf16_t*>(yw + static_cast<uint32_t>((r - 4 * hb) * ld2 + lo2) + j * 64) =
                  f32_to_bf16(acc[i][j][e] * lw[j]);
          }
        }
      }
      // pass 2: squared deviations
      float v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        v[e] = acc[i][0][e] * acc[i][0][e];
#pragma unroll
        for (int j = 1; j < TJ; ++j) v[e] = __builtin_fmaf(acc[i][j][e], acc[i][j][e], v[e]);
      }
      const float ss = rows16_sum(v, l32);
      if ((l32 & 1) == 0) red[wn * BM + wm * WM + i * 32 + rows16_row(l32, hb)] = ss;
    }
  }
  __syncthreads();
  if (tid < unit_rows && m0 + tid < g.M) {
    float m2 = red[tid];
#pragma unroll
    for (int w = 1; w < WGN; ++w) m2 += red[w * BM + tid];
    const int nbn = g.N / kLnBlock;
    typedef __attribute__((ext_vector_type(2))) float f2_t;
    *reinterpret_cast<f2_t*>(g.ln_stats_out + (static_cast<int64_t>(m0 + tid) * nbn + tile_n) * 2) =
        (f2_t){mu[tid], m2};
  }
}

// Consumer, part 1 (threads tid < BM of the workgroup, then a barrier by
// the caller): the unit's per-row LayerNorm values from the producer's block
// moments (copied to LDS at `stage` when the unit's K loop began), combined
// in double (src/tensor.cpp:63-71: mean and population variance in double,
// the inverse std rounded to float).  tab: BM rows of 16 bytes (the bf16
// deviations d_b = mu_b - mu, zero past the row's blocks: an MFMA operand
// row), then BM floats r = 1 / sqrt(var + eps).
__device__ __forceinline__ void ln_fold_table(const GemmArgs& g, const char* stage, char* tab, int tid,
                                              int BM) {
  const int nb = g.K / kLnBlock;
  const float* st = reinterpret_cast<const float*>(stage) + tid * nb * 2;
  double sum = 0.0;
#pragma unroll
  for (int b = 0; b < kLnMaxBlocks; ++b)
    if (b < nb) sum += st[2 * b];
  const double mean = sum / nb;
  double m2 = 0.0;
#pragma unroll
  for (int b = 0; b < kLnMaxBlocks; ++b)
    if (b < nb) {
      const double d = st[2 * b] - mean;
      m2 += st[2 * b + 1] + static_cast<double>(kLnBlock) * d * d;
    }
  const double var = m2 / (static_cast<double>(kLnBlock) * nb);
  reinterpret_cast<float*>(tab + 16 * BM)[tid] = static_cast<float>(1.0 / sqrt(var + static_cast<double>(g.ln_eps)));
  bf16x8_t dv = {};
#pragma unroll
  for (int b = 0; b < kLnMaxBlocks; ++b)
    if (b < nb) dv[b] = static_cast<__bf16>(static_cast<float>(st[2 * b] - mean));
  *reinterpret_cast<bf16x8_t*>(tab + 16 * tid) = dv;
}

// Consumer, part 2 (per wave, before its epilogue): acc += d . c1 as one more
// MFMA per block (the deviations in the K slots of the A side, c1 on the W
// side, zeros in the upper 8 K slots), then acc *= r of the row, then + c2.
template <int BM, int BN, int WM, int WN, int TI, int TJ, int EPI, bool SWAP>
__device__ __forceinline__ void ln_fold_acc(const GemmArgs& g, f32x16_t (&acc)[TI][TJ], int tile_n, int wm,
                                            int wn, int l32, int hb, const char* tab) {
  const bf16x8_t zero = {};
  bf16x8_t df[TI], cf[TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
    df[i] = hb == 0 ? *reinterpret_cast<const bf16x8_t*>(tab + 16 * (wm * WM + i * 32 + l32)) : zero;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int64_t wr = mfma_w_row<BN, WN, EPI>(g, tile_n, wn * WN + j * 32 + l32);
    cf[j] = hb == 0 ? *reinterpret_cast<const bf16x8_t*>(g.ln_c1 + wr * 8) : zero;
  }
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
      acc[i][j] = SWAP ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(cf[j], df[i], acc[i][j], 0, 0, 0)
                       : __builtin_amdgcn_mfma_f32_32x32x16_bf16(df[i], cf[j], acc[i][j], 0, 0, 0);
  const float* tr = reinterpret_cast<const float*>(tab + 16 * BM) + wm * WM;
  if constexpr (SWAP) {
    // lane l32 holds row 32 i + l32 and W rows 8 q + 4 hb + t of each block
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const float r = tr[i * 32 + l32];
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] *= r;
    }
    if (g.ln_c2) {
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float c = g.ln_c2[mfma_w_row<BN, WN, EPI>(g, tile_n, wn * WN + j * 32 + 8 * (e >> 2) + 4 * hb + (e & 3))];
#pragma unroll
          for (int i = 0; i < TI; ++i) acc[i][j][e] += c;
        }
    }
  } else {
    // lane l32 holds W row 32 j + l32 and rows 8 (e / 4) + 4 hb + e % 4
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const f32x4_t r4 = *reinterpret_cast<const f32x4_t*>(tr + i * 32 + 8 * e4 + 4 * hb);
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
          for (int t = 0; t < 4; ++t) acc[i][j][4 * e4 + t] *= r4[t];
      }
    if (g.ln_c2) {
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const float c = g.ln_c2[mfma_w_row<BN, WN, EPI>(g, tile_n, wn * WN + j * 32 + l32)];
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[i][j][e] += c;
      }
    }
  }
}

// ---- the next LayerNorm finished in the residual epilogue ------------------
// (GemmArgs::rln_y).  With every tile of the launch in a workgroup of its own
// and all of them resident, the N / 256 tiles of a 256-row panel hold whole
// rows of the updated residual stream x between them.  Each tile publishes
// its rows' moments over its 256 columns (mean and sum of squared
// deviations from it, fp32), counts itself into the panel's arrival counter
// and waits until every tile of the panel has arrived; it then combines the
// panel's moments per row in double (src/tensor.cpp:63-71: mean and
// population variance, the inverse std rounded to float) and writes LN(x) of
// its own block from the registers, with launch_ln's arithmetic.  The wait is
// bounded (rln_spin polls): a tile that gives up marks its block, and the
// panel's last tile to finish normalises the marked blocks from X in memory
// with the same published moments, so the result does not depend on which
// way it went.  Sync ints of panel p (kRlnSyncInts from 8p): [0] arrivals,
// [1] finishes, [2 + b] block b given up; the last tile to finish clears
// them for the next launch.
//
// Memory ordering: the moments and the sync ints are agent-scope atomics
// (written through to, and read from, the level every XCD sees).  A tile's
// moment stores have completed (vmcnt) before its arrival is counted, and
// the moment loads are issued only after the count was seen complete.  Only
// the give-up path needs X itself seen by another workgroup: a release fence
// before the mark, an acquire fence before the last tile reads X.
__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Row statistics (float mean, inverse std) of row m from the nb blocks'
// published (x0, s, q) (ln_block_combine's arithmetic).
__device__ __forceinline__ void rln_row_stats(const GemmArgs& g, int m, int nb, float& fmean, float& finv) {
  const float* p = g.rln_mom + static_cast<int64_t>(m) * nb * 4;
  float x0[kLnStatMaxBlocks] = {}, sb[kLnStatMaxBlocks] = {}, qb[kLnStatMaxBlocks] = {};
#pragma unroll
  for (int b = 0; b < kLnStatMaxBlocks; ++b)
    if (b < nb) {
      x0[b] = __hip_atomic_load(p + 4 * b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sb[b] = __hip_atomic_load(p + 4 * b + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      qb[b] = __hip_atomic_load(p + 4 * b + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  ln_block_combine(x0, sb, qb, nb, g.rln_eps, fmean, finv);
}

// Every wave of the workgroup calls it (it holds barriers).  lds: (WGN + 3)
// * BM floats and 4 ints past the ring.
template <int BM, int BN, int WM, int WN, int TI, int TJ, int WGN>
__device__ __forceinline__ void resid_rln_epilogue(const GemmArgs& g, f32x16_t (&acc)[TI][TJ], int m0, int tile_m,
                                                   int tile_n, int wm, int wn, int l32, int hb, int tid, char* lds) {
  static_assert(BM == 256 && BN == kLnBlock && TJ == 2 && WN == 64 && WM == 32 * TI,
                "the 16-wave 256 x 256 tile of 64 x 64 waves");
  float* red = reinterpret_cast<float*>(lds);  // [WGN][BM] partial sums
  float* mu = red + WGN * BM;                  // [BM] the block's shifted means s, then the rows' means
  float* rinv = mu + BM;                       // [BM] the rows' inverse std
  float* x0s = rinv + BM;                      // [BM] the block's first value of each row
  int* flag = reinterpret_cast<int*>(x0s + BM);  // [0] panel complete, [1] last to finish, [2] blocks given up
  const int nb = g.N / BN;
  const int c0 = tile_n * BN + wn * WN;
  const int rw = m0 + wm * WM;             // the wave's first row
  const int rows_in = min(g.M - rw, WM);   // its rows below M (may be <= 0)
  const uint32_t ld4 = static_cast<uint32_t>(g.ldx) * 4u;
  const uint32_t lo4 = 4 * hb * ld4 + l32 * 4;
  char* xw = reinterpret_cast<char*>(g.X + static_cast<int64_t>(rw) * g.ldx + c0);
  int* sync = g.rln_sync + kRlnSyncInts * tile_m;
  // lane (l32, hb) holds rows i * 32 + 8 (e / 4) + 4 hb + e % 4 of the wave,
  // columns j * 32 + l32
  auto rowof = [&](int i, int e) { return i * 32 + 8 * (e >> 2) + (e & 3) + 4 * hb; };

  // 1) X += acc + bias, the sum x kept in acc; the X reads of a group of 8
  //    rows go out before the first add (as in the plain residual epilogue).
  //    The waves that publish the moments (threads tid < BM) store their X
  //    after the arrival (3), so that their wait before it covers the moment
  //    stores only; the other waves store theirs here.
  const bool publisher = tid < BM;  // uniform per wave
  float bv[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) bv[j] = g.bias ? g.bias[c0 + j * 32 + l32] : 0.f;
  constexpr int RG = 8;
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int e0 = 0; e0 < 16; e0 += RG) {
      float xv[RG][TJ];
#pragma unroll
      for (int e = 0; e < RG; ++e) {
        const int r = rowof(i, e0 + e);
        const char* xr = xw + static_cast<uint32_t>((r - 4 * hb) * ld4 + lo4);
#pragma unroll
        for (int j = 0; j < TJ; ++j) xv[e][j] = r < rows_in ? *reinterpret_cast<const float*>(xr + j * 128) : 0.f;
      }
#pragma unroll
      for (int e = 0; e < RG; ++e) {
        const int r = rowof(i, e0 + e);
        char* xr = xw + static_cast<uint32_t>((r - 4 * hb) * ld4 + lo4);
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          acc[i][j][e0 + e] = xv[e][j] + (acc[i][j][e0 + e] + bv[j]);
          if (!publisher && r < rows_in) *reinterpret_cast<float*>(xr + j * 128) = acc[i][j][e0 + e];
        }
      }
    }

  // 2) the rows' block moments (ln_block_combine's inputs): the shift x0 is
  //    the block's first column (wave wn = 0, lane column 0); the pairwise
  //    tree is the wave's two column blocks (columns k, k + 32), rows16_sum
  //    over its 32 lane columns (distances 16 .. 1), then the four column
  //    waves as (g0 + g1) + (g2 + g3)
  if (wn == 0 && l32 == 0) {
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) x0s[wm * WM + rowof(i, e)] = acc[i][0][e];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    float v[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4_t x4 = *reinterpret_cast<const f32x4_t*>(x0s + wm * WM + i * 32 + 8 * q + 4 * hb);
#pragma unroll
      for (int t = 0; t < 4; ++t) v[4 * q + t] = (acc[i][0][4 * q + t] - x4[t]) + (acc[i][1][4 * q + t] - x4[t]);
    }
    const float sum = rows16_sum(v, l32);
    if ((l32 & 1) == 0) red[wn * BM + wm * WM + i * 32 + rows16_row(l32, hb)] = sum;
  }
  __syncthreads();
  static_assert(WGN == 4, "the four 64-column groups combine as (g0 + g1) + (g2 + g3)");
  if (tid < BM) mu[tid] = ((red[tid] + red[BM + tid]) + (red[2 * BM + tid] + red[3 * BM + tid])) * (1.0f / BN);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    float v[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4_t x4 = *reinterpret_cast<const f32x4_t*>(x0s + wm * WM + i * 32 + 8 * q + 4 * hb);
      const f32x4_t s4 = *reinterpret_cast<const f32x4_t*>(mu + wm * WM + i * 32 + 8 * q + 4 * hb);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float e0 = (acc[i][0][4 * q + t] - x4[t]) - s4[t], e1 = (acc[i][1][4 * q + t] - x4[t]) - s4[t];
        v[4 * q + t] = ln_pair_sq(e0, e1);
      }
    }
    const float ss = rows16_sum(v, l32);
    if ((l32 & 1) == 0) red[wn * BM + wm * WM + i * 32 + rows16_row(l32, hb)] = ss;
  }
  __syncthreads();
  if (tid < BM && m0 + tid < g.M) {
    const float q = (red[tid] + red[BM + tid]) + (red[2 * BM + tid] + red[3 * BM + tid]);
    float* p = g.rln_mom + (static_cast<int64_t>(m0 + tid) * nb + tile_n) * 4;
    __hip_atomic_store(p, x0s[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p + 1, mu[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p + 2, q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  wait_vm_all();  // this thread's X or moment stores have completed
  __syncthreads();

  // 3) count the tile in (its moment stores have completed), then the
  //    publishers' X stores
  if (tid == 0) __hip_atomic_fetch_add(sync, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (publisher) {
    // (the lane's offset recomputed here, so that no address of step 1 is
    // held through the statistics)
    const int ln = lane_id_here(), hbp = ln >> 5;
    const uint32_t lop = static_cast<uint32_t>(ln & 31) * 4;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rb = i * 32 + 8 * (e >> 2) + (e & 3);  // the row less 4 hb
        char* xr = xw + static_cast<uint32_t>((rb + 4 * hbp) * ld4 + lop);
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          if (rb + 4 * hbp < rows_in) *reinterpret_cast<float*>(xr + j * 128) = acc[i][j][e];
      }
  }
  if (tid == 0) {
    int n = __hip_atomic_load(sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int it = 0; n < nb && it < g.rln_spin; ++it) {
      __builtin_amdgcn_s_sleep(2);
      n = __hip_atomic_load(sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    flag[0] = n >= nb;
  }
  __syncthreads();

  const bool has_b = g.rln_b != nullptr;
  bf16_t* yw = static_cast<bf16_t*>(g.rln_y) + static_cast<int64_t>(rw) * g.rln_ldy + c0 + l32;
  if (__builtin_amdgcn_readfirstlane(flag[0])) {  // uniform
    // 4) every tile of the panel has published its moments
    if (tid < BM && m0 + tid < g.M) rln_row_stats(g, m0 + tid, nb, mu[tid], rinv[tid]);
    __syncthreads();
    float lw[TJ], lb[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      lw[j] = g.rln_w[c0 + j * 32 + l32];
      lb[j] = has_b ? g.rln_b[c0 + j * 32 + l32] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4_t fm = *reinterpret_cast<const f32x4_t*>(mu + wm * WM + i * 32 + 8 * q + 4 * hb);
        const f32x4_t fi = *reinterpret_cast<const f32x4_t*>(rinv + wm * WM + i * 32 + 8 * q + 4 * hb);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int r = rowof(i, 4 * q + t);
          if (r >= rows_in) continue;
#pragma unroll
          for (int j = 0; j < TJ; ++j)
            yw[static_cast<int64_t>(r) * g.rln_ldy + j * 32] =
                f32_to_bf16(ln_apply(acc[i][j][4 * q + t], fm[t], fi[t], lw[j], lb[j], has_b));
        }
      }
  } else {
    // 4') gave up waiting: X of this block to where the panel's last tile
    //     reads it, then the block's mark
    wait_vm_all();
    __syncthreads();
    if (tid == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      __hip_atomic_store(sync + 2 + tile_n, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  wait_vm_all();
  __syncthreads();

  // 5) the panel's last tile to finish normalises the blocks given up, then
  //    clears the panel's sync ints
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(sync + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    flag[1] = old == nb - 1;
    int given_up = 0;
    if (old == nb - 1)
      for (int b = 0; b < nb; ++b)
        given_up |= __hip_atomic_load(sync + 2 + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) << b;
    flag[2] = given_up;
  }
  __syncthreads();
  const int last = __builtin_amdgcn_readfirstlane(flag[1]), given_up = __builtin_amdgcn_readfirstlane(flag[2]);
  if (last && given_up) {  // uniform; rarely taken
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (tid < BM && m0 + tid < g.M) rln_row_stats(g, m0 + tid, nb, mu[tid], rinv[tid]);
    __syncthreads();
    for (int b = 0; b < nb; ++b) {
      if (!((given_up >> b) & 1)) continue;
      for (int k = tid; k < BM * BN; k += 64 * WGN * (BM / WM)) {
        const int r = k / BN, c = b * BN + k % BN;
        if (m0 + r >= g.M) continue;
        const float x = g.X[static_cast<int64_t>(m0 + r) * g.ldx + c];
        static_cast<bf16_t*>(g.rln_y)[static_cast<int64_t>(m0 + r) * g.rln_ldy + c] =
            f32_to_bf16(ln_apply(x, mu[r], rinv[r], g.rln_w[c], has_b ? g.rln_b[c] : 0.f, has_b));
      }
    }
  }
  if (last && tid < 2 + nb) __hip_atomic_store(sync + tid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- direct-to-LDS variant -------------------------------------------------
// Tiles move from HBM to LDS with global_load_lds_dwordx4 (no VGPR staging):
// lane l of an instruction writes its 16 bytes at LDS address base + 16*l, so
// one instruction fills 1 KB of unpadded tile rows (8 rows of a 64-deep K
// step, 16 rows of a 32-deep one).  Bank conflicts on the MFMA operand reads
// are avoided by an XOR swizzle of the 16-byte chunks within a row.  NS
// stages form a ring; the loads for stage kt + NS - 1 are issued right after
// the barrier that opens iteration kt, so NS - 1 stages are in flight while
// stage kt is consumed.
template <int BM, int BN, int WGM, int WGN, int NS, int BK>
struct DTile {
  static constexpr int NW = WGM * WGN;
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int TI = WM / 32, TJ = WN / 32;
  static constexpr int RB = BK * 2;                // bytes per tile row
  static constexpr int CPR = BK / 8;               // 16-byte chunks per row
  static constexpr int RPI = 1024 / RB;            // rows per load instruction
  static constexpr int GROUPS = (BM + BN) / RPI;   // load instructions per stage
  static constexpr int G = GROUPS / NW;            // ... per wave
  static constexpr int STAGE_BYTES = (BM + BN) * RB;
  static_assert(BK == 32 || BK == 64, "K step is 32 or 64");
  static_assert(G * NW == GROUPS && BM % RPI == 0, "row groups must split evenly over waves");
  static_assert(TI >= 1 && TJ >= 1, "tile too small");
  static_assert(NS >= 2 && NS * STAGE_BYTES <= 160 * 1024, "LDS ring does not fit");
  static_assert(G * (NS - 2) <= 63, "vmcnt range");
  // chunk position of logical chunk c in tile row r is c ^ swz(r).  The LDS
  // serves a 16-byte read for 16 lanes at a time across 64 four-byte banks;
  // 16 consecutive rows at one logical chunk then land in 16 distinct
  // 16-byte bank groups.
  static __device__ __forceinline__ int swz(int r) {
    return BK == 64 ? ((r >> 1) & 7) : ((r >> 2) & 3);
  }
};

template <typename OutT>
__device__ void splitk_output(const GemmArgs& g, int S, int m, int n);

template <int BM, int BN, int WGM, int WGN, int NS, int BK, int EPI, typename OutT,
          bool SPLITK = false>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_bf16_dma_kernel(GemmArgs g0) {
  using TT = DTile<BM, BN, WGM, WGN, NS, BK>;
  const GemmArgs g = resolve_rows(g0);
  constexpr int TI = TT::TI, TJ = TT::TJ, G = TT::G, RB = TT::RB, CPR = TT::CPR;
  constexpr int KS = BK / 16;  // MFMA K steps per stage
  extern __shared__ __attribute__((aligned(16))) char dsmem[];

  const int tiles_n = EPI == EPI_GEGLU ? g.N / (BN / 2) : (g.N + BN - 1) / BN;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int tile_m = tile / tiles_n, tile_n = tile - tile_m * tiles_n;
  const int m0 = tile_m * BM;
  if (m0 >= g.M) return;  // a row tile past the device row count (uniform)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int l32 = lane & 31, hb = lane >> 5;

  const bf16_t* A = static_cast<const bf16_t*>(g.A);
  const bf16_t* W = static_cast<const bf16_t*>(g.W);

  // this wave's row groups: q = wave + NW * i; lane moves tile row
  // RPI * q + lane / CPR into chunk slot lane % CPR, reading the logical
  // chunk that the swizzle maps there
  const bf16_t* src[G];
  const int lrow = lane / CPR, cslot = lane % CPR;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int r = TT::RPI * (wave + TT::NW * i) + lrow;
    const int gchunk = cslot ^ TT::swz(r);
    if (r < BM)
      src[i] = A + static_cast<int64_t>(min(m0 + r, g.M - 1)) * g.lda + gchunk * 8;
    else
      src[i] = W + mfma_w_row<BN, TT::WN, EPI>(g, tile_n, r - BM) * g.ldw + gchunk * 8;
  }
  auto issue = [&](int kt, int buf) {
    char* base = dsmem + buf * TT::STAGE_BYTES;
#pragma unroll
    for (int i = 0; i < G; ++i)
      load_lds16(static_cast<const void*>(src[i] + kt * BK), base + (wave + TT::NW * i) * 1024);
  };

  f32x16_t acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // K steps [k_begin, k_begin + nk): all of K, or one split's slice
  int k_begin = 0, nk = g.K / BK;
  if constexpr (SPLITK) {
    k_begin = blockIdx.y * g.k_chunk;
    nk = min(g.k_chunk, nk - k_begin);
  }
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) issue(k_begin + s, s);

  // operand rows of this lane; tile bases are multiples of 32, so the
  // swizzle key of row base + l32 is that of l32
  const int xr = TT::swz(l32);
  const int a_row0 = (wm * TT::WM + l32) * RB, w_row0 = (BM + wn * TT::WN + l32) * RB;
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + NS - 2 < nk)
      wait_vmcnt<G * (NS - 2)>();
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (kt + NS - 1 < nk) issue(k_begin + kt + NS - 1, (kt + NS - 1) % NS);
    const char* sb = dsmem + (kt % NS) * TT::STAGE_BYTES;
    // operand fragments double-buffered across the K steps so the LDS reads
    // of step s + 1 are in flight during the MFMAs of step s
    bf16x8_t af[2][TI], bw[2][TJ];
    auto frag = [&](int s, int buf) {
      const int coff = ((2 * s + hb) ^ xr) * 16;
#pragma unroll
      for (int i = 0; i < TI; ++i)
        af[buf][i] = *reinterpret_cast<const bf16x8_t*>(sb + a_row0 + i * 32 * RB + coff);
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        bw[buf][j] = *reinterpret_cast<const bf16x8_t*>(sb + w_row0 + j * 32 * RB + coff);
    };
    frag(0, 0);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if (s + 1 < KS) frag(s + 1, (s + 1) & 1);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s & 1][i], bw[s & 1][j],
                                                               acc[i][j], 0, 0, 0);
    }
    // Pin the schedule: the reads of step 0, then for each step its MFMAs
    // interleaved one-for-one with the reads of the next step (mask 0x008 =
    // MFMA, 0x100 = LDS read).
#pragma unroll
    for (int r = 0; r < TI + TJ; ++r) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int k = 0; k < TI * TJ; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (s + 1 < KS && k < TI + TJ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      if (s + 1 < KS) {
#pragma unroll
        for (int k = TI * TJ; k < TI + TJ; ++k) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
  }

  if constexpr (!SPLITK) {
    gemm_epilogue<BM, BN, TT::WM, TT::WN, TI, TJ, EPI, OutT>(g, acc, m0, tile_n, wm, wn, l32, hb);
  } else {
    // Split-K: store this split's partial sums at their W row;
    // splitk_epilogue_kernel adds the splits in order and applies the
    // epilogue.  The tile holds every W row its outputs need (GEGLU input and
    // gate rows, both halves of a RoPE head).
    float* part = g.partial + static_cast<int64_t>(blockIdx.y) * g.part_rows * g.n_w;
    if constexpr (EPI != EPI_GEGLU) {
      // W row = output column: the wave's uniform corner plus one 32-bit
      // byte offset per store; the bounds checks only where the wave's rows
      // or columns run past M or N
      const int rw = m0 + wm * TT::WM, c0 = tile_n * BN + wn * TT::WN;
      char* pw = reinterpret_cast<char*>(part + static_cast<int64_t>(rw) * g.n_w + c0);
      const uint32_t ldb = static_cast<uint32_t>(g.n_w) * 4u;
      const uint32_t lo = 4 * hb * ldb + l32 * 4;
      auto body = [&](auto checked) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int r = i * 32 + 8 * (e >> 2) + (e & 3);
            if (decltype(checked)::value && rw + r + 4 * hb >= g.M) continue;
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
              if (decltype(checked)::value && c0 + j * 32 + l32 >= g.n_w) continue;
              *reinterpret_cast<float*>(pw + static_cast<uint32_t>(r * ldb + lo) + j * 128) = acc[i][j][e];
            }
          }
      };
      if (rw + TT::WM <= g.M && c0 + TT::WN <= g.n_w)
        body(std::false_type{});
      else
        body(std::true_type{});
    } else {
      const int row_base = m0 + wm * TT::WM + 4 * hb;
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int64_t wr = mfma_w_row<BN, TT::WN, EPI>(g, tile_n, wn * TT::WN + j * 32 + l32);
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int m = row_base + i * 32 + 8 * (e >> 2) + (e & 3);
            if (m < g.M) part[static_cast<int64_t>(m) * g.n_w + wr] = acc[i][j][e];
          }
      }
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- persistent variant ------------------------------------------------------
// One workgroup per CU walks a static list of output tiles.  The direct-to-LDS
// load ring runs across tile boundaries (the first stages of the next tile are
// in flight while the current tile's epilogue runs), and the MFMAs of the last
// K step of each stage are issued after the next barrier, so the matrix pipe
// keeps working while the first operand reads of the new stage are in flight.
//
// The MFMA computes the transposed product C^T = W . A^T: W rows are the MFMA
// rows and A rows its columns.  Lane l then owns output row l % 32 of a 32x32
// block and, for e = 4q + r, output column 8q + 4(l / 32) + r: four
// consecutive columns per q, so every epilogue reads and writes 8- or 16-byte
// vectors.  For RoPE (head_dim 64) the partner of a dim in block j is the same
// lane and register in block j ^ 1; for GEGLU the input and gate values of an
// output are the same lane and register in blocks j and j + TJ/2.

__device__ __forceinline__ void store4(bf16_t* p, float a, float b, float c, float d) {
  *reinterpret_cast<u32x2_t*>(p) = (u32x2_t){pack_bf16x2(a, b), pack_bf16x2(c, d)};
}
__device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<f32x4_t*>(p) = (f32x4_t){a, b, c, d};
}

// Rows past M and (GEGLU, whose last column tile may be partial) column
// chunks past N are masked; N % 4 == 0.
template <int BM, int BN, int WM, int WN, int TI, int TJ, int EPI, typename OutT>
__device__ __forceinline__ void pers_epilogue(const GemmArgs& g, f32x16_t (&acc)[TI][TJ], int m0,
                                              int tile_n, int wm, int wn, int l32, int hb) {
  const int row0 = m0 + wm * WM + l32;  // + 32 i
  if constexpr (EPI == EPI_GEGLU) {
    OutT* out = static_cast<OutT*>(g.out);
    const int c0 = tile_n * (BN / 2) + wn * (WN / 2) + 4 * hb;  // + 32 j + 8 q
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const int m = row0 + i * 32;
      if (m >= g.M) continue;
      OutT* orow = out + static_cast<int64_t>(m) * g.ldo + c0;
#pragma unroll
      for (int j = 0; j < TJ / 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (c0 + j * 32 + 8 * q >= g.N) continue;  // N % 4 == 0: a chunk is all in or out
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            v[r] = gelu_out<OutT>(acc[i][j][4 * q + r]) * acc[i][j + TJ / 2][4 * q + r];
          store4(orow + j * 32 + 8 * q, v[0], v[1], v[2], v[3]);
        }
    }
  } else if constexpr (EPI == EPI_RESID) {
    const int c0 = tile_n * BN + wn * WN + 4 * hb;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const int m = row0 + i * 32;
      float* xrow = g.X + static_cast<int64_t>(min(m, g.M - 1)) * g.ldx + c0;
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        // the block's four X reads are issued before the first add
        f32x4_t xv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) xv[q] = *reinterpret_cast<const f32x4_t*>(xrow + j * 32 + 8 * q);
        if (g.bias) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4_t b = *reinterpret_cast<const f32x4_t*>(g.bias + c0 + j * 32 + 8 * q);
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[i][j][4 * q + t] += b[t];
          }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) consume(xv[q]);
        if (m < g.M) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            f32x4_t r;
#pragma unroll
            for (int t = 0; t < 4; ++t) r[t] = xv[q][t] + acc[i][j][4 * q + t];
            *reinterpret_cast<f32x4_t*>(xrow + j * 32 + 8 * q) = r;
          }
        }
      }
    }
  } else if constexpr (EPI == EPI_ROPE) {
    static_assert(TJ % 2 == 0, "RoPE pairs need an even number of column blocks");
    OutT* out = static_cast<OutT*>(g.out);
    const int c0 = tile_n * BN + wn * WN + 4 * hb;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const int m = row0 + i * 32;
      const int p = min(max(g.pos[min(m, g.M - 1)], 0), g.rope_rows - 1);
      // dims 8q + 4hb .. +3 at the row's position
      f32x4_t cs[4], sn[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t tb = static_cast<int64_t>(p) * 32 + 8 * q + 4 * hb;
        cs[q] = *reinterpret_cast<const f32x4_t*>(g.rope_cos + tb);
        sn[q] = *reinterpret_cast<const f32x4_t*>(g.rope_sin + tb);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        consume(cs[q]);
        consume(sn[q]);
      }
      if (m >= g.M) continue;
      OutT* orow = out + static_cast<int64_t>(m) * g.ldo + c0;
#pragma unroll
      for (int j = 0; j < TJ; j += 2) {
        const bool rot = tile_n * BN + wn * WN + j * 32 < 2 * g.rope_dim;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float x0[4], x1[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            x0[t] = acc[i][j][4 * q + t];
            x1[t] = acc[i][j + 1][4 * q + t];
            if (rot) {
              const float r0 = rope_lo(x0[t], x1[t], cs[q][t], sn[q][t]);
              const float r1 = rope_hi(x0[t], x1[t], cs[q][t], sn[q][t]);
              x0[t] = r0;
              x1[t] = r1;
              if (tile_n * BN + wn * WN + j * 32 < g.rope_dim) {  // a q head
                x0[t] *= g.q_scale;
                x1[t] *= g.q_scale;
              }
            }
          }
          store4(orow + j * 32 + 8 * q, x0[0], x0[1], x0[2], x0[3]);
          store4(orow + j * 32 + 32 + 8 * q, x1[0], x1[1], x1[2], x1[3]);
        }
      }
    }
  } else {
    OutT* out = static_cast<OutT*>(g.out);
    const int c0 = tile_n * BN + wn * WN + 4 * hb;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const int m = row0 + i * 32;
      if (m >= g.M) continue;
      OutT* orow = out + static_cast<int64_t>(m) * g.ldo + c0;
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4_t b = g.bias ? *reinterpret_cast<const f32x4_t*>(g.bias + c0 + j * 32 + 8 * q)
                                   : (f32x4_t){0, 0, 0, 0};
          float v[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            v[t] = acc[i][j][4 * q + t] + b[t];
            if (g.act == 1)
              v[t] = gelu_out<OutT>(v[t]);
            else if (g.act == 2)
              v[t] = fmaxf(v[t], 0.f);
          }
          store4(orow + j * 32 + 8 * q, v[0], v[1], v[2], v[3]);
        }
    }
  }
}

// RoPE tables of a persistent unit's 256 rows staged in LDS for its epilogue:
// cos rows at row * 128, sin rows 32 KB on (64 KB), copied with direct-to-LDS
// loads of whole 128-byte table rows, so that the epilogue's per-element
// table reads are LDS reads instead of one global gather per (row, dim).  The
// row positions come from pos_lds (the unit's 256 positions, copied there
// when its first K step began).  Each of the 16 waves copies 16 rows (four
// load instructions); the caller provides the waits and barriers.
__device__ __forceinline__ void rope_issue_tables(const GemmArgs& g, char* tab, const int* pos_lds,
                                                  int wave_s, int lane) {
  // byte offsets into the tables (under 4 GiB, checked by the launcher) over
  // the tables' uniform bases
  uint32_t off[2];
#pragma unroll
  for (int k = 0; k < 2; ++k)
    off[k] = static_cast<uint32_t>(min(max(pos_lds[8 * (wave_s + 16 * k) + (lane >> 3)], 0), g.rope_rows - 1)) * 128u +
             (lane & 7) * 16;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const char* t = reinterpret_cast<const char*>((i >> 1) ? g.rope_sin : g.rope_cos);
    load_lds16(t + off[i & 1], tab + (i >> 1) * 32768 + (wave_s + 16 * (i & 1)) * 1024);
  }
}

// Ring geometry of the persistent kernel.  A rows are bf16; W rows are bf16,
// or fp8 (W8: one byte per element, half the bytes per stage).  Each load
// instruction fills 1 KB of LDS (64 lanes x 16 bytes): groups [0, GA) are A
// rows, groups [GA, GA + GW) W rows, and group g lands at byte 1024 g of the
// stage.  16-byte chunks are XOR-swizzled per row so that the operand reads
// are free of bank conflicts (16 lanes per cycle over 64 four-byte banks).
template <int BM, int BN, int WGM, int WGN, int NS, int BK, bool W8>
struct PTile {
  static constexpr int NW = WGM * WGN;
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int TI = WM / 32, TJ = WN / 32;
  static constexpr int RBA = BK * 2, RBW = W8 ? BK : BK * 2;  // bytes per row
  static constexpr int CPRA = RBA / 16, CPRW = RBW / 16;      // 16-byte chunks per row
  static constexpr int RPIA = 1024 / RBA, RPIW = 1024 / RBW;  // rows per load instruction
  static constexpr int GA = BM / RPIA, GW = BN / RPIW;
  static constexpr int G = (GA + GW) / NW;  // load instructions per wave per stage
  static constexpr int W_OFF = BM * RBA;
  static constexpr int STAGE_BYTES = W_OFF + BN * RBW;
  static_assert(BK == 32 || BK == 64, "K step is 32 or 64");
  static_assert(!W8 || BK == 64, "fp8 weights use 64-deep K steps");
  static_assert(G * NW == GA + GW && BM % RPIA == 0 && BN % RPIW == 0,
                "row groups must split evenly over waves");
  static_assert(TI >= 1 && TJ >= 1, "tile too small");
  static_assert(NS >= 2 && NS * STAGE_BYTES <= 160 * 1024, "LDS ring does not fit");
  static_assert(G * (NS - 2) <= 63, "vmcnt range");
  // 128-byte rows: 16 consecutive rows at one logical chunk hit 16 distinct
  // 16-byte bank groups with key (r >> 1) & 7; 64-byte rows need (r >> 2) & 3
  static __device__ __forceinline__ int swz(int row_bytes, int r) {
    return row_bytes == 128 ? ((r >> 1) & 7) : ((r >> 2) & 3);
  }
};

// Workgroups resident per CU: bounded by the 160 KB of LDS and by 16 waves
// (4 per SIMD at <= 128 VGPRs).  Several per CU let one workgroup's barriers
// and epilogue overlap another's MFMAs; the register budget follows from the
// waves that then share a SIMD.
template <int BM, int BN, int WGM, int WGN, int NS, int BK, bool W8>
constexpr int pers_occupancy() {
  return std::max(1, std::min(163840 / (NS * PTile<BM, BN, WGM, WGN, NS, BK, W8>::STAGE_BYTES),
                              16 / (WGM * WGN)));
}
template <int BM, int BN, int WGM, int WGN, int NS, int BK, bool W8>
constexpr int pers_waves_per_simd() {
  return std::max(1, std::min(4, pers_occupancy<BM, BN, WGM, WGN, NS, BK, W8>() * WGM * WGN / 4));
}

// LNF: 0, or a folded LayerNorm's consumer (1) or producer (2, EPI_RESID)
template <int BM, int BN, int WGM, int WGN, int NS, int BK, bool W8, int EPI, typename OutT, int LNF>
__global__ __launch_bounds__(64 * WGM * WGN, (pers_waves_per_simd<BM, BN, WGM, WGN, NS, BK, W8>()))
void gemm_bf16_pers_kernel(GemmArgs g0) {
  using TT = PTile<BM, BN, WGM, WGN, NS, BK, W8>;
  const GemmArgs g = resolve_rows(g0);
  if (g.M <= 0) return;
  constexpr int TI = TT::TI, TJ = TT::TJ, G = TT::G, NW = TT::NW;
  constexpr int RBA = TT::RBA, RBW = TT::RBW;
  constexpr int KS = BK / 16;  // MFMA K steps per stage
  static_assert(KS % 2 == 0, "the deferred step and step 0 use different fragment buffers");
  // Transposed product (vector epilogue) only where the epilogue just stores:
  // its 16-byte accesses span 32 rows, which costs more than it saves where
  // the epilogue also reads (X, RoPE tables).
  constexpr bool kSwap = EPI == EPI_GEGLU;
  // RoPE tables through LDS: needs a 64 KB stage and 16 waves of 256 rows
  constexpr bool kRopeLds = EPI == EPI_ROPE && !kSwap && BM == 256 && WGM * WGN == 16 &&
                            PTile<BM, BN, WGM, WGN, NS, BK, W8>::STAGE_BYTES >= 65536;
  // half units need an even number of wave rows (the lower half computes)
  constexpr bool kHalves = WGM % 2 == 0;
  extern __shared__ __attribute__((aligned(16))) char dsmem[];

  const int tiles_n = EPI == EPI_GEGLU ? (g.N + BN / 2 - 1) / (BN / 2) : (g.N + BN - 1) / BN;
  const int tiles = tiles_n * ((g.M + BM - 1) / BM);
  const int nk = g.K / BK;

  // Static schedule.  Workgroup b runs on XCD b % 8.  The tile list (N
  // fastest) is cut into 8 contiguous ranges, one per XCD, sized by the
  // number of workgroups on that XCD, so the tiles sharing an A row panel stay
  // in one L2; workgroup k of an XCD takes local tiles k, k + c, k + 2c, ...
  // When the range leaves a last, partial round of r <= c/2 tiles, those
  // tiles are cut into 2r half units of BM/2 rows, one per workgroup, so the
  // last round takes about half a tile's time instead of a whole one (in a
  // half unit the waves of the lower half of the tile do the MFMAs and the
  // epilogue; the others only share the loads and barriers).
  const int nwg = gridDim.x, xcd = blockIdx.x & 7, xk = blockIdx.x >> 3;
  const int per = nwg >> 3, rem = nwg & 7;
  const int cx = per + (xcd < rem ? 1 : 0);
  const int offx = xcd * per + min(xcd, rem);
  const int lo = static_cast<int>(static_cast<int64_t>(tiles) * offx / nwg);
  const int hi = static_cast<int>(static_cast<int64_t>(tiles) * (offx + cx) / nwg);
  const int full_x = (hi - lo) / cx, rem_x = (hi - lo) - full_x * cx;
  // (no half units where the epilogue finishes a LayerNorm: its tiles need every wave)
  const bool halves = LNF != 3 && kHalves && full_x >= 1 && rem_x > 0 && 2 * rem_x <= cx;
  const int my_full = halves ? full_x : (xk < hi - lo ? (hi - lo - xk + cx - 1) / cx : 0);
  // (a launch whose epilogue finishes a LayerNorm has one tile per workgroup:
  // the launcher checks that the grid covers every tile)
  const int my_units = LNF == 3 ? min(my_full, 1) : my_full + (halves && xk < 2 * rem_x ? 1 : 0);
  if (my_units == 0) return;
  const int total = my_units * nk;
  // unit u of this workgroup: its tile (m, n) and half (-1: the whole tile)
  auto unit = [&](int u, int& m, int& n, int& h) {
    const int t = u < my_full ? lo + xk + u * cx : lo + full_x * cx + (xk >> 1);
    h = u < my_full ? -1 : (xk & 1);
    m = t / tiles_n;
    n = t - m * tiles_n;
  };

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int l32 = lane & 31, hb = lane >> 5;
  const char* A = static_cast<const char*>(g.A);
  const char* W = static_cast<const char*>(g.W);

  // Load cursor (uniform): unit ld_u of this workgroup's list (tile (ld_m,
  // ld_n), half ld_h) and K step ld_kt.
  int ld_kt = 0, ld_u = 0, ld_m, ld_n, ld_h;
  unit(0, ld_m, ld_n, ld_h);
  // Load addresses: a wave-uniform base (the operand's start plus the K
  // step's byte offset, in scalar registers) plus a per-lane 32-bit byte
  // offset of the source row and chunk, recomputed only when the cursor
  // enters a new unit (the launcher checks that both operands span less than
  // 4 GiB).  The LDS target of each load instruction is wave-uniform too.
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  uint32_t voff[G];
  auto set_src = [&]() {
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int gi = wave + NW * i;
      if (gi < TT::GA) {
        const int row = TT::RPIA * gi + lane / TT::CPRA;
        const int chunk = (lane % TT::CPRA) ^ TT::swz(RBA, row);
        // a half unit stages its BM/2 rows twice (the copy is never read)
        const int arow = ld_h < 0 ? row : (row & (BM / 2 - 1)) + (BM / 2) * ld_h;
        voff[i] = static_cast<uint32_t>(min(ld_m * BM + arow, g.M - 1)) * static_cast<uint32_t>(g.lda * 2) +
                  chunk * 16;
      } else {
        const int row = TT::RPIW * (gi - TT::GA) + lane / TT::CPRW;
        const int chunk = (lane % TT::CPRW) ^ TT::swz(RBW, row);
        voff[i] = static_cast<uint32_t>(mfma_w_row<BN, TT::WN, EPI>(g, ld_n, row)) *
                      static_cast<uint32_t>(g.ldw * (W8 ? 1 : 2)) +
                  chunk * 16;
      }
    }
  };
  set_src();
  auto issue_next = [&](int buf) {
    char* base = dsmem + buf * TT::STAGE_BYTES + wave_s * 1024;
    const char* a_k = A + ld_kt * (BK * 2);
    const char* w_k = W + ld_kt * RBW;
#pragma unroll
    for (int i = 0; i < G; ++i)
      load_lds16(static_cast<const void*>((wave_s + NW * i < TT::GA ? a_k : w_k) + voff[i]),
                 base + NW * i * 1024);
    if (++ld_kt == nk) {  // next unit of the list
      ld_kt = 0;
      if (++ld_u < my_units) {
        unit(ld_u, ld_m, ld_n, ld_h);
        set_src();
      }
    }
  };
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < total) issue_next(s);

  // Operand reads.  bf16 W: step s reads chunk 2s + hb of the A and W rows.
  // fp8 W: one 16-byte read of W chunk 2p + hb holds 16 K values for the
  // step pair (2p, 2p + 1), so the K order is permuted the same way on the A
  // side: step 2p + t reads A chunk 4p + 2hb + t.  The sum over K is the same
  // either way.
  const int xa = TT::swz(RBA, l32), xw = TT::swz(RBW, l32);
  const int a_row0 = (wm * TT::WM + l32) * RBA, w_row0 = TT::W_OFF + (wn * TT::WN + l32) * RBW;
  bf16x8_t af[2][TI];
  bf16x8_t bw[W8 ? 1 : 2][TJ];
  u32x4_t wraw[W8 ? 2 : 1][TJ];  // fp8 codes of a step pair, by pair parity
  auto frag = [&](const char* sb, int s, int buf) {
    const int ca = W8 ? 4 * (s >> 1) + 2 * hb + (s & 1) : 2 * s + hb;
#pragma unroll
    for (int i = 0; i < TI; ++i)
      af[buf][i] = *reinterpret_cast<const bf16x8_t*>(sb + a_row0 + i * 32 * RBA + ((ca ^ xa) << 4));
    if constexpr (!W8) {
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        bw[buf][j] = *reinterpret_cast<const bf16x8_t*>(sb + w_row0 + j * 32 * RBW +
                                                        (((2 * s + hb) ^ xw) << 4));
    } else if ((s & 1) == 0) {
      const int cw = (s & 2) + hb;
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        wraw[(s >> 1) & 1][j] =
            *reinterpret_cast<const u32x4_t*>(sb + w_row0 + j * 32 * RBW + ((cw ^ xw) << 4));
    }
  };
  f32x16_t acc[TI][TJ];
  const int wm_s = __builtin_amdgcn_readfirstlane(wm);
  auto mma = [&](int s) {  // K step s of a stage
    const int buf = s & 1;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      bf16x8_t w;
      if constexpr (W8) {
        const u32x4_t& r = wraw[(s >> 1) & 1][j];
        w = (s & 1) ? fp8x8_to_bf16(r[2], r[3]) : fp8x8_to_bf16(r[0], r[1]);
      } else {
        w = bw[buf][j];
      }
#pragma unroll
      for (int i = 0; i < TI; ++i)
        acc[i][j] = kSwap ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(w, af[buf][i], acc[i][j], 0, 0, 0)
                          : __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[buf][i], w, acc[i][j], 0, 0, 0);
    }
  };
  // LDS reads issued by frag(s)
  auto nreads = [](int s) { return TI + (W8 ? ((s & 1) == 0 ? TJ : 0) : TJ); };

  // Ring slot of stage q: (q + so) % NS.  A RoPE unit with rotated columns
  // and at least two K steps copies its table rows during its last K step,
  // into the slot that step leaves free (where the next unit's first stage
  // would otherwise go); that stage goes instead into the slot the last step
  // consumed, once every wave is done with it, so the slot order flips.
  int so = 0;
  int q = 0;  // global stage counter (ring position)
  for (int r = 0; r < my_units; ++r) {
    int tm, tn, th;  // compute cursor: the unit whose stages are consumed
    unit(r, tm, tn, th);
    // waves with no rows in a half unit only share the loads and barriers
    const bool idle = th >= 0 && wm_s >= WGM / 2;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    // the operands of the first stage's "deferred" step start at zero: its
    // MFMAs add 0 (fp8 code 0 is +0)
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int t = 0; t < 8; ++t) af[1][i][t] = static_cast<__bf16>(0.f);
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      if constexpr (W8) {
        wraw[1][j] = (u32x4_t){0u, 0u, 0u, 0u};
      } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) bw[1][j][t] = static_cast<__bf16>(0.f);
      }
    }
    const int m0 = tm * BM + (th < 0 ? 0 : (BM / 2) * th);
    static_assert(LNF == 0 || (LNF == 1 && EPI != EPI_RESID) || (LNF >= 2 && EPI == EPI_RESID),
                  "folded LayerNorm roles");
    // RoPE units: positions of the unit's 256 rows to LDS (waves 0-3, 64 rows
    // each), copied during the first K step and read at the unit's end
    int* pos_lds = reinterpret_cast<int*>(dsmem + NS * TT::STAGE_BYTES);
    auto copy_pos = [&]() {
      if constexpr (kRopeLds) {
        if (wave_s < 4 && tn * BN < 2 * g.rope_dim)
          __builtin_amdgcn_global_load_lds(g.pos + min(m0 + 64 * wave_s + lane_id_here(), g.M - 1),
                                           (__attribute__((address_space(3))) void*)(pos_lds + 64 * wave_s),
                                           4, 0, 0);
      }
    };
    // a folded LayerNorm's LDS, past the ring and the RoPE positions: the
    // consumer's copy of the unit's row moments and its row table, or the
    // producer's reduction rows
    char* fold_lds = dsmem + NS * TT::STAGE_BYTES + 1024;
    char* fold_tab = fold_lds + BM * kLnMaxBlocks * 8;
    // consumer: the moments of the unit's BM rows (contiguous; the buffer
    // holds rows past M), copied during the first K step
    auto copy_stats = [&]() {
      if constexpr (LNF == 1) {
        const int chunks = BM * (g.K / kLnBlock) * 8 / 1024;
        const char* src = reinterpret_cast<const char*>(g.ln_stats_in) +
                          static_cast<int64_t>(m0) * (g.K / kLnBlock) * 8 + lane_id_here() * 16;
        for (int c = wave_s; c < chunks; c += NW) load_lds16(src + c * 1024, fold_lds + c * 1024);
      }
    };
    // uniform: the unit's tile has rotated columns
    const bool rot = kRopeLds && tn * BN < 2 * g.rope_dim;
    auto kloop = [&](auto busy) {
      for (int kt = 0; kt < nk; ++kt, ++q) {
        // this wave's loads of stage q have landed once at most the younger
        // stages' loads are outstanding (vector memory completes in issue order)
        if (q + NS - 2 < total)
          wait_vmcnt<G * (NS - 2)>();
        else
          wait_vmcnt<0>();
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
        if (rot && nk >= 2 && kt == nk - 1)
          rope_issue_tables(g, dsmem + ((q + NS - 1 + so) % NS) * TT::STAGE_BYTES, pos_lds, wave_s,
                            lane_id_here());
        else if (q + NS - 1 < total)
          issue_next((q + NS - 1 + so) % NS);
        if (kt == 0) {
          copy_pos();
          copy_stats();
        }
        if constexpr (!decltype(busy)::value) continue;
        const char* sb = dsmem + ((q + so) % NS) * TT::STAGE_BYTES;
        // operand reads of step 0 go out first; the previous stage's last K
        // step (deferred past the barrier) covers their latency; then each
        // step's MFMAs interleave one-for-one with the reads of the next step
        frag(sb, 0, 0);
        mma(KS - 1);
#pragma unroll
        for (int s = 0; s + 1 < KS; ++s) {
          frag(sb, s + 1, (s + 1) & 1);
          mma(s);
        }
#pragma unroll
        for (int k = 0; k < nreads(0); ++k) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
        for (int k = 0; k < TI * TJ; ++k) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
        for (int s = 0; s + 1 < KS; ++s) {
#pragma unroll
          for (int k = 0; k < TI * TJ; ++k) {
            if (k < nreads(s + 1)) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          }
#pragma unroll
          for (int k = TI * TJ; k < nreads(s + 1); ++k) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }
      if constexpr (decltype(busy)::value) mma(KS - 1);
    };
    const char* rope_tab = nullptr;
    auto stage_tables = [&]() {  // every wave takes part (loads and barriers)
      if constexpr (kRopeLds) {
        if (rot) {
          static_assert(NS == 2, "the table slot is the ring's other slot");
          const int last = (q - 1 + so) % NS;  // slot of the last K step
          wait_lgkm0();
          if (nk >= 2) {
            // the tables are in flight into the other slot; the next unit's
            // first stage takes the last step's slot once every wave is done
            // with it, and its loads stay in flight through the epilogue
            __builtin_amdgcn_s_barrier();
            rope_tab = dsmem + (1 - last) * TT::STAGE_BYTES;
            const bool more = q < total;
            if (more) issue_next(last);
            so ^= 1;
            if (more)
              wait_vmcnt<G>();
            else
              wait_vmcnt<0>();
          } else {
            // one K step: the positions copied when it began land first, then
            // the tables go into the last step's slot
            wait_vmcnt<0>();
            __builtin_amdgcn_s_barrier();
            rope_tab = dsmem + last * TT::STAGE_BYTES;
            rope_issue_tables(g, const_cast<char*>(rope_tab), pos_lds, wave_s, lane_id_here());
            wait_vmcnt<0>();
          }
          __builtin_amdgcn_s_barrier();  // every wave's table rows have landed
        }
      }
    };
    auto ln_table = [&]() {  // every wave takes part (barriers)
      if constexpr (LNF == 1) {
        // this wave's copy has landed: the loads issued after it (at least
        // NS - 1 stages when the unit has more K steps than the ring) may
        // still be in flight, older ones not
        if (nk >= NS + 1)
          wait_vmcnt<G * (NS - 1)>();
        else
          wait_vmcnt<0>();
        __syncthreads();
        const int tid_e = wave_s * 64 + lane_id_here();
        if (tid_e < BM) ln_fold_table(g, fold_lds, fold_tab, tid_e, BM);
        __syncthreads();
      }
    };
    const int unit_rows = th < 0 ? BM : BM / 2;
    if (idle) {
      kloop(std::false_type{});
      stage_tables();
      ln_table();
      if constexpr (LNF == 2) {
        {  // its barriers
          const int lane_e = lane_id_here();
          resid_ln_epilogue<BM, BN, TT::WM, TT::WN, TI, TJ, WGN>(
              g, acc, m0, unit_rows, tn, wm_s, wave_s % WGN, lane_e & 31, lane_e >> 5, wave_s * 64 + lane_e, false,
              reinterpret_cast<float*>(fold_lds), reinterpret_cast<float*>(fold_lds) + WGN * BM);
        }
      }
      continue;
    }
    kloop(std::true_type{});
    stage_tables();
    ln_table();
    // the epilogue's lane and wave indices, recomputed after the K loop
    // rather than held through it
    const int lane_e = lane_id_here(), l32e = lane_e & 31, hbe = lane_e >> 5;
    const int wme = wm_s, wne = wave_s % WGN;
    if constexpr (W8) {
      // row n of W stands for code * w_scale[n]: scale the accumulators
      if constexpr (kSwap) {
        // the lane's four consecutive W rows 8q + 4hb .. + 3 of block j; a
        // clamped (past-the-end) group reads in-bounds scales of outputs that
        // are never stored
        const int64_t nrows = EPI == EPI_GEGLU ? 2 * static_cast<int64_t>(g.N) : g.N;
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t r0 = min(mfma_w_row<BN, TT::WN, EPI>(g, tn, wne * TT::WN + j * 32 + 8 * q + 4 * hbe),
                                   nrows - 4);
            const f32x4_t sc = *reinterpret_cast<const f32x4_t*>(g.w_scale + r0);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
              for (int i = 0; i < TI; ++i) acc[i][j][4 * q + t] *= sc[t];
          }
      } else {
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          const float sc = g.w_scale[mfma_w_row<BN, TT::WN, EPI>(g, tn, wne * TT::WN + j * 32 + l32e)];
#pragma unroll
          for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] *= sc;
        }
      }
    }
    if constexpr (LNF == 1)  // A holds folded LayerNorm rows
      ln_fold_acc<BM, BN, TT::WM, TT::WN, TI, TJ, EPI, kSwap>(g, acc, tn, wme, wne, l32e, hbe, fold_tab);
    if constexpr (LNF == 2) {  // the next LayerNorm's input rows and moments too
      resid_ln_epilogue<BM, BN, TT::WM, TT::WN, TI, TJ, WGN>(
          g, acc, m0, unit_rows, tn, wme, wne, l32e, hbe, wave_s * 64 + lane_e, true, reinterpret_cast<float*>(fold_lds),
          reinterpret_cast<float*>(fold_lds) + WGN * BM);
      continue;
    }
    if constexpr (LNF == 3) {  // and the next LayerNorm, finished with the panel's other tiles
      resid_rln_epilogue<BM, BN, TT::WM, TT::WN, TI, TJ, WGN>(g, acc, m0, tm, tn, wme, wne, l32e, hbe,
                                                             wave_s * 64 + lane_e, fold_lds);
      continue;
    }
    if constexpr (kSwap)
      pers_epilogue<BM, BN, TT::WM, TT::WN, TI, TJ, EPI, OutT>(g, acc, m0, tn, wme, wne, l32e, hbe);
    else
      gemm_epilogue<BM, BN, TT::WM, TT::WN, TI, TJ, EPI, OutT, kRopeLds>(g, acc, m0, tn, wme, wne, l32e, hbe,
                                                               rope_tab);
  }
}

int num_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    hip_check(hipGetDevice(&dev), "gemm: hipGetDevice");
    hip_check(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev),
              "gemm: CU count");
    n = v > 0 ? v : 256;
  }
  return n;
}

template <int BM, int BN, int WGM, int WGN, int NS, int BK, bool W8, int EPI, typename OutT, int LNF>
void launch_pers_kernel(const GemmArgs& g, hipStream_t st) {
  // (+ 1 KB of row positions for the RoPE epilogue, + a folded LayerNorm's
  // tables: the consumer's moments copy (8 bytes per row and block) and row
  // table (16 + 4 bytes per row), or the producer's WGN + 1 floats per row)
  constexpr int fold = LNF == 1   ? BM * (kLnMaxBlocks * 8 + 20)
                       : LNF == 2 ? 4 * (WGN + 1) * BM
                       : LNF == 3 ? 4 * (WGN + 3) * BM + 16
                                  : 0;
  constexpr int lds = NS * PTile<BM, BN, WGM, WGN, NS, BK, W8>::STAGE_BYTES + 1024 + fold;
  static_assert(lds <= 160 * 1024, "LDS");
  auto kern = gemm_bf16_pers_kernel<BM, BN, WGM, WGN, NS, BK, W8, EPI, OutT, LNF>;
  static bool attr_set = false;
  if (!attr_set) {
    hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, lds),
              "gemm: LDS attribute");
    attr_set = true;
  }
  const int tiles_n = EPI == EPI_GEGLU ? (g.N + BN / 2 - 1) / (BN / 2) : (g.N + BN - 1) / BN;
  const int64_t tiles = static_cast<int64_t>(tiles_n) * ((g.M + BM - 1) / BM);
  require(tiles < (int64_t{1} << 30), "gemm: too many tiles");
  constexpr int occ = pers_occupancy<BM, BN, WGM, WGN, NS, BK, W8>();
  const int grid = static_cast<int>(std::min<int64_t>(tiles, int64_t{occ} * num_cus()));
  // a tile of a LayerNorm-finishing launch waits for its panel's other tiles:
  // each of them needs a workgroup of its own (one round)
  if constexpr (LNF == 3) require(grid == tiles, "gemm: the residual epilogue's LayerNorm needs a workgroup per tile");
  kern<<<grid, 64 * WGM * WGN, lds, st>>>(g);
}

template <int BM, int BN, int WGM, int WGN, int NS, int BK, bool W8>
void launch_pers(const GemmArgs& g, hipStream_t st) {
  const bool bf = g.out_dtype == DT_BF16;
  // a folded LayerNorm's consumer: bf16 outputs of the QKV and GEGLU products
  const bool lni = g.ln_stats_in != nullptr;
  require(!lni || (bf && (g.epi == EPI_ROPE || g.epi == EPI_GEGLU)),
          "gemm: a folded LayerNorm's consumer is a bf16 RoPE or GEGLU product");
  switch (g.epi) {
    case EPI_STORE:
      bf ? launch_pers_kernel<BM, BN, WGM, WGN, NS, BK, W8, EPI_STORE, bf16_t, 0>(g, st)
         : launch_pers_kernel<BM, BN, WGM, WGN, NS, BK, W8, EPI_STORE, float, 0>(g, st);
      break;
    case EPI_RESID:
      if constexpr (!W8 && BM == 256 && BN == 256 && WGM == 4 && WGN == 4) {
        if (g.rln_y) {
          launch_pers_kernel<BM, BN, WGM, WGN, NS, BK, W8, EPI_RESID, float, 3>(g, st);
          break;
        }
      }
      require(!g.rln_y, "gemm: the residual epilogue's LayerNorm needs the bf16 256 x 256 tile");
      g.ln_y ? launch_pers_kernel<BM, BN, WGM, WGN, NS, BK, W8, EPI_RESID, float, 2>(g, st)
             : launch_pers_kernel<BM, BN, WGM, WGN, NS, BK, W8, EPI_RESID, float, 0>(g, st);
      break;
    case EPI_ROPE:
      lni  ? launch_pers_kernel<BM, BN, WGM, WGN, NS, BK, W8, EPI_ROPE, bf16_t, 1>(g, st)
      : bf ? launch_pers_kernel<BM, BN, WGM, WGN, NS, BK, W8, EPI_ROPE, bf16_t, 0>(g, st)
           : launch_pers_kernel<BM, BN, WGM, WGN, NS, BK, W8, EPI_ROPE, float, 0>(g, st);
      break;
    default:
      lni  ? launch_pers_kernel<BM, BN, WGM, WGN, NS, BK, W8, EPI_GEGLU, bf16_t, 1>(g, st)
      : bf ? launch_pers_kernel<BM, BN, WGM, WGN, NS, BK, W8, EPI_GEGLU, bf16_t, 0>(g, st)
           : launch_pers_kernel<BM, BN, WGM, WGN, NS, BK, W8, EPI_GEGLU, float, 0>(g, st);
      break;
  }
}

template <int BM, int BN, int WGM, int WGN, int NS, int BK, int EPI, typename OutT>
void launch_mfma_kernel(const GemmArgs& g, dim3 grid, hipStream_t st) {
  constexpr int lds = NS * DTile<BM, BN, WGM, WGN, NS, BK>::STAGE_BYTES;
  auto kern = gemm_bf16_dma_kernel<BM, BN, WGM, WGN, NS, BK, EPI, OutT>;
  static bool attr_set = false;  // per instantiation; the attribute is per function
  if (!attr_set) {
    hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, lds),
              "gemm: LDS attribute");
    attr_set = true;
  }
  kern<<<grid, 64 * WGM * WGN, lds, st>>>(g);
}

template <int BM, int BN, int WGM, int WGN, int NS, int BK, int EPI>
void launch_mfma_tile(const GemmArgs& g, hipStream_t st) {
  const int tiles_n = EPI == EPI_GEGLU ? g.N / (BN / 2) : (g.N + BN - 1) / BN;
  const int64_t tiles = static_cast<int64_t>(tiles_n) * ((g.M + BM - 1) / BM);
  require(tiles < (int64_t{1} << 31), "gemm: too many tiles");
  dim3 grid(static_cast<unsigned>(tiles));
  if (g.out_dtype == DT_BF16 || EPI == EPI_RESID)
    launch_mfma_kernel<BM, BN, WGM, WGN, NS, BK, EPI, bf16_t>(g, grid, st);
  else
    launch_mfma_kernel<BM, BN, WGM, WGN, NS, BK, EPI, float>(g, grid, st);
}

template <int BM, int BN, int WGM, int WGN, int NS, int BK>
void launch_mfma_epi(const GemmArgs& g, hipStream_t st) {
  switch (g.epi) {
    case EPI_STORE: launch_mfma_tile<BM, BN, WGM, WGN, NS, BK, EPI_STORE>(g, st); break;
    case EPI_RESID: launch_mfma_tile<BM, BN, WGM, WGN, NS, BK, EPI_RESID>(g, st); break;
    case EPI_ROPE: launch_mfma_tile<BM, BN, WGM, WGN, NS, BK, EPI_ROPE>(g, st); break;
    default: launch_mfma_tile<BM, BN, WGM, WGN, NS, BK, EPI_GEGLU>(g, st); break;
  }
}

#ifndef SJH_GEMM_BIG
#define SJH_GEMM_BIG 256, 256, 4, 4, 2, 64
#endif
#ifndef SJH_GEMM_MID
#define SJH_GEMM_MID 128, 128, 2, 2, 2, 64
#endif

// Tile shapes by row count (BM, BN, wave grid, ring stages, K step): 256x256
// with 16 waves of 64x64 (4 waves per SIMD hide the LDS and MFMA latencies)
// for the throughput shapes; 128x128 with 4 waves for mid-size batches;
// 64x64 with 2 waves of 32x64 and a 4-stage ring for short ones (batch-1
// latency): more workgroups spread the weight reads over the CUs, and three
// stages in flight cover the load latency that bounds such a short loop.
#ifndef SJH_GEMM_PERS
#define SJH_GEMM_PERS 256, 256, 4, 4, 2, 64
#endif
// fp8 weights: 48 KB stages (bf16 A rows, fp8 W rows), three in the ring; 16
// waves of 64 x 64 as in the bf16 kernel (one workgroup per CU, 4 waves per
// SIMD; config 5's QKV, Wo and Wo2 products 7-9% faster than with 8 waves of
// 128 x 64, GEGLU equal)
#ifndef SJH_GEMM_PERS_FP8
#define SJH_GEMM_PERS_FP8 256, 256, 4, 4, 3, 64
#endif

#ifndef SJH_GEMM_SMALL
#define SJH_GEMM_SMALL 64, 64, 2, 1, 4, 64
#endif
// Up to SJH_SMALL32_MAX_M rows (batch-1 latency), the GEGLU and plain
// products take 32-column tiles: a CU streams W at ~25 GB/s at most, so half
// the W rows per workgroup on twice the workgroups shortens the K loop
// (batch-1 Wi + GEGLU 10.2 -> 8.1 us per launch).  A GEGLU tile's input and
// gate rows meet in the epilogue by a lane swap, and so do the rotation
// pairs of a RoPE tile (head_dim 64: 16 dims of a head and their partners 32
// higher; batch-1 p50 1.084 -> 1.074 ms against 64-column RoPE tiles).
#ifndef SJH_GEMM_SMALL32
#define SJH_GEMM_SMALL32 64, 32, 2, 1, 4, 64
#endif
#ifndef SJH_SMALL32_MAX_M
#define SJH_SMALL32_MAX_M 256
#endif
#ifndef SJH_SPLITK_MAX_M
#define SJH_SPLITK_MAX_M 256
#endif

// The persistent kernel's epilogues write 8- and 16-byte vectors, and its
// loads address each operand by 32-bit byte offsets.
bool pers_ok(const GemmArgs& g) {
  const int64_t w_rows = g.epi == EPI_GEGLU ? 2 * static_cast<int64_t>(g.N) : g.N;
  const int64_t w_bytes = g.w_dtype == DT_FP8 ? 1 : 2;
  return g.N % 4 == 0 && g.ldo % 4 == 0 && g.ldx % 4 == 0 && aligned16(g.out) &&
         aligned16(g.X) && aligned16(g.bias) && aligned16(g.rope_cos) && aligned16(g.rope_sin) &&
         static_cast<int64_t>(g.M) * g.lda * 2 < (int64_t{1} << 32) &&
         w_rows * g.ldw * w_bytes < (int64_t{1} << 32) &&
         (g.epi != EPI_ROPE || static_cast<int64_t>(g.rope_rows) * 128 < (int64_t{1} << 32));
}

void launch_mfma(const GemmArgs& g, hipStream_t st) {
  if (g.M >= 4096 && pers_ok(g))
    launch_pers<SJH_GEMM_PERS, false>(g, st);
  else if (g.M >= 4096 && (g.epi != EPI_GEGLU || g.N % 128 == 0))
    launch_mfma_epi<SJH_GEMM_BIG>(g, st);
  else if (g.M >= 1024)
    launch_mfma_epi<SJH_GEMM_MID>(g, st);
  else if (g.M <= SJH_SMALL32_MAX_M && g.epi == EPI_GEGLU)
    launch_mfma_tile<SJH_GEMM_SMALL32, EPI_GEGLU>(g, st);
  else if (g.M <= SJH_SMALL32_MAX_M && g.epi == EPI_STORE)
    launch_mfma_tile<SJH_GEMM_SMALL32, EPI_STORE>(g, st);
  else if (g.M <= SJH_SMALL32_MAX_M && g.epi == EPI_ROPE && g.head_dim == 64 && g.N % 64 == 0)
    launch_mfma_tile<SJH_GEMM_SMALL32, EPI_ROPE>(g, st);
  else
    launch_mfma_epi<SJH_GEMM_SMALL>(g, st);
}

// ------------------------------------------------------------------ split-K
// Short batches (M <= 256, e.g. batch-1 latency) have too few output tiles to
// spread the weight reads over the CUs.  K is cut into splits; each split's
// partial product goes to g.partial, and splitk_epilogue_kernel adds the
// splits in order and applies the epilogue (one thread per output).  The
// kernel boundary between the two is what makes every split's partials
// visible to the epilogue, whichever XCD wrote them.
__device__ __forceinline__ float splitk_sum(const GemmArgs& g, int S, int m, int col) {
  float v = 0.f;
  for (int sp = 0; sp < S; ++sp) v += g.partial[(static_cast<int64_t>(sp) * g.part_rows + m) * g.n_w + col];
  return v;
}

// Output (m, n) of a split-K GEMM from the partial sums of all S splits.
template <typename OutT>
__device__ void splitk_output(const GemmArgs& g, int S, int m, int n) {
  if (g.epi == EPI_RESID) {
    float v = splitk_sum(g, S, m, n);
    if (g.bias) v += g.bias[n];
    g.X[static_cast<int64_t>(m) * g.ldx + n] += v;
    return;
  }
  OutT* out = static_cast<OutT*>(g.out) + static_cast<int64_t>(m) * g.ldo + n;
  if (g.epi == EPI_GEGLU) {
    store_f32(out, gelu_out<OutT>(splitk_sum(g, S, m, n)) * splitk_sum(g, S, m, g.N + n));
    return;
  }
  float v = splitk_sum(g, S, m, n);
  if (g.epi == EPI_ROPE) {
    if (n < 2 * g.rope_dim) {
      const int half = g.head_dim >> 1, d = n % g.head_dim;
      const int64_t p = min(max(g.pos[m], 0), g.rope_rows - 1);
      if (d < half) {
        v = rope_lo(v, splitk_sum(g, S, m, n + half), g.rope_cos[p * half + d],
                    g.rope_sin[p * half + d]);
      } else {
        v = rope_hi(splitk_sum(g, S, m, n - half), v, g.rope_cos[p * half + d - half],
                    g.rope_sin[p * half + d - half]);
      }
      if (n < g.rope_dim) v *= g.q_scale;
    }
  } else {
    if (g.bias) v += g.bias[n];
    if (g.act == 1)
      v = gelu_out<OutT>(v);
    else if (g.act == 2)
      v = fmaxf(v, 0.f);
  }
  store_f32(out, v);
}

template <typename OutT>
__global__ __launch_bounds__(256) void splitk_epilogue_kernel(GemmArgs g0, int S) {
  const GemmArgs g = resolve_rows(g0);
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<int64_t>(g.M) * g.N) return;
  const int m = static_cast<int>(idx / g.N);
  splitk_output<OutT>(g, S, m, static_cast<int>(idx - static_cast<int64_t>(m) * g.N));
}

// Split-K tile: 128 x 64 with 4 waves of 64 x 32.
constexpr int kSkBM = 128, kSkBN = 64;

template <int EPI>
void launch_splitk_epi(const GemmArgs& g, dim3 grid, hipStream_t st) {
  constexpr int lds = 2 * DTile<kSkBM, kSkBN, 2, 2, 2, 64>::STAGE_BYTES;
  auto kern = g.out_dtype == DT_BF16 || EPI == EPI_RESID
                  ? gemm_bf16_dma_kernel<kSkBM, kSkBN, 2, 2, 2, 64, EPI, bf16_t, true>
                  : gemm_bf16_dma_kernel<kSkBM, kSkBN, 2, 2, 2, 64, EPI, float, true>;
  kern<<<grid, 256, lds, st>>>(g);
}

// Launches the split-K product (partials only) and returns the number of
// splits, or 0 (nothing launched) when the workspace is too small or K too
// short to split.
int launch_splitk_partials(GemmArgs& g, hipStream_t st) {
  g.n_w = g.epi == EPI_GEGLU ? 2 * g.N : g.N;
  g.part_rows = g.M;
  if (g.epi == EPI_GEGLU && g.N % (kSkBN / 2) != 0) return 0;
  const int tiles_n = g.epi == EPI_GEGLU ? g.N / (kSkBN / 2) : (g.N + kSkBN - 1) / kSkBN;
  const int tiles = ((g.M + kSkBM - 1) / kSkBM) * tiles_n;
  const int nk = g.K / kBK;
  // enough workgroups to cover the CUs, at least two K steps per split
  int S = std::min(std::max(1, (512 + tiles - 1) / tiles), std::max(1, nk / 2));
  S = std::min(S, 16);
  g.k_chunk = (nk + S - 1) / S;
  S = (nk + g.k_chunk - 1) / g.k_chunk;
  if (S < 2 || static_cast<int64_t>(S) * g.M * g.n_w > g.partial_cap) return 0;
  dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(S));
  switch (g.epi) {
    case EPI_STORE: launch_splitk_epi<EPI_STORE>(g, grid, st); break;
    case EPI_RESID: launch_splitk_epi<EPI_RESID>(g, grid, st); break;
    case EPI_ROPE: launch_splitk_epi<EPI_ROPE>(g, grid, st); break;
    default: launch_splitk_epi<EPI_GEGLU>(g, grid, st); break;
  }
  check_launch("gemm_splitk");
  return S;
}

// Returns false (caller takes the regular path) when the workspace is too
// small or K too short to split.
bool launch_splitk(const GemmArgs& g0, hipStream_t st) {
  GemmArgs g = g0;
  const int S = launch_splitk_partials(g, st);
  if (S == 0) return false;
  const int64_t outs = static_cast<int64_t>(g.M) * g.N;
  dim3 eg(static_cast<unsigned>((outs + 255) / 256));
  if (g.out_dtype == DT_BF16 || g.epi == EPI_RESID)
    splitk_epilogue_kernel<bf16_t><<<eg, 256, 0, st>>>(g, S);
  else
    splitk_epilogue_kernel<float><<<eg, 256, 0, st>>>(g, S);
  check_launch("gemm_splitk_epilogue");
  return true;
}

// ------------------------------------------------------------------ generic
constexpr int gBM = 64, gBN = 64, gBK = 16;
constexpr int gLdc = gBN + 4;

template <typename InT, typename OutT>
__global__ __launch_bounds__(256) void gemm_generic_kernel(GemmArgs g0) {
  const GemmArgs g = resolve_rows(g0);
  constexpr int kStage = 2 * gBK * (gBM + 1);  // As[k][m] and Ws[k][n]
  constexpr int kFloats = kStage > gBM * gLdc ? kStage : gBM * gLdc;
  __shared__ float smem[kFloats];
  float* As = smem;
  float* Ws = smem + gBK * (gBM + 1);

  const int tile_n = blockIdx.x, tile_m = blockIdx.y;
  const int m0 = tile_m * gBM;
  if (m0 >= g.M) return;  // uniform
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

// The bf16 MFMA kernels' operand requirements.
bool mfma_ok(const GemmArgs& g) {
  return g.in_dtype == DT_BF16 && g.w_dtype == DT_BF16 && g.K % kBK == 0 && g.lda % 8 == 0 &&
         g.ldw % 8 == 0 && aligned16(g.A) && aligned16(g.W) &&
         (g.epi != EPI_ROPE || g.head_dim == 64) && (g.epi != EPI_GEGLU || g.N % 64 == 0);
}

bool gemm_takes_ln_fold(const GemmArgs& g) {
  if (g.M <= 0 || g.N <= 0 || g.K <= 0 || !g.A || !g.W) return false;
  if (g.w_dtype == DT_FP8)  // the persistent kernel always (launch_gemm's checks)
    return g.in_dtype == DT_BF16 && g.w_scale && aligned16(g.w_scale) && g.K % 64 == 0 &&
           g.lda % 8 == 0 && g.ldw % 16 == 0 && aligned16(g.A) && aligned16(g.W) && pers_ok(g) &&
           (g.epi != EPI_ROPE || g.head_dim == 64);
  return g.w_dtype == DT_BF16 && mfma_ok(g) && g.M >= 4096 && pers_ok(g);  // launch_mfma's first choice
}

bool gemm_takes_rln(const GemmArgs& g) {
  if (g.epi != EPI_RESID || g.w_dtype != DT_BF16 || g.M <= 0 || g.N % kLnBlock != 0 ||
      g.N / kLnBlock > kLnMaxBlocks || !g.A || !g.W || !g.X)
    return false;
  if (!(mfma_ok(g) && g.M >= 4096 && pers_ok(g))) return false;  // launch_mfma's persistent path
  // one round: every tile a workgroup of its own, all resident at once
  const int64_t tiles = static_cast<int64_t>(g.N / kLnBlock) * ((g.M + 255) / 256);
  return tiles <= static_cast<int64_t>(pers_occupancy<SJH_GEMM_PERS, false>()) * num_cus();
}

int launch_gemm_resid_partials(const GemmArgs& g0, hipStream_t st) {
  if (g0.epi != EPI_RESID || g0.M <= 0 || g0.M > SJH_SPLITK_MAX_M || g0.N <= 0 || g0.K <= 0 || !g0.partial ||
      !g0.A || !g0.W || !g0.X || g0.lda < g0.K || g0.ldw < g0.K || g0.ldx < g0.N || !mfma_ok(g0))
    return 0;
  GemmArgs g = g0;
  return launch_splitk_partials(g, st);
}

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
      require(g.pos && g.rope_cos && g.rope_sin && g.rope_rows > 0,
              "gemm: ROPE needs positions and tables");
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
  if (g.rln_y) {
    require(gemm_takes_rln(g), "gemm: the residual epilogue finishes a LayerNorm only on one round of 256 x 256 "
                               "bf16 tiles with N a multiple of 256 up to 1024");
    require(g.rln_w && g.rln_mom && g.rln_sync && g.rln_ldy >= g.N && g.rln_spin > 0 && g.rln_eps > 0.f &&
                !g.ln_y && !g.ln_stats_in,
            "gemm: the residual epilogue's LayerNorm needs weights, moments, sync ints, a poll bound and ldy >= N");
  }
  if (g.ln_y || g.ln_stats_in) {
    require(gemm_takes_ln_fold(g),
            "gemm: a folded LayerNorm needs the persistent kernel (bf16 activations and M >= 4096, or fp8 weights)");
    require(!g.ln_y || (g.epi == EPI_RESID && g.N % kLnBlock == 0 && g.ln_w && g.ln_stats_out &&
                        aligned16(g.ln_y) && aligned16(g.ln_stats_out) && g.ldx % 8 == 0),
            "gemm: a folded LayerNorm's producer is a residual GEMM with N % 256 == 0, weights, moments "
            "and 16-byte aligned rows");
    require(!g.ln_stats_in || (g.K % kLnBlock == 0 && g.K / kLnBlock <= kLnMaxBlocks && g.ln_c1 &&
                               aligned16(g.ln_c1) && aligned16(g.ln_stats_in) && g.ln_eps > 0.f),
            "gemm: a folded LayerNorm's consumer needs K % 256 == 0, K <= 1024, c1 rows and moments");
  }
  if (g.w_dtype == DT_FP8) {
    // fp8 weights: the persistent kernel only (16-byte fp8 rows chunks)
    require(g.in_dtype == DT_BF16, "gemm: fp8 weights need bf16 activations");
    require(g.w_scale && aligned16(g.w_scale), "gemm: fp8 weights need per-row scales");
    require(g.K % 64 == 0 && g.lda % 8 == 0 && g.ldw % 16 == 0 && aligned16(g.A) &&
                aligned16(g.W),
            "gemm: fp8 weights need K % 64 == 0 and 16-byte aligned rows");
    require(pers_ok(g), "gemm: fp8 weights need N % 4 == 0, 16-byte aligned outputs and operands under 4 GiB");
    require(g.epi != EPI_ROPE || g.head_dim == 64, "gemm: fp8 RoPE epilogue needs head_dim 64");
    launch_pers<SJH_GEMM_PERS_FP8, true>(g, st);
    check_launch("gemm_fp8w");
    return;
  }
  require(g.w_dtype == DT_BF16 || g.w_dtype == DT_F32, "gemm: unknown weight type");
  const bool mfma = g.in_dtype == DT_BF16 && g.K % kBK == 0 && g.lda % 8 == 0 &&
                    g.ldw % 8 == 0 && aligned16(g.A) && aligned16(g.W) &&
                    (g.epi != EPI_ROPE || g.head_dim == 64) &&
                    (g.epi != EPI_GEGLU || g.N % 64 == 0);
  if (g.epi == EPI_ROPE && !mfma)
    require(gBN % g.head_dim == 0, "gemm: ROPE epilogue needs head_dim dividing 64");
  // split-K only for the residual epilogue: its few output tiles (N = D)
  // leave most CUs idle otherwise; the wider products (QKV, GEGLU) have
  // enough tiles, and a second epilogue kernel costs more than it saves
  if (mfma && g.partial && g.M <= SJH_SPLITK_MAX_M && g.epi == EPI_RESID && launch_splitk(g, st)) return;
  if (mfma) {
    launch_mfma(g, st);
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

// attn.hip -- non-causal varlen flash attention for gfx950.
//
// Fast path (bf16, head_dim 64): one workgroup = (sequence, head, 128
// queries); 4 waves own 32 queries each.  Key/value tiles of 64 rows move
// from HBM into a 2-stage LDS ring (32 KB) with direct-to-LDS loads,
// row-major and XOR-swizzled; three workgroups share a CU, so one
// workgroup's softmax overlaps the others' MFMAs.  Per tile a wave computes
// S^T = K . Q^T with
// v_mfma_f32_32x32x16_bf16 (the query is the MFMA column, so each lane owns
// one query and 32 of the tile's keys), does the online-softmax update in
// registers (exp2 of log2-domain logits; a first pass without any running
// max, checked afterwards, else the max rule with one cross-half exchange
// for the row max), and accumulates
// O^T += V^T . P^T.  The accumulator of S^T is already laid out as the B
// operand of the second MFMA once the key order inside a 16-key step is taken
// as the MFMA's k order, so P never leaves registers; the V^T operand comes
// straight from the row-major V tile through transposed LDS reads
// (ds_read_b64_tr_b16).
//
// Generic path (fp32 or bf16, head_dim 8/16/32/64/128): one thread per query,
// K/V tiles of 32 keys in LDS (broadcast reads), blocked online softmax with
// expf.  It serves the fp32 parity mode.
//
// Masking follows src/tensor.cpp:186-192: query i sees keys
// [0, k_len) (full) or [max(0, i-w), min(k_len, i+w+1)) (window w).  A query
// with no visible key yields zeros, as the reference does for len = 0.
#include <type_traits>

#include "sjh_common.hpp"
#include "sjh_host.hpp"
#include "sjh_kernels.hpp"

namespace sjh {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kQ = 128;     // queries per workgroup (4 waves x 32)
constexpr int kKey = 64;    // keys per tile
constexpr int kNS = 2;      // LDS ring stages (2 x 16 KB)
constexpr float kLazy = 8.f;  // log2 headroom before the running max is raised
// Pre-scaled queries (q already times scale * log2 e, so the QK^T MFMA gives
// log2-domain logits): the offset subtracted before exp2 is 0 whenever the
// tile's max lies in [kZeroLo, kZeroHi] and is otherwise raised lazily with
// kLazyPre of headroom; with a zero offset the exp2 argument is the MFMA
// result itself (no multiply-add per logit).  exp2 of up to 2^32 and a sum
// of 8192 such terms times V stay far inside fp32 and bf16 range.
constexpr float kLazyPre = 32.f, kZeroLo = -64.f, kZeroHi = 32.f;
constexpr int kStage = 2 * kKey * 128;  // bytes per stage: K tile then V tile, 64 x 128 B each

typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((ext_vector_type(8))) short s16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ float wave_max32(float v) {
  // lanes l and l^32 hold the two halves of one query's keys: one
  // v_permlane32_swap hands each half the other's value (no LDS round trip)
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Chunk position of 16-byte chunk c of tile row r is c ^ kv_swz(r), a
// permutation of (r >> 1) & 7 (rows r and r + 16 share the key).  LDS serves
// 256 bytes (64 banks) per cycle and a 128-byte row covers half of them, so
// even and odd rows fall in different halves: 16 consecutive rows read at one
// logical chunk (K fragments) then hit 16 distinct bank groups, and the four
// rows r0 + [0, 4) that half a wave's transposed V reads cover (chunks
// 4 db + [0, 4) of each) do too, since rows r0 and r0 + 2 differ in the
// key's bit 2.
__device__ __forceinline__ int kv_swz(int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); }

// LDS byte offset of element (row, col) of a 64 x 64 bf16 tile.
__device__ __forceinline__ int kv_off(int row, int col) {
  return row * 128 + (((col >> 3) ^ kv_swz(row)) << 4) + ((col & 7) << 1);
}

// Buffer descriptor over the n_bytes bytes from p on (untyped dword loads:
// word 3 carries gfx9's 32-bit data format).  A load at or past n_bytes
// returns zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t seq_rsrc(const bf16_t* p, uint32_t n_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(p), static_cast<short>(0),
                                           static_cast<int>(n_bytes), 0x00020000);
}

// 16 bytes per lane from buffer r at voff + soff into LDS at lds + 16 * lane
// (buffer_load_dwordx4 ... lds; the LDS base goes through M0).
__device__ __forceinline__ void load_lds16_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, char* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds), 16,
                                           static_cast<int>(voff), static_cast<int>(soff), 0, 0);
}

// Transposed 8-byte LDS read (ds_read_b64_tr_b16) at LDS byte address
// addr + OFF.  Within each 16-lane group, if lane q + 4k addresses element
// (r0 + k, c0 + 4q) of a row-major tile, lane i of the group receives
// elements (r0 + k, c0 + i), k = 0..3.
//
// Inline asm rather than the builtin: before the builtin's read the compiler
// waits for every direct-to-LDS load in flight (vmcnt(0)), which would hold
// each tile's P.V phase until the next tile's K/V loads (into the other ring
// slot) have landed.  The asm is invisible to the compiler's wait insertion,
// so its results are claimed with lgkm_claim before their first use.
template <int OFF>
__device__ __forceinline__ s16x4_t lds_read_tr(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  s16x4_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
  return r;
}
// Waits until at most N LDS operations of this wave are outstanding, tied to
// the four registers it makes valid (the compiler cannot move their uses
// above it).  LDS operations complete in issue order, so N = the number of
// LDS reads issued after the four means those four have returned; LDS
// operations the compiler issues in between only make the wait longer.
template <int N>
__device__ __forceinline__ void lgkm_claim(s16x4_t& a, s16x4_t& b, s16x4_t& c, s16x4_t& d) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt immediate");
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N));
}
// f(integral_constant<int, I>) for I = B .. E - 1 in turn: loop indices that
// the asm operands above need as compile-time constants.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}
// LDS byte address of a pointer into the workgroup's LDS.
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}

// Register budget for three workgroups per CU (168 VGPRs, 3 waves per SIMD):
// a third wave per SIMD lets softmax VALU work, MFMAs and LDS reads of
// different waves overlap.  (The pre-scaled kernel spills 3 VGPRs on the
// max-rule rerun only, past the redo vote; the common path has no scratch
// access.)  PRE: q holds q * scale * log2 e (AttnArgs::
// q_log2_scaled).
// One work item: queries [q0, q0 + kQ) of head h of the sequence whose rows
// start at row0 (q0 < qlen).  half 0: all keys; 1: keys [0, mid), 2: keys
// [mid, klen) with mid = klen / 2 rounded up to a whole tile (full attention
// only), the unnormalised result going to part (kAttnPartFloats floats).
// WO: the output projection folded in (AttnArgs::wo): the workgroup's
// kAttnWoCols rows of Wo (grid y) go to LDS at kWoLds while the item runs,
// and the item writes its partial product instead of O.
constexpr int kWoLds = kNS * kStage + 1024;
template <bool PRE, bool WO = false>
__device__ __forceinline__ void attn_item(const AttnArgs& a, char* smem, int64_t row0, int qlen, int klen,
                                          int h, int q0, int half = 0, float* part = nullptr) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hb = lane >> 5;
  const int n0 = WO ? static_cast<int>(blockIdx.y) * kAttnWoCols : 0;
  if constexpr (WO) {
    // rows n0 + [0, kAttnWoCols) of Wo, columns 64 h + [0, 64): 128-byte
    // rows swizzled as the K/V tiles (kv_off), groups of 8 rows per load,
    // wave w moving groups w, w + 4, ...
    const bf16_t* Wo = static_cast<const bf16_t*>(a.wo) + static_cast<int64_t>(n0) * a.ld_wo + h * 64;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
    for (int i = 0; i < kAttnWoCols / 32; ++i) {
      const int grp = wave_u + 4 * i;
      const int r = 8 * grp + (lane >> 3);
      load_lds16(Wo + static_cast<int64_t>(r) * a.ld_wo + (((lane & 7) ^ kv_swz(r)) << 3),
                 smem + kWoLds + grp * 1024);
    }
  }

  const bf16_t* Q = static_cast<const bf16_t*>(a.q) + h * 64;
  const bf16_t* K = static_cast<const bf16_t*>(a.k) + h * 64;
  const bf16_t* V = static_cast<const bf16_t*>(a.v) + h * 64;

  // this lane's query (clamped for the load; rows past q_len are not stored)
  const int qi = q0 + wave * 32 + l32;
  const bool wave_active = q0 + wave * 32 < qlen;
  const int64_t qrow = row0 + min(qi, qlen - 1);
  bf16x8_t qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    qf[s] = *reinterpret_cast<const bf16x8_t*>(Q + qrow * a.ld_q + 16 * s + 8 * hb);

  int klo = 0, khi = klen;
  if (a.window > 0) {
    klo = max(0, q0 - a.window);
    khi = min(klen, q0 + kQ - 1 + a.window + 1);
  } else if (half > 0) {
    const int mid = ((klen + 1) / 2 + kKey - 1) / kKey * kKey;
    if (half == 1)
      khi = mid;
    else
      klo = mid;
  }
  const int qlo = a.window > 0 ? max(0, qi - a.window) : 0;
  const int qhi = a.window > 0 ? min(klen, qi + a.window + 1) : klen;
  const int ntiles = khi > klo ? (khi - klo + kKey - 1) / kKey : 0;

  // DMA: a stage is 16 row groups of 8 rows x 128 B (groups 0-7 K, 8-15 V);
  // wave w moves groups w, w + 4, w + 8, w + 12.  Lane l carries row
  // 8 * (group % 8) + l / 8 and lands in chunk slot l % 8, so it reads the
  // logical chunk (l % 8) ^ kv_swz(row).
  // Groups i = 0, 1 are K rows, 2, 3 V rows.  The loads go through buffer
  // descriptors based at the sequence's first K and V rows: a full tile is
  // the tile's row offset (scalar) plus the lane's fixed byte offset, with no
  // per-lane address arithmetic; a tile that runs past klen takes 32-bit
  // lane offsets from the sequence's base, and its rows past the last key
  // fall outside the descriptors and load as zeros.
  const int lrow = lane >> 3, cslot = lane & 7;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  uint32_t goff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 8 * ((wave + 4 * i) & 7) + lrow;
    goff[i] = static_cast<uint32_t>(r * (i < 2 ? a.ld_k : a.ld_v) * 2 + ((cslot ^ kv_swz(r)) << 4));
  }
  // the descriptors end with the head's 64 values of key klen - 1: the rows
  // past the keys read as zeros
  const uint32_t kstride = static_cast<uint32_t>(a.ld_k * 2), vstride = static_cast<uint32_t>(a.ld_v * 2);
  const uint32_t klast = static_cast<uint32_t>(max(klen - 1, 0));
  const __amdgpu_buffer_rsrc_t rk = seq_rsrc(K + row0 * a.ld_k, klast * kstride + 128u);
  const __amdgpu_buffer_rsrc_t rv = seq_rsrc(V + row0 * a.ld_v, klast * vstride + 128u);
  auto issue = [&](int t, int buf) {
    char* base = smem + buf * kStage;
    const int k0 = klo + t * kKey;
    if (k0 + kKey <= klen) {
      const uint32_t sk = static_cast<uint32_t>(k0) * kstride, sv = static_cast<uint32_t>(k0) * vstride;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        load_lds16_buf(i < 2 ? rk : rv, goff[i], i < 2 ? sk : sv, base + (wave_s + 4 * i) * 1024);
    } else {
      // the tile that runs past the keys: its rows past klen - 1 lie outside
      // the descriptors' range and land as zeros
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int grp = wave_s + 4 * i;
        const int r = 8 * (grp & 7) + lrow;
        const uint32_t key = static_cast<uint32_t>(k0 + r);
        const uint32_t off = key * (i < 2 ? kstride : vstride) + ((cslot ^ kv_swz(r)) << 4);
        load_lds16_buf(i < 2 ? rk : rv, off, 0u, base + grp * 1024);
      }
    }
  };

  // O^T accumulators; l_i: this lane's share of the softmax denominator,
  // summed from the same bf16 weights the P.V MFMA consumes (two partial
  // sums, v_dot2 with ones); m_i: the running offset.  Each pass sets them.
  f32x16_t o[2];
  float m_i, l_i, l_j;
  const float c = PRE ? 1.f : a.scale * kLog2e;

  // LDS offsets (within a stage) of this lane's operand reads, the same for
  // every tile.  K fragments: row jb*32 + l32, dims 16*st + 8*hb + [0, 8).
  // V^T fragments through transposed reads (see lds_read_tr): lane group
  // g = lane / 16 covers dims 16 * (g % 2) + [0, 16) of a 32-dim block and
  // keys 4 * (g / 2) + [0, 4) of an 8-key half step.  The swizzle key of a
  // row, a function of (row >> 1) & 7, does not see the 32-row block jb or
  // the 16-row step u, so those enter as constants (folded into the LDS
  // instructions' offset fields): koff[st] + 4096 jb; the V reads take the
  // LDS address vaddr[db][hl] (stage 0) plus slot * kStage + 4096 jb + 2048 u.
  int koff[4];
  uint32_t vaddr[2][2];
  {
    const int tq = lane & 3, tk = (lane >> 2) & 3, tg = lane >> 4;
    const int tdim = 16 * (tg & 1) + 4 * tq;
    const int tkey = 4 * (tg >> 1) + tk;
#pragma unroll
    for (int st = 0; st < 4; ++st) koff[st] = kv_off(l32, 16 * st + 8 * hb);
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
        vaddr[db][hl] = lds_addr(smem) + kKey * 128 + kv_off(8 * hl + tkey, db * 32 + tdim);
  }

  // One 64-key tile at key offset kt from the stage at sb.  MASK 0: interior
  // tile of full attention; 1: its last tile (keys >= qhi masked); 2: a
  // sliding window (keys outside [qlo, qhi) masked).  NOMAX (PRE only): the
  // exp2 offset stays 0 and no tile max is taken (see the pass check below).
  // ST >= 0: the tile's ring slot, known to the caller (folded into the LDS
  // offsets); ST < 0: slot `slot`.
  auto tile = [&](auto mask_tag, auto nomax_tag, auto slot_tag, int slot, int kt) {
    constexpr int MASK = decltype(mask_tag)::value;
    constexpr bool NOMAX = decltype(nomax_tag)::value;
    constexpr int ST = decltype(slot_tag)::value;
    const char* sb = smem + (ST >= 0 ? ST : slot) * kStage;
    static_assert(PRE || !NOMAX, "the offset-free pass needs log2-domain logits");
    f32x16_t s[2];
    // S^T[key][query] for keys kt + [0, 32) and kt + [32, 64): every K
    // fragment of the tile is read first, then the two accumulators' MFMAs
    // go in turn (reading each fragment just before its MFMA left a wait on
    // the LDS between MFMAs; the V^T fragments stay where they are used:
    // holding them from here needs more registers than three workgroups per
    // CU leave)
    bf16x8_t kf[2][4];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int st = 0; st < 4; ++st) kf[jb][st] = *reinterpret_cast<const bf16x8_t*>(sb + jb * 4096 + koff[st]);
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int e = 0; e < 16; ++e) s[jb][e] = 0.f;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
        s[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[jb][st], qf[st], s[jb], 0, 0, 0);
    static_assert(!(NOMAX && MASK == 1), "the offset-free pass takes the last tile unmasked");
    if constexpr (MASK != 0) {
      // key of element (jb, e) is kt + 4*hb + 32*jb + 8*(e/4) + e%4
      const int lo = qlo - kt - 4 * hb, hi = qhi - kt - 4 * hb;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int k = 32 * jb + 8 * (e >> 2) + (e & 3);
          const bool out = MASK == 2 ? (k < lo || k >= hi) : k >= hi;
          s[jb][e] = out ? -INFINITY : s[jb][e];
        }
    }
    // Online softmax in the log2 domain (c = scale * log2 e).  A lane keeps
    // its running max m_i unless the tile's max exceeds it by more than
    // kLazy: p = 2^(s*c - m_i) then stays below 2^kLazy, the final 1/l
    // normalisation uses the same m_i, so the result is exact while the
    // rescale of O and l is skipped for most tiles.  PRE: the same with the
    // offset held at 0 while the logits stay near 0 (kZeroLo, kZeroHi).
    if constexpr (!NOMAX) {
      float tmax = -INFINITY;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, s[jb][e]);
      tmax = wave_max32(tmax) * c;
      const bool bump = tmax > m_i + (PRE ? kLazyPre : kLazy);
      if (__any(bump)) {
        asm volatile("" ::: "memory");  // keep this a branch (rarely taken), not a select
        const float m_tgt = PRE && tmax >= kZeroLo && tmax <= kZeroHi ? 0.f : tmax;
        const float m_new = bump ? m_tgt : m_i;
        const float alpha = m_i == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_i - m_new);
        m_i = m_new;
        l_i *= alpha;
        l_j *= alpha;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          o[0][e] *= alpha;
          o[1][e] *= alpha;
        }
      }
    }
    const float m_use = m_i == -INFINITY ? 0.f : m_i;
    if constexpr (PRE) {
      // the logits are already in the log2 domain; the offset is 0 for the
      // whole wave unless a lane's logits left [kZeroLo, kZeroHi]
      if (!NOMAX && __any(m_use != 0.f)) {
        asm volatile("" ::: "memory");  // a branch (rarely taken), not a select
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
#pragma unroll
          for (int e = 0; e < 16; ++e) s[jb][e] -= m_use;
      }
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[jb][e] = __builtin_amdgcn_exp2f(s[jb][e]);
    } else {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[jb][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[jb][e], c, -m_use));
    }
    // O^T[dim][query] += V^T[dim][key] . P^T[key][query].  The MFMA's k index
    // 8 * hb + t of a 16-key step u stands for key 16u + 4hb + t (t < 4) or
    // 16u + 8 + 4hb + (t - 4): the order in which the S^T accumulator holds
    // them, so P^T needs no data movement and V^T is read to match.  The
    // V^T reads go in groups g = 2 jb + u of four, two groups ahead of the
    // MFMAs: group g + 2 is issued after group g's MFMAs, so exactly one
    // group (four reads) is issued after each group but the last when its
    // MFMAs wait for it.
    uint32_t vb[2][2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl) vb[db][hl] = ST >= 0 ? vaddr[db][hl] : vaddr[db][hl] + slot * kStage;
    constexpr int SOFF = ST >= 0 ? ST * kStage : 0;
    s16x4_t vr[4][2][2];
    auto vread = [&](auto g_tag) {
      constexpr int g = decltype(g_tag)::value;
      constexpr int off = SOFF + (g >> 1) * 4096 + (g & 1) * 2048;
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        vr[g][db][0] = lds_read_tr<off>(vb[db][0]);
        vr[g][db][1] = lds_read_tr<off>(vb[db][1]);
      }
    };
    vread(std::integral_constant<int, 0>{});
    vread(std::integral_constant<int, 1>{});
    static_for<0, 4>([&](auto g_tag) {
      constexpr int g = decltype(g_tag)::value, jb = g >> 1, u = g & 1;
      bf16x8_t pf;
#pragma unroll
      for (int e = 0; e < 8; ++e) pf[e] = static_cast<__bf16>(s[jb][8 * u + e]);
      const bf16x2_t ones = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};
      l_i = __builtin_amdgcn_fdot2_f32_bf16((bf16x2_t){pf[0], pf[1]}, ones, l_i, false);
      l_j = __builtin_amdgcn_fdot2_f32_bf16((bf16x2_t){pf[2], pf[3]}, ones, l_j, false);
      l_i = __builtin_amdgcn_fdot2_f32_bf16((bf16x2_t){pf[4], pf[5]}, ones, l_i, false);
      l_j = __builtin_amdgcn_fdot2_f32_bf16((bf16x2_t){pf[6], pf[7]}, ones, l_j, false);
      lgkm_claim<g < 3 ? 4 : 0>(vr[g][0][0], vr[g][0][1], vr[g][1][0], vr[g][1][1]);
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const s16x4_t lo = vr[g][db][0], hi = vr[g][db][1];
        const bf16x8_t vf = __builtin_bit_cast(
            bf16x8_t, (s16x8_t){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[db], 0, 0, 0);
      }
      if constexpr (g + 2 < 4) vread(std::integral_constant<int, g + 2>{});
    });
  };

  // ST: the ring slot of tile t when the caller knows it (t % kNS), so the
  // slot's LDS offset folds into the instructions' offset fields; -1: taken
  // from t
  auto step = [&](int t, auto mask_tag, auto nomax_tag, auto slot_tag) {
    constexpr int ST = decltype(slot_tag)::value;
    const int slot = ST >= 0 ? ST : t % kNS;
    if (t + kNS - 2 < ntiles)
      wait_vmcnt<4 * (kNS - 2)>();
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (t + kNS - 1 < ntiles) issue(t + kNS - 1, ST >= 0 ? (ST + kNS - 1) % kNS : (t + kNS - 1) % kNS);
    if (wave_active) tile(mask_tag, nomax_tag, slot_tag, slot, klo + t * kKey);
  };
  // One pass over the item's key tiles.  The interior tiles of full attention
  // run in a loop of their own, then the masked ones: no branch between the
  // two tile bodies inside the hot loop (such a merge costs register copies
  // of the accumulators on every tile).
  const int n_plain = a.window > 0 ? 0 : (khi - klo) / kKey;
  auto pass = [&](auto nomax_tag) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      o[0][e] = 0.f;
      o[1][e] = 0.f;
    }
    m_i = -INFINITY, l_i = 0.f, l_j = 0.f;
#pragma unroll
    for (int st = 0; st < kNS - 1; ++st)
      if (st < ntiles) issue(st, st);
    using I0 = std::integral_constant<int, 0>;
    using Idyn = std::integral_constant<int, -1>;
    static_assert(kNS == 2, "the interior loop is unrolled by the ring depth");
    // The offset-free pass of full attention takes every tile through the
    // interior body, the last one too: its keys past klen have zero K and V
    // rows (the descriptors end at the last key), so each adds 2^0 = 1 to
    // the weight sum and nothing to O; the caller gives them back.
    constexpr bool NOMAX = decltype(nomax_tag)::value;
    const bool all_plain = NOMAX && a.window == 0;  // uniform
    const int n_int = all_plain ? ntiles : n_plain;
    int t = 0;
    for (; t + 1 < n_int; t += 2) {  // t is even: slots 0 then 1
      step(t, I0{}, nomax_tag, I0{});
      step(t + 1, I0{}, nomax_tag, std::integral_constant<int, 1>{});
    }
    for (; t < n_int; ++t) step(t, I0{}, nomax_tag, Idyn{});
    if (a.window > 0) {
      for (; t < ntiles; ++t) step(t, std::integral_constant<int, 2>{}, nomax_tag, Idyn{});
    } else {
      if constexpr (!NOMAX)
        for (; t < ntiles; ++t) step(t, std::integral_constant<int, 1>{}, nomax_tag, Idyn{});
    }
    l_i += l_j;
    return l_i + __shfl_xor(l_i, 32, 64);
  };
  float l_tot;
  if constexpr (PRE) {
    // First pass without the running max: p = 2^s straight from the MFMA.
    // It stands when every live query's weight sum lies in [2^-60, 2^64]
    // (raised below when the last tile ran past the keys):
    // then no weight, sum or O entry overflowed, and a weight that flushed
    // to zero (below 2^-126) is under 2^-53 of the largest one (>= 2^-60 /
    // 8192), so its loss is far below the bf16 rounding of the weights.
    // Otherwise (or a NaN) the workgroup runs the item again with the max
    // rule.  The decision is per workgroup: its waves share the K/V loads.
    int* redo = reinterpret_cast<int*>(smem + kNS * kStage);
    if (tid == 0) *redo = 0;  // ordered before other waves' writes by pass 1's barriers
    l_tot = pass(std::true_type{});
    float l_min = 0x1p-60f;
    if (a.window == 0 && ntiles > 0) {  // uniform
      // the keys at or past klen in the last tile (none before a half item's
      // middle), each counted once with
      // weight 1 (both wave halves' keys: kt + 8g + 4hb + [0, 4), g = 0..7;
      // with rr = klen - kt - 4hb, groups g > rr / 8 and 4 - rr % 8 of group
      // rr / 8 lie past the end)
      auto n_out = [](int rr) { return rr <= 0 ? 32 : rr >= 60 ? 0 : 4 * (7 - (rr >> 3)) + max(0, 4 - (rr & 7)); };
      const int rr = klen - (klo + (ntiles - 1) * kKey);
      const float units = static_cast<float>(n_out(rr) + n_out(rr - 4));
      l_tot -= units;
      // While those units sit in the sums, each of the last tile's adds
      // rounds by up to 2^-24 of (true sum + units): at most 2^-19 (l + units)
      // over the lane's adds, the two wave halves and the subtraction.  A
      // true sum of at least units * 2^-6 keeps that below 2^-13 of it; a
      // smaller one (every weight of the row tiny) runs again with the max
      // rule, which masks those keys instead.
      l_min = fmaxf(l_min, units * 0x1p-6f);
    }
    if (ntiles > 0) {  // uniform
      const bool bad = wave_active && qi < qlen && qhi > qlo && !(l_tot >= l_min && l_tot <= 0x1p64f);
      if (__any(bad) && lane == 0) *redo = 1;
      __syncthreads();
      if (*redo) l_tot = pass(std::false_type{});
    }
  } else {
    l_tot = pass(std::false_type{});
  }
  if (half > 0) {
    // a half item: O^T as accumulated, then per query the weight sum and the
    // softmax offset (log2 domain; 0 for the offset-free pass), rows past
    // q_len left out
    if (qi < qlen) {
      const int ql = wave * 32 + l32;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq)
          *reinterpret_cast<f32x4_t*>(part + ql * 64 + db * 32 + 8 * gq + 4 * hb) =
              (f32x4_t){o[db][4 * gq], o[db][4 * gq + 1], o[db][4 * gq + 2], o[db][4 * gq + 3]};
      if (hb == 0) {
        part[kQ * 64 + ql] = l_tot;
        part[kQ * 64 + kQ + ql] = m_i == -INFINITY ? 0.f : m_i;
      }
    }
    return;
  }
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if constexpr (WO) {
    // P[q][n] = sum_d O[q][d] Wo[n0 + n][64 h + d] by v_mfma_f32_32x32x16_bf16
    // with A = Wo rows, B = O^T: the B fragment of K step (db, sub) is the
    // accumulator o[db][8 sub + t] itself (lane (q, hb) holds dims 8 (e / 4)
    // + 4 hb + e % 4 of its 32-dim block), so its k slot 8 hb + t stands for
    // dim 16 sub + 4 hb + t (t < 4) or 16 sub + 8 + 4 hb + t - 4, and the A
    // fragments are read in that order (two 8-byte reads).  O is rounded to
    // bf16 after the 1 / l normalisation, as the O store does.
    wait_vmcnt<0>();  // the Wo chunk (all else has landed)
    __syncthreads();  // every wave's share of it
    if (!wave_active) return;
    bf16x8_t ob[2][2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int t = 0; t < 8; ++t) ob[db][sub][t] = static_cast<__bf16>(o[db][8 * sub + t] * inv);
    const char* wl = smem + kWoLds;
    float* P = a.wo_part + h * a.wo_part_stride + (row0 + min(qi, qlen - 1)) * a.wo_ld_part + n0 + 4 * hb;
#pragma unroll
    for (int nb = 0; nb < kAttnWoCols / 32; ++nb) {
      f32x16_t d;
#pragma unroll
      for (int e = 0; e < 16; ++e) d[e] = 0.f;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
          const int row = nb * 32 + l32, col = db * 32 + 16 * sub + 4 * hb;
          const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(wl + kv_off(row, col));
          const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(wl + kv_off(row, col + 8));
          const bf16x8_t af = __builtin_bit_cast(bf16x8_t, (u32x4_t){lo[0], lo[1], hi[0], hi[1]});
          d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, ob[db][sub], d, 0, 0, 0);
        }
      // lane (q, hb): columns nb * 32 + 8 g + 4 hb + [0, 4) of its query's row
      if (qi < qlen) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<f32x4_t*>(P + nb * 32 + 8 * g) = (f32x4_t){d[4 * g], d[4 * g + 1], d[4 * g + 2], d[4 * g + 3]};
      }
    }
    return;
  }
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

template <bool PRE>
__global__ __launch_bounds__(256, 3) void attn_bf16_mfma_kernel(AttnArgs a) {
  // the K/V ring, then the workgroup's redo flag
  __shared__ __attribute__((aligned(16))) char smem[kNS * kStage + 16];
  if (a.items) {  // the work list: this workgroup's slot
    const int4 m = reinterpret_cast<const int4*>(a.items)[blockIdx.x];
    if (m.y <= 0) return;  // an empty slot (uniform over the workgroup)
    const int q0 = static_cast<int>(static_cast<uint32_t>(m.w) >> 16) * kQ;
    if (m.w & 0x8000) {  // a half item of the key split: its pair's partials
      const int half = (m.w >> 14) & 1;
      const int pair = a.items[4 * a.n_slots + blockIdx.x];
      float* part = a.part + (2 * static_cast<int64_t>(pair) + half) * kAttnPartFloats;
      attn_item<PRE>(a, smem, m.x, m.y, m.z, m.w & 0x3fff, q0, 1 + half, part);
    } else {
      attn_item<PRE>(a, smem, m.x, m.y, m.z, m.w & 0x3fff, q0);
    }
    return;
  }
  // Workgroup -> (sequence, head, query block).  Hardware hands workgroup i
  // to XCD i % 8.  The (sequence, head) pairs, in seq_order's order, go to the
  // XCDs round-robin, and an XCD's workgroups take its pairs' query blocks in
  // turn, so the blocks of one pair run on one XCD close together and share
  // its L2 for the pair's K/V tiles.
  const int nblk = (a.max_q + kQ - 1) / kQ;
  const int xcd = blockIdx.x & 7, kx = blockIdx.x >> 3;
  const int pair = xcd + 8 * (kx / nblk);
  if (pair >= a.H * a.B) return;  // uniform over the workgroup
  const int zs = pair / a.H, h = pair - zs * a.H;
  int qlen, klen;
  int64_t row0;
  if (a.seq_meta) {
    const int4 m = reinterpret_cast<const int4*>(a.seq_meta)[zs];
    row0 = m.x;
    qlen = m.y;
    klen = m.z;
  } else {
    const int b = a.seq_order ? a.seq_order[zs] : zs;
    qlen = a.q_len ? a.q_len[b] : a.uniform_L;
    // keys never extend past the rows a sequence owns (a caller's k_len > L
    // in the padded layout is clamped rather than read out of bounds)
    klen = a.seq_start ? a.k_len[b] : max(0, min(a.k_len[b], a.uniform_L));
    row0 = a.seq_start ? a.seq_start[b] : static_cast<int64_t>(b) * a.uniform_L;
  }
  const int q0 = (kx % nblk) * kQ;
  if (q0 >= qlen) return;  // uniform over the workgroup
  attn_item<PRE>(a, smem, row0, qlen, klen, h, q0);
}

// The work list's items with the output projection folded in (AttnArgs::wo):
// workgroup (slot, y) runs slot's item for Wo rows y * kAttnWoCols + [0,
// kAttnWoCols).
template <bool PRE>
__global__ __launch_bounds__(256) void attn_wo_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kWoLds + kAttnWoCols * 128];
  const int4 m = reinterpret_cast<const int4*>(a.items)[blockIdx.x];
  if (m.y <= 0) return;  // an empty slot (uniform over the workgroup)
  const int q0 = static_cast<int>(static_cast<uint32_t>(m.w) >> 16) * kQ;
  attn_item<PRE, true>(a, smem, m.x, m.y, m.z, m.w & 0x3fff, q0);
}

// First rank of the key-split tail (Bb: none): the smallest rank z, at a
// change of length (rank z - 1 longer), such that the sequences from z on
// hold at most a quarter of the batch's query blocks and each at least
// kAttnSplitMinKeys keys.  Empty sequences (ranked last) are passed over.
__device__ int attn_split_rank(const int32_t* table, int Bb) {
  const int32_t* qbp = table + seq_table_qbp(Bb);
  const int32_t* meta = table + seq_table_meta(Bb);
  const int64_t qb_all = qbp[Bb];
  int rs = Bb;
  for (int z = Bb - 1; z >= 0; --z) {
    const int n = meta[4 * z + 1];
    if (n == 0) continue;
    if (4 * (qb_all - qbp[z]) > qb_all || meta[4 * z + 2] < kAttnSplitMinKeys) break;
    if (z == 0 || meta[4 * (z - 1) + 1] != n) rs = z;
  }
  return rs;
}

// Item i (< H * qbp[Bb]) of the batch's order: sequence z (rank), head h and
// query block qb, z by bisection of the table's query-block prefix.
__device__ void attn_item_of(const int32_t* qbp, int Bb, int H, int64_t i, int& z, int& h, int& qb) {
  int lo = 0, hi = Bb;  // H * qbp[lo] <= i < H * qbp[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(H) * qbp[mid] <= i)
      lo = mid;
    else
      hi = mid;
  }
  const int nb = qbp[lo + 1] - qbp[lo];  // >= 1: item i lies in sequence lo's range
  const int r = static_cast<int>(i - static_cast<int64_t>(H) * qbp[lo]);
  z = lo;
  h = r / nb;
  qb = r - h * nb;
}

// Work list (launch_attn_items): one thread per slot.  Slot (workgroup) s
// runs on XCD s % 8 and is place pos = s / 8 of that XCD's list, which holds
// the items of runs x, x + 8, x + 16, ... (runs of kAttnRun items of the
// batch's item order).  With split, the items of the tail ranks follow the
// others as half items, both halves of an item side by side.
__global__ __launch_bounds__(256) void attn_items_kernel(const int32_t* table, int Bb, int H, int n_slots,
                                                         int split, int32_t* items) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s >= n_slots) return;
  const int32_t* qbp = table + seq_table_qbp(Bb);
  const int32_t* meta = table + seq_table_meta(Bb);
  const int pos = s >> 3;
  const int64_t i = (static_cast<int64_t>(pos / kAttnRun) * 8 + (s & 7)) * kAttnRun + pos % kAttnRun;
  const int rs = split ? attn_split_rank(table, Bb) : Bb;
  const int64_t n_whole = static_cast<int64_t>(H) * qbp[rs];
  const int64_t n_half = 2 * static_cast<int64_t>(H) * (qbp[Bb] - qbp[rs]);
  int4 out = {0, 0, 0, 0};
  int pair = 0;
  if (i < n_whole + n_half) {
    const bool halves = i >= n_whole;
    int z, h, qb;
    attn_item_of(qbp, Bb, H, halves ? n_whole + ((i - n_whole) >> 1) : i, z, h, qb);
    int w = h | (qb << 16);
    if (halves) {
      w |= 0x8000 | (static_cast<int>((i - n_whole) & 1) << 14);
      pair = static_cast<int>((i - n_whole) >> 1);
    }
    out = (int4){meta[4 * z], meta[4 * z + 1], meta[4 * z + 2], w};
  }
  reinterpret_cast<int4*>(items)[s] = out;
  if (split) items[4 * static_cast<int64_t>(n_slots) + s] = pair;
}

// Merge of the split items (launch_attn_merge): workgroup p = pair p; thread
// t takes dims 4 (t % 16) + [0, 4) of queries t / 16 + 16 r, r < 8 (a row's
// 16 threads read and write it contiguously).
__global__ __launch_bounds__(256) void attn_merge_kernel(const int32_t* table, int Bb, int H, const float* part,
                                                         bf16_t* o, int64_t ld_o) {
  const int32_t* qbp = table + seq_table_qbp(Bb);
  const int32_t* meta = table + seq_table_meta(Bb);
  const int rs = attn_split_rank(table, Bb);
  const int64_t n_whole = static_cast<int64_t>(H) * qbp[rs];
  const int64_t p = blockIdx.x;
  if (n_whole + p >= static_cast<int64_t>(H) * qbp[Bb]) return;  // uniform
  int z, h, qb;
  attn_item_of(qbp, Bb, H, n_whole + p, z, h, qb);
  const int64_t row0 = meta[4 * z];
  const int qlen = meta[4 * z + 1];
  const float* p1 = part + 2 * p * kAttnPartFloats;
  const float* p2 = p1 + kAttnPartFloats;
  const int c = threadIdx.x & 15;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int q = (threadIdx.x >> 4) + 16 * r;
    const int qi = qb * kQ + q;
    if (qi >= qlen) break;
    const float m1 = p1[kQ * 64 + kQ + q], m2 = p2[kQ * 64 + kQ + q];
    const float mx = fmaxf(m1, m2);
    const float w1 = __builtin_amdgcn_exp2f(m1 - mx), w2 = __builtin_amdgcn_exp2f(m2 - mx);
    const float l = p1[kQ * 64 + q] * w1 + p2[kQ * 64 + q] * w2;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const float s1 = w1 * inv, s2 = w2 * inv;
    const f32x4_t x1 = *reinterpret_cast<const f32x4_t*>(p1 + q * 64 + 4 * c);
    const f32x4_t x2 = *reinterpret_cast<const f32x4_t*>(p2 + q * 64 + 4 * c);
    u32x2_t w;
    w[0] = pack_bf16x2(x1[0] * s1 + x2[0] * s2, x1[1] * s1 + x2[1] * s2);
    w[1] = pack_bf16x2(x1[2] * s1 + x2[2] * s2, x1[3] * s1 + x2[3] * s2);
    *reinterpret_cast<u32x2_t*>(o + (row0 + qi) * ld_o + h * 64 + 4 * c) = w;
  }
}

// ------------------------------------------------------------------ generic
constexpr int gQ = 128;   // queries per workgroup (one per thread)
constexpr int gKey = 32;  // keys per LDS tile

template <typename T, int DH>
__global__ __launch_bounds__(gQ) void attn_generic_kernel(AttnArgs a) {
  const int b = a.seq_order ? a.seq_order[blockIdx.z] : static_cast<int>(blockIdx.z);
  const int h = blockIdx.y;
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
  require(!a.part || (a.items && a.window == 0 && (reinterpret_cast<uintptr_t>(a.part) & 15u) == 0),
          "attention: split items need the work list, full attention and 16-byte aligned partials");
  require(!a.seq_meta || (a.seq_start && a.q_len && (reinterpret_cast<uintptr_t>(a.seq_meta) & 15u) == 0),
          "attention: seq_meta needs the varlen layout and 16-byte alignment");
  const bool mfma = a.dtype == DT_BF16 && a.Dh == 64 && a.ld_q % 8 == 0 && a.ld_k % 8 == 0 &&
                    a.ld_v % 8 == 0 && a.ld_o % 4 == 0 && aligned16(a.q) && aligned16(a.k) &&
                    aligned16(a.v) && (reinterpret_cast<uintptr_t>(a.o) & 7u) == 0;
  if (mfma) {
    // one workgroup per (sequence, head, query block), the pairs padded to a
    // multiple of the 8 XCDs (see the kernel's mapping), or per slot of the
    // work list
    int64_t nwg;
    if (a.items) {
      require(a.n_slots > 0 && (reinterpret_cast<uintptr_t>(a.items) & 15u) == 0,
              "attention: the work list needs slots and 16-byte alignment");
      nwg = a.n_slots;
    } else {
      const int64_t pairs8 = (static_cast<int64_t>(a.H) * a.B + 7) / 8 * 8;
      nwg = pairs8 * ((a.max_q + kQ - 1) / kQ);
    }
    require(nwg < (int64_t{1} << 31), "attention: too many workgroups");
    if (a.wo) {
      require(a.items && !a.part && a.wo_n > 0 && a.wo_n % kAttnWoCols == 0 && a.ld_wo >= 64 * int64_t{a.H} &&
                  a.ld_wo % 8 == 0 && aligned16(a.wo) && a.wo_part && aligned16(a.wo_part) &&
                  a.wo_ld_part >= a.wo_n && a.wo_ld_part % 4 == 0 && a.wo_part_stride % 4 == 0,
              "attention: the folded output projection needs the work list without split items, bf16 Wo rows "
              "of at least 64 H values, a multiple of 128 rows and 16-byte aligned partials");
      const dim3 grid(static_cast<unsigned>(nwg), static_cast<unsigned>(a.wo_n / kAttnWoCols));
      if (a.q_log2_scaled)
        attn_wo_kernel<true><<<grid, dim3(256), 0, st>>>(a);
      else
        attn_wo_kernel<false><<<grid, dim3(256), 0, st>>>(a);
      check_launch("attn_wo");
      return;
    }
    if (a.q_log2_scaled)
      attn_bf16_mfma_kernel<true><<<dim3(static_cast<unsigned>(nwg)), dim3(256), 0, st>>>(a);
    else
      attn_bf16_mfma_kernel<false><<<dim3(static_cast<unsigned>(nwg)), dim3(256), 0, st>>>(a);
    check_launch("attn_bf16_mfma");
    return;
  }
  require(!a.q_log2_scaled, "attention: pre-scaled queries need the bf16 head_dim-64 kernel");
  if (a.dtype == DT_BF16)
    launch_generic<bf16_t>(a, st);
  else
    launch_generic<float>(a, st);
  check_launch("attn_generic");
}

namespace {
// query blocks of any batch of at most Tb rows in at most Bb sequences:
// sum over sequences of ceil(n / kAttnQ) <= (T + (kAttnQ - 1) B) / kAttnQ
int64_t max_query_blocks(int Tb, int Bb) {
  require(Tb >= 0 && Bb >= 0, "attention items: bad shape");
  return (static_cast<int64_t>(Tb) + (kAttnQ - 1) * int64_t{Bb} + kAttnQ - 1) / kAttnQ;
}
}  // namespace

int attn_split_pairs(int Tb, int Bb, int H) {
  require(H > 0, "attention items: bad shape");
  // the tail holds at most a quarter of the query blocks
  const int64_t pairs = static_cast<int64_t>(H) * (max_query_blocks(Tb, Bb) / 4);
  require(pairs < (int64_t{1} << 28), "attention items: too many");
  return static_cast<int>(pairs);
}

int attn_item_slots(int Tb, int Bb, int H, bool split) {
  require(H > 0, "attention items: bad shape");
  int64_t items = static_cast<int64_t>(H) * max_query_blocks(Tb, Bb);
  if (split) items += attn_split_pairs(Tb, Bb, H);  // a split item takes two slots
  const int64_t slots = 8 * ((items + 8 * kAttnRun - 1) / (8 * kAttnRun)) * kAttnRun;
  require(slots < (int64_t{1} << 30), "attention items: too many");
  return static_cast<int>(slots);
}

void launch_attn_items(const int32_t* table, int Bb, int H, int n_slots, bool split, int32_t* items,
                       hipStream_t st) {
  if (n_slots <= 0) return;
  require(table && items && (reinterpret_cast<uintptr_t>(items) & 15u) == 0 && Bb >= 1 && H >= 1 &&
              H < 16384 && n_slots % 8 == 0,
          "attention items: bad arguments");
  // (the caller keeps every sequence below 65536 query blocks: the item
  // holds the block index in 16 bits, the head in 14)
  attn_items_kernel<<<(n_slots + 255) / 256, 256, 0, st>>>(table, Bb, H, n_slots, split ? 1 : 0, items);
  check_launch("attn_items");
}

void launch_attn_merge(const int32_t* table, int Bb, int H, int max_pairs, const float* part, void* o,
                       int64_t ld_o, hipStream_t st) {
  if (max_pairs <= 0) return;
  require(table && part && o && Bb >= 1 && H >= 1 && ld_o >= 64 * int64_t{H} && ld_o % 4 == 0 &&
              (reinterpret_cast<uintptr_t>(part) & 15u) == 0 && (reinterpret_cast<uintptr_t>(o) & 7u) == 0,
          "attention merge: bad arguments");
  attn_merge_kernel<<<max_pairs, 256, 0, st>>>(table, Bb, H, part, static_cast<bf16_t*>(o), ld_o);
  check_launch("attn_merge");
}

}  // namespace sjh

// sjh_kernels.hpp -- host-side launch interface of the gfx950 kernels.
//
// Every launcher validates the shapes its kernel assumes and throws
// std::runtime_error naming the violated condition before anything reaches the
// GPU, so a bad call never becomes an out-of-bounds access.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sjh {

enum DType : int { DT_F32 = 0, DT_BF16 = 1, DT_FP8 = 2 };  // DT_FP8: OCP e4m3fn, GEMM weights only

// GEMM epilogues, applied to an fp32 tile staged in LDS.
enum Epi : int {
  EPI_STORE = 0,  // out = act(acc + bias)                (bias optional)
  EPI_RESID = 1,  // X (fp32) += acc + bias                (bias optional)
  EPI_ROPE = 2,   // packed (q|k|v) output, rotate-half RoPE on q and k
  EPI_GEGLU = 3,  // out[:, j] = gelu(acc_in[:, j]) * acc_gate[:, j]
};

// out[M, N] = epi(A[M, K] . W[N_w, K]^T).  For EPI_GEGLU, N = F and W is the
// reference's [2F, K] Wi (rows [0, F) input half, [F, 2F) gate half).
struct GemmArgs {
  const void* A = nullptr;
  int64_t lda = 0;
  const void* W = nullptr;
  int64_t ldw = 0;
  // M sizes the launch (grid, tile choice, split-K strides).  With M_dev set,
  // the kernels read the real row count (<= M) from device memory at start
  // and touch rows [0, *M_dev) only: one launch, or one captured graph,
  // then serves every row count up to M.
  int M = 0, N = 0, K = 0;
  const int* M_dev = nullptr;
  int in_dtype = DT_BF16;  // A (and W unless w_dtype says otherwise)
  // DT_FP8: W holds e4m3 codes and row n of W stands for code * w_scale[n]
  // (A stays bf16); the scale multiplies the fp32 accumulator.
  int w_dtype = DT_BF16;
  const float* w_scale = nullptr;
  int epi = EPI_STORE;
  void* out = nullptr;  // STORE / ROPE / GEGLU
  int64_t ldo = 0;
  int out_dtype = DT_BF16;
  const float* bias = nullptr;  // [N]
  int act = 0;                  // 0 none, 1 erf-GELU, 2 ReLU (STORE)
  float* X = nullptr;           // RESID
  int64_t ldx = 0;
  const int* pos = nullptr;  // ROPE: position of each row
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;  // [rope_rows, head_dim/2]
  int rope_rows = 0;                // positions are clamped to [0, rope_rows)
  int rope_dim = 0;                 // D: columns [0, 2D) are q and k
  int head_dim = 0;
  // ROPE: the rotated q columns [0, rope_dim) are multiplied by q_scale
  // before the output rounding (attention's scale * log2 e, folded in)
  float q_scale = 1.f;
  // Optional split-K workspace for short batches (M <= 256): partial sums of
  // K slices go to partial[split][M][N_w] (fp32) and a second kernel adds them
  // in split order and applies the epilogue.  Unused when null or too small.
  float* partial = nullptr;
  int64_t partial_cap = 0;  // floats
  // set by the launcher for split-K launches
  int k_chunk = 0;  // K steps (of the MFMA K depth) per split
  int n_w = 0;      // rows of W (= N, or 2F for GEGLU)
  int part_rows = 0;  // the launch's M: split s of row m sits at partial[(s * part_rows + m) * n_w]
  // A LayerNorm folded across a residual GEMM and the GEMM that reads its
  // rows next (persistent bf16-activation path only; the launcher rejects
  // anything else).  Rows are cut into blocks of kLnBlock columns.
  //  Producer (EPI_RESID with ln_y, N % kLnBlock == 0): besides X += acc
  //    (+ bias) it writes ln_y[m][c] = bf16((x[m][c] - mu_b) * ln_w[c]) (row
  //    stride ldx), mu_b the mean of row m over its block b = c / kLnBlock,
  //    and ln_stats_out[(m * N / kLnBlock + b) * 2 + {0, 1}] = {mu_b, M2_b},
  //    M2_b the block's sum of squared deviations from mu_b.
  //  Consumer (ln_stats_in, K % kLnBlock == 0, K <= kLnMaxBlocks * kLnBlock,
  //    a bf16 RoPE or GEGLU product; ln_stats_in holds the moments of at
  //    least round_up(M, 256) + 256 rows, read in whole 256-row tiles): A holds such rows.  The
  //    epilogue first takes acc to r_m * (acc + sum_b d_mb * c1[n][b]) + c2[n]
  //    with d_mb = mu_b - mu_m and r_m = 1 / sqrt(var_m + eps) from the row's
  //    combined moments (src/tensor.cpp:54-79), c1[n][b] = sum over block b of
  //    ln_w[k] W[n][k] and c2 = W . ln_b: that is LN(x) . W^T, with x rounded
  //    to bf16 after centring on its block's mean.
  void* ln_y = nullptr;                 // bf16
  const float* ln_w = nullptr;          // [N]
  float* ln_stats_out = nullptr;
  const float* ln_stats_in = nullptr;
  const uint16_t* ln_c1 = nullptr;      // bf16 [n_w][8], blocks past K / kLnBlock zero
  const float* ln_c2 = nullptr;         // [n_w] or null (an unbiased norm)
  float ln_eps = 1e-5f;
  // The LayerNorm that reads the residual stream next, finished by the
  // residual epilogue itself (EPI_RESID with rln_y; gemm_takes_rln): besides
  // X += acc (+ bias) it writes rln_y[m][c] = bf16(LN(x)[c]) (row stride
  // rln_ldy) with weights rln_w, optional bias rln_b and rln_eps, as
  // launch_ln does, bit for bit (sjh_common.hpp's LayerNorm statistics).
  // The N / 256 tiles of a 256-row panel exchange their rows' 256-column
  // block moments through rln_mom (M x N/256 x 4 floats) and count
  // themselves in through rln_sync (8 ints per panel, zero before the launch,
  // zero again after it); a tile waits at most rln_spin polls for the others.
  void* rln_y = nullptr;
  int64_t rln_ldy = 0;
  const float* rln_w = nullptr;
  const float* rln_b = nullptr;
  float rln_eps = 1e-5f;
  float* rln_mom = nullptr;
  int* rln_sync = nullptr;
  int rln_spin = 0;
};
// Sync ints per 256-row panel of GemmArgs::rln_sync.
constexpr int kRlnSyncInts = 8;
constexpr int kLnBlock = 256;
// The engine does not take the folded path (see Engine::stage_weights).
constexpr bool kLnFoldEnabled = false;
constexpr int kLnMaxBlocks = 4;  // D <= 1024 (c1 rows hold 8 bf16, blocks past 4 zero)
void launch_gemm(const GemmArgs& g, hipStream_t st);
// Whether a GEMM of these arguments takes the persistent kernel, the only
// one that can produce or consume a folded LayerNorm.
bool gemm_takes_ln_fold(const GemmArgs& g);
// The consumer constants of a folded LayerNorm for weights W [n_w, K] (bf16,
// or fp8 codes with per-row scales w_scale: the effective rows code * scale):
// c1[n][b] = sum over block b of ln_w[k] W[n][k] (bf16, [n_w][8]) and, with
// ln_b, c2[n] = sum_k ln_b[k] W[n][k] (fp32), both summed in double.
void launch_ln_fold_consts(const void* W, int w_dtype, const float* w_scale, int n_w, int K,
                           const float* ln_w, const float* ln_b, uint16_t* c1, float* c2,
                           hipStream_t st);
// Whether the residual epilogue can finish the next LayerNorm for these
// arguments (GemmArgs::rln_y): the persistent bf16 kernel, N a multiple of 256
// up to 1024, and at most one tile per workgroup, so that all of a panel's
// tiles run at once.
bool gemm_takes_rln(const GemmArgs& g);
// Short batches (M <= 256) of a residual GEMM (EPI_RESID, bf16 MFMA path):
// launches only the split-K product into g.partial and returns the number of
// splits S >= 2; the caller then adds the splits with the layer norm that
// reads X next (LnArgs::parts), which must then satisfy ln_takes_parts.
// Returns 0, having launched nothing, when the split-K path does not apply.
int launch_gemm_resid_partials(const GemmArgs& g, hipStream_t st);

// Row LayerNorm over [M, D] rows (src/tensor.cpp:54-79 semantics).
//   input row r = in[(ids ? ids[r] : r) * ld_in]
//   if resid: x = in_row + resid_row, written back to xio (fp32)
//   if n_parts: x = in_row + (sum of the n_parts split-K partial rows, in
//     split order, + part_bias), written back to xio (fp32): the residual
//     epilogue of a split-K GEMM, bit for bit
//   y = normalize ? LN(x) * w (+ b) : x
//   x_out (fp32, optional) and y_out (y_dtype, optional) receive y.
struct LnArgs {
  const void* in = nullptr;
  int in_dtype = DT_F32;
  int64_t ld_in = 0;
  const int* ids = nullptr;
  const void* resid = nullptr;  // optional residual added first (resid_dtype)
  int resid_dtype = DT_BF16;
  float* xio = nullptr;  // where x = in + resid is written back (fp32 rows, ld_in)
  const float* parts = nullptr;  // split-K partials: parts[s * part_stride + r * ld_part + c]
  int n_parts = 0;
  int64_t part_stride = 0, ld_part = 0;
  const float* part_bias = nullptr;
  bool normalize = true;
  const float* w = nullptr;
  const float* b = nullptr;
  float eps = 1e-5f;
  float* x_out = nullptr;
  int64_t ld_x = 0;
  void* y_out = nullptr;
  int y_dtype = DT_BF16;
  int64_t ld_y = 0;
  int M = 0, D = 0;
  const int* M_dev = nullptr;  // as GemmArgs::M_dev: rows [0, *M_dev) of the M launched
  // optional second input row added to the first, before the residual:
  // x = in_row + add[add_ids[r] clamped to [0, add_rows)] (fp32 rows, ld_add),
  // the learned position embedding of a BERT-style encoder
  const float* add = nullptr;
  const int* add_ids = nullptr;
  int add_rows = 0;
  int64_t ld_add = 0;
};
void launch_ln(const LnArgs& a, hipStream_t st);
// Whether launch_ln accepts a.n_parts > 0 (split-K partials folded into the
// residual) for rows of this shape: the vector kernel's D % 4 == 0 and
// D <= 1024 with 16-byte aligned fp32 rows.
bool ln_takes_parts(const LnArgs& a);

// Non-causal attention over a varlen batch.  Sequence b owns rows
// [seq_start[b], seq_start[b] + max(q_len[b], k_len[b])); its queries are the
// first q_len[b] rows and its keys/values the first k_len[b] rows.  Head h of
// row t sits at q + t*ld_q + h*Dh (same for k, v, o).  window > 0 restricts
// query i to keys |i - j| <= window (src/tensor.cpp:186-192).  A null
// seq_start means seq_start[b] = b * uniform_L; a null q_len means
// q_len[b] = uniform_L (the reference's padded [B, L] layout).
struct AttnArgs {
  const void* q = nullptr;
  const void* k = nullptr;
  const void* v = nullptr;
  int64_t ld_q = 0, ld_k = 0, ld_v = 0;
  void* o = nullptr;
  int64_t ld_o = 0;
  int dtype = DT_BF16;
  const int* seq_start = nullptr;
  const int* q_len = nullptr;
  const int* k_len = nullptr;
  const int* seq_order = nullptr;  // optional: workgroup z handles sequence seq_order[z]
  // optional, 16-byte aligned: seq_meta[4z .. 4z+3] = {seq_start, q_len,
  // k_len, 0} of the sequence seq_order[z] (one load instead of a chain)
  const int* seq_meta = nullptr;
  int B = 0, H = 0, Dh = 0;
  int max_q = 0;  // upper bound of q_len over the batch (grid size)
  int uniform_L = 0;
  int window = 0;
  float scale = 0.f;  // 1/sqrt(Dh)
  // q already holds q * scale * log2(e) (GemmArgs::q_scale of the QKV
  // projection): the logits come out of the QK^T product in the log2 domain.
  // bf16 with head_dim 64 only.
  bool q_log2_scaled = false;
  // Optional work list of the bf16 head_dim-64 kernel (launch_attn_items),
  // 16-byte aligned: n_slots entries of {first row, q_len, k_len, head |
  // query block << 16}, q_len 0 for an empty slot; workgroup w runs slot w.
  // The grid is then n_slots workgroups whatever B and max_q say.
  const int* items = nullptr;
  int n_slots = 0;
  // Partials of the work list's key-split items (launch_attn_items with
  // split): kAttnPartFloats floats per half item, merged by launch_attn_merge.
  float* part = nullptr;
  // Optional output projection folded in (bf16 head_dim-64 kernel with the
  // work list, no split items): instead of o, item (head h, query block)
  // writes its queries' O_h . Wo[:, 64h : 64h + 64]^T, fp32, to
  // wo_part[h * wo_part_stride + row * wo_ld_part + n] for n < wo_n, so the
  // H slices summed in head order (a LayerNorm with LnArgs::parts) give
  // O . Wo^T.  Wo is bf16 [wo_n][ld_wo], wo_n a multiple of kAttnWoCols (the
  // columns of one workgroup; grid y = wo_n / kAttnWoCols).
  const void* wo = nullptr;
  int64_t ld_wo = 0;
  int wo_n = 0;
  float* wo_part = nullptr;
  int64_t wo_part_stride = 0, wo_ld_part = 0;
};
constexpr int kAttnWoCols = 128;
void launch_attn(const AttnArgs& a, hipStream_t st);

// Attention work list of a batch (AttnArgs::items): the (sequence, head,
// query block of kAttnQ rows) items of the sequences in table order (longest
// first), each sequence's heads in turn and each head's blocks in turn, are
// cut into runs of kAttnRun consecutive items dealt to the 8 XCDs
// round-robin; the workgroups of an XCD take its runs' items in order.
// Items beyond the batch's leave their slots empty.  Only real items reach
// the dispatcher (the padded grid of the (pair, block) mapping hands it an
// empty workgroup for every block a shorter sequence lacks).
constexpr int kAttnQ = 128;
constexpr int kAttnRun = 4;
//
// Key split of the tail (full attention only): the shortest sequences, from
// the first rank z whose length differs from rank z - 1's on, whose query
// blocks are at most a quarter of the batch's and which each hold at least
// kAttnSplitMinKeys keys, run every item as two half items over keys
// [0, mid) and [mid, k_len), mid = k_len / 2 rounded up to 64 keys.  They
// are the list's last items, the two halves of one item side by side; each
// half leaves its unnormalised O^T, weight sums and softmax offsets in
// AttnArgs::part (kAttnPartFloats floats at (2 pair + half) * kAttnPartFloats)
// and launch_attn_merge writes the item's output rows.  The split depends
// only on the batch's multiset of lengths (never on its order).
constexpr int kAttnSplitMinKeys = 2048;
constexpr int kAttnPartFloats = kAttnQ * 64 + 2 * kAttnQ;
// Slots for any batch of at most Tb rows in at most Bb sequences (a multiple
// of 8 * kAttnRun), with room for the split's half items when split.
int attn_item_slots(int Tb, int Bb, int H, bool split = false);
// Item pairs a split can make for such a batch (the merge's grid).
int attn_split_pairs(int Tb, int Bb, int H);
// Ints of the list: n_slots int4 items, then (split) one pair index per slot.
inline size_t attn_items_ints(int n_slots) { return 5u * static_cast<size_t>(n_slots); }
// Fills items[0, n_slots) (and the pair indices when split) from the sequence
// table (its query-block prefix).
void launch_attn_items(const int32_t* table, int Bb, int H, int n_slots, bool split, int32_t* items,
                       hipStream_t st);
// Output rows of the split items: O = (2^(m1-M) O1 + 2^(m2-M) O2) /
// (2^(m1-M) l1 + 2^(m2-M) l2), M = max(m1, m2), bf16 into o (row stride ld_o,
// head h at column 64 h).  Workgroups past the batch's pairs return.
void launch_attn_merge(const int32_t* table, int Bb, int H, int max_pairs, const float* part, void* o,
                       int64_t ld_o, hipStream_t st);

// Standalone RoPE on packed (q|k|v)(head)(dim) rows, position = pos[r]
// (or r % L when pos is null), as src/tensor.cpp:257-279.
void launch_rope(void* qkv, int dtype, int64_t M, int64_t ld, const int* pos, int L, int H,
                 int Dh, const float* cos_t, const float* sin_t, hipStream_t st);

// Fill tok_pos[t] (position inside its sequence) and tok_seq[t] for the rows
// [seq_start[b], seq_start[b] + rows[b]) of every sequence.
void launch_token_index(const int* seq_start, const int* rows, int B, int* tok_pos,
                        int* tok_seq, hipStream_t st);

// X[t, :] += table[sel[tok_seq[t]], :] for t < T (type embedding of a row's
// qtype); with T_dev, for t < *T_dev (<= T).
void launch_add_row_embedding(float* X, int64_t ldx, const float* table, const int* sel,
                              const int* tok_seq, int T, const int* T_dev, int D, hipStream_t st);

// Checkpoint staging conversions (convert.hip), element types of the source:
enum SrcType : int { SRC_F32 = 0, SRC_F16 = 1, SRC_BF16 = 2, SRC_F8 = 3 };
// dst[i] = exact fp32 value of src[i] (bf16 or f16)
void launch_widen_f32(const void* src, int src_dtype, float* dst, int64_t n, hipStream_t st);
// dst[i] = bf16 nearest to src[i] (f32 or f16), ties to even
void launch_narrow_bf16(const void* src, int src_dtype, uint16_t* dst, int64_t n, hipStream_t st);
// Per-row e4m3 codes and scales of a [rows, cols] fp32 matrix, identical to
// the host quantizer (sjh_quantize_fp8)
void launch_quantize_fp8_rows(const float* w, int64_t rows, int64_t cols, uint8_t* q,
                              float* scale, hipStream_t st);

// Per-batch sequence table (device int32), for Bb >= B table entries:
//   [0] total tokens T = sum of lens, [1] B, [2..3] 0,
//   seq_start[Bb] at 4, q_len[Bb], k_len[Bb], qtype[Bb], order[Bb], then,
//   16-byte aligned at seq_table_meta(Bb), meta[4 * Bb] = {seq_start, q_len,
//   k_len, 0} of order[z] for z < Bb, then at seq_table_qbp(Bb) the query
//   block prefix qbp[Bb + 1]: qbp[z] = sum over z' < z of
//   ceil(q_len / kAttnQ) of order[z'].
// Entries b >= B are empty sequences (start T, length 0) that every kernel
// skips; order lists the real sequences longest first (stable), then the
// empty ones.
constexpr int kSeqHdr = 4;
__host__ __device__ inline size_t seq_table_meta(int Bb) { return (static_cast<size_t>(kSeqHdr) + 5u * Bb + 3) / 4 * 4; }
__host__ __device__ inline size_t seq_table_qbp(int Bb) { return seq_table_meta(Bb) + 4u * Bb; }
__host__ __device__ inline size_t seq_table_ints(int Bb) { return (seq_table_qbp(Bb) + Bb + 1 + 3) / 4 * 4; }
// Builds that table on the device from lengths passed by value in the kernel
// arguments (no host staging buffer): q_len = k_len = lens[b], qtype 0.
constexpr int kSeqTableMaxB = 256;
void launch_seq_table(const int32_t* h_lens, int B, int Bb, int32_t* table, hipStream_t st);

// dst[i, :] = idx[i] >= 0 ? src[idx[i], :] : 0   (fp32 rows)
void launch_gather_rows(const float* src, int64_t ld_src, const int* idx, int n, int D,
                        float* dst, int64_t ld_dst, hipStream_t st);

// Decision-head tail on the device (src/model.cpp:484-534): per row b of B,
// logits[b, k] = mmask[b, k] ? s2[b, k] : -1e4 and the act-head input
// ain[b, :] = [cls[b, :D], top1, top1 - top2, entropy, kf / 255]
void launch_act_features(const float* s2, const int* mmask, int B, int K, const float* cls,
                         int64_t ld_cls, int D, float* logits, float* ain, int64_t ld_ain,
                         hipStream_t st);
// act[b, :] = softmax(a[b, :n]) with the reference's float exp / double sums
void launch_act_softmax(const float* a, int B, int n, float* act, hipStream_t st);
// SjModel's act head (src/sj_model.cpp:336-367): masked logits as in
// launch_act_features, then act[b, :] = {top1, 1 - top1} of their softmax
void launch_act_top1(const float* s2, const int* mmask, int B, int K, float* logits, float* act,
                     hipStream_t st);

}  // namespace sjh

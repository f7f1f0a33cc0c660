/*
 * snapjudge_hip.h -- C ABI of the MI355X (gfx950) encoder forward.
 *
 * Drop-in boundary for the reference's GPU fast-path hook.  Two layers:
 *
 *  1. Model level (replaces FastSnapjudge, include/snapjudge/fast.hpp:15-31 of
 *     the reference): stage a DecisionModel's weights on the GPU once, then run
 *     DecisionModel::forward (src/model.cpp:309-536) or ::encode
 *     (src/model.cpp:222-307) on host-side [B][L] batches with exactly the
 *     reference's argument meaning.
 *
 *  2. Kernel level (replaces the extern "C" launchers of cuda/kernels.cu,
 *     bound by cuda/fast.cpp:23-34): GEMM with epilogues, GEGLU, residual +
 *     LayerNorm, RoPE, attention, taking device pointers and a hipStream_t.
 *
 * Conventions (mirroring the reference engine ABI, include/snapjudge/capi.h):
 * every entry point returns 0 on success or a negative SJH_E_* code; the
 * message of the last failure on the calling thread is sjh_last_error().
 * bf16 tensors are passed as raw 16-bit storage (uint16_t / void*).  Nothing
 * here falls back to the CPU: without a usable gfx950 device, calls fail.
 */
#ifndef SNAPJUDGE_HIP_H
#define SNAPJUDGE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* sjh_stream_t; /* == hipStream_t */

enum {
  SJH_OK = 0,
  SJH_E_INVALID = -1, /* bad argument or shape */
  SJH_E_DEVICE = -2,  /* HIP runtime error or no gfx950 device */
  SJH_E_OOM = -3      /* device allocation failed */
};

enum { SJH_F32 = 0, SJH_BF16 = 1 }; /* element types */

/* Numerics mode of a model.
 *  SJH_PREC_FP32: fp32 weights and activations, fp32 accumulation
 *                 (parity mode: hidden states within 1e-4 of the reference).
 *  SJH_PREC_BF16: bf16 weights and activations, fp32 accumulation, fp32
 *                 residual stream and LayerNorm statistics (within 2e-2).
 *  SJH_PREC_FP8W: as SJH_PREC_BF16, but the four encoder projections of every
 *                 layer (Wqkv, Wo, Wi, Wo2) are stored as OCP fp8 e4m3 with
 *                 one fp32 scale per output row (sjh_quantize_fp8); the
 *                 forward equals the reference forward on the dequantized
 *                 weights within the bf16 tolerance.  No counterpart in the
 *                 reference, whose loader rejects fp8 (src/safetensors.cpp:132). */
enum { SJH_PREC_FP32 = 0, SJH_PREC_BF16 = 1, SJH_PREC_FP8W = 2 };

/* One encoder layer: the reference's LayerWeights (include/snapjudge/model.hpp:37-44),
 * fp32 host arrays, row-major, PyTorch Linear layout [out, in]. */
typedef struct sjh_layer_desc {
  const float* attn_norm; /* [D] or NULL (layer 0 has none, src/model.cpp:112-117) */
  const float* wqkv;      /* [3D, D] */
  const float* wo;        /* [D, D] */
  const float* mlp_norm;  /* [D] */
  const float* wi;        /* [2F, D]: rows [0,F) input half, [F,2F) gate half */
  const float* wo2;       /* [D, F] */
  int32_t window;         /* 0 = full attention, else local_attention/2 */
  int32_t sliding;        /* 1 = use the sliding-attention RoPE tables */
} sjh_layer_desc;

/* One decision-head layer (src/model.cpp:107-111). */
typedef struct sjh_head_desc {
  const float *n1w, *n1b, *n2w, *n2b; /* [D] */
  const float *in_w, *in_b;           /* [3D, D], [3D] */
  const float *out_w, *out_b;         /* [D, D], [D] */
  const float *l1w, *l1b;             /* [4D, D], [4D] */
  const float *l2w, *l2b;             /* [D, 4D], [D] */
} sjh_head_desc;

/* Everything DecisionModel::forward reads (src/model.cpp:89-126). */
typedef struct sjh_model_desc {
  int32_t hidden_size, num_heads, intermediate_size, vocab_size, num_layers;
  int32_t max_position; /* rows of the RoPE tables */
  int32_t n_act, head_layers, lora_r;
  float norm_eps;
  double rope_theta_full, rope_theta_sliding; /* used when the tables below are NULL */
  const float* emb_w;      /* [V, D] */
  const float* emb_norm;   /* [D] */
  const float* final_norm; /* [D] */
  const float *rope_cos_full, *rope_sin_full;   /* [max_position, Dh/2] or NULL */
  const float *rope_cos_slide, *rope_sin_slide; /* [max_position, Dh/2] or NULL */
  const sjh_layer_desc* layers;                 /* [num_layers] */
  const float* lora_a;   /* [r, D] or NULL */
  const float* lora_b;   /* [D, r] or NULL */
  const float* type_emb; /* [3, D] */
  const sjh_head_desc* head; /* [head_layers] */
  const float *sc_ln_w, *sc_ln_b; /* [D], [D] or NULL */
  const float *sc_w1, *sc_b1;     /* [D, D], [D] or NULL */
  const float *sc_w2, *sc_b2;     /* [1, D], [1] or NULL */
  const float *act_w1, *act_b1;   /* [256, D+4], [256] */
  const float *act_w2, *act_b2;   /* [n_act, 256], [n_act] */
} sjh_model_desc;

typedef struct sjh_options {
  int32_t precision;  /* SJH_PREC_* */
  int32_t max_len;    /* longest row accepted (the reference's max_len) */
  int32_t use_graphs; /* replay the device work of a repeated batch shape as a hipGraph */
  int32_t pad_rows;   /* 1: also compute padded query rows, as the reference does, so
                         encode() returns its values at padded positions too; 0: work
                         only on valid tokens (padded positions of encode() are 0) */
  int32_t device;     /* HIP device ordinal */
  int32_t fuse_ln;    /* 1 (default): where a residual GEMM's tiles all run at once (bf16,
                         hidden size a multiple of 256 up to 1024, one round of tiles), its
                         epilogue also writes the LayerNorm that reads the residual stream
                         next; 0: that LayerNorm runs as a launch of its own; 2: as 1, but a
                         tile waits for its panel's other tiles for one poll only, so that
                         most tiles take the path of a tile that gave up waiting (the
                         results are the same bits as with 1; for tests) */
  int32_t fuse_attn_wo; /* 1 (default): on short batches (at most 256 tokens, bf16, head_dim
                         64) attention also multiplies each head's output by its slice of
                         Wo, and the LayerNorm that reads the residual stream next adds the
                         heads' partial products (no separate Wo launch); 0: Wo is a GEMM
                         launch of its own */
} sjh_options;

typedef struct sjh_model sjh_model;

const char* sjh_last_error(void);
int sjh_version(void);
void sjh_default_options(sjh_options* opt);

/* FastSnapjudge::FastSnapjudge (cuda/fast.cpp:272-352): copies the weights to
 * the device in the numerics mode's storage type.  The descriptor's arrays may
 * be released after the call. */
int sjh_model_create(const sjh_model_desc* desc, const sjh_options* opt, sjh_model** out);
void sjh_model_destroy(sjh_model* m);

/* Loads a checkpoint directory straight into device memory, with no fp32
 * host copy of the model (the reference materialises one:
 * src/safetensors.cpp:109-135, src/model.cpp:96-171).  model.safetensors is
 * memory-mapped; each tensor is copied to the device in its stored type and
 * converted there (bf16 weights of a bf16 model are copied as they are).
 *   DecisionModel (DecisionModel::load, src/model.cpp:35-205):
 *     rl_agent_config.json, encoder/config.json, model.safetensors.
 *     The four encoder projections may also be stored as "F8_E4M3" codes
 *     with an F32 "<name>_scale" of one scale per output row (the
 *     SJH_PREC_FP8W format, see sjh_quantize_fp8); such a checkpoint needs
 *     SJH_PREC_FP8W.  F32/F16/BF16 projections loaded with SJH_PREC_FP8W are
 *     quantized on the device, bit-identical to sjh_quantize_fp8.
 *   SjModel (SjModel::load, src/sj_model.cpp:87-204): sj_config.json and
 *     model.safetensors with the sj.* tensors.  Its act head is
 *     {top1, 1 - top1} (n_act 2) and positions past max_positions use the
 *     last row of the position table, as the reference does.
 * Same configuration keys, defaults, strict shapes and error cases as the
 * reference loaders (SJH_E_INVALID with the message). */
int sjh_model_load(const char* dir, const sjh_options* opt, sjh_model** out);

/* DecisionModel::encode (src/model.cpp:222-307).  ids, mask: [B, L] int64,
 * right-padded, mask 0/1.  hidden: [B, L, D] fp32, caller-allocated. */
int sjh_model_encode(sjh_model* m, const int64_t* ids, const int64_t* mask, int32_t B, int32_t L,
                     float* hidden);

/* DecisionModel::forward (src/model.cpp:309-536) / FastSnapjudge::forward
 * (cuda/fast.cpp:357-569).  marker_pos [B, K] int64, marker_mask [B, K] uint8,
 * qtype [B] int64 in {0,1,2}.  logits [B, K] (masked = -1e4), act [B, n_act]. */
int sjh_model_forward(sjh_model* m, const int64_t* ids, const int64_t* mask,
                      const int64_t* marker_pos, const uint8_t* marker_mask, const int64_t* qtype,
                      int32_t B, int32_t L, int32_t K, float* logits, float* act);

/* DecisionModel::forward (src/model.cpp:309-536) on B rows that share U
 * token sequences: row b reads sequence row_seq[b] of ids/mask [U, L], with
 * its own marker_pos [B, K], marker_mask [B, K] and qtype [B].  The results
 * are those of sjh_model_forward on the B-row batch ids[row_seq[b]] (the
 * encoder depends on the tokens only, src/model.cpp:332-407).  Each sequence
 * is encoded once; the head layers, whose input is the sequence plus the type
 * embedding of the row's qtype (src/model.cpp:409-459), run once per distinct
 * (sequence, qtype) pair, and the scorer and act head once per row.  The
 * shape of 32 sequences x 8 typed questions: no counterpart in the
 * reference, which runs the 256 rows through DecisionModel::forward. */
int sjh_model_forward_shared(sjh_model* m, const int64_t* ids, const int64_t* mask, int32_t U,
                             int32_t L, const int32_t* row_seq, const int64_t* marker_pos,
                             const uint8_t* marker_mask, const int64_t* qtype, int32_t B,
                             int32_t K, float* logits, float* act);

/* Encoder on a batch already resident in device memory: d_ids [T] int32 holds
 * the B sequences back to back, h_lens [B] (host) their lengths, T = sum.
 * Writes the final hidden states [T, D] fp32 to d_hidden.  Work is enqueued on
 * `stream` (NULL: the model's own stream); the call does not synchronize. */
int sjh_model_encode_device(sjh_model* m, const int32_t* d_ids, const int32_t* h_lens, int32_t B,
                            float* d_hidden, sjh_stream_t stream);

/* sjh_model_encode_device without any device allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, same results bit for bit (the same kernels on the same launch
 * sizes); the work runs launch by launch (no graph) and every intermediate
 * buffer lives in one fixed array of SJH_NOALLOC_SCRATCH_BYTES per device,
 * shared by all models on that device and held until the process ends.
 * Limits: at most 256 sequences, and the batch must fit the array (about
 * 3000 tokens of a 768-wide bf16 model); larger batches fail with
 * SJH_E_INVALID and a message naming the bytes needed.  Calls that overlap on
 * one device (any model, any stream) race on the array: the caller
 * serializes them.  The call waits for earlier calls of the same model on
 * any stream and does not synchronize. */
#define SJH_NOALLOC_SCRATCH_BYTES (32u << 20)
int sjh_model_encode_device_noalloc(sjh_model* m, const int32_t* d_ids, const int32_t* h_lens,
                                    int32_t B, float* d_hidden, sjh_stream_t stream);

/* Hidden size, heads, n_act and the precision a model was built with. */
int sjh_model_info(const sjh_model* m, int32_t* D, int32_t* H, int32_t* n_act,
                   int32_t* precision);

/* Graph cache of a model (use_graphs): graphs held now, captures and replays
 * so far.  A batch is replayed from the graph of its shape bucket (batch size
 * rounded up to a power of two, token count and longest row rounded up), so a
 * serving loop captures once per bucket.  No counterpart in the reference,
 * whose graph map is private (cuda/fast.cpp:376-393). */
int sjh_model_graph_stats(const sjh_model* m, int32_t* cached, int64_t* captures,
                          int64_t* replays);

/* Enable/disable per-kernel timing with hipEvents on the model's launches and
 * read the totals: names[i] (static strings), total_ms[i], launches[i]. */
int sjh_model_profile(sjh_model* m, int32_t enable);
int sjh_model_profile_read(sjh_model* m, int32_t max_entries, const char** names,
                           double* total_ms, int64_t* launches, int32_t* n_entries);

/* ------------------------------------------------------------------------
 * Kernel level.  All pointers are device pointers.
 * ------------------------------------------------------------------------ */

/* sj_gemm (cuda/kernels.cu:88-108): C[M,N] = act(A[M,K] . W[N,K]^T (+ bias)).
 * act 0 none, 1 erf-GELU, 2 ReLU.  dtype applies to A, W and C; bias fp32 or NULL. */
int sjh_gemm(const void* A, const void* W, const float* bias, void* C, int32_t M, int32_t N,
             int32_t K, int32_t act, int32_t dtype, sjh_stream_t stream);

/* Host-side quantizer of SJH_PREC_FP8W (no GPU needed): for each row r of the
 * row-major [rows, cols] fp32 matrix w, scale[r] = max|w[r,:]| / 448 (1 for an
 * all-zero row) and q[r,c] = e4m3(w[r,c] / scale[r]), OCP e4m3fn rounded to
 * nearest even, saturating at 448.  Row r stands for e4m3_decode(q[r,:]) *
 * scale[r].  No counterpart in the reference (fp8 is not loadable there). */
int sjh_quantize_fp8(const float* w, int64_t rows, int64_t cols, uint8_t* q, float* scale);

/* sj_gemm with fp8 weights: C[M,N] (bf16) = act(A[M,K] (bf16) . Wdq[N,K]^T (+ bias))
 * where Wdq[n,:] = e4m3_decode(Wq[n,:]) * w_scale[n].  K % 64 == 0, N % 4 == 0,
 * 16-byte aligned rows.  The GEMM of SJH_PREC_FP8W models; no counterpart in
 * the reference. */
int sjh_gemm_fp8w(const void* A, const uint8_t* Wq, const float* w_scale, const float* bias,
                  void* C, int32_t M, int32_t N, int32_t K, int32_t act, sjh_stream_t stream);

/* sj_gemm_geglu (cuda/kernels.cu:168-174): C[M,F] = gelu(A.Wi[:F]^T) * (A.Wi[F:]^T),
 * Wi [2F, K]. */
int sjh_gemm_geglu(const void* A, const void* Wi, void* C, int32_t M, int32_t F, int32_t K,
                   int32_t dtype, sjh_stream_t stream);

/* X[M,D] (fp32) += C[M,N=D] where C = A[M,K] . W[D,K]^T: the residual-add
 * epilogue that the reference runs as gemm + add_ (src/model.cpp:389-391). */
int sjh_gemm_residual(const void* A, const void* W, float* X, int32_t M, int32_t D, int32_t K,
                      int32_t dtype, sjh_stream_t stream);

/* sj_gemm followed by sj_rope (cuda/fast.cpp:183-190 runs them back to back;
 * src/model.cpp:355-365 on the CPU): qkv[M, 3*H*Dh] = A[M,K] . Wqkv[3*H*Dh, K]^T
 * with rotate-half RoPE applied to the q and k heads of each row, row m at
 * position pos[m] (device int32 [M], clamped to [0, max_pos)); cos/sin fp32
 * [max_pos, Dh/2]. */
int sjh_gemm_qkv_rope(const void* A, const void* Wqkv, void* qkv, const int32_t* pos,
                      const float* cos_t, const float* sin_t, int32_t max_pos, int32_t M,
                      int32_t H, int32_t Dh, int32_t K, int32_t dtype, sjh_stream_t stream);

/* sj_add_ln (cuda/kernels.cu:243-254): if residual, X += R (R of dtype);
 * Y = LN(X) * W (+ B if bias), Y of dtype.  X fp32 [M, D]. */
int sjh_add_ln(float* X, const void* R, const float* W, const float* B, void* Y, int32_t M,
               int32_t D, float eps, int32_t residual, int32_t bias, int32_t dtype,
               sjh_stream_t stream);

/* sj_rope (cuda/kernels.cu:282-288): in-place rotate-half on packed qkv
 * [M, 3*H*Dh], row r at position r % L; cos/sin fp32 [L_max, Dh/2]. */
int sjh_rope(void* qkv, const float* cos_t, const float* sin_t, int64_t M, int32_t L, int32_t H,
             int32_t Dh, int32_t dtype, sjh_stream_t stream);

/* sj_attn (cuda/kernels.cu:351-357): qkv [B, L, 3, H, Dh], lens [B] int32 ->
 * O [B, L, H*Dh]; every query row of each sequence attends to its first
 * lens[b] keys (window > 0: |i-j| <= window).  dtype applies to qkv and O. */
int sjh_attn(const void* qkv, const int32_t* lens, void* O, int32_t B, int32_t L, int32_t H,
             int32_t Dh, int32_t window, int32_t dtype, sjh_stream_t stream);

/* sjh_attn on queries that already hold q * (1/sqrt(64)) * log2(e), bf16 with
 * head_dim 64: the layout the encoder's QKV projection writes (the scale is
 * folded into the projection's epilogue, so the QK^T product yields log2-
 * domain logits).  Same masking and output as sjh_attn.  No counterpart in the
 * reference, which scales the scores (src/tensor.cpp:186-200). */
int sjh_attn_log2(const void* qkv, const int32_t* lens, void* O, int32_t B, int32_t L, int32_t H,
                  int32_t window, sjh_stream_t stream);

/* Embedding gather + LayerNorm (src/model.cpp:332-340): X[r] = LN(table[ids[r]]) * w.
 * table [V, D] of dtype, ids int32 [M], X fp32 [M, D]. */
int sjh_embed_ln(const void* table, const int32_t* ids, const float* w, float* X, int32_t M,
                 int32_t D, float eps, int32_t dtype, sjh_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* SNAPJUDGE_HIP_H */

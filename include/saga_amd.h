/*
 * saga_amd.h -- C ABI of the MI355X (gfx950) SAGA + Atop-N decode-attention
 * library (libsaga_amd.so).
 *
 * The reference (noamelata/SAGA) is Python: its decode path is the module
 * attention/attention.py (torch ops) plus the Triton kernel in
 * attention/triton_atopn.py.  Each entry point below replaces one function of
 * that module; the comment above it names the function and file:line.  A
 * Python caller binds them with ctypes (saga_amd/_lib.py); the same
 * signatures are what a cffi/ctypes stub in the reference would bind.
 *
 * Conventions
 *   - All tensor data live in device memory (HBM) and are owned by the
 *     caller.  No entry point allocates, frees or synchronises; every one
 *     enqueues work on `stream` and returns.  Calls are capturable into a
 *     HIP graph.
 *   - Strides are in elements.  The innermost (head_dim / position) stride
 *     must be 1.  16-bit tensors need 16-byte aligned rows for the vector
 *     loads (head_dim * 2 bytes, i.e. any d in {64, 128} with aligned base).
 *   - query [b, q_h, 1, d]; key [b, k_h, L, d]; value [b, v_h, L, d];
 *     q_h % k_h == 0 and q_h % v_h == 0; query head h reads key head
 *     h / (q_h / k_h) and value head h / (q_h / v_h)
 *     (attention/attention.py:70, 81, 119, 163).
 *   - mask (optional) is an additive mask [b or 1, 1 or q_h, 1, L' >= L];
 *     only its first L columns are used (attention/attention.py:125).  A
 *     SAGA_DTYPE_BOOL mask adds 1.0 where true and 0.0 where false, which is
 *     what `logits + bool_mask` does in torch.
 *   - kv_len (optional, device int32 [b]) truncates batch row i to its first
 *     kv_len[i] positions: results equal the reference applied to
 *     key[i, :, :kv_len[i]] and value[i, :, :kv_len[i]].  No counterpart in
 *     the reference; it lets a static KV cache skip its unfilled slots.
 *   - Return value: SAGA_OK or a negative SAGA_ERR_* code; the message of
 *     the last error on the calling thread is in saga_last_error().  Nothing
 *     aborts and no C++ exception crosses this boundary.
 *   - Workspaces are caller-allocated device buffers of the size the
 *     matching *_workspace_bytes() returns; no initial contents are needed.
 *     Calls that share a workspace must be ordered (same stream): calls on
 *     different streams need workspaces of their own.
 */
#ifndef SAGA_AMD_H
#define SAGA_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SAGA_DTYPE_F32 0
#define SAGA_DTYPE_BF16 1
#define SAGA_DTYPE_F16 2
#define SAGA_DTYPE_BOOL 3 /* one byte, 0 or 1; masks only */
#define SAGA_DTYPE_I32 4
#define SAGA_DTYPE_I64 5

#define SAGA_OK 0
#define SAGA_ERR_INVALID (-1)     /* null pointer, bad shape/stride/dtype */
#define SAGA_ERR_UNSUPPORTED (-2) /* valid but not built (head_dim, group size) */
#define SAGA_ERR_WORKSPACE (-3)   /* workspace missing or too small */
#define SAGA_ERR_HIP (-4)         /* a HIP runtime call failed */

typedef struct saga_tensor {
  void* data;
  int32_t dtype;
  int32_t ndim; /* 1..4 */
  int64_t shape[4];
  int64_t stride[4]; /* elements */
} saga_tensor;

/* hipStream_t; NULL selects the null stream. */
typedef void* saga_stream_t;

/* Byte offsets of the fused decode workspace (for tests and inspection). */
typedef struct saga_atopn_layout {
  int64_t scores;    /* f32 [b*q_h, scores_ld] */
  int64_t scores_ld; /* elements */
  int64_t part_max;  /* f32 [b*q_h, nparts] */
  int64_t part_sum;  /* f32 [b*q_h, nparts] */
  int64_t part_tail; /* f32 [b*q_h, nparts] max over the last min(256, kv_len) positions */
  int64_t nparts;    /* saga_qk_nparts(b, k_h, L) */
  int64_t thresh;    /* f32 [b*q_h] logit threshold (fast step) */
  int64_t sel_idx;   /* i32 [b*q_h, buf_k] ascending positions (calibration; the fast step
                        keeps its list in the slice lists, concatenated and cut at buf_k) */
  int64_t sel_val;   /* f32 [b*q_h, buf_k] their logits */
  int64_t sel_cnt;   /* i32 [b*q_h] kept (<= buf_k) */
  int64_t sel_total; /* i32 [b*q_h] passing before the cap */
  /* fast step: each row's passing positions in nslice ordered lists
     ("slices"), one per 1024 positions, capacity slice_cap = min(1024, buf_k) */
  int64_t nslice;
  int64_t slice_cap;
  int64_t slice_idx; /* i32 [b*q_h, nslice, slice_cap] passing positions per slice */
  int64_t slice_val; /* f32 [b*q_h, nslice, slice_cap] their logits */
  int64_t slice_cnt; /* i32 [b*q_h, nslice] passing per slice */
  int64_t slice_pre; /* i32 [b*q_h, 2, nslice + 1] slice ranks (rows of > 2048 slices) */
  int64_t slice_o;   /* f32 [b*q_h, nslice, d] partial sum_e exp(x_e - m) V[e] of short slices */
  int64_t slice_ml;  /* f32 [b*q_h, nslice, 2] partial (m, sum_e exp(x_e - m)) of short slices */
  int64_t row_part;  /* f32 [b*q_h, 4, d + 4] partials (m, l, -, -, o) of a row's gather split over blocks */
  int64_t row_cnt;   /* i32 [b*q_h] blocks of a split row done (zeroed by the slice kernel) */
  int64_t total_bytes;
} saga_atopn_layout;

/* Library version (major*10000 + minor*100 + patch). */
int saga_version(void);

/* Message of the last error returned on this thread ("" if none). */
const char* saga_last_error(void);

/* Scaled, masked QK logits of one decode step.
 * Replaces _compute_attn_weights, attention/attention.py:113-128
 * (bmm of the grouped queries with K^T, * scaling, + mask).
 * scores: f32 [b, q_h, 1, >=L] (last stride 1), written for positions < L
 * (positions >= kv_len[i] are -inf).  part_max/part_sum (optional, f32
 * [b*q_h, saga_qk_nparts(b, k_h, L)]): max and sum of exp(x - max) of each
 * part of the row (contiguous ranges of positions; a part wholly past kv_len
 * holds (-inf, 0)).  Their log-sum-exp merge is the row's softmax
 * normaliser, so the logit threshold needs no second pass over the scores. */
int64_t saga_qk_nparts(int64_t b, int64_t k_h, int64_t L);
int saga_qk_scores(const saga_tensor* query, const saga_tensor* key, const saga_tensor* mask,
                   const int32_t* kv_len, float scale, saga_tensor* scores, float* part_max,
                   float* part_sum, saga_stream_t stream);

/* Softmax-space -> logit-space threshold per row.
 * Replaces _transform_softmax_threshold, attention/attention.py:136-149:
 * t = m + log(max(p*, 1e-30) * sum_j exp(x_j - m)), m = max of the last
 * min(256, L) logits.  scores f32 [b, q_h, 1, L]; softmax_threshold f32
 * [b*q_h]; logit_threshold f32 [b*q_h] (output). */
int saga_logit_threshold(const saga_tensor* scores, const int32_t* kv_len,
                         const float* softmax_threshold, float* logit_threshold,
                         saga_stream_t stream);

/* Threshold stream compaction.
 * Replaces threshold_topk_fast + threshold_select_fast_kernel,
 * attention/triton_atopn.py:59-113 and :6-53.  x [..., D] (f32/bf16/f16,
 * rows contiguous in D); threshold f32 with threshold_numel == rows (per
 * row), 1 (broadcast) or any other count (repeated, row r uses
 * threshold[r % threshold_numel], :87-96).  Selects x > t (strict, fp32
 * compare), at most k per row, in ascending index order (the reference's
 * order is atomic-race order; on overflow it keeps a race-dependent subset,
 * this keeps the first k).  out_values [..., k] (x's dtype) and out_indices
 * int64 [..., k] are fully written, unfilled slots as (-inf, 0).
 * out_counts (optional, int32 [rows]): passing elements before the cap. */
int saga_threshold_select(const saga_tensor* x, const float* threshold, int64_t threshold_numel,
                          int64_t k, saga_tensor* out_values, int64_t* out_indices,
                          int32_t* out_counts, saga_stream_t stream);

/* Softmax (or renormalisation) over K selected entries per row, then . V.
 * Replaces _atopn_gather_and_output, attention/attention.py:152-170.
 * weights [b, q_h, 1, K] (f32/bf16/f16; logits if input_is_logits, else
 * probabilities), indices int64 or int32 [b, q_h, 1, K], value
 * [b, v_h, L, d], out [b, q_h, 1, d] (f32/bf16/f16).  An all -inf logit row
 * gives NaN, as torch's softmax does; an index outside [0, L) makes its row
 * NaN (the reference's gather raises). */
int saga_sparse_softmax_pv(const saga_tensor* weights, const saga_tensor* indices,
                           const saga_tensor* value, int32_t input_is_logits, saga_tensor* out,
                           saga_stream_t stream);

/* Workspace of the fused decode entry points; buf_k = min(2*top_n, L) for
 * saga_atopn_decode, min(top_n, L) for saga_atopn_calibrate. */
size_t saga_atopn_workspace_bytes(int64_t b, int64_t q_h, int64_t k_h, int64_t L, int64_t d, int64_t buf_k);
int saga_atopn_workspace_layout(int64_t b, int64_t q_h, int64_t k_h, int64_t L, int64_t d, int64_t buf_k,
                                saga_atopn_layout* layout);

/* Atop-N fast decode step: scores, logit threshold from the stored
 * softmax-space thresholds, ordered compaction capped at
 * buf_k = min(2*top_n, L), sparse softmax . V.
 * Replaces approx_top_n_attention_amortized, attention/attention.py:192-209.
 * softmax_threshold: f32 [b*q_h] (the reference reads
 * AMORTIZED_THRESHOLD_TENSOR[layer_idx, :b*q_h], :200-201).
 * out [b, q_h, 1, d] (f32/bf16/f16). */
int saga_atopn_decode(const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
                      const saga_tensor* mask, const int32_t* kv_len, float scale, int64_t top_n,
                      const float* softmax_threshold, saga_tensor* out, void* workspace,
                      size_t workspace_bytes, saga_stream_t stream);

/* saga_atopn_decode with the kernels of its selection and softmax . V chosen
 * per call (no counterpart in the reference; every variant selects the same
 * lists, counts and thresholds and its outputs agree to fp32 rounding -- the
 * sums are grouped by other block shapes -- so this only serves A/B
 * measurement and tests):
 *   SAGA_K2_AUTO       by shape, as saga_atopn_decode;
 *   SAGA_K2_ROW_BLOCK  one block per (batch, head) row: its waves run the
 *                      row's 1024-position slices, the row's list is kept in
 *                      LDS (or, for rows of more than 64 slices or
 *                      buf_k > 2048, written to the workspace and merged
 *                      after a block barrier); the choice of SAGA_K2_AUTO for
 *                      rows of at most 12 slices with buf_k <= 2048;
 *   SAGA_K2_SLICE_ROW  a slice kernel over every (row, slice), then a row
 *                      kernel.
 * Another value returns SAGA_ERR_INVALID. */
#define SAGA_K2_AUTO 0
#define SAGA_K2_ROW_BLOCK 1
#define SAGA_K2_SLICE_ROW 2
int saga_atopn_decode_ex(const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
                         const saga_tensor* mask, const int32_t* kv_len, float scale, int64_t top_n,
                         const float* softmax_threshold, saga_tensor* out, int32_t k2_variant,
                         void* workspace, size_t workspace_bytes, saga_stream_t stream);

/* saga_atopn_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace is a static device array of SAGA_NOALLOC_SCRATCH_BYTES (64 MiB)
 * inside the library's code object, one copy per GPU, held until the
 * process ends; its address is looked up once per device (the stream must
 * be on the current device).  Nothing is allocated or freed.  Shapes whose
 * saga_atopn_workspace_bytes(b, q_h, k_h, L, d, min(2*top_n, L)) exceed the
 * scratch return SAGA_ERR_WORKSPACE (the 12/1/2-head d128 decode at batch 8
 * and 33024 cached positions needs about 41 MB).  Every call on a GPU uses
 * that GPU's one scratch: calls that may overlap on one GPU (other streams,
 * other threads) race and give wrong results; order them on one stream.
 * Results equal saga_atopn_decode's. */
#define SAGA_NOALLOC_SCRATCH_BYTES (64ull << 20)
int saga_atopn_decode_noalloc(const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
                              const saga_tensor* mask, const int32_t* kv_len, float scale, int64_t top_n,
                              const float* softmax_threshold, saga_tensor* out, saga_stream_t stream);

/* Atop-N calibration step: full softmax statistics, exact top-k
 * (k = min(top_n, L), found among the positions of its distance bin below
 * the row max, or by a radix select; equal values: lower index first),
 * stores the k-th largest probability per row into softmax_threshold_out
 * f32 [b*q_h], output = renormalised top-k . V.
 * Replaces approx_top_n_attention_amortized_cal, attention/attention.py:173-189. */
int saga_atopn_calibrate(const saga_tensor* query, const saga_tensor* key,
                         const saga_tensor* value, const saga_tensor* mask, const int32_t* kv_len,
                         float scale, int64_t top_n, float* softmax_threshold_out,
                         saga_tensor* out, void* workspace, size_t workspace_bytes,
                         saga_stream_t stream);

/* saga_atopn_calibrate with its kernels chosen per call (no counterpart in
 * the reference; every variant keeps the same list and p* and its outputs
 * agree to fp32 rounding, so this only serves A/B measurement and tests):
 *   SAGA_K2_AUTO       by shape, as saga_atopn_calibrate;
 *   SAGA_K2_ROW_BLOCK  one block per (batch, head) row;
 *   SAGA_K2_SLICE_ROW  a chunk kernel over every (row, chunk of 4096-32768
 *                      positions) that keeps each chunk's top-k, then a row
 *                      kernel that selects the row's top-k among those
 *                      lists, its V gathers split over up to 4 blocks per
 *                      row; built for top_n <= 2048, L of at least two
 *                      chunks and at most 32768 chunk-list entries per row
 *                      (elsewhere one block per row); the choice of
 *                      SAGA_K2_AUTO for rows of more than 36864 positions,
 *                      and of 16384 or more when b * q_h <= 24 or > 256.
 * Another value returns SAGA_ERR_INVALID. */
int saga_atopn_calibrate_ex(const saga_tensor* query, const saga_tensor* key,
                            const saga_tensor* value, const saga_tensor* mask, const int32_t* kv_len,
                            float scale, int64_t top_n, float* softmax_threshold_out,
                            saga_tensor* out, int32_t k2_variant, void* workspace,
                            size_t workspace_bytes, saga_stream_t stream);

/* Dense decode attention (split-L, one pass over K and V).
 * Replaces full_einsum_forward, attention/attention.py:64-85, for l_q == 1. */
size_t saga_dense_workspace_bytes(int64_t b, int64_t q_h, int64_t L, int64_t d);
int saga_dense_decode(const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
                      const saga_tensor* mask, const int32_t* kv_len, float scale,
                      saga_tensor* out, void* workspace, size_t workspace_bytes,
                      saga_stream_t stream);

/* ---- decode-step kernels around the attention path ---- */

/* RoPE + KV-cache append for N new tokens.
 * Replaces apply_rotary_pos_emb + the cache update of the reference's model
 * (transformers models/qwen2/modeling_qwen2.py:211-214, cache_utils.py:455-487)
 * with the separate key / value caches of speedup.py:119-139.
 * qkv [N, >= (n_q + n_k + n_v) * d]: the fused projection output (bias
 * included), heads in the order q, k, v.  Rotation (rotate-half form, fp32):
 * angle_i = pos * theta^(-2i/d).  q_out [N, n_q, d] receives the rotated
 * queries; k_cache [B, n_k, Lmax, d] / v_cache [B, n_v, Lmax, d] receive the
 * rotated key and the value at [batch[n], :, pos[n]] (batch == NULL: token n
 * is batch row n).  A pos or batch index out of range writes no cache row and
 * NaN queries. */
int saga_rope_kv_append(const saga_tensor* qkv, int64_t n_q, int64_t n_k, int64_t n_v, float theta,
                        const int32_t* pos, const int32_t* batch, saga_tensor* q_out,
                        saga_tensor* k_cache, saga_tensor* v_cache, saga_stream_t stream);

/* y = weight * x / sqrt(mean(x^2) + eps) per row, x and y [N, H] (Qwen2RMSNorm). */
int saga_rmsnorm(const saga_tensor* x, const saga_tensor* weight, float eps, saga_tensor* y,
                 saga_stream_t stream);

/* y[n, i] = silu(x[n, i]) * x[n, H + i]; x [N, 2H] = [gate | up], y [N, H]. */
int saga_silu_mul(const saga_tensor* gate_up, saga_tensor* y, saga_stream_t stream);

/* Skinny GEMM for decode projections (M <= 32 token rows, bf16):
 *   y[m, n] (op)= s[m] * sum_k x[m, k] * w[n, k]  (+ bias[n])
 * s[m] = 1 / sqrt(mean_k x[m, k]^2 + eps) when rms_eps >= 0 (RMSNorm of x
 * fused; its weight is expected folded into w), else 1.  epilogue:
 *   SAGA_GEMV_STORE       y = result
 *   SAGA_GEMV_ADD         y += result (residual stream, in place)
 *   SAGA_GEMV_SILU_PAIRS  w rows are interleaved (gate_i, up_i); y[m, i] =
 *                         silu(gate_i) * up_i, y is [M, N / 2]
 * Replaces the hipBLASLt calls of the decode step (no reference counterpart:
 * the reference's projections are torch nn.Linear).  N % 16 == 0, K % 32 == 0.
 * w is [N, K] (unit column stride), or packed: a contiguous 16-byte aligned
 * 4-D [N/16, K/32, 16, 32] with packed[t][j][r][c] = w[16t + r][32j + c],
 * each MFMA fragment 1 KB contiguous (measured faster: one DRAM region per
 * load instruction); results are bit-identical.  Or, for at most 8 rows of
 * x, packed in 8-row tiles: a contiguous 16-byte aligned 3-D [N/8, K/64, 512]
 * with packed[t][j][32r + c] = w[8t + r % 8][64j + 32 (r / 8) + c] (K % 64 ==
 * 0): one fragment holds 8 rows over 64 columns, so weights of few 16-row
 * tiles are read by twice the workgroups (equal to rounding: the sums run
 * in another order); never split over K.
 * workspace (optional, 256-byte aligned, saga_gemv_workspace_bytes(M, N, K)
 * bytes, no initial contents needed): with it, weights with few 16-row
 * tiles and long rows (the MLP down projection) are read by workgroups over
 * (tile, K range) whose fp32 partial sums a second kernel adds up in a fixed
 * order (results do not depend on scheduling).  Without it, or when the size
 * function returns 0, one workgroup per tile. */
#define SAGA_GEMV_STORE 0
#define SAGA_GEMV_ADD 1
#define SAGA_GEMV_SILU_PAIRS 2
size_t saga_gemv_workspace_bytes(int64_t M, int64_t N, int64_t K);
int saga_gemv(const saga_tensor* x, const saga_tensor* w, const saga_tensor* bias, float rms_eps,
              int32_t epilogue, saga_tensor* y, void* workspace, size_t workspace_bytes,
              saga_stream_t stream);

/* saga_gemv (STORE, bias, fused RMSNorm) of the fused q/k/v projection with
 * saga_rope_kv_append applied in its epilogue: one launch per layer for
 * projection + RoPE + cache append.  x [M, K] (M <= 32 new tokens), w bf16
 * [(n_q + n_k + n_v) * d, K] and bias [(n_q + n_k + n_v) * d] hold the q, k
 * and v heads in that order, with the rows of every q and k head permuted to
 * rotary-pair order [0, d/2, 1, d/2 + 1, ..., d/2 - 1, d - 1] (v heads
 * unpermuted).  The projection output is rounded to bf16 before the rotation,
 * so results equal saga_gemv into an unpermuted qkv followed by
 * saga_rope_kv_append.  Replaces q/k/v_proj + apply_rotary_pos_emb + the
 * cache update (transformers models/qwen2/modeling_qwen2.py:205-214,
 * cache_utils.py:455-487).  d % 16 == 0.  rope_table: NULL (the rotations
 * are computed in the epilogue), or the token rows' rotations from
 * saga_rope_table for the same pos, d and theta (16-byte aligned): a decode
 * step computes them once for all its layers, with identical results. */
int saga_gemv_rope_kv(const saga_tensor* x, const saga_tensor* w, const saga_tensor* bias, float rms_eps,
                      int64_t n_q, int64_t n_k, int64_t n_v, float theta, const int32_t* pos,
                      const int32_t* batch, saga_tensor* q_out, saga_tensor* k_cache,
                      saga_tensor* v_cache, const float* rope_table, saga_stream_t stream);

/* Rotations of N token rows: table [N][d/2][2] fp32 (16-byte aligned) with
 * table[n][i] = (cos, sin)(pos[n] * theta^(-2i/d)), the angles of
 * saga_rope_kv_append.  The cos / sin tables of transformers'
 * Qwen2RotaryEmbedding (models/qwen2/modeling_qwen2.py:51-104), kept in fp32,
 * for saga_gemv_rope_kv's rope_table. */
int saga_rope_table(const int32_t* pos, int64_t N, int64_t d, float theta, float* table,
                    saga_stream_t stream);

/* The opening of a decode step in one launch: x[b, :] = embed[tokens[b], :]
 * for the B = x.shape[0] token rows (embed [V, H], x [B, H], one float
 * dtype; a token id outside [0, V) writes a NaN row), and, when rope_table
 * is given, the rows' rotations for positions pos as saga_rope_table
 * writes them (d even).  Replaces Qwen2Model.forward's embed_tokens and
 * rotary_emb calls (transformers models/qwen2/modeling_qwen2.py:356, 385). */
int saga_embed_rope(const int64_t* tokens, const saga_tensor* embed, saga_tensor* x, const int32_t* pos,
                    int64_t d, float theta, float* rope_table, saga_stream_t stream);

/* The close of a decode step: pos[i] += 1 and kv_len[i] += 1 for i < n
 * (either may be NULL): the one-token growth of the cache that the
 * reference's decode loop gets from past_key_values (speedup.py:164-169;
 * transformers models/qwen2/modeling_qwen2.py:361-364 derives the next
 * position from the cache length). */
int saga_advance_positions(int32_t* pos, int32_t* kv_len, int64_t n, saga_stream_t stream);

/* out[r] = first index of the maximum of row r of x [rows, N] (bf16); the
 * greedy next token of speedup.py:169/193 (logits.argmax(dim=-1)).  NaN is
 * never the maximum.  workspace (optional, 256-byte aligned,
 * saga_argmax_workspace_bytes(rows, N) bytes, no initial contents): with it,
 * long rows are reduced in two passes over many workgroups per row; without
 * it, or when the size is 0, one workgroup per row. */
size_t saga_argmax_workspace_bytes(int64_t rows, int64_t N);
int saga_argmax(const saga_tensor* x, int64_t* out, void* workspace, size_t workspace_bytes,
                saga_stream_t stream);

/* ---- prefill ---- */

/* Prefill attention with separate key and value head counts; replaces the
 * reference's sdpa_attention_forward (attention/attention.py:13-53: torch SDPA
 * over repeat_kv-expanded keys and values) without expanding the caches.
 *   out[b, i, h, :] = sum_j softmax_j(scale * q[b, h, i] . k[b, h / (q_h/k_h), j]
 *                                     + mask[b, h, i, j]) * v[b, h / (q_h/v_h), j]
 * query [b, q_h, Lq, d], key [b, k_h, Lk, d], value [b, v_h, Lk, d] (bf16 or
 * f16, d in {64, 128}, innermost stride 1, 16-byte aligned rows); out
 * [b, Lq, q_h, d] of the same dtype: the layout the reference returns after
 * its transpose(1, 2).  mask (optional) [b | 1, q_h | 1, Lq, Lk]: bool keeps
 * True entries (False -> -inf), f32 / bf16 / f16 are added to the scaled
 * scores, as in torch SDPA.  causal != 0: key j is visible to query i only if
 * j <= i + causal_offset (SDPA's is_causal is causal_offset = 0; a chunk of
 * queries after P cached positions uses causal_offset = P).  A query that
 * sees no key gets 0 (torch SDPA's math path does the same).  scale must be
 * positive (SAGA_ERR_UNSUPPORTED otherwise). */
int saga_prefill_attention(const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
                           const saga_tensor* mask, float scale, int32_t causal, int64_t causal_offset,
                           saga_tensor* out, saga_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SAGA_AMD_H */

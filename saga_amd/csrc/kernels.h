// Launch parameter blocks and host launchers of the SAGA decode kernels.
// Shapes follow the reference's decode tensors (l_q == 1):
//   query [b, q_h, 1, d], key [b, k_h, L, d], value [b, v_h, L, d];
// score / selection rows are r = batch * q_h + head.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/saga_amd.h"

namespace saga {

// K1: scores = (Q_group . K^T) * scale (+ mask), per-chunk (max, sumexp).
struct QKParams {
  const char* q;
  int64_t q_sb, q_sh;  // element strides of batch / head
  const char* k;
  int64_t k_sb, k_sh, k_sl;
  const void* mask;  // nullable additive mask
  int32_t mask_dt;
  int64_t m_sb, m_sh, m_sl;
  const int32_t* kv_len;  // nullable
  int32_t b, q_h, k_h, g, L;
  int32_t ntiles, nparts;  // ceil(L / 16) tiles per row, split into nparts ranges
  float scale;
  float* scores;  // nullable: skip storing scores
  int64_t s_sb, s_sh;
  int32_t vec_store;  // rows 16-byte aligned: store 4 scores at once
  float* pmax;        // nullable: [row * (nparts / 4) + part / 4], one per block of 4 parts
  float* psum;
  float* ptail;       // nullable: max over the part's positions in the tail window
                      // [Leff - min(256, Leff), Leff), -inf if none
};
hipError_t launch_qk_scores(int dtype, int d, const QKParams& p, hipStream_t st);
// K1 tile ranges: at most kQKMaxTiles 16-position tiles per wave; launches are
// planned in whole rounds of kQKResidentWaves (256 CUs x 4 SIMDs x 3 waves, the
// occupancy the kernel is built for: at least 3).
constexpr int kQKMaxTiles = 6;
constexpr int64_t kQKResidentWaves = 256 * 4 * 3;
int64_t qk_plan(int64_t b, int64_t k_h, int64_t L);  // waves (parts) per (batch, key head), % 4 == 0

// Standalone logit threshold from a scores tensor.
struct ThreshParams {
  const float* scores;
  int64_t s_sb, s_sh;
  int32_t q_h, nrows, L;
  const int32_t* kv_len;
  const float* pstar;
  float* t_out;
};
hipError_t launch_logit_threshold(const ThreshParams& p, hipStream_t st);

// Selection-list softmax . V parameters (value tensor, output, row mapping).
struct PVParams {
  const void* w;  // API path: weights per row [nrows][K]
  int32_t w_dt;
  int64_t w_ld;
  const void* idx;  // API path: indices per row
  int32_t idx_i64;
  int64_t i_ld;
  int32_t K;
  const char* v;
  int32_t v_dt;
  int64_t v_sb, v_sh, v_sl;
  int32_t b, q_h, v_h, d, L;
  int32_t probs_mode;
  void* out;
  int32_t out_dt;
  int64_t o_sb, o_sh;
};
// API path of _atopn_gather_and_output: one block per row.
hipError_t launch_sparse_pv(const PVParams& p, hipStream_t st);

// K2: per score row of the fused workspace, threshold (fast step) or exact
// top-k (calibration), ordered compaction, then softmax . V of the list.
struct FusedSelParams {
  const float* scores;
  int64_t ld;
  const float* pmax;
  const float* psum;
  const float* ptail;  // [row * nparts + part] tail-window max of the part
  int32_t nparts;      // K1 block partials per row
  const int32_t* kv_len;
  int32_t q_h, nrows, L;
  const float* pstar;  // fast step: softmax-space thresholds in
  float* pstar_out;    // calibration: k-th largest probability out
  float* t_out;        // fast step: logit thresholds out
  int32_t cap;         // buf_k (fast) ; top_n capped at L (calibration)
  int32_t* sel_idx;
  float* sel_val;
  int32_t* sel_cnt;
  int32_t* sel_total;
  // fast step, split over slices of kSliceLen positions per row
  int32_t nslice, slice_cap;  // slice_cap = min(kSliceLen, cap)
  int32_t* sl_idx;            // [row][slice][slice_cap]
  float* sl_val;
  int32_t* sl_cnt;  // [row][slice] passing count in the slice
  float* sl_o;      // [row][slice][d] unnormalised sum_e w_e V[e] of short slices
  float* sl_ml;     // [row][slice][2] (max logit, sum of weights) of short slices
  int32_t* sl_pre;  // [row][2][nslice + 1] slice ranks (rows of > 2048 slices)
  // a row's gather split over kRowSplit blocks: their (m, l, -, -, o[d])
  // partials and the count of blocks done (zeroed by the slice kernel)
  float* row_part;   // [row][kRowSplit][d + 4]
  int32_t* row_cnt;  // [row]
  int32_t split_min;  // rows gathering more entries than this split (set by the row kernel's launcher)
  int32_t k2_variant;  // fast step: kK2Auto / kK2RowBlock / kK2SliceRow
  int32_t cal_chunk;   // spread calibration: positions per chunk (set by its launcher)
};
// calibrate: one block per row; fast step: slice kernel + per-row gather kernel
hipError_t launch_atopn_select_pv(bool calibrate, const FusedSelParams& p, const PVParams& v, hipStream_t st);
constexpr int kSliceLen = 1024;  // score positions per slice wave of the fast step
constexpr int kRowSplit = 4;     // blocks of the row kernel per row (a heavy row's gather is split over them)
constexpr int kSliceSmall = 96;  // slice lists this short are gathered by their slice wave (<= 2 bursts)
hipError_t launch_atopn_fast(const FusedSelParams& p, const PVParams& v, hipStream_t st);
// Fast-step K2 shape (FusedSelParams::k2_variant): 0 by shape (one block per
// row for rows of few slices), 1 always one block per row, 2 always slice
// kernel + row kernel.  Results are identical in every variant.
constexpr int kK2Auto = SAGA_K2_AUTO, kK2RowBlock = SAGA_K2_ROW_BLOCK, kK2SliceRow = SAGA_K2_SLICE_ROW;
bool k2_row_block(int64_t nslice, int64_t cap, int variant);
// Calibration spread over (row, chunk) blocks and a row kernel
// (calibrate_chunks.hip): built for rows of at least two chunks with
// top_n <= 2048 whose chunk lists fit the workspace's slice lists; the
// choice of kK2Auto for rows longer than kCalSpreadAutoLen, or of at least
// kCalSpreadFewRowsLen positions when there are at most kCalSpreadFewRows
// rows or more than kCalSpreadManyRows (one block per row then takes more
// than one round of the CUs); of kK2SliceRow wherever built; never of
// kK2RowBlock.
constexpr int64_t kCalSpreadAutoLen = 9 * 4096;
constexpr int64_t kCalSpreadFewRowsLen = 16384;
constexpr int64_t kCalSpreadFewRows = 24;
constexpr int64_t kCalSpreadManyRows = 256;
bool cal_spread(int64_t L, int64_t cap, int64_t nslice, int64_t slice_cap, int variant, int64_t nrows);
hipError_t launch_calibrate_spread(const FusedSelParams& p, const PVParams& v, hipStream_t st);
// One block per row on the same selection, rows of up to kCalRowBlockLen
// positions and k <= 2048 (the other rows: the older one-block kernels).
constexpr int64_t kCalRowBlockLen = 36 * 1024;
bool cal_row_block(int64_t L, int64_t cap);
hipError_t launch_calibrate_row_block(const FusedSelParams& p, const PVParams& v, hipStream_t st);

// API selection (threshold_topk_fast): typed rows, typed values out.
struct ApiSelParams {
  const void* x;
  int32_t x_dt;
  int64_t x_ld;
  int32_t nrows;
  int64_t D;
  const float* thresh;
  int64_t thresh_numel;
  int32_t k;
  void* out_val;
  int64_t ov_ld;
  int64_t* out_idx;
  int64_t oi_ld;
  int32_t* out_counts;  // nullable
};
hipError_t launch_select_api(const ApiSelParams& p, hipStream_t st);

// Dense split-L decode (flash-decoding): one pass over K and V.
struct DenseParams {
  const char* q;
  int64_t q_sb, q_sh;
  const char* k;
  int64_t k_sb, k_sh, k_sl;
  const char* v;
  int64_t v_sb, v_sh, v_sl;
  const void* mask;
  int32_t mask_dt;
  int64_t m_sb, m_sh, m_sl;
  const int32_t* kv_len;
  int32_t b, q_h, k_h, v_h, g, L;
  float scale;
  void* out;
  int32_t out_dt;
  int64_t o_sb, o_sh;
  float* part;  // [unit][nsplit][g][2 + d]
  int32_t nsplit, split_len;
};
hipError_t launch_dense_decode(int dtype, int d, const DenseParams& p, hipStream_t st);

// RoPE on q/k of new tokens + k/v append into the separate caches.
struct RopeParams {
  const void* qkv;  // [N, qkv_ld]: n_q, n_k, n_v heads of d, in that order
  int64_t qkv_ld;
  int32_t dt;
  int32_t N, n_q, n_k, n_v, d;
  float theta;
  const int32_t* pos;    // [N]
  const int32_t* batch;  // [N] or null (token n -> batch row n)
  void* q_out;           // [N, n_q, d]
  int64_t q_sn, q_sh;
  void* k_cache;  // [B, n_k, Lmax, d]
  int64_t k_sb, k_sh, k_sl;
  void* v_cache;  // [B, n_v, Lmax, d]
  int64_t v_sb, v_sh, v_sl;
  int32_t B, Lmax;
  // [N][d/2][2] fp32 (cos, sin) of the token rows' rotations (launch_rope_table),
  // or null: computed where they are used
  const float* table;
};
hipError_t launch_rope_kv_append(const RopeParams& p, hipStream_t st);
// table[n][i] = (cos, sin)(pos[n] * theta^(-2i/d)), i < d/2, n < N
hipError_t launch_rope_table(const int32_t* pos, int N, int d, float theta, float* table, hipStream_t st);

// x[b] = embed[tokens[b]] for b < B (+ the rows' rotations into table when given)
struct EmbedParams {
  const int64_t* tokens;
  const void* embed;  // [V, H], row stride e_ld
  int64_t e_ld;
  void* x;  // [B, H], row stride x_ld, dtype dt
  int64_t x_ld;
  int32_t B, H, dt, vec;  // vec: rows copied in 16-byte chunks
  int64_t V;
  const int32_t* pos;  // [B] (with table)
  int32_t d;
  float theta;
  float* table;  // [B][d/2][2] or null
};
hipError_t launch_embed_rope(const EmbedParams& p, hipStream_t st);
hipError_t launch_advance(int32_t* pos, int32_t* kv_len, int n, hipStream_t st);

// Row-wise ops: rmsnorm (y = w * x * rsqrt(mean(x^2) + eps)) and silu_mul.
struct RowParams {
  const void* x;
  int64_t x_ld;
  const void* w;
  void* y;
  int64_t y_ld;
  int32_t dt;
  int32_t N, H;
  float eps;
};
hipError_t launch_rmsnorm(const RowParams& p, hipStream_t st);
hipError_t launch_silu_mul(const RowParams& p, hipStream_t st);

// Skinny GEMM y[m, n] = rms(x)[m] * sum_k x[m, k] W[n, k] (+ epilogue), m < 32.
struct GemvParams {
  const void* x;  // bf16 [M, K]
  int64_t x_ld;
  const void* w;  // bf16 [N, K] (row stride w_ld), or packed [N/16][K/32][16][32]
  int64_t w_ld;
  // 1: packed [N/16][K/32][16][32], every MFMA A fragment (16 rows x 32 k) 1 KB
  // contiguous; 2: packed [N/8][K/64][512] in 8-row tiles (at most 8 token rows)
  int32_t w_packed;
  const void* bias;  // bf16 [N] or null
  void* y;           // bf16 [M, N] (SILU_PAIRS: [M, N / 2])
  int64_t y_ld;
  int32_t M, N, K;
  int32_t rms;  // scale by 1/sqrt(mean(x^2) + eps)
  float eps;
  int32_t epilogue;
  // kGemvRopeKV: y is unused; rows of w are the fused q/k/v projection with
  // the q and k heads in rotary-pair order, written through `rope` (qkv unused)
  RopeParams rope;
  // split-K (part != null): K cut into `splits` ranges, one workgroup each;
  // part [splits][M][N] and part_ssq [splits][M] fp32, finished by an epilogue kernel
  int32_t splits;
  float* part;
  float* part_ssq;
};
int gemv_splits(int64_t N, int64_t K);  // K ranges worth launching for an N x K weight
int gemv_tiles_per_wave(int64_t N, int64_t K);  // 16-row W tiles per wave of the one-range kernel
constexpr int kGemvRopeKV = 3;
hipError_t launch_gemv(const GemvParams& p, hipStream_t st);
// ws (optional, argmax_workspace_bytes): two passes over many blocks per row
int64_t argmax_workspace_bytes(int64_t rows, int64_t N);
hipError_t launch_argmax(const void* x, int64_t ld, int rows, int N, int64_t* out, void* ws, hipStream_t st);

// Prefill attention with separate key / value head maps (csrc/prefill.hip).
// Strides in elements; q [b, q_h, Lq, d], k [b, k_h, Lk, d], v [b, v_h, Lk, d],
// mask [b|1, q_h|1, Lq, Lk] (broadcast dims stride 0), out [b, Lq, q_h, d].
struct PrefillParams {
  const char* q;
  int64_t q_sb, q_sh, q_sl;
  const char* k;
  int64_t k_sb, k_sh, k_sl;
  const char* v;
  int64_t v_sb, v_sh, v_sl;
  const void* mask;  // null: none; bool keeps True, float is added
  int32_t mask_dt;
  int64_t m_sb, m_sh, m_sq, m_sk;
  void* out;
  int64_t o_sb, o_sq, o_sh;
  int32_t b, q_h, k_h, v_h, Lq, Lk;
  int32_t nmb;         // query blocks per (batch, head)
  int32_t causal;      // key j visible to query i iff j <= i + causal_off
  int32_t causal_off;
  float scale;
};
int prefill_query_blocks(int64_t Lq, int d);
hipError_t launch_prefill_attention(int dtype, int d, const PrefillParams& p, hipStream_t st);

}  // namespace saga

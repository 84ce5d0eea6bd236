// K1: decode QK scores for every query head against its shared key head.
//
// Replaces the bmm + scale + mask of _compute_attn_weights
// (attention/attention.py:113-128).  One wave owns one (batch, key head,
// 128-position chunk) item: it streams the chunk's K rows once with 16-byte
// loads straight into MFMA A fragments (16 positions x 32 dims per
// v_mfma_f32_16x16x32_bf16), multiplies by the g = q_h / k_h query heads of
// the group held as the B fragment (g <= 16, padded with zeros), and writes
//   * fp32 scores  x = acc * scale (+ mask), -inf at positions >= kv_len,
//   * the chunk's per-head max m_c and sum_c exp(x - m_c),
// so the logit threshold t = m + log(p* * sum_c s_c exp(m_c - m)) needs no
// second pass over the scores.  The K stream is the only large read.
#include "common.cuh"
#include "kernels.h"

namespace saga {

constexpr int kQKTiles = SAGA_CHUNK / 16;  // 16-position MFMA tiles per chunk item

template <int DT, int D, int TPL>
__global__ void __launch_bounds__(256) qk_scores_kernel(QKParams p) {
  using E = Elt<DT>;
  constexpr int E16 = E::kPer16B;           // elements per 16-byte fragment
  constexpr int NLOAD = D / (4 * E16);      // fragments per K row per lane
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;                // MFMA row (position) / column (head)
  const int s = lane >> 4;                  // k-slot group
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t nitems = static_cast<int64_t>(p.b) * p.k_h * p.nchunk;
  if (item >= nitems) return;
  const int chunk = static_cast<int>(item % p.nchunk);
  const int unit = static_cast<int>(item / p.nchunk);
  const int bi = unit / p.k_h;
  const int kh = unit - bi * p.k_h;
  const bool hvalid = col < p.g;
  const int h = kh * p.g + (hvalid ? col : 0);

  // B fragment: query head (kh*g + col), dims [j*4*E16 + s*E16, +E16).
  u32x4 qf[NLOAD];
  const char* qrow = p.q + (bi * p.q_sb + static_cast<int64_t>(h) * p.q_sh) * E::kBytes;
#pragma unroll
  for (int j = 0; j < NLOAD; ++j) {
    qf[j] = hvalid ? ld16(qrow + (j * 4 * E16 + s * E16) * E::kBytes) : u32x4{0u, 0u, 0u, 0u};
  }

  const char* kbase = p.k + (bi * p.k_sb + static_cast<int64_t>(kh) * p.k_sh) * E::kBytes;
  const int p0 = chunk * SAGA_CHUNK;
  float x[kQKTiles][4];
#pragma unroll
  for (int tb = 0; tb < kQKTiles; tb += TPL) {
    u32x4 kf[TPL][NLOAD];
#pragma unroll
    for (int t = 0; t < TPL; ++t) {
      // A fragment: key row (p0 + 16*(tb+t) + col); rows past L are clamped
      // (their scores are discarded below).
      const int pos = min(p0 + 16 * (tb + t) + col, p.L - 1);
      const char* krow = kbase + static_cast<int64_t>(pos) * p.k_sl * E::kBytes;
#pragma unroll
      for (int j = 0; j < NLOAD; ++j) kf[t][j] = ld16(krow + (j * 4 * E16 + s * E16) * E::kBytes);
    }
    // keep the whole burst in flight: no MFMA may be hoisted between the loads
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < TPL; ++t) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NLOAD; ++j) acc = mfma_16b<DT>(kf[t][j], qf[j], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) x[tb + t][r] = acc[r];
    }
  }

  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  // Lane holds head `col`, positions p0 + 16*t + 4*s + r.
  float m = kNegInf;
#pragma unroll
  for (int t = 0; t < kQKTiles; ++t) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int pos = p0 + 16 * t + 4 * s + r;
      float v = x[t][r] * p.scale;
      if (p.mask) {
        const int mp = min(pos, p.L - 1);
        v = v + load_as_f32(p.mask, p.mask_dt, bi * p.m_sb + static_cast<int64_t>(h) * p.m_sh +
                                                   static_cast<int64_t>(mp) * p.m_sl);
      }
      if (pos >= Leff) v = kNegInf;
      x[t][r] = v;
      m = fmaxf(m, v);
    }
  }

  if (p.scores && hvalid) {
    float* srow = p.scores + bi * p.s_sb + static_cast<int64_t>(h) * p.s_sh;
#pragma unroll
    for (int t = 0; t < kQKTiles; ++t) {
      const int pos0 = p0 + 16 * t + 4 * s;
      if (p.vec_store && pos0 + 3 < p.L) {
        *reinterpret_cast<f32x4*>(srow + pos0) = f32x4{x[t][0], x[t][1], x[t][2], x[t][3]};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (pos0 + r < p.L) srow[pos0 + r] = x[t][r];
      }
    }
  }

  if (p.pmax) {
    float sum = 0.f;
    if (m != kNegInf) {
#pragma unroll
      for (int t = 0; t < kQKTiles; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) sum += __expf(x[t][r] - m);
    }
    // the four lane groups holding the same head
    lse_merge(m, sum, __shfl_xor(m, 16), __shfl_xor(sum, 16));
    lse_merge(m, sum, __shfl_xor(m, 32), __shfl_xor(sum, 32));
    if (s == 0 && hvalid) {
      const int64_t o = static_cast<int64_t>(bi * p.q_h + h) * p.nchunk + chunk;
      p.pmax[o] = m;
      p.psum[o] = sum;
    }
  }
}

template <int DT, int D>
static hipError_t launch_qk_typed(const QKParams& p, hipStream_t st) {
  constexpr int NLOAD = D / (4 * Elt<DT>::kPer16B);
  constexpr int TPL = (NLOAD * kQKTiles <= 32) ? kQKTiles : (32 / NLOAD);
  const int64_t nitems = static_cast<int64_t>(p.b) * p.k_h * p.nchunk;
  const int64_t blocks = (nitems + 3) / 4;
  hipLaunchKernelGGL((qk_scores_kernel<DT, D, TPL>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_qk_scores(int dtype, int d, const QKParams& p, hipStream_t st) {
  if (dtype == SAGA_DTYPE_BF16) return d == 128 ? launch_qk_typed<SAGA_DTYPE_BF16, 128>(p, st)
                                                : launch_qk_typed<SAGA_DTYPE_BF16, 64>(p, st);
  if (dtype == SAGA_DTYPE_F16) return d == 128 ? launch_qk_typed<SAGA_DTYPE_F16, 128>(p, st)
                                               : launch_qk_typed<SAGA_DTYPE_F16, 64>(p, st);
  return d == 128 ? launch_qk_typed<SAGA_DTYPE_F32, 128>(p, st)
                  : launch_qk_typed<SAGA_DTYPE_F32, 64>(p, st);
}

// Standalone logit threshold, attention/attention.py:136-149, one block per
// row over a scores tensor: m = max of the last min(256, L) logits,
// t = m + log(max(p*, 1e-30) * sum exp(x - m)).
__global__ void __launch_bounds__(256) logit_threshold_kernel(ThreshParams p) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const int bi = r / p.q_h, h = r - bi * p.q_h;
  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  const float* row = p.scores + bi * p.s_sb + static_cast<int64_t>(h) * p.s_sh;
  const int tail = min(256, Leff);
  const int tid = threadIdx.x;
  const float v = tid < tail ? row[Leff - tail + tid] : kNegInf;
  const float m = block_max<4>(v, red);
  float acc = 0.f;
  for (int i = tid; i < Leff; i += 256) acc += __expf(row[i] - m);
  const float ssum = block_sum<4>(acc, red);
  if (tid == 0) p.t_out[r] = m + logf(fmaxf(p.pstar[r], 1e-30f) * ssum);
}

hipError_t launch_logit_threshold(const ThreshParams& p, hipStream_t st) {
  hipLaunchKernelGGL(logit_threshold_kernel, dim3(p.nrows), dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace saga

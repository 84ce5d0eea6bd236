// K1: decode QK scores for every query head against its shared key head.
//
// Replaces the bmm + scale + mask of _compute_attn_weights
// (attention/attention.py:113-128).  The key rows of one (batch, key head)
// are split into `nparts` contiguous ranges of 16-position MFMA tiles, with
// the tile counts balanced (they differ by at most one, and are at most
// kQKMaxTiles).  One wave owns one range: it issues every 16-byte load of the
// range's K rows at once, straight into MFMA A fragments (16 positions x 32
// dims per v_mfma_f32_16x16x32_bf16), multiplies by the g = q_h / k_h query
// heads of the group held as the B fragment (g <= 16, padded with zeros), and
// writes
//   * fp32 scores  x = acc * scale (+ mask), -inf at positions >= kv_len,
//   * per block of 4 waves (4 consecutive ranges) and head: the max m_c, the
//     sum_c exp(x - m_c) and the max over the tail window (the last
//     min(256, kv_len) positions),
// so the logit threshold t = m + log(p* * sum_c s_c exp(m_c - m)) needs no
// second pass over the scores.  The K stream is the only large read.  The
// host planner (qk_plan) picks nparts so that all waves of a launch fit the
// GPU in whole rounds: no round runs a handful of leftover waves.
#include <algorithm>

#include "qk_wave.cuh"

namespace saga {

template <int DT, int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 8)))
qk_scores_kernel(QKParams p) {
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;                // MFMA row (position) / column (head)
  const int s = lane >> 4;                  // k-slot group
  __shared__ float red[3][4][16];  // per wave and head: (max, sum, tail max) of the part
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  // nparts % 4 == 0: the block's 4 waves are parts 4j..4j+3 of one (batch, key head)
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave;
  const int part = static_cast<int>(item % p.nparts);
  const int unit = static_cast<int>(item / p.nparts);
  const QKWaveSpan w = qk_wave_span(p, unit, part, col);
  float x[kQKMaxTiles][4];
  int Leff;
  const float m = qk_wave_scores<DT, D>(p, w, s, col, x, Leff);

  if (p.scores && w.hvalid) {
    float* srow = p.scores + w.bi * p.s_sb + static_cast<int64_t>(w.h) * p.s_sh;
#pragma unroll
    for (int t = 0; t < kQKMaxTiles; ++t) {
      if (t >= w.nt) break;
      const int pos0 = 16 * (w.t0 + t) + 4 * s;
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
    // the block's 4 parts merged into one partial per head
    float pm, ps, pt;
    qk_block_partial(x, m, w, Leff, p.ptail != nullptr, s, col, wave, red, pm, ps, pt);
    if (wave == 0 && s == 0 && w.hvalid) {
      const int row = w.bi * p.q_h + w.h;
      const int64_t o = static_cast<int64_t>(row) * (p.nparts / 4) + part / 4;
      p.pmax[o] = pm;
      p.psum[o] = ps;
      if (p.ptail) p.ptail[o] = pt;
    }
  }
}

int64_t qk_plan(int64_t b, int64_t k_h, int64_t L) {
  const int64_t tiles = (L + 15) / 16;
  if (tiles == 0) return 4;
  const int64_t units = b * k_h;
  const int64_t minp = (tiles + kQKMaxTiles - 1) / kQKMaxTiles;
  const int64_t rounds = (units * minp + kQKResidentWaves - 1) / kQKResidentWaves;
  const int64_t fill = rounds * kQKResidentWaves / units;  // whole rounds of resident waves
  const int64_t np = std::max(minp, std::min(tiles, fill));
  return (np + 3) / 4 * 4;  // whole blocks of 4 waves per (batch, key head); a part may hold no tile
}

template <int DT, int D>
static hipError_t launch_qk_typed(const QKParams& p, hipStream_t st) {
  const int64_t nitems = static_cast<int64_t>(p.b) * p.k_h * p.nparts;  // nparts % 4 == 0
  const int64_t blocks = nitems / 4;
  hipLaunchKernelGGL((qk_scores_kernel<DT, D>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, p);
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

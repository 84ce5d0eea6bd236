// One wave's share of the decode QK scores (K1, qk_scores_kernel).
//
// A wave owns tiles [t0, t0 + nt) of 16 positions of one (batch, key head),
// nt <= kQKMaxTiles.  It issues every 16-byte load of its K rows at once,
// straight into MFMA A fragments (16 positions x 32 dims per
// v_mfma_f32_16x16x32_bf16), multiplies by the g = q_h / k_h query heads of
// the group held as the B fragment (g <= 16, padded with zeros) and leaves
//   x[t][r] = acc * scale (+ mask), -inf at positions >= kv_len or past the range,
// for lane (s = lane / 16, col = lane % 16): head col, position
// 16 * (t0 + t) + 4 * s + r.
#pragma once

#include "common.cuh"
#include "kernels.h"

namespace saga {

// Read in place of kv_len[b] when no kv_len is given: no truncation.
static __device__ int32_t g_no_kv_len = 0x7fffffff;

template <int DT, int D>
struct QKShape {
  static constexpr int E16 = Elt<DT>::kPer16B;  // elements per 16-byte fragment
  static constexpr int NLOAD = D / (4 * E16);   // fragments per K row per lane
  // tiles per load burst: at most 24 fragments (96 VGPRs) in flight per lane
  static constexpr int BURST = (24 / NLOAD) < kQKMaxTiles ? (24 / NLOAD) : kQKMaxTiles;
};

// Where a wave's tiles lie: unit = batch * k_h + key head, part in [0, nparts).
struct QKWaveSpan {
  int bi, kh, h, t0, nt;
  bool hvalid;
};

__device__ __forceinline__ QKWaveSpan qk_wave_span(const QKParams& p, int unit, int part, int col) {
  QKWaveSpan w;
  w.bi = unit / p.k_h;
  w.kh = unit - w.bi * p.k_h;
  w.hvalid = col < p.g;
  w.h = w.kh * p.g + (w.hvalid ? col : 0);
  w.t0 = static_cast<int>(static_cast<int64_t>(part) * p.ntiles / p.nparts);
  w.nt = static_cast<int>(static_cast<int64_t>(part + 1) * p.ntiles / p.nparts) - w.t0;
  return w;
}

// Scores of the wave's tiles into x; returns the lane's max and sets Leff
// (the batch row's kv_len capped at L).
template <int DT, int D>
__device__ __forceinline__ float qk_wave_scores(const QKParams& p, const QKWaveSpan& w, int s, int col,
                                                float (&x)[kQKMaxTiles][4], int& Leff) {
  using E = Elt<DT>;
  using S = QKShape<DT, D>;
  constexpr int E16 = S::E16, NLOAD = S::NLOAD, BURST = S::BURST;
  const int t0 = w.t0, nt = w.nt;

  // kv_len first, as a vector load (a relaxed atomic is never turned into a
  // scalar load, whose lgkmcnt wait the next kernel-argument read would share):
  // issued before the K burst it returns with it (loads return in order), so
  // the masking below waits for nothing; read after the burst it would cost
  // every wave one more round trip behind the whole stream
  // (no branch: a load under a branch is waited for at the join)
  int32_t* kvp = p.kv_len ? const_cast<int32_t*>(p.kv_len) + w.bi : &g_no_kv_len;
  const int kvl = __hip_atomic_load(kvp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);

  // B fragment: query head (kh*g + col), dims [j*4*E16 + s*E16, +E16).
  u32x4 qf[NLOAD];
  const char* qrow = p.q + (w.bi * p.q_sb + static_cast<int64_t>(w.h) * p.q_sh) * E::kBytes;
#pragma unroll
  for (int j = 0; j < NLOAD; ++j) {
    qf[j] = w.hvalid ? ld16(qrow + (j * 4 * E16 + s * E16) * E::kBytes) : u32x4{0u, 0u, 0u, 0u};
  }

  const char* kbase = p.k + (w.bi * p.k_sb + static_cast<int64_t>(w.kh) * p.k_sh) * E::kBytes;
#pragma unroll
  for (int tb = 0; tb < kQKMaxTiles; tb += BURST) {
    if (tb >= nt) break;
    u32x4 kf[BURST][NLOAD];
#pragma unroll
    for (int t = 0; t < BURST; ++t) {
      // A fragment: key row (16*(t0+tb+t) + col), rows past L clamped (their
      // scores are discarded below); tiles past the range are not loaded
      const int pos = min(16 * (t0 + tb + t) + col, p.L - 1);
      const char* krow = kbase + static_cast<int64_t>(pos) * p.k_sl * E::kBytes;
#pragma unroll
      for (int j = 0; j < NLOAD; ++j)
        kf[t][j] = tb + t < nt ? ld16(krow + (j * 4 * E16 + s * E16) * E::kBytes) : u32x4{0u, 0u, 0u, 0u};
    }
    // keep the whole burst in flight: no MFMA may be hoisted between the loads
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < BURST; ++t) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NLOAD; ++j) acc = mfma_16b<DT>(kf[t][j], qf[j], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) x[tb + t][r] = acc[r];
    }
  }

  // first use of kvl, after the MFMAs; the empty asm keeps it in a VGPR (a
  // uniform value would be moved to an SGPR, and waited for, right at its load)
  int kv = kvl;
  asm volatile("" : "+v"(kv));
  Leff = min(p.L, max(kv, 0));
#pragma unroll
  for (int t = 0; t < kQKMaxTiles; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) x[t][r] *= p.scale;
  if (p.mask) {
    // every mask element of the wave in one burst (one round trip), the
    // dtype switch outside the loads
    const int64_t mrow = w.bi * p.m_sb + static_cast<int64_t>(w.h) * p.m_sh;
    auto moff = [&](int t, int r) {
      return mrow + static_cast<int64_t>(min(16 * (t0 + t) + 4 * s + r, p.L - 1)) * p.m_sl;
    };
    float mv[kQKMaxTiles][4];
    if (p.mask_dt == SAGA_DTYPE_BOOL) {
      const uint8_t* mp = static_cast<const uint8_t*>(p.mask);
      uint32_t raw[kQKMaxTiles][4];
#pragma unroll
      for (int t = 0; t < kQKMaxTiles; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) raw[t][r] = mp[moff(t, r)];
#pragma unroll
      for (int t = 0; t < kQKMaxTiles; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) mv[t][r] = raw[t][r] ? 1.0f : 0.0f;
    } else if (p.mask_dt == SAGA_DTYPE_F32) {
      const float* mp = static_cast<const float*>(p.mask);
#pragma unroll
      for (int t = 0; t < kQKMaxTiles; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) mv[t][r] = mp[moff(t, r)];
    } else {
      const uint16_t* mp = static_cast<const uint16_t*>(p.mask);
      uint32_t raw[kQKMaxTiles][4];
#pragma unroll
      for (int t = 0; t < kQKMaxTiles; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) raw[t][r] = mp[moff(t, r)];
      const bool bf = p.mask_dt == SAGA_DTYPE_BF16;
#pragma unroll
      for (int t = 0; t < kQKMaxTiles; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          mv[t][r] = bf ? bf16_bits_to_f32(raw[t][r]) : f16_bits_to_f32(static_cast<uint16_t>(raw[t][r]));
    }
#pragma unroll
    for (int t = 0; t < kQKMaxTiles; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) x[t][r] += mv[t][r];
  }
  float m = kNegInf;
#pragma unroll
  for (int t = 0; t < kQKMaxTiles; ++t) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int pos = 16 * (t0 + t) + 4 * s + r;
      if (pos >= Leff || t >= nt) x[t][r] = kNegInf;
      m = fmaxf(m, x[t][r]);
    }
  }
  return m;
}

// The (max, sum of exp(x - max), max over the tail window [Leff - min(256,
// Leff), Leff)) of the block's 4 waves per head, merged through `red`.  The
// result is valid in wave 0, lanes s == 0 (one per head col); every thread of
// the block must call this (it holds a block barrier).
__device__ __forceinline__ void qk_block_partial(const float (&x)[kQKMaxTiles][4], float m, const QKWaveSpan& w,
                                                 int Leff, bool want_tail, int s, int col, int wave,
                                                 float (*red)[4][16], float& pm, float& ps, float& pt) {
  float sum = 0.f;
  if (m != kNegInf) {
#pragma unroll
    for (int t = 0; t < kQKMaxTiles; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) sum += __expf(x[t][r] - m);
  }
  // the four lane groups holding the same head
  lse_merge(m, sum, __shfl_xor(m, 16), __shfl_xor(sum, 16));
  lse_merge(m, sum, __shfl_xor(m, 32), __shfl_xor(sum, 32));
  float tm = kNegInf;
  if (want_tail) {
    const int tail_lo = Leff - min(256, Leff);
#pragma unroll
    for (int t = 0; t < kQKMaxTiles; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (16 * (w.t0 + t) + 4 * s + r >= tail_lo) tm = fmaxf(tm, x[t][r]);
    tm = fmaxf(tm, __shfl_xor(tm, 16));
    tm = fmaxf(tm, __shfl_xor(tm, 32));
  }
  if (s == 0) {
    red[0][wave][col] = m;
    red[1][wave][col] = sum;
    red[2][wave][col] = tm;
  }
  lds_sync();  // K1's score stores may still be in flight: no wait for them
  if (wave == 0 && s == 0) {
#pragma unroll
    for (int q = 1; q < 4; ++q) {
      lse_merge(m, sum, red[0][q][col], red[1][q][col]);
      tm = fmaxf(tm, red[2][q][col]);
    }
  }
  pm = m;
  ps = sum;
  pt = tm;
}

}  // namespace saga

// Skinny GEMM for decode projections: y[m, n] = sum_k x[m, k] * W[n, k], m < 32.
//
// W is row-major [N, K], or packed [N/16][K/32][16][32] (each 16-row x 32-k
// MFMA A fragment 1 KB contiguous: a load instruction reads 1 KB of one
// DRAM region instead of 64 B from 16 rows one row stride apart).
//
// Decode steps multiply a handful of token rows (the batch) by every weight
// matrix once, so the kernel is a weight stream: 16 rows of W per MFMA tile,
// loaded 16 bytes per lane straight into the A fragment of
// v_mfma_f32_16x16x32_bf16 (as K1 streams K rows), with the token rows as
// the B fragment.  A workgroup owns 16 output columns n; its waves split K
// and meet in LDS.  Fused pieces:
//   * RMSNorm of x (Qwen2RMSNorm): the norm weight is folded into W when the
//     model is built, and the per-row 1/sqrt(mean(x^2) + eps) is a scalar of
//     the output row, accumulated from the x fragments the waves load anyway;
//   * epilogues: + bias, += into y (residual stream), or silu(gate) * up for
//     W rows interleaved as [gate_0, up_0, gate_1, up_1, ...].
#include <algorithm>

#include "common.cuh"
#include "kernels.h"

namespace saga {

constexpr int kGemvUnroll = 12;  // 32-wide k steps in flight per wave (K = 1536 over 4 waves: one burst)
constexpr int kSplitBatch = 8;   // split-K partial sums in flight per epilogue thread

// Epilogue inputs of one lane, loaded right behind the first weight burst (as
// loads they return with it; after the reduction each would cost one more
// round trip):
// the residual of output rows n..n+3 of token row m (SAGA_GEMV_ADD), and the
// bias, position, batch row and rotations (with a rotation table) of the
// fused q/k/v projection (kGemvRopeKV).
// Absent inputs read a valid dummy address instead of branching (a load under
// a branch is waited for at the join, ahead of the burst).  Other epilogues
// load their (rare) bias after the reduction, keeping registers for the burst.
struct GemvPre {
  uint16_t bias[4], y[4];
  int pos, batch;
  f32x4 rot;  // (cos, sin) of the rotary pairs j/2 and j/2 + 1, j = n mod d
};

template <int EPI>
__device__ __forceinline__ GemvPre gemv_prefetch(const GemvParams& p, int m, int n, const void* dummy) {
  GemvPre e{};
  if constexpr (EPI == SAGA_GEMV_ADD) {
    const uint16_t* yp = static_cast<const uint16_t*>(p.y) + static_cast<int64_t>(m) * p.y_ld + n;
#pragma unroll
    for (int r = 0; r < 4; ++r) e.y[r] = yp[r];
  }
  if constexpr (EPI == kGemvRopeKV) {
    const uint16_t* bp = p.bias ? static_cast<const uint16_t*>(p.bias) + n : static_cast<const uint16_t*>(dummy);
#pragma unroll
    for (int r = 0; r < 4; ++r) e.bias[r] = bp[r];
    e.pos = p.rope.pos[m];
    e.batch = *(p.rope.batch ? p.rope.batch + m : p.rope.pos + m);
    if (!p.rope.batch) e.batch = m;
    // rows n..n+3 hold the pairs j/2, j/2 + 1 (j % 4 == 0): 16 aligned bytes
    const int j = n % p.rope.d;
    const float* rt = p.rope.table ? p.rope.table + (static_cast<int64_t>(m) * (p.rope.d / 2) + j / 2) * 2
                                   : static_cast<const float*>(dummy);
    e.rot = *reinterpret_cast<const f32x4*>(rt);
  }
  return e;
}

// TPW tiles of 16 W rows per workgroup (rows n0 .. n0 + 16*TPW): each k step
// loads one x fragment and TPW W fragments, so a wave keeps TPW x more weight
// bytes in flight per register of x.
//
// HALF (at most 8 token rows, W packed in 8-row tiles): a tile is 8 W rows
// and a k step 64 wide.  A fragment rows 0-7 are the tile's rows at k
// [64j, 64j + 32) and rows 8-15 the same rows at [64j + 32, 64j + 64); the B
// columns 0-7 are the token rows at the first half and 8-15 at the second.
// Output rows i < 8 of columns c < 8 and rows 8 + i of columns 8 + c then
// hold the two halves of y[c, n0 + i] (the other two quarters are unused
// products), added across lanes before the reduction: lane l = 16s + c
// (s < 2, c < 8) and lane l + 40.  Weights of few 16-row tiles (a 1536-row projection: 96) so
// spread over twice the workgroups, each CU streaming half the bytes, with no
// split over K.  UNROLL: k steps per wave and burst.
//
// MT = 2 (17 to 32 token rows): every W fragment meets two B fragments, token
// rows c and 16 + c of lane column c, into two accumulators; the epilogue
// waves split over (tile, token tile).
template <int WAVES, int EPI, int TPW, bool HALF = false, int UNROLL = kGemvUnroll, int MT = 1>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(TPW == 2 ? 3 : 4, 8)))
gemv_kernel(GemvParams p) {
  static_assert(!HALF || (TPW == 1 && MT == 1), "8-row tiles: one per wave, at most 8 token rows");
  static_assert(WAVES >= TPW * MT, "one epilogue wave per (tile, token tile)");
  constexpr int TR = HALF ? 8 : 16;  // W rows per tile
  __shared__ float red[WAVES][TPW * MT][64][4];
  __shared__ float rsq[WAVES][MT][64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int col = lane & 15, s = lane >> 4;
  const int n0 = blockIdx.x * TR * TPW;
  const int split = blockIdx.y;  // K range of this workgroup (split-K: partial sums out)
  const int mrow = HALF ? (col & 7) : col;  // token row of this lane's x fragments (+ 16 per token tile)
  // the (tile, token tile) this wave finishes (waves 0 .. TPW*MT - 1) and
  // its token row m: the epilogue inputs are loaded for it
  const int tf = w < TPW * MT ? (MT == 1 ? w : w % TPW) : TPW - 1;
  const int mte = MT == 1 ? 0 : (w < TPW * MT ? w / TPW : 0);
  const int tme = mrow + 16 * mte;
  const int m = tme < p.M ? tme : 0;
  // A fragment of tile t at k step j: wrow[t] + j * wstep.  Row-major W:
  // 16 rows x 64 B, one row per W row stride; packed W: 1 KB contiguous
  const int64_t wstep = p.w_packed ? 1024 : 64;
  const int steps = p.K / (HALF ? 64 : 32);
  const char* wrow[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
    wrow[t] = static_cast<const char*>(p.w) +
              (p.w_packed ? static_cast<int64_t>(n0 / TR + t) * steps * 1024 + col * 64 + s * 16
                          : (static_cast<int64_t>(n0 + 16 * t + col) * p.w_ld + 8 * s) * 2);
  // x fragments: 8 k values of token row mrow + 16 mt (HALF: of the k half of column col)
  const int64_t xstep = HALF ? 128 : 64;
  bool xvalid[MT];
  const char* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int mm = mrow + 16 * mt;
    xvalid[mt] = mm < p.M;
    xrow[mt] = static_cast<const char*>(p.x) +
               (static_cast<int64_t>(xvalid[mt] ? mm : 0) * p.x_ld + 8 * s + (HALF ? 32 * (col >> 3) : 0)) * 2;
  }
  // (HALF: lanes s < 2 own rows n0 + 4s .. + 3; lanes s >= 2 load the same)
  const int nf = n0 + TR * tf + 4 * (HALF ? (s & 1) : s);
  // this workgroup's k steps [k0, k1), dealt to its waves round robin (wave
  // w: k0 + w, k0 + w + WAVES, ...): at any moment the workgroup's waves
  // read neighbouring fragments of its tiles (measured faster than a
  // contiguous share per wave, for packed and row-major W)
  const int k0 = split * steps / p.splits, k1 = (split + 1) * steps / p.splits;
  const int nmine = (k1 - k0 - w + WAVES - 1) / WAVES;
  const int jstride = WAVES;
  const int jbase = k0 + w;
  f32x4 acc[TPW][MT];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float ssq[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) ssq[mt] = 0.f;
  // one burst: every k step of [i0, i0 + UNROLL) of the wave (steps past its
  // share repeat its last one, clamped into the workgroup's range: a wave
  // with no step loads valid addresses it never uses)
  auto load_burst = [&](int i0, u32x4 (&a)[UNROLL][TPW], u32x4 (&b)[UNROLL][MT]) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int jj = min(max(jbase + jstride * min(i0 + u, nmine - 1), k0), k1 - 1);
#pragma unroll
      for (int t = 0; t < TPW; ++t) a[u][t] = ld16(wrow[t] + static_cast<int64_t>(jj) * wstep);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        b[u][mt] = xvalid[mt] ? ld16(xrow[mt] + static_cast<int64_t>(jj) * xstep) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto use_burst = [&](int i0, const u32x4 (&a)[UNROLL][TPW], const u32x4 (&b)[UNROLL][MT]) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (i0 + u < nmine) {
#pragma unroll
        for (int t = 0; t < TPW; ++t)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[t][mt] = mfma_16b<SAGA_DTYPE_BF16>(a[u][t], b[u][mt], acc[t][mt]);
        if (p.rms) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            float f[8];
            unpack16<SAGA_DTYPE_BF16>(b[u][mt], f);
#pragma unroll
            for (int i = 0; i < 8; ++i) ssq[mt] += f[i] * f[i];
          }
        }
      }
    }
  };
  // The first burst (the only one for waves of at most UNROLL k steps: every
  // decode projection of K <= 1536 and every split-K range), then the
  // epilogue inputs.  Issued behind the burst they return right after it
  // (loads return in order); issued ahead of a loop they would be waited for
  // at its header, before the burst.
  GemvPre pre;
  {
    u32x4 a[UNROLL][TPW], b[UNROLL][MT];
    load_burst(0, a, b);
    pre = gemv_prefetch<EPI>(p, m, nf, wrow[0]);
    __builtin_amdgcn_sched_barrier(0);
    use_burst(0, a, b);
  }
  for (int i0 = UNROLL; i0 < nmine; i0 += UNROLL) {
    u32x4 a[UNROLL][TPW], b[UNROLL][MT];
    load_burst(i0, a, b);
    __builtin_amdgcn_sched_barrier(0);
    use_burst(i0, a, b);
  }
  if constexpr (HALF) {
    // fold the second k half into lanes l = 16s + c (s < 2, c < 8): + lane l + 40
    // (rows 8 + 4s + r, column 8 + c); the x^2 sums of the two halves of token
    // row c & 7 meet in lanes c and c ^ 8
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[0][0][r] += __shfl(acc[0][0][r], (lane + 40) & 63);
    ssq[0] += __shfl_xor(ssq[0], 8);
  }
  // lane (col, s): rows n0 + 16t + 4s + r of tile t for token row col + 16 mt
  // (HALF: rows n0 + 4s + r, s < 2, col < 8)
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[w][t + TPW * mt][lane][r] = acc[t][mt][r];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) rsq[w][mt][lane] = ssq[mt];
  lds_sync();
  if (w >= TPW * MT) return;
  if (HALF && (s >= 2 || col >= 8)) return;  // folded into the lanes above
  const int t = tf;
  const int tm = tme;  // this lane's output token row
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  float sq = 0.f;
#pragma unroll
  for (int q = 0; q < WAVES; ++q) {
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] += red[q][t + TPW * mte][lane][r];
    if (p.rms) {
#pragma unroll
      for (int g = 0; g < 4; ++g) sq += rsq[q][mte][col + 16 * g];  // all k-slot groups of row tm
    }
  }
  if (tm >= p.M) return;
  const int n = nf;
  if (p.part) {
    // split-K: this K range's sums; gemv_splitk_epilogue finishes the rows
    *reinterpret_cast<f32x4*>(p.part + (static_cast<int64_t>(split) * p.M + tm) * p.N + n) =
        f32x4{v[0], v[1], v[2], v[3]};
    if (s == 0 && blockIdx.x == 0 && t == 0) p.part_ssq[split * p.M + tm] = sq;
    return;
  }
  const float scale = p.rms ? rsqrtf(sq / static_cast<float>(p.K) + p.eps) : 1.f;
  float bias[4] = {0.f, 0.f, 0.f, 0.f};
  if (EPI == kGemvRopeKV) {
#pragma unroll
    for (int r = 0; r < 4; ++r) bias[r] = bf16_bits_to_f32(pre.bias[r]);
  } else if (p.bias) {
#pragma unroll
    for (int r = 0; r < 4; ++r) bias[r] = bf16_bits_to_f32(static_cast<const uint16_t*>(p.bias)[nf + r]);
  }
  if constexpr (EPI == kGemvRopeKV) {
    // token row tm; the 4 rows n..n+3 lie in one head (d % 16 == 0).  q/k
    // heads are stored in rotary-pair order [0, d/2, 1, d/2 + 1, ...], so rows
    // (n, n+1) and (n+2, n+3) are the pairs (i, i + d/2) of i = j/2, j/2 + 1.
    const RopeParams& rp = p.rope;
    const int pos = pre.pos;
    const int b = pre.batch;
    const bool ok = pos >= 0 && pos < rp.Lmax && b >= 0 && b < rp.B;
    const int hh = n / rp.d, j = n - hh * rp.d;
    float o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float tt = v[r] * scale;
      if (p.bias) tt += bias[r];
      o[r] = bf16_bits_to_f32(f32_to_bf16_bits(tt));  // the projection output, rounded as stored
    }
    if (hh < rp.n_q + rp.n_k) {
      const int half = rp.d / 2;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int i = j / 2 + q;
        float cs = pre.rot[2 * q], sn = pre.rot[2 * q + 1];
        if (!rp.table) rope_cos_sin(pos, i, rp.d, rp.theta, cs, sn);
        const float x1 = o[2 * q], x2 = o[2 * q + 1];
        const float y1 = x1 * cs - x2 * sn;
        const float y2 = x2 * cs + x1 * sn;
        if (hh < rp.n_q) {
          uint16_t* qo = static_cast<uint16_t*>(rp.q_out) + static_cast<int64_t>(tm) * rp.q_sn +
                         static_cast<int64_t>(hh) * rp.q_sh;
          qo[i] = f32_to_bf16_bits(ok ? y1 : __builtin_nanf(""));
          qo[i + half] = f32_to_bf16_bits(ok ? y2 : __builtin_nanf(""));
        } else if (ok) {
          uint16_t* ko = static_cast<uint16_t*>(rp.k_cache) + b * rp.k_sb +
                         static_cast<int64_t>(hh - rp.n_q) * rp.k_sh + static_cast<int64_t>(pos) * rp.k_sl;
          ko[i] = f32_to_bf16_bits(y1);
          ko[i + half] = f32_to_bf16_bits(y2);
        }
      }
    } else if (ok) {
      uint16_t* vo = static_cast<uint16_t*>(rp.v_cache) + b * rp.v_sb +
                     static_cast<int64_t>(hh - rp.n_q - rp.n_k) * rp.v_sh + static_cast<int64_t>(pos) * rp.v_sl;
#pragma unroll
      for (int r = 0; r < 4; ++r) vo[j + r] = f32_to_bf16_bits(o[r]);
    }
    return;
  }
  uint16_t* y = static_cast<uint16_t*>(p.y) + static_cast<int64_t>(tm) * p.y_ld;
  if constexpr (EPI == SAGA_GEMV_SILU_PAIRS) {
    // rows (n, n+1) and (n+2, n+3) are (gate, up) pairs -> outputs n/2, n/2 + 1
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float g = v[2 * q] * scale, u = v[2 * q + 1] * scale;
      y[n / 2 + q] = f32_to_bf16_bits(g / (1.0f + expf(-g)) * u);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float o = v[r] * scale;
      if (p.bias) o += bias[r];
      if constexpr (EPI == SAGA_GEMV_ADD) o += bf16_bits_to_f32(pre.y[r]);
      y[n + r] = f32_to_bf16_bits(o);
    }
  }
}

// Split-K finish, one thread per output pair (n, n+1) of a token row m: the
// sums over the K ranges of the partial sums (and of the partial sums of
// squares for the RMS scale), then the epilogue of gemv_kernel.  64-thread
// blocks spread the few thousand threads over many CUs; every partial of a
// thread is loaded in one burst.
template <int EPI>
__global__ void __launch_bounds__(64) gemv_splitk_epilogue(GemvParams p) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
  const int np = p.N / 2;
  if (q >= static_cast<int64_t>(p.M) * np) return;
  const int m = static_cast<int>(q / np), n = 2 * static_cast<int>(q - static_cast<int64_t>(m) * np);
  uint16_t* y = static_cast<uint16_t*>(p.y) + static_cast<int64_t>(m) * p.y_ld;
  // bias and residual issued with the first partials (one round trip)
  const uint16_t* bp = p.bias ? static_cast<const uint16_t*>(p.bias) + n : y + n;
  const uint16_t b0 = bp[0], b1 = bp[1];
  uint16_t r0 = 0, r1 = 0;
  if constexpr (EPI == SAGA_GEMV_ADD) {
    r0 = y[n];
    r1 = y[n + 1];
  }
  float v0 = 0.f, v1 = 0.f, sq = 0.f;
  for (int s0 = 0; s0 < p.splits; s0 += kSplitBatch) {
    f32x2 a[kSplitBatch];
    float b[kSplitBatch];
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u) {
      const int s = s0 + u;
      a[u] = s < p.splits ? *reinterpret_cast<const f32x2*>(p.part + (static_cast<int64_t>(s) * p.M + m) * p.N + n)
                          : f32x2{0.f, 0.f};
      b[u] = (p.rms && s < p.splits) ? p.part_ssq[s * p.M + m] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u) {
      v0 += a[u].x;
      v1 += a[u].y;
      sq += b[u];
    }
  }
  const float scale = p.rms ? rsqrtf(sq / static_cast<float>(p.K) + p.eps) : 1.f;
  if constexpr (EPI == SAGA_GEMV_SILU_PAIRS) {
    // rows (n, n+1) are a (gate, up) pair -> output n/2
    const float g = v0 * scale, u = v1 * scale;
    y[n / 2] = f32_to_bf16_bits(g / (1.0f + expf(-g)) * u);
  } else {
    float o0 = v0 * scale, o1 = v1 * scale;
    if (p.bias) {
      o0 += bf16_bits_to_f32(b0);
      o1 += bf16_bits_to_f32(b1);
    }
    if constexpr (EPI == SAGA_GEMV_ADD) {
      o0 += bf16_bits_to_f32(r0);
      o1 += bf16_bits_to_f32(r1);
    }
    y[n] = f32_to_bf16_bits(o0);
    y[n + 1] = f32_to_bf16_bits(o1);
  }
}

template <int EPI>
static hipError_t launch_gemv_epi(const GemvParams& p, hipStream_t st) {
  if (p.w_packed == 2) {
    // 8-row tiles: 16 waves for long rows (the MLP down projection: 140 k steps
    // of 64, 9 per wave), else 4; the burst sized to the wave's share
    const unsigned tiles8 = static_cast<unsigned>(p.N / 8);
    const int steps = p.K / 64;
    if (steps >= 64) {
      if ((steps + 15) / 16 <= 9)
        hipLaunchKernelGGL((gemv_kernel<16, EPI, 1, true, 9>), dim3(tiles8, 1), dim3(1024), 0, st, p);
      else
        hipLaunchKernelGGL((gemv_kernel<16, EPI, 1, true, 12>), dim3(tiles8, 1), dim3(1024), 0, st, p);
    } else if ((steps + 3) / 4 <= 6) {
      hipLaunchKernelGGL((gemv_kernel<4, EPI, 1, true, 6>), dim3(tiles8, 1), dim3(256), 0, st, p);
    } else {
      hipLaunchKernelGGL((gemv_kernel<4, EPI, 1, true, 12>), dim3(tiles8, 1), dim3(256), 0, st, p);
    }
    return hipGetLastError();
  }
  const unsigned tiles = static_cast<unsigned>(p.N / 16);
  if (p.M > 16) {
    // 17-32 token rows: two token tiles per W fragment, 6 k steps per burst
    // (12 registers of fragments per step), 8 waves per workgroup so that a
    // K = 1536 row or a split-K range is one burst
    if (p.part) {
      hipLaunchKernelGGL((gemv_kernel<8, EPI, 1, false, 6, 2>), dim3(tiles, p.splits), dim3(512), 0, st, p);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      const int64_t pairs = static_cast<int64_t>(p.M) * (p.N / 2);
      hipLaunchKernelGGL((gemv_splitk_epilogue<EPI>), dim3(static_cast<unsigned>((pairs + 63) / 64)), dim3(64), 0,
                         st, p);
    } else if (p.K >= 4096) {
      hipLaunchKernelGGL((gemv_kernel<16, EPI, 1, false, 6, 2>), dim3(tiles, 1), dim3(1024), 0, st, p);
    } else {
      hipLaunchKernelGGL((gemv_kernel<8, EPI, 1, false, 6, 2>), dim3(tiles, 1), dim3(512), 0, st, p);
    }
    return hipGetLastError();
  }
  if (p.part) {
    hipLaunchKernelGGL((gemv_kernel<4, EPI, 1>), dim3(tiles, p.splits), dim3(256), 0, st, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t pairs = static_cast<int64_t>(p.M) * (p.N / 2);
    hipLaunchKernelGGL((gemv_splitk_epilogue<EPI>), dim3(static_cast<unsigned>((pairs + 63) / 64)), dim3(64), 0, st,
                       p);
  } else if (p.K >= 4096) {
    // long rows of W: more waves per workgroup split K
    hipLaunchKernelGGL((gemv_kernel<16, EPI, 1>), dim3(tiles, 1), dim3(1024), 0, st, p);
  } else if (gemv_tiles_per_wave(p.N, p.K) == 2) {
    hipLaunchKernelGGL((gemv_kernel<4, EPI, 2>), dim3(tiles / 2, 1), dim3(256), 0, st, p);
  } else {
    hipLaunchKernelGGL((gemv_kernel<4, EPI, 1>), dim3(tiles, 1), dim3(256), 0, st, p);
  }
  return hipGetLastError();
}

// Two tiles per wave (24 KB of W in flight per wave, 3 waves per SIMD) for
// weights of many tiles (the LM head: 9.3 rounds of 4096 one-tile waves),
// one tile (12 KB, 4 waves per SIMD) otherwise: measured on MI355X, two tiles
// lose below about two rounds (the gate/up projection, 1.1 rounds).
int gemv_tiles_per_wave(int64_t N, int64_t K) {
  if (N % 32 != 0 || K >= 4096) return 1;
  return (N / 16) * 4 > 2 * 4096 ? 2 : 1;
}

int gemv_splits(int64_t N, int64_t K) {
  const int64_t tiles = N / 16, steps = K / 32;
  int64_t s = (512 + tiles - 1) / tiles;       // about 512 workgroups
  s = std::min<int64_t>(s, steps / (4 * 8));   // >= 8 k steps per wave
  return static_cast<int>(std::max<int64_t>(s, 1));
}

hipError_t launch_gemv(const GemvParams& p, hipStream_t st) {
  switch (p.epilogue) {
    case SAGA_GEMV_ADD: return launch_gemv_epi<SAGA_GEMV_ADD>(p, st);
    case SAGA_GEMV_SILU_PAIRS: return launch_gemv_epi<SAGA_GEMV_SILU_PAIRS>(p, st);
    case kGemvRopeKV: return launch_gemv_epi<kGemvRopeKV>(p, st);
    default: return launch_gemv_epi<SAGA_GEMV_STORE>(p, st);
  }
}

// Row-wise argmax (first index of the maximum), one block per row; rows are
// read 8 bf16 per lane (16-byte loads), four loads in flight per lane.
__device__ __forceinline__ void argmax_take(float v, int i, float& best, int& idx) {
  if (v > best || (v == best && i < idx)) {
    best = v;
    idx = i;
  }
}

__global__ void __launch_bounds__(1024) argmax_kernel(const uint16_t* x, int64_t ld, int N, int64_t* out) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint16_t* row = x + static_cast<int64_t>(r) * ld;
  float best = kNegInf;
  int idx = 0x7fffffff;
  const bool vec = (reinterpret_cast<uintptr_t>(row) % 16) == 0;
  const int nv = vec ? N / 8 : 0;  // full 8-element groups
  for (int g0 = tid; g0 < nv; g0 += 4 * 1024) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int g = g0 + u * 1024;
      v[u] = g < nv ? ld16(row + 8 * static_cast<int64_t>(g)) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int g = g0 + u * 1024;
      if (g < nv) {
        float f[8];
        unpack16<SAGA_DTYPE_BF16>(v[u], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) argmax_take(f[e], 8 * g + e, best, idx);
      }
    }
  }
  for (int i = 8 * nv + tid; i < N; i += 1024) argmax_take(bf16_bits_to_f32(row[i]), i, best, idx);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) argmax_take(__shfl_xor(best, o), __shfl_xor(idx, o), best, idx);
  if (lane == 0) {
    bv[w] = best;
    bi[w] = idx;
  }
  __syncthreads();
  if (tid == 0) {
    for (int q = 1; q < 16; ++q) argmax_take(bv[q], bi[q], best, idx);
    out[r] = idx == 0x7fffffff ? 0 : idx;
  }
}

// Two-pass argmax over long rows (the LM head's vocabulary): pass 1 reduces
// chunks of kArgmaxChunk elements, one 256-thread block each (every load of
// a row in flight at once over many CUs), into (value, index) partials;
// pass 2 reduces a row's partials in one wave.  Ties keep the lowest index.
constexpr int kArgmaxChunk = 256 * 16;

__global__ void __launch_bounds__(256) argmax_chunk_kernel(const uint16_t* x, int64_t ld, int N, float* pval,
                                                           int* pidx, int nchunk) {
  __shared__ float bv[4];
  __shared__ int bi[4];
  const int r = blockIdx.y, c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint16_t* row = x + static_cast<int64_t>(r) * ld;
  const int e0 = c * kArgmaxChunk + tid * 8;
  u32x4 v[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int e = e0 + u * 256 * 8;
    v[u] = e + 8 <= N ? ld16(row + e) : u32x4{0u, 0u, 0u, 0u};
  }
  float best = kNegInf;
  int idx = 0x7fffffff;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int e = e0 + u * 256 * 8;
    if (e + 8 <= N) {
      float f[8];
      unpack16<SAGA_DTYPE_BF16>(v[u], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) argmax_take(f[i], e + i, best, idx);
    } else {
      for (int i = e; i < N && i < e + 8; ++i) argmax_take(bf16_bits_to_f32(row[i]), i, best, idx);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) argmax_take(__shfl_xor(best, o), __shfl_xor(idx, o), best, idx);
  if (lane == 0) {
    bv[w] = best;
    bi[w] = idx;
  }
  __syncthreads();
  if (tid == 0) {
    for (int q = 1; q < 4; ++q) argmax_take(bv[q], bi[q], best, idx);
    pval[r * nchunk + c] = best;
    pidx[r * nchunk + c] = idx;
  }
}

__global__ void __launch_bounds__(64) argmax_final_kernel(const float* pval, const int* pidx, int nchunk,
                                                          int64_t* out) {
  const int r = blockIdx.x, lane = threadIdx.x;
  float best = kNegInf;
  int idx = 0x7fffffff;
  for (int c = lane; c < nchunk; c += 64) argmax_take(pval[r * nchunk + c], pidx[r * nchunk + c], best, idx);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) argmax_take(__shfl_xor(best, o), __shfl_xor(idx, o), best, idx);
  if (lane == 0) out[r] = idx == 0x7fffffff ? 0 : idx;
}

int64_t argmax_workspace_bytes(int64_t rows, int64_t N) {
  const int64_t nchunk = (N + kArgmaxChunk - 1) / kArgmaxChunk;
  return nchunk > 1 ? rows * nchunk * 8 : 0;
}

hipError_t launch_argmax(const void* x, int64_t ld, int rows, int N, int64_t* out, void* ws, hipStream_t st) {
  const int nchunk = (N + kArgmaxChunk - 1) / kArgmaxChunk;
  const bool vec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && ld % 8 == 0;
  if (ws && vec && nchunk > 1 && nchunk <= 65535) {
    float* pval = static_cast<float*>(ws);
    int* pidx = reinterpret_cast<int*>(pval + static_cast<int64_t>(rows) * nchunk);
    hipLaunchKernelGGL(argmax_chunk_kernel, dim3(nchunk, rows), dim3(256), 0, st, static_cast<const uint16_t*>(x), ld,
                       N, pval, pidx, nchunk);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, st, pval, pidx, nchunk, out);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(1024), 0, st, static_cast<const uint16_t*>(x), ld, N, out);
  return hipGetLastError();
}

}  // namespace saga

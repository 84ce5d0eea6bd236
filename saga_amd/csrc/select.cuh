// Block-level selection helpers shared by the calibration kernels: the
// histogram pick, the radix select over order-preserving float keys, the
// distance-bin scale and a four-per-thread block scan.  NT is the block's
// thread count (256, 512 or 1024); every thread of the block calls them.
#pragma once

#include "block_pv.cuh"

namespace saga {

constexpr int kNearBins = 2048;      // bins of the distance below the row max
constexpr float kNearScale = 32.0f;  // default bins per unit of logit: the bins span M - 64 .. M

__device__ __forceinline__ unsigned long long lanes_below(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (kWave - lane));
}

// Bin holding the krem-th largest element of sh.hist[0..nb) (bin nb - 1 holds
// the largest, nb <= 2048), the count in the bins above it and the bin's own
// count (read before the last barrier, so a caller may overwrite sh.hist
// right after); bin -1 (count 0) if fewer than krem elements are counted.
// Uses sh.cnt[NT / 64], sh.sel_bin, sh.sel_above, sh.sel_cnt.
template <int NT = kBlkThreads, class SH>
__device__ __forceinline__ void hist_pick(SH& sh, int nb, int krem, int& bin, int& above, int& count) {
  constexpr int BPT = 2048 / NT;  // bins per thread, scanned from the top
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (tid == 0) sh.sel_bin = -1;
  const int b0 = nb - 1 - BPT * tid;  // thread t owns bins b0, b0 - 1, .., b0 - BPT + 1
  int c[BPT];
  int tsum = 0;
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    c[i] = b0 - i >= 0 ? sh.hist[b0 - i] : 0;
    tsum += c[i];
  }
  const int incl = wave_incl_scan(tsum, lane);
  if (lane == kWave - 1) sh.cnt[w] = incl;
  lds_sync();
  int ex = incl - tsum;
#pragma unroll
  for (int i = 0; i < NT / kWave; ++i)  // (all reads in flight together)
    if (i < w) ex += sh.cnt[i];
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    if (c[i] > 0 && ex < krem && krem <= ex + c[i]) {
      sh.sel_bin = b0 - i;
      sh.sel_above = ex;
      sh.sel_cnt = c[i];
    }
    ex += c[i];
  }
  lds_sync();
  bin = sh.sel_bin;
  above = sh.sel_above;
  count = bin >= 0 ? sh.sel_cnt : 0;
  lds_sync();
}

// The krem-th largest of a set of keys, by a 3-pass radix select (11/11/10
// bits of the order-preserving uint32 key) over 2048-bin LDS histograms;
// each(f) calls f(x) for every element of the set (in the calling thread's
// share); krem is left at the count of elements equal to it that are among
// the krem largest.
template <int NT = kBlkThreads, class SH, class EACH>
__device__ __forceinline__ uint32_t radix_select_each(SH& sh, int& krem, EACH each) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0;
  const int shifts[3] = {21, 10, 0};
  const int nbits[3] = {11, 11, 10};
#pragma unroll
  for (int pass = 0; pass < 3; ++pass) {
    const int nb = 1 << nbits[pass];
    const uint32_t hmask = pass == 0 ? 0u : (0xffffffffu << (shifts[pass] + nbits[pass]));
    for (int i = tid; i < 2048; i += NT) sh.hist[i] = 0;
    lds_sync();
    each([&](float xi) {
      const uint32_t key = f32_to_key(xi);
      if ((key & hmask) == prefix) atomicAdd(&sh.hist[(key >> shifts[pass]) & (nb - 1)], 1);
    });
    lds_sync();
    int bin, above, count;
    hist_pick<NT>(sh, nb, krem, bin, above, count);
    prefix |= static_cast<uint32_t>(bin) << shifts[pass];
    krem -= above;
  }
  return prefix;
}

// Exclusive scan over the block of four values per thread (thread t's four
// are entries 4t..4t+3 of the sequence); returns thread t's exclusive base.
template <int NW = kBlkWaves>
__device__ __forceinline__ int block_excl_scan4(int tsum, int* wscan) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int incl = wave_incl_scan(tsum, lane);
  if (lane == kWave - 1) wscan[w] = incl;
  lds_sync();
  int base = incl - tsum;
#pragma unroll
  for (int u = 0; u < NW; ++u)
    if (u < w) base += wscan[u];
  return base;
}

// Scale s of the distance bins (M - x) * s: the largest power of two (at
// most 2^40) with (M - mn) * s <= 2047 for the smallest finite value mn, so
// that every finite value has a bin whatever the spread; a power of two
// keeps M * s exact, so the max sits at distance 0.
__device__ __forceinline__ float near_bin_scale(float M, float mn) {
  float scale = kNearScale;
  const float range = M - mn;
  if (range > 0.f && range < INFINITY) {
    int ex;
    frexpf(fminf(static_cast<float>(kNearBins - 1) / range, 1e30f), &ex);  // in [2^(ex-1), 2^ex)
    scale = ldexpf(1.f, min(max(ex - 1, -100), 40));
  }
  return scale;
}

}  // namespace saga

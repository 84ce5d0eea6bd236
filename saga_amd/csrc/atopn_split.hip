// K2 of the Atop-N fast step: slice kernel + row kernel, or, for rows of
// few slices, one block per row (atopn_rowlds_kernel / atopn_rowblock_kernel
// below); the choice is by shape (k2_row_block) and the results are identical.
//
// Replaces the threshold transform (attention/attention.py:136-149), the
// Triton stream compaction threshold_select_fast_kernel
// (attention/triton_atopn.py:6-53) and _atopn_gather_and_output
// (attention/attention.py:152-170) of approx_top_n_attention_amortized
// (:192-209).
//
// Slice waves (atopn_slice_kernel), one wave per (row, kSliceLen positions),
// four independent waves per block, no block barrier:
//   1. loads of the K1 block partials (max, sum of exp, tail-window max) and
//      of the slice's scores are issued together; t = m + log(max(p*, 1e-30)
//      * sum_j exp(x_j - m)) from the partials with DPP wave reductions
//      (every wave of a row runs the same reduction in the same order, so all
//      of them hold the bit-identical t);
//   2. ordered compaction of {x > t} (strict, triton_atopn.py:42): 64-bit
//      ballots and mbcnt put every passing element at its rank in ascending
//      position order; the slice's list and count go to the workspace;
//   3. a list of at most kSliceSmall entries (the usual case) is gathered by
//      the wave itself, 48 V rows per burst (a second burst only for the
//      slices of a peaked head): its (m, l, o) softmax . V partial.
// Row blocks (atopn_gather_kernel), one block per row (256 threads when buf_k
// <= 1024, else 1024): a block scan
// of the slice counts ranks the slices; exactly the first n = min(total,
// buf_k) passing positions in ascending order count (the reference keeps a
// race-dependent subset when more than buf_k pass).  Short slices wholly
// among them contribute their partials (log-sum-exp merge); the entries of
// long slices and of the slice cut at rank buf_k are gathered here, 256 V
// rows per burst.  So no wave carries a long gather chain: balanced rows stay
// one gather burst deep, skewed or overflowing rows cost at most buf_k
// block-parallel gathers.  The kernel boundary orders the slice writes before
// the row reads (no device-scope fences or counters).
#include "block_pv.cuh"
#include "kernels.h"

namespace saga {

constexpr int kSliceThreads = 256;                    // 4 independent slice waves per block
constexpr int kSliceWaves = kSliceThreads / kWave;    // 4
constexpr int kSliceLoads = kSliceLen / (4 * kWave);  // f32x4 loads per lane: 4
constexpr int kSlicePrefetch = 8;                     // partials per lane in the first burst
// row kernel block: 256 threads when at most 1024 positions count per row
// (buf_k <= 1024: the partial merge dominates, a small block launches and
// synchronises faster), 1024 threads for longer lists (block-wide gathers)
constexpr int kRowThreadsSmall = 256;
constexpr int kRowThreadsLarge = 1024;
constexpr int kRowSmallCap = 1024;
constexpr int kRowBatch = 2048;                       // list entries per LDS batch
constexpr int kRowMaxSlices = 2048;                   // slice ranks kept in LDS
constexpr int kRowUnroll = 16;                        // V rows in flight per lane group
constexpr int kWaveUnroll = 12;                       // slice wave: 4 groups x 12 = 48 V rows in flight
constexpr int kRowMergeSlices = 8;                    // slice partials per merge thread in one burst
// A row kernel of at most kRowSplitThreads threads (unsplit) splits the
// gathers of rows with more than split_min entries over its kRowSplit blocks
// per row (one CU draws ~28 GB/s of V rows: an overflowing row's 1024 kept
// rows took 9 us in one block).  With more rows the blocks already spread
// over the chip and the split blocks' release fences cost more than the split
// gains (b32 16k N 256: 74.5 against 62.3 us; b8 16k N 1024 on 1024-thread
// blocks: 50.3 against 44.6); with few, split (b8 32k N 512: 44.5 against
// 50.0; b4 128k N 1024: 63.7 against 68.0).  split_min: 384 for kernels of at
// most kRowSplitSmallThreads threads (b1 16k N 256: 23.9 against 24.8 us),
// else 768 (b8 16k N 256, lists of <= 512: 34.6 against 35.1 us).
constexpr int64_t kRowSplitThreads = 65536;
constexpr int64_t kRowSplitSmallThreads = 16384;
// auto mode: one block per row when a row has at most this many slices and
// its list fits one LDS batch (measured on MI355X, attention call at b1-b32,
// d 64 and 128: 1.02-1.48x at 4k-12k positions; from 16k positions a row's
// scores and V rows are too much for one CU and the spread slice waves win:
// 0.84-0.99x)
constexpr int kRowBlockAutoSlices = 12;

static_assert(kSliceLen == kSliceLoads * 4 * kWave, "slice = whole f32x4 loads of every lane");
static_assert(kSliceSmall % (4 * kWaveUnroll) == 0 && kSliceSmall <= 2 * kWave,
              "a short slice list is whole gather bursts of its wave, at most two entries per lane");

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One wave's softmax . V over n <= kSliceSmall entries, in bursts of 48 V
// rows (one for the usual short list, two for a peaked head's): 4 lane
// groups of 16 lanes, lane c of group G owns dims [c*DPL, c*DPL + DPL) and
// loads the rows G, G+4, ...; weights are relative to the list's max m.
// The bursts reuse the same registers (a second burst costs a round trip,
// not occupancy: 7 waves per SIMD at d128).  Writes o (unnormalised, D floats) and returns (m, l) in
// every lane.
template <int DT, int D>
__device__ void wave_pv_small(int n, const int* sidx, const float* sval, const char* vbase, int64_t vrow,
                              float* scratch, float* o, float& m, float& l) {
  using PV = BlockPV<DT, D>;
  constexpr int DPL = D / 16;
  constexpr int BURST = 4 * kWaveUnroll;
  const int lane = threadIdx.x & 63, G = lane >> 4, c = lane & 15;
  const float x0 = lane < n ? sval[lane] : kNegInf;
  const float x1 = lane + kWave < n ? sval[lane + kWave] : kNegInf;
  m = wave_max(fmaxf(x0, x1));
  l = wave_sum((lane < n ? __expf(x0 - m) : 0.f) + (lane + kWave < n ? __expf(x1 - m) : 0.f));
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
  const char* vb = vbase + static_cast<int64_t>(c) * PV::BYTES;
  auto burst = [&](int e0) {
    // the burst's positions first (LDS reads issued back to back and waited
    // for once), then every gather: each load would otherwise wait for its
    // own LDS read
    int id[kWaveUnroll];
#pragma unroll
    for (int u = 0; u < kWaveUnroll; ++u) {
      const int e = e0 + G + 4 * u;
      id[u] = sidx[min(e, kSliceSmall - 1)];
    }
    u32x4 raw[kWaveUnroll][PV::NV];
#pragma unroll
    for (int u = 0; u < kWaveUnroll; ++u) {
      const int e = e0 + G + 4 * u;
      if (e < n) PV::load_raw(vb + static_cast<int64_t>(id[u]) * vrow, raw[u]);
    }
    // the entries' logits, read while the rows are in flight
    float xs[kWaveUnroll];
#pragma unroll
    for (int u = 0; u < kWaveUnroll; ++u) xs[u] = sval[min(e0 + G + 4 * u, kSliceSmall - 1)];
    __builtin_amdgcn_sched_barrier(0);  // all gathers of the burst in flight before the FMAs
#pragma unroll
    for (int u = 0; u < kWaveUnroll; ++u) {
      const int e = e0 + G + 4 * u;
      if (e < n) {
        const float w = __expf(xs[u] - m);
        float f[DPL];
        PV::unpack(raw[u], f);
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] += w * f[i];
      }
    }
  };
  burst(0);
  if (n > BURST) burst(BURST);  // wave-uniform
  // the 4 groups summed through the wave's LDS scratch (>= 4 * D floats)
  wave_lds_sync();
#pragma unroll
  for (int i = 0; i < DPL; ++i) scratch[G * D + c * DPL + i] = acc[i];
  wave_lds_sync();
  for (int i = lane; i < D; i += kWave) o[i] = (scratch[i] + scratch[D + i]) + (scratch[2 * D + i] + scratch[3 * D + i]);
}

struct SliceWaveShared {
  int sidx[kSliceSmall];
  float sval[kSliceSmall];
  float scratch[4 * 128];
};

// The K1 block partials of row r held by one wave (kSlicePrefetch per lane:
// 512 parts, b >= 2 at 128k positions, in the first burst; longer rows read
// the rest in row_threshold, one more round trip).
struct RowPartials {
  float pm[kSlicePrefetch], ps[kSlicePrefetch], pt[kSlicePrefetch];
  float pstar;
};

__device__ __forceinline__ void load_row_partials(const FusedSelParams& p, int r, int lane, RowPartials& rp) {
  const float* prow_m = p.pmax + static_cast<int64_t>(r) * p.nparts;
  const float* prow_s = p.psum + static_cast<int64_t>(r) * p.nparts;
  const float* prow_t = p.ptail + static_cast<int64_t>(r) * p.nparts;
  // unconditional loads (index clamped into the row, nparts >= 1), selected
  // after they return: a load under a branch is waited for at the branch's
  // join, which would hold back every later load of the wave (the scores)
  // by one round trip
#pragma unroll
  for (int k = 0; k < kSlicePrefetch; ++k) {
    const int c = lane + k * kWave;
    const int cc = min(c, p.nparts - 1);
    const float vm = prow_m[cc], vs = prow_s[cc], vt = prow_t[cc];
    rp.pm[k] = c < p.nparts ? vm : kNegInf;
    rp.ps[k] = c < p.nparts ? vs : 0.f;
    rp.pt[k] = c < p.nparts ? vt : kNegInf;
  }
  rp.pstar = p.pstar[r];
}

// t = m + log(max(p*, 1e-30) * sum_j exp(x_j - m)) from the partials
// (attention/attention.py:142-147: m = max of the last min(256, L) logits);
// every wave of a row runs the same reductions in the same order, so all of
// them hold the bit-identical t.
__device__ __forceinline__ float row_threshold(const FusedSelParams& p, int r, int lane, const RowPartials& rp) {
  const float* prow_m = p.pmax + static_cast<int64_t>(r) * p.nparts;
  const float* prow_s = p.psum + static_cast<int64_t>(r) * p.nparts;
  const float* prow_t = p.ptail + static_cast<int64_t>(r) * p.nparts;
  float tl = kNegInf;
#pragma unroll
  for (int k = 0; k < kSlicePrefetch; ++k) tl = fmaxf(tl, rp.pt[k]);
  for (int c = lane + kSlicePrefetch * kWave; c < p.nparts; c += kWave) tl = fmaxf(tl, prow_t[c]);
  const float mt = wave_max(tl);
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < kSlicePrefetch; ++k)
    if (rp.pm[k] != kNegInf) acc += rp.ps[k] * __expf(rp.pm[k] - mt);
  for (int c = lane + kSlicePrefetch * kWave; c < p.nparts; c += kWave) {
    const float m2 = prow_m[c];
    if (m2 != kNegInf) acc += prow_s[c] * __expf(m2 - mt);
  }
  const float ssum = wave_sum(acc);
  return mt + logf(fmaxf(rp.pstar, 1e-30f) * ssum);
}

// The scores of slice sl of row r: element (k, lane, j) is position
// sl * kSliceLen + 4*(k*64 + lane) + j (-inf past the row).
__device__ __forceinline__ void load_slice_scores(const FusedSelParams& p, int r, int sl, int lane,
                                                  f32x4 (&xv)[kSliceLoads]) {
  const float* x = p.scores + static_cast<int64_t>(r) * p.ld;
  const int s0 = sl * kSliceLen;
#pragma unroll
  for (int k = 0; k < kSliceLoads; ++k) {
    const int64_t e = s0 + 4 * (k * kWave + lane);
    xv[k] = e < p.ld ? *reinterpret_cast<const f32x4*>(x + e) : f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
  }
}

// Number of {x > t} in a slice (the predicate of compact_slice).
__device__ __forceinline__ int count_slice(int s0, float t, int Leff, const f32x4 (&xv)[kSliceLoads], int lane) {
  int n = 0;
#pragma unroll
  for (int k = 0; k < kSliceLoads; ++k) {
    const int e = s0 + 4 * (k * kWave + lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) n += __popcll(__ballot(e + j < Leff && xv[k][j] > t));
  }
  return n;
}

// Where compact_slice writes the slice's workspace list: element by element
// (kListDirect), not at all (kListNone: the caller copies it from LDS), or
// element by element only when it does not fit the LDS list (kListIfLong;
// else the caller copies the LDS list with one coalesced store per lane).
enum ListStores { kListDirect, kListNone, kListIfLong };

// Ordered compaction of {x > t} over a slice into its workspace list (ranks
// past slice_cap = min(kSliceLen, buf_k) can never be among a row's first
// buf_k) and into sidx / sval (if given) at lds_off + rank, below lds_lim.
// Ballot j of load k holds flag j of every lane; a passing element's rank is
// the passing elements of earlier loads + those of lower lanes (mbcnt of the
// four ballots) + its own lower flags.  Returns the slice's count.
template <ListStores LS = kListDirect>
__device__ __forceinline__ int compact_slice(const FusedSelParams& p, int64_t gw, int s0, float t, int Leff,
                                             const f32x4 (&xv)[kSliceLoads], int lane, int* sidx, float* sval,
                                             int lds_off, int lds_lim) {
  unsigned long long bal[kSliceLoads][4];
  int n = 0;
  int base[kSliceLoads];
#pragma unroll
  for (int k = 0; k < kSliceLoads; ++k) {
    const int e = s0 + 4 * (k * kWave + lane);
    base[k] = n;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bal[k][j] = __ballot(e + j < Leff && xv[k][j] > t);
      n += __popcll(bal[k][j]);
    }
  }
  int32_t* gidx = p.sl_idx + gw * p.slice_cap;
  float* gval = p.sl_val + gw * p.slice_cap;
  const bool to_global = LS == kListDirect || (LS == kListIfLong && lds_off + n > lds_lim);
#pragma unroll
  for (int k = 0; k < kSliceLoads; ++k) {
    int pos = base[k];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = static_cast<uint32_t>(bal[k][j]), hi = static_cast<uint32_t>(bal[k][j] >> 32);
      pos += __builtin_amdgcn_mbcnt_hi(hi, __builtin_amdgcn_mbcnt_lo(lo, 0u));
    }
    const int e = s0 + 4 * (k * kWave + lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if ((bal[k][j] >> lane) & 1ull) {
        if (to_global && pos < p.slice_cap) {
          gidx[pos] = e + j;
          gval[pos] = xv[k][j];
        }
        if (sidx && lds_off + pos < lds_lim) {
          sidx[lds_off + pos] = e + j;
          sval[lds_off + pos] = xv[k][j];
        }
        ++pos;
      }
    }
  }
  return n;
}

// One slice wave: slice sl of row r (see the file comment), LDS scratch sh.
template <int DT, int D>
__device__ __forceinline__ void slice_wave(const FusedSelParams& p, const PVParams& v, int r, int sl,
                                           SliceWaveShared& sh) {
  const int lane = threadIdx.x & 63;
  const int64_t gw = static_cast<int64_t>(r) * p.nslice + sl;
  const int bi = r / p.q_h;
  // 1. the block partials and the slice's scores in flight together; nothing
  //    waits for kv_len, which only masks
  RowPartials rp;
  load_row_partials(p, r, lane, rp);
  f32x4 xv[kSliceLoads];
  load_slice_scores(p, r, sl, lane, xv);
  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  __builtin_amdgcn_sched_barrier(0);
  const float t = row_threshold(p, r, lane, rp);
  // 2. ordered compaction
  const int n = compact_slice<kListIfLong>(p, gw, sl * kSliceLen, t, Leff, xv, lane, sh.sidx, sh.sval, 0, kSliceSmall);
  if (lane == 0) {
    p.sl_cnt[gw] = n;
    if (sl == 0 && p.t_out) p.t_out[r] = t;
    if (sl == 0) p.row_cnt[r] = 0;  // the row kernel's split count starts at zero
  }
  if (n > 0 && n <= kSliceSmall) {  // the list is in LDS: coalesced stores, one or two per lane
    wave_lds_sync();
    for (int i = lane; i < min(n, p.slice_cap); i += kWave) {
      p.sl_idx[gw * p.slice_cap + i] = sh.sidx[i];
      p.sl_val[gw * p.slice_cap + i] = sh.sval[i];
    }
  }
  // 3. a short list is gathered here (one burst, two for a peaked head):
  //    (m, l, o) partial of the slice (its count tells the row kernel that
  //    the partial exists)
  if (n > 0 && n <= kSliceSmall) {
    wave_lds_sync();
    const int h = r - bi * p.q_h;
    const int vh = h / (v.q_h / v.v_h);
    const char* vbase = v.v + (bi * v.v_sb + static_cast<int64_t>(vh) * v.v_sh) * Elt<DT>::kBytes;
    float m, l;
    wave_pv_small<DT, D>(n, sh.sidx, sh.sval, vbase, v.v_sl * Elt<DT>::kBytes, sh.scratch,
                         p.sl_o + gw * D, m, l);
    if (lane == 0) {
      p.sl_ml[2 * gw] = m;
      p.sl_ml[2 * gw + 1] = l;
    }
  }
}

template <int DT, int D>
__global__ void __launch_bounds__(kSliceThreads) atopn_slice_kernel(FusedSelParams p, PVParams v) {
  __shared__ SliceWaveShared shw[kSliceWaves];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t gw = static_cast<int64_t>(blockIdx.x) * kSliceWaves + w;
  if (gw >= static_cast<int64_t>(p.nrows) * p.nslice) return;
  const int r = static_cast<int>(gw / p.nslice), sl = static_cast<int>(gw - static_cast<int64_t>(r) * p.nslice);
  slice_wave<DT, D>(p, v, r, sl, shw[w]);
}

// The slice phase of a row block: wave w of nw handles slices w, w + nw, ...
// of row r.  The partials and the scores of up to kRowBlockBurst of its
// slices are in flight together; t is computed once; every slice is
// compacted into its workspace list (no short-list gathers: the block
// gathers every kept entry after its barrier).
constexpr int kRowBlockBurst = 4;
constexpr int kRowLdsMaxSlices = 64;  // slices of a row in the all-LDS row block

__device__ __forceinline__ void rowblock_slices(const FusedSelParams& p, int r, int w, int nw) {
  const int lane = threadIdx.x & 63;
  const int bi = r / p.q_h;
  RowPartials rp;
  load_row_partials(p, r, lane, rp);
  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  float t = 0.f;
  bool have_t = false;
  for (int g0 = w; g0 < p.nslice; g0 += nw * kRowBlockBurst) {
    f32x4 xv[kRowBlockBurst][kSliceLoads];
#pragma unroll
    for (int u = 0; u < kRowBlockBurst; ++u) {
      const int sl = g0 + nw * u;
      if (sl < p.nslice) {
        load_slice_scores(p, r, sl, lane, xv[u]);
      } else {
#pragma unroll
        for (int k = 0; k < kSliceLoads; ++k) xv[u][k] = f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (!have_t) {
      t = row_threshold(p, r, lane, rp);
      have_t = true;
      if (g0 == 0 && lane == 0 && p.t_out) p.t_out[r] = t;
    }
#pragma unroll
    for (int u = 0; u < kRowBlockBurst; ++u) {
      const int sl = g0 + nw * u;
      if (sl < p.nslice) {
        const int64_t gw = static_cast<int64_t>(r) * p.nslice + sl;
        const int n = compact_slice(p, gw, sl * kSliceLen, t, Leff, xv[u], lane, nullptr, nullptr, 0, 0);
        if (lane == 0) p.sl_cnt[gw] = n;
      }
    }
  }
}

// The slice holding list entry j of a row (pre[s] <= j < pre[s+1]).
__device__ __forceinline__ int slice_of(const int* pre, int nslice, int j) {
  int lo = 0, hi = nslice - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (pre[mid] <= j) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Exclusive block scans of a(s) and b(s) over s in [0, ns) into pa / pb
// [0..ns] (pa[ns], pb[ns] = totals; pa may be null); returns the totals.
template <int NT, class FA, class FB>
__device__ int2 block_scan_slices(int ns, int* pa, int* pb, int2* wsum, FA fa, FB fb) {
  constexpr int NW = NT / kWave;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int ra = 0, rb = 0;
  for (int c0 = 0; c0 < ns; c0 += NT) {
    const int s = c0 + tid;
    const int xa = s < ns ? fa(s) : 0;
    const int xb = s < ns ? fb(s) : 0;
    const int ia = wave_incl_scan(xa, lane), ib = wave_incl_scan(xb, lane);
    if (lane == kWave - 1) wsum[w] = int2{ia, ib};
    __syncthreads();
    int ba = ra, bb = rb, ta = 0, tb = 0;
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      const int2 v = wsum[q];
      if (q < w) {
        ba += v.x;
        bb += v.y;
      }
      ta += v.x;
      tb += v.y;
    }
    if (s < ns) {
      if (pa) pa[s] = ba + ia - xa;
      pb[s] = bb + ib - xb;
    }
    ra += ta;
    rb += tb;
    __syncthreads();
  }
  if (tid == 0) {
    if (pa) pa[ns] = ra;
    pb[ns] = rb;
  }
  __threadfence_block();
  __syncthreads();
  return int2{ra, rb};
}

// LDS of one row merge (NT threads).
template <int NT>
struct RowShared {
  f32x4 accs[NT];
  float red[NT / kWave];
  int2 wsum[NT / kWave];
  int spre[kRowMaxSlices + 1];
  int sgpre[kRowMaxSlices + 1];
  int sidx[kRowBatch];
  float sval[kRowBatch];
  int last;  // this block merges the row's split partials
};

// The row merge of row r by the NT threads of a block (see the file comment).
// ALL_GATHER: the slices carry no partials; every kept entry is gathered here.
// LONG: rows of more than kRowMaxSlices slices, whose slice ranks live in the
// workspace instead of LDS (a host-side choice: with the address space known
// at compile time the ranks are LDS reads, not flat loads that wait on both
// the LDS and the memory counters at every use).
// piece / pieces: this block's share of the row (pieces blocks per row, the
// row kernel's grid y).  Every block ranks the row's slices; a row with more
// than p.split_min entries to gather splits them in contiguous rank ranges
// over the blocks (block 0 also merges the slice partials), each block writes
// its (m, l, o) partial, and the last block to finish -- counted with an
// agent-scope atomic after a release fence, no block waits for another --
// merges the partials in block order.  Other rows are merged by block 0 alone.
template <int DT, int D, int NT, bool ALL_GATHER = false, bool LONG = false>
__device__ __forceinline__ void row_merge(const FusedSelParams& p, const PVParams& v, int r, RowShared<NT>& sh,
                                          int piece = 0, int pieces = 1) {
  constexpr int NW = NT / kWave;
  float* red = sh.red;
  int2* wsum = sh.wsum;
  int* spre = sh.spre;
  int* sgpre = sh.sgpre;
  int* sidx = sh.sidx;
  float* sval = sh.sval;
  f32x4* accs = sh.accs;
  constexpr int C = D / 4;             // 16-byte chunks of an output row
  constexpr int G = NT / C;            // slice groups of the partial merge
  const int tid = threadIdx.x;
  const int c = tid % C, g = tid / C;
  const int ns = p.nslice;
  const int64_t row0 = static_cast<int64_t>(r) * ns;
  const int bi = r / p.q_h, h = r - bi * p.q_h;
  // the row's slice ranks: LDS, or the workspace for very long rows
  int* pre = LONG ? p.sl_pre + static_cast<int64_t>(r) * 2 * (ns + 1) : spre;
  int* gpre = LONG ? pre + (ns + 1) : sgpre;

  // 0. the first merge batch's slice partials, loaded before the counts
  //    (whether a slice's partial counts is known only after the scan; the
  //    loads of unused ones are discarded): counts and partials arrive in one
  //    round trip instead of two (16-bit V only: the f32 kernel has no
  //    registers to spare at 1024 threads)
  constexpr bool kPrefetch = DT != SAGA_DTYPE_F32 && !ALL_GATHER;
  float ms0[kRowMergeSlices], ls0[kRowMergeSlices];
  f32x4 ov0[kRowMergeSlices];
#pragma unroll
  for (int u = 0; u < kRowMergeSlices; ++u) {
    const int s = g + G * u;
    const bool in = kPrefetch && s < ns && piece == 0;
    ms0[u] = in ? p.sl_ml[2 * (row0 + s)] : kNegInf;
    ls0[u] = in ? p.sl_ml[2 * (row0 + s) + 1] : 0.f;
    ov0[u] = in ? *reinterpret_cast<const f32x4*>(p.sl_o + (row0 + s) * D + 4 * c) : f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // 1. ranks of the slices (pre) and of the entries gathered here (gpre); the
  //    first n = min(total, buf_k) passing positions count.  One pass when no
  //    more than buf_k pass (every slice is then taken whole); a second one
  //    re-ranks the gathers of an overflowing row.
  auto cnt_of = [&](int s) { return p.sl_cnt[row0 + s]; };
  auto whole_gather = [&](int s) {
    const int cnt = p.sl_cnt[row0 + s];
    return ALL_GATHER || cnt > kSliceSmall ? cnt : 0;
  };
  const int2 tot = block_scan_slices<NT>(ns, pre, gpre, wsum, cnt_of, whole_gather);
  const int total = tot.x;
  const int n = min(total, p.cap);
  // sel_cnt / sel_total are stored at the end: a global store here would make
  // every later block barrier wait for its acknowledgement
  // slice s contributes its first take(s) entries; a short slice contributing
  // all of them has its partial from the slice wave, the rest are gathered here
  auto take = [&](int s) { return max(0, min(n - pre[s], pre[s + 1] - pre[s])); };
  auto has_partial = [&](int s) {
    const int cnt = pre[s + 1] - pre[s];
    return !ALL_GATHER && cnt > 0 && cnt <= kSliceSmall && take(s) == cnt;
  };
  int ng = tot.y;
  if (total > p.cap) {
    ng = block_scan_slices<NT>(ns, static_cast<int*>(nullptr), gpre, wsum, cnt_of,
                           [&](int s) { return has_partial(s) ? 0 : take(s); }).y;
  }
  const bool split = pieces > 1 && ng > p.split_min;  // the same in every block of the row
  if (!split && piece > 0) return;
  // this block's gather ranks [j0, j1)
  const int j0 = split ? static_cast<int>(static_cast<int64_t>(ng) * piece / pieces) : 0;
  const int j1 = split ? static_cast<int>(static_cast<int64_t>(ng) * (piece + 1) / pieces) : ng;

  // 2. log-sum-exp merge of the slice partials (block 0)
  float M = kNegInf, lsum = 0.f;
  f32x4 on = {0.f, 0.f, 0.f, 0.f};
  for (int b0 = 0; b0 < (ALL_GATHER || piece > 0 ? 0 : ns); b0 += G * kRowMergeSlices) {
    float ms[kRowMergeSlices], lsv[kRowMergeSlices];
    f32x4 ov[kRowMergeSlices];
#pragma unroll
    for (int u = 0; u < kRowMergeSlices; ++u) {
      const int s = b0 + g + G * u;
      const bool use = s < ns && has_partial(s);
      if (kPrefetch && b0 == 0) {  // prefetched
        ms[u] = use ? ms0[u] : kNegInf;
        lsv[u] = use ? ls0[u] : 0.f;
        ov[u] = use ? ov0[u] : f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
        ms[u] = use ? p.sl_ml[2 * (row0 + s)] : kNegInf;
        lsv[u] = use ? p.sl_ml[2 * (row0 + s) + 1] : 0.f;
        ov[u] = use ? *reinterpret_cast<const f32x4*>(p.sl_o + (row0 + s) * D + 4 * c) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    float mb = kNegInf;
#pragma unroll
    for (int u = 0; u < kRowMergeSlices; ++u) mb = fmaxf(mb, ms[u]);
    const float Mn = fmaxf(M, block_max<NW>(mb, red));
    const float rescale = M == kNegInf ? 0.f : __expf(M - Mn);
    lsum *= rescale;
#pragma unroll
    for (int i = 0; i < 4; ++i) on[i] *= rescale;
    M = Mn;
#pragma unroll
    for (int u = 0; u < kRowMergeSlices; ++u) {
      if (ms[u] != kNegInf) {
        const float wgt = __expf(ms[u] - M);
        lsum += lsv[u] * wgt;
#pragma unroll
        for (int i = 0; i < 4; ++i) on[i] += ov[u][i] * wgt;
      }
    }
  }
  // l is the same in every thread of a slice group: one thread per group adds it
  float L = block_sum<NW>(c == 0 ? lsum : 0.f, red);
  accs[tid] = on;
  __syncthreads();
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  if (tid < C) {
    o = accs[tid];
#pragma unroll
    for (int q = 1; q < G; ++q) {
      const f32x4 a = accs[q * C + tid];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] += a[i];
    }
  }

  // 3. the remaining entries (long slices, the slice cut at rank buf_k), batch
  //    by batch through softmax . V (block-uniform branch)
  if (j1 > j0) {
    const int vh = h / (v.q_h / v.v_h);
    const char* vbase = v.v + (bi * v.v_sb + static_cast<int64_t>(vh) * v.v_sh) * Elt<DT>::kBytes;
    BlockPV<DT, D, NT, kRowUnroll> pv;
    pv.init();
    for (int b0 = j0; b0 < j1; b0 += kRowBatch) {
      const int nb = min(kRowBatch, j1 - b0);
      __syncthreads();  // the LDS list of the previous batch (or accs) is free
      for (int i = tid; i < nb; i += NT) {
        const int j = b0 + i;
        const int s = slice_of(gpre, ns, j);
        const int64_t src = (row0 + s) * p.slice_cap + (j - gpre[s]);
        sidx[i] = p.sl_idx[src];
        sval[i] = p.sl_val[src];
      }
      __syncthreads();
      pv.add(nb, sidx, sval, vbase, v.v_sl * Elt<DT>::kBytes, false, red);
    }
    float* accs_f = reinterpret_cast<float*>(accs);
    __syncthreads();
    const float og = pv.reduce(accs_f);  // thread i < D: dim i
    __syncthreads();
    if (tid < D) accs_f[tid] = og;
    __syncthreads();
    const float Mn = fmaxf(M, pv.m);
    const float a = M == kNegInf ? 0.f : __expf(M - Mn);
    const float bw = pv.m == kNegInf ? 0.f : __expf(pv.m - Mn);
    L = L * a + pv.l * bw;
    if (tid < C) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = o[i] * a + accs_f[4 * tid + i] * bw;
    }
    M = Mn;
  }
  if (split) {
    // this block's partial out; the last block of the row merges all of them
    constexpr int PW = D + 4;  // floats per partial: m, l, two unused, o
    float* part = p.row_part + static_cast<int64_t>(r) * pieces * PW;
    if (tid < C) *reinterpret_cast<f32x4*>(part + piece * PW + 4 + 4 * tid) = o;
    if (tid == 0) *reinterpret_cast<f32x2*>(part + piece * PW) = f32x2{M, L};
    // the block's stores complete at the barrier; one agent-scope release
    // fence (an L2 write-back) then orders them before the count, and one
    // acquire fence in the last block (the block's waves share its CU's
    // caches) makes the other blocks' partials visible
    __syncthreads();
    if (tid == 0) {
      __threadfence();
      sh.last = atomicAdd(p.row_cnt + r, 1) == pieces - 1;
      if (sh.last) __threadfence();
    }
    __syncthreads();
    if (!sh.last) return;
    if (tid < C) {
      float Mx = kNegInf;
      for (int q = 0; q < pieces; ++q) Mx = fmaxf(Mx, part[q * PW]);
      L = 0.f;
      o = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int q = 0; q < pieces; ++q) {
        const f32x2 ml = *reinterpret_cast<const f32x2*>(part + q * PW);
        const f32x4 oq = *reinterpret_cast<const f32x4*>(part + q * PW + 4 + 4 * tid);
        const float w = ml.x == kNegInf ? 0.f : __expf(ml.x - Mx);
        L += ml.y * w;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] += oq[i] * w;
      }
    }
    if (tid == 0) p.row_cnt[r] = 0;  // ready for the next call
  }
  if (tid < C) {
    const int64_t ooff = bi * v.o_sb + static_cast<int64_t>(h) * v.o_sh;
    // no passing position: softmax over an empty (all -inf) list is NaN
#pragma unroll
    for (int i = 0; i < 4; ++i)
      store_from_f32(v.out, v.out_dt, ooff + 4 * tid + i, n == 0 ? __builtin_nanf("") : o[i] / L);
  }
  if (tid == 0) {
    p.sel_cnt[r] = n;
    if (p.sel_total) p.sel_total[r] = total;
  }
}

template <int DT, int D, int NT, bool LONG>
__global__ void __launch_bounds__(NT) atopn_gather_kernel(FusedSelParams p, PVParams v) {
  __shared__ RowShared<NT> sh;
  row_merge<DT, D, NT, false, LONG>(p, v, blockIdx.x, sh, blockIdx.y, gridDim.y);
}

// One block per row: its waves compact the row's slices (t once per wave,
// the scores of several slices in flight together), then, after a block
// barrier (which orders their workspace writes before the reads), the whole
// block gathers every kept entry and computes softmax . V -- one launch, no
// kernel boundary and no per-slice partials.
template <int DT, int D, int NT, bool LONG>
__global__ void __launch_bounds__(NT) atopn_rowblock_kernel(FusedSelParams p, PVParams v) {
  __shared__ RowShared<NT> sh;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = blockIdx.x;
  rowblock_slices(p, r, w, NT / kWave);
  __syncthreads();
  row_merge<DT, D, NT, true, LONG>(p, v, r, sh);
}

// One block per row with the whole selection in LDS (rows of at most
// NT / 64 * kRowBlockBurst slices, buf_k <= kRowBatch): the waves hold the
// scores of their slices in registers, count them into LDS, one wave scans
// the counts, the waves write every kept entry at its rank in the row's list
// (the first buf_k in position order) in LDS, the block copies that list to
// the workspace slice lists (for inspection; coalesced, nothing waits for
// it) and gathers the V rows of the list: no global round trip between the
// slice phase and the gather.
template <int NT, int D>
struct RowLdsShared {
  float accs[(NT / kWave) * D];
  float red[NT / kWave];
  int cnt[kRowLdsMaxSlices];
  int pre[kRowLdsMaxSlices + 1];
  int sidx[kRowBatch];
  float sval[kRowBatch];
};

template <int DT, int D, int NT>
__global__ void __launch_bounds__(NT) atopn_rowlds_kernel(FusedSelParams p, PVParams v) {
  constexpr int NW = NT / kWave;
  static_assert(NW * kRowBlockBurst <= kRowLdsMaxSlices, "slice counts fit the LDS arrays");
  __shared__ RowLdsShared<NT, D> sh;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = blockIdx.x;
  const int bi = r / p.q_h, h = r - bi * p.q_h;
  const int ns = p.nslice;  // <= NW * kRowBlockBurst (host-checked)

  // A. partials and the scores of the wave's slices w, w + NW, ... in flight
  //    together; t; the slice counts
  RowPartials rp;
  load_row_partials(p, r, lane, rp);
  f32x4 xv[kRowBlockBurst][kSliceLoads];
#pragma unroll
  for (int u = 0; u < kRowBlockBurst; ++u) {
    const int sl = w + NW * u;
    if (sl < ns) {
      load_slice_scores(p, r, sl, lane, xv[u]);
    } else {
#pragma unroll
      for (int k = 0; k < kSliceLoads; ++k) xv[u][k] = f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
    }
  }
  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  __builtin_amdgcn_sched_barrier(0);
  const float t = row_threshold(p, r, lane, rp);
#pragma unroll
  for (int u = 0; u < kRowBlockBurst; ++u) {
    const int sl = w + NW * u;
    if (sl < ns) {
      const int c = count_slice(sl * kSliceLen, t, Leff, xv[u], lane);
      if (lane == 0) sh.cnt[sl] = c;
    }
  }
  lds_sync();
  // B. slice ranks (one wave: ns <= 64)
  if (w == 0) {
    const int c = lane < ns ? sh.cnt[lane] : 0;
    const int incl = wave_incl_scan(c, lane);
    if (lane < ns) sh.pre[lane] = incl - c;
    if (lane == ns - 1) sh.pre[ns] = incl;
  }
  lds_sync();
  const int total = sh.pre[ns];
  const int n = min(total, p.cap);
  // C. every kept entry at its rank (LDS list of the first n), the workspace lists and counts
#pragma unroll
  for (int u = 0; u < kRowBlockBurst; ++u) {
    const int sl = w + NW * u;
    if (sl < ns) {
      const int64_t gw = static_cast<int64_t>(r) * ns + sl;
      const int c = compact_slice<kListNone>(p, gw, sl * kSliceLen, t, Leff, xv[u], lane, sh.sidx, sh.sval, sh.pre[sl], n);
      if (lane == 0) p.sl_cnt[gw] = c;
    }
  }
  if (w == 0 && lane == 0 && p.t_out) p.t_out[r] = t;
  lds_sync();
  // the kept entries to their slices' workspace lists (inspection only;
  // entries past the row's first n are not written), coalesced
  for (int i = tid; i < n; i += NT) {
    const int sl = slice_of(sh.pre, ns, i);
    const int64_t dst = (static_cast<int64_t>(r) * ns + sl) * p.slice_cap + (i - sh.pre[sl]);
    p.sl_idx[dst] = sh.sidx[i];
    p.sl_val[dst] = sh.sval[i];
  }
  // D. softmax . V over the list
  const int vh = h / (v.q_h / v.v_h);
  const char* vbase = v.v + (bi * v.v_sb + static_cast<int64_t>(vh) * v.v_sh) * Elt<DT>::kBytes;
  BlockPV<DT, D, NT, kRowUnroll> pv;
  pv.init();
  if (n > 0) pv.add(n, sh.sidx, sh.sval, vbase, v.v_sl * Elt<DT>::kBytes, false, sh.red);
  const float o = pv.reduce(sh.accs);  // thread i < D: dim i
  if (tid < D) {
    const int64_t ooff = bi * v.o_sb + static_cast<int64_t>(h) * v.o_sh;
    // no passing position: softmax over an empty (all -inf) list is NaN
    store_from_f32(v.out, v.out_dt, ooff + tid, n == 0 ? __builtin_nanf("") : o / pv.l);
  }
  if (tid == 0) {
    p.sel_cnt[r] = n;
    if (p.sel_total) p.sel_total[r] = total;
  }
}

template <int DT, int D>
static hipError_t launch_rows_typed(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  // rows of more than kRowMaxSlices slices keep their ranks in the workspace,
  // shared by a row's blocks: one block per row (no split)
  const bool lng = p.nslice > kRowMaxSlices;
  const int nt = p.cap <= kRowSmallCap ? kRowThreadsSmall : kRowThreadsLarge;
  const int64_t threads = static_cast<int64_t>(p.nrows) * nt;
  const unsigned pieces = lng || threads > kRowSplitThreads ? 1u : static_cast<unsigned>(kRowSplit);
  FusedSelParams q = p;
  q.split_min = threads <= kRowSplitSmallThreads ? 384 : 768;
  if (nt == kRowThreadsSmall) {
    if (lng)
      hipLaunchKernelGGL((atopn_gather_kernel<DT, D, kRowThreadsSmall, true>), dim3(q.nrows, 1),
                         dim3(kRowThreadsSmall), 0, st, q, v);
    else
      hipLaunchKernelGGL((atopn_gather_kernel<DT, D, kRowThreadsSmall, false>), dim3(q.nrows, pieces),
                         dim3(kRowThreadsSmall), 0, st, q, v);
  } else {
    if (lng)
      hipLaunchKernelGGL((atopn_gather_kernel<DT, D, kRowThreadsLarge, true>), dim3(q.nrows, 1),
                         dim3(kRowThreadsLarge), 0, st, q, v);
    else
      hipLaunchKernelGGL((atopn_gather_kernel<DT, D, kRowThreadsLarge, false>), dim3(q.nrows, pieces),
                         dim3(kRowThreadsLarge), 0, st, q, v);
  }
  return hipGetLastError();
}

bool k2_row_block(int64_t nslice, int64_t cap, int variant) {
  if (variant == kK2RowBlock) return true;
  if (variant == kK2SliceRow) return false;
  return nslice <= kRowBlockAutoSlices && cap <= kRowBatch;
}

template <int DT, int D>
static hipError_t launch_split(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  if (k2_row_block(p.nslice, p.cap, p.k2_variant)) {
    if (p.cap <= kRowBatch && p.nslice <= 4)
      hipLaunchKernelGGL((atopn_rowlds_kernel<DT, D, 256>), dim3(p.nrows), dim3(256), 0, st, p, v);
    else if (p.cap <= kRowBatch && p.nslice <= 16 * kRowBlockBurst)
      hipLaunchKernelGGL((atopn_rowlds_kernel<DT, D, 1024>), dim3(p.nrows), dim3(1024), 0, st, p, v);
    else if (p.nslice <= kRowMaxSlices)
      hipLaunchKernelGGL((atopn_rowblock_kernel<DT, D, 1024, false>), dim3(p.nrows), dim3(1024), 0, st, p, v);
    else
      hipLaunchKernelGGL((atopn_rowblock_kernel<DT, D, 1024, true>), dim3(p.nrows), dim3(1024), 0, st, p, v);
    return hipGetLastError();
  }
  const int64_t waves = static_cast<int64_t>(p.nslice) * p.nrows;
  const unsigned blocks = static_cast<unsigned>((waves + kSliceWaves - 1) / kSliceWaves);
  hipLaunchKernelGGL((atopn_slice_kernel<DT, D>), dim3(blocks), dim3(kSliceThreads), 0, st, p, v);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_rows_typed<DT, D>(p, v, st);
}

template <int DT>
static hipError_t launch_split_d(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  return v.d == 128 ? launch_split<DT, 128>(p, v, st) : launch_split<DT, 64>(p, v, st);
}

hipError_t launch_atopn_fast(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  if (v.v_dt == SAGA_DTYPE_BF16) return launch_split_d<SAGA_DTYPE_BF16>(p, v, st);
  if (v.v_dt == SAGA_DTYPE_F16) return launch_split_d<SAGA_DTYPE_F16>(p, v, st);
  return launch_split_d<SAGA_DTYPE_F32>(p, v, st);
}

}  // namespace saga

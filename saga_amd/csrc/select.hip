// K2 of the calibration step and the threshold_topk_fast API kernel, one
// 1024-thread block per score row (the fast step's K2 is atopn_split.hip).
//
// Replaces torch.topk + the renormalised gather of
// approx_top_n_attention_amortized_cal (attention/attention.py:173-189) and
// the Triton stream compaction threshold_select_fast_kernel
// (attention/triton_atopn.py:6-53).  Ordered, deterministic compactions.
// API kernel: a row is read in tiles of 1024 x 16 elements; each wave turns
// its pass flags into 64-bit ballots, the per-(slot, wave) counts are
// prefix-summed in LDS in ascending index order, and every passing element
// goes to base + prefix + popcount(ballot & lanes_below).  Calibration: each
// wave takes 1024 consecutive elements of a tile, so a rank is the lower
// waves' total + the wave's running count + mbcnt.
#include <type_traits>

#include "kernels.h"
#include "select.cuh"

namespace saga {

constexpr int kSelEPT = 16;                       // elements per thread per tile
constexpr int kSelSlots = kSelEPT * kBlkWaves;    // 256 (slot, wave) counters
constexpr int kSelTile = kBlkThreads * kSelEPT;   // 16384 elements
constexpr int kListLDS = 4096;                    // selection entries kept in LDS

static_assert(kSelSlots == 4 * kWave, "wave-0 scan handles 4 counters per lane");

// Exclusive scan of cnt[0..256) into pre[0..256], pre[256] = total (one wave).
__device__ __forceinline__ void scan_slots(const int* cnt, int* pre, int lane) {
  const int c0 = cnt[4 * lane], c1 = cnt[4 * lane + 1], c2 = cnt[4 * lane + 2], c3 = cnt[4 * lane + 3];
  const int tot = c0 + c1 + c2 + c3;
  const int incl = wave_incl_scan(tot, lane);
  const int ex = incl - tot;
  pre[4 * lane] = ex;
  pre[4 * lane + 1] = ex + c0;
  pre[4 * lane + 2] = ex + c0 + c1;
  pre[4 * lane + 3] = ex + c0 + c1 + c2;
  if (lane == kWave - 1) pre[kSelSlots] = incl;
}

struct SelShared {
  static constexpr int kList = kListLDS;  // selection entries kept in LDS
  float red[kBlkWaves];
  int cnt[kSelSlots];
  int pre[kSelSlots + 1];
  int cntE[kSelSlots];
  int preE[kSelSlots + 1];
  int hist[2048];
  int sel_bin, sel_above, sel_cnt;
  int sidx[kList];
  float sval[kList];
};

// Run the PV phase over a row's list: from LDS when it fits, otherwise in
// LDS-sized batches re-read from the workspace copy.
template <int DT, int D, class SH>
__device__ void row_pv(SH& sh, float* accs, int n, const int32_t* gidx, const float* gval, const PVParams& v,
                       int bi, int h, bool probs) {
  constexpr int kListLDS = SH::kList;
  const int vh = h / (v.q_h / v.v_h);
  const char* vbase = v.v + (bi * v.v_sb + static_cast<int64_t>(vh) * v.v_sh) * Elt<DT>::kBytes;
  const int64_t vrow = v.v_sl * Elt<DT>::kBytes;
  BlockPV<DT, D> pv;
  pv.init();
  if (n <= kListLDS) {
    pv.add(n, sh.sidx, sh.sval, vbase, vrow, probs, sh.red);
  } else {
    for (int b0 = 0; b0 < n; b0 += kListLDS) {
      const int nb = min(kListLDS, n - b0);
      __syncthreads();
      for (int i = threadIdx.x; i < nb; i += kBlkThreads) {
        sh.sidx[i] = gidx[b0 + i];
        sh.sval[i] = gval[b0 + i];
      }
      __syncthreads();
      pv.add(nb, sh.sidx, sh.sval, vbase, vrow, probs, sh.red);
    }
  }
  pv.finish(accs, v.out, v.out_dt, bi * v.o_sb + static_cast<int64_t>(h) * v.o_sh, probs);
}

// f(x[i]) for every i < n of a score row (ld floats, 16-byte aligned, n <= ld),
// in tiles of 16 elements per thread whose four 16-byte loads are in flight
// together (one load per element and step would wait out a round trip each).
template <class F>
__device__ __forceinline__ void row_tiles(const float* x, int64_t ld, int n, F f) {
  const int tid = threadIdx.x;
  for (int st = 0; st < n; st += 16 * kBlkThreads) {
    f32x4 v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t e = st + 4 * (q * kBlkThreads + tid);
      v[q] = e < ld ? *reinterpret_cast<const f32x4*>(x + e) : f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (st + 4 * (q * kBlkThreads + tid) + j < n) f(v[q][j]);
  }
}

// radix_select_each over the score row x (ROW) or the LDS candidates sh.sval.
template <bool ROW, class SH>
__device__ __forceinline__ uint32_t radix_select(SH& sh, const float* x, int64_t ld, int n, int& krem) {
  if constexpr (ROW) {
    return radix_select_each(sh, krem, [&](auto f) { row_tiles(x, ld, n, f); });
  } else {
    return radix_select_each(sh, krem, [&](auto f) {
      for (int i = threadIdx.x; i < n; i += kBlkThreads) f(sh.sval[i]);
    });
  }
}

// The krem-th largest score of the row without a radix pass over it: one
// pass counts every position into its bin of distance (M - x) * 32 below the
// row max M (the bins are monotone in x, so every element of a nearer bin is
// strictly larger than every element of a farther one), a second gathers
// the elements of the bin that holds the krem-th largest into LDS, and the
// radix select runs over those few.  On N(0,1)-like scores the counts spread
// over hundreds of bins, where the top bits of the float key put them into a
// handful (LDS atomics serialised up to 64 ways).  Returns false, leaving the
// work to the full-row select, for a NaN or non-finite max, a k-th value more
// than 64 below M, or more candidates than the LDS list holds.  kth and krem
// as radix_select.
// The distance histogram (pass 1 of near_pick): every position of the row
// into its bin; false for a NaN or a non-finite max (block-uniform).
template <class SH>
__device__ __forceinline__ bool near_hist(SH& sh, const float* x, int64_t ld, int Leff, float M) {
  const int tid = threadIdx.x;
  if (!(M > -INFINITY && M < INFINITY)) return false;  // block-uniform
  for (int i = tid; i < kNearBins; i += kBlkThreads) sh.hist[i] = 0;
  lds_sync();
  int odd = 0;
  row_tiles(x, ld, Leff, [&](float xi) {
    if (!(xi <= M)) {  // NaN
      odd = 1;
      return;
    }
    const float dd = (M - xi) * kNearScale;
    if (dd < kNearBins) atomicAdd(&sh.hist[kNearBins - 1 - static_cast<int>(dd)], 1);
  });
  return !__syncthreads_or(odd);
}

// The rest of near_pick, over the histogram of near_hist: the bin holding
// the krem-th largest, its elements gathered into LDS, the radix select
// over them.
template <class SH>
__device__ __forceinline__ bool near_select(SH& sh, const float* x, int64_t ld, int Leff, float M, int& krem,
                                            uint32_t& kth) {
  const int tid = threadIdx.x;
  int bin, above, c;
  hist_pick(sh, kNearBins, krem, bin, above, c);
  if (bin < 0) return false;
  if (c > SH::kList) return false;
  const int want = kNearBins - 1 - bin;  // distance bin of the candidates
  if (tid == 0) sh.sel_bin = 0;          // candidate count
  lds_sync();
  row_tiles(x, ld, Leff, [&](float xi) {
    const float dd = (M - xi) * kNearScale;
    if (dd < kNearBins && static_cast<int>(dd) == want) sh.sval[atomicAdd(&sh.sel_bin, 1)] = xi;
  });
  lds_sync();
  krem -= above;
  kth = radix_select<false>(sh, nullptr, 0, c, krem);
  return true;
}

template <class SH>
__device__ __forceinline__ bool near_pick(SH& sh, const float* x, int64_t ld, int Leff, float M, int& krem,
                                          uint32_t& kth) {
  return near_hist(sh, x, ld, Leff, M) && near_select(sh, x, ld, Leff, M, krem, kth);
}

// Calibration: exact top-k of the row (k = min(top_n, L)), for rows past
// the block-resident kernel below (more than 17 * 4096 positions, top_n >
// 4096, or top_n > 2048 past 13 * 4096 positions), the row re-read from
// memory by each pass.
//   1. full-row max M and sum S of exp(x - M) from the K1 partials;
//   2. the k-th largest value: by a radix select over the few elements of
//      its bin of distance below M (near_pick), else over the whole row;
//   3. ordered compaction of the elements above it plus the first (by index)
//      elements equal to it, exactly k;
//   4. p* = exp(x_k - M) / S, the k-th largest probability, into the
//      threshold table (attention/attention.py:185-187);
//   5. softmax over the k logits . V == renormalised top-k probabilities . V.
template <int DT, int D>
__global__ void __launch_bounds__(kBlkThreads) atopn_calibrate_kernel(FusedSelParams p, PVParams v) {
  __shared__ SelShared sh;
  __shared__ float accs[kBlkWaves * D];
  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int bi = r / p.q_h, h = r - bi * p.q_h;
  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  const float* x = p.scores + static_cast<int64_t>(r) * p.ld;
  const float* prow_m = p.pmax + static_cast<int64_t>(r) * p.nparts;
  const float* prow_s = p.psum + static_cast<int64_t>(r) * p.nparts;

  const int nch = p.nparts;  // parts past kv_len hold (-inf, 0)
  float mloc = kNegInf;
  for (int c = tid; c < nch; c += kBlkThreads) mloc = fmaxf(mloc, prow_m[c]);
  const float M = block_max<kBlkWaves>(mloc, sh.red);
  float sloc = 0.f;
  for (int c = tid; c < nch; c += kBlkThreads) {
    const float pm = prow_m[c];
    if (pm != kNegInf) sloc += prow_s[c] * __expf(pm - M);
  }
  const float S = block_sum<kBlkWaves>(sloc, sh.red);

  const int k = min(p.cap, Leff);
  int32_t* gidx = p.sel_idx + static_cast<int64_t>(r) * p.cap;
  float* gval = p.sel_val + static_cast<int64_t>(r) * p.cap;
  if (k <= 0) {
    if (tid == 0) {
      p.sel_cnt[r] = 0;
      if (p.sel_total) p.sel_total[r] = 0;
      p.pstar_out[r] = 0.f;
    }
    row_pv<DT, D>(sh, accs, 0, gidx, gval, v, bi, h, false);
    return;
  }

  // the k-th largest key: among the few elements of its bin of distance
  // below M when that is cheap (near_pick), else over the whole row
  int krem = k;
  uint32_t kth = 0;
  if (!near_pick(sh, x, p.ld, Leff, M, krem, kth)) {
    krem = k;
    kth = radix_select<true>(sh, x, p.ld, Leff, krem);
  }
  const int need = krem;  // elements equal to the k-th value that are taken

  // Ordered compaction, tile by tile (LDS-only barriers: the list's global
  // copy is read back only by row_pv's batches, after a full barrier): wave w takes the kSelEPT * 64
  // consecutive elements [st + 1024 w, st + 1024 (w + 1)) of the tile, so the
  // index order is (tile, wave, step, lane) and an element's rank is its
  // wave's offset (the totals of the lower waves) + the running count of its
  // wave + its lane's mbcnt; loads are clamped, not branched (a load under a
  // branch is waited for at the join).
  int baseG = 0, baseE = 0;
  for (int st = 0; st < Leff; st += kSelTile) {
    const int w0 = st + w * (kSelEPT * kWave);
    float xv[kSelEPT];
#pragma unroll
    for (int kk = 0; kk < kSelEPT; ++kk) xv[kk] = x[min(w0 + kk * kWave + lane, Leff - 1)];
    unsigned long long bg[kSelEPT], be[kSelEPT];
    int cg = 0, ce = 0;
#pragma unroll
    for (int kk = 0; kk < kSelEPT; ++kk) {
      const bool in = w0 + kk * kWave + lane < Leff;
      const uint32_t key = f32_to_key(xv[kk]);
      bg[kk] = __ballot(in && key > kth);
      be[kk] = __ballot(in && key == kth);
      cg += __popcll(bg[kk]);
      ce += __popcll(be[kk]);
    }
    if (lane == 0) {
      sh.cnt[w] = cg;
      sh.cntE[w] = ce;
    }
    lds_sync();
    int g_off = baseG, e_off = baseE, totG = 0, totE = 0;
#pragma unroll
    for (int q = 0; q < kBlkWaves; ++q) {
      const int a = sh.cnt[q], b = sh.cntE[q];
      if (q < w) {
        g_off += a;
        e_off += b;
      }
      totG += a;
      totE += b;
    }
#pragma unroll
    for (int kk = 0; kk < kSelEPT; ++kk) {
      if ((bg[kk] | be[kk]) != 0ull) {  // wave-uniform: most steps hold no taken element
        const int g_before = g_off + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
            static_cast<uint32_t>(bg[kk] >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bg[kk]), 0u)));
        const int e_before = e_off + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
            static_cast<uint32_t>(be[kk] >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(be[kk]), 0u)));
        int pos = -1;
        if ((bg[kk] >> lane) & 1ull) pos = g_before + min(e_before, need);
        else if (((be[kk] >> lane) & 1ull) && e_before < need) pos = g_before + e_before;
        if (pos >= 0) {
          const int i = w0 + kk * kWave + lane;
          gidx[pos] = i;
          gval[pos] = xv[kk];
          if (pos < kListLDS) {
            sh.sidx[pos] = i;
            sh.sval[pos] = xv[kk];
          }
        }
      }
      g_off += __popcll(bg[kk]);
      e_off += __popcll(be[kk]);
    }
    baseG += totG;
    baseE += totE;
    lds_sync();
  }
  if (tid == 0) {
    p.sel_cnt[r] = k;
    if (p.sel_total) p.sel_total[r] = k;
    p.pstar_out[r] = expf(key_to_f32(kth) - M) / S;
  }
  row_pv<DT, D>(sh, accs, k, gidx, gval, v, bi, h, false);
}

// ---------------------------------------------------------------------------
// Calibration with the score row held in registers: rows of up to
// CH * 4096 positions are read from HBM once, every later pass runs over the
// registers.  Wave w holds positions [w * 256 CH, (w + 1) * 256 CH): chunk q
// of the wave is the 256 positions from w * 256 CH + 256 q, lane l holding
// its four from 4 l (16-byte loads, 1 KiB per wave and load).  Index order is
// (wave, chunk, lane, element), so a position's rank among the selected ones
// is its wave's offset + its chunk's offset in the wave + a wave scan.
//
// Selection by classes: with the k-th largest value's distance bin B
// (2048 bins of (M - x) * s below the max M, s a power of two fitted to the
// row's spread; elements of nearer bins are all larger than every element of
// B, as in near_pick), the positions of nearer bins are all kept ("nearer") and the
// krem largest of bin B's elements ("candidates", by value, then lowest
// index) complete the k.  The candidates -- a few dozen on N(0,1)-like rows
// -- go to LDS in index order and are ranked there; a kept position's slot
// in the list is the nearer positions before it + the kept candidates
// before it.  When the distance bins cannot be used (a NaN or non-finite
// max, more candidates than LDS holds: ties, or one bin of a row stretched by
// a far outlier) the classes are by key: above the k-th key (from a radix
// select over the registers) and equal to it, the first `need` of which are
// kept.
constexpr int kRegList = 4096;   // k <= kRegList: the kept list in LDS
constexpr int kRegChunks = 13;   // chunks kept in registers (more: thread-private LDS slots)
constexpr int kRegListLong = 2048;  // the 17-chunk rows: kept list (k <= 2048),
constexpr int kRegCandLong = 1024;  //   candidates in LDS,
constexpr int kRegChunksLong = 12;  //   chunks in registers (5 in LDS)
constexpr int kRegCand = 2048;   // candidates of the distance classes kept in LDS
constexpr int kRegRank = 128;    // candidates ranked pairwise; more: radix select

template <int LIST, int CAND>
struct RegShared {
  static constexpr int kList = LIST;
  float red[kBlkWaves];
  int cnt[kBlkWaves];      // hist_pick's per-wave totals
  int wtot[2][kBlkWaves];  // per-wave class totals (nearer, candidates)
  int scan[kBlkWaves];     // per-wave totals of the taken-flag scan
  int hist[2048];
  int sel_bin, sel_above, sel_cnt, sel_key;
  int sidx[LIST];           // the kept list (key classes) / the nearer positions (distance classes),
  float sval[LIST];         //   their values
  int ncb[LIST];            //   and the candidates before each nearer position
  float cval[CAND];         // candidates in index order: value,
  int cidx[CAND];           // position,
  int cnb[CAND];            // nearer positions before it,
  int ctp[CAND + 1];        // kept candidates before it (ctp[c] = all kept)
  int cflag[CAND];          // kept?
};

template <int DT, int D, int CH, int LIST>
__global__ void __launch_bounds__(kBlkThreads) atopn_calibrate_reg_kernel(FusedSelParams p, PVParams v) {
  // chunks [0, CHR) in registers, the rest in thread-private LDS slots (at
  // 14 register chunks and more the compiler spills the row itself)
  constexpr int CHR = CH <= kRegChunks ? CH : kRegChunksLong;
  constexpr int CHL = CH - CHR;
  constexpr int CAND = CHL > 0 ? kRegCandLong : kRegCand;
  __shared__ RegShared<LIST, CAND> sh;
  __shared__ float accs[kBlkWaves * D];
  __shared__ f32x4 rowl[CHL > 0 ? CHL * kBlkThreads : 1];
  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int bi = r / p.q_h, h = r - bi * p.q_h;
  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  const float* x = p.scores + static_cast<int64_t>(r) * p.ld;
  const float* prow_m = p.pmax + static_cast<int64_t>(r) * p.nparts;
  const float* prow_s = p.psum + static_cast<int64_t>(r) * p.nparts;
  const int nch = p.nparts;  // parts past kv_len hold (-inf, 0)

  // K1's partials first, then the whole row: the row's loads stay in flight
  // through the max / sum reductions
  const float pm0 = tid < nch ? prow_m[tid] : kNegInf;
  const float ps0 = tid < nch ? prow_s[tid] : 0.f;
  const int wbase = w * (CH * 256) + 4 * lane;  // chunk q: wbase + 256 q + j
  const int lastq = max(0, (Leff + 3) / 4 * 4 - 4);  // loads past Leff are clamped (and never used)
  f32x4 xr[CHR], xl[CHL > 0 ? CHL : 1];
#pragma unroll
  for (int q = 0; q < CH; ++q) {
    const f32x4 v4 = *reinterpret_cast<const f32x4*>(x + min(wbase + 256 * q, lastq));
    if (q < CHR) xr[q < CHR ? q : 0] = v4;
    else xl[q >= CHR ? q - CHR : 0] = v4;
  }
  for (int i = tid; i < 2048; i += kBlkThreads) sh.hist[i] = 0;

  float mloc = pm0;
  for (int c = tid + kBlkThreads; c < nch; c += kBlkThreads) mloc = fmaxf(mloc, prow_m[c]);
  const float M = block_max<kBlkWaves>(mloc, sh.red);  // (its barriers also publish the zeroed histogram)
  float sloc = pm0 != kNegInf ? ps0 * __expf(pm0 - M) : 0.f;
  for (int c = tid + kBlkThreads; c < nch; c += kBlkThreads) {
    const float pm = prow_m[c];
    if (pm != kNegInf) sloc += prow_s[c] * __expf(pm - M);
  }
  const float S = block_sum<kBlkWaves>(sloc, sh.red);
#pragma unroll
  for (int q = 0; q < CHL; ++q) rowl[q * kBlkThreads + tid] = xl[q];  // (read back by this thread only)
  // chunk q of the thread's share of the row
  auto chunk = [&](int q) -> f32x4 {
    if (q < CHR) return xr[q < CHR ? q : 0];
    return rowl[(q >= CHR ? q - CHR : 0) * kBlkThreads + tid];
  };

  const int k = min(p.cap, Leff);
  int32_t* gidx = p.sel_idx + static_cast<int64_t>(r) * p.cap;
  float* gval = p.sel_val + static_cast<int64_t>(r) * p.cap;
  using PV = BlockPV<DT, D>;
  const int vh = h / (v.q_h / v.v_h);
  const char* vbase = v.v + (bi * v.v_sb + static_cast<int64_t>(vh) * v.v_sh) * Elt<DT>::kBytes;
  const int64_t vrow = v.v_sl * Elt<DT>::kBytes;
  const int64_t ooff = bi * v.o_sb + static_cast<int64_t>(h) * v.o_sh;
  if (k <= 0) {
    if (tid == 0) {
      p.sel_cnt[r] = 0;
      if (p.sel_total) p.sel_total[r] = 0;
      p.pstar_out[r] = 0.f;
    }
    PV pv;
    pv.init();
    pv.finish(accs, v.out, v.out_dt, ooff, false);  // 0 / 0: an empty row's output is NaN
    return;
  }

  // every in-row element of the thread's share: f(value, position)
  auto each_in = [&](auto f) {
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      const int lim = Leff - (wbase + 256 * q);  // elements of this chunk in the row
      const f32x4 xq = chunk(q);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < lim) f(xq[j]);
    }
  };

  // the bins' scale from the smallest finite score mn (near_bin_scale)
  float mnl = INFINITY;
#pragma unroll
  for (int q = 0; q < CH; ++q) {
    const int lim = Leff - (wbase + 256 * q);
    const f32x4 xq = chunk(q);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float xi = xq[j];
      mnl = fminf(mnl, (j < lim && xi > -INFINITY) ? xi : INFINITY);  // (no branch per element)
    }
  }
  const float mn = -block_max<kBlkWaves>(-mnl, sh.red);
  const float scale = near_bin_scale(M, mn);

  // pass 1: distance bins (M - x) * s below the max; a NaN, or a max
  // that is not finite, sends the row to the key classes
  const float Ms = M * scale;
  int odd = (M > -INFINITY && M < INFINITY) ? 0 : 1;
  if (!odd) {
    each_in([&](float xi) {
      const float dd = fmaf(-xi, scale, Ms);
      if (!(dd >= 0.f)) odd = 1;
      else if (dd < static_cast<float>(kNearBins)) atomicAdd(&sh.hist[kNearBins - 1 - static_cast<int>(dd)], 1);
    });
  }
  bool near = !__syncthreads_or(odd);
  int krem = k, bin = -1, above = 0;
  if (near) {
    int bcnt;
    hist_pick(sh, kNearBins, k, bin, above, bcnt);
    near = bin >= 0 && bcnt <= CAND;  // block-uniform
  }
  uint32_t kth = 0;
  float wantf = 0.f;
  if (near) {
    krem = k - above;
    wantf = static_cast<float>(kNearBins - 1 - bin);
  } else {
    krem = k;
    kth = radix_select_each(sh, krem, each_in);  // krem -> need (keys equal to kth that are kept)
  }
  const int need = krem;

  // class pass: per chunk, 4-bit masks of nearer / candidate elements and
  // one wave scan of both counts (packed: 16 bits each; a wave chunk holds
  // at most 256 of a class); positions past Leff are masked per chunk
  // the lane's class masks, 8 bits per chunk (nearer | candidates << 4);
  // the lane's counts before it in the chunk are re-scanned where needed
  uint32_t msk[(CH + 3) / 4];
#pragma unroll
  for (int u = 0; u < (CH + 3) / 4; ++u) msk[u] = 0u;
  int base[CH];  // the wave's nearer | candidates << 16 before chunk q (wave-uniform)
  int wN = 0, wC = 0;
  auto classify = [&](auto cls) {
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      uint32_t mN = 0, mC = 0;
      const f32x4 xq = chunk(q);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bool n, c;
        cls(xq[j], n, c);
        mN |= static_cast<uint32_t>(n) << j;
        mC |= static_cast<uint32_t>(c) << j;
      }
      const int lim = Leff - (wbase + 256 * q);
      const uint32_t valid = lim >= 4 ? 15u : (lim > 0 ? (1u << lim) - 1u : 0u);
      mN &= valid;
      mC &= valid & ~mN;
      const int cntv = __popc(mN) | (__popc(mC) << 16);
      const int inc = wave_incl_scan(cntv, lane);
      msk[q >> 2] |= (mN | (mC << 4)) << (8 * (q & 3));
      base[q] = wN | (wC << 16);
      const int tot = __builtin_amdgcn_readlane(inc, kWave - 1);
      wN += tot & 0xffff;
      wC += tot >> 16;
    }
  };
  if (near) {
    const float wantf1 = wantf + 1.f;
    classify([&](float xi, bool& n, bool& c) {  // (in-row elements have dd >= 0)
      const float dd = fmaf(-xi, scale, Ms);
      n = dd < wantf;
      c = dd < wantf1;  // minus the nearer ones
    });
  } else {
    classify([&](float xi, bool& n, bool& c) {
      const uint32_t key = f32_to_key(xi);
      n = key > kth;
      c = key == kth;
    });
  }
  if (lane == 0) {
    sh.wtot[0][w] = wN;
    sh.wtot[1][w] = wC;
  }
  lds_sync();
  int WN = 0, WC = 0, TN = 0, TC = 0;
#pragma unroll
  for (int u = 0; u < kBlkWaves; ++u) {
    const int a = sh.wtot[0][u], b = sh.wtot[1][u];
    if (u < w) {
      WN += a;
      WC += b;
    }
    TN += a;
    TC += b;
  }
  // chunk q's masks and the nearer / candidates before the lane's first
  // element of it (every lane calls it: it holds a wave scan)
  auto chunk_bases = [&](int q, uint32_t& mN, uint32_t& mC, int& nb0, int& cb0) {
    const uint32_t m8 = (msk[q >> 2] >> (8 * (q & 3))) & 0xffu;
    mN = m8 & 15u;
    mC = m8 >> 4;
    const int cntv = __popc(mN) | (__popc(mC) << 16);
    const int ex = wave_incl_scan(cntv, lane) - cntv;
    nb0 = WN + (base[q] & 0xffff) + (ex & 0xffff);
    cb0 = WC + (base[q] >> 16) + (ex >> 16);
  };

  // the kept list (key classes: in LDS in position order) or the nearer
  // positions + the candidates (distance classes) are the softmax . V
  // entries: the first nl from sidx / sval, then c candidates
  int nl = k, c = 0;
  if (!near) {
    // key classes: every kept position is placed by its owner, the first
    // need equal ones by their rank among the equal ones
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      uint32_t mN, mC;
      int nb0, cb0;
      chunk_bases(q, mN, mC, nb0, cb0);
      if (mN | mC) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t below = (1u << j) - 1u;
          const int cb = cb0 + __popc(mC & below);
          if (((mN >> j) & 1u) || (((mC >> j) & 1u) && cb < need)) {
            const int pos = nb0 + __popc(mN & below) + min(cb, need);
            if (pos < k) {
              sh.sidx[pos] = wbase + 256 * q + j;
              sh.sval[pos] = chunk(q)[j];
            }
          }
        }
      }
    }
    __syncthreads();
    for (int i = tid; i < k; i += kBlkThreads) {  // the kept list for inspection, coalesced
      gidx[i] = sh.sidx[i];
      gval[i] = sh.sval[i];
    }
  } else {
    // distance classes: the nearer positions go to LDS at their rank among
    // the nearer ones (with the candidates before each), the candidates in
    // index order, where they are ranked
    c = TC;  // == the bin's count <= CAND
    nl = TN;  // (== k - krem) nearer positions, all kept
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      uint32_t mN, mC;
      int nb0, cb0;
      chunk_bases(q, mN, mC, nb0, cb0);
      if (mN | mC) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t below = (1u << j) - 1u;
          const int nb = nb0 + __popc(mN & below), cb = cb0 + __popc(mC & below);
          if ((mN >> j) & 1u) {
            if (nb < LIST) {
              sh.sidx[nb] = wbase + 256 * q + j;
              sh.sval[nb] = chunk(q)[j];
              sh.ncb[nb] = cb;
            }
          } else if ((mC >> j) & 1u) {
            if (cb < CAND) {
              sh.cval[cb] = chunk(q)[j];
              sh.cidx[cb] = wbase + 256 * q + j;
              sh.cnb[cb] = nb;
            }
          }
        }
      }
    }
    lds_sync();

    // which candidates are kept, and the k-th key (block-uniform branches)
    if (c <= kRegRank) {
      // pairwise ranks by (value desc, index asc), 8 threads per candidate:
      // rank < krem is kept, rank krem - 1 is the k-th
      const int i = tid >> 3, sub = tid & 7;
      int rank = 0;
      uint32_t ki = 0;
      if (i < c) {
        ki = f32_to_key(sh.cval[i]);
#pragma unroll 4
        for (int u = sub; u < c; u += 8) {
          const uint32_t ku = f32_to_key(sh.cval[u]);
          rank += (ku > ki || (ku == ki && u < i)) ? 1 : 0;
        }
      }
      rank += __shfl_xor(rank, 1);
      rank += __shfl_xor(rank, 2);
      rank += __shfl_xor(rank, 4);
      if (i < c && sub == 0) {
        sh.cflag[i] = rank < krem ? 1 : 0;
        if (rank == krem - 1) sh.sel_key = static_cast<int>(ki);
      }
      lds_sync();
      kth = static_cast<uint32_t>(sh.sel_key);
      // prefix of the flags, 8 threads per candidate
      int before = 0;
      if (i < c) {
#pragma unroll 4
        for (int u = sub; u < i; u += 8) before += sh.cflag[u];
      }
      before += __shfl_xor(before, 1);
      before += __shfl_xor(before, 2);
      before += __shfl_xor(before, 4);
      if (i < c && sub == 0) sh.ctp[i] = before;
      if (tid == 0) sh.ctp[c] = krem;
    } else {
      int nd = krem;
      kth = radix_select_each(sh, nd, [&](auto f) {
        for (int t = tid; t < c; t += kBlkThreads) f(sh.cval[t]);
      });
      // kept: above kth, or equal to it and among the first nd equal ones
      int tflag[4] = {0, 0, 0, 0};  // candidates 4 tid .. 4 tid + 3
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 4 * tid + j;
        if (t < c) {
          const uint32_t kt = f32_to_key(sh.cval[t]);
          if (kt > kth) {
            tflag[j] = 1;
          } else if (kt == kth) {
            int eq = 0;
            for (int u = 0; u < t; ++u) eq += f32_to_key(sh.cval[u]) == kth ? 1 : 0;
            tflag[j] = eq < nd ? 1 : 0;
          }
          sh.cflag[t] = tflag[j];
        }
      }
      const int ts = tflag[0] + tflag[1] + tflag[2] + tflag[3];
      const int tb = block_excl_scan4(ts, sh.scan);
      if (4 * tid < c) {
        sh.ctp[4 * tid] = tb;
        if (4 * tid + 1 <= c) sh.ctp[4 * tid + 1] = tb + tflag[0];
        if (4 * tid + 2 <= c) sh.ctp[4 * tid + 2] = tb + tflag[0] + tflag[1];
        if (4 * tid + 3 <= c) sh.ctp[4 * tid + 3] = tb + tflag[0] + tflag[1] + tflag[2];
        if (4 * tid + 4 <= c) sh.ctp[4 * tid + 4] = ts + tb;
      }
    }
    lds_sync();

    // the kept list, in position order, straight to the workspace: slot =
    // nearer before + kept candidates before
    for (int e = tid; e < TN; e += kBlkThreads) {
      const int pos = e + sh.ctp[min(sh.ncb[e], c)];
      if (pos < k) {
        gidx[pos] = sh.sidx[e];
        gval[pos] = sh.sval[e];
      }
    }
    for (int t = tid; t < c; t += kBlkThreads) {
      if (sh.cflag[t]) {
        const int pos = sh.cnb[t] + sh.ctp[t];
        if (pos < k) {
          gidx[pos] = sh.cidx[t];
          gval[pos] = sh.cval[t];
        }
      }
    }
  }
  if (tid == 0) {
    p.sel_cnt[r] = k;
    if (p.sel_total) p.sel_total[r] = k;
    p.pstar_out[r] = expf(key_to_f32(kth) - M) / S;
  }

  // softmax . V over the entries: weight exp(x - M) (the row max is always
  // kept; 0 for a candidate not kept)
  const int nE = nl + c;
  const int G = tid >> 4;
  const char* vb = vbase + static_cast<int64_t>(tid & 15) * PV::BYTES;
  auto entry_pos = [&](int e) { return e < nl ? sh.sidx[e] : sh.cidx[e - nl]; };
  auto weight = [&](int e) {
    if (e < nl) return __expf(sh.sval[e] - M);
    return sh.cflag[e - nl] ? __expf(sh.cval[e - nl] - M) : 0.f;
  };
  PV pv;
  pv.init();
  pv.m = M;
  u32x4 raw[kPVUnroll][PV::NV];
  for (int e0 = G; e0 < nE; e0 += kPVUnroll * kBlkGroups) {
#pragma unroll
    for (int u = 0; u < kPVUnroll; ++u) {
      const int e = e0 + u * kBlkGroups;
      if (e < nE) PV::load_raw(vb + static_cast<int64_t>(entry_pos(e)) * vrow, raw[u]);
    }
    __builtin_amdgcn_sched_barrier(0);  // all gathers in flight before the FMAs
#pragma unroll
    for (int u = 0; u < kPVUnroll; ++u) {
      const int e = e0 + u * kBlkGroups;
      if (e < nE) {
        const float wt = weight(e);
        float f[PV::DPL];
        PV::unpack(raw[u], f);
#pragma unroll
        for (int i = 0; i < PV::DPL; ++i) pv.acc[i] += wt * f[i];
      }
    }
  }
  float ls = 0.f;
  for (int e = tid; e < nE; e += kBlkThreads) ls += weight(e);
  pv.l = block_sum<kBlkWaves>(ls, sh.red);
  pv.finish(accs, v.out, v.out_dt, ooff, false);
}

template <int DT, int D>
static hipError_t launch_calibrate(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  const dim3 grid(p.nrows), block(kBlkThreads);
  // the row resident in the block, chunks of 4096 positions: up to 13 in
  // registers, 17 with 4 in LDS (a 2048-entry list then leaves room for them)
  if (p.cap <= kRegList && p.L <= 13 * 4096) {
    if (p.L <= 2 * 4096)
      hipLaunchKernelGGL((atopn_calibrate_reg_kernel<DT, D, 2, kRegList>), grid, block, 0, st, p, v);
    else if (p.L <= 4 * 4096)
      hipLaunchKernelGGL((atopn_calibrate_reg_kernel<DT, D, 4, kRegList>), grid, block, 0, st, p, v);
    else if (p.L <= 9 * 4096)
      hipLaunchKernelGGL((atopn_calibrate_reg_kernel<DT, D, 9, kRegList>), grid, block, 0, st, p, v);
    else
      hipLaunchKernelGGL((atopn_calibrate_reg_kernel<DT, D, 13, kRegList>), grid, block, 0, st, p, v);
  } else if (p.cap <= kRegListLong && p.L <= 17 * 4096) {
    hipLaunchKernelGGL((atopn_calibrate_reg_kernel<DT, D, 17, kRegListLong>), grid, block, 0, st, p, v);
  } else {
    hipLaunchKernelGGL((atopn_calibrate_kernel<DT, D>), grid, block, 0, st, p, v);
  }
  return hipGetLastError();
}

template <int DT>
static hipError_t launch_calibrate_d(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  return v.d == 128 ? launch_calibrate<DT, 128>(p, v, st) : launch_calibrate<DT, 64>(p, v, st);
}

hipError_t launch_atopn_select_pv(bool calibrate, const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  if (!calibrate) return launch_atopn_fast(p, v, st);
  // long rows: spread over (row, chunk) blocks
  if (cal_spread(p.L, p.cap, p.nslice, p.slice_cap, p.k2_variant, p.nrows)) return launch_calibrate_spread(p, v, st);
  if (cal_row_block(p.L, p.cap)) return launch_calibrate_row_block(p, v, st);
  if (v.v_dt == SAGA_DTYPE_BF16) return launch_calibrate_d<SAGA_DTYPE_BF16>(p, v, st);
  if (v.v_dt == SAGA_DTYPE_F16) return launch_calibrate_d<SAGA_DTYPE_F16>(p, v, st);
  return launch_calibrate_d<SAGA_DTYPE_F32>(p, v, st);
}

// threshold_topk_fast API (attention/triton_atopn.py:59-113): typed rows,
// per-row / broadcast / repeated thresholds (:87-96), values kept in the
// input dtype, int64 indices, every slot of the k-wide outputs written
// (unfilled: -inf, 0 as the reference pre-fills them, :82-84).
template <int DT>
__global__ void __launch_bounds__(kBlkThreads) select_api_kernel(ApiSelParams p) {
  __shared__ int cnt[kSelSlots];
  __shared__ int pre[kSelSlots + 1];
  using Raw = typename std::conditional<DT == SAGA_DTYPE_F32, uint32_t, uint16_t>::type;
  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const float t = p.thresh[r % p.thresh_numel];
  const int n = static_cast<int>(p.D);
  const Raw* x = static_cast<const Raw*>(p.x) + static_cast<int64_t>(r) * p.x_ld;
  Raw* ov = static_cast<Raw*>(p.out_val) + static_cast<int64_t>(r) * p.ov_ld;
  int64_t* oi = p.out_idx + static_cast<int64_t>(r) * p.oi_ld;
  int base = 0;
  for (int st = 0; st < n; st += kSelTile) {
    Raw xr[kSelEPT];
    unsigned long long bal[kSelEPT];
#pragma unroll
    for (int k = 0; k < kSelEPT; ++k) {
      const int i = st + k * kBlkThreads + tid;
      xr[k] = i < n ? x[i] : Raw(0);
    }
#pragma unroll
    for (int k = 0; k < kSelEPT; ++k) {
      const int i = st + k * kBlkThreads + tid;
      bal[k] = __ballot(i < n && Elt<DT>::to_f32(xr[k]) > t);
      if (lane == 0) cnt[k * kBlkWaves + w] = __popcll(bal[k]);
    }
    __syncthreads();
    if (w == 0) scan_slots(cnt, pre, lane);
    __syncthreads();
    if (base < p.k) {
#pragma unroll
      for (int k = 0; k < kSelEPT; ++k) {
        if ((bal[k] >> lane) & 1ull) {
          const int pos = base + pre[k * kBlkWaves + w] + __popcll(bal[k] & lanes_below(lane));
          if (pos < p.k) {
            oi[pos] = st + k * kBlkThreads + tid;
            ov[pos] = xr[k];
          }
        }
      }
    }
    base += pre[kSelSlots];
    __syncthreads();
  }
  const Raw ninf = DT == SAGA_DTYPE_F32 ? Raw(0xff800000u) : (DT == SAGA_DTYPE_BF16 ? Raw(0xff80u) : Raw(0xfc00u));
  for (int j = min(base, p.k) + tid; j < p.k; j += kBlkThreads) {
    oi[j] = 0;
    ov[j] = ninf;
  }
  if (tid == 0 && p.out_counts) p.out_counts[r] = base;
}

hipError_t launch_select_api(const ApiSelParams& p, hipStream_t st) {
  switch (p.x_dt) {
    case SAGA_DTYPE_F32:
      hipLaunchKernelGGL(select_api_kernel<SAGA_DTYPE_F32>, dim3(p.nrows), dim3(kBlkThreads), 0, st, p);
      break;
    case SAGA_DTYPE_BF16:
      hipLaunchKernelGGL(select_api_kernel<SAGA_DTYPE_BF16>, dim3(p.nrows), dim3(kBlkThreads), 0, st, p);
      break;
    default:
      hipLaunchKernelGGL(select_api_kernel<SAGA_DTYPE_F16>, dim3(p.nrows), dim3(kBlkThreads), 0, st, p);
      break;
  }
  return hipGetLastError();
}

}  // namespace saga

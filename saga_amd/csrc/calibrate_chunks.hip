// Calibration spread over many blocks per row: the exact top-k of each
// chunk of a score row, then the exact top-k of the row among those lists;
// and the same selection with one block per row over a short row's scores.
//
// Replaces torch.topk + the renormalised gather of
// approx_top_n_attention_amortized_cal (attention/attention.py:173-189):
// spread over chunks for rows of more than 36864 positions (and from 16384
// when the rows are few or outnumber the CUs), where one block per row is
// bound by a single CU's memory draw (one CU moves about 25 GB/s: 128 KB of
// scores and 128 KB of V rows take 10 us); one block per row (the row
// kernel's body over the scores themselves) for rows of up to 24576.
//
// Chunk kernel, one block per (row, chunk of C positions): the k largest
// positions of the chunk (k = min(top_n, L); ordered by value, then lowest
// index) in position order, into the chunk's slot of k entries.  The row's
// top-k is a subset of the union of its chunks' top-k (fewer than k
// positions of the row precede one of its top-k in that order, so fewer
// than k of its chunk do), and every full chunk keeps exactly k, so a row's
// entries are one dense list in position order.
//
// Row kernel, one block per row: the row's top-k among the entries (the
// same selection, run over the entries instead of the positions), the kept
// list, p* and softmax . V over the kept entries.
//
// The selection (block_topk): 2048 bins of the distance (M - x) * s below
// the set's max M (s a power of two fitted to the set's spread); the bin of
// the k-th largest splits the set into nearer entries (all kept) and that
// bin's candidates, ranked by (value desc, position asc); a NaN, a
// non-finite max or too many candidates (ties) take a radix select over the
// order-preserving keys instead.  Each thread holds E consecutive entries,
// so an entry's rank within its class is the lower waves' total + one wave
// scan + the thread's own count below it; or, for one block per row, each
// wave holds 64 E consecutive entries quad-interleaved (every 16-byte load
// of the wave reads 1 KB in a row), and a rank takes one wave scan per quad.
#include <algorithm>
#include <type_traits>

#include "kernels.h"
#include "select.cuh"

namespace saga {

constexpr int kSpreadRank = 128;      // candidates ranked pairwise; more: radix select over them
constexpr int kChunkCand = 512;       // chunk kernel: candidates of the k-th's bin held in LDS
constexpr int kMergeCand = 1024;      // row kernel: the same
constexpr int kMergeList = 2048;      // row kernel: kept list in LDS (k <= 2048)
constexpr int kMergeBlocksMax = 256;  // row kernel: past this many rows, 512-thread blocks (two per CU)
constexpr int kSpareBins = 32;        // histogram bins past kNearBins for positions out of range (one per bank)
constexpr uint32_t kPadBits = 0xffffffffu;  // a NaN whose order key is 0: below every other float

// Which of the c candidates sh.cval[0..c) (index order) are among the krem
// largest by (value desc, index asc); returns the key of the krem-th.  At
// most 64 candidates (the usual few): every wave ranks them all, lane t
// candidate t, into the block-uniform mask km (bit t: kept), with no LDS
// writes or barriers.  More (c <= 4 NT): sh.cflag[t], and the kept ones
// before t in sh.ctp[t] (sh.ctp[c] = krem).  CandKept reads either form.
template <int NT, class SH>
__device__ __forceinline__ uint32_t rank_candidates(SH& sh, int c, int krem, uint64_t& km) {
  constexpr int NW = NT / kWave, TPC = NT / kSpreadRank;  // threads per candidate
  const int tid = threadIdx.x;
  uint32_t kth;
  km = 0ull;
  if (c <= kWave) {
    const int lane = tid & 63;
    const bool in = lane < c;
    const uint32_t ki = in ? f32_to_key(sh.cval[lane]) : 0u;
    int rank = 0;
    for (int u = 0; u < c; ++u) {
      const uint32_t ku = f32_to_key(sh.cval[u]);  // (the same address in every lane)
      rank += (ku > ki || (ku == ki && u < lane)) ? 1 : 0;
    }
    km = __ballot(in && rank < krem);
    const uint64_t kb = __ballot(in && rank == krem - 1);  // exactly one lane
    return static_cast<uint32_t>(__shfl(static_cast<int>(ki), __builtin_ctzll(kb)));
  }
  if (c <= kSpreadRank) {
    const int i = tid / TPC, sub = tid % TPC;
    int rank = 0;
    uint32_t ki = 0;
    if (i < c) {
      ki = f32_to_key(sh.cval[i]);
#pragma unroll 4
      for (int u = sub; u < c; u += TPC) {
        const uint32_t ku = f32_to_key(sh.cval[u]);
        rank += (ku > ki || (ku == ki && u < i)) ? 1 : 0;
      }
    }
#pragma unroll
    for (int o = 1; o < TPC; o <<= 1) rank += __shfl_xor(rank, o);
    if (i < c && sub == 0) {
      sh.cflag[i] = rank < krem ? 1 : 0;
      if (rank == krem - 1) sh.sel_key = static_cast<int>(ki);
    }
    lds_sync();
    kth = static_cast<uint32_t>(sh.sel_key);
    int before = 0;
    if (i < c) {
#pragma unroll 4
      for (int u = sub; u < i; u += TPC) before += sh.cflag[u];
    }
#pragma unroll
    for (int o = 1; o < TPC; o <<= 1) before += __shfl_xor(before, o);
    if (i < c && sub == 0) sh.ctp[i] = before;
    if (tid == 0) sh.ctp[c] = krem;
  } else {
    int nd = krem;
    kth = radix_select_each<NT>(sh, nd, [&](auto f) {
      for (int t = tid; t < c; t += NT) f(sh.cval[t]);
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
    const int tb = block_excl_scan4<NW>(ts, sh.scan);
    if (4 * tid < c) {
      sh.ctp[4 * tid] = tb;
      if (4 * tid + 1 <= c) sh.ctp[4 * tid + 1] = tb + tflag[0];
      if (4 * tid + 2 <= c) sh.ctp[4 * tid + 2] = tb + tflag[0] + tflag[1];
      if (4 * tid + 3 <= c) sh.ctp[4 * tid + 3] = tb + tflag[0] + tflag[1] + tflag[2];
      if (4 * tid + 4 <= c) sh.ctp[4 * tid + 4] = ts + tb;
    }
  }
  lds_sync();
  return kth;
}

// Kept flags and kept-before counts of the ranked candidates, from the mask
// (c <= 64) or from LDS.
template <class SH>
struct CandKept {
  const SH& sh;
  int c;
  uint64_t km;
  __device__ __forceinline__ bool kept(int t) const { return c <= kWave ? ((km >> t) & 1ull) != 0ull : sh.cflag[t] != 0; }
  // kept candidates among the first cb (cb <= c)
  __device__ __forceinline__ int before(int cb) const {
    if (c <= kWave) return __popcll(cb >= kWave ? km : (km & ((1ull << cb) - 1ull)));
    return sh.ctp[cb];
  }
};

// Elements past the end of a block's share (the partial last chunk of a
// row, the entries past a row's list) are set to kPadBits: its key is 0, so
// in key order it follows every other value (and, at the highest indices,
// every element equal to it), and as a NaN it takes no distance bin.  The
// selection over the padded share then equals the one over the real
// elements (which number at least k), with no range checks per element.
template <int NQ>
__device__ __forceinline__ void pad_past(f32x4* xr, int lp, int n) {  // xr[u][j]: element lp + 4 u + j
#pragma unroll
  for (int u = 0; u < NQ; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (lp + 4 * u + j >= n) xr[u][j] = __uint_as_float(kPadBits);
}

// The same for the quad-interleaved share (xr[u][j]: element wbase + 256 u +
// 4 lane + j).
template <int NQ>
__device__ __forceinline__ void pad_past_qi(f32x4* xr, int wbase, int lane, int n) {
#pragma unroll
  for (int u = 0; u < NQ; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (wbase + kWave * 4 * u + 4 * lane + j >= n) xr[u][j] = __uint_as_float(kPadBits);
}

// Every element of the share into its distance bin below M; elements out of
// the bins' range (padding, -inf, NaN) into a spare bin, so that no lane
// branches.  sh.hist has kNearBins + kSpareBins entries.
template <int CH, class SH>
__device__ __forceinline__ void near_histogram(SH& sh, const f32x4* xr, float scale, float Ms) {
  const int spare = kNearBins + (threadIdx.x & (kSpareBins - 1));
#pragma unroll
  for (int q = 0; q < CH; ++q) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float dd = fmaf(-xr[q][j], scale, Ms);
      atomicAdd(&sh.hist[dd < static_cast<float>(kNearBins) ? kNearBins - 1 - static_cast<int>(dd) : spare], 1);
    }
  }
}

// Entries per row of the chunk lists: rows are cs apart (a multiple of 4
// entries, for 16-byte loads).
__device__ __forceinline__ int64_t spread_row_stride(const FusedSelParams& p) {
  return static_cast<int64_t>(p.nslice) * p.slice_cap / 4 * 4;
}

// ---------------------------------------------------------------------------
// LDS of the selection: LIST staging slots (+ one spare per lane), CAND
// candidate slots.
template <int NW, int LIST, int CAND>
struct TopkShared {
  static constexpr int kList = LIST;
  float red[2 * NW];
  float red2[NW];
  int cnt[NW];     // hist_pick's per-wave totals
  int wtot[NW];    // per-wave class totals (nearer | candidates << 16)
  int scan[NW];    // NaN flags; block_excl_scan4's per-wave totals
  int hist[kNearBins + kSpareBins];
  int sel_bin, sel_above, sel_cnt, sel_key, last;
  alignas(16) int sidx[LIST + kWave];    // the nearer entries' positions by rank (key classes: the kept list)
  alignas(16) float sval[LIST + kWave];  //   and values (16-byte aligned: read back as vectors)
  float cval[CAND];  // candidates in index order: value,
  int cidx[CAND];    // position,
  int cnb[CAND];     // nearer entries before it,
  int ctp[CAND + 1];  // (more than 64 candidates: kept ones before it,
  int cflag[CAND];    //  kept?)
  int kf[CAND];       // kept candidates: final slot in the list,
  int kix[CAND];      // position,
  float kvl[CAND];    // value
};

// The exact k largest (value desc, position asc) of a set held E per thread
// (thread t: entries t E .. t E + E - 1 of the set, which is in position
// order; QI: wave w holds entries [64 E w, 64 E (w + 1)), its quad u the 256
// entries from 64 E w + 256 u, lane l entries 4 l .. 4 l + 3 of each quad,
// so that every 16-byte load of a wave reads 1 KB in a row; values xr,
// positions pos(i) of the thread's entry i = 4 u + j; entries past the set
// are kPadBits), k <= the set's size <= LIST... for the nearer ones.
// M: the set's max (every value <= M unless near is false), mn: a lower
// bound of its finite values; near (in): M finite and no NaN.  sh.hist must
// be zero and published.  Out, published: near mode (near true): nl nearer
// entries in sh.sidx / sval by rank, nk kept candidates in sh.kf / kix / kvl
// (kf ascending); key mode: the k kept entries in sh.sidx / sval in order
// (nl = k, nk = 0).  Returns the k-th largest's key.
template <int NT, int E, bool QI = false, class SH, class POS>
__device__ __forceinline__ uint32_t block_topk(SH& sh, f32x4 (&xr)[E / 4], POS pos, int k, float M, float mn,
                                                bool& near, int& nl, int& nk) {
  constexpr int NW = NT / kWave, NQ = E / 4, LIST = SH::kList;
  constexpr int CAND = sizeof(sh.kf) / sizeof(int);
  static_assert(E % 4 == 0 && E <= 64 && NT * E < 65536, "class counts are packed in 16 bits");
  using MT = typename std::conditional<(E > 32), uint64_t, uint32_t>::type;  // one bit per entry of the thread
  auto popc = [](MT m) -> int {
    if constexpr (sizeof(MT) == 8) return __popcll(m);
    else return __popc(m);
  };
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  auto each_in = [&](auto f) {
#pragma unroll
    for (int u = 0; u < NQ; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) f(xr[u][j]);
  };
  const float scale = near_bin_scale(M, mn), Ms = M * scale;
  int bin = -1, above = 0;
  if (near) {  // (block-uniform)
    near_histogram<NQ>(sh, xr, scale, Ms);  // (dd >= 0: every value <= M)
    lds_sync();
    int bcnt;
    hist_pick<NT>(sh, kNearBins, k, bin, above, bcnt);
    near = bin >= 0 && bcnt <= CAND;  // block-uniform
  }
  int krem = k;
  uint32_t kth = 0;
  float wantf = 0.f;
  if (near) {
    krem = k - above;
    wantf = static_cast<float>(kNearBins - 1 - bin);
  } else {
    kth = radix_select_each<NT>(sh, krem, each_in);  // krem -> keys equal to kth that are kept
  }
  const int need = krem;

  // classes: the thread's E-bit masks of nearer / candidate entries
  MT mN = 0, mC = 0;
  if (near) {
    // the distances again (the same bits); an opaque copy of the scale keeps
    // the compiler from holding the histogram pass's ones in registers
    float sc2 = scale;
    asm volatile("" : "+v"(sc2));
    const float wantf1 = wantf + 1.f;
#pragma unroll
    for (int u = 0; u < NQ; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float dd = fmaf(-xr[u][j], sc2, Ms);
        mN |= MT(dd < wantf ? 1 : 0) << (4 * u + j);
        mC |= MT(dd < wantf1 ? 1 : 0) << (4 * u + j);
      }
    mC &= ~mN;
  } else {
#pragma unroll
    for (int u = 0; u < NQ; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t key = f32_to_key(xr[u][j]);
        mN |= MT(key > kth ? 1 : 0) << (4 * u + j);
        mC |= MT(key == kth ? 1 : 0) << (4 * u + j);
      }
  }
  // ranks: the lower waves' totals + the lower lanes' (one packed scan, nearer
  // | candidates << 16; a class of the block holds fewer than 65536
  // entries); QI: one scan per quad, whose wave totals precede the next quad
  const int cntv = popc(mN) | (popc(mC) << 16);
  int qpre[QI ? NQ : 1];  // QI: entries of the wave before the lane's entries of quad u (packed)
  int incl = 0;
  if constexpr (QI) {
    int run = 0;  // (wave-uniform)
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int c = __popc(static_cast<uint32_t>(mN >> (4 * u)) & 15u) |
                    (__popc(static_cast<uint32_t>(mC >> (4 * u)) & 15u) << 16);
      const int inc = wave_incl_scan(c, lane);
      qpre[u] = run + inc - c;
      run += __builtin_amdgcn_readlane(inc, kWave - 1);
    }
    incl = run;
  } else {
    incl = wave_incl_scan(cntv, lane);
  }
  if (lane == kWave - 1) sh.wtot[w] = incl;
  lds_sync();
  int WB = 0, TT = 0;
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    const int t = sh.wtot[u];
    if (u < w) WB += t;
    TT += t;
  }
  const int pre = WB + incl - cntv;
  const int nb0 = pre & 0xffff, cb0 = pre >> 16;  // nearer / candidates before the thread's first entry
  // QI: nearer / candidates before entry i of the thread, in set order
  auto before_n = [&](int i) -> int {
    return ((WB + qpre[QI ? i >> 2 : 0]) & 0xffff) +
           __popc(static_cast<uint32_t>(mN >> (i & ~3)) & ((1u << (i & 3)) - 1u));
  };
  auto before_c = [&](int i) -> int {
    return ((WB + qpre[QI ? i >> 2 : 0]) >> 16) +
           __popc(static_cast<uint32_t>(mC >> (i & ~3)) & ((1u << (i & 3)) - 1u));
  };

  if (near) {
    const int c = TT >> 16;  // == the bin's count <= CAND
    nl = TT & 0xffff;        // (== k - krem)
    nk = krem;
    if (__ballot(mC != 0) != 0ull) {  // (wave-uniform) the candidates to LDS in index order
#pragma unroll
      for (int i = 0; i < E; ++i) {
        if (__ballot((mC >> i) & 1) != 0ull && ((mC >> i) & 1)) {
          const MT below = (MT(1) << i) - 1;
          const int cb = QI ? before_c(i) : cb0 + popc(mC & below);
          sh.cval[cb] = xr[i >> 2][i & 3];
          sh.cidx[cb] = pos(i);
          sh.cnb[cb] = QI ? before_n(i) : nb0 + popc(mN & below);
        }
      }
    }
    int slot = nb0;  // the nearer entries by rank (the thread's others to its lane's spare slot)
#pragma unroll
    for (int i = 0; i < E; ++i) {
      if (QI && (i & 3) == 0) slot = before_n(i);
      const int n = static_cast<int>((mN >> i) & 1);
      const int at = n ? slot : LIST + lane;
      sh.sidx[at] = pos(i);
      sh.sval[at] = xr[i >> 2][i & 3];
      slot += n;
    }
    lds_sync();
    uint64_t km;
    kth = rank_candidates<NT>(sh, c, krem, km);
    const CandKept<SH> ck{sh, c, km};
    for (int t = tid; t < c; t += NT) {  // the kept candidates at their final slots
      if (ck.kept(t)) {
        const int kt = ck.before(t);
        sh.kf[kt] = sh.cnb[t] + kt;
        sh.kix[kt] = sh.cidx[t];
        sh.kvl[kt] = sh.cval[t];
      }
    }
  } else {
    nl = k;
    nk = 0;
    // key classes: above the k-th key, and the first `need` equal to it
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const MT below = (MT(1) << i) - 1;
      const int cb = QI ? before_c(i) : cb0 + popc(mC & below);
      const bool kept = ((mN >> i) & 1) || (((mC >> i) & 1) && cb < need);
      const int at = kept ? (QI ? before_n(i) : nb0 + popc(mN & below)) + min(cb, need) : LIST + lane;
      sh.sidx[at] = pos(i);
      sh.sval[at] = xr[i >> 2][i & 3];
    }
  }
  lds_sync();
  return kth;
}

// The kept list of block_topk in position order, coalesced: slot o holds the
// kept candidate whose final slot is o, else nearer entry o - (kept
// candidates before o).
template <int NT, class SH>
__device__ __forceinline__ void write_list(const SH& sh, int k, int nk, int32_t* oidx, float* oval) {
  for (int o = threadIdx.x; o < k; o += NT) {
    int lo = 0, hi = nk;  // the kept candidates with final slot <= o: [0, lo)
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (sh.kf[mid] <= o) lo = mid + 1;
      else hi = mid;
    }
    if (lo > 0 && sh.kf[lo - 1] == o) {
      oidx[o] = sh.kix[lo - 1];
      oval[o] = sh.kvl[lo - 1];
    } else {
      oidx[o] = sh.sidx[o - lo];
      oval[o] = sh.sval[o - lo];
    }
  }
}

// Chunk kernel: NT threads hold the chunk's C = NT * E positions, E
// consecutive per thread (E / 4 16-byte loads).
constexpr int chunk_waves_per_simd(int NT, int E) { return E > 16 ? 4 : (NT >= 512 ? 8 : 5); }

template <int NT, int E>
__global__ void __launch_bounds__(NT, chunk_waves_per_simd(NT, E)) atopn_cal_chunk_kernel(FusedSelParams p) {
  constexpr int NW = NT / kWave, C = NT * E, NQ = E / 4;
  constexpr int KEEP = C / 16;  // kept per chunk at most (k <= C / 16)
  static_assert(E % 4 == 0 && E <= 32, "4 to 32 positions per thread, in 16-byte loads");
  __shared__ TopkShared<NW, KEEP, kChunkCand> sh;
  const int r = blockIdx.x, ck = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int bi = r / p.q_h;
  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  const int base = ck * C;
  const int nv = min(Leff - base, C);  // positions of the chunk inside the row
  if (nv <= 0) return;
  const int64_t cs = spread_row_stride(p);
  int32_t* oidx = p.sl_idx + r * cs + static_cast<int64_t>(ck) * p.cap;
  float* oval = p.sl_val + r * cs + static_cast<int64_t>(ck) * p.cap;
  const float* x = p.scores + static_cast<int64_t>(r) * p.ld + base;
  if (nv <= p.cap) {  // (the row's last chunk) every position is kept
    for (int e = tid; e < nv; e += NT) {
      oidx[e] = base + e;
      oval[e] = x[e];
    }
    return;
  }
  const int kc = p.cap;  // < nv

  const int lp = tid * E;                   // the thread's first position in the chunk
  const int lastq = (nv + 3) / 4 * 4 - 4;   // loads past nv are clamped (and never used)
  f32x4 xr[NQ];
#pragma unroll
  for (int u = 0; u < NQ; ++u) xr[u] = *reinterpret_cast<const f32x4*>(x + min(lp + 4 * u, lastq));
  for (int i = tid; i < kNearBins + kSpareBins; i += NT) sh.hist[i] = 0;
  auto each_in = [&](auto f) {
#pragma unroll
    for (int u = 0; u < NQ; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) f(xr[u][j]);
  };

  // a NaN among the chunk's positions, before the row's last chunk is padded
  bool odd = false;
  if (nv < C) {  // (block-uniform)
#pragma unroll
    for (int u = 0; u < NQ; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) odd = odd || (lp + 4 * u + j < nv && xr[u][j] != xr[u][j]);
    pad_past<NQ>(xr, lp, nv);
  } else {
    each_in([&](float xi) { odd = odd || xi != xi; });
  }
  // the chunk's max and min (NaN aside; one barrier, which also publishes
  // the zeroed histogram)
  float mx = kNegInf, mnl = INFINITY;
  each_in([&](float xi) {
    mx = fmaxf(mx, xi);
    mnl = fminf(mnl, xi);
  });
  mx = wave_max(mx);
  mnl = -wave_max(-mnl);
  const int wodd = __ballot(odd) != 0ull ? 1 : 0;
  if (lane == 0) {
    sh.red[w] = mx;
    sh.red[NW + w] = mnl;
    sh.scan[w] = wodd;
  }
  lds_sync();
  float M = sh.red[0], mn = sh.red[NW];
  int anyodd = sh.scan[0];
#pragma unroll
  for (int u = 1; u < NW; ++u) {
    M = fmaxf(M, sh.red[u]);
    mn = fminf(mn, sh.red[NW + u]);
    anyodd |= sh.scan[u];
  }
  bool near = !anyodd && M > kNegInf && M < INFINITY;  // block-uniform
  if (near && !(mn > kNegInf)) {  // (block-uniform) masked positions: the smallest finite value
    float m2 = INFINITY;
    each_in([&](float xi) { m2 = fminf(m2, xi > kNegInf ? xi : INFINITY); });
    mn = -block_max<NW>(-m2, sh.red2);
  }
  int nl = 0, nk = 0;
  block_topk<NT, E>(sh, xr, [&](int i) { return base + lp + i; }, kc, M, mn, near, nl, nk);
  write_list<NT>(sh, kc, nk, oidx, oval);
}

// Row body, one block per row: NT threads hold up to NT * E entries (value,
// position), E per thread: LISTS, of the row's chunk lists; else the row's
// scores themselves, positions implicit.  The kept entries (the nearer ones
// by rank, then the kept candidates) are the row's softmax . V.
template <int NW, int D>
struct RowShared {
  TopkShared<NW, kMergeList, kMergeCand> t;
  float accs[NW * D];
};

template <int DT, int D, int NT, int E, bool LISTS>
__device__ __forceinline__ void cal_row_body(const FusedSelParams& p, const PVParams& v,
                                             RowShared<NT / kWave, D>& shr) {
  constexpr int NW = NT / kWave, NG = NT / 16, NQ = E / 4;
  static_assert(E % 4 == 0 && E <= 64, "4 to 64 entries per thread, in 16-byte loads");
  auto& sh = shr.t;
  float* accs = shr.accs;
  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int bi = r / p.q_h, h = r - bi * p.q_h;
  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  const float* prow_m = p.pmax + static_cast<int64_t>(r) * p.nparts;
  const float* prow_s = p.psum + static_cast<int64_t>(r) * p.nparts;
  const int nch = p.nparts;  // parts past kv_len hold (-inf, 0)
  int T = Leff;  // entries: the row's positions, or
  const float* ev = p.scores + static_cast<int64_t>(r) * p.ld;
  const int32_t* ei = nullptr;
  if constexpr (LISTS) {  // the entries of its chunk lists
    const int C = p.cal_chunk;
    T = Leff / C * p.cap + min(p.cap, Leff % C);
    const int64_t cs = spread_row_stride(p);
    ev = p.sl_val + r * cs;
    ei = p.sl_idx + r * cs;
  }

  // K1's partials first, then the entries: their loads stay in flight
  // through the max / sum reductions
  const float pm0 = tid < nch ? prow_m[tid] : kNegInf;
  const float ps0 = tid < nch ? prow_s[tid] : 0.f;
  // the entries: E consecutive per thread from the chunk lists; the score
  // row quad-interleaved (wave w: entries [wbase, wbase + 64 E), quad u the
  // 256 from wbase + 256 u, lane l 4 of each), every load 1 KB in a row
  constexpr bool QI = !LISTS;
  const int lp = tid * E;  // the thread's first entry (E consecutive)
  const int wbase = w * kWave * E;
  auto entry = [&](int u) { return QI ? wbase + kWave * 4 * u + 4 * lane : lp + 4 * u; };
  const int lastq = max(0, (T + 3) / 4 * 4 - 4);
  f32x4 xr[NQ];
  i32x4 ir[LISTS ? NQ : 1];
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int o = min(entry(u), lastq);
    xr[u] = *reinterpret_cast<const f32x4*>(ev + o);
    if constexpr (LISTS) ir[u] = *reinterpret_cast<const i32x4*>(ei + o);
  }
  for (int i = tid; i < kNearBins + kSpareBins; i += NT) sh.hist[i] = 0;
  float mloc = pm0;
  for (int c = tid + NT; c < nch; c += NT) mloc = fmaxf(mloc, prow_m[c]);
  const float M = block_max<NW>(mloc, sh.red);  // (its barriers also publish the zeroed histogram)
  float sloc = pm0 != kNegInf ? ps0 * __expf(pm0 - M) : 0.f;
  for (int c = tid + NT; c < nch; c += NT) {
    const float pm = prow_m[c];
    if (pm != kNegInf) sloc += prow_s[c] * __expf(pm - M);
  }
  const float S = block_sum<NW>(sloc, sh.red);

  const int k = min(p.cap, Leff);
  int32_t* gidx = p.sel_idx + static_cast<int64_t>(r) * p.cap;
  float* gval = p.sel_val + static_cast<int64_t>(r) * p.cap;
  using PV = BlockPV<DT, D, NT>;
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

  if (T < NT * E) {  // (block-uniform)
    if constexpr (QI) pad_past_qi<NQ>(xr, wbase, lane, T);
    else pad_past<NQ>(xr, lp, T);
  }
  // the smallest entry and a NaN entry or one above M (padding aside; one barrier)
  float mnl = INFINITY;
  bool odd = false;
#pragma unroll
  for (int u = 0; u < NQ; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float xi = xr[u][j];
      mnl = fminf(mnl, xi);  // (ignores NaN)
      odd = odd || (xi != xi && __float_as_uint(xi) != kPadBits) || xi > M;
    }
  mnl = -wave_max(-mnl);
  const int wodd = __ballot(odd) != 0ull ? 1 : 0;
  if (lane == 0) {
    sh.red2[w] = mnl;
    sh.scan[w] = wodd;
  }
  lds_sync();
  float mn = sh.red2[0];
  int anyodd = sh.scan[0];
#pragma unroll
  for (int u = 1; u < NW; ++u) {
    mn = fminf(mn, sh.red2[u]);
    anyodd |= sh.scan[u];
  }
  bool near = !anyodd && M > kNegInf && M < INFINITY;  // block-uniform
  if (near && !(mn > kNegInf)) {  // (block-uniform) masked positions: the smallest finite entry
    float m2 = INFINITY;
#pragma unroll
    for (int u = 0; u < NQ; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) m2 = fminf(m2, xr[u][j] > kNegInf ? xr[u][j] : INFINITY);
    mn = -block_max<NW>(-m2, sh.red);
  }
  int nl = 0, nk = 0;
  const uint32_t kth = block_topk<NT, E, QI>(
      sh, xr, [&](int i) { return LISTS ? ir[LISTS ? i >> 2 : 0][i & 3] : entry(i >> 2) + (i & 3); }, k, M, mn, near,
      nl, nk);
  write_list<NT>(sh, k, nk, gidx, gval);
  if (tid == 0) {
    p.sel_cnt[r] = k;
    if (p.sel_total) p.sel_total[r] = k;
    p.pstar_out[r] = expf(key_to_f32(kth) - M) / S;
  }

  // softmax . V over the kept entries [0, nl + nk), weight exp(x - M) (the
  // row max is always kept).  One block gathers the row's V rows: splitting
  // them over several blocks per row (each repeating the selection, the last
  // one adding the shares after an agent-scope fence) measured slower
  // wherever it applied (b8 x 32769: 17.4 against 12.6 us)
  const int e0 = 0, e1 = nl + nk;
  const int grp = tid >> 4;
  const char* vb = vbase + static_cast<int64_t>(tid & 15) * PV::BYTES;
  auto entry_pos = [&](int e) { return e < nl ? sh.sidx[e] : sh.kix[e - nl]; };
  auto weight = [&](int e) { return __expf((e < nl ? sh.sval[e] : sh.kvl[e - nl]) - M); };
  PV pv;
  pv.init();
  pv.m = M;
  u32x4 raw[kPVUnroll][PV::NV];
  for (int ea = e0 + grp; ea < e1; ea += kPVUnroll * NG) {
#pragma unroll
    for (int u = 0; u < kPVUnroll; ++u) {
      const int e = ea + u * NG;
      if (e < e1) PV::load_raw(vb + static_cast<int64_t>(entry_pos(e)) * vrow, raw[u]);
    }
    __builtin_amdgcn_sched_barrier(0);  // all gathers in flight before the FMAs
#pragma unroll
    for (int u = 0; u < kPVUnroll; ++u) {
      const int e = ea + u * NG;
      if (e < e1) {
        const float wt = weight(e);
        float f[PV::DPL];
        PV::unpack(raw[u], f);
#pragma unroll
        for (int i = 0; i < PV::DPL; ++i) pv.acc[i] += wt * f[i];
      }
    }
  }
  float ls = 0.f;
  for (int e = e0 + tid; e < e1; e += NT) ls += weight(e);
  pv.l = block_sum<NW>(ls, sh.red);
  pv.finish(accs, v.out, v.out_dt, ooff, false);
}

template <int DT, int D, int NT, int E>
__global__ void __launch_bounds__(NT) atopn_cal_merge_kernel(FusedSelParams p, PVParams v) {
  __shared__ RowShared<NT / kWave, D> sh;
  cal_row_body<DT, D, NT, E, true>(p, v, sh);
}

// One block per row over the row's scores (rows of at most 1024 * 36
// positions, k <= 2048).
template <int DT, int D, int E>
__global__ void __launch_bounds__(kBlkThreads) atopn_cal_row_kernel(FusedSelParams p, PVParams v) {
  __shared__ RowShared<kBlkWaves, D> sh;
  cal_row_body<DT, D, kBlkThreads, E, false>(p, v, sh);
}

// ---------------------------------------------------------------------------
// Shapes: positions per chunk C = 4096 for k <= 256, then 8192, 16384 and
// 32768 up to k = 2048 (a chunk keeps at most 1/16 of itself); the row
// kernel holds up to 8 * 4096 entries.
static int spread_chunk(int64_t cap) {
  return cap <= 256 ? 4096 : (cap <= 512 ? 8192 : (cap <= 1024 ? 16384 : 32768));
}

bool cal_spread(int64_t L, int64_t cap, int64_t nslice, int64_t slice_cap, int variant, int64_t nrows) {
  if (variant == kK2RowBlock || cap > kMergeList || cap < 1) return false;
  // by shape: rows past one block per row's 36864 positions (measured: 27.1
  // against 43.9 us at b8 x 65537, 23.2 against 77.9 at b1 x 131073; at
  // 32769 positions one block per row is ahead at b8, 21.7 against 22.7 us),
  // and from 16384 positions when the rows are few (at most 24: 19.1-19.8
  // against 20.7-21.8 us at b1 x 32769) or more than the CUs (29.8 against
  // 36.7 us at b32 x 16385, 41.4 against 49.7 at b32 x 32769; one block per
  // row ahead at b16 x 16385, 19.1 against 24.2)
  const bool by_rows = nrows <= kCalSpreadFewRows || nrows > kCalSpreadManyRows;
  if (variant == kK2Auto && L <= kCalSpreadAutoLen && !(L >= kCalSpreadFewRowsLen && by_rows)) return false;
  const int64_t C = spread_chunk(cap);
  if (L < 2 * C) return false;
  const int64_t slots = (L + C - 1) / C * cap;  // chunk slots of the longest row
  return slots <= 8 * 4096 && slots <= nslice * slice_cap / 4 * 4;
}

template <int DT, int D>
static hipError_t launch_spread(FusedSelParams p, const PVParams& v, hipStream_t st) {
  const int C = spread_chunk(p.cap);
  p.cal_chunk = C;
  const int nck = (p.L + C - 1) / C;
  const dim3 ga(p.nrows, nck);
  if (C == 4096)
    hipLaunchKernelGGL((atopn_cal_chunk_kernel<256, 16>), ga, dim3(256), 0, st, p);
  else if (C == 8192)
    hipLaunchKernelGGL((atopn_cal_chunk_kernel<512, 16>), ga, dim3(512), 0, st, p);
  else if (C == 16384)
    hipLaunchKernelGGL((atopn_cal_chunk_kernel<1024, 16>), ga, dim3(1024), 0, st, p);
  else
    hipLaunchKernelGGL((atopn_cal_chunk_kernel<1024, 32>), ga, dim3(1024), 0, st, p);
  // entries of the longest row: full chunks keep cap, the last min(cap, rest)
  const int64_t tmax = static_cast<int64_t>(p.L / C) * p.cap + std::min<int64_t>(p.cap, p.L % C);
  const dim3 gb(p.nrows);
  // more rows than CUs: 512-thread blocks, two per CU, while their share of
  // the entries stays in registers
  if (p.nrows > kMergeBlocksMax && tmax <= 16 * 512) {
    const dim3 blk(512);
    if (tmax <= 4 * 512)
      hipLaunchKernelGGL((atopn_cal_merge_kernel<DT, D, 512, 4>), gb, blk, 0, st, p, v);
    else if (tmax <= 8 * 512)
      hipLaunchKernelGGL((atopn_cal_merge_kernel<DT, D, 512, 8>), gb, blk, 0, st, p, v);
    else if (tmax <= 12 * 512)
      hipLaunchKernelGGL((atopn_cal_merge_kernel<DT, D, 512, 12>), gb, blk, 0, st, p, v);
    else
      hipLaunchKernelGGL((atopn_cal_merge_kernel<DT, D, 512, 16>), gb, blk, 0, st, p, v);
    return hipGetLastError();
  }
  const dim3 blk(kBlkThreads);
  if (tmax <= 4 * 1024)
    hipLaunchKernelGGL((atopn_cal_merge_kernel<DT, D, 1024, 4>), gb, blk, 0, st, p, v);
  else if (tmax <= 8 * 1024)
    hipLaunchKernelGGL((atopn_cal_merge_kernel<DT, D, 1024, 8>), gb, blk, 0, st, p, v);
  else if (tmax <= 12 * 1024)
    hipLaunchKernelGGL((atopn_cal_merge_kernel<DT, D, 1024, 12>), gb, blk, 0, st, p, v);
  else if (tmax <= 16 * 1024)
    hipLaunchKernelGGL((atopn_cal_merge_kernel<DT, D, 1024, 16>), gb, blk, 0, st, p, v);
  else if (tmax <= 24 * 1024)
    hipLaunchKernelGGL((atopn_cal_merge_kernel<DT, D, 1024, 24>), gb, blk, 0, st, p, v);
  else
    hipLaunchKernelGGL((atopn_cal_merge_kernel<DT, D, 1024, 32>), gb, blk, 0, st, p, v);
  return hipGetLastError();
}

template <int DT>
static hipError_t launch_spread_d(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  return v.d == 128 ? launch_spread<DT, 128>(p, v, st) : launch_spread<DT, 64>(p, v, st);
}

bool cal_row_block(int64_t L, int64_t cap) { return cap >= 1 && cap <= kMergeList && L <= kCalRowBlockLen; }

template <int DT, int D>
static hipError_t launch_row_block(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  // the fewest whole quads per wave that hold the row: a context of a power
  // of two plus the decoded tokens (8193, 16385, 32769) takes one more quad,
  // not the next power of two's share
  const dim3 grid(p.nrows), blk(kBlkThreads);
  switch ((p.L + 4095) / 4096) {
    case 0:
    case 1:
    case 2: hipLaunchKernelGGL((atopn_cal_row_kernel<DT, D, 8>), grid, blk, 0, st, p, v); break;
    case 3: hipLaunchKernelGGL((atopn_cal_row_kernel<DT, D, 12>), grid, blk, 0, st, p, v); break;
    case 4: hipLaunchKernelGGL((atopn_cal_row_kernel<DT, D, 16>), grid, blk, 0, st, p, v); break;
    case 5: hipLaunchKernelGGL((atopn_cal_row_kernel<DT, D, 20>), grid, blk, 0, st, p, v); break;
    case 6: hipLaunchKernelGGL((atopn_cal_row_kernel<DT, D, 24>), grid, blk, 0, st, p, v); break;
    case 7: hipLaunchKernelGGL((atopn_cal_row_kernel<DT, D, 28>), grid, blk, 0, st, p, v); break;
    case 8: hipLaunchKernelGGL((atopn_cal_row_kernel<DT, D, 32>), grid, blk, 0, st, p, v); break;
    default: hipLaunchKernelGGL((atopn_cal_row_kernel<DT, D, 36>), grid, blk, 0, st, p, v); break;
  }
  return hipGetLastError();
}

template <int DT>
static hipError_t launch_row_block_d(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  return v.d == 128 ? launch_row_block<DT, 128>(p, v, st) : launch_row_block<DT, 64>(p, v, st);
}

hipError_t launch_calibrate_row_block(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  if (v.v_dt == SAGA_DTYPE_BF16) return launch_row_block_d<SAGA_DTYPE_BF16>(p, v, st);
  if (v.v_dt == SAGA_DTYPE_F16) return launch_row_block_d<SAGA_DTYPE_F16>(p, v, st);
  return launch_row_block_d<SAGA_DTYPE_F32>(p, v, st);
}

hipError_t launch_calibrate_spread(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  if (v.v_dt == SAGA_DTYPE_BF16) return launch_spread_d<SAGA_DTYPE_BF16>(p, v, st);
  if (v.v_dt == SAGA_DTYPE_F16) return launch_spread_d<SAGA_DTYPE_F16>(p, v, st);
  return launch_spread_d<SAGA_DTYPE_F32>(p, v, st);
}

}  // namespace saga

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

#include "block_pv.cuh"
#include "kernels.h"

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

__device__ __forceinline__ unsigned long long lanes_below(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (kWave - lane));
}

struct SelShared {
  float red[kBlkWaves];
  int cnt[kSelSlots];
  int pre[kSelSlots + 1];
  int cntE[kSelSlots];
  int preE[kSelSlots + 1];
  int hist[2048];
  int sel_bin, sel_above;
  int sidx[kListLDS];
  float sval[kListLDS];
};

// Run the PV phase over a row's list: from LDS when it fits, otherwise in
// LDS-sized batches re-read from the workspace copy.
template <int DT, int D>
__device__ void row_pv(SelShared& sh, float* accs, int n, const int32_t* gidx, const float* gval, const PVParams& v,
                       int bi, int h, bool probs) {
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

// Bin holding the krem-th largest element of sh.hist[0..nb) (bin nb - 1 holds
// the largest) and the count in the bins above it; bin -1 if fewer than krem
// elements are counted.  Every thread of the block calls it.
__device__ __forceinline__ void hist_pick(SelShared& sh, int nb, int krem, int& bin, int& above) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (tid == 0) sh.sel_bin = -1;
  // bins scanned from the top: thread t owns bins nb-1-2t and nb-2-2t
  const int b0 = nb - 1 - 2 * tid, b1 = b0 - 1;
  const int c0 = b0 >= 0 ? sh.hist[b0] : 0;
  const int c1 = b1 >= 0 ? sh.hist[b1] : 0;
  const int tsum = c0 + c1;
  const int incl = wave_incl_scan(tsum, lane);
  if (lane == kWave - 1) sh.cnt[w] = incl;
  __syncthreads();
  int woff = 0;
  for (int i = 0; i < w; ++i) woff += sh.cnt[i];
  const int ex = woff + incl - tsum;
  if (c0 > 0 && ex < krem && krem <= ex + c0) {
    sh.sel_bin = b0;
    sh.sel_above = ex;
  } else if (c1 > 0 && ex + c0 < krem && krem <= ex + tsum) {
    sh.sel_bin = b1;
    sh.sel_above = ex + c0;
  }
  __syncthreads();
  bin = sh.sel_bin;
  above = sh.sel_above;
  __syncthreads();
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

// The krem-th largest of n keys -- of the score row x (ROW) or of the LDS
// candidates sh.sval -- by a 3-pass radix select (11/11/10 bits of the
// order-preserving uint32 key) over 2048-bin LDS histograms; krem is left at
// the count of elements equal to it that are among the krem largest.
template <bool ROW>
__device__ __forceinline__ uint32_t radix_select(SelShared& sh, const float* x, int64_t ld, int n, int& krem) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0;
  const int shifts[3] = {21, 10, 0};
  const int nbits[3] = {11, 11, 10};
#pragma unroll
  for (int pass = 0; pass < 3; ++pass) {
    const int nb = 1 << nbits[pass];
    const uint32_t hmask = pass == 0 ? 0u : (0xffffffffu << (shifts[pass] + nbits[pass]));
    for (int i = tid; i < 2048; i += kBlkThreads) sh.hist[i] = 0;
    __syncthreads();
    auto count = [&](float xi) {
      const uint32_t key = f32_to_key(xi);
      if ((key & hmask) == prefix) atomicAdd(&sh.hist[(key >> shifts[pass]) & (nb - 1)], 1);
    };
    if constexpr (ROW) {
      row_tiles(x, ld, n, count);
    } else {
      for (int i = tid; i < n; i += kBlkThreads) count(sh.sval[i]);
    }
    __syncthreads();
    int bin, above;
    hist_pick(sh, nb, krem, bin, above);
    prefix |= static_cast<uint32_t>(bin) << shifts[pass];
    krem -= above;
  }
  return prefix;
}

constexpr int kNearBins = 2048;      // bins of the distance below the row max
constexpr float kNearScale = 32.0f;  // bins per unit of logit: the bins span M - 64 .. M

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
__device__ __forceinline__ bool near_pick(SelShared& sh, const float* x, int64_t ld, int Leff, float M, int& krem,
                                          uint32_t& kth) {
  const int tid = threadIdx.x;
  if (!(M > -INFINITY && M < INFINITY)) return false;  // block-uniform
  for (int i = tid; i < kNearBins; i += kBlkThreads) sh.hist[i] = 0;
  __syncthreads();
  int odd = 0;
  row_tiles(x, ld, Leff, [&](float xi) {
    if (!(xi <= M)) {  // NaN
      odd = 1;
      return;
    }
    const float dd = (M - xi) * kNearScale;
    if (dd < kNearBins) atomicAdd(&sh.hist[kNearBins - 1 - static_cast<int>(dd)], 1);
  });
  if (__syncthreads_or(odd)) return false;
  int bin, above;
  hist_pick(sh, kNearBins, krem, bin, above);
  if (bin < 0) return false;
  const int c = sh.hist[bin];
  if (c > kListLDS) return false;
  const int want = kNearBins - 1 - bin;  // distance bin of the candidates
  if (tid == 0) sh.sel_bin = 0;          // candidate count
  __syncthreads();
  row_tiles(x, ld, Leff, [&](float xi) {
    const float dd = (M - xi) * kNearScale;
    if (dd < kNearBins && static_cast<int>(dd) == want) sh.sval[atomicAdd(&sh.sel_bin, 1)] = xi;
  });
  __syncthreads();
  krem -= above;
  kth = radix_select<false>(sh, nullptr, 0, c, krem);
  return true;
}

// Calibration: exact top-k of the row (k = min(top_n, L)).
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

  // Ordered compaction, tile by tile: wave w takes the kSelEPT * 64
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
    __syncthreads();
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
    __syncthreads();
  }
  if (tid == 0) {
    p.sel_cnt[r] = k;
    if (p.sel_total) p.sel_total[r] = k;
    p.pstar_out[r] = expf(key_to_f32(kth) - M) / S;
  }
  row_pv<DT, D>(sh, accs, k, gidx, gval, v, bi, h, false);
}

template <int DT, int D>
static hipError_t launch_calibrate(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  hipLaunchKernelGGL((atopn_calibrate_kernel<DT, D>), dim3(p.nrows), dim3(kBlkThreads), 0, st, p, v);
  return hipGetLastError();
}

template <int DT>
static hipError_t launch_calibrate_d(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  return v.d == 128 ? launch_calibrate<DT, 128>(p, v, st) : launch_calibrate<DT, 64>(p, v, st);
}

hipError_t launch_atopn_select_pv(bool calibrate, const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  if (!calibrate) return launch_atopn_fast(p, v, st);
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

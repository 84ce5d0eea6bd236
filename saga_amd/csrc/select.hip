// K2: Atop-N selection kernels (one 1024-thread block per score row).
//
// Replaces the Triton stream compaction threshold_select_fast_kernel
// (attention/triton_atopn.py:6-53) and, for calibration, torch.topk over the
// softmax (attention/attention.py:179-187).  The compaction is ordered and
// deterministic: a row is processed in super-tiles of 1024 x 16 elements;
// each wave turns its pass flags into 64-bit ballots, wave counts are
// prefix-summed in LDS in (element-slot, wave) order -- which is ascending
// index order -- and every passing element is written to
// base + prefix + popcount(ballot & lanes_below).  The result is the list of
// passing positions in ascending order; past `cap` entries nothing is
// written (the reference's atomic-order output keeps a race-dependent
// subset there).
#include "common.cuh"
#include "kernels.h"

namespace saga {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / kWave;      // 16
constexpr int kSelEPT = 16;                         // elements per thread per super-tile
constexpr int kSelSlots = kSelEPT * kSelWaves;      // 256 (slot, wave) counters
constexpr int kSelTile = kSelThreads * kSelEPT;     // 16384 elements

static_assert(kSelSlots == 4 * kWave, "wave-0 scan handles 4 counters per lane");

// Exclusive scan of cnt[0..256) into pre[0..256], pre[256] = total (wave 0).
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

// Ordered compaction of {i < n : v(i) > t}; emit(pos, i, v) for pos < cap.
// Returns the number of passing elements (before the cap).
template <class LoadF, class EmitF>
__device__ int ordered_compact(int n, float t, int cap, LoadF load, EmitF emit, int* cnt, int* pre) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int base = 0;
  for (int st = 0; st < n; st += kSelTile) {
    float xv[kSelEPT];
    unsigned long long bal[kSelEPT];
#pragma unroll
    for (int k = 0; k < kSelEPT; ++k) {
      const int i = st + k * kSelThreads + tid;
      xv[k] = i < n ? load(i) : kNegInf;
    }
#pragma unroll
    for (int k = 0; k < kSelEPT; ++k) {
      const int i = st + k * kSelThreads + tid;
      bal[k] = __ballot(i < n && xv[k] > t);
      if (lane == 0) cnt[k * kSelWaves + w] = __popcll(bal[k]);
    }
    __syncthreads();
    if (w == 0) scan_slots(cnt, pre, lane);
    __syncthreads();
    if (base < cap) {
#pragma unroll
      for (int k = 0; k < kSelEPT; ++k) {
        if ((bal[k] >> lane) & 1ull) {
          const int pos = base + pre[k * kSelWaves + w] + __popcll(bal[k] & lanes_below(lane));
          if (pos < cap) emit(pos, st + k * kSelThreads + tid, xv[k]);
        }
      }
    }
    base += pre[kSelSlots];
    __syncthreads();
  }
  return base;
}

// Fast step: logit threshold from the K1 chunk partials (no extra pass over
// the scores), then ordered compaction capped at buf_k.
__global__ void __launch_bounds__(kSelThreads) select_fast_kernel(FusedSelParams p) {
  __shared__ float red[kSelWaves];
  __shared__ int cnt[kSelSlots];
  __shared__ int pre[kSelSlots + 1];
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const int bi = r / p.q_h;
  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  const float* x = p.scores + static_cast<int64_t>(r) * p.ld;

  // attention/attention.py:142-143: approximate max over the last 256 logits.
  const int tail = min(256, Leff);
  const float mt = block_max<kSelWaves>(tid < tail ? x[Leff - tail + tid] : kNegInf, red);
  // :145 sum_j exp(x_j - m) = sum_c s_c * exp(m_c - m)
  const int nch = (Leff + SAGA_CHUNK - 1) / SAGA_CHUNK;
  float acc = 0.f;
  for (int c = tid; c < nch; c += kSelThreads) {
    const float pm = p.pmax[static_cast<int64_t>(r) * p.nchunk + c];
    if (pm != kNegInf) acc += p.psum[static_cast<int64_t>(r) * p.nchunk + c] * __expf(pm - mt);
  }
  const float ssum = block_sum<kSelWaves>(acc, red);
  // :147 t = m + log(clamp(p*, 1e-30) * s)
  const float t = mt + logf(fmaxf(p.pstar[r], 1e-30f) * ssum);
  if (tid == 0 && p.t_out) p.t_out[r] = t;

  int32_t* oi = p.sel_idx + static_cast<int64_t>(r) * p.cap;
  float* ov = p.sel_val + static_cast<int64_t>(r) * p.cap;
  const int total = ordered_compact(
      Leff, t, p.cap, [&](int i) { return x[i]; },
      [&](int pos, int i, float v) { oi[pos] = i; ov[pos] = v; }, cnt, pre);
  if (tid == 0) {
    p.sel_cnt[r] = min(total, p.cap);
    if (p.sel_total) p.sel_total[r] = total;
  }
}

hipError_t launch_select_fast(const FusedSelParams& p, hipStream_t st) {
  hipLaunchKernelGGL(select_fast_kernel, dim3(p.nrows), dim3(kSelThreads), 0, st, p);
  return hipGetLastError();
}

// threshold_topk_fast API (attention/triton_atopn.py:59-113): typed rows,
// per-row / broadcast / repeated thresholds (:87-96), values kept in the
// input dtype, int64 indices, every slot of the k-wide outputs written
// (unfilled: -inf, 0 as the reference pre-fills them, :82-84).
template <int DT>
__global__ void __launch_bounds__(kSelThreads) select_api_kernel(ApiSelParams p) {
  __shared__ int cnt[kSelSlots];
  __shared__ int pre[kSelSlots + 1];
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const float t = p.thresh[r % p.thresh_numel];
  const int n = static_cast<int>(p.D);
  int64_t* oi = p.out_idx + static_cast<int64_t>(r) * p.oi_ld;
  int total;
  if constexpr (DT == SAGA_DTYPE_F32) {
    const float* x = static_cast<const float*>(p.x) + static_cast<int64_t>(r) * p.x_ld;
    float* ov = static_cast<float*>(p.out_val) + static_cast<int64_t>(r) * p.ov_ld;
    total = ordered_compact(
        n, t, p.k, [&](int i) { return x[i]; },
        [&](int pos, int i, float v) { oi[pos] = i; ov[pos] = v; }, cnt, pre);
    for (int j = min(total, p.k) + tid; j < p.k; j += kSelThreads) { oi[j] = 0; ov[j] = kNegInf; }
  } else {
    const uint16_t* x = static_cast<const uint16_t*>(p.x) + static_cast<int64_t>(r) * p.x_ld;
    uint16_t* ov = static_cast<uint16_t*>(p.out_val) + static_cast<int64_t>(r) * p.ov_ld;
    total = ordered_compact(
        n, t, p.k, [&](int i) { return Elt<DT>::to_f32(x[i]); },
        [&](int pos, int i, float) { oi[pos] = i; ov[pos] = x[i]; }, cnt, pre);
    const uint16_t ninf = DT == SAGA_DTYPE_BF16 ? 0xff80u : 0xfc00u;
    for (int j = min(total, p.k) + tid; j < p.k; j += kSelThreads) { oi[j] = 0; ov[j] = ninf; }
  }
  if (tid == 0 && p.out_counts) p.out_counts[r] = total;
}

hipError_t launch_select_api(const ApiSelParams& p, hipStream_t st) {
  switch (p.x_dt) {
    case SAGA_DTYPE_F32:
      hipLaunchKernelGGL(select_api_kernel<SAGA_DTYPE_F32>, dim3(p.nrows), dim3(kSelThreads), 0, st, p);
      break;
    case SAGA_DTYPE_BF16:
      hipLaunchKernelGGL(select_api_kernel<SAGA_DTYPE_BF16>, dim3(p.nrows), dim3(kSelThreads), 0, st, p);
      break;
    default:
      hipLaunchKernelGGL(select_api_kernel<SAGA_DTYPE_F16>, dim3(p.nrows), dim3(kSelThreads), 0, st, p);
      break;
  }
  return hipGetLastError();
}

// Calibration: exact top-k of each score row (k = min(top_n, L)).
//   1. full-row max M and sum S of exp(x - M) from the K1 partials;
//   2. the k-th largest value by a 3-pass radix select (11/11/10 bits of the
//      order-preserving uint32 key) with 2048-bin LDS histograms;
//   3. ordered compaction of the elements above it plus the first (by index)
//      elements equal to it, to exactly k;
//   4. p* = exp(x_k - M) / S, the k-th largest probability, into the
//      threshold table (attention/attention.py:185-187).
__global__ void __launch_bounds__(kSelThreads) select_calibrate_kernel(FusedSelParams p) {
  __shared__ float red[kSelWaves];
  __shared__ int hist[2048];
  __shared__ int wsum[kSelWaves];
  __shared__ int sel_bin, sel_above;
  __shared__ int cntG[kSelSlots], cntE[kSelSlots];
  __shared__ int preG[kSelSlots + 1], preE[kSelSlots + 1];
  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int bi = r / p.q_h;
  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  const float* x = p.scores + static_cast<int64_t>(r) * p.ld;

  const int nch = (Leff + SAGA_CHUNK - 1) / SAGA_CHUNK;
  float mloc = kNegInf;
  for (int c = tid; c < nch; c += kSelThreads) mloc = fmaxf(mloc, p.pmax[static_cast<int64_t>(r) * p.nchunk + c]);
  const float M = block_max<kSelWaves>(mloc, red);
  float sloc = 0.f;
  for (int c = tid; c < nch; c += kSelThreads) {
    const float pm = p.pmax[static_cast<int64_t>(r) * p.nchunk + c];
    if (pm != kNegInf) sloc += p.psum[static_cast<int64_t>(r) * p.nchunk + c] * __expf(pm - M);
  }
  const float S = block_sum<kSelWaves>(sloc, red);

  const int k = min(p.cap, Leff);
  if (k <= 0) {
    if (tid == 0) {
      p.sel_cnt[r] = 0;
      if (p.sel_total) p.sel_total[r] = 0;
      p.pstar_out[r] = 0.f;
    }
    return;
  }

  uint32_t prefix = 0;
  int krem = k;
  const int shifts[3] = {21, 10, 0};
  const int nbits[3] = {11, 11, 10};
#pragma unroll
  for (int pass = 0; pass < 3; ++pass) {
    const int nb = 1 << nbits[pass];
    const uint32_t hmask = pass == 0 ? 0u : (0xffffffffu << (shifts[pass] + nbits[pass]));
    for (int i = tid; i < 2048; i += kSelThreads) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < Leff; i += kSelThreads) {
      const uint32_t key = f32_to_key(x[i]);
      if ((key & hmask) == prefix) atomicAdd(&hist[(key >> shifts[pass]) & (nb - 1)], 1);
    }
    __syncthreads();
    // bins scanned from the top: thread t owns bins nb-1-2t and nb-2-2t
    const int b0 = nb - 1 - 2 * tid, b1 = b0 - 1;
    const int c0 = b0 >= 0 ? hist[b0] : 0;
    const int c1 = b1 >= 0 ? hist[b1] : 0;
    const int tsum = c0 + c1;
    const int incl = wave_incl_scan(tsum, lane);
    if (lane == kWave - 1) wsum[w] = incl;
    __syncthreads();
    int woff = 0;
    for (int i = 0; i < w; ++i) woff += wsum[i];
    const int ex = woff + incl - tsum;
    if (c0 > 0 && ex < krem && krem <= ex + c0) {
      sel_bin = b0;
      sel_above = ex;
    } else if (c1 > 0 && ex + c0 < krem && krem <= ex + tsum) {
      sel_bin = b1;
      sel_above = ex + c0;
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(sel_bin) << shifts[pass];
    krem -= sel_above;
    __syncthreads();
  }
  const uint32_t kth = prefix;
  const int need = krem;  // elements equal to the k-th value that are taken

  int32_t* oi = p.sel_idx + static_cast<int64_t>(r) * p.cap;
  float* ov = p.sel_val + static_cast<int64_t>(r) * p.cap;
  int baseG = 0, baseE = 0;
  for (int st = 0; st < Leff; st += kSelTile) {
    float xv[kSelEPT];
    unsigned long long bg[kSelEPT], be[kSelEPT];
#pragma unroll
    for (int kk = 0; kk < kSelEPT; ++kk) {
      const int i = st + kk * kSelThreads + tid;
      xv[kk] = i < Leff ? x[i] : kNegInf;
    }
#pragma unroll
    for (int kk = 0; kk < kSelEPT; ++kk) {
      const int i = st + kk * kSelThreads + tid;
      const uint32_t key = f32_to_key(xv[kk]);
      bg[kk] = __ballot(i < Leff && key > kth);
      be[kk] = __ballot(i < Leff && key == kth);
      if (lane == 0) {
        cntG[kk * kSelWaves + w] = __popcll(bg[kk]);
        cntE[kk * kSelWaves + w] = __popcll(be[kk]);
      }
    }
    __syncthreads();
    if (w == 0) scan_slots(cntG, preG, lane);
    if (w == 1) scan_slots(cntE, preE, lane);
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kSelEPT; ++kk) {
      const int slot = kk * kSelWaves + w;
      const int i = st + kk * kSelThreads + tid;
      const int g_before = baseG + preG[slot] + __popcll(bg[kk] & lanes_below(lane));
      const int e_before = baseE + preE[slot] + __popcll(be[kk] & lanes_below(lane));
      if ((bg[kk] >> lane) & 1ull) {
        const int pos = g_before + min(e_before, need);
        oi[pos] = i;
        ov[pos] = xv[kk];
      } else if (((be[kk] >> lane) & 1ull) && e_before < need) {
        const int pos = g_before + e_before;
        oi[pos] = i;
        ov[pos] = xv[kk];
      }
    }
    baseG += preG[kSelSlots];
    baseE += preE[kSelSlots];
    __syncthreads();
  }
  if (tid == 0) {
    p.sel_cnt[r] = k;
    if (p.sel_total) p.sel_total[r] = k;
    p.pstar_out[r] = expf(key_to_f32(kth) - M) / S;
  }
}

hipError_t launch_select_calibrate(const FusedSelParams& p, hipStream_t st) {
  hipLaunchKernelGGL(select_calibrate_kernel, dim3(p.nrows), dim3(kSelThreads), 0, st, p);
  return hipGetLastError();
}

}  // namespace saga

// K2 of the Atop-N fast step, split across the GPU: each score row is cut
// into slices of kSliceLen positions, one wave per (row, slice), with no
// block barrier (wave-level DPP reductions, ballot ranks); then one merge
// block per row.
//
// Replaces the threshold transform (attention/attention.py:136-149), the
// Triton stream compaction threshold_select_fast_kernel
// (attention/triton_atopn.py:6-53) and _atopn_gather_and_output
// (attention/attention.py:152-170) of approx_top_n_attention_amortized
// (:192-209).
//
// Slice wave (atopn_slice_kernel):
//   1. loads of the K1 block partials (max, sum of exp, tail-window max) and
//      of the slice's scores are issued together; t = m + log(max(p*, 1e-30)
//      * sum_j exp(x_j - m)) from the partials (every wave of a row runs the
//      same reduction in the same order, so all of them hold the
//      bit-identical t);
//   2. ordered compaction of {x > t} (strict, triton_atopn.py:42) within the
//      slice: 64-bit ballots and mbcnt put every passing element at its rank
//      in ascending position order; the slice's list goes to LDS and to the
//      workspace;
//   3. softmax . V over the slice's list relative to its own max:
//      (m_s, l_s, o_s = sum_e exp(x_e - m_s) V[e]) to the workspace.
// Merge block (atopn_merge_kernel), per row: the log-sum-exp merge of the
// slice partials; when more than buf_k positions pass, exactly the first
// buf_k in ascending order count (the reference keeps a race-dependent subset
// there): slices past rank buf_k are dropped and the slice straddling it is
// recomputed over its first entries.  The selected list stays in the slice
// lists of the workspace (concatenated in slice order, cut at buf_k).
// The kernel boundary between the two orders the slice writes before the
// merge reads (no device-scope fences or counters).
#include "block_pv.cuh"
#include "kernels.h"

namespace saga {

constexpr int kSliceThreads = 256;                    // 4 independent slice waves per block
constexpr int kSliceWaves = kSliceThreads / kWave;    // 4
constexpr int kSliceLoads = kSliceLen / (4 * kWave);  // f32x4 loads per lane: 4
constexpr int kSlicePrefetch = 4;                     // partials per lane in the first burst
constexpr int kMergeSlices = 8;                       // slices per merge thread in one burst
constexpr int kMergeMaxSlices = 2048;                 // slice ranks kept in LDS

static_assert(kSliceLen == kSliceLoads * 4 * kWave, "slice = whole f32x4 loads of every lane");

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wave-level sparse softmax . V with a running max (online softmax over
// batches): 4 lane groups of 16 lanes, lane c of group G owns dims
// [c*DPL, c*DPL + DPL) and walks entries G, G+4, ...; eight V rows per group
// in flight.
template <int DT, int D>
struct WavePV {
  static constexpr int DPL = D / 16;
  float acc[DPL];
  float m, l;

  __device__ void init() {
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
    m = kNegInf;
    l = 0.f;
  }

  __device__ void add(int n, const int* sidx, const float* sval, const char* vbase, int64_t vrow) {
    const int lane = threadIdx.x & 63;
    float cm = kNegInf;
    for (int i = lane; i < n; i += kWave) cm = fmaxf(cm, sval[i]);
    const float mn = fmaxf(m, wave_max(cm));
    const float scale_old = m == kNegInf ? 0.f : __expf(m - mn);
    float ls = 0.f;
    if (mn != kNegInf)
      for (int i = lane; i < n; i += kWave) ls += __expf(sval[i] - mn);
    l = l * scale_old + wave_sum(ls);
    m = mn;
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] *= scale_old;
    if (mn == kNegInf) return;
    const int G = lane >> 4, c = lane & 15;
    const char* vb = vbase + static_cast<int64_t>(c) * BlockPV<DT, D>::BYTES;
    for (int e0 = G; e0 < n; e0 += 4 * kPVUnroll) {
      u32x4 raw[kPVUnroll][BlockPV<DT, D>::NV];
#pragma unroll
      for (int u = 0; u < kPVUnroll; ++u) {
        const int e = e0 + 4 * u;
        if (e < n) BlockPV<DT, D>::load_raw(vb + static_cast<int64_t>(sidx[e]) * vrow, raw[u]);
      }
      __builtin_amdgcn_sched_barrier(0);  // all gathers in flight before the FMAs
#pragma unroll
      for (int u = 0; u < kPVUnroll; ++u) {
        const int e = e0 + 4 * u;
        if (e < n) {
          const float w = __expf(sval[e] - mn);
          float f[DPL];
          BlockPV<DT, D>::unpack(raw[u], f);
#pragma unroll
          for (int i = 0; i < DPL; ++i) acc[i] += w * f[i];
        }
      }
    }
  }

  // Sum the 4 groups through the wave's LDS scratch (>= 4 * D floats); o[q]
  // then holds dim lane + 64 q (< D) of sum_e w_e V[e].
  template <int DQ>
  __device__ void reduce(float* scratch, float (&o)[DQ]) {
    const int lane = threadIdx.x & 63, G = lane >> 4, c = lane & 15;
#pragma unroll
    for (int i = 0; i < DPL; ++i) scratch[G * D + c * DPL + i] = acc[i];
    wave_lds_sync();
#pragma unroll
    for (int q = 0; q < DQ; ++q) {
      const int i = lane + q * kWave;
      o[q] = i < D ? (scratch[i] + scratch[D + i]) + (scratch[2 * D + i] + scratch[3 * D + i]) : 0.f;
    }
    wave_lds_sync();
  }
};

struct SliceWaveShared {
  int sidx[kSliceLen];
  float sval[kSliceLen];
};

// The slice holding list entry j of a row (pre[s] <= j < pre[s+1]).
__device__ __forceinline__ int slice_of(const int* pre, int nslice, int j) {
  int lo = 0, hi = nslice - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (pre[mid] <= j) lo = mid; else hi = mid - 1;
  }
  return lo;
}

template <int DT, int D>
__global__ void __launch_bounds__(kSliceThreads) atopn_slice_kernel(FusedSelParams p, PVParams v) {
  __shared__ SliceWaveShared shw[kSliceWaves];
  constexpr int DQ = (D + kWave - 1) / kWave;  // output dims per lane
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t gw = static_cast<int64_t>(blockIdx.x) * kSliceWaves + w;
  if (gw >= static_cast<int64_t>(p.nrows) * p.nslice) return;
  const int r = static_cast<int>(gw / p.nslice), sl = static_cast<int>(gw - static_cast<int64_t>(r) * p.nslice);
  SliceWaveShared& sh = shw[w];
  const int bi = r / p.q_h, h = r - bi * p.q_h;
  const float* x = p.scores + static_cast<int64_t>(r) * p.ld;
  const float* prow_m = p.pmax + static_cast<int64_t>(r) * p.nparts;
  const float* prow_s = p.psum + static_cast<int64_t>(r) * p.nparts;
  const float* prow_t = p.ptail + static_cast<int64_t>(r) * p.nparts;
  const int s0 = sl * kSliceLen;

  // 1. the block partials and the slice's scores in flight together; nothing
  //    waits for kv_len, which only masks
  float pm[kSlicePrefetch], ps[kSlicePrefetch], pt[kSlicePrefetch];
#pragma unroll
  for (int k = 0; k < kSlicePrefetch; ++k) {
    const int c = lane + k * kWave;
    pm[k] = c < p.nparts ? prow_m[c] : kNegInf;
    ps[k] = c < p.nparts ? prow_s[c] : 0.f;
    pt[k] = c < p.nparts ? prow_t[c] : kNegInf;
  }
  f32x4 xv[kSliceLoads];
#pragma unroll
  for (int k = 0; k < kSliceLoads; ++k) {
    const int64_t e = s0 + 4 * (k * kWave + lane);
    xv[k] = e < p.ld ? *reinterpret_cast<const f32x4*>(x + e) : f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
  }
  const float pstar = p.pstar[r];
  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  __builtin_amdgcn_sched_barrier(0);

  // attention/attention.py:142-147: m = max of the last min(256, L) logits
  float tl = kNegInf;
#pragma unroll
  for (int k = 0; k < kSlicePrefetch; ++k) tl = fmaxf(tl, pt[k]);
  for (int c = lane + kSlicePrefetch * kWave; c < p.nparts; c += kWave) tl = fmaxf(tl, prow_t[c]);
  const float mt = wave_max(tl);
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < kSlicePrefetch; ++k)
    if (pm[k] != kNegInf) acc += ps[k] * __expf(pm[k] - mt);
  for (int c = lane + kSlicePrefetch * kWave; c < p.nparts; c += kWave) {
    const float m2 = prow_m[c];
    if (m2 != kNegInf) acc += prow_s[c] * __expf(m2 - mt);
  }
  const float ssum = wave_sum(acc);
  const float t = mt + logf(fmaxf(pstar, 1e-30f) * ssum);

  // 2. ordered compaction; element (k, lane, j) is position s0 + 4*(k*64 + lane) + j.
  //    Ballot j of load k holds flag j of every lane; a passing element's rank
  //    is the passing elements of earlier loads + those of lower lanes (mbcnt
  //    of the four ballots) + its own lower flags.
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
        sh.sidx[pos] = e + j;
        sh.sval[pos] = xv[k][j];
        if (pos < p.slice_cap) {
          gidx[pos] = e + j;
          gval[pos] = xv[k][j];
        }
        ++pos;
      }
    }
  }
  if (lane == 0) {
    p.sl_cnt[gw] = n;
    if (sl == 0 && p.t_out) p.t_out[r] = t;
  }
  wave_lds_sync();

  // 3. the slice's softmax . V partial (skipped when the row overflows for
  //    sure: the merge recomputes it from the capped list)
  const int vh = h / (v.q_h / v.v_h);
  const char* vbase = v.v + (bi * v.v_sb + static_cast<int64_t>(vh) * v.v_sh) * Elt<DT>::kBytes;
  WavePV<DT, D> pv;
  pv.init();
  if (n <= p.cap) pv.add(n, sh.sidx, sh.sval, vbase, v.v_sl * Elt<DT>::kBytes);
  wave_lds_sync();
  float o[DQ];
  pv.reduce(sh.sval, o);  // the list is consumed: its LDS is the scratch
#pragma unroll
  for (int q = 0; q < DQ; ++q)
    if (lane + q * kWave < D) p.sl_o[gw * D + lane + q * kWave] = o[q];
  if (lane == 0) {
    p.sl_ml[2 * gw] = pv.m;
    p.sl_ml[2 * gw + 1] = pv.l;
  }
}

// Merge of row r's slice partials, one 256-thread block per row.
//   1. the slice counts and a first batch of partials in one burst; a block
//      scan of the counts gives each slice's first rank;
//   2. slices whose passing positions all rank below buf_k ("included") are
//      merged from their partials: out = sum_s o_s exp(m_s - M) / sum_s l_s
//      exp(m_s - M), thread t owning dims [4c, 4c + 4), c = t % (D/4), of the
//      slices g, g + G, ... (g = t / (D/4));
//   3. overflow (total > buf_k): the one slice straddling rank buf_k
//      contributes softmax . V over its first k* entries, recomputed here;
//      later slices are dropped.
template <int DT, int D>
__global__ void __launch_bounds__(kSliceThreads) atopn_merge_kernel(FusedSelParams p, PVParams v) {
  __shared__ float red[kSliceWaves];
  __shared__ int wsum[kSliceWaves];
  __shared__ int spre[kMergeMaxSlices + 1];
  __shared__ int sidx[kSliceLen];
  __shared__ float sval[kSliceLen];
  __shared__ f32x4 accs[kSliceThreads];
  constexpr int C = D / 4;              // 16-byte chunks per output row
  constexpr int G = kSliceThreads / C;  // slice groups
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = tid % C, g = tid / C;
  const int ns = p.nslice;
  const int64_t row0 = static_cast<int64_t>(r) * ns;
  const int bi = r / p.q_h, h = r - bi * p.q_h;
  const int64_t ooff = bi * v.o_sb + static_cast<int64_t>(h) * v.o_sh;
  // the row's slice ranks: LDS, or the workspace for very long rows
  int* pre = ns <= kMergeMaxSlices ? spre : p.sl_pre + static_cast<int64_t>(r) * (ns + 1);

  // 1. counts + the first batch of partials, then the block scan of the counts
  float ms[kMergeSlices], lsv[kMergeSlices];
  f32x4 ov[kMergeSlices];
  auto load_batch = [&](int b0) {
#pragma unroll
    for (int u = 0; u < kMergeSlices; ++u) {
      const int s = b0 + g + G * u;
      ms[u] = s < ns ? p.sl_ml[2 * (row0 + s)] : kNegInf;
      lsv[u] = s < ns ? p.sl_ml[2 * (row0 + s) + 1] : 0.f;
      ov[u] = s < ns ? *reinterpret_cast<const f32x4*>(p.sl_o + (row0 + s) * D + 4 * c) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  int run = 0;
  for (int c0 = 0; c0 < ns; c0 += kSliceThreads) {
    const int s = c0 + tid;
    const int cnt = s < ns ? p.sl_cnt[row0 + s] : 0;
    if (c0 == 0) load_batch(0);
    const int incl = wave_incl_scan(cnt, lane);
    if (lane == kWave - 1) wsum[w] = incl;
    __syncthreads();
    int before = run, tot = 0;
#pragma unroll
    for (int q = 0; q < kSliceWaves; ++q) {
      before += q < w ? wsum[q] : 0;
      tot += wsum[q];
    }
    if (s < ns) pre[s] = before + incl - cnt;
    run += tot;
    __syncthreads();
  }
  if (tid == 0) pre[ns] = run;
  __threadfence_block();
  __syncthreads();
  const int total = run;
  // included slices: pre[s + 1] <= cap; the straddling slice s_cut takes its
  // first k_cut entries
  int s_cut = ns, k_cut = 0;
  if (total > p.cap) {
    s_cut = slice_of(pre, ns, p.cap - 1);
    k_cut = p.cap - pre[s_cut];
    if (k_cut == pre[s_cut + 1] - pre[s_cut]) {  // the cut falls on a slice boundary
      ++s_cut;
      k_cut = 0;
    }
  }
  if (tid == 0) {
    p.sel_cnt[r] = min(total, p.cap);
    if (p.sel_total) p.sel_total[r] = total;
  }

  // 2. log-sum-exp merge of the included slices
  float M = kNegInf, lsum = 0.f;
  f32x4 on = {0.f, 0.f, 0.f, 0.f};
  for (int b0 = 0; b0 < ns; b0 += G * kMergeSlices) {
    if (b0 > 0) load_batch(b0);
    float mb = kNegInf;
#pragma unroll
    for (int u = 0; u < kMergeSlices; ++u)
      if (b0 + g + G * u < s_cut) mb = fmaxf(mb, ms[u]);
    const float Mn = fmaxf(M, block_max<kSliceWaves>(mb, red));
    const float rescale = M == kNegInf ? 0.f : __expf(M - Mn);
    lsum *= rescale;
#pragma unroll
    for (int i = 0; i < 4; ++i) on[i] *= rescale;
    M = Mn;
#pragma unroll
    for (int u = 0; u < kMergeSlices; ++u) {
      if (b0 + g + G * u < s_cut && ms[u] != kNegInf) {
        const float wgt = __expf(ms[u] - M);
        lsum += lsv[u] * wgt;
#pragma unroll
        for (int i = 0; i < 4; ++i) on[i] += ov[u][i] * wgt;
      }
    }
  }
  // l is the same in every thread of a slice group: one thread per group adds it
  float L = block_sum<kSliceWaves>(c == 0 ? lsum : 0.f, red);
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

  // 3. the straddling slice's first k_cut entries (block-uniform branch)
  if (k_cut > 0) {
    const int64_t src = (row0 + s_cut) * p.slice_cap;
    for (int i = tid; i < k_cut; i += kSliceThreads) {
      sidx[i] = p.sl_idx[src + i];
      sval[i] = p.sl_val[src + i];
    }
    __syncthreads();
    const int vh = h / (v.q_h / v.v_h);
    const char* vbase = v.v + (bi * v.v_sb + static_cast<int64_t>(vh) * v.v_sh) * Elt<DT>::kBytes;
    BlockPV<DT, D, kSliceThreads> pv;
    pv.init();
    pv.add(k_cut, sidx, sval, vbase, v.v_sl * Elt<DT>::kBytes, false, red);
    float* accs_f = reinterpret_cast<float*>(accs);
    __syncthreads();
    const float oc = pv.reduce(accs_f);  // thread i < D: dim i of the slice prefix
    __syncthreads();
    if (tid < D) accs_f[tid] = oc;
    __syncthreads();
    const float Mn = fmaxf(M, pv.m);
    const float a = M == kNegInf ? 0.f : __expf(M - Mn);
    const float bw = pv.m == kNegInf ? 0.f : __expf(pv.m - Mn);
    L = L * a + pv.l * bw;
    if (tid < C) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = o[i] * a + accs_f[4 * tid + i] * bw;
    }
  }
  if (tid < C) {
    // no passing position: softmax over an empty (all -inf) list is NaN
#pragma unroll
    for (int i = 0; i < 4; ++i)
      store_from_f32(v.out, v.out_dt, ooff + 4 * tid + i, total == 0 ? __builtin_nanf("") : o[i] / L);
  }
}

template <int DT, int D>
static hipError_t launch_split(const FusedSelParams& p, const PVParams& v, hipStream_t st) {
  const int64_t waves = static_cast<int64_t>(p.nslice) * p.nrows;
  const unsigned blocks = static_cast<unsigned>((waves + kSliceWaves - 1) / kSliceWaves);
  hipLaunchKernelGGL((atopn_slice_kernel<DT, D>), dim3(blocks), dim3(kSliceThreads), 0, st, p, v);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((atopn_merge_kernel<DT, D>), dim3(p.nrows), dim3(kSliceThreads), 0, st, p, v);
  return hipGetLastError();
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

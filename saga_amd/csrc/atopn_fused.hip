// Fused Atop-N fast step: scores, logit threshold, ordered compaction and
// the short lists' softmax . V in one kernel; the per-row merge and the long
// lists' gathers in the row kernel (atopn_gather_kernel) after it.
//
// Replaces _compute_attn_weights (attention/attention.py:113-128),
// _transform_softmax_threshold (:136-149), threshold_select_fast_kernel
// (attention/triton_atopn.py:6-53) and _atopn_gather_and_output
// (attention/attention.py:152-170) of approx_top_n_attention_amortized
// (:192-209), for shapes whose whole grid is resident on the GPU at once.
//
// Grid: the K1 plan (qk_plan): every (batch, key head) "unit" is cut into
// nparts ranges of 16-position tiles, 4 ranges per 256-thread block, nb =
// nparts / 4 blocks per unit.  A block:
//   1. scores its 4 ranges exactly as K1 (qk_wave_scores) and keeps them in
//      registers; merges (max, sum of exp, tail-window max) per head;
//   2. publishes that block partial and its arrival flag, then waits until
//      every block of its unit has arrived (a flag barrier over the unit's
//      nb blocks, all of them resident, see below);
//   3. reads the unit's nb partials per head and computes, in every block
//      identically, the logit threshold t = m + log(max(p*, 1e-30) * sum_j
//      exp(x_j - m)) (m = max of the last min(256, kv_len) logits) and the
//      row max M;
//   4. compacts {x > t} (strict, triton_atopn.py:42) per head in ascending
//      position order into the block's list ("slice") of the row, capped at
//      min(block positions, buf_k);
//   5. gathers the V rows of every list of at most kSliceSmall entries
//      itself: an (M, l, o) partial with weights exp(x - M) <= 1.
// The row kernel then ranks the block lists of each row, keeps exactly the
// first buf_k passing positions, merges the partials and gathers the rest.
//
// Barrier.  Cross-block data (partials, flags, epochs) moves through
// agent-scope relaxed atomic stores and loads (global_store / global_load
// sc1: coherent across the XCDs' L2 caches, no L2 write-back fences).  A
// block publishes its partial, waits until its own stores are acknowledged
// (s_waitcnt 0), then stores flag[unit][j] = epoch[unit] + 1.  Wave 0 polls
// the unit's nb flags until all equal epoch + 1.  Block 0 of the unit then
// advances epoch[unit] (every block of the unit has read it before storing
// its flag).  Flags sit at fixed per-(unit, block) addresses and only grow,
// so calls with other block counts never see a stale equal flag; the region
// must be zero before the first call on a workspace.  Deadlock freedom: the
// host launches this kernel only when units * nb blocks fit the GPU at once
// (kFusedBlocksPerCU per CU; the kernel's occupancy is checked), every block
// arrives before it waits, and no block waits on another unit.  A wait that
// exceeds kFusedSpinLimit polls sets the sync error word, empties the
// block's lists and returns, so the kernel always ends.
#include <atomic>

#include "block_pv.cuh"
#include "qk_wave.cuh"

namespace saga {

constexpr int kFusedThreads = 256;
constexpr int kFusedSpinLimit = 1 << 20;

__device__ __forceinline__ int ld_agent(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(int32_t* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct FusedShared {
  float red[3][4][16];         // block partial merge
  float th[16], rmax[16];      // per head: logit threshold, row max
  int cnt[4][16];              // per wave and head: passing positions
  int ok;
  int lidx[16][kSliceSmall];   // short lists per head (block-local ascending order)
  float lval[16][kSliceSmall];
  float scratch[4][4 * 128];   // per wave: the 4 lane groups' sums of one head
};

template <int DT, int D>
__global__ void __launch_bounds__(kFusedThreads) __attribute__((amdgpu_waves_per_eu(3, 8)))
atopn_fused_kernel(QKParams q, FusedSelParams p, PVParams v, FusedSync sy) {
  using PV = BlockPV<DT, D>;
  constexpr int DPL = PV::DPL;
  // V rows per lane group in one gather burst: 64 entries per burst for 16-byte
  // row chunks, 32 for the 32-byte chunks of f32 d128 (register budget)
  constexpr int UNROLL = PV::NV > 1 ? kSliceSmall / 8 : kSliceSmall / 4;
  constexpr int BURST = 4 * UNROLL;
  __shared__ FusedShared sh;
  const int lane = threadIdx.x & 63;
  const int col = lane & 15, s = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nb = q.nparts >> 2;
  int unit, j;
  if (sy.xcd_map) {  // units % 8 == 0: unit u's blocks are the ids == u (mod 8), one XCD
    const int x8 = blockIdx.x & 7, k = blockIdx.x >> 3;
    unit = x8 + 8 * (k / nb);
    j = k - (k / nb) * nb;
  } else {
    unit = blockIdx.x / nb;
    j = blockIdx.x - unit * nb;
  }
  const QKWaveSpan w = qk_wave_span(q, unit, 4 * j + wave, col);
  const int row = unit * q.g + col;  // = batch * q_h + head for hvalid lanes
  // loaded unconditionally, before the K burst (a load under a branch makes the
  // compiler wait for it at the join, ahead of the stream); used by wave 0
  const int epoch = ld_agent(sy.epoch + unit);
  const float pstar = p.pstar[w.hvalid ? row : unit * q.g];

  // 1. scores and the block partial
  float x[kQKMaxTiles][4];
  int Leff;
  const float m = qk_wave_scores<DT, D>(q, w, s, col, x, Leff);
  float pm, ps, pt;
  qk_block_partial(x, m, w, Leff, true, s, col, wave, sh.red, pm, ps, pt);

  // 2. publish, arrive, wait (wave 0)
  if (wave == 0) {
    if (s == 0 && w.hvalid) {
      const int64_t o = static_cast<int64_t>(row) * nb + j;
      st_agent(q.pmax + o, pm);
      st_agent(q.psum + o, ps);
      st_agent(q.ptail + o, pt);
    }
    // the partial stores are acknowledged before the flag is stored: a compiler
    // barrier (no instruction) on each side of the hardware wait
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    int32_t* flags = sy.flags + static_cast<int64_t>(unit) * kFusedMaxBlocks;
    if (lane == 0) st_agent(flags + j, epoch + 1);
    int ok = 0;
    for (int it = 0; it < kFusedSpinLimit; ++it) {
      bool arrived = true;
      for (int jj = lane; jj < nb; jj += kWave) arrived &= ld_agent(flags + jj) == epoch + 1;
      if (__all(arrived)) {
        ok = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);  // no partial load moves above the poll
    if (lane == 0) {
      sh.ok = ok;
      if (!ok) st_agent(sy.error, 1);
      if (ok && j == 0) st_agent(sy.epoch + unit, epoch + 1);
    }
  }
  __syncthreads();
  if (!sh.ok) {
    if (wave == 0 && s == 0 && w.hvalid) p.sl_cnt[static_cast<int64_t>(row) * p.nslice + j] = 0;
    return;
  }

  // 3. thresholds: wave `wave` reduces heads wave, wave + 4, ... over the nb
  //    partials (lanes jj = lane, lane + 64); the same code and order in every
  //    block gives every block the bit-identical t
  {
    constexpr int kHeads = 4, kPer = 2;  // g <= 16, nb <= 128
    float cm[kHeads][kPer], cs[kHeads][kPer], ct[kHeads][kPer];
#pragma unroll
    for (int k = 0; k < kHeads; ++k) {
      const int hk = wave + 4 * k;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int jj = lane + kWave * i;
        const bool use = hk < q.g && jj < nb;
        const int64_t o = static_cast<int64_t>(unit * q.g + hk) * nb + jj;
        cm[k][i] = use ? ld_agent(q.pmax + o) : kNegInf;
        cs[k][i] = use ? ld_agent(q.psum + o) : 0.f;
        ct[k][i] = use ? ld_agent(q.ptail + o) : kNegInf;
      }
    }
#pragma unroll
    for (int k = 0; k < kHeads; ++k) {
      const int hk = wave + 4 * k;
      if (hk >= q.g) break;
      const float mt = wave_max(fmaxf(ct[k][0], ct[k][1]));
      const float M = wave_max(fmaxf(cm[k][0], cm[k][1]));
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < kPer; ++i)
        if (cm[k][i] != kNegInf) acc += cs[k][i] * __expf(cm[k][i] - mt);
      const float ssum = wave_sum(acc);
      const float ps_k = lane_f(pstar, hk);
      if (lane == 0) {
        sh.th[hk] = mt + logf(fmaxf(ps_k, 1e-30f) * ssum);
        sh.rmax[hk] = M;
      }
    }
  }
  lds_sync();
  const float th = sh.th[col];

  // 4. ordered compaction per head.  Lane (s, col) holds positions
  //    16*(t0 + t) + 4*s + r of head col as bit 4t + r of F; a head's order is
  //    (wave, t, s, r).
  uint32_t F = 0;
  if (w.hvalid) {
#pragma unroll
    for (int t = 0; t < kQKMaxTiles; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (x[t][r] > th) F |= 1u << (4 * t + r);
  }
  const uint32_t F0 = __shfl(F, col), F1 = __shfl(F, col + 16), F2 = __shfl(F, col + 32), F3 = __shfl(F, col + 48);
  const int nw = __popc(F0) + __popc(F1) + __popc(F2) + __popc(F3);
  if (s == 0) sh.cnt[wave][col] = nw;
  lds_sync();
  int off = 0, N = 0;
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    const int c = sh.cnt[q4][col];
    if (q4 < wave) off += c;
    N += c;
  }
  const int64_t slot = static_cast<int64_t>(row) * p.nslice + j;
  if (F) {
    int32_t* gidx = p.sl_idx + slot * p.slice_cap;
    float* gval = p.sl_val + slot * p.slice_cap;
    const bool small = N <= kSliceSmall;
#pragma unroll
    for (int t = 0; t < kQKMaxTiles; ++t) {
      const uint32_t below = (1u << (4 * t)) - 1u;
      const int sh4 = 4 * t;
      int base = off + __popc(F0 & below) + __popc(F1 & below) + __popc(F2 & below) + __popc(F3 & below);
      base += (s > 0 ? __popc((F0 >> sh4) & 15u) : 0) + (s > 1 ? __popc((F1 >> sh4) & 15u) : 0) +
              (s > 2 ? __popc((F2 >> sh4) & 15u) : 0);
      const uint32_t nib = (F >> sh4) & 15u;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if ((nib >> r) & 1u) {
          const int e = base + __popc(nib & ((1u << r) - 1u));
          const int pos = 16 * (w.t0 + t) + 4 * s + r;
          if (e < p.slice_cap) {
            gidx[e] = pos;
            gval[e] = x[t][r];
          }
          if (small) {
            sh.lidx[col][e] = pos;
            sh.lval[col][e] = x[t][r];
          }
        }
      }
    }
  }
  if (wave == 0 && s == 0 && w.hvalid) {
    p.sl_cnt[slot] = N;
    if (j == 0 && p.t_out) p.t_out[row] = th;
  }
  lds_sync();  // the LDS lists; the global list stores complete in the background

  // 5. short lists: wave `wave` gathers heads wave, wave + 4, ... (at most 4),
  //    their entries concatenated, BURST rows per burst
  int nk[4], ck[5];
  ck[0] = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int hk = wave + 4 * k;
    int n = 0;
    if (hk < q.g) {
      n = sh.cnt[0][hk] + sh.cnt[1][hk] + sh.cnt[2][hk] + sh.cnt[3][hk];
      if (n > kSliceSmall) n = 0;
    }
    nk[k] = n;
    ck[k + 1] = ck[k] + n;
  }
  const int E = ck[4];
  if (E == 0) return;
  const int G = lane >> 4, c = lane & 15;
  const int gq = v.q_h / v.v_h;
  const int64_t vrow = v.v_sl * Elt<DT>::kBytes;
  float Mk[4];
  const char* vb[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int hk = min(wave + 4 * k, q.g - 1);
    Mk[k] = sh.rmax[hk];
    const int vh = (w.kh * q.g + hk) / gq;
    vb[k] = v.v + (w.bi * v.v_sb + static_cast<int64_t>(vh) * v.v_sh) * Elt<DT>::kBytes +
            static_cast<int64_t>(c) * PV::BYTES;
  }
  float acc[4][DPL];
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[k][i] = 0.f;
  float lk[4] = {0.f, 0.f, 0.f, 0.f};
  for (int e0 = 0; e0 < E; e0 += BURST) {
    u32x4 raw[UNROLL][PV::NV];
    int ek[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int e = e0 + G + 4 * u;
      const int k = (e >= ck[1]) + (e >= ck[2]) + (e >= ck[3]);
      ek[u] = e < E ? k : -1;
      if (e < E) {
        const int hk = wave + 4 * k;
        const char* base = k == 0 ? vb[0] : k == 1 ? vb[1] : k == 2 ? vb[2] : vb[3];
        PV::load_raw(base + static_cast<int64_t>(sh.lidx[hk][e - ck[k]]) * vrow, raw[u]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every gather in flight before the FMAs
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int k = ek[u];
      if (k >= 0) {
        const int e = e0 + G + 4 * u;
        const int hk = wave + 4 * k;
        const float mk = k == 0 ? Mk[0] : k == 1 ? Mk[1] : k == 2 ? Mk[2] : Mk[3];
        const float wt = __expf(sh.lval[hk][e - ck[k]] - mk);
        float f[DPL];
        PV::unpack(raw[u], f);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const float wk = k == kk ? wt : 0.f;
#pragma unroll
          for (int i = 0; i < DPL; ++i) acc[kk][i] += wk * f[i];
        }
      }
    }
  }
  // l per head: every entry once (lane e mod 64)
  for (int e = lane; e < E; e += kWave) {
    const int k = (e >= ck[1]) + (e >= ck[2]) + (e >= ck[3]);
    const int hk = wave + 4 * k;
    const float mk = k == 0 ? Mk[0] : k == 1 ? Mk[1] : k == 2 ? Mk[2] : Mk[3];
    const float wt = __expf(sh.lval[hk][e - ck[k]] - mk);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) lk[kk] += k == kk ? wt : 0.f;
  }
  float* scr = sh.scratch[wave];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (nk[k] == 0) continue;  // wave-uniform
    const int hk = wave + 4 * k;
    const float l = wave_sum(lk[k]);
    wave_lds_fence();
#pragma unroll
    for (int i = 0; i < DPL; ++i) scr[G * D + c * DPL + i] = acc[k][i];
    wave_lds_fence();
    const int64_t hslot = static_cast<int64_t>(unit * q.g + hk) * p.nslice + j;
    for (int i = lane; i < D; i += kWave)
      p.sl_o[hslot * D + i] = (scr[i] + scr[D + i]) + (scr[2 * D + i] + scr[3 * D + i]);
    if (lane == 0) {
      p.sl_ml[2 * hslot] = Mk[k];
      p.sl_ml[2 * hslot + 1] = l;
    }
  }
}

hipError_t launch_atopn_rows(const FusedSelParams& p, const PVParams& v, hipStream_t st);

namespace {

// Per-device facts queried once (a racing first call stores the same values).
struct FusedDev {
  std::atomic<int> cus{0};
  std::atomic<int> checked{0};  // bit per (dtype, d) instantiation: occupancy verified
};
FusedDev g_fused_dev[64];

template <int DT, int D>
hipError_t fused_occupancy_ok(int dev, int bit) {
  FusedDev& fd = g_fused_dev[dev];
  if (fd.checked & (1 << bit)) return hipSuccess;
  int per = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, atopn_fused_kernel<DT, D>, kFusedThreads, 0);
  if (e != hipSuccess) return e;
  if (per < kFusedBlocksPerCU) return hipErrorLaunchOutOfResources;
  fd.checked |= 1 << bit;
  return hipSuccess;
}

template <int DT, int D>
hipError_t launch_fused_typed(const QKParams& q, const FusedSelParams& p, const PVParams& v, const FusedSync& sy,
                              int dev, int bit, hipStream_t st) {
  hipError_t e = fused_occupancy_ok<DT, D>(dev, bit);
  if (e != hipSuccess) return e;
  const unsigned blocks = static_cast<unsigned>(static_cast<int64_t>(q.b) * q.k_h * (q.nparts / 4));
  hipLaunchKernelGGL((atopn_fused_kernel<DT, D>), dim3(blocks), dim3(kFusedThreads), 0, st, q, p, v, sy);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_atopn_rows(p, v, st);
}

}  // namespace

// Off by default: measured slower than the three-kernel path at every shape
// it covers on MI355X (see the A/B switch saga_set_fused_fast_step).
static std::atomic<int> g_fused_enabled{0};

int set_fused_enabled(int enable) { return g_fused_enabled.exchange(enable ? 1 : 0); }

int fused_device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  FusedDev& fd = g_fused_dev[dev];
  if (fd.cus == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    fd.cus = n;
  }
  return fd.cus;
}

bool atopn_fused_fits(int64_t b, int64_t k_h, int64_t g, int64_t L) {
  const int64_t units = b * k_h;
  const int64_t nb = qk_plan(b, k_h, L) / 4;
  const int cus = fused_device_cus();
  return g_fused_enabled.load() && L > 0 && g <= 16 && units <= kFusedMaxUnits && nb <= kFusedMaxBlocks &&
         units * nb <= static_cast<int64_t>(cus) * kFusedBlocksPerCU;
}

int64_t atopn_fused_slice_cap(int64_t b, int64_t k_h, int64_t L, int64_t buf_k) {
  const int64_t nparts = qk_plan(b, k_h, L);
  const int64_t ntiles = (L + 15) / 16;
  const int64_t per_wave = (ntiles + nparts - 1) / nparts;  // balanced ranges: at most this many tiles
  return std::min<int64_t>(4 * 16 * per_wave, buf_k);
}

hipError_t launch_atopn_fused(int dtype, int d, const QKParams& q, const FusedSelParams& p, const PVParams& v,
                              const FusedSync& sy, hipStream_t st) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  if (dtype == SAGA_DTYPE_BF16)
    return d == 128 ? launch_fused_typed<SAGA_DTYPE_BF16, 128>(q, p, v, sy, dev, 0, st)
                    : launch_fused_typed<SAGA_DTYPE_BF16, 64>(q, p, v, sy, dev, 1, st);
  if (dtype == SAGA_DTYPE_F16)
    return d == 128 ? launch_fused_typed<SAGA_DTYPE_F16, 128>(q, p, v, sy, dev, 2, st)
                    : launch_fused_typed<SAGA_DTYPE_F16, 64>(q, p, v, sy, dev, 3, st);
  return d == 128 ? launch_fused_typed<SAGA_DTYPE_F32, 128>(q, p, v, sy, dev, 4, st)
                  : launch_fused_typed<SAGA_DTYPE_F32, 64>(q, p, v, sy, dev, 5, st);
}

}  // namespace saga

// Dense decode attention, split-L (flash-decoding), one pass over K and V.
//
// Replaces full_einsum_forward (attention/attention.py:64-85) for l_q == 1:
// it serves the layers exempt from Atop-N, SAGA with full attention and the
// dense-GQA comparator.  Kernel 1 gives a block one (batch, key head) unit
// and one split of the positions; its four waves step through
// sub-chunks of 16 positions, each with one burst of loads (the K rows and
// the V rows of up to two value heads):
//   * QK on MFMA exactly as the score kernel (K rows -> A fragments, the
//     g <= 16 query heads of the unit -> B fragment),
//   * online softmax per head (running max / sum, rescale factor alpha),
//   * P (fp32) through wave-private LDS, then P . V on the VALU in fp32, one
//     V row per wave load (d / 64 dims per lane); heads read value head
//     h / (q_h / v_h), so a unit may touch several value heads (SAGA: 1 key
//     head, 2 value heads).
// Waves merge in LDS; with several splits each writes a (max, sum, o[d])
// partial per head and kernel 2 (one block per head) merges them.
#include <type_traits>

#include "common.cuh"
#include "kernels.h"

namespace saga {

constexpr int kDenseSubDefault = 16;  // positions per wave step (MFMA tiles of 16)

// Wave-local LDS ordering: the P and alpha buffers of a wave are private to it.
__device__ __forceinline__ void dense_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One V row per wave load: lane l holds dims [l*DL, l*DL + DL), DL = D / 64.
template <int DT, int DL>
struct VLane {
  static constexpr int BYTES = DL * Elt<DT>::kBytes;  // 2, 4 or 8
  using Raw = typename std::conditional<BYTES == 8, u32x2, typename std::conditional<BYTES == 4, uint32_t, uint16_t>::type>::type;
  __device__ static Raw load(const char* p) { return *reinterpret_cast<const Raw*>(p); }
  __device__ static void unpack(const Raw& r, float* f) {
    if constexpr (DT == SAGA_DTYPE_F32) {
      if constexpr (DL == 2) {
        f[0] = __uint_as_float(r.x);
        f[1] = __uint_as_float(r.y);
      } else {
        f[0] = __uint_as_float(r);
      }
    } else if constexpr (DL == 2) {
      f[0] = Elt<DT>::to_f32(r & 0xffffu);
      f[1] = Elt<DT>::to_f32(r >> 16);
    } else {
      f[0] = Elt<DT>::to_f32(r);
    }
  }
};

template <int DT, int D, int kDenseSub>
__global__ void __launch_bounds__(256) dense_split_kernel(DenseParams p) {
  using E = Elt<DT>;
  constexpr int E16 = E::kPer16B;
  constexpr int NLOAD = D / (4 * E16);
  constexpr int DL = D / kWave;  // dims per lane in the P . V phase
  using VL = VLane<DT, DL>;
  __shared__ float Ps[4][16][kDenseSub];  // per wave: P[head][position]
  __shared__ float Al[4][16];
  __shared__ float Wm[4][16], Wl[4][16];
  __shared__ float Wo[4][16][D];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int col = lane & 15, s = lane >> 4;
  const int split = blockIdx.x % p.nsplit;
  const int unit = blockIdx.x / p.nsplit;
  const int bi = unit / p.k_h, kh = unit - bi * p.k_h;
  const int g = p.g;
  const int g_v = p.q_h / p.v_h;
  int Leff = p.L;
  if (p.kv_len) Leff = min(Leff, max(p.kv_len[bi], 0));
  const bool hvalid = col < g;
  const int h0 = kh * g;
  const int h = h0 + (hvalid ? col : 0);

  u32x4 qf[NLOAD];
  const char* qrow = p.q + (bi * p.q_sb + static_cast<int64_t>(h) * p.q_sh) * E::kBytes;
#pragma unroll
  for (int j = 0; j < NLOAD; ++j)
    qf[j] = hvalid ? ld16(qrow + (j * 4 * E16 + s * E16) * E::kBytes) : u32x4{0u, 0u, 0u, 0u};
  const char* kbase = p.k + (bi * p.k_sb + static_cast<int64_t>(kh) * p.k_sh) * E::kBytes;

  const int vh_first = h0 / g_v, vh_last = (h0 + g - 1) / g_v;
  const int64_t vrow = p.v_sl * E::kBytes;
  const char* vlane = p.v + (bi * p.v_sb + static_cast<int64_t>(lane) * DL) * E::kBytes;

  float acc[16][DL];
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int d = 0; d < DL; ++d) acc[i][d] = 0.f;
  float m_run = kNegInf, l_run = 0.f;  // for head `col` (replicated over s)

  const int beg = split * p.split_len;
  const int end = min(beg + p.split_len, Leff);
  const int n_iter = end > beg ? (end - beg + 4 * kDenseSub - 1) / (4 * kDenseSub) : 0;
  for (int it = 0; it < n_iter; ++it) {
    const int c0 = beg + (it * 4 + w) * kDenseSub;
    const bool active = c0 < end;
    // V rows of the unit's first two value heads ride in the K load burst
    typename VL::Raw v0[kDenseSub], v1[kDenseSub];
    if (active) {
      constexpr int NT = kDenseSub / 16;
      u32x4 kf[NT][NLOAD];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int pos = min(c0 + 16 * t + col, p.L - 1);
        const char* krow = kbase + static_cast<int64_t>(pos) * p.k_sl * E::kBytes;
#pragma unroll
        for (int j = 0; j < NLOAD; ++j) kf[t][j] = ld16(krow + (j * 4 * E16 + s * E16) * E::kBytes);
      }
      const char* vb0 = vlane + static_cast<int64_t>(vh_first) * p.v_sh * E::kBytes;
#pragma unroll
      for (int i = 0; i < kDenseSub; ++i) v0[i] = VL::load(vb0 + static_cast<int64_t>(min(c0 + i, p.L - 1)) * vrow);
      if (vh_last > vh_first) {
        const char* vb1 = vlane + static_cast<int64_t>(vh_first + 1) * p.v_sh * E::kBytes;
#pragma unroll
        for (int i = 0; i < kDenseSub; ++i) v1[i] = VL::load(vb1 + static_cast<int64_t>(min(c0 + i, p.L - 1)) * vrow);
      }
      __builtin_amdgcn_sched_barrier(0);  // the K and V burst stays in flight together
      float x[NT][4];
      float mt = kNegInf;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NLOAD; ++j) a = mfma_16b<DT>(kf[t][j], qf[j], a);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int pos = c0 + 16 * t + 4 * s + r;
          float v = a[r] * p.scale;
          if (p.mask) {
            const int mp = min(pos, p.L - 1);
            v = v + load_as_f32(p.mask, p.mask_dt, bi * p.m_sb + static_cast<int64_t>(h) * p.m_sh +
                                                       static_cast<int64_t>(mp) * p.m_sl);
          }
          if (pos >= end) v = kNegInf;
          x[t][r] = v;
          mt = fmaxf(mt, v);
        }
      }
      mt = fmaxf(mt, __shfl_xor(mt, 16));
      mt = fmaxf(mt, __shfl_xor(mt, 32));
      const float m_new = fmaxf(m_run, mt);
      const float alpha = (m_run == kNegInf) ? (m_new == kNegInf ? 1.f : 0.f) : __expf(m_run - m_new);
      float ps = 0.f;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f32x4 e4;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float e = m_new == kNegInf ? 0.f : __expf(x[t][r] - m_new);
          ps += e;
          e4[r] = e;
        }
        *reinterpret_cast<f32x4*>(&Ps[w][col][16 * t + 4 * s]) = e4;
      }
      ps += __shfl_xor(ps, 16);
      ps += __shfl_xor(ps, 32);
      l_run = l_run * alpha + ps;
      m_run = m_new;
      if (s == 0) Al[w][col] = alpha;
    }
    dense_wave_sync();  // this wave's P and alpha (waves advance independently)
    if (active) {
      {
        const f32x4* a4 = reinterpret_cast<const f32x4*>(&Al[w][0]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 a = a4[q];
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int d = 0; d < DL; ++d) acc[4 * q + e][d] *= a[e];
        }
      }
      for (int vh = vh_first; vh <= vh_last; ++vh) {
        const int u = vh - vh_first;
        float vf[kDenseSub][DL];
        if (u == 1) {
#pragma unroll
          for (int i = 0; i < kDenseSub; ++i) VL::unpack(v1[i], vf[i]);
        } else {
          if (u >= 2) {  // further value heads: a load burst of their own
            const char* vb = vlane + static_cast<int64_t>(vh) * p.v_sh * E::kBytes;
#pragma unroll
            for (int i = 0; i < kDenseSub; ++i) v0[i] = VL::load(vb + static_cast<int64_t>(min(c0 + i, p.L - 1)) * vrow);
          }
#pragma unroll
          for (int i = 0; i < kDenseSub; ++i) VL::unpack(v0[i], vf[i]);
        }
        const int hb = max(vh * g_v, h0) - h0, he = min((vh + 1) * g_v, h0 + g) - h0;  // unit-local heads
#pragma unroll
        for (int hh = 0; hh < 16; ++hh) {
          if (hh >= hb && hh < he) {
            const f32x4* p4 = reinterpret_cast<const f32x4*>(&Ps[w][hh][0]);
#pragma unroll
            for (int i4 = 0; i4 < kDenseSub / 4; ++i4) {
              const f32x4 pw = p4[i4];
#pragma unroll
              for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int d = 0; d < DL; ++d) acc[hh][d] += pw[k] * vf[4 * i4 + k][d];
            }
          }
        }
      }
    }
    dense_wave_sync();  // P is rewritten by this wave's next step
  }

  if (s == 0) {
    Wm[w][col] = m_run;
    Wl[w][col] = l_run;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int d = 0; d < DL; ++d) Wo[w][i][lane * DL + d] = acc[i][d];
  __syncthreads();

  // merge the four waves: the split's partial, or the output when nsplit == 1
  float* part = p.part + (static_cast<int64_t>(unit) * p.nsplit + split) * g * (2 + D);
  for (int e = tid; e < g * D; e += 256) {
    const int hh = e / D, dd = e - hh * D;
    float M = kNegInf;
#pragma unroll
    for (int q = 0; q < 4; ++q) M = fmaxf(M, Wm[q][hh]);
    float l = 0.f, o = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float f = Wm[q][hh] == kNegInf ? 0.f : __expf(Wm[q][hh] - M);
      l += Wl[q][hh] * f;
      o += Wo[q][hh][dd] * f;
    }
    if (p.nsplit == 1) {
      store_from_f32(p.out, p.out_dt, bi * p.o_sb + static_cast<int64_t>(h0 + hh) * p.o_sh + dd, o / l);
    } else {
      part[hh * (2 + D) + 2 + dd] = o;
      if (dd == 0) {
        part[hh * (2 + D)] = M;
        part[hh * (2 + D) + 1] = l;
      }
    }
  }
}

// Merge the split partials of one (batch, head): block of D threads.
// Kernel 2: one block per head, kMergeGroups x D threads: thread (grp, i)
// sums dim i of the splits grp, grp + kMergeGroups, ... (all of its loads in
// one burst for up to kMergeGroups x kMergeBurst splits), then the groups
// are added in LDS in a fixed order.
constexpr int kMergeGroups = 8;
constexpr int kMergeBurst = 8;

template <int D>
__global__ void __launch_bounds__(kMergeGroups * D) dense_merge_kernel(DenseParams p) {
  constexpr int NT = kMergeGroups * D;
  __shared__ float fm[1024];
  __shared__ float red[NT / kWave];
  __shared__ float og[kMergeGroups][D];
  const int unit = blockIdx.x / p.g, hh = blockIdx.x - unit * p.g;
  const int bi = unit / p.k_h, kh = unit - bi * p.k_h;
  const int tid = threadIdx.x, grp = tid / D, i = tid - grp * D;
  const int64_t stride = static_cast<int64_t>(p.g) * (2 + D);  // between splits
  const float* base = p.part + static_cast<int64_t>(unit) * p.nsplit * stride + hh * (2 + D);
  // (max, sum) of every split, then the common max
  float mloc = kNegInf;
  for (int q = tid; q < p.nsplit; q += NT) {
    const float m = base[q * stride];
    fm[q] = m;
    mloc = fmaxf(mloc, m);
  }
  const float M = block_max<NT / kWave>(mloc, red);
  float lloc = 0.f;
  for (int q = tid; q < p.nsplit; q += NT) {
    const float f = fm[q] == kNegInf ? 0.f : __expf(fm[q] - M);
    lloc += base[q * stride + 1] * f;
    fm[q] = f;
  }
  const float l = block_sum<NT / kWave>(lloc, red);  // orders the fm writes too
  // dim i of this group's splits: independent loads, kMergeBurst in flight
  float o = 0.f;
  for (int q0 = grp; q0 < p.nsplit; q0 += kMergeGroups * kMergeBurst) {
    float ov[kMergeBurst];
#pragma unroll
    for (int u = 0; u < kMergeBurst; ++u) {
      const int q = q0 + u * kMergeGroups;
      ov[u] = q < p.nsplit ? base[q * stride + 2 + i] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kMergeBurst; ++u) {
      const int q = q0 + u * kMergeGroups;
      if (q < p.nsplit) o += ov[u] * fm[q];
    }
  }
  og[grp][i] = o;
  __syncthreads();
  if (grp == 0) {
    float t = og[0][i];
#pragma unroll
    for (int g2 = 1; g2 < kMergeGroups; ++g2) t += og[g2][i];
    store_from_f32(p.out, p.out_dt, bi * p.o_sb + static_cast<int64_t>(kh * p.g + hh) * p.o_sh + i, t / l);
  }
}

template <int DT>
static hipError_t launch_dense_typed(int d, const DenseParams& p, hipStream_t st) {
  const unsigned blocks = static_cast<unsigned>(p.b * p.k_h * p.nsplit);
  const unsigned heads = static_cast<unsigned>(p.b * p.k_h * p.g);
  if (d == 128) {
    hipLaunchKernelGGL((dense_split_kernel<DT, 128, kDenseSubDefault>), dim3(blocks), dim3(256), 0, st, p);
    if (p.nsplit > 1)
      hipLaunchKernelGGL((dense_merge_kernel<128>), dim3(heads), dim3(kMergeGroups * 128), 0, st, p);
  } else {
    hipLaunchKernelGGL((dense_split_kernel<DT, 64, kDenseSubDefault>), dim3(blocks), dim3(256), 0, st, p);
    if (p.nsplit > 1)
      hipLaunchKernelGGL((dense_merge_kernel<64>), dim3(heads), dim3(kMergeGroups * 64), 0, st, p);
  }
  return hipGetLastError();
}

hipError_t launch_dense_decode(int dtype, int d, const DenseParams& p, hipStream_t st) {
  if (dtype == SAGA_DTYPE_BF16) return launch_dense_typed<SAGA_DTYPE_BF16>(d, p, st);
  if (dtype == SAGA_DTYPE_F16) return launch_dense_typed<SAGA_DTYPE_F16>(d, p, st);
  return launch_dense_typed<SAGA_DTYPE_F32>(d, p, st);
}

}  // namespace saga

// Dense decode attention, split-L (flash-decoding), one pass over K and V.
//
// Replaces full_einsum_forward (attention/attention.py:64-85) for l_q == 1:
// it serves the layers exempt from Atop-N, SAGA with full attention and the
// dense-GQA comparator.  A block owns one (batch, key head) unit and one
// split of the positions; its four waves step through 32-position
// sub-chunks in lockstep:
//   * QK on MFMA exactly as the score kernel (K rows -> A fragments, the
//     g <= 16 query heads of the unit -> B fragment),
//   * online softmax per head (running max / sum, rescale factor alpha),
//   * P (fp32) through LDS, then P . V on the VALU in fp32: one V row per
//     wave instruction, two dims per lane, accumulators for every head of
//     the unit; heads read value head h / (q_h / v_h), so a unit may touch
//     several value heads (SAGA: 1 key head, 2 value heads).
// Waves merge in LDS, splits write (max, sum, o[d]) partials, and the last
// block of a unit to arrive merges them and writes the output.
#include "common.cuh"
#include "kernels.h"

namespace saga {

constexpr int kDenseSub = 32;  // positions per wave step (2 MFMA tiles)

template <int DT>
__device__ __forceinline__ void load_v2(const char* p, float& a, float& b) {
  if constexpr (DT == SAGA_DTYPE_F32) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(p);
    a = __uint_as_float(v.x);
    b = __uint_as_float(v.y);
  } else {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(p);
    a = Elt<DT>::to_f32(v & 0xffffu);
    b = Elt<DT>::to_f32(v >> 16);
  }
}

template <int DT, int D>
__global__ void __launch_bounds__(256) dense_decode_kernel(DenseParams p) {
  using E = Elt<DT>;
  constexpr int E16 = E::kPer16B;
  constexpr int NLOAD = D / (4 * E16);
  constexpr int LPR = D / 2;            // lanes per V row, 2 dims each
  constexpr int RPI = kWave / LPR;      // V rows per wave load (1 or 2)
  constexpr int NVL = kDenseSub / RPI;  // V loads per value head per sub-chunk
  __shared__ float Ps[4][kDenseSub][16];
  __shared__ float Al[4][16];
  __shared__ float Wm[4][16], Wl[4][16];
  __shared__ float Wo[4][16][D];
  __shared__ int is_last;

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
  const int dim = 2 * (lane % LPR);  // this lane's two dims of a V row
  const int rpar = lane / LPR;       // row parity for D = 64

  float acc[16][2];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i][0] = acc[i][1] = 0.f;
  float m_run = kNegInf, l_run = 0.f;  // for head `col` (replicated over s)

  const int beg = split * p.split_len;
  const int end = min(beg + p.split_len, Leff);
  const int n_iter = end > beg ? (end - beg + 4 * kDenseSub - 1) / (4 * kDenseSub) : 0;
  for (int it = 0; it < n_iter; ++it) {
    const int c0 = beg + (it * 4 + w) * kDenseSub;
    const bool active = c0 < end;
    float x[2][4];
    if (active) {
      u32x4 kf[2][NLOAD];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int pos = min(c0 + 16 * t + col, p.L - 1);
        const char* krow = kbase + static_cast<int64_t>(pos) * p.k_sl * E::kBytes;
#pragma unroll
        for (int j = 0; j < NLOAD; ++j) kf[t][j] = ld16(krow + (j * 4 * E16 + s * E16) * E::kBytes);
      }
      float mt = kNegInf;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
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
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float e = m_new == kNegInf ? 0.f : __expf(x[t][r] - m_new);
          ps += e;
          Ps[w][16 * t + 4 * s + r][col] = e;
        }
      ps += __shfl_xor(ps, 16);
      ps += __shfl_xor(ps, 32);
      l_run = l_run * alpha + ps;
      m_run = m_new;
      if (s == 0) Al[w][col] = alpha;
    }
    __syncthreads();
    if (active) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float a = Al[w][i];
        acc[i][0] *= a;
        acc[i][1] *= a;
      }
      for (int vh = vh_first; vh <= vh_last; ++vh) {
        const int hb = max(vh * g_v, h0) - h0, he = min((vh + 1) * g_v, h0 + g) - h0;  // unit-local heads
        const char* vbase = p.v + (bi * p.v_sb + static_cast<int64_t>(vh) * p.v_sh + dim) * E::kBytes;
        float va[NVL], vb[NVL];
#pragma unroll
        for (int i = 0; i < NVL; ++i) {
          const int pos = min(c0 + i * RPI + rpar, p.L - 1);
          load_v2<DT>(vbase + static_cast<int64_t>(pos) * p.v_sl * E::kBytes, va[i], vb[i]);
        }
#pragma unroll
        for (int i = 0; i < NVL; ++i) {
          const int prow = i * RPI + rpar;
#pragma unroll
          for (int hh = 0; hh < 16; ++hh) {
            if (hh >= hb && hh < he) {
              const float pw = Ps[w][prow][hh];
              acc[hh][0] += pw * va[i];
              acc[hh][1] += pw * vb[i];
            }
          }
        }
      }
    }
    __syncthreads();
  }

  // rows of the other parity (D = 64) hold the same dims
  if constexpr (RPI == 2) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc[i][0] += __shfl_xor(acc[i][0], 32);
      acc[i][1] += __shfl_xor(acc[i][1], 32);
    }
  }
  if (s == 0) {
    Wm[w][col] = m_run;
    Wl[w][col] = l_run;
  }
  if (lane < LPR) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      Wo[w][i][dim] = acc[i][0];
      Wo[w][i][dim + 1] = acc[i][1];
    }
  }
  __syncthreads();

  // merge the four waves; split partial (or the output when nsplit == 1)
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
  if (p.nsplit == 1) return;

  __threadfence();
  __syncthreads();
  if (tid == 0) is_last = atomicAdd(p.counters + unit, 1) == p.nsplit - 1;
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  const float* pu = p.part + static_cast<int64_t>(unit) * p.nsplit * g * (2 + D);
  for (int e = tid; e < g * D; e += 256) {
    const int hh = e / D, dd = e - hh * D;
    float M = kNegInf;
    for (int q = 0; q < p.nsplit; ++q) M = fmaxf(M, pu[(q * g + hh) * (2 + D)]);
    float l = 0.f, o = 0.f;
    for (int q = 0; q < p.nsplit; ++q) {
      const float* pp = pu + (q * g + hh) * (2 + D);
      const float f = pp[0] == kNegInf ? 0.f : __expf(pp[0] - M);
      l += pp[1] * f;
      o += pp[2 + dd] * f;
    }
    store_from_f32(p.out, p.out_dt, bi * p.o_sb + static_cast<int64_t>(h0 + hh) * p.o_sh + dd, o / l);
  }
  if (tid == 0) p.counters[unit] = 0;
}

template <int DT>
static hipError_t launch_dense_typed(int d, const DenseParams& p, hipStream_t st) {
  const unsigned blocks = static_cast<unsigned>(p.b * p.k_h * p.nsplit);
  if (d == 128)
    hipLaunchKernelGGL((dense_decode_kernel<DT, 128>), dim3(blocks), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((dense_decode_kernel<DT, 64>), dim3(blocks), dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_dense_decode(int dtype, int d, const DenseParams& p, hipStream_t st) {
  if (dtype == SAGA_DTYPE_BF16) return launch_dense_typed<SAGA_DTYPE_BF16>(d, p, st);
  if (dtype == SAGA_DTYPE_F16) return launch_dense_typed<SAGA_DTYPE_F16>(d, p, st);
  return launch_dense_typed<SAGA_DTYPE_F32>(d, p, st);
}

}  // namespace saga

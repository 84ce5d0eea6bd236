// Block-level sparse softmax . V (NT threads = NT / 16 lane groups of 16 lanes).
//
// The selected positions and their logits (or probabilities) sit in LDS.
// Lane c of group G owns dims [c*DPL, c*DPL + DPL) of the head dim and walks
// entries G, G + NT/16, ...; UNROLL V rows per group are in flight at a time
// (raw 16-byte fragments): a 1024-thread block with the default 8 keeps 512
// rows (128 KiB of bf16 V) of gathers outstanding.  Lists longer than one LDS batch are
// accumulated with a running max and rescaled sums (online softmax).
#pragma once

#include "common.cuh"

namespace saga {

constexpr int kBlkThreads = 1024;
constexpr int kBlkWaves = kBlkThreads / kWave;  // 16
constexpr int kBlkGroups = kBlkThreads / 16;    // 64 lane groups
constexpr int kPVUnroll = 8;

template <int DT, int D, int NT = kBlkThreads, int UNROLL = kPVUnroll>
struct BlockPV {
  static constexpr int NW = NT / kWave;      // waves
  static constexpr int NG = NT / 16;         // lane groups
  static constexpr int DPL = D / 16;                   // dims per lane
  static constexpr int BYTES = DPL * Elt<DT>::kBytes;  // bytes per lane per row (8, 16 or 32)
  static constexpr int NV = BYTES >= 16 ? BYTES / 16 : 1;
  float acc[DPL];
  float m;  // running max (logits) -- identical in every thread
  float l;  // running sum of weights

  __device__ void init() {
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
    m = kNegInf;
    l = 0.f;
  }

  __device__ static void load_raw(const char* p, u32x4* raw) {
    if constexpr (BYTES >= 16) {
#pragma unroll
      for (int i = 0; i < NV; ++i) raw[i] = ld16(p + 16 * i);
    } else {
      const u32x2 v = *reinterpret_cast<const u32x2*>(p);
      raw[0] = u32x4{v.x, v.y, 0u, 0u};
    }
  }

  __device__ static void unpack(const u32x4* raw, float* f) {
    if constexpr (BYTES >= 16) {
#pragma unroll
      for (int i = 0; i < NV; ++i) unpack16<DT>(raw[i], f + i * (16 / Elt<DT>::kBytes));
    } else {
      f[0] = Elt<DT>::to_f32(raw[0].x & 0xffffu);
      f[1] = Elt<DT>::to_f32(raw[0].x >> 16);
      f[2] = Elt<DT>::to_f32(raw[0].y & 0xffffu);
      f[3] = Elt<DT>::to_f32(raw[0].y >> 16);
    }
  }

  // Add n entries: positions sidx[0..n), logits / probabilities sval[0..n)
  // (overwritten with the weights).  vbase points at dim 0 of position 0 of
  // the value head; vrow is the byte stride between positions.  All threads
  // of the block must call it.
  __device__ void add(int n, const int* sidx, float* sval, const char* vbase, int64_t vrow, bool probs,
                      float* red) {
    const int tid = threadIdx.x;
    float scale_old = 1.f;
    if (!probs) {
      float cm = kNegInf;
      for (int i = tid; i < n; i += NT) cm = fmaxf(cm, sval[i]);
      cm = block_max<NW>(cm, red);
      const float mn = fmaxf(m, cm);
      scale_old = (m == kNegInf) ? 0.f : __expf(m - mn);
      float ls = 0.f;
      for (int i = tid; i < n; i += NT) {
        const float w = mn == kNegInf ? 0.f : __expf(sval[i] - mn);
        sval[i] = w;
        ls += w;
      }
      ls = block_sum<NW>(ls, red);  // also orders the weight writes
      l = l * scale_old + ls;
      m = mn;
    } else {
      float ls = 0.f;
      for (int i = tid; i < n; i += NT) ls += sval[i];
      ls = block_sum<NW>(ls, red);
      l += ls;
    }
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] *= scale_old;

    const int G = tid >> 4, c = tid & 15;
    const char* vb = vbase + static_cast<int64_t>(c) * BYTES;
    for (int e0 = G; e0 < n; e0 += NG * UNROLL) {
      u32x4 raw[UNROLL][NV];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int e = e0 + u * NG;
        if (e < n) load_raw(vb + static_cast<int64_t>(sidx[e]) * vrow, raw[u]);
      }
      __builtin_amdgcn_sched_barrier(0);  // all gathers in flight before the FMAs
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int e = e0 + u * NG;
        if (e < n) {
          const float w = sval[e];
          float f[DPL];
          unpack(raw[u], f);
#pragma unroll
          for (int i = 0; i < DPL; ++i) acc[i] += w * f[i];
        }
      }
    }
  }

  // Sum the lane groups: on return, thread i < D holds sum_e w_e * V[e, i]
  // (unnormalised).  accs: LDS of NW * D floats.
  __device__ float reduce(float* accs) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, c = tid & 15;
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      acc[i] += __shfl_xor(acc[i], 16);
      acc[i] += __shfl_xor(acc[i], 32);
    }
    if (lane < 16) {
#pragma unroll
      for (int i = 0; i < DPL; ++i) accs[w * D + c * DPL + i] = acc[i];
    }
    __syncthreads();
    float o = 0.f;
    if (tid < D) {
#pragma unroll
      for (int q = 0; q < NW; ++q) o += accs[q * D + tid];
    }
    return o;
  }

  // Reduce and write out[off + i] = o_i / l (probs: / max(l, 1e-12)).
  __device__ void finish(float* accs, void* out, int out_dt, int64_t off, bool probs) {
    const float o = reduce(accs);
    if (threadIdx.x < D) {
      const float den = probs ? fmaxf(l, 1e-12f) : l;
      store_from_f32(out, out_dt, off + threadIdx.x, o / den);
    }
  }
};

}  // namespace saga

// K3: sparse softmax . V over the selected positions of each row.
//
// Replaces _atopn_gather_and_output (attention/attention.py:152-170): the
// reference materialises value[:, :, None].expand(...).gather(...) -- a copy
// of every selected V row per query head -- and runs a bmm over it.  Here a
// block owns one piece (`piece` entries) of one row's selection list: it
// computes the piece-local max, exp weights and their sum, and streams only
// the selected V rows (16 lanes x 16 bytes per 128-dim bf16 row), keeping
// an fp32 accumulator per lane.  Pieces write (max, sum, o[d]) partials; the
// last block of a row to arrive (device-scope counter) merges them and
// writes the output, then rearms the counter.  Blocks are mapped so that the
// pieces of one (batch, value head) group run on the same XCD, where the V
// rows shared by the heads of the group stay in that XCD's L2.
#include "common.cuh"
#include "kernels.h"

namespace saga {

constexpr int kPVThreads = 256;
constexpr int kPVGroups = kPVThreads / 16;  // lane groups of 16, one V row each

// Load DPL consecutive elements of a V row as floats.
template <int DT, int DPL>
__device__ __forceinline__ void load_row_piece(const char* ptr, float* out) {
  constexpr int kBytes = Elt<DT>::kBytes * DPL;
  if constexpr (kBytes == 16) {
    unpack16<DT>(ld16(ptr), out);
  } else if constexpr (kBytes == 32) {
    unpack16<DT>(ld16(ptr), out);
    unpack16<DT>(ld16(ptr + 16), out + 16 / Elt<DT>::kBytes);
  } else {  // 8 bytes: 4 x 16-bit
    const u32x2 v = *reinterpret_cast<const u32x2*>(ptr);
    out[0] = Elt<DT>::to_f32(v.x & 0xffffu);
    out[1] = Elt<DT>::to_f32(v.x >> 16);
    out[2] = Elt<DT>::to_f32(v.y & 0xffffu);
    out[3] = Elt<DT>::to_f32(v.y >> 16);
  }
}

template <int DT, int D>
__global__ void __launch_bounds__(kPVThreads) sparse_pv_kernel(PVParams p) {
  constexpr int DPL = D / 16;  // dims per lane
  __shared__ float wts[kPVThreads];
  __shared__ int ids[kPVThreads];
  __shared__ float red[4];
  __shared__ float accs[4][D];
  __shared__ int is_last;

  // XCD-aware mapping: hardware dispatches block i to XCD i % 8, so XCD x
  // gets the contiguous item range [x*per_xcd, (x+1)*per_xcd).  Items are
  // row-major (row, piece) and rows of one value group are adjacent.
  const int nitems = p.b * p.q_h * p.npiece;
  const int per_xcd = (nitems + 7) / 8;
  const int slot = blockIdx.x >> 3;
  const int item = (blockIdx.x & 7) * per_xcd + slot;
  if (slot >= per_xcd || item >= nitems) return;
  const int r = item / p.npiece;
  const int pc = item - r * p.npiece;
  const int bi = r / p.q_h, h = r - bi * p.q_h;
  const int vh = h / (p.q_h / p.v_h);
  const int tid = threadIdx.x;

  const int n_all = p.cnt ? min(p.cnt[r], p.K) : p.K;
  const int lo = pc * p.piece;
  const int n = max(min(lo + p.piece, n_all) - lo, 0);

  float xv = kNegInf;
  int id = 0;
  if (tid < n) {
    const int64_t o = static_cast<int64_t>(r) * p.w_ld + lo + tid;
    xv = load_as_f32(p.w, p.w_dt, o);
    const int64_t io = static_cast<int64_t>(r) * p.i_ld + lo + tid;
    const int64_t raw = p.idx_i64 ? static_cast<const int64_t*>(p.idx)[io]
                                  : static_cast<int64_t>(static_cast<const int32_t*>(p.idx)[io]);
    // An index outside [0, L) (torch.gather would raise) poisons the row
    // with NaN instead of reading out of bounds.
    if (raw < 0 || raw >= p.L) {
      xv = __builtin_nanf("");
      id = 0;
    } else {
      id = static_cast<int>(raw);
    }
  }
  float m, wgt;
  if (p.probs_mode) {
    m = 0.f;
    wgt = tid < n ? xv : 0.f;
  } else {
    m = block_max<4>(xv, red);
    wgt = (tid < n && m != kNegInf) ? __expf(xv - m) : 0.f;
  }
  const float l = block_sum<4>(wgt, red);
  wts[tid] = wgt;
  ids[tid] = id;
  __syncthreads();

  const int G = tid >> 4, c = tid & 15;
  const int64_t vrow_stride = p.v_sl * Elt<DT>::kBytes;
  const char* vbase = p.v + (bi * p.v_sb + static_cast<int64_t>(vh) * p.v_sh + c * DPL) * Elt<DT>::kBytes;
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
  // four rows in flight per lane group per iteration
  for (int e0 = G; e0 < n; e0 += 4 * kPVGroups) {
    float vv[4][DPL];
    float we[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = e0 + u * kPVGroups;
      const bool ok = e < n;
      we[u] = ok ? wts[e] : 0.f;
      const int pos = ok ? ids[e] : ids[0];
      load_row_piece<DT, DPL>(vbase + static_cast<int64_t>(pos) * vrow_stride, vv[u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (e0 + u * kPVGroups < n) {
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] += we[u] * vv[u][i];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    acc[i] += __shfl_xor(acc[i], 16);
    acc[i] += __shfl_xor(acc[i], 32);
  }
  const int lane = tid & 63, w = tid >> 6;
  if (lane < 16) {
#pragma unroll
    for (int i = 0; i < DPL; ++i) accs[w][c * DPL + i] = acc[i];
  }
  __syncthreads();

  if (p.npiece == 1) {
    if (tid < D) {
      const float o = accs[0][tid] + accs[1][tid] + accs[2][tid] + accs[3][tid];
      const float den = p.probs_mode ? fmaxf(l, 1e-12f) : l;
      store_from_f32(p.out, p.out_dt, bi * p.o_sb + static_cast<int64_t>(h) * p.o_sh + tid, o / den);
    }
    return;
  }

  float* part = p.part + (static_cast<int64_t>(r) * p.npiece + pc) * (2 + D);
  if (tid < D) part[2 + tid] = accs[0][tid] + accs[1][tid] + accs[2][tid] + accs[3][tid];
  if (tid == 0) {
    part[0] = m;
    part[1] = l;
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) is_last = atomicAdd(p.counters + r, 1) == p.npiece - 1;
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  const float* prow = p.part + static_cast<int64_t>(r) * p.npiece * (2 + D);
  float M = kNegInf;
  for (int q = 0; q < p.npiece; ++q) M = fmaxf(M, prow[q * (2 + D)]);
  float Ls = 0.f, O = 0.f;
  for (int q = 0; q < p.npiece; ++q) {
    const float mq = prow[q * (2 + D)];
    const float f = p.probs_mode ? 1.f : (mq == kNegInf ? 0.f : __expf(mq - M));
    Ls += prow[q * (2 + D) + 1] * f;
    if (tid < D) O += prow[q * (2 + D) + 2 + tid] * f;
  }
  if (tid < D) {
    const float den = p.probs_mode ? fmaxf(Ls, 1e-12f) : Ls;
    store_from_f32(p.out, p.out_dt, bi * p.o_sb + static_cast<int64_t>(h) * p.o_sh + tid, O / den);
  }
  if (tid == 0) p.counters[r] = 0;
}

template <int DT>
static hipError_t launch_pv_typed(const PVParams& p, hipStream_t st) {
  const int nitems = p.b * p.q_h * p.npiece;
  const int blocks = 8 * ((nitems + 7) / 8);
  if (p.d == 128)
    hipLaunchKernelGGL((sparse_pv_kernel<DT, 128>), dim3(blocks), dim3(kPVThreads), 0, st, p);
  else
    hipLaunchKernelGGL((sparse_pv_kernel<DT, 64>), dim3(blocks), dim3(kPVThreads), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_sparse_pv(const PVParams& p, hipStream_t st) {
  if (p.v_dt == SAGA_DTYPE_BF16) return launch_pv_typed<SAGA_DTYPE_BF16>(p, st);
  if (p.v_dt == SAGA_DTYPE_F16) return launch_pv_typed<SAGA_DTYPE_F16>(p, st);
  return launch_pv_typed<SAGA_DTYPE_F32>(p, st);
}

}  // namespace saga

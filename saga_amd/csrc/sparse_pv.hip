// Sparse softmax . V over caller-given selections (API path).
//
// Replaces _atopn_gather_and_output (attention/attention.py:152-170): the
// reference materialises value[:, :, None].expand(...).gather(...) -- a copy
// of every selected V row per query head -- and runs a bmm over it.  Here one
// 1024-thread block owns one row: it stages the K (weight, index) pairs in
// LDS in batches of 4096, applies softmax (logits, -inf padding weighs 0, an
// all -inf row gives NaN) or renormalisation (probabilities, 1e-12 floor),
// and gathers only the listed V rows (BlockPV).  An index outside [0, L)
// (torch.gather would raise) makes the row NaN instead of reading out of
// bounds.
#include "block_pv.cuh"
#include "kernels.h"

namespace saga {

constexpr int kPVBatch = 4096;

template <int DT, int D>
__global__ void __launch_bounds__(kBlkThreads) sparse_pv_kernel(PVParams p) {
  __shared__ int sidx[kPVBatch];
  __shared__ float sval[kPVBatch];
  __shared__ float red[kBlkWaves];
  __shared__ float accs[kBlkWaves * D];
  const int r = blockIdx.x;
  const int bi = r / p.q_h, h = r - bi * p.q_h;
  const int vh = h / (p.q_h / p.v_h);
  const int tid = threadIdx.x;
  const bool probs = p.probs_mode != 0;
  const char* vbase = p.v + (bi * p.v_sb + static_cast<int64_t>(vh) * p.v_sh) * Elt<DT>::kBytes;
  const int64_t vrow = p.v_sl * Elt<DT>::kBytes;
  BlockPV<DT, D> pv;
  pv.init();
  for (int b0 = 0; b0 < p.K; b0 += kPVBatch) {
    const int nb = min(kPVBatch, p.K - b0);
    __syncthreads();
    for (int i = tid; i < nb; i += kBlkThreads) {
      float xv = load_as_f32(p.w, p.w_dt, static_cast<int64_t>(r) * p.w_ld + b0 + i);
      const int64_t io = static_cast<int64_t>(r) * p.i_ld + b0 + i;
      const int64_t raw = p.idx_i64 ? static_cast<const int64_t*>(p.idx)[io]
                                    : static_cast<int64_t>(static_cast<const int32_t*>(p.idx)[io]);
      int id = static_cast<int>(raw);
      if (raw < 0 || raw >= p.L) {
        xv = __builtin_nanf("");
        id = 0;
      }
      sidx[i] = id;
      sval[i] = xv;
    }
    __syncthreads();
    pv.add(nb, sidx, sval, vbase, vrow, probs, red);
  }
  pv.finish(accs, p.out, p.out_dt, bi * p.o_sb + static_cast<int64_t>(h) * p.o_sh, probs);
}

template <int DT>
static hipError_t launch_pv_typed(const PVParams& p, hipStream_t st) {
  const unsigned blocks = static_cast<unsigned>(p.b * p.q_h);
  if (p.d == 128)
    hipLaunchKernelGGL((sparse_pv_kernel<DT, 128>), dim3(blocks), dim3(kBlkThreads), 0, st, p);
  else
    hipLaunchKernelGGL((sparse_pv_kernel<DT, 64>), dim3(blocks), dim3(kBlkThreads), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_sparse_pv(const PVParams& p, hipStream_t st) {
  if (p.v_dt == SAGA_DTYPE_BF16) return launch_pv_typed<SAGA_DTYPE_BF16>(p, st);
  if (p.v_dt == SAGA_DTYPE_F16) return launch_pv_typed<SAGA_DTYPE_F16>(p, st);
  return launch_pv_typed<SAGA_DTYPE_F32>(p, st);
}

}  // namespace saga

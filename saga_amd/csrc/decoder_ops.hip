// Decode-step kernels around the attention path (one launch each):
//   * rope_kv_append: the new tokens' q/k/v from the fused projection, RoPE on
//     q and k, k/v written into the separate key-head / value-head caches
//     (replaces apply_rotary_pos_emb + StaticLayer.update's index_copy_,
//     transformers models/qwen2/modeling_qwen2.py:211-214 and
//     cache_utils.py:455-487, with the caches laid out as speedup.py:119-139);
//   * rmsnorm: y = w * x / sqrt(mean(x^2) + eps) per row (Qwen2RMSNorm);
//   * silu_mul: act = silu(gate) * up over a fused [gate | up] projection.
// All arithmetic in fp32, one rounding to the storage dtype.
#include "common.cuh"
#include "kernels.h"

namespace saga {

// One 64-lane block per (token n, head hh); heads are ordered q, k, v as in
// the fused projection row.  q and k heads rotate pairs (i, i + d/2), v heads
// are copied.
__global__ void __launch_bounds__(64) rope_kv_append_kernel(RopeParams p) {
  const int n = blockIdx.x, hh = blockIdx.y;
  const int half = p.d / 2;
  const int pos = p.pos[n];
  const int b = p.batch ? p.batch[n] : n;
  const bool ok = pos >= 0 && pos < p.Lmax && b >= 0 && b < p.B;
  const int64_t base = static_cast<int64_t>(n) * p.qkv_ld + static_cast<int64_t>(hh) * p.d;
  if (hh < p.n_q + p.n_k) {
    for (int i = threadIdx.x; i < half; i += 64) {
      float cs, sn;
      rope_cos_sin(pos, i, p.d, p.theta, cs, sn);
      const float x1 = load_as_f32(p.qkv, p.dt, base + i);
      const float x2 = load_as_f32(p.qkv, p.dt, base + i + half);
      const float y1 = x1 * cs - x2 * sn;
      const float y2 = x2 * cs + x1 * sn;
      if (hh < p.n_q) {
        const int64_t qo = static_cast<int64_t>(n) * p.q_sn + static_cast<int64_t>(hh) * p.q_sh;
        store_from_f32(p.q_out, p.dt, qo + i, ok ? y1 : __builtin_nanf(""));
        store_from_f32(p.q_out, p.dt, qo + i + half, ok ? y2 : __builtin_nanf(""));
      } else if (ok) {
        const int kh = hh - p.n_q;
        const int64_t ko = b * p.k_sb + static_cast<int64_t>(kh) * p.k_sh + static_cast<int64_t>(pos) * p.k_sl;
        store_from_f32(p.k_cache, p.dt, ko + i, y1);
        store_from_f32(p.k_cache, p.dt, ko + i + half, y2);
      }
    }
  } else if (ok) {
    const int vh = hh - p.n_q - p.n_k;
    const int64_t vo = b * p.v_sb + static_cast<int64_t>(vh) * p.v_sh + static_cast<int64_t>(pos) * p.v_sl;
    for (int i = threadIdx.x; i < p.d; i += 64) store_from_f32(p.v_cache, p.dt, vo + i, load_as_f32(p.qkv, p.dt, base + i));
  }
}

hipError_t launch_rope_kv_append(const RopeParams& p, hipStream_t st) {
  hipLaunchKernelGGL(rope_kv_append_kernel, dim3(p.N, p.n_q + p.n_k + p.n_v), dim3(64), 0, st, p);
  return hipGetLastError();
}

// The rotations of a decode step's token rows, computed once per step for
// every layer's fused q/k/v projection (the same rope_cos_sin as the kernels
// that compute them in place: identical values).
__global__ void __launch_bounds__(256) rope_table_kernel(const int32_t* pos, int N, int d, float theta,
                                                         float* table) {
  const int half = d / 2;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= N * half) return;
  const int n = t / half, i = t - n * half;
  float cs, sn;
  rope_cos_sin(pos[n], i, d, theta, cs, sn);
  *reinterpret_cast<f32x2*>(table + 2 * static_cast<int64_t>(t)) = f32x2{cs, sn};
}

hipError_t launch_rope_table(const int32_t* pos, int N, int d, float theta, float* table, hipStream_t st) {
  const int total = N * (d / 2);
  hipLaunchKernelGGL(rope_table_kernel, dim3((total + 255) / 256), dim3(256), 0, st, pos, N, d, theta, table);
  return hipGetLastError();
}

// The opening of a decode step, one block per token row b: x[b] =
// embed[tokens[b]] (16-byte chunks when rows allow, else element by element,
// exact for every float dtype; a token id outside [0, V) writes a NaN row)
// and, with a table, the row's rotations as rope_table_kernel computes them.
__global__ void __launch_bounds__(256) embed_rope_kernel(EmbedParams p) {
  const int b = blockIdx.x, tid = threadIdx.x;
  const int64_t tok = p.tokens[b];
  const bool ok = tok >= 0 && tok < p.V;
  if (ok && p.vec) {
    const int64_t es = p.dt == SAGA_DTYPE_F32 ? 4 : 2;
    const char* src = static_cast<const char*>(p.embed) + tok * p.e_ld * es;
    char* dst = static_cast<char*>(p.x) + static_cast<int64_t>(b) * p.x_ld * es;
    const int chunks = static_cast<int>(p.H * es / 16);
    for (int c = tid; c < chunks; c += 256) *reinterpret_cast<u32x4*>(dst + 16 * c) = ld16(src + 16 * c);
  } else {
    for (int i = tid; i < p.H; i += 256)
      store_from_f32(p.x, p.dt, static_cast<int64_t>(b) * p.x_ld + i,
                     ok ? load_as_f32(p.embed, p.dt, tok * p.e_ld + i) : __builtin_nanf(""));
  }
  if (p.table) {
    const int half = p.d / 2;
    const int pos = p.pos[b];
    for (int i = tid; i < half; i += 256) {
      float cs, sn;
      rope_cos_sin(pos, i, p.d, p.theta, cs, sn);
      *reinterpret_cast<f32x2*>(p.table + 2 * (static_cast<int64_t>(b) * half + i)) = f32x2{cs, sn};
    }
  }
}

hipError_t launch_embed_rope(const EmbedParams& p, hipStream_t st) {
  hipLaunchKernelGGL(embed_rope_kernel, dim3(p.B), dim3(256), 0, st, p);
  return hipGetLastError();
}

// The close of a decode step: every row's position and cache length + 1.
__global__ void __launch_bounds__(256) advance_kernel(int32_t* pos, int32_t* kv_len, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  if (pos) pos[i] += 1;
  if (kv_len) kv_len[i] += 1;
}

hipError_t launch_advance(int32_t* pos, int32_t* kv_len, int n, hipStream_t st) {
  hipLaunchKernelGGL(advance_kernel, dim3((n + 255) / 256), dim3(256), 0, st, pos, kv_len, n);
  return hipGetLastError();
}

__global__ void __launch_bounds__(256) rmsnorm_kernel(RowParams p) {
  __shared__ float red[4];
  const int n = blockIdx.x;
  const int64_t xi = static_cast<int64_t>(n) * p.x_ld;
  float ss = 0.f;
  for (int i = threadIdx.x; i < p.H; i += 256) {
    const float v = load_as_f32(p.x, p.dt, xi + i);
    ss += v * v;
  }
  ss = block_sum<4>(ss, red);
  const float r = rsqrtf(ss / static_cast<float>(p.H) + p.eps);
  const int64_t yi = static_cast<int64_t>(n) * p.y_ld;
  for (int i = threadIdx.x; i < p.H; i += 256) {
    const float v = load_as_f32(p.x, p.dt, xi + i);
    store_from_f32(p.y, p.dt, yi + i, load_as_f32(p.w, p.dt, i) * (v * r));
  }
}

hipError_t launch_rmsnorm(const RowParams& p, hipStream_t st) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(p.N), dim3(256), 0, st, p);
  return hipGetLastError();
}

// y[n, i] = silu(x[n, i]) * x[n, H + i]; H = width of the output row.
__global__ void __launch_bounds__(256) silu_mul_kernel(RowParams p) {
  const int n = blockIdx.y;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= p.H) return;
  const int64_t xi = static_cast<int64_t>(n) * p.x_ld;
  const float g = load_as_f32(p.x, p.dt, xi + i);
  const float u = load_as_f32(p.x, p.dt, xi + p.H + i);
  store_from_f32(p.y, p.dt, static_cast<int64_t>(n) * p.y_ld + i, g / (1.0f + expf(-g)) * u);
}

hipError_t launch_silu_mul(const RowParams& p, hipStream_t st) {
  hipLaunchKernelGGL(silu_mul_kernel, dim3((p.H + 255) / 256, p.N), dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace saga

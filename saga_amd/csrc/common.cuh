// Device-side building blocks shared by the SAGA decode kernels (gfx950).
//
// Wave64 everywhere.  16-byte vector loads feed the MFMA operands directly:
// for v_mfma_f32_16x16x32_{bf16,f16} a lane holds 8 consecutive k-slots of
// row (lane % 16); for v_mfma_f32_16x16x4_f32 it holds 1 k-slot per MFMA, so
// one 16-byte load of 4 floats feeds 4 MFMAs.  The reduction dimension (head
// dim) may be permuted freely as long as both operands use the same
// permutation; every kernel loads lane group s = lane / 16 with the 16-byte
// piece at dims [j*4*E16 + s*E16, +E16) of MFMA step j.  The 16x16 result
// layout is row = 4*(lane/16) + reg, col = lane % 16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/saga_amd.h"

namespace saga {

constexpr int kWave = 64;
constexpr float kNegInf = -__builtin_huge_valf();

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even float -> bfloat16 bits (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  _Float16 h = __builtin_bit_cast(_Float16, b);
  return static_cast<float>(h);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

// Scalar element access by runtime dtype code (masks, small side inputs).
__device__ __forceinline__ float load_as_f32(const void* base, int dtype, int64_t off) {
  switch (dtype) {
    case SAGA_DTYPE_F32: return static_cast<const float*>(base)[off];
    case SAGA_DTYPE_BF16: return bf16_bits_to_f32(static_cast<const uint16_t*>(base)[off]);
    case SAGA_DTYPE_F16: return f16_bits_to_f32(static_cast<const uint16_t*>(base)[off]);
    case SAGA_DTYPE_BOOL: return static_cast<const uint8_t*>(base)[off] ? 1.0f : 0.0f;
    default: return 0.0f;
  }
}

__device__ __forceinline__ void store_from_f32(void* base, int dtype, int64_t off, float v) {
  switch (dtype) {
    case SAGA_DTYPE_F32: static_cast<float*>(base)[off] = v; break;
    case SAGA_DTYPE_BF16: static_cast<uint16_t*>(base)[off] = f32_to_bf16_bits(v); break;
    case SAGA_DTYPE_F16: static_cast<uint16_t*>(base)[off] = f32_to_f16_bits(v); break;
    default: break;
  }
}

// Compile-time traits of the K/Q/V element type.
template <int DT> struct Elt;
template <> struct Elt<SAGA_DTYPE_BF16> {
  static constexpr int kBytes = 2;
  static constexpr int kPer16B = 8;
  __device__ static float to_f32(uint32_t bits) { return bf16_bits_to_f32(bits & 0xffffu); }
};
template <> struct Elt<SAGA_DTYPE_F16> {
  static constexpr int kBytes = 2;
  static constexpr int kPer16B = 8;
  __device__ static float to_f32(uint32_t bits) { return f16_bits_to_f32(bits & 0xffffu); }
};
template <> struct Elt<SAGA_DTYPE_F32> {
  static constexpr int kBytes = 4;
  static constexpr int kPer16B = 4;
  __device__ static float to_f32(uint32_t bits) { return __uint_as_float(bits); }
};

// Unpack a 16-byte vector of elements to floats (8 for 16-bit types, 4 for f32).
template <int DT>
__device__ __forceinline__ void unpack16(const u32x4& v, float* out) {
  if constexpr (DT == SAGA_DTYPE_F32) {
    out[0] = __uint_as_float(v.x); out[1] = __uint_as_float(v.y);
    out[2] = __uint_as_float(v.z); out[3] = __uint_as_float(v.w);
  } else {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = Elt<DT>::to_f32(w[i] & 0xffffu);
      out[2 * i + 1] = Elt<DT>::to_f32(w[i] >> 16);
    }
  }
}

// acc += A(16 rows from a_frag lanes) * B(16 cols from b_frag lanes) over the
// k-slots held in one 16-byte fragment per lane.
template <int DT>
__device__ __forceinline__ f32x4 mfma_16b(const u32x4& a, const u32x4& b, f32x4 acc) {
  if constexpr (DT == SAGA_DTYPE_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  } else if constexpr (DT == SAGA_DTYPE_F16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
  } else {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
    return acc;
  }
}

__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Cross-lane steps on the DPP path (no LDS round trip).  GFX9 DPP controls:
// quad_perm [1,0,3,2] / [2,3,0,1], row_half_mirror, row_mirror, row_shr:n,
// row_bcast:15 / :31.
constexpr int kDppQuadXor1 = 0xB1;
constexpr int kDppQuadXor2 = 0x4E;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowShr = 0x110;
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int dpp_i(int old, int src) {
  return __builtin_amdgcn_update_dpp(old, src, CTRL, ROW_MASK, 0xf, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(v), __float_as_int(v)));
}

__device__ __forceinline__ float lane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Max / sum over the 64 lanes, returned in every lane: the four 16-lane rows
// reduce by quad and mirror permutes, then the row results are read out.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppRowMirror>(v));
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<kDppQuadXor1>(v);
  v += dpp_f<kDppQuadXor2>(v);
  v += dpp_f<kDppRowHalfMirror>(v);
  v += dpp_f<kDppRowMirror>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

// Inclusive prefix sum over the 64 lanes: row_shr 1, 2, 4, 8 scan each
// 16-lane row (lanes without a source add 0), then row_bcast:15 adds row 0's
// total to row 1 and row 2's to row 3, and row_bcast:31 adds rows 0-1 to 2-3.
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
  (void)lane;
  v += dpp_i<kDppRowShr | 1>(0, v);
  v += dpp_i<kDppRowShr | 2>(0, v);
  v += dpp_i<kDppRowShr | 4>(0, v);
  v += dpp_i<kDppRowShr | 8>(0, v);
  v += dpp_i<kDppRowBcast15, 0xa>(0, v);
  v += dpp_i<kDppRowBcast31, 0xc>(0, v);
  return v;
}

// Block barrier that publishes LDS only: it waits for the wave's LDS
// operations, not for its outstanding global stores (__syncthreads' release
// fence waits for those, one memory round trip).  Global loads after it may
// still be reordered above it: use __syncthreads where they depend on the
// barrier.
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Merge two (max, sum of exp(x - max)) pairs.  Empty sets are (-inf, 0).
__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  if (M == kNegInf) {
    m = M;
    s = 0.0f;
    return;
  }
  s = s * __expf(m - M) + s2 * __expf(m2 - M);
  m = M;
}

// Block-wide reductions; `scratch` holds one float per wave.
template <int NWAVES>
__device__ __forceinline__ float block_max(float v, float* scratch) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_max(v);
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  float r = scratch[0];
#pragma unroll
  for (int i = 1; i < NWAVES; ++i) r = fmaxf(r, scratch[i]);
  __syncthreads();
  return r;
}

template <int NWAVES>
__device__ __forceinline__ float block_sum(float v, float* scratch) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_sum(v);
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  float r = 0.0f;
#pragma unroll
  for (int i = 0; i < NWAVES; ++i) r += scratch[i];
  __syncthreads();
  return r;
}

// Order-preserving map float -> uint32 (larger float -> larger key).
__device__ __forceinline__ uint32_t f32_to_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_to_f32(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// RoPE angle of rotary pair i at position pos (Qwen2RotaryEmbedding,
// transformers models/qwen2/modeling_qwen2.py:86-120): inv_freq_i =
// 1 / theta^(2i/d) and angle = pos * inv_freq_i, both in fp32.
__device__ __forceinline__ void rope_cos_sin(int pos, int i, int d, float theta, float& c, float& s) {
  const float inv_freq = 1.0f / powf(theta, static_cast<float>(2 * i) / static_cast<float>(d));
  sincosf(static_cast<float>(pos) * inv_freq, &s, &c);
}

}  // namespace saga

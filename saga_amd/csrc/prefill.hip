// Prefill attention with separate key-head and value-head counts.
//
// The reference's prefill is torch SDPA on keys and values expanded to the
// query heads: key head h / (q_h / k_h), value head h / (q_h / v_h)
// (attention/attention.py:13-53, repeat_kv).  This kernel computes
//   out[b, q, h, :] = softmax_k(scale * q_h . k + mask) . v
// with that head map, over the caches as they lie, without expanding them.
//
// One block of NW waves (8 for d = 128, 4 for d = 64) owns 32 * NW queries of
// one (batch, query head); each wave owns 32 of them as two 16-query MFMA
// columns.  Keys are visited in tiles of
// 64 (two 32-key chunks) that the block stages in LDS, with the next tile's
// global loads in flight while the current one is multiplied:
//  * scores are computed transposed, S^T = K . Q^T (v_mfma_f32_16x16x32_bf16,
//    A = 16 key rows from LDS, B = the wave's queries held in registers), so a
//    lane holds 4 keys of one query per 16-key tile.  The K rows of a 32-key
//    chunk are stored permuted in LDS (tile t, row i <-> key 8*(i/4) + 4*t +
//    i%4), which leaves every lane with 8 consecutive keys of its query after
//    the chunk's two tiles: exactly the B operand of
//  * O^T = V^T . P^T, whose A operand (8 consecutive keys of one value dim)
//    comes from a transposed copy of the V tile in LDS, written once per tile
//    with the 16-byte units of each row XOR-swizzled by the row so that both
//    the transposed writes and the fragment reads spread over the banks;
//  * online softmax in base 2: per lane partial sums, reduced across the
//    four lane groups of a query only at the end; the running max is moved
//    (and O rescaled) only when a score exceeds it by 2^8, and the causal /
//    length masks are applied only to the tiles that cross them.
// Blocks are ordered heaviest first (causal: the last query blocks see the
// most keys) and, within one query block, by head: blocks in flight together
// share the key / value head.
#include "common.cuh"
#include "kernels.h"

namespace saga {
namespace {

constexpr int kPfBN = 64;  // keys per tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kPfRescale = 8.0f;  // log2 headroom of the running max

// waves per block: the tile loads are spread over 512 threads for d = 128
// (two 16-byte fragments per thread and operand, which keeps the kernel
// within 256 VGPRs at 2 waves per SIMD)
constexpr int pf_waves(int d) { return d == 128 ? 8 : 4; }

template <int D>
struct PfShape {
  static constexpr int NW = pf_waves(D);
  static constexpr int THREADS = 64 * NW;
  static constexpr int BM = 32 * NW;                       // queries per block
  static constexpr int NDC = D / 8;                        // 16-byte chunks per row
  static constexpr int KPT = kPfBN * NDC / THREADS;        // keys per thread in a tile load (2)
  static constexpr int NJ = D / 32;                        // MFMA k-steps over d
  static constexpr int NDT = D / 16;                       // 16-dim output tiles
  static constexpr int KROW = D / 2 + 4;                   // K row stride in dwords (4-dword pad)
  static constexpr int VROW = kPfBN / 2;                   // V^T row stride in dwords (swizzled)
};

// LDS row of tile-local key k: chunk c = k / 32, within it key 8a + 4t + b
// goes to row 16t + 4a + b.
__device__ __forceinline__ int pf_krow(int k) {
  const int w = k & 31;
  return (k & 32) + ((w >> 2) & 1) * 16 + (w >> 3) * 4 + (w & 3);
}

// 16-byte unit swizzle of V^T row d.
__device__ __forceinline__ int pf_swz(int d) { return (d ^ (d >> 3)) & 7; }

__device__ __forceinline__ u32x4 lds16(const uint32_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// Two floats -> two 16-bit elements, round to nearest even
// (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const f32x2 v = {a, b};
  if constexpr (DT == SAGA_DTYPE_BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
  }
}

// MASKED: the per-element mask path (a separate instantiation: its 64-bit
// offsets would push the unmasked kernel into spills).
template <int DT, int D, bool MASKED>
__global__ __launch_bounds__(PfShape<D>::THREADS, 2) void prefill_attn_kernel(PrefillParams p) {
  using S = PfShape<D>;
  using E = Elt<DT>;
  __shared__ __attribute__((aligned(16))) uint32_t ks[kPfBN * S::KROW];
  __shared__ __attribute__((aligned(16))) uint32_t vt[D * S::VROW];

  // the wave index through readfirstlane: every per-wave condition below is
  // then a scalar branch, not an exec-masked region issued by every wave
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int s = lane >> 4, c = lane & 15;
  const int nhb = p.q_h * p.b;
  const int id = blockIdx.x;
  const int mb = p.nmb - 1 - id / nhb;
  const int h = (id % nhb) % p.q_h, bi = (id % nhb) / p.q_h;
  const int kh = h / (p.q_h / p.k_h), vh = h / (p.q_h / p.v_h);
  const int q0 = mb * S::BM, q0w = q0 + 32 * wave;

  // keys the block needs: key <= q + causal_off for its last query
  int kend = p.Lk;
  if (p.causal) kend = min(kend, q0 + S::BM + p.causal_off);
  kend = max(kend, 0);
  const int ntiles = (kend + kPfBN - 1) / kPfBN;

  const char* kb = p.k + (bi * p.k_sb + static_cast<int64_t>(kh) * p.k_sh) * E::kBytes;
  const char* vb = p.v + (bi * p.v_sb + static_cast<int64_t>(vh) * p.v_sh) * E::kBytes;

  // the wave's queries as B fragments: lane (s, c) holds query q0w + 16 ct + c, dims 32 j + 8 s ..
  u32x4 qf[2][S::NJ];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int q = q0w + 16 * ct + c;
    const char* qr = p.q + (bi * p.q_sb + static_cast<int64_t>(h) * p.q_sh + static_cast<int64_t>(min(q, p.Lq - 1)) *
                            p.q_sl) * E::kBytes;
#pragma unroll
    for (int j = 0; j < S::NJ; ++j)
      qf[ct][j] = q < p.Lq ? ld16(qr + (32 * j + 8 * s) * E::kBytes) : u32x4{0u, 0u, 0u, 0u};
  }

  // tile loads: thread (chunk lc, key group lg) holds keys lg*KPT + i, dims 8 lc ..
  // (row pointers advance one tile per call; rows at or past Lk are not read)
  const int lc = tid % S::NDC, lg = tid / S::NDC;
  u32x4 kr[S::KPT], vr[S::KPT];
  const char* kcur = kb + (static_cast<int64_t>(lg * S::KPT) * p.k_sl + 8 * lc) * E::kBytes;
  const char* vcur = vb + (static_cast<int64_t>(lg * S::KPT) * p.v_sl + 8 * lc) * E::kBytes;
  const int64_t krow = p.k_sl * E::kBytes, vrow = p.v_sl * E::kBytes;
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < S::KPT; ++i) {
      const bool ok = k0 + lg * S::KPT + i < p.Lk;
      kr[i] = ok ? ld16(kcur + i * krow) : u32x4{0u, 0u, 0u, 0u};
      vr[i] = ok ? ld16(vcur + i * vrow) : u32x4{0u, 0u, 0u, 0u};
    }
    kcur += kPfBN * krow;
    vcur += kPfBN * vrow;
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < S::KPT; ++i) {
      *reinterpret_cast<u32x4*>(ks + pf_krow(lg * S::KPT + i) * S::KROW + 4 * lc) = kr[i];
    }
    const int kl = lg * S::KPT;  // first tile-local key of the thread
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = 8 * lc + e;
      uint32_t* row = vt + d * S::VROW + 4 * ((kl >> 3) ^ pf_swz(d)) + ((kl & 7) >> 1);
      uint32_t el[S::KPT];
#pragma unroll
      for (int i = 0; i < S::KPT; ++i) {
        const uint32_t w = vr[i][e >> 1];
        el[i] = (e & 1) ? (w >> 16) : (w & 0xffffu);
      }
      static_assert(S::KPT == 2, "one dword of two keys per V^T row write");
      *row = el[0] | (el[1] << 16);
    }
  };

  f32x4 o[2][S::NDT];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int dt = 0; dt < S::NDT; ++dt) o[ct][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mrun[2] = {kNegInf, kNegInf}, lsum[2] = {0.f, 0.f};
  const float sl2 = p.scale * kLog2e;  // > 0 (checked by the host)
  const float inv_scale = 1.0f / p.scale;

  if (ntiles > 0) load_tile(0);
  for (int it = 0; it < ntiles; ++it) {
    const int k0 = it * kPfBN;
    store_tile();
    __syncthreads();
    if (it + 1 < ntiles) load_tile(k0 + kPfBN);

    // keys of this tile that any query of the wave may see
    const bool active = !p.causal || k0 <= q0w + 31 + p.causal_off;
    if (active) {
      // S^T tiles: sc[ch][t][ct], lane (s, c) row r <-> key k0 + 32 ch + 8 s + 4 t + r, query col c
      f32x4 sc[2][2][2];
#pragma unroll
      for (int ch = 0; ch < 2; ++ch)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          u32x4 kf[S::NJ];
          const uint32_t* kp = ks + (32 * ch + 16 * t + c) * S::KROW + 4 * s;
#pragma unroll
          for (int j = 0; j < S::NJ; ++j) kf[j] = lds16(kp + 16 * j);
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < S::NJ; ++j) acc = mfma_16b<DT>(kf[j], qf[ct][j], acc);
            sc[ch][t][ct] = acc;
          }
        }

      // per-element masks only where needed: the wave's diagonal, the last
      // (partial) tile, an explicit mask
      const bool edge = MASKED || (p.causal && k0 + kPfBN - 1 > q0w + p.causal_off) || k0 + kPfBN > p.Lk;
      u32x4 pf[2][2];  // [ct][ch]: B fragments of P^T
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const int q = q0w + 16 * ct + c;
        // raw scores q.k (scaled only inside the exponent below)
        float x[2][2][4];
#pragma unroll
        for (int ch = 0; ch < 2; ++ch)
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) x[ch][t][r] = sc[ch][t][ct][r];
        if (edge) {
#pragma unroll
          for (int ch = 0; ch < 2; ++ch)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int key = k0 + 32 * ch + 8 * s + 4 * t + r;
                float v = x[ch][t][r];
                if constexpr (MASKED) {
                  const int64_t mo = bi * p.m_sb + static_cast<int64_t>(h) * p.m_sh +
                                     static_cast<int64_t>(min(q, p.Lq - 1)) * p.m_sq +
                                     static_cast<int64_t>(min(key, p.Lk - 1)) * p.m_sk;
                  if (p.mask_dt == SAGA_DTYPE_BOOL) {
                    if (!static_cast<const uint8_t*>(p.mask)[mo]) v = kNegInf;
                  } else {
                    v += load_as_f32(p.mask, p.mask_dt, mo) * inv_scale;
                  }
                }
                if (key >= p.Lk || (p.causal && key > q + p.causal_off)) v = kNegInf;
                x[ch][t][r] = v;
              }
        }
        float mx = kNegInf;
#pragma unroll
        for (int ch = 0; ch < 2; ++ch)
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, x[ch][t][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        mx *= sl2;  // base-2 units (scale > 0 keeps the max)
        // lazy rescale: the reference max moves only when a score exceeds it
        // by more than 2^8, so p <= 256 and most tiles skip the O rescale
        const bool grow = mx > mrun[ct] + kPfRescale;
        if (__any(grow)) {
          asm volatile("" ::: "memory");  // a real branch: not flattened into every tile
          const float alpha = grow ? __builtin_amdgcn_exp2f(mrun[ct] - mx) : 1.0f;
          mrun[ct] = grow ? mx : mrun[ct];
          lsum[ct] *= alpha;
#pragma unroll
          for (int dt = 0; dt < S::NDT; ++dt) o[ct][dt] *= alpha;
        }
        const float msub = mrun[ct] == kNegInf ? 0.f : mrun[ct];
        float ps = 0.f;
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) {
          float pv[8];
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              pv[4 * t + r] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[ch][t][r], sl2, -msub));
              ps += pv[4 * t + r];
            }
          pf[ct][ch] = u32x4{pack2<DT>(pv[0], pv[1]), pack2<DT>(pv[2], pv[3]), pack2<DT>(pv[4], pv[5]),
                             pack2<DT>(pv[6], pv[7])};
        }
        lsum[ct] += ps;
      }

      // O^T += V^T . P^T; A fragment: V^T row 16 dt + c, keys 32 ch + 8 s ..
#pragma unroll
      for (int dt = 0; dt < S::NDT; ++dt) {
        const int d = 16 * dt + c;
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) {
          const u32x4 vf = lds16(vt + d * S::VROW + 4 * ((4 * ch + s) ^ pf_swz(d)));
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) o[ct][dt] = mfma_16b<DT>(vf, pf[ct][ch], o[ct][dt]);
        }
      }
    }
    __syncthreads();
  }

  // out[b, q, h, 16 dt + 4 s + r] = O^T[d][q] / l; a query with no visible key gets 0
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    float l = lsum[ct];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    const int q = q0w + 16 * ct + c;
    if (q >= p.Lq) continue;
    char* orow = static_cast<char*>(p.out) +
                 (bi * p.o_sb + static_cast<int64_t>(q) * p.o_sq + static_cast<int64_t>(h) * p.o_sh) * E::kBytes;
#pragma unroll
    for (int dt = 0; dt < S::NDT; ++dt) {
      const f32x4 a = o[ct][dt] * inv;
      *reinterpret_cast<u32x2*>(orow + (16 * dt + 4 * s) * E::kBytes) =
          u32x2{pack2<DT>(a[0], a[1]), pack2<DT>(a[2], a[3])};
    }
  }
}

template <int DT>
hipError_t launch_prefill_typed(int d, const PrefillParams& p, hipStream_t st) {
  const unsigned blocks = static_cast<unsigned>(p.nmb) * static_cast<unsigned>(p.q_h * p.b);
  if (blocks == 0) return hipSuccess;
  const bool m = p.mask != nullptr;
  if (d == 128) {
    if (m) hipLaunchKernelGGL((prefill_attn_kernel<DT, 128, true>), dim3(blocks), dim3(PfShape<128>::THREADS), 0, st, p);
    else hipLaunchKernelGGL((prefill_attn_kernel<DT, 128, false>), dim3(blocks), dim3(PfShape<128>::THREADS), 0, st, p);
  } else {
    if (m) hipLaunchKernelGGL((prefill_attn_kernel<DT, 64, true>), dim3(blocks), dim3(PfShape<64>::THREADS), 0, st, p);
    else hipLaunchKernelGGL((prefill_attn_kernel<DT, 64, false>), dim3(blocks), dim3(PfShape<64>::THREADS), 0, st, p);
  }
  return hipGetLastError();
}

}  // namespace

int prefill_query_blocks(int64_t Lq, int d) {
  const int bm = 32 * pf_waves(d);
  return static_cast<int>((Lq + bm - 1) / bm);
}

hipError_t launch_prefill_attention(int dtype, int d, const PrefillParams& p, hipStream_t st) {
  if (dtype == SAGA_DTYPE_BF16) return launch_prefill_typed<SAGA_DTYPE_BF16>(d, p, st);
  return launch_prefill_typed<SAGA_DTYPE_F16>(d, p, st);
}

}  // namespace saga

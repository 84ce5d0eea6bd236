// Randomised argument fuzzing of the C ABI's host-side validation, built with
// AddressSanitizer and UndefinedBehaviorSanitizer on the host code of
// capi.hip.  Every call gets descriptors with random ndim, dtypes, shapes
// and strides (zero, negative, huge, misaligned), null or fake data
// pointers and random scalars; it must return without a sanitizer report.
// Fake pointers are never dereferenced on the host: the library validates
// first and hands device pointers only to kernels, and this program refuses
// to run where a GPU is visible (a call that passed validation would launch
// on them).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <initializer_list>

#include "saga_amd.h"

namespace {

uint64_t g_state = 0x9e3779b97f4a7c15ull;

uint64_t next() {  // splitmix64
  uint64_t z = (g_state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

template <class T, size_t N>
T pick(const T (&a)[N]) {
  return a[next() % N];
}

const int64_t kSizes[] = {-1, 0, 1, 2, 3, 5, 12, 15, 16, 63, 64, 65, 128, 1024, 4097, 1 << 20,
                          int64_t(1) << 31, int64_t(1) << 40, INT64_MAX, INT64_MIN};

int64_t rnd_size() { return (next() % 4 == 0) ? pick(kSizes) : int64_t(next() % 200); }

uintptr_t rnd_ptr() {
  const uintptr_t p[] = {0, 0x10000, 0x10002, 0x10010, 0x7fff0000};
  return pick(p);
}

saga_tensor rnd_tensor() {
  saga_tensor t;
  std::memset(&t, 0, sizeof(t));
  t.data = reinterpret_cast<void*>(rnd_ptr());
  const int32_t dts[] = {-1, 0, 1, 2, 3, 4, 5, 6, 99};
  t.dtype = pick(dts);
  const int32_t nds[] = {-1, 0, 1, 2, 3, 4, 4, 4, 5, 1000};
  t.ndim = pick(nds);
  for (int i = 0; i < 4; ++i) {
    t.shape[i] = rnd_size();
    t.stride[i] = (next() % 3 == 0) ? rnd_size() : 1;
  }
  if (next() % 2) {  // often contiguous, so that later checks run too
    int64_t acc = 1;
    for (int i = 3; i >= 0; --i) {
      t.stride[i] = acc;
      if (t.shape[i] > 0 && acc < (int64_t(1) << 40)) acc *= t.shape[i] < (1 << 20) ? t.shape[i] : 1;
    }
  }
  return t;
}

const saga_tensor* maybe(const saga_tensor& t) { return next() % 8 == 0 ? nullptr : &t; }
float rnd_float() {
  const float f[] = {0.f, -1.f, 1e-6f, 0.125f, 1.f, 1e4f, 1e30f, __builtin_inff(), __builtin_nanf("")};
  return pick(f);
}
template <class T>
T* fake(uintptr_t p) {
  return reinterpret_cast<T*>(p);
}

// A contiguous descriptor of the given shape (ndim = shape count).
saga_tensor contig(int32_t dtype, std::initializer_list<int64_t> shape, uintptr_t data = 0x100000) {
  saga_tensor t;
  std::memset(&t, 0, sizeof(t));
  t.data = reinterpret_cast<void*>(data);
  t.dtype = dtype;
  t.ndim = static_cast<int32_t>(shape.size());
  int i = 0;
  for (int64_t n : shape) t.shape[i++] = n;
  int64_t acc = 1;
  for (int j = t.ndim - 1; j >= 0; --j) {
    t.stride[j] = acc;
    if (t.shape[j] > 0 && acc <= (int64_t(1) << 40) / t.shape[j]) acc *= t.shape[j];
  }
  return t;
}

// 0-2 random edits of a well-formed descriptor.
void mutate(saga_tensor& t) {
  const int k = int(next() % 3);
  for (int m = 0; m < k; ++m) {
    const int i = int(next() % 4);
    switch (next() % 6) {
      case 0: t.shape[i] = pick(kSizes); break;
      case 1: t.stride[i] = pick(kSizes); break;
      case 2: t.dtype = int32_t(next() % 7) - 1; break;
      case 3: t.data = reinterpret_cast<void*>(rnd_ptr()); break;
      case 4: t.ndim = int32_t(next() % 6); break;
      default: t.shape[i] = int64_t(next() % 300); break;
    }
  }
}

// Shapes near the real ones and the limits: (b, q_h, k_h, v_h, L, d).
struct Cfg {
  int64_t b, q_h, k_h, v_h, L, d;
};
Cfg rnd_cfg() {
  const int64_t bs[] = {1, 2, 8, 32, 1 << 20, int64_t(1) << 31};
  const int64_t groups[][3] = {{12, 1, 2}, {15, 1, 5}, {16, 2, 8}, {6, 3, 1}, {32, 1, 2}, {4, 4, 4}};
  const int64_t Ls[] = {1, 63, 64, 4097, 33024, int64_t(1) << 29, (int64_t(1) << 30) - 1, int64_t(1) << 30};
  const int64_t ds[] = {64, 128, 96, 256};
  const auto& g = groups[next() % 6];
  return Cfg{pick(bs), g[0], g[1], g[2], pick(Ls), pick(ds)};
}

int structured(int which) {
  const Cfg c = rnd_cfg();
  const int32_t dt = next() % 4 == 0 ? SAGA_DTYPE_F32 : SAGA_DTYPE_BF16;
  saga_tensor q = contig(dt, {c.b, c.q_h, 1, c.d}), k = contig(dt, {c.b, c.k_h, c.L, c.d}),
              v = contig(dt, {c.b, c.v_h, c.L, c.d}), out = contig(dt, {c.b, c.q_h, 1, c.d}),
              mask = contig(SAGA_DTYPE_BOOL, {c.b, 1, 1, c.L});
  mutate(q);
  mutate(k);
  mutate(v);
  mutate(out);
  const saga_tensor* m = next() % 3 == 0 ? &mask : nullptr;
  const int64_t top_n = next() % 2 ? int64_t(next() % 4096) : pick(kSizes);
  void* ws = reinterpret_cast<void*>(uintptr_t(0x200000));
  const size_t wsb = next() % 2 ? (size_t(1) << 40) : size_t(next() % 100000);
  switch (which % 8) {
    case 0: return saga_atopn_decode(&q, &k, &v, m, nullptr, 0.125f, top_n, reinterpret_cast<float*>(0x300000), &out,
                                     ws, wsb, nullptr);
    case 1: return saga_atopn_calibrate(&q, &k, &v, m, nullptr, 0.125f, top_n, reinterpret_cast<float*>(0x300000),
                                        &out, ws, wsb, nullptr);
    case 2: return saga_dense_decode(&q, &k, &v, m, nullptr, 0.125f, &out, ws, wsb, nullptr);
    case 3: {
      const int64_t lq = next() % 2 ? c.L : int64_t(next() % 600);
      saga_tensor pq = contig(dt, {c.b, c.q_h, lq, c.d}), po = contig(dt, {c.b, lq, c.q_h, c.d});
      mutate(pq);
      mutate(po);
      return saga_prefill_attention(&pq, &k, &v, nullptr, 0.125f, int32_t(next() % 2), rnd_size(), &po, nullptr);
    }
    case 4: {
      saga_tensor s = contig(SAGA_DTYPE_F32, {c.b, c.q_h, 1, c.L});
      mutate(s);
      return saga_qk_scores(&q, &k, m, nullptr, 0.125f, &s, reinterpret_cast<float*>(0x400000),
                            reinterpret_cast<float*>(0x500000), nullptr);
    }
    case 5: {
      const int64_t M = int64_t(next() % 20), N = pick(kSizes) & ~int64_t(15), K = c.d * 12;
      saga_tensor x = contig(SAGA_DTYPE_BF16, {M, K}), w = contig(SAGA_DTYPE_BF16, {N, K}),
                  y = contig(SAGA_DTYPE_BF16, {M, N});
      mutate(x);
      mutate(w);
      mutate(y);
      return saga_gemv(&x, &w, nullptr, next() % 2 ? 1e-6f : 0.f, int32_t(next() % 4), &y, ws, wsb, nullptr);
    }
    case 6: {
      saga_tensor x = contig(SAGA_DTYPE_BF16, {c.b, c.L});
      mutate(x);
      return saga_argmax(&x, reinterpret_cast<int64_t*>(0x600000), ws, wsb, nullptr);
    }
    default: {
      saga_tensor w = contig(dt, {c.b * c.q_h, top_n > 0 && top_n < 4096 ? top_n : 64}),
                  idx = contig(SAGA_DTYPE_I64, {c.b * c.q_h, top_n > 0 && top_n < 4096 ? top_n : 64});
      mutate(w);
      mutate(idx);
      return saga_sparse_softmax_pv(&w, &idx, &v, int32_t(next() % 2), &out, nullptr);
    }
  }
}

}  // namespace

int main(int argc, char** argv) {
  int n = 0;
  if (hipGetDeviceCount(&n) == hipSuccess && n > 0) {
    std::printf("a GPU is visible: the fuzzer runs on hosts without one\n");
    return 0;
  }
  const long iters = argc > 1 ? std::atol(argv[1]) : 20000;
  long errors = 0, passed = 0, reached_hip = 0;
  for (long it = 0; it < iters; ++it) {
    saga_tensor a = rnd_tensor(), b = rnd_tensor(), c = rnd_tensor(), d = rnd_tensor(), e = rnd_tensor(),
                f = rnd_tensor();
    const uintptr_t p1 = rnd_ptr(), p2 = rnd_ptr(), p3 = rnd_ptr(), p4 = rnd_ptr();
    int rc = 0;
    switch (next() % 32) {
      case 0: rc = saga_qk_scores(maybe(a), maybe(b), maybe(c), fake<int32_t>(p1), rnd_float(), &d,
                                  fake<float>(p2), fake<float>(p3), nullptr); break;
      case 1: rc = saga_logit_threshold(maybe(a), fake<int32_t>(p1), fake<float>(p2), fake<float>(p3), nullptr); break;
      case 2: rc = saga_threshold_select(maybe(a), fake<float>(p1), rnd_size(), rnd_size(), &b, fake<int64_t>(p2),
                                         fake<int32_t>(p3), nullptr); break;
      case 3: rc = saga_sparse_softmax_pv(maybe(a), maybe(b), maybe(c), int32_t(next() % 3), &d, nullptr); break;
      case 4: (void)saga_atopn_workspace_bytes(rnd_size(), rnd_size(), rnd_size(), rnd_size(), rnd_size(), rnd_size());
              (void)saga_dense_workspace_bytes(rnd_size(), rnd_size(), rnd_size(), rnd_size());
              (void)saga_gemv_workspace_bytes(rnd_size(), rnd_size(), rnd_size());
              (void)saga_argmax_workspace_bytes(rnd_size(), rnd_size());
              (void)saga_qk_nparts(rnd_size(), rnd_size(), rnd_size());
              rc = -1; break;
      case 5: {
        saga_atopn_layout lay;
        rc = saga_atopn_workspace_layout(rnd_size(), rnd_size(), rnd_size(), rnd_size(), rnd_size(), rnd_size(),
                                         next() % 8 ? &lay : nullptr);
        break;
      }
      case 6: rc = saga_atopn_decode(maybe(a), maybe(b), maybe(c), next() % 2 ? nullptr : &d, fake<int32_t>(p1),
                                     rnd_float(), rnd_size(), fake<float>(p2), &e, fake<void>(p3 & ~uintptr_t(255)),
                                     size_t(rnd_size()), nullptr); break;
      case 7: rc = saga_atopn_calibrate(maybe(a), maybe(b), maybe(c), next() % 2 ? nullptr : &d, fake<int32_t>(p1),
                                        rnd_float(), rnd_size(), fake<float>(p2), &e, fake<void>(p3),
                                        size_t(rnd_size()), nullptr); break;
      case 8: rc = saga_dense_decode(maybe(a), maybe(b), maybe(c), next() % 2 ? nullptr : &d, fake<int32_t>(p1),
                                     rnd_float(), &e, fake<void>(p2), size_t(rnd_size()), nullptr); break;
      case 9: rc = saga_rope_kv_append(maybe(a), rnd_size(), rnd_size(), rnd_size(), rnd_float(), fake<int32_t>(p1),
                                       fake<int32_t>(p2), &b, &c, &d, nullptr); break;
      case 10: rc = saga_rmsnorm(maybe(a), maybe(b), rnd_float(), &c, nullptr); break;
      case 11: rc = saga_silu_mul(maybe(a), &b, nullptr); break;
      case 12: rc = saga_gemv(maybe(a), maybe(b), next() % 2 ? nullptr : &c, rnd_float(), int32_t(next() % 6) - 1, &d,
                              fake<void>(p1), size_t(rnd_size()), nullptr); break;
      case 13: rc = saga_gemv_rope_kv(maybe(a), maybe(b), next() % 2 ? nullptr : &c, rnd_float(), rnd_size(),
                                      rnd_size(), rnd_size(), rnd_float(), fake<int32_t>(p1), fake<int32_t>(p2), &d,
                                      &e, &f, next() % 2 ? nullptr : fake<float>(p3), nullptr); break;
      case 14: rc = saga_argmax(maybe(a), fake<int64_t>(p1), fake<void>(p2), size_t(rnd_size()), nullptr); break;
      case 15: rc = saga_prefill_attention(maybe(a), maybe(b), maybe(c), next() % 2 ? nullptr : &d, rnd_float(),
                                           int32_t(next() % 3), rnd_size(), &e, nullptr); break;
      case 16: rc = saga_atopn_decode_ex(maybe(a), maybe(b), maybe(c), next() % 2 ? nullptr : &d, fake<int32_t>(p1),
                                         rnd_float(), rnd_size(), fake<float>(p2), &e, int32_t(next() % 5) - 1,
                                         fake<void>(p3), size_t(rnd_size()), nullptr); break;
      case 17: rc = saga_rope_table(next() % 2 ? nullptr : fake<int32_t>(p1), rnd_size(), rnd_size(), rnd_float(),
                                    next() % 2 ? nullptr : fake<float>(p2), nullptr); break;
      case 18: rc = saga_atopn_decode(nullptr, nullptr, nullptr, nullptr, nullptr, 0.f, 0, nullptr, nullptr,
                                      nullptr, 0, nullptr); break;
      case 19: rc = saga_qk_scores(&a, &b, nullptr, nullptr, rnd_float(), maybe(c) ? &c : nullptr, nullptr,
                                   nullptr, nullptr); break;
      case 20: rc = saga_sparse_softmax_pv(&a, &b, &c, 0, &d, nullptr); (void)p4; break;
      case 21: case 22: case 23: case 24: case 25: case 26: case 27: case 28:
        rc = structured(int(next() % 8));
        break;
      case 29: rc = saga_embed_rope(next() % 2 ? nullptr : fake<int64_t>(p1), maybe(a), &b,
                                    next() % 2 ? nullptr : fake<int32_t>(p2), rnd_size(), rnd_float(),
                                    next() % 2 ? nullptr : fake<float>(p3), nullptr); break;
      case 30: rc = saga_advance_positions(next() % 2 ? nullptr : fake<int32_t>(p1),
                                           next() % 2 ? nullptr : fake<int32_t>(p2), rnd_size(), nullptr); break;
      default: rc = saga_version() == 100 ? -1 : 0; break;
    }
    if (rc == SAGA_ERR_HIP) ++reached_hip;  // validated: the launch itself found no device
    if (rc < 0) {
      ++errors;
      const char* msg = saga_last_error();
      if (!msg || std::strlen(msg) > 4096) {
        std::printf("bad error message at iteration %ld\n", it);
        return 2;
      }
    } else {
      ++passed;
    }
  }
  std::printf("calls %ld: %ld rejected (%ld of them past validation, at the launch), %ld accepted\n", iters,
              errors, reached_hip, passed);
  return 0;
}

// C ABI of libsaga_amd.so: argument validation, workspace layout and the
// launch sequences of the fused decode entry points.  Declarations and the
// reference function each entry point replaces: include/saga_amd.h.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <mutex>

#include "../../include/saga_amd.h"
#include "kernels.h"

using namespace saga;

// Scratch of saga_atopn_decode_noalloc: one copy per GPU, part of the code
// object, held until the process ends.  On the host this name is only a
// stand-in for the device copy: kernels and copies use the device address
// from hipGetSymbolAddress (scratch_ptr below), never the name itself.
static __device__ __align__(256) unsigned char scratch[SAGA_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = 0;
  return SAGA_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(SAGA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return SAGA_OK;
}

int64_t elt_size(int dt) {
  switch (dt) {
    case SAGA_DTYPE_F32: return 4;
    case SAGA_DTYPE_BF16: return 2;
    case SAGA_DTYPE_F16: return 2;
    case SAGA_DTYPE_BOOL: return 1;
    case SAGA_DTYPE_I32: return 4;
    case SAGA_DTYPE_I64: return 8;
    default: return 0;
  }
}

bool is_float(int dt) {
  return dt == SAGA_DTYPE_F32 || dt == SAGA_DTYPE_BF16 || dt == SAGA_DTYPE_F16;
}

constexpr int64_t kMaxLen = (1LL << 30);  // positions are int32 inside kernels
constexpr int kMaxGroup = 16;             // query heads per key head (one MFMA column tile)

int64_t align256(int64_t x) { return (x + 255) & ~static_cast<int64_t>(255); }

// Sizes whose Atop-N workspace arithmetic stays far inside int64 (every
// region below 2^58 bytes): the layout query and the entry points refuse others.
bool atopn_sizes_ok(int64_t b, int64_t q_h, int64_t k_h, int64_t L, int64_t d, int64_t buf_k) {
  if (b < 1 || q_h < 1 || k_h < 1 || k_h > q_h || L < 1 || L >= kMaxLen || d < 1 || d > 1024 || buf_k < 1 ||
      buf_k >= kMaxLen)
    return false;
  if (b > ((1LL << 31) - 1) / q_h) return false;
  const int64_t widest = std::max<int64_t>((L + 15) / 16 * 16 + kSliceLen, buf_k);
  return b * q_h <= (1LL << 55) / widest;
}

// Sizes >= 1, strides >= 0, and element counts and offsets that the
// index arithmetic of the entry points holds without overflow.
constexpr int64_t kMaxDim = (1LL << 31);   // a size (positions are int32 inside kernels)
constexpr int64_t kMaxSpan = (1LL << 48);  // elements, a stride, and the last element's offset
int check_dims(const saga_tensor* t, const char* name) {
  int64_t elems = 1, span = 0;
  for (int i = 0; i < t->ndim; ++i) {
    const int64_t n = t->shape[i], st = t->stride[i];
    if (n < 1) return fail(SAGA_ERR_INVALID, "%s: dim %d has size %lld", name, i, (long long)n);
    if (n >= kMaxDim || st < 0 || st > kMaxSpan)
      return fail(SAGA_ERR_INVALID, "%s: dim %d size %lld or stride %lld out of range", name, i, (long long)n,
                  (long long)st);
    if (elems > kMaxSpan / n) return fail(SAGA_ERR_UNSUPPORTED, "%s: too many elements", name);
    elems *= n;
    if (st > 0 && n - 1 > (kMaxSpan - span) / st) return fail(SAGA_ERR_UNSUPPORTED, "%s: offsets too large", name);
    span += (n - 1) * st;
  }
  return SAGA_OK;
}

int check_tensor(const saga_tensor* t, const char* name, int ndim) {
  if (!t) return fail(SAGA_ERR_INVALID, "%s: null tensor descriptor", name);
  if (!t->data) return fail(SAGA_ERR_INVALID, "%s: null data pointer", name);
  if (t->ndim != ndim) return fail(SAGA_ERR_INVALID, "%s: expected %d dims, got %d", name, ndim, t->ndim);
  int rc;
  if ((rc = check_dims(t, name))) return rc;
  if (elt_size(t->dtype) == 0) return fail(SAGA_ERR_INVALID, "%s: unknown dtype %d", name, t->dtype);
  return SAGA_OK;
}

// 16-byte vector loads of rows: aligned base and strides.
int check_vec_rows(const saga_tensor* t, const char* name) {
  const int64_t es = elt_size(t->dtype);
  if (t->stride[t->ndim - 1] != 1) return fail(SAGA_ERR_INVALID, "%s: innermost stride must be 1", name);
  if (reinterpret_cast<uintptr_t>(t->data) % 16)
    return fail(SAGA_ERR_INVALID, "%s: data pointer must be 16-byte aligned", name);
  for (int i = 0; i + 1 < t->ndim; ++i)
    if (t->shape[i] > 1 && (t->stride[i] * es) % 16)
      return fail(SAGA_ERR_INVALID, "%s: stride of dim %d must be a multiple of 16 bytes", name, i);
  return SAGA_OK;
}

struct Shape {
  int64_t b, q_h, k_h, v_h, d, L;
  int dt;
};

int check_qk(const saga_tensor* q, const saga_tensor* k, const saga_tensor* mask, Shape* s) {
  int rc;
  if ((rc = check_tensor(q, "query", 4)) || (rc = check_tensor(k, "key", 4))) return rc;
  s->b = q->shape[0];
  s->q_h = q->shape[1];
  s->d = q->shape[3];
  s->k_h = k->shape[1];
  s->L = k->shape[2];
  s->dt = q->dtype;
  if (q->shape[2] != 1) return fail(SAGA_ERR_UNSUPPORTED, "query: decode path needs l_q == 1, got %lld", (long long)q->shape[2]);
  if (!is_float(q->dtype)) return fail(SAGA_ERR_INVALID, "query: dtype must be f32, bf16 or f16");
  if (k->dtype != q->dtype) return fail(SAGA_ERR_INVALID, "key: dtype differs from query");
  if (k->shape[0] != s->b || k->shape[3] != s->d)
    return fail(SAGA_ERR_INVALID, "key: shape [%lld,%lld,%lld,%lld] does not match query [b=%lld, d=%lld]",
                (long long)k->shape[0], (long long)k->shape[1], (long long)k->shape[2], (long long)k->shape[3],
                (long long)s->b, (long long)s->d);
  if (s->d != 64 && s->d != 128) return fail(SAGA_ERR_UNSUPPORTED, "head_dim %lld not built (64, 128)", (long long)s->d);
  if (s->q_h % s->k_h) return fail(SAGA_ERR_INVALID, "q_h (%lld) not a multiple of k_h (%lld)", (long long)s->q_h, (long long)s->k_h);
  if (s->q_h / s->k_h > kMaxGroup)
    return fail(SAGA_ERR_UNSUPPORTED, "q_h / k_h = %lld > %d not built", (long long)(s->q_h / s->k_h), kMaxGroup);
  if (s->L >= kMaxLen) return fail(SAGA_ERR_UNSUPPORTED, "key length %lld too large", (long long)s->L);
  if (s->b * s->q_h >= (1LL << 31)) return fail(SAGA_ERR_UNSUPPORTED, "b * q_h too large");
  if ((rc = check_vec_rows(q, "query")) || (rc = check_vec_rows(k, "key"))) return rc;
  if (mask) {
    if ((rc = check_tensor(mask, "mask", 4))) return rc;
    if (!is_float(mask->dtype) && mask->dtype != SAGA_DTYPE_BOOL)
      return fail(SAGA_ERR_INVALID, "mask: dtype must be f32, bf16, f16 or bool");
    if ((mask->shape[0] != 1 && mask->shape[0] != s->b) || (mask->shape[1] != 1 && mask->shape[1] != s->q_h) ||
        mask->shape[2] != 1 || mask->shape[3] < s->L)
      return fail(SAGA_ERR_INVALID, "mask: shape [%lld,%lld,%lld,%lld] does not broadcast to [b, q_h, 1, L=%lld]",
                  (long long)mask->shape[0], (long long)mask->shape[1], (long long)mask->shape[2],
                  (long long)mask->shape[3], (long long)s->L);
  }
  return SAGA_OK;
}

int check_v(const saga_tensor* v, Shape* s) {
  int rc;
  if ((rc = check_tensor(v, "value", 4))) return rc;
  s->v_h = v->shape[1];
  if (v->dtype != s->dt) return fail(SAGA_ERR_INVALID, "value: dtype differs from query");
  if (v->shape[0] != s->b || v->shape[2] != s->L || v->shape[3] != s->d)
    return fail(SAGA_ERR_INVALID, "value: shape [%lld,%lld,%lld,%lld] does not match [b, v_h, L=%lld, d=%lld]",
                (long long)v->shape[0], (long long)v->shape[1], (long long)v->shape[2], (long long)v->shape[3],
                (long long)s->L, (long long)s->d);
  if (s->q_h % s->v_h) return fail(SAGA_ERR_INVALID, "q_h (%lld) not a multiple of v_h (%lld)", (long long)s->q_h, (long long)s->v_h);
  return check_vec_rows(v, "value");
}

int check_out(const saga_tensor* out, const Shape& s) {
  int rc;
  if ((rc = check_tensor(out, "out", 4))) return rc;
  if (!is_float(out->dtype)) return fail(SAGA_ERR_INVALID, "out: dtype must be f32, bf16 or f16");
  if (out->shape[0] != s.b || out->shape[1] != s.q_h || out->shape[2] != 1 || out->shape[3] != s.d)
    return fail(SAGA_ERR_INVALID, "out: shape must be [b, q_h, 1, d]");
  if (out->stride[3] != 1) return fail(SAGA_ERR_INVALID, "out: innermost stride must be 1");
  return SAGA_OK;
}

QKParams make_qk(const saga_tensor* q, const saga_tensor* k, const saga_tensor* mask, const int32_t* kv_len,
                 float scale, const Shape& s) {
  QKParams p{};
  p.q = static_cast<const char*>(q->data);
  p.q_sb = q->stride[0];
  p.q_sh = q->stride[1];
  p.k = static_cast<const char*>(k->data);
  p.k_sb = k->stride[0];
  p.k_sh = k->stride[1];
  p.k_sl = k->stride[2];
  if (mask) {
    p.mask = mask->data;
    p.mask_dt = mask->dtype;
    p.m_sb = mask->shape[0] == 1 ? 0 : mask->stride[0];
    p.m_sh = mask->shape[1] == 1 ? 0 : mask->stride[1];
    p.m_sl = mask->stride[3];
  }
  p.kv_len = kv_len;
  p.b = static_cast<int32_t>(s.b);
  p.q_h = static_cast<int32_t>(s.q_h);
  p.k_h = static_cast<int32_t>(s.k_h);
  p.g = static_cast<int32_t>(s.q_h / s.k_h);
  p.L = static_cast<int32_t>(s.L);
  p.ntiles = static_cast<int32_t>((s.L + 15) / 16);
  p.nparts = static_cast<int32_t>(qk_plan(s.b, s.k_h, s.L));
  p.scale = scale;
  return p;
}

void atopn_layout(int64_t b, int64_t q_h, int64_t k_h, int64_t L, int64_t d, int64_t buf_k, saga_atopn_layout* o) {
  const int64_t nr = b * q_h;
  const int64_t ld = (L + 15) / 16 * 16;
  const int64_t nparts = qk_plan(b, k_h, L) / 4;  // K1 partials: one per block of 4 waves
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = off;
    off = align256(off + bytes);
    return at;
  };
  o->scores_ld = ld;
  o->nparts = nparts;
  o->scores = take(nr * ld * 4);
  o->part_max = take(nr * nparts * 4);
  o->part_sum = take(nr * nparts * 4);
  o->part_tail = take(nr * nparts * 4);
  o->thresh = take(nr * 4);
  o->sel_idx = take(nr * buf_k * 4);
  o->sel_val = take(nr * buf_k * 4);
  o->sel_cnt = take(nr * 4);
  o->sel_total = take(nr * 4);
  // fast-step lists: one per 1024-position slice of a row
  const int64_t ns_max = (L + kSliceLen - 1) / kSliceLen;
  const int64_t ent_max = ns_max * std::min<int64_t>(kSliceLen, buf_k);
  o->nslice = ns_max;
  o->slice_cap = std::min<int64_t>(kSliceLen, buf_k);
  o->slice_idx = take(nr * ent_max * 4);
  o->slice_val = take(nr * ent_max * 4);
  o->slice_cnt = take(nr * ns_max * 4);
  o->slice_pre = take(nr * 2 * (ns_max + 1) * 4);
  o->slice_o = take(nr * ns_max * d * 4);
  o->slice_ml = take(nr * ns_max * 2 * 4);
  o->row_part = take(nr * kRowSplit * (d + 4) * 4);
  o->row_cnt = take(nr * 4);
  o->total_bytes = off;
}

PVParams make_pv(const saga_tensor* v, const saga_tensor* out, const Shape& s) {
  PVParams p{};
  p.v = static_cast<const char*>(v->data);
  p.v_dt = v->dtype;
  p.v_sb = v->stride[0];
  p.v_sh = v->stride[1];
  p.v_sl = v->stride[2];
  p.b = static_cast<int32_t>(s.b);
  p.q_h = static_cast<int32_t>(s.q_h);
  p.v_h = static_cast<int32_t>(s.v_h);
  p.d = static_cast<int32_t>(s.d);
  p.L = static_cast<int32_t>(s.L);
  p.out = out->data;
  p.out_dt = out->dtype;
  p.o_sb = out->stride[0];
  p.o_sh = out->stride[1];
  return p;
}

// Shared body of the two fused Atop-N entry points.
int atopn_run(bool calibrate, const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
              const saga_tensor* mask, const int32_t* kv_len, float scale, int64_t top_n,
              const float* pstar_in, float* pstar_out, saga_tensor* out, int32_t k2_variant, void* workspace,
              size_t workspace_bytes, saga_stream_t stream) {
  Shape s{};
  int rc;
  if ((rc = check_qk(query, key, mask, &s)) || (rc = check_v(value, &s)) || (rc = check_out(out, s))) return rc;
  if (top_n < 1) return fail(SAGA_ERR_INVALID, "top_n must be >= 1, got %lld", (long long)top_n);
  if (calibrate ? !pstar_out : !pstar_in) return fail(SAGA_ERR_INVALID, "threshold table row is null");
  if (k2_variant != kK2Auto && k2_variant != kK2RowBlock && k2_variant != kK2SliceRow)
    return fail(SAGA_ERR_INVALID, "k2_variant must be 0, 1 or 2, got %d", k2_variant);
  const int64_t buf_k = calibrate ? (top_n < s.L ? top_n : s.L) : (top_n < (s.L + 1) / 2 ? 2 * top_n : s.L);
  if (!atopn_sizes_ok(s.b, s.q_h, s.k_h, s.L, s.d, buf_k)) return fail(SAGA_ERR_UNSUPPORTED, "workspace too large");
  saga_atopn_layout lay;
  atopn_layout(s.b, s.q_h, s.k_h, s.L, s.d, buf_k, &lay);
  if (!workspace || workspace_bytes < static_cast<size_t>(lay.total_bytes))
    return fail(SAGA_ERR_WORKSPACE, "workspace of %zu bytes, need %lld", workspace_bytes, (long long)lay.total_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(SAGA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nr = s.b * s.q_h;
  if (nr * lay.nslice >= (1LL << 31)) return fail(SAGA_ERR_UNSUPPORTED, "too many score rows x slices");

  QKParams qp = make_qk(query, key, mask, kv_len, scale, s);
  qp.pmax = reinterpret_cast<float*>(ws + lay.part_max);
  qp.psum = reinterpret_cast<float*>(ws + lay.part_sum);
  qp.ptail = reinterpret_cast<float*>(ws + lay.part_tail);
  qp.scores = reinterpret_cast<float*>(ws + lay.scores);
  qp.s_sb = s.q_h * lay.scores_ld;
  qp.s_sh = lay.scores_ld;
  qp.vec_store = 1;
  if ((rc = hip_status(launch_qk_scores(s.dt, static_cast<int>(s.d), qp, st), "qk_scores launch"))) return rc;

  FusedSelParams sp{};
  sp.scores = qp.scores;
  sp.ld = lay.scores_ld;
  sp.pmax = qp.pmax;
  sp.psum = qp.psum;
  sp.ptail = qp.ptail;
  sp.nparts = static_cast<int32_t>(lay.nparts);
  sp.kv_len = kv_len;
  sp.q_h = static_cast<int32_t>(s.q_h);
  sp.nrows = static_cast<int32_t>(nr);
  sp.L = static_cast<int32_t>(s.L);
  sp.pstar = pstar_in;
  sp.pstar_out = pstar_out;
  sp.t_out = reinterpret_cast<float*>(ws + lay.thresh);
  sp.cap = static_cast<int32_t>(buf_k);
  sp.sel_idx = reinterpret_cast<int32_t*>(ws + lay.sel_idx);
  sp.sel_val = reinterpret_cast<float*>(ws + lay.sel_val);
  sp.sel_cnt = reinterpret_cast<int32_t*>(ws + lay.sel_cnt);
  sp.sel_total = reinterpret_cast<int32_t*>(ws + lay.sel_total);
  sp.nslice = static_cast<int32_t>(lay.nslice);
  sp.slice_cap = static_cast<int32_t>(lay.slice_cap);
  sp.sl_idx = reinterpret_cast<int32_t*>(ws + lay.slice_idx);
  sp.sl_val = reinterpret_cast<float*>(ws + lay.slice_val);
  sp.sl_cnt = reinterpret_cast<int32_t*>(ws + lay.slice_cnt);
  sp.sl_pre = reinterpret_cast<int32_t*>(ws + lay.slice_pre);
  sp.sl_o = reinterpret_cast<float*>(ws + lay.slice_o);
  sp.sl_ml = reinterpret_cast<float*>(ws + lay.slice_ml);
  sp.row_part = reinterpret_cast<float*>(ws + lay.row_part);
  sp.row_cnt = reinterpret_cast<int32_t*>(ws + lay.row_cnt);
  sp.k2_variant = k2_variant;
  // calibration: softmax over the top-k logits == renormalised top-k probabilities
  const PVParams pp = make_pv(value, out, s);
  if ((rc = hip_status(launch_atopn_select_pv(calibrate, sp, pp, st), "atopn select/pv launch"))) return rc;
  return ok();
}

// Dense split plan: about 512 blocks over the (batch, key head) units,
// splits of >= 512 positions, or up to 256 splits of >= 64 positions where
// that gives more (a batch-1 4k decode ran on 8 blocks, 32k on 64), split
// length a multiple of the 32-position wave step.  The split count never
// grows with the number of units, so the workspace bound computed for
// k_h = 1 covers every k_h.
constexpr int64_t kDenseHeadSplitBatch = 4;  // one key head and fewer batch rows: heads split over two units

void dense_plan(int64_t units, int64_t L, int64_t* nsplit, int64_t* split_len) {
  units = std::max<int64_t>(units, 1);
  L = std::max<int64_t>(L, 1);
  int64_t ns = (512 + units - 1) / units;
  const int64_t by_len = std::max<int64_t>((L + 511) / 512, std::min<int64_t>((L + 63) / 64, 256));
  if (ns > by_len) ns = by_len;
  if (ns < 1) ns = 1;
  int64_t sl = (L + ns - 1) / ns;
  sl = (sl + 31) / 32 * 32;
  *nsplit = (L + sl - 1) / sl;
  *split_len = sl;
}

// Rows of a [..., D] tensor must be uniformly strided (collapsible leading dims).
int rows_of(const saga_tensor* t, const char* name, int64_t* rows, int64_t* ld) {
  if (!t) return fail(SAGA_ERR_INVALID, "%s: null tensor descriptor", name);
  if (!t->data) return fail(SAGA_ERR_INVALID, "%s: null data pointer", name);
  if (t->ndim < 1 || t->ndim > 4) return fail(SAGA_ERR_INVALID, "%s: 1 to 4 dims expected", name);
  if (t->stride[t->ndim - 1] != 1) return fail(SAGA_ERR_INVALID, "%s: innermost stride must be 1", name);
  int rc;
  if ((rc = check_dims(t, name))) return rc;
  int64_t r = 1;
  for (int i = 0; i + 1 < t->ndim; ++i) r *= t->shape[i];
  *rows = r;
  *ld = t->ndim >= 2 ? t->stride[t->ndim - 2] : t->shape[0];
  for (int i = 0; i + 2 < t->ndim; ++i)
    if (t->shape[i] > 1 && t->stride[i] != t->stride[i + 1] * t->shape[i + 1])
      return fail(SAGA_ERR_INVALID, "%s: leading dims must be collapsible into rows", name);
  return SAGA_OK;
}

// Device address of `scratch` on the current device, looked up once per
// device with that device current (each GPU holds its own copy at its own
// address).  Returns SAGA_OK and sets *out, or an error code.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_ptr(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SAGA_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(SAGA_ERR_UNSUPPORTED, "device %d out of range", dev);
  if (stream) {
    int sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return fail(SAGA_ERR_HIP, "hipStreamGetDevice: %s", hipGetErrorString(e));
    if (sdev != dev)
      return fail(SAGA_ERR_INVALID, "stream is on device %d, the current device is %d: make it current", sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(SAGA_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SAGA_OK;
}

}  // namespace

extern "C" {

int saga_version(void) { return 100; }

const char* saga_last_error(void) { return g_err; }

int saga_qk_scores(const saga_tensor* query, const saga_tensor* key, const saga_tensor* mask,
                   const int32_t* kv_len, float scale, saga_tensor* scores, float* part_max,
                   float* part_sum, saga_stream_t stream) {
  Shape s{};
  int rc;
  if ((rc = check_qk(query, key, mask, &s))) return rc;
  if ((rc = check_tensor(scores, "scores", 4))) return rc;
  if (scores->dtype != SAGA_DTYPE_F32) return fail(SAGA_ERR_INVALID, "scores: dtype must be f32");
  if (scores->shape[0] != s.b || scores->shape[1] != s.q_h || scores->shape[2] != 1 || scores->shape[3] < s.L)
    return fail(SAGA_ERR_INVALID, "scores: shape must be [b, q_h, 1, >=L]");
  if (scores->stride[3] != 1) return fail(SAGA_ERR_INVALID, "scores: innermost stride must be 1");
  if ((part_max == nullptr) != (part_sum == nullptr))
    return fail(SAGA_ERR_INVALID, "part_max and part_sum must both be given or both be null");
  QKParams p = make_qk(query, key, mask, kv_len, scale, s);
  p.scores = static_cast<float*>(scores->data);
  p.s_sb = scores->stride[0];
  p.s_sh = scores->stride[1];
  p.vec_store = (reinterpret_cast<uintptr_t>(scores->data) % 16 == 0) && (p.s_sb % 4 == 0) && (p.s_sh % 4 == 0);
  p.pmax = part_max;
  p.psum = part_sum;
  if ((rc = hip_status(launch_qk_scores(s.dt, static_cast<int>(s.d), p, static_cast<hipStream_t>(stream)),
                       "qk_scores launch")))
    return rc;
  return ok();
}

int saga_logit_threshold(const saga_tensor* scores, const int32_t* kv_len, const float* softmax_threshold,
                         float* logit_threshold, saga_stream_t stream) {
  int rc;
  if ((rc = check_tensor(scores, "scores", 4))) return rc;
  if (scores->dtype != SAGA_DTYPE_F32) return fail(SAGA_ERR_INVALID, "scores: dtype must be f32");
  if (scores->shape[2] != 1 || scores->stride[3] != 1) return fail(SAGA_ERR_INVALID, "scores: [b, q_h, 1, L], innermost stride 1");
  if (!softmax_threshold || !logit_threshold) return fail(SAGA_ERR_INVALID, "threshold pointers must not be null");
  if (scores->shape[3] >= kMaxLen) return fail(SAGA_ERR_UNSUPPORTED, "length too large");
  ThreshParams p{};
  p.scores = static_cast<const float*>(scores->data);
  p.s_sb = scores->stride[0];
  p.s_sh = scores->stride[1];
  p.q_h = static_cast<int32_t>(scores->shape[1]);
  p.nrows = static_cast<int32_t>(scores->shape[0] * scores->shape[1]);
  p.L = static_cast<int32_t>(scores->shape[3]);
  p.kv_len = kv_len;
  p.pstar = softmax_threshold;
  p.t_out = logit_threshold;
  if ((rc = hip_status(launch_logit_threshold(p, static_cast<hipStream_t>(stream)), "logit_threshold launch"))) return rc;
  return ok();
}

int saga_threshold_select(const saga_tensor* x, const float* threshold, int64_t threshold_numel, int64_t k,
                          saga_tensor* out_values, int64_t* out_indices, int32_t* out_counts,
                          saga_stream_t stream) {
  int rc;
  int64_t rows, ld, orows, old;
  if ((rc = rows_of(x, "x", &rows, &ld))) return rc;
  if (!is_float(x->dtype)) return fail(SAGA_ERR_INVALID, "x: dtype must be f32, bf16 or f16");
  const int64_t D = x->shape[x->ndim - 1];
  if (D < 1 || D >= kMaxLen) return fail(SAGA_ERR_UNSUPPORTED, "row length %lld unsupported", (long long)D);
  if (rows < 1 || rows >= (1LL << 31)) return fail(SAGA_ERR_UNSUPPORTED, "row count %lld unsupported", (long long)rows);
  if (!threshold || threshold_numel < 1) return fail(SAGA_ERR_INVALID, "threshold: null or empty");
  if (k < 0 || k >= kMaxLen) return fail(SAGA_ERR_INVALID, "k = %lld out of range", (long long)k);
  if ((rc = rows_of(out_values, "out_values", &orows, &old))) return rc;
  if (out_values->dtype != x->dtype) return fail(SAGA_ERR_INVALID, "out_values: dtype must match x");
  if (orows != rows || out_values->shape[out_values->ndim - 1] != k)
    return fail(SAGA_ERR_INVALID, "out_values: shape must be x.shape[:-1] + (k,)");
  if (!out_indices) return fail(SAGA_ERR_INVALID, "out_indices: null");
  if (k == 0) return ok();
  ApiSelParams p{};
  p.x = x->data;
  p.x_dt = x->dtype;
  p.x_ld = ld;
  p.nrows = static_cast<int32_t>(rows);
  p.D = D;
  p.thresh = threshold;
  p.thresh_numel = threshold_numel;
  p.k = static_cast<int32_t>(k);
  p.out_val = out_values->data;
  p.ov_ld = old;
  p.out_idx = out_indices;
  p.oi_ld = k;
  p.out_counts = out_counts;
  if ((rc = hip_status(launch_select_api(p, static_cast<hipStream_t>(stream)), "threshold_select launch"))) return rc;
  return ok();
}

int saga_sparse_softmax_pv(const saga_tensor* weights, const saga_tensor* indices, const saga_tensor* value,
                           int32_t input_is_logits, saga_tensor* out, saga_stream_t stream) {
  int rc;
  if ((rc = check_tensor(weights, "weights", 4)) || (rc = check_tensor(indices, "indices", 4))) return rc;
  Shape s{};
  s.b = weights->shape[0];
  s.q_h = weights->shape[1];
  s.L = value ? value->shape[2] : 0;
  s.d = value ? value->shape[3] : 0;
  s.dt = value ? value->dtype : -1;
  if ((rc = check_v(value, &s)) || (rc = check_out(out, s))) return rc;
  if (!is_float(s.dt)) return fail(SAGA_ERR_INVALID, "value: dtype must be f32, bf16 or f16");
  if (s.d != 64 && s.d != 128) return fail(SAGA_ERR_UNSUPPORTED, "head_dim %lld not built (64, 128)", (long long)s.d);
  if (s.L >= kMaxLen) return fail(SAGA_ERR_UNSUPPORTED, "value length too large");
  const int64_t K = weights->shape[3];
  if (weights->shape[2] != 1 || indices->shape[0] != s.b || indices->shape[1] != s.q_h || indices->shape[2] != 1 ||
      indices->shape[3] != K)
    return fail(SAGA_ERR_INVALID, "weights/indices: shapes must both be [b, q_h, 1, K]");
  if (!is_float(weights->dtype)) return fail(SAGA_ERR_INVALID, "weights: dtype must be f32, bf16 or f16");
  if (indices->dtype != SAGA_DTYPE_I64 && indices->dtype != SAGA_DTYPE_I32)
    return fail(SAGA_ERR_INVALID, "indices: dtype must be int64 or int32");
  if (weights->stride[3] != 1 || indices->stride[3] != 1 || (s.b > 1 && weights->stride[0] != s.q_h * weights->stride[1]) ||
      (s.b > 1 && indices->stride[0] != s.q_h * indices->stride[1]))
    return fail(SAGA_ERR_INVALID, "weights/indices: rows must be uniformly strided with unit innermost stride");
  if (K >= kMaxLen) return fail(SAGA_ERR_UNSUPPORTED, "K too large");
  PVParams p = make_pv(value, out, s);
  p.w = weights->data;
  p.w_dt = weights->dtype;
  p.w_ld = weights->stride[1];
  p.idx = indices->data;
  p.idx_i64 = indices->dtype == SAGA_DTYPE_I64;
  p.i_ld = indices->stride[1];
  p.K = static_cast<int32_t>(K);
  p.probs_mode = input_is_logits ? 0 : 1;
  if ((rc = hip_status(launch_sparse_pv(p, static_cast<hipStream_t>(stream)), "sparse_pv launch"))) return rc;
  return ok();
}

int64_t saga_qk_nparts(int64_t b, int64_t k_h, int64_t L) {
  if (b < 1 || k_h < 1 || L < 1 || L >= kMaxLen || b > ((1LL << 31) - 1) / k_h) return 0;
  return qk_plan(b, k_h, L) / 4;
}

size_t saga_atopn_workspace_bytes(int64_t b, int64_t q_h, int64_t k_h, int64_t L, int64_t d, int64_t buf_k) {
  if (!atopn_sizes_ok(b, q_h, k_h, L, d, buf_k)) return 0;
  saga_atopn_layout lay;
  atopn_layout(b, q_h, k_h, L, d, buf_k, &lay);
  return static_cast<size_t>(lay.total_bytes);
}

int saga_atopn_workspace_layout(int64_t b, int64_t q_h, int64_t k_h, int64_t L, int64_t d, int64_t buf_k,
                                saga_atopn_layout* layout) {
  if (!layout) return fail(SAGA_ERR_INVALID, "layout: null");
  if (!atopn_sizes_ok(b, q_h, k_h, L, d, buf_k))
    return fail(SAGA_ERR_INVALID, "sizes must be >= 1 (k_h <= q_h) and the workspace must fit int64");
  atopn_layout(b, q_h, k_h, L, d, buf_k, layout);
  return ok();
}

int saga_atopn_decode(const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
                      const saga_tensor* mask, const int32_t* kv_len, float scale, int64_t top_n,
                      const float* softmax_threshold, saga_tensor* out, void* workspace, size_t workspace_bytes,
                      saga_stream_t stream) {
  return atopn_run(false, query, key, value, mask, kv_len, scale, top_n, softmax_threshold, nullptr, out, kK2Auto,
                   workspace, workspace_bytes, stream);
}

int saga_atopn_decode_ex(const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
                         const saga_tensor* mask, const int32_t* kv_len, float scale, int64_t top_n,
                         const float* softmax_threshold, saga_tensor* out, int32_t k2_variant, void* workspace,
                         size_t workspace_bytes, saga_stream_t stream) {
  return atopn_run(false, query, key, value, mask, kv_len, scale, top_n, softmax_threshold, nullptr, out, k2_variant,
                   workspace, workspace_bytes, stream);
}

int saga_atopn_decode_noalloc(const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
                              const saga_tensor* mask, const int32_t* kv_len, float scale, int64_t top_n,
                              const float* softmax_threshold, saga_tensor* out, saga_stream_t stream) {
  // the scratch bound first: a shape whose workspace exceeds it is refused
  // before anything is looked up or launched
  Shape s{};
  int rc;
  if ((rc = check_qk(query, key, mask, &s)) || (rc = check_v(value, &s)) || (rc = check_out(out, s))) return rc;
  if (top_n < 1) return fail(SAGA_ERR_INVALID, "top_n must be >= 1, got %lld", (long long)top_n);
  const int64_t buf_k = top_n < (s.L + 1) / 2 ? 2 * top_n : s.L;
  if (!atopn_sizes_ok(s.b, s.q_h, s.k_h, s.L, s.d, buf_k)) return fail(SAGA_ERR_UNSUPPORTED, "workspace too large");
  saga_atopn_layout lay;
  atopn_layout(s.b, s.q_h, s.k_h, s.L, s.d, buf_k, &lay);
  if (lay.total_bytes > static_cast<int64_t>(SAGA_NOALLOC_SCRATCH_BYTES))
    return fail(SAGA_ERR_WORKSPACE, "this shape needs %lld bytes of scratch; the static scratch holds %lld",
                (long long)lay.total_bytes, (long long)SAGA_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if ((rc = scratch_ptr(static_cast<hipStream_t>(stream), &ws))) return rc;
  return atopn_run(false, query, key, value, mask, kv_len, scale, top_n, softmax_threshold, nullptr, out, kK2Auto, ws,
                   SAGA_NOALLOC_SCRATCH_BYTES, stream);
}

int saga_atopn_calibrate(const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
                         const saga_tensor* mask, const int32_t* kv_len, float scale, int64_t top_n,
                         float* softmax_threshold_out, saga_tensor* out, void* workspace, size_t workspace_bytes,
                         saga_stream_t stream) {
  return atopn_run(true, query, key, value, mask, kv_len, scale, top_n, nullptr, softmax_threshold_out, out,
                   kK2Auto, workspace, workspace_bytes, stream);
}

int saga_atopn_calibrate_ex(const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
                            const saga_tensor* mask, const int32_t* kv_len, float scale, int64_t top_n,
                            float* softmax_threshold_out, saga_tensor* out, int32_t k2_variant, void* workspace,
                            size_t workspace_bytes, saga_stream_t stream) {
  return atopn_run(true, query, key, value, mask, kv_len, scale, top_n, nullptr, softmax_threshold_out, out,
                   k2_variant, workspace, workspace_bytes, stream);
}

// (the head split of saga_dense_decode only lowers the split count: the plan
// for b units bounds it)
size_t saga_dense_workspace_bytes(int64_t b, int64_t q_h, int64_t L, int64_t d) {
  if (b < 1 || q_h < 1 || L < 1 || L >= kMaxLen || d < 1 || d > 1024 || b > ((1LL << 31) - 1) / q_h) return 0;
  int64_t ns, sl;
  dense_plan(b, L, &ns, &sl);
  return static_cast<size_t>(align256(b * q_h * ns * (2 + d) * 4));
}

int saga_dense_decode(const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
                      const saga_tensor* mask, const int32_t* kv_len, float scale, saga_tensor* out, void* workspace,
                      size_t workspace_bytes, saga_stream_t stream) {
  Shape s{};
  int rc;
  if ((rc = check_qk(query, key, mask, &s)) || (rc = check_v(value, &s)) || (rc = check_out(out, s))) return rc;
  // one key head (the merged SAGA shape) at small batch: the query heads are
  // split over two units that read the same key head (a key-head stride of
  // 0), which doubles the blocks of a latency-bound decode
  const int64_t hs = (s.k_h == 1 && (s.q_h / s.k_h) % 2 == 0 && s.b < kDenseHeadSplitBatch) ? 2 : 1;
  int64_t ns, sl;
  dense_plan(s.b * s.k_h * hs, s.L, &ns, &sl);
  const size_t need = static_cast<size_t>(s.b * s.q_h * ns * (2 + s.d) * 4);
  if (ns > 1 && (!workspace || workspace_bytes < need))
    return fail(SAGA_ERR_WORKSPACE, "workspace of %zu bytes, need %zu", workspace_bytes, need);
  if (ns > 1 && reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(SAGA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  QKParams qp = make_qk(query, key, mask, kv_len, scale, s);
  DenseParams p{};
  p.q = qp.q;
  p.q_sb = qp.q_sb;
  p.q_sh = qp.q_sh;
  p.k = qp.k;
  p.k_sb = qp.k_sb;
  p.k_sh = qp.k_sh;
  p.k_sl = qp.k_sl;
  p.v = static_cast<const char*>(value->data);
  p.v_sb = value->stride[0];
  p.v_sh = value->stride[1];
  p.v_sl = value->stride[2];
  p.mask = qp.mask;
  p.mask_dt = qp.mask_dt;
  p.m_sb = qp.m_sb;
  p.m_sh = qp.m_sh;
  p.m_sl = qp.m_sl;
  p.kv_len = kv_len;
  p.b = qp.b;
  p.q_h = qp.q_h;
  p.k_h = qp.k_h;
  p.v_h = static_cast<int32_t>(s.v_h);
  p.g = qp.g;
  if (hs > 1) {
    p.k_h = static_cast<int32_t>(qp.k_h * hs);
    p.g = static_cast<int32_t>(qp.g / hs);
    p.k_sh = 0;
  }
  p.L = qp.L;
  p.scale = scale;
  p.out = out->data;
  p.out_dt = out->dtype;
  p.o_sb = out->stride[0];
  p.o_sh = out->stride[1];
  p.nsplit = static_cast<int32_t>(ns);
  p.split_len = static_cast<int32_t>(sl);
  p.part = static_cast<float*>(workspace);
  if ((rc = hip_status(launch_dense_decode(s.dt, static_cast<int>(s.d), p, static_cast<hipStream_t>(stream)),
                       "dense_decode launch")))
    return rc;
  return ok();
}

}  // extern "C"

namespace {

// Validates the RoPE / cache-append operands shared by saga_rope_kv_append and
// saga_gemv_rope_kv: N token rows of dtype dt, q_out [N, n_q, d], caches
// [B, n_k, Lmax, d] / [B, n_v, Lmax, d].
int make_rope(int64_t N, int32_t dt, int64_t n_q, int64_t n_k, int64_t n_v, float theta, const int32_t* pos,
              const int32_t* batch, saga_tensor* q_out, saga_tensor* k_cache, saga_tensor* v_cache, RopeParams& p) {
  int rc;
  if ((rc = check_tensor(q_out, "q_out", 3)) || (rc = check_tensor(k_cache, "k_cache", 4)) ||
      (rc = check_tensor(v_cache, "v_cache", 4)))
    return rc;
  if (!pos) return fail(SAGA_ERR_INVALID, "pos: null");
  if (n_q < 1 || n_k < 1 || n_v < 1) return fail(SAGA_ERR_INVALID, "head counts must be >= 1");
  const int64_t d = q_out->shape[2];
  if (d % 2 || d < 2) return fail(SAGA_ERR_INVALID, "head_dim must be even");
  if (q_out->dtype != dt || k_cache->dtype != dt || v_cache->dtype != dt)
    return fail(SAGA_ERR_INVALID, "q_out and the caches must have the dtype of the projection");
  if (q_out->shape[0] != N || q_out->shape[1] != n_q) return fail(SAGA_ERR_INVALID, "q_out: shape must be [N, n_q, d]");
  if (k_cache->shape[1] != n_k || k_cache->shape[3] != d || v_cache->shape[1] != n_v || v_cache->shape[3] != d ||
      v_cache->shape[0] != k_cache->shape[0] || v_cache->shape[2] != k_cache->shape[2])
    return fail(SAGA_ERR_INVALID, "caches: shapes must be [B, n_k, Lmax, d] and [B, n_v, Lmax, d]");
  if (q_out->stride[2] != 1 || k_cache->stride[3] != 1 || v_cache->stride[3] != 1)
    return fail(SAGA_ERR_INVALID, "innermost strides must be 1");
  if (!batch && N > k_cache->shape[0]) return fail(SAGA_ERR_INVALID, "without batch indices N must be <= B");
  if (N >= (1LL << 31) || k_cache->shape[2] >= kMaxLen || n_q + n_k + n_v > 65535)
    return fail(SAGA_ERR_UNSUPPORTED, "sizes too large");
  p = RopeParams{};
  p.dt = dt;
  p.N = static_cast<int32_t>(N);
  p.n_q = static_cast<int32_t>(n_q);
  p.n_k = static_cast<int32_t>(n_k);
  p.n_v = static_cast<int32_t>(n_v);
  p.d = static_cast<int32_t>(d);
  p.theta = theta;
  p.pos = pos;
  p.batch = batch;
  p.q_out = q_out->data;
  p.q_sn = q_out->stride[0];
  p.q_sh = q_out->stride[1];
  p.k_cache = k_cache->data;
  p.k_sb = k_cache->stride[0];
  p.k_sh = k_cache->stride[1];
  p.k_sl = k_cache->stride[2];
  p.v_cache = v_cache->data;
  p.v_sb = v_cache->stride[0];
  p.v_sh = v_cache->stride[1];
  p.v_sl = v_cache->stride[2];
  p.B = static_cast<int32_t>(k_cache->shape[0]);
  p.Lmax = static_cast<int32_t>(k_cache->shape[2]);
  return SAGA_OK;
}

// Validates x [M, K] and w [N, K] (bf16, 16-byte aligned rows) and an optional
// bias [N] of a skinny GEMM and fills the shared fields of p.
int make_gemv(const saga_tensor* x, const saga_tensor* w, const saga_tensor* bias, float rms_eps, GemvParams& p) {
  int rc;
  if ((rc = check_tensor(x, "x", 2))) return rc;
  const bool packed = w && w->ndim == 4;   // 16-row tiles
  const bool packed8 = w && w->ndim == 3;  // 8-row tiles
  if ((rc = check_tensor(w, "w", packed ? 4 : packed8 ? 3 : 2))) return rc;
  if (x->dtype != SAGA_DTYPE_BF16 || w->dtype != SAGA_DTYPE_BF16) return fail(SAGA_ERR_UNSUPPORTED, "gemv: bf16 only");
  const int64_t M = x->shape[0], K = x->shape[1];
  const int64_t N = packed ? w->shape[0] * 16 : packed8 ? w->shape[0] * 8 : w->shape[0];
  if (packed) {
    // [N/16][K/32][16][32], contiguous (the stride of a size-1 dim is immaterial)
    if (w->shape[2] != 16 || w->shape[3] != 32 || w->shape[1] * 32 != K || w->stride[3] != 1 || w->stride[2] != 32 ||
        (w->shape[1] > 1 && w->stride[1] != 512) || (w->shape[0] > 1 && w->stride[0] != w->shape[1] * 512))
      return fail(SAGA_ERR_INVALID, "gemv: packed w must be contiguous [N/16, K/32, 16, 32] with K = x.shape[1]");
    if (reinterpret_cast<uintptr_t>(w->data) % 16) return fail(SAGA_ERR_INVALID, "gemv: packed w must be 16-byte aligned");
  } else if (packed8) {
    // [N/8][K/64][512], contiguous
    if (w->shape[2] != 512 || w->shape[1] * 64 != K || w->stride[2] != 1 ||
        (w->shape[1] > 1 && w->stride[1] != 512) || (w->shape[0] > 1 && w->stride[0] != w->shape[1] * 512))
      return fail(SAGA_ERR_INVALID, "gemv: 8-row packed w must be contiguous [N/8, K/64, 512] with K = x.shape[1]");
    if (reinterpret_cast<uintptr_t>(w->data) % 16) return fail(SAGA_ERR_INVALID, "gemv: packed w must be 16-byte aligned");
    if (M > 8) return fail(SAGA_ERR_UNSUPPORTED, "gemv: 8-row packed w takes at most 8 rows of x");
  } else if (w->shape[1] != K) {
    return fail(SAGA_ERR_INVALID, "gemv: w must be [N, K] with K = x.shape[1]");
  }
  if (M > 32) return fail(SAGA_ERR_UNSUPPORTED, "gemv: at most 32 rows");
  if (N % 16 || K % 32 || K >= (1LL << 30) || N >= (1LL << 30))
    return fail(SAGA_ERR_UNSUPPORTED, "gemv: N %% 16 == 0 and K %% 32 == 0 required");
  if ((rc = check_vec_rows(x, "x")) || (!packed && (rc = check_vec_rows(w, "w")))) return rc;
  if (bias) {
    if ((rc = check_tensor(bias, "bias", 1))) return rc;
    if (bias->dtype != SAGA_DTYPE_BF16 || bias->shape[0] != N || bias->stride[0] != 1)
      return fail(SAGA_ERR_INVALID, "bias must be bf16 [N]");
  }
  p = GemvParams{};
  p.x = x->data;
  p.x_ld = x->stride[0];
  p.w = w->data;
  p.w_ld = packed || packed8 ? 0 : w->stride[0];
  p.w_packed = packed ? 1 : packed8 ? 2 : 0;
  p.bias = bias ? bias->data : nullptr;
  p.M = static_cast<int32_t>(M);
  p.N = static_cast<int32_t>(N);
  p.K = static_cast<int32_t>(K);
  p.rms = rms_eps >= 0.f;
  p.eps = rms_eps;
  p.splits = 1;
  return SAGA_OK;
}

}  // namespace

extern "C" {

int saga_rope_kv_append(const saga_tensor* qkv, int64_t n_q, int64_t n_k, int64_t n_v, float theta,
                        const int32_t* pos, const int32_t* batch, saga_tensor* q_out, saga_tensor* k_cache,
                        saga_tensor* v_cache, saga_stream_t stream) {
  int rc;
  if ((rc = check_tensor(qkv, "qkv", 2))) return rc;
  if (!is_float(qkv->dtype)) return fail(SAGA_ERR_INVALID, "qkv: float dtype required");
  const int64_t N = qkv->shape[0];
  RopeParams p;
  if ((rc = make_rope(N, qkv->dtype, n_q, n_k, n_v, theta, pos, batch, q_out, k_cache, v_cache, p))) return rc;
  if (qkv->shape[1] < (n_q + n_k + n_v) * p.d) return fail(SAGA_ERR_INVALID, "qkv: row shorter than (n_q + n_k + n_v) * d");
  if (qkv->stride[1] != 1) return fail(SAGA_ERR_INVALID, "innermost strides must be 1");
  if (N == 0) return ok();
  p.qkv = qkv->data;
  p.qkv_ld = qkv->stride[0];
  if ((rc = hip_status(launch_rope_kv_append(p, static_cast<hipStream_t>(stream)), "rope_kv_append launch"))) return rc;
  return ok();
}

int saga_rope_table(const int32_t* pos, int64_t N, int64_t d, float theta, float* table, saga_stream_t stream) {
  if (N < 0 || d < 2 || d % 2) return fail(SAGA_ERR_INVALID, "rope_table: N >= 0 and an even head_dim >= 2 required");
  if (N > 0 && (!pos || !table)) return fail(SAGA_ERR_INVALID, "rope_table: null pos or table");
  if (N >= (1LL << 31) || d > 65536 || N * (d / 2) >= (1LL << 31))
    return fail(SAGA_ERR_UNSUPPORTED, "rope_table: sizes too large");
  if (reinterpret_cast<uintptr_t>(table) % 16) return fail(SAGA_ERR_INVALID, "rope_table: table must be 16-byte aligned");
  if (N == 0) return ok();
  int rc;
  if ((rc = hip_status(launch_rope_table(pos, static_cast<int>(N), static_cast<int>(d), theta, table,
                                         static_cast<hipStream_t>(stream)),
                       "rope_table launch")))
    return rc;
  return ok();
}

int saga_embed_rope(const int64_t* tokens, const saga_tensor* embed, saga_tensor* x, const int32_t* pos, int64_t d,
                    float theta, float* rope_table, saga_stream_t stream) {
  int rc;
  if ((rc = check_tensor(embed, "embed", 2)) || (rc = check_tensor(x, "x", 2))) return rc;
  if (!is_float(embed->dtype) || x->dtype != embed->dtype)
    return fail(SAGA_ERR_INVALID, "embed_rope: embed and x must share one float dtype");
  if (x->shape[1] != embed->shape[1]) return fail(SAGA_ERR_INVALID, "embed_rope: x must be [B, H] of embed [V, H]");
  if (embed->stride[1] != 1 || x->stride[1] != 1) return fail(SAGA_ERR_INVALID, "innermost strides must be 1");
  if (!tokens) return fail(SAGA_ERR_INVALID, "embed_rope: null tokens");
  if (rope_table) {
    if (!pos) return fail(SAGA_ERR_INVALID, "embed_rope: a rope_table needs pos");
    if (d < 2 || d % 2 || d > 65536) return fail(SAGA_ERR_INVALID, "embed_rope: an even head_dim >= 2 required");
    if (reinterpret_cast<uintptr_t>(rope_table) % 16)
      return fail(SAGA_ERR_INVALID, "embed_rope: rope_table must be 16-byte aligned");
  }
  EmbedParams p{};
  p.tokens = tokens;
  p.embed = embed->data;
  p.e_ld = embed->stride[0];
  p.x = x->data;
  p.x_ld = x->stride[0];
  p.B = static_cast<int32_t>(x->shape[0]);
  p.H = static_cast<int32_t>(x->shape[1]);
  p.dt = x->dtype;
  p.V = embed->shape[0];
  const int64_t es = elt_size(x->dtype);
  p.vec = (p.H * es) % 16 == 0 && reinterpret_cast<uintptr_t>(embed->data) % 16 == 0 &&
          reinterpret_cast<uintptr_t>(x->data) % 16 == 0 && (p.e_ld * es) % 16 == 0 && (p.x_ld * es) % 16 == 0;
  p.pos = pos;
  p.d = static_cast<int32_t>(d);
  p.theta = theta;
  p.table = rope_table;
  if ((rc = hip_status(launch_embed_rope(p, static_cast<hipStream_t>(stream)), "embed_rope launch"))) return rc;
  return ok();
}

int saga_advance_positions(int32_t* pos, int32_t* kv_len, int64_t n, saga_stream_t stream) {
  if (n < 0 || n >= (1LL << 31)) return fail(SAGA_ERR_INVALID, "advance_positions: 0 <= n < 2^31 required");
  if (n > 0 && !pos && !kv_len) return fail(SAGA_ERR_INVALID, "advance_positions: null pos and kv_len");
  if (n == 0) return ok();
  int rc;
  if ((rc = hip_status(launch_advance(pos, kv_len, static_cast<int>(n), static_cast<hipStream_t>(stream)),
                       "advance_positions launch")))
    return rc;
  return ok();
}

int saga_gemv_rope_kv(const saga_tensor* x, const saga_tensor* w, const saga_tensor* bias, float rms_eps,
                      int64_t n_q, int64_t n_k, int64_t n_v, float theta, const int32_t* pos, const int32_t* batch,
                      saga_tensor* q_out, saga_tensor* k_cache, saga_tensor* v_cache, const float* rope_table,
                      saga_stream_t stream) {
  int rc;
  GemvParams p;
  if ((rc = make_gemv(x, w, bias, rms_eps, p))) return rc;
  if ((rc = make_rope(p.M, SAGA_DTYPE_BF16, n_q, n_k, n_v, theta, pos, batch, q_out, k_cache, v_cache, p.rope)))
    return rc;
  if (p.rope.d % 16) return fail(SAGA_ERR_UNSUPPORTED, "gemv_rope_kv: head_dim %% 16 == 0 required");
  if (reinterpret_cast<uintptr_t>(rope_table) % 16)
    return fail(SAGA_ERR_INVALID, "gemv_rope_kv: rope_table must be 16-byte aligned");
  p.rope.table = rope_table;
  if (p.N != (n_q + n_k + n_v) * p.rope.d) return fail(SAGA_ERR_INVALID, "gemv_rope_kv: w must have (n_q + n_k + n_v) * d rows");
  if (p.M == 0) return ok();
  p.epilogue = kGemvRopeKV;
  if ((rc = hip_status(launch_gemv(p, static_cast<hipStream_t>(stream)), "gemv_rope_kv launch"))) return rc;
  return ok();
}

static int row_op(bool silu, const saga_tensor* x, const saga_tensor* w, float eps, saga_tensor* y, saga_stream_t stream) {
  int rc;
  if ((rc = check_tensor(x, "x", 2)) || (rc = check_tensor(y, "y", 2))) return rc;
  if (!is_float(x->dtype) || y->dtype != x->dtype) return fail(SAGA_ERR_INVALID, "x and y must share one float dtype");
  const int64_t H = y->shape[1];
  if (x->shape[0] != y->shape[0] || x->shape[1] != (silu ? 2 * H : H))
    return fail(SAGA_ERR_INVALID, silu ? "x must be [N, 2H] for y [N, H]" : "x and y must have the same shape");
  if (x->stride[1] != 1 || y->stride[1] != 1) return fail(SAGA_ERR_INVALID, "innermost strides must be 1");
  if (!silu) {
    if ((rc = check_tensor(w, "weight", 1))) return rc;
    if (w->dtype != x->dtype || w->shape[0] != H || w->stride[0] != 1) return fail(SAGA_ERR_INVALID, "weight must be [H], same dtype");
  }
  if (x->shape[0] == 0 || H == 0) return ok();
  RowParams p{};
  p.x = x->data;
  p.x_ld = x->stride[0];
  p.w = silu ? nullptr : w->data;
  p.y = y->data;
  p.y_ld = y->stride[0];
  p.dt = x->dtype;
  p.N = static_cast<int32_t>(x->shape[0]);
  p.H = static_cast<int32_t>(H);
  p.eps = eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if ((rc = hip_status(silu ? launch_silu_mul(p, st) : launch_rmsnorm(p, st), "row op launch"))) return rc;
  return ok();
}

int saga_rmsnorm(const saga_tensor* x, const saga_tensor* weight, float eps, saga_tensor* y, saga_stream_t stream) {
  return row_op(false, x, weight, eps, y, stream);
}

int saga_silu_mul(const saga_tensor* gate_up, saga_tensor* y, saga_stream_t stream) {
  return row_op(true, gate_up, nullptr, 0.f, y, stream);
}

size_t saga_gemv_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > 32 || N < 16 || K < 32 || N >= (1LL << 31) || K >= (1LL << 31)) return 0;
  const int s = gemv_splits(N, K);
  if (s <= 1) return 0;
  return static_cast<size_t>(align256(s * M * N * 4) + align256(s * M * 4));
}

int saga_gemv(const saga_tensor* x, const saga_tensor* w, const saga_tensor* bias, float rms_eps, int32_t epilogue,
              saga_tensor* y, void* workspace, size_t workspace_bytes, saga_stream_t stream) {
  int rc;
  GemvParams p;
  if ((rc = make_gemv(x, w, bias, rms_eps, p))) return rc;
  if ((rc = check_tensor(y, "y", 2))) return rc;
  if (y->dtype != SAGA_DTYPE_BF16) return fail(SAGA_ERR_UNSUPPORTED, "gemv: bf16 only");
  if (epilogue != SAGA_GEMV_STORE && epilogue != SAGA_GEMV_ADD && epilogue != SAGA_GEMV_SILU_PAIRS)
    return fail(SAGA_ERR_INVALID, "gemv: unknown epilogue %d", epilogue);
  const int64_t ny = epilogue == SAGA_GEMV_SILU_PAIRS ? p.N / 2 : p.N;
  if (y->shape[0] != p.M || y->shape[1] != ny) return fail(SAGA_ERR_INVALID, "gemv: y must be [M, %lld]", (long long)ny);
  if (y->stride[1] != 1) return fail(SAGA_ERR_INVALID, "y: innermost stride must be 1");
  if (bias && epilogue == SAGA_GEMV_SILU_PAIRS) return fail(SAGA_ERR_UNSUPPORTED, "bias with SILU_PAIRS");
  if (p.M == 0 || p.N == 0) return ok();
  p.y = y->data;
  p.y_ld = y->stride[0];
  p.epilogue = epilogue;
  const int splits = gemv_splits(p.N, p.K);
  const size_t need = saga_gemv_workspace_bytes(p.M, p.N, p.K);
  if (workspace && splits > 1 && workspace_bytes >= need && p.w_packed != 2) {
    if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(SAGA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
    p.splits = splits;
    p.part = static_cast<float*>(workspace);
    p.part_ssq = reinterpret_cast<float*>(static_cast<char*>(workspace) + align256(int64_t(splits) * p.M * p.N * 4));
  }
  if ((rc = hip_status(launch_gemv(p, static_cast<hipStream_t>(stream)), "gemv launch"))) return rc;
  return ok();
}

size_t saga_argmax_workspace_bytes(int64_t rows, int64_t N) {
  if (rows < 1 || N < 1 || rows >= (1LL << 31) || N >= (1LL << 31)) return 0;
  return static_cast<size_t>(argmax_workspace_bytes(rows, N));
}

int saga_argmax(const saga_tensor* x, int64_t* out, void* workspace, size_t workspace_bytes, saga_stream_t stream) {
  int rc;
  if ((rc = check_tensor(x, "x", 2))) return rc;
  if (x->dtype != SAGA_DTYPE_BF16 || x->stride[1] != 1) return fail(SAGA_ERR_UNSUPPORTED, "argmax: bf16 rows with unit stride");
  if (!out) return fail(SAGA_ERR_INVALID, "out: null");
  if (x->shape[0] >= (1LL << 31) || x->shape[1] >= (1LL << 31)) return fail(SAGA_ERR_UNSUPPORTED, "argmax: too large");
  if (x->shape[0] == 0) return ok();
  const int64_t need = argmax_workspace_bytes(x->shape[0], x->shape[1]);
  void* ws = workspace && need > 0 && workspace_bytes >= static_cast<size_t>(need) ? workspace : nullptr;
  if (ws && reinterpret_cast<uintptr_t>(ws) % 256) return fail(SAGA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if ((rc = hip_status(launch_argmax(x->data, x->stride[0], static_cast<int>(x->shape[0]), static_cast<int>(x->shape[1]),
                                     out, ws, static_cast<hipStream_t>(stream)),
                       "argmax launch")))
    return rc;
  return ok();
}

}  // extern "C"

extern "C" {

int saga_prefill_attention(const saga_tensor* query, const saga_tensor* key, const saga_tensor* value,
                           const saga_tensor* mask, float scale, int32_t causal, int64_t causal_offset,
                           saga_tensor* out, saga_stream_t stream) {
  int rc;
  if ((rc = check_tensor(query, "query", 4)) || (rc = check_tensor(key, "key", 4)) ||
      (rc = check_tensor(value, "value", 4)) || (rc = check_tensor(out, "out", 4)))
    return rc;
  const int64_t b = query->shape[0], q_h = query->shape[1], Lq = query->shape[2], d = query->shape[3];
  const int64_t k_h = key->shape[1], Lk = key->shape[2], v_h = value->shape[1];
  const int dt = query->dtype;
  if (dt != SAGA_DTYPE_BF16 && dt != SAGA_DTYPE_F16)
    return fail(SAGA_ERR_UNSUPPORTED, "prefill: query dtype must be bf16 or f16");
  if (key->dtype != dt || value->dtype != dt || out->dtype != dt)
    return fail(SAGA_ERR_INVALID, "prefill: key, value and out must have the query's dtype");
  if (d != 64 && d != 128) return fail(SAGA_ERR_UNSUPPORTED, "prefill: head_dim %lld not built (64, 128)", (long long)d);
  if (key->shape[0] != b || key->shape[3] != d || value->shape[0] != b || value->shape[2] != Lk || value->shape[3] != d)
    return fail(SAGA_ERR_INVALID, "prefill: key [b, k_h, Lk, d] / value [b, v_h, Lk, d] do not match the query");
  if (q_h % k_h || q_h % v_h)
    return fail(SAGA_ERR_INVALID, "prefill: q_h (%lld) must be a multiple of k_h (%lld) and v_h (%lld)", (long long)q_h,
                (long long)k_h, (long long)v_h);
  if (out->shape[0] != b || out->shape[1] != Lq || out->shape[2] != q_h || out->shape[3] != d)
    return fail(SAGA_ERR_INVALID, "prefill: out must be [b, Lq, q_h, d]");
  if (Lq >= kMaxLen || Lk >= kMaxLen) return fail(SAGA_ERR_UNSUPPORTED, "prefill: sequence too long");
  if (causal_offset < -kMaxLen || causal_offset > kMaxLen)
    return fail(SAGA_ERR_INVALID, "prefill: causal_offset out of range");
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(SAGA_ERR_UNSUPPORTED, "prefill: scale must be positive and finite");
  const int64_t nmb = prefill_query_blocks(Lq, static_cast<int>(d));
  if (nmb * q_h * b >= (1LL << 31)) return fail(SAGA_ERR_UNSUPPORTED, "prefill: grid too large");
  if ((rc = check_vec_rows(query, "query")) || (rc = check_vec_rows(key, "key")) || (rc = check_vec_rows(value, "value")))
    return rc;
  // 8-byte stores of 4 output dims
  if (out->stride[3] != 1 || reinterpret_cast<uintptr_t>(out->data) % 8 || out->stride[0] % 4 || out->stride[1] % 4 ||
      out->stride[2] % 4)
    return fail(SAGA_ERR_INVALID, "prefill: out needs unit innermost stride, 8-byte aligned rows");
  PrefillParams p{};
  if (mask) {
    if ((rc = check_tensor(mask, "mask", 4))) return rc;
    if (!is_float(mask->dtype) && mask->dtype != SAGA_DTYPE_BOOL)
      return fail(SAGA_ERR_INVALID, "mask: dtype must be f32, bf16, f16 or bool");
    if ((mask->shape[0] != 1 && mask->shape[0] != b) || (mask->shape[1] != 1 && mask->shape[1] != q_h) ||
        mask->shape[2] != Lq || mask->shape[3] != Lk)
      return fail(SAGA_ERR_INVALID, "mask: shape [%lld,%lld,%lld,%lld] does not broadcast to [b, q_h, Lq, Lk]",
                  (long long)mask->shape[0], (long long)mask->shape[1], (long long)mask->shape[2],
                  (long long)mask->shape[3]);
    p.mask = mask->data;
    p.mask_dt = mask->dtype;
    p.m_sb = mask->shape[0] == 1 ? 0 : mask->stride[0];
    p.m_sh = mask->shape[1] == 1 ? 0 : mask->stride[1];
    p.m_sq = mask->stride[2];
    p.m_sk = mask->stride[3];
  }
  p.q = static_cast<const char*>(query->data);
  p.q_sb = query->stride[0];
  p.q_sh = query->stride[1];
  p.q_sl = query->stride[2];
  p.k = static_cast<const char*>(key->data);
  p.k_sb = key->stride[0];
  p.k_sh = key->stride[1];
  p.k_sl = key->stride[2];
  p.v = static_cast<const char*>(value->data);
  p.v_sb = value->stride[0];
  p.v_sh = value->stride[1];
  p.v_sl = value->stride[2];
  p.out = out->data;
  p.o_sb = out->stride[0];
  p.o_sq = out->stride[1];
  p.o_sh = out->stride[2];
  p.b = static_cast<int32_t>(b);
  p.q_h = static_cast<int32_t>(q_h);
  p.k_h = static_cast<int32_t>(k_h);
  p.v_h = static_cast<int32_t>(v_h);
  p.Lq = static_cast<int32_t>(Lq);
  p.Lk = static_cast<int32_t>(Lk);
  p.nmb = static_cast<int32_t>(nmb);
  p.causal = causal ? 1 : 0;
  p.causal_off = static_cast<int32_t>(causal_offset);
  p.scale = scale;
  if ((rc = hip_status(launch_prefill_attention(dt, static_cast<int>(d), p, static_cast<hipStream_t>(stream)),
                       "prefill launch")))
    return rc;
  return ok();
}

}  // extern "C"

// C ABI of the EPTQ gfx950 library (declarations and contract: include/eptq_hip.h).
//
// Host-side validation mirrors and extends the reference dispatcher's checks
// (csrc/eptq_kernels.cu:478-494): null pointers, sizes, alignment of every
// 16-byte vector operand, S_group group size, then a launch and a
// hipGetLastError check.

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "eptq_hip.h"
#include "eptq_llama.h"
#include "kernels.h"

// Scratch of eptq_e8d4_forward_multi_noalloc: the matrix-core decode's
// split-K workspace (tile counters, then partial sums for up to 256 CUs), a
// file-scope device array; each GPU holds its own copy until the process
// ends.  Host code uses only the per-device address from
// hipGetSymbolAddress (in host code the array's name is a stand-in, not a
// device address).
constexpr size_t kNoAllocScratchBytes = eptq::kSplitCounterBytes + 256 * eptq::kSplitPartBytes;
static_assert(kNoAllocScratchBytes == EPTQ_NOALLOC_SCRATCH_BYTES, "header constant");
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(EPTQ_EHIP, "%s: %s", what, hipGetErrorString(e));
  return EPTQ_OK;
}

int check_common(const char* fn, const void* Q, const void* codes, const void* g,
                 const void* h, const void* O_vals, const void* O_col,
                 const void* O_row_ptr, const void* S_group, int n_groups, int M, int N,
                 int* qb) {
  if (!Q || !codes || !g || !h || !O_row_ptr)
    return fail(EPTQ_EINVAL, "%s: null Q/codes/g/h/O_row_ptr", fn);
  if (M <= 0 || N <= 0) return fail(EPTQ_EINVAL, "%s: M=%d N=%d must be positive", fn, M, N);
  if ((int64_t)M * 8 > 0x7fffffff) return fail(EPTQ_EINVAL, "%s: M=%d too large", fn, M);
  if ((!O_vals || !O_col) && (O_vals || O_col))
    return fail(EPTQ_EINVAL, "%s: O_vals and O_col must both be given or both be null", fn);
  if (O_vals && !aligned16(O_vals))
    return fail(EPTQ_EUNSUPPORTED, "%s: O_vals must be 16-byte aligned", fn);
  *qb = 1;
  if (S_group) {
    if (n_groups <= 0 || (8 * M) % n_groups != 0)
      return fail(EPTQ_EINVAL, "%s: n_groups=%d must divide out_features=%d", fn, n_groups, 8 * M);
    *qb = (8 * M) / n_groups;
    if (*qb % 8 != 0)
      return fail(EPTQ_EUNSUPPORTED, "%s: group size %d is not a multiple of 8", fn, *qb);
  }
  return EPTQ_OK;
}

// Validate one layer's operands and fill its kernel arguments (y, ldy set by
// the caller).
int layer_args(const char* fn, int kind, const void* Q, const void* codes, int codes_dtype,
               const void* g, const void* h, const void* x, int x_dtype, const void* O_vals,
               const void* O_col, const void* O_row_ptr, const void* bias, const void* S_group,
               int n_groups, int M, int N, int B, eptq::LinearArgs* a) {
  int qb = 1;
  int rc = check_common(fn, Q, codes, g, h, O_vals, O_col, O_row_ptr, S_group, n_groups, M, N, &qb);
  if (rc) return rc;
  if (B < 0) return fail(EPTQ_EINVAL, "%s: B=%d", fn, B);
  if (B > 0 && !x) return fail(EPTQ_EINVAL, "%s: null x/y", fn);
  if (codes_dtype != EPTQ_F16 && codes_dtype != EPTQ_F32)
    return fail(EPTQ_EINVAL, "%s: codes_dtype must be EPTQ_F16 or EPTQ_F32", fn);
  if (x_dtype != EPTQ_F16 && x_dtype != EPTQ_BF16)
    return fail(EPTQ_EINVAL, "%s: x_dtype must be EPTQ_F16 or EPTQ_BF16", fn);
  if (N % 8 != 0) return fail(EPTQ_EUNSUPPORTED, "%s: in_features=%d not a multiple of 8", fn, N);
  if (!aligned16(Q) || (B > 0 && !aligned16(x)) || !aligned16(h) || (S_group && !aligned16(S_group)))
    return fail(EPTQ_EUNSUPPORTED, "%s: Q, x, h and S_group must be 16-byte aligned", fn);
  if (kind == eptq::KIND_E8 && !aligned16(codes))
    return fail(EPTQ_EUNSUPPORTED, "%s: E8 codebook must be 16-byte aligned", fn);
  a->Q = (const int16_t*)Q;
  a->codes = codes;
  a->codes_f32 = codes_dtype == EPTQ_F32;
  a->g = (const eptq::f16*)g;
  a->h = (const eptq::f16*)h;
  a->x = (const uint16_t*)x;
  a->x_bf16 = x_dtype == EPTQ_BF16;
  a->O = (const eptq::f16*)O_vals;
  a->O_col = (const int32_t*)O_col;
  a->O_row_ptr = (const int32_t*)O_row_ptr;
  a->bias = (const eptq::f16*)bias;
  a->S = (const eptq::f16*)S_group;
  a->qb = qb;
  a->M = M;
  a->N = N;
  a->B = B;
  a->y = nullptr;
  a->ldy = 8 * M;
  a->prep = 0;
  a->ldx = N;
  a->x2 = nullptr;
  a->nw = nullptr;
  a->xsum = nullptr;
  a->eps = 0.0f;
  a->pad_ = 0;
  a->res = nullptr;
  return EPTQ_OK;
}

// Launch one layer on the kernel for its codebook and batch size (work: an
// optional decode workspace, see eptq_e8d4_forward_multi).
int dispatch(const char* fn, int kind, const eptq::LinearArgs& a, hipStream_t s, void* work = nullptr,
             long long work_bytes = 0) {
  int rc = 0;
  if (a.B <= eptq::kMatvecMaxBatch) {
    if (kind == eptq::KIND_E8D4) {
      rc = eptq::launch_decode_e8d4(a, s);
      if (rc) rc = eptq::launch_matvec<eptq::KIND_E8D4>(a, s);
    } else {
      rc = eptq::launch_matvec<eptq::KIND_E8>(a, s);
    }
  } else if (kind == eptq::KIND_E8D4) {
    rc = eptq::launch_gemm<eptq::KIND_E8D4>(a, s, work, work_bytes);
  } else {
    rc = eptq::launch_gemm<eptq::KIND_E8>(a, s);
  }
  if (rc) return fail(EPTQ_EUNSUPPORTED, "%s: no kernel for M=%d N=%d B=%d", fn, a.M, a.N, a.B);
  return EPTQ_OK;
}

int linear_common(int kind, const void* Q, const void* codes, int codes_dtype, const void* g,
                  const void* h, const void* x, int x_dtype, const void* O_vals,
                  const void* O_col, const void* O_row_ptr, const void* bias,
                  const void* S_group, int n_groups, int M, int N, int B, void* y,
                  void* stream) {
  const char* fn = kind == eptq::KIND_E8D4 ? "eptq_e8d4_forward" : "eptq_e8_forward";
  eptq::LinearArgs a;
  int rc = layer_args(fn, kind, Q, codes, codes_dtype, g, h, x, x_dtype, O_vals, O_col, O_row_ptr,
                      bias, S_group, n_groups, M, N, B, &a);
  if (rc) return rc;
  if (B == 0) return EPTQ_OK;
  if (!y) return fail(EPTQ_EINVAL, "%s: null x/y", fn);
  a.y = (uint16_t*)y;
  rc = dispatch(fn, kind, a, (hipStream_t)stream);
  if (rc) return rc;
  return check_launch(fn);
}

int dequant_common(int kind, const void* Q, const void* codes_f32, const void* g,
                   const void* h, const void* O_vals, const void* O_col,
                   const void* O_row_ptr, const void* S_group, int n_groups, int M, int N,
                   void* W, void* stream) {
  const char* fn = kind == eptq::KIND_E8D4 ? "eptq_e8d4_dequant" : "eptq_e8_dequant";
  int qb = 1;
  int rc = check_common(fn, Q, codes_f32, g, h, O_vals, O_col, O_row_ptr, S_group, n_groups, M,
                        N, &qb);
  if (rc) return rc;
  if (!W) return fail(EPTQ_EINVAL, "%s: null W", fn);
  if (!aligned16(codes_f32)) return fail(EPTQ_EUNSUPPORTED, "%s: table must be 16-byte aligned", fn);
  if ((N & 3) == 0 && ((uintptr_t)W & 7u))
    return fail(EPTQ_EUNSUPPORTED, "%s: W must be 8-byte aligned", fn);
  eptq::DequantArgs a;
  a.Q = (const int16_t*)Q;
  a.table = (const float*)codes_f32;
  a.g = (const eptq::f16*)g;
  a.h = (const eptq::f16*)h;
  a.O = (const eptq::f16*)O_vals;
  a.O_col = (const int32_t*)O_col;
  a.O_row_ptr = (const int32_t*)O_row_ptr;
  a.S = (const eptq::f16*)S_group;
  a.qb = qb;
  a.M = M;
  a.N = N;
  a.W = (eptq::f16*)W;
  hipStream_t s = (hipStream_t)stream;
  rc = kind == eptq::KIND_E8D4 ? eptq::launch_dequant<eptq::KIND_E8D4>(a, s)
                               : eptq::launch_dequant<eptq::KIND_E8>(a, s);
  if (rc) return fail(EPTQ_EUNSUPPORTED, "%s: layer too large (M=%d N=%d)", fn, M, N);
  return check_launch(fn);
}

bool overlaps(const void* a, const void* b, size_t bytes) {
  if (!a || !b) return false;
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + bytes && y < x + bytes;
}

// [a, a + a_bytes) and [b, b + b_bytes) share a byte.
bool ranges_overlap(const void* a, size_t a_bytes, const void* b, size_t b_bytes) {
  if (!a || !b || !a_bytes || !b_bytes) return false;
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + b_bytes && y < x + a_bytes;
}

// Layers reading an activation that the decode kernel forms itself (prep 1:
// residual add + RMSNorm); see LinearArgs.
// pair: layers[0] = gate, layers[1] = up of equal M; y (B, 8M) = silu(gate) ⊙ up
// (ldy = 8M, the layers' y offsets unused).
int fused_linear(const char* fn, int n, const eptq_layer* layers, const void* codes, const void* x,
                 int ldx, int prep, const void* x2, const void* nw, float eps, void* xsum, int N, int B,
                 void* y, int ldy, void* stream, bool pair = false) {
  if (n < 1 || n > eptq::kMaxLayers || !layers) return fail(EPTQ_EINVAL, "%s: n_layers=%d (1..%d)", fn, n, eptq::kMaxLayers);
  if (pair && layers[0].M != layers[1].M)
    return fail(EPTQ_EINVAL, "%s: gate M=%d and up M=%d differ", fn, layers[0].M, layers[1].M);
  const int bmax = pair ? 2 : 8;
  if (B < 0 || B > bmax) return fail(B < 0 ? EPTQ_EINVAL : EPTQ_EUNSUPPORTED, "%s: B=%d (0..%d)", fn, B, bmax);
  if (B > 0 && (!x || !y)) return fail(EPTQ_EINVAL, "%s: null input/y", fn);
  if (prep == 1 && !nw) return fail(EPTQ_EINVAL, "%s: null norm weight", fn);
  if ((x && !aligned16(x)) || (x2 && !aligned16(x2)) || (nw && !aligned16(nw)) || (xsum && !aligned16(xsum)))
    return fail(EPTQ_EUNSUPPORTED, "%s: activation pointers must be 16-byte aligned", fn);
  const size_t row_bytes = (size_t)B * N * 2;
  if (overlaps(xsum, x, row_bytes) || overlaps(xsum, x2, row_bytes))
    return fail(EPTQ_EINVAL, "%s: resid_out overlaps resid or delta", fn);
  eptq::LinearArgs a[eptq::kMaxLayers];
  for (int l = 0; l < n; ++l) {
    const eptq_layer& L = layers[l];
    int rc = layer_args(fn, eptq::KIND_E8D4, L.Q, codes, EPTQ_F16, L.g, L.h, x, EPTQ_F16, L.O_vals, L.O_col,
                        L.O_row_ptr, L.bias, L.S_group, L.n_groups, L.M, N, B, &a[l]);
    if (rc) return rc;
    if (!pair && (L.y_offset < 0 || L.y_offset + 8LL * L.M > (long long)ldy || (L.y_offset & 3)))
      return fail(EPTQ_EINVAL, "%s: layer %d columns [%lld, %lld) outside a y row of %d (offset %% 4 == 0)",
                  fn, l, L.y_offset, L.y_offset + 8LL * L.M, ldy);
    a[l].y = (uint16_t*)y + (pair ? 0 : L.y_offset);
    a[l].ldy = ldy;
    a[l].prep = prep;
    a[l].ldx = ldx;
    a[l].x2 = (const uint16_t*)x2;
    a[l].nw = (const eptq::f16*)nw;
    a[l].eps = eps;
    a[l].xsum = (uint16_t*)xsum;
  }
  if (B == 0) return EPTQ_OK;
  const int lrc = pair ? eptq::launch_decode_e8d4_pair(a, (hipStream_t)stream)
                       : eptq::launch_decode_e8d4_multi(a, n, (hipStream_t)stream);
  if (lrc != 0) return fail(EPTQ_EUNSUPPORTED, "%s: the decode kernel does not take N=%d B=%d here", fn, N, B);
  return check_launch(fn);
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
std::atomic<char*> g_scratch[kMaxDevices];

__global__ void k_clear_words(uint32_t* p, int n) {
  for (int i = (int)(blockIdx.x * blockDim.x + threadIdx.x); i < n; i += (int)(gridDim.x * blockDim.x)) p[i] = 0u;
}

// Device address of the current device's scratch.  The first call on a
// device looks it up (with that device current) and queues on `s` a kernel
// that zeroes the tile counters; every launch that uses a counter afterwards
// returns it to zero, so later calls find them cleared.  The partial sums
// need no clearing (each is written before it is read).
int scratch_of_device(const char* fn, hipStream_t s, char** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(EPTQ_EHIP, "%s: hipGetDevice failed", fn);
  if (dev < 0 || dev >= kMaxDevices) return fail(EPTQ_EUNSUPPORTED, "%s: device %d (at most %d)", fn, dev, kMaxDevices);
  char* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      void* q = nullptr;
      const hipError_t e = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !q)
        return fail(EPTQ_EHIP, "%s: hipGetSymbolAddress(scratch): %s", fn, hipGetErrorString(e));
      k_clear_words<<<eptq::kSplitCounters / 256, 256, 0, s>>>((uint32_t*)q, eptq::kSplitCounters);
      if (const int rc = check_launch(fn)) return rc;
      p = (char*)q;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return EPTQ_OK;
}

// Body of eptq_e8d4_forward_multi and of its allocation-free variant
// (use_scratch: `work` is the library's own scratch, looked up once every
// argument has passed the same checks).
int forward_multi(const char* fn, int n_layers, const eptq_layer* layers, const void* codes, int codes_dtype,
                  const void* x, int x_dtype, int N, int B, void* y, int ldy, void* work, long long work_bytes,
                  void* stream, bool use_scratch = false) {
  if (n_layers <= 0 || !layers) return fail(EPTQ_EINVAL, "%s: n_layers=%d", fn, n_layers);
  if (work && (!aligned16(work) || work_bytes < 0))
    return fail(EPTQ_EINVAL, "%s: work must be 16-byte aligned with work_bytes >= 0", fn);
  if (B < 0) return fail(EPTQ_EINVAL, "%s: B=%d", fn, B);
  if (B > 0 && (!x || !y)) return fail(EPTQ_EINVAL, "%s: null x/y", fn);
  eptq::LinearArgs a[eptq::kMaxLayers];
  const int n = n_layers;
  // Validate every layer first; each writes columns [y_offset, y_offset + 8M) of y.
  for (int l = 0; l < n; ++l) {
    const eptq_layer& L = layers[l];
    eptq::LinearArgs t;
    int rc = layer_args(fn, eptq::KIND_E8D4, L.Q, codes, codes_dtype, L.g, L.h, x, x_dtype, L.O_vals,
                        L.O_col, L.O_row_ptr, L.bias, L.S_group, L.n_groups, L.M, N, B, &t);
    if (rc) return rc;
    if (L.y_offset < 0 || L.y_offset + 8LL * L.M > (long long)ldy || (L.y_offset & 3))
      return fail(EPTQ_EINVAL, "%s: layer %d columns [%lld, %lld) outside a y row of %d (offset %% 4 == 0)",
                  fn, l, L.y_offset, L.y_offset + 8LL * L.M, ldy);
    t.y = (uint16_t*)y + L.y_offset;
    t.ldy = ldy;
    if (l < eptq::kMaxLayers) a[l] = t;
  }
  if (B == 0) return EPTQ_OK;
  hipStream_t s = (hipStream_t)stream;
  if (use_scratch) {
    char* p = nullptr;
    if (const int rc = scratch_of_device(fn, s, &p)) return rc;
    work = p;
    work_bytes = (long long)kNoAllocScratchBytes;
  }
  // 17..128 rows: 16-row slices of the matrix-core decode kernel, every layer
  // in each slice's launch (its eligibility does not depend on the slice's
  // row count, so a first slice that launches means every slice does).
  if (B > eptq::kMatvecMaxBatch && B <= eptq::kSliceMaxTokens && n <= eptq::kMaxLayers) {
    int rc = 0;
    for (int b0 = 0; b0 < B && rc == 0; b0 += eptq::kMatvecMaxBatch) {
      eptq::LinearArgs sl[eptq::kMaxLayers];
      for (int l = 0; l < n; ++l) {
        sl[l] = a[l];
        sl[l].B = B - b0 < eptq::kMatvecMaxBatch ? B - b0 : eptq::kMatvecMaxBatch;
        sl[l].x = a[l].x + (size_t)b0 * a[l].ldx;
        sl[l].y = a[l].y + (size_t)b0 * ldy;
      }
      rc = eptq::launch_decode_mfma_multi(sl, n, s, work, work ? work_bytes : 0);
    }
    if (rc == 0) return check_launch(fn);
  }
  // One launch when the decode kernel takes them all, else one per layer.
  if (n > eptq::kMaxLayers || eptq::launch_decode_e8d4_multi(a, n, s, work, work ? work_bytes : 0) != 0) {
    for (int l = 0; l < n; ++l) {
      eptq::LinearArgs t;
      const eptq_layer& L = layers[l];
      layer_args(fn, eptq::KIND_E8D4, L.Q, codes, codes_dtype, L.g, L.h, x, x_dtype, L.O_vals, L.O_col,
                 L.O_row_ptr, L.bias, L.S_group, L.n_groups, L.M, N, B, &t);
      t.y = (uint16_t*)y + L.y_offset;
      t.ldy = ldy;
      const int rc = dispatch(fn, eptq::KIND_E8D4, t, s, work, work ? work_bytes : 0);
      if (rc) return rc;
    }
  }
  return check_launch(fn);
}


}  // namespace

extern "C" {

int eptq_abi_version(void) { return 3; }

const char* eptq_last_error(void) { return g_err; }

int eptq_e8d4_forward(const void* Q, const void* codes, int codes_dtype, const void* g,
                      const void* h, const void* x, int x_dtype, const void* O_vals,
                      const void* O_col, const void* O_row_ptr, const void* bias,
                      const void* S_group, int n_groups, int M, int N, int B, void* y,
                      void* stream) {
  return linear_common(eptq::KIND_E8D4, Q, codes, codes_dtype, g, h, x, x_dtype, O_vals, O_col,
                       O_row_ptr, bias, S_group, n_groups, M, N, B, y, stream);
}

int eptq_e8_forward(const void* Q, const void* codes, int codes_dtype, const void* g,
                    const void* h, const void* x, int x_dtype, const void* O_vals,
                    const void* O_col, const void* O_row_ptr, const void* bias,
                    const void* S_group, int n_groups, int M, int N, int B, void* y,
                    void* stream) {
  return linear_common(eptq::KIND_E8, Q, codes, codes_dtype, g, h, x, x_dtype, O_vals, O_col,
                       O_row_ptr, bias, S_group, n_groups, M, N, B, y, stream);
}

int eptq_e8d4_forward_multi(int n_layers, const eptq_layer* layers, const void* codes,
                            int codes_dtype, const void* x, int x_dtype, int N, int B, void* y,
                            int ldy, void* work, long long work_bytes, void* stream) {
  return forward_multi("eptq_e8d4_forward_multi", n_layers, layers, codes, codes_dtype, x, x_dtype, N, B, y, ldy,
                       work, work_bytes, stream);
}

int eptq_e8d4_forward_multi_noalloc(int n_layers, const eptq_layer* layers, const void* codes,
                                    int codes_dtype, const void* x, int x_dtype, int N, int B, void* y,
                                    int ldy, void* stream) {
  return forward_multi("eptq_e8d4_forward_multi_noalloc", n_layers, layers, codes, codes_dtype, x, x_dtype, N, B,
                       y, ldy, nullptr, 0, stream, true);
}

long long eptq_e8d4_work_bytes(void) {
  return eptq::decode_mfma_work_bytes() + (long long)eptq::kPrefillSplitBytes;
}

int eptq_llama_norm_linear(int n_layers, const eptq_layer* layers, const void* codes,
                           const void* resid, const void* delta, const void* w, float eps,
                           void* resid_out, int N, int B, void* y, int ldy, void* stream) {
  return fused_linear("eptq_llama_norm_linear", n_layers, layers, codes, resid, N, 1, delta, w, eps, resid_out,
                      N, B, y, ldy, stream);
}

int eptq_llama_norm_swiglu(const eptq_layer* gate_up, const void* codes, const void* resid, const void* delta,
                           const void* w, float eps, void* resid_out, int N, int B, void* out, void* stream) {
  if (!gate_up) return fail(EPTQ_EINVAL, "eptq_llama_norm_swiglu: null layers");
  return fused_linear("eptq_llama_norm_swiglu", 2, gate_up, codes, resid, N, 1, delta, w, eps, resid_out, N, B, out,
                      8 * gate_up[0].M, stream, true);
}

// eptq_llama_linear, and with act (B, 8M of the first layer) its SwiGLU form.
static int llama_linear(const char* fn, int n_layers, const eptq_layer* layers, const void* codes, const void* x,
                        int N, int B, const void* norm_w, float eps, const void* resid, void* y, int ldy,
                        void* work, long long work_bytes, void* stream, void* act) {
  const int n = n_layers;
  if (n < 1 || n > eptq::kMaxLayers || !layers) return fail(EPTQ_EINVAL, "%s: n_layers=%d (1..%d)", fn, n, eptq::kMaxLayers);
  if (B < 0 || B > 16) return fail(B < 0 ? EPTQ_EINVAL : EPTQ_EUNSUPPORTED, "%s: B=%d (0..16)", fn, B);
  if (B > 0 && (!x || !y)) return fail(EPTQ_EINVAL, "%s: null x/y", fn);
  if (work && (!aligned16(work) || work_bytes < 0))
    return fail(EPTQ_EINVAL, "%s: work must be 16-byte aligned with work_bytes >= 0", fn);
  if ((x && !aligned16(x)) || (norm_w && !aligned16(norm_w)))
    return fail(EPTQ_EUNSUPPORTED, "%s: x and norm_w must be 16-byte aligned", fn);
  if (resid && ((uintptr_t)resid & 3) != 0) return fail(EPTQ_EUNSUPPORTED, "%s: resid must be 4-byte aligned", fn);
  const size_t x_bytes = (size_t)B * N * 2, y_bytes = (size_t)B * (size_t)(ldy > 0 ? ldy : 0) * 2;
  if (ranges_overlap(x, x_bytes, y, y_bytes) || ranges_overlap(x, x_bytes, resid, y_bytes))
    return fail(EPTQ_EINVAL, "%s: x overlaps y or resid", fn);
  eptq::LinearArgs a[eptq::kMaxLayers];
  for (int l = 0; l < n; ++l) {
    const eptq_layer& L = layers[l];
    int rc = layer_args(fn, eptq::KIND_E8D4, L.Q, codes, EPTQ_F16, L.g, L.h, x, EPTQ_F16, L.O_vals, L.O_col,
                        L.O_row_ptr, L.bias, L.S_group, L.n_groups, L.M, N, B, &a[l]);
    if (rc) return rc;
    if (L.y_offset < 0 || L.y_offset + 8LL * L.M > (long long)ldy || (L.y_offset & 3))
      return fail(EPTQ_EINVAL, "%s: layer %d columns [%lld, %lld) outside a y row of %d (offset %% 4 == 0)",
                  fn, l, L.y_offset, L.y_offset + 8LL * L.M, ldy);
    a[l].y = (uint16_t*)y + L.y_offset;
    a[l].ldy = ldy;
    a[l].prep = norm_w ? 1 : 0;
    a[l].nw = (const eptq::f16*)norm_w;
    a[l].eps = eps;
    a[l].res = resid ? (const uint16_t*)resid + L.y_offset : nullptr;
  }
  if (B == 0) return EPTQ_OK;
  if (eptq::launch_decode_mfma_multi(a, n, (hipStream_t)stream, work, work ? work_bytes : 0, (uint16_t*)act) != 0)
    return fail(EPTQ_EUNSUPPORTED, "%s: the matrix-core decode kernel does not take N=%d B=%d%s", fn, N, B,
                norm_w ? " with the norm" : "");
  return check_launch(fn);
}

int eptq_llama_linear(int n_layers, const eptq_layer* layers, const void* codes, const void* x, int N, int B,
                      const void* norm_w, float eps, const void* resid, void* y, int ldy, void* work,
                      long long work_bytes, void* stream) {
  return llama_linear("eptq_llama_linear", n_layers, layers, codes, x, N, B, norm_w, eps, resid, y, ldy, work,
                      work_bytes, stream, nullptr);
}

int eptq_llama_linear_swiglu(const eptq_layer* gate_up, const void* codes, const void* x, int N, int B,
                             const void* norm_w, float eps, void* gu, void* out, void* work, long long work_bytes,
                             void* stream) {
  const char* fn = "eptq_llama_linear_swiglu";
  if (!gate_up) return fail(EPTQ_EINVAL, "%s: null layers", fn);
  if (gate_up[0].M != gate_up[1].M || gate_up[0].M <= 0)
    return fail(EPTQ_EINVAL, "%s: gate and up need equal M > 0 (%d, %d)", fn, gate_up[0].M, gate_up[1].M);
  if (!work) return fail(EPTQ_EINVAL, "%s: the SwiGLU form needs a workspace", fn);
  if (B > 0 && (!gu || !out)) return fail(EPTQ_EINVAL, "%s: null gu/out", fn);
  if (out && ((uintptr_t)out & 3) != 0) return fail(EPTQ_EUNSUPPORTED, "%s: out must be 4-byte aligned", fn);
  const int F = 8 * gate_up[0].M;
  const size_t out_bytes = (size_t)(B > 0 ? B : 0) * F * 2;
  if (ranges_overlap(out, out_bytes, gu, 2 * out_bytes) || ranges_overlap(out, out_bytes, x, (size_t)(B > 0 ? B : 0) * N * 2))
    return fail(EPTQ_EINVAL, "%s: out overlaps gu or x", fn);
  eptq_layer l2[2] = {gate_up[0], gate_up[1]};
  l2[0].y_offset = 0;
  l2[1].y_offset = F;
  return llama_linear(fn, 2, l2, codes, x, N, B, norm_w, eps, nullptr, gu, 2 * F, work, work_bytes, stream, out);
}

int eptq_f16_gemm_rows(const void* W, const void* x, const void* bias, int F, int N, int T, const void* row_scale,
                       void* y, int y_dtype, int ldy, void* stream) {
  const char* fn = "eptq_f16_gemm";
  if (F <= 0 || N <= 0 || T < 0 || ldy < F) return fail(EPTQ_EINVAL, "%s: F=%d N=%d T=%d ldy=%d", fn, F, N, T, ldy);
  if (y_dtype != EPTQ_F16 && y_dtype != EPTQ_BF16) return fail(EPTQ_EINVAL, "%s: y_dtype=%d", fn, y_dtype);
  if (T == 0) return EPTQ_OK;
  if (!W || !x || !y) return fail(EPTQ_EINVAL, "%s: null W/x/y", fn);
  if (row_scale && ((uintptr_t)row_scale & 3) != 0) return fail(EPTQ_EUNSUPPORTED, "%s: row_scale alignment", fn);
  // y's extent ends at its last row's F columns: y may be a column slice of
  // a wider output, allocated right before x or W.
  const size_t y_bytes = ((size_t)(T - 1) * ldy + F) * 2;
  if (ranges_overlap(y, y_bytes, x, (size_t)T * N * 2) || ranges_overlap(y, y_bytes, W, (size_t)F * N * 2) ||
      ranges_overlap(y, y_bytes, row_scale, (size_t)T * 4))
    return fail(EPTQ_EINVAL, "%s: y overlaps x, W or row_scale", fn);
  if (eptq::launch_gemm_f16w((const uint16_t*)W, (const uint16_t*)x, (const eptq::f16*)bias, F, N, T, N, (uint16_t*)y,
                             ldy, (hipStream_t)stream, (const float*)row_scale, y_dtype == EPTQ_BF16) != 0)
    return fail(EPTQ_EUNSUPPORTED, "%s: F=%d N=%d ldy=%d (multiples of 64, 64, 4) or alignment", fn, F, N, ldy);
  return check_launch(fn);
}

int eptq_f16_gemm(const void* W, const void* x, const void* bias, int F, int N, int T, void* y, int ldy,
                  void* stream) {
  return eptq_f16_gemm_rows(W, x, bias, F, N, T, nullptr, y, EPTQ_F16, ldy, stream);
}

int eptq_bf16_rows_to_f16(const void* x, int N, int T, void* x16, void* row_scale, void* stream) {
  const char* fn = "eptq_bf16_rows_to_f16";
  if (N <= 0 || T < 0) return fail(EPTQ_EINVAL, "%s: N=%d T=%d", fn, N, T);
  if (T == 0) return EPTQ_OK;
  if (!x || !x16 || !row_scale) return fail(EPTQ_EINVAL, "%s: null x/x16/row_scale", fn);
  if (ranges_overlap(x16, (size_t)T * N * 2, x, (size_t)T * N * 2) ||
      ranges_overlap(row_scale, (size_t)T * 4, x, (size_t)T * N * 2) ||
      ranges_overlap(row_scale, (size_t)T * 4, x16, (size_t)T * N * 2))
    return fail(EPTQ_EINVAL, "%s: x, x16 and row_scale must not overlap", fn);
  if (eptq::launch_bf16_rows_to_f16((const uint16_t*)x, N, T, (uint16_t*)x16, (float*)row_scale,
                                    (hipStream_t)stream) != 0)
    return fail(EPTQ_EUNSUPPORTED, "%s: N=%d (a multiple of 8 up to 16384) or alignment", fn, N);
  return check_launch(fn);
}

int eptq_e8d4_dequant(const void* Q, const void* codes_f32, const void* g, const void* h,
                      const void* O_vals, const void* O_col, const void* O_row_ptr,
                      const void* S_group, int n_groups, int M, int N, void* W, void* stream) {
  return dequant_common(eptq::KIND_E8D4, Q, codes_f32, g, h, O_vals, O_col, O_row_ptr, S_group,
                        n_groups, M, N, W, stream);
}

int eptq_e8_dequant(const void* Q, const void* codes_f32, const void* g, const void* h,
                    const void* O_vals, const void* O_col, const void* O_row_ptr,
                    const void* S_group, int n_groups, int M, int N, void* W, void* stream) {
  return dequant_common(eptq::KIND_E8, Q, codes_f32, g, h, O_vals, O_col, O_row_ptr, S_group,
                        n_groups, M, N, W, stream);
}

}  // extern "C"

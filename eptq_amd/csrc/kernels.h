// Internal launch interface between the C ABI (abi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace eptq {

enum { KIND_E8D4 = 0, KIND_E8 = 1 };


struct DequantArgs {
  const int16_t* Q;
  const float* table;
  const f16* g;
  const f16* h;
  const f16* O;
  const int32_t* O_col;
  const int32_t* O_row_ptr;
  const f16* S;   // nullable
  int qb;
  int M, N;
  f16* W;
};

struct LinearArgs {
  const int16_t* Q;
  const void* codes;
  int codes_f32;        // table element type: 1 fp32, 0 fp16
  const f16* g;
  const f16* h;
  const uint16_t* x;    // fp16 or bf16 words
  int x_bf16;
  const f16* O;
  const int32_t* O_col;
  const int32_t* O_row_ptr;
  const f16* bias;      // nullable
  const f16* S;         // nullable
  int qb;
  int M, N, B;
  uint16_t* y;          // same element type as x
  int ldy;              // elements between consecutive rows of y (>= 8M)
  // Activation preparation fused into the decode launch (fp16 x; decode
  // kernel only): the Linear's input is
  //   prep 0: x
  //   prep 1: RMSNorm(x + x2) = nw ⊙ r / rms(r), r = fp16(x + x2) (x2 may be
  //           null); the first workgroup writes r to xsum (if non-null).
  //           The matrix-core kernel takes prep 1 with x2 and xsum null: it
  //           multiplies the weights by nw ⊙ x and the sums by 1/rms(x).
  int prep;
  int ldx;              // elements between consecutive rows of x
  const uint16_t* x2;
  const f16* nw;
  uint16_t* xsum;
  float eps;
  int pad_;
  // Residual (matrix-core kernel only; null elsewhere): y = fp16(res + fp16(out)),
  // res laid out like y (it may be y itself).
  const uint16_t* res;
};
static_assert(sizeof(LinearArgs) % 16 == 0, "LinearArgs is a whole number of 16-byte words");

// Up to kMaxLayers layers that share x (e.g. q, k and v): one decode launch,
// workgroups [start[l], start[l+1]) serve layer l.
constexpr int kMaxLayers = 4;
struct MultiArgs {
  LinearArgs l[kMaxLayers];
  int start[kMaxLayers + 1];
  int n;
  // Matrix-core kernel only (null elsewhere): with two layers gate and up of
  // equal M whose outputs sit side by side in y, also act (B, 8M) =
  // silu(gate) ⊙ up, written by whichever of a row tile's two workgroups
  // finishes last.
  uint16_t* act;
};

template <int KIND> int launch_dequant(const DequantArgs& a, hipStream_t s);
template <int KIND> int launch_matvec(const LinearArgs& a, hipStream_t s);
// MFMA prefill GEMM (B > 16); batch tiles of the matvec where it does not apply.
// work (nullable, work_bytes long): a decode workspace; past its first
// decode_mfma_work_bytes() bytes, launches whose tiles leave half the CUs
// idle or more split K over up to kPrefillMaxParts parts (fp32 sums there,
// added in part order by a second launch).  Launches sharing it must not
// overlap in time.
template <int KIND> int launch_gemm(const LinearArgs& a, hipStream_t s, void* work = nullptr,
                                    long long work_bytes = 0);
constexpr int kPrefillMaxParts = 4;
// The prefill area of a decode workspace (eptq_e8d4_work_bytes() includes it).
constexpr size_t kPrefillSplitBytes = (size_t)64 << 20;
// Persistent E8-D4 decode (B <= 8); -1 when the layer/batch is outside its range.
int launch_decode_e8d4(const LinearArgs& a, hipStream_t s);
// Several layers sharing x (same N, B, table, dtypes) in one launch; -1 when
// any of them is outside the decode kernel's range.
// work (nullable, work_bytes long, zero-filled before its first use): lets the
// matrix-core kernel split the columns of layers with few row tiles over
// several workgroups; launches sharing it must not overlap in time.
int launch_decode_e8d4_multi(const LinearArgs* layers, int n, hipStream_t s, void* work = nullptr,
                             long long work_bytes = 0);

// SwiGLU pair (B <= 2, fp16): layers[0] = gate and layers[1] = up of equal
// shape in one launch, y = silu(gate) ⊙ up written at layers[0].y with
// layers[0].ldy; -1 when the pair is outside the kernel's range.
int launch_decode_e8d4_pair(const LinearArgs* layers, hipStream_t s);

// Matrix-core E8-D4 decode (B <= 16, fp16 or bf16 x, fp16 table; prep 1 and a
// residual for fp16 x, B <= 8, N a multiple of 64);
// -1 when the layers are outside its range.  act (fp16 x, n = 2, equal M,
// layers[1].y = layers[0].y + 8M, a workspace): also act (B, 8M) =
// silu(gate) ⊙ up with the roundings of the separate SwiGLU kernel.
int launch_decode_mfma_multi(const LinearArgs* layers, int n, hipStream_t s, void* work = nullptr,
                             long long work_bytes = 0, uint16_t* act = nullptr);
// Split-K workspace of the matrix-core decode kernel: kSplitCounters int
// arrival counters (one per 64-row tile of a launch), then fp32 partial sums,
// kSplitPartBytes per (split tile, part): [16 batch rows][64 outputs], then
// the part's sum of squares of x per batch row (prep 1).
constexpr int kSplitCounters = 16384;
constexpr size_t kSplitCounterBytes = (size_t)kSplitCounters * 4;
constexpr size_t kSplitPartBytes = (16 * 64 + 16) * 4;
constexpr int kSplitTileRows = 64;
// Prefill GEMM over dequantized fp16 weights: y (T, F) = rs[t] · (x (T, N) ·
// Wᵀ) + bias for W (F, N) row-major, rs NULL for 1, y fp16 or (ybf) bf16;
// -1 when the shape is outside the kernel.
int launch_gemm_f16w(const uint16_t* W, const uint16_t* x, const f16* bias, int F, int N, int T, int ldx,
                     uint16_t* y, int ldy, hipStream_t s, const float* rs = nullptr, int ybf = 0);
// bf16 rows to fp16 for it: x16[t] = fp16(x[t] · 2^-e_t), rs[t] = 2^e_t.
int launch_bf16_rows_to_f16(const uint16_t* x, int N, int T, uint16_t* x16, float* rs, hipStream_t s);
// Workspace bytes that let the matrix-core decode split every launch it takes.
long long decode_mfma_work_bytes();
namespace dec { int mfma_min_batch_init(); }
inline int mfma_min_batch() {
  static const int v = dec::mfma_min_batch_init();
  return v;
}

// Largest batch served by the decode matvec; larger batches take the GEMM.
constexpr int kMatvecMaxBatch = 16;
// Up to this many rows an E8-D4 launch runs as 16-row slices of the
// matrix-core decode kernel: its 64-row tiles spread a layer over far more
// workgroups than the GEMM's 128-token tiles can at these token counts (one
// token tile: 32 workgroups for 4096 rows), and the slices re-read the weight
// from cache.  Measured at 32 / 128 / 256 tokens on 4096x4096: slices 27 /
// 106 / 214 us against 112 us for the GEMM; 4096x11008: 59 / 226 / 459 us
// against 285-290 us.
constexpr int kSliceMaxTokens = 128;

}  // namespace eptq

// Bit-exact dequantization of an EPTQ layer to fp16 W (8M, N).
//
// Device counterpart of dequantize_layer (reference algorithms/eptq.py:406-471).
// Per element, in IEEE fp32 with round-to-nearest-even and no contraction:
//   v = table row (E8-D4: codes[t,i] | codes[t,j]; E8: points[u])
//   v = v * fp32(S_group[row / qb, n])            (if S_group)
//   v = fp32(O[rank])  for critical blocks          (not multiplied by S)
//   W = fp16((v * fp32(g[row])) * fp32(h[n]))
// The table must be the fp32 one the reference's loader produces
// (reconstruct.py:52-62), so the bits match eptq.reconstruct.
//
// Layout: a thread takes (Q-row m, 8 consecutive columns) items with a
// grid stride (consecutive threads, consecutive column chunks of one row):
// one 16-byte index load and 16-byte g and h loads, and one 16-byte store in
// each of the 8 output rows.  Workgroups stay resident and stage the E8-D4
// table in LDS once.  The kernel is write-bound (16 bytes out per 2-byte
// index).

#include "common.h"
#include "kernels.h"

namespace eptq {

// First CSR slot in [lo, hi) whose column is >= n (columns ascend per row).
__device__ __forceinline__ int csr_lower_bound(const int32_t* __restrict__ col,
                                               int lo, int hi, int n) {
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (col[mid] < n) lo = mid + 1; else hi = mid;
  }
  return lo;
}

constexpr int kDqPerCu = 16;  // resident workgroups per CU (8: ~3% slower on the 11008-wide layers)

template <int KIND, bool HAS_S>
__global__ __launch_bounds__(256) void k_dequant(
    const int16_t* __restrict__ Q, const float* __restrict__ table,
    const f16* __restrict__ g, const f16* __restrict__ h,
    const f16* __restrict__ O, const int32_t* __restrict__ O_col,
    const int32_t* __restrict__ O_row_ptr, const f16* __restrict__ S, int qb,
    int M, int N, int chunks_per_row, int vec, f16* __restrict__ W) {
  __shared__ f32x4 tab[KIND == KIND_E8D4 ? 512 : 1];
  if (KIND == KIND_E8D4) {
    for (int i = threadIdx.x; i < 512; i += 256) tab[i] = ((const f32x4*)table)[i];
    __syncthreads();
  }
  const int64_t items = (int64_t)M * chunks_per_row;
  const int64_t stride = (int64_t)gridDim.x * 256;
  // 16-byte path: the next item's index, g and h chunks are requested before
  // the current item is computed (one item in flight per thread).
  u16x8 qnext = {};
  f16x8 hnext = {}, gnext = {};
  auto fetch = [&](int64_t i) {
    if (vec && i < items) {
      const int mm = (int)(i / chunks_per_row);
      const int nn = (int)(i - (int64_t)mm * chunks_per_row) * 8;
      qnext = *(const u16x8*)(Q + (size_t)mm * N + nn);
      hnext = *(const f16x8*)(h + nn);
      gnext = *(const f16x8*)(g + 8 * mm);
    }
  };
  fetch((int64_t)blockIdx.x * 256 + threadIdx.x);
  for (int64_t it = (int64_t)blockIdx.x * 256 + threadIdx.x; it < items; it += stride) {
    const int m = (int)(it / chunks_per_row);
    const int n0 = (int)(it - (int64_t)m * chunks_per_row) * 8;
    // 16-byte accesses when the host found N % 8 == 0 and Q, g, h, W 16-byte
    // aligned (every chunk then is whole); element by element otherwise.
    const bool full = vec && n0 + 8 <= N;
    const int r0 = O_row_ptr[m], r1 = O_row_ptr[m + 1];
    float gk[8];
    int16_t q8[8];
    f16 h8[8];
    if (vec) {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        gk[c] = (float)gnext[c];
        q8[c] = (int16_t)qnext[c];
        h8[c] = hnext[c];
      }
      fetch(it + stride);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) gk[k] = (float)g[8 * m + k];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        q8[c] = n0 + c < N ? Q[(size_t)m * N + n0 + c] : (int16_t)0;
        h8[c] = n0 + c < N ? h[n0 + c] : (f16)0.0f;
      }
    }
    // out[k] word c/2: the fp16 pair (column c, column c + 1) of output row
    // 8m + k, converted two at a time (one v_cvt_pk_f16_f32).
    u32x4 out[8];
#pragma unroll
    for (int c = 0; c < 8; c += 2) {
      float v[2][8];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const int n = n0 + c + cc;
        const unsigned u = (unsigned)((int)q8[c + cc] + 32768);
        if (u == 65535u) {
          const int i = csr_lower_bound(O_col, r0, r1, n);
          const bool hit = (i < r1) && (O_col[i] == n);
#pragma unroll
          for (int k = 0; k < 8; ++k) v[cc][k] = hit ? (float)O[(size_t)i * 8 + k] : 0.0f;
        } else {
          f32x4 a, b;
          if (KIND == KIND_E8D4) {
            a = tab[u >> 7];
            b = tab[((u >> 14) << 7) | (u & 127u)];
          } else {
            const f32x4* p = (const f32x4*)(table + (size_t)u * 8);
            a = p[0];
            b = p[1];
          }
          v[cc][0] = a.x; v[cc][1] = a.y; v[cc][2] = a.z; v[cc][3] = a.w;
          v[cc][4] = b.x; v[cc][5] = b.y; v[cc][6] = b.z; v[cc][7] = b.w;
          if (HAS_S) {
#pragma unroll
            for (int k = 0; k < 8; ++k)
              v[cc][k] = n < N ? v[cc][k] * (float)S[(size_t)((8 * m + k) / qb) * N + n] : v[cc][k];
          }
        }
      }
      const float h0 = (float)h8[c], h1 = (float)h8[c + 1];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        float w0 = (v[0][k] * gk[k]) * h0;
        float w1 = (v[1][k] * gk[k]) * h1;
        // The reference rounds twice: to fp32 at the multiply, then to fp16.
        // Materialize the fp32 products so the compiler cannot fold multiply
        // and conversion into one single-rounding mix instruction.
        asm volatile("" : "+v"(w0), "+v"(w1));
        out[k][c >> 1] = __builtin_bit_cast(uint32_t, (f16x2){(f16)w0, (f16)w1});
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      f16* dst = W + (size_t)(8 * m + k) * N + n0;
      if (full) {
        __builtin_nontemporal_store(out[k], (u32x4*)dst);   // streamed out, not re-read here
      } else {
        for (int c = 0; c < 8 && n0 + c < N; ++c) {
          // Through a local: this compiler's __builtin_bit_cast of a vector
          // element lvalue reads element 0.
          const uint32_t wd = out[k][c >> 1];
          dst[c] = __builtin_bit_cast(f16x2, wd)[c & 1];
        }
      }
    }
  }
}

template <int KIND>
int launch_dequant(const DequantArgs& a, hipStream_t s) {
  const int chunks = (a.N + 7) / 8;
  const int64_t items = (int64_t)a.M * chunks;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int vec = (a.N % 8 == 0) &&
                  ((((uintptr_t)a.Q | (uintptr_t)a.g | (uintptr_t)a.h | (uintptr_t)a.W) & 15u) == 0);
  int64_t blocks = (items + 255) / 256;
  if (blocks > (int64_t)cus * kDqPerCu) blocks = (int64_t)cus * kDqPerCu;
  if (blocks < 1) return 0;
  if (a.S)
    k_dequant<KIND, true><<<(unsigned)blocks, 256, 0, s>>>(
        a.Q, a.table, a.g, a.h, a.O, a.O_col, a.O_row_ptr, a.S, a.qb, a.M, a.N, chunks, vec, a.W);
  else
    k_dequant<KIND, false><<<(unsigned)blocks, 256, 0, s>>>(
        a.Q, a.table, a.g, a.h, a.O, a.O_col, a.O_row_ptr, nullptr, 1, a.M, a.N, chunks, vec, a.W);
  return 0;
}

template int launch_dequant<KIND_E8D4>(const DequantArgs&, hipStream_t);
template int launch_dequant<KIND_E8>(const DequantArgs&, hipStream_t);

}  // namespace eptq

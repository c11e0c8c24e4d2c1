// Fused decode matvec for E8-D4 and E8-lattice layers, batch 1..16.
//
// y[b, 8m+k] = g[8m+k] * ( sum_n v_k(Q[m,n]) * S[grp,n] * h[n] * x[b,n]
//                        + sum_{i in CSR(m)} O[i][k] * h[c_i] * x[b,c_i] ) + bias[8m+k]
// Same math as the reference decode kernels (csrc/eptq_kernels.cu:161-292,
// kernels/triton_e8d4.py:47-157) plus the fused S_group factor.
//
// Work split: a workgroup of 256 threads owns R consecutive Q-rows over all N
// columns; 256/R threads share a row, each taking 16-byte chunks (8 indices)
// at a stride of 256/R chunks.  No cross-workgroup reduction is needed.
//
// Latency structure (a 4096x4096 layer is only 4 MiB, so the kernel is a
// handful of memory round trips long):
//  * every lane issues all of its loads first — the table slice, then the
//    index chunks (non-temporal: Q is read once), then h / x / S chunks — so
//    one round trip covers the whole row;
//  * the E8-D4 table is staged in LDS as fp16 (4 KB) while those loads are in
//    flight; the E8 table (65535 x 8) is gathered from L2/MALL;
//  * the wave reduction uses DPP and permlane swaps (no LDS round trips
//    except one swizzle/bpermute per value above 8 lanes).
//
// E8-D4 index decode without a sign fix-up: the LDS table is stored at
// position e ^ 0x100 for table row e, so both halves are addressed straight
// from the stored int16 bits v (u = v ^ 0x8000):
//   rows 0..3: table[(u >> 7)]                      -> byte (v >> 4) & 0xFF8
//   rows 4..7: table[((u >> 14) << 7) | (u & 127)]   -> bits 10-11 of the
//              first address with bits 3-9 replaced by (v & 127) << 3.
// Critical blocks (v = 32767) decode as table row 511 in both halves (E8:
// row 0); the CSR pass adds O·(h x) minus that decoded vector, so the main
// loop has no per-index branch.

#include "common.h"
#include "kernels.h"

namespace eptq {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

template <int BT> struct MatvecCfg;
template <> struct MatvecCfg<1>  { static constexpr int MAXJ = 8; };
template <> struct MatvecCfg<2>  { static constexpr int MAXJ = 8; };
template <> struct MatvecCfg<4>  { static constexpr int MAXJ = 4; };
template <> struct MatvecCfg<8>  { static constexpr int MAXJ = 2; };
template <> struct MatvecCfg<16> { static constexpr int MAXJ = 1; };

template <int KIND, int BT, int R, bool HAS_S, bool CODES_F32, typename XT>
__global__ __launch_bounds__(kThreads) void k_matvec(LinearArgs a) {
  constexpr int MAXJ = MatvecCfg<BT>::MAXJ;
  constexpr int V = BT * 8;
  constexpr int TPR = kThreads / R;            // threads per row
  constexpr int WPR = TPR / 64;                // waves per row (0 when a row is < 1 wave)
  static_assert(TPR >= 64, "a row must span at least one wave");
  __shared__ f16x4 tab[KIND == KIND_E8D4 ? 512 : 1];
  __shared__ float red[kWaves][V];

  const int tid = threadIdx.x;
  const int r_local = tid / TPR;
  const int rl = tid % TPR;                    // lane index within the row
  const int m = blockIdx.x * R + r_local;
  const bool row_ok = m < a.M;
  const int N = a.N;
  const int nch = N >> 3;
  const int B = a.B;
  const int mm = row_ok ? m : a.M - 1;         // clamp for address math only
  const u32x4* __restrict__ qrow = (const u32x4*)(a.Q + (size_t)mm * N);
  const int grp = HAS_S ? (8 * mm) / a.qb : 0;

  // ---- issue every load of the first round up front ----
  f16x4 tload[2];
  if (KIND == KIND_E8D4) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int e = tid + kThreads * p;        // table row
      if (a.codes_f32) {
        const f32x4 f = ((const f32x4*)a.codes)[e];
        tload[p] = (f16x4){(f16)f.x, (f16)f.y, (f16)f.z, (f16)f.w};
      } else {
        tload[p] = ((const f16x4*)a.codes)[e];
      }
    }
  }
  u32x4 qv[MAXJ];
  f16x8 hv[MAXJ];
  f16x8 sv[MAXJ];
  u16x8 xv[MAXJ][BT];
  auto load_round = [&](int base) {
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
      const int c = base + rl + TPR * j;
      if (row_ok && c < nch) qv[j] = __builtin_nontemporal_load(qrow + c);
      else qv[j] = (u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
      const int c = base + rl + TPR * j;
      if (c < nch) {
        const int n0 = c << 3;
        hv[j] = *(const f16x8*)(a.h + n0);
        if (HAS_S) sv[j] = *(const f16x8*)(a.S + (size_t)grp * N + n0);
#pragma unroll
        for (int b = 0; b < BT; ++b)
          xv[j][b] = (b < B) ? *(const u16x8*)(a.x + (size_t)b * N + n0) : (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
  };
  load_round(0);

  if (KIND == KIND_E8D4) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int e = tid + kThreads * p;
      tab[e ^ 0x100] = tload[p];
    }
    __syncthreads();
  }
  const char* __restrict__ tabB = (const char*)tab;

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;

  for (int base = 0; base < nch; base += TPR * MAXJ) {
    if (base > 0) load_round(base);
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
      if (base + rl + TPR * j >= nch) break;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t w = qv[j][d];
        float c8[2][8];
        if (KIND == KIND_E8D4) {
          const uint32_t a1lo = (w >> 4) & 0xFF8u;
          const uint32_t a1hi = (w >> 20) & 0xFF8u;
          const uint32_t a2lo = bfi(0x3F8u, w << 3, a1lo);
          const uint32_t a2hi = bfi(0x3F8u, w >> 13, a1hi);
          const f16x4 t1l = *(const f16x4*)(tabB + a1lo);
          const f16x4 t2l = *(const f16x4*)(tabB + a2lo);
          const f16x4 t1h = *(const f16x4*)(tabB + a1hi);
          const f16x4 t2h = *(const f16x4*)(tabB + a2hi);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            c8[0][k] = (float)t1l[k]; c8[0][k + 4] = (float)t2l[k];
            c8[1][k] = (float)t1h[k]; c8[1][k + 4] = (float)t2h[k];
          }
        } else {
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            uint32_t u = ((s ? (w >> 16) : w) & 0xffffu) ^ 0x8000u;
            u = (u == 0xffffu) ? 0u : u;
            if (CODES_F32) {
              const f32x4* p = (const f32x4*)((const float*)a.codes + (size_t)u * 8);
              const f32x4 lo = p[0], hi = p[1];
              c8[s][0] = lo.x; c8[s][1] = lo.y; c8[s][2] = lo.z; c8[s][3] = lo.w;
              c8[s][4] = hi.x; c8[s][5] = hi.y; c8[s][6] = hi.z; c8[s][7] = hi.w;
            } else {
              const f16x8 t = *((const f16x8*)a.codes + u);
#pragma unroll
              for (int k = 0; k < 8; ++k) c8[s][k] = (float)t[k];
            }
          }
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const int e = 2 * d + s;
          f16 hs = hv[j][e];
          if (HAS_S) hs = (f16)((float)hs * (float)sv[j][e]);
#pragma unroll
          for (int b = 0; b < BT; ++b) {
            const float xh = HAS_S ? Act<XT>::to_f32(xv[j][b][e]) * ((float)hv[j][e] * (float)sv[j][e])
                                   : Act<XT>::mul_f16(xv[j][b][e], hs);
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[b * 8 + k] = fmaf(c8[s][k], xh, acc[b * 8 + k]);
          }
        }
      }
    }
  }

  // ---- critical blocks: add O·(h x), remove the decoded marker vector ----
  if (row_ok) {
    const int r0 = a.O_row_ptr[m], r1 = a.O_row_ptr[m + 1];
    if (r0 < r1) {
      float mk[8];
      if (KIND == KIND_E8D4) {
        const f16x4 t5 = tab[511 ^ 0x100];
#pragma unroll
        for (int k = 0; k < 4; ++k) { mk[k] = (float)t5[k]; mk[k + 4] = (float)t5[k]; }
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k)
          mk[k] = CODES_F32 ? ((const float*)a.codes)[k] : (float)((const f16*)a.codes)[k];
      }
      for (int i = r0 + rl; i < r1; i += TPR) {
        const int col = a.O_col[i];
        const f16x8 o = *(const f16x8*)(a.O + (size_t)i * 8);
        const float hn = (float)a.h[col];
        const float hsn = HAS_S ? hn * (float)a.S[(size_t)grp * N + col] : hn;
#pragma unroll
        for (int b = 0; b < BT; ++b) {
          if (b < B) {
            const float xb = Act<XT>::to_f32(a.x[(size_t)b * N + col]);
            const float xh = xb * hn, xhs = xb * hsn;
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[b * 8 + k] += (float)o[k] * xh - mk[k] * xhs;
          }
        }
      }
    }
  }

  // ---- reduce: lanes of the wave, then the waves of the row ----
  const int base_idx = wave_reduce_halving<V>(acc);
  const int wave = tid >> 6, lane = tid & 63;
  if (WaveReduceOut<V>::writer(lane)) {
#pragma unroll
    for (int p = 0; p < WaveReduceOut<V>::per_lane; ++p) red[wave][base_idx + p] = acc[p];
  }
  __syncthreads();
  if (row_ok) {
    for (int t = rl; t < V; t += TPR) {
      const int b = t >> 3, k = t & 7;
      if (b < B) {
        float s = 0.0f;
        const int w0 = r_local * WPR;
#pragma unroll
        for (int w = 0; w < WPR; ++w) s += red[w0 + w][t];
        const int row = 8 * m + k;
        s = s * (float)a.g[row];
        if (a.bias) s += (float)a.bias[row];
        a.y[(size_t)b * a.ldy + row] = Act<XT>::from_f32(s);
      }
    }
  }
}

// Rows per workgroup: enough workgroups to cover the chip, fewer table fills
// and reductions per row when rows are plentiful or short.
static int pick_rows(int M, int N) {
  const int nch = N >> 3;
  if (nch <= 64 * 8) {                       // a wave covers the row in <= 8 chunks
    if (M >= 4 * 1024 || nch <= 64 * 2) return 4;
  }
  if (M >= 2 * 1024 && nch <= 128 * 8) return 2;
  return 1;
}

template <int KIND, int BT, bool HAS_S, bool CODES_F32, typename XT>
static void launch_r(const LinearArgs& a, hipStream_t s) {
  const int R = pick_rows(a.M, a.N);
  const unsigned grid = (unsigned)((a.M + R - 1) / R);
  if (R == 4)
    k_matvec<KIND, BT, 4, HAS_S, CODES_F32, XT><<<grid, kThreads, 0, s>>>(a);
  else if (R == 2)
    k_matvec<KIND, BT, 2, HAS_S, CODES_F32, XT><<<grid, kThreads, 0, s>>>(a);
  else
    k_matvec<KIND, BT, 1, HAS_S, CODES_F32, XT><<<grid, kThreads, 0, s>>>(a);
}

template <int KIND, int BT, bool HAS_S, bool CODES_F32>
static void launch_bt(const LinearArgs& a, hipStream_t s) {
  if (a.x_bf16) launch_r<KIND, BT, HAS_S, CODES_F32, bf16>(a, s);
  else launch_r<KIND, BT, HAS_S, CODES_F32, f16>(a, s);
}

template <int KIND, bool HAS_S, bool CODES_F32>
static void launch_b(const LinearArgs& a, hipStream_t s) {
  if (a.B <= 1) launch_bt<KIND, 1, HAS_S, CODES_F32>(a, s);
  else if (a.B <= 2) launch_bt<KIND, 2, HAS_S, CODES_F32>(a, s);
  else if (a.B <= 4) launch_bt<KIND, 4, HAS_S, CODES_F32>(a, s);
  else if (a.B <= 8) launch_bt<KIND, 8, HAS_S, CODES_F32>(a, s);
  else launch_bt<KIND, 16, HAS_S, CODES_F32>(a, s);
}

template <int KIND>
int launch_matvec(const LinearArgs& a, hipStream_t s) {
  if (a.B < 1 || a.B > kMatvecMaxBatch) return -1;
  if (KIND == KIND_E8D4) {
    // The E8-D4 table is converted into LDS, so its precision is a runtime flag.
    if (a.S) launch_b<KIND, true, false>(a, s);
    else launch_b<KIND, false, false>(a, s);
  } else {
    if (a.codes_f32) {
      if (a.S) launch_b<KIND, true, true>(a, s); else launch_b<KIND, false, true>(a, s);
    } else {
      if (a.S) launch_b<KIND, true, false>(a, s); else launch_b<KIND, false, false>(a, s);
    }
  }
  return 0;
}

template int launch_matvec<KIND_E8D4>(const LinearArgs&, hipStream_t);
template int launch_matvec<KIND_E8>(const LinearArgs&, hipStream_t);

}  // namespace eptq

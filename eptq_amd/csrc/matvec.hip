// Fused decode matvec for E8-D4 and E8-lattice layers, batch 1..16.
//
// y[b, 8m+k] = g[8m+k] * ( sum_n v_k(Q[m,n]) * S[grp,n] * h[n] * x[b,n]
//                        + sum_{i in CSR(m)} O[i][k] * h[c_i] * x[b,c_i] ) + bias[8m+k]
// Same math as the reference decode kernels (csrc/eptq_kernels.cu:161-292,
// kernels/triton_e8d4.py:47-157) plus the fused S_group factor.
//
// HBM-bound design (one workgroup of 4 waves per Q-row, all N columns):
//  * every lane first issues all of its 16-byte index loads (8 indices each,
//    non-temporal: Q is streamed once), so the whole row is in flight;
//  * the E8-D4 table (512 x 4) is staged in LDS as fp16 (4 KB) while those
//    loads are outstanding; the E8 table (65535 x 8) stays in L2/MALL;
//  * h, x (and S) are read as 16-byte vectors per 8-column chunk;
//  * critical blocks decode like any index (E8-D4: table row 511 twice; E8:
//    row 0) and the CSR pass adds O·xh minus that decoded vector, so the
//    main loop carries no per-index branch;
//  * partial sums are reduced across the wave by recursive halving and across
//    the 4 waves through LDS; g, bias and the output conversion are fused.

#include "common.h"
#include "kernels.h"

namespace eptq {

template <int BT> struct MatvecCfg;
template <> struct MatvecCfg<1>  { static constexpr int MAXJ = 8; };
template <> struct MatvecCfg<2>  { static constexpr int MAXJ = 4; };
template <> struct MatvecCfg<4>  { static constexpr int MAXJ = 4; };
template <> struct MatvecCfg<8>  { static constexpr int MAXJ = 2; };
template <> struct MatvecCfg<16> { static constexpr int MAXJ = 2; };

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

template <int KIND, int BT, bool HAS_S, bool CODES_F32, typename XT>
__global__ __launch_bounds__(kThreads) void k_matvec(LinearArgs a) {
  constexpr int MAXJ = MatvecCfg<BT>::MAXJ;
  constexpr int V = BT * 8;
  __shared__ f16x4 tab[KIND == KIND_E8D4 ? 512 : 1];
  __shared__ float red[kWaves][V];

  const int m = blockIdx.x;
  const int tid = threadIdx.x;
  const int N = a.N;
  const int nch = N >> 3;
  const int B = a.B;
  const u32x4* __restrict__ qrow = (const u32x4*)(a.Q + (size_t)m * N);
  const int grp = HAS_S ? (8 * m) / a.qb : 0;

  // Issue the first round of index loads before anything else.
  u32x4 qv[MAXJ];
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) {
    const int c = tid + kThreads * j;
    if (c < nch) qv[j] = __builtin_nontemporal_load(qrow + c);
    else qv[j] = (u32x4){0u, 0u, 0u, 0u};
  }

  if (KIND == KIND_E8D4) {
    for (int i = tid; i < 512; i += kThreads) {
      f16x4 t;
      if (a.codes_f32) {
        const f32x4 f = ((const f32x4*)a.codes)[i];
        t = (f16x4){(f16)f.x, (f16)f.y, (f16)f.z, (f16)f.w};
      } else {
        t = ((const f16x4*)a.codes)[i];
      }
      tab[i] = t;
    }
    __syncthreads();
  }

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;

  const uint16_t* __restrict__ xg = a.x;
  for (int base = 0; base < nch; base += kThreads * MAXJ) {
    if (base > 0) {
#pragma unroll
      for (int j = 0; j < MAXJ; ++j) {
        const int c = base + tid + kThreads * j;
        if (c < nch) qv[j] = __builtin_nontemporal_load(qrow + c);
      }
    }
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
      const int c = base + tid + kThreads * j;
      if (c >= nch) break;
      const int n0 = c << 3;
      const f16x8 hv = *(const f16x8*)(a.h + n0);
      f16x8 sv;
      if (HAS_S) sv = *(const f16x8*)(a.S + (size_t)grp * N + n0);
      u16x8 xv[BT];
#pragma unroll
      for (int b = 0; b < BT; ++b) {
        if (b < B) xv[b] = *(const u16x8*)(xg + (size_t)b * N + n0);
        else xv[b] = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t w = qv[j][e >> 1];
        uint32_t u = (((e & 1) ? (w >> 16) : w) & 0xffffu) ^ 0x8000u;
        float c8[8];
        if (KIND == KIND_E8D4) {
          const f16x4 a1 = tab[u >> 7];
          const f16x4 a2 = tab[((u >> 7) & 0x180u) | (u & 0x7fu)];
#pragma unroll
          for (int k = 0; k < 4; ++k) { c8[k] = (float)a1[k]; c8[k + 4] = (float)a2[k]; }
        } else {
          u = (u == 0xffffu) ? 0u : u;
          if (CODES_F32) {
            const f32x4* p = (const f32x4*)((const float*)a.codes + (size_t)u * 8);
            const f32x4 lo = p[0], hi = p[1];
            c8[0] = lo.x; c8[1] = lo.y; c8[2] = lo.z; c8[3] = lo.w;
            c8[4] = hi.x; c8[5] = hi.y; c8[6] = hi.z; c8[7] = hi.w;
          } else {
            const f16x8 t = *((const f16x8*)a.codes + u);
#pragma unroll
            for (int k = 0; k < 8; ++k) c8[k] = (float)t[k];
          }
        }
        float hs = (float)hv[e];
        if (HAS_S) hs *= (float)sv[e];
#pragma unroll
        for (int b = 0; b < BT; ++b) {
          const float xh = Act<XT>::to_f32(xv[b][e]) * hs;
#pragma unroll
          for (int k = 0; k < 8; ++k) acc[b * 8 + k] = fmaf(c8[k], xh, acc[b * 8 + k]);
        }
      }
    }
  }

  // Critical blocks: add O·(h x) and remove what the main loop accumulated
  // for the marker index (decoded vector times h·S·x).
  {
    const int r0 = a.O_row_ptr[m], r1 = a.O_row_ptr[m + 1];
    float mk[8];
    if (KIND == KIND_E8D4) {
      const f16x4 t5 = tab[511];
#pragma unroll
      for (int k = 0; k < 4; ++k) { mk[k] = (float)t5[k]; mk[k + 4] = (float)t5[k]; }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        mk[k] = CODES_F32 ? ((const float*)a.codes)[k] : (float)((const f16*)a.codes)[k];
    }
    for (int i = r0 + tid; i < r1; i += kThreads) {
      const int col = a.O_col[i];
      const f16x8 o = *(const f16x8*)(a.O + (size_t)i * 8);
      const float hn = (float)a.h[col];
      const float hsn = HAS_S ? hn * (float)a.S[(size_t)grp * N + col] : hn;
#pragma unroll
      for (int b = 0; b < BT; ++b) {
        if (b < B) {
          const float xb = Act<XT>::to_f32(xg[(size_t)b * N + col]);
          const float xh = xb * hn, xhs = xb * hsn;
#pragma unroll
          for (int k = 0; k < 8; ++k)
            acc[b * 8 + k] += (float)o[k] * xh - mk[k] * xhs;
        }
      }
    }
  }

  const int base_idx = wave_reduce_halving<V>(acc);
  const int wave = tid >> 6, lane = tid & 63;
  if ((lane & WaveReduceOut<V>::writer_mask) == 0) {
#pragma unroll
    for (int p = 0; p < WaveReduceOut<V>::per_lane; ++p) red[wave][base_idx + p] = acc[p];
  }
  __syncthreads();
  if (tid < V) {
    const int b = tid >> 3, k = tid & 7;
    if (b < B) {
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) s += red[w][tid];
      const int row = 8 * m + k;
      s = s * (float)a.g[row];
      if (a.bias) s += (float)a.bias[row];
      a.y[(size_t)b * (8 * a.M) + row] = Act<XT>::from_f32(s);
    }
  }
}

template <int KIND, int BT, bool HAS_S, bool CODES_F32>
static void launch_bt(const LinearArgs& a, hipStream_t s) {
  if (a.x_bf16)
    k_matvec<KIND, BT, HAS_S, CODES_F32, bf16><<<a.M, kThreads, 0, s>>>(a);
  else
    k_matvec<KIND, BT, HAS_S, CODES_F32, f16><<<a.M, kThreads, 0, s>>>(a);
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

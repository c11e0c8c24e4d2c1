// Prefill GEMM for E8-D4 and E8 layers: y = (decode(Q)·diag(h·S)) · xᵀ ⊙ g + CSR + bias.
//
// Counterpart of the reference's large-batch path e8d4_wmma_v2_kernel +
// at::mul(x, h) (csrc/eptq_kernels.cu:309-461, :520-537), rebuilt for gfx950
// MFMA.  The contraction is a genuine dense GEMM on v_mfma_f32_16x16x32_f16.
// Three kernels (each with its own comment below):
//  * k_gemm_lds_e8d4 (E8-D4 without S_group, fp16 x, in_features a multiple
//    of 64: the Llama prefill case): producer waves decode the weight tile
//    into LDS and bring the activation tile in by LDS DMA while eight waves
//    run the MFMAs;
//  * k_gemm_rows_e8d4 (E8-D4 without S_group, bf16 x or in_features an odd
//    multiple of 32): each wave decodes its 64 rows of the weight straight
//    into MFMA A operands in registers;
//  * k_gemm_e8d4 / k_gemm_e8 (S_group layers, E8, shapes the others do not
//    take): the weight is dequantized tile by tile into LDS, as below.
//
// E8 layers (1 MB table, larger than LDS) gather each index's 16-byte table
// row from global memory (L2-resident after first use) one K-step ahead,
// through a buffer resource bounded at the table's 65535 rows, so the marker
// index reads zeros; otherwise the pipeline is the same.
//
// Tiling: a workgroup (4 waves) computes 128 output features (16 Q-rows) ×
// 128 tokens; each wave a 64 × 64 sub-tile as 4 × 4 MFMA tiles of 16 × 16,
// accumulated in fp32 over K-steps of 32 input columns.  Per K-step:
//  * every thread decodes one 32-bit word of Q (two adjacent columns of one
//    Q-row) through the LDS table (4 lookups), pairs the two columns per
//    output row with byte permutes, scales the pairs by (h·S) of the two
//    columns in fp16 and writes 8 words of the W tile (rows × K, fp16);
//  * the activation tile x[t, k0..k0+31] is copied to LDS unscaled (h lives on
//    the weight side, so x is never rounded);
//  * the step is software-pipelined: the table lookups of step s+1 are issued
//    before the MFMAs of step s and its W/X tiles written after them, into
//    the other half of a double-buffered LDS tile (one barrier per step);
//    the global loads run kPF steps ahead in a register ring.
// Critical blocks are written into the W tile itself: the workgroup stages
// its rows' CSR entries in LDS once (fp16(O·h) per output row), 16 walker
// threads list the entries whose column falls in each K-step two steps
// ahead, and the thread that decodes a marker index writes the entry's
// values in place of the table row, so the MFMA loop needs no correction.
// (Entries beyond the LDS cap, only in very dense layers, are added after the
// loop from global memory.)  The output is g ⊙ acc + bias, written as fp16.

#include <stdlib.h>

#include "common.h"
#include "kernels.h"
#include "mfma_decode.h"

namespace eptq {

namespace {

constexpr int kGT = 256;            // threads
constexpr int kBM = 128;            // output features per workgroup (16 Q-rows)
constexpr int kBQ = kBM / 8;        // Q-rows per workgroup
constexpr int kBN = 128;            // tokens per workgroup
constexpr int kTJ = kBN / 32;       // 16-token MFMA tiles per wave (waves split the tokens in two)
constexpr int kXC = kBN / 64;       // 16-byte activation chunks per thread per K-step
constexpr int kBK = 32;             // input columns per K-step
constexpr int kLd = kBK + 8;        // LDS row stride in halves (80 bytes)
constexpr int kEntCap = 512;        // CSR entries staged in LDS per workgroup
constexpr int kPerStep = kBK;       // max entries of one Q-row inside one K-step

typedef f16 h2 __attribute__((ext_vector_type(2)));
typedef f16 h8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t gperm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}
// By value: __builtin_bit_cast applied directly to a vector-element lvalue
// reads element 0 with this compiler.
__device__ __forceinline__ uint32_t bits16(f16 v) { return (uint32_t)__builtin_bit_cast(uint16_t, v); }
__device__ __forceinline__ uint32_t gpk_mul(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) * __builtin_bit_cast(h2, b));
}

}  // namespace

template <int KIND, bool HAS_S>
__device__ __forceinline__ void gemm_tile(const LinearArgs& a, int OB) {
  __shared__ f16x4 tab[KIND == KIND_E8D4 ? 512 : 1];
  __shared__ __attribute__((aligned(16))) f16 Ws[2][kBM][kLd];
  __shared__ __attribute__((aligned(16))) f16 Xs[2][kBN][kLd];
  __shared__ int ent_col[kEntCap];
  __shared__ __attribute__((aligned(16))) h8 ent_val[kEntCap];
  __shared__ uint16_t lst[3][kBQ][kPerStep];
  __shared__ int lcnt[3][kBQ];
  __shared__ int rps[kBQ + 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;      // wave's 64 x 64 sub-tile
  const int N = a.N, M = a.M, T = a.B;
  const int ob = blockIdx.x % OB;               // consecutive workgroups share a token tile
  const int tb = blockIdx.x / OB;
  const int m0 = ob * kBQ;                      // first Q-row
  const int t0 = tb * kBN;                      // first token
  const int nsteps = N / kBK;
  const char* __restrict__ tabB = (const char*)tab;

  // ---- per-thread roles for the tile loads ----
  const int dq = tid >> 4;                      // Q-row of the word this thread decodes
  const int dc = (tid & 15) * 2;                // its first column inside the step
  const int qrow = m0 + dq;                      // < M: the launcher requires M % 16 == 0
  const uint32_t* __restrict__ qsrc = (const uint32_t*)(a.Q + (size_t)qrow * N);
  const int grp = HAS_S ? (8 * qrow) / a.qb : 0;
  // x chunks: kXC 16-byte pieces, token xt[i], column chunk xc[i].  Sixteen
  // consecutive lanes take 16 tokens at one chunk, so each 16-lane pass of
  // the 16-byte LDS writes hits 64 distinct banks (80-byte rows); a wave
  // still reads whole 64-byte pieces of 16 token rows from global memory.
  int xt[kXC], xc[kXC];
#pragma unroll
  for (int i = 0; i < kXC; ++i) {
    const int idx = tid + kGT * i;
    xt[i] = (idx & 15) | ((idx >> 6) << 4);
    xc[i] = ((idx >> 4) & 3) * 8;
  }

  // ---- table and CSR staging ----
  if constexpr (KIND == KIND_E8D4) {
#pragma unroll
    for (int p = 0; p < 2; ++p) tab[(tid + kGT * p) ^ 0x100] = ((const f16x4*)a.codes)[tid + kGT * p];
  }
  if (tid <= kBQ) rps[tid] = a.O_row_ptr[m0 + tid < M ? m0 + tid : M];
  __syncthreads();
  const int e0 = rps[0];
  const int ecount = rps[kBQ] - e0;
  // What a marker index leaves in the tile before its entry replaces it:
  // E8-D4 table row 511 in both halves, E8 zeros (out of the table's range).
  f16x4 t5 = {(f16)0.0f, (f16)0.0f, (f16)0.0f, (f16)0.0f};
  if constexpr (KIND == KIND_E8D4) t5 = tab[511 ^ 0x100];
  for (int e = tid; e < ecount && e < kEntCap; e += kGT) {
    const int gi = e0 + e;
    const int col = a.O_col[gi];
    const f16x8 o = *(const f16x8*)(a.O + (size_t)gi * 8);
    const f16 hc = a.h[col];
    h8 d;   // the tile's value for the block: O·h (the reference applies no S to O)
#pragma unroll
    for (int k = 0; k < 8; ++k) d[k] = (f16)((float)o[k] * (float)hc);
    ent_col[e] = col;
    ent_val[e] = d;
  }
  __syncthreads();   // staged entries are read by the walkers and the decoders
  // Walker thread q (tid < 16) owns Q-row q's entry cursor.
  int wcur = 0, wend = 0;
  if (tid < kBQ) {
    wcur = rps[tid] - e0;
    wend = rps[tid + 1] - e0;
  }

  // ---- register ring: the global loads of the next kPF steps are in flight ----
  constexpr int kPF = 3;
  uint32_t qw[kPF], hsw[kPF];
  u32x4 xr[kPF][kXC];
  auto load_step = [&](int slot, int s) {
    const int k0 = (s < nsteps ? s : nsteps - 1) * kBK;
    qw[slot] = qsrc[(k0 + dc) >> 1];
    uint32_t hw = *(const uint32_t*)(a.h + k0 + dc);
    if (HAS_S) hw = gpk_mul(hw, *(const uint32_t*)(a.S + (size_t)grp * N + k0 + dc));
    hsw[slot] = hw;
#pragma unroll
    for (int i = 0; i < kXC; ++i) {
      // Tokens past T read a valid row; their output columns are never stored.
      const int tt = t0 + xt[i];
      xr[slot][i] = *(const u32x4*)(a.x + (size_t)(tt < T ? tt : T - 1) * N + k0 + xc[i]);
    }
  };

  // Step pipeline: the 4 table lookups of the next step are issued before
  // this step's MFMAs and the W/X tiles of the next step are written after
  // them, so LDS latency and dequantization overlap the matrix work.
  u32x2 lk[4];    // E8-D4: the four LDS table lookups of the word
  u32x4 lk8[2];   // E8: the two gathered table rows (low and high index)
  const __amdgpu_buffer_rsrc_t rtab = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.codes, (short)0, KIND == KIND_E8 ? 65535 * 16 : 0, 0x00020000);
  auto lookups = [&](int slot) {
    const uint32_t w = qw[slot];
    if constexpr (KIND == KIND_E8D4) {
      const uint32_t a1lo = (w >> 4) & 0xFF8u;
      const uint32_t a1hi = (w >> 20) & 0xFF8u;
      const uint32_t a2lo = bfi(0x3F8u, w << 3, a1lo);
      const uint32_t a2hi = bfi(0x3F8u, w >> 13, a1hi);
      lk[0] = *(const u32x2*)(tabB + a1lo);
      lk[1] = *(const u32x2*)(tabB + a2lo);
      lk[2] = *(const u32x2*)(tabB + a1hi);
      lk[3] = *(const u32x2*)(tabB + a2hi);
    } else {
      // u = Q + 32768 = raw bits ^ 0x8000; the marker (u = 65535) is past
      // the resource and reads zeros.
      const uint32_t ulo = (w & 0xFFFFu) ^ 0x8000u, uhi = (w >> 16) ^ 0x8000u;
      lk8[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rtab, ulo * 16, 0, 0));
      lk8[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rtab, uhi * 16, 0, 0));
    }
  };
  // Walkers: list the critical blocks of K-step s per Q-row (in list
  // buffer s % 3, two steps before the decoders read it).
  auto walk = [&](int s) {
    if (tid < kBQ) {
      const int b3 = s % 3;
      const int kend = (s + 1) * kBK;
      int nw = 0;
      while (wcur < wend && wcur < kEntCap && ent_col[wcur] < kend) {
        lst[b3][tid][nw++] = (uint16_t)wcur;
        ++wcur;
      }
      lcnt[b3][tid] = nw;
    }
  };
  auto write_tiles = [&](int slot, int buf, int k0) {
    // pr[k] = (row k at column dc, row k at column dc + 1), fp16 pairs.
    uint32_t pr[8];
    if constexpr (KIND == KIND_E8D4) {
      const u32x2 t1l = lk[0], t2l = lk[1], t1h = lk[2], t2h = lk[3];
      pr[0] = gperm(t1h[0], t1l[0], 0x05040100u);
      pr[1] = gperm(t1h[0], t1l[0], 0x07060302u);
      pr[2] = gperm(t1h[1], t1l[1], 0x05040100u);
      pr[3] = gperm(t1h[1], t1l[1], 0x07060302u);
      pr[4] = gperm(t2h[0], t2l[0], 0x05040100u);
      pr[5] = gperm(t2h[0], t2l[0], 0x07060302u);
      pr[6] = gperm(t2h[1], t2l[1], 0x05040100u);
      pr[7] = gperm(t2h[1], t2l[1], 0x07060302u);
    } else {
      const u32x4 lo = lk8[0], hi = lk8[1];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        pr[2 * d] = gperm(hi[d], lo[d], 0x05040100u);
        pr[2 * d + 1] = gperm(hi[d], lo[d], 0x07060302u);
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) pr[k] = gpk_mul(pr[k], hsw[slot]);
    // Marker indices (raw 0x7FFF) take their entry's values instead.
    const uint32_t w = qw[slot];
    const bool mlo = (w & 0xFFFFu) == 0x7FFFu, mhi = (w >> 16) == 0x7FFFu;
    if (mlo || mhi) {
      const int b3 = (k0 / kBK) % 3;
      const int n = lcnt[b3][dq];
      for (int e = 0; e < n; ++e) {
        const int idx = lst[b3][dq][e];
        const int c = ent_col[idx] - k0 - dc;   // 0: low half, 1: high half
        if ((c == 0 && mlo) || (c == 1 && mhi)) {
          const h8 v = ent_val[idx];
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const uint32_t vb = bits16(v[k]);
            pr[k] = c == 0 ? (pr[k] & 0xFFFF0000u) | vb : (pr[k] & 0x0000FFFFu) | (vb << 16);
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) *(uint32_t*)&Ws[buf][8 * dq + k][dc] = pr[k];
#pragma unroll
    for (int i = 0; i < kXC; ++i) *(u32x4*)&Xs[buf][xt[i]][xc[i]] = xr[slot][i];
  };

#pragma unroll
  for (int p = 0; p < kPF; ++p) load_step(p, p);

  f32x4 acc[4][kTJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kTJ; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // prologue: the lists of steps 0 and 1, then step 0's tiles
  walk(0);
  if (nsteps > 1) walk(1);
  __syncthreads();
  lookups(0);
  write_tiles(0, 0, 0);
  load_step(0, kPF);
  __syncthreads();

  for (int s0 = 0; s0 < nsteps; s0 += kPF) {
#pragma unroll
  for (int p = 0; p < kPF; ++p) {
    const int s = s0 + p;
    if (s >= nsteps) break;
    const int buf = s & 1;
    const int k0 = s * kBK;
    const int pn = (p + 1) % kPF;              // ring slot holding step s + 1
    const bool more = s + 1 < nsteps;

    h8 af[4], bf[kTJ];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      af[i] = *(const h8*)&Ws[buf][64 * wm + 16 * i + (lane & 15)][8 * (lane >> 4)];
#pragma unroll
    for (int j = 0; j < kTJ; ++j)
      bf[j] = *(const h8*)&Xs[buf][(kBN / 2) * wn + 16 * j + (lane & 15)][8 * (lane >> 4)];
    if (more) lookups(pn);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < kTJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    if (more) {
      write_tiles(pn, buf ^ 1, k0 + kBK);
      load_step(pn, s + 1 + kPF);
    }
    if (s + 2 < nsteps) walk(s + 2);

    __syncthreads();
  }
  }

  // Entries beyond the LDS cap (only for very dense critical-block layers):
  // apply them from global memory.
  if (ecount > kEntCap) {
    __syncthreads();
    for (int qq = 0; qq < 8; ++qq) {
      const int q = 8 * wm + qq;
      const int lo = rps[q] - e0, hi = rps[q + 1] - e0;
      const int ti = qq >> 1;
      const int lg = lane >> 4;
      const bool mine = (lg >> 1) == (qq & 1);
      for (int e = (lo > kEntCap ? lo : kEntCap); e < hi; ++e) {
        const int gi = e0 + e;
        const int col = a.O_col[gi];
        const f16x8 o = *(const f16x8*)(a.O + (size_t)gi * 8);
        const f16 hc = a.h[col];
        f16 hs = hc;
        if (HAS_S) hs = (f16)((float)hc * (float)a.S[(size_t)((8 * (m0 + q)) / a.qb) * N + col]);
        if (mine) {
          const int kb = 4 * (lg & 1);
#pragma unroll
          for (int j = 0; j < kTJ; ++j) {
            const int tt = t0 + (kBN / 2) * wn + 16 * j + (lane & 15);
            const float xv = tt < T ? (float)__builtin_bit_cast(f16, a.x[(size_t)tt * N + col]) : 0.f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int k = kb + v;
              const f16 wmk = (f16)((float)t5[k & 3] * (float)hs);
              const float dv = (float)(f16)((float)o[k] * (float)hc - (float)wmk);
              acc[ti][j][v] += dv * xv;
            }
          }
        }
      }
    }
  }

  // ---- epilogue: g, bias, fp16 ----
  const int lg = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r0 = 8 * m0 + 64 * wm + 16 * i + 4 * lg;   // first of this lane's 4 rows
    if (r0 >= 8 * M) continue;
    float gv[4], bv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      gv[v] = (float)a.g[r0 + v];
      bv[v] = a.bias ? (float)a.bias[r0 + v] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kTJ; ++j) {
      const int tt = t0 + (kBN / 2) * wn + 16 * j + (lane & 15);
      if (tt >= T) continue;
      f16x4 o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = (f16)(acc[i][j][v] * gv[v] + bv[v]);
      *(f16x4*)((f16*)a.y + (size_t)tt * a.ldy + r0) = o;
    }
  }
}


// ---------------------------------------------------------------------------
// E8-D4 prefill GEMM with the weights decoded in registers (no S_group).
//
// A workgroup (kW waves) computes 64·kW output features × 128 tokens; each
// wave owns 64 features (8 Q-rows) for all 128 tokens.  Per K-step of 32
// columns a lane decodes its 8 indices straight into v_mfma_f32_16x16x32_f16
// A operands (the matrix-core decode matvec's mapping: 8 table lookups, 16
// byte permutes, no lane exchange) and reuses them for the 8 MFMA token
// tiles, so the decoded weight never goes through LDS.  The B operands are
// the shared activation tile fp16(x · h·2^-e) in LDS (tokens × 32 columns,
// double-buffered, written once per step by the whole workgroup; h lives on
// the activation side, as in the reference's at::mul(x, h) before its WMMA
// GEMM, csrc/eptq_kernels.cu:520-537), with 2^-e a workgroup-uniform power
// of two that keeps |x·h·2^-e| <= |x|.  A critical block replaces the
// lane's four looked-up values with its O values in registers: each lane
// walks its Q-row's CSR entries (the first kEnt of the workgroup staged in
// LDS) with a cursor; entries past the stage keep the marker's table row in
// the K loop and are corrected after it.  D of MFMA c, token tile j, lane (n, lg),
// element v is feature 16·lg + 4v + c of the wave's 64 for token 16j + n, so
// a lane stores 16 consecutive features of one token.
namespace g2 {
constexpr int kTok = 128;                  // tokens per workgroup
constexpr int kJ = kTok / 16;              // MFMA token tiles per wave
constexpr int kBK = 32;                    // input columns per K-step
constexpr int kXLd = kBK + 8;              // activation tile row stride in halves (80 bytes)
constexpr int kEnt = 1024;                 // critical blocks staged in LDS per workgroup
constexpr int kPF = 2;                     // K-steps of indices in flight per lane

__host__ __device__ inline size_t dyn_bytes(int N) { return (size_t)N * 2; }
}  // namespace g2

// kBF: bf16 x and y (the activation operand is still fp16(x·h·2^-e), from
// the exact fp32 product; the reference casts bf16 x to fp16 for its GEMM,
// kernels/linear.py:200-203).
template <int kW, bool kBF>
__global__ __launch_bounds__(64 * kW, 8 / kW) void k_gemm_rows_e8d4(LinearArgs a, int OB) {
  constexpr int kT = 64 * kW, kQR = 8 * kW;
  constexpr int kTok = g2::kTok, kJ = g2::kJ, kBK = g2::kBK;
  constexpr int kXLd = g2::kXLd, kPF = g2::kPF;
  // Critical blocks staged in LDS: 0.2% of a five-wave workgroup's 40 rows
  // of 13824 columns is ~1100 (one workgroup per CU leaves the LDS for it).
  constexpr int kEnt = kW == 5 ? 2 * g2::kEnt : g2::kEnt;
  constexpr int kXCH = kTok * kBK / 8;   // 16-byte activation chunks per K-step
  __shared__ f16x4 tab[512];
  __shared__ __attribute__((aligned(16))) uint16_t Xs[2][kTok][kXLd];
  __shared__ int ecol[kEnt];
  __shared__ __attribute__((aligned(16))) u32x4 eov[kEnt];
  __shared__ int rps[kQR + 1];
  __shared__ float wmx[kW];
  extern __shared__ __attribute__((aligned(16))) char dyn[];
  uint16_t* const hs = (uint16_t*)dyn;   // fp16(h·2^-e), N entries

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = a.N, T = a.B, ldx = a.ldx;
  const int ob = (int)blockIdx.x % OB, tb = (int)blockIdx.x / OB;
  const int m0 = ob * kQR;      // first Q-row (the launcher requires M % kQR == 0)
  const int t0 = tb * kTok;     // first token
  const int nsteps = N / kBK, nch = N / 8;

  // ---- table, h (max |h|), CSR row pointers ----
  constexpr int kTabP = (512 + kT - 1) / kT;
  f16x4 tl[kTabP];
#pragma unroll
  for (int p = 0; p < kTabP; ++p)
    if (tid + kT * p < 512) tl[p] = ((const f16x4*)a.codes)[tid + kT * p];
  if (tid <= kQR) rps[tid] = a.O_row_ptr[m0 + tid];
  float mx = 0.0f;
  for (int c = tid; c < nch; c += kT) {
    const u32x4 hv = ((const u32x4*)a.h)[c];
    *(u32x4*)(hs + 8 * c) = hv;
    const f16x8 hf = __builtin_bit_cast(f16x8, hv);
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf((float)hf[e]));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) wmx[wave] = mx;
#pragma unroll
  for (int p = 0; p < kTabP; ++p)
    if (tid + kT * p < 512) tab[(tid + kT * p) ^ 0x100] = tl[p];
  __syncthreads();
  mx = wmx[0];
#pragma unroll
  for (int w = 1; w < kW; ++w) mx = fmaxf(mx, wmx[w]);
  int ex = 0;
  if (mx > 1.0f) ex = (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xff) - 126;   // 2^ex >= mx
  const float out_scale = __builtin_ldexpf(1.0f, ex);
  const f16 down = (f16)__builtin_ldexpf(1.0f, -ex);
  const uint32_t down2 = __builtin_bit_cast(uint32_t, (h2){down, down});
  for (int c = tid; c < nch; c += kT) {   // the chunks this thread wrote
    u32x4 hv = *(const u32x4*)(hs + 8 * c);
#pragma unroll
    for (int d = 0; d < 4; ++d) hv[d] = gpk_mul(hv[d], down2);
    *(u32x4*)(hs + 8 * c) = hv;
  }
  const int e0 = rps[0];
  const int nst = rps[kQR] - e0 < kEnt ? rps[kQR] - e0 : kEnt;
  for (int e = tid; e < nst; e += kT) {
    ecol[e] = a.O_col[e0 + e];
    eov[e] = ((const u32x4*)a.O)[e0 + e];
  }

  // ---- per-lane roles ----
  const int i = lane & 15, kg = lane >> 4;
  const mdec::Half half(i);
  const int hsel = i & 1;
  const int lq = 8 * wave + (i >> 1);                          // this lane's Q-row in the workgroup
  const int16_t* __restrict__ qp = a.Q + (size_t)(m0 + lq) * N + 8 * kg;
  u32x4 qv[kPF];
#pragma unroll
  for (int p = 0; p < kPF; ++p) qv[p] = *(const u32x4*)(qp + (p < nsteps ? p : nsteps - 1) * kBK);
  // Activation chunks: chunk c = tid + kT·p is token c/4, columns 8(c%4)..+7.
  constexpr int kXC = (kXCH + kT - 1) / kT;   // chunks per thread (the last pass partial for kW = 5)
  static_assert(kPF % 2 == 0, "activation slots follow the step parity");
  u32x4 xr[2][kXC];   // activation loads two K-steps ahead (slot = step parity)
  // Every load is issued unconditionally (steps past the end and the partial
  // last pass of a five-wave workgroup reload valid addresses and are never
  // stored), so the compiler can count the loads in flight and wait for
  // exactly the one it needs.
  auto load_x = [&](int st, int slot) {
    const int stc = st < nsteps ? st : nsteps - 1;
#pragma unroll
    for (int p = 0; p < kXC; ++p) {
      const int c0 = tid + kT * p;
      const int c = c0 < kXCH ? c0 : c0 - kT;
      const int tt = t0 + (c >> 2);
      xr[slot][p] = *(const u32x4*)(a.x + (size_t)(tt < T ? tt : T - 1) * ldx + stc * kBK + 8 * (c & 3));
    }
  };
  auto store_x = [&](int buf, int st, int slot) {
#pragma unroll
    for (int p = 0; p < kXC; ++p) {
      const int c = tid + kT * p;
      if (kXCH % kT != 0 && c >= kXCH) break;
      const u32x4 hv = *(const u32x4*)(hs + st * kBK + 8 * (c & 3));
      u32x4 v;
      if constexpr (kBF) {
        const f16x8 hf = __builtin_bit_cast(f16x8, hv);
        const u16x8 xb = __builtin_bit_cast(u16x8, xr[slot][p]);
        f16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (f16)(Act<bf16>::to_f32(xb[e]) * (float)hf[e]);
        v = __builtin_bit_cast(u32x4, o);
      } else {
#pragma unroll
        for (int d = 0; d < 4; ++d) v[d] = gpk_mul(xr[slot][p][d], hv[d]);
      }
      *(u32x4*)&Xs[buf][c >> 2][8 * (c & 3)] = v;
    }
  };
  load_x(0, 0);
  __syncthreads();   // hs scaled, entries staged
  load_x(1, 1);
  store_x(0, 0, 0);
  load_x(2, 0);
  __syncthreads();

  f32x4 acc[4][kJ];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int j = 0; j < kJ; ++j) acc[c][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const char* __restrict__ tabB = (const char*)tab;

  // The cursor reads LDS only (a load from memory in the loop would make the
  // compiler wait for every index and activation load in flight): entries
  // past the stage keep the marker's table row in the loop and are
  // corrected after it.
  int ec = rps[lq] - e0;
  const int ee = rps[lq + 1] - e0 < kEnt ? rps[lq + 1] - e0 : kEnt;
  int ncol = ec < ee ? ecol[ec] : 0x7fffffff;
  for (int s0 = 0; s0 < nsteps; s0 += kPF) {
#pragma unroll
    for (int p = 0; p < kPF; ++p) {
      const int s = s0 + p;
      if (s >= nsteps) break;
      const int buf = s & 1;
      u32x2 lo[4], hi[4];
      half.lookup(qv[p], tabB, lo, hi);
      qv[p] = *(const u32x4*)(qp + (s + kPF < nsteps ? s + kPF : nsteps - 1) * kBK);
      u32x4 bf[kJ];
#pragma unroll
      for (int j = 0; j < kJ; ++j) bf[j] = *(const u32x4*)&Xs[buf][16 * j + i][8 * kg];
      // Critical blocks in this lane's 8 columns take the table values' place.
      const int klo = s * kBK + 8 * kg;
      while (ncol < klo + 8) {
        if (ncol >= klo) {
          const u32x4 o = eov[ec];
          const u32x2 oh = hsel ? (u32x2){o[2], o[3]} : (u32x2){o[0], o[1]};
          const int jc = ncol - klo;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            if (jc == 2 * d) lo[d] = oh;
            if (jc == 2 * d + 1) hi[d] = oh;
          }
        }
        ++ec;
        ncol = ec < ee ? ecol[ec] : 0x7fffffff;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f16x8 aw = __builtin_bit_cast(f16x8, mdec::Half::operand(lo, hi, c));
#pragma unroll
        for (int j = 0; j < kJ; ++j)
          acc[c][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw, __builtin_bit_cast(f16x8, bf[j]), acc[c][j], 0, 0, 0);
      }
      // kPF is even and s0 a multiple of it: slot (s + 1) & 1 = (p + 1) & 1.
      if (s + 1 < nsteps) store_x(buf ^ 1, s + 1, (p + 1) & 1);
      load_x(s + 3, (p + 1) & 1);
      __syncthreads();
    }
  }

  // Entries past the LDS stage (dense critical blocks only): the loop
  // multiplied table row 511 by fp16(x·h·2^-e) at their columns; add
  // (O - row 511) times the same operand.  Lane group kg holds Q-rows
  // 2kg, 2kg + 1 of the wave (features 16kg .. 16kg + 15).
  if (rps[kQR] - e0 > kEnt) {
    const f16x4 t5 = tab[511 ^ 0x100];
#pragma unroll
    for (int qq = 0; qq < 8; ++qq) {
      if ((qq >> 1) != kg) continue;
      const int lqq = 8 * wave + qq;
      const int elo = rps[lqq] - e0 > kEnt ? rps[lqq] - e0 : kEnt;
      const int ehi = rps[lqq + 1] - e0;
      for (int e = elo; e < ehi; ++e) {
        const int col = a.O_col[e0 + e];
        const f16x8 o = ((const f16x8*)a.O)[e0 + e];
        const f16 hc = __builtin_bit_cast(f16, hs[col]);
        float dv[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) dv[k] = (float)o[k] - (float)t5[k & 3];
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
          const int tt = t0 + 16 * j + i;
          const uint16_t xw = a.x[(size_t)(tt < T ? tt : T - 1) * ldx + col];
          float xh;
          if constexpr (kBF) xh = (float)(f16)(Act<bf16>::to_f32(xw) * (float)hc);
          else xh = (float)(f16)(__builtin_bit_cast(f16, xw) * hc);
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const int r = 8 * (qq & 1) + k;   // this lane's feature index 4v + c
            acc[r & 3][j][r >> 2] += dv[k] * xh;
          }
        }
      }
    }
  }

  // ---- epilogue: y = acc·2^e·g + bias, 16 consecutive features per lane and token ----
  const int r0 = 8 * m0 + 64 * wave + 16 * kg;
  const f16x8 g0 = *(const f16x8*)(a.g + r0), g1 = *(const f16x8*)(a.g + r0 + 8);
  f16x8 b0 = {}, b1 = {};
  if (a.bias) {
    b0 = *(const f16x8*)(a.bias + r0);
    b1 = *(const f16x8*)(a.bias + r0 + 8);
  }
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const int tt = t0 + 16 * j + i;
    if (tt >= T) continue;
    u16x8 o0, o1;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float y0 = acc[q & 3][j][q >> 2] * out_scale * (float)g0[q] + (float)b0[q];
      const float y1 = acc[q & 3][j][2 + (q >> 2)] * out_scale * (float)g1[q] + (float)b1[q];
      if constexpr (kBF) {
        o0[q] = Act<bf16>::from_f32(y0);
        o1[q] = Act<bf16>::from_f32(y1);
      } else {
        o0[q] = Act<f16>::from_f32(y0);
        o1[q] = Act<f16>::from_f32(y1);
      }
    }
    uint16_t* yp = a.y + (size_t)tt * a.ldy + r0;
    *(u16x8*)yp = o0;
    *(u16x8*)(yp + 8) = o1;
  }
}

// ---------------------------------------------------------------------------
// E8-D4 prefill GEMM with the weight tile decoded into LDS and the activation
// tile brought in by LDS DMA (fp16 x, no S_group).
//
// A workgroup of 8 + NPW waves computes BF output features (BF/8 Q-rows) ×
// 256 tokens.  Waves 0-7 only multiply: wave w owns features (w & 1)·BF/2 ..
// +BF/2 of tokens 64·(w >> 1) .. +63 as (BF/32) × 4 tiles of
// v_mfma_f32_16x16x32_f16, reading both operands from LDS.  Waves 8 ..
// 8 + NPW - 1 (one or two per SIMD) produce, one K-step of 64 columns ahead:
//  * X: 256 rows × 128 bytes of raw fp16 x written to LDS by
//    global_load_lds_dwordx4 (no register staging), rows XOR-swizzled by
//    16-byte chunk so the MFMA fragment reads (16 rows at one chunk) hit
//    distinct banks; the index tile (BF/8 Q-rows × 64 int16) and the step's
//    64 h values the same way;
//  * W: each lane decodes units of 8 indices × one half (rows 0-3 or 4-7) of
//    an 8-row block through the LDS table (8 lookups, the matrix-core decode's
//    operand mapping), multiplies by h and writes 4 rows × 8 columns of fp16
//    W·h·2^-e into a tile whose layout spreads each row's chunks over both
//    halves of a 256-byte bank row (conflict-free writes and reads); critical
//    blocks are then patched in from the workgroup's CSR entries staged in
//    LDS (a per-lane cursor).
// X, W, indices and h are double-buffered; one barrier per K-step.  h sits on
// the weight side and the table is scaled by 2^-e once (2^e ≥ max|h|, so
// W·h·2^-e cannot overflow fp16); y = acc·2^e·g + bias.  Entries past the LDS
// stage keep table row 511 in the loop and are corrected after it.  One
// workgroup per CU (LDS).
namespace g3 {
constexpr int kBK = 64;      // columns per K-step: 128-byte rows
constexpr int kBT = 256;     // tokens per workgroup
constexpr int kLds = 160 * 1024;
__device__ __forceinline__ int xpos(int t, int c) { return t * 128 + ((c ^ ((t >> 1) & 7)) << 4); }
// Row r's 16-byte chunk c: the chunks of rows r and r ^ 1 alternate across the
// 256-byte bank row they share, XOR-swizzled by r / 2, so 16 consecutive rows
// at one chunk and rows c, c + 4 of one 8-row block (the decode's 16-lane
// write groups) each cover 16 distinct 16-byte bank slots.
__device__ __forceinline__ int wpos(int r, int c) {
  const int b = (r ^ (r >> 2)) & 1;
  return (r >> 1) * 256 + (((2 * c + b) ^ (2 * ((r >> 1) & 7))) << 4);
}
template <int BF> struct Lay {
  static constexpr int QR = BF / 8, QRp = (QR + 7) / 8 * 8;
  static constexpr int X0 = 0, XS = kBT * 128;                   // 2 stages
  static constexpr int W0 = 2 * XS, WS = BF * 128;             // 2 stages, then 1 KB for idle lanes' writes
  static constexpr int I0 = W0 + 2 * WS + 1024, IS = QRp * 128;  // 2 stages
  static constexpr int H0 = I0 + 2 * IS, HS = 128;               // 2 stages
  static constexpr int T0 = H0 + 2 * HS;                         // 4 KB table
  static constexpr int R0 = T0 + 4096;                           // CSR row pointers
  static constexpr int M0 = R0 + ((QR + 1) * 4 + 15) / 16 * 16;  // per-wave max |h|
  static constexpr int C0 = M0 + 64;                             // staged entry columns
  static constexpr int kEnt = ((kLds - C0) / 20) / 16 * 16;      // 2272 (BF 160), 944 (BF 256)
  static constexpr int O0 = C0 + kEnt * 4;                       // staged entry O values
  static constexpr int Bytes = O0 + kEnt * 16;
  static_assert(Bytes <= kLds, "LDS budget");
};
}  // namespace g3

// NPW producer waves: 4, or 8 when the MFMA waves' registers allow four
// waves per SIMD.
//
// Split K (part != null): the grid is P copies of the OB × TB tiles, copy p
// taking K-steps [p·nk/P, (p+1)·nk/P); each writes its fp32 sums times 2^e
// to part[p][token][feature] (8M features per token) and k_gemm_split_sum
// adds the P copies in part order, then applies g and bias.
template <int BF, int NPW>
__global__ __launch_bounds__(64 * (8 + NPW), (8 + NPW) / 4) void k_gemm_lds_e8d4(LinearArgs a, int OB, int P,
                                                                               float* __restrict__ part) {
  using L = g3::Lay<BF>;
  constexpr int kBK = g3::kBK, kBT = g3::kBT, kNT = 64 * (8 + NPW);
  static_assert(NPW == 4 || NPW == 8, "producer waves");
  constexpr int QR = L::QR, QRp = L::QRp, kEnt = L::kEnt;
  constexpr int FW = BF / 2, FA = FW / 16, TW = kBT / 4, TB = TW / 16;
  static_assert(FW % 16 == 0 && QRp <= 32, "whole MFMA tiles, index tile in 4 DMA rows of waves");
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  int* const rps = (int*)(smem + L::R0);
  float* const wmx = (float*)(smem + L::M0);
  int* const ecol = (int*)(smem + L::C0);
  u32x4* const eov = (u32x4*)(smem + L::O0);
  char* const tabB = smem + L::T0;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = a.N, T = a.B, ldx = a.ldx;
  // Workgroups are dealt to the 8 XCDs round-robin: give each XCD a run of
  // consecutive tiles (same token tile, neighbouring feature tiles).
  int blk = blockIdx.x;
  const int G = gridDim.x;
  if ((G & 7) == 0) blk = (blk & 7) * (G >> 3) + (blk >> 3);
  const int tiles = G / P;
  const int pp = blk / tiles;
  blk -= pp * tiles;
  const int ob = blk % OB, tb = blk / OB;
  const int m0 = ob * QR, f0 = 8 * m0, t0 = tb * kBT;
  const int nk = N / kBK, nch = N / 8;
  // This workgroup's K-steps [k0, k1) (all of them without a split).
  const int k0 = pp * nk / P, k1 = (pp + 1) * nk / P, nkp = k1 - k0;

  // ---- table scaled by 2^-e (2^e >= max |h|), CSR rows, staged entries ----
  const f16x4 tl = ((const f16x4*)a.codes)[tid & 511];
  if (tid <= QR) rps[tid] = a.O_row_ptr[m0 + tid];
  float mx = 0.0f;
  for (int c = tid; c < nch; c += kNT) {
    const f16x8 hf = ((const f16x8*)a.h)[c];
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf((float)hf[e]));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) wmx[wave] = mx;
  __syncthreads();
  mx = wmx[0];
#pragma unroll
  for (int w = 1; w < kNT / 64; ++w) mx = fmaxf(mx, wmx[w]);
  int ex = 0;
  if (mx > 1.0f) ex = (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xff) - 126;
  const float out_scale = __builtin_ldexpf(1.0f, ex);
  const f16 down = (f16)__builtin_ldexpf(1.0f, -ex);
  const uint32_t down2 = __builtin_bit_cast(uint32_t, (h2){down, down});
  if (tid < 512) {
    u32x2 tw = __builtin_bit_cast(u32x2, tl);
    tw[0] = gpk_mul(tw[0], down2);
    tw[1] = gpk_mul(tw[1], down2);
    *(u32x2*)(tabB + 8 * (tid ^ 0x100)) = tw;
  }
  const int e0 = rps[0];
  const int nst = rps[QR] - e0 < kEnt ? rps[QR] - e0 : kEnt;
  for (int e = tid; e < nst; e += kNT) {
    ecol[e] = a.O_col[e0 + e];
    eov[e] = ((const u32x4*)a.O)[e0 + e];
  }

  if (wave >= 8) {
    // ================= producer waves 8 .. 8 + NPW - 1 =================
    const int dw = wave - 8;
    constexpr int kXI = 32 / NPW;   // x DMA instructions per producer per step
    // LDS DMA: wave instruction j of a tile covers rows 8j .. 8j+7; lane l
    // loads the 16 bytes that land at byte 16l of that kilobyte.
    auto issue_x = [&](int s, int st) {
      char* base = smem + L::X0 + st * L::XS;
#pragma unroll
      for (int p = 0; p < kXI; ++p) {
        const int j = NPW * p + dw;
        const int r = 8 * j + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        const int tt = t0 + r < T ? t0 + r : T - 1;
        __builtin_amdgcn_global_load_lds((const void*)(a.x + (size_t)tt * ldx + s * kBK + 8 * c),
                                         (__attribute__((address_space(3))) void*)(base + j * 1024), 16, 0, 0);
      }
    };
    auto issue_i = [&](int s, int st) {
      if (dw < QRp / 8) {
        const int r = 8 * dw + (lane >> 3);
        const int rr = r < QR ? r : QR - 1;   // rows past QR: loaded, never read
        __builtin_amdgcn_global_load_lds((const void*)(a.Q + (size_t)(m0 + rr) * N + s * kBK + 8 * (lane & 7)),
                                         (__attribute__((address_space(3))) void*)(smem + L::I0 + st * L::IS + dw * 1024),
                                         16, 0, 0);
      }
      if (dw == NPW - 1 && lane < 8) {
        __builtin_amdgcn_global_load_lds((const void*)(a.h + s * kBK + 8 * lane),
                                         (__attribute__((address_space(3))) void*)(smem + L::H0 + st * L::HS), 16, 0, 0);
      }
    };
    // Decode units (Q-row, 8-column group, half): 16·QR / NPW per producer wave
    // in NP passes of 64 lanes; lanes past a wave's units repeat one of its units
    // (same LDS addresses, so no extra bank conflicts) and write to a
    // scratch slot.
    constexpr int UPD = 16 * QR / NPW, NP = (UPD + 63) / 64;
    static_assert(UPD * NPW == 16 * QR, "whole units per producer");
    int dq[NP], dg[NP], dh[NP], ec[NP], ee[NP], ncol[NP];
    bool twin[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int l = 64 * p + lane;
      twin[p] = l >= UPD;
      const int u = dw * UPD + (twin[p] ? 64 * p + (lane & 15) : l);
      dq[p] = u >> 4; dh[p] = (u >> 3) & 1; dg[p] = u & 7;
      ec[p] = 0; ee[p] = 0;
      if (!twin[p]) {
        ec[p] = rps[dq[p]] - e0;
        ee[p] = rps[dq[p] + 1] - e0 < kEnt ? rps[dq[p] + 1] - e0 : kEnt;
      }
    }
    // All passes' index/h reads and table lookups first (one dependency chain
    // per wave), then the arithmetic and writes, then the rare critical blocks
    // patched in after the lane's own writes.
    auto decode = [&](int s, int st) {
      u32x2 lo[NP][4], hi[NP][4];
      u32x4 hv[NP];
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const u32x4 qv = *(const u32x4*)(smem + L::I0 + st * L::IS + dq[p] * 128 + 16 * dg[p]);
        hv[p] = *(const u32x4*)(smem + L::H0 + st * L::HS + 16 * dg[p]);
        const mdec::Half half(dh[p]);
        half.lookup(qv, tabB, lo[p], hi[p]);
      }
      char* wb = smem + L::W0 + st * L::WS;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          u32x4 aw = mdec::Half::operand(lo[p], hi[p], c);
#pragma unroll
          for (int d = 0; d < 4; ++d) aw[d] = gpk_mul(aw[d], hv[p][d]);
          const int off = twin[p] ? (2 - st) * L::WS + 16 * lane : g3::wpos(8 * dq[p] + 4 * dh[p] + c, dg[p]);
          *(u32x4*)(wb + off) = aw;
        }
      }
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int klo = s * kBK + 8 * dg[p];
        while (ncol[p] < klo + 8) {
          if (ncol[p] >= klo) {
            const int jc = ncol[p] - klo;
            const f16 hc = *(const f16*)(smem + L::H0 + st * L::HS + 2 * (8 * dg[p] + jc));
            const f16x8 o = __builtin_bit_cast(f16x8, eov[ec[p]]);
#pragma unroll
            for (int c = 0; c < 4; ++c)
              *(f16*)(wb + g3::wpos(8 * dq[p] + 4 * dh[p] + c, dg[p]) + 2 * jc) =
                  (f16)((f16)(o[4 * dh[p] + c] * down) * hc);
          }
          ++ec[p];
          ncol[p] = ec[p] < ee[p] ? ecol[ec[p]] : 0x7fffffff;
        }
      }
    };

    // Stages alternate by step within this workgroup's range: step k0 + j
    // uses stage j & 1.  The entry cursors start at each row's first entry;
    // the first decode walks past the entries left of column 64·k0.
    issue_i(k0, 0);
    if (nkp > 1) issue_i(k0 + 1, 1);
    issue_x(k0, 0);
    __syncthreads();   // table, entries, row pointers
#pragma unroll
    for (int p = 0; p < NP; ++p) ncol[p] = ec[p] < ee[p] ? ecol[ec[p]] : 0x7fffffff;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    decode(k0, 0);
    for (int j = 0; j < nkp; ++j) {
      // Before the barrier: X(k0 + j), indices(k0 + j + 1) landed, W(k0 + j) written.
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (j + 2 < nkp) issue_i(k0 + j + 2, j & 1);
      if (j + 1 < nkp) {
        issue_x(k0 + j + 1, (j + 1) & 1);
        decode(k0 + j + 1, (j + 1) & 1);
      }
    }
    return;
  }

  // ================= MFMA waves 0-7 =================
  const int wf = wave & 1, wt = wave >> 1;
  const int i = lane & 15, kg = lane >> 4;
  f32x4 acc[FA][TB];
#pragma unroll
  for (int x = 0; x < FA; ++x)
#pragma unroll
    for (int q = 0; q < TB; ++q) acc[x][q] = (f32x4){0.f, 0.f, 0.f, 0.f};
  __syncthreads();   // the producers' first barrier
  for (int j = 0; j < nkp; ++j) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const char* xb = smem + L::X0 + (j & 1) * L::XS;
    const char* wb = smem + L::W0 + (j & 1) * L::WS;
    f16x8 af[2][FA], bf[2][TB];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int x = 0; x < FA; ++x) af[ks][x] = *(const f16x8*)(wb + g3::wpos(wf * FW + 16 * x + i, 4 * ks + kg));
#pragma unroll
      for (int q = 0; q < TB; ++q) bf[ks][q] = *(const f16x8*)(xb + g3::xpos(wt * TW + 16 * q + i, 4 * ks + kg));
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int x = 0; x < FA; ++x)
#pragma unroll
        for (int q = 0; q < TB; ++q)
          acc[x][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[ks][x], bf[ks][q], acc[x][q], 0, 0, 0);
  }

  // ---- entries past the LDS stage: the loop used table row 511 at their
  // columns; add (fp16(O·2^-e·h) - fp16(row511·h)) · x per output row ----
  if (rps[QR] - e0 > kEnt) {
    const f16x4 t5 = *(const f16x4*)(tabB + 8 * (511 ^ 0x100));   // scaled by 2^-e
    const int lg = lane >> 4;
    for (int q = 0; q < QR; ++q) {
      const int fl0 = 8 * q - wf * FW;   // the block's first feature in this wave's range
      if (fl0 < 0 || fl0 >= FW) continue;
      const int elo = rps[q] - e0 > kEnt ? rps[q] - e0 : kEnt;
      const int ehi = rps[q + 1] - e0;
      for (int e = elo; e < ehi; ++e) {
        const int col = a.O_col[e0 + e];
        if (col < kBK * k0 || col >= kBK * k1) continue;   // another part's columns
        const f16x8 o = ((const f16x8*)a.O)[e0 + e];
        const f16 hc = __builtin_bit_cast(f16, a.h[col]);
        float dv[4];   // this lane's 4 features 16·(fl0/16) + 4·lg + v
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int k = 4 * lg + v - (fl0 & 15);
          float d = 0.0f;
#pragma unroll
          for (int kk = 0; kk < 8; ++kk)
            if (kk == k) d = (float)(f16)((f16)(o[kk] * down) * hc) - (float)(f16)(t5[kk & 3] * hc);
          dv[v] = d;
        }
#pragma unroll
        for (int x = 0; x < FA; ++x) {
          if (x != (fl0 >> 4)) continue;
#pragma unroll
          for (int q2 = 0; q2 < TB; ++q2) {
            const int tt = t0 + wt * TW + 16 * q2 + i < T ? t0 + wt * TW + 16 * q2 + i : T - 1;
            const float xv = (float)__builtin_bit_cast(f16, a.x[(size_t)tt * ldx + col]);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[x][q2][v] += dv[v] * xv;
          }
        }
      }
    }
  }

  // ---- split K: this part's sums times 2^e, for k_gemm_split_sum ----
  if (part) {
    const size_t F = 8 * (size_t)a.M;
#pragma unroll
    for (int x = 0; x < FA; ++x) {
      const int f = f0 + wf * FW + 16 * x + 4 * kg;
#pragma unroll
      for (int q = 0; q < TB; ++q) {
        const int tt = t0 + wt * TW + 16 * q + i;
        if (tt >= T) continue;
        f32x4 o;
#pragma unroll
        for (int v = 0; v < 4; ++v) o[v] = acc[x][q][v] * out_scale;
        *(f32x4*)(part + ((size_t)pp * T + tt) * F + f) = o;
      }
    }
    return;
  }

  // ---- y = acc·2^e·g + bias: lane (n, lg) holds 4 consecutive features of token n ----
#pragma unroll
  for (int x = 0; x < FA; ++x) {
    const int f = f0 + wf * FW + 16 * x + 4 * kg;
    const f16x4 g4 = *(const f16x4*)(a.g + f);
    f16x4 b4 = {};
    if (a.bias) b4 = *(const f16x4*)(a.bias + f);
#pragma unroll
    for (int q = 0; q < TB; ++q) {
      const int tt = t0 + wt * TW + 16 * q + i;
      if (tt >= T) continue;
      f16x4 o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = (f16)(acc[x][q][v] * out_scale * (float)g4[v] + (float)b4[v]);
      *(f16x4*)(a.y + (size_t)tt * a.ldy + f) = o;
    }
  }
}

// Four outputs of one token: y = acc · sc + bias, rounded to fp16 or (ybf)
// bf16; sc is the token's power-of-two activation scale (1 for fp16 x).
__device__ __forceinline__ void store_out(uint16_t* p, const f32x4& acc, float sc, const f16x4& b4, int ybf) {
  uint32_t w[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float v0 = acc[2 * h] * sc + (float)b4[2 * h], v1 = acc[2 * h + 1] * sc + (float)b4[2 * h + 1];
    const uint32_t lo = ybf ? Act<bf16>::from_f32(v0) : Act<f16>::from_f32(v0);
    const uint32_t hi = ybf ? Act<bf16>::from_f32(v1) : Act<f16>::from_f32(v1);
    w[h] = lo | (hi << 16);
  }
  *(u32x2*)p = (u32x2){w[0], w[1]};
}

// Prefill GEMM over weights already dequantized: y = x·Wᵀ + bias for fp16 W
// (F × N, row-major, F = out_features) and x (T × N).  The tiles and MFMA
// waves of k_gemm_lds_e8d4 (BF features × 256 tokens, 64-column K-steps, NS
// stages, one barrier per step); the producer waves bring both the x tile and
// the W tile in by LDS DMA, W in the swizzled layout the decode writes (the
// swizzle is in the source addresses: LDS DMA writes each lane's 16 bytes at
// 16·lane of the instruction's kilobyte).  With W from k_dequant this is the
// two-pass prefill: every weight decoded once, rather than once per 256-token
// tile as in the fused kernel.  The launcher runs it for 256 × 256 tiles
// only (two stages: three do not fit the LDS), k_gemm_f16w4 below for the
// rest; F is a multiple of BF here, rs and ybf as in k_gemm_f16w4.
template <int BF, int NPW, int NS, int GT = 4>
__global__ __launch_bounds__(64 * (8 + NPW), (8 + NPW) / 4) void k_gemm_f16w(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ x, const f16* __restrict__ bias, int N, int T,
    int ldx, uint16_t* __restrict__ y, int ldy, int OB, int F, const float* __restrict__ rs, int ybf) {
  constexpr int kBK = g3::kBK, kBT = g3::kBT;
  constexpr int XS = kBT * 128, WS = BF * 128, W0 = NS * XS;
  static_assert(NS == 2 || NS == 3, "stages");
  constexpr int FW = BF / 2, FA = FW / 16, TW = kBT / 4, TB = TW / 16;
  static_assert(NPW == 4 || NPW == 8, "producer waves");
  static_assert(FW % 16 == 0 && BF % 8 == 0, "whole MFMA tiles, whole W kilobytes");
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroups are dealt to the 8 XCDs round-robin: give each XCD a run of
  // consecutive tiles (same token tile, neighbouring feature tiles).
  int blk = blockIdx.x;
  const int G = gridDim.x;
  if ((G & 7) == 0) blk = (blk & 7) * (G >> 3) + (blk >> 3);
  // Tiles in bands of GT token tiles, token tile fastest: the 32 consecutive
  // tiles one XCD runs at a time cover GT token tiles x 32/GT feature tiles,
  // so each x and W slice comes from the last-level cache once per XCD and
  // from the XCD's L2 for the rest.
  const int TBn = G / OB;
  const int band = blk / (GT * OB), r = blk - band * GT * OB;
  const int gt = min(GT, TBn - band * GT);
  const int ob = r / gt, tb = band * GT + r % gt;
  const int f0 = ob * BF, t0 = tb * kBT;
  const int nk = N / kBK;

  if (wave >= 8) {
    // ================= producer waves 8 .. 8 + NPW - 1 =================
    const int dw = wave - 8;
    constexpr int kXI = 32 / NPW;
    auto issue_x = [&](int s, int st) {
      char* base = smem + st * XS;
#pragma unroll
      for (int p = 0; p < kXI; ++p) {
        const int j = NPW * p + dw;
        const int r = 8 * j + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        const int tt = t0 + r < T ? t0 + r : T - 1;
        __builtin_amdgcn_global_load_lds((const void*)(x + (size_t)tt * ldx + s * kBK + 8 * c),
                                         (__attribute__((address_space(3))) void*)(base + j * 1024), 16, 0, 0);
      }
    };
    // Kilobyte j of a W stage holds rows 8j .. 8j+7 (row pairs rp = 4j + lane/16);
    // lane l's 16 bytes land at slot l % 16 of its pair's 256 bytes, which
    // g3::wpos gives to chunk c = v/2 of row 2·rp + t, v = slot ^ 2(rp % 8),
    // t = (v & 1) ^ ((rp / 2) & 1).  Every wave issues WI instructions (a
    // wave with fewer kilobytes repeats its last one: the same bytes to the
    // same place), so a wait can count them.
    constexpr int WI = (BF / 8 + NPW - 1) / NPW;
    auto issue_w = [&](int s, int st) {
      char* base = smem + W0 + st * WS;
#pragma unroll
      for (int u = 0; u < WI; ++u) {
        const int j0 = dw + NPW * u, j = j0 < BF / 8 ? j0 : j0 - NPW;
        const int rp = 4 * j + (lane >> 4);
        const int v = (lane & 15) ^ (2 * (rp & 7));
        const int c = v >> 1, r = 2 * rp + ((v & 1) ^ ((rp >> 1) & 1));
        __builtin_amdgcn_global_load_lds((const void*)(W + (size_t)(f0 + r) * N + s * kBK + 8 * c),
                                         (__attribute__((address_space(3))) void*)(base + j * 1024), 16, 0, 0);
      }
    };
    // NS stages: the loads of step j + NS - 1 go out after barrier j, so
    // each step's loads have NS - 1 steps to land.
#pragma unroll
    for (int j = 0; j < NS - 1; ++j) {
      if (j < nk) {
        issue_x(j, j);
        issue_w(j, j);
      }
    }
    for (int j = 0; j < nk; ++j) {
      // Before the barrier: X(j) and W(j) landed (the NS - 2 later steps'
      // loads may still be in flight; every step issues the same count).
      if (NS == 3 && j + 1 < nk) {
        asm volatile("s_waitcnt vmcnt(%0)" :: "n"(kXI + WI) : "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (j + NS - 1 < nk) {
        issue_x(j + NS - 1, (j + NS - 1) % NS);
        issue_w(j + NS - 1, (j + NS - 1) % NS);
      }
    }
    return;
  }

  // ================= MFMA waves 0-7 =================
  const int wf = wave & 1, wt = wave >> 1;
  const int i = lane & 15, kg = lane >> 4;
  f32x4 acc[FA][TB];
#pragma unroll
  for (int xx = 0; xx < FA; ++xx)
#pragma unroll
    for (int q = 0; q < TB; ++q) acc[xx][q] = (f32x4){0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < nk; ++j) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const char* xb = smem + (j % NS) * XS;
    const char* wb = smem + W0 + (j % NS) * WS;
    f16x8 af[2][FA], bf[2][TB];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int xx = 0; xx < FA; ++xx) af[ks][xx] = *(const f16x8*)(wb + g3::wpos(wf * FW + 16 * xx + i, 4 * ks + kg));
#pragma unroll
      for (int q = 0; q < TB; ++q) bf[ks][q] = *(const f16x8*)(xb + g3::xpos(wt * TW + 16 * q + i, 4 * ks + kg));
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int xx = 0; xx < FA; ++xx)
#pragma unroll
        for (int q = 0; q < TB; ++q)
          acc[xx][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[ks][xx], bf[ks][q], acc[xx][q], 0, 0, 0);
  }
  // ---- y = acc + bias: lane (n, lg) holds 4 consecutive features of token n ----
#pragma unroll
  for (int xx = 0; xx < FA; ++xx) {
    const int f = f0 + wf * FW + 16 * xx + 4 * kg;
    f16x4 b4 = {};
    if (bias) b4 = *(const f16x4*)(bias + f);
#pragma unroll
    for (int q = 0; q < TB; ++q) {
      const int tt = t0 + wt * TW + 16 * q + i;
      if (tt >= T) continue;
      store_out(y + (size_t)tt * ldy + f, acc[xx][q], rs ? rs[tt] : 1.0f, b4, ybf);
    }
  }
}

// k_gemm_f16w with BF x BT tiles and four matrix-core waves, one per SIMD,
// each holding a (BF/2) x (BT/2) block of the tile, and their LDS reads a
// half-step ahead of their MFMAs: the reads for the second half of step j
// (k 32..63) go out column by column among the MFMAs of its first half, the
// barrier of step j + 1 sits between the two halves, and the reads of step
// j + 1's first half go out among the MFMAs of step j's second half.  So the
// MFMAs never wait for LDS, and the barrier no longer lines every wave's
// reads up into one burst.  Four producer waves (one per SIMD) bring x and W
// in by LDS DMA, three stages deep.  Eight waves in all: 256 registers per
// wave for up to 160 fp32 accumulators and two sets of fragments.  The last
// feature tile may be ragged (rows past F read row F - 1, stores stop at F);
// the output is rs[t] · acc + bias in fp16 or (ybf) bf16.
template <int BF, int BT, int GT = 4>
__global__ __launch_bounds__(512, 2) void k_gemm_f16w4(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ x, const f16* __restrict__ bias, int N, int T,
    int ldx, uint16_t* __restrict__ y, int ldy, int OB, int F, const float* __restrict__ rs, int ybf) {
  constexpr int kBK = g3::kBK, kBT = BT, NS = 3, NPW = 4;
  constexpr int XS = kBT * 128, WS = BF * 128, W0 = NS * XS;
  constexpr int FW = BF / 2, FA = FW / 16, TW = kBT / 2, TB = TW / 16;
  static_assert(FW % 16 == 0 && TW % 16 == 0 && FA * TB <= 40, "whole MFMA tiles, accumulators fit");
  static_assert(NS * (XS + WS) <= g3::kLds, "three stages fit the LDS");
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int blk = blockIdx.x;
  const int G = gridDim.x;
  if ((G & 7) == 0) blk = (blk & 7) * (G >> 3) + (blk >> 3);
  // Tiles in bands of GT token tiles, token tile fastest (as k_gemm_f16w).
  const int TBn = G / OB;
  const int band = blk / (GT * OB), r = blk - band * GT * OB;
  const int gt = min(GT, TBn - band * GT);
  const int ob = r / gt, tb = band * GT + r % gt;
  const int f0 = ob * BF, t0 = tb * kBT;
  const int nk = N / kBK;

  if (wave >= 4) {
    // ================= producer waves 4 .. 7 =================
    const int dw = wave - 4;
    constexpr int kXI = kBT / 8 / NPW;
    auto issue_x = [&](int s, int st) {
      char* base = smem + st * XS;
#pragma unroll
      for (int p = 0; p < kXI; ++p) {
        const int j = NPW * p + dw;
        const int rr = 8 * j + (lane >> 3);
        const int c = (lane & 7) ^ ((rr >> 1) & 7);
        const int tt = t0 + rr < T ? t0 + rr : T - 1;
        __builtin_amdgcn_global_load_lds((const void*)(x + (size_t)tt * ldx + s * kBK + 8 * c),
                                         (__attribute__((address_space(3))) void*)(base + j * 1024), 16, 0, 0);
      }
    };
    // The W kilobytes as in k_gemm_f16w; every wave issues WI instructions
    // (repeating its last kilobyte where it has fewer) so a wait can count.
    constexpr int WI = (BF / 8 + NPW - 1) / NPW;
    auto issue_w = [&](int s, int st) {
      char* base = smem + W0 + st * WS;
#pragma unroll
      for (int u = 0; u < WI; ++u) {
        const int j0 = dw + NPW * u, j = j0 < BF / 8 ? j0 : j0 - NPW;
        const int rp = 4 * j + (lane >> 4);
        const int v = (lane & 15) ^ (2 * (rp & 7));
        const int c = v >> 1, rr = 2 * rp + ((v & 1) ^ ((rp >> 1) & 1));
        const int fr = f0 + rr < F ? f0 + rr : F - 1;   // a ragged last tile repeats row F - 1
        __builtin_amdgcn_global_load_lds((const void*)(W + (size_t)fr * N + s * kBK + 8 * c),
                                         (__attribute__((address_space(3))) void*)(base + j * 1024), 16, 0, 0);
      }
    };
    // The loads of step j + 2 go out after barrier j, into the stage that
    // step j - 1 used: every MFMA wave finished reading it before barrier j.
    issue_x(0, 0);
    issue_w(0, 0);
    if (nk > 1) {
      issue_x(1, 1);
      issue_w(1, 1);
    }
    for (int j = 0; j < nk; ++j) {
      // Before barrier j: X(j) and W(j) landed (step j + 1's may be in flight).
      if (j + 1 < nk) {
        asm volatile("s_waitcnt vmcnt(%0)" :: "n"(kXI + WI) : "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (j + 2 < nk) {
        issue_x(j + 2, (j + 2) % NS);
        issue_w(j + 2, (j + 2) % NS);
      }
    }
    return;
  }

  // ================= MFMA waves 0-3 =================
  const int wf = wave & 1, wt = wave >> 1;
  const int i = lane & 15, kg = lane >> 4;
  f32x4 acc[FA][TB];
#pragma unroll
  for (int xx = 0; xx < FA; ++xx)
#pragma unroll
    for (int q = 0; q < TB; ++q) acc[xx][q] = (f32x4){0.f, 0.f, 0.f, 0.f};
  f16x8 a0[FA], b0[TB], a1[FA], b1[TB];
  // Rows 16 apart sit 2 KB apart in both layouts (the swizzles depend on
  // the row mod 16 only): one lane offset per half-step, immediates after.
  const int wl0 = W0 + g3::wpos(wf * FW + i, kg), wl1 = W0 + g3::wpos(wf * FW + i, 4 + kg);
  const int xl0 = g3::xpos(wt * TW + i, kg), xl1 = g3::xpos(wt * TW + i, 4 + kg);
  auto rd_a = [&](f16x8& v, int st, int ks, int xx) {
    v = *(const f16x8*)(smem + st * WS + (ks ? wl1 : wl0) + 2048 * xx);
  };
  auto rd_b = [&](f16x8& v, int st, int ks, int q) {
    v = *(const f16x8*)(smem + st * XS + (ks ? xl1 : xl0) + 2048 * q);
  };
  // The MFMAs of one half-step, token column by column; after column q the
  // reads of the next half-step's column q (and A fragment q) go out, so
  // each fragment's registers come free as the next one's load is issued,
  // and the first MFMAs of a half-step wait on no read just issued.  The
  // scheduling barriers keep that order (left alone, the scheduler gathers
  // the reads after most of the MFMAs and then waits on them).
  auto mm_rd = [&](const f16x8* a, const f16x8* b, f16x8* an, f16x8* bn, int st, int ks) {
#pragma unroll
    for (int q = 0; q < TB; ++q) {
#pragma unroll
      for (int xx = 0; xx < FA; ++xx)
        acc[xx][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[xx], b[q], acc[xx][q], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (q < FA) rd_a(an[q], st, ks, q);
      rd_b(bn[q], st, ks, q);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int xx = TB; xx < FA; ++xx) rd_a(an[xx], st, ks, xx);
  };
  __builtin_amdgcn_s_barrier();   // barrier 0: step 0 landed
  asm volatile("" ::: "memory");
#pragma unroll
  for (int xx = 0; xx < FA; ++xx) rd_a(a0[xx], 0, 0, xx);
#pragma unroll
  for (int q = 0; q < TB; ++q) rd_b(b0[q], 0, 0, q);
  // The loop runs from barrier to barrier (the second half of step j, then
  // the first half of step j + 1), so its first MFMAs follow the wait at the
  // barrier and the reads issued just before the back edge are not waited
  // for there.
  mm_rd(a0, b0, a1, b1, 0, 1);
  for (int j = 0; j + 1 < nk; ++j) {
    // Every read of stage j % NS done before barrier j + 1: the producers
    // refill it after that barrier.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    mm_rd(a1, b1, a0, b0, (j + 1) % NS, 0);
    mm_rd(a0, b0, a1, b1, (j + 1) % NS, 1);
  }
#pragma unroll
  for (int q = 0; q < TB; ++q)
#pragma unroll
    for (int xx = 0; xx < FA; ++xx)
      acc[xx][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[xx], b1[q], acc[xx][q], 0, 0, 0);
  // ---- y = acc + bias: lane (n, lg) holds 4 consecutive features of token n ----
#pragma unroll
  for (int xx = 0; xx < FA; ++xx) {
    const int f = f0 + wf * FW + 16 * xx + 4 * kg;
    if (f >= F) continue;   // past a ragged last tile (F is a multiple of 4)
    f16x4 b4 = {};
    if (bias) b4 = *(const f16x4*)(bias + f);
#pragma unroll
    for (int q = 0; q < TB; ++q) {
      const int tt = t0 + wt * TW + 16 * q + i;
      if (tt >= T) continue;
      store_out(y + (size_t)tt * ldy + f, acc[xx][q], rs ? rs[tt] : 1.0f, b4, ybf);
    }
  }
}

// y[t][f] = fp16((Σ_p part[p][t][f]) · g[f] + bias[f]), the parts added in
// order (deterministic); 8 features per thread.
__global__ __launch_bounds__(256) void k_gemm_split_sum(LinearArgs a, int P, const float* __restrict__ part) {
  const size_t F = 8 * (size_t)a.M;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;   // (token, 8-feature chunk)
  const size_t nc = F / 8;
  if (i >= (size_t)a.B * nc) return;
  const size_t t = i / nc, f = (i - t * nc) * 8;
  f32x4 s0 = *(const f32x4*)(part + t * F + f), s1 = *(const f32x4*)(part + t * F + f + 4);
  for (int p = 1; p < P; ++p) {
    const float* q = part + ((size_t)p * a.B + t) * F + f;
    s0 += *(const f32x4*)q;
    s1 += *(const f32x4*)(q + 4);
  }
  const f16x8 g8 = *(const f16x8*)(a.g + f);
  f16x8 b8 = {};
  if (a.bias) b8 = *(const f16x8*)(a.bias + f);
  u16x8 o;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    o[v] = Act<f16>::from_f32(s0[v] * (float)g8[v] + (float)b8[v]);
    o[4 + v] = Act<f16>::from_f32(s1[v] * (float)g8[4 + v] + (float)b8[4 + v]);
  }
  // Two 8-byte stores: y rows are 8-byte aligned (the GEMM's own stores).
  const u32x4 w = __builtin_bit_cast(u32x4, o);
  u32x2* yp = (u32x2*)(a.y + t * a.ldy + f);
  yp[0] = (u32x2){w[0], w[1]};
  yp[1] = (u32x2){w[2], w[3]};
}

template <bool HAS_S>
__global__ __launch_bounds__(kGT, 2) void k_gemm_e8d4(LinearArgs a, int OB) {
  gemm_tile<KIND_E8D4, HAS_S>(a, OB);
}

template <bool HAS_S>
__global__ __launch_bounds__(kGT, 2) void k_gemm_e8(LinearArgs a, int OB) {
  gemm_tile<KIND_E8, HAS_S>(a, OB);
}

namespace {
constexpr size_t kLdsBytes = 160 * 1024;

// Static LDS of a kernel (0 if the runtime cannot say, which the launch's
// own check then catches).
size_t static_lds(const void* kern) {
  hipFuncAttributes fa;
  return hipFuncGetAttributes(&fa, kern) == hipSuccess ? fa.sharedSizeBytes : 0;
}
}  // namespace

template <int KIND>
int launch_gemm(const LinearArgs& a, hipStream_t s, void* work, long long work_bytes) {
  if (KIND == KIND_E8D4 && a.B <= kSliceMaxTokens && a.prep == 0) {
    // Eligibility does not depend on the slice (B = 1..16 all qualify), so a
    // first slice that launches means every slice does.
    int rc = 0;
    for (int b0 = 0; b0 < a.B && rc == 0; b0 += kMatvecMaxBatch) {
      LinearArgs t = a;
      t.B = a.B - b0 < kMatvecMaxBatch ? a.B - b0 : kMatvecMaxBatch;
      t.x = a.x + (size_t)b0 * a.ldx;
      t.y = a.y + (size_t)b0 * a.ldy;
      rc = launch_decode_mfma_multi(&t, 1, s);
    }
    if (rc == 0) return 0;
  }
  // LDS-decode kernel: fp16 x and table, no S_group, K-steps of 64, whole
  // 8-, 16-, 20- or 32-Q-row tiles, 16-byte x rows and 8-byte y stores.  Of the two
  // tile widths, the one with less work per CU (rounds of the CUs × tile
  // width) wins; on a tie the wider tile.
  if (KIND == KIND_E8D4 && !a.x_bf16 && !a.codes_f32 && !a.S && a.prep == 0 && (a.N % g3::kBK) == 0 &&
      (a.ldx % 8) == 0 && ((uintptr_t)a.x & 15) == 0 && (a.ldy % 4) == 0 && ((uintptr_t)a.y & 7) == 0) {
    const long TB = (a.B + g3::kBT - 1) / g3::kBT;
    const long cus = dec::cu_count();
    long cost160 = -1, cost256 = -1;
    if (a.M % 20 == 0) cost160 = ((a.M / 20) * TB + cus - 1) / cus * 160;
    if (a.M % 32 == 0) cost256 = ((a.M / 32) * TB + cus - 1) / cus * 256;
    int bf = cost160 < 0 ? (cost256 < 0 ? 0 : 256) : (cost256 < 0 || cost160 < cost256 ? 160 : 256);
    // 128-feature tiles in place of 256: twice the workgroups, each ~0.8 of
    // the time (its producers decode in one pass), so they win when
    // 0.8 x their rounds of the CUs is below the 256 tiles' rounds.
    if (bf != 160 && a.M % 16 == 0) {
      const long r128 = ((a.M / 16) * TB + cus - 1) / cus, r256 = ((a.M / 32) * TB + cus - 1) / cus;
      if (bf == 0 || 4 * r128 < 5 * r256) bf = 128;
      // 64-feature tiles when they still fit one round of the CUs: a launch
      // with few token tiles is bound by each workgroup's serial K-steps,
      // and narrower tiles shorten each step.
      if (bf == 128 && (long)(a.M / 8) * TB <= cus) bf = 64;
    }
    // With a workspace the tile width and the K split are chosen together:
    // time ~ rounds of the CUs x K-steps per part x a tile's step time
    // (measured ~1.09 / 1.33 / 1.66 / 1.66 us for 64 / 128 / 160 / 256
    // features on 4096-5120-column layers), plus the parts' fp32 sums
    // written and read once at ~4 TB/s and the summing launch (~3 us).
    int P = 1;
    const size_t woff = (size_t)decode_mfma_work_bytes();
    const size_t wavail = work && work_bytes > (long long)woff ? (size_t)work_bytes - woff : 0;
    if (bf && wavail) {
      const int nk = a.N / g3::kBK;
      const double per = (double)a.B * 8 * a.M * 4;
      const int widths[4] = {64, 128, 160, 256};
      const double step[4] = {1.09, 1.33, 1.66, 1.66};
      double best = -1;
      int bw = bf, bp = 1;
      for (int wi = 0; wi < 4; ++wi) {
        const int w = widths[wi];
        if (a.M % (w / 8) != 0) continue;
        const long gw = (a.M / (w / 8)) * TB;
        for (int pp = 1; pp <= kPrefillMaxParts; ++pp) {
          if (pp > 1 && (gw * pp > cus || nk / pp < 8 || (size_t)(pp * per) > wavail)) break;
          const double t = (double)((gw * pp + cus - 1) / cus) * ((nk + pp - 1) / pp) * step[wi] +
                           (pp > 1 ? 2.0 * pp * per / 4.0e6 + 3.0 : 0.0);
          if (best < 0 || t < best) {
            best = t;
            bw = w;
            bp = pp;
          }
        }
      }
      // An unsplit choice keeps the measured width rule above.
      if (bp > 1) {
        bf = bw;
        P = bp;
      }
    }
    const long grid = bf ? (a.M / (bf / 8)) * TB : 0;
    if (bf && grid <= 0x7fffffff) {
      // 160-feature tiles: 8 producer waves (the MFMA waves fit four waves per
      // SIMD); 256-feature tiles: 4.
      const int v = bf == 256 ? 0 : bf == 160 ? 1 : bf == 128 ? 2 : 3;
      const void* kerns[4] = {(const void*)k_gemm_lds_e8d4<256, 4>, (const void*)k_gemm_lds_e8d4<160, 8>,
                              (const void*)k_gemm_lds_e8d4<128, 8>, (const void*)k_gemm_lds_e8d4<64, 8>};
      const int bytes[4] = {g3::Lay<256>::Bytes, g3::Lay<160>::Bytes, g3::Lay<128>::Bytes, g3::Lay<64>::Bytes};
      static bool attr[4] = {false, false, false, false};
      if (!attr[v]) attr[v] = hipFuncSetAttribute(kerns[v], hipFuncAttributeMaxDynamicSharedMemorySize, bytes[v]) == hipSuccess;
      if (attr[v]) {
        const int OB = a.M / (bf / 8);
        float* part = P > 1 ? (float*)((char*)work + woff) : nullptr;
        const unsigned g = (unsigned)(grid * P);
        if (v == 0) k_gemm_lds_e8d4<256, 4><<<g, 768, bytes[0], s>>>(a, OB, P, part);
        else if (v == 1) k_gemm_lds_e8d4<160, 8><<<g, 1024, bytes[1], s>>>(a, OB, P, part);
        else if (v == 2) k_gemm_lds_e8d4<128, 8><<<g, 1024, bytes[2], s>>>(a, OB, P, part);
        else k_gemm_lds_e8d4<64, 8><<<g, 1024, bytes[3], s>>>(a, OB, P, part);
        if (part) {
          const size_t chunks = (size_t)a.B * a.M;   // 8-feature chunks
          k_gemm_split_sum<<<(unsigned)((chunks + 255) / 256), 256, 0, s>>>(a, P, part);
        }
        return 0;
      }
    }
  }
  // MFMA path: fp16 activations, fp16 table, whole 16-Q-row tiles, K-steps
  // of 32.  Anything else takes batch tiles of the decode matvec.
  const bool mfma_ok = !a.x_bf16 && !a.codes_f32 && (a.N % kBK) == 0 && (a.M % kBQ) == 0 &&
                       (!a.S || (a.qb % 8) == 0);
  // Rows-in-registers kernel: no S_group, whole 32-Q-row workgroups, y
  // stored 16 bytes at a time; fp16 or bf16 activations.
  const bool rows_ok = KIND == KIND_E8D4 && !a.codes_f32 && !a.S && a.prep == 0 && (a.N % kBK) == 0 &&
                       (a.M % 32) == 0 && (a.ldy % 8) == 0 && ((uintptr_t)a.y & 15) == 0 && (a.ldx % 8) == 0;
  if (rows_ok) {
    const int TB = (a.B + g2::kTok - 1) / g2::kTok;
    const size_t dyn = g2::dyn_bytes(a.N);
    // Five-wave workgroups (one per CU) when they cover the layer in one
    // round of the device's CUs; else four-wave workgroups, two per CU.
    const void* kerns[4] = {(const void*)k_gemm_rows_e8d4<4, false>, (const void*)k_gemm_rows_e8d4<5, false>,
                            (const void*)k_gemm_rows_e8d4<4, true>, (const void*)k_gemm_rows_e8d4<5, true>};
    // A variant fits when its static LDS plus the activation rows stay
    // within the CU's 160 KB.
    static const size_t st[4] = {static_lds(kerns[0]), static_lds(kerns[1]), static_lds(kerns[2]),
                                 static_lds(kerns[3])};
    auto fits = [&](int v) { return dyn <= 96 * 1024 && st[v] + dyn <= kLdsBytes; };
    bool five = (a.M % 40) == 0 && (long)(a.M / 40) * TB <= dec::cu_count() && fits(1 | (a.x_bf16 ? 2 : 0));
    const int OB = five ? a.M / 40 : a.M / 32;
    const long grid = (long)OB * TB;
    if (grid <= 0x7fffffff && fits((five ? 1 : 0) | (a.x_bf16 ? 2 : 0))) {
      const int v = (five ? 1 : 0) | (a.x_bf16 ? 2 : 0);
      static size_t attr[4] = {0, 0, 0, 0};
      bool ok = true;
      if (dyn > attr[v]) {
        ok = hipFuncSetAttribute(kerns[v], hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn) == hipSuccess;
        if (ok) attr[v] = dyn;
      }
      if (ok) {
        switch (v) {
          case 0: k_gemm_rows_e8d4<4, false><<<(unsigned)grid, 256, dyn, s>>>(a, OB); break;
          case 1: k_gemm_rows_e8d4<5, false><<<(unsigned)grid, 320, dyn, s>>>(a, OB); break;
          case 2: k_gemm_rows_e8d4<4, true><<<(unsigned)grid, 256, dyn, s>>>(a, OB); break;
          default: k_gemm_rows_e8d4<5, true><<<(unsigned)grid, 320, dyn, s>>>(a, OB); break;
        }
        return 0;
      }
    }
  }
  if (mfma_ok) {
    const int OB = a.M / kBQ;
    const int TB = (a.B + kBN - 1) / kBN;
    const long grid = (long)OB * TB;
    if (grid <= 0x7fffffff) {
      if (KIND == KIND_E8D4) {
        if (a.S) k_gemm_e8d4<true><<<(unsigned)grid, kGT, 0, s>>>(a, OB);
        else k_gemm_e8d4<false><<<(unsigned)grid, kGT, 0, s>>>(a, OB);
      } else {
        if (a.S) k_gemm_e8<true><<<(unsigned)grid, kGT, 0, s>>>(a, OB);
        else k_gemm_e8<false><<<(unsigned)grid, kGT, 0, s>>>(a, OB);
      }
      return 0;
    }
  }
  for (int b0 = 0; b0 < a.B; b0 += kMatvecMaxBatch) {
    LinearArgs t = a;
    t.B = a.B - b0 < kMatvecMaxBatch ? a.B - b0 : kMatvecMaxBatch;
    t.x = a.x + (size_t)b0 * a.N;
    t.y = a.y + (size_t)b0 * a.ldy;
    const int rc = launch_matvec<KIND>(t, s);
    if (rc) return rc;
  }
  return 0;
}

// Returns 0 if launched, -1 if the shape is outside k_gemm_f16w: F a
// multiple of 64, N of 64, x rows 16-byte aligned, y rows 8-byte aligned.
int launch_gemm_f16w(const uint16_t* W, const uint16_t* x, const f16* bias, int F, int N, int T, int ldx,
                     uint16_t* y, int ldy, hipStream_t s, const float* rs, int ybf) {
  if (T <= 0 || F % 64 != 0 || N % g3::kBK != 0 || ldx % 8 != 0 || ((uintptr_t)x & 15) != 0 || ldy % 4 != 0 ||
      ((uintptr_t)y & 7) != 0 || ((uintptr_t)W & 15) != 0 || (bias && ((uintptr_t)bias & 7) != 0))
    return -1;
  // Tile: the one with the least time, rounds of the CUs x one tile's
  // K-step time (measured 1.08 / 1.64 / 0.88 / 0.65 us at 64 columns for
  // 160 / 256 / 128 / 64 features x 256 tokens: per unit of area the
  // narrowest is ~1.5x the others), the earlier one on ties.  The
  // three-stage kernel takes a ragged last feature tile (F a multiple of
  // 64, not of the tile), the two-stage 256 x 256 one whole tiles only.  (A
  // 288 x 128 tile, three whole rounds for 13824 features at 2048 tokens,
  // measured slower than 256 x 256 with its second round partly idle.)
  struct Tile { int bf, bt, step; bool ragged; };
  constexpr Tile tiles[4] = {{160, 256, 108, true}, {256, 256, 164, false}, {128, 256, 88, true}, {64, 256, 65, true}};
  const long cus = dec::cu_count();
  int k = -1;
  long best = -1;
  for (int c = 0; c < 4; ++c) {
    if (F % tiles[c].bf != 0 && !tiles[c].ragged) continue;
    const long n = (long)((F + tiles[c].bf - 1) / tiles[c].bf) * ((T + tiles[c].bt - 1) / tiles[c].bt);
    const long cost = (n + cus - 1) / cus * tiles[c].step;
    if (k < 0 || cost < best) {
      best = cost;
      k = c;
    }
  }
  const int OB = (F + tiles[k].bf - 1) / tiles[k].bf;
  const long grid = (long)OB * ((T + tiles[k].bt - 1) / tiles[k].bt);
  if (grid > 0x7fffffff) return -1;
  auto run = [&](auto kern, int threads, int bytes, int v) {
    static bool attr[4] = {false, false, false, false};
    if (!attr[v]) attr[v] = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) == hipSuccess;
    if (!attr[v]) return -1;
    kern<<<(unsigned)grid, threads, bytes, s>>>(W, x, bias, N, T, ldx, y, ldy, OB, F, rs, ybf);
    return 0;
  };
  // Three stages where they fit the CU's 160 KB of LDS (all but 256 x 256).
  // The 256 x 256 tile runs the two-stage kernel with 8-token-tile bands
  // (measured 4% faster than 4 at 13824 features).
  switch (k) {
    case 0: return run(k_gemm_f16w4<160, 256>, 512, 3 * (256 + 160) * 128, 0);
    case 1: return run(k_gemm_f16w<256, 4, 2, 8>, 768, 2 * (256 + 256) * 128, 1);
    case 2: return run(k_gemm_f16w4<128, 256>, 512, 3 * (256 + 128) * 128, 2);
    default: return run(k_gemm_f16w4<64, 256>, 512, 3 * (256 + 64) * 128, 3);
  }
}

// bf16 activations for the W-streaming GEMM: row t of x becomes
// x16[t] = fp16(x[t] · 2^-e_t) with e_t = floor(log2 max_n |x[t][n]|) - 14,
// so the row's largest magnitude lands in [2^14, 2^15): exact for every
// element that stays in fp16's normal range (bf16 carries 8 significand
// bits, fp16 11), i.e. all but those below 2^-28 of the row's maximum.
// rs[t] = 2^e_t restores the scale at the GEMM's output.  One 256-thread
// workgroup per row, the row in registers (N <= 256 · 8 · kRowChunks).
constexpr int kRowChunks = 8;
__global__ __launch_bounds__(256) void k_bf16_rows_to_f16(const uint16_t* __restrict__ x, int N,
                                                          uint16_t* __restrict__ x16, float* __restrict__ rs) {
  __shared__ float wm[4];
  const int t = blockIdx.x, tid = threadIdx.x;
  const int nch = N / 8;
  const uint16_t* xr = x + (size_t)t * N;
  u32x4 v[kRowChunks];
  float mx = 0.0f;
#pragma unroll
  for (int k = 0; k < kRowChunks; ++k) {
    const int c = tid + 256 * k;
    v[k] = c < nch ? *(const u32x4*)(xr + 8 * c) : (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      mx = fmaxf(mx, fabsf(__builtin_bit_cast(float, v[k][d] << 16)));
      mx = fmaxf(mx, fabsf(__builtin_bit_cast(float, v[k][d] & 0xffff0000u)));
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if ((tid & 63) == 0) wm[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
  // floor(log2 mx) from the exponent bits (mx is a bf16 value widened, so
  // normal or zero; a subnormal or zero row keeps e = -100, harmless).
  int e = (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xff) - 127 - 14;
  if (mx == 0.0f || e < -100) e = -100;
  if (mx != mx || e > 100) e = 100;   // inf / NaN rows: their non-finite values stay non-finite
  const float down = __builtin_ldexpf(1.0f, -e);
  uint16_t* orow = x16 + (size_t)t * N;
#pragma unroll
  for (int k = 0; k < kRowChunks; ++k) {
    const int c = tid + 256 * k;
    if (c >= nch) continue;
    u32x4 w;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float a = __builtin_bit_cast(float, v[k][d] << 16) * down;
      const float b = __builtin_bit_cast(float, v[k][d] & 0xffff0000u) * down;
      w[d] = __builtin_bit_cast(uint32_t, (f16x2){(f16)a, (f16)b});
    }
    *(u32x4*)(orow + 8 * c) = w;
  }
  if (tid == 0) rs[t] = __builtin_ldexpf(1.0f, e);
}

// Returns 0 if launched, -1 outside the kernel's range (N a multiple of 8 up
// to 16384, 16-byte aligned rows).
int launch_bf16_rows_to_f16(const uint16_t* x, int N, int T, uint16_t* x16, float* rs, hipStream_t s) {
  if (T <= 0 || N <= 0 || N % 8 != 0 || N > 256 * 8 * kRowChunks || ((uintptr_t)x & 15) != 0 ||
      ((uintptr_t)x16 & 15) != 0 || ((uintptr_t)rs & 3) != 0)
    return -1;
  k_bf16_rows_to_f16<<<(unsigned)T, 256, 0, s>>>(x, N, x16, rs);
  return 0;
}

template int launch_gemm<KIND_E8D4>(const LinearArgs&, hipStream_t, void*, long long);
template int launch_gemm<KIND_E8>(const LinearArgs&, hipStream_t, void*, long long);

}  // namespace eptq

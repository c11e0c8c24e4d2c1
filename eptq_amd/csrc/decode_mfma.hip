// E8-D4 decode matvec for batches of 1..16 on the matrix cores.
//
// Same result as the reference decode kernels (csrc/eptq_kernels.cu:161-292,
// kernels/triton_e8d4.py:47-157): y = g ⊙ (decode(Q)·(h ⊙ S ⊙ x)ᵀ + CSR(O)) + bias,
// here for the batches where the vector kernel (decode_layer.h) would spend
// one dot-product per batch row and weight: the contraction runs on
// v_mfma_f32_16x16x32_f16 with the batch as the MFMA's 16 columns.
//
// Tiles.  A workgroup owns one tile of 8 block rows (64 output rows) of one
// layer and all N columns; S "column" waves split the columns in blocks of 64
// and one more wave stages the tile's critical blocks.  The S partial sums
// meet in LDS at the end, where the critical-block corrections, g, bias and
// the activation scale are applied and y is written.
//
// MFMA operands.  D(16 x 16) += A(16 x 32)·B(32 x 16) with lane l holding
// A[l%16][8(l/16) .. +7], B[8(l/16) .. +7][l%16] and D[4(l/16) .. +3][l%16]:
//   * B = x·h: lane (b = l%16, kg = l/16) holds the activation of batch row b
//     at the 8 columns of its K group (one 16-byte load per column half of a
//     block);
//   * A = weights: lane (i = l%16, kg) decodes the 8 indices of block row
//     i/2 at those same 8 columns through the LDS table, half i%2 of each
//     vector (rows 0-3 or 4-7 of the block).  Each table lookup gives 4 rows
//     of one column; 4 MFMAs per 32 columns take row c (c = 0..3) of the
//     lane's half, so the operand of MFMA c is a byte-permute of the lookups
//     and no lane exchanges data with another.
//   D of MFMA c: lane (b, lg = l/16), element v = output row 16·lg + 4v + c of
//   the tile for batch row b.
//
// Activation scaling is the vector kernel's for B >= 2: h is scaled by a
// workgroup-uniform power of two 2^-e with max|h|·2^-e <= 1, so the fp16
// operand |x·h·2^-e| <= |x| cannot overflow; MFMA products of fp16 operands
// are exact in the fp32 accumulators and 2^e is restored at the output.
//
// Critical blocks (v = 32767) decode as table row 511 in both halves; the
// staging wave loads the tile's CSR entries (column, O, and x·h at that
// column for each batch row) into LDS while the column waves run, and the
// output stage adds O·(x h) minus what the marker contributed.

#include <type_traits>

#include "mfma_decode.h"

namespace eptq {
namespace dmf {

using dec::gp;
using dec::h2;
using dec::kNonTemporal;
using dec::pk_mul;
using mdec::as_f16;
using mdec::bits;
using mdec::ld16;
using mdec::ld2;
using mdec::rsrc;

constexpr int kTile = 8;        // block rows per tile (64 output rows)
constexpr int kBlk = 64;        // columns per block: 4 K groups x 16
constexpr int kDepth = 6;       // blocks of indices and activations in flight per lane (long waves)
constexpr int kFar = 0x40000000;  // a buffer offset past every operand (a load there reads zeros)
constexpr int kEntCap = 256;    // critical blocks of a tile prefetched before the column loop
constexpr int kRedLd = 68;      // floats per batch row of a wave's partial sums
constexpr int kS = 8;           // column waves per workgroup (one workgroup per CU)


// Split-K workspace: per-tile arrival counters, then the fp32 partial sums
// [split tile][part][16][64] of the tiles whose columns are split over P
// workgroups.
constexpr int kMaxCounters = kSplitCounters;
constexpr size_t kCntBytes = kSplitCounterBytes;
constexpr size_t kPartBytes = kSplitPartBytes;
static_assert(kTile * 8 == kSplitTileRows, "one counter per tile");
constexpr int kMaxParts = 4;

__device__ __forceinline__ void st_pair(float* p, float a, float b) {
  const uint64_t v = (uint64_t)__builtin_bit_cast(uint32_t, a) | ((uint64_t)__builtin_bit_cast(uint32_t, b) << 32);
  __hip_atomic_store((uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 ld_pair(const float* p) {
  const uint64_t v = __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__builtin_bit_cast(float, (uint32_t)v), __builtin_bit_cast(float, (uint32_t)(v >> 32)));
}

// Columns rounded up to whole blocks: the activation-scale rows in LDS are
// zero past N, so the last block's extra columns contribute nothing.
__host__ __device__ inline int padded_cols(int N) { return (N + kBlk - 1) / kBlk * kBlk; }

// Dynamic LDS: hs[Np] = fp16(h·2^-e) and, with S_group, hss[Np] = fp16(hs·S)
// during the column loop; the partial sums red[S][16][kRedLd] afterwards.
__host__ __device__ inline size_t dyn_bytes(int N, bool has_s, int S) {
  const size_t act = (size_t)padded_cols(N) * 2 * (has_s ? 2 : 1);
  const size_t red = (size_t)S * 16 * kRedLd * 4;
  return act > red ? act : red;
}

template <int S, bool HAS_S, typename XT, bool XH, bool NORM>
// At most 168 VGPRs (3 waves per SIMD): one 9-wave workgroup per CU.
// XT: activation and output type (bf16 x is taken to fp16 exactly in fp16's
// normal range before the scale; y is rounded from the fp32 sums to XT).
// XH (B <= 8): each lane loads half of its batch row pair's activations (see
// the column waves' loads below).
// NORM (prep 1, fp16 x, B <= 8, N a multiple of 64): the input is
// RMSNorm(x) = nw ⊙ x / rms(x).  The column scale becomes fp16(h·nw) (before
// the power of two), the column waves add up x² over the activations they
// load, and each batch row's sums are multiplied by 1/rms at the output (a
// split tile's parts leave their x² sums with their partial sums).
// a.res (fp16 x): y = fp16(res + fp16(out)).
// Work split: tiles [0, T1) take one workgroup each; the tiles from T1 on
// have their columns split over P workgroups (T1 = 0: every tile).  ma.start
// counts tiles.
__global__ __launch_bounds__((S + 1) * 64, 3) void k_decode_mfma(MultiArgs ma, int P, int T1, int* wcnt,
                                                                 float* wpart) {
  constexpr int NT = (S + 1) * 64;
  __shared__ f16x4 tab[512];
  // The tile's critical blocks as the output stage reads them: O, and the
  // activation operand at the block's column, fp16(x·hs) (xo) and
  // fp16(x·hsa) (xm: what the main loop multiplied the marker's row by).
  __shared__ __attribute__((aligned(16))) u32x4 eov[kEntCap];
  __shared__ __attribute__((aligned(16))) uint16_t exo[kEntCap][16];
  __shared__ __attribute__((aligned(16))) uint16_t exm[HAS_S ? kEntCap : 1][16];
  __shared__ int erow[kTile + 1];   // entry index (from the tile's first) where each block row starts
  __shared__ int ebase;             // the tile's first entry
  __shared__ float wmax[S + 1];
  __shared__ float wss[NORM ? S : 1][8];   // NORM: per column wave, Σx² per batch row
  __shared__ float sinv[8];                // NORM: 1/rms per batch row
  extern __shared__ __attribute__((aligned(16))) char dyn[];

  // This workgroup's tile (index among all tiles of the launch) and part:
  // part p of Pt takes the p-th Pt-th of the tile's column blocks.
  const int g = (int)blockIdx.x;
  const int Pt = g < T1 ? 1 : P;
  const int tile_g = g < T1 ? g : T1 + (g - T1) / P;
  const int part = g < T1 ? 0 : (g - T1) - (tile_g - T1) * P;
  int li = 0;
#pragma unroll
  for (int l = 1; l < kMaxLayers; ++l)
    if (l < ma.n && tile_g >= ma.start[l]) li = l;
  const LinearArgs a = li == 0 ? ma.l[0] : li == 1 ? ma.l[1] : li == 2 ? ma.l[2] : ma.l[3];
  const int tile = tile_g - ma.start[li];         // within layer li

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = a.M, N = a.N, B = a.B, ldx = a.ldx;
  const int Np = padded_cols(N), nchp = Np >> 3;
  const int m0 = tile * kTile;
  const int grp = HAS_S ? (8 * m0) / a.qb : 0;
  uint16_t* __restrict__ hs = (uint16_t*)dyn;
  uint16_t* __restrict__ hss = hs + Np;
  float (*red)[16][kRedLd] = (float (*)[16][kRedLd])dyn;

  const __amdgpu_buffer_rsrc_t rh = rsrc(a.h, N * 2);
  const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, ((B - 1) * ldx + N) * 2);
  const __amdgpu_buffer_rsrc_t rs = rsrc(HAS_S ? a.S + (size_t)grp * N : nullptr, HAS_S ? N * 2 : 0);
  const __amdgpu_buffer_rsrc_t rnw = rsrc(NORM ? a.nw : nullptr, NORM ? N * 2 : 0);

  // Table, h and the S row first (the column waves' ring follows them into
  // LDS).  Loads skipped on some path are left undefined there (never merged with
  // a constant: the compiler would wait for every load in flight at such a
  // merge, before the ring is issued) and used only under the same
  // condition.  Only waves with a chunk below nchp load h: every load
  // instruction costs address-unit time, in range or not.
  f16x4 tload;
  if (tid < 512) tload = *gp((const f16x4*)a.codes + tid);
  u32x4 hw[4], sw[4], ww[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = tid + NT * k;
    if (NT * k + 64 * wave < nchp) {             // wave-uniform
      hw[k] = ld16(rh, c * 16);                  // zero past N
      if (HAS_S) sw[k] = ld16(rs, c * 16);
      if (NORM) ww[k] = ld16(rnw, c * 16);
    }
  }
  // g and bias of this thread's two outputs (thread t < 512: rows 2(t%32), +1
  // of the tile), read long before the output stage needs them.
  const int orow = 8 * m0 + (tid & 31) * 2;
  const int oi = orow < 8 * M ? orow : 0;
  const uint32_t gpair = *gp((const uint32_t*)(a.g + oi));
  const __amdgpu_buffer_rsrc_t rbias = rsrc(a.bias, a.bias ? 16 * M : 0);
  const uint32_t bpair = __builtin_amdgcn_raw_buffer_load_b32(rbias, oi * 2, 0, 0);
  // The residual of this thread's output pair (batch row tid / 32; zeros when
  // absent or past the batch).
  static_assert(NT >= 512, "one output pair per thread");
  const __amdgpu_buffer_rsrc_t rres = rsrc(a.res, a.res ? B * a.ldy * 2 : 0);
  const uint32_t rpair = __builtin_amdgcn_raw_buffer_load_b32(rres, (((tid >> 5) & 15) * a.ldy + orow) * 2, 0, 0);

  // Column waves: blocks [blo, bhi) of the tile's rows, the first kDepth of
  // them in flight.  Lane (i, kg) reads the 16 indices of block row m0 + i/2
  // at columns 64·blk + 16·kg .. +15; lane (b, kg) the activations of batch
  // row b at the same columns (rows past M and batch rows past B read zeros).
  const int nb = Np / kBlk;
  const int plo = part * nb / Pt, pnb = (part + 1) * nb / Pt - plo;
  const int blo = plo + wave * pnb / S, bhi = plo + (wave + 1) * pnb / S;
  const int i = lane & 15, kg = lane >> 4;
  const int qrow = m0 + (i >> 1);
  const __amdgpu_buffer_rsrc_t rq = rsrc(a.Q, M * N * 2);
  // Address-unit economy (every 16-byte load instruction costs the CU's
  // address unit the same time, whatever it reads): the two lanes of a block
  // row (i, i ^ 1) each load half of the row's 16 indices and take the other
  // half from their partner (DPP); with XH, lane (b, kg) loads half of batch
  // row b & 7's 16 activations (columns 8·(b >> 3) ..) and lane b < 8 takes
  // the other half from lane b ^ 8 (lanes b >= 8 then hold values of no
  // batch row: their MFMA columns are never read).
  int qo = qrow < M ? (qrow * N + blo * kBlk + 16 * kg + 8 * (i & 1)) * 2 : 0x40000000;
  int xo = XH ? ((lane & 7) * ldx + blo * kBlk + 16 * kg + 8 * ((lane >> 3) & 1)) * 2
              : ((lane & 15) * ldx + blo * kBlk + 16 * kg) * 2;
  constexpr int XL = XH ? 1 : 2;   // activation loads per block
  constexpr int kShort = 8;        // most blocks per wave loaded at once
  // The tile's CSR row pointers (part 0 applies the critical blocks; the
  // other parts see an empty range), for the staging wave (the compiler
  // moves the load into that wave's path).
  const __amdgpu_buffer_rsrc_t rp = rsrc(a.O_row_ptr, (M + 1) * 4);
  const int rrow = m0 + (part == 0 && lane <= kTile ? lane : part == 0 ? kTile : 0);
  const int rpv = (int)__builtin_amdgcn_raw_buffer_load_b32(rp, (rrow < M ? rrow : M) * 4, 0, 0);

  // h (times nw with NORM; and the S row) into LDS as loaded; max|h|.
  float mx = 0.0f;
  auto put = [&](int c, u32x4 h, const u32x4 sv, const u32x4 wv) {
    if (c < nchp) {
      if (NORM) {
#pragma unroll
        for (int d = 0; d < 4; ++d) h[d] = pk_mul(h[d], wv[d]);
      }
      *(u32x4*)(hs + c * 8) = h;
      if (HAS_S) *(u32x4*)(hss + c * 8) = sv;
      const f16x8 hv = __builtin_bit_cast(f16x8, h);
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf((float)hv[e]));
    }
  };
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (NT * k + 64 * wave < nchp) put(tid + NT * k, hw[k], HAS_S ? sw[k] : hw[k], NORM ? ww[k] : hw[k]);
  for (int c = tid + 4 * NT; c < nchp; c += NT)
    put(c, ld16(rh, c * 16), HAS_S ? ld16(rs, c * 16) : u32x4{}, NORM ? ld16(rnw, c * 16) : u32x4{});
  mx = fmaxf(mx, partner<1>(mx));
  mx = fmaxf(mx, partner<2>(mx));
  mx = fmaxf(mx, partner<4>(mx));
  mx = fmaxf(mx, partner<8>(mx));
  mx = fmaxf(mx, partner<16>(mx));
  mx = fmaxf(mx, partner<32>(mx));
  if (lane == 0) wmax[wave] = mx;
  if (tid < 512) tab[tid ^ 0x100] = tload;
  const char* __restrict__ tabB = (const char*)tab;
  const uint16_t* __restrict__ hsa = HAS_S ? hss : hs;   // the scale row of the main loop

  // The two barriers around the scaling, run by every wave on its own path
  // (a load issued before them and used after must not cross a merge of
  // paths that issued different numbers of loads: the compiler would then
  // wait for every load in flight).  Workgroup scale 2^-e with
  // max|h|·2^-e <= 1; hs = fp16(h·2^-e), hss = fp16(hs·S).
  float out_scale = 1.0f;
  f16 down = (f16)1.0f;
  auto scale = [&]() {
    __syncthreads();
    float m = wmax[0];
#pragma unroll
    for (int w = 1; w <= S; ++w) m = fmaxf(m, wmax[w]);
    int ex = 0;
    if (m > 1.0f) ex = (int)((__builtin_bit_cast(uint32_t, m) >> 23) & 0xff) - 126;   // 2^ex >= m
    out_scale = __builtin_ldexpf(1.0f, ex);
    down = (f16)__builtin_ldexpf(1.0f, -ex);
    const uint32_t down2 = __builtin_bit_cast(uint32_t, (h2){down, down});
    for (int c = tid; c < nchp; c += NT) {
      u32x4 h = *(const u32x4*)(hs + c * 8);
#pragma unroll
      for (int d = 0; d < 4; ++d) h[d] = pk_mul(h[d], down2);
      *(u32x4*)(hs + c * 8) = h;
      if (HAS_S) {
        u32x4 sv = *(const u32x4*)(hss + c * 8);
#pragma unroll
        for (int d = 0; d < 4; ++d) sv[d] = pk_mul(h[d], sv[d]);
        *(u32x4*)(hss + c * 8) = sv;
      }
    }
    __syncthreads();
  };

  f32x4 acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  float ssq = 0.0f;   // NORM: Σx² of this lane's activations (batch row lane & 7)
  const mdec::Half half(i);

    auto block = [&](const u32x4 qh, const u32x4 (&xh)[XL], int blk) {
      // The 16 indices of the lane's block row (columns 16·kg ..): q[0] from
      // the even lane of the pair, q[1] from the odd one (DPP quad_perm
      // [0,0,2,2] and [1,1,3,3]); the activations likewise (row_ror:8).
      u32x4 q[2], x[2];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        q[0][d] = (uint32_t)__builtin_amdgcn_mov_dpp((int)qh[d], 0xA0, 0xF, 0xF, false);
        q[1][d] = (uint32_t)__builtin_amdgcn_mov_dpp((int)qh[d], 0xF5, 0xF, 0xF, false);
      }
      x[0] = xh[0];
      if constexpr (NORM) {
#pragma unroll
        for (int d = 0; d < 4; ++d) ssq = dec::dot2(xh[0][d], xh[0][d], ssq);
      }
      if constexpr (XH) {
#pragma unroll
        for (int d = 0; d < 4; ++d) x[1][d] = (uint32_t)__builtin_amdgcn_mov_dpp((int)xh[0][d], 0x128, 0xF, 0xF, false);
      } else {
        x[1] = xh[XL - 1];
      }
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        const u32x4 sc = *(const u32x4*)(hsa + blk * kBlk + 16 * kg + 8 * g2);
        u32x4 bx;
#pragma unroll
        for (int d = 0; d < 4; ++d) bx[d] = pk_mul(to_f16x2<XT>(x[g2][d]), sc[d]);
        u32x2 lo[4], hi[4];
        half.lookup(q[g2], tabB, lo, hi);
#pragma unroll
        for (int c = 0; c < 4; ++c)
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, mdec::Half::operand(lo, hi, c)),
                                                          __builtin_bit_cast(f16x8, bx), acc[c], 0, 0, 0);
      }
    };

  if (wave < S) {
    // ---- column wave --------------------------------------------------------
    // The ring goes out once h and the table are in LDS; its round trip runs
    // under the barriers and the scaling.  (Issued before h has arrived, the
    // ring's load instructions hold up the other waves' h loads in the CU's
    // address unit, and so the barriers: 7% slower at B = 8.)  Up to kShort
    // blocks: the wave's blocks rounded up to an even count are all loaded
    // at once, unconditionally (at most one placeholder block, read past the
    // buffer), so that the compiler counts them and block d waits only for
    // its own loads.  More blocks: a ring of kDepth, refilled as blocks are
    // done (its loads are conditional: those waits are for every load in
    // flight).
    const int n = bhi - blo;   // wave-uniform
    auto exact = [&](auto nv) {
      constexpr int V = decltype(nv)::value;
      u32x4 qe[V], xe[V][XL];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int d = 0; d < V; ++d) {
        const int oq = d < n ? qo + d * kBlk * 2 : kFar;
        const int ox = d < n ? xo + d * kBlk * 2 : kFar;
        qe[d] = ld16<kNonTemporal>(rq, oq);
#pragma unroll
        for (int u = 0; u < XL; ++u) xe[d][u] = ld16(rx, ox + 16 * u);
        __builtin_amdgcn_sched_barrier(0);   // in block order
      }
      scale();
      __builtin_amdgcn_sched_barrier(0);   // no block's work above the barriers
#pragma unroll
      for (int d = 0; d < V; ++d)
        if ((V > 2 && d < V - 1) || d < n) block(qe[d], xe[d], blo + d);
    };
    if (n <= 2) {
      exact(std::integral_constant<int, 2>{});
    } else if (n <= 4) {
      exact(std::integral_constant<int, 4>{});
    } else if (n <= 6) {
      exact(std::integral_constant<int, 6>{});
    } else if (kShort >= 8 && n <= 8) {
      exact(std::integral_constant<int, (kShort >= 8 ? 8 : 6)>{});
    } else {
      u32x4 qv[kDepth], xv[kDepth][XL];
    __builtin_amdgcn_sched_barrier(0);
    if (wave < S) {
  #pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        if (blo + d < bhi) {
          qv[d] = ld16<kNonTemporal>(rq, qo + d * kBlk * 2);
  #pragma unroll
          for (int u = 0; u < XL; ++u) xv[d][u] = ld16(rx, xo + d * kBlk * 2 + 16 * u);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
      scale();
      for (int k = blo; k < bhi; k += kDepth) {
  #pragma unroll
        for (int d = 0; d < kDepth; ++d) {
          const int blk = k + d;
          if (blk >= bhi) break;                     // uniform
          block(qv[d], xv[d], blk);
          if (blk + kDepth < bhi) {
            const int off = (blk - blo + kDepth) * kBlk * 2;
            qv[d] = ld16<kNonTemporal>(rq, qo + off);
  #pragma unroll
            for (int u = 0; u < XL; ++u) xv[d][u] = ld16(rx, xo + off + 16 * u);
          }
        }
      }
    }
  } else {
    // ---- staging wave: the tile's entries (columns, O) --------------------------
    // (The row pointers are read by this wave alone: a column wave reading
    // them would wait for its whole ring.)
    constexpr int kPass = kEntCap / 64;
    int scol[kPass];
    u32x4 so[kPass];
    const int rsv = __builtin_amdgcn_readlane(rpv, 0);
    const int nent = __builtin_amdgcn_readlane(rpv, kTile) - rsv;
    const int nst = nent < kEntCap ? nent : kEntCap;
    if (lane <= kTile) erow[lane] = rpv - rsv;
    if (lane == 0) ebase = rsv;
    const __amdgpu_buffer_rsrc_t rc = rsrc(a.O_col + rsv, nst * 4);
    const __amdgpu_buffer_rsrc_t ro = rsrc(a.O + (size_t)rsv * 8, nst * 16);
#pragma unroll
    for (int p = 0; p < kPass; ++p) {
      scol[p] = (int)__builtin_amdgcn_raw_buffer_load_b32(rc, (lane + 64 * p) * 4, 0, 0);
      so[p] = ld16(ro, (lane + 64 * p) * 16);
    }
    scale();
    // The tile's first kEntCap critical blocks into LDS.
#pragma unroll
    for (int p = 0; p < kPass; ++p) {
      if (64 * p >= nst) break;                    // uniform
      const int e = lane + 64 * p;
      const int col = scol[p];
      const int cc = e < nst && (unsigned)col < (unsigned)N ? col : 0;
      uint16_t xb[16];
#pragma unroll
      for (int bb = 0; bb < 16; ++bb) xb[bb] = ld2(rx, bb < B ? (bb * ldx + cc) * 2 : 0x7ffffff0);
      const f16 h1 = as_f16(hs[cc]), hm = as_f16(hsa[cc]);
      if (e < nst) {
        eov[e] = so[p];
        u32x4 wo[2], wm[2];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const f16 x0 = to_f16<XT>(xb[2 * q]), x1 = to_f16<XT>(xb[2 * q + 1]);
          wo[q >> 2][q & 3] = (uint32_t)bits(x0 * h1) | ((uint32_t)bits(x1 * h1) << 16);
          if (HAS_S) wm[q >> 2][q & 3] = (uint32_t)bits(x0 * hm) | ((uint32_t)bits(x1 * hm) << 16);
        }
        *(u32x4*)&exo[e][0] = wo[0];
        *(u32x4*)&exo[e][8] = wo[1];
        if (HAS_S) {
          *(u32x4*)&exm[HAS_S ? e : 0][0] = wm[0];
          *(u32x4*)&exm[HAS_S ? e : 0][8] = wm[1];
        }
      }
    }
  }
  // The activation-scale rows are no longer read: the partial sums take
  // their place.  red[wave][b][16 lg + 4v + c] = acc[c][v].
  __syncthreads();
  if (wave < S) {
    const int b = lane & 15, lg = lane >> 4;
#pragma unroll
    for (int v = 0; v < 4; ++v)
      *(f32x4*)&red[wave][b][16 * lg + 4 * v] = (f32x4){acc[0][v], acc[1][v], acc[2][v], acc[3][v]};
    if constexpr (NORM) {
      ssq += partner<8>(ssq);
      ssq += partner<16>(ssq);
      ssq += partner<32>(ssq);
      if (lane < 8) wss[wave][lane] = ssq;
    }
  }
  __syncthreads();
  // NORM: this part's Σx² of batch row tid (tid < 8), the waves in order.
  float ssl = 0.0f;
  if (NORM && tid < 8) {
#pragma unroll
    for (int w = 0; w < S; ++w) ssl += wss[NORM ? w : 0][tid];
  }

  // ---- output: item t (< 512) -> batch row t/32, rows 2(t%32), +1; thread
  // tid takes items tid, tid + NT (NT is a multiple of 32: one row pair).
  const f16x4 t5 = tab[511 ^ 0x100];
  constexpr int kItems = (512 + NT - 1) / NT;
  const int r = (tid & 31) * 2;
  const int br = r >> 3, k = r & 7;
  const h2 t5p = {t5[k & 3], t5[(k + 1) & 3]};
  float s0[kItems], s1[kItems];
  bool ok[kItems];
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int oi = tid + NT * it, b = (oi >> 5) & 15;
    ok[it] = oi < 512 && b < B && orow < 8 * M;
    s0[it] = 0.0f;
    s1[it] = 0.0f;
    if (ok[it]) {
      float t0 = 0.0f, t1 = 0.0f;
#pragma unroll
      for (int w = 0; w < S; ++w) {
        const float2 p = *(const float2*)&red[w][b][r];
        t0 += p.x;
        t1 += p.y;
      }
      // Critical blocks of this block row: rows k, k+1 of each O (one 4-byte
      // read), two entries per step so the LDS reads of one overlap the other.
      const int e0 = erow[br], e1 = erow[br + 1];
      const int es = e1 < kEntCap ? e1 : kEntCap;
      auto corr1 = [&](int e) {
        const h2 o = __builtin_bit_cast(h2, *((const uint32_t*)&eov[e] + (k >> 1)));
        const float xo = (float)as_f16(exo[e][b]);
        const float xm = HAS_S ? (float)as_f16(exm[HAS_S ? e : 0][b]) : xo;
        t0 += (float)o[0] * xo - (float)t5p[0] * xm;
        t1 += (float)o[1] * xo - (float)t5p[1] * xm;
      };
      int e = e0;
      for (; e + 1 < es; e += 2) {
        corr1(e);
        corr1(e + 1);
      }
      if (e < es) corr1(e);
      // Beyond the staged entries: straight from memory (the activation
      // scales are no longer in LDS).
      for (int e2 = es > e0 ? es : e0; e2 < e1; ++e2) {
        const int ge = ebase + e2;
        const int col = gp(a.O_col)[ge];
        const f16x8 o = *gp((const f16x8*)(a.O + (size_t)ge * 8));
        const f16 x16 = to_f16<XT>(gp(a.x)[(size_t)b * ldx + col]);
        const f16 hc = as_f16(gp((const uint16_t*)a.h)[col]);
        const f16 h1 = (NORM ? (f16)(hc * as_f16(gp((const uint16_t*)a.nw)[col])) : hc) * down;
        const float xo = (float)(f16)(x16 * h1);
        const float xm = HAS_S ? (float)(f16)(x16 * (f16)(h1 * as_f16(gp((const uint16_t*)a.S)[(size_t)grp * N + col]))) : xo;
        t0 += (float)o[k] * xo - (float)t5p[0] * xm;
        t1 += (float)o[k + 1] * xo - (float)t5p[1] * xm;
      }
      s0[it] = t0;
      s1[it] = t1;
    }
  }
  // Split columns: every part leaves its partial sums (device-coherent
  // stores, complete before the tile's counter is raised); the last part to
  // arrive adds all Pt of them in part order, so the result does not depend
  // on which part came last, writes y and resets the counter.  Publication
  // uses gfx950's coherence, not C++ release/acquire: the sums are
  // agent-scope atomic stores (sc1, written through to the level every XCD
  // reads), every wave waits for their completion (vmcnt(0)) before the
  // barrier that precedes the count, the count is an atomic at that level,
  // and the last part reads the sums with agent-scope atomic loads (sc1).
  // An agent-scope release on the count would add an L2 writeback in every
  // part and the acquire an L2 invalidate: measured +2 us per split launch
  // (the B=8 Llama-2-7B step 1.71 -> 1.91 ms), so the count stays relaxed.
  bool fin = true;
  if (Pt > 1) {
    __shared__ int last_part;
    float* base = wpart + (size_t)(tile_g - T1) * Pt * (kPartBytes / 4) + r;
    float* ssb = wpart + (size_t)(tile_g - T1) * Pt * (kPartBytes / 4) + 16 * 64;   // Σx² slots
#pragma unroll
    for (int it = 0; it < kItems; ++it)
      if (ok[it]) st_pair(base + part * (kPartBytes / 4) + (((tid + NT * it) >> 5) & 15) * 64, s0[it], s1[it]);
    if (NORM && tid < 8)
      __hip_atomic_store((uint32_t*)(ssb + part * (kPartBytes / 4) + tid), __builtin_bit_cast(uint32_t, ssl),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();
    if (tid == 0) {
      const int old = __hip_atomic_fetch_add(wcnt + tile_g, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_part = old == Pt - 1;
      if (old == Pt - 1) __hip_atomic_store(wcnt + tile_g, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    fin = last_part != 0;
    if (fin) {
#pragma unroll
      for (int it = 0; it < kItems; ++it) {
        if (!ok[it]) continue;
        const int b = ((tid + NT * it) >> 5) & 15;
        float t0 = 0.0f, t1 = 0.0f;
        for (int q = 0; q < Pt; ++q) {
          float2 v = make_float2(s0[it], s1[it]);
          if (q != part) v = ld_pair(base + q * (kPartBytes / 4) + b * 64);
          t0 += v.x;
          t1 += v.y;
        }
        s0[it] = t0;
        s1[it] = t1;
      }
      if (NORM && tid < 8) {   // the parts' Σx², in part order
        float t = 0.0f;
        for (int q = 0; q < Pt; ++q)
          t += q == part ? ssl
                         : __builtin_bit_cast(float, __hip_atomic_load((const uint32_t*)(ssb + q * (kPartBytes / 4) + tid),
                                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        ssl = t;
      }
    }
  }
  if (NORM && fin) {   // fin is uniform over the workgroup
    if (tid < 8) sinv[tid] = rsqrtf(ssl / (float)N + a.eps);
    __syncthreads();
  }
  uint32_t pks[kItems];
  if (fin) {
    const h2 gg = __builtin_bit_cast(h2, gpair), bb = __builtin_bit_cast(h2, bpair);
    const h2 rr = __builtin_bit_cast(h2, rpair);
#pragma unroll
    for (int it = 0; it < kItems; ++it) {
      if (!ok[it]) continue;
      const int b = ((tid + NT * it) >> 5) & 15;
      const float sc = NORM ? out_scale * sinv[b & 7] : out_scale;
      const float y0 = s0[it] * sc * (float)gg[0] + (float)bb[0];
      const float y1 = s1[it] * sc * (float)gg[1] + (float)bb[1];
      uint32_t pk = (uint32_t)Act<XT>::from_f32(y0) | ((uint32_t)Act<XT>::from_f32(y1) << 16);
      if (a.res) {   // fp16 only (the launcher's check): y = fp16(res + fp16(out))
        const h2 o = __builtin_bit_cast(h2, pk);
        pk = (uint32_t)Act<XT>::from_f32((float)rr[0] + (float)o[0]) |
             ((uint32_t)Act<XT>::from_f32((float)rr[1] + (float)o[1]) << 16);
      }
      uint32_t* yp = (uint32_t*)(a.y + (size_t)b * a.ldy + orow);
      if (ma.act) __hip_atomic_store(yp, pk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else *gp(yp) = pk;
      pks[it] = pk;
    }
  }
  // SwiGLU (ma.act: layer 0 gate, layer 1 up, up's columns right after
  // gate's in y): the two workgroups that finish row tile `tile` of the two
  // layers meet at a counter past the split counters; the second to arrive
  // reads the other's outputs and writes act = silu(gate) ⊙ up.  Publication
  // as for the split sums above: agent-scope atomic stores of y, vmcnt(0)
  // before the barrier that precedes the count, agent-scope atomic loads.
  if (ma.act && fin) {   // uniform over the workgroup
    __shared__ int pair_last;
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();
    if (tid == 0) {
      int* pc = wcnt + ma.start[2] + tile;
      const int old = __hip_atomic_fetch_add(pc, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      pair_last = old == 1;
      if (old == 1) __hip_atomic_store(pc, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (pair_last) {
      const int F = 8 * M;
#pragma unroll
      for (int it = 0; it < kItems; ++it) {
        if (!ok[it]) continue;
        const int b = ((tid + NT * it) >> 5) & 15;
        const uint32_t other = __hip_atomic_load((const uint32_t*)(a.y + (size_t)b * a.ldy + orow + (li == 0 ? F : -F)),
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const h2 gv = __builtin_bit_cast(h2, li == 0 ? pks[it] : other);
        const h2 uv = __builtin_bit_cast(h2, li == 0 ? other : pks[it]);
        const float g0 = (float)gv[0], g1 = (float)gv[1];
        float o0 = g0 / (1.0f + __expf(-g0)) * (float)uv[0];
        float o1 = g1 / (1.0f + __expf(-g1)) * (float)uv[1];
        // The fp32 rounding of the product before the fp16 one, as the
        // separate SwiGLU kernel computes it (the compiler would otherwise
        // fuse the multiply and the conversion).
        asm volatile("" : "+v"(o0), "+v"(o1));
        *gp((uint32_t*)(ma.act + (size_t)b * F + orow)) =
            (uint32_t)Act<f16>::from_f32(o0) | ((uint32_t)Act<f16>::from_f32(o1) << 16);
      }
    }
  }
}

// Parts for `split` tiles: as many as keep them within one workgroup per CU
// (a further round of workgroups would add a whole tile's time), within the
// workspace (none: one part).
inline int parts_for(int split, int tiles, void* work, long long work_bytes) {
  if (!work || tiles > kMaxCounters || split <= 0) return 1;
  int P = dec::cu_count() / split;
  P = P < 1 ? 1 : P > kMaxParts ? kMaxParts : P;
  while (P > 1 && (long long)(kCntBytes + (size_t)split * P * kPartBytes) > work_bytes) --P;
  return P;
}

template <int S, bool HAS_S, typename XT, bool XH, bool NORM = false>
int launch_t(const LinearArgs* l, int n, hipStream_t s, void* work, long long work_bytes, uint16_t* act) {
  int tiles = 0;
  for (int k = 0; k < n; ++k) tiles += (l[k].M + kTile - 1) / kTile;
  // SwiGLU pairs: one counter per row tile of a layer, after the tiles' own.
  if (act && (!work || work_bytes < (long long)kCntBytes || tiles + tiles / 2 > kMaxCounters)) return -1;
  // One workgroup per CU.  Up to one round of tiles: each tile's columns
  // split P ways.  More tiles than CUs: the first round takes whole tiles,
  // and the tiles left for the second round are split so that it is shorter.
  const int cu = dec::cu_count();
  int T1 = tiles > cu ? cu : 0;
  int P = parts_for(tiles - T1, tiles, work, work_bytes);
  if (P == 1) T1 = 0;
  MultiArgs ma;
  ma.n = n;
  ma.act = act;
  ma.start[0] = 0;
  for (int k = 0; k < kMaxLayers; ++k) {
    ma.l[k] = l[k < n ? k : 0];
    ma.start[k + 1] = ma.start[k] + (k < n ? (l[k].M + kTile - 1) / kTile : 0);   // tiles
  }
  const int grid = T1 + (tiles - T1) * P;
  auto kern = k_decode_mfma<S, HAS_S, XT, XH, NORM>;
  const size_t dyn = dyn_bytes(l[0].N, HAS_S, S);
  static size_t attr = 0;
  if (dyn > attr) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn) != hipSuccess)
      return -1;
    attr = dyn;
  }
  int* cnt = P > 1 || act ? (int*)work : nullptr;
  float* part = P > 1 ? (float*)((char*)work + kCntBytes) : nullptr;
  kern<<<grid, (S + 1) * 64, dyn, s>>>(ma, P, T1, cnt, part);
  return 0;
}

}  // namespace dmf

// Returns 0 if launched, -1 if the layers are outside this kernel's range
// (then the vector decode kernel or the generic matvec takes them).
int launch_decode_mfma_multi(const LinearArgs* l, int n, hipStream_t s, void* work, long long work_bytes,
                             uint16_t* act) {
  if (n < 1 || n > kMaxLayers) return -1;
  const LinearArgs& a = l[0];
  // SwiGLU: gate and up of equal M, up's outputs right after gate's, fp16,
  // 4-byte aligned act, no residual.
  if (act && (n != 2 || l[1].M != a.M || l[1].y != a.y + 8 * (size_t)a.M || l[1].ldy != a.ldy || a.x_bf16 ||
              a.res || l[1].res || ((uintptr_t)act & 3) != 0))
    return -1;
  if (a.B < 1 || a.B > 16 || a.codes_f32 || (a.N & 7) != 0) return -1;
  // prep 1 (the norm at the output; no residual add before it, no xsum) and
  // the residual: fp16 x, B <= 8, whole 64-column blocks (so Σx² sees no
  // column past N).
  const bool norm = a.prep == 1;
  if (a.prep != 0 && (!norm || a.x2 || a.xsum || !a.nw || a.B > 8 || (a.N & 63) != 0 || a.x_bf16)) return -1;
  if (norm && (((uintptr_t)a.nw & 15) != 0)) return -1;
  // y is written in pairs of fp16 (4-byte stores).
  if ((a.ldy & 1) != 0 || ((uintptr_t)a.y & 3) != 0) return -1;
  for (int i = 0; i < n; ++i) {
    const LinearArgs& b = l[i];
    if (b.N != a.N || b.B != a.B || b.x != a.x || b.ldx != a.ldx || b.codes != a.codes ||
        b.codes_f32 != a.codes_f32 || b.x_bf16 != a.x_bf16 || (b.S != nullptr) != (a.S != nullptr) ||
        b.prep != a.prep || b.nw != a.nw || b.eps != a.eps || b.x2 || b.xsum || ((uintptr_t)b.y & 3) != 0)
      return -1;
    if (b.res && (a.x_bf16 || ((uintptr_t)b.res & 3) != 0)) return -1;
    // S_group: one scale row per 64-row tile.
    if (b.S && (b.qb <= 0 || b.qb % 64 != 0)) return -1;
    if ((long)b.M * b.N * 2 >= (1L << 30)) return -1;   // 32-bit buffer offsets
  }
  if ((long)(a.B - 1) * a.ldx + a.N >= (1L << 30)) return -1;
  // The activation-scale rows and the staged entries share the 160 KB of LDS.
  if (dmf::dyn_bytes(a.N, a.S != nullptr, dmf::kS) > 120 * 1024) return -1;
  // (Two 6-wave workgroups per CU for layers with more tiles than CUs, so
  // that they run in one round, measured slower than two rounds of 9-wave
  // workgroups: gate|up 11008x4096 at B=8 24.6 us against 22.2 us.)
  using namespace dmf;
  const bool xh = a.B <= 8;
  if (norm) return a.S ? launch_t<kS, true, f16, true, true>(l, n, s, work, work_bytes, act)
                       : launch_t<kS, false, f16, true, true>(l, n, s, work, work_bytes, act);
  if (a.x_bf16) {
    if (a.S) return xh ? launch_t<kS, true, bf16, true>(l, n, s, work, work_bytes, act)
                       : launch_t<kS, true, bf16, false>(l, n, s, work, work_bytes, act);
    return xh ? launch_t<kS, false, bf16, true>(l, n, s, work, work_bytes, act)
              : launch_t<kS, false, bf16, false>(l, n, s, work, work_bytes, act);
  }
  if (a.S) return xh ? launch_t<kS, true, f16, true>(l, n, s, work, work_bytes, act)
                     : launch_t<kS, true, f16, false>(l, n, s, work, work_bytes, act);
  return xh ? launch_t<kS, false, f16, true>(l, n, s, work, work_bytes, act)
            : launch_t<kS, false, f16, false>(l, n, s, work, work_bytes, act);
}

long long decode_mfma_work_bytes() {
  return (long long)(dmf::kCntBytes + (size_t)dec::cu_count() * dmf::kPartBytes);
}

}  // namespace eptq

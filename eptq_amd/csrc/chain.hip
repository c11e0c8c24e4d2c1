// Batch-1 chains of dependent E8-D4 Linears in one persistent launch
// (contract: include/eptq_chain.h).
//
// Why: launched one stage at a time, every stage of a decode step pays the
// launch gap, the round trip of its first index loads and the drain of its
// last workgroups (about 4 us of a 4096x4096 Linear's 5.3 us in a graph).
// Here one workgroup per compute unit walks all stages; a stage's index
// chunks, h, g, bias and row pointers are requested before its input
// exists, so only the input's trip from its producers remains between
// stages.
//
// Stage s in workgroup wg (1024 threads, 16 waves, one workgroup per CU):
//  * rows: Q-rows [wg·Mt/G, (wg+1)·Mt/G) of the stage's layers laid end to
//    end (at most 16 rows and two layers per workgroup);
//  * chunks: the rows' 16-byte index chunks (8 columns) in row-major order,
//    split into 16 equal wave ranges; lane l of a wave takes chunks
//    start + l + 64k.  A range spans at most two rows (range <= one row), so
//    a lane keeps two sets of 8 fp32 accumulators and a chunk's sums go to
//    the set of its row;
//  * input: every thread waits for the tagged words of its 8-column input
//    chunks (their tag is this run's number), forms the input (slice or
//    SwiGLU, fp32), and, with an RMSNorm, adds its squares to the workgroup
//    sum; then the activation tables x·w·h are written to LDS per layer of
//    the workgroup's rows, fp16 scaled per chunk by a power of two with the
//    chunk's maximum in [0.5, 1) (the batch-1 scheme of decode_layer.h);
//  * decode: the E8-D4 table sits in LDS in COPIES interleaved copies (lane
//    l reads copy l % COPIES, so lanes reading the same table row hit
//    different banks); per chunk 16 lookups, 8 packed fp16 FMAs per word,
//    then one mixed FMA per output moves the chunk sum into fp32 times the
//    chunk scale;
//  * critical blocks: decoded as table row 511 in the loop; each staged CSR
//    entry of the rows adds O·x − c511·x at its column (LDS, summed per row
//    in entry order after the partial sums, so results do not depend on
//    timing);
//  * output: the 16 waves' partial sums are added in wave order, times the
//    RMSNorm scale, g and + bias; fp16 outputs go to the caller's y and, two
//    per 8-byte word with the run number, to the stage's tagged buffer.
//
// Run numbers: the run's tag is the workspace's counter + 1; the last
// workgroup to leave stores it as the new counter, so no buffer is reset
// between runs.  Every wait is bounded (s_memrealtime); one that expires
// sets the error word, which every waiting thread also polls, and all
// workgroups leave.  Every workgroup must be resident at once: the grid is
// the number of CUs, one workgroup per CU by its LDS and register use
// (checked with the occupancy query at plan time).

#include <string.h>

#include <vector>

#include "decode_layer.h"
#include "eptq_chain.h"
#include "kernels.h"

namespace eptq {
namespace chain {

using dec::as_h2;
using dec::fma_hi;
using dec::fma_lo;
using dec::gp;
using dec::h2;

constexpr int kT = 1024;       // threads per workgroup
constexpr int kW = kT / 64;    // waves
constexpr int kMaxJ = 6;       // index chunks per lane per stage
constexpr int kMaxRows = 16;   // Q-rows per workgroup per stage
constexpr int kMaxEnt = 256;   // critical-block entries staged per workgroup per stage
constexpr int kMaxN = 16384;   // input length (two 8-column chunks per thread)
constexpr int kXC = 2;
constexpr long long kDefaultSpin = 25000000;   // 0.25 s of the 100 MHz real-time counter

struct LayerD {
  const int16_t* Q;
  const f16* g;
  const f16* h;
  const f16* O;
  const int32_t* O_col;
  const int32_t* O_row_ptr;
  const f16* bias;
  int M, row0, y_off, pad;
};

struct StageD {
  LayerD L[kMaxLayers];
  const uint64_t* src;   // tagged words of the source stage (null: the chain input)
  const f16* nw;         // RMSNorm weight (null: none)
  uint16_t* y;           // the caller's fp16 output (null: none)
  uint64_t* yt;          // tagged output words
  int nl, N, Mt, src_col, act, pad;
  float eps, pad2;
};

// The plan does not change during a launch: constant address space, so its
// fields are read with scalar loads.
typedef const __attribute__((address_space(4))) StageD CStageD;

__device__ __forceinline__ uint64_t ld_tag(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_u32(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ __attribute__((address_space(3))) void* lds(char* p) {
  return (__attribute__((address_space(3))) void*)p;
}

__device__ __forceinline__ float f16_of(uint32_t w, int hi) {
  return (float)__builtin_bit_cast(f16, (uint16_t)(hi ? w >> 16 : w & 0xffffu));
}

// Layer (0..nl-1) of stage row gr (gr uniform: scalar code).
__device__ __forceinline__ int layer_of(CStageD* S, int nl, int gr) {
  int l = 0;
#pragma unroll
  for (int i = 1; i < kMaxLayers; ++i)
    if (i < nl && gr >= S->L[i].row0) l = i;
  return __builtin_amdgcn_readfirstlane(l);
}

// A layer's descriptor in scalar registers: a workgroup's rows lie in at most
// two layers (A and Z), and each thread selects between the two copies, so
// no thread indexes the descriptors with a per-thread layer number (that
// would make every field a dependent vector load).
struct LayerU {
  const int16_t* Q;
  const f16* g;
  const f16* h;
  const f16* O;
  const int32_t* O_col;
  const int32_t* O_row_ptr;
  const f16* bias;
  int row0, y_off;
};

__device__ __forceinline__ LayerU layer_u(CStageD* S, int l) {
  LayerU u;
  u.Q = S->L[l].Q;
  u.g = S->L[l].g;
  u.h = S->L[l].h;
  u.O = S->L[l].O;
  u.O_col = S->L[l].O_col;
  u.O_row_ptr = S->L[l].O_row_ptr;
  u.bias = S->L[l].bias;
  u.row0 = S->L[l].row0;
  u.y_off = S->L[l].y_off;
  return u;
}

template <int COPIES>
__device__ __forceinline__ void lookups(uint32_t w, const char* __restrict__ tabB, uint32_t coff, u32x2& t1l,
                                        u32x2& t2l, u32x2& t1h, u32x2& t2h) {
  constexpr int SH = COPIES == 32 ? 5 : COPIES == 16 ? 4 : COPIES == 8 ? 3 : COPIES == 4 ? 2 : 0;
  const uint32_t lo = (w >> 4) & 0xFF8u;                               // rows 0-3, lower index
  const uint32_t lo2 = ((w >> 4) & 0xC00u) | ((w & 127u) << 3);        // rows 4-7
  const uint32_t hi = (w >> 20) & 0xFF8u;                              // upper index
  const uint32_t hi2 = ((w >> 20) & 0xC00u) | (((w >> 16) & 127u) << 3);
  t1l = *(const u32x2*)(tabB + ((lo << SH) | coff));
  t2l = *(const u32x2*)(tabB + ((lo2 << SH) | coff));
  t1h = *(const u32x2*)(tabB + ((hi << SH) | coff));
  t2h = *(const u32x2*)(tabB + ((hi2 << SH) | coff));
}

// dyn LDS: [COPIES x 4 KB table][slot 0: xs (fp16, N; whole KB) | csc (fp32, N/8)][slot 1][norm weight (whole KB)]
template <int COPIES>
__global__ __launch_bounds__(kT, 1) void k_chain(const StageD* __restrict__ plan_, int ns, unsigned* __restrict__ ctl,
                                                 const f16x4* __restrict__ codes, const uint16_t* __restrict__ x,
                                                 long long spin, int slot_bytes, int csc_off) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ float part[kW][16];
  __shared__ float corr[kMaxEnt][8];
  __shared__ int s_rp[kMaxRows][2];
  __shared__ float s_red[kW];

  CStageD* plan = (CStageD*)plan_;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const unsigned G = gridDim.x, wg = blockIdx.x;
  const unsigned run = __builtin_amdgcn_readfirstlane(ld_u32(ctl) + 1u);
  char* const tabB = dyn;
  char* const act0 = dyn + COPIES * 4096;
  char* const nwb = act0 + 2 * slot_bytes;   // RMSNorm weight

  for (int i = threadIdx.x; i < 512 * COPIES; i += kT) ((f16x4*)tabB)[i] = codes[(i / COPIES) ^ 0x100];
  __syncthreads();

  bool stop = false;
  bool ovf = false;   // the previous stage read activation tables after its last barrier
  for (int s = 0; s < ns; ++s) {
    CStageD* S = plan + s;
    const int Mt = S->Mt;
    const int r0 = (int)(wg * (unsigned)Mt / G), r1 = (int)((wg + 1) * (unsigned)Mt / G);
    const int R = r1 - r0;
    if (R == 0) continue;
    // Per-thread values are derived afresh in every stage (the empty asm
    // hides that they do not change), so none is held in a register across
    // the whole stage loop: the decode loop needs every register.
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const uint32_t coff = (uint32_t)(lane % COPIES) * 8u;
    const f16x4 t5 = ((const f16x4*)tabB)[(511 ^ 0x100) * COPIES];   // the marker's decode
    const int N = S->N, nch = N >> 3, C = R * nch, nl = S->nl;
    const int la = layer_of(S, nl, r0), lz = layer_of(S, nl, r1 - 1);
    const bool two = lz != la;
    if (ovf) __syncthreads();   // before this stage's DMA overwrites the tables

    // This wave's chunk range [fs, fe): rows rowA and rowA + 1 (local).
    const int fs = (int)((unsigned)(wave * C) / kW), fe = (int)((unsigned)((wave + 1) * C) / kW);
    const int rowA = fs / nch, bnd = (rowA + 1) * nch;
    const int grA = r0 + rowA, grB = r0 + (rowA + 1 < R ? rowA + 1 : rowA);
    const LayerU A = layer_u(S, la), Z = layer_u(S, lz);
    const bool zA = two && grA >= Z.row0, zB = two && grB >= Z.row0;   // wave-uniform
    const int16_t* QA = (zA ? Z.Q : A.Q) + (size_t)(grA - (zA ? Z.row0 : A.row0)) * N;
    const int16_t* QB = (zB ? Z.Q : A.Q) + (size_t)(grB - (zB ? Z.row0 : A.row0)) * N;

    // 1. Everything that does not depend on the input, requested first.
    u32x4 ring[kMaxJ];
#pragma unroll
    for (int k = 0; k < kMaxJ; ++k) {
      const int f = fs + lane + 64 * k;
      if (f < fe) {
        const int16_t* q = f < bnd ? QA + (size_t)(f - rowA * nch) * 8 : QB + (size_t)(f - bnd) * 8;
        ring[k] = __builtin_nontemporal_load(gp((const u32x4*)q));
      }
    }
    f16 og = (f16)0.0f, ob = (f16)0.0f;
    const int olr = tid >> 3, ok = tid & 7;
    if (tid < R * 8) {
      const int gr = r0 + olr;
      const bool z = two && gr >= Z.row0;
      const int oi = 8 * (gr - (z ? Z.row0 : A.row0)) + ok;
      og = gp(z ? Z.g : A.g)[oi];
      const f16* b = z ? Z.bias : A.bias;
      if (b) ob = gp(b)[oi];
    }
    int rpb = 0, rpe = 0;
    if (tid < R) {
      const int gr = r0 + tid;
      const bool z = two && gr >= Z.row0;
      const int32_t* rp = (z ? Z.O_row_ptr : A.O_row_ptr) + (gr - (z ? Z.row0 : A.row0));
      rpb = gp(rp)[0];
      rpe = gp(rp)[1];
    }
    // h of the workgroup's layers into the activation slots and the RMSNorm
    // weight into its area, by LDS DMA (no registers held across the wait):
    // each wave instruction fills 1 KB, lane l's 16 bytes at byte 16·l, so
    // chunk c lands at byte 16·c; lanes past the last chunk re-read it into
    // the area's padding (areas are whole KB).
    const f16* nw = S->nw;
#pragma unroll
    for (int i = 0; i < kXC; ++i) {
      const int w2 = wave + kW * i;
      if (64 * w2 < nch) {
        const int c = 64 * w2 + lane < nch ? 64 * w2 + lane : nch - 1;
        __builtin_amdgcn_global_load_lds((const void*)(A.h + 8 * c), lds(act0 + w2 * 1024), 16, 0, 0);
        if (two)
          __builtin_amdgcn_global_load_lds((const void*)(Z.h + 8 * c), lds(act0 + slot_bytes + w2 * 1024), 16,
                                           0, 0);
        if (nw) __builtin_amdgcn_global_load_lds((const void*)(nw + 8 * c), lds(nwb + w2 * 1024), 16, 0, 0);
      }
    }

    // 2. The input, as packed fp16: tagged words of the source stage (their
    // run number is this run's) or the chain input.
    u32x4 xv[kXC];
    const uint64_t* src = S->src;
    const int scol = S->src_col, act = S->act;
    bool abort_ = false;
    if (src == nullptr) {
#pragma unroll
      for (int i = 0; i < kXC; ++i) {
        const int c = tid + kT * i;
        if (c < nch) xv[i] = *gp((const u32x4*)(x + scol + 8 * c));
      }
    } else {
      const uint64_t* pa = src + (scol >> 1);
      const uint64_t* pb = src + ((scol + N) >> 1);
      u32x4 ub[kXC];
      bool got[kXC];
#pragma unroll
      for (int i = 0; i < kXC; ++i) got[i] = tid + kT * i >= nch;
      const long long t0 = __builtin_amdgcn_s_memrealtime();
      for (;;) {
        bool all = true;
#pragma unroll
        for (int i = 0; i < kXC; ++i) {
          const int c = tid + kT * i;
          if (!got[i]) {
            // The chunk's last word first; the rest once it has arrived.
            bool ok = (unsigned)(ld_tag(pa + 4 * c + 3) >> 32) == run;
            if (act) ok = ok && (unsigned)(ld_tag(pb + 4 * c + 3) >> 32) == run;
            if (ok) {
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const uint64_t wa = ld_tag(pa + 4 * c + j);
                xv[i][j] = (uint32_t)wa;
                ok = ok && (unsigned)(wa >> 32) == run;
                if (act) {
                  const uint64_t wb = ld_tag(pb + 4 * c + j);
                  ub[i][j] = (uint32_t)wb;
                  ok = ok && (unsigned)(wb >> 32) == run;
                }
              }
            }
            got[i] = ok;
          }
          all = all && got[i];
        }
        if (all) break;
        if (ld_u32(ctl + 2) != 0u) {
          abort_ = true;
          break;
        }
        if (__builtin_amdgcn_s_memrealtime() - t0 > spin) {
          __hip_atomic_store(ctl + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          abort_ = true;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      if (act && !abort_) {
        // SwiGLU with the separate kernel's roundings: fp32 product, then fp16.
#pragma unroll
        for (int i = 0; i < kXC; ++i) {
          if (tid + kT * i < nch) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              float o0 = f16_of(xv[i][j], 0), o1 = f16_of(xv[i][j], 1);
              o0 = o0 / (1.0f + __expf(-o0)) * f16_of(ub[i][j], 0);
              o1 = o1 / (1.0f + __expf(-o1)) * f16_of(ub[i][j], 1);
              asm volatile("" : "+v"(o0), "+v"(o1));
              xv[i][j] = __builtin_bit_cast(uint32_t, (h2){(f16)o0, (f16)o1});
            }
          }
        }
      }
    }
    // RMSNorm: the workgroup's sum of squares.
    if (nw) {
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < kXC; ++i)
        if (tid + kT * i < nch && !abort_) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float t = f16_of(xv[i][e >> 1], e & 1);
            ss += t * t;
          }
        }
      ss = butterfly<1>(ss);
      ss = butterfly<2>(ss);
      ss = butterfly<4>(ss);
      ss = butterfly<8>(ss);
      ss = butterfly<16>(ss);
      ss = butterfly<32>(ss);
      if (lane == 0) s_red[wave] = ss;
    }
    if (__syncthreads_or(abort_)) {
      stop = true;
      break;
    }
    float inv = 1.0f;
    if (nw) {
      float t = 0.0f;
#pragma unroll
      for (int w = 0; w < kW; ++w) t += s_red[w];
      inv = rsqrtf(t / (float)N + S->eps);
    }

    // 3. Activation tables of the workgroup's layers, in place of their h
    // (this thread's chunks, which its own lane's DMA brought in).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    auto build = [&](char* slot, int c, const u32x4 xw) {
      const u32x4 hv = *(const u32x4*)(slot + c * 16);
      u32x4 wv = {0u, 0u, 0u, 0u};
      if (nw) wv = *(const u32x4*)(nwb + c * 16);
      float xf[8], mx = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float t = f16_of(xw[e >> 1], e & 1);
        if (nw) t *= f16_of(wv[e >> 1], e & 1);
        xf[e] = t * f16_of(hv[e >> 1], e & 1);
        mx = fmaxf(mx, fabsf(xf[e]));
      }
      const int ex = mx > 0.0f ? (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xff) - 126 : 0;
      const float down = __builtin_ldexpf(1.0f, -ex);
      u32x4 o;
#pragma unroll
      for (int d = 0; d < 4; ++d)
        o[d] = __builtin_bit_cast(uint32_t, (h2){(f16)(xf[2 * d] * down), (f16)(xf[2 * d + 1] * down)});
      *(u32x4*)(slot + c * 16) = o;
      ((float*)(slot + csc_off))[c] = __builtin_ldexpf(1.0f, ex);
    };
#pragma unroll
    for (int i = 0; i < kXC; ++i) {
      const int c = tid + kT * i;
      if (c < nch) {
        build(act0, c, xv[i]);
        if (two) build(act0 + slot_bytes, c, xv[i]);
      }
    }
    if (tid < R) {
      s_rp[tid][0] = rpb;
      s_rp[tid][1] = rpe;
    }
    __syncthreads();

    // 4. Critical-block entries of the rows (loaded now, used after the loop).
    int erow = -1, eidx = 0;
    {
      int E = 0;
      for (int r = 0; r < R; ++r) {
        const int cnt = s_rp[r][1] - s_rp[r][0];
        if (tid >= E && tid < E + cnt) {
          erow = r;
          eidx = s_rp[r][0] + tid - E;
        }
        E += cnt;
      }
      ovf = E > kMaxEnt;
    }
    int ecol = 0;
    u32x4 eo = {0u, 0u, 0u, 0u};
    if (erow >= 0 && tid < kMaxEnt) {
      const bool z = two && r0 + erow >= Z.row0;
      ecol = gp(z ? Z.O_col : A.O_col)[eidx];
      eo = *gp((const u32x4*)((z ? Z.O : A.O) + (size_t)eidx * 8));
    }

    // 5. The decode: two accumulator sets (rows rowA, rowA + 1 of the wave).
    const char* xsA = act0 + (zA ? slot_bytes : 0);
    const char* xsB = act0 + (zB ? slot_bytes : 0);
    float accA[8], accB[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      accA[k] = 0.0f;
      accB[k] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < kMaxJ; ++k) {
      const int f = fs + lane + 64 * k;
      if (f < fe) {
        const bool inA = f < bnd;
        const int cc = inA ? f - rowA * nch : f - bnd;
        const char* xsb = inA ? xsA : xsB;
        u32x2 t1l[4], t2l[4], t1h[4], t2h[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) lookups<COPIES>(ring[k][d], tabB, coff, t1l[d], t2l[d], t1h[d], t2h[d]);
        const u32x4 xw = *(const u32x4*)(xsb + cc * 16);
        const float sc = ((const float*)(xsb + csc_off))[cc];
        h2 acc16[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const h2 xx = as_h2(xw[d]);
          const h2 xl = {xx.x, xx.x}, xh = {xx.y, xx.y};
          const h2 cv[8] = {as_h2(t1l[d][0]), as_h2(t1l[d][1]), as_h2(t2l[d][0]), as_h2(t2l[d][1]),
                            as_h2(t1h[d][0]), as_h2(t1h[d][1]), as_h2(t2h[d][0]), as_h2(t2h[d][1])};
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            acc16[p] = d == 0 ? cv[p] * xl : __builtin_elementwise_fma(cv[p], xl, acc16[p]);
            acc16[p] = __builtin_elementwise_fma(cv[p + 4], xh, acc16[p]);
          }
        }
        const float sa = inA ? sc : 0.0f, sb = inA ? 0.0f : sc;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t pq = __builtin_bit_cast(uint32_t, acc16[p]);
          accA[2 * p] = fma_lo(pq, sa, accA[2 * p]);
          accA[2 * p + 1] = fma_hi(pq, sa, accA[2 * p + 1]);
          accB[2 * p] = fma_lo(pq, sb, accB[2 * p]);
          accB[2 * p + 1] = fma_hi(pq, sb, accB[2 * p + 1]);
        }
      }
    }

    // 6. Corrections of the staged entries; the waves' partial sums.
    auto xval = [&](int gr, int col) {
      const char* sl = act0 + (two && gr >= Z.row0 ? slot_bytes : 0);
      return (float)__builtin_bit_cast(f16, ((const uint16_t*)sl)[col]) * ((const float*)(sl + csc_off))[col >> 3];
    };
    if (erow >= 0 && tid < kMaxEnt) {
      const float xo = xval(r0 + erow, (unsigned)ecol < (unsigned)N ? ecol : 0);
      const f16x8 o = __builtin_bit_cast(f16x8, eo);
#pragma unroll
      for (int k = 0; k < 8; ++k) corr[tid][k] = (float)o[k] * xo - (float)t5[k & 3] * xo;
    }
    {
      float v[16];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        v[k] = accA[k];
        v[8 + k] = accB[k];
      }
      const int base = wave_reduce_halving<16>(v);
      if (WaveReduceOut<16>::writer(lane)) part[wave][base] = v[0];
    }
    __syncthreads();

    // 7. Outputs: partial sums in wave order, then the row's entries in order.
    if (tid < R * 8) {
      float sum = 0.0f;
#pragma unroll
      for (int w = 0; w < kW; ++w) {
        const int ws = (int)((unsigned)(w * C) / kW), we = (int)((unsigned)((w + 1) * C) / kW);
        if (we > ws) {
          const int ra = ws / nch;
          if (ra == olr) sum += part[w][ok];
          else if (ra + 1 == olr && we > (ra + 1) * nch) sum += part[w][8 + ok];
        }
      }
      int eb = 0;
      for (int r = 0; r < olr; ++r) eb += s_rp[r][1] - s_rp[r][0];
      const int rb = s_rp[olr][0], cnt = s_rp[olr][1] - rb;
      const int gr = r0 + olr;
      const bool z = two && gr >= Z.row0;
      for (int i = 0; i < cnt; ++i) {
        if (eb + i < kMaxEnt) {
          sum += corr[eb + i][ok];
        } else {
          const int col = gp(z ? Z.O_col : A.O_col)[rb + i];
          const float xo = xval(gr, (unsigned)col < (unsigned)N ? col : 0);
          sum += (float)gp(z ? Z.O : A.O)[(size_t)(rb + i) * 8 + ok] * xo - (float)t5[ok & 3] * xo;
        }
      }
      const f16 y16 = (f16)(sum * inv * (float)og + (float)ob);
      const int oi = (z ? Z.y_off : A.y_off) + 8 * (gr - (z ? Z.row0 : A.row0)) + ok;
      uint16_t* yp = S->y;
      if (yp) gp(yp)[oi] = __builtin_bit_cast(uint16_t, y16);
      const uint32_t mine = __builtin_bit_cast(uint16_t, y16);
      const uint32_t other = (uint32_t)__builtin_amdgcn_mov_dpp((int)mine, 0xB1, 0xF, 0xF, false);   // lane ^ 1
      if ((ok & 1) == 0)
        __hip_atomic_store(S->yt + (oi >> 1), (uint64_t)(mine | (other << 16)) | ((uint64_t)run << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  (void)stop;
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == G - 1) {
      __hip_atomic_store(ctl + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(ctl, run, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

constexpr size_t kCtlBytes = 256;

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
inline int align16(int v) { return (v + 15) & ~15; }

// Validate the stages and describe them for the kernel (tagged buffers at
// work + offsets).  Returns EPTQ_OK or an error code (message set).
int describe(const eptq_chain_stage* st, int n, int G, std::vector<StageD>* out, std::vector<size_t>* tag_offs,
             size_t* bytes, int* max_n) {
  const char* fn = "eptq_e8d4_chain";
  if (n <= 0 || !st) return set_error(EPTQ_EINVAL, "%s: n_stages=%d", fn, n);
  size_t off = kCtlBytes + align256((size_t)n * sizeof(StageD));
  *max_n = 8;
  for (int s = 0; s < n; ++s) {
    const eptq_chain_stage& a = st[s];
    if (a.n_layers < 1 || a.n_layers > kMaxLayers || !a.layers)
      return set_error(EPTQ_EINVAL, "%s: stage %d: n_layers=%d (1..%d)", fn, s, a.n_layers, kMaxLayers);
    if (a.N < 8 || a.N % 8 != 0 || a.N > kMaxN)
      return set_error(EPTQ_EUNSUPPORTED, "%s: stage %d: N=%d (a multiple of 8, at most %d)", fn, s, a.N, kMaxN);
    if (a.out_features <= 0 || (a.out_features & 1))
      return set_error(EPTQ_EINVAL, "%s: stage %d: out_features=%d (positive, even)", fn, s, a.out_features);
    if (a.src < -1 || a.src >= s) return set_error(EPTQ_EINVAL, "%s: stage %d: src=%d (-1 or an earlier stage)", fn, s, a.src);
    if (a.act != EPTQ_CHAIN_SLICE && a.act != EPTQ_CHAIN_SWIGLU)
      return set_error(EPTQ_EINVAL, "%s: stage %d: act=%d", fn, s, a.act);
    if (a.act == EPTQ_CHAIN_SWIGLU && a.src < 0)
      return set_error(EPTQ_EUNSUPPORTED, "%s: stage %d: SwiGLU reads a stage output, not the chain input", fn, s);
    if (a.src_col < 0 || (a.src_col & 1) || (a.src < 0 && a.src_col % 8 != 0))
      return set_error(EPTQ_EINVAL, "%s: stage %d: src_col=%d (even; a multiple of 8 for the chain input)", fn, s,
                       a.src_col);
    if (a.src >= 0 && (long long)a.src_col + (long long)a.N * (a.act == EPTQ_CHAIN_SWIGLU ? 2 : 1) > st[a.src].out_features)
      return set_error(EPTQ_EINVAL, "%s: stage %d reads past the %d columns of stage %d", fn, s,
                       st[a.src].out_features, a.src);
    if (a.norm_weight && ((uintptr_t)a.norm_weight & 15))
      return set_error(EPTQ_EUNSUPPORTED, "%s: stage %d: norm_weight must be 16-byte aligned", fn, s);
    if (a.y && ((uintptr_t)a.y & 3)) return set_error(EPTQ_EUNSUPPORTED, "%s: stage %d: y must be 4-byte aligned", fn, s);
    StageD d;
    memset(&d, 0, sizeof(d));
    int Mt = 0;
    for (int l = 0; l < a.n_layers; ++l) {
      const eptq_layer& L = a.layers[l];
      if (!L.Q || !L.g || !L.h || !L.O_row_ptr || L.M <= 0)
        return set_error(EPTQ_EINVAL, "%s: stage %d layer %d: null Q/g/h/O_row_ptr or M=%d", fn, s, l, L.M);
      if ((!L.O_vals) != (!L.O_col))
        return set_error(EPTQ_EINVAL, "%s: stage %d layer %d: O_vals and O_col both or neither", fn, s, l);
      if (L.S_group) return set_error(EPTQ_EUNSUPPORTED, "%s: stage %d layer %d: S_group layers are not chained", fn, s, l);
      if (((uintptr_t)L.Q & 15) || ((uintptr_t)L.h & 15) || ((uintptr_t)L.O_vals & 15))
        return set_error(EPTQ_EUNSUPPORTED, "%s: stage %d layer %d: Q, h and O_vals must be 16-byte aligned", fn, s, l);
      if (L.y_offset < 0 || (L.y_offset & 1) || L.y_offset + 8LL * L.M > a.out_features)
        return set_error(EPTQ_EINVAL, "%s: stage %d layer %d: columns [%lld, %lld) outside the %d outputs", fn, s, l,
                         L.y_offset, L.y_offset + 8LL * L.M, a.out_features);
      LayerD& D = d.L[l];
      D.Q = (const int16_t*)L.Q;
      D.g = (const f16*)L.g;
      D.h = (const f16*)L.h;
      D.O = (const f16*)L.O_vals;
      D.O_col = (const int32_t*)L.O_col;
      D.O_row_ptr = (const int32_t*)L.O_row_ptr;
      D.bias = (const f16*)L.bias;
      D.M = L.M;
      D.row0 = Mt;
      D.y_off = (int)L.y_offset;
      Mt += L.M;
    }
    // Rows per workgroup, chunks per lane and layers per workgroup.
    const int nch = a.N / 8;
    for (int w = 0; w < G; ++w) {
      const int r0 = (int)((long long)w * Mt / G), r1 = (int)((long long)(w + 1) * Mt / G);
      const int R = r1 - r0;
      if (R == 0) continue;
      if (R > kMaxRows)
        return set_error(EPTQ_EUNSUPPORTED, "%s: stage %d: %d rows per workgroup (at most %d on %d CUs)", fn, s, R,
                         kMaxRows, G);
      const int per_wave = (R * nch + kW - 1) / kW;
      if ((per_wave + 63) / 64 > kMaxJ)
        return set_error(EPTQ_EUNSUPPORTED, "%s: stage %d: %d index chunks per lane (at most %d)", fn, s,
                         (per_wave + 63) / 64, kMaxJ);
      int la = 0, lz = 0;
      for (int l = 0; l < a.n_layers; ++l) {
        if (r0 >= d.L[l].row0) la = l;
        if (r1 - 1 >= d.L[l].row0) lz = l;
      }
      if (lz - la > 1)
        return set_error(EPTQ_EUNSUPPORTED, "%s: stage %d: a workgroup's rows span %d layers (at most 2)", fn, s,
                         lz - la + 1);
    }
    d.nl = a.n_layers;
    d.N = a.N;
    d.Mt = Mt;
    d.src_col = a.src_col;
    d.act = a.act;
    d.nw = (const f16*)a.norm_weight;
    d.eps = a.eps;
    d.y = (uint16_t*)a.y;
    tag_offs->push_back(off);
    off += align256((size_t)(a.out_features / 2) * 8);
    out->push_back(d);
    if (a.N > *max_n) *max_n = a.N;
  }
  *bytes = off;
  return EPTQ_OK;
}

// One activation slot: xs (fp16, N) in whole KB, then the chunk scales;
// the RMSNorm weight area after the two slots is another align(2N, 1 KB).
inline int slot_bytes_of(int n_max, int* csc_off) {
  *csc_off = (2 * n_max + 1023) & ~1023;
  return align16(*csc_off + 4 * (n_max / 8));
}

constexpr int kStaticLds = (kW * 16 + kMaxEnt * 8 + kW) * 4 + kMaxRows * 2 * 4;

template <int COPIES>
const void* kernel_of() {
  return (const void*)k_chain<COPIES>;
}

const void* kernel_for(int copies) {
  switch (copies) {
    case 32: return kernel_of<32>();
    case 16: return kernel_of<16>();
    case 8: return kernel_of<8>();
    default: return kernel_of<1>();
  }
}

}  // namespace chain
}  // namespace eptq

using namespace eptq;
using namespace eptq::chain;

extern "C" {

long long eptq_e8d4_chain_work_bytes(const eptq_chain_stage* stages, int n_stages) {
  std::vector<StageD> d;
  std::vector<size_t> offs;
  size_t bytes = 0;
  int nmax = 0;
  if (describe(stages, n_stages, dec::cu_count(), &d, &offs, &bytes, &nmax) != EPTQ_OK) return 0;
  return (long long)bytes;
}

int eptq_e8d4_chain_plan(const eptq_chain_stage* stages, int n_stages, const void* codes, void* work,
                         long long work_bytes, eptq_chain_plan* plan, void* stream) {
  const char* fn = "eptq_e8d4_chain_plan";
  if (!codes || !work || !plan) return set_error(EPTQ_EINVAL, "%s: null codes/work/plan", fn);
  if (((uintptr_t)work & 255) || ((uintptr_t)codes & 7))
    return set_error(EPTQ_EUNSUPPORTED, "%s: work must be 256-byte and codes 8-byte aligned", fn);
  const int G = dec::cu_count();
  std::vector<StageD> d;
  std::vector<size_t> offs;
  size_t bytes = 0;
  int nmax = 0;
  if (const int rc = describe(stages, n_stages, G, &d, &offs, &bytes, &nmax)) return rc;
  // Every operand the kernel reads or writes must be device memory of the
  // current device (a host pointer would fault inside the persistent launch).
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(EPTQ_EHIP, "%s: hipGetDevice failed", fn);
  auto on_device = [&](const void* p) {
    if (!p) return true;
    hipPointerAttribute_t at;
    if (hipPointerGetAttributes(&at, p) != hipSuccess) {
      (void)hipGetLastError();
      return false;
    }
    return at.type == hipMemoryTypeDevice && at.device == dev;
  };
  if (!on_device(codes) || !on_device(work))
    return set_error(EPTQ_EINVAL, "%s: codes and work must be device memory of device %d", fn, dev);
  for (int s = 0; s < n_stages; ++s) {
    const eptq_chain_stage& a = stages[s];
    if (!on_device(a.norm_weight) || !on_device(a.y))
      return set_error(EPTQ_EINVAL, "%s: stage %d: norm_weight and y must be device memory of device %d", fn, s, dev);
    for (int l = 0; l < a.n_layers; ++l) {
      const eptq_layer& L = a.layers[l];
      if (!on_device(L.Q) || !on_device(L.g) || !on_device(L.h) || !on_device(L.O_vals) || !on_device(L.O_col) ||
          !on_device(L.O_row_ptr) || !on_device(L.bias))
        return set_error(EPTQ_EINVAL, "%s: stage %d layer %d: every operand must be device memory of device %d", fn, s,
                         l, dev);
    }
  }
  if (work_bytes < (long long)bytes)
    return set_error(EPTQ_EINVAL, "%s: work_bytes=%lld, the chain needs %zu", fn, work_bytes, bytes);
  char* base = (char*)work;
  for (int s = 0; s < n_stages; ++s) {
    d[s].yt = (uint64_t*)(base + offs[s]);
    d[s].src = stages[s].src >= 0 ? (const uint64_t*)(base + offs[stages[s].src]) : nullptr;
  }
  // LDS: the activation slots, then as many table copies as fit.
  int csc_off = 0;
  const int slot = slot_bytes_of(nmax, &csc_off);
  hipFuncAttributes fa;
  const int static_lds = hipFuncGetAttributes(&fa, kernel_for(16)) == hipSuccess ? (int)fa.sharedSizeBytes : kStaticLds;
  const int avail = 160 * 1024 - (static_lds > kStaticLds ? static_lds : kStaticLds) - 2 * slot - csc_off;
  int copies = 32;
  while (copies > 1 && copies * 4096 > avail) copies /= 2;
  if (copies < 8) copies = 1;
  if (copies * 4096 > avail) return set_error(EPTQ_EUNSUPPORTED, "%s: N=%d leaves no LDS for the table", fn, nmax);
  const int lds = copies * 4096 + 2 * slot + csc_off;
  const void* kern = kernel_for(copies);
  if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
    return set_error(EPTQ_EHIP, "%s: %d bytes of dynamic LDS refused", fn, lds);
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kT, lds) != hipSuccess || per_cu < 1)
    return set_error(EPTQ_EUNSUPPORTED, "%s: the chain kernel cannot be resident (occupancy %d)", fn, per_cu);
  hipStream_t s = (hipStream_t)stream;
  if (hipMemsetAsync(work, 0, bytes, s) != hipSuccess ||
      hipMemcpyAsync(base + kCtlBytes, d.data(), d.size() * sizeof(StageD), hipMemcpyHostToDevice, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return set_error(EPTQ_EHIP, "%s: writing the plan failed", fn);
  plan->codes = codes;
  plan->n_stages = n_stages;
  plan->grid = G;
  plan->lds_bytes = lds;
  plan->copies = copies;
  plan->slot_bytes = slot;
  plan->csc_offset = csc_off;
  plan->pad = 0;
  plan->spin_ticks = kDefaultSpin;
  plan->work_bytes = (long long)bytes;
  return EPTQ_OK;
}

int eptq_e8d4_chain_run(const eptq_chain_plan* plan, void* work, const void* x, void* stream) {
  const char* fn = "eptq_e8d4_chain_run";
  if (!plan || !work || !x || !plan->codes) return set_error(EPTQ_EINVAL, "%s: null plan/work/x", fn);
  if ((uintptr_t)x & 15) return set_error(EPTQ_EUNSUPPORTED, "%s: x must be 16-byte aligned", fn);
  if (plan->n_stages <= 0 || plan->grid <= 0 || plan->spin_ticks < 0 || plan->slot_bytes <= 0 ||
      plan->lds_bytes != plan->copies * 4096 + 2 * plan->slot_bytes + plan->csc_offset)
    return set_error(EPTQ_EINVAL, "%s: the plan was not filled by eptq_e8d4_chain_plan", fn);
  const int slot = plan->slot_bytes, csc_off = plan->csc_offset;
  const StageD* dplan = (const StageD*)((char*)work + kCtlBytes);
  unsigned* ctl = (unsigned*)work;
  hipStream_t s = (hipStream_t)stream;
  switch (plan->copies) {
    case 32:
      k_chain<32><<<plan->grid, kT, plan->lds_bytes, s>>>(dplan, plan->n_stages, ctl, (const f16x4*)plan->codes,
                                                          (const uint16_t*)x, plan->spin_ticks, slot, csc_off);
      break;
    case 16:
      k_chain<16><<<plan->grid, kT, plan->lds_bytes, s>>>(dplan, plan->n_stages, ctl, (const f16x4*)plan->codes,
                                                          (const uint16_t*)x, plan->spin_ticks, slot, csc_off);
      break;
    case 8:
      k_chain<8><<<plan->grid, kT, plan->lds_bytes, s>>>(dplan, plan->n_stages, ctl, (const f16x4*)plan->codes,
                                                         (const uint16_t*)x, plan->spin_ticks, slot, csc_off);
      break;
    default:
      k_chain<1><<<plan->grid, kT, plan->lds_bytes, s>>>(dplan, plan->n_stages, ctl, (const f16x4*)plan->codes,
                                                         (const uint16_t*)x, plan->spin_ticks, slot, csc_off);
      break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(EPTQ_EHIP, "%s: %s", fn, hipGetErrorString(e));
  return EPTQ_OK;
}

int eptq_e8d4_chain_error(void* work, int clear, int* err, void* stream) {
  const char* fn = "eptq_e8d4_chain_error";
  if (!work || !err) return set_error(EPTQ_EINVAL, "%s: null work/err", fn);
  hipStream_t s = (hipStream_t)stream;
  unsigned v = 0;
  if (hipMemcpyAsync(&v, (char*)work + 8, 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return set_error(EPTQ_EHIP, "%s: reading the error word failed", fn);
  *err = (int)v;
  if (clear && v) {
    const unsigned z = 0;
    if (hipMemcpyAsync((char*)work + 8, &z, 4, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
      return set_error(EPTQ_EHIP, "%s: clearing the error word failed", fn);
  }
  return EPTQ_OK;
}

}  // extern "C"

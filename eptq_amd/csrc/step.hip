// Persistent batch-1 E8-D4 decode-step engine: a whole sequence of dependent
// Linear stages (a decode step's q|k|v, o, gate|up, down for every layer) in
// one launch, one workgroup per compute unit.
//
// Why: as one launch per stage, every stage pays the launch gap, the first
// index loads' latency and the drain (~4 us fixed per launch, more than half
// of a Llama-2-7B step at batch 1).  Here the index stream of later stages is
// already in flight while a stage waits for its input.
//
// Workgroup (16 waves, all of a CU's activation side in one place):
//  * waves 4..15 (compute): stream the stage rows' index chunks through an
//    8-deep register ring per lane (16 bytes = 8 indices per lane per item,
//    an item is 64 chunks = 1 KB of one row) and run the decode arithmetic of
//    the batch-1 decode kernel (decode_layer.h) against the LDS activation
//    table.  The ring runs across stage boundaries: the chunks of the next
//    stages are requested while the current stage computes and waits.  These
//    waves issue no other global memory operation, so a wait for a ring load
//    never waits behind anything else (vmcnt counts in issue order).
//  * waves 0..3 (sync): everything else that touches global memory — the
//    stage input (polled, see below), the next stage's h, RMSNorm weight,
//    g/bias and critical-block entries, the critical-block corrections, and
//    the epilogue that writes the stage output.
// Per stage s: [A] input in LDS -> all waves build the activation tables
// x·h (one per layer of the stage, scaled per 8-column chunk) -> [B] ->
// compute waves run their items, sync waves add corrections and prefetch
// stage s+1 -> [C] -> sync waves sum the partials and write the output.
//
// Stage outputs are flagged: every 8-byte word holds two fp16 outputs and a
// 32-bit flag (epoch·kMaxStages + s + 1), written with one device-scope
// store.  A reader polls the words it needs until every flag matches, so a
// stage boundary is one store and one poll, with no counter, no fence and no
// wait for store completion.  The epoch (first word of the work area) grows
// by one per launch: the last workgroup to leave increments it.
//
// Every workgroup must be resident at once (grid = number of CUs, one
// workgroup per CU by its LDS use).  A poll that spins past its limit sets
// the error word and goes on, so every wave reaches the end.

#include <stddef.h>

#include "decode_layer.h"
#include "kernels.h"
#include "step.h"

namespace eptq {
namespace step {

using dec::h2;
using dec::as_h2;
using dec::fma_hi;
using dec::fma_lo;
using dec::kBufferWord3;
using dec::kCoherent;
using dec::kNonTemporal;
using dec::gp;

constexpr int kT = 1024;      // threads per workgroup
constexpr int kSyncW = 4;     // waves 0..3
constexpr int kCompW = 12;    // waves 4..15
constexpr int kChunks = 2;    // 16-byte index chunks per lane per item (an item: 64·kChunks chunks of a row)
constexpr int kRing = 4;      // ring depth (items) per compute wave (the item loop has up to 8 slots)
constexpr int kSlots = 16;    // partial-sum slots per row: compute waves 0..11, corrections at 12
constexpr int kCorrSlot = 12;
constexpr int kHRegs = 6;     // h chunks per sync thread (L·nch <= 1536)
constexpr int kWRegs = 2;     // RMSNorm weight chunks per sync thread (nch <= 512)
constexpr int kXRegs = 6;     // 16-byte input loads per sync thread and poll round (two rounds: N <= 12288)
constexpr int kRowsPerSyncWave = kRowsMax / kSyncW;
constexpr int kSpinLimit = 1 << 16;

typedef int i32x4 __attribute__((ext_vector_type(4)));

// The plan as constant memory: it does not change during a launch, so its
// fields are read with scalar loads (which the compute waves' vmcnt waits do
// not see) rather than vector loads.
typedef const __attribute__((address_space(4))) Stage CStage;
typedef const __attribute__((address_space(4))) Layer CLayer;

// The ring slot's loads have landed: (kRing - 1)·kChunks ring loads were
// issued after them and the compute waves issue no other vector memory
// operation.
__device__ __forceinline__ void ring_wait(u32x4 (&slot)[kChunks]) {
  if constexpr (kChunks == 1) {
    asm volatile("s_waitcnt vmcnt(%1)" : "+v"(slot[0]) : "n"((kRing - 1) * kChunks));
  } else {
    asm volatile("s_waitcnt vmcnt(%2)" : "+v"(slot[0]), "+v"(slot[1]) : "n"((kRing - 1) * kChunks));
  }
}

struct Offs {                 // dynamic LDS layout (bytes)
  int h, w, act, csc;         // xbuf at 0
};

__device__ __forceinline__ int rd_dev(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave-uniform copies (scalar registers): values the compiler cannot prove
// uniform through the cursor's control flow.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
template <typename T>
__device__ __forceinline__ const T* uni(const T* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const T*)(((uint64_t)hi << 32) | lo);
}

// This workgroup's rows [r0, r0 + rows) of a stage with M Q-rows (M·G < 2^31).
__device__ __forceinline__ void wg_rows(int M, int& r0, int& rows) {
  const unsigned G = gridDim.x, c = blockIdx.x;
  r0 = (int)(c * (unsigned)M / G);
  rows = (int)((c + 1) * (unsigned)M / G) - r0;
}

// Item range [a, b) of compute wave k among I items.
__device__ __forceinline__ void wave_items(int I, int k, int& a, int& b) {
  a = k * I / kCompW;
  b = (k + 1) * I / kCompW;
}

// Where compute wave k's work lies in stage s: items [a, b) of the
// workgroup's rows, and the layer of its first row.  Returns false when the
// wave has no item there.
struct Span {
  int a, b, r0, nseg, nch, N, lyr, rem;   // rem: rows left in layer lyr from the first row
};
__device__ __forceinline__ bool span_of(CStage* plan, int s, int k, Span& sp) {
  CStage* S = plan + s;
  int r0, rows;
  wg_rows(uni(S->M_tot), r0, rows);
  const int ns = uni(S->nseg);
  wave_items(rows * ns, k, sp.a, sp.b);
  if (sp.a >= sp.b) return false;
  sp.a = uni(sp.a);
  sp.b = uni(sp.b);
  sp.r0 = uni(r0);
  sp.nseg = ns;
  sp.nch = uni(S->nch);
  sp.N = uni(S->N);
  const int rg = sp.r0 + uni((unsigned)sp.a / (unsigned)ns);
  const int nl = uni(S->n_layers);
  const int b1 = nl > 1 ? uni(S->l[1].row0) : 0x7fffffff;
  const int b2 = nl > 2 ? uni(S->l[2].row0) : 0x7fffffff;
  sp.lyr = rg >= b2 ? 2 : rg >= b1 ? 1 : 0;
  sp.rem = uni(S->l[sp.lyr].row0 + S->l[sp.lyr].M - rg);
  return true;
}

// Producer: the next item to request.  State is wave-uniform: the current
// row's index pointer advances by N per row and switches layer when the
// layer's rows run out (descriptor read then).
struct Prod {
  CStage* plan;
  int n_stages, k;
  int s, i, b, seg, nseg, N, lyr, rem;
  int nrec;             // bytes of the current row (0 once exhausted: loads read nothing)
  const int16_t* rowQ;

  __device__ __forceinline__ void enter(int s_) {
    nrec = 0;
    pend = false;
    for (s = uni(s_); s < n_stages; s = uni(s + 1)) {
      Span sp;
      if (!span_of(plan, s, k, sp)) continue;
      i = sp.a;
      b = sp.b;
      nseg = sp.nseg;
      N = sp.N;
      const int row = uni((unsigned)i / (unsigned)nseg);
      seg = uni(i - row * nseg);
      lyr = sp.lyr;
      rem = sp.rem;
      CLayer* L = &plan[s].l[lyr];
      const int rg = sp.r0 + row;
      rowQ = L->Q + (size_t)(rg - L->row0) * N;
      nrec = N * 2;
      return;
    }
    rowQ = nullptr;   // with 0 records no lane reads anything
  }
  bool pend;            // the next item needs fix(): a new stage or layer
  // Next item, in-line part only (the common case: same row or next row of
  // the same layer); a layer or stage change is left to fix().
  __device__ __forceinline__ void advance_fast() {
    i = uni(i + 1);
    seg = uni(seg + 1);
    if (seg == nseg) {
      seg = 0;
      rem = uni(rem - 1);
      rowQ = uni(rowQ + N);
      if (rem == 0) pend = true;
    }
    if (i == b) pend = true;
  }
  __device__ __forceinline__ void fix() {
    pend = false;
    if (i == b) {
      enter(s + 1);
    } else {
      lyr = uni(lyr + 1);
      CLayer* L = &plan[s].l[lyr];
      rowQ = L->Q;
      rem = L->M;
    }
  }
  __device__ __forceinline__ void advance() {
    advance_fast();
    if (pend) fix();
  }
  // The 16 index bytes of lane `lane` (chunks past the row end read zero
  // through the buffer resource's bound; once exhausted nothing is read).
  //
  // Issued as inline assembly: the compiler does not track it, so it adds no
  // wait of its own; the consumer waits with ring_wait (exactly kRing - 1
  // newer ring loads in flight), which is tied to the slot's registers.
  __device__ __forceinline__ void load(u32x4 (&dst)[kChunks], int lane) const {
    const uint64_t a = (uint64_t)rowQ;
    const i32x4 rs = {uni((int)(uint32_t)a), uni((int)((uint32_t)(a >> 32) & 0xffffu)), uni(nrec), kBufferWord3};
    const int o = (seg * 64 * kChunks + lane) * 16;
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen nt" : "=v"(dst[0]) : "v"(o), "s"(rs));
    if constexpr (kChunks == 2)
      asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen offset:1024 nt" : "=v"(dst[1]) : "v"(o), "s"(rs));
  }
};

// Consumer: the item being computed, with the LDS offsets of its layer's
// activation table and chunk scales.
struct Cons {
  CStage* plan;
  int n_stages, k;
  int s, i, b, seg, nseg, nch, row, lyr, rem;
  int act_off, csc_off;   // elements

  __device__ __forceinline__ void set_layer(int N) {
    act_off = uni(lyr * (N + 8));
    csc_off = uni(lyr * (nch + 1));
  }
  __device__ __forceinline__ void enter(int s_) {
    pend = false;
    for (s = uni(s_); s < n_stages; s = uni(s + 1)) {
      Span sp;
      if (!span_of(plan, s, k, sp)) continue;
      i = sp.a;
      b = sp.b;
      nseg = sp.nseg;
      nch = sp.nch;
      row = uni((unsigned)i / (unsigned)nseg);
      seg = uni(i - row * nseg);
      lyr = sp.lyr;
      rem = sp.rem;
      set_layer(sp.N);
      return;
    }
  }
  bool pend;            // the next item needs fix(): a new stage or layer
  __device__ __forceinline__ void advance_fast() {
    i = uni(i + 1);
    seg = uni(seg + 1);
    if (seg == nseg) {
      seg = 0;
      row = uni(row + 1);
      rem = uni(rem - 1);
      if (rem == 0) pend = true;
    }
    if (i == b) pend = true;
  }
  __device__ __forceinline__ void fix() {
    pend = false;
    if (i == b) {
      enter(s + 1);
    } else {
      lyr = uni(lyr + 1);
      rem = uni(plan[s].l[lyr].M);
      set_layer(uni(plan[s].N));
    }
  }
};

// Two chunks (8 columns each) of one row against the activation table: the
// batch-1 arithmetic of the vector decode kernel (packed fp16 FMAs over a
// chunk, flushed into fp32 with the chunk's power-of-two scale).  All 32
// table lookups are issued before the arithmetic, so their LDS latency is
// paid once per item.
__device__ __forceinline__ void lookups(const u32x4 q, const char* __restrict__ tabB, u32x2 (&t1l)[4],
                                        u32x2 (&t2l)[4], u32x2 (&t1h)[4], u32x2 (&t2h)[4]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t w = q[d];
    const uint32_t w4 = w >> 4;
    const uint32_t a1lo = w4 & 0xFF8u;
    const uint32_t a1hi = hi_addr(w4);
    const uint32_t a2lo = bfi(0x3F8u, w << 3, a1lo);
    const uint32_t a2hi = bfi(0x3F8u, w >> 13, a1hi);
    t1l[d] = *(const u32x2*)(tabB + a1lo);
    t2l[d] = *(const u32x2*)(tabB + a2lo);
    t1h[d] = *(const u32x2*)(tabB + a1hi);
    t2h[d] = *(const u32x2*)(tabB + a2hi);
  }
}

__device__ __forceinline__ void accumulate(const u32x2 (&t1l)[4], const u32x2 (&t2l)[4], const u32x2 (&t1h)[4],
                                           const u32x2 (&t2h)[4], const u32x4 xw, float sc, float (&acc)[8]) {
  h2 acc16[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const h2 xx = as_h2(xw[d]);   // by value: a bit_cast of the element itself reads element 0
    const h2 xl = {xx.x, xx.x}, xh = {xx.y, xx.y};
    const h2 c[8] = {as_h2(t1l[d][0]), as_h2(t1l[d][1]), as_h2(t2l[d][0]), as_h2(t2l[d][1]),
                     as_h2(t1h[d][0]), as_h2(t1h[d][1]), as_h2(t2h[d][0]), as_h2(t2h[d][1])};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      acc16[p] = d == 0 ? c[p] * xl : __builtin_elementwise_fma(c[p], xl, acc16[p]);
      acc16[p] = __builtin_elementwise_fma(c[p + 4], xh, acc16[p]);
    }
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t pq = __builtin_bit_cast(uint32_t, acc16[p]);
    acc[2 * p] = fma_lo(pq, sc, acc[2 * p]);
    acc[2 * p + 1] = fma_hi(pq, sc, acc[2 * p + 1]);
  }
}

__global__ __launch_bounds__(kT) void k_step_b1(const Stage* __restrict__ plan, int n_stages,
                                                 int* __restrict__ sync, const f16x4* __restrict__ codes,
                                                 Offs off) {
  __shared__ f16x4 tab[512];
  __shared__ float red[kRowsMax][kSlots][8];
  __shared__ float s_rms[kSyncW];
  __shared__ int s_epoch;
  extern __shared__ __align__(16) char dyn[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint16_t* const xbuf = (uint16_t*)dyn;
  uint16_t* const hbuf = (uint16_t*)(dyn + off.h);
  uint16_t* const wbuf = (uint16_t*)(dyn + off.w);
  uint16_t* const act = (uint16_t*)(dyn + off.act);
  float* const csc = (float*)(dyn + off.csc);
  const char* tabB = (const char*)tab;

  if (tid < 512) tab[tid ^ 0x100] = codes[tid];
  for (int i = tid; i < kRowsMax * kSlots * 8; i += kT) (&red[0][0][0])[i] = 0.0f;
  if (tid == 0) s_epoch = rd_dev(sync + kEpochWord);
  __syncthreads();
  const unsigned epoch = (unsigned)s_epoch;
  auto flag_of = [&](int s) { return epoch * (unsigned)kMaxStages + (unsigned)s + 1u; };

  // Activation tables of stage S from xbuf, hbuf (and wbuf): every thread.
  CStage* const cplan = (CStage*)plan;
  auto build = [&](CStage& S) {
    const int N = S.N, nch = S.nch, nl = S.n_layers;
    float inv = 1.0f;
    if (S.prep) inv = rsqrtf((s_rms[0] + s_rms[1] + s_rms[2] + s_rms[3]) / (float)N + S.eps);
    // At most two (layer, chunk) items per thread (nl·nch <= 2·kT): both
    // read before either is computed.
    f16x8 xv[2], hv[2], wv[2];
    int qs[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int q = tid + r * kT;
      qs[r] = q;
      if (q < nl * nch) {
        const int l = q >= 2 * nch ? 2 : q >= nch ? 1 : 0;
        const int c = q - l * nch;
        xv[r] = *(const f16x8*)(xbuf + c * 8);
        hv[r] = *(const f16x8*)(hbuf + l * N + c * 8);
        if (S.prep) wv[r] = *(const f16x8*)(wbuf + c * 8);
      }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int q = qs[r];
      if (q >= nl * nch) continue;
      const int l = q >= 2 * nch ? 2 : q >= nch ? 1 : 0;
      const int c = q - l * nch;
      f16x8 xn = xv[r];
      if (S.prep) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xn[e] = (f16)((float)xv[r][e] * inv * (float)wv[r][e]);
      }
      float xf[8], mx = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xf[e] = __builtin_fmaf((float)xn[e], (float)hv[r][e], 0.0f);
        mx = fmaxf(mx, fabsf(xf[e]));
      }
      const int ex = mx > 0.0f ? (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xff) - 126 : 0;
      const float down = __builtin_ldexpf(1.0f, -ex);
      u32x4 w;
#pragma unroll
      for (int d = 0; d < 4; ++d)
        w[d] = __builtin_bit_cast(uint32_t, (h2){(f16)(xf[2 * d] * down), (f16)(xf[2 * d + 1] * down)});
      *(u32x4*)(act + l * (N + 8) + c * 8) = w;
      csc[l * (nch + 1) + c] = __builtin_ldexpf(1.0f, ex);
    }
    if (tid < nl) {
      *(u32x4*)(act + tid * (N + 8) + nch * 8) = (u32x4){0u, 0u, 0u, 0u};
      csc[tid * (nch + 1) + nch] = 1.0f;
    }
  };

  if (wave >= kSyncW) {
    // ------------------------------------------------------------ compute
    const int k = wave - kSyncW;
    Prod prod{(CStage*)plan, n_stages, k};
    prod.enter(0);
    Cons cons{(CStage*)plan, n_stages, k};
    cons.enter(0);
    // Exactly one ring load per item slot, always (past the last item the
    // producer re-reads its last row: a harmless load), so the loads of the
    // unrolled loop below come in a fixed order and the compiler waits for
    // exactly the slot in use (vmcnt 7), not for the whole ring.
    u32x4 ring[kRing][kChunks];
    auto refill = [&](u32x4 (&slot)[kChunks]) {
      prod.load(slot, lane);
      if (prod.s < n_stages) prod.advance();
    };
#pragma unroll
    for (int j = 0; j < kRing; ++j) refill(ring[j]);
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
    int cur_row = -1;
    auto flush = [&]() {
      if (cur_row < 0) return;
      const int base = wave_reduce_halving<8>(acc);
      if (WaveReduceOut<8>::writer(lane)) red[cur_row][k][base] = acc[0];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
      cur_row = -1;
    };
    // Stage 0 opens: input [A], tables, [B].
    __syncthreads();
    build(cplan[0]);
    __syncthreads();
    int cur = 0;
    // The rare part of moving on (a cursor entering a new stage or layer,
    // closing stage cur [C] and opening the next ones: [A], tables, [B]),
    // kept out of the unrolled item slots below so that the loop stays small
    // in the instruction cache.  False once every stage is closed.
    auto slow_path = [&]() -> bool {
      if (prod.pend) prod.fix();
      if (cons.pend) cons.fix();
      while (cons.s != cur) {
        flush();
        __syncthreads();   // [C] partials of stage cur are in red[]
        if (++cur >= n_stages) return false;
        __syncthreads();   // [A] input of stage cur in xbuf
        build(cplan[cur]);
        __syncthreads();   // [B]
      }
      return true;
    };
    // One item from ring slot `slot`; false (nothing done) when the slow
    // path has to run first.
    auto item = [&](u32x4 (&slot)[kChunks]) -> bool {
      if (cons.pend || prod.pend || cons.s != cur) return false;
      if (cons.row != cur_row) flush();
      cur_row = cons.row;
      int cj[kChunks];
      u32x4 xw[kChunks];
      float sc[kChunks];
#pragma unroll
      for (int c = 0; c < kChunks; ++c) {
        const int c0 = cons.seg * 64 * kChunks + 64 * c + lane;
        cj[c] = c0 < cons.nch ? c0 : cons.nch;   // past the row: the zero chunk
        xw[c] = *(const u32x4*)(act + cons.act_off + cj[c] * 8);
        sc[c] = csc[cons.csc_off + cj[c]];
      }
      ring_wait(slot);
      u32x2 t1l[kChunks][4], t2l[kChunks][4], t1h[kChunks][4], t2h[kChunks][4];
#pragma unroll
      for (int c = 0; c < kChunks; ++c) lookups(slot[c], tabB, t1l[c], t2l[c], t1h[c], t2h[c]);
#pragma unroll
      for (int c = 0; c < kChunks; ++c) accumulate(t1l[c], t2l[c], t1h[c], t2h[c], xw[c], sc[c], acc);
      prod.load(slot, lane);
      if (prod.s < n_stages) prod.advance_fast();
      cons.advance_fast();
      return true;
    };
    // The ring slots in item order; after the slow path, items resume at the
    // slot where they stopped.  The ring's registers are only read after
    // ring_wait and only written by the loads, so entering the loop at any
    // slot keeps every slot's load in flight.
    int phase = 0;
    for (;;) {
      switch (phase) {
#define EPTQ_SLOT(j)                                                  \
  case j:                                                             \
    if constexpr (j < kRing) {                                        \
      if (!item(ring[j < kRing ? j : 0])) {                           \
        phase = j;                                                    \
        break;                                                        \
      }                                                               \
      if (j == kRing - 1) {                                           \
        phase = -1;                                                   \
        break;                                                        \
      }                                                               \
    }                                                                 \
    [[fallthrough]];
        EPTQ_SLOT(0) EPTQ_SLOT(1) EPTQ_SLOT(2) EPTQ_SLOT(3) EPTQ_SLOT(4) EPTQ_SLOT(5) EPTQ_SLOT(6) EPTQ_SLOT(7)
#undef EPTQ_SLOT
        default:
          break;
      }
      if (phase < 0) {
        phase = 0;
        continue;
      }
      if (!slow_path()) break;
    }
  done:
    asm volatile("s_waitcnt vmcnt(0)");   // no ring load outlives the wave's registers
  } else {
    // --------------------------------------------------------------- sync
    const int st = tid;   // 0..255
    uint16_t gb[4];       // g, g, bias, bias of this thread's output pair (current stage)
    uint16_t gbn[4];      // the same for the next stage
    int e_cnt[kRowsPerSyncWave];
    int e_col[kRowsPerSyncWave];
    u32x4 e_o[kRowsPerSyncWave];
    int e_ptr[kRowsPerSyncWave];
    u32x4 hreg[kHRegs], wreg[kWRegs];
    bool err = false;

    // Layer of stage-row rg and its local row.
    auto layer_of = [&](CStage& S, int rg, int& lr) {
      const int l = (S.n_layers > 2 && rg >= S.l[2].row0) ? 2 : (S.n_layers > 1 && rg >= S.l[1].row0) ? 1 : 0;
      lr = rg - S.l[l].row0;
      return l;
    };
    // Row pointers of stage s's rows (one per sync wave row slot), left in
    // vector registers so that issuing them does not wait for them: they are
    // read one stage later, by fetch_meta.
    auto fetch_ptrs = [&](int s, int (&ptr0)[kRowsPerSyncWave], int (&ptr1)[kRowsPerSyncWave]) {
      CStage& S = cplan[s];
      int r0, rows;
      wg_rows(S.M_tot, r0, rows);
#pragma unroll
      for (int j = 0; j < kRowsPerSyncWave; ++j) {
        const int r = wave + kSyncW * j;
        ptr0[j] = ptr1[j] = 0;
        if (r < rows) {
          int lr;
          const int l = layer_of(S, r0 + r, lr);
          const int32_t* rp = S.l[l].O_row_ptr;
          ptr0[j] = gp(rp)[lr];
          ptr1[j] = gp(rp)[lr + 1];
        }
      }
    };
    // Everything else stage s needs that does not depend on its input: h, the
    // RMSNorm weight, g/bias of this thread's output pair, and the first 64
    // critical-block entries of each row (lane i: entry i).  Issued without
    // waiting; the registers are read at stage s.
    auto fetch_h = [&](int s) {
      CStage& S = cplan[s];
      const int nl = S.n_layers, N = S.N, nch = S.nch;
#pragma unroll
      for (int j = 0; j < kHRegs; ++j) {
        const int q = st + 256 * j;
        if (q < nl * nch) {
          const int l = q >= 2 * nch ? 2 : q >= nch ? 1 : 0;
          hreg[j] = *gp((const u32x4*)(S.l[l].h + (q - l * nch) * 8));
        }
      }
      if (S.prep) {
#pragma unroll
        for (int j = 0; j < kWRegs; ++j) {
          const int c = st + 256 * j;
          if (c < nch) wreg[j] = *gp((const u32x4*)(S.nw + c * 8));
        }
      }
    };
    auto fetch_meta = [&](int s, const int (&ptr0)[kRowsPerSyncWave], const int (&ptr1)[kRowsPerSyncWave]) {
      CStage& S = cplan[s];
      int r0, rows;
      wg_rows(S.M_tot, r0, rows);
      if (st < rows * 4) {
        int lr;
        const int l = layer_of(S, r0 + (st >> 2), lr);
        const int o = 8 * lr + 2 * (st & 3);
        gbn[0] = __builtin_bit_cast(uint16_t, gp(S.l[l].g)[o]);
        gbn[1] = __builtin_bit_cast(uint16_t, gp(S.l[l].g)[o + 1]);
        const f16* bs = S.l[l].bias;
        gbn[2] = bs ? __builtin_bit_cast(uint16_t, gp(bs)[o]) : 0;
        gbn[3] = bs ? __builtin_bit_cast(uint16_t, gp(bs)[o + 1]) : 0;
      }
#pragma unroll
      for (int j = 0; j < kRowsPerSyncWave; ++j) {
        const int r = wave + kSyncW * j;
        const int pa = __builtin_amdgcn_readfirstlane(ptr0[j]);
        e_cnt[j] = __builtin_amdgcn_readfirstlane(ptr1[j]) - pa;
        e_ptr[j] = pa;
        e_col[j] = 0;
        e_o[j] = (u32x4){0u, 0u, 0u, 0u};
        if (r < rows && lane < e_cnt[j]) {
          int lr;
          const int l = layer_of(S, r0 + r, lr);
          e_col[j] = gp(S.l[l].O_col)[pa + lane];
          e_o[j] = *gp((const u32x4*)(S.l[l].O + (size_t)(pa + lane) * 8));
        }
      }
    };
    // h and the RMSNorm weight of stage s into LDS (after stage s-1's tables are built).
    auto store_h = [&](int s) {
      CStage& S = cplan[s];
      const int nl = S.n_layers, nch = S.nch;
#pragma unroll
      for (int j = 0; j < kHRegs; ++j) {
        const int q = st + 256 * j;
        if (q < nl * nch) *(u32x4*)(hbuf + q * 8) = hreg[j];
      }
      if (S.prep) {
#pragma unroll
        for (int j = 0; j < kWRegs; ++j) {
          const int c = st + 256 * j;
          if (c < nch) *(u32x4*)(wbuf + c * 8) = wreg[j];
        }
      }
    };
    // Corrections of stage s: O·xh − c511·xh per critical block, into slot kCorrSlot.
    auto corrections = [&](int s) {
      CStage& S = cplan[s];
      const int N = S.N, nch = S.nch;
      int r0, rows;
      wg_rows(S.M_tot, r0, rows);
      const f16x4 t5 = tab[511 ^ 0x100];
#pragma unroll
      for (int j = 0; j < kRowsPerSyncWave; ++j) {
        const int r = wave + kSyncW * j;
        if (r >= rows) continue;
        int lr;
        const int l = layer_of(S, r0 + r, lr);
        const uint16_t* actl = act + l * (N + 8);
        const float* cscl = csc + l * (nch + 1);
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
        auto add = [&](int col, u32x4 ow) {
          const f16x8 o = __builtin_bit_cast(f16x8, ow);
          const int cc = (unsigned)col < (unsigned)N ? col : 0;
          const float xo = (float)__builtin_bit_cast(f16, actl[cc]) * cscl[cc >> 3];
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += (float)o[e] * xo - (float)t5[e & 3] * xo;
        };
        if (lane < e_cnt[j]) add(e_col[j], e_o[j]);
        for (int i = 64 + lane; i < e_cnt[j]; i += 64)
          add(gp(S.l[l].O_col)[e_ptr[j] + i], *gp((const u32x4*)(S.l[l].O + (size_t)(e_ptr[j] + i) * 8)));
        const int base = wave_reduce_halving<8>(acc);
        if (WaveReduceOut<8>::writer(lane)) red[r][kCorrSlot][base] = acc[0];
      }
    };
    // Poll stage s's input into xbuf (and the RMSNorm sum of squares).
    auto load_input = [&](int s) {
      CStage& S = cplan[s];
      const int N = S.N, nq = N >> 2;   // 16-byte loads of 4 inputs
      float ss = 0.0f;
      if (S.src < 0) {
        for (int q = st; q < nq; q += 256) {
          const u32x2 v = *gp((const u32x2*)(S.x + q * 4));
          *(u32x2*)(xbuf + q * 4) = v;
          const h2 a = as_h2(v[0]), b = as_h2(v[1]);
          ss += (float)a.x * (float)a.x + (float)a.y * (float)a.y + (float)b.x * (float)b.x + (float)b.y * (float)b.y;
        }
      } else {
        const unsigned want = flag_of(S.src);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(S.x_ll + (S.col >> 1)), (short)0, N * 4, kBufferWord3);
        for (int round = 0; round < 2; ++round) {
          const int q0 = st + 256 * kXRegs * round;
          u32x4 v[kXRegs];
          unsigned pending = 0;
#pragma unroll
          for (int j = 0; j < kXRegs; ++j)
            if (q0 + 256 * j < nq) pending |= 1u << j;
          for (int it = 0; pending; ++it) {
#pragma unroll
            for (int j = 0; j < kXRegs; ++j)
              if (pending & (1u << j))
                v[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (q0 + 256 * j) * 16, 0,
                                                                                        kCoherent));
#pragma unroll
            for (int j = 0; j < kXRegs; ++j) {
              if ((pending & (1u << j)) && v[j][1] == want && v[j][3] == want) {
                pending &= ~(1u << j);
                const int q = q0 + 256 * j;
                *(u32x2*)(xbuf + q * 4) = (u32x2){v[j][0], v[j][2]};
                const h2 a = as_h2(v[j][0]), b = as_h2(v[j][2]);
                ss += (float)a.x * (float)a.x + (float)a.y * (float)a.y + (float)b.x * (float)b.x +
                      (float)b.y * (float)b.y;
              }
            }
            if (!pending) break;
            if (it >= kSpinLimit || err) {
              __hip_atomic_store(sync + kErrorWord, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              err = true;
              break;
            }
            __builtin_amdgcn_s_sleep(2);
          }
        }
        // Another workgroup gave up: stop waiting for the rest of this launch.
        if (__builtin_amdgcn_readfirstlane((int)err)) err = true;
      }
      if (S.prep) {
        ss += partner<1>(ss);
        ss += partner<2>(ss);
        ss += partner<4>(ss);
        ss += partner<8>(ss);
        ss += partner<16>(ss);
        ss += partner<32>(ss);
        if (lane == 0) s_rms[wave] = ss;
      }
    };
    // Epilogue of stage s: partial sums + corrections, g, bias -> flagged output.
    auto epilogue = [&](int s) {
      CStage& S = cplan[s];
      int r0, rows;
      wg_rows(S.M_tot, r0, rows);
      if (st < rows * 4) {
        const int r = st >> 2, k0 = 2 * (st & 3);
        float2 v[kSlots];
#pragma unroll
        for (int kk = 0; kk <= kCorrSlot; ++kk) v[kk] = *(const float2*)&red[r][kk][k0];
        // Slots of waves that held no part of the row are zero: every
        // epilogue clears the compute slots it read.
#pragma unroll
        for (int kk = 0; kk < kCompW; ++kk) *(float2*)&red[r][kk][k0] = make_float2(0.0f, 0.0f);
        float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
        for (int kk = 0; kk <= kCorrSlot; ++kk) {
          v0 += v[kk].x;
          v1 += v[kk].y;
        }
        const float o0 = v0 * (float)__builtin_bit_cast(f16, gb[0]) + (float)__builtin_bit_cast(f16, gb[2]);
        const float o1 = v1 * (float)__builtin_bit_cast(f16, gb[1]) + (float)__builtin_bit_cast(f16, gb[3]);
        const uint32_t pr = __builtin_bit_cast(uint32_t, (h2){(f16)o0, (f16)o1});
        const size_t w = (size_t)(r0 + r) * 4 + (st & 3);
        const uint64_t word = (uint64_t)pr | ((uint64_t)flag_of(s) << 32);
        __hip_atomic_store(S.y_ll + w, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (S.y) *(uint32_t*)(S.y + 2 * w) = pr;
      }
    };

    // Prefetch pipeline: during stage s the sync waves issue stage s+1's
    // data (h, g/bias, entries, with the row pointers fetched during stage
    // s-1) and stage s+2's row pointers, and wait for none of it before [C].
    int pa0[kRowsPerSyncWave], pa1[kRowsPerSyncWave], pb0[kRowsPerSyncWave], pb1[kRowsPerSyncWave];
    fetch_ptrs(0, pa0, pa1);
    fetch_meta(0, pa0, pa1);
    if (n_stages > 1) fetch_ptrs(1, pb0, pb1);
#pragma unroll
    for (int e = 0; e < 4; ++e) gb[e] = gbn[e];
    fetch_h(0);
    load_input(0);
    store_h(0);
    __syncthreads();   // [A] stage 0
    build(cplan[0]);
    __syncthreads();   // [B]
    for (int s = 0;; ++s) {
      corrections(s);
      const bool more = s + 1 < n_stages;
      if (more) {
        // Stage s+1's g/bias and entries (row pointers fetched a stage ago)
        // and stage s+2's row pointers: issued, not waited for.
        fetch_meta(s + 1, pb0, pb1);
        if (s + 2 < n_stages) {
          fetch_ptrs(s + 2, pa0, pa1);
#pragma unroll
          for (int j = 0; j < kRowsPerSyncWave; ++j) {
            pb0[j] = pa0[j];
            pb1[j] = pa1[j];
          }
        }
      }
      __syncthreads();   // [C] stage s
      epilogue(s);
      if (!more) break;
#pragma unroll
      for (int e = 0; e < 4; ++e) gb[e] = gbn[e];
      // h of stage s+1 is requested before the input poll, which waits for it.
      fetch_h(s + 1);
      load_input(s + 1);
      store_h(s + 1);
      __syncthreads();   // [A] stage s+1
      build(cplan[s + 1]);
      __syncthreads();   // [B]
    }
    // The last workgroup out advances the epoch for the next launch.
    if (tid == 0 &&
        __hip_atomic_fetch_add(sync + kExitWord, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (int)gridDim.x - 1) {
      __hip_atomic_store(sync + kExitWord, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(sync + kEpochWord, (int)(epoch + 1u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace step

// Host side -----------------------------------------------------------------

namespace {
constexpr size_t kStaticLds = 512 * 8 + step::kRowsMax * step::kSlots * 8 * 4 + 64;
constexpr size_t kLdsCu = 160 * 1024;
size_t up16(size_t v) { return (v + 15) & ~(size_t)15; }
}  // namespace

// Dynamic LDS layout for the plan's largest stage sizes; 0 when it does not fit.
size_t step_lds_layout(int n, const step::Stage* h_stages, int* off /* 4 ints */) {
  size_t X = 0, H = 0, W = 0, A = 0, C = 0;
  for (int s = 0; s < n; ++s) {
    const step::Stage& S = h_stages[s];
    X = X > (size_t)(S.N + 8) * 2 ? X : (size_t)(S.N + 8) * 2;
    H = H > (size_t)S.n_layers * S.N * 2 ? H : (size_t)S.n_layers * S.N * 2;
    if (S.prep) W = W > (size_t)S.N * 2 ? W : (size_t)S.N * 2;
    A = A > (size_t)S.n_layers * (S.N + 8) * 2 ? A : (size_t)S.n_layers * (S.N + 8) * 2;
    C = C > (size_t)S.n_layers * (S.nch + 1) * 4 ? C : (size_t)S.n_layers * (S.nch + 1) * 4;
  }
  off[0] = (int)up16(X);
  off[1] = off[0] + (int)up16(H);
  off[2] = off[1] + (int)up16(W);
  off[3] = off[2] + (int)up16(A);
  const size_t total = (size_t)off[3] + up16(C);
  return kStaticLds + total <= kLdsCu ? total : 0;
}

int step_check_stage(const step::Stage& S, int* why) {
  using step::kChunks;
  using step::kT;
  // Limits of the kernel's fixed register and LDS budgets.
  if (S.n_layers < 1 || S.n_layers > step::kMaxStageLayers) return *why = 1, -1;
  if (S.N % 8 || S.nch != S.N / 8 || S.nseg != (S.nch + 64 * kChunks - 1) / (64 * kChunks)) return *why = 2, -1;
  if (S.n_layers * S.nch > 2 * kT) return *why = 6, -1;
  if (S.n_layers * S.nch > step::kHRegs * 256) return *why = 3, -1;
  if (S.prep && S.nch > step::kWRegs * 256) return *why = 4, -1;
  if (S.N > 2 * step::kXRegs * 256 * 4) return *why = 5, -1;
  return 0;
}

int step_grid() { return dec::cu_count(); }

int step_launch(const step::Stage* d_plan, int n, int* sync, const void* codes, const int* off, size_t dyn,
                hipStream_t s) {
  step::Offs o{off[0], off[1], off[2], off[3]};
  static bool attr = false;
  if (!attr) {
    if (hipFuncSetAttribute((const void*)step::k_step_b1, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)(kLdsCu - kStaticLds)) != hipSuccess)
      return -1;
    attr = true;
  }
  step::k_step_b1<<<step_grid(), step::kT, dyn, s>>>(d_plan, n, sync, (const f16x4*)codes, o);
  return 0;
}

int step_occupancy(size_t dyn) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void*)step::k_step_b1, step::kT, dyn) != hipSuccess)
    return 0;
  return n;
}

}  // namespace eptq

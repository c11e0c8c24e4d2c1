// One layer of the E8-D4 decode matvec (batch 1..8) as seen by one workgroup
// of the one-launch-per-layer kernels (decode.hip).
//
// Same result as the reference decode kernels (csrc/eptq_kernels.cu:161-292,
// kernels/triton_e8d4.py:47-157): y = g ⊙ (decode(Q)·(h ⊙ S ⊙ x)ᵀ + CSR(O)) + bias.
//
// Work split.  A workgroup is 4 waves; S waves (1, 2 or 4) share a Q-row, so
// a workgroup works on R = 4/S adjacent rows at a time and walks row groups
// wg, wg+G, wg+2G, ...  Lane `lane` of segment wave `seg` owns the 16-byte
// column chunks c = seg·64 + lane + 64·S·j (j < J) of every row, so the
// activation side (x·h) is prepared once per workgroup in LDS and the E8-D4
// table is staged in LDS once.  Whole-row waves (S = 1) need no cross-wave
// reduction and no barrier; S > 1 combines the S partial sums through LDS
// with one barrier per row group.  The index chunks of the next P row groups
// are kept in flight in a register ring of 8 chunks (128 bytes per lane) so
// HBM latency is covered.
//
// Arithmetic:
//  * B = 1: x·h is formed in fp32 and stored in fp16 scaled per chunk of 8
//    columns by a power of two 2^-e with max|x·h|·2^-e in [0.5, 1); packed
//    fp16 FMAs accumulate a chunk (two rows per op), and one mixed-precision
//    FMA per row moves the chunk sum into fp32 times 2^e.
//  * B >= 2 (bf16 x taken to fp16 first, exactly in fp16's normal range):
//    the two indices of a 32-bit word (adjacent columns) are paired:
//    byte permutes turn their two table vectors into (c_k(n), c_k(n+1)) fp16
//    pairs and one v_dot2_f32_f16 per (k, b) accumulates both columns in
//    fp32.  The activation pairs x·h are rounded to fp16 after scaling h by a
//    workgroup-uniform power of two 2^-e with max|h|·2^-e <= 1, so |x·h·2^-e|
//    <= |x| cannot overflow; 2^e is restored in fp32 at the output.  With
//    S_group the pairs are multiplied by the row group's scales in fp16.
//
// Index decode from the raw int16 bits v, with the LDS table stored at
// position e ^ 0x100 for table row e (u = v ^ 0x8000 needs no fix-up):
//   rows 0..3 of the block: byte address (v >> 4) & 0xFF8
//   rows 4..7:              same bits 10-11, bits 3-9 = (v & 127) << 3.
// Critical blocks (v = 32767) decode as table row 511 in both halves; the
// CSR pass adds O·(h x) minus exactly what the main loop accumulated for them.
#pragma once

#include "common.h"
#include "kernels.h"

namespace eptq {
namespace dec {

constexpr int kT = 256;                    // threads per workgroup
constexpr int kW = kT / 64;                // waves per workgroup
constexpr int kBufferWord3 = 0x00020000;   // buffer resource word 3 (gfx9 family)
constexpr int kNonTemporal = 2;            // buffer load cache policy: nt
constexpr int kRing = 8;                   // index chunks in flight per lane

typedef f16 h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
}

// By value: __builtin_bit_cast applied directly to a vector-element lvalue
// (v[1], v.y) reads element 0 with this compiler.
__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }

// acc + (float)(lo or hi half of a packed fp16 pair) · s, one mixed-precision FMA.
__device__ __forceinline__ float fma_lo(uint32_t p, float s, float acc) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(p), "v"(s), "v"(acc));
  return r;
}
__device__ __forceinline__ float fma_hi(uint32_t p, float s, float acc) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(p), "v"(s), "v"(acc));
  return r;
}

__device__ __forceinline__ uint32_t pk_mul(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) * __builtin_bit_cast(h2, b));
}

// A layer pointer as a global-memory pointer.  A generic pointer (one the
// compiler cannot place in the global address space) is accessed with flat
// instructions, which count on both vmcnt and lgkmcnt and make every wait a
// full one.
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gp(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}

__device__ __forceinline__ void store_y(uint16_t* p, uint16_t v) { *gp(p) = v; }

// Dynamic LDS of the activation side: BT padded fp16 rows, plus the per-chunk
// scales for B = 1.
__host__ __device__ inline size_t act_lds_bytes(int N, int BT) {
  return (size_t)BT * (N + 8) * 2 + (BT == 1 ? (size_t)((N >> 3) + 1) * 4 : 0);
}

// Host side of the launch shape.
int cu_count();   // compute units of the current device

// Chunks per lane for a row split S ways (0 if beyond the kernel's range).
inline int chunks_for(int nch, int S) {
  const int j = (nch + 64 * S - 1) / (64 * S);
  if (j <= 2) return 2;
  if (j <= 4) return 4;
  if (j <= 8) return 8;
  return 0;
}

constexpr size_t kActLdsMax = 64 * 1024;   // activation table limit per workgroup
constexpr size_t kLdsPerCu = 160 * 1024;

inline bool fits(int J, int N, int BT) { return J > 0 && act_lds_bytes(N, BT) <= kActLdsMax; }

// LDS shared by the layer code of one workgroup.
template <int BT>
struct Smem {
  f16x4* tab;                  // [512], row e at e ^ 0x100
  float (*red)[kW][BT * 8];    // [2][kW][V] cross-wave partial sums (S > 1)
  float* wmax;                 // [kW]
  uint16_t* xs;                // [BT][N + 8] activation table
  float* csc;                  // [N/8 + 1] chunk scales (B = 1)
};

// State a workgroup carries from the prefetch of its first row groups into
// the row loop: the index ring (slot p·K + j = chunk j of the p-th row group
// ahead), critical-block entry ranges of this and the next row group, this
// lane's first-pass entry and the epilogue operands of this thread's output.
struct RowState {
  u32x4 ring[kRing];
  int crb, cre, nrb, nre;
  int ecol;
  u32x4 eo;
  f16 og, ob;
};

// Where one workgroup's work lies in a layer split S ways with J chunks per
// lane: the row groups wg, wg + G, ...  (Runtime fields; with compile-time S
// and J the arithmetic folds away.)
struct Walk {
  const LinearArgs& a;
  int wg, G, S, J, K, R, slot, seg, lane, tid, V;
  bool strided;

  // pair: the workgroup serves two layers of equal shape (SwiGLU gate and
  // up), wave w layer w % 2 at row slot w / 2 (S = 1): R = 2 rows per layer.
  // strided (the single-row-group form): the workgroup's one row group is
  // rows wg, wg + G, wg + 2G, ... (one per row slot), so G may exceed the
  // number of row groups: rows then spread evenly over the workgroups.
  __device__ __forceinline__ Walk(const LinearArgs& a_, int wg_, int G_, int S_, int J_, int V_, bool pair = false,
                                  bool strided_ = false)
      : a(a_), wg(wg_), G(G_), S(S_), J(J_), K(J_ > 4 ? 4 : J_), R(pair ? kW / S_ / 2 : kW / S_),
        slot(pair ? (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) / S_) >> 1
                  : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) / S_),
        seg(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) % S_), lane(threadIdx.x & 63),
        tid(threadIdx.x), V(V_), strided(strided_) {}

  // The row of row slot sl in row group rg.
  __device__ __forceinline__ int row_of(int rg, int sl) const { return strided ? sl * G + rg : rg * R + sl; }

  __device__ __forceinline__ int chunk(int j) const { return seg * 64 + lane + 64 * S * j; }

  // Critical-block rows [rb, re) of O_col/O for this wave's row of row group
  // rg; rows past the end give an empty range.  Vector loads (the values are
  // wave-uniform): a scalar load would share lgkmcnt with the LDS lookups,
  // and since scalar loads complete out of order every LDS wait would also
  // wait for it.
  __device__ __forceinline__ void row_range(int rg, int& rb, int& re) const {
    const int M = a.M;
    const int row = row_of(rg, slot);          // wave-uniform
    const int rr = row < M ? row : M - 1;
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.O_row_ptr, (short)0, (M + 1) * 4, kBufferWord3);
    // Both pointers in one load instruction; rows past M: the empty range at
    // the end.
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(rp, rr * 4, 0, 0);
    rb = (int)(row < M ? v[0] : v[1]);
    re = (int)v[1];
  }

  // Index chunks are read through a buffer resource spanning one row (an
  // empty one past the last row): out-of-range chunks read as zero, so the
  // loads need no branches or clamps, and the compiler can wait for exactly
  // the load it needs (vmcnt counts loads in issue order).
  __device__ __forceinline__ void load_chunk(u32x4& dst, int rg, int j) const {
    const int M = a.M, N = a.N;
    const int row = row_of(rg, slot);         // wave-uniform
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.Q + (size_t)(row < M ? row : 0) * N), (short)0, row < M ? N * 2 : 0, kBufferWord3);
    dst = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, chunk(j) * 16, 0, kNonTemporal));
  }

  // Critical blocks, first 64·S entries of a row: lane `ent` of the row's S
  // waves holds entry rb + ent (its column and O vector).  Buffer resources
  // span exactly the row's entries, so lanes past the end read zeros.
  __device__ __forceinline__ void load_entries(RowState& st, int rb_v, int re_v) const {
    const int ent = seg * 64 + lane;
    const int rb = __builtin_amdgcn_readfirstlane(rb_v);
    const int cnt = __builtin_amdgcn_readfirstlane(re_v) - rb;
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.O_col + rb), (short)0, cnt * 4, kBufferWord3);
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.O + (size_t)rb * 8), (short)0, cnt * 16, kBufferWord3);
    st.ecol = (int)__builtin_amdgcn_raw_buffer_load_b32(rc, ent * 4, 0, 0);
    st.eo = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, ent * 16, 0, 0));
  }

  // The output row this thread writes for row group rg, and its (batch row,
  // row-in-block) position.
  __device__ __forceinline__ int out_row(int rg) const {
    return S == 1 ? row_of(rg, slot) : row_of(rg, tid < R * V ? tid / V : 0);
  }
  template <int VV>
  __device__ __forceinline__ int wbase() const {
    return S == 1 ? reduce_base<VV>(lane) : (tid < R * VV ? tid % VV : 0);
  }
  // g and bias of this thread's output in row group rg (rows past the end
  // read the last row; bias through a resource that is empty when null).
  template <int VV>
  __device__ __forceinline__ void load_epilogue(int rg, f16& og, f16& ob) const {
    const int M = a.M;
    const int orow = out_row(rg);
    const int oidx = 8 * (orow < M ? orow : M - 1) + (wbase<VV>() & 7);
    const __amdgpu_buffer_rsrc_t rbias = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.bias, (short)0, a.bias ? 16 * M : 0, kBufferWord3);
    og = gp(a.g)[oidx];
    ob = __builtin_bit_cast(f16, (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rbias, oidx * 2, 0, 0));
  }

  // Entry ranges of the first two row groups (issued early: the entry loads
  // need them); ONE: the workgroup has one row group.
  template <bool ONE>
  __device__ __forceinline__ void rows_first(RowState& st) const {
    row_range(wg, st.crb, st.cre);
    if (ONE) st.nrb = st.nre = 0;
    else row_range(wg + G, st.nrb, st.nre);
  }

  // Index chunks in flight: K of each of the kRing/K row groups of the ring,
  // then the first row group's critical-block entries and epilogue operands.
  // ONE: the workgroup has one row group; only its first K chunks.  (The
  // entry and bias loads stay unconditional: a load skipped on one path
  // merges with a constant on the other, and the compiler waits for every
  // load in flight at that merge.)
  template <int VV, bool ONE>
  __device__ __forceinline__ void issue_ring(RowState& st) const {
#pragma unroll
    for (int k = 0; k < (ONE ? K : kRing); ++k) {
      const int p = K == 4 ? k >> 2 : K == 2 ? k >> 1 : k;
      const int j = k - p * K;
      load_chunk(st.ring[k], wg + p * G, j);
    }
    load_entries(st, st.crb, st.cre);
    load_epilogue<VV>(wg, st.og, st.ob);
  }
};

// PAIR (S = 1): two layers of equal shape in one workgroup, wave w computing
// layer w % 2 (gate, up) at row slot w / 2; the output is the SwiGLU product
// silu(gate) ⊙ up, each factor rounded to the activation type first, as the
// unfused Linear outputs are.
// ONE: every workgroup has exactly one row group (G = RG), so nothing is
// prefetched for a next one.  Every load instruction costs the CU's address
// unit the same time whether it reads memory or falls past its buffer, so
// the general form's look-ahead loads (ring slots, entry ranges, entries and
// epilogue operands of row groups that do not exist) are not free.
template <int BT, int J, int P, int S, bool HAS_S, typename XT, bool PAIR = false, bool ONE = false>
struct Layer {
  static constexpr int V = BT * 8;
  static constexpr int R = PAIR ? kW / S / 2 : kW / S;   // rows per row group (per layer)
  static_assert(!PAIR || S == 1, "pairs: whole-row waves, one launch per layer pair");
  static constexpr int K = J > 4 ? 4 : J;                 // chunks of a row in flight
  static_assert(P * K == kRing, "the ring holds kRing chunks");
  static_assert(J % K == 0, "chunks per row must be a multiple of the chunks in flight");
  static_assert(V <= 64 && R * V <= kT, "one output per thread after the reduction");
  // Activation chunks per thread (>= ceil(nch / kT)), the first CAP loaded together.
  static constexpr int CA = (J * S) / 4 < 1 ? 1 : (J * S) / 4;
  static constexpr int CAP = CA < 18 / (BT + 1) ? CA : 18 / (BT + 1);

  using State = RowState;

  const LinearArgs& a;
  const int wg, G;
  const int tid, lane, wave, slot, seg;
  const int N, M, B, nch, NP, RG;
  const Walk w;

  __device__ __forceinline__ Layer(const LinearArgs& a_, int wg_, int G_)
      : a(a_), wg(wg_), G(G_), tid(threadIdx.x), lane(threadIdx.x & 63),
        wave(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)), slot(PAIR ? (wave / S) >> 1 : wave / S),
        seg(wave % S), N(a_.N), M(a_.M), B(a_.B), nch(a_.N >> 3), NP(a_.N + 8), RG((a_.M + R - 1) / R),
        w(a_, wg_, G_, S, J, V, PAIR, ONE) {}

  __device__ __forceinline__ int chunk(int j) const { return w.chunk(j); }
  __device__ __forceinline__ void rows_first(State& st) const { w.template rows_first<ONE>(st); }
  __device__ __forceinline__ void issue_ring(State& st) const { w.template issue_ring<V, ONE>(st); }

  // The activation table x·h (scaled) into LDS; returns the output scale.
  // The loads are issued first (h and x rows through buffer resources whose
  // offsets past the end read zero), then the LDS table is written.  Needs a
  // barrier before the row loop reads it.  With a.prep == 1 the Linear's
  // input is formed here first: the RMSNorm of a residual sum (see
  // LinearArgs).  TWO: a second table from the same x and a second h (hup)
  // into sm2, its output scale into *out_scale2 (the layer pair's up side).
  template <bool TWO = false>
  __device__ __forceinline__ float build_act(const Smem<BT>& sm, const f16* hup = nullptr,
                                             const Smem<BT>* sm2 = nullptr, float* out_scale2 = nullptr) const {
    uint16_t* __restrict__ xs = sm.xs;
    float* __restrict__ csc = sm.csc;
    const int prep = a.prep, ldx = a.ldx;
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc((void*)a.h, (short)0, N * 2, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rh2 =
        __builtin_amdgcn_make_buffer_rsrc((void*)hup, (short)0, TWO ? N * 2 : 0, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, B * ldx * 2, kBufferWord3);
    // The residual delta (prep 1; an empty resource when absent).
    const __amdgpu_buffer_rsrc_t r2 = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.x2, (short)0, prep == 1 && a.x2 ? B * ldx * 2 : 0, kBufferWord3);
    auto load_hx = [&](int c, u32x4& hw, u32x4 (&xw)[BT], u32x4 (&dw)[BT]) {
      const bool cv = c < nch;
      hw = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rh, cv ? c * 16 : N * 2, 0, 0));
#pragma unroll
      for (int b = 0; b < BT; ++b)
        xw[b] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
            rx, cv && b < B ? b * ldx * 2 + c * 16 : B * ldx * 2, 0, 0));
      if (prep != 0) {
#pragma unroll
        for (int b = 0; b < BT; ++b)
          dw[b] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
              r2, cv && b < B ? b * ldx * 2 + c * 16 : B * ldx * 2, 0, 0));
      }
    };
    u32x4 hpre[CAP], xpre[CAP][BT], dpre[CAP][BT];
#pragma unroll
    for (int k = 0; k < CAP; ++k) load_hx(tid + kT * k, hpre[k], xpre[k], dpre[k]);
    u32x4 h2pre[TWO ? CAP : 1];
    auto load_h2 = [&](int c) {
      return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rh2, c < nch ? c * 16 : N * 2, 0, 0));
    };
    if constexpr (TWO) {
#pragma unroll
      for (int k = 0; k < CAP; ++k) h2pre[k] = load_h2(tid + kT * k);
    }
    if (prep == 1) {
      // r = fp16(x + x2) (every chunk is among the first CAP: the launch
      // checks N <= CAP·kT·8), sum of squares per batch row, then
      // fp16(r · rsqrt(mean + eps) · w).
      const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)a.nw, (short)0, N * 2, kBufferWord3);
      u32x4 wpre[CAP];
#pragma unroll
      for (int k = 0; k < CAP; ++k) {
        const int c = tid + kT * k;
        wpre[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, c < nch ? c * 16 : N * 2, 0, 0));
      }
      float ss[BT];
#pragma unroll
      for (int b = 0; b < BT; ++b) ss[b] = 0.0f;
#pragma unroll
      for (int k = 0; k < CAP; ++k) {
        const int c = tid + kT * k;
#pragma unroll
        for (int b = 0; b < BT; ++b) {
          const f16x8 xv = __builtin_bit_cast(f16x8, xpre[k][b]), dv = __builtin_bit_cast(f16x8, dpre[k][b]);
          f16x8 r;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            r[e] = (f16)((float)xv[e] + (float)dv[e]);
            ss[b] += (float)r[e] * (float)r[e];
          }
          xpre[k][b] = __builtin_bit_cast(u32x4, r);
          if (blockIdx.x == 0 && blockIdx.y == 0 && a.xsum && c < nch && b < B)
            *gp((u32x4*)(a.xsum + (size_t)b * N + c * 8)) = xpre[k][b];
        }
      }
      // Workgroup sums of the BT rows (LDS partials of the 4 waves).
#pragma unroll
      for (int b = 0; b < BT; ++b) {
        float v = ss[b];
        v += partner<1>(v);
        v += partner<2>(v);
        v += partner<4>(v);
        v += partner<8>(v);
        v += partner<16>(v);
        v += partner<32>(v);
        if (lane == 0) sm.red[0][wave][b] = v;
      }
      __syncthreads();
      float inv[BT];
#pragma unroll
      for (int b = 0; b < BT; ++b) {
        float t = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < kW; ++w2) t += sm.red[0][w2][b];
        inv[b] = rsqrtf(t / (float)N + a.eps);
      }
      __syncthreads();   // red[] is reused by the row loop
#pragma unroll
      for (int k = 0; k < CAP; ++k) {
        const f16x8 wv = __builtin_bit_cast(f16x8, wpre[k]);
#pragma unroll
        for (int b = 0; b < BT; ++b) {
          const f16x8 r = __builtin_bit_cast(f16x8, xpre[k][b]);
          f16x8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (f16)((float)r[e] * inv[b] * (float)wv[e]);
          xpre[k][b] = __builtin_bit_cast(u32x4, o);
        }
      }
    }
    // Chunks past the first CAP (wide layers, prep 0), one at a time.
    auto load_more = [&](int c, u32x4& hw, u32x4 (&xw)[BT]) {
      u32x4 dw[BT];
      load_hx(c, hw, xw, dw);
    };

    float out_scale = 1.0f;
    if constexpr (TWO) *out_scale2 = 1.0f;
    if (tid == 0) {   // the zero chunk past the end of every row
#pragma unroll
      for (int b = 0; b < BT; ++b) *(u32x4*)(xs + b * NP + nch * 8) = (u32x4){0u, 0u, 0u, 0u};
      if (BT == 1) csc[nch] = 1.0f;
      if constexpr (TWO) {
#pragma unroll
        for (int b = 0; b < BT; ++b) *(u32x4*)(sm2->xs + b * NP + nch * 8) = (u32x4){0u, 0u, 0u, 0u};
        if (BT == 1) sm2->csc[nch] = 1.0f;
      }
    }
    if constexpr (BT == 1) {
      // Per chunk of 8 columns: xs = fp16(x·h·2^-e), csc = 2^e with
      // max|x·h|·2^-e in [0.5, 1), so the fp16 accumulation of a chunk (|c| < 2,
      // 8 columns) cannot overflow; the main loop applies 2^e in fp32.
      auto prep = [&](uint16_t* __restrict__ xsd, float* __restrict__ cscd, int c, const u32x4 hw, const u32x4 xw) {
        const f16x8 hv = __builtin_bit_cast(f16x8, hw);
        const u16x8 xv = __builtin_bit_cast(u16x8, xw);
        float xf[8], mx = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xf[e] = Act<XT>::mul_f16(xv[e], hv[e]);
          mx = fmaxf(mx, fabsf(xf[e]));
        }
        const int ex = mx > 0.0f ? (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xff) - 126 : 0;
        const float down = __builtin_ldexpf(1.0f, -ex);
        u32x4 w;
#pragma unroll
        for (int d = 0; d < 4; ++d)
          w[d] = __builtin_bit_cast(uint32_t, (h2){(f16)(xf[2 * d] * down), (f16)(xf[2 * d + 1] * down)});
        if (c < nch) {
          *(u32x4*)(xsd + c * 8) = w;
          cscd[c] = __builtin_ldexpf(1.0f, ex);
        }
      };
#pragma unroll
      for (int k = 0; k < CAP; ++k) {
        prep(xs, csc, tid + kT * k, hpre[k], xpre[k][0]);
        if constexpr (TWO) prep(sm2->xs, sm2->csc, tid + kT * k, h2pre[k], xpre[k][0]);
      }
      for (int c = tid + kT * CAP; c < nch; c += kT) {
        u32x4 hw, xw[BT];
        load_more(c, hw, xw);
        u32x4 hw2 = hw;
        if constexpr (TWO) hw2 = load_h2(c);
        prep(xs, csc, c, hw, xw[0]);
        if constexpr (TWO) prep(sm2->xs, sm2->csc, c, hw2, xw[0]);
      }
    } else {
      // Workgroup-uniform power-of-two scale with max|h|·2^-e <= 1, so the fp16
      // pairs |x·h·2^-e| <= |x| cannot overflow (dot2 accumulates in fp32).
      float mx = 0.0f, mx2 = 0.0f;
      auto hmax = [&](float& m, const u32x4 hw) {
        const f16x8 hv = __builtin_bit_cast(f16x8, hw);
#pragma unroll
        for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf((float)hv[e]));
      };
#pragma unroll
      for (int k = 0; k < CAP; ++k) {
        hmax(mx, hpre[k]);
        if constexpr (TWO) hmax(mx2, h2pre[k]);
      }
      for (int c = tid + kT * CAP; c < nch; c += kT) {
        hmax(mx, __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rh, c * 16, 0, 0)));
        if constexpr (TWO) hmax(mx2, load_h2(c));
      }
      auto wave_max = [&](float m) {
        m = fmaxf(m, partner<1>(m));
        m = fmaxf(m, partner<2>(m));
        m = fmaxf(m, partner<4>(m));
        m = fmaxf(m, partner<8>(m));
        m = fmaxf(m, partner<16>(m));
        return fmaxf(m, partner<32>(m));
      };
      mx = wave_max(mx);
      if (lane == 0) sm.wmax[wave] = mx;
      if constexpr (TWO) {
        mx2 = wave_max(mx2);
        if (lane == 0) sm2->wmax[wave] = mx2;
      }
      __syncthreads();
      // Workgroup-uniform scale 2^ex >= max|h| (ex = 0 when max|h| <= 1).
      auto scale_of = [&](const float* wm, float& osc) {
        const float m = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
        int ex = 0;
        if (m > 1.0f) ex = (int)((__builtin_bit_cast(uint32_t, m) >> 23) & 0xff) - 126;
        osc = __builtin_ldexpf(1.0f, ex);
        const f16 down = (f16)__builtin_ldexpf(1.0f, -ex);
        return __builtin_bit_cast(uint32_t, (h2){down, down});
      };
      const uint32_t down2 = scale_of(sm.wmax, out_scale);
      uint32_t down2b = down2;
      if constexpr (TWO) down2b = scale_of(sm2->wmax, *out_scale2);
      auto prep = [&](uint16_t* __restrict__ xsd, uint32_t dn, int c, const u32x4 hw, const u32x4 (&xw)[BT]) {
        if (c < nch) {
#pragma unroll
          for (int b = 0; b < BT; ++b) {
            u32x4 w;
#pragma unroll
            for (int d = 0; d < 4; ++d) w[d] = pk_mul(to_f16x2<XT>(xw[b][d]), pk_mul(hw[d], dn));
            *(u32x4*)(xsd + b * NP + c * 8) = w;
          }
        }
      };
#pragma unroll
      for (int k = 0; k < CAP; ++k) {
        prep(xs, down2, tid + kT * k, hpre[k], xpre[k]);
        if constexpr (TWO) prep(sm2->xs, down2b, tid + kT * k, h2pre[k], xpre[k]);
      }
      for (int c = tid + kT * CAP; c < nch; c += kT) {
        u32x4 hw, xw[BT];
        load_more(c, hw, xw);
        prep(xs, down2, c, hw, xw);
        if constexpr (TWO) prep(sm2->xs, down2b, c, load_h2(c), xw);
      }
    }
    return out_scale;
  }

  // The row groups of this workgroup, starting from the state the ring and
  // entry prefetch left.  The LDS table and activation table must be ready.
  // PAIR: pairx is LDS for the up side's outputs, [2][2][64].
  __device__ __forceinline__ void rows(State& st, const Smem<BT>& sm, float out_scale,
                                       uint16_t (*pairx)[2][64] = nullptr) const {
    const char* __restrict__ tabB = (const char*)sm.tab;
    const uint16_t* __restrict__ xs = sm.xs;
    const float* __restrict__ csc = sm.csc;
    const int ent = seg * 64 + lane;
    // Marker vector as the main loop sees it.
    const f16x4 t5 = sm.tab[511 ^ 0x100];
    // The output (batch row, block row) this thread writes after the reduction.
    const int wbase = w.wbase<V>();
    const int wb = wbase >> 3, wk = wbase & 7;

    int par = 0;
    // ONE: exactly one pass, rg = wg (its rows wg + G·slot).
    for (int rg0 = wg; ONE ? rg0 == wg : rg0 < RG; rg0 += P * G) {
#pragma unroll
    for (int p = 0; p < (ONE ? 1 : P); ++p) {
      const int rg = rg0 + p * G;
      if (!ONE && rg >= RG) break;               // uniform across the workgroup
      const int m = w.row_of(rg, slot);
      const bool row_ok = m < M;
      const int grp = HAS_S ? (8 * (row_ok ? m : 0)) / a.qb : 0;

      // Epilogue operands: this row group's (loaded a row group ago), and the
      // next one's.
      const int orow = w.out_row(rg);
      const f16 og = st.og, ob = st.ob;
      if (!ONE) w.load_epilogue<V>(rg + G, st.og, st.ob);
      // Row pointers two row groups ahead (their entries are loaded next).
      int frb = 0, fre = 0;
      if (!ONE) w.row_range(rg + 2 * G, frb, fre);
      // S at the critical blocks' columns (grouped layers), issued part-way
      // through the chunk loop once the entry columns have arrived.
      f16 gs = (f16)1.0f;
      auto load_gather = [&]() {
        if constexpr (HAS_S) {
          const int col = (unsigned)st.ecol < (unsigned)N ? st.ecol : 0;
          gs = gp(a.S)[(size_t)grp * N + col];
        }
      };

      float acc[V];
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = 0.0f;

#pragma unroll
      for (int j = 0; j < J; ++j) {
        const bool live = seg * 64 + 64 * S * j < nch;   // uniform: some lane has this chunk
        if (j == J / 2) load_gather();
        const int cj = chunk(j) < nch ? chunk(j) : nch;   // past the end: the zero chunk
        f16x8 sv;
        u32x4 xw[BT];
        // All 16 table lookups of the chunk first, then the arithmetic, so the
        // LDS latency is paid once per chunk rather than once per word.
        u32x2 t1l[4], t2l[4], t1h[4], t2h[4];
        if (live) {
          if (HAS_S) sv = *gp((const f16x8*)(a.S + (size_t)grp * N + ((cj < nch ? cj : 0) << 3)));
#pragma unroll
          for (int b = 0; b < BT; ++b) xw[b] = *(const u32x4*)(xs + b * NP + cj * 8);
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const uint32_t q = st.ring[p * K + j % K][d];
            const uint32_t q4 = q >> 4;
            const uint32_t a1lo = q4 & 0xFF8u;
            const uint32_t a1hi = hi_addr(q4);   // (q >> 20) & 0xFF8
            const uint32_t a2lo = bfi(0x3F8u, q << 3, a1lo);
            const uint32_t a2hi = bfi(0x3F8u, q >> 13, a1hi);
            t1l[d] = *(const u32x2*)(tabB + a1lo);
            t2l[d] = *(const u32x2*)(tabB + a2lo);
            t1h[d] = *(const u32x2*)(tabB + a1hi);
            t2h[d] = *(const u32x2*)(tabB + a2hi);
          }
        }
        // Refill this chunk's ring slot: the chunk K ahead in the same row,
        // else the matching chunk of the row group P·G ahead.
        if (j + K < J) w.load_chunk(st.ring[p * K + j % K], rg, j + K);
        else if (!ONE) w.load_chunk(st.ring[p * K + j % K], rg + P * G, j + K - J);
        if (!live) continue;
        if constexpr (BT == 1) {
          const float sc = csc[cj];
          h2 acc16[4];   // rows (0,1) (2,3) (4,5) (6,7) of this chunk, fp16
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            // Packed fp16 FMAs, two rows per op, both columns of the word.
            const uint32_t xp = HAS_S ? pk_mul(xw[0][d], __builtin_bit_cast(u32x4, sv)[d]) : xw[0][d];
            const h2 xx = __builtin_bit_cast(h2, xp);
            const h2 xl = {xx.x, xx.x}, xh = {xx.y, xx.y};
            const h2 c[8] = {as_h2(t1l[d][0]), as_h2(t1l[d][1]), as_h2(t2l[d][0]), as_h2(t2l[d][1]),
                             as_h2(t1h[d][0]), as_h2(t1h[d][1]), as_h2(t2h[d][0]), as_h2(t2h[d][1])};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              acc16[q] = d == 0 ? c[q] * xl : __builtin_elementwise_fma(c[q], xl, acc16[q]);
              acc16[q] = __builtin_elementwise_fma(c[q + 4], xh, acc16[q]);
            }
          }
          // Chunk partial sums (8 columns) into the fp32 accumulators, times 2^e.
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t pq = __builtin_bit_cast(uint32_t, acc16[q]);
            acc[2 * q] = fma_lo(pq, sc, acc[2 * q]);
            acc[2 * q + 1] = fma_hi(pq, sc, acc[2 * q + 1]);
          }
        } else {
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            // (c_k(lo), c_k(hi)) fp16 pairs for k = 0..7
            uint32_t pr[8];
            pr[0] = perm(t1h[d][0], t1l[d][0], 0x05040100u);
            pr[1] = perm(t1h[d][0], t1l[d][0], 0x07060302u);
            pr[2] = perm(t1h[d][1], t1l[d][1], 0x05040100u);
            pr[3] = perm(t1h[d][1], t1l[d][1], 0x07060302u);
            pr[4] = perm(t2h[d][0], t2l[d][0], 0x05040100u);
            pr[5] = perm(t2h[d][0], t2l[d][0], 0x07060302u);
            pr[6] = perm(t2h[d][1], t2l[d][1], 0x05040100u);
            pr[7] = perm(t2h[d][1], t2l[d][1], 0x07060302u);
            uint32_t sp = 0;
            if (HAS_S) sp = __builtin_bit_cast(u32x4, sv)[d];
#pragma unroll
            for (int b = 0; b < BT; ++b) {
              const uint32_t xp = HAS_S ? pk_mul(xw[b][d], sp) : xw[b][d];
#pragma unroll
              for (int k = 0; k < 8; ++k) acc[b * 8 + k] = dot2(pr[k], xp, acc[b * 8 + k]);
            }
          }
        }
      }

      // Critical blocks: add O·(x h) in the accumulator's units, minus what the
      // marker index contributed in the main loop (table row 511 against the
      // same activation operand).  x·h for O is the activation table's value.
      auto correct = [&](const f16x8 o, int col, float sc) {
        const float csx = BT == 1 ? csc[col >> 3] : 1.0f;
#pragma unroll
        for (int b = 0; b < BT; ++b) {
          if (b < B) {
            const f16 x16 = __builtin_bit_cast(f16, xs[b * NP + col]);
            const float xo = (float)x16 * csx;
            const float xm = HAS_S ? (float)(f16)((float)x16 * sc) * csx : xo;
#pragma unroll
            for (int k = 0; k < 8; ++k)
              acc[b * 8 + k] += (float)o[k] * xo - (float)t5[k & 3] * xm;
          }
        }
      };
      if (row_ok && ent < st.cre - st.crb)
        correct(__builtin_bit_cast(f16x8, st.eo), (unsigned)st.ecol < (unsigned)N ? st.ecol : 0, (float)gs);
      // Rows with more than 64·S critical blocks: the rest, synchronously.
      if (row_ok) {
        for (int i = st.crb + 64 * S + ent; i < st.cre; i += 64 * S) {
          const int col = gp(a.O_col)[i];
          const float sc = HAS_S ? (float)gp(a.S)[(size_t)grp * N + col] : 1.0f;
          correct(*gp((const f16x8*)(a.O + (size_t)i * 8)), col, sc);
        }
      }

      // Next row group's entries.
      if (!ONE) {
        w.load_entries(st, st.nrb, st.nre);
        st.crb = st.nrb; st.cre = st.nre;
        st.nrb = frb; st.nre = fre;
      }

      const int base = wave_reduce_halving<V>(acc);
      if constexpr (PAIR) {
        // The up wave hands its rounded outputs to the gate wave of the same
        // row slot through LDS (same reducing lanes), which writes
        // silu(gate) * up with the roundings of the separate SwiGLU kernel.
        (void)base;
        const bool writer = WaveReduceOut<V>::writer(lane);
        const uint16_t v16 = Act<XT>::from_f32(acc[0] * out_scale * (float)og + (float)ob);
        if ((wave & 1) && writer) pairx[par][slot][lane] = v16;
        // One barrier per row group; pairx alternates like red[] below.
        __syncthreads();
        if (!(wave & 1) && row_ok && writer && wb < B) {
          const float gf = Act<XT>::to_f32(v16), uf = Act<XT>::to_f32(pairx[par][slot][lane]);
          float o = gf / (1.0f + __expf(-gf)) * uf;
          // The fp32 rounding of the product before the fp16 one, as the
          // separate kernel computes it (without this the compiler fuses the
          // multiply and the conversion into one mixed-precision FMA).
          asm volatile("" : "+v"(o));
          store_y(a.y + (size_t)wb * a.ldy + 8 * m + wk, Act<XT>::from_f32(o));
        }
        par ^= 1;
      } else if constexpr (S == 1) {
        // The wave owns the row: write straight from the reducing lanes.
        (void)base;
        if (row_ok && WaveReduceOut<V>::writer(lane) && wb < B) {
          const float sum = acc[0] * out_scale * (float)og + (float)ob;
          store_y(a.y + (size_t)wb * a.ldy + 8 * m + wk, Act<XT>::from_f32(sum));
        }
      } else {
        if (WaveReduceOut<V>::writer(lane)) {
#pragma unroll
          for (int i = 0; i < WaveReduceOut<V>::per_lane; ++i) sm.red[par][wave][base + i] = acc[i];
        }
        // One barrier per row group: red[] alternates, and the next barrier
        // orders these reads of red[par] before its reuse two groups later.
        __syncthreads();
        if (tid < R * V) {
          const int sl = tid / V;
          if (orow < M && wb < B) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < S; ++w) sum += sm.red[par][sl * S + w][wbase];
            sum = sum * out_scale * (float)og + (float)ob;
            store_y(a.y + (size_t)wb * a.ldy + 8 * orow + wk, Act<XT>::from_f32(sum));
          }
        }
        par ^= 1;
      }
    }
    }
  }
};

}  // namespace dec
}  // namespace eptq

// Persistent E8-D4 decode matvec (batch 1..8), the HBM-bound hot path.
//
// Same result as the reference decode kernels (csrc/eptq_kernels.cu:161-292,
// kernels/triton_e8d4.py:47-157): y = g ⊙ (decode(Q)·(h ⊙ S ⊙ x)ᵀ + CSR(O)) + bias.
//
// Work split.  A workgroup is 4 waves; S waves (1, 2 or 4) share a Q-row, so
// a workgroup works on R = 4/S adjacent rows at a time and walks row groups
// blockIdx.x, +G, +2G, ...  Lane `lane` of segment wave `seg` owns the
// 16-byte column chunks c = seg·64 + lane + 64·S·j (j < J) of every row, so
// the activation side (x·h) is prepared once per workgroup and kept in
// registers and the E8-D4 table is staged in LDS once.  S is the smallest
// split that still gives the chip enough waves: whole-row waves (S = 1) need
// no cross-wave reduction and no barrier; S > 1 combines the S partial sums
// through LDS with one barrier per row group.  The index chunks of the next
// P row groups are kept in flight in a register ring (about 8 chunks = 128
// bytes per lane) so HBM latency is covered, and the grid holds as many
// workgroups per CU as the registers allow so LDS latency is covered.
//
// Arithmetic:
//  * B = 1: x·h is formed exactly in fp32 (product of two fp16 values) and
//    each table component is accumulated with one mixed fp16×fp32 FMA.
//  * B >= 2: the two indices of a 32-bit word (adjacent columns) are paired:
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

#include "common.h"
#include "kernels.h"

namespace eptq {

namespace {

constexpr int kT = 256;          // threads per workgroup
constexpr int kBufferWord3 = 0x00020000;   // buffer resource word 3 (gfx9 family)
constexpr int kNonTemporal = 2;            // buffer load cache policy: nt
constexpr int kW = kT / 64;      // waves per workgroup

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

}  // namespace

template <int BT, int J, int P, int S, bool HAS_S, typename XT>
__global__ __launch_bounds__(kT) void k_decode_e8d4(MultiArgs ma) {
  constexpr int V = BT * 8;
  constexpr int R = kW / S;                    // rows per row group
  static_assert(V <= 64 && R * V <= kT, "one output per thread after the reduction");
  __shared__ f16x4 tab[512];
  __shared__ float red[S > 1 ? 2 : 1][kW][S > 1 ? V : 1];
  __shared__ float wmax[kW];
  // Activation side, shared by the workgroup: xs[b][n] = fp16 x·h (scaled),
  // rows padded by one zero chunk; for B = 1 also csc[c] = the scale of chunk c.
  extern __shared__ __align__(16) char dyn[];

  // This workgroup's layer and its index among the layer's workgroups.
  int li = 0;
#pragma unroll
  for (int l = 1; l < kMaxLayers; ++l)
    if (l < ma.n && (int)blockIdx.x >= ma.start[l]) li = l;
  const LinearArgs a = li == 0 ? ma.l[0] : li == 1 ? ma.l[1] : li == 2 ? ma.l[2] : ma.l[3];
  const int wg = (int)blockIdx.x - ma.start[li];
  const int G = ma.start[li + 1] - ma.start[li];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slot = wave / S, seg = wave % S;
  const int N = a.N, M = a.M, B = a.B;
  const int nch = N >> 3;
  const int NP = N + 8;
  const int RG = (M + R - 1) / R;              // row groups
  const char* __restrict__ tabB = (const char*)tab;
  uint16_t* __restrict__ xs = (uint16_t*)dyn;
  float* __restrict__ csc = (float*)(dyn + BT * NP * 2);

  auto chunk = [&](int j) { return seg * 64 + lane + 64 * S * j; };

  // ---- critical-block rows: [rb, re) of O_col/O for this wave's row ----
  // Scalar loads, kept one row group ahead of their use so that the entry
  // loads they address never wait for them.
  auto row_range = [&](int rg, int& rb, int& re) {
    const int row = rg * R + slot;             // wave-uniform
    const int rr = row < M ? row : M;
    rb = a.O_row_ptr[rr];
    re = a.O_row_ptr[row < M ? rr + 1 : rr];
  };
  int crb, cre, nrb, nre;
  row_range(wg, crb, cre);
  row_range(wg + G, nrb, nre);

  // ---- loads: table and activations first; the activation table is built
  // before the index stream is requested, so its loads are not queued behind
  // the HBM index traffic (vmcnt also counts loads in issue order). ----
  f16x4 tload[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) tload[p] = ((const f16x4*)a.codes)[tid + kT * p];   // fp16 table

  // h and x rows through buffer resources (offsets past the end read zero).
  // Each thread prepares chunks c = tid + kT·k of the activation table; the
  // first CAP of them are loaded together up front, any others one by one.
  constexpr int CA = (J * S) / 4 < 1 ? 1 : (J * S) / 4;   // >= ceil(nch / kT)
  constexpr int CAP = CA < 18 / (BT + 1) ? CA : 18 / (BT + 1);
  const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc((void*)a.h, (short)0, N * 2, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, B * N * 2, kBufferWord3);
  auto load_hx = [&](int c, u32x4& hw, u32x4 (&xw)[BT]) {
    const bool cv = c < nch;
    hw = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rh, cv ? c * 16 : N * 2, 0, 0));
#pragma unroll
    for (int b = 0; b < BT; ++b)
      xw[b] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
          rx, cv && b < B ? b * N * 2 + c * 16 : B * N * 2, 0, 0));
  };
  u32x4 hpre[CAP], xpre[CAP][BT];
#pragma unroll
  for (int k = 0; k < CAP; ++k) load_hx(tid + kT * k, hpre[k], xpre[k]);

  // ---- activation side into LDS ----
  float out_scale = 1.0f;
  if (tid == 0) {   // the zero chunk past the end of every row
#pragma unroll
    for (int b = 0; b < BT; ++b) *(u32x4*)(xs + b * NP + nch * 8) = (u32x4){0u, 0u, 0u, 0u};
    if (BT == 1) csc[nch] = 1.0f;
  }
  if constexpr (BT == 1) {
    // Per chunk of 8 columns: xs = fp16(x·h·2^-e), csc = 2^e with
    // max|x·h|·2^-e in [0.5, 1), so the fp16 accumulation of a chunk (|c| < 2,
    // 8 columns) cannot overflow; the main loop applies 2^e in fp32.
    auto prep = [&](int c, const u32x4 hw, const u32x4 xw) {
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
        *(u32x4*)(xs + c * 8) = w;
        csc[c] = __builtin_ldexpf(1.0f, ex);
      }
    };
#pragma unroll
    for (int k = 0; k < CAP; ++k) prep(tid + kT * k, hpre[k], xpre[k][0]);
    for (int c = tid + kT * CAP; c < nch; c += kT) {
      u32x4 hw, xw[BT];
      load_hx(c, hw, xw);
      prep(c, hw, xw[0]);
    }
  } else {
    // Workgroup-uniform power-of-two scale with max|h|·2^-e <= 1, so the fp16
    // pairs |x·h·2^-e| <= |x| cannot overflow (dot2 accumulates in fp32).
    float mx = 0.0f;
    auto hmax = [&](const u32x4 hw) {
      const f16x8 hv = __builtin_bit_cast(f16x8, hw);
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf((float)hv[e]));
    };
#pragma unroll
    for (int k = 0; k < CAP; ++k) hmax(hpre[k]);
    for (int c = tid + kT * CAP; c < nch; c += kT)
      hmax(__builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rh, c * 16, 0, 0)));
    mx = fmaxf(mx, partner<1>(mx));
    mx = fmaxf(mx, partner<2>(mx));
    mx = fmaxf(mx, partner<4>(mx));
    mx = fmaxf(mx, partner<8>(mx));
    mx = fmaxf(mx, partner<16>(mx));
    mx = fmaxf(mx, partner<32>(mx));
    if (lane == 0) wmax[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int ex = 0;
    if (mx > 1.0f) ex = (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xff) - 126;  // 2^ex >= mx
    out_scale = __builtin_ldexpf(1.0f, ex);
    const f16 down = (f16)__builtin_ldexpf(1.0f, -ex);
    const uint32_t down2 = __builtin_bit_cast(uint32_t, (h2){down, down});
    auto prep = [&](int c, const u32x4 hw, const u32x4 (&xw)[BT]) {
      if (c < nch) {
#pragma unroll
        for (int b = 0; b < BT; ++b) {
          u32x4 w;
#pragma unroll
          for (int d = 0; d < 4; ++d) w[d] = pk_mul(xw[b][d], pk_mul(hw[d], down2));
          *(u32x4*)(xs + b * NP + c * 8) = w;
        }
      }
    };
#pragma unroll
    for (int k = 0; k < CAP; ++k) prep(tid + kT * k, hpre[k], xpre[k]);
    for (int c = tid + kT * CAP; c < nch; c += kT) {
      u32x4 hw, xw[BT];
      load_hx(c, hw, xw);
      prep(c, hw, xw);
    }
  }

  // Index chunks in flight: K of each of the P row groups of the ring.  A
  // slot is refilled as soon as its chunk's table addresses are formed —
  // with the chunk K ahead in the same row, else the matching chunk of the row
  // group P·G ahead — so each wave's requests reach HBM in a steady stream.
  constexpr int K = J > 4 ? 4 : J;
  static_assert(J % K == 0, "chunks per row must be a multiple of the chunks in flight");
  u32x4 qv[P][K];
  // Index chunks are read through a buffer resource spanning one row (an
  // empty one past the last row): out-of-range chunks read as zero, so the
  // loads need no branches or clamps, and the compiler can wait for exactly
  // the load it needs (vmcnt counts loads in issue order).
  auto load_chunk = [&](u32x4& dst, int rg, int j) {
    const int row = rg * R + slot;            // wave-uniform
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.Q + (size_t)(row < M ? row : 0) * N), (short)0, row < M ? N * 2 : 0, kBufferWord3);
    dst = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, chunk(j) * 16, 0, kNonTemporal));
  };
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int j = 0; j < K; ++j) load_chunk(qv[p][j], wg + p * G, j);

  // Critical blocks, first 64·S entries of a row: lane `ent` of the row's
  // S waves holds entry rb + ent (its column and O vector).  Buffer resources
  // span exactly the row's entries, so lanes past the end read zeros.
  const int ent = seg * 64 + lane;
  int ecol;
  u32x4 eo;
  auto load_entries = [&](int rb, int re) {
    const int cnt = re - rb;
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.O_col + rb), (short)0, cnt * 4, kBufferWord3);
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.O + (size_t)rb * 8), (short)0, cnt * 16, kBufferWord3);
    ecol = (int)__builtin_amdgcn_raw_buffer_load_b32(rc, ent * 4, 0, 0);
    eo = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, ent * 16, 0, 0));
  };
  load_entries(crb, cre);
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int p = 0; p < 2; ++p) tab[(tid + kT * p) ^ 0x100] = tload[p];
  __syncthreads();

  // Marker vector as the main loop sees it.
  const f16x4 t5 = tab[511 ^ 0x100];
  // bias (or nothing: an empty resource reads zeros).
  const __amdgpu_buffer_rsrc_t rbias = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.bias, (short)0, a.bias ? 16 * M : 0, kBufferWord3);
  // The output (batch row, block row) this thread writes after the reduction.
  const int wbase = S == 1 ? reduce_base<V>(lane) : (tid < R * V ? tid % V : 0);
  const int wb = wbase >> 3, wk = wbase & 7;

  int par = 0;
  for (int rg0 = wg; rg0 < RG; rg0 += P * G) {
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int rg = rg0 + p * G;
    if (rg >= RG) break;                       // uniform across the workgroup
    const int m = rg * R + slot;
    const bool row_ok = m < M;
    const int grp = HAS_S ? (8 * (row_ok ? m : 0)) / a.qb : 0;

    // Epilogue operands for this thread's output row, fetched early.
    const int orow = S == 1 ? m : rg * R + (tid < R * V ? tid / V : 0);
    const int oidx = 8 * (orow < M ? orow : M - 1) + wk;
    const f16 og = a.g[oidx];
    const f16 ob = __builtin_bit_cast(f16, (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rbias, oidx * 2, 0, 0));
    // Row pointers two row groups ahead (their entries are loaded next).
    int frb, fre;
    row_range(rg + 2 * G, frb, fre);
    // S at the critical blocks' columns (grouped layers), issued part-way
    // through the chunk loop once the entry columns have arrived.
    f16 gs = (f16)1.0f;
    auto load_gather = [&]() {
      if constexpr (HAS_S) {
        const int col = (unsigned)ecol < (unsigned)N ? ecol : 0;
        gs = a.S[(size_t)grp * N + col];
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
        if (HAS_S) sv = *(const f16x8*)(a.S + (size_t)grp * N + ((cj < nch ? cj : 0) << 3));
#pragma unroll
        for (int b = 0; b < BT; ++b) xw[b] = *(const u32x4*)(xs + b * NP + cj * 8);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t w = qv[p][j % K][d];
          const uint32_t a1lo = (w >> 4) & 0xFF8u;
          const uint32_t a1hi = (w >> 20) & 0xFF8u;
          const uint32_t a2lo = bfi(0x3F8u, w << 3, a1lo);
          const uint32_t a2hi = bfi(0x3F8u, w >> 13, a1hi);
          t1l[d] = *(const u32x2*)(tabB + a1lo);
          t2l[d] = *(const u32x2*)(tabB + a2lo);
          t1h[d] = *(const u32x2*)(tabB + a1hi);
          t2h[d] = *(const u32x2*)(tabB + a2hi);
        }
      }
      // Refill this chunk's ring slot.
      if (j + K < J) load_chunk(qv[p][j % K], rg, j + K);
      else load_chunk(qv[p][j % K], rg + P * G, j + K - J);
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
    if (row_ok && ent < cre - crb)
      correct(__builtin_bit_cast(f16x8, eo), (unsigned)ecol < (unsigned)N ? ecol : 0, (float)gs);
    // Rows with more than 64·S critical blocks: the rest, synchronously.
    if (row_ok) {
      for (int i = crb + 64 * S + ent; i < cre; i += 64 * S) {
        const int col = a.O_col[i];
        const float sc = HAS_S ? (float)a.S[(size_t)grp * N + col] : 1.0f;
        correct(*(const f16x8*)(a.O + (size_t)i * 8), col, sc);
      }
    }

    // Next row group's entries.
    load_entries(nrb, nre);
    crb = nrb; cre = nre;
    nrb = frb; nre = fre;

    const int base = wave_reduce_halving<V>(acc);
    if constexpr (S == 1) {
      // The wave owns the row: write straight from the reducing lanes.
      (void)base;
      if (row_ok && WaveReduceOut<V>::writer(lane) && wb < B) {
        const float sum = acc[0] * out_scale * (float)og + (float)ob;
        a.y[(size_t)wb * a.ldy + 8 * m + wk] = Act<XT>::from_f32(sum);
      }
    } else {
      if (WaveReduceOut<V>::writer(lane)) {
#pragma unroll
        for (int i = 0; i < WaveReduceOut<V>::per_lane; ++i) red[par][wave][base + i] = acc[i];
      }
      // One barrier per row group: red[] alternates, and the next barrier
      // orders these reads of red[par] before its reuse two groups later.
      __syncthreads();
      if (tid < R * V) {
        const int sl = tid / V;
        if (orow < M && wb < B) {
          float sum = 0.0f;
#pragma unroll
          for (int w = 0; w < S; ++w) sum += red[par][sl * S + w][wbase];
          sum = sum * out_scale * (float)og + (float)ob;
          a.y[(size_t)wb * a.ldy + 8 * orow + wk] = Act<XT>::from_f32(sum);
        }
      }
      par ^= 1;
    }
  }
  }
}

namespace {

int g_cu_count = 0;

int cu_count() {
  if (g_cu_count == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      g_cu_count = n;
    else
      g_cu_count = 256;
  }
  return g_cu_count;
}

// Chunks per lane for a row split S ways (0 if beyond the kernel's range).
int chunks_for(int nch, int S) {
  const int j = (nch + 64 * S - 1) / (64 * S);
  if (j <= 2) return 2;
  if (j <= 4) return 4;
  if (j <= 8) return 8;
  return 0;
}

// Dynamic LDS of the activation side: BT padded fp16 rows, plus the per-chunk
// scales for B = 1.
size_t act_lds_bytes(int N, int BT) {
  return (size_t)BT * (N + 8) * 2 + (BT == 1 ? (size_t)((N >> 3) + 1) * 4 : 0);
}
constexpr size_t kActLdsMax = 64 * 1024;
constexpr size_t kLdsPerCu = 160 * 1024;

bool fits(int J, int N, int BT) { return J > 0 && act_lds_bytes(N, BT) <= kActLdsMax; }

template <int BT, int J, int S, bool HAS_S, typename XT>
void launch_k(const LinearArgs* layers, int n, hipStream_t s) {
  // About 8 index chunks (128 bytes) per lane in flight: P row groups of
  // min(J, 4) chunks.
  constexpr int P = 8 / (J > 4 ? 4 : J);
  constexpr int R = kW / S;
  auto kern = k_decode_e8d4<BT, J, P, S, HAS_S, XT>;
  // As many workgroups per CU as registers and LDS allow (one wave of each
  // workgroup per SIMD): occupancy hides the LDS lookup latency.
  static int reg_cu = 0;
  static size_t static_lds = 0;
  if (reg_cu == 0) {
    hipFuncAttributes fa;
    int v = 128;
    if (hipFuncGetAttributes(&fa, (const void*)kern) == hipSuccess) {
      if (fa.numRegs > 0) v = fa.numRegs;
      static_lds = fa.sharedSizeBytes;
    }
    const int waves = 512 / ((v + 7) / 8 * 8);
    reg_cu = waves < 1 ? 1 : (waves > 8 ? 8 : waves);
  }
  const size_t dyn = act_lds_bytes(layers[0].N, BT);
  int per_cu = (int)(kLdsPerCu / (static_lds + dyn + 256));
  if (per_cu > reg_cu) per_cu = reg_cu;
  if (per_cu < 1) per_cu = 1;
  MultiArgs ma;
  ma.n = n;
  ma.start[0] = 0;
  for (int l = 0; l < kMaxLayers; ++l) {
    if (l < n) {
      ma.l[l] = layers[l];
      const int RG = (layers[l].M + R - 1) / R;
      const int g = cu_count() * per_cu < RG ? cu_count() * per_cu : RG;
      ma.start[l + 1] = ma.start[l] + g;
    } else {
      ma.l[l] = layers[0];
      ma.start[l + 1] = ma.start[l];
    }
  }
  kern<<<ma.start[n], kT, dyn, s>>>(ma);
}

template <int BT, int S, bool HAS_S, typename XT>
int launch_s(const LinearArgs* l, int n, hipStream_t s) {
  const int J = chunks_for(l[0].N >> 3, S);
  if (!fits(J, l[0].N, BT)) return -1;
  if (J == 2) { launch_k<BT, 2, S, HAS_S, XT>(l, n, s); return 0; }
  if (J == 4) { launch_k<BT, 4, S, HAS_S, XT>(l, n, s); return 0; }
  if (J == 8) { launch_k<BT, 8, S, HAS_S, XT>(l, n, s); return 0; }
  return -1;
}

template <int BT, bool HAS_S, typename XT>
int launch_bt(const LinearArgs* l, int n, hipStream_t s) {
  const int N = l[0].N;
  const int nch = N >> 3;
  long Mt = 0;
  for (int i = 0; i < n; ++i) Mt += l[i].M;
  // Smallest row split that gives the chip about 8 waves per CU (and keeps
  // the chunks per lane within the kernel's range).
  const int want = cu_count() * 8;
  int S = 4;
  for (int cand = 1; cand <= 4; cand *= 2) {
    if (!fits(chunks_for(nch, cand), N, BT)) continue;
    S = cand;
    if (Mt * cand >= want) break;
  }
  if (!fits(chunks_for(nch, S), N, BT)) return -1;
  if (S == 1) return launch_s<BT, 1, HAS_S, XT>(l, n, s);
  if (S == 2) return launch_s<BT, 2, HAS_S, XT>(l, n, s);
  return launch_s<BT, 4, HAS_S, XT>(l, n, s);
}

template <bool HAS_S, typename XT>
int launch_b(const LinearArgs* l, int n, hipStream_t s) {
  const int B = l[0].B;
  if (B == 1) return launch_bt<1, HAS_S, XT>(l, n, s);
  if (B == 2) return launch_bt<2, HAS_S, XT>(l, n, s);
  if (B <= 4) return launch_bt<4, HAS_S, XT>(l, n, s);
  if (B <= 8) return launch_bt<8, HAS_S, XT>(l, n, s);
  return -1;
}

}  // namespace

// Returns 0 if launched, -1 if the layers/batch are outside the kernel's range.
int launch_decode_e8d4_multi(const LinearArgs* l, int n, hipStream_t s) {
  if (n < 1 || n > kMaxLayers) return -1;
  const LinearArgs& a = l[0];
  for (int i = 1; i < n; ++i)
    if (l[i].N != a.N || l[i].B != a.B || l[i].x != a.x || l[i].codes != a.codes ||
        l[i].codes_f32 != a.codes_f32 || l[i].x_bf16 != a.x_bf16 || (l[i].S != nullptr) != (a.S != nullptr))
      return -1;
  if (a.B < 1 || a.B > 8) return -1;
  if (a.codes_f32) return -1;  // fp32 tables take the generic kernel
  if (a.x_bf16) {
    if (a.B >= 2) return -1;   // the B >= 2 pairs are formed in fp16 arithmetic
    return a.S ? launch_bt<1, true, bf16>(l, n, s) : launch_bt<1, false, bf16>(l, n, s);
  }
  return a.S ? launch_b<true, f16>(l, n, s) : launch_b<false, f16>(l, n, s);
}

int launch_decode_e8d4(const LinearArgs& a, hipStream_t s) { return launch_decode_e8d4_multi(&a, 1, s); }

}  // namespace eptq

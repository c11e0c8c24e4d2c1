// E8-D4 decode matvec (batch 1..8), one launch per layer group: the
// HBM-bound hot path.  The per-workgroup layer code (work split, arithmetic,
// index decode) is in decode_layer.h; this file selects the layer of each
// workgroup and sizes the launch.

#include <stdlib.h>

#include "decode_layer.h"

namespace eptq {

using namespace dec;

template <int BT, int J, int P, int S, bool HAS_S, typename XT, bool ONE>
__global__ __launch_bounds__(kT) void k_decode_e8d4(MultiArgs ma) {
  __shared__ __attribute__((aligned(16))) f16x4 tab[512];
  __shared__ float red[2][kW][BT * 8];
  __shared__ float wmax[kW];
  // Activation side, shared by the workgroup: xs[b][n] = fp16 x·h (scaled),
  // rows padded by one zero chunk; for B = 1 also csc[c] = the scale of chunk c.
  extern __shared__ __align__(16) char dyn[];

  // This workgroup's layer (grid row) and its index among the layer's
  // workgroups.  The layer is the grid row rather than a search of the
  // launch's layer boundaries, so the layer's arguments are read in the
  // workgroup's first scalar loads, not in a second round trip after them.
  const int li = (int)blockIdx.y;
  const int wg = (int)blockIdx.x;
  const int G = ma.start[li + 1] - ma.start[li];
  if (wg >= G) return;   // rows of the grid past this layer's workgroups
  const LinearArgs a = ma.l[li];

  using L = Layer<BT, J, P, S, HAS_S, XT, false, ONE>;
  const L layer(a, wg, G);
  const Smem<BT> sm{tab, red, wmax, (uint16_t*)dyn, (float*)(dyn + BT * (a.N + 8) * 2)};
  typename L::State st;
  // Critical-block row ranges first (scalar loads, one row group ahead of use).
  layer.rows_first(st);
  // Table and activations before the index stream, so their loads are not
  // queued behind the HBM index traffic (vmcnt counts loads in issue order).
  const int tid = threadIdx.x;
  static_assert(2 * kT == 512, "one 16-byte table load per thread");
  const u32x4 tload = *gp((const u32x4*)a.codes + tid);   // fp16 table rows 2·tid, 2·tid + 1
  const float out_scale = layer.build_act(sm);
  layer.issue_ring(st);
  __builtin_amdgcn_sched_barrier(0);
  *(u32x4*)&tab[(2 * tid) ^ 0x100] = tload;   // rows 2·tid, 2·tid + 1 stay adjacent
  __syncthreads();
  layer.rows(st, sm, out_scale);
}

// One activation table of a pair, rounded up to 16 bytes (the tables are
// read with 16-byte LDS loads).
__host__ __device__ inline size_t pair_table_bytes(int N, int BT) { return (act_lds_bytes(N, BT) + 15) & ~(size_t)15; }

// SwiGLU pair: layers ma.l[0] (gate) and ma.l[1] (up) of equal shape, every
// workgroup serving the same rows of both (wave w: layer w % 2, row slot
// w / 2); y = silu(gate) ⊙ up at ma.l[0].y.  Both activation tables are
// built from one read of x (and one RMSNorm, prep 1).
template <int BT, int J, int P, bool HAS_S, bool ONE>
__global__ __launch_bounds__(kT) void k_decode_e8d4_pair(MultiArgs ma) {
  __shared__ __attribute__((aligned(16))) f16x4 tab[512];
  __shared__ float red[2][kW][BT * 8];
  __shared__ float wmax[2][kW];
  __shared__ uint16_t pairx[2][2][64];
  extern __shared__ __align__(16) char dyn[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool up = wave & 1;
  const LinearArgs a = up ? ma.l[1] : ma.l[0];
  using L = Layer<BT, J, P, 1, HAS_S, f16, true, ONE>;
  const L layer(a, (int)blockIdx.x, (int)gridDim.x);
  const size_t act = pair_table_bytes(a.N, BT);   // the second table 16-byte aligned
  const Smem<BT> sm0{tab, red, wmax[0], (uint16_t*)dyn, (float*)(dyn + BT * (a.N + 8) * 2)};
  const Smem<BT> sm1{tab, red, wmax[1], (uint16_t*)(dyn + act), (float*)(dyn + act + BT * (a.N + 8) * 2)};
  typename L::State st;
  layer.rows_first(st);
  const int tid = threadIdx.x;
  static_assert(2 * kT == 512, "one 16-byte table load per thread");
  const u32x4 tload = *gp((const u32x4*)a.codes + tid);   // fp16 table rows 2·tid, 2·tid + 1
  float scale1;
  const float scale0 =
      L(ma.l[0], (int)blockIdx.x, (int)gridDim.x).template build_act<true>(sm0, ma.l[1].h, &sm1, &scale1);
  layer.issue_ring(st);
  __builtin_amdgcn_sched_barrier(0);
  *(u32x4*)&tab[(2 * tid) ^ 0x100] = tload;   // rows 2·tid, 2·tid + 1 stay adjacent
  __syncthreads();
  layer.rows(st, up ? sm1 : sm0, up ? scale1 : scale0, pairx);
}

namespace dec {

// Smallest batch that takes the matrix-core decode kernel (EPTQ_MFMA_MIN_BATCH
// overrides, for tests and tuning).
int mfma_min_batch_init() {
  const char* e = getenv("EPTQ_MFMA_MIN_BATCH");
  if (e && *e) return atoi(e);
  // Below 3 the vector kernel (one dot product per batch row) is faster on
  // Llama shapes; from 3 on the MFMA kernel (whose cost barely grows with B)
  // is.  Llama-2-7B decode step: B=2 1.15 against 1.53 ms, B=3 1.54 against
  // 1.64 (the vector kernel runs B=3 as 4), B=4 1.55 against 1.66.
  return 3;
}

int cu_count() {
  static int n_cu = 0;
  if (n_cu == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      n_cu = n;
    else
      n_cu = 256;
  }
  return n_cu;
}

}  // namespace dec

namespace {

template <int BT, int J, int S, bool HAS_S, typename XT, bool ONE>
int launch_one(const LinearArgs* layers, int n, hipStream_t s, int per_cu, size_t dyn) {
  constexpr int P = 8 / (J > 4 ? 4 : J);
  constexpr int R = kW / S;
  const int cap = cu_count() * per_cu;
  // ONE: the launch's row groups fit in one round (sum RG <= cap).  Workgroups
  // are raised to a whole number of CU rounds (within cap), given to the
  // layers in proportion to their rows and never more than a layer's rows:
  // with the strided row map every CU then holds about the same number of
  // rows (688 row groups of 4 rows on 256 CUs left CUs with 3 and with 2).
  long rg_sum = 0, m_sum = 0;
  for (int l = 0; l < n; ++l) {
    rg_sum += (layers[l].M + R - 1) / R;
    m_sum += layers[l].M;
  }
  long total = (rg_sum + cu_count() - 1) / cu_count() * cu_count();
  if (total > cap) total = cap;
  MultiArgs ma;
  ma.n = n;
  ma.act = nullptr;
  ma.start[0] = 0;
  for (int l = 0; l < kMaxLayers; ++l) {
    if (l < n) {
      ma.l[l] = layers[l];
      const int RG = (layers[l].M + R - 1) / R;
      int g = cap < RG ? cap : RG;
      if (ONE) {
        long extra = (total - rg_sum) * layers[l].M / (m_sum > 0 ? m_sum : 1);
        g = RG + (int)(extra > 0 ? extra : 0);
        if (g > layers[l].M) g = layers[l].M;
      }
      ma.start[l + 1] = ma.start[l] + g;
    } else {
      ma.l[l] = layers[0];
      ma.start[l + 1] = ma.start[l];
    }
  }
  int gx = 1;
  for (int l = 0; l < n; ++l) gx = ma.start[l + 1] - ma.start[l] > gx ? ma.start[l + 1] - ma.start[l] : gx;
  k_decode_e8d4<BT, J, P, S, HAS_S, XT, ONE><<<dim3(gx, n), kT, dyn, s>>>(ma);
  return 0;
}

template <int BT, int J, int S, bool HAS_S, typename XT>
int launch_k(const LinearArgs* layers, int n, hipStream_t s) {
  // About 8 index chunks (128 bytes) per lane in flight: P row groups of
  // min(J, 4) chunks.
  constexpr int P = 8 / (J > 4 ? 4 : J);
  constexpr int R = kW / S;
  // The fused RMSNorm keeps a whole row in the first CAP chunks per thread.
  if (layers[0].prep == 1 && Layer<BT, J, P, S, HAS_S, XT>::CAP * kT * 8 < layers[0].N) return -1;
  // As many workgroups per CU as registers and LDS allow (one wave of each
  // workgroup per SIMD): occupancy hides the LDS lookup latency.
  const size_t dyn = act_lds_bytes(layers[0].N, BT);
  auto per_cu_of = [&](const void* kern, int& reg_cu, size_t& static_lds) {
    if (reg_cu == 0) {
      hipFuncAttributes fa;
      int v = 128;
      if (hipFuncGetAttributes(&fa, kern) == hipSuccess) {
        if (fa.numRegs > 0) v = fa.numRegs;
        static_lds = fa.sharedSizeBytes;
      }
      const int waves = 512 / ((v + 7) / 8 * 8);
      reg_cu = waves < 1 ? 1 : (waves > 8 ? 8 : waves);
    }
    int per_cu = (int)(kLdsPerCu / (static_lds + dyn + 256));
    if (per_cu > reg_cu) per_cu = reg_cu;
    return per_cu < 1 ? 1 : per_cu;
  };
  // One row group per workgroup in every layer (the Llama decode shapes at
  // B <= 2): the form without look-ahead loads, sized by its own registers.
  if constexpr (BT <= 2) {
    static int reg_one = 0;
    static size_t lds_one = 0;
    const int per_cu = per_cu_of((const void*)k_decode_e8d4<BT, J, P, S, HAS_S, XT, true>, reg_one, lds_one);
    bool one = true;
    for (int l = 0; l < n; ++l)
      if ((layers[l].M + R - 1) / R > cu_count() * per_cu) one = false;
    if (one) return launch_one<BT, J, S, HAS_S, XT, true>(layers, n, s, per_cu, dyn);
  }
  static int reg_gen = 0;
  static size_t lds_gen = 0;
  const int per_cu = per_cu_of((const void*)k_decode_e8d4<BT, J, P, S, HAS_S, XT, false>, reg_gen, lds_gen);
  return launch_one<BT, J, S, HAS_S, XT, false>(layers, n, s, per_cu, dyn);
}

template <int BT, int J, bool HAS_S>
int launch_pair_k(const LinearArgs* l, hipStream_t s) {
  constexpr int P = 8 / (J > 4 ? 4 : J);
  using L = Layer<BT, J, P, 1, HAS_S, f16, true>;
  // The fused RMSNorm keeps a whole row in the first CAP chunks per thread.
  if (l[0].prep == 1 && L::CAP * kT * 8 < l[0].N) return -1;
  const size_t dyn = 2 * pair_table_bytes(l[0].N, BT);
  auto per_cu_of = [&](const void* kern, int& reg_cu, size_t& static_lds) {
    if (reg_cu == 0) {
      hipFuncAttributes fa;
      int v = 128;
      if (hipFuncGetAttributes(&fa, kern) == hipSuccess) {
        if (fa.numRegs > 0) v = fa.numRegs;
        static_lds = fa.sharedSizeBytes;
      }
      const int waves = 512 / ((v + 7) / 8 * 8);
      reg_cu = waves < 1 ? 1 : (waves > 8 ? 8 : waves);
    }
    int per_cu = (int)(kLdsPerCu / (static_lds + dyn + 256));
    if (per_cu > reg_cu) per_cu = reg_cu;
    return per_cu < 1 ? 1 : per_cu;
  };
  const int RG = (l[0].M + L::R - 1) / L::R;
  MultiArgs ma;
  ma.n = 2;
  ma.act = nullptr;
  ma.l[0] = l[0];
  ma.l[1] = l[1];
  ma.l[2] = ma.l[3] = l[0];
  ma.start[0] = 0;
  // One row group per workgroup: the form without look-ahead loads.
  static int reg_one = 0, reg_gen = 0;
  static size_t lds_one = 0, lds_gen = 0;
  const int pc1 = per_cu_of((const void*)k_decode_e8d4_pair<BT, J, P, HAS_S, true>, reg_one, lds_one);
  if (RG <= cu_count() * pc1) {
    ma.start[1] = ma.start[2] = ma.start[3] = ma.start[4] = RG;
    k_decode_e8d4_pair<BT, J, P, HAS_S, true><<<RG, kT, dyn, s>>>(ma);
    return 0;
  }
  const int pc = per_cu_of((const void*)k_decode_e8d4_pair<BT, J, P, HAS_S, false>, reg_gen, lds_gen);
  const int G = cu_count() * pc < RG ? cu_count() * pc : RG;
  ma.start[1] = ma.start[2] = ma.start[3] = ma.start[4] = G;
  k_decode_e8d4_pair<BT, J, P, HAS_S, false><<<G, kT, dyn, s>>>(ma);
  return 0;
}

template <int BT, bool HAS_S>
int launch_pair_bt(const LinearArgs* l, hipStream_t s) {
  const int J = chunks_for(l[0].N >> 3, 1);
  if (J == 0 || 2 * pair_table_bytes(l[0].N, BT) > kActLdsMax) return -1;
  if (J == 2) return launch_pair_k<BT, 2, HAS_S>(l, s);
  if (J == 4) return launch_pair_k<BT, 4, HAS_S>(l, s);
  return launch_pair_k<BT, 8, HAS_S>(l, s);
}

template <int BT, int S, bool HAS_S, typename XT>
int launch_s(const LinearArgs* l, int n, hipStream_t s) {
  const int J = chunks_for(l[0].N >> 3, S);
  if (!fits(J, l[0].N, BT)) return -1;
  if (J == 2) return launch_k<BT, 2, S, HAS_S, XT>(l, n, s);
  if (J == 4) return launch_k<BT, 4, S, HAS_S, XT>(l, n, s);
  if (J == 8) return launch_k<BT, 8, S, HAS_S, XT>(l, n, s);
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
int launch_decode_e8d4_multi(const LinearArgs* l, int n, hipStream_t s, void* work, long long work_bytes) {
  if (n < 1 || n > kMaxLayers) return -1;
  const LinearArgs& a = l[0];
  if (a.B >= mfma_min_batch() && launch_decode_mfma_multi(l, n, s, work, work_bytes) == 0) return 0;
  for (int i = 1; i < n; ++i)
    if (l[i].N != a.N || l[i].B != a.B || l[i].x != a.x || l[i].codes != a.codes ||
        l[i].codes_f32 != a.codes_f32 || l[i].x_bf16 != a.x_bf16 || (l[i].S != nullptr) != (a.S != nullptr) ||
        l[i].prep != a.prep || l[i].ldx != a.ldx || l[i].x2 != a.x2 || l[i].nw != a.nw ||
        l[i].xsum != a.xsum || l[i].eps != a.eps)
      return -1;
  if (a.prep != 0 && a.x_bf16) return -1;
  for (int i = 0; i < n; ++i)
    if (l[i].res) return -1;   // residual epilogue: matrix-core kernel only
  if (a.B < 1 || a.B > 8) return -1;
  if (a.codes_f32) return -1;  // fp32 tables take the generic kernel
  if (a.x_bf16) return a.S ? launch_b<true, bf16>(l, n, s) : launch_b<false, bf16>(l, n, s);
  return a.S ? launch_b<true, f16>(l, n, s) : launch_b<false, f16>(l, n, s);
}

int launch_decode_e8d4(const LinearArgs& a, hipStream_t s) { return launch_decode_e8d4_multi(&a, 1, s); }

// Returns 0 if launched, -1 if the pair is outside the kernel's range.
int launch_decode_e8d4_pair(const LinearArgs* l, hipStream_t s) {
  const LinearArgs& a = l[0];
  const LinearArgs& b = l[1];
  if (b.M != a.M || b.N != a.N || b.B != a.B || b.x != a.x || b.codes != a.codes || b.codes_f32 || a.codes_f32 ||
      a.x_bf16 || b.x_bf16 || (b.S != nullptr) != (a.S != nullptr) || b.prep != a.prep || b.ldx != a.ldx ||
      b.x2 != a.x2 || b.nw != a.nw || b.xsum != a.xsum || b.eps != a.eps || a.res || b.res)
    return -1;
  const int B = a.B;
  if (B == 1) return a.S ? launch_pair_bt<1, true>(l, s) : launch_pair_bt<1, false>(l, s);
  if (B == 2) return a.S ? launch_pair_bt<2, true>(l, s) : launch_pair_bt<2, false>(l, s);
  return -1;   // B >= 3: two activation tables exceed the workgroup's activation LDS at N = 4096
}

}  // namespace eptq

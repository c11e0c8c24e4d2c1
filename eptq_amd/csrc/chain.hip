// Decode chain: a sequence of E8-D4 layer stages (batch 1) in one persistent
// launch.  A decode step runs 4 dependent Linear stages per transformer layer
// (q|k|v, o, gate|up, down); as separate launches each stage pays the launch
// gap, the first index loads' latency and the drain.  Here every workgroup
// stays resident and walks the stages in order: before waiting for a stage's
// input it already issues that stage's index ring (the index stream does not
// depend on the input), so HBM keeps streaming across stage boundaries.
//
// Stage boundary.  A stage that waits starts reading its x only after every
// workgroup has finished the previous stage (hence every earlier one):
//  * writers: y is stored with device-coherent (sc1) stores; each wave waits
//    for its stores (vmcnt), the workgroup meets at a barrier, and one thread
//    adds 1 to its group's counter (NG groups of workgroups, one 128-byte line
//    each).  The last arriver of a group adds 1 to the stage's top counter;
//    the last group sets the stage's per-group flags.
//  * readers: one thread polls its group's flag (bounded spin with s_sleep),
//    then the workgroup meets at a barrier and reads x with sc1 loads.
// No L2 writeback or invalidate is needed: every cross-workgroup access goes
// to the device-coherent level, which keeps a boundary near 1.5 us on
// MI355X where a fenced barrier costs 8-20 us.
//
// Counters are never reset: a launch reads the plan's epoch e at its start
// and counts to multiples of e + 1; the last workgroup to leave stores e + 1.
// A wait that spins past its limit sets the plan's error word and goes on
// (results are then wrong, but every wave still reaches the end), and later
// waits see the word and stop spinning; eptq_e8d4_chain_check reports it.
//
// Workgroups must all be resident: the plan sizes the grid from the
// occupancy of this kernel (at most what the CUs hold at once), and one plan
// runs one launch at a time.

#include <stddef.h>
#include <stdlib.h>

#include "decode_layer.h"
#include "chain.h"

namespace eptq {

using namespace dec;

namespace {

constexpr int kLine = 32;                 // ints per 128-byte line
constexpr int kEpoch = 0, kErr = kLine, kExit = 2 * kLine, kStages = 3 * kLine;
constexpr int kSpinLimit = 1 << 20;       // polls (each >= one device round trip)
// s_waitcnt operand (gfx9 encoding): vmcnt 0, expcnt and lgkmcnt not waited.
constexpr int kWaitVmcnt0 = 0x0F70;

__host__ __device__ inline int stage_sync_base(int s, int NG) { return kStages + s * (2 * NG + 1) * kLine; }

__device__ __forceinline__ int ld_dev(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int add_dev(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Thread 0: this workgroup has finished stage s (its y stores are complete).
// Returns true for the last arriver, which sets the stage's flags and so
// need not poll them.
__device__ __forceinline__ bool arrive(int* sync, int s, int NG, int grp, int gsz, int E1) {
  int* base = sync + stage_sync_base(s, NG);
  if ((unsigned)add_dev(base + kLine * (1 + grp), 1) == (unsigned)E1 * gsz - 1u) {
    if ((unsigned)add_dev(base, 1) == (unsigned)E1 * NG - 1u) {
      for (int g = 0; g < NG; ++g) st_dev(base + kLine * (1 + NG + g), E1);
      return true;
    }
  }
  return false;
}

// Thread 0: wait until every workgroup has finished stage s.
__device__ __forceinline__ void wait_stage(int* sync, int s, int NG, int grp, int E1) {
  const int* flag = sync + stage_sync_base(s, NG) + kLine * (1 + NG + grp);
  for (int it = 0;; ++it) {
    if ((int)((unsigned)ld_dev(flag) - (unsigned)E1) >= 0) return;
    if (it >= kSpinLimit) {
      st_dev(sync + kErr, 1);
      return;
    }
    if ((it & 63) == 63 && ld_dev(sync + kErr) != 0) return;   // another workgroup gave up
    __builtin_amdgcn_s_sleep(1);
  }
}

// A stage as one workgroup sees it, read from the stage descriptor that a
// wave-wide vector load left in `d` (lane i holds bytes 16i..16i+15 of the
// ChainStage): wave-uniform values via readlane, no scalar loads.
constexpr int kArgWords = sizeof(LinearArgs) / 4;   // a multiple of 4
static_assert(sizeof(ChainStage) <= 64 * 16, "a stage descriptor fits one wave-wide load");
static_assert(sizeof(ChainStage) % 16 == 0, "stage descriptors are 16-byte aligned");

__device__ __forceinline__ int desc_word(const u32x4& d, int k) {
  // dword k: lane k / 4, component k % 4 (k is a compile-time constant here)
  return (int)__builtin_amdgcn_readlane(d[k & 3], k >> 2);
}

struct StageView {
  int cfg, wait, wg, Gl;
  bool active;
  LinearArgs a;
};

__device__ __forceinline__ StageView view_stage(const u32x4& d) {
  constexpr int kStart = offsetof(ChainStage, start) / 4;
  constexpr int kN = offsetof(ChainStage, n) / 4;
  constexpr int kCfg = offsetof(ChainStage, cfg) / 4;
  constexpr int kWait = offsetof(ChainStage, wait) / 4;
  StageView v;
  const int n = desc_word(d, kN);
  int start[kMaxLayers + 1];
#pragma unroll
  for (int l = 0; l <= kMaxLayers; ++l) start[l] = desc_word(d, kStart + l);
  int li = 0;
#pragma unroll
  for (int l = 1; l < kMaxLayers; ++l)
    if (l < n && (int)blockIdx.x >= start[l]) li = l;
  int s0 = start[0], s1 = start[1];
#pragma unroll
  for (int l = 1; l < kMaxLayers; ++l)
    if (li == l) { s0 = start[l]; s1 = start[l + 1]; }
  v.cfg = desc_word(d, kCfg);
  v.wait = desc_word(d, kWait);
  v.wg = (int)blockIdx.x - s0;
  v.Gl = s1 - s0;
  v.active = v.wg < v.Gl;
  uint32_t w[kArgWords];
#pragma unroll
  for (int k = 0; k < kArgWords; ++k) w[k] = __builtin_amdgcn_readlane(d[k & 3], li * (kArgWords / 4) + (k >> 2));
  __builtin_memcpy(&v.a, w, sizeof(LinearArgs));
  return v;
}

__device__ __forceinline__ int cfg_J(int cfg) { return cfg < 3 ? 2 : cfg < 6 ? 4 : 8; }
__device__ __forceinline__ int cfg_S(int cfg) { const int r = cfg % 3; return r == 0 ? 1 : r == 1 ? 2 : 4; }

// Prefetch of a stage's first row groups that does not depend on its input:
// the index ring, the first entries, the epilogue operands (entry ranges
// were loaded earlier into st).
__device__ __forceinline__ void prefetch_stage(const StageView& v, RowState& st) {
  if (!v.active) return;
  const Walk w(v.a, v.wg, v.Gl, cfg_S(v.cfg), cfg_J(v.cfg), 8);
  w.issue_ring<8>(st);
}

__device__ __forceinline__ void prefetch_rows(const StageView& v, RowState& st) {
  if (!v.active) return;
  const Walk w(v.a, v.wg, v.Gl, cfg_S(v.cfg), cfg_J(v.cfg), 8);
  w.rows_first(st);
}

template <int J, int S, bool HAS_S>
__device__ __forceinline__ void run_stage(const LinearArgs& a, int wg, int G, bool active, bool wait,
                                          const Smem<1>& sm, RowState& st, int* sync, int s, int NG,
                                          int grp, int E1, bool last) {
  constexpr int P = kRing / (J > 4 ? 4 : J);
  using L = Layer<1, J, P, S, HAS_S, f16, true>;
  const L layer(a, wg, G);
  if (wait) {   // workgroup-uniform: every thread meets the barrier
    if (threadIdx.x == 0 && !last) wait_stage(sync, s - 1, NG, grp, E1);
    __syncthreads();
  }
  if (active) {
    const float out_scale = layer.build_act(sm);
    __syncthreads();
    layer.rows(st, sm, out_scale);
  }
}

template <bool HAS_S>
__global__ __launch_bounds__(kT) void k_decode_chain(const ChainStage* __restrict__ prog, int n_stages,
                                                        int* __restrict__ sync, int NG) {
  __shared__ f16x4 tab[512];
  __shared__ float red[2][kW][8];
  __shared__ float wmax[kW];
  __shared__ int s_epoch;
  extern __shared__ __align__(16) char dyn[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int G = gridDim.x;
  const int grp = blockIdx.x % NG;
  const int gsz = G / NG + (grp < G % NG ? 1 : 0);
  // Stage descriptors, two ahead: one 16-byte load per lane each.
  const __amdgpu_buffer_rsrc_t rprog = __builtin_amdgcn_make_buffer_rsrc(
      (void*)prog, (short)0, n_stages * (int)sizeof(ChainStage), kBufferWord3);
  auto load_desc = [&](int s) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
        rprog, s * (int)sizeof(ChainStage) + lane * 16, 0, 0));
  };
  u32x4 dcur = load_desc(0), dnext = load_desc(1);
  if (tid == 0) s_epoch = ld_dev(sync + kEpoch);
#pragma unroll
  for (int p = 0; p < 2; ++p) tab[(tid + kT * p) ^ 0x100] = gp((const f16x4*)prog[0].l[0].codes)[tid + kT * p];
  RowState st;
  {
    const StageView v0 = view_stage(dcur);
    prefetch_rows(v0, st);
    prefetch_stage(v0, st);
  }
  __syncthreads();
  const int E1 = s_epoch + 1;
  bool last = false;   // thread 0 only: this workgroup completed the previous stage

  for (int s = 0; s < n_stages; ++s) {
    const u32x4 dnn = load_desc(s + 2);
    // The next stage's entry ranges, in flight during this stage.
    RowState nx;
    if (s + 1 < n_stages) prefetch_rows(view_stage(dnext), nx);
    {
      const StageView v = view_stage(dcur);
      const bool wait = s > 0 && v.wait;
      const Smem<1> sm{tab, red, wmax, (uint16_t*)dyn, (float*)(dyn + (v.a.N + 8) * 2)};
      switch (v.cfg) {
#define EPTQ_STAGE(J_, S_)                                                                              \
  case ChainStage::cfg_of(J_, S_):                                                                       \
    run_stage<J_, S_, HAS_S>(v.a, v.wg, v.Gl, v.active, wait, sm, st, sync, s, NG, grp, E1, last); \
    break;
        EPTQ_STAGE(2, 1) EPTQ_STAGE(2, 2) EPTQ_STAGE(2, 4)
        EPTQ_STAGE(4, 1) EPTQ_STAGE(4, 2) EPTQ_STAGE(4, 4)
        EPTQ_STAGE(8, 1) EPTQ_STAGE(8, 2) EPTQ_STAGE(8, 4)
#undef EPTQ_STAGE
        default: break;
      }
    }
    // Every wave's y stores complete at device scope, then the workgroup
    // arrives (this barrier also ends all LDS reads of the stage).
    // (The builtin, not inline asm: the compiler's wait-count tracking sees
    // it and knows every earlier load has landed.)
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (tid == 0) last = arrive(sync, s, NG, grp, gsz, E1);
    // The next stage's index ring right away: it streams while the other
    // workgroups finish and while this one waits for its input.
    if (s + 1 < n_stages) {
      st.crb = nx.crb; st.cre = nx.cre; st.nrb = nx.nrb; st.nre = nx.nre;
      prefetch_stage(view_stage(dnext), st);
    }
    dcur = dnext;
    dnext = dnn;
  }
  if (tid == 0 && (unsigned)add_dev(sync + kExit, 1) == (unsigned)E1 * G - 1u) st_dev(sync + kEpoch, E1);
}

}  // namespace

struct ChainPlan {
  ChainStage* prog = nullptr;   // device
  int* sync = nullptr;          // device
  int n_stages = 0;
  int G = 0, NG = 0;
  size_t dyn = 0;
  bool has_s = false;
};

// Workgroups per layer in proportion to its row groups (each at least one,
// none more than its row groups); returns the most row groups any workgroup
// walks, or -1 if the layers outnumber the workgroups.
static int split_groups(const ChainStage& cs, int R, int G, int* start) {
  long RGt = 0;
  int RG[kMaxLayers];
  for (int i = 0; i < cs.n; ++i) {
    RG[i] = (cs.l[i].M + R - 1) / R;
    RGt += RG[i];
  }
  start[0] = 0;
  if (RGt <= G) {
    for (int i = 0; i < cs.n; ++i) start[i + 1] = start[i] + RG[i];
    return 1;
  }
  if (G < cs.n) return -1;
  int left = G, steps = 0;
  for (int i = 0; i < cs.n; ++i) {
    const int rest = cs.n - i - 1;
    int g = (int)((long)G * RG[i] / RGt);
    if (g < 1) g = 1;
    if (g > RG[i]) g = RG[i];
    if (g > left - rest) g = left - rest;
    start[i + 1] = start[i] + g;
    left -= g;
    const int st = (RG[i] + g - 1) / g;
    if (st > steps) steps = st;
  }
  return steps;
}

// Row split and workgroup ranges of each stage for a grid of G workgroups.
static int plan_stage(ChainStage& cs, int G) {
  const int N = cs.l[0].N;
  const int nch = N >> 3;
  // Row split S: the one whose slowest workgroup has the least work, with
  // workgroups shared among the layers in proportion to their row groups.
  // A workgroup's time ~ (row groups it walks) x (live chunks per lane + one
  // for the per-row-group epilogue and reduction).
  int best = -1, bestS = 0;
  int bestStart[kMaxLayers + 1];
  for (int S = 1; S <= 4; S *= 2) {
    const int J = chunks_for(nch, S);
    if (!fits(J, N, 1)) continue;
    const int R = kW / S;
    int start[kMaxLayers + 1];
    const int steps = split_groups(cs, R, G, start);
    if (steps < 0) continue;
    const int live = (nch + 64 * S - 1) / (64 * S);
    const int cost = steps * (live + 1);
    if (best < 0 || cost < best) {
      best = cost;
      bestS = S;
      for (int i = 0; i <= cs.n; ++i) bestStart[i] = start[i];
    }
  }
  if (best < 0) return -1;
  cs.cfg = ChainStage::cfg_of(chunks_for(nch, bestS), bestS);
  for (int i = 0; i <= cs.n; ++i) cs.start[i] = bestStart[i];
  for (int i = cs.n; i < kMaxLayers; ++i) {
    cs.start[i + 1] = cs.start[cs.n];
    cs.l[i] = cs.l[0];
  }
  return 0;
}

int chain_create(const ChainStage* stages, int n_stages, ChainPlan** out) {
  *out = nullptr;
  if (n_stages <= 0) return -1;
  ChainPlan* p = new ChainPlan();
  p->n_stages = n_stages;
  p->has_s = stages[0].l[0].S != nullptr;
  size_t dyn = 0;
  for (int s = 0; s < n_stages; ++s) {
    const size_t d = act_lds_bytes(stages[s].l[0].N, 1);
    if (d > dyn) dyn = d;
  }
  p->dyn = dyn;
  const void* kern = p->has_s ? (const void*)k_decode_chain<true> : (const void*)k_decode_chain<false>;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kT, dyn) != hipSuccess || per_cu < 1) {
    delete p;
    return -2;
  }
  if (per_cu > 4) per_cu = 4;
  p->G = cu_count() * per_cu;
  p->NG = p->G >= 32 ? 32 : p->G;
  ChainStage* host = (ChainStage*)malloc(sizeof(ChainStage) * n_stages);
  if (!host) {
    delete p;
    return -2;
  }
  for (int s = 0; s < n_stages; ++s) {
    host[s] = stages[s];
    if (plan_stage(host[s], p->G) != 0) {
      free(host);
      delete p;
      return -1;
    }
  }
  const size_t sync_bytes = (size_t)stage_sync_base(n_stages, p->NG) * sizeof(int);
  bool ok = hipMalloc((void**)&p->prog, sizeof(ChainStage) * n_stages) == hipSuccess &&
            hipMalloc((void**)&p->sync, sync_bytes) == hipSuccess &&
            hipMemcpy(p->prog, host, sizeof(ChainStage) * n_stages, hipMemcpyHostToDevice) == hipSuccess &&
            hipMemset(p->sync, 0, sync_bytes) == hipSuccess && hipDeviceSynchronize() == hipSuccess;
  free(host);
  if (!ok) {
    chain_destroy(p);
    return -2;
  }
  *out = p;
  return 0;
}

int chain_run(const ChainPlan* p, hipStream_t s) {
  if (p->has_s)
    k_decode_chain<true><<<p->G, kT, p->dyn, s>>>(p->prog, p->n_stages, p->sync, p->NG);
  else
    k_decode_chain<false><<<p->G, kT, p->dyn, s>>>(p->prog, p->n_stages, p->sync, p->NG);
  return 0;
}

int chain_check(ChainPlan* p) {
  int err = 0;
  if (hipMemcpy(&err, p->sync + kErr, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess) return -2;
  if (err) {
    const int zero = 0;
    if (hipMemcpy(p->sync + kErr, &zero, sizeof(int), hipMemcpyHostToDevice) != hipSuccess) return -2;
    return 1;
  }
  return 0;
}

int chain_grid(const ChainPlan* p) { return p->G; }

void chain_destroy(ChainPlan* p) {
  if (!p) return;
  if (p->prog) (void)hipFree(p->prog);
  if (p->sync) (void)hipFree(p->sync);
  delete p;
}

}  // namespace eptq

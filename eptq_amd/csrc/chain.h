// Internal interface of the persistent decode chain (chain.hip).
#pragma once

#include "kernels.h"

namespace eptq {

// One stage: up to kMaxLayers E8-D4 layers (batch 1) that read the same x.
// Filled by the C ABI (l, n, wait); the plan adds cfg and start.
struct ChainStage {
  LinearArgs l[kMaxLayers];
  int start[kMaxLayers + 1];   // workgroups [start[i], start[i+1]) serve layer i
  int n;                       // layers
  int cfg;                     // (chunks per lane J, row split S) variant
  int wait;                    // read x only after every earlier stage is done
  static constexpr __host__ __device__ int cfg_of(int J, int S) {
    return (J == 2 ? 0 : J == 4 ? 1 : 2) * 3 + (S == 1 ? 0 : S == 2 ? 1 : 2);
  }
};

struct ChainPlan;

// 0, -1 (a stage outside the kernel's range) or -2 (HIP error).
int chain_create(const ChainStage* stages, int n_stages, ChainPlan** out);
int chain_run(const ChainPlan* p, hipStream_t s);
// 0, 1 (a wait timed out since the last check; cleared) or -2 (HIP error).
int chain_check(ChainPlan* p);
int chain_grid(const ChainPlan* p);
void chain_destroy(ChainPlan* p);

}  // namespace eptq

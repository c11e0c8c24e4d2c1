// Device-side plan of the persistent batch-1 decode-step engine (step.hip):
// one descriptor per stage, written by eptq_step_init into caller memory.
#pragma once

#include <stdint.h>

#include "common.h"

namespace eptq {
namespace step {

constexpr int kMaxStageLayers = 3;   // layers sharing one stage input (q|k|v)
constexpr int kMaxStages = 1024;     // flag stride per launch epoch
constexpr int kRowsMax = 16;         // Q rows of one stage per workgroup

// One E8-D4 layer of a stage; its Q rows occupy [row0, row0 + M) of the
// stage's row space, so its outputs are columns [8·row0, 8·(row0 + M)) of the
// stage output.
struct Layer {
  const int16_t* Q;
  const f16* g;
  const f16* h;
  const f16* bias;        // nullable
  const f16* O;           // nullable when the layer has no critical block
  const int32_t* O_col;
  const int32_t* O_row_ptr;
  int M;
  int row0;
};
static_assert(sizeof(Layer) == 64, "layer descriptor layout");

// Stage input: plain fp16 x (src < 0: ready when the launch starts) or the
// flagged output of an earlier stage src (columns [col, col + N)).
// prep 1: the input is RMSNorm'd first, fp16(x · rsqrt(mean(x²) + eps) · nw).
struct Stage {
  Layer l[kMaxStageLayers];
  const uint16_t* x;      // plain input (src < 0)
  const uint64_t* x_ll;   // flagged output of stage src
  const f16* nw;          // RMSNorm weight (prep 1)
  uint64_t* y_ll;         // this stage's flagged output: word w = outputs 2w, 2w+1 | flag
  uint16_t* y;            // optional plain fp16 copy of the output
  int n_layers, N, nch, nseg;
  int M_tot, src, col, prep;
  float eps;
  int pad_[1];
};
static_assert(sizeof(Stage) % 16 == 0, "stage descriptors are 16-byte aligned");

// Synchronization words at the start of the work area (one 256-byte block),
// then each stage's flagged output.
enum { kEpochWord = 0, kExitWord = 1, kErrorWord = 2 };
constexpr int kSyncBytes = 256;

}  // namespace step
}  // namespace eptq

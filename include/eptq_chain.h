/*
 * eptq_chain.h — batch-1 chains of dependent E8-D4 Linears in one launch.
 *
 * No counterpart in the reference, whose decoder runs one EPTQLinear launch
 * per projection (kernels/linear.py:154-212, timed as a decode step in
 * bench_decode.py:50-71).  A chain is a sequence of stages; each stage is one
 * or more E8-D4 layers that read the same input vector (q|k|v, gate|up), and
 * a stage's input is a slice of the chain input x or of an earlier stage's
 * output, optionally through SwiGLU and an RMSNorm.  One persistent launch
 * runs every stage: one workgroup per compute unit, each stage's index
 * stream requested before its input exists, and stage outputs handed on as
 * tagged words (two fp16 outputs and a 32-bit run number per 8-byte word,
 * one device-coherent store; readers wait for exactly the words they read),
 * so stages need no launch, counter, fence or reset between them.
 *
 * Per stage (layers as in eptq_e8d4_forward_multi, fp16 table, no S_group):
 *   in[c]  = src[src_col + c]                                  (SLICE)
 *          = fp16(silu(src[src_col + c]) * src[src_col + N + c])  (SWIGLU)
 *   with norm_weight: in <- in * w / sqrt(mean(in^2) + eps)
 *   y      = g ⊙ (decode(Q) · (h ⊙ in)ᵀ + CSR(O)) + bias per layer, fp16,
 *            written to the stage's y at each layer's y_offset.
 * The RMSNorm's scalar is applied to the fp32 sums (the Linear is linear), its
 * weight with h; results match an fp32 evaluation of the formula within the
 * decode kernels' 1e-2 relative-L2 bar.
 */
#ifndef EPTQ_CHAIN_H
#define EPTQ_CHAIN_H

#include "eptq_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { EPTQ_CHAIN_SLICE = 0, EPTQ_CHAIN_SWIGLU = 1 };

typedef struct {
  int n_layers;               /* 1..4 E8-D4 layers sharing the stage input */
  const eptq_layer* layers;   /* y_offset: first column of the layer in the stage output (even) */
  int out_features;           /* columns of the stage output */
  int src;                    /* -1: the chain input x; else the index of an earlier stage */
  int src_col;                /* first source column read (even; a multiple of 8 for x) */
  int N;                      /* input length: every layer's in_features (multiple of 8, <= 16384) */
  int act;                    /* EPTQ_CHAIN_SLICE or EPTQ_CHAIN_SWIGLU (stage sources only) */
  const void* norm_weight;    /* NULL, or fp16 (N) RMSNorm weight */
  float eps;                  /* RMSNorm epsilon */
  void* y;                    /* fp16 (out_features) stage output, 4-byte aligned */
} eptq_chain_stage;

/* Filled by eptq_e8d4_chain_plan; read by eptq_e8d4_chain_run.  spin_ticks
 * bounds every wait for a stage input (s_memrealtime ticks, 100 MHz); a
 * wait that expires sets the error word and every workgroup leaves. */
typedef struct {
  const void* codes;
  int n_stages;
  int grid;          /* workgroups: one per compute unit */
  int lds_bytes;     /* dynamic LDS per workgroup */
  int copies;        /* E8-D4 table copies in LDS */
  int slot_bytes;    /* LDS of one activation table */
  int csc_offset;    /* chunk scales within an activation table */
  int pad;
  long long spin_ticks;
  long long work_bytes;
} eptq_chain_plan;

/* Bytes of the chain workspace for these stages (0 and an error if the
 * stages are outside what the kernel takes). */
long long eptq_e8d4_chain_work_bytes(const eptq_chain_stage* stages, int n_stages);

/*
 * Validate the stages, write the device plan into `work` (work_bytes from
 * eptq_e8d4_chain_work_bytes, 256-byte aligned) and clear its run counter,
 * error word and tagged buffers.  Synchronous (it copies the plan from host
 * memory); the stages' layers and outputs must stay allocated while the plan
 * is in use.
 */
int eptq_e8d4_chain_plan(const eptq_chain_stage* stages, int n_stages, const void* codes, void* work,
                         long long work_bytes, eptq_chain_plan* plan, void* stream);

/* Run the chain once on fp16 input x (the length its x-sourced stages
 * read).  Asynchronous, no allocation, no host synchronization; runs of one
 * workspace must not overlap in time. */
int eptq_e8d4_chain_run(const eptq_chain_plan* plan, void* work, const void* x, void* stream);

/* The workspace's error word (1: a stage input wait expired; every run since
 * has left at once), read after `stream` drains; clear != 0 resets it. */
int eptq_e8d4_chain_error(void* work, int clear, int* err, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EPTQ_CHAIN_H */

/*
 * eptq_hip.h — C ABI of the MI355X (gfx950) EPTQ quantized-Linear library.
 *
 * Every entry point takes plain device pointers and sizes, allocates no
 * device memory, keeps no pointer after returning, and returns EPTQ_OK or an
 * error code; eptq_last_error() then describes the failure (per host
 * thread).  The compute entry points take a hipStream_t (passed as void*) and
 * launch asynchronously on it; the two exceptions, eptq_step_init and
 * eptq_step_status, synchronize and say so where they are declared.
 *
 * Layer format (reference config.py:98-159, kernels/linear.py:83-152):
 *   Q          int16 (M, N) row-major, stored as index - 32768; 32767 marks a
 *              critical 8-row block.  M = out_features / 8, N = in_features.
 *   g          fp16 (8M)          row scales
 *   h          fp16 (N)           column scales
 *   O_vals     fp16 (nnz, 8)      critical blocks, row-major marker order
 *   O_col      int32 (nnz)        column of each critical block
 *   O_row_ptr  int32 (M + 1)      CSR row pointers into O_vals / O_col
 *   bias       fp16 (8M) or NULL
 *   S_group    fp16 (n_groups, N) or NULL; qb = 8M / n_groups must be a
 *              multiple of 8 (reference algorithms/eptq.py:74, :440-449)
 *   codes      E8-D4: (512, 4) table, E8: (65535, 8) table, fp16 or fp32
 *              (codes_dtype), already divided by the layer's radius.
 *   x          fp16 or bf16 (B, N) row-major; y same dtype as x_dtype
 *              (B, 8M) row-major.
 *
 * Alignment: Q, x, h, O_vals and S_group must be 16-byte aligned and N a
 * multiple of 8 (EPTQ_EUNSUPPORTED otherwise).
 */
#ifndef EPTQ_HIP_H
#define EPTQ_HIP_H

#ifdef __cplusplus
extern "C" {
#endif

enum {
  EPTQ_OK = 0,
  EPTQ_EINVAL = 1,        /* null pointer / negative size / inconsistent args */
  EPTQ_EUNSUPPORTED = 2,  /* shape or alignment outside what the kernels take */
  EPTQ_EHIP = 3,          /* HIP runtime reported an error at launch */
  EPTQ_ETIMEOUT = 4       /* a decode-step stage wait gave up (results invalid) */
};

enum { EPTQ_F16 = 0, EPTQ_F32 = 1, EPTQ_BF16 = 2 };

/* ABI revision; bumped on any signature change. */
int eptq_abi_version(void);

/* Text of the last error on this host thread ("" if none). */
const char* eptq_last_error(void);

/*
 * Fused E8-D4 quantized Linear: y = g ⊙ (decode(Q) · (h ⊙ x)ᵀ + CSR(O)) + bias.
 * Replaces e8d4_forward (reference csrc/eptq_kernels.h:31-41, dispatch
 * csrc/eptq_kernels.cu:466-558) and the Triton decode path
 * (kernels/triton_e8d4.py:160-193).  Adds the optional S_group operand that
 * the reference serves with a materialized fp16 W (kernels/linear.py:97-120).
 * B <= 16 runs the HBM-bound decode matvec; larger B the dequant-to-LDS
 * MFMA GEMM.
 */
int eptq_e8d4_forward(const void* Q, const void* codes, int codes_dtype,
                      const void* g, const void* h, const void* x, int x_dtype,
                      const void* O_vals, const void* O_col, const void* O_row_ptr,
                      const void* bias, const void* S_group, int n_groups,
                      int M, int N, int B, void* y, void* stream);

/* Per-layer operands of eptq_e8d4_forward_multi (meaning as in
 * eptq_e8d4_forward); the layer writes columns [y_offset, y_offset + 8M) of
 * every row of y. */
typedef struct {
  const void* Q;
  const void* g;
  const void* h;
  const void* O_vals;
  const void* O_col;
  const void* O_row_ptr;
  const void* bias;      /* or NULL */
  const void* S_group;   /* or NULL */
  int n_groups;
  int M;
  long long y_offset;    /* multiple of 4 */
} eptq_layer;

/*
 * Several E8-D4 layers that read the same activations x (B, N) — e.g. q, k
 * and v, or gate and up — into one output y (B, ldy), in one launch of the
 * decode matvec when it takes them all (up to 4 layers, B <= 16, fp16 table;
 * fp16 x for B > 8; B of 17..128 as one such launch per 16 rows, fp16 x),
 * otherwise one launch per layer.  Each layer keeps its own h, g, CSR, bias
 * and S_group, so unlike a concatenated weight it needs no shared column
 * scales.  No counterpart in the reference, whose decoder calls one
 * EPTQLinear per projection (kernels/linear.py:154-212); its callers are
 * decode steps that want fewer launches per token.
 *
 * work: NULL, or a 16-byte aligned device buffer of work_bytes bytes,
 * zero-filled before its first use (eptq_e8d4_work_bytes() bytes cover every
 * launch).  With it, batches (or 16-row slices) of 5..16 rows on layers with
 * few 64-row tiles have
 * each tile's columns split over up to 4 workgroups, whose fp32 partial sums
 * meet in the buffer; the kernel leaves its counters at zero.  Calls that
 * share a buffer must not run at the same time.
 */
int eptq_e8d4_forward_multi(int n_layers, const eptq_layer* layers, const void* codes,
                            int codes_dtype, const void* x, int x_dtype, int N, int B, void* y,
                            int ldy, void* work, long long work_bytes, void* stream);

/* Bytes of the eptq_e8d4_forward_multi workspace for the current device. */
long long eptq_e8d4_work_bytes(void);

/*
 * eptq_e8d4_forward_multi with no workspace argument and no allocation: the
 * split-K workspace is the library's own scratch, a static device array of
 * EPTQ_NOALLOC_SCRATCH_BYTES per GPU (tile counters, then partial sums),
 * held by each GPU the library runs on until the process ends.  No
 * counterpart in the reference; for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, checks and results as eptq_e8d4_forward_multi with a
 * workspace of that size.
 *
 * Limit: at most 16384 tiles of 64 output rows (1048576 rows) over all layers
 * of a call, else EPTQ_EUNSUPPORTED.  The first call on a device looks the
 * array up and queues a kernel on `stream` that zeroes its counters (make
 * that call outside graph capture); every launch that uses a counter returns
 * it to zero.  All calls on one GPU share its array, which keeps the last
 * call's contents: calls that overlap in time on one GPU race (wrong
 * results), whatever their streams.
 */
#define EPTQ_NOALLOC_SCRATCH_BYTES 1114112
int eptq_e8d4_forward_multi_noalloc(int n_layers, const eptq_layer* layers, const void* codes,
                                    int codes_dtype, const void* x, int x_dtype, int N, int B, void* y,
                                    int ldy, void* stream);

/*
 * Decode-step engine (batch 1, E8-D4, fp16): a sequence of dependent Linear
 * stages — a decode step's q|k|v, o, gate|up and down for every transformer
 * layer — run by ONE persistent launch, one workgroup per compute unit.  The
 * index stream of later stages is in flight while a stage waits for its
 * input, so the per-launch fixed cost of eptq_e8d4_forward_multi (launch gap,
 * first-load latency, drain) is paid once per step instead of once per stage.
 *
 * A stage is 1..3 layers that read the same input (outputs side by side in
 * layer order, as eptq_e8d4_forward_multi with consecutive y_offsets; the
 * layers' y_offset fields are ignored; no S_group).  Its input is either a
 * plain fp16 (1, N) vector x (src = -1) or columns [col, col + N) of the
 * output of an earlier stage src; with norm_w it is RMSNorm'd first:
 * fp16(x · rsqrt(mean(x²) + eps) · norm_w).  Stage outputs live in the work
 * area in a flagged form (each 8-byte word: two fp16 outputs and a 32-bit
 * flag), so a stage boundary costs one store and one poll; y, if given,
 * receives a plain fp16 copy of the stage's output.
 *
 * Limits: N a multiple of 8 and <= 11264; n_layers·N <= 12288; N <= 4096
 * for a stage with norm_w; col a multiple of 4; at most 16 Q rows of a stage
 * per compute unit (ΣM <= 16 · CUs); at most 1024 stages.
 *
 * No counterpart in the reference, whose decode step calls one Linear per
 * projection (bench_decode.py:44-71, kernels/linear.py:154-212); its callers
 * are batch-1 decode loops.
 */
typedef struct {
  int n_layers;               /* 1..3 */
  const eptq_layer* layers;
  int N;                      /* in_features of the layers */
  int src;                    /* -1: plain input x; else an earlier stage */
  const void* x;              /* (1, N) fp16 device, 16-byte aligned (src < 0) */
  int col;                    /* first input column of stage src's output */
  const void* norm_w;         /* fp16 (N) RMSNorm weight, or NULL */
  float eps;
  void* y;                    /* (1, 8·ΣM) fp16 device copy of the output, or NULL */
} eptq_step_stage;

/* Launch parameters filled by eptq_step_init (host memory). */
typedef struct {
  int n_stages;
  int grid;
  int dyn_lds;
  int lds[4];
} eptq_step_launch;

/* Bytes of the device plan for n_stages stages. */
long long eptq_step_plan_bytes(int n_stages);

/* Bytes of the device work area (synchronization words and every stage's
 * flagged output) for these stages. */
long long eptq_step_work_bytes(int n_stages, const eptq_step_stage* stages);

/* Validate the stages and write the plan (plan: eptq_step_plan_bytes bytes,
 * 16-byte aligned device memory) and a zeroed work area (work:
 * eptq_step_work_bytes bytes, 256-byte aligned device memory), both
 * caller-owned; codes: the fp16 (512, 4) table.  Synchronizes the stream:
 * call outside graph capture.  Allocates nothing. */
int eptq_step_init(int n_stages, const eptq_step_stage* stages, const void* codes, void* plan, void* work,
                   eptq_step_launch* launch, void* stream);

/* One run of every stage of the plan: one launch on the stream, no
 * allocation, no synchronization (graph-capturable).  Runs that share a work
 * area must not overlap in time. */
int eptq_step_run(const void* plan, const void* codes, void* work, const eptq_step_launch* launch,
                  void* stream);

/* EPTQ_ETIMEOUT if a stage input wait of an earlier run gave up (its outputs
 * are then invalid), else EPTQ_OK.  Synchronous (reads the work area). */
int eptq_step_status(const void* work);

/*
 * Fused E8-lattice quantized Linear (same math, 8-vector = codes[u]).
 * Replaces e8_forward (reference csrc/eptq_kernels.h:15-25,
 * kernel csrc/eptq_kernels.cu:39-150).
 */
int eptq_e8_forward(const void* Q, const void* codes, int codes_dtype,
                    const void* g, const void* h, const void* x, int x_dtype,
                    const void* O_vals, const void* O_col, const void* O_row_ptr,
                    const void* bias, const void* S_group, int n_groups,
                    int M, int N, int B, void* y, void* stream);

/*
 * Bit-exact dequantization to fp16 W (8M, N) row-major, the device
 * counterpart of dequantize_layer (reference algorithms/eptq.py:406-471):
 * W = fp16_rne((v [· S]) · g · h) with v = fp32 table row, critical blocks
 * overwritten by fp32(O) before the g/h scaling.  codes must be fp32.
 */
int eptq_e8d4_dequant(const void* Q, const void* codes_f32,
                      const void* g, const void* h,
                      const void* O_vals, const void* O_col, const void* O_row_ptr,
                      const void* S_group, int n_groups,
                      int M, int N, void* W, void* stream);

int eptq_e8_dequant(const void* Q, const void* codes_f32,
                    const void* g, const void* h,
                    const void* O_vals, const void* O_col, const void* O_row_ptr,
                    const void* S_group, int n_groups,
                    int M, int N, void* W, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EPTQ_HIP_H */

/*
 * eptq_hip.h — C ABI of the MI355X (gfx950) EPTQ quantized-Linear library.
 *
 * Every entry point takes plain device pointers and sizes, allocates no
 * device memory, keeps no pointer after returning, and returns EPTQ_OK or an
 * error code; eptq_last_error() then describes the failure (per host
 * thread).  The compute entry points take a hipStream_t (passed as void*) and
 * launch asynchronously on it and never synchronize.
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
  EPTQ_ETIMEOUT = 4       /* reserved: no entry point of this revision returns it */
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
 * launch).  With it, batches (or 16-row slices) of 3..16 rows on layers with
 * few 64-row tiles have each tile's columns split over up to 4 workgroups,
 * whose fp32 partial sums meet in the buffer (the kernel leaves its counters
 * at zero), and prefill launches above 128 rows whose tiles leave half the
 * CUs idle or more split K over up to 4 parts whose fp32 sums a second launch
 * adds in part order (a 64 MiB area past the decode part; a smaller buffer
 * only takes the decode split).  Calls that share a buffer must not run at
 * the same time.
 */
int eptq_e8d4_forward_multi(int n_layers, const eptq_layer* layers, const void* codes,
                            int codes_dtype, const void* x, int x_dtype, int N, int B, void* y,
                            int ldy, void* work, long long work_bytes, void* stream);

/* Bytes of the eptq_e8d4_forward_multi workspace for the current device
 * (the decode split-K area, then the 64 MiB prefill split-K area). */
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
 * Limit: the scratch holds 16384 tile counters and partial sums for 256
 * CUs; a launch with more than 16384 tiles of 64 output rows (1048576 rows
 * over its layers) runs unsplit, exactly as eptq_e8d4_forward_multi does
 * with a workspace of this size.  The first call on a device looks the
 * array up and queues a kernel on `stream` that zeroes its counters (make
 * that call outside graph capture); every launch that uses a counter returns
 * it to zero.  All calls on one GPU share its array, which keeps the last
 * call's contents: calls that overlap in time on one GPU race (wrong
 * results), whatever their streams.
 */
#define EPTQ_NOALLOC_SCRATCH_BYTES 1130496
int eptq_e8d4_forward_multi_noalloc(int n_layers, const eptq_layer* layers, const void* codes,
                                    int codes_dtype, const void* x, int x_dtype, int N, int B, void* y,
                                    int ldy, void* stream);

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

/*
 * Second pass of a two-pass prefill: y (T, ldy) fp16 = x (T, N) fp16 · Wᵀ +
 * bias for fp16 W (F, N) row-major, e.g. from eptq_e8d4_dequant (F = 8M),
 * bias NULL or (F) fp16.  The LDS-DMA GEMM of the fused prefill kernel with
 * W streamed from memory instead of decoded per 256-token tile, so every
 * weight is decoded once per call (by the dequantization) rather than once
 * per token tile.  F and N multiples of 64, ldy >= F and a multiple of 4;
 * W, x 16-byte aligned, y 8-byte aligned; EPTQ_EUNSUPPORTED otherwise.  No
 * counterpart in the reference, whose module runs the fused kernel
 * (csrc/eptq_kernels.cu:309-461) or a dense matmul; callers are prefills
 * long enough that decoding W once pays for writing and reading it.
 */
int eptq_f16_gemm(const void* W, const void* x, const void* bias, int F, int N, int T,
                  void* y, int ldy, void* stream);

/*
 * eptq_f16_gemm with a per-token scale and a choice of output type:
 * y[t] = row_scale[t] · (x[t] · Wᵀ) + bias, rounded to fp16 (y_dtype
 * EPTQ_F16) or bf16 (EPTQ_BF16); row_scale NULL (1) or T fp32 values, 4-byte
 * aligned.  With eptq_bf16_rows_to_f16 below it is the two-pass prefill for
 * bf16 activations.  No counterpart in the reference (as eptq_f16_gemm).
 */
int eptq_f16_gemm_rows(const void* W, const void* x, const void* bias, int F, int N, int T,
                       const void* row_scale, void* y, int y_dtype, int ldy, void* stream);

/*
 * bf16 activations x (T, N) to the fp16 operand of eptq_f16_gemm_rows:
 * x16[t] = fp16(x[t] · 2^-e_t), row_scale[t] = 2^e_t (fp32), e_t chosen so
 * the row's largest magnitude lands in [2^14, 2^15) — exact for every element
 * within 2^-28 of the row's maximum (bf16 has 8 significand bits, fp16 11).
 * N a multiple of 8 up to 16384, x and x16 16-byte aligned, no overlap;
 * EPTQ_EUNSUPPORTED / EPTQ_EINVAL otherwise.  No counterpart in the
 * reference; the caller owns x16 (T·N·2 bytes) and row_scale (T·4 bytes).
 */
int eptq_bf16_rows_to_f16(const void* x, int N, int T, void* x16, void* row_scale, void* stream);

int eptq_e8_dequant(const void* Q, const void* codes_f32,
                    const void* g, const void* h,
                    const void* O_vals, const void* O_col, const void* O_row_ptr,
                    const void* S_group, int n_groups,
                    int M, int N, void* W, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EPTQ_HIP_H */

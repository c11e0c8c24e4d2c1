/*
 * eptq_llama.h — fused decode-step operators of the synthetic Llama harness
 * (eptq_amd/llama.py), in the same library as eptq_hip.h.
 *
 * No counterpart in the reference's kernel API: the reference runs these
 * parts of a decoder layer as HuggingFace/PyTorch ops (LlamaRMSNorm, rotary
 * embedding, attention over a StaticCache, SiLU gating) driven by
 * bench_decode.py:44-71.  Same conventions as eptq_hip.h: device pointers,
 * fp16 data, asynchronous on `stream`, no allocation; 0 = ok, 1 = invalid
 * argument, 2 = unsupported shape, 3 = HIP launch error.
 */
#ifndef EPTQ_LLAMA_H
#define EPTQ_LLAMA_H

#include "eptq_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* x (B, H) += delta (B, H) when delta is not NULL (the residual add), then
 * y (B, H) = w ⊙ x · rsqrt(mean(x²) + eps).  H % 8 == 0, H <= 16384. */
int eptq_llama_rmsnorm(void* x, const void* delta, const void* w, void* y, int B, int H, float eps,
                       void* stream);

/* Decode attention at position *pos (int64 on the device) for every (head,
 * batch row): rotary on q and k (cos/sin (L, D) fp32 tables), k and v written
 * to the caches (B, Hk, L, D) at pos, out (B, H·D) = softmax(q·Kᵀ/√D)·V over
 * positions 0..pos.  qkv is (B, (H + 2 Hk)·D): [q heads | k heads | v heads].
 * D == 128, H % Hk == 0, L <= 1024.
 * work: NULL (one workgroup per (head, batch row)) or a 16-byte aligned
 * device buffer of eptq_llama_attn_work_bytes(B, H) bytes, zero-filled
 * before its first use, with which the positions of each (head, batch row)
 * are split over several workgroups (softmax partials combined by the last
 * one).  The kernel leaves the buffer's counters at zero; calls that share a
 * buffer must not run concurrently. */
int eptq_llama_rope_attn(const void* qkv, const void* pos, const void* cos_tab, const void* sin_tab,
                         void* k_cache, void* v_cache, void* out, int B, int H, int Hk, int D, int L,
                         void* work, void* stream);

/* Bytes of the eptq_llama_rope_attn workspace for B batch rows and H heads. */
long long eptq_llama_attn_work_bytes(int B, int H);

/* out (B, F) = silu(gate) ⊙ up with gate_up (B, 2F) = [gate | up].  F % 8 == 0. */
int eptq_llama_silu_mul(const void* gate_up, void* out, int B, int F, void* stream);

/* The decoder's RMSNorm fused into the E8-D4 layers that read its output
 * (q|k|v or gate|up): r = resid + delta (delta may be NULL), the layers'
 * input is w ⊙ r · rsqrt(mean(r²) + eps) (the same roundings as
 * eptq_llama_rmsnorm), and r is written to resid_out (may be NULL; must not
 * overlap resid or delta).  layers, codes (fp16 table), y and ldy as in
 * eptq_e8d4_forward_multi; resid, delta, resid_out (B, N) fp16; B <= 8.
 * Error codes and eptq_last_error as in eptq_hip.h: EPTQ_EUNSUPPORTED when
 * the decode kernel cannot take the shape (then run eptq_llama_rmsnorm and
 * the Linear apart). */
int eptq_llama_norm_linear(int n_layers, const eptq_layer* layers, const void* codes,
                           const void* resid, const void* delta, const void* w, float eps,
                           void* resid_out, int N, int B, void* y, int ldy, void* stream);

/* The feed-forward input of a decoder layer in one launch (SwiGLU): the
 * RMSNorm of eptq_llama_norm_linear (r = resid + delta written to resid_out,
 * t = w ⊙ r · rsqrt(mean(r²) + eps)), then out (B, F) = silu(gate(t)) ⊙ up(t)
 * with gate_up[0] = gate, gate_up[1] = up of equal M and F = 8·M; each factor
 * is rounded to fp16 before the product, so out is bit-identical to
 * eptq_llama_norm_linear followed by eptq_llama_silu_mul when both layers
 * run whole-row waves there.  The layers' y_offset fields are not used.
 * B <= 2; EPTQ_EUNSUPPORTED for larger batches or shapes the kernel does not
 * take (then run eptq_llama_norm_linear and eptq_llama_silu_mul).  No
 * counterpart in the reference, whose decode step runs the gate and up
 * Linears and the SiLU product as separate operators (bench_decode.py). */
int eptq_llama_norm_swiglu(const eptq_layer* gate_up, const void* codes, const void* resid, const void* delta,
                           const void* w, float eps, void* resid_out, int N, int B, void* out, void* stream);

/* A decoder Linear group on the matrix-core decode kernel, with the RMSNorm
 * before it and the residual add after it folded in (the fused forms of
 * eptq_llama_norm_linear and eptq_llama_norm_swiglu take B <= 2 only):
 *   y = Linear(t) (+ resid),  t = x, or t = RMSNorm(x) = norm_w ⊙ x ·
 *   rsqrt(mean(x²) + eps) when norm_w is not NULL.
 * The norm is applied as Linear(norm_w ⊙ x) · rsqrt(mean(x²) + eps) per batch
 * row, so t is not rounded to fp16 (the result agrees with eptq_llama_rmsnorm
 * then the Linear to fp16 rounding, not bit for bit).  With resid (laid out
 * like y; it may be y itself) y = fp16(resid + fp16(Linear)), bit-identical to
 * the Linear followed by the residual add of eptq_llama_rmsnorm.  layers,
 * codes (fp16 table), y, ldy, work and work_bytes as in
 * eptq_e8d4_forward_multi; x (B, N) fp16 must not overlap y or resid; norm_w
 * (N) fp16, 16-byte aligned.  EPTQ_EUNSUPPORTED when the matrix-core kernel
 * does not take the call (B > 16, or B > 8 or N % 64 != 0 with norm_w; then
 * run eptq_llama_rmsnorm, the Linear and the add apart).  No counterpart in
 * the reference, whose decode step runs the norms, Linears and residual adds
 * as separate operators (bench_decode.py:44-71). */
int eptq_llama_linear(int n_layers, const eptq_layer* layers, const void* codes, const void* x, int N, int B,
                      const void* norm_w, float eps, const void* resid, void* y, int ldy, void* work,
                      long long work_bytes, void* stream);

/* eptq_llama_linear for the feed-forward gate and up layers with the SwiGLU
 * product in the same launch: gu (B, 2F) fp16 = [gate(t) | up(t)] as
 * eptq_llama_linear writes them (F = 8·M, the layers' y_offset fields are
 * not used), and out (B, F) = silu(gate) ⊙ up, bit-identical to
 * eptq_llama_linear followed by eptq_llama_silu_mul.  Whichever of a row
 * tile's two workgroups finishes second forms the product, meeting the
 * other at a counter in work, which is required (as in eptq_llama_linear;
 * the counters return to zero).  out 4-byte aligned, not overlapping gu or
 * x.  EPTQ_EUNSUPPORTED where eptq_llama_linear is, for a work buffer
 * smaller than its counter area, or for tile counts past it.  No
 * counterpart in the reference, whose decode step runs the gate and up
 * Linears and the SiLU product as separate operators (bench_decode.py). */
int eptq_llama_linear_swiglu(const eptq_layer* gate_up, const void* codes, const void* x, int N, int B,
                             const void* norm_w, float eps, void* gu, void* out, void* work, long long work_bytes,
                             void* stream);

/* Bytes of the eptq_llama_lm_head_argmax workspace for B batch rows
 * (zero-filled before its first use; every call leaves it zeroed). */
long long eptq_llama_lm_head_work_bytes(int B);

/* The decode step's tail in one launch: t = w ⊙ r · rsqrt(mean(r²) + eps) for
 * r = x + delta (delta may be NULL; the roundings of eptq_llama_rmsnorm),
 * logits (B, V) fp16 = t · Wᵀ for the fp16 lm_head weight W (V, H) row-major,
 * tok[b] (int64) = the index of the largest fp16 logit of row b (the smallest
 * index among equal ones), and *pos += 1 (int64) when pos is not NULL.
 * work: eptq_llama_lm_head_work_bytes(B) bytes, 8-byte aligned; calls sharing
 * it must not overlap in time.  B <= 8, H in {4096, 6144, 8192} and B·H·2 <=
 * 128 KB; 2 (unsupported) otherwise.  No counterpart in the reference, which runs the
 * final norm, lm_head and argmax as separate ops (bench_decode.py:44-71). */
int eptq_llama_lm_head_argmax(const void* x, const void* delta, const void* w, float eps, const void* W, int V,
                              int H, int B, void* logits, void* tok, void* pos, void* work, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EPTQ_LLAMA_H */

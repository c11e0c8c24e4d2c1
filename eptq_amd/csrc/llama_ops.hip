// Fused decode-step operators of the synthetic Llama harness (gfx950).
//
// The reference runs these parts of a decoder layer as HuggingFace/PyTorch
// ops (LlamaRMSNorm, rotary embedding, SDPA attention over a StaticCache, SiLU
// gating; bench_decode.py:44-71 drives them); here each group of them is one
// kernel so that a decode step is 8 launches per layer.  They have no
// counterpart in the reference's kernel API (include/eptq_llama.h).
//
//  * k_rmsnorm:     x += delta (optional, the residual add), y = w ⊙ x / rms(x).
//  * k_rope_attn:   one workgroup per (head, batch row) at decode position
//                   pos: rotary on q and the head's k, k/v written to the cache
//                   at pos, softmax(q·Kᵀ/√D)·V over positions 0..pos.
//  * k_silu_mul:    a = silu(gate) ⊙ up from the fused gate|up projection.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "eptq_llama.h"

namespace eptq {
namespace {

constexpr int kT = 256;
constexpr int kMaxSplit = 16;   // position splits per (batch row, head)

__device__ __forceinline__ float block_sum(float v, float* sh) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) sh[w] = v;
  __syncthreads();
  float t = 0.0f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += sh[i];
  return t;
}

__device__ __forceinline__ float block_max(float v, float* sh) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) sh[w] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t = fmaxf(t, sh[i]);
  return t;
}

// One workgroup per row; H a multiple of 8, H <= 8 * kT * 8.
__global__ __launch_bounds__(kT) void k_rmsnorm(f16* __restrict__ x, const f16* __restrict__ delta,
                                               const f16* __restrict__ w, f16* __restrict__ y,
                                               int H, float eps) {
  __shared__ float sh[kT / 64];
  const int row = blockIdx.x;
  f16* xr = x + (size_t)row * H;
  const f16* dr = delta ? delta + (size_t)row * H : nullptr;
  constexpr int MAXV = 8;   // 8-element vectors per thread (H <= 16384)
  f16x8 v[MAXV];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < MAXV; ++k) {
    const int c = threadIdx.x + kT * k;
    if (c * 8 < H) {
      f16x8 a = *(const f16x8*)(xr + c * 8);
      if (dr) {
        const f16x8 d = *(const f16x8*)(dr + c * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = (f16)((float)a[e] + (float)d[e]);
        *(f16x8*)(xr + c * 8) = a;
      }
      v[k] = a;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (float)a[e] * (float)a[e];
    }
  }
  const float inv = rsqrtf(block_sum(ss, sh) / (float)H + eps);
#pragma unroll
  for (int k = 0; k < MAXV; ++k) {
    const int c = threadIdx.x + kT * k;
    if (c * 8 < H) {
      const f16x8 wv = *(const f16x8*)(w + c * 8);
      f16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (f16)((float)v[k][e] * inv * (float)wv[e]);
      *(f16x8*)(y + (size_t)row * H + c * 8) = o;
    }
  }
}

// Decode attention for head h of batch row b, head_dim D = 128, positions
// 0..pos split over ns workgroups (blockIdx.z): each computes the softmax
// partial of its positions (local max m, sum l of exp(s - m), o = Σ exp(s - m)
// V), and the last of the ns to finish (an atomic count per (b, h)) rescales
// and sums them:  out = Σ_s o_s e^(m_s - M) / Σ_s l_s e^(m_s - M), M = max m_s.
// Partials move through device-coherent (sc1) stores and loads, and each
// split waits for its stores (vmcnt) before it counts itself, so no cache
// writeback or invalidate is needed across XCDs; the last split resets the
// count to zero for the next call.  ns = 1 (no workspace) writes directly.
// qkv: (B, (H + 2 Hk) D) = [q heads | k heads | v heads]; caches (B, Hk, L, D);
// cos/sin: (L, D) fp32 (HF rotary layout: frequencies repeated over both halves).
constexpr int kPart = 2 + 128;   // floats per partial: m, l, o[128]

__device__ __forceinline__ void st_coh(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coh(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(kT) void k_rope_attn(const f16* __restrict__ qkv, const int64_t* __restrict__ posp,
                                                 const float* __restrict__ cosv, const float* __restrict__ sinv,
                                                 f16* __restrict__ kc, f16* __restrict__ vc, f16* __restrict__ out,
                                                 int H, int Hk, int L, float scale, float* __restrict__ part,
                                                 int* __restrict__ cnt) {
  constexpr int D = 128;
  __shared__ float qs[D], ks[D], vs[D];
  __shared__ float prob[1024];
  __shared__ float sh[kT / 64];
  __shared__ float opart[16][D];
  __shared__ int s_last;
  const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int sp = blockIdx.z, ns = gridDim.z;
  const int hk = h / (H / Hk);
  const int64_t pos64 = *posp;
  if (pos64 < 0 || pos64 >= L) {   // outside the cache: no cache access, zero output
    if (sp == 0 && t < D) out[(size_t)b * H * D + (size_t)h * D + t] = (f16)0.0f;
    return;
  }
  const int pos = (int)pos64;
  // This split's positions [p0, p1) of 0..pos.
  const int per = (pos + 1 + ns - 1) / ns;
  const int p0 = sp * per;
  const int p1 = p0 + per < pos + 1 ? p0 + per : pos + 1;
  const size_t row = (size_t)b * (H + 2 * Hk) * D;
  const f16* q = qkv + row + (size_t)h * D;
  const f16* k = qkv + row + (size_t)(H + hk) * D;
  const f16* v = qkv + row + (size_t)(H + Hk + hk) * D;
  if (t < D) {
    qs[t] = (float)q[t];
    ks[t] = (float)k[t];
    vs[t] = (float)v[t];
  }
  __syncthreads();
  float qr = 0.0f, kr = 0.0f;
  if (t < D) {
    const float c = cosv[(size_t)pos * D + t], s = sinv[(size_t)pos * D + t];
    const float qrot = t < D / 2 ? -qs[t + D / 2] : qs[t - D / 2];
    const float krot = t < D / 2 ? -ks[t + D / 2] : ks[t - D / 2];
    // fp16 rounding of the rotated q and k, as a fp16 model holds them
    qr = (float)(f16)(qs[t] * c + qrot * s);
    kr = (float)(f16)(ks[t] * c + krot * s);
  }
  __syncthreads();
  if (t < D) {
    qs[t] = qr;
    ks[t] = kr;
  }
  const size_t kvbase = ((size_t)b * Hk + hk) * L * D;
  if (sp == 0 && h % (H / Hk) == 0 && t < D) {   // one writer per kv head
    kc[kvbase + (size_t)pos * D + t] = (f16)kr;
    vc[kvbase + (size_t)pos * D + t] = (f16)vs[t];
  }
  __syncthreads();

  // Scores for positions p = p0 + t, + kT, ... < p1 (the current one from
  // LDS): each thread reads its key rows with 16-byte loads, issued together.
  float mx = -INFINITY;
  for (int p = p0 + t; p < p1; p += kT) {
    float s = 0.0f;
    if (p == pos) {
      for (int d = 0; d < D; ++d) s += qs[d] * ks[d];
    } else {
      const f16x8* kp = (const f16x8*)(kc + kvbase + (size_t)p * D);
      f16x8 kv8[D / 8];
#pragma unroll
      for (int c = 0; c < D / 8; ++c) kv8[c] = kp[c];
#pragma unroll
      for (int c = 0; c < D / 8; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) s += qs[c * 8 + e] * (float)kv8[c][e];
    }
    s *= scale;
    prob[p - p0] = s;
    mx = fmaxf(mx, s);
  }
  mx = block_max(mx, sh);
  float sum = 0.0f;
  for (int p = p0 + t; p < p1; p += kT) {
    const float e = __expf(prob[p - p0] - mx);
    prob[p - p0] = e;
    sum += e;
  }
  sum = block_sum(sum, sh);   // block_sum synchronizes: prob[] complete
  // o = Σ_p prob[p] V[p]: thread (pg, dc) takes 8 dims dc·8.. of the
  // positions p ≡ p0 + pg (mod 16), four rows in flight, then the 16 position
  // groups are summed through LDS.
  const int dc = t & 15, pg = t >> 4;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const f16* vb = vc + kvbase + dc * 8;
  int p = p0 + pg;
  for (; p + 48 < p1 && p + 48 < pos; p += 64) {
    f16x8 v4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v4[u] = *(const f16x8*)(vb + (size_t)(p + 16 * u) * D);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float pr = prob[p + 16 * u - p0];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += pr * (float)v4[u][e];
    }
  }
  for (; p < p1; p += 16) {
    const float pr = prob[p - p0];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float vv = p == pos ? vs[dc * 8 + e] : (float)vb[(size_t)p * D + e];
      acc[e] += pr * vv;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) opart[pg][dc * 8 + e] = acc[e];
  __syncthreads();
  float o = 0.0f;
  if (t < D) {
#pragma unroll
    for (int g2 = 0; g2 < 16; ++g2) o += opart[g2][t];
  }
  f16* orow = out + (size_t)b * H * D + (size_t)h * D;
  if (ns == 1) {
    if (t < D) orow[t] = (f16)(o / sum);
    return;
  }
  // Publish this split's partial, then count it.
  const int bh = b * H + h;
  float* mine = part + ((size_t)bh * ns + sp) * kPart;
  if (t < D) st_coh(mine + 2 + t, o);
  if (t == 0) {
    st_coh(mine, mx);
    st_coh(mine + 1, sum);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the stores are complete
  __syncthreads();
  if (t == 0) {
    const int prev = __hip_atomic_fetch_add(cnt + bh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == ns - 1;
    if (prev == ns - 1) __hip_atomic_store(cnt + bh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  const float* all = part + (size_t)bh * ns * kPart;
  float M = -INFINITY;
  for (int s2 = 0; s2 < ns; ++s2) M = fmaxf(M, ld_coh(all + s2 * kPart));
  float lsum = 0.0f, osum = 0.0f;
  for (int s2 = 0; s2 < ns; ++s2) {
    const float* ps = all + s2 * kPart;
    const float w = __expf(ld_coh(ps) - M);   // empty splits: m = -inf, weight 0
    lsum += ld_coh(ps + 1) * w;
    if (t < D) osum += ld_coh(ps + 2 + t) * w;
  }
  if (t < D) orow[t] = (f16)(osum / lsum);
}

__global__ __launch_bounds__(kT) void k_silu_mul(const f16* __restrict__ gu, f16* __restrict__ a, int F) {
  const int b = blockIdx.y;
  const int c = blockIdx.x * kT + threadIdx.x;   // 8-element vector index
  if (c * 8 >= F) return;
  const f16x8 g = *(const f16x8*)(gu + (size_t)b * 2 * F + c * 8);
  const f16x8 u = *(const f16x8*)(gu + (size_t)b * 2 * F + F + c * 8);
  f16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float gf = (float)g[e];
    o[e] = (f16)(gf / (1.0f + __expf(-gf)) * (float)u[e]);
  }
  *(f16x8*)(a + (size_t)b * F + c * 8) = o;
}

}  // namespace
}  // namespace eptq

extern "C" {

// Return codes as in eptq_hip.h: 0 ok, 1 invalid argument, 3 HIP launch error.

int eptq_llama_rmsnorm(void* x, const void* delta, const void* w, void* y, int B, int H, float eps,
                       void* stream) {
  if (!x || !w || !y || B <= 0 || H <= 0 || H % 8 || H > 8 * 256 * 8) return 1;
  hipLaunchKernelGGL(eptq::k_rmsnorm, dim3(B), dim3(256), 0, (hipStream_t)stream, (eptq::f16*)x,
                     (const eptq::f16*)delta, (const eptq::f16*)w, (eptq::f16*)y, H, eps);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

long long eptq_llama_attn_work_bytes(int B, int H) {
  if (B <= 0 || H <= 0) return 0;
  return (long long)B * H * (eptq::kMaxSplit * eptq::kPart * 4 + 4);
}

int eptq_llama_rope_attn(const void* qkv, const void* pos, const void* cos_tab, const void* sin_tab,
                         void* k_cache, void* v_cache, void* out, int B, int H, int Hk, int D, int L,
                         void* work, void* stream) {
  if (!qkv || !pos || !cos_tab || !sin_tab || !k_cache || !v_cache || !out) return 1;
  if (B <= 0 || H <= 0 || Hk <= 0 || H % Hk || D != 128 || L <= 0 || L > 1024) return 1;
  if (work && ((uintptr_t)work & 15)) return 1;
  // Position splits: enough workgroups to cover the CUs (the cache reads are
  // the work), at most kMaxSplit; one without a workspace.
  int ns = 1;
  if (work) {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    ns = (cus + B * H - 1) / (B * H);
    if (ns > eptq::kMaxSplit) ns = eptq::kMaxSplit;
    if (ns < 1) ns = 1;
  }
  float* part = (float*)work;
  int* cnt = work ? (int*)(part + (size_t)B * H * eptq::kMaxSplit * eptq::kPart) : nullptr;
  hipLaunchKernelGGL(eptq::k_rope_attn, dim3(H, B, ns), dim3(256), 0, (hipStream_t)stream,
                     (const eptq::f16*)qkv, (const int64_t*)pos, (const float*)cos_tab,
                     (const float*)sin_tab, (eptq::f16*)k_cache, (eptq::f16*)v_cache, (eptq::f16*)out,
                     H, Hk, L, 1.0f / sqrtf((float)D), part, cnt);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int eptq_llama_silu_mul(const void* gate_up, void* out, int B, int F, void* stream) {
  if (!gate_up || !out || B <= 0 || F <= 0 || F % 8) return 1;
  const int nv = F / 8;
  hipLaunchKernelGGL(eptq::k_silu_mul, dim3((nv + 255) / 256, B), dim3(256), 0, (hipStream_t)stream,
                     (const eptq::f16*)gate_up, (eptq::f16*)out, F);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

}  // extern "C"

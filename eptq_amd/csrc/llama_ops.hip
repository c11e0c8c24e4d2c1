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
//  * k_lm_head_argmax: the step's tail — final RMSNorm, the fp16 lm_head
//                   matvec, the logits, the greedy next token and the position
//                   advance — in one launch (B <= 8).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "decode_layer.h"
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
// 0..pos split over ns workgroups (blockIdx.z).
//
// Layout: thread (pg = t / 16, dc = t % 16) holds dims 8dc..8dc+7 of the
// cache rows p ≡ pg (mod 16) of a 256-row chunk, so one wave load covers four
// whole 256-byte rows (K as well as V: no lane strides across rows).  A
// row's score is the sum of its 16 lanes' partial dot products; the 16 rows of
// a lane group are reduced together by a transposed butterfly (15 DPP adds),
// after which lane dc holds the score of row pg + 16 dc.  Each lane group keeps
// its own online softmax (running max m, rescaled sum l and o = Σ e^(s-m) V),
// so no workgroup-wide barrier separates the chunks; the 16 groups are
// combined once at the end:  out = Σ_g o_g e^(m_g - M) / Σ_g l_g e^(m_g - M).
//
// Unsplit (ns = 1) the first 256 rows are requested at entry, before pos has
// arrived: rows at or past pos are loaded but not used.  Split, the workgroup
// computes the same partial (M, l, o) over its positions [p0, p1), and the
// last of the ns to finish (an atomic count per (b, h)) rescales and sums
// them.  Partials move through device-coherent (sc1) stores and loads, and
// each split waits for its stores (vmcnt) before it counts itself, so no cache
// writeback or invalidate is needed across XCDs; the last split resets the
// count to zero for the next call.
// qkv: (B, (H + 2 Hk) D) = [q heads | k heads | v heads]; caches (B, Hk, L, D);
// cos/sin: (L, D) fp32 (HF rotary layout: frequencies repeated over both halves).
// pos outside [0, L): zero output, no cache access.
constexpr int kPart = 2 + 128;   // floats per partial: m, l, o[128]

__device__ __forceinline__ void st_coh(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coh(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Lane moves within each row of 16 lanes (gfx9 dpp_ctrl): lane i reads lane
// i ^ 15 (row_mirror), i ^ 7 (row_half_mirror), i ^ 3 (quad_perm 3,2,1,0) or
// i ^ 1 (quad_perm 1,0,3,2).  The four masks span all 16 lanes.
constexpr int kX15 = 0x140, kX7 = 0x141, kX3 = 0x1B, kX1 = 0xB1;
template <int CTRL>
__device__ __forceinline__ float dpp16(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, dpp16<kX15>(v));
  v = fmaxf(v, dpp16<kX7>(v));
  v = fmaxf(v, dpp16<kX3>(v));
  return fmaxf(v, dpp16<kX1>(v));
}
__device__ __forceinline__ float sum16(float v) {
  v += dpp16<kX15>(v);
  v += dpp16<kX7>(v);
  v += dpp16<kX3>(v);
  return v + dpp16<kX1>(v);
}
// One halving step of the transposed sum: lanes whose bit B (of lane & 15)
// is clear keep values [0, n), the others [n, 2n), each adding its partner's
// (lane ^ mask, which differs in bit B and agrees in the higher bits).
template <int N, int CTRL>
__device__ __forceinline__ void halve(float (&v)[16], bool hi) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float keep = hi ? v[i + N] : v[i], send = hi ? v[i] : v[i + N];
    v[i] = keep + dpp16<CTRL>(send);
  }
}
// v[u] = this lane's part of row u (u < 16) -> sum over the 16 lanes of row
// (lane & 15).
__device__ __forceinline__ float transpose_sum16(float (&v)[16], int l16) {
  halve<8, kX15>(v, l16 & 8);
  halve<4, kX7>(v, l16 & 4);
  halve<2, kX3>(v, l16 & 2);
  halve<1, kX1>(v, l16 & 1);
  return v[0];
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t cache_rsrc(const f16* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, bytes, 0x00020000);
}
// Rows c + pg + 16u (u < 16), dims 8dc..: keys first (the scores need them
// first), then values.  Offsets past the resource's size read as zero.
__device__ __forceinline__ void load_rows(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv, int c, int pg,
                                          int dc, f16x8 (&kk)[16], f16x8 (&vv)[16]) {
#pragma unroll
  for (int u = 0; u < 16; ++u)
    kk[u] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, ((c + pg + 16 * u) * 128 + dc * 8) * 2, 0, 0));
#pragma unroll
  for (int u = 0; u < 16; ++u)
    vv[u] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, ((c + pg + 16 * u) * 128 + dc * 8) * 2, 0, 0));
}

// Head h of batch row b, split sp of ns.
__device__ __forceinline__ void rope_attn(const f16* __restrict__ qkv, const int64_t* __restrict__ posp,
                                          const float* __restrict__ cosv, const float* __restrict__ sinv,
                                          f16* __restrict__ kc, f16* __restrict__ vc, f16* __restrict__ out,
                                          int H, int Hk, int L, float scale, float* __restrict__ part,
                                          int* __restrict__ cnt, int h, int b, int sp, int ns) {
  constexpr int D = 128;
  __shared__ float probl[16][16];
  __shared__ float opart[16][D];
  __shared__ float gmax[16], gsum[16];
  __shared__ int s_last;
  const int t = threadIdx.x;
  const int grp = H / Hk, hk = h / grp;
  const int dc = t & 15, pg = t >> 4, d0 = dc * 8;
  const size_t kvbase = ((size_t)b * Hk + hk) * L * D;
  f16x8 ka[16], va[16];
  {  // unsplit: rows 0..255 now (an empty resource when split)
    const int bytes = ns == 1 ? L * D * 2 : 0;
    load_rows(cache_rsrc(kc + kvbase, bytes), cache_rsrc(vc + kvbase, bytes), 0, pg, dc, ka, va);
  }
  // This lane's 8 dims of q, k, v and the rotary partners (dims d ± 64).
  const size_t row = (size_t)b * (H + 2 * Hk) * D;
  const f16* q = qkv + row + (size_t)h * D;
  const f16* k = qkv + row + (size_t)(H + hk) * D;
  const f16* v = qkv + row + (size_t)(H + Hk + hk) * D;
  const f16x8 q8 = *(const f16x8*)(q + d0), qp8 = *(const f16x8*)(q + (d0 ^ 64));
  const f16x8 k8 = *(const f16x8*)(k + d0), kp8 = *(const f16x8*)(k + (d0 ^ 64));
  const f16x8 v8 = *(const f16x8*)(v + d0);
  const int64_t pos64 = *posp;
  const bool ok = pos64 >= 0 && pos64 < L;
  const int pos = ok ? (int)pos64 : 0;
  // This split's positions [p0, p1) of 0..pos.
  const int per = (pos + 1 + ns - 1) / ns;
  const int p0 = sp * per;
  const int p1 = p0 + per < pos + 1 ? p0 + per : pos + 1;
  const __amdgpu_buffer_rsrc_t rk = cache_rsrc(kc + kvbase, p1 * D * 2);
  const __amdgpu_buffer_rsrc_t rv = cache_rsrc(vc + kvbase, p1 * D * 2);
  if (ns > 1) load_rows(rk, rv, p0, pg, dc, ka, va);
  // Rotary (q·cos + rotate_half(q)·sin), rounded to fp16 as a fp16 model
  // holds the rotated q and k.
  float qv[8], kv[8];
  {
    const float4* cr = (const float4*)(cosv + (size_t)pos * D + d0);
    const float4* sr = (const float4*)(sinv + (size_t)pos * D + d0);
    const float4 c0 = cr[0], c1 = cr[1], s0 = sr[0], s1 = sr[1];
    const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const float sg = dc < 8 ? -1.0f : 1.0f;   // rotate_half: (-x2, x1)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      qv[e] = (float)(f16)((float)q8[e] * cs[e] + sg * (float)qp8[e] * sn[e]);
      kv[e] = (float)(f16)((float)k8[e] * cs[e] + sg * (float)kp8[e] * sn[e]);
    }
  }
  if (ok && sp == 0 && h % grp == 0 && pg == 0) {   // one writer per kv head
    f16x8 ko;
#pragma unroll
    for (int e = 0; e < 8; ++e) ko[e] = (f16)kv[e];
    *(f16x8*)(kc + kvbase + (size_t)pos * D + d0) = ko;
    *(f16x8*)(vc + kvbase + (size_t)pos * D + d0) = v8;
  }
  // q as fp16 pairs (exact: it is fp16-rounded) for the dot2 products; the
  // current row's k and v come from registers, not the cache.
  f16x2 qh[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) qh[i] = f16x2{(f16)qv[2 * i], (f16)qv[2 * i + 1]};
  float dself = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) dself += qv[e] * kv[e];
  float m = -INFINITY, lsum = 0.0f;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  auto chunk = [&](int c, const f16x8(&kk)[16], const f16x8(&vv)[16]) {
    float pt[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) s = __builtin_amdgcn_fdot2(qh[i], f16x2{kk[u][2 * i], kk[u][2 * i + 1]}, s, false);
      pt[u] = c + pg + 16 * u == pos ? dself : s;
    }
    float s = transpose_sum16(pt, dc) * scale;   // row c + pg + 16 dc
    if (c + pg + 16 * dc >= p1) s = -INFINITY;
    const float mn = fmaxf(m, max16(s));
    const float alpha = mn == -INFINITY ? 1.0f : __expf(m - mn);
    const float e = s == -INFINITY ? 0.0f : __expf(s - mn);
    m = mn;
    lsum = lsum * alpha + e;
    // The group's 16 weights to every lane of the group (one wave: LDS
    // operations of a wave complete in order).
    probl[pg][dc] = e;
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const float4* pr4 = (const float4*)probl[pg];
    const float4 w0 = pr4[0], w1 = pr4[1], w2 = pr4[2], w3 = pr4[3];
    const float w[16] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w,
                         w2.x, w2.y, w2.z, w2.w, w3.x, w3.y, w3.z, w3.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= alpha;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int r = c + pg + 16 * u;
      f16x8 x = r == pos ? v8 : vv[u];
      if (r >= p1) x = f16x8{};   // rows past the range: weight 0, contents unknown
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += w[u] * (float)x[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  };
  if (p0 + 256 < p1) {   // a second chunk: requested before the first is used
    f16x8 kb[16], vb[16];
    load_rows(rk, rv, p0 + 256, pg, dc, kb, vb);
    chunk(p0, ka, va);
    for (int c = p0 + 256; c < p1; c += 256) {
      chunk(c, kb, vb);
      if (c + 256 < p1) load_rows(rk, rv, c + 256, pg, dc, kb, vb);
    }
  } else {
    chunk(p0, ka, va);
  }
  // Combine the 16 lane groups.
  const float lg = sum16(lsum);
#pragma unroll
  for (int i = 0; i < 8; ++i) opart[pg][d0 + i] = acc[i];
  if (dc == 0) {
    gmax[pg] = m;
    gsum[pg] = lg;
  }
  __syncthreads();
  float M = -INFINITY, o = 0.0f, l = 0.0f;
  if (t < D) {
#pragma unroll
    for (int g = 0; g < 16; ++g) M = fmaxf(M, gmax[g]);
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      const float wg = gmax[g] == -INFINITY ? 0.0f : __expf(gmax[g] - M);
      o += wg * opart[g][t];
      l += wg * gsum[g];
    }
  }
  f16* orow = out + (size_t)b * H * D + (size_t)h * D;
  if (ns == 1) {
    if (t < D) {
      const f16 r = ok ? (f16)(o / l) : (f16)0.0f;
      orow[t] = r;
    }
    return;
  }
  // Publish this split's partial (an empty split: M = -inf, l = o = 0), then
  // count it.
  const int bh = b * H + h;
  float* mine = part + ((size_t)bh * ns + sp) * kPart;
  if (t < D) st_coh(mine + 2 + t, o);
  if (t == 0) {
    st_coh(mine, M);
    st_coh(mine + 1, l);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the stores are complete
  __syncthreads();
  // Agent-scope acquire-release count: releases this split's partial, and
  // the last split's acquire makes every partial visible to its reads.
  if (t == 0) {
    const int prev = __hip_atomic_fetch_add(cnt + bh, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == ns - 1;
    if (prev == ns - 1) __hip_atomic_store(cnt + bh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  const float* all = part + (size_t)bh * ns * kPart;
  float Ms = -INFINITY;
  for (int s2 = 0; s2 < ns; ++s2) Ms = fmaxf(Ms, ld_coh(all + s2 * kPart));
  float lsum2 = 0.0f, osum = 0.0f;
  for (int s2 = 0; s2 < ns; ++s2) {
    const float* ps = all + s2 * kPart;
    const float ms = ld_coh(ps);
    const float w = ms == -INFINITY ? 0.0f : __expf(ms - Ms);   // empty splits weigh 0
    lsum2 += ld_coh(ps + 1) * w;
    if (t < D) osum += ld_coh(ps + 2 + t) * w;
  }
  if (t < D) orow[t] = ok ? (f16)(osum / lsum2) : (f16)0.0f;
}

__global__ __launch_bounds__(kT) void k_rope_attn(const f16* __restrict__ qkv, const int64_t* __restrict__ posp,
                                                 const float* __restrict__ cosv, const float* __restrict__ sinv,
                                                 f16* __restrict__ kc, f16* __restrict__ vc, f16* __restrict__ out,
                                                 int H, int Hk, int L, float scale, float* __restrict__ part,
                                                 int* __restrict__ cnt) {
  rope_attn(qkv, posp, cosv, sinv, kc, vc, out, H, Hk, L, scale, part, cnt, blockIdx.x, blockIdx.y,
                   blockIdx.z, gridDim.z);
}

}  // namespace

namespace {

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

// ---- the decode step's tail: final RMSNorm + lm_head + greedy argmax -------
//
// Every workgroup forms t = RMSNorm(x + delta) for the nb <= B rows in LDS
// with the chunk order and roundings of k_rmsnorm (so t is bit-identical to
// it), then each wave streams vocab rows v = wave id + k · waves: lane l
// holds columns 8(64c + l) .. +7 (c < CH) of W row v (a wave load covers 1 KB
// of the row) and of t — in registers for B <= 2, read from LDS per row
// otherwise (1 KB contiguous per wave load, no bank conflicts) — fp32 dot2
// sums, a wave reduction, and lane 0 writes fp16 logits[b][v].  The greedy choice is the largest fp16 logit,
// the smallest index among equal ones (as torch.argmax): an order-preserving
// 64-bit key per (b, v), reduced per workgroup and combined with one
// device-scope atomic max per batch row; the last workgroup to finish (an
// atomic count) writes tok[b], adds 1 to *pos (if given) and clears the keys
// and the count for the next call.  The next row is requested before the
// current one is summed (two rows in flight per wave).

__device__ __forceinline__ unsigned long long head_key(f16 v, int idx) {
  const uint32_t b = __builtin_bit_cast(uint16_t, v);
  const uint32_t o = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);   // fp16 order as unsigned
  return ((unsigned long long)o << 32) | (0xFFFFFFFFu - (uint32_t)idx);
}

// By value: __builtin_bit_cast applied directly to a vector element (a[d])
// reads element 0 with this compiler.
__device__ __forceinline__ float dot2w(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc, false);
}
__device__ __forceinline__ float dot8(const u32x4 a, const u32x4 b, float acc) {
#pragma unroll
  for (int d = 0; d < 4; ++d) acc = dot2w(a[d], b[d], acc);
  return acc;
}

template <int B, int CH>
__global__ __launch_bounds__(kT) void k_lm_head_argmax(const f16* __restrict__ x, const f16* __restrict__ delta,
                                                       const f16* __restrict__ nw, float eps,
                                                       const f16* __restrict__ W, int V, int nb,
                                                       f16* __restrict__ logits, int64_t* __restrict__ tok,
                                                       int64_t* __restrict__ pos,
                                                       unsigned long long* __restrict__ keys, int* __restrict__ cnt) {
  constexpr int H = CH * 512;
  constexpr int MAXV = H / 8 / kT;   // 16-byte chunks per thread in the norm (H/8 chunks over kT threads)
  static_assert(MAXV * kT * 8 == H, "H is a multiple of 2048");
  constexpr bool TREG = B <= 2;      // t in registers (else read from LDS per row)
  extern __shared__ __attribute__((aligned(16))) char head_dyn[];
  f16 (*ts)[H] = (f16 (*)[H])head_dyn;   // [B][H]
  __shared__ float sh[kT / 64];
  __shared__ unsigned long long wbest[B][kT / 64];
  __shared__ int s_last;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  // t = fp16(w ⊙ r · rsqrt(mean(r²) + eps)), r = fp16(x + delta): k_rmsnorm's steps.
#pragma unroll
  for (int b = 0; b < B; ++b) {
    if (b >= nb) break;   // uniform
    f16x8 v[MAXV];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < MAXV; ++k) {
      const int c = t + kT * k;
      f16x8 a = *(const f16x8*)(x + (size_t)b * H + c * 8);
      if (delta) {
        const f16x8 d = *(const f16x8*)(delta + (size_t)b * H + c * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = (f16)((float)a[e] + (float)d[e]);
      }
      v[k] = a;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (float)a[e] * (float)a[e];
    }
    const float inv = rsqrtf(block_sum(ss, sh) / (float)H + eps);
#pragma unroll
    for (int k = 0; k < MAXV; ++k) {
      const int c = t + kT * k;
      const f16x8 wv = *(const f16x8*)(nw + c * 8);
      f16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (f16)((float)v[k][e] * inv * (float)wv[e]);
      *(f16x8*)&ts[b][c * 8] = o;
    }
  }
  __syncthreads();
  u32x4 tr[TREG ? B : 1][CH];
  if constexpr (TREG) {
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
      for (int c = 0; c < CH; ++c) tr[b][c] = *(const u32x4*)&ts[b][(c * 64 + lane) * 8];
  }

  const int waves = (int)gridDim.x * (kT / 64);
  unsigned long long best[B];
#pragma unroll
  for (int b = 0; b < B; ++b) best[b] = 0ull;
  auto load_row = [&](int v, u32x4 (&w)[CH]) {
    const u32x4* p = (const u32x4*)(W + (size_t)v * H);
#pragma unroll
    for (int c = 0; c < CH; ++c) w[c] = __builtin_nontemporal_load(p + c * 64 + lane);
  };
  auto row = [&](int v, const u32x4 (&w)[CH]) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
      if (b >= nb) break;   // uniform
      float s = 0.0f;
#pragma unroll
      for (int c = 0; c < CH; ++c)
        s = dot8(w[c], TREG ? tr[TREG ? b : 0][c] : *(const u32x4*)&ts[b][(c * 64 + lane) * 8], s);
      s += partner<1>(s);
      s += partner<2>(s);
      s += partner<4>(s);
      s += partner<8>(s);
      s += partner<16>(s);
      s += partner<32>(s);
      if (lane == 0) {
        const f16 l16 = (f16)s;
        logits[(size_t)b * V + v] = l16;
        const unsigned long long k = head_key(l16, v);
        best[b] = k > best[b] ? k : best[b];
      }
    }
  };
  u32x4 wa[CH], wb[CH];
  int v = (int)blockIdx.x * (kT / 64) + wave;
  if (v < V) load_row(v, wa);
  while (v < V) {
    const int v1 = v + waves;
    if (v1 < V) load_row(v1, wb);
    row(v, wa);
    if (v1 >= V) break;
    const int v2 = v1 + waves;
    if (v2 < V) load_row(v2, wa);
    row(v1, wb);
    v = v2;
  }
  // Workgroup maximum per batch row, one device-scope atomic each; the last
  // workgroup to arrive finishes the step.
  if (lane == 0) {
#pragma unroll
    for (int b = 0; b < B; ++b) wbest[b][wave] = best[b];
  }
  __syncthreads();
  if (t < nb) {
    unsigned long long m = wbest[t][0];
#pragma unroll
    for (int w2 = 1; w2 < kT / 64; ++w2) m = wbest[t][w2] > m ? wbest[t][w2] : m;
    __hip_atomic_fetch_max(keys + t, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the atomics are complete
  __syncthreads();
  // Agent-scope acquire-release count: orders this workgroup's key maxima
  // before it, and the last workgroup's acquire before its key reads.
  if (t == 0) {
    const int prev = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == (int)gridDim.x - 1;
    if (s_last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  if (t < nb) {
    const unsigned long long k = __hip_atomic_load(keys + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    tok[t] = (int64_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
    __hip_atomic_store(keys + t, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (t == 0 && pos) pos[0] = pos[0] + 1;
}

template <int B, int CH>
int launch_head(const f16* x, const f16* delta, const f16* w, float eps, const f16* W, int V, int nb, f16* logits,
                int64_t* tok, int64_t* pos, unsigned long long* keys, int* cnt, hipStream_t s) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  // Workgroups per CU: one for B <= 2 (t in registers; every extra workgroup
  // repeats the norm prologue: 46 us against 53 with two, 86 with four, for
  // the Llama-2-7B lm_head at B = 1), two above (t read from LDS: 77.5 us
  // against 109 with one at B = 8).
  int G = cus * (B <= 2 ? 1 : 2);
  const int rows_per_wg = kT / 64;
  if (G * rows_per_wg > V) G = (V + rows_per_wg - 1) / rows_per_wg;
  auto kern = k_lm_head_argmax<B, CH>;
  const size_t dyn = (size_t)B * CH * 512 * 2;
  static size_t attr = 0;
  if (dyn > 64 * 1024 && dyn > attr) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn) != hipSuccess)
      return 3;
    attr = dyn;
  }
  hipLaunchKernelGGL(kern, dim3(G), dim3(kT), dyn, s, x, delta, w, eps, W, V, nb, logits, tok, pos, keys, cnt);
  return 0;
}

}  // namespace
}  // namespace eptq

extern "C" {

// Return codes: 0 ok, 1 invalid argument, 2 unsupported shape, 3 HIP launch error.

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

long long eptq_llama_lm_head_work_bytes(int B) {
  if (B <= 0) return 0;
  return (long long)B * 8 + 8;   // one 64-bit key per batch row, then the count
}

int eptq_llama_lm_head_argmax(const void* x, const void* delta, const void* w, float eps, const void* W, int V,
                              int H, int B, void* logits, void* tok, void* pos, void* work, void* stream) {
  if (!x || !w || !W || !logits || !tok || !work || V <= 0 || B <= 0) return 1;
  if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)W | (uintptr_t)(delta ? delta : x)) & 15) return 1;
  if (((uintptr_t)work & 7) || ((uintptr_t)logits & 1) || ((uintptr_t)tok & 7) || ((uintptr_t)pos & 7)) return 1;
  if (B > 8 || (H != 4096 && H != 6144 && H != 8192) || (size_t)B * H * 2 > 128 * 1024) return 2;
  using eptq::f16;
  auto* keys = (unsigned long long*)work;
  int* cnt = (int*)(keys + B);
  const hipStream_t s = (hipStream_t)stream;
  const f16 *px = (const f16*)x, *pd = (const f16*)delta, *pw = (const f16*)w, *pW = (const f16*)W;
  f16* pl = (f16*)logits;
  int64_t *pt = (int64_t*)tok, *pp = (int64_t*)pos;
  const int CH = H / 512;
  int rc = 0;
#define EPTQ_HEAD(BT)                                                                                   \
  rc = CH == 8    ? eptq::launch_head<BT, 8>(px, pd, pw, eps, pW, V, B, pl, pt, pp, keys, cnt, s)      \
       : CH == 12 ? eptq::launch_head<BT, 12>(px, pd, pw, eps, pW, V, B, pl, pt, pp, keys, cnt, s)     \
                  : eptq::launch_head<BT, 16>(px, pd, pw, eps, pW, V, B, pl, pt, pp, keys, cnt, s)
  if (B == 1) { EPTQ_HEAD(1); }
  else if (B == 2) { EPTQ_HEAD(2); }
  else if (B <= 4) { EPTQ_HEAD(4); }
  else { EPTQ_HEAD(8); }
#undef EPTQ_HEAD
  if (rc) return rc;
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

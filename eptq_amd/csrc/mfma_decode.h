// E8-D4 indices decoded straight into v_mfma_f32_16x16x32_f16 A operands,
// as the matrix-core decode matvec (decode_mfma.hip) uses them.
//
// Operand mapping.  For an MFMA over 16 output rows x 32 input columns, lane
// l = i + 16·kg holds A[i][8kg .. 8kg+7].  Row i of the 16 is half i%2 (rows
// 0-3 or 4-7 of an 8-row block) of block row i/2, so 8 block rows (64 output
// rows) fill 4 MFMAs: MFMA c (c = 0..3) takes row 4·(i%2) + c of block row
// i/2.  A lane therefore decodes the 8 indices of its block row at its 8
// columns, one 8-byte table lookup each (4 rows of one column, its half), and
// the A operand of MFMA c is 4 byte-permutes of those lookups: no lane
// exchanges data with another.  D of MFMA c in lane (n = l%16, lg = l/16),
// element v, is output row 16·lg + 4v + c of the 64 for column n of B.
//
// Table: the 512-row fp16 E8-D4 table in LDS at row e ^ 0x100, so the raw
// int16 bits address it: rows 0-3 of a block at byte (v >> 4) & 0xFF8, rows
// 4-7 with bits 3-9 replaced by (v & 127) << 3.  The marker 32767 decodes as
// table row 511 in both halves.
#pragma once

#include "decode_layer.h"

namespace eptq {
namespace mdec {

using dec::kBufferWord3;
using dec::perm;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, bytes, kBufferWord3);
}
template <int AUX = 0>
__device__ __forceinline__ u32x4 ld16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
}
__device__ __forceinline__ uint16_t ld2(__amdgpu_buffer_rsrc_t r, int off) {
  return (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
// Bitfield insert with a per-lane mask: (mask & a) | (~mask & b).
__device__ __forceinline__ uint32_t bfi_v(uint32_t mask, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask), "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ f16 as_f16(uint16_t v) { return __builtin_bit_cast(f16, v); }
__device__ __forceinline__ uint16_t bits(f16 v) { return __builtin_bit_cast(uint16_t, v); }

// This lane's half of the block: byte addresses of the two indices of a word
// w are (t & 0xFF8) and ((t >> 16) & 0xFF8) with
//   rows 0-3: t = w >> 4;  rows 4-7: t = bfi(0x0C000C00, w >> 4, w << 3)
// (bits 10-11 of each half from v >> 4, bits 3-9 = (v & 127) << 3).
struct Half {
  uint32_t tmask, tsh;
  __device__ __forceinline__ explicit Half(int i)
      : tmask((i & 1) ? 0x0C000C00u : 0xFFFFFFFFu), tsh((i & 1) ? 3u : 0u) {}

  // The 8 table lookups of 8 indices q (columns 0..7 of this lane's K
  // group): lo[d], hi[d] = the lane's half of columns 2d and 2d + 1.
  __device__ __forceinline__ void lookup(const u32x4 q, const char* __restrict__ tabB, u32x2 (&lo)[4],
                                         u32x2 (&hi)[4]) const {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t w0 = q[d];
      const uint32_t t = bfi_v(tmask, w0 >> 4, w0 << tsh);
      lo[d] = *(const u32x2*)(tabB + (t & 0xFF8u));
      hi[d] = *(const u32x2*)(tabB + hi_addr(t));
    }
  }
  // The A operand of MFMA c (0..3) from those lookups: row c of the lane's
  // half at the 8 columns.
  __device__ __forceinline__ static u32x4 operand(const u32x2 (&lo)[4], const u32x2 (&hi)[4], int c) {
    u32x4 aw;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t l = c < 2 ? lo[d][0] : lo[d][1];
      const uint32_t h = c < 2 ? hi[d][0] : hi[d][1];
      aw[d] = perm(h, l, (c & 1) ? 0x07060302u : 0x05040100u);
    }
    return aw;
  }
};

}  // namespace mdec
}  // namespace eptq

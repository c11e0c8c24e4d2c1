// Shared device types and helpers for the gfx950 EPTQ kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eptq {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

// Activation element types: fp16 or bf16, stored as 16-bit words.
template <typename T> struct Act;
template <> struct Act<f16> {
  __device__ __forceinline__ static float to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(f16, b);
  }
  __device__ __forceinline__ static uint16_t from_f32(float v) {
    return __builtin_bit_cast(uint16_t, (f16)v);
  }
  // Exact fp32 product of an activation and an fp16 scale (the product of two
  // 11-bit significands fits in fp32), one fused mixed-precision op.
  __device__ __forceinline__ static float mul_f16(uint16_t a, f16 s) {
    return __builtin_fmaf((float)__builtin_bit_cast(f16, a), (float)s, 0.0f);
  }
};
template <> struct Act<bf16> {
  __device__ __forceinline__ static float to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
  }
  __device__ __forceinline__ static uint16_t from_f32(float v) {
    return __builtin_bit_cast(uint16_t, (bf16)v);
  }
  __device__ __forceinline__ static float mul_f16(uint16_t a, f16 s) {
    return to_f32(a) * (float)s;
  }
};

// Two activation elements (one 32-bit word) as an fp16 pair.  bf16 values
// convert exactly while they lie in fp16's normal range (bf16 carries 8
// significand bits, fp16 11), so round-toward-zero conversion loses nothing
// there; beyond it values saturate at the largest finite fp16.
template <typename T> __device__ __forceinline__ uint32_t to_f16x2(uint32_t w);
template <> __device__ __forceinline__ uint32_t to_f16x2<f16>(uint32_t w) { return w; }
template <> __device__ __forceinline__ uint32_t to_f16x2<bf16>(uint32_t w) {
  const auto p = __builtin_amdgcn_cvt_pkrtz(__builtin_bit_cast(float, w << 16),
                                            __builtin_bit_cast(float, w & 0xffff0000u));
  return __builtin_bit_cast(uint32_t, p);
}
// One element as fp16 (same conversion).
template <typename T> __device__ __forceinline__ f16 to_f16(uint16_t b) {
  return __builtin_bit_cast(f16, (uint16_t)(to_f16x2<T>((uint32_t)b) & 0xffffu));
}

// Bitfield insert: (mask & a) | (~mask & b) in one VALU op.
// (t >> 16) & 0xFF8 in one op (SDWA word select of the second operand): the
// table byte address of the upper index of a 32-bit word t = w >> 4.
__device__ __forceinline__ uint32_t hi_addr(uint32_t t) {
  uint32_t r;
  asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_1"
      : "=v"(r) : "s"(0xFF8u), "v"(t));
  return r;
}

__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(a), "v"(b));
  return r;
}

// ---------------------------------------------------------------------------
// Cross-lane exchange with the partner lane = lane ^ O (exactly: halving
// reductions need partners that agree on every other lane bit).
//   O = 1, 2   DPP quad_perm (VALU)
//   O = 4, 8   ds_swizzle in xor mode (LDS crossbar, no memory access)
//   O = 16, 32 gfx950 permlane16/32 swaps (VALU): with both operands = x the
//              swap returns r[0] = x of the lower row/half, r[1] = x of the
//              upper one, in every lane.
// ---------------------------------------------------------------------------
template <int O>
__device__ __forceinline__ float partner(float v) {
  const int iv = __builtin_bit_cast(int, v);
  const int lane = threadIdx.x & 63;
  if constexpr (O == 1) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, false));
  } else if constexpr (O == 2) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, false));
  } else if constexpr (O == 4) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(iv, 0x101F));
  } else if constexpr (O == 8) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(iv, 0x201F));
  } else if constexpr (O == 16) {
    auto r = __builtin_amdgcn_permlane16_swap((unsigned)iv, (unsigned)iv, false, false);
    return __builtin_bit_cast(float, (unsigned)((lane & 16) ? r[0] : r[1]));
  } else {
    auto r = __builtin_amdgcn_permlane32_swap((unsigned)iv, (unsigned)iv, false, false);
    return __builtin_bit_cast(float, (unsigned)((lane & 32) ? r[0] : r[1]));
  }
}

// v + partner<O>(v) in every lane.
template <int O>
__device__ __forceinline__ float butterfly(float v) {
  if constexpr (O == 16) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
  } else if constexpr (O == 32) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
  } else {
    return v + partner<O>(v);
  }
}

// Lane bits in the order the reduction consumes them (cheapest exchanges
// first for the stages that move the most values).
constexpr int kReduceBits[6] = {1, 2, 16, 32, 4, 8};

constexpr int log2_ceil(int v) { return v <= 1 ? 0 : 1 + log2_ceil((v + 1) / 2); }

// Reduce V partial sums (V a power of two) across the 64 lanes of a wave by
// recursive halving: at the exchange on a lane bit, a lane keeps half of its
// values and adds its partner's copy of that half.  Afterwards the lane holds
// max(V/64, 1) fully reduced values whose indices start at the returned base;
// when V < 64 the first log2(V) bits of kReduceBits select the value and the
// other lane bits are replicas (WaveReduceOut::writer picks one of each).
template <int V>
__device__ __forceinline__ int wave_reduce_halving(float (&v)[V]) {
  const int lane = threadIdx.x & 63;
  int base = 0;
  int cnt = V;
#define EPTQ_STAGE(O)                                                   \
  if (cnt > 1) {                                                        \
    const bool up = (lane & (O)) != 0;                                  \
    const int half = cnt >> 1;                                          \
    _Pragma("unroll") for (int p = 0; p < (V >> 1); ++p) {              \
      if (p < half) {                                                   \
        const float send = up ? v[p] : v[p + half];                     \
        const float keep = up ? v[p + half] : v[p];                     \
        v[p] = keep + partner<O>(send);                                 \
      }                                                                 \
    }                                                                   \
    if (up) base += half;                                               \
    cnt = half;                                                         \
  } else {                                                              \
    v[0] = butterfly<O>(v[0]);                                          \
  }
  EPTQ_STAGE(1)
  EPTQ_STAGE(2)
  EPTQ_STAGE(16)
  EPTQ_STAGE(32)
  EPTQ_STAGE(4)
  EPTQ_STAGE(8)
#undef EPTQ_STAGE
  return base;
}

// The value index that wave_reduce_halving<V> leaves in `lane` (a function
// of the lane bits only, so epilogue operands can be fetched before the sums).
template <int V>
__device__ __forceinline__ int reduce_base(int lane) {
  int base = 0, cnt = V;
#pragma unroll
  for (int s = 0; s < 6; ++s) {
    if (cnt > 1) {
      const int half = cnt >> 1;
      if (lane & kReduceBits[s]) base += half;
      cnt = half;
    }
  }
  return base;
}

template <int V> struct WaveReduceOut {
  static constexpr int per_lane = V >= 64 ? V / 64 : 1;
  static constexpr int used_bits() {
    int m = 0;
    for (int i = 0; i < log2_ceil(V) && i < 6; ++i) m |= kReduceBits[i];
    return m;
  }
  // One writer per distinct value: the lane whose replica bits are all zero.
  __device__ static bool writer(int lane) { return (lane & (63 & ~used_bits())) == 0; }
};

}  // namespace eptq

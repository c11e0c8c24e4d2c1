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
};
template <> struct Act<bf16> {
  __device__ __forceinline__ static float to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
  }
  __device__ __forceinline__ static uint16_t from_f32(float v) {
    return __builtin_bit_cast(uint16_t, (bf16)v);
  }
};

__device__ __forceinline__ float h2f(f16 v) { return (float)v; }

// Reduce V partial sums (V a power of two) across the 64 lanes of a wave by
// recursive halving: at each exchange a lane keeps half of its values and
// adds its partner's copy of that half.  Afterwards the lane holds
// max(V/64, 1) fully reduced values whose indices start at the returned base;
// when V < 64 the 64/V lanes that share a base hold identical sums.
template <int V>
__device__ __forceinline__ int wave_reduce_halving(float (&v)[V]) {
  const int lane = threadIdx.x & 63;
  int base = 0;
#pragma unroll
  for (int step = 0; step < 6; ++step) {
    const int o = 32 >> step;
    const int cnt = (V >> step) > 0 ? (V >> step) : 1;
    if (cnt > 1) {
      const bool up = (lane & o) != 0;
      const int half = cnt >> 1;
#pragma unroll
      for (int p = 0; p < half; ++p) {
        const float send = up ? v[p] : v[p + half];
        const float keep = up ? v[p + half] : v[p];
        v[p] = keep + __shfl_xor(send, o, 64);
      }
      if (up) base += half;
    } else {
      v[0] += __shfl_xor(v[0], o, 64);
    }
  }
  return base;
}

// Number of distinct reduced values per lane after wave_reduce_halving<V>.
template <int V> struct WaveReduceOut {
  static constexpr int per_lane = V >= 64 ? V / 64 : 1;
  // Lanes that write: for V < 64 only one lane per group of 64/V identical lanes.
  static constexpr int writer_mask = V >= 64 ? 0 : (64 / V) - 1;
};

}  // namespace eptq

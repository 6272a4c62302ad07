// Device-side helpers shared by the GDN kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

constexpr int kHQK = 4;    // q/k heads
constexpr int kHV = 8;     // v heads; v-head h reads q/k head h / 2
constexpr int kDK = 128;   // key head size
constexpr int kDV = 128;   // value head size
constexpr int kChunk = 64; // prefill chunk length

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// float -> bf16 bits, round to nearest even; NaN -> 0x7FC0 (torch's choice).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Data-parallel-primitive lane moves.  CTRL is a DPP control word:
//   0xB1 quad_perm[1,0,3,2] (lane ^ 1)   0x4E quad_perm[2,3,0,1] (lane ^ 2)
//   0x141 row_half_mirror (i <-> 7-i within 8 lanes)
//   0x140 row_mirror      (i <-> 15-i within 16 lanes)
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum over each aligned group of 16 lanes (one DPP "row"); every lane of the
// group receives the total.  Four DPP adds, no LDS traffic.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  x += dpp<0x141>(x);
  x += dpp<0x140>(x);
  return x;
}

// softplus with torch's threshold (x > 20 -> x), as F.softplus(beta=1, threshold=20).
__device__ __forceinline__ float softplus20(float x) {
  return x > 20.0f ? x : log1pf(expf(x));
}

// Log-space decay -exp(A_log) * softplus(a + dt_bias).
__device__ __forceinline__ float gdn_log_decay(float A_log, float a, float dt_bias) {
  return -expf(A_log) * softplus20(a + dt_bias);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

}  // namespace gdn

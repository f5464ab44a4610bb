// Shared device helpers for the gfx950 DSA decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dsa_mli.h"

namespace dsa {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// Order-preserving map fp32 -> u32 used by every ranking in this library:
// larger key == ranks higher.  -0.0 is folded onto +0.0 and every NaN onto
// the top key, so the order is total and matches the comparison the
// reference's select makes (torch.topk treats NaN as largest, -0.0 == +0.0).
// Same transform as the reference's hp_exact_key (K:1132-1135) apart from the
// canonicalisation of NaN and -0.0.
__device__ __forceinline__ uint32_t rank_key(float x) {
  uint32_t b = __float_as_uint(x);
  if (x != x) return 0xffffffffu;
  if ((b & 0x7fffffffu) == 0u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// -inf maps to this key, +inf to 0xff800000; NaN to 0xffffffff.
constexpr uint32_t kKeyNegInf = 0x007fffffu;
constexpr uint32_t kKeyPosInf = 0xff800000u;
__device__ __forceinline__ bool key_is_finite(uint32_t k) {
  return k > kKeyNegInf && k < kKeyPosInf;
}

// fp32 -> bf16 bits, round to nearest even (finite and inf inputs; the
// dequantised values here are never NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_rn(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_rn(lo) | (f32_to_bf16_rn(hi) << 16);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Four OCP e4m3 (one 32-bit word, byte i = element i) -> fp32, exact.
__device__ __forceinline__ void e4m3x4_to_f32(uint32_t w, float* o) {
  auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  o[0] = lo[0];
  o[1] = lo[1];
  o[2] = hi[0];
  o[3] = hi[1];
}

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
}

__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

}  // namespace dsa

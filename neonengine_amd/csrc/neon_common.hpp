// neon_common.hpp -- device helpers shared by the gfx950 kernels.
//
// bf16 tensors travel as uint16_t bit patterns; arithmetic is fp32.  Wave
// size is 64 (CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace neon {

constexpr int kWave = 64;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// ---- bf16 <-> fp32 --------------------------------------------------------
__host__ __device__ __forceinline__ float bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  return __builtin_bit_cast(float, u);
}
__device__ __forceinline__ float bf_lo(uint32_t w) {
  return __builtin_bit_cast(float, w << 16);
}
__device__ __forceinline__ float bf_hi(uint32_t w) {
  return __builtin_bit_cast(float, w & 0xffff0000u);
}
// round to nearest even; NaN stays a quiet NaN
__host__ __device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

// acc + a.lo*b.lo + a.hi*b.hi  (v_dot2_f32_bf16)
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc,
                                         false);
}
// 8 bf16 x 8 bf16
__device__ __forceinline__ float dot8_bf16(const uint4& w, const uint4& x,
                                           float acc) {
  acc = dot2_bf16(w.x, x.x, acc);
  acc = dot2_bf16(w.y, x.y, acc);
  acc = dot2_bf16(w.z, x.z, acc);
  acc = dot2_bf16(w.w, x.w, acc);
  return acc;
}

// ---- MXFP4 -----------------------------------------------------------------
// Two E2M1 values of byte `sel` of `w` as a bf16 pair (lo = low nibble),
// unscaled (v_cvt_scalef32_pk_bf16_fp4 with scale 1.0: exact).
template <int SEL>
__device__ __forceinline__ uint32_t fp4x2_to_bf16x2(uint32_t w) {
  bf16x2_t r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, SEL);
  return __builtin_bit_cast(uint32_t, r);
}
// 32 E2M1 values (16 bytes) dotted with 32 bf16 x values (4 x uint4).
__device__ __forceinline__ float fp4_unit_dot(const uint4& c, const uint4* x) {
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
  float acc = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    acc = dot2_bf16(fp4x2_to_bf16x2<0>(cw[q]), x[q].x, acc);
    acc = dot2_bf16(fp4x2_to_bf16x2<1>(cw[q]), x[q].y, acc);
    acc = dot2_bf16(fp4x2_to_bf16x2<2>(cw[q]), x[q].z, acc);
    acc = dot2_bf16(fp4x2_to_bf16x2<3>(cw[q]), x[q].w, acc);
  }
  return acc;
}
// v * 2^(s - 127); E8M0 0xFF is NaN.
__device__ __forceinline__ float e8m0_scale(float v, uint32_t s) {
  float r = __builtin_amdgcn_ldexpf(v, (int)s - 127);
  return s == 0xFFu ? __builtin_nanf("") : r;
}

// ---- wave reductions (xor butterfly over 64 lanes) ------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float half_wave_sum(float v) {
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---- counter-based RNG (SplitMix64 finaliser), identical to the oracle ----
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z ^= z >> 30;
  z *= 0xBF58476D1CE4E5B9ull;
  z ^= z >> 27;
  z *= 0x94D049BB133111EBull;
  z ^= z >> 31;
  return z;
}
__host__ __device__ __forceinline__ uint64_t stream_key(uint64_t seed,
                                                        uint64_t stream) {
  return mix64(seed + stream * 0x9E3779B97F4A7C15ull);
}
__host__ __device__ __forceinline__ uint64_t hash_k(uint64_t key, uint64_t i) {
  return mix64(key ^ (i * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull));
}
__host__ __device__ __forceinline__ int32_t gauss_int(uint64_t h) {
  return (int32_t)((h & 0xFFFF) + ((h >> 16) & 0xFFFF) + ((h >> 32) & 0xFFFF) +
                   (h >> 48)) -
         131070;
}
__host__ __device__ __forceinline__ uint64_t stream_id(int layer, int kind) {
  return ((uint64_t)(layer + 1) << 16) | (uint64_t)kind;
}

}  // namespace neon

// neon_common.hpp -- device helpers shared by the gfx950 kernels.
//
// bf16 tensors travel as uint16_t bit patterns; arithmetic is fp32.  Wave
// size is 64 (CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "neon_internal.hpp"  // the device status bits (kDevErr*)

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
// fp32 -> bf16, round to nearest even; a NaN keeps its sign and top payload
// bits and gets the quiet bit (the oracle's or_f2bf).  gfx950 does this in
// one instruction, v_cvt_pk_bf16_f32 (two values per instruction); its
// results equal the integer form (u + 0x7fff + lsb) >> 16, NaN -> (u >> 16) |
// 0x40, for all 2^32 inputs (compared exhaustively on an MI355X).
typedef __bf16 neon_bf16x2 __attribute__((ext_vector_type(2)));
typedef float neon_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  const neon_f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, neon_bf16x2));
}

// ---- canonical dot products ---------------------------------------------
// Every reduction on the decode path uses one fixed order of IEEE fp32 fused
// multiply-adds so the CPU oracle (oracle/neon_oracle.c, or_c_* functions)
// reproduces it bit for bit.  (v_dot2_f32_bf16 is not used: on gfx950 its
// result is not the correctly rounded 3-term sum, so it cannot be mirrored.)

// 8 bf16 weights x 8 fp32 x values, element order 0..7, one fmaf each.
__device__ __forceinline__ float fma8_bf16(const uint4& w, const float* x,
                                           float acc) {
  acc = __builtin_fmaf(bf_lo(w.x), x[0], acc);
  acc = __builtin_fmaf(bf_hi(w.x), x[1], acc);
  acc = __builtin_fmaf(bf_lo(w.y), x[2], acc);
  acc = __builtin_fmaf(bf_hi(w.y), x[3], acc);
  acc = __builtin_fmaf(bf_lo(w.z), x[4], acc);
  acc = __builtin_fmaf(bf_hi(w.z), x[5], acc);
  acc = __builtin_fmaf(bf_lo(w.w), x[6], acc);
  acc = __builtin_fmaf(bf_hi(w.w), x[7], acc);
  return acc;
}
// 8 bf16 x 8 bf16 (both packed), element order 0..7.
__device__ __forceinline__ float fma8_bf16x2(const uint4& w, const uint4& x,
                                             float acc) {
  acc = __builtin_fmaf(bf_lo(w.x), bf_lo(x.x), acc);
  acc = __builtin_fmaf(bf_hi(w.x), bf_hi(x.x), acc);
  acc = __builtin_fmaf(bf_lo(w.y), bf_lo(x.y), acc);
  acc = __builtin_fmaf(bf_hi(w.y), bf_hi(x.y), acc);
  acc = __builtin_fmaf(bf_lo(w.z), bf_lo(x.z), acc);
  acc = __builtin_fmaf(bf_hi(w.z), bf_hi(x.z), acc);
  acc = __builtin_fmaf(bf_lo(w.w), bf_lo(x.w), acc);
  acc = __builtin_fmaf(bf_hi(w.w), bf_hi(x.w), acc);
  return acc;
}

// ---- MXFP4 -----------------------------------------------------------------
typedef float float2_v __attribute__((ext_vector_type(2)));
// E2M1 values of byte `SEL` of `w` (x = low nibble = even element), exact
// (v_cvt_scalef32_pk_f32_fp4 with scale 1.0).
template <int SEL>
__device__ __forceinline__ float2_v fp4x2_to_f32(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, SEL);
}
// Canonical MXFP4 unit (32 elements, 16 code bytes): t = fmaf chain over the
// 32 elements in increasing k of E2M1(code) * x, starting from 0.
__device__ __forceinline__ float fp4_unit_dot(const uint4& c, const float* x) {
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
  float t = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float2_v v0 = fp4x2_to_f32<0>(cw[q]), v1 = fp4x2_to_f32<1>(cw[q]);
    float2_v v2 = fp4x2_to_f32<2>(cw[q]), v3 = fp4x2_to_f32<3>(cw[q]);
    t = __builtin_fmaf(v0.x, x[8 * q + 0], t);
    t = __builtin_fmaf(v0.y, x[8 * q + 1], t);
    t = __builtin_fmaf(v1.x, x[8 * q + 2], t);
    t = __builtin_fmaf(v1.y, x[8 * q + 3], t);
    t = __builtin_fmaf(v2.x, x[8 * q + 4], t);
    t = __builtin_fmaf(v2.y, x[8 * q + 5], t);
    t = __builtin_fmaf(v3.x, x[8 * q + 6], t);
    t = __builtin_fmaf(v3.y, x[8 * q + 7], t);
  }
  return t;
}
// v * 2^(s - 127) (exact, IEEE ldexp); E8M0 0xFF is NaN.
__device__ __forceinline__ float e8m0_scale(float v, uint32_t s) {
  float r = __builtin_amdgcn_ldexpf(v, (int)s - 127);
  return s == 0xFFu ? __builtin_nanf("") : r;
}

// 16 bytes written by other blocks of the same launch: two 8-byte agent-scope
// loads, served at the device's coherence point rather than from this XCD's
// L2 (which may hold an older copy or none).
__device__ __forceinline__ uint4 load_agent16(const uint16_t* p) {
  const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
  const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
}

// Element offset of (row r, column k) in the packed activation layout of the
// matrix-core GEMVs, [ceil(R/16)][NCH][4][64][8] bf16 with NCH = ceil(K/128):
// one 16 x 32 MFMA operand (16 rows, 32 columns) is 1 KB contiguous, lane
// r % 16 + 16 (u % 4) holding the 8 elements of unit u = k / 8.
__device__ __forceinline__ size_t mx_packed_at(int r, int k, int NCH) {
  const int u = k >> 3;
  return ((((size_t)(r >> 4) * NCH + (u >> 4)) * 4 + ((u & 15) >> 2)) * 64 + (r & 15) +
          16 * (u & 3)) * 8 + (k & 7);
}

// Sets status bits in the caller's status word (a vector-memory atomic).
__device__ __forceinline__ void flag_dev_err(int32_t* err, int32_t bits) {
  if (err != nullptr) atomicOr(err, bits);
}

// RoPE (HFM:149-231) on one (x1, x2) = (dim d, dim d + 32) pair of a head:
// o1 = x1 c - x2 s, o2 = x2 c + x1 s, each product rounded.
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s,
                                          float& o1, float& o2) {
  o1 = __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, s));
  o2 = __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, s));
}

// ---- correctly rounded square root for positive normal x: the hardware
// estimate (v_sqrt_f32, within 1 ulp) corrected by one step that compares x
// with s_dn * s and s_up * s through exact fused residuals (the candidate
// whose half-ulp interval contains sqrt(x) wins).  Equal to IEEE sqrtf.
__device__ __forceinline__ float sqrt_rn(float x) {
  float s = __builtin_amdgcn_sqrtf(x);
  const float s_dn = __builtin_bit_cast(float, __builtin_bit_cast(int32_t, s) - 1);
  const float s_up = __builtin_bit_cast(float, __builtin_bit_cast(int32_t, s) + 1);
  const float r_dn = __builtin_fmaf(-s_dn, s, x);
  const float r_up = __builtin_fmaf(-s_up, s, x);
  s = (r_dn <= 0.0f) ? s_dn : s;
  s = (r_up > 0.0f) ? s_up : s;
  return s;
}

// ---- exp: Cody-Waite reduction by ln 2 (two-part constant) and a degree-7
// Taylor polynomial in Horner form, all fp32 fmaf.  The oracle evaluates the
// same operation sequence, so both sides agree bit for bit.
__host__ __device__ __forceinline__ float neon_expf_core(float x) {
  const float n = __builtin_rintf(x * 0x1.715476p+0f);
  float r = __builtin_fmaf(-n, 0x1.62e4p-1f, x);
  r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

// The range checks are selects, not branches (a divergent branch costs a
// wave both paths and the exec-mask bookkeeping); the polynomial runs on
// every x, and its result is kept only where x is in range.
__host__ __device__ __forceinline__ float neon_expf(float x) {
  const float v = neon_expf_core(x);
  const float r = x > 0x1.62e43p+6f ? __builtin_inff() : (x < -0x1.9fe36ap+6f ? 0.0f : v);
  return x != x ? x : r;
}

// SwiGLU with clamp (HFM:83-87) on g = gate + bias, u = up + bias:
// g = min(g, limit); u = clamp(u, -limit, limit);
// act = (u + 1) * (g * (1 / (1 + exp(-(g * alpha))))), each step rounded.
__device__ __forceinline__ float swiglu_clamp(float g, float u, float alpha,
                                              float limit) {
  g = g > limit ? limit : g;
  u = u > limit ? limit : (u < -limit ? -limit : u);
  const float e = neon_expf(-__fmul_rn(g, alpha));
  const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, e));
  return __fmul_rn(__fadd_rn(u, 1.0f), __fmul_rn(g, sig));
}

// Pairs of every used expert for the matrix-core expert kernels, from the
// experts ids[0 .. nk) of the pairs q = b k + s (nk <= 256, E <= 256; ids in
// LDS, 16-byte aligned):
// route[y] = the y-th used expert (ascending id; -1 past the last),
// route[S + y] = its pair count, route[2 S + 64 y + r] = its r-th pair in
// ascending q.  Every thread of the block calls it (threads 0 .. 255 work);
// cnt_e / slot_of hold 256 ints, wave_used 4, all in LDS.  Slots come from a
// lane-parallel ballot prefix over the 256 expert flags.
// It also lists the expert kernels' work items, one per (slot, group of 16
// pairs): route[kMxItemOff] = the item count n, route[kMxItemOff + 1 + y]
// (y < n) = item y packed by mx_item_pack.  Group 0 of every used slot comes
// first (item y = slot y), then group 1 of the slots with more than 16 pairs,
// and so on, so a launch has one block row per item instead of one per
// (slot, possible group).  n <= (nk + 15 S) / 16 <= 256.
constexpr int kMxItemOff = 66 * 256;
constexpr int kMxRouteWords = kMxItemOff + 1 + 256;
__host__ __device__ __forceinline__ int32_t mx_item_pack(int slot, int grp, int e, int cnt) {
  return slot | (grp << 8) | (e << 10) | (cnt << 19);  // 8 + 2 + 9 + 7 bits
}
__host__ __device__ __forceinline__ void mx_item_unpack(int32_t v, int& slot, int& grp, int& e,
                                                        int& cnt) {
  slot = v & 255; grp = (v >> 8) & 3; e = (v >> 10) & 511; cnt = (v >> 19) & 127;
}
// Block rows a launch needs to cover every item (the bound above).
__host__ __device__ __forceinline__ int mx_item_rows(int nk, int S) {
  return (nk + 15 * S) / 16 < 256 ? (nk + 15 * S) / 16 : 256;
}
__device__ __forceinline__ void mx_route_lists(const int32_t* ids, int nk, int E, int S,
                                               int32_t* __restrict__ route, int* cnt_e,
                                               int* slot_of, int* wave_used) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  if (t < 256) cnt_e[t] = 0;
  __syncthreads();
  const int e = t < nk ? ids[t] : -1;
  if (e >= 0) atomicAdd(&cnt_e[e], 1);
  __syncthreads();
  const int c = (t < 256 && t < E) ? cnt_e[t] : 0;
  const unsigned long long bal = __ballot(c > 0);
  if (t < 256 && lane == 0) wave_used[w] = __popcll(bal);
  __syncthreads();
  if (t < 256) {
    const int before = (w > 0 ? wave_used[0] : 0) + (w > 1 ? wave_used[1] : 0) +
                       (w > 2 ? wave_used[2] : 0);
    const int slot = before + __popcll(bal & ((1ull << lane) - 1ull));
    const int n_used = wave_used[0] + wave_used[1] + wave_used[2] + wave_used[3];
    if (c > 0) {
      slot_of[t] = slot;
      route[slot] = t;
      route[S + slot] = c;
    }
    if (t >= n_used && t < S) {
      route[t] = -1;
      route[S + t] = 0;
    }
  }
  __syncthreads();
  if (e >= 0) {
    // rank of pair t among its expert's pairs: the ids before it, read 4 at a
    // time (ids is 16-byte aligned LDS; every lane reads the same words, a
    // broadcast), several reads in flight per iteration
    const int4* iv = reinterpret_cast<const int4*>(ids);
    int r = 0;
    const int t4 = t >> 2;
#pragma unroll 4
    for (int q4 = 0; q4 < t4; ++q4) {
      const int4 v = iv[q4];
      r += (v.x == e) + (v.y == e) + (v.z == e) + (v.w == e);
    }
    for (int q = 4 * t4; q < t; ++q) r += ids[q] == e;
    route[2 * S + 64 * slot_of[e] + r] = t;
  }
  // work items: the four groups' ballots at once; each wave's counts go to
  // cnt_e[4 q + w] (every thread read its count long before; one barrier)
  unsigned long long bq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) bq[q] = __ballot(t < 256 && c > 16 * q);
  __syncthreads();
  if (t < 256 && lane == 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) cnt_e[4 * q + w] = __popcll(bq[q]);
  }
  __syncthreads();
  int base = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (t < 256 && c > 16 * q) {
      const int before = (w > 0 ? cnt_e[4 * q] : 0) + (w > 1 ? cnt_e[4 * q + 1] : 0) +
                         (w > 2 ? cnt_e[4 * q + 2] : 0);
      const int y = base + before + __popcll(bq[q] & ((1ull << lane) - 1ull));
      route[kMxItemOff + 1 + y] = mx_item_pack(slot_of[t], q, t, c < 64 ? c : 64);
    }
    base += cnt_e[4 * q] + cnt_e[4 * q + 1] + cnt_e[4 * q + 2] + cnt_e[4 * q + 3];
  }
  if (t == 0) route[kMxItemOff] = base;
}

// One expert block's share of mx_route_lists, built from the pair ids by the
// block itself (blockDim 256, nk <= 256, E <= 256): work item y's (slot,
// group, expert, min(count, 64)) and the pair indices 16 group .. 16 group +
// 15 of that expert, in ascending pair index, in rows[].  It is the same item
// and the same pairs as the route table's item y (the same per-expert counts
// and the same ballot ranks), so a launch that reads the ids directly needs
// no table, and the launch before it no step that waits for all its rows.
// Pair ids outside [0, E) join no expert (flagged by block (0, 0)).  False
// when y is past the last item (uniform for the block).
struct MxRouteLds {
  int cnt[256];     // pairs per expert
  int wq[4][4];     // [group q][wave]: experts with more than 16 q pairs
  int we[4];        // [wave]: pairs of the block's expert
  int item[4];      // slot, group, expert, count; expert -1 for no item
  int32_t rows[16];
};
__device__ __forceinline__ bool mx_route_item(const int32_t* __restrict__ ids, int nk, int E,
                                              int y, int32_t* err, MxRouteLds& s, int& slot,
                                              int& grp, int& e, int& cnt) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int id = t < nk ? ids[t] : -1;
  if (t < nk && (unsigned)id >= (unsigned)E) {
    if (blockIdx.x == 0 && blockIdx.y == 0) flag_dev_err(err, kDevErrExpertId);
    id = -1;
  }
  s.cnt[t] = 0;
  if (t == 0) s.item[2] = -1;
  __syncthreads();
  if (id >= 0) atomicAdd(&s.cnt[id], 1);
  __syncthreads();
  const int c = t < E ? s.cnt[t] : 0;
  unsigned long long bq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) bq[q] = __ballot(c > 16 * q);
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) s.wq[q][w] = __popcll(bq[q]);
  }
  __syncthreads();
  // items: group 0 of every used expert in ascending id (item = slot), then
  // group 1 of the experts with more than 16 pairs, ...
  const unsigned long long lt = (1ull << lane) - 1ull;
  const int slot_t = (w > 0 ? s.wq[0][0] : 0) + (w > 1 ? s.wq[0][1] : 0) +
                     (w > 2 ? s.wq[0][2] : 0) + __popcll(bq[0] & lt);
  int base = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (c > 16 * q) {
      const int before = (w > 0 ? s.wq[q][0] : 0) + (w > 1 ? s.wq[q][1] : 0) +
                         (w > 2 ? s.wq[q][2] : 0);
      if (base + before + __popcll(bq[q] & lt) == y) {
        s.item[0] = slot_t; s.item[1] = q; s.item[2] = t; s.item[3] = c < 64 ? c : 64;
      }
    }
    base += s.wq[q][0] + s.wq[q][1] + s.wq[q][2] + s.wq[q][3];
  }
  __syncthreads();
  slot = s.item[0]; grp = s.item[1]; e = s.item[2]; cnt = s.item[3];
  if (e < 0) return false;
  // the expert's pairs ranked 16 grp .. 16 grp + 15
  const unsigned long long be = __ballot(id == e);
  if (lane == 0) s.we[w] = __popcll(be);
  __syncthreads();
  if (id == e) {
    const int r = (w > 0 ? s.we[0] : 0) + (w > 1 ? s.we[1] : 0) + (w > 2 ? s.we[2] : 0) +
                  __popcll(be & lt) - 16 * grp;
    if (r >= 0 && r < 16) s.rows[r] = t;
  }
  __syncthreads();
  return true;
}

// A load that stays where it is written.  The compiler sinks a plain load
// whose only use sits in a branch (a lane-0 epilogue) into that branch, where
// it issues last and is waited for alone; a relaxed atomic load is never
// moved, and at workgroup scope it is the same hardware load.
__device__ __forceinline__ uint32_t load_pinned_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint16_t load_pinned_u16(const uint16_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ float load_pinned_f32(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Two ways an early load still gets waited for at once, and their remedies:
//   - a load under a condition (`p ? load(p) : 0`) is waited for where the
//     branches join: load from an address that is always valid instead and
//     select the value afterwards;
//   - a value the compiler proves uniform across the wave (a load from a
//     block-uniform address) is copied to a scalar register right after the
//     load, so it is waited for there: add lane_zero(n) to its index, which
//     is 0 at run time for n >= 0 but depends on the lane as far as the
//     compiler can tell, so the value stays in vector registers and is
//     waited for at its first use.
__device__ __forceinline__ int lane_zero(int n) { return (int)threadIdx.x & (n >> 31); }

// ---- lane exchange: lane l receives lane (l ^ OFF)'s value ----------------
// The values __shfl_xor(v, OFF, 64) gives, without the LDS permute unit (a
// round trip through the LDS queue per step): DPP quad permutes for OFF 1
// and 2, two row shifts and a select for 4, a row rotate by 8 for 8, and the
// gfx950 permlane swaps for 16 and 32.  Reductions written with it are
// bit-identical to the __shfl_xor form.
template <int OFF>
__device__ __forceinline__ int xor_lane_i(int v) {
  const int lane = threadIdx.x & 63;
  if constexpr (OFF == 1) {
    return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true);  // quad_perm [1,0,3,2]
  } else if constexpr (OFF == 2) {
    return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, true);  // quad_perm [2,3,0,1]
  } else if constexpr (OFF == 4) {
    const int up = __builtin_amdgcn_update_dpp(0, v, 0x104, 0xF, 0xF, true);  // row_shl 4
    const int dn = __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);  // row_shr 4
    return (lane & 4) ? dn : up;
  } else if constexpr (OFF == 8) {
    return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, true);  // row_ror 8
  } else if constexpr (OFF == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16) ? (int)p[0] : (int)p[1];
  } else {
    static_assert(OFF == 32, "xor_lane: OFF must be 1, 2, 4, 8, 16 or 32");
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane & 32) ? (int)p[0] : (int)p[1];
  }
}
template <int OFF>
__device__ __forceinline__ float xor_lane(float v) {
  return __builtin_bit_cast(float, xor_lane_i<OFF>(__builtin_bit_cast(int, v)));
}

// ---- wave reductions (xor butterfly over 64 lanes, off = 32 .. 1) ---------
template <int OFF = 32>
__device__ __forceinline__ float wave_sum(float v) {
  v += xor_lane<OFF>(v);
  if constexpr (OFF > 1) return wave_sum<OFF / 2>(v);
  else return v;
}
template <int OFF = 32>
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, xor_lane<OFF>(v));
  if constexpr (OFF > 1) return wave_max<OFF / 2>(v);
  else return v;
}
__device__ __forceinline__ float half_wave_sum(float v) { return wave_sum<16>(v); }

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

// ---- MXFP8 (E4M3) activations: the two-term image of a bf16 32-block ----
// (OCP MX v1.0 E4M3 and shared-exponent rule, without saturation; the CPU
// oracle's or_mx8_quant states the same arithmetic, bit for bit.)
__device__ __forceinline__ int ilog2f_dev(float a) {
  const uint32_t b = __float_as_uint(a);
  const int ef = (b >> 23) & 255;
  if (ef) return ef - 127;
  return (31 - __builtin_clz(b & 0x7FFFFFu)) - 149;
}

// smallest shared exponent with amax / 2^e <= 448: floor(log2 amax) - 8, one
// more when amax's significand exceeds 1.75
__device__ __forceinline__ uint32_t mx8_scale_byte(float amax) {
  if (!(amax > 0.0f)) return 127u;
  int e = ilog2f_dev(amax);
  if (__builtin_amdgcn_ldexpf(amax, -e) > 1.75f) e += 1;
  e = e - 8 + 127;
  return (uint32_t)(e < 0 ? 0 : (e > 254 ? 254 : e));
}

// Four E4M3 codes (one dword, element j in byte j) of f[0..3], each of
// magnitude <= 448, by the hardware conversion (round to nearest even; it
// gives the CPU oracle's or_e4m3_encode bytes for every bf16 value of
// magnitude <= 448, every midpoint between E4M3 neighbours and the fp32
// values one unit either side, and 1M random fp32 values, all checked on
// gfx950)
__device__ __forceinline__ uint32_t e4m3x4(float f0, float f1, float f2, float f3) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(f0, f1, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(f2, f3, w, true);
  return (uint32_t)w;
}

// The 8 elements v of this lane, one quarter (q = lane & 3 of four adjacent
// lanes) of a 32-element block: its hi and lo E4M3 codes (4 per dword) and
// the block's two scale bytes.  Every lane of the quad must take part.
__device__ __forceinline__ void mx8_quant8(const float (&v)[8], uint32_t (&qh)[2],
                                           uint32_t (&ql)[2], uint32_t& b1, uint32_t& b2) {
  float amax = 0.0f;
  uint32_t nonfin = 0;  // bit j: element j is NaN or infinite
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float a = fabsf(v[j]);
    if (a < INFINITY) amax = fmaxf(amax, a);
    else nonfin |= 1u << j;
  }
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  b1 = mx8_scale_byte(amax);
  float t[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    t[j] = (nonfin >> j) & 1 ? 0.0f : __builtin_amdgcn_ldexpf(v[j], 127 - (int)b1);
  qh[0] = e4m3x4(t[0], t[1], t[2], t[3]);
  qh[1] = e4m3x4(t[4], t[5], t[6], t[7]);
  const float hv[8] = {__builtin_amdgcn_cvt_f32_fp8((int)qh[0], 0),
                       __builtin_amdgcn_cvt_f32_fp8((int)qh[0], 1),
                       __builtin_amdgcn_cvt_f32_fp8((int)qh[0], 2),
                       __builtin_amdgcn_cvt_f32_fp8((int)qh[0], 3),
                       __builtin_amdgcn_cvt_f32_fp8((int)qh[1], 0),
                       __builtin_amdgcn_cvt_f32_fp8((int)qh[1], 1),
                       __builtin_amdgcn_cvt_f32_fp8((int)qh[1], 2),
                       __builtin_amdgcn_cvt_f32_fp8((int)qh[1], 3)};
  float res[8], rmax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    res[j] = (nonfin >> j) & 1 ? 0.0f
                               : __fsub_rn(v[j], __builtin_amdgcn_ldexpf(hv[j], (int)b1 - 127));
    rmax = fmaxf(rmax, fabsf(res[j]));
  }
  // a non-finite element: the NaN code in hi, 0 in lo
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if ((nonfin >> j) & 1) qh[j >> 2] = (qh[j >> 2] & ~(0xFFu << (8 * (j & 3)))) | (0x7Fu << (8 * (j & 3)));
  rmax = fmaxf(rmax, __shfl_xor(rmax, 1, 64));
  rmax = fmaxf(rmax, __shfl_xor(rmax, 2, 64));
  b2 = mx8_scale_byte(rmax);
#pragma unroll
  for (int j = 0; j < 8; ++j) t[j] = __builtin_amdgcn_ldexpf(res[j], 127 - (int)b2);
  ql[0] = e4m3x4(t[0], t[1], t[2], t[3]);
  ql[1] = e4m3x4(t[4], t[5], t[6], t[7]);
}

}  // namespace neon

// neon_kernels.hip -- hand-written gfx950 (CDNA4) kernels of the gpt-oss
// token loop, plus their host launchers (declared in neon_internal.hpp).
//
// Decode at small batch is HBM-bound: every kernel streams its weights once
// with 16-byte-per-lane loads, keeps the activation vector in registers, and
// reduces with wave-wide butterflies.  Batch rows are a grid dimension.
//
// Semantics follow the gpt-oss model maths (HF transformers modeling_gpt_oss
// .py, cited as HFM:<line>); the reference repository has no implementation
// of this path.
#include "neon_common.hpp"
#include "neon_internal.hpp"

#include <math.h>
#include <stdlib.h>
#include <string.h>

namespace neon {

// Weight words are read once per step: a non-temporal load (streaming hint,
// no reuse expected in the caches) measured 4.5% faster over the whole step
// than a plain load.
typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_weight16(const void* p) {
  const nt_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint8_t load_weight1(const uint8_t* p) {
  return __builtin_nontemporal_load(p);
}


// ===========================================================================
// Deterministic init (identical integer/fp32 steps to the CPU oracle)
// ===========================================================================
__global__ void k_fill_bf16(uint16_t* __restrict__ out, int64_t n, uint64_t key,
                            float mean, float mul) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += stride) {
    float g = __fmul_rn((float)gauss_int(hash_k(key, (uint64_t)i)), mul);
    out[i] = f2bf(__fadd_rn(mean, g));
  }
}

__global__ void k_fill_bytes(uint8_t* __restrict__ out, int64_t n,
                             uint64_t key) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t nw = (n + 7) / 8;
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < nw;
       w += stride) {
    uint64_t h = hash_k(key, (uint64_t)w);
    if (w * 8 + 8 <= n) {
      *reinterpret_cast<uint64_t*>(out + w * 8) = h;  // little endian bytes
    } else {
      for (int j = 0; j < 8 && w * 8 + j < n; ++j)
        out[w * 8 + j] = (uint8_t)(h >> (8 * j));
    }
  }
}

__global__ void k_fill_scales(uint8_t* __restrict__ out, int64_t n,
                              uint64_t key, int lo, int range) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += stride) {
    uint64_t h = hash_k(key, (uint64_t)i);
    out[i] = (uint8_t)(lo + (int)(((h >> 32) * (uint64_t)range) >> 32));
  }
}

static int fill_grid(int64_t n) {
  int64_t g = (n + 255) / 256;
  return (int)(g < 8192 ? (g < 1 ? 1 : g) : 8192);
}

void launch_fill_bf16(uint16_t* out, int64_t n, uint64_t seed, uint64_t stream,
                      float mean, float mul, hipStream_t st) {
  hipLaunchKernelGGL(k_fill_bf16, dim3(fill_grid(n)), dim3(256), 0, st, out, n,
                     stream_key(seed, stream), mean, mul);
}
void launch_fill_bytes(uint8_t* out, int64_t n, uint64_t seed, uint64_t stream,
                       hipStream_t st) {
  hipLaunchKernelGGL(k_fill_bytes, dim3(fill_grid((n + 7) / 8)), dim3(256), 0,
                     st, out, n, stream_key(seed, stream));
}
void launch_fill_scales(uint8_t* out, int64_t n, uint64_t seed,
                        uint64_t stream, int lo, int range, hipStream_t st) {
  hipLaunchKernelGGL(k_fill_scales, dim3(fill_grid(n)), dim3(256), 0, st, out,
                     n, stream_key(seed, stream), lo, range);
}

// ===========================================================================
// MXFP4 dequantisation (OCP MX v1.0; gpt-oss LUT and nibble order as in HF
// integrations/mxfp4.py:29-46, 298-304).  Exact fp32 values, for tests and
// tools; the GEMVs never materialise dequantised weights.
// ===========================================================================
__constant__ float c_e2m1[16] = {+0.0f, +0.5f, +1.0f, +1.5f, +2.0f, +3.0f,
                                 +4.0f, +6.0f, -0.0f, -0.5f, -1.0f, -1.5f,
                                 -2.0f, -3.0f, -4.0f, -6.0f};

__global__ void k_mxfp4_dequant(const uint8_t* __restrict__ codes,
                                const uint8_t* __restrict__ scales,
                                int64_t n_bytes, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_bytes) return;
  const uint32_t byte = codes[i];
  const uint32_t s = scales[i >> 4];
  float2 r;
  r.x = e8m0_scale(c_e2m1[byte & 15u], s);
  r.y = e8m0_scale(c_e2m1[byte >> 4], s);
  reinterpret_cast<float2*>(out)[i] = r;
}

void launch_mxfp4_dequant(const uint8_t* codes, const uint8_t* scales,
                          int64_t n_blocks, float* out, hipStream_t st) {
  const int64_t nb = n_blocks * 16;
  hipLaunchKernelGGL(k_mxfp4_dequant, dim3((unsigned)((nb + 255) / 256)),
                     dim3(256), 0, st, codes, scales, nb, out);
}


// ===========================================================================
// Shared GEMV machinery.  Lane l of a wave owns the 16-byte units
// u = l + 64 p (p < P) of every row it processes; x for those units stays in
// registers as fp32, so each weight byte is loaded exactly once, 1 KB
// contiguous per wave instruction.  MXFP4 unit = 32 elements (16 B codes + 1
// scale byte); bf16 unit = 8 elements.
//
// Canonical row dot (restated bit for bit by the oracle's or_c_* GEMVs):
//   lane partial a_l, for p = 0..P-1, u = l + 64 p < U:
//     bf16 : a = fmaf(w_k, x_k, a) for the unit's 8 elements in increasing k
//     MXFP4: t = fmaf(E2M1_k, x_k, t) from t = 0 over the unit's 32 elements,
//            then a = a + t * 2^(s_u - 127)   (exact scaling, one rounding)
//   then the xor butterfly a_l = a_l + a_{l^off}, off = 32, 16, 8, 4, 2, 1.
// ===========================================================================
__device__ __forceinline__ void unpack8(const uint4& v, float* o) {
  o[0] = bf_lo(v.x); o[1] = bf_hi(v.x); o[2] = bf_lo(v.y); o[3] = bf_hi(v.y);
  o[4] = bf_lo(v.z); o[5] = bf_hi(v.z); o[6] = bf_lo(v.w); o[7] = bf_hi(v.w);
}

template <int P>
struct Fp4Row {
  uint4 c[P];
  uint32_t s[P];
};

// Loads without branches: a lane past U re-reads the row's last unit and
// fp4_row_partial drops it.  A load under a divergent branch would make the
// compiler wait for every outstanding load before the first use.
template <int P>
__device__ __forceinline__ void fp4_load_row(Fp4Row<P>& r,
                                             const uint8_t* __restrict__ codes,
                                             const uint8_t* __restrict__ scales,
                                             int U, int lane) {
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = min(lane + 64 * p, U - 1);
    r.c[p] = load_weight16(codes + (size_t)u * 16);
    r.s[p] = load_weight1(scales + u);
  }
}

template <int P>
__device__ __forceinline__ float fp4_row_partial(const Fp4Row<P>& r,
                                                 const float (&xr)[P][32],
                                                 int U, int lane) {
  float acc = 0.0f;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const float t = __fadd_rn(acc, e8m0_scale(fp4_unit_dot(r.c[p], xr[p]), r.s[p]));
    acc = (lane + 64 * p < U) ? t : acc;  // padded units leave acc untouched
  }
  return acc;
}

// x (bf16, global) -> fp32 registers for the lane's MXFP4 units
// u = lane + 64 p (32 elements = 4 x 16 B each); lanes past U get zeros.
// Issue and finish are separate so that callers can put the loads ahead of
// the weight rows and wait for them alone.
template <int P>
__device__ __forceinline__ void x_fp4_issue(uint4 (&raw)[P][4],
                                            const uint16_t* __restrict__ x, int U,
                                            int lane) {
  const uint4* xv = reinterpret_cast<const uint4*>(x);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = min(lane + 64 * p, U - 1);
#pragma unroll
    for (int q = 0; q < 4; ++q) raw[p][q] = xv[u * 4 + q];
  }
}
template <int P>
__device__ __forceinline__ void x_fp4_finish(float (&xr)[P][32],
                                             const uint4 (&raw)[P][4], int U,
                                             int lane) {
  const uint4 zero = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      unpack8((lane + 64 * p < U) ? raw[p][q] : zero, &xr[p][8 * q]);
}
template <int P>
__device__ __forceinline__ void wave_load_x_fp4(float (&xr)[P][32],
                                                const uint16_t* __restrict__ x,
                                                int U, int lane) {
  uint4 raw[P][4];
  x_fp4_issue<P>(raw, x, U, lane);
  x_fp4_finish<P>(xr, raw, U, lane);
}

// Two rows with the partial last pass shared.  With P passes over U units,
// the last pass has r = U - 64 (P - 1) units; when r <= 32 one pass covers
// both rows' tails: lanes [0, r) take row A's units 64 (P - 1) + l, lanes
// [r, 2r) row B's (lanes past 2r re-read a valid unit and are ignored).  Row
// B's tail value then moves to lane l - r, so every lane adds the same unit
// values in the same order as the one-row form (bit-identical), with a
// quarter fewer unit computations at U = 90.
template <int P>
struct Fp4RowPair {
  uint4 c[2][P - 1];
  uint32_t s[2][P - 1];
  uint4 tc;
  uint32_t ts;
};

template <int P>
__device__ __forceinline__ void fp4_load_pair(Fp4RowPair<P>& q,
                                              const uint8_t* __restrict__ ca,
                                              const uint8_t* __restrict__ sa,
                                              const uint8_t* __restrict__ cb,
                                              const uint8_t* __restrict__ sb, int U,
                                              int lane) {
#pragma unroll
  for (int p = 0; p < P - 1; ++p) {
    const int u = lane + 64 * p;  // < 64 (P - 1) < U
    q.c[0][p] = load_weight16(ca + (size_t)u * 16);
    q.s[0][p] = load_weight1(sa + u);
    q.c[1][p] = load_weight16(cb + (size_t)u * 16);
    q.s[1][p] = load_weight1(sb + u);
  }
  const int r = U - 64 * (P - 1);
  const bool in_b = lane >= r;
  const int ut = 64 * (P - 1) + min(in_b ? lane - r : lane, r - 1);
  q.tc = load_weight16((in_b ? cb : ca) + (size_t)ut * 16);
  q.ts = load_weight1((in_b ? sb : sa) + ut);
}

// x for the paired form: full passes as usual, the last pass at the lane's
// tail unit (lanes [r, 2r) repeat lanes [0, r)).
template <int P>
__device__ __forceinline__ void x_fp4_issue_pair(uint4 (&raw)[P][4],
                                                 const uint16_t* __restrict__ x, int U,
                                                 int lane) {
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  const int r = U - 64 * (P - 1);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = p < P - 1 ? lane + 64 * p
                            : 64 * (P - 1) + min(lane >= r ? lane - r : lane, r - 1);
#pragma unroll
    for (int q = 0; q < 4; ++q) raw[p][q] = xv[u * 4 + q];
  }
}
template <int P>
__device__ __forceinline__ void x_fp4_finish_pair(float (&xr)[P][32],
                                                  const uint4 (&raw)[P][4]) {
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int q = 0; q < 4; ++q) unpack8(raw[p][q], &xr[p][8 * q]);
}

// Canonical lane partials of both rows (see fp4_row_partial).
template <int P>
__device__ __forceinline__ void fp4_pair_partials(const Fp4RowPair<P>& q,
                                                  const float (&xr)[P][32], int U,
                                                  int lane, float& a, float& b) {
  const int r = U - 64 * (P - 1);
  a = 0.0f;
  b = 0.0f;
#pragma unroll
  for (int p = 0; p < P - 1; ++p) {
    a = __fadd_rn(a, e8m0_scale(fp4_unit_dot(q.c[0][p], xr[p]), q.s[0][p]));
    b = __fadd_rn(b, e8m0_scale(fp4_unit_dot(q.c[1][p], xr[p]), q.s[1][p]));
  }
  const float t = e8m0_scale(fp4_unit_dot(q.tc, xr[P - 1]), q.ts);
  const float tb = __shfl(t, min(lane + r, 63), 64);  // row B's tail, from lane l + r
  const float a2 = __fadd_rn(a, t), b2 = __fadd_rn(b, tb);
  a = lane < r ? a2 : a;
  b = lane < r ? b2 : b;
}

// Host side: the paired form applies when the last pass has at most 32 units.
inline bool fp4_pair_ok(int U, int P) { return P >= 2 && U - 64 * (P - 1) <= 32; }

// The loads of x (and of the norm weights) are issued on their own, before
// any weight-row loads, so that waiting for x does not wait for the rows
// (the vector-memory counter drains in issue order).  NORM is a template
// argument, not a run-time test, so that no branch separates the norm-weight
// loads from their use (the compiler would sink them into it).
template <int P>
struct XBf16Raw {
  uint4 x[P], w[P];
};
template <int P, bool NORM>
__device__ __forceinline__ void wave_x_bf16_issue(XBf16Raw<P>& r,
                                                  const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ nw,
                                                  int K, int lane) {
  // unconditional, clamped loads (no branch, see bf16_load_row); padded units
  // are zeroed in wave_x_bf16_finish
  const int U = K / 8;
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  const uint4* wv = reinterpret_cast<const uint4*>(nw);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = min(lane + 64 * p, U - 1);
    r.x[p] = xv[u];
    if (NORM) r.w[p] = wv[u];
  }
}
template <int P, bool NORM>
__device__ __forceinline__ void wave_x_bf16_finish(float (&xr)[P][8],
                                                   const XBf16Raw<P>& r,
                                                   float eps, int K, int lane,
                                                   uint16_t* __restrict__ xn_out) {
  const int U = K / 8;
  const uint4 zero = make_uint4(0, 0, 0, 0);
  if (!NORM) {
#pragma unroll
    for (int p = 0; p < P; ++p) unpack8((lane + 64 * p < U) ? r.x[p] : zero, xr[p]);
    return;
  }
  // padded units are zeroed and add exactly +0, so no divergent branch is needed
  float ss = 0.0f;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    float f[8];
    unpack8((lane + 64 * p < U) ? r.x[p] : zero, f);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(f[j], f[j], ss);
  }
  ss = wave_sum(ss);
  const float rs = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)K), eps)));
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = lane + 64 * p;
    float a[8], w8[8];
    unpack8(r.x[p], a);
    unpack8(r.w[p], w8);
    uint32_t o4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o4[j] = pack_bf2(__fmul_rn(w8[2 * j], __fmul_rn(a[2 * j], rs)),
                       __fmul_rn(w8[2 * j + 1], __fmul_rn(a[2 * j + 1], rs)));
    const uint4 o = make_uint4(o4[0], o4[1], o4[2], o4[3]);
    unpack8((u < U) ? o : zero, xr[p]);
    if (xn_out != nullptr && u < U) reinterpret_cast<uint4*>(xn_out)[u] = o;
  }
}

// x (bf16, global) -> fp32 registers for the lane's bf16 units u = lane + 64 p,
// optionally RMS-normalised (HFM:57-62).  The canonical RMSNorm (oracle
// or_c_rmsnorm) sums squares with exactly these lane partials: ss = fmaf(x_k,
// x_k, ss) over the lane's units in increasing k, then the xor butterfly, so
// every wave forms the identical r = 1 / sqrt(ss / K + eps) (correctly rounded
// division and square root) on its own, with no LDS and no barrier;
// y_k = bf16(w_k * (x_k * r)).  If xn_out is not NULL the wave also stores the
// normalised vector there (callers pass it from one wave per row).
template <int P>
__device__ __forceinline__ void wave_load_x_bf16(float (&xr)[P][8],
                                                 const uint16_t* __restrict__ x,
                                                 const uint16_t* __restrict__ nw,
                                                 float eps, int K, int lane,
                                                 uint16_t* __restrict__ xn_out) {
  XBf16Raw<P> r;
  if (nw != nullptr) {
    wave_x_bf16_issue<P, true>(r, x, nw, K, lane);
    wave_x_bf16_finish<P, true>(xr, r, eps, K, lane, xn_out);
  } else {
    wave_x_bf16_issue<P, false>(r, x, nw, K, lane);
    wave_x_bf16_finish<P, false>(xr, r, eps, K, lane, xn_out);
  }
}

template <int P>
__device__ __forceinline__ void bf16_load_row(uint4 (&w)[P],
                                              const uint16_t* __restrict__ row,
                                              int U, int lane) {
  // Every load is issued (padded units re-read the row's last unit and are
  // dropped by bf16_row_partial): a load under a divergent branch forces the
  // compiler to wait for all outstanding loads before any use.
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = min(lane + 64 * p, U - 1);
    w[p] = load_weight16(row + (size_t)u * 8);
  }
}

template <int P>
__device__ __forceinline__ float bf16_row_partial(const uint4 (&w)[P],
                                                  const float (&xr)[P][8],
                                                  int U, int lane) {
  float acc = 0.0f;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const float t = fma8_bf16(w[p], xr[p], acc);
    acc = (lane + 64 * p < U) ? t : acc;  // padded units leave acc untouched
  }
  return acc;
}


// xor butterfly (off = 32 .. 1) of 8 rows at once, on named scalars.  Both
// lanes of an xor pair hold the same sum after every step (fp32 addition
// commutes), so at step `off` a lane keeps half of its rows and sends the
// other half: 7 + 3 shuffles, bit-identical to 8 separate butterflies.  Lane
// l returns the total of row l >> 3.
template <int OFF>
__device__ __forceinline__ float xchg(float keep, float send) {
  return __fadd_rn(keep, xor_lane<OFF>(send));
}
__device__ __forceinline__ float wave_sum_8rows(float a0, float a1, float a2,
                                                float a3, float a4, float a5,
                                                float a6, float a7, int lane) {
  const bool u32 = (lane & 32) != 0, u16 = (lane & 16) != 0, u8 = (lane & 8) != 0;
  // off 32: lanes without bit 5 keep rows 0-3, the others rows 4-7
  const float b0 = xchg<32>(u32 ? a4 : a0, u32 ? a0 : a4);
  const float b1 = xchg<32>(u32 ? a5 : a1, u32 ? a1 : a5);
  const float b2 = xchg<32>(u32 ? a6 : a2, u32 ? a2 : a6);
  const float b3 = xchg<32>(u32 ? a7 : a3, u32 ? a3 : a7);
  // off 16: keep rows {0,1} or {2,3} of the group
  const float c0 = xchg<16>(u16 ? b2 : b0, u16 ? b0 : b2);
  const float c1 = xchg<16>(u16 ? b3 : b1, u16 ? b1 : b3);
  // off 8: keep row 0 or 1
  float t = xchg<8>(u8 ? c1 : c0, u8 ? c0 : c1);
  t = __fadd_rn(t, xor_lane<4>(t));
  t = __fadd_rn(t, xor_lane<2>(t));
  t = __fadd_rn(t, xor_lane<1>(t));
  return t;
}

// xor butterfly of 4 rows at once (see wave_sum_8rows); lane l returns the
// total of row l >> 4.
__device__ __forceinline__ float wave_sum_4rows(float a0, float a1, float a2,
                                                float a3, int lane) {
  const bool u32 = (lane & 32) != 0, u16 = (lane & 16) != 0;
  const float b0 = __fadd_rn(u32 ? a2 : a0, xor_lane<32>(u32 ? a0 : a2));
  const float b1 = __fadd_rn(u32 ? a3 : a1, xor_lane<32>(u32 ? a1 : a3));
  float t = __fadd_rn(u16 ? b1 : b0, xor_lane<16>(u16 ? b0 : b1));
  t = __fadd_rn(t, xor_lane<8>(t));
  t = __fadd_rn(t, xor_lane<4>(t));
  t = __fadd_rn(t, xor_lane<2>(t));
  t = __fadd_rn(t, xor_lane<1>(t));
  return t;
}

// xor butterfly of 2 rows at once (see wave_sum_8rows); lane l returns the
// total of row l >> 5.
__device__ __forceinline__ float wave_sum_2rows(float a0, float a1, int lane) {
  const bool u32 = (lane & 32) != 0;
  float t = __fadd_rn(u32 ? a1 : a0, xor_lane<32>(u32 ? a0 : a1));
  t = __fadd_rn(t, xor_lane<16>(t));
  t = __fadd_rn(t, xor_lane<8>(t));
  t = __fadd_rn(t, xor_lane<4>(t));
  t = __fadd_rn(t, xor_lane<2>(t));
  t = __fadd_rn(t, xor_lane<1>(t));
  return t;
}

// ===========================================================================
// Standalone MXFP4 GEMV: y[b][n] = bf16(dot(W[n], x[b]) + bias[n]).
// grid (ceil(N / (4 rpw)), 1, B), block 256; wave w of block i owns rows
// [(4i + w) rpw, +rpw).  The next row's codes load while the current row is
// reduced.
// ===========================================================================
template <int P>
__global__ __launch_bounds__(256) void k_mxfp4_gemv(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ scales,
    const uint16_t* __restrict__ bias, const uint16_t* __restrict__ x,
    uint16_t* __restrict__ y, int N, int K, int rpw) {
  const int U = K / 32, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.z;
  const int r0 = (blockIdx.x * 4 + wave) * rpw;
  const int r1 = min(r0 + rpw, N);
  if (r0 >= r1) return;
  Fp4Row<P> cur;
  fp4_load_row<P>(cur, codes + (size_t)r0 * (K / 2), scales + (size_t)r0 * U, U, lane);
  float xr[P][32];
  wave_load_x_fp4<P>(xr, x + (size_t)b * K, U, lane);
  for (int r = r0; r < r1; ++r) {
    // the row's bias is requested before its dot product (a load issued
    // after the butterfly would be one more round trip per row)
    const uint16_t br = bias != nullptr ? load_pinned_u16(bias + r) : (uint16_t)0;
    Fp4Row<P> nxt;
    if (r + 1 < r1)
      fp4_load_row<P>(nxt, codes + (size_t)(r + 1) * (K / 2),
                      scales + (size_t)(r + 1) * U, U, lane);
    float acc = wave_sum(fp4_row_partial<P>(cur, xr, U, lane));
    if (lane == 0) {
      if (bias) acc = __fadd_rn(acc, bf2f(br));
      y[(size_t)b * N + r] = f2bf(acc);
    }
    cur = nxt;
  }
}

template <int P>
static void launch_mxfp4_gemv_p(const uint8_t* codes, const uint8_t* scales,
                                const uint16_t* bias, const uint16_t* x,
                                uint16_t* y, int N, int K, int B,
                                hipStream_t st) {
  int rpw = 1;
  while (rpw < 8 && (N + 4 * rpw * 2 - 1) / (4 * rpw * 2) >= 512) rpw *= 2;
  const int nblk = (N + 4 * rpw - 1) / (4 * rpw);
  hipLaunchKernelGGL(k_mxfp4_gemv<P>, dim3(nblk, 1, B), dim3(256), 0, st,
                     codes, scales, bias, x, y, N, K, rpw);
}

// Register "copies" the compiler cannot see through: inside the per-pair
// loops the weight words are laundered once per iteration, so the E2M1
// conversions are not hoisted out of the loop (which keeps every converted
// value live and drops the kernel to one wave per SIMD).  No code is emitted.
__device__ __forceinline__ void launder(uint4& v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}
__device__ __forceinline__ void launder(uint32_t& v) { asm volatile("" : "+v"(v)); }
template <int P>
__device__ __forceinline__ void launder(Fp4RowPair<P>& q) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int p = 0; p < P - 1; ++p) { launder(q.c[i][p]); launder(q.s[i][p]); }
  launder(q.tc);
  launder(q.ts);
}
template <int P>
__device__ __forceinline__ void launder(Fp4Row<P>& r) {
#pragma unroll
  for (int p = 0; p < P; ++p) { launder(r.c[p]); launder(r.s[p]); }
}

// Batched form (B >= 2): every weight row is read once for all B input rows.
// Wave w of block i owns rows 4 (4 i + w) .. +3, held in registers; it walks
// the batch rows, the next row's x loading while the current one is reduced.
// Each (row, batch row) dot is the canonical one above (x of a pass unpacked
// when it is used), so y is bit-identical to B separate batch-1 launches.
template <int P, bool PAIR>
__global__ __launch_bounds__(256) void k_mxfp4_gemv_bt(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ scales,
    const uint16_t* __restrict__ bias, const uint16_t* __restrict__ x,
    uint16_t* __restrict__ y, int N, int K, int B) {
  const int U = K / 32, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * 4;
  if (n0 >= N) return;
  const uint16_t bq =  // unconditional (the input when there is no bias): no branch to join
      load_pinned_u16(bias != nullptr ? bias + min(n0 + (lane >> 4), N - 1) : x);
  const uint16_t bl = bias != nullptr ? bq : (uint16_t)0;
  Fp4RowPair<P> rp[2];
  Fp4Row<P> rw[PAIR ? 1 : 4];
  if constexpr (PAIR) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int na = min(n0 + 2 * c, N - 1), nb = min(n0 + 2 * c + 1, N - 1);
      fp4_load_pair<P>(rp[c], codes + (size_t)na * (K / 2), scales + (size_t)na * U,
                       codes + (size_t)nb * (K / 2), scales + (size_t)nb * U, U, lane);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = min(n0 + r, N - 1);
      fp4_load_row<P>(rw[r], codes + (size_t)n * (K / 2), scales + (size_t)n * U, U, lane);
    }
  }
  uint4 xraw[P][4];
  if (PAIR) x_fp4_issue_pair<P>(xraw, x, U, lane);
  else x_fp4_issue<P>(xraw, x, U, lane);
  __builtin_amdgcn_sched_barrier(0);
  const int r_tail = U - 64 * (P - 1);
  for (int b = 0; b < B; ++b) {
    if constexpr (PAIR) {
#pragma unroll
      for (int c = 0; c < 2; ++c) launder(rp[c]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int p = 0; p < P; ++p) { launder(rw[r].c[p]); launder(rw[r].s[p]); }
      }
    }
    uint4 cur[P][4];
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int q = 0; q < 4; ++q) cur[p][q] = xraw[p][q];
    if (b + 1 < B) {
      if (PAIR) x_fp4_issue_pair<P>(xraw, x + (size_t)(b + 1) * K, U, lane);
      else x_fp4_issue<P>(xraw, x + (size_t)(b + 1) * K, U, lane);
    }
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (PAIR) {
#pragma unroll
      for (int p = 0; p < P - 1; ++p) {
        float xp[32];
#pragma unroll
        for (int q = 0; q < 4; ++q) unpack8(cur[p][q], &xp[8 * q]);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          a[2 * c] = __fadd_rn(a[2 * c], e8m0_scale(fp4_unit_dot(rp[c].c[0][p], xp), rp[c].s[0][p]));
          a[2 * c + 1] =
              __fadd_rn(a[2 * c + 1], e8m0_scale(fp4_unit_dot(rp[c].c[1][p], xp), rp[c].s[1][p]));
        }
      }
      float xp[32];
#pragma unroll
      for (int q = 0; q < 4; ++q) unpack8(cur[P - 1][q], &xp[8 * q]);
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const float tt = e8m0_scale(fp4_unit_dot(rp[c].tc, xp), rp[c].ts);
        const float tb = __shfl(tt, min(lane + r_tail, 63), 64);  // row B's tail
        const float a2 = __fadd_rn(a[2 * c], tt), b2 = __fadd_rn(a[2 * c + 1], tb);
        a[2 * c] = lane < r_tail ? a2 : a[2 * c];
        a[2 * c + 1] = lane < r_tail ? b2 : a[2 * c + 1];
      }
    } else {
      const uint4 zero = make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const bool on = lane + 64 * p < U;
        float xp[32];
#pragma unroll
        for (int q = 0; q < 4; ++q) unpack8(on ? cur[p][q] : zero, &xp[8 * q]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float t2 = __fadd_rn(a[r], e8m0_scale(fp4_unit_dot(rw[r].c[p], xp), rw[r].s[p]));
          a[r] = on ? t2 : a[r];  // padded units leave the partial untouched
        }
      }
    }
    const float t = wave_sum_4rows(a[0], a[1], a[2], a[3], lane);
    const int n = n0 + (lane >> 4);
    if ((lane & 15) == 0 && n < N) {
      float v = t;
      if (bias != nullptr) v = __fadd_rn(v, bf2f(bl));
      y[(size_t)b * N + n] = f2bf(v);
    }
  }
}

void launch_mxfp4_gemv(const uint8_t* codes, const uint8_t* scales,
                       const uint16_t* bias, const uint16_t* x, uint16_t* y,
                       int N, int K, int B, hipStream_t st) {
  const int P = (K / 32 + 63) / 64;
  if (B >= kMxfp4GemvMfmaMinB) {  // a dense contraction: the matrix cores
    launch_mxfp4_gemv_mfma(codes, scales, bias, x, y, N, K, B, st);
    return;
  }
  // (the one-row kernel with one grid slice per row measured slower at B = 4:
  // 8.8 against 7.0 us at N = 2880 -- every slice re-reads the weights)
  if (B >= 2) {
    const int nblk = (N + 15) / 16;
    const bool pr = fp4_pair_ok(K / 32, P);
#define BT_CASE(PP)                                                                          \
  case PP:                                                                                   \
    if (pr) hipLaunchKernelGGL((k_mxfp4_gemv_bt<PP, true>), dim3(nblk), dim3(256), 0, st,   \
                               codes, scales, bias, x, y, N, K, B);                         \
    else hipLaunchKernelGGL((k_mxfp4_gemv_bt<PP, false>), dim3(nblk), dim3(256), 0, st,     \
                            codes, scales, bias, x, y, N, K, B);                            \
    return;
    switch (P) {
      BT_CASE(1) BT_CASE(2) BT_CASE(3)
      default: BT_CASE(4)
    }
#undef BT_CASE
  }
  switch (P) {
    case 1: launch_mxfp4_gemv_p<1>(codes, scales, bias, x, y, N, K, B, st); break;
    case 2: launch_mxfp4_gemv_p<2>(codes, scales, bias, x, y, N, K, B, st); break;
    case 3: launch_mxfp4_gemv_p<3>(codes, scales, bias, x, y, N, K, B, st); break;
    default: launch_mxfp4_gemv_p<4>(codes, scales, bias, x, y, N, K, B, st); break;
  }
}

// ===========================================================================
// bf16 GEMV with fused prologue (optional RMSNorm of x) and epilogue:
//   MODE_STORE : y[b][n] = bf16(dot + bias[n])
//   MODE_RESID : y[b][n] = bf16(y[b][n] + bf16(dot + bias[n]))  (residual add,
//                HFM:365,375)
//   MODE_LOGITS: logits[b][n] = dot (fp32), plus the block's (max, lowest
//                argmax) written to part_val/part_idx [B][gridDim.x]
// grid (nblk, 1, B), block 256; a wave takes groups of R consecutive rows
// (grid-strided, so huge N such as lm_head runs on a bounded grid), loads
// all R rows before any arithmetic and reduces them together with the
// R-row xor butterfly (bit-identical to R separate butterflies); lane
// (64 / R) r then holds row r, so the R epilogues run in parallel lanes.
// R = 2 for the projections (more waves in flight), 4 for lm_head.
// ===========================================================================
// (value, index) candidates of lanes l ^ OFF for OFF = LO, 2 LO, .. HI: keep
// the larger value, the lower index on ties (an order-free reduction)
template <int LO, int HI>
__device__ __forceinline__ void argmax_steps(float& v, int32_t& i) {
  if constexpr (LO <= HI) {
    const float ov = xor_lane<LO>(v);
    const int32_t oi = xor_lane_i<LO>(i);
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
    argmax_steps<2 * LO, HI>(v, i);
  }
}

enum { MODE_STORE = 0, MODE_RESID = 1, MODE_LOGITS = 2, MODE_QKV = 3 };


// Row r of wave group g.  MODE_QKV pairs dims d and d + 32 of one 64-dim
// head (group g: head g / 32, d = g % 32) so that the RoPE pair of a q or k
// head finishes in one wave; the other modes take R consecutive rows.
template <int MODE, int R>
__device__ __forceinline__ int group_row(int g, int r) {
  if constexpr (MODE == MODE_QKV) return ((g >> 5) << 6) + (g & 31) + 32 * r;
  else return g * R + r;
}


template <int R>
constexpr int log2_rows() { return R == 4 ? 2 : (R == 2 ? 1 : 0); }

// One group of R rows.  FIRST: the wave's first group, which also finishes
// the input (and its RMSNorm) from the raw loads issued before the rows, so
// that work overlaps the row loads; later groups reuse xr.
template <int P, int MODE, bool NORM, bool FIRST, int R, bool AGENT_Y = false>
__device__ __forceinline__ void gemv_bf16_group(
    int g, const uint16_t* __restrict__ W, const uint16_t* __restrict__ bias,
    uint16_t bias_first, float (&xr)[P][8], const XBf16Raw<P>& xraw, float eps,
    uint16_t* __restrict__ y, float* __restrict__ logits, int b, int N, int K,
    int lane, float& best_v, int32_t& best_i, const RopeArgs& rp, int p, int sq) {
  const int U = K / 8;
  constexpr int LS = 6 - log2_rows<R>();  // lane (1 << LS) r holds row r after the sum
  const int my_row = lane >> LS;
  const int r0 = g * R;
  const int nr = MODE == MODE_QKV ? R : min(R, N - r0);  // QKV: N is a multiple of 64
  uint4 w[R][P];
#pragma unroll
  for (int r = 0; r < R; ++r)
    bf16_load_row<P>(w[r], W + (size_t)min(group_row<MODE, R>(g, r), N - 1) * K, U, lane);
  float rc = 0.0f, rs = 0.0f;  // RoPE cos / sin of dim g % 32 at position p
  if (MODE == MODE_QKV) {
    rc = load_pinned_f32(rp.cos_t + (size_t)p * 32 + (g & 31));
    rs = load_pinned_f32(rp.sin_t + (size_t)p * 32 + (g & 31));
  }
  uint16_t bias_b = bias_first;  // the first group's bias was loaded before x
  if (!FIRST && MODE != MODE_LOGITS && bias != nullptr)
    bias_b = bias[group_row<MODE, R>(g, min(my_row, nr - 1))];
  if (FIRST) {
    __builtin_amdgcn_sched_barrier(0);  // all row loads issue before the norm's math
    wave_x_bf16_finish<P, NORM>(xr, xraw, eps, K, lane, nullptr);
  }
  float tot;
  if constexpr (R == 4)
    tot = wave_sum_4rows(bf16_row_partial<P>(w[0], xr, U, lane),
                         bf16_row_partial<P>(w[1], xr, U, lane),
                         bf16_row_partial<P>(w[2], xr, U, lane),
                         bf16_row_partial<P>(w[3], xr, U, lane), lane);
  else if constexpr (R == 2)
    tot = wave_sum_2rows(bf16_row_partial<P>(w[0], xr, U, lane),
                         bf16_row_partial<P>(w[1], xr, U, lane), lane);
  else
    tot = wave_sum(bf16_row_partial<P>(w[0], xr, U, lane));
  const int r = group_row<MODE, R>(g, my_row);
  constexpr int kLead = (1 << LS) - 1;  // lanes with (lane & kLead) == 0 store
  if constexpr (MODE == MODE_QKV) {
    // lanes 0-31 hold dim d of head g / 32, lanes 32-63 dim d + 32: the
    // projection row is stored as is; q and k heads are rotated (the decode
    // attention reads q from q_out) and k, v go to cache row p
    const int head = g >> 5, dd = (g & 31) + 32 * my_row;
    const uint16_t yv = f2bf(bias ? __fadd_rn(tot, bf2f(bias_b)) : tot);
    const float yf = bf2f(yv);
    const float other = xor_lane<32>(yf);
    if ((lane & kLead) == 0) {
      y[(size_t)b * N + r] = yv;
      if (head < rp.Hq + rp.Hkv) {
        float o1, o2;
        rope_pair(my_row ? other : yf, my_row ? yf : other, rc, rs, o1, o2);
        const uint16_t o = f2bf(my_row ? o2 : o1);
        if (head < rp.Hq)
          rp.q_out[((size_t)b * rp.Hq + head) * 64 + dd] = o;
        else
          rp.kc[(((size_t)sq * rp.Hkv + head - rp.Hq) * rp.T_max + (p & rp.key_mask)) * 64 + dd] = o;
      } else {
        rp.vc[(((size_t)sq * rp.Hkv + head - rp.Hq - rp.Hkv) * rp.T_max + (p & rp.key_mask)) * 64 + dd] = yv;
      }
    }
  } else if (my_row < nr) {
    if (MODE == MODE_LOGITS) {
      if (tot > best_v) { best_v = tot; best_i = r; }  // rows rise within a lane
      if ((lane & kLead) == 0) logits[(size_t)b * N + r] = tot;
    } else if ((lane & kLead) == 0) {
      const float v = bias ? __fadd_rn(tot, bf2f(bias_b)) : tot;
      const size_t o = (size_t)b * N + r;
      if (MODE == MODE_STORE) {
        y[o] = f2bf(v);
      } else {
        const uint16_t yo = f2bf(__fadd_rn(bf2f(y[o]), bf2f(f2bf(v))));
        if (AGENT_Y)  // read by other blocks of this launch
          __hip_atomic_store(y + o, yo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          y[o] = yo;
      }
    }
  }
}

template <int P, int MODE, bool NORM, int R>
__global__ __launch_bounds__(256) void k_gemv_bf16(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ bias,
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ nw, float eps,
    uint16_t* __restrict__ y, float* __restrict__ logits,
    float* __restrict__ part_val, int32_t* __restrict__ part_idx, int N, int K,
    RopeArgs rp) {
  __shared__ float bv_s[4];
  __shared__ int32_t bi_s[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.z;
  const int ngroups = (N + R - 1) / R;
  const int gstride = gridDim.x * 4;
  const int g0 = blockIdx.x * 4 + wave;
  // The first group's bias, then the input, go out before any row load:
  // waiting for them then does not wait for the rows (the vector-memory
  // counter drains in issue order).  Both loads are unconditional (clamped
  // addresses) so that no branch makes the compiler wait for everything.
  // (The position and sequence below are block-uniform, so the compiler
  // reads them into scalar registers and waits for them first; keeping them
  // in vector registers (lane_zero) so that the rows go out before that wait
  // measured 0.3% slower over the 20b step: 1.2271 against 1.2230 ms.)
  const int p = MODE == MODE_QKV ? (int)load_pinned_u32(
                                        reinterpret_cast<const uint32_t*>(rp.pos) + b)
                                  : 0;
  // the KV-cache sequence of row b (rows of one prompt share a sequence)
  const int sq = (MODE == MODE_QKV && rp.seq != nullptr)
                     ? (int)load_pinned_u32(reinterpret_cast<const uint32_t*>(rp.seq) + b)
                     : b;
  uint16_t bias_first = 0;
  if (MODE != MODE_LOGITS) {
    const int rb = min(group_row<MODE, R>(g0, lane >> (6 - log2_rows<R>())), N - 1);
    bias_first = (bias != nullptr ? bias : W)[rb];
  }
  float xr[P][8];
  XBf16Raw<P> xraw;
  wave_x_bf16_issue<P, NORM>(xraw, x + (size_t)b * K, nw, K, lane);
  __builtin_amdgcn_sched_barrier(0);  // keep the scheduler from mixing them with the rows
  float best_v = -INFINITY;
  int32_t best_i = 0x7fffffff;
  if (g0 < ngroups) {
    gemv_bf16_group<P, MODE, NORM, true, R>(g0, W, bias, bias_first, xr, xraw, eps, y,
                                            logits, b, N, K, lane, best_v, best_i, rp, p, sq);
    for (int g = g0 + gstride; g < ngroups; g += gstride)
      gemv_bf16_group<P, MODE, NORM, false, R>(g, W, bias, 0, xr, xraw, eps, y, logits, b,
                                               N, K, lane, best_v, best_i, rp, p, sq);
  }
  if (MODE == MODE_LOGITS) {
    // lanes 64 r / R hold the wave's candidates: keep the larger value, the
    // lower row on ties
    argmax_steps<64 / R, 32>(best_v, best_i);
    if (lane == 0) { bv_s[wave] = best_v; bi_s[wave] = best_i; }
    __syncthreads();
    if (threadIdx.x == 0) {
      float v = bv_s[0];
      int32_t i = bi_s[0];
      for (int w = 1; w < 4; ++w)
        if (bv_s[w] > v || (bv_s[w] == v && bi_s[w] < i)) { v = bv_s[w]; i = bi_s[w]; }
      part_val[(size_t)b * gridDim.x + blockIdx.x] = v;
      part_idx[(size_t)b * gridDim.x + blockIdx.x] = i;
    }
  }
}

// rows per wave group, measured at the 20b shapes: QKV (store) 8.7 us with 2
// rows against 9.4 with 1 or 4; O (residual) 7.1 us with 1 against 7.5 with
// 2; lm_head (logits) 4
template <int MODE>
constexpr int gemv_rows() { return MODE == MODE_LOGITS ? 4 : (MODE == MODE_RESID ? 1 : 2); }

static RopeArgs rope_args(const GemvArgs& a) {
  RopeArgs r;
  r.pos = a.pos; r.cos_t = a.cos_t; r.sin_t = a.sin_t; r.q_out = a.q_out;
  r.kc = a.kc; r.vc = a.vc; r.seq = a.seq; r.Hq = a.Hq; r.Hkv = a.Hkv; r.T_max = a.T_max;
  r.key_mask = a.key_mask;
  return r;
}

template <int P, int MODE>
static void launch_gemv_bf16_p(const GemvArgs& a, hipStream_t st) {
  constexpr int R = gemv_rows<MODE>();
  if (a.norm_w != nullptr)
    hipLaunchKernelGGL((k_gemv_bf16<P, MODE, true, R>), dim3(a.nblk, 1, a.B), dim3(256),
                       0, st, a.W, a.bias, a.x, a.norm_w, a.eps, a.y, a.logits,
                       a.part_val, a.part_idx, a.N, a.K, rope_args(a));
  else
    hipLaunchKernelGGL((k_gemv_bf16<P, MODE, false, R>), dim3(a.nblk, 1, a.B), dim3(256),
                       0, st, a.W, a.bias, a.x, a.norm_w, a.eps, a.y, a.logits,
                       a.part_val, a.part_idx, a.N, a.K, rope_args(a));
}

template <int MODE>
static void launch_gemv_bf16_m(const GemvArgs& a, hipStream_t st) {
  const int P = (a.K / 8 + 63) / 64;
  switch (P) {
    case 1: launch_gemv_bf16_p<1, MODE>(a, st); break;
    case 2: launch_gemv_bf16_p<2, MODE>(a, st); break;
    case 3: launch_gemv_bf16_p<3, MODE>(a, st); break;
    case 4: launch_gemv_bf16_p<4, MODE>(a, st); break;
    case 5: launch_gemv_bf16_p<5, MODE>(a, st); break;
    case 6: launch_gemv_bf16_p<6, MODE>(a, st); break;
    case 7: launch_gemv_bf16_p<7, MODE>(a, st); break;
    case 8: launch_gemv_bf16_p<8, MODE>(a, st); break;
    default: launch_gemv_bf16_p<16, MODE>(a, st); break;
  }
}

int gemv_default_grid(int N, int mode) {
  const int R = mode == MODE_LOGITS ? gemv_rows<MODE_LOGITS>()
                : mode == MODE_RESID ? gemv_rows<MODE_RESID>()
                : mode == MODE_QKV   ? gemv_rows<MODE_QKV>()
                                     : gemv_rows<MODE_STORE>();
  const int ngroups = (N + R - 1) / R;
  const int nblk = (ngroups + 3) / 4;
  return nblk < 4096 ? nblk : 4096;  // lm_head: 4096 blocks measured 1% faster than 2048
}

void launch_gemv_bf16(const GemvArgs& a, hipStream_t st) {
  switch (a.mode) {
    case MODE_STORE: launch_gemv_bf16_m<MODE_STORE>(a, st); break;
    case MODE_RESID: launch_gemv_bf16_m<MODE_RESID>(a, st); break;
    case MODE_QKV: launch_gemv_bf16_m<MODE_QKV>(a, st); break;
    default: launch_gemv_bf16_m<MODE_LOGITS>(a, st); break;
  }
}

// ===========================================================================
// Batched bf16 GEMV (2 <= B): every weight row is read from HBM once per step
// and dotted with up to BT inputs held in LDS.  Block = 8 waves; its rows
// b0 .. b0 + BT - 1 are RMS-normalised (or copied) into LDS as bf16 units
// first (waves w and w + 8 of the row index), then the waves grid-stride
// over groups of R weight rows.
//
// Every (row, b) total is the canonical one of the batch-1 kernel: lane l
// accumulates its units u = l + 64 p in order with 8 fmaf each, and the R BT
// lane partials are reduced by one multi-value xor butterfly (bit-identical
// to R BT separate butterflies, see wave_sum_nvals), so batch b's outputs
// equal a batch-1 step's bit for bit.
// ===========================================================================

// xor butterfly (off = 32 .. 1) of N values at once: at each step a lane keeps
// half of its values and sends the other half (fp32 addition commutes, so
// both lanes of a pair hold the same sums); lane l returns value
// l >> (6 - log2 N) when N <= 64.
template <int N, int OFF = 32>
__device__ __forceinline__ float wave_sum_nvals(const float (&a)[N], int lane) {
  if constexpr (N == 1) {
    if constexpr (OFF >= 1) return wave_sum<OFF>(a[0]);
    else return a[0];
  } else {
    static_assert(OFF >= 1, "wave_sum_nvals: at most 64 values");
    const bool up = (lane & OFF) != 0;
    float h[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; ++i)
      h[i] = __fadd_rn(up ? a[i + N / 2] : a[i], xor_lane<OFF>(up ? a[i] : a[i + N / 2]));
    return wave_sum_nvals<N / 2, OFF / 2>(h, lane);
  }
}

template <int N>
constexpr int log2_n() { return N <= 1 ? 0 : 1 + log2_n<N / 2>(); }

template <int P, int MODE, bool NORM, int R, int BT>
__global__ __launch_bounds__(512) void k_gemv_bf16_bt(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ bias,
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ nw, float eps,
    uint16_t* __restrict__ y, float* __restrict__ logits,
    float* __restrict__ part_val, int32_t* __restrict__ part_idx, int N, int K, int B,
    RopeArgs rp) {
  extern __shared__ __align__(16) uint4 xs[];  // [BT][U] normalised inputs (bf16 units)
  __shared__ float bv_s[8][BT];
  __shared__ int32_t bi_s[8][BT];
  constexpr int NV = R * BT;                    // values per lane group
  constexpr int LS = 6 - log2_n<NV>();          // lane (1 << LS) v holds value v
  static_assert(NV <= 64, "R * BT must be at most 64");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int U = K / 8;
  const int b0 = blockIdx.z * BT;
  // ---- inputs into LDS ----------------------------------------------------
  for (int bb = wave; bb < BT; bb += 8) {
    const int b = b0 + bb;
    if (b < B) {
      XBf16Raw<P> raw;
      float xr[P][8];
      wave_x_bf16_issue<P, NORM>(raw, x + (size_t)b * K, nw, K, lane);
      wave_x_bf16_finish<P, NORM>(xr, raw, eps, K, lane, nullptr);
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int u = lane + 64 * p;
        if (u < U)
          xs[bb * U + u] = make_uint4(pack_bf2(xr[p][0], xr[p][1]), pack_bf2(xr[p][2], xr[p][3]),
                                      pack_bf2(xr[p][4], xr[p][5]), pack_bf2(xr[p][6], xr[p][7]));
      }
    } else {
      for (int u = lane; u < U; u += 64) xs[bb * U + u] = make_uint4(0, 0, 0, 0);
    }
  }
  __syncthreads();
  // the value this lane holds after the butterfly: (row r, batch row bb)
  const int v_l = lane >> LS, r_l = v_l / BT, bb_l = v_l % BT, b_l = b0 + bb_l;
  const bool lead = (lane & ((1 << LS) - 1)) == 0 && b_l < B;
  // position and sequence of the lane's row: vector registers, no branch
  // (lane_zero), so the rows' loads below are not held up by them
  int p_l = 0, s_l = b_l;
  if constexpr (MODE == MODE_QKV) {
    const int bi = min(b_l, B - 1) + lane_zero(B);
    const uint32_t* pp = reinterpret_cast<const uint32_t*>(rp.pos) + bi;
    const uint32_t* sp = rp.seq != nullptr ? reinterpret_cast<const uint32_t*>(rp.seq) + bi : pp;
    p_l = (int)load_pinned_u32(pp);
    const int sv = (int)load_pinned_u32(sp);
    s_l = rp.seq != nullptr ? sv : b_l;
  }
  float best_v = -INFINITY;
  int32_t best_i = 0x7fffffff;
  const int ngroups = (N + R - 1) / R;
  for (int g = blockIdx.x * 8 + wave; g < ngroups; g += gridDim.x * 8) {
    uint4 w[R][P];
#pragma unroll
    for (int r = 0; r < R; ++r)
      bf16_load_row<P>(w[r], W + (size_t)min(group_row<MODE, R>(g, r), N - 1) * K, U, lane);
    const int row_l = group_row<MODE, R>(g, r_l);
    // unconditional (the weights when there is no bias): no branch to join
    const uint16_t bias_l =
        MODE != MODE_LOGITS ? load_pinned_u16((bias != nullptr ? bias : W) + min(row_l, N - 1)) : 0;
    float rc = 0.0f, rs = 0.0f;
    if (MODE == MODE_QKV) {
      rc = load_pinned_f32(rp.cos_t + (size_t)p_l * 32 + (g & 31));
      rs = load_pinned_f32(rp.sin_t + (size_t)p_l * 32 + (g & 31));
    }
    float acc[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const bool in = lane + 64 * p < U;  // padded units leave the sums untouched
      const int u = min(lane + 64 * p, U - 1);
      float wf[R][8];  // the R rows' unit p, unpacked once for all BT inputs
#pragma unroll
      for (int r = 0; r < R; ++r) unpack8(w[r][p], wf[r]);
#pragma unroll
      for (int b4 = 0; b4 < BT; b4 += 4) {
        // four inputs at a time; the barrier keeps the scheduler from hoisting
        // every LDS read of the unit (BT x 4 registers) ahead of the math
        constexpr int NB = BT < 4 ? BT : 4;
        uint4 xv[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) xv[i] = xs[(b4 + i) * U + u];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
          float xf[8];
          unpack8(xv[i], xf);
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float t = acc[r * BT + b4 + i];
#pragma unroll
            for (int e = 0; e < 8; ++e) t = __builtin_fmaf(wf[r][e], xf[e], t);
            acc[r * BT + b4 + i] = in ? t : acc[r * BT + b4 + i];
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    const float tot = wave_sum_nvals<NV>(acc, lane);
    if constexpr (MODE == MODE_QKV) {
      // R = 2: lanes with r_l = 0 hold dim d, r_l = 1 dim d + 32 of head g / 32
      const int head = g >> 5, dd = (g & 31) + 32 * r_l;
      const uint16_t yv = f2bf(bias ? __fadd_rn(tot, bf2f(bias_l)) : tot);
      const float yf = bf2f(yv);
      const float other = xor_lane<32>(yf);
      if (lead) {
        y[(size_t)b_l * N + row_l] = yv;
        if (head < rp.Hq + rp.Hkv) {
          float o1, o2;
          rope_pair(r_l ? other : yf, r_l ? yf : other, rc, rs, o1, o2);
          const uint16_t o = f2bf(r_l ? o2 : o1);
          if (head < rp.Hq)
            rp.q_out[((size_t)b_l * rp.Hq + head) * 64 + dd] = o;
          else
            rp.kc[(((size_t)s_l * rp.Hkv + head - rp.Hq) * rp.T_max + (p_l & rp.key_mask)) * 64 + dd] = o;
        } else {
          rp.vc[(((size_t)s_l * rp.Hkv + head - rp.Hq - rp.Hkv) * rp.T_max + (p_l & rp.key_mask)) * 64 + dd] = yv;
        }
      }
    } else if constexpr (MODE == MODE_LOGITS) {
      if (row_l < N) {
        if (tot > best_v) { best_v = tot; best_i = row_l; }  // rows rise within a lane
        if (lead) logits[(size_t)b_l * N + row_l] = tot;
      }
    } else {
      if (lead && row_l < N) {
        const float v = bias ? __fadd_rn(tot, bf2f(bias_l)) : tot;
        const size_t o = (size_t)b_l * N + row_l;
        if (MODE == MODE_STORE) y[o] = f2bf(v);
        else y[o] = f2bf(__fadd_rn(bf2f(y[o]), bf2f(f2bf(v))));
      }
    }
  }
  if constexpr (MODE == MODE_LOGITS) {
    // lanes with r_l = 0 (lane < 64 / R) end with their batch row's best
    argmax_steps<64 / R, 32>(best_v, best_i);
    if (lane < 64 / R && (lane & ((1 << LS) - 1)) == 0) { bv_s[wave][bb_l] = best_v; bi_s[wave][bb_l] = best_i; }
    __syncthreads();
    if (threadIdx.x < BT && b0 + (int)threadIdx.x < B) {
      const int bb = threadIdx.x;
      float v = bv_s[0][bb];
      int32_t i = bi_s[0][bb];
      for (int w8 = 1; w8 < 8; ++w8)
        if (bv_s[w8][bb] > v || (bv_s[w8][bb] == v && bi_s[w8][bb] < i)) { v = bv_s[w8][bb]; i = bi_s[w8][bb]; }
      part_val[(size_t)(b0 + bb) * gridDim.x + blockIdx.x] = v;
      part_idx[(size_t)(b0 + bb) * gridDim.x + blockIdx.x] = i;
    }
  }
}

template <int MODE>
constexpr int gemv_bt_rows() { return 2; }  // R BT <= 32 values per lane group

// inputs per block for a batch of B (>= 2) rows
static int gemv_bt_width(int B) { return B <= 2 ? 2 : (B <= 4 ? 4 : (B <= 8 ? 8 : 16)); }

int gemv_bt_grid(int N, int mode) {
  const int R = mode == MODE_LOGITS ? gemv_bt_rows<MODE_LOGITS>() : gemv_bt_rows<MODE_STORE>();
  const int ngroups = (N + R - 1) / R;
  const int nblk = (ngroups + 7) / 8;
  return nblk < 256 ? nblk : 256;  // one 8-wave block per CU; waves stride over the groups
}

// Inputs in LDS: BT x K / 8 16-byte units (up to 128 KB for 16 rows of
// K = 4096), more than the 64 KB a launch gets without opting in.
template <int P, int MODE, bool NORM, int BT>
static hipError_t gemv_bt_optin() {
  constexpr int R = gemv_bt_rows<MODE>();
  constexpr size_t lds_max = (size_t)BT * 64 * P * 16;
  if (lds_max <= 65536) return hipSuccess;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemv_bf16_bt<P, MODE, NORM, R, BT>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_max);
}

template <int P, int MODE, bool NORM, int BT>
static hipError_t launch_gemv_bt_pbt(const GemvArgs& a, hipStream_t st) {
  constexpr int R = gemv_bt_rows<MODE>();
  const size_t lds = (size_t)BT * (a.K / 8) * 16;
  hipLaunchKernelGGL((k_gemv_bf16_bt<P, MODE, NORM, R, BT>), dim3(a.nblk, 1, (a.B + BT - 1) / BT),
                     dim3(512), lds, st, a.W, a.bias, a.x, a.norm_w, a.eps, a.y, a.logits,
                     a.part_val, a.part_idx, a.N, a.K, a.B, rope_args(a));
  return hipSuccess;
}

template <int P, int MODE, bool NORM>
static hipError_t gemv_bt_optin_p() {
  hipError_t e = gemv_bt_optin<P, MODE, NORM, 2>();
  if (e == hipSuccess) e = gemv_bt_optin<P, MODE, NORM, 4>();
  if (e == hipSuccess) e = gemv_bt_optin<P, MODE, NORM, 8>();
  if (e == hipSuccess) e = gemv_bt_optin<P, MODE, NORM, 16>();
  return e;
}

template <int MODE, bool NORM>
static hipError_t gemv_bt_optin_m() {
  hipError_t e = gemv_bt_optin_p<1, MODE, NORM>();
  if (e == hipSuccess) e = gemv_bt_optin_p<2, MODE, NORM>();
  if (e == hipSuccess) e = gemv_bt_optin_p<3, MODE, NORM>();
  if (e == hipSuccess) e = gemv_bt_optin_p<4, MODE, NORM>();
  if (e == hipSuccess) e = gemv_bt_optin_p<6, MODE, NORM>();
  if (e == hipSuccess) e = gemv_bt_optin_p<8, MODE, NORM>();
  return e;
}

hipError_t gemv_batched_prepare() {
  hipError_t e = gemv_bt_optin_m<MODE_QKV, true>();
  if (e == hipSuccess) e = gemv_bt_optin_m<MODE_RESID, false>();
  if (e == hipSuccess) e = gemv_bt_optin_m<MODE_LOGITS, true>();
  return e;
}

template <int P, int MODE, bool NORM>
static hipError_t launch_gemv_bt_pn(const GemvArgs& a, hipStream_t st) {
  switch (gemv_bt_width(a.B)) {
    case 2: return launch_gemv_bt_pbt<P, MODE, NORM, 2>(a, st);
    case 4: return launch_gemv_bt_pbt<P, MODE, NORM, 4>(a, st);
    case 8: return launch_gemv_bt_pbt<P, MODE, NORM, 8>(a, st);
    default: return launch_gemv_bt_pbt<P, MODE, NORM, 16>(a, st);
  }
}

// The step's three batched projections: QKV and lm_head with the RMSNorm
// prologue, O without it.
template <int MODE, bool NORM>
static hipError_t launch_gemv_bt_m(const GemvArgs& a, hipStream_t st) {
  switch ((a.K / 8 + 63) / 64) {
    case 1: return launch_gemv_bt_pn<1, MODE, NORM>(a, st);
    case 2: return launch_gemv_bt_pn<2, MODE, NORM>(a, st);
    case 3: return launch_gemv_bt_pn<3, MODE, NORM>(a, st);
    case 4: return launch_gemv_bt_pn<4, MODE, NORM>(a, st);
    case 6: return launch_gemv_bt_pn<6, MODE, NORM>(a, st);
    case 8: return launch_gemv_bt_pn<8, MODE, NORM>(a, st);
    default: return hipErrorInvalidValue;
  }
}

bool gemv_batched_supported(const GemvArgs& a) {
  const int P = (a.K / 8 + 63) / 64;
  const bool p_ok = P == 1 || P == 2 || P == 3 || P == 4 || P == 6 || P == 8;
  const bool form_ok = (a.mode == MODE_QKV && a.norm_w != nullptr) ||
                       (a.mode == MODE_RESID && a.norm_w == nullptr) ||
                       (a.mode == MODE_LOGITS && a.norm_w != nullptr);
  return p_ok && form_ok && a.K % 8 == 0;
}

hipError_t launch_gemv_bf16_batched(const GemvArgs& a, hipStream_t st) {
  if (!gemv_batched_supported(a)) return hipErrorInvalidValue;
  switch (a.mode) {
    case MODE_QKV: return launch_gemv_bt_m<MODE_QKV, true>(a, st);
    case MODE_RESID: return launch_gemv_bt_m<MODE_RESID, false>(a, st);
    default: return launch_gemv_bt_m<MODE_LOGITS, true>(a, st);
  }
}

// ===========================================================================
// Final argmax over the lm_head partials; advances the sequence.
// grid B, block 256.  Greedy id = largest logit, ties to the lowest index.
// tokens[b][pos+1] receives it unless that slot still belongs to the prompt
// (teacher forcing); pos[b] += 1.  A free batch row (prompt_len < 0: a slot
// no sequence holds) is left as it is.
// ===========================================================================
__global__ __launch_bounds__(256) void k_argmax_advance(
    const float* __restrict__ part_val, const int32_t* __restrict__ part_idx,
    int nparts, int32_t* __restrict__ tokens, int tok_stride,
    int32_t* __restrict__ pos, const int32_t* __restrict__ prompt_len,
    int32_t* __restrict__ last_ids) {
  __shared__ float sv[4];
  __shared__ int32_t si[4];
  const int b = blockIdx.x;
  float v = -INFINITY;
  int32_t i = 0x7fffffff;
  for (int t = threadIdx.x; t < nparts; t += blockDim.x) {
    const float pv = part_val[(size_t)b * nparts + t];
    const int32_t pi = part_idx[(size_t)b * nparts + t];
    if (pv > v || (pv == v && pi < i)) { v = pv; i = pi; }
  }
  argmax_steps<1, 32>(v, i);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) { sv[wave] = v; si[wave] = i; }
  __syncthreads();
  if (threadIdx.x == 0) {
    v = sv[0];
    i = si[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
      if (sv[w] > v || (sv[w] == v && si[w] < i)) { v = sv[w]; i = si[w]; }
    if (i == 0x7fffffff) i = 0;
    const int p = pos[b], pl = prompt_len[b];
    if (pl >= 0) {
      if (p + 1 >= pl) tokens[(size_t)b * tok_stride + p + 1] = i;
      last_ids[b] = i;
      pos[b] = p + 1;
    }
  }
}

void launch_argmax_advance(const float* part_val, const int32_t* part_idx,
                           int nparts, int32_t* tokens, int tok_stride,
                           int32_t* pos, const int32_t* prompt_len,
                           int32_t* last_ids, int B, hipStream_t st) {
  hipLaunchKernelGGL(k_argmax_advance, dim3(B), dim3(256), 0, st, part_val,
                     part_idx, nparts, tokens, tok_stride, pos, prompt_len,
                     last_ids);
}

// ===========================================================================
// Sampling (temperature T > 0, nucleus top_p in (0, 1]) for one row per
// block of 1024 threads:
//   m = max_i l_i;  e_i = exp((l_i - m) / T);  Z = sum e_i
//   t = the largest fp32 value with  sum_{e_i >= t} e_i >= top_p Z
//       (a bit-by-bit search over the positive floats; t = 0 keeps all)
//   u = uniform [0, 1) from SplitMix64(seed, row, position)
//   id = the first vocab index where the running sum of kept e_i exceeds
//        u sum_{e_i >= t} e_i
// The e_i go to scratch [B][V] once; every sum is per thread over a fixed
// index set, then over the waves in order, so a draw is reproducible.
// With `advance` the block also writes the token and advances pos like the
// greedy argmax (teacher forcing inside the prompt).
// ===========================================================================
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// sum over the block (1024 threads) in wave order; every thread gets it
__device__ __forceinline__ float block_sum_1024(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();  // red is free
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int w = 0; w < 16; ++w) t = __fadd_rn(t, red[w]);
  return t;
}
__device__ __forceinline__ float block_max_1024(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < 16; ++w) t = fmaxf(t, red[w]);
  return t;
}

__global__ __launch_bounds__(1024) void k_sample(
    const float* __restrict__ logits, int V, float inv_temp, float top_p, uint64_t seed,
    int32_t* __restrict__ pos, float* __restrict__ scratch, int32_t* __restrict__ out_ids,
    int32_t* __restrict__ tokens, int tok_stride, const int32_t* __restrict__ prompt_len,
    int advance, int row0) {
  __shared__ float red[16];
  __shared__ float scan[1024];
  __shared__ int32_t pick;
  const int b = blockIdx.x, tid = threadIdx.x;
  const float* l = logits + (size_t)b * V;
  float* e = scratch + (size_t)b * V;
  const int p = pos[b];
  float m = -INFINITY;
  for (int i = tid; i < V; i += 1024) m = fmaxf(m, l[i]);
  m = block_max_1024(m, red);
  float z = 0.0f;
  for (int i = tid; i < V; i += 1024) {
    const float v = neon_expf(__fmul_rn(__fsub_rn(l[i], m), inv_temp));
    e[i] = v;
    z = __fadd_rn(z, v);
  }
  z = block_sum_1024(z, red);  // also orders the e[] stores before the reads below
  uint32_t t_bits = 0;          // threshold as positive-float bits (0: keep all)
  float kept = z;
  if (top_p < 1.0f) {
    const float goal = __fmul_rn(top_p, z);
    for (int bit = 30; bit >= 0; --bit) {
      const uint32_t cand = t_bits | (1u << bit);
      const float t = __builtin_bit_cast(float, cand);
      float s = 0.0f;
      for (int i = tid; i < V; i += 1024) {
        const float v = e[i];
        s = __fadd_rn(s, v >= t ? v : 0.0f);
      }
      s = block_sum_1024(s, red);
      if (s >= goal) { t_bits = cand; kept = s; }  // uniform: every thread has s
    }
  }
  const float t = __builtin_bit_cast(float, t_bits);
  // the RNG key is the batch row (row0 + b: a launch for one row of a batch
  // keys it like the batch step) and the position
  const uint64_t r = splitmix64(seed ^ splitmix64(((uint64_t)(uint32_t)(row0 + b) << 32) |
                                                  (uint32_t)p));
  const float u = (float)(r >> 40) * 0x1.0p-24f;
  const float target = __fmul_rn(u, kept);
  // running sums in vocab order: thread tid owns the contiguous slice
  // [tid C, tid C + C) of kept values; block prefix over the threads
  const int C = (V + 1023) / 1024;
  const int i0 = min(tid * C, V), i1 = min(i0 + C, V);
  float local = 0.0f;
  for (int i = i0; i < i1; ++i) { const float v = e[i]; local = __fadd_rn(local, v >= t ? v : 0.0f); }
  scan[tid] = local;
  if (tid == 0) pick = -1;
  __syncthreads();
  if (tid == 0) {  // exclusive prefix in thread order (one thread: a fixed order)
    float acc = 0.0f;
    for (int k2 = 0; k2 < 1024; ++k2) { const float x = scan[k2]; scan[k2] = acc; acc = __fadd_rn(acc, x); }
  }
  __syncthreads();
  {
    // the thread whose slice holds the target walks it; its own running sum
    // may round differently from the prefix, so it ends on its last kept
    // index if the walk does not cross the target
    float run = scan[tid];
    if (run <= target && local > 0.0f && __fadd_rn(run, local) > target) {
      int last = -1, found = -1;
      for (int i = i0; i < i1; ++i) {
        const float v = e[i];
        if (v >= t) {
          last = i;
          run = __fadd_rn(run, v);
          if (run > target) { found = i; break; }
        }
      }
      pick = found >= 0 ? found : last;
    }
  }
  __syncthreads();
  if (tid == 0) {
    int32_t id = pick;
    if (id < 0) {  // target at the very top (rounding): the last kept index
      for (int i = V - 1; i >= 0; --i) if (e[i] >= t) { id = i; break; }
      if (id < 0) id = 0;
    }
    if (!advance) {
      out_ids[b] = id;
    } else if (prompt_len[b] >= 0) {  // a free batch row is left as it is
      out_ids[b] = id;
      if (p + 1 >= prompt_len[b]) tokens[(size_t)b * tok_stride + p + 1] = id;
      pos[b] = p + 1;
    }
  }
}

void launch_sample(const float* logits, int B, int V, float temperature, float top_p,
                   uint64_t seed, int32_t* pos, float* scratch, int32_t* out_ids,
                   int32_t* tokens, int tok_stride, const int32_t* prompt_len, bool advance,
                   hipStream_t st, int row0) {
  hipLaunchKernelGGL(k_sample, dim3(B), dim3(1024), 0, st, logits, V, 1.0f / temperature,
                     top_p, seed, pos, scratch, out_ids, tokens, tok_stride, prompt_len,
                     advance ? 1 : 0, row0);
}

// ===========================================================================
// Embedding gather: h[b] = embed[tokens[b][pos[b]]]
// ===========================================================================
__global__ void k_embed(const int32_t* __restrict__ tokens, int tok_stride,
                        const int32_t* __restrict__ pos, const int32_t* __restrict__ seq,
                        const uint16_t* __restrict__ embed,
                        uint16_t* __restrict__ h, int H) {
  const int b = blockIdx.x;
  const int sq = seq != nullptr ? seq[b] : b;  // row b embeds token pos[b] of sequence sq
  const int32_t id = tokens[(size_t)sq * tok_stride + pos[b]];
  const uint4* src = reinterpret_cast<const uint4*>(embed + (size_t)id * H);
  uint4* dst = reinterpret_cast<uint4*>(h + (size_t)b * H);
  for (int i = threadIdx.x; i < H / 8; i += blockDim.x) dst[i] = src[i];
}

void launch_embed(const int32_t* tokens, int tok_stride, const int32_t* pos,
                  const int32_t* seq, const uint16_t* embed, uint16_t* h, int H, int B,
                  hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3(B), dim3(256), 0, st, tokens, tok_stride,
                     pos, seq, embed, h, H);
}

// ===========================================================================
// Standalone RMSNorm (canonical form of wave_load_x_bf16), one wave per row
// ===========================================================================
template <int P>
__global__ __launch_bounds__(64) void k_rmsnorm(const uint16_t* __restrict__ x,
                                                const uint16_t* __restrict__ w,
                                                uint16_t* __restrict__ out,
                                                int H, float eps) {
  const int b = blockIdx.x;
  float xr[P][8];
  wave_load_x_bf16<P>(xr, x + (size_t)b * H, w, eps, H, threadIdx.x,
                      out + (size_t)b * H);
}

void launch_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out, int B,
                    int H, float eps, hipStream_t st) {
  const int P = (H / 8 + 63) / 64;
  switch (P) {
#define N_CASE(PP)                                                             \
  case PP:                                                                     \
    hipLaunchKernelGGL(k_rmsnorm<PP>, dim3(B), dim3(64), 0, st, x, w, out, H,  \
                       eps);                                                   \
    break;
    N_CASE(1) N_CASE(2) N_CASE(3) N_CASE(4) N_CASE(5) N_CASE(6) N_CASE(7)
    N_CASE(8)
    default: N_CASE(16)
#undef N_CASE
  }
}

// The same normalised rows written in the matrix-core activation layout
// [ceil(B/16)][NCH][4][64][8] (NCH = ceil(H / 128)): the 8 elements 8 u ..
// 8 u + 7 of row r go to piece ((r / 16 * NCH + u / 16) * 4 + u % 16 / 4) * 64
// + r % 16 + 16 (u % 4), so that one 16 x 16 x 32 MFMA operand (16 rows x 32
// elements) is 1 KB contiguous.  Rows B .. 16 ceil(B/16) - 1 and units
// H / 8 .. 16 NCH - 1 are written as zeros (one wave per row of the padded
// tile).  Same arithmetic as k_rmsnorm.
template <int P>
__global__ __launch_bounds__(64) void k_rmsnorm_packed(const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ w,
                                                       uint16_t* __restrict__ out, int B, int H,
                                                       float eps) {
  const int r = blockIdx.x, lane = threadIdx.x;
  const int U = H / 8, NCH = (H + 127) / 128;
  uint4* o = reinterpret_cast<uint4*>(out);
  const size_t tile = (size_t)(r / 16) * NCH * 4 * 64;
  auto piece = [&](int u) { return tile + ((size_t)(u / 16) * 4 + (u % 16) / 4) * 64 + r % 16 + 16 * (u % 4); };
  if (r >= B) {  // padding row (uniform)
    for (int u = lane; u < 16 * NCH; u += 64) o[piece(u)] = make_uint4(0, 0, 0, 0);
    return;
  }
  XBf16Raw<P> raw;
  wave_x_bf16_issue<P, true>(raw, x + (size_t)r * H, w, H, lane);
  float xr[P][8];
  wave_x_bf16_finish<P, true>(xr, raw, eps, H, lane, nullptr);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = lane + 64 * p;
    if (u < U) {
      uint32_t q[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) q[j] = pack_bf2(xr[p][2 * j], xr[p][2 * j + 1]);
      o[piece(u)] = make_uint4(q[0], q[1], q[2], q[3]);
    }
  }
  for (int u = U + lane; u < 16 * NCH; u += 64) o[piece(u)] = make_uint4(0, 0, 0, 0);
}

void launch_rmsnorm_packed(const uint16_t* x, const uint16_t* w, uint16_t* out, int B, int H,
                           float eps, hipStream_t st) {
  const int P = (H / 8 + 63) / 64;
  const int rows = 16 * ((B + 15) / 16);
  switch (P) {
#define NP_CASE(PP)                                                                      \
  case PP:                                                                               \
    hipLaunchKernelGGL(k_rmsnorm_packed<PP>, dim3(rows), dim3(64), 0, st, x, w, out, B, \
                       H, eps);                                                          \
    break;
    NP_CASE(1) NP_CASE(2) NP_CASE(3) NP_CASE(4) NP_CASE(5) NP_CASE(6) NP_CASE(7)
    NP_CASE(8)
    default: NP_CASE(16)
#undef NP_CASE
  }
}

// The matrix-core steps' expert combine and the next RMSNorm in one launch:
// block r (256 threads) owns row r of the padded tile.  Wave w combines the
// row's units u = lane + 64 p for the passes p = w, w + 4, ... with
// k_mx_combine's arithmetic (y = fmaf chain over the KSL slots in order from
// 0, then h = bf16(h + bf16(y))), stores them to h and to LDS, and after the
// barrier wave 0 normalises the row from LDS with k_rmsnorm_packed's
// arithmetic (wave_x_bf16_finish) and writes its packed pieces.  Rows past B
// write the zero pieces only.  Every load is issued before any is used
// (units past the row re-read its last unit and are not stored).
template <int P, int KSL>
__global__ __launch_bounds__(256) void k_mx_combine_norm(const float* __restrict__ ybuf,
                                                         const float* __restrict__ score,
                                                         uint16_t* __restrict__ h,
                                                         const uint16_t* __restrict__ nw,
                                                         uint16_t* __restrict__ out, int B,
                                                         int H, float eps) {
  constexpr int PW = (P + 3) / 4;  // passes per wave
  __shared__ uint4 hs[64 * P];
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int U = H / 8, NCH = (H + 127) / 128;
  uint4* o = reinterpret_cast<uint4*>(out);
  const size_t tile = (size_t)(r / 16) * NCH * 4 * 64;
  auto piece = [&](int u) { return tile + ((size_t)(u / 16) * 4 + (u % 16) / 4) * 64 + r % 16 + 16 * (u % 4); };
  if (r >= B) {  // padding row (uniform)
    for (int u = tid; u < 16 * NCH; u += 256) o[piece(u)] = make_uint4(0, 0, 0, 0);
    return;
  }
  XBf16Raw<P> raw;
  const uint4* wv = reinterpret_cast<const uint4*>(nw);
#pragma unroll
  for (int p = 0; p < P; ++p) raw.w[p] = wv[min(lane + 64 * p, U - 1)];  // used by wave 0
  float sc[KSL];
#pragma unroll
  for (int s = 0; s < KSL; ++s) sc[s] = score[r * KSL + s];
  uint4* hrow = reinterpret_cast<uint4*>(h + (size_t)r * H);
  float4 yv[PW][KSL][2];
  uint4 hv[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int u = min(lane + 64 * min(w + 4 * i, P - 1), U - 1);
#pragma unroll
    for (int s = 0; s < KSL; ++s) {
      const float4* src = reinterpret_cast<const float4*>(ybuf + ((size_t)r * KSL + s) * H + 8 * u);
      yv[i][s][0] = src[0];
      yv[i][s][1] = src[1];
    }
    hv[i] = hrow[u];
  }
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int p = w + 4 * i, u = lane + 64 * p;
    float y[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < KSL; ++s) {
      const float e[8] = {yv[i][s][0].x, yv[i][s][0].y, yv[i][s][0].z, yv[i][s][0].w,
                          yv[i][s][1].x, yv[i][s][1].y, yv[i][s][1].z, yv[i][s][1].w};
#pragma unroll
      for (int q = 0; q < 8; ++q) y[q] = __builtin_fmaf(sc[s], e[q], y[q]);
    }
    const uint32_t cw[4] = {hv[i].x, hv[i].y, hv[i].z, hv[i].w};
    uint32_t ow[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float lo = __fadd_rn(bf2f((uint16_t)(cw[q] & 0xFFFFu)), bf2f(f2bf(y[2 * q])));
      const float hi = __fadd_rn(bf2f((uint16_t)(cw[q] >> 16)), bf2f(f2bf(y[2 * q + 1])));
      ow[q] = (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
    }
    if (p < P && u < U) {
      const uint4 nv = make_uint4(ow[0], ow[1], ow[2], ow[3]);
      hrow[u] = nv;
      hs[u] = nv;
    }
  }
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int p = 0; p < P; ++p) raw.x[p] = hs[min(lane + 64 * p, U - 1)];
  float xr[P][8];
  wave_x_bf16_finish<P, true>(xr, raw, eps, H, lane, nullptr);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = lane + 64 * p;
    if (u < U) {
      uint32_t q[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) q[j] = pack_bf2(xr[p][2 * j], xr[p][2 * j + 1]);
      o[piece(u)] = make_uint4(q[0], q[1], q[2], q[3]);
    }
  }
  for (int u = U + lane; u < 16 * NCH; u += 64) o[piece(u)] = make_uint4(0, 0, 0, 0);
}

bool launch_mx_combine_norm(const float* ybuf, const float* score, uint16_t* h,
                            const uint16_t* nw, uint16_t* out, int B, int H, int k, float eps,
                            hipStream_t st) {
  const int P = (H / 8 + 63) / 64;
  if (k != 4 || H % 8 != 0 || P > 8) return false;
  const dim3 grid(16 * ((B + 15) / 16));
  switch (P) {
#define CN_CASE(PP)                                                                          \
  case PP:                                                                                   \
    hipLaunchKernelGGL((k_mx_combine_norm<PP, 4>), grid, dim3(256), 0, st, ybuf, score, h, \
                       nw, out, B, H, eps);                                                  \
    break;
    CN_CASE(1) CN_CASE(2) CN_CASE(3) CN_CASE(4) CN_CASE(5) CN_CASE(6) CN_CASE(7)
    default: CN_CASE(8)
#undef CN_CASE
  }
  return true;
}

// ===========================================================================
// RoPE (HFM:215-222): half-split rotation with the host-built YaRN table
// (cos/sin [n_pos][D/2] fp32, HF modeling_rope_utils.py:429-483):
//   o1 = x1 c - x2 s,  o2 = x2 c + x1 s   (each product and sum rounded)
// ===========================================================================

// In-place RoPE on x [n_tok][n_heads][D] with per-token positions.
__global__ void k_rope_apply(uint16_t* __restrict__ x,
                             const int32_t* __restrict__ pos,
                             const float* __restrict__ cos_t,
                             const float* __restrict__ sin_t, int n_tok,
                             int n_heads, int D) {
  const int half = D / 2;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)n_tok * n_heads * half) return;
  const int f = (int)(i % half);
  const int64_t th = i / half;  // token * n_heads + head
  const int t = (int)(th / n_heads);
  const int p = pos[t];
  uint16_t* hx = x + th * D;
  float o1, o2;
  rope_pair(bf2f(hx[f]), bf2f(hx[f + half]), cos_t[(size_t)p * half + f],
            sin_t[(size_t)p * half + f], o1, o2);
  hx[f] = f2bf(o1);
  hx[f + half] = f2bf(o2);
}

void launch_rope_apply(uint16_t* x, const int32_t* pos, const float* cos_t,
                       const float* sin_t, int n_tok, int n_heads, int D,
                       hipStream_t st) {
  const int64_t n = (int64_t)n_tok * n_heads * (D / 2);
  hipLaunchKernelGGL(k_rope_apply, dim3((unsigned)((n + 255) / 256)), dim3(256),
                     0, st, x, pos, cos_t, sin_t, n_tok, n_heads, D);
}

// ===========================================================================
// Router (HFM:117-130).
// k_router_logits: grid (E, B), one wave per (expert, row) forms the row's
// (optionally RMS-normalised) input in registers and the expert's logit =
// canonical bf16 row dot + bias (fp32 add).  Wave (0, b) stores the
// normalised row to xn_out for the experts.
// wave_topk: one wave chooses a row's experts.  The router's total order is
// larger logit first, NaN after every number, ties (equal values, or both
// NaN) to the lower expert index.  Each logit maps to a 64-bit key that is
// larger exactly when the expert comes earlier (an order-preserving integer
// image of the float in the high half, NaN as 0, -0 as +0; the complement of
// the index in the low half); an expert's rank is the number of larger keys.
// The keys go to LDS and every lane counts over them with broadcast reads
// (at E <= 32 the two halves of the wave each count half of the keys).  The
// experts of rank t < k are the chosen ones, in rank order; their weights
// are e_t = exp(v_t - v_0) (neon_expf), s = sum in rank order, e_t / s.  Each
// MoE block runs it on the logits itself, so no block waits on another.
// ===========================================================================
constexpr int kMaxExperts = 256;
constexpr int kMaxTopK = 16;

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}


__device__ __forceinline__ float readlane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

__device__ __forceinline__ uint64_t route_key(float v, int i) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  u = (u == 0x80000000u) ? 0u : u;                         // -0 ranks as +0
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);          // order-preserving
  u = (v != v) ? 0u : u;                                   // NaN after numbers
  return ((uint64_t)u << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
}

// Chosen experts of one row, in the routing wave's LDS.
struct TopK {
  int32_t id[kMaxTopK];
  float sc[kMaxTopK];  // weights (when asked for), else the chosen logits
  uint64_t key[kMaxExperts];  // the row's route keys (ranking scratch)
};

// One wave; lg = the row's E logits (global).  On return t.id[0..k) (and,
// with WEIGHTS, t.sc[0..k)) are visible to the wave.
constexpr int kRouteQ = kMaxExperts / 64;  // logits per lane

// The row's logits, one per lane per 64 experts (unconditional, clamped
// loads; lanes past E are masked in wave_topk_rank).
__device__ __forceinline__ void wave_topk_issue(const float* __restrict__ lg, int E,
                                                int lane, float (&v)[kRouteQ]) {
#pragma unroll
  for (int q = 0; q < kRouteQ; ++q) v[q] = lg[min(lane + 64 * q, E - 1)];
}

template <bool WEIGHTS>
__device__ __forceinline__ void wave_topk_rank(const float (&vin)[kRouteQ], int E,
                                               int k, int lane, TopK& t) {
  constexpr int NQ = kRouteQ;
  float v[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int e = lane + 64 * q;
    v[q] = (e < E) ? vin[q] : 0.0f;
    if (e < E) t.key[e] = route_key(v[q], e);
  }
  wave_lds_sync();
  // rank = number of larger keys; keys are read back from LDS (broadcast
  // reads), so the loop is plain vector compares with no scalar round trips
  if (E <= 32) {
    // lanes l and l + 32 share expert l: each counts over half of the keys
    const int i = lane & 31, h = lane >> 5;
    const uint64_t ki = t.key[min(i, E - 1)];
    int r0 = 0, r1 = 0;
#pragma unroll
    for (int jj = 0; jj < 16; jj += 2) {
      const int j = 16 * h + jj;
      r0 += (j < E && t.key[min(j, E - 1)] > ki) ? 1 : 0;
      r1 += (j + 1 < E && t.key[min(j + 1, E - 1)] > ki) ? 1 : 0;
    }
    int r = r0 + r1;
    r += xor_lane_i<32>(r);
    if (lane < E && r < k) { t.id[r] = lane; t.sc[r] = v[0]; }
  } else {
    uint64_t ki[NQ];
    int rank[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      ki[q] = t.key[min(lane + 64 * q, E - 1)];
      rank[q] = 0;
    }
    for (int j = 0; j < E; ++j) {
      const uint64_t kj = t.key[j];
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        if (64 * q < E) rank[q] += kj > ki[q] ? 1 : 0;
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int e = lane + 64 * q;
      if (e < E && rank[q] < k) { t.id[rank[q]] = e; t.sc[rank[q]] = v[q]; }
    }
  }
  wave_lds_sync();
  if (WEIGHTS) {
    const float et = lane < k ? neon_expf(__fsub_rn(t.sc[lane], t.sc[0])) : 0.0f;
    float sum = 0.0f;
    for (int i = 0; i < k; ++i) sum = __fadd_rn(sum, readlane_f(et, i));
    wave_lds_sync();  // every lane has read t.sc before it is overwritten
    if (lane < k) t.sc[lane] = __fdiv_rn(et, sum);
    wave_lds_sync();
  }
}

template <bool WEIGHTS>
__device__ __forceinline__ void wave_topk(const float* __restrict__ lg, int E,
                                          int k, int lane, TopK& t) {
  float v[kRouteQ];
  wave_topk_issue(lg, E, lane, v);
  wave_topk_rank<WEIGHTS>(v, E, k, lane, t);
}

// Router logits, a wave per (expert e, row b).  With row_arrive given, the
// row's top-k finishes in the same launch (k_topk's ranking and weights): the
// wave stores its logit at agent scope (written through to the device's
// coherence point), waits for the store (vmcnt 0) and arrives on its row's
// counter (row_arrive[b kMoeSyncStride], its own 256-byte line) with an
// agent-scope fetch_add; the row's last wave reads the E logits with
// agent-scope loads, ranks them into idx / score and sets the counter back
// to 0 (0 at launch).
template <int P, bool NORM>
__global__ __launch_bounds__(64) void k_router_logits(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ nw, float eps,
    uint16_t* __restrict__ xn_out, const uint16_t* __restrict__ W,
    const uint16_t* __restrict__ bias, float* __restrict__ lg_out, int E,
    int H, int32_t* __restrict__ zero, int zero_n, uint8_t* __restrict__ xq_hi,
    uint8_t* __restrict__ xq_lo, uint8_t* __restrict__ xs_hi, uint8_t* __restrict__ xs_lo,
    int32_t* __restrict__ idx, float* __restrict__ score, int k, int32_t* row_arrive) {
  const int e = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  if (e == 0 && b == 0 && lane < zero_n) zero[(size_t)lane * kMoeSyncStride] = 0;
  const int U = H / 8;
  const uint16_t bias_e = bias[e];  // bias, x and norm loads first, then the row
  XBf16Raw<P> xraw;
  wave_x_bf16_issue<P, NORM>(xraw, x + (size_t)b * H, nw, H, lane);
  __builtin_amdgcn_sched_barrier(0);
  uint4 w[P];
  bf16_load_row<P>(w, W + (size_t)e * H, U, lane);
  __builtin_amdgcn_sched_barrier(0);
  float xr[P][8];
  wave_x_bf16_finish<P, NORM>(xr, xraw, eps, H, lane,
                              (xn_out != nullptr && e == 0) ? xn_out + (size_t)b * H
                                                            : nullptr);
  if (xq_hi != nullptr) {  // uniform: the MXFP8 image of the bf16 row
    // unit u = lane + 64 p holds elements 8 u .. 8 u + 7; four adjacent lanes
    // make one 32-block (U % 4 == 0, so a quad is valid or padding as a
    // whole); every wave holds the whole row, and wave e takes the passes
    // p = e (mod E)
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if (p % E != e) continue;  // uniform
      const int u = lane + 64 * p;
      uint32_t qh[2], ql[2], b1, b2;
      mx8_quant8(xr[p], qh, ql, b1, b2);
      if (u < U) {
        const size_t o = (size_t)b * H + 8 * (size_t)u;
        *reinterpret_cast<uint2*>(xq_hi + o) = make_uint2(qh[0], qh[1]);
        *reinterpret_cast<uint2*>(xq_lo + o) = make_uint2(ql[0], ql[1]);
        if ((u & 3) == 0) {
          xs_hi[(size_t)b * (H / 32) + u / 4] = (uint8_t)b1;
          xs_lo[(size_t)b * (H / 32) + u / 4] = (uint8_t)b2;
        }
      }
    }
  }
  const float acc = wave_sum(bf16_row_partial<P>(w, xr, U, lane));
  const float lv = __fadd_rn(acc, bf2f(bias_e));
  if (row_arrive == nullptr) {  // uniform
    if (lane == 0) lg_out[(size_t)b * E + e] = lv;
    return;
  }
  __shared__ TopK t;
  __shared__ int is_last;
  if (lane == 0) {
    __hip_atomic_store(lg_out + (size_t)b * E + e, lv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the logit has reached the coherence point
    is_last = __hip_atomic_fetch_add(row_arrive + (size_t)b * kMoeSyncStride, 1, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) == E - 1;
  }
  wave_lds_sync();
  if (!is_last) return;  // uniform
  float v[kRouteQ];
#pragma unroll
  for (int q = 0; q < kRouteQ; ++q)
    v[q] = __hip_atomic_load(lg_out + (size_t)b * E + min(lane + 64 * q, E - 1), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  wave_topk_rank<true>(v, E, k, lane, t);
  if (lane < k) { idx[b * k + lane] = t.id[lane]; score[b * k + lane] = t.sc[lane]; }
  if (lane == 0)
    __hip_atomic_store(row_arrive + (size_t)b * kMoeSyncStride, 0, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(64) void k_topk(const float* __restrict__ lg,
                                             int32_t* __restrict__ idx,
                                             float* __restrict__ score, int E,
                                             int k) {
  __shared__ TopK t;
  const int b = blockIdx.x, lane = threadIdx.x;
  wave_topk<true>(lg + (size_t)b * E, E, k, lane, t);
  if (lane < k) { idx[b * k + lane] = t.id[lane]; score[b * k + lane] = t.sc[lane]; }
}

// Top-k of every row (k_topk's ranking) and the matrix-core experts' route
// lists (mx_route_lists) in one launch: wave w of 16 ranks rows w, w + 16, ...
// Each pass requests the logits of the wave's next 4 rows together and then
// ranks them, so a batch of 64 waits for one load round trip instead of 4
// (13.4 us per launch at batch 64 before).
__global__ __launch_bounds__(1024) void k_topk_route(const float* __restrict__ lg, int B, int E,
                                                     int k, int32_t* __restrict__ idx,
                                                     float* __restrict__ score, int S,
                                                     int32_t* __restrict__ route) {
  __shared__ TopK t[16];
  __shared__ __align__(16) int32_t pair_e[256];
  __shared__ int cnt_e[256], slot_of[256], wave_used[4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int b0 = w; b0 < B; b0 += 64) {
    float v[4][kRouteQ];
#pragma unroll
    for (int i = 0; i < 4; ++i)  // rows past B re-read row B - 1 (never ranked)
      wave_topk_issue(lg + (size_t)min(b0 + 16 * i, B - 1) * E, E, lane, v[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = b0 + 16 * i;
      if (b >= B) break;  // uniform for the wave
      wave_topk_rank<true>(v[i], E, k, lane, t[w]);
      if (lane < k) {
        const int32_t id = t[w].id[lane];
        idx[b * k + lane] = id;
        score[b * k + lane] = t[w].sc[lane];
        pair_e[b * k + lane] = id;
      }
      wave_lds_sync();  // every lane has read t[w] before the next row's ranking writes it
    }
  }
  __syncthreads();
  mx_route_lists(pair_e, B * k, E, S, route, cnt_e, slot_of, wave_used);
}

// Router logits, top-k and the matrix-core route lists in one launch (B >= 2,
// no MXFP8 image): block b owns row b.  Its 8 waves each request their
// router rows (experts w, w + 8, w + 16, w + 24 of each 32) together with the
// input row, normalise the row (k_router_logits' wave_x_bf16 operations,
// wave 0 writing xn) and form the logits with k_router_logits' dot and bias
// add, so every logit has its bits (16 waves of two rows each, which waited
// for the normalised row before requesting their rows, ran B = 64 at 16,133
// against 16,200 tok/s); wave 0 then ranks the row (k_topk's ranking) from
// LDS.  With route NULL the block ends there: the expert kernels build
// their work items from the ids (mx_route_item).  Given a route table, the
// row's expert ids are stored at agent scope (written through to the
// device's coherence point), every wave waits for its stores (vmcnt 0), the
// block meets at a barrier, and one thread arrives on arrive[0] with an
// agent-scope fetch_add.  The block that arrives last reads every row's ids
// with agent-scope loads, builds the route lists (mx_route_lists) and sets
// arrive[0] back to 0 (it must be 0 at launch).  At the 20b shape, B = 64:
// 15.3 us per layer with the table against 5.1 + 12.0 us for
// k_router_logits + k_topk_route (14,764 against 14,615 tok/s).
constexpr int kRRWaves = 8;  // k_router_route: waves per block
template <int P>
__global__ __launch_bounds__(64 * kRRWaves) void k_router_route(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ nw, float eps,
    uint16_t* __restrict__ xn_out, const uint16_t* __restrict__ W,
    const uint16_t* __restrict__ bias, float* __restrict__ lg_out, int32_t* idx,
    float* score, int B, int E, int H, int k, int S, int32_t* __restrict__ route,
    int32_t* arrive, int32_t* __restrict__ zero, int zero_n) {
  __shared__ float lg_s[kMaxExperts];
  __shared__ TopK t;
  __shared__ __align__(16) int32_t pair_e[256];
  __shared__ int cnt_e[256], slot_of[256], wave_used[4];
  __shared__ int is_last;
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (b == 0 && tid < zero_n) zero[(size_t)tid * kMoeSyncStride] = 0;
  const int U = H / 8;
  XBf16Raw<P> xraw;
  wave_x_bf16_issue<P, true>(xraw, x + (size_t)b * H, nw, H, lane);
  // the wave's router rows (experts w + 8 q of each group of 32) go out
  // before the input row is normalised: they do not depend on it
  uint4 wr[4][P];
  uint16_t bvv[4];
  auto load_rows = [&](int e0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = min(e0 + kRRWaves * q, E - 1);
      bvv[q] = bias[e];
      bf16_load_row<P>(wr[q], W + (size_t)e * H, U, lane);
    }
  };
  load_rows(w);
  __builtin_amdgcn_sched_barrier(0);
  float xr[P][8];
  wave_x_bf16_finish<P, true>(xr, xraw, eps, H, lane,
                              (xn_out != nullptr && w == 0) ? xn_out + (size_t)b * H : nullptr);
  for (int e0 = w; e0 < E; e0 += 4 * kRRWaves) {  // uniform per wave
    if (e0 != w) load_rows(e0);
    float acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = wave_sum(bf16_row_partial<P>(wr[q], xr, U, lane));
    if (lane == 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = e0 + kRRWaves * q;
        if (e < E) {
          const float v = __fadd_rn(acc[q], bf2f(bvv[q]));
          lg_s[e] = v;
          lg_out[(size_t)b * E + e] = v;
        }
      }
    }
  }
  __syncthreads();
  if (w == 0) {
    float v[kRouteQ];
#pragma unroll
    for (int q = 0; q < kRouteQ; ++q) v[q] = lg_s[min(lane + 64 * q, E - 1)];
    wave_topk_rank<true>(v, E, k, lane, t);
    if (lane < k) {
      __hip_atomic_store(idx + (size_t)b * k + lane, t.id[lane], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      // (read by later launches only; agent scope like the ids, so that every
      // store before the arrival is written through)
      __hip_atomic_store(score + (size_t)b * k + lane, t.sc[lane], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    if (route != nullptr)
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ids have reached the coherence point
  }
  if (route == nullptr) return;  // (uniform) no table: the expert blocks read the ids
  __syncthreads();
  if (tid == 0)
    is_last = __hip_atomic_fetch_add(arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              B - 1;
  __syncthreads();
  if (!is_last) return;  // uniform
  const int nk = B * k;
  for (int q = tid; q < nk; q += 64 * kRRWaves)
    pair_e[q] = __hip_atomic_load(idx + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  mx_route_lists(pair_e, nk, E, S, route, cnt_e, slot_of, wave_used);
  if (tid == 0) __hip_atomic_store(arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

bool router_route_supported(const RouterArgs& a) {
  return a.B >= 2 && a.B * a.k <= 256 && a.E <= 256 && a.E <= kMaxExperts && a.k <= kMaxTopK &&
         a.norm_w != nullptr && a.xq_hi == nullptr && a.H % 8 == 0 &&
         (a.H / 8 + 63) / 64 <= 6 && a.arrive != nullptr;  // H <= 3072: no spills
}

void launch_router_route(const RouterArgs& a, int32_t* idx, float* score, int32_t* route,
                         hipStream_t st) {
  const int S = a.B * a.k < a.E ? a.B * a.k : a.E;
  const int P = (a.H / 8 + 63) / 64;
#define RR_CASE(PP)                                                                       \
  case PP:                                                                                \
    hipLaunchKernelGGL((k_router_route<PP>), dim3(a.B), dim3(64 * kRRWaves), 0, st, a.x,    \
                       a.norm_w, a.eps, a.xn_out, a.W, a.bias, a.lg_out, idx, score, a.B, \
                       a.E, a.H, a.k, S, route, a.arrive, a.zero, a.zero_n);             \
    break;
  switch (P) {
    RR_CASE(1) RR_CASE(2) RR_CASE(3) RR_CASE(4) RR_CASE(5)
    default: RR_CASE(6)
  }
#undef RR_CASE
}

void launch_topk_route(const float* lg, int32_t* idx, float* score, int B, int E, int k,
                       int32_t* route, hipStream_t st) {
  const int S = B * k < E ? B * k : E;
  hipLaunchKernelGGL(k_topk_route, dim3(1), dim3(1024), 0, st, lg, B, E, k, idx, score, S,
                     route);
}

void launch_topk(const float* lg, int32_t* idx, float* score, int B, int E, int k,
                 hipStream_t st) {
  hipLaunchKernelGGL(k_topk, dim3(B), dim3(64), 0, st, lg, idx, score, E, k);
}

void launch_router(const RouterArgs& a, hipStream_t st) {
  const int P = (a.H / 8 + 63) / 64;
  dim3 grid(a.E, a.B);
  // the top-k in the logits launch (row arrival) when counters are given
  int32_t* ra = (a.idx != nullptr && a.row_arrive != nullptr) ? a.row_arrive : nullptr;
  switch (P) {
#define R_CASE(PP)                                                               \
  case PP:                                                                       \
    if (a.norm_w != nullptr)                                                     \
      hipLaunchKernelGGL((k_router_logits<PP, true>), grid, dim3(64), 0, st, a.x, \
                         a.norm_w, a.eps, a.xn_out, a.W, a.bias, a.lg_out, a.E,  \
                         a.H, a.zero, a.zero_n, a.xq_hi, a.xq_lo, a.xs_hi,       \
                         a.xs_lo, a.idx, a.score, a.k, ra);                      \
    else                                                                         \
      hipLaunchKernelGGL((k_router_logits<PP, false>), grid, dim3(64), 0, st,    \
                         a.x, a.norm_w, a.eps, a.xn_out, a.W, a.bias, a.lg_out,  \
                         a.E, a.H, a.zero, a.zero_n, a.xq_hi, a.xq_lo, a.xs_hi,  \
                         a.xs_lo, a.idx, a.score, a.k, ra);                      \
    break;
    R_CASE(1) R_CASE(2) R_CASE(3) R_CASE(4) R_CASE(5) R_CASE(6) R_CASE(7)
    R_CASE(8)
    default: R_CASE(16)
#undef R_CASE
  }
  if (a.idx != nullptr && ra == nullptr)
    hipLaunchKernelGGL(k_topk, dim3(a.B), dim3(64), 0, st, a.lg_out, a.idx,
                       a.score, a.E, a.k);
}

// ===========================================================================
// O projection + residual, then the router logits, in one launch (batch 1).
// Blocks 0 .. nblk - 1 are k_gemv_bf16<P, MODE_RESID, false, 1>'s blocks,
// except that their residual stores are agent-scope (they complete at the
// device's coherence point) and each block then arrives on arr[0].  The
// ceil(E / 4) blocks after them are k_router_logits' waves, one expert each:
// every input that does not depend on h (bias, norm weights, router row) is
// loaded first, then wave 0 polls arr[0] until all nblk blocks have arrived,
// then h is read at agent scope and the logit formed with exactly
// k_router_logits' operations (same norm, same dot), so the bits match the
// two-launch form.  The O blocks never wait and the whole grid is far below
// the device's capacity, so the wait always ends; it is bounded anyway
// (kDevErrSyncTimeout).  The O blocks arrive on kMoeSyncWords shards (block i
// on shard i % kMoeSyncWords, each on its own 256-byte line: hundreds of
// atomics on one address queue behind each other), which the polling wave
// sums.  Each router block then counts itself on the word after the shards;
// the last one sets every word back to 0, ready for the next launch (they
// must be 0 at launch).
// ===========================================================================
__device__ __forceinline__ int wave_isum(int v) {
  v += xor_lane_i<32>(v);
  v += xor_lane_i<16>(v);
  v += xor_lane_i<8>(v);
  v += xor_lane_i<4>(v);
  v += xor_lane_i<2>(v);
  v += xor_lane_i<1>(v);
  return v;
}

template <int P, int PR>
__global__ __launch_bounds__(256) void k_gemv_o_router(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ bias,
    const uint16_t* __restrict__ x, uint16_t* y, int N, int K, int nblk,
    const uint16_t* __restrict__ nw, float eps, uint16_t* __restrict__ xn_out,
    const uint16_t* __restrict__ Wr, const uint16_t* __restrict__ br, float* __restrict__ lg_out,
    int E, int32_t* __restrict__ zero, int zero_n, int32_t* arr, int32_t* __restrict__ err,
    int spin_limit) {
  __shared__ int32_t wait_ok;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if ((int)blockIdx.x < nblk) {
    // ---- O + residual (k_gemv_bf16's block body, batch row 0) ----
    const int ngroups = N;  // one row per wave group
    const int gstride = nblk * 4;
    const int g0 = blockIdx.x * 4 + wave;
    const uint16_t bias_first = (bias != nullptr ? bias : W)[min(g0, N - 1)];
    float xr[P][8];
    XBf16Raw<P> xraw;
    wave_x_bf16_issue<P, false>(xraw, x, nullptr, K, lane);
    __builtin_amdgcn_sched_barrier(0);
    float best_v = -INFINITY;
    int32_t best_i = 0;
    RopeArgs rp{};
    if (g0 < ngroups) {
      gemv_bf16_group<P, MODE_RESID, false, true, 1, true>(g0, W, bias, bias_first, xr, xraw,
                                                           0.0f, y, nullptr, 0, N, K, lane,
                                                           best_v, best_i, rp, 0, 0);
      for (int g = g0 + gstride; g < ngroups; g += gstride)
        gemv_bf16_group<P, MODE_RESID, false, false, 1, true>(g, W, bias, 0, xr, xraw, 0.0f, y,
                                                              nullptr, 0, N, K, lane, best_v,
                                                              best_i, rp, 0, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's h stores have completed
    __syncthreads();
    if (threadIdx.x == 0)
      __hip_atomic_fetch_add(arr + (size_t)(blockIdx.x % kMoeSyncWords) * kMoeSyncStride, 1,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  // ---- router logits: expert e per wave ----
  const int e = ((int)blockIdx.x - nblk) * 4 + wave;
  const int ec = min(e, E - 1);
  if (e == 0 && lane < zero_n) zero[(size_t)lane * kMoeSyncStride] = 0;
  const int H = N, U = H / 8;
  const uint16_t bias_e = br[ec];
  XBf16Raw<PR> xraw;
  {
    const uint4* wv = reinterpret_cast<const uint4*>(nw);
#pragma unroll
    for (int p = 0; p < PR; ++p) xraw.w[p] = wv[min(lane + 64 * p, U - 1)];
  }
  uint4 w[PR];
  bf16_load_row<PR>(w, Wr + (size_t)ec * H, U, lane);
  int32_t* done_w = arr + (size_t)kMoeSyncWords * kMoeSyncStride;
  if (wave == 0) {
    const int32_t* mine = arr + (size_t)min(lane, kMoeSyncWords - 1) * kMoeSyncStride;
    bool ok = false;
    for (int it = 0; it < spin_limit; ++it) {
      const int v = __hip_atomic_load(mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (wave_isum(lane < kMoeSyncWords ? v : 0) >= nblk) {  // uniform
        ok = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) wait_ok = ok;
  }
  __syncthreads();
  int32_t done = 0;
  if (threadIdx.x == 0) {
    if (!wait_ok) flag_dev_err(err, kDevErrSyncTimeout);
    done = __hip_atomic_fetch_add(done_w, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int p = 0; p < PR; ++p) xraw.x[p] = load_agent16(y + 8 * (size_t)min(lane + 64 * p, U - 1));
  float xr[PR][8];
  wave_x_bf16_finish<PR, true>(xr, xraw, eps, H, lane, e == 0 ? xn_out : nullptr);
  const float acc = wave_sum(bf16_row_partial<PR>(w, xr, U, lane));
  if (e < E && lane == 0) lg_out[e] = __fadd_rn(acc, bf2f(bias_e));
  // every router block has seen all arrivals: ready for the next launch
  if (wave == 0 && __builtin_amdgcn_readfirstlane(done) == (int32_t)gridDim.x - nblk - 1 &&
      lane <= kMoeSyncWords)
    __hip_atomic_store(arr + (size_t)lane * kMoeSyncStride, 0, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

bool o_router_supported(const GemvArgs& o, const RouterArgs& r) {
  return o.B == 1 && r.B == 1 && o.mode == MODE_RESID && o.norm_w == nullptr &&
         r.norm_w != nullptr && r.idx == nullptr && r.xq_hi == nullptr && r.x == o.y &&
         r.H == o.N && o.N % 8 == 0 && o.K % 8 == 0 && r.E >= 1 && r.arrive != nullptr &&
         (o.K / 8 + 63) / 64 <= 8 && (r.H / 8 + 63) / 64 <= 8;
}

void launch_gemv_o_router(const GemvArgs& o, const RouterArgs& r, hipStream_t st) {
  const int P = (o.K / 8 + 63) / 64, PR = (r.H / 8 + 63) / 64;
  const int grid = o.nblk + (r.E + 3) / 4;
#define OR_LAUNCH(PP, QQ)                                                                 \
  hipLaunchKernelGGL((k_gemv_o_router<PP, QQ>), dim3(grid), dim3(256), 0, st, o.W, o.bias, \
                     o.x, o.y, o.N, o.K, o.nblk, r.norm_w, r.eps, r.xn_out, r.W, r.bias,  \
                     r.lg_out, r.E, r.zero, r.zero_n, r.arrive, r.err, kMoeSpinLimit)
#define OR_P(PP)                                       \
  switch (PR) {                                        \
    case 1: OR_LAUNCH(PP, 1); break;                   \
    case 2: OR_LAUNCH(PP, 2); break;                   \
    case 3: OR_LAUNCH(PP, 3); break;                   \
    case 4: OR_LAUNCH(PP, 4); break;                   \
    case 5: OR_LAUNCH(PP, 5); break;                   \
    case 6: OR_LAUNCH(PP, 6); break;                   \
    case 7: OR_LAUNCH(PP, 7); break;                   \
    default: OR_LAUNCH(PP, 8); break;                  \
  }
  switch (P) {
    case 1: OR_P(1); break;
    case 2: OR_P(2); break;
    case 3: OR_P(3); break;
    case 4: OR_P(4); break;
    case 5: OR_P(5); break;
    case 6: OR_P(6); break;
    case 7: OR_P(7); break;
    default: OR_P(8); break;
  }
#undef OR_P
#undef OR_LAUNCH
}

// Row b's experts into the wave's LDS slice t: chosen from the router logits
// when lg is given, else copied from idx (and score, when WEIGHTS).  The
// loads (moe_route_issue) are separate from the choice (moe_route_finish) so
// that a kernel issues them, and its activation loads, before anything waits.
// Both ways the ids/weights are then read from LDS.
// Logits (lg path), or the given id (bits) and weight in v[0], v[1] (idx
// path): one set of slots for both, so the compiler cannot merge the two
// paths' loads into a store through a pointer chosen at run time (which
// would put the struct in scratch memory).
struct RouteRaw {
  float v[kRouteQ];
};

template <bool WEIGHTS>
__device__ __forceinline__ void moe_route_issue(const float* __restrict__ lg,
                                                const int32_t* __restrict__ idx,
                                                const float* __restrict__ score,
                                                int b, int E, int k, int lane,
                                                RouteRaw& r) {
  if (lg != nullptr) {
    wave_topk_issue(lg + (size_t)b * E, E, lane, r.v);
  } else {
    const int t = min(lane, k - 1);
    r.v[0] = __builtin_bit_cast(float, idx[b * k + t]);
    if (WEIGHTS) r.v[1] = score[b * k + t];
  }
}

// Returns the expert of `slot`.
template <bool WEIGHTS>
__device__ __forceinline__ int moe_route_finish(const float* __restrict__ lg, int E,
                                                int k, int slot, int lane,
                                                const RouteRaw& r, TopK& t) {
  if (lg != nullptr) {
    wave_topk_rank<WEIGHTS>(r.v, E, k, lane, t);
  } else {
    if (lane < k) {
      t.id[lane] = __builtin_bit_cast(int32_t, r.v[0]);
      if (WEIGHTS) t.sc[lane] = r.v[1];
    }
    wave_lds_sync();
  }
  return t.id[slot];
}

template <bool WEIGHTS>
__device__ __forceinline__ int moe_expert(const float* __restrict__ lg,
                                          const int32_t* __restrict__ idx,
                                          const float* __restrict__ score, int b,
                                          int E, int k, int slot, int lane, TopK& t) {
  RouteRaw r;
  moe_route_issue<WEIGHTS>(lg, idx, score, b, E, k, lane, r);
  return moe_route_finish<WEIGHTS>(lg, E, k, slot, lane, r, t);
}

// ===========================================================================
// MoE expert FFN (HFM:82-112).
// gate_up + SwiGLU: grid (ceil(I / (4 jpw)), k, B), block 256.  Wave w of
// block i owns intermediate columns j in [(4i + w) jpw, +jpw); the gate row
// 2j and up row 2j+1 (interleaved, HFM:83) are computed together:
//   g = dot + bias, u = dot + bias (fp32 adds)
//   g = min(g, limit); u = clamp(u, -limit, limit)              (HFM:84-85)
//   act = bf16((u + 1) * (g * (1 / (1 + exp(-(g * alpha))))))  (HFM:86-87)
// each product, sum and quotient rounded separately (no contraction).
// ===========================================================================

// gate_up's expert for (b, slot); wave 0 of block (0, slot 0) also writes
// the row's chosen ids and weights to idx_out/score_out when given.
__device__ __forceinline__ int moe_gate_up_expert(
    const float* __restrict__ lg, const RouteRaw& rr, int32_t* __restrict__ idx_out,
    float* __restrict__ score_out, int b, int E, int k, int slot, int lane, int wave,
    TopK& t) {
  if (lg != nullptr && idx_out != nullptr && blockIdx.x == 0 && slot == 0 && wave == 0) {
    const int e = moe_route_finish<true>(lg, E, k, slot, lane, rr, t);
    if (lane < k) { idx_out[b * k + lane] = t.id[lane]; score_out[b * k + lane] = t.sc[lane]; }
    return e;
  }
  return moe_route_finish<false>(lg, E, k, slot, lane, rr, t);
}

// One routing per block: wave 0 chooses (into the block's t), the others
// wait at the barrier and read t.  Saves the other waves' top-k work, which
// would otherwise compete for the SIMDs with the expert math.
__device__ __forceinline__ void moe_gate_up_route_block(
    const float* __restrict__ lg, const RouteRaw& rr, int32_t* __restrict__ idx_out,
    float* __restrict__ score_out, int b, int E, int k, int slot, int lane, int wave,
    TopK& t) {
  if (wave == 0) (void)moe_gate_up_expert(lg, rr, idx_out, score_out, b, E, k, slot, lane, 0, t);
  __syncthreads();
}

constexpr int kMoeJpw = 4;  // gate_up: intermediate columns per wave
constexpr int kMoeRpw = 4;  // down: output rows per block

// Load order of both row kernels: routing inputs and the activation vector
// (neither depends on the expert), then the routing choice, then the bias and
// every weight row of the wave at once (unconditional, clamped addresses);
// the math then waits for one load at a time, in issue order.
template <int P, bool PAIR>
__global__ __launch_bounds__(256) void k_moe_gate_up(
    const uint8_t* __restrict__ gu_codes, const uint8_t* __restrict__ gu_scales,
    const uint16_t* __restrict__ gu_bias, const float* __restrict__ router_lg,
    const int32_t* __restrict__ idx, int32_t* __restrict__ idx_out,
    float* __restrict__ score_out, int E, const uint16_t* __restrict__ xn,
    uint16_t* __restrict__ act, int H, int I, int k, float alpha, float limit,
    int32_t* __restrict__ err) {
  __shared__ TopK tk;
  const int slot = blockIdx.y, b = blockIdx.z;
  const int U = H / 32, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  RouteRaw rr;
  if (wave == 0) moe_route_issue<false>(router_lg, idx, nullptr, b, E, k, lane, rr);
  uint4 xraw[P][4];
  if (PAIR) x_fp4_issue_pair<P>(xraw, xn + (size_t)b * H, U, lane);
  else x_fp4_issue<P>(xraw, xn + (size_t)b * H, U, lane);
  __builtin_amdgcn_sched_barrier(0);
  moe_gate_up_route_block(router_lg, rr, idx_out, score_out, b, E, k, slot, lane, wave, tk);
  const int e = tk.id[slot];
  if ((unsigned)e >= (unsigned)E) {  // a caller-given id out of range (uniform)
    if (threadIdx.x == 0 && blockIdx.x == 0) flag_dev_err(err, kDevErrExpertId);
    return;  // the down kernel drops this slot
  }
  const int j0 = (blockIdx.x * 4 + wave) * kMoeJpw;
  if (j0 >= I) return;
  const size_t rows = (size_t)2 * I;
  const uint8_t* codes = gu_codes + (size_t)e * rows * (H / 2);
  const uint8_t* scales = gu_scales + (size_t)e * rows * U;
  const uint16_t* bias = gu_bias + (size_t)e * rows;
  // lane 16 c (+8) will hold column j0 + c's gate (up) total
  const int jl = min(j0 + (lane >> 4), I - 1);
  const uint32_t bgu = load_pinned_u32(reinterpret_cast<const uint32_t*>(bias + 2 * jl));
  // gate row 2j and up row 2j+1 are adjacent (HFM:83); rows g0 u0 g1 u1 ...
  float a[2 * kMoeJpw];
  if constexpr (PAIR) {
    Fp4RowPair<P> rp[kMoeJpw];  // the (gate, up) rows of column j0 + c as a pair
#pragma unroll
    for (int c = 0; c < kMoeJpw; ++c) {
      const int row = 2 * min(j0 + c, I - 1);
      fp4_load_pair<P>(rp[c], codes + (size_t)row * (H / 2), scales + (size_t)row * U,
                       codes + (size_t)(row + 1) * (H / 2), scales + (size_t)(row + 1) * U,
                       U, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    float xr[P][32];
    x_fp4_finish_pair<P>(xr, xraw);
#pragma unroll
    for (int c = 0; c < kMoeJpw; ++c) fp4_pair_partials<P>(rp[c], xr, U, lane, a[2 * c], a[2 * c + 1]);
  } else {
    Fp4Row<P> rw[2 * kMoeJpw];
#pragma unroll
    for (int r = 0; r < 2 * kMoeJpw; ++r) {
      const int row = 2 * min(j0 + r / 2, I - 1) + (r & 1);
      fp4_load_row<P>(rw[r], codes + (size_t)row * (H / 2), scales + (size_t)row * U, U,
                      lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    float xr[P][32];
    x_fp4_finish<P>(xr, xraw, U, lane);
#pragma unroll
    for (int r = 0; r < 2 * kMoeJpw; ++r) a[r] = fp4_row_partial<P>(rw[r], xr, U, lane);
  }
  // lane l holds row l >> 3 (bit-identical to separate butterflies)
  const float t = wave_sum_8rows(a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7], lane);
  const float tu = xor_lane<8>(t);  // lane 16 c receives the up total
  const int j = j0 + (lane >> 4);
  if ((lane & 15) == 0 && j < I) {
    const float gb = __fadd_rn(t, bf_lo(bgu));
    const float ub = __fadd_rn(tu, bf_hi(bgu));
    act[((size_t)b * k + slot) * I + j] = f2bf(swiglu_clamp(gb, ub, alpha, limit));
  }
}

// down + weighted sum (+ residual): grid (ceil(H / kMoeRpw), B), block 64 k
// (wave s handles top-k slot s).  The k waves compute the same kMoeRpw rows
// for their experts; the block combines y = fmaf(score_s, dot_s + bias_s, y)
// in slot order from y = 0 (HFM:111-112), one rounding to bf16, then
// out = bf16(residual + y) when residual is given.
template <int P, bool PAIR>
__global__ __launch_bounds__(1024) void k_moe_down(
    const uint8_t* __restrict__ dn_codes, const uint8_t* __restrict__ dn_scales,
    const uint16_t* __restrict__ dn_bias, const float* __restrict__ router_lg,
    const int32_t* __restrict__ idx, const float* __restrict__ score, int E,
    const uint16_t* __restrict__ act, const uint16_t* residual, uint16_t* out,
    int H, int I, int k, int32_t* __restrict__ err) {
  __shared__ float red[kMaxTopK][kMoeRpw];
  __shared__ TopK tk;  // wave 0 routes for the block
  const int b = blockIdx.y;
  const int U = I / 32, lane = threadIdx.x & 63, slot = threadIdx.x >> 6;
  const int n0 = blockIdx.x * kMoeRpw;
  RouteRaw rr;
  if (slot == 0) moe_route_issue<true>(router_lg, idx, score, b, E, k, lane, rr);
  uint4 xraw[P][4];
  if (PAIR) x_fp4_issue_pair<P>(xraw, act + ((size_t)b * k + slot) * I, U, lane);
  else x_fp4_issue<P>(xraw, act + ((size_t)b * k + slot) * I, U, lane);
  // wave 0, lane t < kMoeRpw combines row n0 + t (out stands in for a
  // missing residual: same shape, read and ignored)
  const uint16_t res = load_pinned_u16((residual != nullptr ? residual : out) +
                                       (size_t)b * H + min(n0 + (lane & 3), H - 1));
  __builtin_amdgcn_sched_barrier(0);
  if (slot == 0) (void)moe_route_finish<true>(router_lg, E, k, 0, lane, rr, tk);
  __syncthreads();
  // a caller-given id out of range (uniform per wave): the slot reads expert
  // 0's rows (in bounds) and contributes 0
  const int e_raw = tk.id[slot];
  const bool e_ok = (unsigned)e_raw < (unsigned)E;
  const int e = e_ok ? e_raw : 0;
  if (!e_ok && lane == 0 && blockIdx.x == 0) flag_dev_err(err, kDevErrExpertId);
  const uint8_t* codes = dn_codes + (size_t)e * H * (I / 2);
  const uint8_t* scales = dn_scales + (size_t)e * H * U;
  const uint16_t* bias = dn_bias + (size_t)e * H;
  const uint16_t bl = load_pinned_u16(bias + min(n0 + (lane >> 4), H - 1));  // lane 16 r: row r
  float a[kMoeRpw];
  if constexpr (PAIR) {
    Fp4RowPair<P> rp[kMoeRpw / 2];
#pragma unroll
    for (int c = 0; c < kMoeRpw / 2; ++c) {
      const int na = min(n0 + 2 * c, H - 1), nb = min(n0 + 2 * c + 1, H - 1);
      fp4_load_pair<P>(rp[c], codes + (size_t)na * (I / 2), scales + (size_t)na * U,
                       codes + (size_t)nb * (I / 2), scales + (size_t)nb * U, U, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    float xr[P][32];
    x_fp4_finish_pair<P>(xr, xraw);
#pragma unroll
    for (int c = 0; c < kMoeRpw / 2; ++c) fp4_pair_partials<P>(rp[c], xr, U, lane, a[2 * c], a[2 * c + 1]);
  } else {
    Fp4Row<P> rw[kMoeRpw];
#pragma unroll
    for (int r = 0; r < kMoeRpw; ++r) {
      const int n = min(n0 + r, H - 1);
      fp4_load_row<P>(rw[r], codes + (size_t)n * (I / 2), scales + (size_t)n * U, U, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    float xr[P][32];
    x_fp4_finish<P>(xr, xraw, U, lane);
#pragma unroll
    for (int r = 0; r < kMoeRpw; ++r) a[r] = fp4_row_partial<P>(rw[r], xr, U, lane);
  }
  const float t = wave_sum_4rows(a[0], a[1], a[2], a[3], lane);
  if ((lane & 15) == 0) red[slot][lane >> 4] = e_ok ? __fadd_rn(t, bf2f(bl)) : 0.0f;
  __syncthreads();
  if (threadIdx.x < min(kMoeRpw, H - n0)) {
    const int r = threadIdx.x, n = n0 + r;
    float y = 0.0f;
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s)
      if (s < k) y = __builtin_fmaf(tk.sc[s], red[s][r], y);
    const uint16_t m = f2bf(y);
    const size_t o = (size_t)b * H + n;
    out[o] = residual ? f2bf(__fadd_rn(bf2f(res), bf2f(m))) : m;
  }
}

// ===========================================================================
// Batched experts (2 <= B, B k <= 64): rows that chose the same expert share
// one read of its weights.  idx / score [B][k] come from the top-k kernel.
// Pair q = b k + s is row b's slot s; lane q of a wave holds idx[q], and
// __ballot(idx == e) lists the pairs of expert e in row order.
//
// gate_up: grid (ceil(I / 16), min(E, B k)); block (x, u) serves the u-th
// used expert (ascending id) on intermediate columns 16 x .. 16 x + 15 for
// every pair that chose it.  down: grid ceil(H / 4); block serves output rows
// 4 x .. 4 x + 3 for every row b: each wave takes every fourth used expert,
// reads its 4 rows once and dots them with the act row of each pair that
// chose it; the block then combines row b's k slots in slot order (the same
// fmaf chain as the batch-1 kernel) and adds the residual.  Each (row, pair)
// dot is the canonical one of the batch-1 kernels, so the outputs are
// bit-identical to a batch-1 step.
// ===========================================================================
template <int P, bool PAIR>
__global__ __launch_bounds__(256) void k_moe_gate_up_bt(
    const uint8_t* __restrict__ gu_codes, const uint8_t* __restrict__ gu_scales,
    const uint16_t* __restrict__ gu_bias, const int32_t* __restrict__ idx, int E,
    const uint16_t* __restrict__ xn, uint16_t* __restrict__ act, int B, int H, int I,
    int k, float alpha, float limit) {
  const int U = H / 32, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nk = B * k;
  const int my_id = lane < nk ? idx[lane] : -1;
  // the u-th used expert and its pairs (uniform across the block)
  int e = -1;
  uint64_t pairs = 0;
  for (int ee = 0, cnt = 0; ee < E; ++ee) {
    const uint64_t bal = __ballot(my_id == ee);
    if (bal != 0) {
      if (cnt == (int)blockIdx.y) { e = ee; pairs = bal; break; }
      ++cnt;
    }
  }
  if (e < 0) return;  // fewer used experts than blocks in y
  const int j0 = (blockIdx.x * 4 + wave) * kMoeJpw;
  if (j0 >= I) return;
  const size_t rows = (size_t)2 * I;
  const uint8_t* codes = gu_codes + (size_t)e * rows * (H / 2);
  const uint8_t* scales = gu_scales + (size_t)e * rows * U;
  const uint16_t* bias = gu_bias + (size_t)e * rows;
  const int jl = min(j0 + (lane >> 4), I - 1);
  const uint32_t bgu = load_pinned_u32(reinterpret_cast<const uint32_t*>(bias + 2 * jl));
  // the wave's 8 rows, once for all pairs
  Fp4RowPair<P> rp[kMoeJpw];
  Fp4Row<P> rw[PAIR ? 1 : 2 * kMoeJpw];
  if constexpr (PAIR) {
#pragma unroll
    for (int c = 0; c < kMoeJpw; ++c) {
      const int row = 2 * min(j0 + c, I - 1);
      fp4_load_pair<P>(rp[c], codes + (size_t)row * (H / 2), scales + (size_t)row * U,
                       codes + (size_t)(row + 1) * (H / 2), scales + (size_t)(row + 1) * U,
                       U, lane);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 2 * kMoeJpw; ++r) {
      const int row = 2 * min(j0 + r / 2, I - 1) + (r & 1);
      fp4_load_row<P>(rw[r], codes + (size_t)row * (H / 2), scales + (size_t)row * U, U, lane);
    }
  }
  // pairs in row order; the next pair's input loads while this one is reduced
  int q = __builtin_ctzll(pairs);
  uint4 xraw[P][4];
  if (PAIR) x_fp4_issue_pair<P>(xraw, xn + (size_t)(q / k) * H, U, lane);
  else x_fp4_issue<P>(xraw, xn + (size_t)(q / k) * H, U, lane);
  while (true) {
    if constexpr (PAIR) {
#pragma unroll
      for (int c = 0; c < kMoeJpw; ++c) launder(rp[c]);
    } else {
#pragma unroll
      for (int r = 0; r < 2 * kMoeJpw; ++r) launder(rw[r]);
    }
    float xr[P][32];
    if (PAIR) x_fp4_finish_pair<P>(xr, xraw);
    else x_fp4_finish<P>(xr, xraw, U, lane);
    pairs &= pairs - 1;
    const int qn = pairs ? __builtin_ctzll(pairs) : q;
    if (pairs) {
      if (PAIR) x_fp4_issue_pair<P>(xraw, xn + (size_t)(qn / k) * H, U, lane);
      else x_fp4_issue<P>(xraw, xn + (size_t)(qn / k) * H, U, lane);
    }
    float a[2 * kMoeJpw];
    if constexpr (PAIR) {
#pragma unroll
      for (int c = 0; c < kMoeJpw; ++c) fp4_pair_partials<P>(rp[c], xr, U, lane, a[2 * c], a[2 * c + 1]);
    } else {
#pragma unroll
      for (int r = 0; r < 2 * kMoeJpw; ++r) a[r] = fp4_row_partial<P>(rw[r], xr, U, lane);
    }
    const float t = wave_sum_8rows(a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7], lane);
    const float tu = xor_lane<8>(t);  // lane 16 c receives the up total
    const int j = j0 + (lane >> 4);
    if ((lane & 15) == 0 && j < I) {
      const float gb = __fadd_rn(t, bf_lo(bgu));
      const float ub = __fadd_rn(tu, bf_hi(bgu));
      act[(size_t)q * I + j] = f2bf(swiglu_clamp(gb, ub, alpha, limit));
    }
    if (!pairs) break;
    q = qn;
  }
}

template <int P, bool PAIR>
__global__ __launch_bounds__(256) void k_moe_down_bt(
    const uint8_t* __restrict__ dn_codes, const uint8_t* __restrict__ dn_scales,
    const uint16_t* __restrict__ dn_bias, const int32_t* __restrict__ idx,
    const float* __restrict__ score, int E, const uint16_t* __restrict__ act,
    const uint16_t* residual, uint16_t* out, int B, int H, int I, int k,
    int32_t* __restrict__ err) {
  __shared__ float red[64][kMoeRpw];  // [pair][row]: dot + bias
  const int U = I / 32, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nk = B * k;
  const int n0 = blockIdx.x * kMoeRpw;
  const int my_id = lane < nk ? idx[lane] : -1;
  // a pair whose id lies outside [0, E) matches no expert and contributes 0
  for (int i = threadIdx.x; i < 64 * kMoeRpw; i += blockDim.x) (&red[0][0])[i] = 0.0f;
  if (blockIdx.x == 0 && wave == 0 &&
      __ballot(lane < nk && (unsigned)my_id >= (unsigned)E) != 0 && lane == 0)
    flag_dev_err(err, kDevErrExpertId);
  __syncthreads();
  // every fourth used expert, starting at this wave's index
  for (int ee = 0, cnt = 0; ee < E; ++ee) {
    const uint64_t bal = __ballot(my_id == ee);
    if (bal == 0) continue;
    if ((cnt++ & 3) != wave) continue;
    const uint8_t* codes = dn_codes + (size_t)ee * H * (I / 2);
    const uint8_t* scales = dn_scales + (size_t)ee * H * U;
    const uint16_t bl = load_pinned_u16(dn_bias + (size_t)ee * H + min(n0 + (lane >> 4), H - 1));
    Fp4RowPair<P> rp[kMoeRpw / 2];
    Fp4Row<P> rw[PAIR ? 1 : kMoeRpw];
    if constexpr (PAIR) {
#pragma unroll
      for (int c = 0; c < kMoeRpw / 2; ++c) {
        const int na = min(n0 + 2 * c, H - 1), nb = min(n0 + 2 * c + 1, H - 1);
        fp4_load_pair<P>(rp[c], codes + (size_t)na * (I / 2), scales + (size_t)na * U,
                         codes + (size_t)nb * (I / 2), scales + (size_t)nb * U, U, lane);
      }
    } else {
#pragma unroll
      for (int r = 0; r < kMoeRpw; ++r) {
        const int n = min(n0 + r, H - 1);
        fp4_load_row<P>(rw[r], codes + (size_t)n * (I / 2), scales + (size_t)n * U, U, lane);
      }
    }
    uint64_t pairs = bal;
    int q = __builtin_ctzll(pairs);
    uint4 xraw[P][4];
    if (PAIR) x_fp4_issue_pair<P>(xraw, act + (size_t)q * I, U, lane);
    else x_fp4_issue<P>(xraw, act + (size_t)q * I, U, lane);
    while (true) {
      if constexpr (PAIR) {
#pragma unroll
        for (int c = 0; c < kMoeRpw / 2; ++c) launder(rp[c]);
      } else {
#pragma unroll
        for (int r = 0; r < kMoeRpw; ++r) launder(rw[r]);
      }
      float xr[P][32];
      if (PAIR) x_fp4_finish_pair<P>(xr, xraw);
      else x_fp4_finish<P>(xr, xraw, U, lane);
      pairs &= pairs - 1;
      const int qn = pairs ? __builtin_ctzll(pairs) : q;
      if (pairs) {
        if (PAIR) x_fp4_issue_pair<P>(xraw, act + (size_t)qn * I, U, lane);
        else x_fp4_issue<P>(xraw, act + (size_t)qn * I, U, lane);
      }
      float a[kMoeRpw];
      if constexpr (PAIR) {
#pragma unroll
        for (int c = 0; c < kMoeRpw / 2; ++c) fp4_pair_partials<P>(rp[c], xr, U, lane, a[2 * c], a[2 * c + 1]);
      } else {
#pragma unroll
        for (int r = 0; r < kMoeRpw; ++r) a[r] = fp4_row_partial<P>(rw[r], xr, U, lane);
      }
      const float t = wave_sum_4rows(a[0], a[1], a[2], a[3], lane);
      if ((lane & 15) == 0) red[q][lane >> 4] = __fadd_rn(t, bf2f(bl));
      if (!pairs) break;
      q = qn;
    }
  }
  __syncthreads();
  // row b, output row n0 + r: y = fmaf(score_s, red_s, y) over the slots in order
  for (int t = threadIdx.x; t < B * kMoeRpw; t += blockDim.x) {
    const int b = t / kMoeRpw, r = t % kMoeRpw, n = n0 + r;
    if (n >= H) continue;
    float y = 0.0f;
    for (int s2 = 0; s2 < k; ++s2) y = __builtin_fmaf(score[b * k + s2], red[b * k + s2][r], y);
    const uint16_t m = f2bf(y);
    const size_t o = (size_t)b * H + n;
    out[o] = residual ? f2bf(__fadd_rn(bf2f(residual[o]), bf2f(m))) : m;
  }
}

// ===========================================================================
// The expert FFN of one row in ONE launch (batch 1): the work of k_moe_gate_up
// and k_moe_down with a grid-wide wait between them instead of a kernel
// boundary, so down's weight rows are already on their way while the last
// gate_up columns finish.  Every dot product is the batch-1 kernels' (same
// lane units and butterflies), so the output bits are the same.
//
//   1. each block routes (wave 0) and loads x once;
//   2. gate_up: wave task t = (slot, 4 intermediate columns), tasks dealt
//      round-robin over the grid's waves; the 4 act values of a task are
//      published with one 8-byte agent-scope store (it completes at the
//      device's coherence point, past this XCD's L2);
//   3. each wave waits for its stores (vmcnt 0), the block arrives on one of
//      kMoeSyncWords counters (agent-scope atomic add);
//   4. down: block task d = 4 output rows, wave = slot; the task's weight rows
//      are requested, then wave 0 polls the counters until all gridDim.x
//      blocks have arrived (a bounded spin: on time-out it flags
//      kDevErrSyncTimeout and goes on, so every wave exits), then act is read
//      with agent-scope loads and the slots are combined as in k_moe_down.
// The grid must be co-resident (the host caps it at the occupancy limit), so
// every block that others wait for is running.  The counters must be 0 at
// launch (the router kernel before it zeroes them).
// ===========================================================================
// How the down phase reads act after the grid-wide wait: false = agent-scope
// loads (each block fetches its own copy past the L2; measured 3.2 us after
// the wait at the 20b shape); true = one agent-scope acquire (L1/L2
// invalidate) per block, then plain loads that the XCD's L2 serves to all its
// blocks (measured 5.6 us: the invalidations cost more than they share).
#ifndef NEON_ACT_ACQUIRE
#define NEON_ACT_ACQUIRE 0
#endif
constexpr bool kActAcquire = NEON_ACT_ACQUIRE != 0;

// x_fp4_issue / x_fp4_issue_pair over agent-scope loads
template <int P, bool PAIR>
__device__ __forceinline__ void x_fp4_issue_agent(uint4 (&raw)[P][4],
                                                  const uint16_t* __restrict__ x, int U,
                                                  int lane) {
  const int r = U - 64 * (P - 1);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    int u;
    if (PAIR) u = p < P - 1 ? lane + 64 * p : 64 * (P - 1) + min(lane >= r ? lane - r : lane, r - 1);
    else u = min(lane + 64 * p, U - 1);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      raw[p][q] = kActAcquire ? reinterpret_cast<const uint4*>(x)[u * 4 + q]
                              : load_agent16(x + (size_t)(u * 4 + q) * 8);
  }
}

// Grid-wide wait of the one-launch kernels.  Layout of the sync words (all
// zero at launch): arrival shard s at ctr[s * kMoeSyncStride], s <
// kMoeSyncWords, then go flag copy c at ctr[(kMoeSyncWords + c) *
// kMoeSyncStride], c < kMoeGoCopies, each word on its own 256-byte line, so
// the arrivals and the polls do not queue on one line.
//
// Block 0's wave 0 is the aggregator: it polls the shards until they add up
// to `target` and then sets every go copy; every other block's wave 0 polls
// one go copy, with a back-off (its polls compete with the weight streams).
// Both loops are bounded (spin_limit polls); false on time-out.
__device__ __forceinline__ bool wave_wait_grid(int32_t* ctr, int target, int spin_limit,
                                               int lane) {
  if (blockIdx.x == 0) {
    const int32_t* mine = ctr + (size_t)min(lane, kMoeSyncWords - 1) * kMoeSyncStride;
    for (int it = 0; it < spin_limit; ++it) {
      const int v = __hip_atomic_load(mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (wave_isum(lane < kMoeSyncWords ? v : 0) >= target) {  // uniform
        if (lane < kMoeGoCopies)
          __hip_atomic_store(ctr + (size_t)(kMoeSyncWords + lane) * kMoeSyncStride, 1,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return true;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    return false;
  }
  const int32_t* go = ctr + (size_t)(kMoeSyncWords + blockIdx.x % kMoeGoCopies) * kMoeSyncStride;
  for (int it = 0; it < spin_limit; ++it) {
    if (__hip_atomic_load(go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) return true;
    __builtin_amdgcn_s_sleep(8);
  }
  return false;
}

template <int P, bool PAIR>
__global__ __launch_bounds__(256) void k_moe_fused(
    const uint8_t* __restrict__ gu_codes, const uint8_t* __restrict__ gu_scales,
    const uint16_t* __restrict__ gu_bias, const uint8_t* __restrict__ dn_codes,
    const uint8_t* __restrict__ dn_scales, const uint16_t* __restrict__ dn_bias,
    const float* __restrict__ router_lg, const int32_t* __restrict__ idx,
    const float* __restrict__ score, int32_t* __restrict__ idx_out,
    float* __restrict__ score_out, int E, const uint16_t* __restrict__ xn, uint16_t* act,
    const uint16_t* residual, uint16_t* out, int H, int I, int k, float alpha, float limit,
    int32_t* __restrict__ err, int32_t* sync, int spin_limit) {
  __shared__ TopK tk;
  __shared__ float red[kMaxTopK][kMoeRpw];
  // x in fp32, unit u's 32 elements at xs[u * 33 ..]: the lanes of a wave read
  // 64 different units at one element, 33 floats apart (all 64 banks)
  __shared__ float xs[kMoeFusedMaxUnits * 33];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int Ug = H / 32, Ud = I / 32;
  // ---- routing (wave 0, with weights) and x, loaded once ----
  RouteRaw rr;
  if (wave == 0) moe_route_issue<true>(router_lg, idx, score, 0, E, k, lane, rr);
  for (int i = threadIdx.x; i < H / 8; i += 256) {  // 8 elements per thread and step
    const uint4 v = reinterpret_cast<const uint4*>(xn)[i];
    float f[8];
    unpack8(v, f);
    const int u = i >> 2, e0 = (i & 3) * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) xs[u * 33 + e0 + j] = f[j];
  }
  __builtin_amdgcn_sched_barrier(0);
  if (wave == 0) {
    (void)moe_route_finish<true>(router_lg, E, k, 0, lane, rr, tk);
    if (blockIdx.x == 0 && idx_out != nullptr && lane < k) {
      idx_out[lane] = tk.id[lane];
      score_out[lane] = tk.sc[lane];
    }
  }
  __syncthreads();
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    bool bad = false;
    for (int s = 0; s < k; ++s) bad |= (unsigned)tk.id[s] >= (unsigned)E;
    if (bad) flag_dev_err(err, kDevErrExpertId);
  }
  // ---- gate_up + SwiGLU, 4 columns per wave task ----
  const int tiles = I / kMoeJpw;  // I % 4 == 0 (host-checked)
  const size_t rows = (size_t)2 * I;
  for (int t = blockIdx.x * 4 + wave; t < k * tiles; t += gridDim.x * 4) {
    const int slot = t / tiles, j0 = (t % tiles) * kMoeJpw;
    const int e = tk.id[slot];
    if ((unsigned)e >= (unsigned)E) continue;  // dropped slot (uniform)
    const uint8_t* codes = gu_codes + (size_t)e * rows * (H / 2);
    const uint8_t* scales = gu_scales + (size_t)e * rows * Ug;
    const uint16_t* bias = gu_bias + (size_t)e * rows;
    const uint32_t bgu =
        load_pinned_u32(reinterpret_cast<const uint32_t*>(bias + 2 * (j0 + (lane >> 4))));
    float a[2 * kMoeJpw];
    if constexpr (PAIR) {
      Fp4RowPair<P> rp[kMoeJpw];
#pragma unroll
      for (int c = 0; c < kMoeJpw; ++c) {
        const int row = 2 * (j0 + c);
        fp4_load_pair<P>(rp[c], codes + (size_t)row * (H / 2), scales + (size_t)row * Ug,
                         codes + (size_t)(row + 1) * (H / 2), scales + (size_t)(row + 1) * Ug,
                         Ug, lane);
      }
      // every row load issued before any use (else the scheduler waits for
      // the first pass's loads before it issues the rest: one memory round
      // trip per pass)
      __builtin_amdgcn_sched_barrier(0);
      // the rows' lane partials pass by pass (the same per-row order as
      // fp4_pair_partials), x of each pass read from LDS when it is needed
      const int r_tail = Ug - 64 * (P - 1);
#pragma unroll
      for (int c = 0; c < kMoeJpw; ++c) { a[2 * c] = 0.0f; a[2 * c + 1] = 0.0f; }
#pragma unroll
      for (int p = 0; p < P - 1; ++p) {
        float xp[32];
        const float* src = xs + (lane + 64 * p) * 33;
#pragma unroll
        for (int j = 0; j < 32; ++j) xp[j] = src[j];
#pragma unroll
        for (int c = 0; c < kMoeJpw; ++c) {
          a[2 * c] = __fadd_rn(a[2 * c], e8m0_scale(fp4_unit_dot(rp[c].c[0][p], xp), rp[c].s[0][p]));
          a[2 * c + 1] =
              __fadd_rn(a[2 * c + 1], e8m0_scale(fp4_unit_dot(rp[c].c[1][p], xp), rp[c].s[1][p]));
        }
      }
      {
        float xp[32];
        const int ut = 64 * (P - 1) + min(lane >= r_tail ? lane - r_tail : lane, r_tail - 1);
        const float* src = xs + ut * 33;
#pragma unroll
        for (int j = 0; j < 32; ++j) xp[j] = src[j];
#pragma unroll
        for (int c = 0; c < kMoeJpw; ++c) {
          const float tt = e8m0_scale(fp4_unit_dot(rp[c].tc, xp), rp[c].ts);
          const float tb = __shfl(tt, min(lane + r_tail, 63), 64);  // row B's tail
          const float a2 = __fadd_rn(a[2 * c], tt), b2 = __fadd_rn(a[2 * c + 1], tb);
          a[2 * c] = lane < r_tail ? a2 : a[2 * c];
          a[2 * c + 1] = lane < r_tail ? b2 : a[2 * c + 1];
        }
      }
    } else {
      Fp4Row<P> rw[2 * kMoeJpw];
#pragma unroll
      for (int r = 0; r < 2 * kMoeJpw; ++r) {
        const int row = 2 * (j0 + r / 2) + (r & 1);
        fp4_load_row<P>(rw[r], codes + (size_t)row * (H / 2), scales + (size_t)row * Ug, Ug, lane);
      }
      __builtin_amdgcn_sched_barrier(0);  // every row load issued before any use
#pragma unroll
      for (int r = 0; r < 2 * kMoeJpw; ++r) a[r] = 0.0f;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        float xp[32];
        const bool on = lane + 64 * p < Ug;
        const float* src = xs + min(lane + 64 * p, Ug - 1) * 33;
#pragma unroll
        for (int j = 0; j < 32; ++j) xp[j] = src[j];
#pragma unroll
        for (int r = 0; r < 2 * kMoeJpw; ++r) {
          const float t2 = __fadd_rn(a[r], e8m0_scale(fp4_unit_dot(rw[r].c[p], xp), rw[r].s[p]));
          a[r] = on ? t2 : a[r];  // padded units leave the partial untouched
        }
      }
    }
    const float tg = wave_sum_8rows(a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7], lane);
    const float tu = xor_lane<8>(tg);  // lane 16 c: column j0 + c's (gate, up) totals
    const float gb = __fadd_rn(tg, bf_lo(bgu));
    const float ub = __fadd_rn(tu, bf_hi(bgu));
    const uint32_t v = f2bf(swiglu_clamp(gb, ub, alpha, limit));
    const uint64_t packed = (uint64_t)__builtin_amdgcn_readlane(v, 0) |
                            ((uint64_t)__builtin_amdgcn_readlane(v, 16) << 16) |
                            ((uint64_t)__builtin_amdgcn_readlane(v, 32) << 32) |
                            ((uint64_t)__builtin_amdgcn_readlane(v, 48) << 48);
    if (lane == 0)
      __hip_atomic_store(reinterpret_cast<uint64_t*>(act + (size_t)slot * I + j0), packed,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // ---- arrive: this block's act stores have completed ----
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(sync + (size_t)(blockIdx.x % kMoeSyncWords) * kMoeSyncStride, 1,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // ---- down + weighted sum (+ residual), 4 output rows per block task ----
  const int slot = wave;
  const int slot_c = min(slot, k - 1);
  int e = tk.id[slot_c];
  const bool e_ok = slot < k && (unsigned)e < (unsigned)E;
  if (!e_ok) e = 0;  // expert 0's rows are read (in bounds) and dropped
  const uint8_t* dcodes = dn_codes + (size_t)e * H * (I / 2);
  const uint8_t* dscales = dn_scales + (size_t)e * H * Ud;
  const uint16_t* dbias = dn_bias + (size_t)e * H;
  // act of this wave's slot, kept as bf16 and unpacked one pass at a time
  uint4 araw[P][4];
  bool waited = false;
  for (int d = blockIdx.x; d * kMoeRpw < H; d += gridDim.x) {
    const int n0 = d * kMoeRpw;
    const uint16_t res = load_pinned_u16((residual != nullptr ? residual : out) +
                                         min(n0 + (lane & 3), H - 1));
    const uint16_t bl = load_pinned_u16(dbias + min(n0 + (lane >> 4), H - 1));
    float a[kMoeRpw];
    if constexpr (PAIR) {
      Fp4RowPair<P> rp[kMoeRpw / 2];
#pragma unroll
      for (int c = 0; c < kMoeRpw / 2; ++c) {
        const int na = min(n0 + 2 * c, H - 1), nb = min(n0 + 2 * c + 1, H - 1);
        fp4_load_pair<P>(rp[c], dcodes + (size_t)na * (I / 2), dscales + (size_t)na * Ud,
                         dcodes + (size_t)nb * (I / 2), dscales + (size_t)nb * Ud, Ud, lane);
      }
      __builtin_amdgcn_sched_barrier(0);  // every row load issued before the wait or any use
      if (!waited) {  // the first task's rows are in flight during the wait
        bool ok = true;
        if (wave == 0) ok = wave_wait_grid(sync, gridDim.x, spin_limit, lane);
        if (!ok && lane == 0) flag_dev_err(err, kDevErrSyncTimeout);
        // acquire: act lines cached in this CU's L1 or XCD's L2 are dropped
        if (kActAcquire && wave == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        __syncthreads();
        x_fp4_issue_agent<P, true>(araw, act + (size_t)slot_c * I, Ud, lane);
        waited = true;
      }
      // fp4_pair_partials, pass by pass (same per-row order)
      const int r_tail = Ud - 64 * (P - 1);
#pragma unroll
      for (int c = 0; c < kMoeRpw / 2; ++c) { a[2 * c] = 0.0f; a[2 * c + 1] = 0.0f; }
#pragma unroll
      for (int p = 0; p < P - 1; ++p) {
        float xp[32];
#pragma unroll
        for (int q = 0; q < 4; ++q) unpack8(araw[p][q], &xp[8 * q]);
#pragma unroll
        for (int c = 0; c < kMoeRpw / 2; ++c) {
          a[2 * c] = __fadd_rn(a[2 * c], e8m0_scale(fp4_unit_dot(rp[c].c[0][p], xp), rp[c].s[0][p]));
          a[2 * c + 1] =
              __fadd_rn(a[2 * c + 1], e8m0_scale(fp4_unit_dot(rp[c].c[1][p], xp), rp[c].s[1][p]));
        }
      }
      {
        float xp[32];
#pragma unroll
        for (int q = 0; q < 4; ++q) unpack8(araw[P - 1][q], &xp[8 * q]);
#pragma unroll
        for (int c = 0; c < kMoeRpw / 2; ++c) {
          const float tt = e8m0_scale(fp4_unit_dot(rp[c].tc, xp), rp[c].ts);
          const float tb = __shfl(tt, min(lane + r_tail, 63), 64);  // row B's tail
          const float a2 = __fadd_rn(a[2 * c], tt), b2 = __fadd_rn(a[2 * c + 1], tb);
          a[2 * c] = lane < r_tail ? a2 : a[2 * c];
          a[2 * c + 1] = lane < r_tail ? b2 : a[2 * c + 1];
        }
      }
    } else {
      Fp4Row<P> rw[kMoeRpw];
#pragma unroll
      for (int r = 0; r < kMoeRpw; ++r) {
        const int n = min(n0 + r, H - 1);
        fp4_load_row<P>(rw[r], dcodes + (size_t)n * (I / 2), dscales + (size_t)n * Ud, Ud, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (!waited) {
        bool ok = true;
        if (wave == 0) ok = wave_wait_grid(sync, gridDim.x, spin_limit, lane);
        if (!ok && lane == 0) flag_dev_err(err, kDevErrSyncTimeout);
        // acquire: act lines cached in this CU's L1 or XCD's L2 are dropped
        if (kActAcquire && wave == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        __syncthreads();
        x_fp4_issue_agent<P, false>(araw, act + (size_t)slot_c * I, Ud, lane);
        waited = true;
      }
#pragma unroll
      for (int r = 0; r < kMoeRpw; ++r) a[r] = 0.0f;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        float xp[32];
        const bool on = lane + 64 * p < Ud;
#pragma unroll
        for (int q = 0; q < 4; ++q) unpack8(araw[p][q], &xp[8 * q]);
#pragma unroll
        for (int r = 0; r < kMoeRpw; ++r) {
          const float t2 = __fadd_rn(a[r], e8m0_scale(fp4_unit_dot(rw[r].c[p], xp), rw[r].s[p]));
          a[r] = on ? t2 : a[r];  // padded units leave the partial untouched
        }
      }
    }
    const float t = wave_sum_4rows(a[0], a[1], a[2], a[3], lane);
    if ((lane & 15) == 0) red[slot][lane >> 4] = e_ok ? __fadd_rn(t, bf2f(bl)) : 0.0f;
    __syncthreads();
    if (threadIdx.x < min(kMoeRpw, H - n0)) {
      const int r = threadIdx.x, n = n0 + r;
      float y = 0.0f;
#pragma unroll
      for (int s = 0; s < kMaxTopK; ++s)
        if (s < k) y = __builtin_fmaf(tk.sc[s], red[s][r], y);
      const uint16_t m = f2bf(y);
      out[n] = residual ? f2bf(__fadd_rn(bf2f(res), bf2f(m))) : m;
    }
    __syncthreads();  // red is reused by the next task
  }
}

bool moe_fused_supported(const MoeArgs& a) {
  return a.sync != nullptr && a.B == 1 && a.k >= 1 && a.k <= 4 && a.I % kMoeJpw == 0 &&
         a.H / 32 <= kMoeFusedMaxUnits &&
         (a.router_lg != nullptr || (a.idx != nullptr && a.score != nullptr));
}

template <int P, bool PR>
static int moe_fused_capacity() {
  static int cap = -1;
  if (cap < 0) {
    int per_cu = 0, dev = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_moe_fused<P, PR>, 256, 0) !=
            hipSuccess ||
        hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      per_cu = cus = 0;
    cap = per_cu * cus;
  }
  return cap;
}

// Returns false (nothing launched) when the grid could not be co-resident.
template <int P, bool PR>
static bool launch_moe_fused_p(const MoeArgs& a, hipStream_t st) {
  const int n_dn = (a.H + kMoeRpw - 1) / kMoeRpw;
  const int cap = moe_fused_capacity<P, PR>();
  const int grid = min(n_dn, cap);
  if (grid < 1) return false;
  hipLaunchKernelGGL((k_moe_fused<P, PR>), dim3(grid), dim3(256), 0, st, a.gu_codes,
                     a.gu_scales, a.gu_bias, a.dn_codes, a.dn_scales, a.dn_bias, a.router_lg,
                     a.idx, a.score, a.idx_out, a.score_out, a.E, a.xn, a.act, a.residual, a.out,
                     a.H, a.I, a.k, a.alpha, a.limit, a.err, a.sync, kMoeSpinLimit);
  return true;
}

bool launch_moe_fused(const MoeArgs& a, hipStream_t st) {
  const int Pg = (a.H / 32 + 63) / 64, Pd = (a.I / 32 + 63) / 64;
  if (Pg != Pd) return false;  // one P for both halves
  const bool pr = fp4_pair_ok(a.H / 32, Pg) && fp4_pair_ok(a.I / 32, Pd);
  switch (Pg) {
    case 1: return launch_moe_fused_p<1, false>(a, st);
    case 2: return pr ? launch_moe_fused_p<2, true>(a, st) : launch_moe_fused_p<2, false>(a, st);
    case 3: return pr ? launch_moe_fused_p<3, true>(a, st) : launch_moe_fused_p<3, false>(a, st);
    default: return false;
  }
}

bool moe_batched_supported(const MoeArgs& a) {
  return a.B >= 2 && a.B * a.k <= 64 && a.idx != nullptr && a.score != nullptr &&
         a.router_lg == nullptr && a.k <= kMaxTopK;
}

void launch_moe_batched(const MoeArgs& a, hipStream_t st) {
  const int Pg = (a.H / 32 + 63) / 64, Pd = (a.I / 32 + 63) / 64;
  const int gblk = (a.I + 4 * kMoeJpw - 1) / (4 * kMoeJpw);
  const int dblk = (a.H + kMoeRpw - 1) / kMoeRpw;
  const int used_max = a.E < a.B * a.k ? a.E : a.B * a.k;
  const bool pg = fp4_pair_ok(a.H / 32, Pg), pd = fp4_pair_ok(a.I / 32, Pd);
#define GB_LAUNCH(PP, PR)                                                                    \
  hipLaunchKernelGGL((k_moe_gate_up_bt<PP, PR>), dim3(gblk, used_max), dim3(256), 0, st,    \
                     a.gu_codes, a.gu_scales, a.gu_bias, a.idx, a.E, a.xn, a.act, a.B, a.H, \
                     a.I, a.k, a.alpha, a.limit)
#define DB_LAUNCH(PP, PR)                                                                    \
  hipLaunchKernelGGL((k_moe_down_bt<PP, PR>), dim3(dblk), dim3(256), 0, st, a.dn_codes,     \
                     a.dn_scales, a.dn_bias, a.idx, a.score, a.E, a.act, a.residual, a.out,  \
                     a.B, a.H, a.I, a.k, a.err)
  switch (Pg) {
    case 1: GB_LAUNCH(1, false); break;
    case 2: if (pg) GB_LAUNCH(2, true); else GB_LAUNCH(2, false); break;
    case 3: if (pg) GB_LAUNCH(3, true); else GB_LAUNCH(3, false); break;
    default: if (pg) GB_LAUNCH(4, true); else GB_LAUNCH(4, false); break;
  }
  switch (Pd) {
    case 1: DB_LAUNCH(1, false); break;
    case 2: if (pd) DB_LAUNCH(2, true); else DB_LAUNCH(2, false); break;
    case 3: if (pd) DB_LAUNCH(3, true); else DB_LAUNCH(3, false); break;
    default: if (pd) DB_LAUNCH(4, true); else DB_LAUNCH(4, false); break;
  }
#undef GB_LAUNCH
#undef DB_LAUNCH
}

void launch_moe(const MoeArgs& a, hipStream_t st) {
  if (moe_fused_supported(a) && launch_moe_fused(a, st)) return;
  const int Pg = (a.H / 32 + 63) / 64;  // gate_up reduces over H
  const int Pd = (a.I / 32 + 63) / 64;  // down reduces over I
  const int gblk = (a.I + 4 * kMoeJpw - 1) / (4 * kMoeJpw);
  const int dblk = (a.H + kMoeRpw - 1) / kMoeRpw;
  const bool pg = fp4_pair_ok(a.H / 32, Pg), pd = fp4_pair_ok(a.I / 32, Pd);
#define G_LAUNCH(PP, PR)                                                           \
  hipLaunchKernelGGL((k_moe_gate_up<PP, PR>), dim3(gblk, a.k, a.B), dim3(256), 0, \
                     st, a.gu_codes, a.gu_scales, a.gu_bias, a.router_lg, a.idx,  \
                     a.idx_out, a.score_out, a.E, a.xn, a.act, a.H, a.I, a.k,     \
                     a.alpha, a.limit, a.err)
  // When gate_up records the chosen experts and weights (idx_out/score_out),
  // down reads them instead of ranking the logits again: gate_up has finished
  // before down starts (same stream), and the values are the same.
  const bool dn_ids = a.router_lg != nullptr && a.idx_out != nullptr && a.score_out != nullptr;
  const float* dn_lg = dn_ids ? nullptr : a.router_lg;
  const int32_t* dn_idx = dn_ids ? a.idx_out : a.idx;
  const float* dn_score = dn_ids ? a.score_out : a.score;
#define D_LAUNCH(PP, PR)                                                            \
  hipLaunchKernelGGL((k_moe_down<PP, PR>), dim3(dblk, a.B), dim3(64 * a.k), 0, st, \
                     a.dn_codes, a.dn_scales, a.dn_bias, dn_lg, dn_idx, dn_score,   \
                     a.E, a.act, a.residual, a.out, a.H, a.I, a.k, a.err)
  switch (Pg) {
    case 1: G_LAUNCH(1, false); break;
    case 2: if (pg) G_LAUNCH(2, true); else G_LAUNCH(2, false); break;
    case 3: if (pg) G_LAUNCH(3, true); else G_LAUNCH(3, false); break;
    default: if (pg) G_LAUNCH(4, true); else G_LAUNCH(4, false); break;
  }
  switch (Pd) {
    case 1: D_LAUNCH(1, false); break;
    case 2: if (pd) D_LAUNCH(2, true); else D_LAUNCH(2, false); break;
    case 3: if (pd) D_LAUNCH(3, true); else D_LAUNCH(3, false); break;
    default: if (pd) D_LAUNCH(4, true); else D_LAUNCH(4, false); break;
  }
#undef G_LAUNCH
#undef D_LAUNCH
}

// ===========================================================================
// GQA decode attention with sinks (HFM:235-263): softmax over
// [q.k_j / sqrt(D) for keys j in window] + [sink_h], sink column dropped
// before P.V.  Keys j in [lo, pos] with lo = pos - window + 1 on sliding
// layers (HF mask kv_idx > q_idx - window).
//
// Canonical form (oracle or_c_attn_decode), S splits:
//   chunks of 64 keys from lo; split s takes chunks [s nch / S, (s+1) nch / S).
//   score (lane = key): a = fmaf(q_d, k_d, a) over d = 0..63, times 1/8.
//   per chunk: m' = max(m, max_j s_j); alpha = exp(m - m');
//     p_j = exp(s_j - m'); l = fmaf(l, alpha, butterfly_sum(p_j));
//     lane (kg = lane>>3, dq = lane&7) accumulators o *= alpha, then
//     o = fmaf(p_j, v_j[8 dq + e], o) over the lane's keys j = kg + 8 i.
//   o reduced over kg with xor 8, 16, 32.
//   merge (split order s = 0..S-1): M = max(sink, m_s...);
//     den = exp(sink - M); f_s = exp(m_s - M) (0 for empty splits);
//     den = fmaf(l_s, f_s, den); acc = fmaf(f_s, o_s, acc); out = bf16(acc * (1/den))
//
// k_attn_split: grid (Hkv NHB S, B) with NHB = G / HB (G = Hq / Hkv query
// heads per kv head), block 64 max(HB, 4).  Block (g, hb, s) serves split s
// of kv head g for the HB query heads g G + hb HB + w, one wave each: each
// 64-key chunk of K and V is loaded from HBM once per block into LDS (one
// 16-byte word per thread) and read by its HB waves.  HB = G shares a chunk
// among all heads of the group (many splits); HB = 1 spreads a one-split span
// (the sliding window) over G times more CUs.  The words of two chunks are in
// flight at once: both first tiles are staged before the loop, then chunk
// c + 2 loads while chunk c is computed.  K rows sit in LDS with their eight
// 16-byte words rotated by the key index, so the 64 lanes of a wave, one key
// each, read distinct banks.  q is rotated and k / v of position pos are in
// the cache already (the QKV projection writes them).  Each wave writes its
// split's (o, m, l) partial, or with one split the finished output.
// k_attn_merge: grid (Hq, B), 64 lanes (lane = output dim), merges the S
// partials of a head in split order with the sink.
// ===========================================================================
constexpr int kD = 64;
constexpr int kMaxSplits = 32;

// Words of the 64-key chunk starting at key CB: word WD = 8 j + ch is
// 16-byte word ch of key CB + j; a thread owns words tid and tid + nt
// (nt >= 256).  Keys past p read as zero.  (Macros on plain locals: the
// words stay in registers while the loads are in flight.)
#define ATTN_LOAD_WORD(KW, VW, WD, CB)                                          \
  do {                                                                          \
    KW = make_uint4(0, 0, 0, 0);                                                \
    VW = make_uint4(0, 0, 0, 0);                                                \
    const int key_ = (CB) + ((WD) >> 3);                                        \
    if ((WD) < 512 && key_ <= p) {                                              \
      const size_t row_ = kv_base + (uint32_t)(key_ & key_mask);                \
      KW = reinterpret_cast<const uint4*>(kc + row_ * kD)[(WD) & 7];            \
      VW = reinterpret_cast<const uint4*>(vc + row_ * kD)[(WD) & 7];            \
    }                                                                           \
  } while (0)
#define ATTN_STORE_WORD(KW, VW, WD, BUF)                                        \
  do {                                                                          \
    if ((WD) < 512) {                                                           \
      const int j_ = (WD) >> 3, ch_ = (WD) & 7;                                 \
      kt[BUF][j_ * 8 + ((ch_ + j_) & 7)] = (KW);                                \
      vt[BUF][j_ * 8 + ch_] = (VW);                                             \
    }                                                                           \
  } while (0)

// Splits' partials written by other blocks of the same launch (AGENT):
// agent-scope loads, served at the device's coherence point rather than from
// this XCD's L2, which may hold none of them.
template <bool AGENT>
__device__ __forceinline__ float attn_part_load(const float* p) {
  if (AGENT)
    return __builtin_bit_cast(float, __hip_atomic_load(reinterpret_cast<const uint32_t*>(p),
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  return *p;
}

// One wave merges the S partials of head h (rows pi0 .. pi0 + S - 1 of
// part_o / part_ml) with the sink, lane = output dim.  Every load goes out
// first; each lane t < S computes its split's factor f_t = exp(m_t - M) (0 for
// an empty split), then den and acc take the splits in order with fmaf.
template <bool AGENT>
__device__ __forceinline__ void attn_merge_head(const float* __restrict__ part_o,
                                                const float* __restrict__ part_ml,
                                                size_t pi0, int S, float sk, int lane,
                                                uint16_t* __restrict__ out_row,
                                                uint16_t* __restrict__ outp = nullptr,
                                                size_t outp_at = 0) {
  float ov[kMaxSplits];
#pragma unroll
  for (int t = 0; t < kMaxSplits; ++t)
    ov[t] = t < S ? attn_part_load<AGENT>(part_o + (pi0 + t) * kD + lane) : 0.0f;
  const float mt_l = lane < S ? attn_part_load<AGENT>(part_ml + (pi0 + lane) * 2) : -INFINITY;
  const float lt_l = lane < S ? attn_part_load<AGENT>(part_ml + (pi0 + lane) * 2 + 1) : 0.0f;
  const float M = fmaxf(sk, wave_max(mt_l));
  const float f_l = (mt_l == -INFINITY) ? 0.0f : neon_expf(__fsub_rn(mt_l, M));
  float den = neon_expf(__fsub_rn(sk, M));
  float acc = 0.0f;
#pragma unroll
  for (int t = 0; t < kMaxSplits; ++t) {
    if (t < S) {
      const float f = readlane_f(f_l, t);
      den = __builtin_fmaf(readlane_f(lt_l, t), f, den);
      acc = __builtin_fmaf(f, ov[t], acc);
    }
  }
  const uint16_t o = f2bf(__fmul_rn(acc, __fdiv_rn(1.0f, den)));
  out_row[lane] = o;
  // the packed copy: lane's column k0 + lane sits at outp_at + the offset of
  // lane (units of 8 are contiguous, 16 B apart per 16-row lane group)
  if (outp != nullptr) outp[outp_at + (size_t)(lane >> 5) * 512 + ((lane & 31) >> 3) * 128 + (lane & 7)] = o;
}

__global__ __launch_bounds__(512) void k_attn_split(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ pos_arr,
    float* __restrict__ part_o, float* __restrict__ part_ml,
    const uint16_t* __restrict__ sinks, uint16_t* __restrict__ out,
    const int32_t* __restrict__ seq, int Hq, int Hkv, int G, int HB, int T_max, int key_mask,
    int window, int S, int q_stride, int32_t* __restrict__ arrive) {
  __shared__ __align__(16) uint4 kt[2][64 * 8];  // [key][word], words rotated by key
  __shared__ __align__(16) uint4 vt[2][64 * 8];  // [key][word]
  __shared__ __align__(16) float qs[8][kD];
  __shared__ float ps[8][64];
  __shared__ int merge_here;
  // blockDim = 64 max(HB, 4): waves w >= HB only help stage the tiles
  const int nt = blockDim.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const bool active = w < HB;
  const int NHB = G / HB;
  const int g = blockIdx.x % Hkv, hb = (blockIdx.x / Hkv) % NHB, s = blockIdx.x / (Hkv * NHB);
  const int b = blockIdx.y;
  const int h = g * G + hb * HB + (active ? w : 0);
  // q first (it does not depend on the position), then the position
  const uint16_t qv = q[(size_t)b * q_stride + (size_t)h * kD + lane];
  const uint16_t sink_raw = load_pinned_u16(sinks + h);  // used at the end (one split)
  const int p = pos_arr[b];
  const int sq = seq != nullptr ? seq[b] : b;  // the row's KV-cache sequence
  const int lo = (window > 0 && p - window + 1 > 0) ? p - window + 1 : 0;
  const int n = p - lo + 1;
  const int nch = (n + 63) >> 6;
  const int c0 = (int)((int64_t)s * nch / S), c1 = (int)((int64_t)(s + 1) * nch / S);
  const size_t kv_base = ((size_t)sq * Hkv + g) * T_max;

  // the first two chunks' words into registers: both tiles are staged before
  // the loop, so a split of two chunks (the 128-key sliding window) never
  // waits for memory inside it
  uint4 nk0, nk1, nv0, nv1;  // chunk c0, later the chunk two ahead
  uint4 pk0, pk1, pv0, pv1;  // chunk c0 + 1
  if (c0 < c1) {
    ATTN_LOAD_WORD(nk0, nv0, tid, lo + c0 * 64);
    ATTN_LOAD_WORD(nk1, nv1, tid + nt, lo + c0 * 64);
  }
  if (c0 + 1 < c1) {
    ATTN_LOAD_WORD(pk0, pv0, tid, lo + (c0 + 1) * 64);
    ATTN_LOAD_WORD(pk1, pv1, tid + nt, lo + (c0 + 1) * 64);
  }
  if (active) qs[w][lane] = bf2f(qv);
  if (c0 < c1) {
    ATTN_STORE_WORD(nk0, nv0, tid, 0);
    ATTN_STORE_WORD(nk1, nv1, tid + nt, 0);
  }
  if (c0 + 1 < c1) {
    ATTN_STORE_WORD(pk0, pv0, tid, 1);
    ATTN_STORE_WORD(pk1, pv1, tid + nt, 1);
  }
  __syncthreads();

  // q of this wave's head in registers (one LDS pass for all chunks)
  float qf[kD];
  {
    const float4* q4 = reinterpret_cast<const float4*>(qs[w]);
#pragma unroll
    for (int i = 0; i < kD / 4; ++i) {
      const float4 v = q4[i];
      qf[4 * i] = v.x; qf[4 * i + 1] = v.y; qf[4 * i + 2] = v.z; qf[4 * i + 3] = v.w;
    }
  }
  float m = -INFINITY, l = 0.0f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.0f;
  const int kg = lane >> 3, dq = lane & 7;

  for (int c = c0; c < c1; ++c) {
    const int buf = (c - c0) & 1;
    if (c + 2 < c1) {  // chunk c + 2 goes into this tile once it is consumed
      ATTN_LOAD_WORD(nk0, nv0, tid, lo + (c + 2) * 64);
      ATTN_LOAD_WORD(nk1, nv1, tid + nt, lo + (c + 2) * 64);
    }
    const int cb = lo + c * 64;
    if (active) {
      const bool valid = cb + lane <= p;
      // the key row of this lane: all eight words first, then the chain
      uint4 kw[kD / 8];
#pragma unroll
      for (int u = 0; u < kD / 8; ++u) kw[u] = kt[buf][lane * 8 + ((u + lane) & 7)];
      float a = 0.0f;
#pragma unroll
      for (int u = 0; u < kD / 8; ++u) {
        float kf[8];
        unpack8(kw[u], kf);
#pragma unroll
        for (int e = 0; e < 8; ++e) a = __builtin_fmaf(qf[8 * u + e], kf[e], a);
      }
      const float sc = valid ? __fmul_rn(a, 0.125f) : -INFINITY;  // 1/sqrt(64), HFM:277
      const float mn = fmaxf(m, wave_max(sc));
      const float alpha = neon_expf(__fsub_rn(m, mn));
      const float pj = valid ? neon_expf(__fsub_rn(sc, mn)) : 0.0f;
      l = __builtin_fmaf(l, alpha, wave_sum(pj));
      m = mn;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = __fmul_rn(o[e], alpha);
      // p of key j at (j % 8) * 8 + j / 8: lane (kg, dq) reads its keys
      // kg + 8 i as eight consecutive floats
      ps[w][(lane & 7) * 8 + (lane >> 3)] = pj;
      wave_lds_sync();
      uint4 vw[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) vw[i] = vt[buf][(kg + 8 * i) * 8 + dq];
      const float4 pa = *reinterpret_cast<const float4*>(&ps[w][kg * 8]);
      const float4 pb = *reinterpret_cast<const float4*>(&ps[w][kg * 8 + 4]);
      const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
      // keys past p have p = 0 and zero words: fmaf(0, 0, o) == o exactly
      // (o is never -0), so they need no branch
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float vf[8];
        unpack8(vw[i], vf);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf(pv[i], vf[e], o[e]);
      }
    }  // active
    __syncthreads();  // tile buf and ps are consumed
    if (c + 2 < c1) {  // visible to the readers of iteration c + 2 after the
                       // barrier that ends iteration c + 1
      ATTN_STORE_WORD(nk0, nv0, tid, buf);
      ATTN_STORE_WORD(nk1, nv1, tid + nt, buf);
    }
  }
  // with `arrive` every wave of the block reaches the arrival barrier below,
  // so the helper waves stay until then
  if (!active && (S == 1 || arrive == nullptr)) return;
  // reduce o over the 8 key groups (lane bits 3..5)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float v = o[e];
    v = __fadd_rn(v, xor_lane<8>(v));
    v = __fadd_rn(v, xor_lane<16>(v));
    v = __fadd_rn(v, xor_lane<32>(v));
    o[e] = v;
  }
  if (S == 1) {
    // one split: the merge with the sink happens here, with exactly the
    // operations k_attn_merge applies to a single partial
    if (kg == 0) {
      const float sk = bf2f(sink_raw);
      const float M = fmaxf(sk, m);
      float den = neon_expf(__fsub_rn(sk, M));
      const float f = (m == -INFINITY) ? 0.0f : neon_expf(__fsub_rn(m, M));
      den = __builtin_fmaf(l, f, den);
      const float inv = __fdiv_rn(1.0f, den);
      uint32_t w4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w4[e] = pack_bf2(__fmul_rn(__builtin_fmaf(f, o[2 * e], 0.0f), inv),
                         __fmul_rn(__builtin_fmaf(f, o[2 * e + 1], 0.0f), inv));
      *reinterpret_cast<uint4*>(out + ((size_t)b * Hq + h) * kD + dq * 8) =
          make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }
    return;
  }
  const size_t pi = ((size_t)b * Hq + h) * S + s;
  if (arrive == nullptr) {  // the partials go to k_attn_merge
    if (kg == 0) {
      float4* po = reinterpret_cast<float4*>(part_o + pi * kD + dq * 8);
      po[0] = make_float4(o[0], o[1], o[2], o[3]);
      po[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
    if (lane == 0) { part_ml[pi * 2] = m; part_ml[pi * 2 + 1] = l; }
    return;
  }
  // Merge in this launch: the partials are stored at agent scope (they
  // complete at the device's coherence point, past this XCD's L2), each
  // block arrives on its (row, kv head) counter once its stores are done,
  // and the block that arrives last merges the G heads of that kv head
  // (attn_merge_head, reading the partials at agent scope) and sets the
  // counter back to 0 for the next launch.  No block waits for another.
  if (active) {
    auto pack = [](float a, float c) {
      return (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(c) << 32);
    };
    if (kg == 0) {
      uint64_t* po = reinterpret_cast<uint64_t*>(part_o + pi * kD + dq * 8);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        __hip_atomic_store(po + e, pack(o[2 * e], o[2 * e + 1]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane == 0)
      __hip_atomic_store(reinterpret_cast<uint64_t*>(part_ml + pi * 2), pack(m, l),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's stores have completed
  __syncthreads();
  int32_t* ctr = arrive + ((size_t)b * Hkv + g) * kAttnArriveStride;
  if (tid == 0)
    merge_here = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 S - 1;
  __syncthreads();
  if (!merge_here) return;
  if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (active)
    attn_merge_head<true>(part_o, part_ml, ((size_t)b * Hq + h) * S, S, bf2f(sink_raw), lane,
                          out + ((size_t)b * Hq + h) * kD);
}

__global__ __launch_bounds__(64) void k_attn_merge(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    const uint16_t* __restrict__ sinks, uint16_t* __restrict__ out, int Hq,
    int S, uint16_t* __restrict__ outp) {
  const int h = blockIdx.x, b = blockIdx.y;
  // head h's 64 columns start at k0 = 64 h: unit 8 h (a multiple of 8), so
  // they fill lanes b % 16 + 16 q (q = 0..3) of steps 2 (h % 2), +1 of chunk h / 2
  const size_t at = outp != nullptr ? mx_packed_at(b, kD * h, Hq * kD / 128) : 0;
  attn_merge_head<false>(part_o, part_ml, ((size_t)b * Hq + h) * S, S, bf2f(sinks[h]),
                         threadIdx.x, out + ((size_t)b * Hq + h) * kD, outp, at);
}

#undef ATTN_LOAD_WORD
#undef ATTN_STORE_WORD

void launch_attn_merge(const AttnArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k_attn_merge, dim3(a.Hq, a.B), dim3(64), 0, st, a.part_o, a.part_ml,
                     a.sinks, a.out, a.Hq, a.S, a.out_packed);
}

void launch_attn(const AttnArgs& a, hipStream_t st) {
  const int G = a.Hq / a.Hkv;  // 1, 2, 4 or 8 (checked on the host)
  // one split: a block per query head (more CUs for a short span); several:
  // a block per (kv head, split) serving the whole group
  const int HB = a.S == 1 ? 1 : G;
  hipLaunchKernelGGL(k_attn_split, dim3(a.Hkv * (G / HB) * a.S, a.B),
                     dim3(64 * (HB < 4 ? 4 : HB)), 0, st, a.q, a.kc, a.vc, a.pos,
                     a.part_o, a.part_ml, a.sinks, a.out, a.seq, a.Hq, a.Hkv, G, HB,
                     a.T_max, a.key_mask, a.window, a.S, a.q_stride,
                     a.S > 1 ? a.arrive : nullptr);
  // one split finishes in the split kernel; several merge there too when the
  // arrival counters are given, else in k_attn_merge
  if (a.S > 1 && a.arrive == nullptr)
    hipLaunchKernelGGL(k_attn_merge, dim3(a.Hq, a.B), dim3(64), 0, st, a.part_o,
                       a.part_ml, a.sinks, a.out, a.Hq, a.S, nullptr);
}

// Key splits for a cache of T_max rows: spans of at most 4 chunks (256 keys,
// e.g. the 128-key sliding window) stay in one split, which finishes in the
// split kernel (no merge launch); longer spans use one split per 64-key
// chunk, at most 32.
int attn_splits(int T_max, int window) {
  const int span = window > 0 ? (window < T_max ? window : T_max) : T_max;
  const int s = (span + 63) / 64;
  return s <= 4 ? 1 : (s > kMaxSplits ? kMaxSplits : s);
}

}  // namespace neon

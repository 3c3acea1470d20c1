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

namespace neon {

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

template <int P>
__device__ __forceinline__ void fp4_load_row(Fp4Row<P>& r,
                                             const uint8_t* __restrict__ codes,
                                             const uint8_t* __restrict__ scales,
                                             int U, int lane) {
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = lane + 64 * p;
    if (u < U) {
      r.c[p] = *reinterpret_cast<const uint4*>(codes + (size_t)u * 16);
      r.s[p] = scales[u];
    } else {
      r.c[p] = make_uint4(0, 0, 0, 0);
      r.s[p] = 127;
    }
  }
}

template <int P>
__device__ __forceinline__ float fp4_row_partial(const Fp4Row<P>& r,
                                                 const float (&xr)[P][32],
                                                 int U, int lane) {
  float acc = 0.0f;
#pragma unroll
  for (int p = 0; p < P; ++p)
    if (lane + 64 * p < U)
      acc = __fadd_rn(acc, e8m0_scale(fp4_unit_dot(r.c[p], xr[p]), r.s[p]));
  return acc;
}

// x (bf16 [K] in LDS) -> fp32 registers for the lane's MXFP4 units
template <int P>
__device__ __forceinline__ void fp4_load_x(float (&xr)[P][32],
                                           const uint4* __restrict__ xs, int U,
                                           int lane) {
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = lane + 64 * p;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      unpack8((u < U) ? xs[u * 4 + q] : make_uint4(0, 0, 0, 0), &xr[p][8 * q]);
  }
}

template <int P>
__device__ __forceinline__ void bf16_load_x(float (&xr)[P][8],
                                            const uint4* __restrict__ xs,
                                            int U, int lane) {
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = lane + 64 * p;
    unpack8((u < U) ? xs[u] : make_uint4(0, 0, 0, 0), xr[p]);
  }
}

template <int P>
__device__ __forceinline__ void bf16_load_row(uint4 (&w)[P],
                                              const uint16_t* __restrict__ row,
                                              int U, int lane) {
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int u = lane + 64 * p;
    w[p] = (u < U) ? *reinterpret_cast<const uint4*>(row + (size_t)u * 8)
                   : make_uint4(0, 0, 0, 0);
  }
}

template <int P>
__device__ __forceinline__ float bf16_row_partial(const uint4 (&w)[P],
                                                  const float (&xr)[P][8],
                                                  int U, int lane) {
  float acc = 0.0f;
#pragma unroll
  for (int p = 0; p < P; ++p)
    if (lane + 64 * p < U) acc = fma8_bf16(w[p], xr[p], acc);
  return acc;
}

// Block-wide: x[K] (bf16, global) -> LDS, optionally RMS-normalised with
// weight nw (HFM:57-62).  Canonical form (oracle or_c_rmsnorm): wave 0 forms
// ss with lane partials ss = fmaf(x_k, x_k, ss) over the units
// u = l + 64 p (8 elements each, increasing k) and the xor butterfly; then
// r = 1 / sqrt(ss / K + eps) with correctly rounded fp32 division and square
// root; y_k = bf16(w_k * (x_k * r)).  If xn_out is not NULL the block also
// writes the normalised vector there (callers pass it from one block per row).
__device__ void block_load_x(uint4* __restrict__ xs,
                             const uint16_t* __restrict__ x,
                             const uint16_t* __restrict__ nw, float eps, int K,
                             uint16_t* __restrict__ xn_out) {
  __shared__ float r_s;
  const int U8 = K / 8;
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  if (nw == nullptr) {
    for (int i = threadIdx.x; i < U8; i += blockDim.x) xs[i] = xv[i];
    __syncthreads();
    return;
  }
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    float ss = 0.0f;
    for (int u = lane; u < U8; u += 64) {
      float f[8];
      unpack8(xv[u], f);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(f[j], f[j], ss);
    }
    ss = wave_sum(ss);
    if (lane == 0)
      r_s = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)K), eps)));
  }
  __syncthreads();
  const float r = r_s;
  const uint4* wv = reinterpret_cast<const uint4*>(nw);
  for (int i = threadIdx.x; i < U8; i += blockDim.x) {
    float a[8], b[8];
    unpack8(xv[i], a);
    unpack8(wv[i], b);
    uint32_t o4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o4[j] = pack_bf2(__fmul_rn(b[2 * j], __fmul_rn(a[2 * j], r)),
                       __fmul_rn(b[2 * j + 1], __fmul_rn(a[2 * j + 1], r)));
    const uint4 o = make_uint4(o4[0], o4[1], o4[2], o4[3]);
    xs[i] = o;
    if (xn_out != nullptr) reinterpret_cast<uint4*>(xn_out)[i] = o;
  }
  __syncthreads();
}

constexpr int kMaxK = 8192;  // LDS holds x [K] bf16 (16 KB)

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
  __shared__ uint4 xs[kMaxK / 8];
  const int U = K / 32, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.z;
  const int r0 = (blockIdx.x * 4 + wave) * rpw;
  const int r1 = min(r0 + rpw, N);
  Fp4Row<P> cur;
  if (r0 < r1)
    fp4_load_row<P>(cur, codes + (size_t)r0 * (K / 2), scales + (size_t)r0 * U,
                    U, lane);
  block_load_x(xs, x + (size_t)b * K, nullptr, 0.0f, K, nullptr);
  float xr[P][32];
  fp4_load_x<P>(xr, xs, U, lane);
  for (int r = r0; r < r1; ++r) {
    Fp4Row<P> nxt;
    if (r + 1 < r1)
      fp4_load_row<P>(nxt, codes + (size_t)(r + 1) * (K / 2),
                      scales + (size_t)(r + 1) * U, U, lane);
    float acc = wave_sum(fp4_row_partial<P>(cur, xr, U, lane));
    if (lane == 0) {
      if (bias) acc = __fadd_rn(acc, bf2f(bias[r]));
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

void launch_mxfp4_gemv(const uint8_t* codes, const uint8_t* scales,
                       const uint16_t* bias, const uint16_t* x, uint16_t* y,
                       int N, int K, int B, hipStream_t st) {
  const int P = (K / 32 + 63) / 64;
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
// grid (nblk, 1, B), block 256; rows are grid-strided in groups of rpw per
// wave so huge N (lm_head) runs on a bounded grid.
// ===========================================================================
enum { MODE_STORE = 0, MODE_RESID = 1, MODE_LOGITS = 2 };

template <int P, int MODE>
__global__ __launch_bounds__(256) void k_gemv_bf16(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ bias,
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ nw, float eps,
    uint16_t* __restrict__ y, float* __restrict__ logits,
    float* __restrict__ part_val, int32_t* __restrict__ part_idx, int N, int K,
    int rpw) {
  __shared__ uint4 xs[kMaxK / 8];
  __shared__ float bv_s[4];
  __shared__ int32_t bi_s[4];
  const int U = K / 8, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.z;
  const int ngroups = (N + rpw - 1) / rpw;
  const int gstride = gridDim.x * 4;
  int g = blockIdx.x * 4 + wave;
  uint4 cur[P];
  if (g < ngroups) bf16_load_row<P>(cur, W + (size_t)g * rpw * K, U, lane);
  block_load_x(xs, x + (size_t)b * K, nw, eps, K, nullptr);
  float xr[P][8];
  bf16_load_x<P>(xr, xs, U, lane);
  float best_v = -INFINITY;
  int32_t best_i = 0x7fffffff;
  for (; g < ngroups; g += gstride) {
    const int r0 = g * rpw, r1 = min(r0 + rpw, N);
    for (int r = r0; r < r1; ++r) {
      uint4 nxt[P];
      const int rn = (r + 1 < r1) ? r + 1
                                  : ((g + gstride < ngroups) ? (g + gstride) * rpw : -1);
      if (rn >= 0) bf16_load_row<P>(nxt, W + (size_t)rn * K, U, lane);
      const float acc = wave_sum(bf16_row_partial<P>(cur, xr, U, lane));
      if (MODE == MODE_LOGITS) {
        if (acc > best_v) { best_v = acc; best_i = r; }
        if (lane == 0) logits[(size_t)b * N + r] = acc;
      } else if (lane == 0) {
        const float v = bias ? __fadd_rn(acc, bf2f(bias[r])) : acc;
        const size_t o = (size_t)b * N + r;
        if (MODE == MODE_STORE) y[o] = f2bf(v);
        else y[o] = f2bf(__fadd_rn(bf2f(y[o]), bf2f(f2bf(v))));
      }
#pragma unroll
      for (int p = 0; p < P; ++p) cur[p] = nxt[p];
    }
  }
  if (MODE == MODE_LOGITS) {
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

template <int P, int MODE>
static void launch_gemv_bf16_p(const GemvArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((k_gemv_bf16<P, MODE>), dim3(a.nblk, 1, a.B), dim3(256), 0,
                     st, a.W, a.bias, a.x, a.norm_w, a.eps, a.y, a.logits,
                     a.part_val, a.part_idx, a.N, a.K, a.rpw);
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

int gemv_default_grid(int N, int rpw) {
  const int ngroups = (N + rpw - 1) / rpw;
  const int nblk = (ngroups + 3) / 4;
  return nblk < 2048 ? nblk : 2048;
}

void launch_gemv_bf16(const GemvArgs& a, hipStream_t st) {
  switch (a.mode) {
    case MODE_STORE: launch_gemv_bf16_m<MODE_STORE>(a, st); break;
    case MODE_RESID: launch_gemv_bf16_m<MODE_RESID>(a, st); break;
    default: launch_gemv_bf16_m<MODE_LOGITS>(a, st); break;
  }
}

// ===========================================================================
// Final argmax over the lm_head partials; advances the sequence.
// grid B, block 256.  Greedy id = largest logit, ties to the lowest index.
// tokens[b][pos+1] receives it unless that slot still belongs to the prompt
// (teacher forcing); pos[b] += 1.
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
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const int32_t oi = __shfl_xor(i, off, 64);
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) { sv[wave] = v; si[wave] = i; }
  __syncthreads();
  if (threadIdx.x == 0) {
    v = sv[0];
    i = si[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
      if (sv[w] > v || (sv[w] == v && si[w] < i)) { v = sv[w]; i = si[w]; }
    if (i == 0x7fffffff) i = 0;
    const int p = pos[b];
    if (p + 1 >= prompt_len[b]) tokens[(size_t)b * tok_stride + p + 1] = i;
    last_ids[b] = i;
    pos[b] = p + 1;
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
// Embedding gather: h[b] = embed[tokens[b][pos[b]]]
// ===========================================================================
__global__ void k_embed(const int32_t* __restrict__ tokens, int tok_stride,
                        const int32_t* __restrict__ pos,
                        const uint16_t* __restrict__ embed,
                        uint16_t* __restrict__ h, int H) {
  const int b = blockIdx.x;
  const int32_t id = tokens[(size_t)b * tok_stride + pos[b]];
  const uint4* src = reinterpret_cast<const uint4*>(embed + (size_t)id * H);
  uint4* dst = reinterpret_cast<uint4*>(h + (size_t)b * H);
  for (int i = threadIdx.x; i < H / 8; i += blockDim.x) dst[i] = src[i];
}

void launch_embed(const int32_t* tokens, int tok_stride, const int32_t* pos,
                  const uint16_t* embed, uint16_t* h, int H, int B,
                  hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3(B), dim3(256), 0, st, tokens, tok_stride,
                     pos, embed, h, H);
}

// ===========================================================================
// Standalone RMSNorm (canonical form of block_load_x)
// ===========================================================================
__global__ __launch_bounds__(256) void k_rmsnorm(const uint16_t* __restrict__ x,
                                                 const uint16_t* __restrict__ w,
                                                 uint16_t* __restrict__ out,
                                                 int H, float eps) {
  __shared__ uint4 xs[kMaxK / 8];
  const int b = blockIdx.x;
  block_load_x(xs, x + (size_t)b * H, w, eps, H, out + (size_t)b * H);
}

void launch_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out, int B,
                    int H, float eps, hipStream_t st) {
  hipLaunchKernelGGL(k_rmsnorm, dim3(B), dim3(256), 0, st, x, w, out, H, eps);
}

// ===========================================================================
// RoPE (HFM:215-222): half-split rotation with the host-built YaRN table
// (cos/sin [n_pos][D/2] fp32, HF modeling_rope_utils.py:429-483):
//   o1 = x1 c - x2 s,  o2 = x2 c + x1 s   (each product and sum rounded)
// ===========================================================================
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s,
                                          float& o1, float& o2) {
  o1 = __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, s));
  o2 = __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, s));
}

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
// Router (HFM:117-130), one block per batch row, 8 waves.  Optional fused
// RMSNorm prologue (then the normalised x is also written to xn_out for the
// experts).  Logits: the canonical bf16 row dot + bias (fp32 add).  Top-k by
// value, ties to the lower expert index; softmax over the k selected values:
// e_t = exp(v_t - v_0) (neon_expf), s = sum in rank order, score_t = e_t / s.
// ===========================================================================
constexpr int kMaxExperts = 256;

template <int P>
__global__ __launch_bounds__(512) void k_router(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ nw, float eps,
    uint16_t* __restrict__ xn_out, const uint16_t* __restrict__ W,
    const uint16_t* __restrict__ bias, int32_t* __restrict__ idx,
    float* __restrict__ score, float* __restrict__ logits_out, int E, int H,
    int k) {
  __shared__ uint4 xs[kMaxK / 8];
  __shared__ float lg[kMaxExperts];
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int U = H / 8;
  block_load_x(xs, x + (size_t)b * H, nw, eps, H,
               xn_out ? xn_out + (size_t)b * H : nullptr);
  float xr[P][8];
  bf16_load_x<P>(xr, xs, U, lane);
  for (int e = wave; e < E; e += nwaves) {
    uint4 w[P];
    bf16_load_row<P>(w, W + (size_t)e * H, U, lane);
    const float acc = wave_sum(bf16_row_partial<P>(w, xr, U, lane));
    if (lane == 0) lg[e] = __fadd_rn(acc, bf2f(bias[e]));
  }
  __syncthreads();
  if (wave == 0) {
    if (logits_out)
      for (int e = lane; e < E; e += 64) logits_out[(size_t)b * E + e] = lg[e];
    float vals[16];
    int32_t ids[16];
    uint64_t used[kMaxExperts / 64] = {0, 0, 0, 0};
    for (int t = 0; t < k; ++t) {
      float v = -INFINITY;
      int32_t i = 0x7fffffff;
      for (int e = lane; e < E; e += 64) {
        if ((used[e >> 6] >> (e & 63)) & 1ull) continue;
        if (i == 0x7fffffff || lg[e] > v) { v = lg[e]; i = e; }
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int32_t oi = __shfl_xor(i, off, 64);
        const bool take = (oi != 0x7fffffff) &&
                          (i == 0x7fffffff || ov > v || (ov == v && oi < i));
        if (take) { v = ov; i = oi; }
      }
      used[i >> 6] |= 1ull << (i & 63);
      vals[t] = v;
      ids[t] = i;
    }
    if (lane == 0) {
      float ex[16], s = 0.0f;
      for (int t = 0; t < k; ++t) {
        ex[t] = neon_expf(__fsub_rn(vals[t], vals[0]));
        s = __fadd_rn(s, ex[t]);
      }
      for (int t = 0; t < k; ++t) {
        idx[b * k + t] = ids[t];
        score[b * k + t] = __fdiv_rn(ex[t], s);
      }
    }
  }
}

void launch_router(const uint16_t* x, const uint16_t* nw, float eps,
                   uint16_t* xn_out, const uint16_t* W, const uint16_t* bias,
                   int32_t* idx, float* score, float* logits_out, int B, int E,
                   int H, int k, hipStream_t st) {
  const int P = (H / 8 + 63) / 64;
  switch (P) {
#define R_CASE(PP)                                                           \
  case PP:                                                                   \
    hipLaunchKernelGGL(k_router<PP>, dim3(B), dim3(512), 0, st, x, nw, eps,  \
                       xn_out, W, bias, idx, score, logits_out, E, H, k);    \
    break;
    R_CASE(1) R_CASE(2) R_CASE(3) R_CASE(4) R_CASE(5) R_CASE(6) R_CASE(7)
    R_CASE(8)
    default:
      hipLaunchKernelGGL(k_router<16>, dim3(B), dim3(512), 0, st, x, nw, eps,
                         xn_out, W, bias, idx, score, logits_out, E, H, k);
#undef R_CASE
  }
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
__device__ __forceinline__ float swiglu_clamp(float g, float u, float alpha,
                                              float limit) {
  g = g > limit ? limit : g;
  u = u > limit ? limit : (u < -limit ? -limit : u);
  const float e = neon_expf(-__fmul_rn(g, alpha));
  const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, e));
  return __fmul_rn(__fadd_rn(u, 1.0f), __fmul_rn(g, sig));
}

template <int P>
__global__ __launch_bounds__(256) void k_moe_gate_up(
    const uint8_t* __restrict__ gu_codes, const uint8_t* __restrict__ gu_scales,
    const uint16_t* __restrict__ gu_bias, const int32_t* __restrict__ idx,
    const uint16_t* __restrict__ xn, uint16_t* __restrict__ act, int H, int I,
    int k, int jpw, float alpha, float limit) {
  __shared__ uint4 xs[kMaxK / 8];
  const int slot = blockIdx.y, b = blockIdx.z;
  const int U = H / 32, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = idx[b * k + slot];
  const size_t rows = (size_t)2 * I;
  const uint8_t* codes = gu_codes + (size_t)e * rows * (H / 2);
  const uint8_t* scales = gu_scales + (size_t)e * rows * U;
  const uint16_t* bias = gu_bias + (size_t)e * rows;
  const int j0 = (blockIdx.x * 4 + wave) * jpw;
  const int j1 = min(j0 + jpw, I);
  Fp4Row<P> cg, cu;
  if (j0 < j1) {
    fp4_load_row<P>(cg, codes + (size_t)(2 * j0) * (H / 2),
                    scales + (size_t)(2 * j0) * U, U, lane);
    fp4_load_row<P>(cu, codes + (size_t)(2 * j0 + 1) * (H / 2),
                    scales + (size_t)(2 * j0 + 1) * U, U, lane);
  }
  block_load_x(xs, xn + (size_t)b * H, nullptr, 0.0f, H, nullptr);
  float xr[P][32];
  fp4_load_x<P>(xr, xs, U, lane);
  uint16_t* out = act + ((size_t)b * k + slot) * I;
  for (int j = j0; j < j1; ++j) {
    Fp4Row<P> ng, nu;
    if (j + 1 < j1) {
      fp4_load_row<P>(ng, codes + (size_t)(2 * j + 2) * (H / 2),
                      scales + (size_t)(2 * j + 2) * U, U, lane);
      fp4_load_row<P>(nu, codes + (size_t)(2 * j + 3) * (H / 2),
                      scales + (size_t)(2 * j + 3) * U, U, lane);
    }
    const float g = wave_sum(fp4_row_partial<P>(cg, xr, U, lane));
    const float u = wave_sum(fp4_row_partial<P>(cu, xr, U, lane));
    if (lane == 0) {
      const float gb = __fadd_rn(g, bf2f(bias[2 * j]));
      const float ub = __fadd_rn(u, bf2f(bias[2 * j + 1]));
      out[j] = f2bf(swiglu_clamp(gb, ub, alpha, limit));
    }
    cg = ng;
    cu = nu;
  }
}

// down + weighted sum (+ residual): grid (ceil(H / rpw), B), block 64 k (wave
// s handles top-k slot s).  All k waves compute the same rows; the block
// combines y = fmaf(score_s, dot_s + bias_s, y) in slot order from y = 0
// (HFM:111-112), one rounding to bf16, then out = bf16(residual + y) when
// residual is given.
template <int P>
__global__ __launch_bounds__(1024) void k_moe_down(
    const uint8_t* __restrict__ dn_codes, const uint8_t* __restrict__ dn_scales,
    const uint16_t* __restrict__ dn_bias, const int32_t* __restrict__ idx,
    const float* __restrict__ score, const uint16_t* __restrict__ act,
    const uint16_t* residual, uint16_t* out, int H, int I, int k, int rpw) {
  __shared__ float red[16][64];
  const int b = blockIdx.y;
  const int U = I / 32, lane = threadIdx.x & 63, slot = threadIdx.x >> 6;
  const int e = idx[b * k + slot];
  const uint8_t* codes = dn_codes + (size_t)e * H * (I / 2);
  const uint8_t* scales = dn_scales + (size_t)e * H * U;
  const uint16_t* bias = dn_bias + (size_t)e * H;
  const int n0 = blockIdx.x * rpw, n1 = min(n0 + rpw, H);
  Fp4Row<P> cur;
  if (n0 < n1)
    fp4_load_row<P>(cur, codes + (size_t)n0 * (I / 2), scales + (size_t)n0 * U,
                    U, lane);
  float xr[P][32];
  fp4_load_x<P>(xr, reinterpret_cast<const uint4*>(act + ((size_t)b * k + slot) * I),
                U, lane);
  for (int n = n0; n < n1; ++n) {
    Fp4Row<P> nxt;
    if (n + 1 < n1)
      fp4_load_row<P>(nxt, codes + (size_t)(n + 1) * (I / 2),
                      scales + (size_t)(n + 1) * U, U, lane);
    const float acc = wave_sum(fp4_row_partial<P>(cur, xr, U, lane));
    if (lane == 0) red[slot][n - n0] = __fadd_rn(acc, bf2f(bias[n]));
    cur = nxt;
  }
  __syncthreads();
  if (threadIdx.x < n1 - n0) {
    const int t = threadIdx.x, n = n0 + t;
    float y = 0.0f;
    for (int s = 0; s < k; ++s) y = __builtin_fmaf(score[b * k + s], red[s][t], y);
    const uint16_t m = f2bf(y);
    const size_t o = (size_t)b * H + n;
    out[o] = residual ? f2bf(__fadd_rn(bf2f(residual[o]), bf2f(m))) : m;
  }
}

void launch_moe(const MoeArgs& a, hipStream_t st) {
  const int P = (a.H / 32 + 63) / 64;
  const int jpw = 4;
  const int gblk = (a.I + 4 * jpw - 1) / (4 * jpw);
  const int rpw = 8;
  const int dblk = (a.H + rpw - 1) / rpw;
  switch (P) {
#define M_CASE(PP)                                                            \
  case PP:                                                                    \
    hipLaunchKernelGGL(k_moe_gate_up<PP>, dim3(gblk, a.k, a.B), dim3(256), 0, \
                       st, a.gu_codes, a.gu_scales, a.gu_bias, a.idx, a.xn,   \
                       a.act, a.H, a.I, a.k, jpw, a.alpha, a.limit);          \
    hipLaunchKernelGGL(k_moe_down<PP>, dim3(dblk, a.B), dim3(64 * a.k), 0,   \
                       st, a.dn_codes, a.dn_scales, a.dn_bias, a.idx,         \
                       a.score, a.act, a.residual, a.out, a.H, a.I, a.k,      \
                       rpw);                                                  \
    break;
    M_CASE(1) M_CASE(2) M_CASE(3)
    default: M_CASE(4)
#undef M_CASE
  }
}

// ===========================================================================
// GQA decode attention with sinks (HFM:235-263): softmax over
// [q.k_j / sqrt(D) for keys j in window] + [sink_h], sink column dropped
// before P.V.  Keys j in [lo, pos] with lo = pos - window + 1 on sliding
// layers (HF mask kv_idx > q_idx - window).
//
// grid (S, Hkv, B), one wave per block.  Canonical form (oracle
// or_c_attn_decode):
//   chunks of 64 keys from lo; split s takes chunks [s nch / S, (s+1) nch / S).
//   score (lane = key): a = fmaf(q_d, k_d, a) over d = 0..63, times 1/8.
//   per chunk and head: m' = max(m, max_j s_j); alpha = exp(m - m');
//     p_j = exp(s_j - m'); l = fmaf(l, alpha, butterfly_sum(p_j));
//     lane (kg = lane>>3, dq = lane&7) accumulators o *= alpha, then
//     o = fmaf(p_j, v_j[8 dq + e], o) over the lane's keys j = kg + 8 i.
//   o reduced over kg with xor 8, 16, 32.
//   merge (split order s = 0..S-1): M = max(sink, m_s...);
//     den = exp(sink - M); f_s = exp(m_s - M) (0 for empty splits);
//     den = fmaf(l_s, f_s, den); acc = fmaf(f_s, o_s, acc); out = bf16(acc * (1/den))
// S > 1: partials go to global memory and the last split block to arrive
// (agent-scope atomic counter) merges them; S == 1 merges in registers.
// fused != 0: q_src is the raw qkv row ([Hq + 2 Hkv] heads); the block rotates
// q itself (YaRN table), and the block owning key `pos` also rotates k and
// appends k/v to the caches (stream order makes them visible to later steps).
// ===========================================================================
constexpr int kD = 64;

template <int G>
__global__ __launch_bounds__(64) void k_attn_decode(
    const uint16_t* __restrict__ q_src, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, const uint16_t* __restrict__ sinks,
    const int32_t* __restrict__ pos_arr, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, uint16_t* __restrict__ out,
    float* __restrict__ part_o, float* __restrict__ part_ml,
    int32_t* __restrict__ counters, int Hq, int Hkv, int T_max, int window,
    int fused, int q_stride) {
  __shared__ float qf[G][kD];          // rotated q (bf16 values) as fp32
  __shared__ uint4 knew[kD / 8], vnew[kD / 8];
  __shared__ float ps[G][64];          // probabilities of the current chunk
  __shared__ int is_last_s;
  const int S = gridDim.x, s = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  const int p = pos_arr[b];
  const int lo = (window > 0 && p - window + 1 > 0) ? p - window + 1 : 0;
  const int n = p - lo + 1;
  const int nch = (n + 63) >> 6;
  const int c0 = (int)((int64_t)s * nch / S), c1 = (int)((int64_t)(s + 1) * nch / S);
  const bool owns_new = fused && c0 < c1 && c1 == nch;
  const size_t kv_base = ((size_t)b * Hkv + g) * T_max;

  // ---- q (and the new k/v) into LDS -------------------------------------
  {
    const uint16_t* qrow = q_src + (size_t)b * q_stride;
    if (fused) {
      const float* cr = cos_t + (size_t)p * (kD / 2);
      const float* sr = sin_t + (size_t)p * (kD / 2);
      for (int t = lane; t < G * (kD / 2); t += 64) {
        const int hh = t / (kD / 2), f = t % (kD / 2);
        const uint16_t* qh = qrow + (size_t)(g * G + hh) * kD;
        float o1, o2;
        rope_pair(bf2f(qh[f]), bf2f(qh[f + kD / 2]), cr[f], sr[f], o1, o2);
        qf[hh][f] = bf2f(f2bf(o1));
        qf[hh][f + kD / 2] = bf2f(f2bf(o2));
      }
      if (owns_new && lane < kD / 2) {
        const uint16_t* kh = qrow + (size_t)(Hq + g) * kD;
        float o1, o2;
        rope_pair(bf2f(kh[lane]), bf2f(kh[lane + kD / 2]), cr[lane], sr[lane],
                  o1, o2);
        uint16_t* kn16 = reinterpret_cast<uint16_t*>(knew);
        kn16[lane] = f2bf(o1);
        kn16[lane + kD / 2] = f2bf(o2);
        const uint32_t* vh =
            reinterpret_cast<const uint32_t*>(qrow + (size_t)(Hq + Hkv + g) * kD);
        reinterpret_cast<uint32_t*>(vnew)[lane] = vh[lane];
      }
    } else {
      for (int t = lane; t < G * kD; t += 64) {
        const int hh = t / kD, d = t % kD;
        qf[hh][d] = bf2f(qrow[(size_t)(g * G + hh) * kD + d]);
      }
    }
    __syncthreads();
    if (owns_new && lane < kD / 8) {
      reinterpret_cast<uint4*>(kc + (kv_base + p) * kD)[lane] = knew[lane];
      reinterpret_cast<uint4*>(vc + (kv_base + p) * kD)[lane] = vnew[lane];
    }
  }

  float m[G], l[G], o[G][8];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    m[hh] = -INFINITY;
    l[hh] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[hh][e] = 0.0f;
  }
  const int kg = lane >> 3, dq = lane & 7;

  for (int c = c0; c < c1; ++c) {
    // ---- scores: lane = key -------------------------------------------
    const int j = lo + c * 64 + lane;
    const bool valid = j <= p;
    float kf[kD];
    {
      uint4 kr[kD / 8];
      if (valid) {
        if (fused && j == p) {
#pragma unroll
          for (int u = 0; u < kD / 8; ++u) kr[u] = knew[u];
        } else {
          const uint4* src = reinterpret_cast<const uint4*>(kc + (kv_base + j) * kD);
#pragma unroll
          for (int u = 0; u < kD / 8; ++u) kr[u] = src[u];
        }
      } else {
#pragma unroll
        for (int u = 0; u < kD / 8; ++u) kr[u] = make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kD / 8; ++u) unpack8(kr[u], &kf[8 * u]);
    }
    float sc[G];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      float a = 0.0f;
#pragma unroll
      for (int d = 0; d < kD; ++d) a = __builtin_fmaf(qf[hh][d], kf[d], a);
      sc[hh] = valid ? __fmul_rn(a, 0.125f) : -INFINITY;  // 1/sqrt(64), HFM:277
    }
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      const float mn = fmaxf(m[hh], wave_max(sc[hh]));
      const float alpha = neon_expf(__fsub_rn(m[hh], mn));
      const float pj = valid ? neon_expf(__fsub_rn(sc[hh], mn)) : 0.0f;
      l[hh] = __builtin_fmaf(l[hh], alpha, wave_sum(pj));
      m[hh] = mn;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[hh][e] = __fmul_rn(o[hh][e], alpha);
      ps[hh][lane] = pj;
    }
    __syncthreads();
    // ---- P.V: lane = (key group, dim octet) ---------------------------
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int jj = kg + 8 * i;
      const int jk = lo + c * 64 + jj;
      if (jk <= p) {
        uint4 v;
        if (fused && jk == p) v = vnew[dq];
        else v = reinterpret_cast<const uint4*>(vc + (kv_base + jk) * kD)[dq];
        float vf[8];
        unpack8(v, vf);
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
          const float pv = ps[hh][jj];
#pragma unroll
          for (int e = 0; e < 8; ++e) o[hh][e] = __builtin_fmaf(pv, vf[e], o[hh][e]);
        }
      }
    }
    __syncthreads();
  }
  // reduce o over the 8 key groups (lane bits 3..5)
#pragma unroll
  for (int hh = 0; hh < G; ++hh)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = o[hh][e];
      v = __fadd_rn(v, __shfl_xor(v, 8, 64));
      v = __fadd_rn(v, __shfl_xor(v, 16, 64));
      v = __fadd_rn(v, __shfl_xor(v, 32, 64));
      o[hh][e] = v;
    }

  if (S == 1) {
    if (kg == 0) {
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
        const float sk = bf2f(sinks[g * G + hh]);
        const float M = fmaxf(sk, m[hh]);
        float den = neon_expf(__fsub_rn(sk, M));
        const float f = (m[hh] == -INFINITY) ? 0.0f : neon_expf(__fsub_rn(m[hh], M));
        den = __builtin_fmaf(l[hh], f, den);
        const float inv = __fdiv_rn(1.0f, den);
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = pack_bf2(__fmul_rn(__builtin_fmaf(f, o[hh][2 * e], 0.0f), inv),
                          __fmul_rn(__builtin_fmaf(f, o[hh][2 * e + 1], 0.0f), inv));
        reinterpret_cast<uint4*>(out + (size_t)b * Hq * kD +
                                 (size_t)(g * G + hh) * kD)[dq] =
            make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
    return;
  }

  // ---- split-KV: publish the partial, the last block merges -------------
  const size_t pbase = ((size_t)b * Hkv + g) * S;
  if (kg == 0) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      float4* dst = reinterpret_cast<float4*>(part_o + ((pbase + s) * G + hh) * kD + dq * 8);
      dst[0] = make_float4(o[hh][0], o[hh][1], o[hh][2], o[hh][3]);
      dst[1] = make_float4(o[hh][4], o[hh][5], o[hh][6], o[hh][7]);
    }
  }
  if (lane < G) {
    float mv = m[0], lv = l[0];
#pragma unroll
    for (int hh = 1; hh < G; ++hh)
      if (lane == hh) { mv = m[hh]; lv = l[hh]; }
    part_ml[((pbase + s) * G + lane) * 2 + 0] = mv;
    part_ml[((pbase + s) * G + lane) * 2 + 1] = lv;
  }
  __threadfence();
  if (lane == 0) {
    const int prev = __hip_atomic_fetch_add(&counters[b * Hkv + g], 1,
                                            __ATOMIC_ACQ_REL,
                                            __HIP_MEMORY_SCOPE_AGENT);
    is_last_s = (prev == S - 1);
  }
  __syncthreads();
  if (!is_last_s) return;
  __threadfence();
  // lane -> (head hh = lane / 8, dims dq*8 .. +8)
  {
    const int hh = lane >> 3;
    if (hh < G) {
      const float sk = bf2f(sinks[g * G + hh]);
      float M = sk;
      for (int t = 0; t < S; ++t) M = fmaxf(M, part_ml[((pbase + t) * G + hh) * 2]);
      float den = neon_expf(__fsub_rn(sk, M));
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int t = 0; t < S; ++t) {
        const float mt = part_ml[((pbase + t) * G + hh) * 2];
        const float lt = part_ml[((pbase + t) * G + hh) * 2 + 1];
        const float f = (mt == -INFINITY) ? 0.0f : neon_expf(__fsub_rn(mt, M));
        den = __builtin_fmaf(lt, f, den);
        const float* src = part_o + ((pbase + t) * G + hh) * kD + dq * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(f, src[e], acc[e]);
      }
      const float inv = __fdiv_rn(1.0f, den);
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = pack_bf2(__fmul_rn(acc[2 * e], inv), __fmul_rn(acc[2 * e + 1], inv));
      reinterpret_cast<uint4*>(out + (size_t)b * Hq * kD +
                               (size_t)(g * G + hh) * kD)[dq] =
          make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  if (lane == 0)
    __hip_atomic_store(&counters[b * Hkv + g], 0, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

void launch_attn(const AttnArgs& a, hipStream_t st) {
  const int G = a.Hq / a.Hkv;
  dim3 grid(a.S, a.Hkv, a.B);
#define A_CASE(GG)                                                             \
  case GG:                                                                     \
    hipLaunchKernelGGL(k_attn_decode<GG>, grid, dim3(64), 0, st, a.q_src,      \
                       a.kc, a.vc, a.sinks, a.pos, a.cos_t, a.sin_t, a.out,    \
                       a.part_o, a.part_ml, a.counters, a.Hq, a.Hkv, a.T_max,  \
                       a.window, a.fused, a.q_stride);                         \
    break;
  switch (G) {
    A_CASE(1) A_CASE(2) A_CASE(4)
    default: A_CASE(8)
  }
#undef A_CASE
}

int attn_splits(int T_max, int window) {
  const int span = window > 0 ? (window < T_max ? window : T_max) : T_max;
  const int s = (span + 63) / 64;
  return s < 1 ? 1 : (s > 32 ? 32 : s);
}

}  // namespace neon

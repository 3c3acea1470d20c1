// neon_prefill.hip -- batched prompt processing (prefill) on gfx950.
//
// A prompt of M tokens runs every layer over all M rows at once, so the
// projections and the experts become dense contractions on the matrix cores
// (v_mfma_f32_32x32x16_bf16, fp32 accumulate):
//   - bf16 GEMM  C[M][N] = A[M][K] W[N][K]^T (QKV, O + residual, router);
//   - grouped MXFP4 GEMM over the tokens routed to each expert, with the
//     expert rows dequantised exactly to bf16 in LDS (E2M1 x 2^(s-127) is a
//     bf16 value), SwiGLU fused into the gate_up epilogue;
//   - tiled causal sink attention over the KV cache the prefill fills, on
//     the matrix cores as well (S^T = K Q^T, O^T += V^T P^T).
// The maths is the decode path's (HFM:82-112, 235-263, 347-376); the
// accumulation order of a matrix-core dot product differs from the decode
// kernels' canonical fp32 chain, so prefill agrees with it within fp32
// rounding, not bit for bit.
#include "neon_common.hpp"
#include "neon_internal.hpp"

#include <cstdlib>

namespace neon {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));  // staging (no struct copies)
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ void unpack8(const uint4& v, float* o) {
  o[0] = bf_lo(v.x); o[1] = bf_hi(v.x); o[2] = bf_lo(v.y); o[3] = bf_hi(v.y);
  o[4] = bf_lo(v.z); o[5] = bf_hi(v.z); o[6] = bf_lo(v.w); o[7] = bf_hi(v.w);
}

// ===========================================================================
// Row gather: h[t] = embed[ids[t]]
// ===========================================================================
__global__ void k_embed_rows(const int32_t* __restrict__ ids,
                             const uint16_t* __restrict__ embed,
                             uint16_t* __restrict__ h, int H) {
  const int t = blockIdx.x;
  const uint4* src = reinterpret_cast<const uint4*>(embed + (size_t)ids[t] * H);
  uint4* dst = reinterpret_cast<uint4*>(h + (size_t)t * H);
  for (int u = threadIdx.x; u < H / 8; u += blockDim.x) dst[u] = src[u];
}

void launch_embed_rows(const int32_t* ids, int M, const uint16_t* embed,
                       uint16_t* h, int H, hipStream_t st) {
  hipLaunchKernelGGL(k_embed_rows, dim3(M), dim3(256), 0, st, ids, embed, h, H);
}

// ===========================================================================
// Matrix-core GEMM.  Block tile 128 x 128, K step 64, 4 waves in 2 x 2, each
// wave a 64 x 64 tile of 2 x 2 MFMA 32x32x16 blocks.  Both operands are
// "row of the matrix, 8 consecutive k" per lane (lane l: row l % 32, k
// 8 (l / 32) .. + 8), so A [M][K] and W [N][K] are staged the same way:
// global -> registers (next step) -> LDS (double buffer, row stride 40 bf16
// so rows spread over the banks) -> ds_read_b128 operands.
//
// Rows past M or N read a clamped valid row and are never stored.  K must be
// a multiple of 32; when it is not one of 64, the last step's upper 32
// elements are zeros (a zero A value and a zero code add nothing).  With FP4,
// W is an MXFP4 matrix (codes [N][K/2], scales [N][K/32]); a thread stages
// one scale block (32 values) of one row per step, dequantised as
// E2M1 (v_cvt_scalef32_pk_f32_fp4, exact) x 2^(s-127) (ldexp, exact) and
// rounded to bf16 (exact: every such value is a bf16 value or overflows).
//
// Grouped (MoE) form: blockIdx.y is a tile of the expert-sorted row list;
// tile_e / tile_r0 give its expert and first list row, and rows past the
// expert's count are masked.  The A row of list row i is a_rows[i] (token)
// when a_rows is given, else i itself.
// ===========================================================================
constexpr int kGM = 128, kGN = 128, kGK = 64, kGS = 72;  // tile, LDS row stride

constexpr int kNarrowMaxN = 64;   // k_gemm_narrow_f32: columns per launch (4 tiles)
constexpr int kNarrowBatch = 6;   // its K chunks per wave loaded before their MFMAs
enum {
  GEMM_STORE = 0,    // C = bf16(acc + bias)
  GEMM_RESID = 1,    // C = bf16(C + bf16(acc + bias))  (C holds the residual)
  GEMM_F32 = 2,      // Cf = acc + bias
  GEMM_SWIGLU = 3,   // act[i][j] = bf16(swiglu(acc_2j + b_2j, acc_2j+1 + b_2j+1))
  GEMM_SCATTER = 4   // ybuf[token][slot][n] = acc + bias (fp32)
};

struct GemmParams {
  const uint16_t* A; int lda;
  const uint16_t* W; int ldw;          // bf16 weights [N][K]
  const uint8_t* codes;                // MXFP4 weights (FP4): [E][N][K/2]
  const uint8_t* scales;               // [E][N][K/32]
  const uint16_t* bias;                // [E][N] (grouped) or [N]; may be NULL
  uint16_t* C; float* Cf; int ldc;
  int M, N, K;
  // grouped form
  const int32_t* tile_e; const int32_t* tile_r0; const int32_t* n_tiles;
  const int32_t* e_off;                // [E+1] list offsets
  const int32_t* list_tok; const int32_t* list_slot;
  const int32_t* a_rows;               // token of each list row (gate_up), or NULL
  float* ybuf; int topk;
  float alpha, limit;
  // MXFP8 A operand (k_gemm_mx8), in step lines: per row and 64-element
  // step 128 bytes (64 E4M3 hi, 64 lo) and one scale dword (s_hi of the two
  // 32-blocks, then s_lo); a row's scale dwords are mx8_scale_stride(K)
  // apart (a multiple of 4, so 4 steps' scales are one aligned 16 bytes)
  const uint8_t* qa; const uint32_t* qsc;
};

__device__ __forceinline__ float swiglu_clamp_p(float g, float u, float alpha, float limit) {
  g = g > limit ? limit : g;
  u = u > limit ? limit : (u < -limit ? -limit : u);
  const float e = neon_expf(-__fmul_rn(g, alpha));
  const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, e));
  return __fmul_rn(__fadd_rn(u, 1.0f), __fmul_rn(g, sig));
}

// 16 E2M1 values of 8 code bytes, times 2^(s - 127), as 16 bf16 (two uint4)
__device__ __forceinline__ void fp4x16_to_bf16(u32x2_t c, uint32_t s, u32x4_t& lo, u32x4_t& hi) {
  const int ex = (int)s - 127;
  const bool nan = s == 0xFFu;
  uint32_t o[8];
  const uint32_t w[2] = {c.x, c.y};
#pragma unroll
  for (int q = 0; q < 2; ++q) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      float2_v v;
      switch (b) {
        case 0: v = fp4x2_to_f32<0>(w[q]); break;
        case 1: v = fp4x2_to_f32<1>(w[q]); break;
        case 2: v = fp4x2_to_f32<2>(w[q]); break;
        default: v = fp4x2_to_f32<3>(w[q]); break;
      }
      float a = __builtin_amdgcn_ldexpf(v.x, ex), bb = __builtin_amdgcn_ldexpf(v.y, ex);
      a = nan ? __builtin_nanf("") : a;
      bb = nan ? __builtin_nanf("") : bb;
      o[q * 4 + b] = pack_bf2(a, bb);
    }
  }
  lo = u32x4_t{o[0], o[1], o[2], o[3]};
  hi = u32x4_t{o[4], o[5], o[6], o[7]};
}

// What the epilogue of a 128 x 128 tile reads besides the accumulators,
// fetched when the block starts (gemm_epi_issue) so that the epilogue does
// not wait on dependent loads one 32 x 32 block at a time (measured: 15 of
// the 61 us a gate_up block of the MXFP8 expert GEMM lived): the lane's two
// column biases, and for the scatter epilogue the (token, slot) of every row
// of the tile (thread t < kGM holds row t's; gemm_epi_stage puts them in LDS
// after the K loop).
struct GemmEpi {
  float bcol[2];
  uint32_t tok, slot;  // scatter: row threadIdx.x's (token, slot), threads < kGM
};
struct GemmEpiLds {
  int32_t tok[kGM], slot[kGM];
};

template <int MODE, bool GROUPED>
__device__ __forceinline__ void gemm_epi_issue(const GemmParams& p, int lane, int wn, int n0,
                                               int r0, int rows, int e, GemmEpi& ep,
                                               GemmEpiLds& el) {
  const uint16_t* bias = p.bias ? p.bias + (GROUPED ? (size_t)e * p.N : 0) : nullptr;
#pragma unroll
  for (int in = 0; in < 2; ++in) {
    const int col = n0 + wn * 64 + in * 32 + (lane & 31);
    // unconditional (clamped; the weights when there is no bias): a load under
    // a branch is waited for where the branches join, before the operands
    const uint16_t bq = load_pinned_u16(
        bias ? bias + min(col, p.N - 1)
             : (GROUPED ? reinterpret_cast<const uint16_t*>(p.codes) : p.W));
    ep.bcol[in] = (bias && col < p.N) ? bf2f(bq) : 0.0f;
  }
  if (MODE == GEMM_SCATTER) {  // every thread loads (threads >= kGM repeat row kGM - 1)
    const size_t gr = (size_t)r0 + min(min((int)threadIdx.x, kGM - 1), rows - 1);
    ep.tok = load_pinned_u32(reinterpret_cast<const uint32_t*>(p.list_tok + gr));
    ep.slot = load_pinned_u32(reinterpret_cast<const uint32_t*>(p.list_slot + gr));
  }
}

// After the K loop: the scatter rows' (token, slot) into LDS for the epilogue.
template <int MODE>
__device__ __forceinline__ void gemm_epi_stage(const GemmEpi& ep, GemmEpiLds& el) {
  if (MODE != GEMM_SCATTER) return;
  if (threadIdx.x < kGM) {
    el.tok[threadIdx.x] = (int32_t)ep.tok;
    el.slot[threadIdx.x] = (int32_t)ep.slot;
  }
  __syncthreads();
}

// Epilogue of the 128 x 128 GEMM tiles (both operand kinds): acc[im][in][i]
// is row 8 (i/4) + 4 (lane/32) + i%4, column lane%32 of the wave's 32 x 32
// block (im, in) -- the D layout of the 32 x 32 MFMA shapes.  el was written
// by gemm_epi_stage.
template <int MODE, bool GROUPED>
__device__ __forceinline__ void gemm_epilogue(const f32x16_t (&acc)[2][2], const GemmParams& p,
                                              int lane, int wm, int wn, int n0, int r0,
                                              int rows, const GemmEpi& ep,
                                              const GemmEpiLds& el) {
  const bool has_bias = p.bias != nullptr;
#pragma unroll
  for (int im = 0; im < 2; ++im)
#pragma unroll
    for (int in = 0; in < 2; ++in) {
      const int col = n0 + wn * 64 + in * 32 + (lane & 31);
      const float bcol = ep.bcol[in];
      if constexpr (MODE == GEMM_SWIGLU) {
        // gate (even column) and up (odd column) sit in adjacent lanes, and
        // values i, i + 1 are rows r, r + 1: the even lane keeps row r's
        // gate and receives its up, the odd lane keeps row r + 1's up and
        // receives its gate, so every lane forms one SwiGLU per two values
        const bool odd = (lane & 1) != 0;
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const int r = wm * 64 + im * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3) + (odd ? 1 : 0);
          const float v0 = has_bias ? __fadd_rn(acc[im][in][i], bcol) : acc[im][in][i];
          const float v1 = has_bias ? __fadd_rn(acc[im][in][i + 1], bcol) : acc[im][in][i + 1];
          const float got = __shfl_xor(odd ? v0 : v1, 1, 64);
          const float gate = odd ? got : v0, up = odd ? v1 : got;
          if (r < rows && (col | 1) < p.N)
            p.C[(size_t)(r0 + r) * p.ldc + col / 2] = f2bf(swiglu_clamp_p(gate, up, p.alpha, p.limit));
        }
        continue;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = wm * 64 + im * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        const float v = has_bias ? __fadd_rn(acc[im][in][i], bcol) : acc[im][in][i];
        if (r >= rows || col >= p.N) continue;
        const size_t gr = (size_t)(r0 + r);
        if (MODE == GEMM_STORE) {
          p.C[gr * p.ldc + col] = f2bf(v);
        } else if (MODE == GEMM_RESID) {
          uint16_t* c = p.C + gr * p.ldc + col;
          *c = f2bf(__fadd_rn(bf2f(*c), bf2f(f2bf(v))));
        } else if (MODE == GEMM_F32) {
          p.Cf[gr * p.ldc + col] = v;
        } else {  // GEMM_SCATTER
          const int t = el.tok[r], sl = el.slot[r];
          p.ybuf[((size_t)t * p.topk + sl) * p.N + col] = v;
        }
      }
    }
}

template <int MODE, bool FP4, bool GROUPED>
__global__ __launch_bounds__(256) void k_gemm(GemmParams p) {
  __shared__ __align__(16) uint16_t As[2][kGM * kGS];
  __shared__ __align__(16) uint16_t Ws[2][kGN * kGS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = blockIdx.x * kGN;
  int e = 0, r0, rows;  // rows: valid A rows of this tile (from r0)
  if (GROUPED) {
    if ((int)blockIdx.y >= *p.n_tiles) return;  // uniform for the block
    e = p.tile_e[blockIdx.y];
    const int lo = p.e_off[e];
    r0 = lo + p.tile_r0[blockIdx.y];
    rows = min(kGM, p.e_off[e + 1] - r0);
  } else {
    r0 = blockIdx.y * kGM;
    rows = min(kGM, p.M - r0);
  }
  const int K = p.K;
  __shared__ GemmEpiLds epl;
  GemmEpi ep;
  gemm_epi_issue<MODE, GROUPED>(p, lane, wn, n0, r0, rows, e, ep, epl);
  // this thread's staging rows: A/W chunk c = tid + 256 i (i = 0, 1):
  // row c >> 2, k (c & 3) * 8; FP4 W: row tid >> 1, k half (tid & 1) * 16
  // staging: thread tid copies the 8-element piece (tid & 7) of rows
  // (tid + 256 i) >> 3, i = 0..3 (128 rows x 64 elements per step)
  const int pc = (tid & 7) * 8;
  const uint16_t* arow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (tid + 256 * i) >> 3;
    const int lr = r0 + min(r, rows - 1);
    const int ar = GROUPED && p.a_rows ? p.a_rows[lr] : lr;
    arow[i] = p.A + (size_t)ar * p.lda + pc;
  }
  const uint16_t* wrow[4] = {nullptr, nullptr, nullptr, nullptr};
  const uint8_t* crow = nullptr;
  const uint8_t* srow = nullptr;
  const int half = tid & 1;  // FP4: which scale block (32 values) of the step
  if (FP4) {
    const int r = tid >> 1;
    const size_t nr = (size_t)e * p.N + min(n0 + r, p.N - 1);
    crow = p.codes + nr * (K / 2) + half * 16;
    srow = p.scales + nr * (K / 32) + half;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (tid + 256 * i) >> 3;
      wrow[i] = p.W + (size_t)min(n0 + r, p.N - 1) * p.ldw + pc;
    }
  }
  const u32x4_t z4 = {0u, 0u, 0u, 0u};
  u32x4_t ra[4], rw[4] = {z4, z4, z4, z4};
  u32x4_t rc = z4;
  uint32_t rs = 127;
  // the loads of the step at element ko; pieces past K are zeros
  auto load_step = [&](int ko) {
    const bool aok = ko + pc < K;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ra[i] = aok ? *reinterpret_cast<const u32x4_t*>(arow[i] + ko) : z4;
    if (FP4) {
      const bool cok = ko + 32 * half < K;
      rc = cok ? *reinterpret_cast<const u32x4_t*>(crow + ko / 2) : z4;
      rs = cok ? srow[ko / 32] : 127u;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        rw[i] = aok ? *reinterpret_cast<const u32x4_t*>(wrow[i] + ko) : z4;
    }
  };
  load_step(0);
  f32x16_t acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

  const int nk = (K + kGK - 1) / kGK;
  // registers -> LDS buffer `buf`
#define GEMM_STAGE(buf)                                                                 \
  do {                                                                                  \
    for (int i = 0; i < 4; ++i)                                                         \
      *reinterpret_cast<u32x4_t*>(&As[buf][((tid + 256 * i) >> 3) * kGS + pc]) = ra[i]; \
    if (FP4) {                                                                          \
      u32x4_t lo, hi;                                                                   \
      uint16_t* d = &Ws[buf][(tid >> 1) * kGS + half * 32];                             \
      fp4x16_to_bf16(u32x2_t{rc.x, rc.y}, rs, lo, hi);                                  \
      *reinterpret_cast<u32x4_t*>(d) = lo;                                              \
      *reinterpret_cast<u32x4_t*>(d + 8) = hi;                                          \
      fp4x16_to_bf16(u32x2_t{rc.z, rc.w}, rs, lo, hi);                                  \
      *reinterpret_cast<u32x4_t*>(d + 16) = lo;                                         \
      *reinterpret_cast<u32x4_t*>(d + 24) = hi;                                         \
    } else {                                                                            \
      for (int i = 0; i < 4; ++i)                                                       \
        *reinterpret_cast<u32x4_t*>(&Ws[buf][((tid + 256 * i) >> 3) * kGS + pc]) = rw[i]; \
    }                                                                                   \
  } while (0)
  GEMM_STAGE(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_step((kt + 1) * kGK);  // next step's loads before this step's math
#pragma unroll
    for (int ks = 0; ks < kGK / 16; ++ks) {
      bf16x8_t af[2], bf[2];
#pragma unroll
      for (int im = 0; im < 2; ++im)
        af[im] = *reinterpret_cast<const bf16x8_t*>(
            &As[cur][(wm * 64 + im * 32 + (lane & 31)) * kGS + ks * 16 + 8 * (lane >> 5)]);
#pragma unroll
      for (int in = 0; in < 2; ++in)
        bf[in] = *reinterpret_cast<const bf16x8_t*>(
            &Ws[cur][(wn * 64 + in * 32 + (lane & 31)) * kGS + ks * 16 + 8 * (lane >> 5)]);
#pragma unroll
      for (int im = 0; im < 2; ++im)
#pragma unroll
        for (int in = 0; in < 2; ++in)
          acc[im][in] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[im], bf[in], acc[im][in], 0, 0, 0);
    }
    if (kt + 1 < nk) GEMM_STAGE(cur ^ 1);
    __syncthreads();
  }
#undef GEMM_STAGE

  gemm_epi_stage<MODE>(ep, epl);
  gemm_epilogue<MODE, GROUPED>(acc, p, lane, wm, wn, n0, r0, rows, ep, epl);
}

// ===========================================================================
// MXFP8 activations x MXFP4 experts on the scaled matrix instruction
// (v_mfma_scale_f32_32x32x64_f8f6f4: A E4M3, B E2M1, one E8M0 scale per
// 32-element block of each operand, fp32 accumulate).
//
// Activation quantisation (k_mx8_quant): each 32-element block of a bf16
// row becomes two MXFP8 terms, hi = the OCP MX rule (shared exponent
// floor(log2 amax) - 8, one more when amax's significand exceeds 1.75 so
// nothing saturates; round to nearest even) and lo = the same rule on the
// exact fp32 residual x - hi.  Together they carry the bf16 value to within
// 2^(floor(log2 amax) - 8), half a bf16 unit of the block maximum, so the
// expert GEMM runs two instructions per 64-deep step (A_hi B, A_lo B) into
// one accumulator.  The CPU oracle's or_mx8_quant states the same rule and
// this kernel matches it bit for bit.
//
// Operand lanes of the 32x32x64 shape, measured on gfx950 with an in-bounds
// probe (random E4M3 / E2M1 data and scales, exact fp32 match):
//   - B (E2M1, 16 bytes in the first 4 VGPRs): lane n + 32 h holds column n,
//     k 32 h .. 32 h + 31, low nibble first -- exactly one stored MXFP4 block
//     of a weight row, so the expert rows are read straight from memory;
//   - A (E4M3, 32 bytes): lane i + 32 h holds row i, bytes 0-15 = k 16 h ..
//     16 h + 15 and bytes 16-31 = k 32 + 16 h .. 32 + 16 h + 15;
//   - scales: the scale of (row / column i, k block b) is byte 0 of lane
//     i + 32 b's scale operand;
//   - D: as the other 32x32 shapes (row 8 (r/4) + 4 (lane/32) + r%4,
//     column lane%32).
// ===========================================================================
// Four lanes per 32-element block (8 elements each; the block maxima by a
// quad exchange): rows x K/32 x 4 threads.  LINES: hi / lo into step lines
// (hi = the lines, K % 64 == 0; block b of a row goes to line b / 2 at bytes
// 32 (b % 2) (hi) and 64 + 32 (b % 2) (lo), its scale bytes to bytes b % 2
// and 2 + b % 2 of the step's dword in s_hi, the row's dwords
// mx8_scale_stride(K) apart, the padding dwords never written); else the
// four arrays of the kernel-level layout.
template <bool LINES>
__global__ __launch_bounds__(256) void k_mx8_quant(const uint16_t* __restrict__ x, int64_t n_blocks,
                                                   int K, uint8_t* __restrict__ hi,
                                                   uint8_t* __restrict__ lo,
                                                   uint8_t* __restrict__ s_hi,
                                                   uint8_t* __restrict__ s_lo) {
  const int64_t tq = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int q = (int)(tq & 3);
  const bool on = (tq >> 2) < n_blocks;  // the same for the 4 lanes of a block
  const int64_t t = on ? (tq >> 2) : n_blocks - 1;  // past the end: lanes stay for the exchange
  const int nb = K / 32;
  const int64_t r = t / nb, blk = t - r * nb;
  const int64_t o = r * K + blk * 32 + 8 * q;
  float v[8];
  unpack8(*reinterpret_cast<const uint4*>(x + o), v);
  uint32_t qh[2], ql[2], b1, b2;
  mx8_quant8(v, qh, ql, b1, b2);
  if (!on) return;
  uint2 *dh, *dl;
  if (LINES) {
    const int64_t line = r * (K / 64) + (blk >> 1);
    const int64_t sline = r * mx8_scale_stride(K) + (blk >> 1);
    const int half = (int)(blk & 1);
    dh = reinterpret_cast<uint2*>(hi + line * 128 + 32 * half + 8 * q);
    dl = reinterpret_cast<uint2*>(hi + line * 128 + 64 + 32 * half + 8 * q);
    if (q == 0) {
      s_hi[sline * 4 + half] = (uint8_t)b1;
      s_hi[sline * 4 + 2 + half] = (uint8_t)b2;
    }
  } else {
    dh = reinterpret_cast<uint2*>(hi + o);
    dl = reinterpret_cast<uint2*>(lo + o);
    if (q == 0) {
      s_hi[t] = (uint8_t)b1;
      s_lo[t] = (uint8_t)b2;
    }
  }
  *dh = make_uint2(qh[0], qh[1]);
  *dl = make_uint2(ql[0], ql[1]);
}

void launch_mx8_quant(const uint16_t* x, int64_t rows, int K, uint8_t* hi, uint8_t* lo,
                      uint8_t* s_hi, uint8_t* s_lo, hipStream_t st) {
  const int64_t n = rows * (K / 32);
  if (n <= 0) return;
  hipLaunchKernelGGL(k_mx8_quant<false>, dim3((unsigned)((4 * n + 255) / 256)), dim3(256), 0, st,
                     x, n, K, hi, lo, s_hi, s_lo);
}

void launch_mx8_quant_lines(const uint16_t* x, int64_t rows, int K, uint8_t* q, uint32_t* qs,
                            hipStream_t st) {
  const int64_t n = rows * (K / 32);
  if (n <= 0) return;
  hipLaunchKernelGGL(k_mx8_quant<true>, dim3((unsigned)((4 * n + 255) / 256)), dim3(256), 0, st,
                     x, n, K, q, nullptr, reinterpret_cast<uint8_t*>(qs), nullptr);
}

// Grouped expert GEMM on the scaled matrix instruction.  What bounds this
// shape is operand fetch (the matrix units idle most of the time
// otherwise), so every global fetch uses whole 128-byte lines:
//   - A (the two MXFP8 terms of the input rows, step-line layout: one line
//     per row and 64-deep step) is staged through LDS a step at a time
//     (row stride kQS = 64 hi + 64 lo + 16 padding, two buffers), fetched
//     kRingA - 1 steps ahead through a register ring;
//   - B (the expert's MXFP4 rows as stored) is staged through LDS a group
//     of kPipe steps (128 bytes of each row) at a time, fetched a group
//     ahead (two buffers, column stride kQS), with its scale bytes.
// Same tiles, grouping and epilogues as k_gemm<MODE, true, true>.
// K % 64 == 0.
__device__ __forceinline__ int h_of(int lane) { return lane >> 5; }
constexpr int kQS = 144;
constexpr int kPipe = 4;   // B steps per group
constexpr int kRingA = 4;  // A register sets (A runs kRingA - 1 steps ahead)

// Block -> (expert tile, column block) map of the expert GEMMs.  Blocks are
// handed to the 8 XCDs round-robin in linear id order (id = x + gridDim.x y),
// and each XCD has its own L2, so linear id P runs logical block
// L = (P mod 8) per + P / 8: each XCD takes one contiguous range of logical
// blocks.  Logical blocks go expert by expert, and within an expert column
// block by column block over the expert's row tiles, so an XCD holds the A
// rows of about one expert at a time and each weight column block is read by
// the expert's tiles back to back (measured at the 2048-token 20b shape:
// gate_up 471 -> 453 us).  The grid has at least 8 per blocks (mx8_grid adds
// the rows for it); blocks past the work exit.
__device__ __forceinline__ bool mx8_block_map(const GemmParams& p, int& n0, int& e, int& r0,
                                              int& rows) {
  const int NB = gridDim.x;
  const int total = NB * *p.n_tiles;
  const int per = (total + 7) >> 3;
  const int P = blockIdx.y * NB + blockIdx.x;
  const int L = (P & 7) * per + (P >> 3);
  if ((P >> 3) >= per || L >= total) return false;
  const int T = L / NB;                       // a tile of the block's expert
  e = p.tile_e[T];
  const int tb = T - p.tile_r0[T] / kGM;      // the expert's first tile
  const int lo = p.e_off[e], hi = p.e_off[e + 1];
  const int ne = (hi - lo + kGM - 1) / kGM;   // the expert's tiles
  const int li = L - tb * NB;                 // the block's index within the expert
  n0 = (li / ne) * kGN;
  r0 = lo + (li % ne) * kGM;
  rows = min(kGM, hi - r0);
  return true;
}

// grid of k_gemm_mx8 for N output columns and at most max_tiles row tiles:
// 8 ceil(NB max_tiles / 8) <= NB max_tiles + 7 blocks must exist
static dim3 mx8_grid(int N, int max_tiles) {
  const int NB = (N + kGN - 1) / kGN;
  return dim3(NB, max_tiles + (7 + NB - 1) / NB);
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void k_gemm_mx8(GemmParams p) {
  __shared__ __align__(16) uint8_t Aq[2][kGM * kQS];
  __shared__ uint32_t Asc[2][kGM];              // per row: s_hi b0, s_hi b1, s_lo b0, s_lo b1
  __shared__ __align__(16) uint8_t Bq[2][kGN * kQS];   // per column: kPipe steps x 32 B
  __shared__ uint16_t Bsc[2][kGN * kPipe];       // per column and step: the 2 blocks' scales
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int n0, e, r0, rows;
  if (!mx8_block_map(p, n0, e, r0, rows)) return;  // uniform for the block
  __shared__ GemmEpiLds epl;
  GemmEpi ep;
  gemm_epi_issue<MODE, true>(p, lane, wn, n0, r0, rows, e, ep, epl);
  const int K = p.K, KB = K / 32, KS = K / 64;
  const int nk = KS;
  // staging map shared by A and B: piece c = tid + 256 i (i = 0..3) is row /
  // column c >> 3, 16-byte piece c & 7 of its 128 bytes
  const int pc = tid & 7;
  const uint8_t* asrc[4];
  const uint8_t* bsrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (tid + 256 * i) >> 3;
    const int lr = r0 + min(r, rows - 1);
    const int ar = p.a_rows ? p.a_rows[lr] : lr;
    asrc[i] = p.qa + (size_t)ar * KS * 128 + 16 * pc;
    bsrc[i] = p.codes + ((size_t)e * p.N + min(n0 + r, p.N - 1)) * (K / 2) + 16 * (pc & 1);
  }
  // A scales: every thread fetches row (tid & 127)'s 4 dwords of a group
  // of kPipe steps (one 16-byte load per group: a dword load per step, each
  // lane on another row, costs the address unit 64 lines per instruction;
  // measured at the 2048-token 20b shape: gate_up 453 -> 445 us, down
  // 229 -> 212 us, the same bits); threads
  // < 128 stage the step's dword (one load per thread keeps every wave's load
  // count equal)
  const uint32_t* ssrc;
  {
    const int lr = r0 + min(tid & 127, rows - 1);
    const int ar = p.a_rows ? p.a_rows[lr] : lr;
    ssrc = p.qsc + (size_t)ar * mx8_scale_stride(K);
  }
  const int ng = (nk + kPipe - 1) / kPipe;  // groups
  // B scales: thread tid fetches column (tid & 127)'s two blocks of steps
  // 2 (tid >> 7) and 2 (tid >> 7) + 1 of a group
  const uint8_t* bssrc = p.scales + ((size_t)e * p.N + min(n0 + (tid & 127), p.N - 1)) * KB;
  const int bsj = 2 * (tid >> 7);
  u32x4_t ra[kRingA][4];
  u32x4_t rsg_cur, rsg_next;  // A scales of this group and the next
  u32x4_t rbq[4];
  uint32_t rbs[2];
  f32x16_t acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;
  // Every load is unconditional (steps past the end re-read the last one and
  // are never used), so each iteration issues the same loads and the wait
  // before a step's first use counts only the loads issued after it.
#define MX8_LOAD_A(u, kt)                                                            \
  do {                                                                               \
    for (int i = 0; i < 4; ++i)                                                      \
      ra[u][i] = *reinterpret_cast<const u32x4_t*>(asrc[i] + (size_t)(kt) * 128);    \
  } while (0)
  // group g of B: piece pc of each column is step g kPipe + pc / 2, half pc % 2
#define MX8_LOAD_B(g)                                                                \
  do {                                                                               \
    const int st = min((g) * kPipe + (pc >> 1), nk - 1);                             \
    for (int i = 0; i < 4; ++i)                                                      \
      rbq[i] = *reinterpret_cast<const u32x4_t*>(bsrc[i] + (size_t)st * 32);         \
    for (int j = 0; j < 2; ++j) {                                                    \
      const int sj = min((g) * kPipe + bsj + j, nk - 1);                             \
      rbs[j] = *reinterpret_cast<const uint16_t*>(bssrc + 2 * sj);                   \
    }                                                                                \
  } while (0)
#define MX8_STAGE_A(u, buf, sv)                                                      \
  do {                                                                               \
    for (int i = 0; i < 4; ++i) {                                                    \
      const int r = (tid + 256 * i) >> 3;                                            \
      *reinterpret_cast<u32x4_t*>(&Aq[buf][r * kQS + 16 * pc]) = ra[u][i];           \
    }                                                                                \
    if (tid < kGM) Asc[buf][tid] = (sv);                                             \
  } while (0)
#define MX8_STAGE_B(buf)                                                             \
  do {                                                                               \
    for (int i = 0; i < 4; ++i) {                                                    \
      const int c = (tid + 256 * i) >> 3;                                            \
      *reinterpret_cast<u32x4_t*>(&Bq[buf][c * kQS + 16 * pc]) = rbq[i];             \
    }                                                                                \
    for (int j = 0; j < 2; ++j) Bsc[buf][(tid & 127) * kPipe + bsj + j] = (uint16_t)rbs[j]; \
  } while (0)
#pragma unroll
  for (int u = 0; u < kRingA; ++u) MX8_LOAD_A(u, min(u, nk - 1));
  MX8_LOAD_B(0);
  rsg_cur = *reinterpret_cast<const u32x4_t*>(ssrc);
  rsg_next = rsg_cur;
  MX8_STAGE_A(0, 0, rsg_cur.x);
  MX8_STAGE_B(0);
  __syncthreads();
  static_assert(kPipe % kRingA == 0 || kRingA % kPipe == 0, "ring and group must nest");
  static_assert(kPipe == 4, "a group's A scales are one 16-byte load");
  for (int kt0 = 0; kt0 < nk; kt0 += kPipe) {
    const int gb = (kt0 / kPipe) & 1;
    MX8_LOAD_B(kt0 / kPipe + 1);  // the next group, staged at this group's end
    if (kt0 > 0) rsg_cur = rsg_next;
    rsg_next = *reinterpret_cast<const u32x4_t*>(ssrc + 4 * min(kt0 / kPipe + 1, ng - 1));
#pragma unroll
    for (int u = 0; u < kPipe; ++u) {
      const int kt = kt0 + u;
      const int cur = kt & 1;
      const int ua = u % kRingA;
      // A of step kt + kRingA into the set staged at the end of the last step
      MX8_LOAD_A(ua, min(kt + kRingA, nk - 1));
      __builtin_amdgcn_sched_barrier(0);
      if (kt < nk) {  // uniform for the block
        // all operands first, then the four independent hi products, then
        // the lo ones (each lo MFMA is four instructions behind the hi one
        // that wrote its accumulator)
        i32x8_t ahi[2], alo[2], bq[2];
        int sa_hi[2], sa_lo[2], s_b[2];
#pragma unroll
        for (int im = 0; im < 2; ++im) {
          const int rr = wm * 64 + im * 32 + (lane & 31);
          const uint8_t* base = &Aq[cur][rr * kQS + 16 * h_of(lane)];
          const u32x4_t h0 = *reinterpret_cast<const u32x4_t*>(base);
          const u32x4_t h1 = *reinterpret_cast<const u32x4_t*>(base + 32);
          const u32x4_t l0 = *reinterpret_cast<const u32x4_t*>(base + 64);
          const u32x4_t l1 = *reinterpret_cast<const u32x4_t*>(base + 96);
          const uint32_t sc = Asc[cur][rr];
          sa_hi[im] = (int)((sc >> (8 * h_of(lane))) & 0xFFu);
          sa_lo[im] = (int)((sc >> (16 + 8 * h_of(lane))) & 0xFFu);
          ahi[im] = i32x8_t{(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w,
                            (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
          alo[im] = i32x8_t{(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w,
                            (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
        }
#pragma unroll
        for (int in = 0; in < 2; ++in) {
          const int cn = wn * 64 + in * 32 + (lane & 31);
          const u32x4_t b4 =
              *reinterpret_cast<const u32x4_t*>(&Bq[gb][cn * kQS + u * 32 + 16 * h_of(lane)]);
          bq[in] = i32x8_t{(int)b4.x, (int)b4.y, (int)b4.z, (int)b4.w, 0, 0, 0, 0};
          s_b[in] = (int)((Bsc[gb][cn * kPipe + u] >> (8 * h_of(lane))) & 0xFFu);
        }
#pragma unroll
        for (int im = 0; im < 2; ++im)
#pragma unroll
          for (int in = 0; in < 2; ++in)
            acc[im][in] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                ahi[im], bq[in], acc[im][in], 0, 4, 0, sa_hi[im], 0, s_b[in]);
#pragma unroll
        for (int im = 0; im < 2; ++im)
#pragma unroll
          for (int in = 0; in < 2; ++in)
            acc[im][in] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                alo[im], bq[in], acc[im][in], 0, 4, 0, sa_lo[im], 0, s_b[in]);
      }
      // A of step kt + 1 (fetched kRingA - 1 steps ago) into the other buffer
      // (past the last step it is never read); at the group's last step, the
      // next group of B (fetched at the group's start)
      MX8_STAGE_A((ua + 1) % kRingA, cur ^ 1,
                  u == 0 ? rsg_cur.y : u == 1 ? rsg_cur.z : u == 2 ? rsg_cur.w : rsg_next.x);
      if (u == kPipe - 1) MX8_STAGE_B(gb ^ 1);
      __syncthreads();
    }
  }
#undef MX8_LOAD_A
#undef MX8_LOAD_B
#undef MX8_STAGE_A
#undef MX8_STAGE_B
  gemm_epi_stage<MODE>(ep, epl);
  gemm_epilogue<MODE, true>(acc, p, lane, wm, wn, n0, r0, rows, ep, epl);
}

static void launch_gemm_narrow_f32(const uint16_t* A, const uint16_t* W, const uint16_t* bias,
                                   float* C, int M, int N, int K, hipStream_t st);

// ===========================================================================
// Dense bf16 GEMM of the prompt projections, C[M][N] = A[M][K] W[N][K]^T
// (+ bias; STORE, RESID or F32 epilogue as k_gemm), K a multiple of BK.
//
// Block tile BM x 32 NB, WM x WN waves (8: two per SIMD): wave (wm, wn)
// owns IM 32-row blocks and JN 32-column blocks, so each A fragment feeds
// JN MFMAs and each W fragment IM (v_mfma_f32_32x32x16_bf16).  The tiles
// reach LDS by direct global -> LDS loads (global_load_lds_dwordx4: no
// register staging, no ds_write): one load instruction fills 64 consecutive
// 16-byte LDS units, RPI rows x CH chunks of BK / 8 elements, lane l writing
// row l / CH, slot l % CH of its rows; the lane fetches chunk slot ^ swz(row)
// of its row, so chunk c of row r sits at slot c ^ swz(r) and the rows of a
// fragment read fall on different banks (no bank conflicts measured).  As
// many stages of BK as fit in LDS (NS); NS - 1 are in flight while one is
// multiplied, one barrier per stage, the next 16-deep step's fragments read
// while the current one's MFMAs run.  Blocks are renumbered so that each XCD
// takes whole weight-column tiles.  The STORE / RESID epilogue goes through
// an LDS copy of the tile, so C is read and written in 16-byte row pieces.
// Rows past M / N read a clamped valid row and are never stored.
// ===========================================================================
template <int BM_, int NB, int BK_, int WM_, int WN_>
struct GemmLdsCfg {
  static constexpr int BM = BM_, BN = 32 * NB, BK = BK_;
  // waves WM x WN: wave (wm, wn) owns IM 32-row blocks from 32 IM wm and JN
  // 32-column blocks from 32 JN wn
  static constexpr int WM = WM_, WN = WN_, WAVES = WM * WN;
  static constexpr int IM = BM / 32 / WM, JN = NB / WN;
  static constexpr int CH = BK / 8;                 // 16-byte chunks per row piece
  static constexpr int RPI = 64 / CH;               // rows per load instruction
  static constexpr int A_UNITS = BM * CH, B_UNITS = BN * CH, STAGE = A_UNITS + B_UNITS;
  static constexpr int NS = (160 * 1024 - 8 * 1024) / (STAGE * 16);  // stages in LDS
  static constexpr int A_LOADS = BM / RPI / WAVES, B_LOADS = BN / RPI / WAVES;  // per wave
  static constexpr int LOADS = A_LOADS + B_LOADS;  // load instructions per wave per stage
  static constexpr size_t LDS_BYTES = (size_t)NS * STAGE * 16;
  static_assert(BM % (WAVES * RPI) == 0 && BN % (WAVES * RPI) == 0 && IM >= 1 &&
                    JN * WN == NB && NS >= 2 && NS * LOADS <= 63,
                "tile shape");
  // chunk c of row r sits at slot c ^ swz(r): the rows one LDS pass serves
  // fall on different banks
  static __device__ __forceinline__ int swz(int r) { return CH == 8 ? (r & 7) : ((r >> 2) & 3); }
};

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt at their maxima): the gfx9
// encoding puts vmcnt bits 3:0 at 3:0 and bits 5:4 at 15:14.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// k_gemm_mx8 with the A operand (the input rows' MXFP8 step lines) copied
// into LDS by global_load_lds instead of through a register ring, and the
// next step's fragments read from LDS while this step's MFMAs run (two
// register sets).  A goes through two stages: step k + 2 is copied while
// step k multiplies, into the stage whose fragments (step k) were read
// during step k - 1; lane l of a copy writes the 16 bytes at base + 16 l and
// fetches 16-byte slot (l % 8) ^ swa(row) of its row's line, so the reads of
// 8 or 16 consecutive rows hit different banks.  B (the expert's MXFP4
// rows, a group of kPipe steps = one 128-byte line per column) and the
// scales keep k_gemm_mx8's register staging; a group's B is staged two
// steps after its loads go out, a step's A scale dword two steps ahead.
// One barrier per step.  Same MFMA sequence and operands as k_gemm_mx8, so
// the outputs are bit-identical to it.
__device__ __forceinline__ int mx8b_swa(int r) { return (r ^ (r >> 3)) & 7; }
template <int MODE>
__global__ __launch_bounds__(256, 2) void k_gemm_mx8b(GemmParams p) {
  // A step lines of the two stages, slot s of row r at s ^ swa(r) (two
  // arrays: the compiler then sees that a copy into one stage does not touch
  // the other, and does not wait for it before reading the other)
  __shared__ __align__(16) uint4 Ar0[kGM * 8], Ar1[kGM * 8];
  __shared__ uint32_t Asc[2][kGM];                // per row: s_hi b0, s_hi b1, s_lo b0, s_lo b1
  __shared__ __align__(16) uint8_t Bq[2][kGN * kQS];   // per column: kPipe steps x 32 B
  __shared__ uint16_t Bsc[2][kGN * kPipe];       // per column and step: the 2 blocks' scales
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int n0, e, r0, rows;
  if (!mx8_block_map(p, n0, e, r0, rows)) return;  // uniform for the block
  __shared__ GemmEpiLds epl;
  GemmEpi ep;
  gemm_epi_issue<MODE, true>(p, lane, wn, n0, r0, rows, e, ep, epl);
  const int K = p.K, KB = K / 32, nk = K / 64;
  // A copies: wave w copies pieces w + 4 i (rows 8 p .. 8 p + 7 of the tile)
  const uint8_t* asrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 8 * (wave + 4 * i) + (lane >> 3);
    const int lr = r0 + min(r, rows - 1);
    const int ar = p.a_rows ? p.a_rows[lr] : lr;
    asrc[i] = p.qa + (size_t)ar * nk * 128 + 16 * ((lane & 7) ^ mx8b_swa(r));
  }
  // B staging map (k_gemm_mx8's): piece c = tid + 256 i is column c >> 3,
  // 16-byte piece c & 7 of its group line
  const int pc = tid & 7;
  const uint8_t* bsrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = (tid + 256 * i) >> 3;
    bsrc[i] = p.codes + ((size_t)e * p.N + min(n0 + c, p.N - 1)) * (K / 2) + 16 * (pc & 1);
  }
  const uint32_t* ssrc;
  {
    const int lr = r0 + min(tid & 127, rows - 1);
    const int ar = p.a_rows ? p.a_rows[lr] : lr;
    ssrc = p.qsc + (size_t)ar * mx8_scale_stride(K);
  }
  const int ng = (nk + kPipe - 1) / kPipe;
  const uint8_t* bssrc = p.scales + ((size_t)e * p.N + min(n0 + (tid & 127), p.N - 1)) * KB;
  const int bsj = 2 * (tid >> 7);
  u32x4_t rsg_cur, rsg_next;  // A scales of this group and the next
  u32x4_t rbq[4];
  uint32_t rbs[2];
#if defined(__HIP_DEVICE_COMPILE__)
#define MX8B_COPY(g, l) __builtin_amdgcn_global_load_lds((g), (l), 16, 0, 0)
#else
#define MX8B_COPY(g, l) ((void)(g), (void)(l))
#endif
  auto issue_a = [&](int kt, int slot) {
    const int st = min(kt, nk - 1);  // past the last step: a copy never read
#pragma unroll
    for (int i = 0; i < 4; ++i)
      MX8B_COPY(asrc[i] + (size_t)st * 128, (slot ? Ar1 : Ar0) + (wave + 4 * i) * 64);
  };
#undef MX8B_COPY
  auto load_b = [&](int g) {
    const int st = min(g * kPipe + (pc >> 1), nk - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      rbq[i] = *reinterpret_cast<const u32x4_t*>(bsrc[i] + (size_t)st * 32);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int sj = min(g * kPipe + bsj + j, nk - 1);
      rbs[j] = *reinterpret_cast<const uint16_t*>(bssrc + 2 * sj);
    }
  };
  auto stage_b = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = (tid + 256 * i) >> 3;
      *reinterpret_cast<u32x4_t*>(&Bq[buf][c * kQS + 16 * pc]) = rbq[i];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) Bsc[buf][(tid & 127) * kPipe + bsj + j] = (uint16_t)rbs[j];
  };
  struct Frag {
    i32x8_t ahi[2], alo[2], bq[2];
    int sa_hi[2], sa_lo[2], s_b[2];
  };
  const int h = h_of(lane);
  // the fragments of step kt (A stage kt % 2, B group buffer gb, step u of it)
  auto read_frag = [&](int slot, int gb, int u, Frag& f) {
#pragma unroll
    for (int im = 0; im < 2; ++im) {
      const int rr = wm * 64 + im * 32 + (lane & 31);
      const uint4* row = (slot ? Ar1 : Ar0) + rr * 8;
      const int sw = mx8b_swa(rr);
      const u32x4_t h0 = *reinterpret_cast<const u32x4_t*>(row + ((h + 0) ^ sw));
      const u32x4_t h1 = *reinterpret_cast<const u32x4_t*>(row + ((h + 2) ^ sw));
      const u32x4_t l0 = *reinterpret_cast<const u32x4_t*>(row + ((h + 4) ^ sw));
      const u32x4_t l1 = *reinterpret_cast<const u32x4_t*>(row + ((h + 6) ^ sw));
      const uint32_t sc = Asc[slot][rr];
      f.sa_hi[im] = (int)((sc >> (8 * h)) & 0xFFu);
      f.sa_lo[im] = (int)((sc >> (16 + 8 * h)) & 0xFFu);
      f.ahi[im] = i32x8_t{(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w,
                          (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
      f.alo[im] = i32x8_t{(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w,
                          (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
    }
#pragma unroll
    for (int in = 0; in < 2; ++in) {
      const int cn = wn * 64 + in * 32 + (lane & 31);
      const u32x4_t b4 = *reinterpret_cast<const u32x4_t*>(&Bq[gb][cn * kQS + u * 32 + 16 * h]);
      f.bq[in] = i32x8_t{(int)b4.x, (int)b4.y, (int)b4.z, (int)b4.w, 0, 0, 0, 0};
      f.s_b[in] = (int)((Bsc[gb][cn * kPipe + u] >> (8 * h)) & 0xFFu);
    }
  };
  f32x16_t acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;
  auto mfma = [&](const Frag& f) {
#pragma unroll
    for (int im = 0; im < 2; ++im)
#pragma unroll
      for (int in = 0; in < 2; ++in)
        acc[im][in] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            f.ahi[im], f.bq[in], acc[im][in], 0, 4, 0, f.sa_hi[im], 0, f.s_b[in]);
#pragma unroll
    for (int im = 0; im < 2; ++im)
#pragma unroll
      for (int in = 0; in < 2; ++in)
        acc[im][in] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            f.alo[im], f.bq[in], acc[im][in], 0, 4, 0, f.sa_lo[im], 0, f.s_b[in]);
  };
  // prologue: A of steps 0 and 1, B and scales of group 0, staged
  issue_a(0, 0);
  issue_a(1, 1);
  load_b(0);
  rsg_cur = *reinterpret_cast<const u32x4_t*>(ssrc);
  rsg_next = *reinterpret_cast<const u32x4_t*>(ssrc + 4 * min(1, ng - 1));
  stage_b(0);
  if (tid < kGM) {
    Asc[0][tid] = rsg_cur.x;
    Asc[1][tid] = rsg_cur.y;
  }
  wait_vmcnt<0>();
  __syncthreads();
  Frag fr[2];
  read_frag(0, 0, 0, fr[0]);
  for (int kt0 = 0; kt0 < nk; kt0 += kPipe) {
    const int g = kt0 / kPipe, gb = g & 1;
#pragma unroll
    for (int u = 0; u < kPipe; ++u) {
      const int kt = kt0 + u;
      if (kt >= nk) break;  // uniform for the block
      // A of step kt + 1 (copied during step kt - 1; then group g's B loads
      // went out after it at u = 1) has landed for this wave; the barrier:
      // for every wave, and every wave's reads of step kt's stage and of the
      // scale dwords staged two steps back are done
      if (u == 1) wait_vmcnt<7>();
      else wait_vmcnt<0>();
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      issue_a(kt + 2, u & 1);  // into the stage of step kt, read during step kt - 1
      if (u == 0) {
        load_b(g + 1);  // group g + 1's B, staged at u = 2
        if (g > 0) rsg_cur = rsg_next;
        rsg_next = *reinterpret_cast<const u32x4_t*>(ssrc + 4 * min(g + 1, ng - 1));
      }
      __builtin_amdgcn_sched_barrier(0);
      if (kt + 1 < nk)  // uniform
        read_frag((u + 1) & 1, u == kPipe - 1 ? gb ^ 1 : gb, (u + 1) % kPipe, fr[(u + 1) & 1]);
      mfma(fr[u & 1]);
      // the scale dword of step kt + 2 into its stage (that of step kt)
      if (tid < kGM)
        Asc[u & 1][tid] = u == 0 ? rsg_cur.z : u == 1 ? rsg_cur.w : u == 2 ? rsg_next.x : rsg_next.y;
      if (u == 2) stage_b(gb ^ 1);  // group g + 1 (its buffer's last reads were in step 4 g - 2)
    }
  }
  wait_vmcnt<0>();  // the last (unread) copies have landed before LDS is reused
  gemm_epi_stage<MODE>(ep, epl);
  gemm_epilogue<MODE, true>(acc, p, lane, wm, wn, n0, r0, rows, ep, epl);
}

// The MXFP8 expert GEMMs run k_gemm_mx8b: at the 2048-token 20b shape 367 /
// 201 us per layer (gate_up / down) against 388 / 215 us for k_gemm_mx8 in
// the same run, the same bits.  NEON_MX8_GEMM = "a" selects k_gemm_mx8, for
// comparisons.
static bool mx8_gemm_b() {
  static const bool v = !(getenv("NEON_MX8_GEMM") && getenv("NEON_MX8_GEMM")[0] == 'a');
  return v;
}

template <int MODE, int BM, int NB, int BK, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN, 1) void k_gemm_lds(GemmParams p) {
  using G = GemmLdsCfg<BM, NB, BK, WM, WN>;
  constexpr int IM = G::IM, JN = G::JN, WAVES = G::WAVES;
  extern __shared__ __align__(16) uint4 lds[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w / WN, wn = w % WN;
  const int M = p.M, N = p.N, nk = p.K / G::BK;
  // Block order: the dispatcher deals blocks to the 8 XCDs round-robin
  // (linear id % 8).  Renumbered so that each XCD gets a contiguous range of
  // logical tiles, taken column by column: the row tiles of one weight
  // column tile then share that XCD's L2 copy of it.
  const int gx = gridDim.x, gy = gridDim.y, nb = gx * gy;
  const int bid = blockIdx.y * gx + blockIdx.x;
  const int per = (nb + 7) / 8, full = nb - 8 * (per - 1);  // XCDs with `per` blocks
  const int xcd = bid % 8, slot = bid / 8;
  const int lid = (xcd < full ? xcd * per : full * per + (xcd - full) * (per - 1)) + slot;
  const int m0 = (lid % gy) * G::BM, n0 = (lid / gy) * G::BN;
  // epilogue inputs first (their loads precede every stage's in the counter)
  float bcol[JN];
#pragma unroll
  for (int in = 0; in < JN; ++in) {
    const int col = n0 + 32 * (JN * wn + in) + (lane & 31);
    const uint16_t bq =  // unconditional: see gemm_epi_issue
        load_pinned_u16(p.bias != nullptr ? p.bias + min(col, N - 1) : p.W);
    bcol[in] = (p.bias != nullptr && col < N) ? bf2f(bq) : 0.0f;
  }
  // this lane's rows and chunk for the direct loads: instruction j covers
  // rows RPI j .. RPI j + RPI - 1; lane l fills row RPI j + l / CH, slot
  // l % CH, with chunk slot ^ swz(row) of that row
  const int lr = lane / G::CH, ls = lane % G::CH;
  const uint16_t* ag[G::A_LOADS];
#pragma unroll
  for (int i = 0; i < G::A_LOADS; ++i) {
    const int rt = G::RPI * (w + WAVES * i) + lr;
    const int r = min(m0 + rt, M - 1);
    ag[i] = p.A + (size_t)r * p.lda + 8 * (ls ^ G::swz(rt));
  }
  const uint16_t* bg[G::B_LOADS];
#pragma unroll
  for (int i = 0; i < G::B_LOADS; ++i) {
    const int rt = G::RPI * (w + WAVES * i) + lr;
    const int r = min(n0 + rt, N - 1);
    bg[i] = p.W + (size_t)r * p.ldw + 8 * (ls ^ G::swz(rt));
  }
  f32x16_t acc[IM][JN];
#pragma unroll
  for (int a = 0; a < IM; ++a)
#pragma unroll
    for (int b = 0; b < JN; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;
  // the direct loads of step kt (BK of K) into its stage: wave w's
  // instructions j = w + WAVES i of the A tile and of the W tile.  The
  // builtin is compiled in the device pass only: the host pass of this
  // kernel drops its launch stub without a diagnostic when it sees it.
#if defined(__HIP_DEVICE_COMPILE__)
#define GEMM_LDS_LOAD(g, l) __builtin_amdgcn_global_load_lds((g), (l), 16, 0, 0)
#else
#define GEMM_LDS_LOAD(g, l) ((void)(g), (void)(l))
#endif
  // every wave issues the same copies at every step (past the last step the
  // last one again, into a stage that is not read any more), so one vmcnt
  // value covers a step
#define GEMM_LDS_ISSUE(kt_, slot_)                                                         \
  do {                                                                                     \
    uint4* base_ = lds + (slot_) * G::STAGE;                                               \
    const int ko_ = min((kt_), nk - 1) * G::BK;                                            \
    _Pragma("unroll") for (int i = 0; i < G::A_LOADS; ++i)                                 \
      GEMM_LDS_LOAD(ag[i] + ko_, base_ + (w + WAVES * i) * 64);                            \
    _Pragma("unroll") for (int i = 0; i < G::B_LOADS; ++i)                                 \
      GEMM_LDS_LOAD(bg[i] + ko_, base_ + G::A_UNITS + (w + WAVES * i) * 64);               \
  } while (0)
#pragma unroll
  for (int s = 0; s < G::NS - 1; ++s) GEMM_LDS_ISSUE(s, s);
  // fragment units: row r, 16-k step ks -> chunk 2 ks + lane / 32 at slot c ^ swz(r)
  const int fr = lane & 31, fh = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    // stage kt complete (the stages after it that were issued may still load)
    wait_vmcnt<(G::NS - 2) * G::LOADS>();  // this wave's copies of step kt have landed
    // every wave's have, and every wave's reads of stage (kt - 1) % NS are
    // complete (lgkmcnt 0), so it may be refilled.  Not __syncthreads(): its
    // fence waits for every outstanding copy (vmcnt 0), the later stages'
    // too, which leaves the ring one stage deep
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    GEMM_LDS_ISSUE(kt + G::NS - 1, (kt + G::NS - 1) % G::NS);
    __builtin_amdgcn_sched_barrier(0);  // the copies go out before this step's reads
    const uint4* st = lds + (kt % G::NS) * G::STAGE;
    // fragments of 16-k step ks into register set ks % 2; the next step's
    // reads are issued before this step's MFMAs, so LDS latency hides behind
    // them
    bf16x8_t af[2][IM], bf[2][JN];
#define GEMM_LDS_FRAGS(ks_)                                                                  \
    do {                                                                                     \
      const int c_ = 2 * (ks_) + fh, b_ = (ks_) & 1;                                         \
      _Pragma("unroll") for (int im = 0; im < IM; ++im) {                                    \
        const int r = 32 * IM * wm + 32 * im + fr;                                           \
        af[b_][im] = *reinterpret_cast<const bf16x8_t*>(st + r * G::CH + (c_ ^ G::swz(r))); \
      }                                                                                      \
      _Pragma("unroll") for (int in = 0; in < JN; ++in) {                                    \
        const int r = 32 * (JN * wn + in) + fr;                                              \
        bf[b_][in] = *reinterpret_cast<const bf16x8_t*>(st + G::A_UNITS + r * G::CH +       \
                                                        (c_ ^ G::swz(r)));                   \
      }                                                                                      \
    } while (0)
    constexpr int KS = G::BK / 16;
    GEMM_LDS_FRAGS(0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) GEMM_LDS_FRAGS(ks + 1);
#pragma unroll
      for (int im = 0; im < IM; ++im)
#pragma unroll
        for (int in = 0; in < JN; ++in)
          acc[im][in] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks & 1][im], bf[ks & 1][in],
                                                                acc[im][in], 0, 0, 0);
    }
#undef GEMM_LDS_FRAGS
  }
  wait_vmcnt<0>();  // the ring's last (unread) copies have landed before LDS is reused
#undef GEMM_LDS_ISSUE
#undef GEMM_LDS_LOAD
  // epilogue: acc[im][in][i] is row 32 IM wm + 32 im + 8 (i / 4) + 4 (lane / 32) + i % 4,
  // column 32 (JN wn + in) + lane % 32 of the tile
  if constexpr (MODE == GEMM_F32) {
#pragma unroll
    for (int im = 0; im < IM; ++im)
#pragma unroll
      for (int in = 0; in < JN; ++in) {
        const int col = n0 + 32 * (JN * wn + in) + (lane & 31);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int row = m0 + 32 * IM * wm + 32 * im + 8 * (i >> 2) + 4 * fh + (i & 3);
          if (row < M && col < N)
            p.Cf[(size_t)row * p.ldc + col] = p.bias != nullptr ? __fadd_rn(acc[im][in][i], bcol[in])
                                                                : acc[im][in][i];
        }
      }
    return;
  }
  // STORE / RESID: bf16(acc + bias) into an LDS copy of the tile (row stride
  // BN + 8 elements), then the whole block writes C in 16-byte row pieces,
  // RESID adding each to the residual it reads the same way:
  // C = bf16(C + bf16(acc + bias))
  constexpr int TS = G::BN + 8;
  static_assert((size_t)G::BM * TS * 2 <= G::LDS_BYTES, "the output tile fits the stages' LDS");
  uint16_t* tile = reinterpret_cast<uint16_t*>(lds);
  __syncthreads();  // every wave has finished reading the last stage
#pragma unroll
  for (int im = 0; im < IM; ++im)
#pragma unroll
    for (int in = 0; in < JN; ++in) {
      const int ct = 32 * (JN * wn + in) + (lane & 31);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rt = 32 * IM * wm + 32 * im + 8 * (i >> 2) + 4 * fh + (i & 3);
        const float v = p.bias != nullptr ? __fadd_rn(acc[im][in][i], bcol[in]) : acc[im][in][i];
        tile[rt * TS + ct] = f2bf(v);
      }
    }
  __syncthreads();
  constexpr int CPR = G::BN / 8;  // 16-byte pieces per tile row
  for (int q = tid; q < G::BM * CPR; q += 64 * WAVES) {
    const int rt = q / CPR, cp = q % CPR;
    const int row = m0 + rt, col = n0 + 8 * cp;
    if (row >= M || col >= N) continue;  // N % 8 == 0: a piece is wholly in or out
    const uint4 v = *reinterpret_cast<const uint4*>(tile + rt * TS + 8 * cp);
    uint4* dst = reinterpret_cast<uint4*>(p.C + (size_t)row * p.ldc + col);
    if constexpr (MODE == GEMM_RESID) {
      const uint4 c = *dst;
      const uint32_t cw[4] = {c.x, c.y, c.z, c.w}, vw[4] = {v.x, v.y, v.z, v.w};
      uint32_t o[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        o[t] = pack_bf2(__fadd_rn(bf_lo(cw[t]), bf_lo(vw[t])), __fadd_rn(bf_hi(cw[t]), bf_hi(vw[t])));
      *dst = make_uint4(o[0], o[1], o[2], o[3]);
    } else {
      *dst = v;
    }
  }
}

template <int MODE, int BM, int NB, int BK, int WM, int WN>
static void launch_gemm_lds_v(const GemmParams& p, hipStream_t st) {
  using G = GemmLdsCfg<BM, NB, BK, WM, WN>;
  static const hipError_t optin = hipFuncSetAttribute(
      reinterpret_cast<const void*>(k_gemm_lds<MODE, BM, NB, BK, WM, WN>),
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)G::LDS_BYTES);
  (void)optin;  // a refused opt-in surfaces as the launch's error
  const dim3 grid((p.N + G::BN - 1) / G::BN, (p.M + G::BM - 1) / G::BM);
  hipLaunchKernelGGL((k_gemm_lds<MODE, BM, NB, BK, WM, WN>), grid, dim3(64 * G::WAVES),
                     G::LDS_BYTES, st, p);
}

// Tile of an M x N product: of 256 x 192, 256 x 128, 128 x 192 and 128 x 128,
// the one with the fewest rounds of the device times per-block MFMA work
// (BM x BN), ties to the larger tile (fewer operand re-reads).  Every tile
// runs 8 waves, two per SIMD, with 64-deep K steps.  Measured at the
// prompt pass's shapes (M = 2047): QKV (N 5120, K 2880, 256 x 192, 2
// stages) 69 us, O + residual (N 2880, K 4096, 128 x 192, 3 stages) 62 us
// (71 us while the step barrier also waited for the later stages' copies);
// QKV on 128 x 192 tiles 85 us; 32-deep steps with 5-9 stages in flight
// (256 x 128 and 128 x 128) 108-117 us for QKV and 72-94 us for O; 4 waves
// per block 3 to 25% slower.
static void gemm_lds_tile(int M, int N, int& bm, int& nb) {
  long best = -1;
  for (int b : {256, 128})
    for (int n : {6, 4}) {
      const long blocks = (long)((N + 32 * n - 1) / (32 * n)) * ((M + b - 1) / b);
      const long cost = ((blocks + 255) / 256) * b * n;
      if (best < 0 || cost < best) { best = cost; bm = b; nb = n; }
    }
}

// NEON_GEMM_LDS = "BM,NB,64" forces one of the shapes below, for comparisons
template <int MODE>
static void launch_gemm_lds(const GemmParams& p, hipStream_t st) {
  int bm = 256, nb = 6;
  gemm_lds_tile(p.M, p.N, bm, nb);
  static int force[3] = {-1, 0, 0};
  if (force[0] == -1) {
    force[0] = 0;
    if (const char* e = getenv("NEON_GEMM_LDS")) sscanf(e, "%d,%d,%d", &force[0], &force[1], &force[2]);
  }
  if (force[0] > 0 && force[2] == 64 && (force[0] == 256 || force[0] == 128) &&
      (force[1] == 6 || force[1] == 4)) {
    bm = force[0];
    nb = force[1];
  }
  if (bm == 256) {
    if (nb == 6) launch_gemm_lds_v<MODE, 256, 6, 64, 8, 1>(p, st);
    else launch_gemm_lds_v<MODE, 256, 4, 64, 8, 1>(p, st);
  } else {
    if (nb == 6) launch_gemm_lds_v<MODE, 128, 6, 64, 4, 2>(p, st);
    else launch_gemm_lds_v<MODE, 128, 4, 64, 4, 2>(p, st);
  }
}

// The prompt pass's QKV and O projections (bias; O adds into the residual):
// the hand-written direct-load GEMM above.
void launch_prompt_proj(const uint16_t* A, const uint16_t* W, const uint16_t* bias,
                        uint16_t* C, int M, int N, int K, int mode, hipStream_t st) {
  launch_gemm_bf16(A, K, W, K, bias, C, nullptr, N, M, N, K, mode, st);
}

void launch_gemm_bf16(const uint16_t* A, int lda, const uint16_t* W, int ldw,
                      const uint16_t* bias, uint16_t* C, float* Cf, int ldc, int M,
                      int N, int K, int mode, hipStream_t st) {
  if (mode == GEMM_F32 && N <= kNarrowMaxN && K % 32 == 0 && lda == K && ldw == K && ldc == N) {
    // a narrow fp32 product (the prompt router logits, N = E): 128-wide
    // column tiles would leave most of the device idle
    launch_gemm_narrow_f32(A, W, bias, Cf, M, N, K, st);
    return;
  }
  GemmParams p{};
  p.A = A; p.lda = lda; p.W = W; p.ldw = ldw; p.bias = bias; p.C = C; p.Cf = Cf;
  p.ldc = ldc; p.M = M; p.N = N; p.K = K;
  if (K % 64 == 0 && lda % 8 == 0 && ldw % 8 == 0 && ldc % 8 == 0 && N % 8 == 0 && N >= 128) {
    // the direct-load pipeline (16-byte row pieces, 32-deep steps)
    switch (mode) {
      case GEMM_STORE: launch_gemm_lds<GEMM_STORE>(p, st); return;
      case GEMM_RESID: launch_gemm_lds<GEMM_RESID>(p, st); return;
      default: launch_gemm_lds<GEMM_F32>(p, st); return;
    }
  }
  dim3 grid((N + kGN - 1) / kGN, (M + kGM - 1) / kGM);
  switch (mode) {
    case GEMM_STORE: hipLaunchKernelGGL((k_gemm<GEMM_STORE, false, false>), grid, dim3(256), 0, st, p); break;
    case GEMM_RESID: hipLaunchKernelGGL((k_gemm<GEMM_RESID, false, false>), grid, dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL((k_gemm<GEMM_F32, false, false>), grid, dim3(256), 0, st, p); break;
  }
}

// ===========================================================================
// Expert grouping: the (token, slot) pairs of idx [M][k] sorted by expert,
// stable in (token, slot) order, plus the 128-row GEMM tiles of each
// expert's run.  One block of 1024 threads; for each expert the block counts
// its pairs in each thread's consecutive chunk and places them with a block
// prefix sum.
// ===========================================================================
__device__ __forceinline__ int block_excl_scan_1024(int v, int* lds) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) lds[wave] = x;
  __syncthreads();
  if (tid == 0) {
    int s = 0;
    for (int w = 0; w < 16; ++w) { const int t = lds[w]; lds[w] = s; s += t; }
    lds[16] = s;
  }
  __syncthreads();
  const int r = lds[wave] + x - v;
  __syncthreads();
  return r;
}

// Expert grouping, step 1 (one block): pairs per expert (LDS atomics), the
// offsets e_off[0..E] and the 128-row tiles (tile_e, tile_r0, n_tiles).
__global__ __launch_bounds__(1024) void k_moe_count(
    const int32_t* __restrict__ idx, int n_pairs, int E, int32_t* __restrict__ e_off,
    int32_t* __restrict__ tile_e, int32_t* __restrict__ tile_r0, int32_t* __restrict__ n_tiles,
    int32_t* __restrict__ err) {
  __shared__ int cnt[256];
  const int tid = threadIdx.x;
  if (tid < 256) cnt[tid] = 0;
  __syncthreads();
  bool bad = false;
  for (int q = tid; q < n_pairs; q += 1024) {
    const int e = idx[q];
    // a pair whose id lies outside [0, E) joins no group; the combine drops it
    if ((unsigned)e < (unsigned)E) atomicAdd(&cnt[e], 1);
    else bad = true;
  }
  if (bad) flag_dev_err(err, kDevErrExpertId);
  __syncthreads();
  if (tid == 0) {
    int base = 0, t = 0;
    for (int e = 0; e < E; ++e) {
      e_off[e] = base;
      const int c = cnt[e];
      for (int r = 0; r < c; r += kGM) { tile_e[t] = e; tile_r0[t] = r; ++t; }
      base += c;
    }
    e_off[E] = base;
    *n_tiles = t;
  }
}

// Expert grouping, step 2 (block e): the pairs q that chose expert e, in
// increasing q, at e_off[e] ..: (token q / k, slot q % k).  Thread tid holds
// pairs tid * per .. tid * per + per - 1; one block scan orders the threads.
__global__ __launch_bounds__(1024) void k_moe_group(
    const int32_t* __restrict__ idx, int n_pairs, int k, const int32_t* __restrict__ e_off,
    int32_t* __restrict__ list_tok, int32_t* __restrict__ list_slot) {
  __shared__ int scan_lds[17];
  const int e = blockIdx.x, tid = threadIdx.x;
  const int per = (n_pairs + 1023) / 1024;
  const int p0 = tid * per, p1 = min(p0 + per, n_pairs);
  int c = 0;
  for (int q = p0; q < p1; ++q) c += idx[q] == e;
  const int pos = block_excl_scan_1024(c, scan_lds);
  int o = e_off[e] + pos;
  for (int q = p0; q < p1; ++q)
    if (idx[q] == e) { list_tok[o] = q / k; list_slot[o] = q % k; ++o; }
}

// Expert grouping in one launch (block e of E): every block counts the pairs
// of every expert (LDS atomics, k_moe_count's counts), two block scans over
// the experts give the offsets and the first tile of each, then block e
// writes e_off[e] and its expert's tiles (block 0 also e_off[E] and
// n_tiles) and places the expert's pairs as k_moe_group does.  The same
// lists and tiles as k_moe_count + k_moe_group, one launch and one
// dependent round trip fewer.
__global__ __launch_bounds__(1024) void k_moe_group1(
    const int32_t* __restrict__ idx, int n_pairs, int k, int E, int32_t* __restrict__ e_off,
    int32_t* __restrict__ tile_e, int32_t* __restrict__ tile_r0, int32_t* __restrict__ n_tiles,
    int32_t* __restrict__ list_tok, int32_t* __restrict__ list_slot, int32_t* __restrict__ err) {
  __shared__ int cnt[256];
  __shared__ int scan_lds[17];
  __shared__ int mine[2];
  const int e = blockIdx.x, tid = threadIdx.x;
  if (tid < 256) cnt[tid] = 0;
  __syncthreads();
  const int per = (n_pairs + 1023) / 1024;
  const int p0 = tid * per, p1 = min(p0 + per, n_pairs);
  int c = 0;
  bool bad = false;
  for (int q = p0; q < p1; ++q) {
    const int id = idx[q];
    // a pair whose id lies outside [0, E) joins no group; the combine drops it
    if ((unsigned)id < (unsigned)E) atomicAdd(&cnt[id], 1);
    else bad = true;
    c += id == e;
  }
  if (bad && e == 0) flag_dev_err(err, kDevErrExpertId);
  __syncthreads();
  const int ce = tid < E ? cnt[tid] : 0;
  const int off = block_excl_scan_1024(ce, scan_lds);  // pairs of the experts before tid
  const int total = scan_lds[16];
  const int toff = block_excl_scan_1024((ce + kGM - 1) / kGM, scan_lds);  // their tiles
  const int ttot = scan_lds[16];
  if (tid == e) { mine[0] = off; mine[1] = toff; }
  if (e == 0 && tid == 0) { e_off[E] = total; *n_tiles = ttot; }
  __syncthreads();
  const int base = mine[0], t0 = mine[1], ne = cnt[e];
  if (tid == 0) e_off[e] = base;
  for (int r = tid * kGM; r < ne; r += 1024 * kGM) {
    tile_e[t0 + r / kGM] = e;
    tile_r0[t0 + r / kGM] = r;
  }
  int o = base + block_excl_scan_1024(c, scan_lds);
  for (int q = p0; q < p1; ++q)
    if (idx[q] == e) { list_tok[o] = q / k; list_slot[o] = q % k; ++o; }
}

// out[t] = bf16(residual[t] + bf16(sum_s score[t][s] * y[t][s]))  in slot
// order with fmaf, as the decode combine (HFM:111-112).
__global__ void k_moe_combine(const float* __restrict__ ybuf,
                              const float* __restrict__ score,
                              const int32_t* __restrict__ idx, int E, int k, int H,
                              uint16_t* __restrict__ h) {
  const int t = blockIdx.x;
  for (int n = threadIdx.x; n < H; n += blockDim.x) {
    float y = 0.0f;
    for (int s = 0; s < k; ++s) {
      // pairs with an id outside [0, E) were never computed: they add 0
      const bool ok = (unsigned)idx[t * k + s] < (unsigned)E;
      y = __builtin_fmaf(score[t * k + s], ok ? ybuf[((size_t)t * k + s) * H + n] : 0.0f, y);
    }
    uint16_t* c = h + (size_t)t * H + n;
    *c = f2bf(__fadd_rn(bf2f(*c), bf2f(f2bf(y))));
  }
}

// k_moe_combine with 8 consecutive columns per thread (32-byte loads of each
// slot's fp32 row, 16-byte load and store of the residual): the same
// operations per element in the same order, for KSL slots (the model's
// top-k).  The slots' ids and scores are read once per block.  H % 8 == 0.
template <int KSL>
__global__ __launch_bounds__(384) void k_moe_combine8(const float* __restrict__ ybuf,
                                                      const float* __restrict__ score,
                                                      const int32_t* __restrict__ idx, int E,
                                                      int H, uint16_t* __restrict__ h) {
  const int t = blockIdx.x;
  float sc[KSL];
  bool ok[KSL];
#pragma unroll
  for (int s = 0; s < KSL; ++s) {
    sc[s] = score[t * KSL + s];
    // pairs with an id outside [0, E) were never computed: they add 0
    ok[s] = (unsigned)idx[t * KSL + s] < (unsigned)E;
  }
  for (int n = 8 * threadIdx.x; n < H; n += 8 * blockDim.x) {
    float4 v[KSL][2];
#pragma unroll
    for (int s = 0; s < KSL; ++s) {
      const float4* src = reinterpret_cast<const float4*>(ybuf + ((size_t)t * KSL + s) * H + n);
      v[s][0] = src[0];
      v[s][1] = src[1];
    }
    uint4* cp = reinterpret_cast<uint4*>(h + (size_t)t * H + n);
    const uint4 c = *cp;
    float y[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < KSL; ++s) {
      const float e[8] = {v[s][0].x, v[s][0].y, v[s][0].z, v[s][0].w,
                          v[s][1].x, v[s][1].y, v[s][1].z, v[s][1].w};
#pragma unroll
      for (int q = 0; q < 8; ++q) y[q] = __builtin_fmaf(sc[s], ok[s] ? e[q] : 0.0f, y[q]);
    }
    const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float lo = __fadd_rn(bf2f((uint16_t)(cw[q] & 0xFFFFu)), bf2f(f2bf(y[2 * q])));
      const float hi = __fadd_rn(bf2f((uint16_t)(cw[q] >> 16)), bf2f(f2bf(y[2 * q + 1])));
      o[q] = (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
    }
    *cp = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// MoE layer over M tokens: experts from idx/score [M][k], input xn [M][H],
// residual stream h [M][H] updated in place.  Scratch: list_tok/list_slot
// [M k], e_off [E+1], tile_e/tile_r0 [max_tiles], n_tiles [1], act [M k][I]
// bf16, ybuf [M][k][H] fp32.
void launch_moe_prefill(const MoePrefillArgs& a, hipStream_t st) {
  const int n_pairs = a.M * a.k;
  // the grouping in one launch (NEON_PREFILL_GROUP=2: k_moe_count, then
  // k_moe_group; the same lists)
  static const bool two = getenv("NEON_PREFILL_GROUP") && getenv("NEON_PREFILL_GROUP")[0] == '2';
  if (two) {
    hipLaunchKernelGGL(k_moe_count, dim3(1), dim3(1024), 0, st, a.idx, n_pairs, a.E, a.e_off,
                       a.tile_e, a.tile_r0, a.n_tiles, a.err);
    hipLaunchKernelGGL(k_moe_group, dim3(a.E), dim3(1024), 0, st, a.idx, n_pairs, a.k, a.e_off,
                       a.list_tok, a.list_slot);
  } else {
    hipLaunchKernelGGL(k_moe_group1, dim3(a.E), dim3(1024), 0, st, a.idx, n_pairs, a.k, a.E,
                       a.e_off, a.tile_e, a.tile_r0, a.n_tiles, a.list_tok, a.list_slot, a.err);
  }
  const int max_tiles = moe_prefill_max_tiles(a.M, a.k, a.E);
  GemmParams p{};
  p.tile_e = a.tile_e; p.tile_r0 = a.tile_r0; p.n_tiles = a.n_tiles; p.e_off = a.e_off;
  p.list_tok = a.list_tok; p.list_slot = a.list_slot; p.topk = a.k;
  p.alpha = a.alpha; p.limit = a.limit;
  p.qa = a.q; p.qsc = a.qs;
  const bool mx8 = a.q != nullptr;
  // gate_up + SwiGLU: A = xn rows of the listed tokens, N = 2 I, out act [list][I]
  if (mx8) launch_mx8_quant_lines(a.xn, a.M, a.H, a.q, a.qs, st);
  p.A = a.xn; p.lda = a.H; p.a_rows = a.list_tok;
  p.codes = a.gu_codes; p.scales = a.gu_scales; p.bias = a.gu_bias;
  p.C = a.act; p.ldc = a.I; p.N = 2 * a.I; p.K = a.H;
  if (mx8 && mx8_gemm_b())
    hipLaunchKernelGGL((k_gemm_mx8b<GEMM_SWIGLU>), mx8_grid(2 * a.I, max_tiles),
                       dim3(256), 0, st, p);
  else if (mx8)
    hipLaunchKernelGGL((k_gemm_mx8<GEMM_SWIGLU>), mx8_grid(2 * a.I, max_tiles),
                       dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((k_gemm<GEMM_SWIGLU, true, true>),
                       dim3((2 * a.I + kGN - 1) / kGN, max_tiles), dim3(256), 0, st, p);
  // down: A = act rows in list order, N = H, out ybuf[token][slot]
  if (mx8) launch_mx8_quant_lines(a.act, (int64_t)a.M * a.k, a.I, a.q, a.qs, st);
  p.A = a.act; p.lda = a.I; p.a_rows = nullptr;
  p.codes = a.dn_codes; p.scales = a.dn_scales; p.bias = a.dn_bias;
  p.ybuf = a.ybuf; p.N = a.H; p.K = a.I; p.C = nullptr;
  if (mx8 && mx8_gemm_b())
    hipLaunchKernelGGL((k_gemm_mx8b<GEMM_SCATTER>), mx8_grid(a.H, max_tiles),
                       dim3(256), 0, st, p);
  else if (mx8)
    hipLaunchKernelGGL((k_gemm_mx8<GEMM_SCATTER>), mx8_grid(a.H, max_tiles),
                       dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((k_gemm<GEMM_SCATTER, true, true>), dim3((a.H + kGN - 1) / kGN, max_tiles),
                       dim3(256), 0, st, p);
  if (a.H % 8 == 0 && a.k == 4)  // the gpt-oss top-4
    hipLaunchKernelGGL(k_moe_combine8<4>, dim3(a.M), dim3(min(384, (a.H / 8 + 63) / 64 * 64)),
                       0, st, a.ybuf, a.score, a.idx, a.E, a.H, a.h);
  else
    hipLaunchKernelGGL(k_moe_combine, dim3(a.M), dim3(256), 0, st, a.ybuf, a.score, a.idx, a.E,
                       a.k, a.H, a.h);
}

int moe_prefill_max_tiles(int M, int k, int E) {
  return (M * k + kGM - 1) / kGM + E;
}

// ===========================================================================
// RoPE + KV append for M prompt rows (positions 0 .. M-1): q heads rotated
// into q_out [M][Hq][64] (bf16, as the decode kernel rounds them), k heads
// rotated and v copied into the cache rows [Hkv][T_max][64].
// ===========================================================================
__global__ void k_rope_kv_rows(const uint16_t* __restrict__ qkv, int q_stride,
                               const float* __restrict__ cos_t,
                               const float* __restrict__ sin_t, int Hq, int Hkv,
                               int T_max, uint16_t* __restrict__ q_out,
                               uint16_t* __restrict__ kc, uint16_t* __restrict__ vc) {
  const int t = blockIdx.x;
  const int half = 32;
  const uint16_t* row = qkv + (size_t)t * q_stride;
  const float* cr = cos_t + (size_t)t * half;
  const float* sr = sin_t + (size_t)t * half;
  for (int i = threadIdx.x; i < (Hq + Hkv) * half; i += blockDim.x) {
    const int hh = i / half, f = i % half;
    const uint16_t* x = row + (size_t)hh * 64;
    float o1, o2;
    const float x1 = bf2f(x[f]), x2 = bf2f(x[f + half]);
    o1 = __fsub_rn(__fmul_rn(x1, cr[f]), __fmul_rn(x2, sr[f]));
    o2 = __fadd_rn(__fmul_rn(x2, cr[f]), __fmul_rn(x1, sr[f]));
    uint16_t* dst = hh < Hq ? q_out + ((size_t)t * Hq + hh) * 64
                            : kc + ((size_t)(hh - Hq) * T_max + t) * 64;
    dst[f] = f2bf(o1);
    dst[f + half] = f2bf(o2);
  }
  for (int i = threadIdx.x; i < Hkv * 64; i += blockDim.x) {
    const int g = i / 64, d = i % 64;
    vc[((size_t)g * T_max + t) * 64 + d] = row[(size_t)(Hq + Hkv + g) * 64 + d];
  }
}

void launch_rope_kv_rows(const uint16_t* qkv, int q_stride, const float* cos_t,
                         const float* sin_t, int M, int Hq, int Hkv, int T_max,
                         uint16_t* q_out, uint16_t* kc, uint16_t* vc, hipStream_t st) {
  hipLaunchKernelGGL(k_rope_kv_rows, dim3(M), dim3(256), 0, st, qkv, q_stride, cos_t,
                     sin_t, Hq, Hkv, T_max, q_out, kc, vc);
}

// Keys / values of prompt rows t0 .. M-1, staged as [Hkv][S][64], into a
// sliding layer's ring cache [Hkv][R][64] (R a power of two, row t at t & (R-1)).
__global__ void k_kv_ring_store(const uint16_t* __restrict__ ks,
                                const uint16_t* __restrict__ vs, int S, int t0, int Hkv,
                                int R, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc) {
  const int t = t0 + blockIdx.x;
  const int r = t & (R - 1);
  for (int i = threadIdx.x; i < Hkv * 64; i += blockDim.x) {
    const int g = i >> 6, d = i & 63;
    kc[((size_t)g * R + r) * 64 + d] = ks[((size_t)g * S + t) * 64 + d];
    vc[((size_t)g * R + r) * 64 + d] = vs[((size_t)g * S + t) * 64 + d];
  }
}

void launch_kv_ring_store(const uint16_t* ks, const uint16_t* vs, int S, int t0, int M,
                          int Hkv, int R, uint16_t* kc, uint16_t* vc, hipStream_t st) {
  if (M <= t0) return;
  hipLaunchKernelGGL(k_kv_ring_store, dim3(M - t0), dim3(256), 0, st, ks, vs, S, t0, Hkv,
                     R, kc, vc);
}

// ===========================================================================
// Causal sink attention over a prompt (HFM:235-263) on the matrix cores.
// grid (Hkv, ceil(M/64)), block 64 G: wave w is q head g G + w for the 64
// query rows t0 .. t0+63 of block row y.  Per tile of 64 keys (staged once per
// block in LDS: K as [key][dim], V transposed as [dim][key]):
//   S^T = K Q^T  (v_mfma_f32_16x16x32_bf16: A = 16 keys x 32 dims from LDS,
//                 B = 32 dims x 16 queries from registers); lane (j, g) holds
//                 S^T[key 16 kt + 4 g + r][query 16 qt + j];
//   scores x 1/8 (HFM:277), causal / window mask, online softmax per query
//   (max over the 4 lane groups by xor 16, 32);
//   O^T += V^T P^T  (A = 16 dims x 8 keys of V^T, B = the same 8 keys of P^T
//                    as the lane already holds them: keys 32 p + 4 g + r and
//                    32 p + 16 + 4 g + r), with P split into bf16 hi + lo so
//                    the products keep ~16 bits of P.
// The sink joins the denominator at the end.  Sliding layers see keys
// (t - window, t].
// ===========================================================================
typedef __bf16 pf_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pf_f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ pf_bf16x8 pf_as_bf16x8(const uint4& v) {
  return __builtin_bit_cast(pf_bf16x8, v);
}

// Scores of one tile for the 16 query columns (qt, j) of this lane: the
// softmax state m (log2 domain), l, o, and the P^T fragments (hi, lo) for
// V^T P^T.  s2 = (q.k) * log2(e) / 8 in one rounding; p = 2^(s2 - m).
// MASK: the tile crosses the causal diagonal or the window's lower edge, so
// each key is checked; other tiles are valid for every query of the block.
template <bool MASK, int QT>
__device__ __forceinline__ void attn_prefill_softmax(
    const pf_f32x4 (&sacc)[4][QT], int qt, int t0, int j0, int j, int g, int window,
    float& m, float& l, pf_f32x4 (&o)[4], uint4 (&phi)[2], uint4 (&plo)[2]) {
  constexpr float kScale = 0.125f * 1.44269504088896340736f;  // 1/sqrt(64) * log2(e)
  const int t = t0 + 16 * qt + j;
  const int lo_t = window > 0 ? max(0, t - window + 1) : 0;
  float sv[4][4];
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = __fmul_rn(sacc[kt][qt][r], kScale);
      if (MASK) {
        const int key = j0 + 16 * kt + 4 * g + r;
        v = (key >= lo_t && key <= t) ? v : -INFINITY;
      }
      sv[kt][r] = v;
      mx = fmaxf(mx, v);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float mt = fmaxf(m, mx);
  // no valid key yet (a window's first tile): every p and the rescale are 0
  const float mb = mt == -INFINITY ? 0.0f : mt;
  const float sc = __builtin_amdgcn_exp2f(m - mb);  // 2^(-inf) = 0
  l *= sc;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    o[dt][0] *= sc; o[dt][1] *= sc; o[dt][2] *= sc; o[dt][3] *= sc;
  }
  m = mt;
  float pv[4][4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pv[kt][r] = __builtin_amdgcn_exp2f(sv[kt][r] - mb);  // masked: 2^(-inf) = 0
      l += pv[kt][r];
    }
  // P^T as bf16 hi + lo, two values per conversion
#pragma unroll
  for (int pp = 0; pp < 2; ++pp) {
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int r2 = 0; r2 < 2; ++r2) {
        const float a0 = pv[2 * pp + half][2 * r2], a1 = pv[2 * pp + half][2 * r2 + 1];
        const uint32_t hv = pack_bf2(a0, a1);
        const float h0 = __uint_as_float(hv << 16), h1 = __uint_as_float(hv & 0xFFFF0000u);
        hw[2 * half + r2] = hv;
        lw[2 * half + r2] = pack_bf2(a0 - h0, a1 - h1);
      }
    phi[pp] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    plo[pp] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  }
}

// NWD = 512 / blockDim: the 16-byte words of a K (and a V) tile per thread.
// QT: query tiles of 16 per block (a block serves 16 QT consecutive
// queries); blocks run from the last query tile down, so the longest
// (causal) blocks start first and short ones fill the CUs they free.
template <int NWD, int QT>
__global__ __launch_bounds__(512) void k_attn_prefill(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const uint16_t* __restrict__ sinks,
    uint16_t* __restrict__ out, int M, int Hq, int Hkv, int T_max, int window) {
  constexpr int VT = 64 + 8;  // V^T row stride (bf16): 8 pad breaks bank conflicts
  __shared__ __align__(16) uint16_t ks[64 * 64];
  __shared__ __align__(16) uint16_t vt[64 * VT];
  const int gkv = blockIdx.x, G = Hq / Hkv;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int j = lane & 15, g = lane >> 4;
  const int h = gkv * G + w;
  const int t0 = (gridDim.y - 1 - blockIdx.y) * 16 * QT;
  // Q^T fragments: query 16 qt + j, dims 32 h2 + 8 g .. + 7
  uint4 qf[QT][2];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int t = min(t0 + 16 * qt + j, M - 1);
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2)
      qf[qt][h2] = *reinterpret_cast<const uint4*>(q + ((size_t)t * Hq + h) * 64 + 32 * h2 + 8 * g);
  }
  pf_f32x4 o[QT][4];  // [qt][dt]: O^T[dim 16 dt + 4 g + r][query 16 qt + j]
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[qt][dt] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m[QT], l[QT];  // per query column (qt, j), log2 domain; l is this lane's partial sum
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) { m[qt] = -INFINITY; l[qt] = 0.0f; }
  const int hi_blk = min(M - 1, t0 + 16 * QT - 1);
  const int lo_blk = window > 0 ? max(0, t0 - window + 1) : 0;
  const uint16_t* kg = kc + (size_t)gkv * T_max * 64;
  const uint16_t* vg = vc + (size_t)gkv * T_max * 64;
  // a tile is 64 keys x 8 words of 16 bytes for K and for V; thread tid owns
  // words tid + i 512 / NWD (i < NWD), and the next tile's words are loaded
  // while the current one is computed
  constexpr int nthr = 512 / NWD;
  uint4 kn[NWD], vn[NWD];
  auto load_tile = [&](int jb) {
#pragma unroll
    for (int i = 0; i < NWD; ++i) {
      const int c = tid + i * nthr;
      const int key = min(jb + (c >> 3), T_max - 1);
      kn[i] = *reinterpret_cast<const uint4*>(kg + (size_t)key * 64 + (c & 7) * 8);
      vn[i] = *reinterpret_cast<const uint4*>(vg + (size_t)key * 64 + (c & 7) * 8);
    }
  };
  const int jstart = (lo_blk / 64) * 64;
  load_tile(jstart);
  for (int j0 = jstart; j0 <= hi_blk; j0 += 64) {
    __syncthreads();  // the previous tile is consumed
#pragma unroll
    for (int i = 0; i < NWD; ++i) {
      const int c = tid + i * nthr;
      const int kl = c >> 3, dq = (c & 7) * 8;
      *reinterpret_cast<uint4*>(&ks[kl * 64 + dq]) = kn[i];
      const uint32_t vw[4] = {vn[i].x, vn[i].y, vn[i].z, vn[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vt[(dq + 2 * e) * VT + kl] = (uint16_t)(vw[e] & 0xFFFFu);
        vt[(dq + 2 * e + 1) * VT + kl] = (uint16_t)(vw[e] >> 16);
      }
    }
    if (j0 + 64 <= hi_blk) load_tile(j0 + 64);  // in flight during this tile
    __syncthreads();
    // S^T tiles
    pf_f32x4 sacc[4][QT];  // [kt][qt]
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const uint4 ka0 = *reinterpret_cast<const uint4*>(&ks[(16 * kt + j) * 64 + 8 * g]);
      const uint4 ka1 = *reinterpret_cast<const uint4*>(&ks[(16 * kt + j) * 64 + 32 + 8 * g]);
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        pf_f32x4 acc = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pf_as_bf16x8(ka0), pf_as_bf16x8(qf[qt][0]),
                                                     acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pf_as_bf16x8(ka1), pf_as_bf16x8(qf[qt][1]),
                                                     acc, 0, 0, 0);
        sacc[kt][qt] = acc;
      }
    }
    // scale, mask (tiles that cross the diagonal or the window edge only),
    // online softmax; P^T (hi, lo) packed per key pair p
    const bool full = j0 + 63 <= t0 && (window <= 0 || j0 >= t0 + 16 * QT - window);
    uint4 phi[QT][2], plo[QT][2];  // [qt][p]
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      if (full)  // uniform
        attn_prefill_softmax<false, QT>(sacc, qt, t0, j0, j, g, window, m[qt], l[qt], o[qt],
                                        phi[qt], plo[qt]);
      else
        attn_prefill_softmax<true, QT>(sacc, qt, t0, j0, j, g, window, m[qt], l[qt], o[qt],
                                       phi[qt], plo[qt]);
    }
    // O^T += V^T P^T
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const uint16_t* vrow = &vt[(16 * dt + j) * VT];
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const uint2 va = *reinterpret_cast<const uint2*>(vrow + 32 * pp + 4 * g);
        const uint2 vb = *reinterpret_cast<const uint2*>(vrow + 32 * pp + 16 + 4 * g);
        const uint4 vfrag = make_uint4(va.x, va.y, vb.x, vb.y);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              pf_as_bf16x8(vfrag), pf_as_bf16x8(phi[qt][pp]), o[qt][dt], 0, 0, 0);
          o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              pf_as_bf16x8(vfrag), pf_as_bf16x8(plo[qt][pp]), o[qt][dt], 0, 0, 0);
        }
      }
    }
  }
  const float sk = __fmul_rn(bf2f(sinks[h]), 1.44269504088896340736f);  // log2 domain
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    float lt = l[qt];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    const float mt = fmaxf(m[qt], sk);
    const float sc = __builtin_amdgcn_exp2f(m[qt] - mt);
    const float inv = 1.0f / (lt * sc + __builtin_amdgcn_exp2f(sk - mt));
    const int t = t0 + 16 * qt + j;
    if (t < M) {
      uint16_t* dst = out + (size_t)t * Hq * 64 + (size_t)h * 64;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint32_t w0 = pack_bf2(o[qt][dt][0] * sc * inv, o[qt][dt][1] * sc * inv);
        const uint32_t w1 = pack_bf2(o[qt][dt][2] * sc * inv, o[qt][dt][3] * sc * inv);
        *reinterpret_cast<uint2*>(dst + 16 * dt + 4 * g) = make_uint2(w0, w1);
      }
    }
  }
}

// fp32 C[M][N] = A[M][K] W[N][K]^T + bias[N] for N <= kNarrowMaxN (the router
// logits of the prompt pass, N = E): a block owns 16 rows of A and all N
// columns (NT tiles of 16) on v_mfma_f32_16x16x32_bf16; its kNarrowWaves
// waves take the 32-element K chunks c = w, w + kNarrowWaves, ..., loading
// kNarrowBatch chunks at a time before their MFMAs (every load is used by
// an MFMA, chunks past K with both operands zeroed: a load used only under
// a branch is sunk into it by the compiler and waited for alone, which made
// this kernel one memory round trip per chunk, 26 us per prompt layer), then
// wave 0 adds the partial tiles in wave order and the bias.
constexpr int kNarrowWaves = 8;
template <int NT>
__global__ __launch_bounds__(64 * kNarrowWaves) void k_gemm_narrow_f32(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ W,
    const uint16_t* __restrict__ bias, float* __restrict__ C, int M, int N, int K) {
  __shared__ pf_f32x4 red[kNarrowWaves - 1][NT][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int r0 = blockIdx.x * 16;
  const uint16_t* arow = A + (size_t)min(r0 + j, M - 1) * K + 8 * g;
  const uint16_t* wrow[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) wrow[nt] = W + (size_t)min(16 * nt + j, N - 1) * K + 8 * g;
  pf_f32x4 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int nch = K / 32;
  const uint4 z = make_uint4(0u, 0u, 0u, 0u);
  for (int c0 = w; c0 < nch; c0 += kNarrowWaves * kNarrowBatch) {
    uint4 av[kNarrowBatch], wv[kNarrowBatch][NT];
#pragma unroll
    for (int i = 0; i < kNarrowBatch; ++i) {
      const bool ok = c0 + kNarrowWaves * i < nch;
      const int c = min(c0 + kNarrowWaves * i, nch - 1);  // past the end: re-read, zeroed
      const uint4 a = *reinterpret_cast<const uint4*>(arow + 32 * (size_t)c);
      av[i] = ok ? a : z;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const uint4 b = *reinterpret_cast<const uint4*>(wrow[nt] + 32 * (size_t)c);
        wv[i][nt] = ok ? b : z;
      }
    }
    // keep the scheduler from placing the selects (which wait for their
    // loads) between the loads
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kNarrowBatch; ++i)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pf_as_bf16x8(av[i]),
                                                          pf_as_bf16x8(wv[i][nt]), acc[nt], 0,
                                                          0, 0);
  }
  if (w > 0) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) red[w - 1][nt][lane] = acc[nt];
  }
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    pf_f32x4 tot = acc[nt];
#pragma unroll
    for (int v = 0; v < kNarrowWaves - 1; ++v) {
      const pf_f32x4 p = red[v][nt][lane];
      tot[0] += p[0]; tot[1] += p[1]; tot[2] += p[2]; tot[3] += p[3];
    }
    const int col = 16 * nt + j;
    if (col >= N) continue;
    const float b = bias != nullptr ? bf2f(bias[col]) : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = r0 + 4 * g + r;  // D row of lane (j, g), register r
      if (row < M) C[(size_t)row * N + col] = tot[r] + b;
    }
  }
}

static void launch_gemm_narrow_f32(const uint16_t* A, const uint16_t* W, const uint16_t* bias,
                                   float* C, int M, int N, int K, hipStream_t st) {
  const dim3 grid((M + 15) / 16);
  switch ((N + 15) / 16) {
    case 1: hipLaunchKernelGGL(k_gemm_narrow_f32<1>, grid, dim3(64 * kNarrowWaves), 0, st, A, W, bias, C, M, N, K); break;
    case 2: hipLaunchKernelGGL(k_gemm_narrow_f32<2>, grid, dim3(64 * kNarrowWaves), 0, st, A, W, bias, C, M, N, K); break;
    case 3: hipLaunchKernelGGL(k_gemm_narrow_f32<3>, grid, dim3(64 * kNarrowWaves), 0, st, A, W, bias, C, M, N, K); break;
    default: hipLaunchKernelGGL(k_gemm_narrow_f32<4>, grid, dim3(64 * kNarrowWaves), 0, st, A, W, bias, C, M, N, K); break;
  }
}

void launch_attn_prefill(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                         const uint16_t* sinks, uint16_t* out, int M, int Hq, int Hkv,
                         int T_max, int window, hipStream_t st) {
  // 32 queries per block: 2047 prompt rows give 64 blocks per kv head, run
  // longest first (26.4 ms per MXFP8 20b pass against 27.3 with 64 queries
  // and 26.5 with 16)
  constexpr int QT = 2;
  dim3 grid(Hkv, (M + 16 * QT - 1) / (16 * QT));
  const int G = Hq / Hkv;  // 1, 2, 4 or 8 (checked by the callers)
#define AP_LAUNCH(NWD)                                                                      \
  hipLaunchKernelGGL((k_attn_prefill<NWD, QT>), grid, dim3(64 * G), 0, st, q, kc, vc, sinks, \
                     out, M, Hq, Hkv, T_max, window)
  if (G == 8) AP_LAUNCH(1);
  else if (G == 4) AP_LAUNCH(2);
  else if (G == 2) AP_LAUNCH(4);
  else AP_LAUNCH(8);
#undef AP_LAUNCH
}

}  // namespace neon

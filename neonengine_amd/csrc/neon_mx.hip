// neon_mx.hip -- batched decode steps (2 <= B <= 64 rows) on the matrix cores.
//
// The exact batched kernels keep every dot product in the canonical fp32
// order of the batch-1 kernels, which makes them VALU-bound from B = 16 on.
// Here each weight row is read once per step and the B rows ride in the M
// dimension of v_mfma_f32_16x16x32_bf16 (fp32 accumulate):
//   - projections and lm_head (k_mx_gemv): a block owns 16 weight rows and
//     its 4 waves split K;
//   - experts (k_mx_moe16): a block owns 64 kMxMoeTiles rows of one used
//     expert for up to 16 of its (row, slot) pairs, whose activation rows it
//     stages in LDS; the used experts and their pairs come from
//     k_topk_route; MXFP4 rows go through v_cvt_scalef32_pk_bf16_fp4 (E2M1 x
//     2^(s-127) is a bf16 value, so the dequantisation is exact);
//   - the weights come from copies packed in MFMA lane order (k_mx_pack_*),
//     so that a load instruction reads 1 KB contiguous;
//   - attention (k_mx_attn): K Q^T and V^T P^T with a kv head's query heads
//     as the query columns.
// Only the order of fp32 additions differs from the exact path (products
// of two bf16 values are exact in fp32), and every rounding point, bias,
// SwiGLU clamp and the slot-ordered combine are the exact path's
// (HFM:82-112, 347-376).
#include "neon_common.hpp"
#include "neon_internal.hpp"

namespace neon {

typedef __bf16 mx_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 mx_bf16x2 __attribute__((ext_vector_type(2)));
typedef float mx_f32x4 __attribute__((ext_vector_type(4)));

enum { MX_STORE = 0, MX_RESID = 1, MX_LOGITS = 2, MX_GATE_UP = 3, MX_DOWN = 4 };

typedef uint32_t mx_u32x4 __attribute__((ext_vector_type(4)));

// weights are read once per step: non-temporal loads keep them out of the way
__device__ __forceinline__ uint4 mx_load_nt(const void* p) {
  const mx_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const mx_u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ mx_bf16x8 mx_as_bf16x8(const uint4& v) {
  return __builtin_bit_cast(mx_bf16x8, v);
}

// 8 E2M1 codes (one dword, low nibble = even element) times 2^(s-127) as bf16
__device__ __forceinline__ mx_bf16x8 mx_fp4x8(uint32_t c, float scale) {
  const mx_bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, scale, 0);
  const mx_bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, scale, 1);
  const mx_bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, scale, 2);
  const mx_bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, scale, 3);
  mx_bf16x8 r;
  r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
  r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
  return r;
}

__device__ __forceinline__ void mx_argmax_step(float& v, int& i, int off) {
  const float ov = __shfl_xor(v, off);
  const int oi = __shfl_xor(i, off);
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

// Epilogue of the dense matrix-core GEMVs.  Every wave hands its partial
// tiles to LDS; row tile bt is then finished by wave bt % WAVES, which adds
// the WAVES partials in wave order and applies the mode's bias / residual /
// bf16 rounding (or fp32 logits and the per-block (max, lowest index)
// partials).  The bias and the residual values a wave will need are
// requested when the kernel starts (mx_epi_prefetch), so the finishing waves
// do not wait for a load round trip at the end.  At the 20b O shape
// (2880 x 4096, B = 64) wave 0 finishing all four tiles with the loads at
// the end took 17.6 against 12.8 us for the bare product.
template <int BT, int WAVES>
struct MxEpiPre {
  static constexpr int TPW = (BT + WAVES - 1) / WAVES;  // tiles a wave finishes
  float bias;
  uint16_t res[TPW][4];
};

template <int BT, int MODE, int WAVES>
__device__ __forceinline__ void mx_epi_prefetch(const MxArgs& a, MxEpiPre<BT, WAVES>& p, int w,
                                                int n0, int j, int g, int N, int R) {
  const int n = n0 + j;
  // unconditional (a valid address when there is no bias): a load under a
  // branch would be waited for where the branches join
  p.bias = 0.0f;
  if constexpr (MODE != MX_LOGITS) {
    const uint16_t bq = load_pinned_u16(a.bias != nullptr ? a.bias + min(n, N - 1) : a.y);
    p.bias = a.bias != nullptr ? bf2f(bq) : 0.0f;
  }
  if constexpr (MODE == MX_RESID) {
#pragma unroll
    for (int i = 0; i < MxEpiPre<BT, WAVES>::TPW; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ri = 16 * (w + WAVES * i) + 4 * g + r;
        p.res[i][r] = load_pinned_u16(a.y + (size_t)min(ri, R - 1) * N + n);
      }
  }
}

template <int BT, int MODE, int WAVES = 4>
__device__ __forceinline__ void mx_gemv_epilogue(const MxArgs& a, const mx_f32x4 (&acc)[BT],
                                                 mx_f32x4 (&red)[WAVES][BT][64],
                                                 const MxEpiPre<BT, WAVES>& pre, int lane,
                                                 int w, int n0, int j, int g, int N, int R) {
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) red[w][bt][lane] = acc[bt];
  __syncthreads();
  const int n = n0 + j;
#pragma unroll
  for (int i = 0; i < MxEpiPre<BT, WAVES>::TPW; ++i) {
    const int bt = w + WAVES * i;
    if (bt >= BT || 16 * bt >= R) break;  // uniform per wave
    mx_f32x4 tot = red[0][bt][lane];
#pragma unroll
    for (int v = 1; v < WAVES; ++v) {
      const mx_f32x4 p = red[v][bt][lane];
      tot[0] = __fadd_rn(tot[0], p[0]); tot[1] = __fadd_rn(tot[1], p[1]);
      tot[2] = __fadd_rn(tot[2], p[2]); tot[3] = __fadd_rn(tot[3], p[3]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ri = 16 * bt + 4 * g + r;  // row of A / output row
      const bool ok = ri < R;
      const float d = tot[r];
      if constexpr (MODE == MX_LOGITS) {
        if (ok) a.out_f[(size_t)ri * N + n] = d;
        float bv = ok ? d : -INFINITY;
        int bi = n;
        mx_argmax_step(bv, bi, 1);
        mx_argmax_step(bv, bi, 2);
        mx_argmax_step(bv, bi, 4);
        mx_argmax_step(bv, bi, 8);
        if (ok && j == 0) {
          a.part_val[(size_t)ri * gridDim.x + blockIdx.x] = bv;
          a.part_idx[(size_t)ri * gridDim.x + blockIdx.x] = bi;
        }
      } else if (ok) {
        const float v = a.bias ? __fadd_rn(d, pre.bias) : d;
        const size_t o = (size_t)ri * N + n;
        if (MODE == MX_STORE) a.y[o] = f2bf(v);
        else a.y[o] = f2bf(__fadd_rn(bf2f(pre.res[i][r]), bf2f(f2bf(v))));
      }
    }
  }
}

// Projections and lm_head: a block owns weight rows n0 .. n0 + 15 for all B
// rows, and its 4 waves split K.  BT = row tiles of 16 (B <= 16 BT); IT = K
// iterations per wave (K <= 512 IT).  Lane (j, g) reads elements
// 128 (4 i + w) + 32 t + 8 g .. + 7 of its row in step t of iteration i: one
// load instruction covers 64 contiguous bytes of each of 16 rows in the
// checkpoint layout, or 1 KB contiguous in the packed copy (PACKED).
template <int BT, int IT, int MODE, bool PACKED>
__global__ __launch_bounds__(256) void k_mx_gemv(MxArgs a) {
  __shared__ mx_f32x4 red[4][BT][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int N = a.N, K = a.K, R = a.B;
  const int n0 = blockIdx.x * 16;
  MxEpiPre<BT, 4> pre;
  mx_epi_prefetch<BT, MODE, 4>(a, pre, w, n0, j, g, N, R);
  // weight loads first (the stream), then the activation rows
  uint4 wq[IT][4];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    if constexpr (PACKED) {
      // [N/16][NCH][t][g][j][8]: lane l = j + 16 g reads piece ... * 64 + l
      const int NCH = (K + 127) / 128;
      const int ch = min(4 * it + w, NCH - 1);
      const uint16_t* P = static_cast<const uint16_t*>(a.Wp);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        wq[it][t] = mx_load_nt(P + ((((size_t)blockIdx.x * NCH + ch) * 4 + t) * 64 + lane) * 8);
    } else {
      const uint16_t* wrow = static_cast<const uint16_t*>(a.W) + (size_t)(n0 + j) * K;
      const int base = 128 * (4 * it + w);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int el = base + 32 * t < K ? base + 32 * t + 8 * g : 8 * g;
        wq[it][t] = mx_load_nt(wrow + el);
      }
    }
  }
  const uint16_t* xrow[BT];
  bool rv[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) {
    const int r = 16 * bt + j;
    rv[bt] = r < R;
    xrow[bt] = a.x + (size_t)(rv[bt] ? r : R - 1) * K;
  }
  mx_f32x4 acc[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) acc[bt] = mx_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int base = 128 * (4 * it + w);
    uint4 xq[BT][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const bool ok = base + 32 * t < K;
      const int el = ok ? base + 32 * t + 8 * g : 8 * g;
#pragma unroll
      for (int bt = 0; bt < BT; ++bt) {
        const uint4 v = *reinterpret_cast<const uint4*>(xrow[bt] + el);
        // a zero A value drops a padded element range or row
        xq[bt][t] = (ok && rv[bt]) ? v : make_uint4(0u, 0u, 0u, 0u);
      }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const mx_bf16x8 bw = mx_as_bf16x8(wq[it][t]);
#pragma unroll
      for (int bt = 0; bt < BT; ++bt)
        if (16 * bt < R)
          acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mx_as_bf16x8(xq[bt][t]), bw, acc[bt],
                                                            0, 0, 0);
    }
  }
  mx_gemv_epilogue<BT, MODE, 4>(a, acc, red, pre, lane, w, n0, j, g, N, R);
}

// k_mx_gemv over the packed copy with the weights and activation rows of
// each K iteration loaded one iteration ahead (two register sets), instead
// of all of the wave's weight loads up front: more waves per SIMD and the
// next iteration's loads in flight during this one's MFMAs.  Same lane map,
// same order of every fp32 addition, so the same bits as k_mx_gemv.
// Measured faster for one row tile (B <= 16: QKV 13.0 -> 11.5 us, O
// 11.0 -> 9.7 us at the 20b shape, B = 16) and slower from BT = 2 on (two
// sets of BT activation tiles), where k_mx_gemv stays.
template <int BT, int IT, int MODE, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_mx_gemv_db(MxArgs a) {
  __shared__ mx_f32x4 red[WAVES][BT][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int N = a.N, K = a.K, R = a.B;
  const int n0 = blockIdx.x * 16;
  MxEpiPre<BT, WAVES> pre;
  mx_epi_prefetch<BT, MODE, WAVES>(a, pre, w, n0, j, g, N, R);
  const int NCH = (K + 127) / 128;
  const uint16_t* P = static_cast<const uint16_t*>(a.Wp);
  const uint16_t* xrow[BT];
  bool rv[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) {
    const int r = 16 * bt + j;
    rv[bt] = r < R;
    xrow[bt] = a.x + (size_t)(rv[bt] ? r : R - 1) * K;
  }
  auto load_w = [&](int it, uint4 (&wq)[4]) {
    const int ch = min(WAVES * it + w, NCH - 1);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      wq[t] = mx_load_nt(P + ((((size_t)blockIdx.x * NCH + ch) * 4 + t) * 64 + lane) * 8);
  };
  auto load_x = [&](int it, uint4 (&xq)[BT][4]) {
    const int base = 128 * (WAVES * it + w);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const bool ok = base + 32 * t < K;
      const int el = ok ? base + 32 * t + 8 * g : 8 * g;
#pragma unroll
      for (int bt = 0; bt < BT; ++bt) {
        const uint4 v = *reinterpret_cast<const uint4*>(xrow[bt] + el);
        xq[bt][t] = (ok && rv[bt]) ? v : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  mx_f32x4 acc[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) acc[bt] = mx_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  uint4 wc[4], wn[4], xc[BT][4], xn[BT][4];
  load_w(0, wc);
  load_x(0, xc);
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    if (it + 1 < IT) { load_w(it + 1, wn); load_x(it + 1, xn); }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const mx_bf16x8 bw = mx_as_bf16x8(wc[t]);
#pragma unroll
      for (int bt = 0; bt < BT; ++bt)
        if (16 * bt < R)
          acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mx_as_bf16x8(xc[bt][t]), bw, acc[bt],
                                                            0, 0, 0);
    }
    if (it + 1 < IT) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        wc[t] = wn[t];
#pragma unroll
        for (int bt = 0; bt < BT; ++bt) xc[bt][t] = xn[bt][t];
      }
    }
  }
  mx_gemv_epilogue<BT, MODE, WAVES>(a, acc, red, pre, lane, w, n0, j, g, N, R);
}

// k_mx_gemv over the packed weights with the activation rows in the packed
// activation layout (MxArgs::xp, written by launch_rmsnorm_packed): every
// operand load is 1 KB contiguous, the weights stream one K iteration ahead
// (two register sets) and each iteration's activation tiles are loaded as it
// starts.  Same lane map and the same order of every fp32 addition as
// k_mx_gemv, so the same bits.  Measured at the 20b shape, B = 16 / 32 / 64:
// QKV 11.6 / 19.4 / 38.2 -> 9.8 / 13.9 / 23.3 us, lm_head 276 / 405 / 753 ->
// 245 / 293 / 582 us (377 us at B = 64 with 8 waves).  The O projection
// (K = 4096, 8 iterations) runs faster with all of its weights requested at
// the start (DEEP): 10.4 / 16.0 / 28.3 -> 9.5 / 12.9 / 19.9 us; QKV does not
// (34.0 us at B = 64).
template <int BT, int IT, int MODE, int WAVES, bool DEEP = false>
__global__ __launch_bounds__(64 * WAVES) void k_mx_gemv_px(MxArgs a) {
  __shared__ mx_f32x4 red[WAVES][BT][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int N = a.N, K = a.K, R = a.B;
  const int n0 = blockIdx.x * 16;
  MxEpiPre<BT, WAVES> pre;
  mx_epi_prefetch<BT, MODE, WAVES>(a, pre, w, n0, j, g, N, R);
  const int NCH = (K + 127) / 128;
  const uint16_t* P = static_cast<const uint16_t*>(a.Wp);
  const uint16_t* X = a.xp;
  // weights DEPTH iterations ahead: one (two register sets), or all of the
  // wave's at the start (DEEP)
  constexpr int DEPTH = DEEP ? IT : 1;
  uint4 wq[DEPTH + 1][4];
  auto load_w = [&](int it, uint4 (&dst)[4]) {
    const int ch = min(WAVES * it + w, NCH - 1);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      dst[t] = mx_load_nt(P + ((((size_t)blockIdx.x * NCH + ch) * 4 + t) * 64 + lane) * 8);
  };
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) load_w(d, wq[d]);
  mx_f32x4 acc[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) acc[bt] = mx_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    if (it + DEPTH < IT) load_w(it + DEPTH, wq[(it + DEPTH) % (DEPTH + 1)]);
    // chunks past K: a zero A operand (the packed rows are zero past K only
    // up to the last chunk)
    const bool okc = WAVES * it + w < NCH;
    const int ch = min(WAVES * it + w, NCH - 1);
    uint4 xq[BT][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int bt = 0; bt < BT; ++bt) {
        const uint4 v = *reinterpret_cast<const uint4*>(
            X + ((((size_t)bt * NCH + ch) * 4 + t) * 64 + lane) * 8);
        xq[bt][t] = okc ? v : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const mx_bf16x8 bw = mx_as_bf16x8(wq[it % (DEPTH + 1)][t]);
#pragma unroll
      for (int bt = 0; bt < BT; ++bt)
        if (16 * bt < R)
          acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mx_as_bf16x8(xq[bt][t]), bw, acc[bt],
                                                            0, 0, 0);
    }
  }
  mx_gemv_epilogue<BT, MODE, WAVES>(a, acc, red, pre, lane, w, n0, j, g, N, R);
}

// k_mx_gemv over the packed weights and packed activations with the
// activations shared through LDS.  A block holds WT weight tiles (16 rows
// each) and splits K into KS parts: wave w owns tile w % WT over the 128-
// element K chunks of part w / WT, and the WT waves of a part read each
// chunk of the BT activation tiles from one LDS copy instead of each
// fetching it from L2.  Every operand piece (1 KB: the activation tiles of a
// chunk, each wave's weight tile of a chunk) is copied into LDS by
// global_load_lds_dwordx4 (lane l writes bytes 16 l .. 16 l + 15 of the
// piece), NS - 1 chunks ahead in a ring of NS stages, so no register holds
// an operand in flight.  A wave issues the same number of pieces for every
// step (past its part's end it re-reads the last chunk into a stage that is
// never consumed), so "the step's pieces have landed" is one fixed vmcnt.
// Per tile the fp32 sums run over each part's chunks in order, with each
// chunk's 4 MFMAs in order, and the parts are added in part order; only the
// order of fp32 additions differs from k_mx_gemv.  Measured at the 20b
// shape, B = 64, weights cold (one launch in isolation, one part): lm_head
// (8 tiles, 3 stages) 380 -> 251 us, QKV (2 tiles, 4 stages) 15.6 -> 12.0
// us; in the step, QKV and O gain from shorter chains (K in 2 or 4 parts,
// mx_lx_shape).
#if defined(__HIP_DEVICE_COMPILE__)
#define MX_LDS_LOAD(g, l) __builtin_amdgcn_global_load_lds((g), (l), 16, 0, 0)
#else
#define MX_LDS_LOAD(g, l) ((void)(g), (void)(l))
#endif
template <int N>
__device__ __forceinline__ void mx_wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int BT, int MODE, int WT, int KS, int NS>
__global__ __launch_bounds__(64 * WT * KS) void k_mx_gemv_lx(MxArgs a) {
  // WT weight tiles per block, K split KS ways: wave w owns tile w % WT for
  // the K chunks of part kh = w / WT; the parts' partial tiles are added in
  // part order at the end.  Every stage holds, per part, the chunk's PX
  // activation pieces and the WT tiles' 4 weight pieces each.
  extern __shared__ uint4 mx_lds[];
  constexpr int PX = 4 * BT;                 // activation pieces per chunk (shared)
  constexpr int PART = PX + 4 * WT;          // pieces per part and stage
  constexpr int STAGE = KS * PART;
  constexpr int LX = (PX + WT - 1) / WT;
  constexpr int LT = LX + 4;                 // pieces one wave issues per chunk
  static_assert(NS >= 2 && (NS - 2) * LT <= 63, "chunk arrival must fit one vmcnt");
  // the launcher picks BT = ceil(B / 16), so every row tile holds rows
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wt = w % WT, kh = w / WT;
  const int j = lane & 15, g = lane >> 4;
  const int N = a.N, K = a.K, R = a.B;
  const int NCH = (K + 127) / 128, NT = N / 16;
  const int CPK = (NCH + KS - 1) / KS;       // chunks per part
  const int cb = kh * CPK;                   // this wave's first chunk
  const int tile = blockIdx.x * WT + wt;
  const int tl = min(tile, NT - 1);          // waves past N load a real tile, store nothing
  const uint16_t* P = static_cast<const uint16_t*>(a.Wp);
  const uint16_t* X = a.xp;
  // the epilogue's bias and residual values, requested now (see
  // mx_gemv_epilogue)
  const int nl = 16 * tl + j;
  float bias_n = 0.0f;
  if constexpr (MODE != MX_LOGITS) {  // unconditional: see mx_epi_prefetch
    const uint16_t bq = load_pinned_u16(a.bias != nullptr ? a.bias + nl : a.y);
    bias_n = a.bias != nullptr ? bf2f(bq) : 0.0f;
  }
  uint16_t res[BT][4];
  if constexpr (MODE == MX_RESID) {
#pragma unroll
    for (int bt = 0; bt < BT; ++bt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        res[bt][r] = load_pinned_u16(a.y + (size_t)min(16 * bt + 4 * g + r, R - 1) * N + nl);
  }
  auto issue = [&](int i, int stage) {
    const int ch = min(cb + i, NCH - 1);  // past the part's end: a copy never consumed
    uint4* base = mx_lds + (stage * STAGE + kh * PART) * 64;
#pragma unroll
    for (int ii = 0; ii < LX; ++ii) {
      const int q = min(wt + WT * ii, PX - 1);  // a duplicate writes the same bytes
      MX_LDS_LOAD(X + ((((size_t)(q >> 2) * NCH + ch) * 4 + (q & 3)) * 64 + lane) * 8,
                  base + q * 64);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
      MX_LDS_LOAD(P + ((((size_t)tl * NCH + ch) * 4 + t) * 64 + lane) * 8,
                  base + (PX + 4 * wt + t) * 64);
  };
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) issue(s, s);
  mx_f32x4 acc[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) acc[bt] = mx_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int i0 = 0; i0 < CPK; i0 += NS) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int i = i0 + s;
      if (i >= CPK) break;  // uniform
      mx_wait_vmcnt<(NS - 2) * LT>();  // this wave's pieces of step i have landed
      // every wave's have, and every wave's reads of stage (i - 1) % NS are
      // complete (lgkmcnt 0), so the copies issued next may overwrite it.  No
      // fence: the waits on the copies are the vmcnt above
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      issue(i + NS - 1, (s + NS - 1) % NS);
      __builtin_amdgcn_sched_barrier(0);
      if (cb + i < NCH) {  // uniform per wave (the last part may be shorter)
        const uint4* st = mx_lds + (s * STAGE + kh * PART) * 64;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const mx_bf16x8 bw = mx_as_bf16x8(st[(PX + 4 * wt + t) * 64 + lane]);
#pragma unroll
          for (int bt = 0; bt < BT; ++bt)  // BT = ceil(R / 16): every tile has rows
            acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                mx_as_bf16x8(st[(4 * bt + t) * 64 + lane]), bw, acc[bt], 0, 0, 0);
        }
      }
    }
  }
  mx_wait_vmcnt<0>();  // the ring's last (unused) copies have landed
  if constexpr (KS > 1) {
    // parts 1 .. KS - 1 hand their tiles over through the (now idle) ring
    mx_f32x4* red = reinterpret_cast<mx_f32x4*>(mx_lds);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (kh > 0) {
#pragma unroll
      for (int bt = 0; bt < BT; ++bt) red[(((kh - 1) * WT + wt) * BT + bt) * 64 + lane] = acc[bt];
    }
    __syncthreads();
    if (kh > 0) return;
#pragma unroll
    for (int v = 1; v < KS; ++v)
#pragma unroll
      for (int bt = 0; bt < BT; ++bt) {
        const mx_f32x4 p = red[(((v - 1) * WT + wt) * BT + bt) * 64 + lane];
        acc[bt][0] = __fadd_rn(acc[bt][0], p[0]); acc[bt][1] = __fadd_rn(acc[bt][1], p[1]);
        acc[bt][2] = __fadd_rn(acc[bt][2], p[2]); acc[bt][3] = __fadd_rn(acc[bt][3], p[3]);
      }
  }
  if (tile >= NT) return;
  const int n = 16 * tile + j;
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ri = 16 * bt + 4 * g + r;
      const bool ok = ri < R;
      const float d = acc[bt][r];
      if constexpr (MODE == MX_LOGITS) {
        if (ok) a.out_f[(size_t)ri * N + n] = d;
        float bv = ok ? d : -INFINITY;
        int bi = n;
        mx_argmax_step(bv, bi, 1);
        mx_argmax_step(bv, bi, 2);
        mx_argmax_step(bv, bi, 4);
        mx_argmax_step(bv, bi, 8);
        if (ok && j == 0) {  // partials per 16-column tile, as k_mx_gemv's per block
          a.part_val[(size_t)ri * NT + tile] = bv;
          a.part_idx[(size_t)ri * NT + tile] = bi;
        }
      } else if (ok) {
        const float v = a.bias ? __fadd_rn(d, bias_n) : d;
        const size_t o = (size_t)ri * N + n;
        if (MODE == MX_STORE) a.y[o] = f2bf(v);
        else a.y[o] = f2bf(__fadd_rn(bf2f(res[bt][r]), bf2f(f2bf(v))));
      }
    }
  }
}
#undef MX_LDS_LOAD

template <int BT, int MODE, int WT, int KS, int NS>
static void launch_mx_gemv_lx(const MxArgs& a, hipStream_t st) {
  constexpr int bytes = NS * KS * (4 * BT + 4 * WT) * 1024;
  static_assert(bytes <= 160 * 1024, "LDS");
  static const hipError_t optin =
      hipFuncSetAttribute(reinterpret_cast<const void*>(k_mx_gemv_lx<BT, MODE, WT, KS, NS>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  (void)optin;  // a refused opt-in surfaces as the launch's error
  const int nt = a.N / 16;
  hipLaunchKernelGGL((k_mx_gemv_lx<BT, MODE, WT, KS, NS>), dim3((nt + WT - 1) / WT),
                     dim3(64 * WT * KS), bytes, st, a);
}

// Block shape of k_mx_gemv_lx per mode: weight tiles per block, ring stages
// and K parts; tiles 0 = k_mx_gemv_px instead.  Defaults measured on the 20b
// step (tok/s at B = 64 / 32 / 16 after 16-token prompts): one K part for
// every mode, QKV 2 tiles x 4 stages and lm_head 8 x 3, O on k_mx_gemv_px:
// 15,832 / 8977 / 5078; QKV with its K in two parts (2 tiles, 3 stages) and
// O on 1 tile with 2 parts (4 stages): 16,240 / 9118 / 5121; O with 4 parts
// (2 stages): 16,353 / 9081 / 5062.  The K parts are used from 49 rows: below
// that they gained under 2%, and at B = 16 their summation order flipped
// more routing near-ties in the free-routing check against the oracle
// (median row error 0.446 against its 0.433 bar).  At B = 64 one block of
// these shapes fills a CU's LDS, so QKV runs 160 blocks and O 180 on the 256
// CUs; shapes with half the LDS or less (two or more blocks per CU: QKV
// 1,2,2 / 2,2,2 / 1,2,1 / 2,2,1, O 1,2,2 / 2,2,2 / 1,2,1) were all slower
// (17,479 / 17,808 / 17,042 / 17,230 and 17,591 / 17,494 / 16,415 tok/s
// against 17,982).  NEON_MX_LX_STORE / _RESID / _LOGITS =
// "W,NS[,KS]" override them for comparisons (the shapes listed in
// launch_mx_gemv_lx_sel).
struct MxLxShape { int waves, ns, ks; };
static MxLxShape mx_lx_shape(int mode, int bt) {
  static MxLxShape env[3] = {{-2, 0, 1}, {-2, 0, 1}, {-2, 0, 1}};
  if (mode < 0 || mode > 2) return {0, 0, 1};
  if (env[mode].waves == -2) {
    static const char* names[3] = {"NEON_MX_LX_STORE", "NEON_MX_LX_RESID", "NEON_MX_LX_LOGITS"};
    MxLxShape v = {-1, 0, 1};  // -1: the default below
    if (const char* e = getenv(names[mode])) {
      int w = -1, ns = -1, ks = 1;
      if (sscanf(e, "%d,%d,%d", &w, &ns, &ks) >= 1) {
        v.waves = w;
        v.ns = ns > 0 ? ns : 3;
        v.ks = ks > 0 ? ks : 1;
      }
    }
    env[mode] = v;
  }
  if (env[mode].waves >= 0) return env[mode];
  if (mode == MX_STORE) return bt >= 4 ? MxLxShape{2, 3, 2} : MxLxShape{2, 4, 1};
  if (mode == MX_RESID) return bt >= 4 ? MxLxShape{1, 2, 4} : MxLxShape{0, 0, 1};
  return {8, 3, 1};
}

template <int MODE>
static bool launch_mx_gemv_lx_sel(const MxArgs& a, hipStream_t st) {
  const int bt = (a.B + 15) / 16;
  if (bt > 4) return false;
  const MxLxShape v = mx_lx_shape(MODE, bt);
#define LX_SEL(W, NS, KS)                                                   \
  if (v.waves == W && v.ns == NS && v.ks == KS) {                           \
    switch (bt) {                                                           \
      case 1: launch_mx_gemv_lx<1, MODE, W, KS, NS>(a, st); break;          \
      case 2: launch_mx_gemv_lx<2, MODE, W, KS, NS>(a, st); break;          \
      case 3: launch_mx_gemv_lx<3, MODE, W, KS, NS>(a, st); break;          \
      default: launch_mx_gemv_lx<4, MODE, W, KS, NS>(a, st); break;         \
    }                                                                       \
    return true;                                                            \
  }
  LX_SEL(1, 4, 1) LX_SEL(2, 4, 1) LX_SEL(4, 3, 1) LX_SEL(8, 3, 1)
  LX_SEL(1, 4, 2) LX_SEL(2, 3, 2) LX_SEL(1, 2, 4) LX_SEL(4, 2, 2)
#undef LX_SEL
  return false;  // 0 (or an unsupported shape): k_mx_gemv_px
}

// Standalone MXFP4 GEMV on the matrix cores (neon_mxfp4_gemv at B >= 16):
// y[b][n] = bf16(sum_k x[b][k] dq(W[n][k]) + bias[n]) with the weights in the
// checkpoint layout (codes [N][K/2], scales [N][K/32]).  A block owns rows
// n0 .. n0 + 15 and up to 64 batch rows (BT tiles of 16); its 4 waves split
// K.  In K step q (128 elements = 4 MXFP4 units) lane (j, g) loads all of
// unit 4 q + g of row n0 + j (16 code bytes and its scale) and feeds it to
// 4 MFMAs, 8 elements each; the x operand is loaded with the same lane-to-
// unit map, so every k is summed exactly once (in another order than the
// checkpoint's).  E2M1 x 2^(s - 127) converts exactly to bf16 (scale byte
// 0xFF gives NaN), products of two bf16 values are exact in fp32, and the
// 4 waves' partial tiles are added in wave order; only the order of the fp32
// additions differs from the canonical GEMV.
template <int BT, int IT, int WV>
__global__ __launch_bounds__(64 * WV) void k_mxfp4_gemv_mfma(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ scales,
    const uint16_t* __restrict__ bias, const uint16_t* __restrict__ x,
    uint16_t* __restrict__ y, int N, int K, int B) {
  __shared__ mx_f32x4 red[WV][BT][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int U = K / 32;
  const int n0 = blockIdx.x * 16;
  const int nr = min(n0 + j, N - 1);  // rows past N re-read row N - 1 (not stored)
  // the bias of column n0 + j, requested now (the epilogue then waits for no load)
  const uint16_t bq = load_pinned_u16(bias != nullptr ? bias + nr : x);  // unconditional
  const float bv = (bias != nullptr && n0 + j < N) ? bf2f(bq) : 0.0f;
  const int b0 = blockIdx.y * 16 * BT;
  // this wave's units: 4 (w + WV i) + g for i < IT (clamped; zero A past U)
  uint4 wc[IT];
  uint32_t ws[IT];
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int u = min(4 * (w + WV * i) + g, U - 1);
    wc[i] = mx_load_nt(codes + (size_t)nr * (K / 2) + (size_t)u * 16);
    ws[i] = __builtin_nontemporal_load(scales + (size_t)nr * U + u);
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint16_t* xrow[BT];
  bool rv[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) {
    const int r = b0 + 16 * bt + j;
    rv[bt] = r < B;
    xrow[bt] = x + (size_t)(rv[bt] ? r : B - 1) * K;
  }
  mx_f32x4 acc[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) acc[bt] = mx_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // each iteration's input rows load as it starts (loading the next
  // iteration's during this one's MFMAs measured no faster)
  auto x_load = [&](int i, uint4 (&xq)[BT][4]) {
    const int u_raw = 4 * (w + WV * i) + g;
    const bool uok = u_raw < U;
    const int u = min(u_raw, U - 1);
#pragma unroll
    for (int bt = 0; bt < BT; ++bt)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint4 v = reinterpret_cast<const uint4*>(xrow[bt] + (size_t)u * 32)[t];
        xq[bt][t] = (uok && rv[bt]) ? v : make_uint4(0u, 0u, 0u, 0u);  // zero A drops it
      }
  };
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    uint4 xq[BT][4];
    x_load(i, xq);
    const float sc = ws[i] == 0xFFu ? __builtin_nanf("")
                                    : __builtin_amdgcn_ldexpf(1.0f, (int)ws[i] - 127);
    const uint32_t cw[4] = {wc[i].x, wc[i].y, wc[i].z, wc[i].w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const mx_bf16x8 bw = mx_fp4x8(cw[t], sc);
#pragma unroll
      for (int bt = 0; bt < BT; ++bt)
        acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mx_as_bf16x8(xq[bt][t]), bw, acc[bt],
                                                          0, 0, 0);
    }
  }
  // every wave hands its partial tiles to LDS; tile bt is finished by wave
  // bt % WV, adding the WV partials in wave order
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) red[w][bt][lane] = acc[bt];
  __syncthreads();
  const int n = n0 + j;
  if (n >= N) return;
#pragma unroll
  for (int bt = w; bt < BT; bt += WV) {
    mx_f32x4 tot = red[0][bt][lane];
#pragma unroll
    for (int v = 1; v < WV; ++v) {
      const mx_f32x4 p = red[v][bt][lane];
      tot[0] = __fadd_rn(tot[0], p[0]); tot[1] = __fadd_rn(tot[1], p[1]);
      tot[2] = __fadd_rn(tot[2], p[2]); tot[3] = __fadd_rn(tot[3], p[3]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ri = b0 + 16 * bt + 4 * g + r;
      if (ri < B) {
        const float v = bias != nullptr ? __fadd_rn(tot[r], bv) : tot[r];
        y[(size_t)ri * N + n] = f2bf(v);
      }
    }
  }
}

template <int BT>
static void launch_mxfp4_gemv_mfma_bt(const uint8_t* codes, const uint8_t* scales,
                                      const uint16_t* bias, const uint16_t* x, uint16_t* y,
                                      int N, int K, int B, hipStream_t st) {
  const int steps = (K / 32 + 3) / 4;        // K steps of 4 units
  const int it = (steps + 3) / 4;            // per wave (8 waves of half the K measured slower)
  const dim3 grid((N + 15) / 16, (B + 16 * BT - 1) / (16 * BT));
#define MF_CASE(ITV)                                                                     \
  if (it <= ITV) {                                                                       \
    hipLaunchKernelGGL((k_mxfp4_gemv_mfma<BT, ITV, 4>), grid, dim3(256), 0, st, codes,  \
                       scales, bias, x, y, N, K, B);                                     \
    return;                                                                              \
  }
  MF_CASE(2) MF_CASE(4) MF_CASE(6) MF_CASE(8) MF_CASE(12) MF_CASE(16)
#undef MF_CASE
}

// k_mxfp4_gemv_mfma with its operands copied into LDS by global_load_lds
// through a ring of NS stages (no register staging).  A block owns WT
// 16-row weight tiles and BT 16-row batch tiles; its K chunks (128
// elements, 4 MXFP4 units) are split into KS contiguous parts, wave
// w = kh WT + wt taking tile wt over part kh, and the parts' partial tiles
// are added in part order at the end.  Per part a stage holds:
//   - the chunk of the block's input rows, 256 bytes a row, copied a whole
//     row segment at a time (4 rows per 1 KB copy, each row's 256 bytes one
//     contiguous read) with 16-byte slot s of row r at physical slot
//     s ^ (r % 16), so that the MFMA operand reads of 16 rows (one slot
//     each) fall on 16 different bank groups;
//   - per weight tile the 16 code bytes of unit 4 q + g of row 16 tl + j
//     for lane (j, g) -- the operand order itself, one 1 KB copy -- and that
//     unit's scale byte inside the aligned dword that holds it (a dword
//     copy; an aligned dword never crosses a page).
// Every wave issues the same number of copies a chunk (duplicates where the
// input pieces do not divide evenly), so one vmcnt covers a chunk.  Units
// past K read the last unit and their input operand is zeroed; rows past N
// or B read the last row and are not stored.  Lane (j, g) multiplies the
// same k values as in k_mxfp4_gemv_mfma; only the order of the fp32
// additions differs (the chunks of a part in order, then the parts).
constexpr int kMxgX = 64;   // uint4 per input piece (4 rows x 256 B)
constexpr int kMxgW = 80;   // uint4 per weight tile: 64 code + 16 scale (256 B)
template <int BT, int WT, int KS, int NS>
struct MxgCfg {
  static constexpr int PX = 4 * BT;                   // input pieces per chunk
  static constexpr int PART = PX * kMxgX + WT * kMxgW;  // uint4 per part and stage
  static constexpr int STAGE = KS * PART;
  static constexpr int LX = (PX + WT - 1) / WT;       // input copies per wave
  static constexpr int LT = LX + 2;                   // copies per wave and chunk
  static constexpr size_t BYTES = (size_t)NS * STAGE * 16;
};
template <int BT, int WT, int KS, int NS>
__global__ __launch_bounds__(64 * WT * KS) void k_mxfp4_gemv_lx(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ scales,
    const uint16_t* __restrict__ bias, const uint16_t* __restrict__ x,
    uint16_t* __restrict__ y, int N, int K, int B) {
  using C = MxgCfg<BT, WT, KS, NS>;
  constexpr int PX = C::PX, PART = C::PART, STAGE = C::STAGE, LX = C::LX, LT = C::LT;
  static_assert(NS >= 2 && (NS - 2) * LT <= 63, "chunk arrival must fit one vmcnt");
  extern __shared__ uint4 mxg_lds[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wt = w % WT, kh = w / WT;
  const int j = lane & 15, g = lane >> 4;
  const int U = K / 32, NCH = (K + 127) / 128, NT = (N + 15) / 16;
  const int CPK = (NCH + KS - 1) / KS;  // chunks per part
  const int cb = kh * CPK;              // this wave's first chunk
  const int tile = blockIdx.x * WT + wt;
  const int tl = min(tile, NT - 1);     // waves past N load a real tile, store nothing
  const int b0 = blockIdx.y * 16 * BT;
  const int nr = min(16 * tl + j, N - 1);
  const int n = 16 * tile + j;
  // the epilogue's bias, requested now from an address that is always valid
  // (a conditional load would be waited for where the branches join)
  const uint16_t bq = load_pinned_u16(bias != nullptr ? bias + min(n, N - 1) : x);
  const float bv = (bias != nullptr && n < N) ? bf2f(bq) : 0.0f;
  const uint8_t* crow = codes + (size_t)nr * (K / 2);
  const uint8_t* srow = scales + (size_t)nr * U;
  const int spar = (int)(reinterpret_cast<uintptr_t>(srow) & 3);
#if defined(__HIP_DEVICE_COMPILE__)
#define MXG_LOAD(gp, lp, sz) __builtin_amdgcn_global_load_lds((gp), (lp), (sz), 0, 0)
#else
#define MXG_LOAD(gp, lp, sz) ((void)(gp), (void)(lp))
#endif
  auto issue = [&](int i, int stage) {
    const int ch = min(cb + i, NCH - 1);  // past the part's end: a copy never consumed
    uint4* base = mxg_lds + stage * STAGE + kh * PART;
#pragma unroll
    for (int ii = 0; ii < LX; ++ii) {
      const int q = min(wt + WT * ii, PX - 1);  // a duplicate writes the same bytes
      const int rr = 4 * q + (lane >> 4);       // the block's row
      const int ls = (lane & 15) ^ (rr & 15);   // logical 16-byte slot of the row's chunk
      const int u = min(4 * ch + (ls >> 2), U - 1);
      const int gr = min(b0 + rr, B - 1);
      MXG_LOAD(x + (size_t)gr * K + u * 32 + 8 * (ls & 3), base + q * kMxgX, 16);
    }
    const int u = min(4 * ch + g, U - 1);
    uint4* wb = base + PX * kMxgX + wt * kMxgW;
    MXG_LOAD(crow + (size_t)u * 16, wb, 16);
    const uintptr_t sa = reinterpret_cast<uintptr_t>(srow + u) & ~(uintptr_t)3;
    MXG_LOAD(reinterpret_cast<const void*>(sa), reinterpret_cast<uint32_t*>(wb + 64), 4);
  };
#undef MXG_LOAD
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) issue(s, s);
  mx_f32x4 acc[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) acc[bt] = mx_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int i0 = 0; i0 < CPK; i0 += NS) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int i = i0 + s;
      if (i >= CPK) break;  // uniform
      mx_wait_vmcnt<(NS - 2) * LT>();  // this wave's copies of chunk i have landed
      // every wave's have, and every wave's reads of stage (i - 1) % NS are
      // complete (lgkmcnt 0), so the copies issued next may overwrite it.  No
      // fence: the waits on the copies are the vmcnt above
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      issue(i + NS - 1, (s + NS - 1) % NS);
      __builtin_amdgcn_sched_barrier(0);
      const int ch = cb + i;
      if (ch < NCH) {  // uniform per wave (the last part may be shorter)
        const uint4* st = mxg_lds + s * STAGE + kh * PART;
        const uint4* wb = st + PX * kMxgX + wt * kMxgW;
        const bool uok = 4 * ch + g < U;
        const int u = min(4 * ch + g, U - 1);
        const uint32_t sd = reinterpret_cast<const uint32_t*>(wb + 64)[lane];
        const uint32_t sb = (sd >> (8 * ((spar + u) & 3))) & 0xFFu;
        const float sc = sb == 0xFFu ? __builtin_nanf("") : __builtin_amdgcn_ldexpf(1.0f, (int)sb - 127);
        const mx_u32x4 cw = *reinterpret_cast<const mx_u32x4*>(wb + lane);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const mx_bf16x8 bw = mx_fp4x8(cw[t], sc);
#pragma unroll
          for (int bt = 0; bt < BT; ++bt) {
            // row 16 bt + j, logical slot 4 g + t
            const mx_u32x4 xv = *reinterpret_cast<const mx_u32x4*>(
                st + (4 * bt + (j >> 2)) * kMxgX + ((j & 3) << 4) + ((4 * g + t) ^ j));
            const mx_u32x4 xa = uok ? xv : mx_u32x4{0u, 0u, 0u, 0u};  // zero A drops the unit
            acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(mx_bf16x8, xa), bw, acc[bt], 0, 0, 0);
          }
        }
      }
    }
  }
  mx_wait_vmcnt<0>();  // the ring's last (unused) copies have landed
  if constexpr (KS > 1) {
    // parts 1 .. KS - 1 hand their tiles over through the (now idle) ring
    mx_f32x4* red = reinterpret_cast<mx_f32x4*>(mxg_lds);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (kh > 0) {
#pragma unroll
      for (int bt = 0; bt < BT; ++bt) red[(((kh - 1) * WT + wt) * BT + bt) * 64 + lane] = acc[bt];
    }
    __syncthreads();
    if (kh > 0) return;
#pragma unroll
    for (int v = 1; v < KS; ++v)
#pragma unroll
      for (int bt = 0; bt < BT; ++bt) {
        const mx_f32x4 p = red[(((v - 1) * WT + wt) * BT + bt) * 64 + lane];
        acc[bt][0] = __fadd_rn(acc[bt][0], p[0]); acc[bt][1] = __fadd_rn(acc[bt][1], p[1]);
        acc[bt][2] = __fadd_rn(acc[bt][2], p[2]); acc[bt][3] = __fadd_rn(acc[bt][3], p[3]);
      }
  }
  if (n >= N || tile >= NT) return;
#pragma unroll
  for (int bt = 0; bt < BT; ++bt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ri = b0 + 16 * bt + 4 * g + r;
      if (ri < B) {
        const float v = bias != nullptr ? __fadd_rn(acc[bt][r], bv) : acc[bt][r];
        y[(size_t)ri * N + n] = f2bf(v);
      }
    }
}

template <int BT, int WT, int KS, int NS>
static void launch_mxfp4_gemv_lx(const uint8_t* codes, const uint8_t* scales,
                                 const uint16_t* bias, const uint16_t* x, uint16_t* y, int N,
                                 int K, int B, hipStream_t st) {
  constexpr size_t bytes = MxgCfg<BT, WT, KS, NS>::BYTES;
  static_assert(bytes <= 160 * 1024 && bytes >= (size_t)(KS - 1) * WT * BT * 1024,
                "LDS (ring, and the part hand-over)");
  static const hipError_t optin =
      hipFuncSetAttribute(reinterpret_cast<const void*>(k_mxfp4_gemv_lx<BT, WT, KS, NS>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  (void)optin;  // a refused opt-in surfaces as the launch's error
  const int nt = (N + 15) / 16;
  hipLaunchKernelGGL((k_mxfp4_gemv_lx<BT, WT, KS, NS>),
                     dim3((nt + WT - 1) / WT, (B + 16 * BT - 1) / (16 * BT)),
                     dim3(64 * WT * KS), bytes, st, codes, scales, bias, x, y, N, K, B);
}

// Block shape of k_mxfp4_gemv_lx: batch tiles, weight tiles, K parts,
// stages.  Measured over BASELINE config 1 (K = 2880, N = 2880 / 5760 /
// 4096, us; the register-fed k_mxfp4_gemv_mfma in brackets):
//   B = 16: (1,1,8,3) 5.81 / 10.06 / 5.98, (1,2,4,3) 6.65 / 6.95 / 6.74
//           [6.45 / 10.61 / 6.61];
//   B = 64: (2,2,4,3) 8.78 / 14.87 / 8.81, (2,4,2,3) 10.88 / 11.37 / 11.02,
//           (1,2,2,4) 9.66 / 14.44 / 10.85, (1,4,2,4) 9.49 / 14.65 / 9.41
//           [14.99 / 26.51 / 15.23].
// The 8-wave shapes hold 126 KB of LDS (one block per CU): up to 256 blocks
// they all start at once, beyond that the shapes with more weight tiles per
// block keep the grid within one round.  NEON_MXFP4_LX = "BT,WT,KS,NS" picks
// one of the shapes listed in launch_mxfp4_gemv_lx_sel for comparisons, "0"
// the register-fed kernel.
struct MxgShape { int bt, wt, ks, ns; };
static MxgShape mxg_shape(int B, int N) {
  static MxgShape env = {-2, 0, 0, 0};
  if (env.bt == -2) {
    MxgShape v = {-1, 0, 0, 0};
    if (const char* e = getenv("NEON_MXFP4_LX")) {
      int a = -1, b = 0, c = 0, d = 0;
      if (sscanf(e, "%d,%d,%d,%d", &a, &b, &c, &d) >= 1) v = {a, b, c, d};
    }
    env = v;
  }
  if (env.bt >= 0) return env;
  const bool one_round = (N + 15) / 16 <= 256;
  if (B <= 16) return one_round ? MxgShape{1, 1, 8, 3} : MxgShape{1, 2, 4, 3};
  return one_round ? MxgShape{2, 2, 4, 3} : MxgShape{2, 4, 2, 3};
}

static bool launch_mxfp4_gemv_lx_sel(const uint8_t* codes, const uint8_t* scales,
                                     const uint16_t* bias, const uint16_t* x, uint16_t* y,
                                     int N, int K, int B, hipStream_t st) {
  // its 16-byte copies read whole 16-byte pieces of x and of the code rows
  if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(codes)) & 15) != 0)
    return false;
  const MxgShape v = mxg_shape(B, N);
#define MXG_SEL(BT, WT, KS, NS)                                                     \
  if (v.bt == BT && v.wt == WT && v.ks == KS && v.ns == NS) {                       \
    launch_mxfp4_gemv_lx<BT, WT, KS, NS>(codes, scales, bias, x, y, N, K, B, st);   \
    return true;                                                                    \
  }
  MXG_SEL(1, 2, 2, 4) MXG_SEL(1, 4, 1, 4) MXG_SEL(1, 1, 4, 4) MXG_SEL(1, 2, 4, 3)
  MXG_SEL(1, 1, 2, 4) MXG_SEL(1, 2, 1, 4) MXG_SEL(2, 2, 2, 4) MXG_SEL(2, 4, 2, 3)
  MXG_SEL(4, 2, 2, 3) MXG_SEL(4, 4, 1, 4) MXG_SEL(1, 1, 8, 3) MXG_SEL(2, 1, 4, 3)
  MXG_SEL(1, 2, 2, 6) MXG_SEL(1, 4, 2, 4) MXG_SEL(1, 4, 4, 3) MXG_SEL(1, 2, 4, 4)
  MXG_SEL(1, 2, 8, 3) MXG_SEL(2, 4, 4, 2) MXG_SEL(2, 2, 4, 3)
#undef MXG_SEL
  return false;
}

void launch_mxfp4_gemv_mfma(const uint8_t* codes, const uint8_t* scales, const uint16_t* bias,
                            const uint16_t* x, uint16_t* y, int N, int K, int B,
                            hipStream_t st) {
  // batch tiles per block (B past 64 rows runs several blocks in y).  One
  // or two tiles per block with more blocks in y measured slower at B = 64
  // (16.5 / 16.8 against 15.6 us at N = 2880, 20.8 / 16.8 against 15.8 at
  // N = 4096); only N = 5760 gained with two (24.1 against 28.0 us)
  if (launch_mxfp4_gemv_lx_sel(codes, scales, bias, x, y, N, K, B, st)) return;
  const int bt = B >= 64 ? 4 : (B + 15) / 16;
  switch (bt) {
    case 1: launch_mxfp4_gemv_mfma_bt<1>(codes, scales, bias, x, y, N, K, B, st); break;
    case 2: launch_mxfp4_gemv_mfma_bt<2>(codes, scales, bias, x, y, N, K, B, st); break;
    case 3: launch_mxfp4_gemv_mfma_bt<3>(codes, scales, bias, x, y, N, K, B, st); break;
    default: launch_mxfp4_gemv_mfma_bt<4>(codes, scales, bias, x, y, N, K, B, st); break;
  }
}

// weight tiles of 16 rows per wave and rows per block.  Measured at the 20b
// shape (tok/s at B = 16 / 64): 4 tiles (228 VGPRs, 2 waves per SIMD)
// 3754 / 7924, 2 tiles (146 VGPRs) 4141 / 9400, 1 tile 4206 / 9499 -- more
// waves in flight beat the activation reuse of wider waves.  Likewise 8
// waves of one tile per block (128 rows sharing each staged input chunk,
// half the blocks): 4711 / 15,454 against 4943 / 15,836 with 4.
constexpr int kMxMoeTiles = 1, kMxMoeRows = 64 * kMxMoeTiles;

// The work item of block row blockIdx.y (one load: the item count and the
// packed item are read together, the item slot in bounds for any y < 256).
// False for rows past the item count and for items whose expert is out of
// range (a corrupt table: flagged, never read past the experts) or whose
// group lies past the expert's pairs.
__device__ __forceinline__ bool mx_block_item(const MxArgs& a, int tid, int& slot, int& grp,
                                              int& e, int& cnt) {
  const int n = a.route[kMxItemOff];
  const int32_t v = a.route[kMxItemOff + 1 + blockIdx.y];
  if ((int)blockIdx.y >= n) return false;
  mx_item_unpack(v, slot, grp, e, cnt);
  if (e >= a.E || slot >= min(a.E, a.B * a.k)) {
    if (tid == 0) flag_dev_err(a.err, kDevErrExpertId);
    return false;
  }
  return 16 * grp < cnt;
}

// The block's work item and its 16 pair rows in s.rows (entries from the
// item's pair count R = min(16, cnt - 16 grp) on are not read): from the
// route table when the router step wrote one (a.route), else built by the
// block from the pair ids (mx_route_item: the same item, the same pairs).
__device__ __forceinline__ bool mx_block_work(const MxArgs& a, int tid, MxRouteLds& s,
                                              int& slot, int& grp, int& e, int& cnt) {
  if (a.route == nullptr)
    return mx_route_item(a.idx, a.B * a.k, a.E, blockIdx.y, a.err, s, slot, grp, e, cnt);
  if (!mx_block_item(a, tid, slot, grp, e, cnt)) return false;  // (uniform)
  const int S = min(a.E, a.B * a.k);
  if (tid < 16) s.rows[tid] = a.route[2 * S + 64 * slot + 16 * grp + tid];  // within the 64-entry list
  __syncthreads();
  return true;
}

template <int MODE>
__global__ __launch_bounds__(256) void k_mx_moe16(MxArgs a) {
  constexpr int CKU = 16, CK = 32 * CKU, XS = CK + 8;
  constexpr int TT = kMxMoeTiles;  // weight tiles of 16 rows per wave
  __shared__ __align__(16) uint16_t xs[2][16][XS];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int N = a.N, K = a.K, U = K / 32;
  // block row y = work item y (the route table's order): rows 16 group ..
  // 16 group + 15 of the slot's pair list
  __shared__ MxRouteLds rl;
  int slot, grp, e, Rall;
  if (!mx_block_work(a, tid, rl, slot, grp, e, Rall)) return;  // (uniform)
  const int R = min(16, Rall - 16 * grp);
  const int32_t* rows = rl.rows;
  const int nw0 = blockIdx.x * 64 * TT + 16 * TT * w;  // the wave's first row
  const bool wave_on = nw0 < N;               // uniform per wave
  const int nch = (U + CKU - 1) / CKU;
  // the epilogue's bias values and output rows, requested now so that the
  // end of the kernel waits for no load (a load after the K loop is one more
  // round trip per block)
  float bias_pre[TT];
  int32_t row_pre[4];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
    bias_pre[tt] = bf2f(load_pinned_u16(  // unconditional (clamped): no branch to join
        a.bias + (size_t)e * N + min(nw0 + 16 * tt + j, N - 1)));
#pragma unroll
  for (int r = 0; r < 4; ++r) row_pre[r] = rows[min(4 * g + r, R - 1)];
  // staging: thread tid copies 8-element pieces (tid & 15) + 16 q of row tid >> 4
  const int sr = tid >> 4, sp = tid & 15;
  const bool s_ok = sr < R;
  int xr = 0;
  if (s_ok) {
    // pair index -> input row (clamped: a corrupt list still reads in bounds)
    const unsigned q = min((unsigned)rows[sr], (unsigned)(a.B * a.k - 1));
    xr = MODE == MX_GATE_UP ? (int)q / a.k : (int)q;
  }
  const uint16_t* xsrc = a.x + (size_t)xr * K;
  auto x_load = [&](int c, uint4 (&xv)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int el = c * CK + 8 * (sp + 16 * q);
      xv[q] = (s_ok && el < K) ? *reinterpret_cast<const uint4*>(xsrc + el)
                               : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto x_store = [&](int buf, const uint4 (&xv)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<uint4*>(&xs[buf][sr][8 * (sp + 16 * q)]) = xv[q];
  };
  // packed codes [E][N/16][nch][su][g][j] pieces of 16 bytes (scales: one
  // byte each): lane l = j + 16 g reads piece ... * 64 + l
  const uint8_t* Pc = static_cast<const uint8_t*>(a.Wp);
  auto w_load = [&](int c, uint4 (&wv)[TT][4], float (&sv)[TT][4]) {
    if (!wave_on) return;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const size_t et = (size_t)e * (N / 16) + nw0 / 16 + tt;
#pragma unroll
      for (int su = 0; su < 4; ++su) {
        const size_t piece = ((et * nch + c) * 4 + su) * 64 + lane;
        wv[tt][su] = mx_load_nt(Pc + piece * 16);
        sv[tt][su] = __builtin_amdgcn_ldexpf(1.0f, (int)a.sp[piece] - 127);
      }
    }
  };
  mx_f32x4 acc[TT];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) acc[tt] = mx_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](int c, int buf, const uint4 (&wv)[TT][4], const float (&sv)[TT][4]) {
#pragma unroll
    for (int su = 0; su < 4; ++su) {
      // units past K (the last chunk's padding) hold zero codes at scale
      // 2^0 in the packed copy and zero inputs in xs (x_load), so their
      // products are +0 like those of any zero input: no mask is needed
      uint4 af[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        af[t] = *reinterpret_cast<const uint4*>(&xs[buf][j][32 * (4 * g + su) + 8 * t]);
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const uint4 cw = wv[tt][su];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint32_t word = t == 0 ? cw.x : t == 1 ? cw.y : t == 2 ? cw.z : cw.w;
          acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              mx_as_bf16x8(af[t]), mx_fp4x8(word, sv[tt][su]), acc[tt], 0, 0, 0);
        }
      }
    }
  };
  uint4 wA[TT][4], wB[TT][4];
  float sA[TT][4], sB[TT][4];
  uint4 xv[4];
  x_load(0, xv);
  w_load(0, wA, sA);
  x_store(0, xv);
  for (int c = 0; c < nch; c += 2) {
    const bool has1 = c + 1 < nch, has2 = c + 2 < nch;
    if (has1) x_load(c + 1, xv);
    __builtin_amdgcn_sched_barrier(0);
    if (has1) w_load(c + 1, wB, sB);
    __syncthreads();  // chunk c staged; chunk c - 1's buffer is free
    if (wave_on) compute(c, 0, wA, sA);
    if (has1) x_store(1, xv);
    if (!has1) break;
    if (has2) x_load(c + 2, xv);
    __builtin_amdgcn_sched_barrier(0);
    if (has2) w_load(c + 2, wA, sA);
    __syncthreads();  // chunk c + 1 staged; chunk c's buffer is free
    if (wave_on) compute(c + 1, 1, wB, sB);
    if (has2) x_store(0, xv);
  }
  if (!wave_on) return;
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    const int n = nw0 + 16 * tt + j;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ri = 4 * g + r;
      const bool ok = ri < R && (unsigned)row_pre[r] < (unsigned)(a.B * a.k);
      const float d = acc[tt][r];
      if constexpr (MODE == MX_GATE_UP) {
        const float v = __fadd_rn(d, bias_pre[tt]);
        const float other = __shfl_xor(v, 1);
        if (ok && (j & 1) == 0)
          a.y[(size_t)row_pre[r] * (N / 2) + n / 2] = f2bf(swiglu_clamp(v, other, a.alpha, a.limit));
      } else {
        if (ok) a.out_f[(size_t)row_pre[r] * N + n] = __fadd_rn(d, bias_pre[tt]);
      }
    }
  }
}

// Decode attention of the matrix-core steps (HFM:235-263): block = one wave
// for (kv head g, key split s, row b); the G query heads of g are the query
// columns of v_mfma_f32_16x16x32_bf16 (columns G .. 15 are zero).  The split's
// 64-key chunks go through LDS (K as [key][dim], V transposed), loaded 1 KB
// contiguous per instruction with each key at its cache row (pos & key_mask
// for a ring); S^T = K Q^T, scores x 1/8, keys past the row's position
// masked, online softmax per head, O^T += V^T P^T with P in bf16 hi + lo.
// One split finishes with the sink here; several leave (o, m, l) partials in
// the exact kernels' layout for k_attn_merge.
// RoPE of dims f, f + 1 (a, packed bf16) with their partners f + 32, f + 33
// (c): rope_pair at the position whose table rows cp / sp are given.
__device__ __forceinline__ void mx_rope2(uint32_t& a, uint32_t& c, const float* cp,
                                         const float* sp, int f) {
  float o1a, o2a, o1b, o2b;
  rope_pair(bf_lo(a), bf_lo(c), cp[f], sp[f], o1a, o2a);
  rope_pair(bf_hi(a), bf_hi(c), cp[f + 1], sp[f + 1], o1b, o2b);
  a = (uint32_t)f2bf(o1a) | ((uint32_t)f2bf(o1b) << 16);
  c = (uint32_t)f2bf(o2a) | ((uint32_t)f2bf(o2b) << 16);
}
// dims f0 .. f0 + 7 (x1) and their partners f0 + 32 .. f0 + 39 (x2)
__device__ __forceinline__ void mx_rope8(uint4& x1, uint4& x2, const float* cp, const float* sp,
                                         int f0) {
  mx_rope2(x1.x, x2.x, cp, sp, f0);
  mx_rope2(x1.y, x2.y, cp, sp, f0 + 2);
  mx_rope2(x1.z, x2.z, cp, sp, f0 + 4);
  mx_rope2(x1.w, x2.w, cp, sp, f0 + 6);
}

__global__ __launch_bounds__(64) void k_mx_attn(
    const uint16_t* __restrict__ q, const uint16_t* kc,
    const uint16_t* vc, const int32_t* __restrict__ pos_arr,
    const int32_t* __restrict__ seq, float* __restrict__ part_o, float* __restrict__ part_ml,
    const uint16_t* __restrict__ sinks, uint16_t* __restrict__ out, int Hq, int Hkv, int G,
    int T_max, int key_mask, int window, int S, int q_stride, uint16_t* __restrict__ outp,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    uint16_t* kc_w, uint16_t* vc_w) {
  // kc / vc and kc_w / vc_w are the same caches (read by every block, the
  // new row written by the block of the last split): no __restrict__ on them
  constexpr int VT = 64 + 8;
  __shared__ __align__(16) uint16_t ks[64 * 64];
  __shared__ __align__(16) uint16_t vt[64 * VT];
  const int lane = threadIdx.x, j = lane & 15, gq = lane >> 4;
  const int g = blockIdx.x % Hkv, sp = blockIdx.x / Hkv, b = blockIdx.y;
  const int p = pos_arr[b];
  const int sq = seq != nullptr ? seq[b] : b;
  const int lo = (window > 0 && p - window + 1 > 0) ? p - window + 1 : 0;
  const int nch = (p - lo + 1 + 63) >> 6;
  const int c0 = (int)((int64_t)sp * nch / S), c1 = (int)((int64_t)(sp + 1) * nch / S);
  const size_t kv_base = ((size_t)sq * Hkv + g) * T_max;
  const bool hv = j < G;
  const int h = g * G + (hv ? j : 0);
  uint4 qf[2];
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2)
    qf[h2] = hv ? *reinterpret_cast<const uint4*>(q + (size_t)b * q_stride + (size_t)h * 64 +
                                                  32 * h2 + 8 * gq)
                : make_uint4(0u, 0u, 0u, 0u);
  // Raw projection output (cos_t given): the lane's q dims 8 gq + e and
  // 32 + 8 gq + e are RoPE partners, rotated here.  The block whose split
  // holds position p (the last: its last chunk ends at p) also rotates the
  // kv head's new key, appends key and value to the caches, and stages them
  // for every key index >= p (keys past p are masked) instead of reading
  // them back.  Each rotation is rope_pair at position p, as in
  // k_mx_rope_append, so the bits are those of the separate launch.
  const bool fused = cos_t != nullptr;
  const bool owner = fused && sp == S - 1;
  uint4 knew = make_uint4(0u, 0u, 0u, 0u), vnew = knew;
  const int dql = (lane & 7) * 8;  // the 8 dims this lane stages for every key
  if (fused) {
    const float* cp = cos_t + (size_t)p * 32;
    const float* spn = sin_t + (size_t)p * 32;
    if (hv) {
      uint4 q0 = qf[0], q1 = qf[1];
      mx_rope8(q0, q1, cp, spn, 8 * gq);
      qf[0] = q0;
      qf[1] = q1;
    }
    if (owner) {
      // lane stages dims dql .. dql + 7: its partner dims are dql ^ 32
      const uint16_t* kr = q + (size_t)b * q_stride + (size_t)(Hq + g) * 64;
      const uint16_t* vr = q + (size_t)b * q_stride + (size_t)(Hq + Hkv + g) * 64;
      const int f0 = dql & 31;
      uint4 k1 = *reinterpret_cast<const uint4*>(kr + f0);
      uint4 k2 = *reinterpret_cast<const uint4*>(kr + f0 + 32);
      vnew = *reinterpret_cast<const uint4*>(vr + dql);
      mx_rope8(k1, k2, cp, spn, f0);
      const bool lo_half = dql < 32;  // the lane's dims are k1's, else k2's
      knew = make_uint4(lo_half ? k1.x : k2.x, lo_half ? k1.y : k2.y, lo_half ? k1.z : k2.z,
                        lo_half ? k1.w : k2.w);
      if (lane < 8) {  // one lane per 8 dims writes the cache row
        const size_t crow = kv_base + (size_t)(p & key_mask);
        *reinterpret_cast<uint4*>(kc_w + crow * 64 + dql) = knew;
        *reinterpret_cast<uint4*>(vc_w + crow * 64 + dql) = vnew;
      }
    }
  }
  mx_f32x4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = mx_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m = -INFINITY, l = 0.0f;
  // a chunk's K and V pieces (lane: keys 8 i + lane / 8, dims 8 (lane % 8)
  // .. + 7); the next chunk's are requested before this one is staged and
  // multiplied, so a split of several chunks pays one memory round trip
  // instead of one per chunk
  uint4 kq[8], vq[8];
  auto load_chunk = [&](int c, uint4 (&kd)[8], uint4 (&vd)[8]) {
    const int kb = lo + 64 * c;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int kl = 8 * i + (lane >> 3), dq = (lane & 7) * 8;
      const int key = min(kb + kl, p);  // keys past p are masked below
      const size_t row = kv_base + (size_t)(key & key_mask);
      kd[i] = *reinterpret_cast<const uint4*>(kc + row * 64 + dq);
      vd[i] = *reinterpret_cast<const uint4*>(vc + row * 64 + dq);
    }
  };
  // chunk c (its pieces in kd / vd) into LDS, then into the running state
  auto process = [&](int c, const uint4 (&kd)[8], const uint4 (&vd)[8]) {
    const int kb = lo + 64 * c;
    __syncthreads();  // the previous chunk is consumed
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int kl = 8 * i + (lane >> 3), dq = (lane & 7) * 8;
      const int key = min(kb + kl, p);  // keys past p are masked below
      const bool fresh = owner && key == p;  // (dq == dql)
      // both rows loaded, then selected word by word (a select between a
      // load and a register value would put the value in private memory)
      const uint4 kg = kd[i];
      const uint4 vg = vd[i];
      const uint4 kv = make_uint4(fresh ? knew.x : kg.x, fresh ? knew.y : kg.y,
                                  fresh ? knew.z : kg.z, fresh ? knew.w : kg.w);
      const uint4 vv = make_uint4(fresh ? vnew.x : vg.x, fresh ? vnew.y : vg.y,
                                  fresh ? vnew.z : vg.z, fresh ? vnew.w : vg.w);
      *reinterpret_cast<uint4*>(&ks[kl * 64 + dq]) = kv;
      const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vt[(dq + 2 * e) * VT + kl] = (uint16_t)(vw[e] & 0xFFFFu);
        vt[(dq + 2 * e + 1) * VT + kl] = (uint16_t)(vw[e] >> 16);
      }
    }
    __syncthreads();
    float sv[4][4];
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const uint4 ka0 = *reinterpret_cast<const uint4*>(&ks[(16 * kt + j) * 64 + 8 * gq]);
      const uint4 ka1 = *reinterpret_cast<const uint4*>(&ks[(16 * kt + j) * 64 + 32 + 8 * gq]);
      mx_f32x4 acc = mx_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mx_as_bf16x8(ka0), mx_as_bf16x8(qf[0]), acc,
                                                   0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mx_as_bf16x8(ka1), mx_as_bf16x8(qf[1]), acc,
                                                   0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool valid = kb + 16 * kt + 4 * gq + r <= p;
        sv[kt][r] = valid ? __fmul_rn(acc[r], 0.125f) : -INFINITY;
        mx = fmaxf(mx, sv[kt][r]);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mt = fmaxf(m, mx);
    const float sc = mt == -INFINITY ? 1.0f : __expf(m - mt);  // m = -inf -> 0
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
        pv[kt][r] = sv[kt][r] == -INFINITY ? 0.0f : __expf(sv[kt][r] - mt);
        l += pv[kt][r];
      }
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int r2 = 0; r2 < 2; ++r2) {
          const float a0 = pv[2 * pp + half][2 * r2], a1 = pv[2 * pp + half][2 * r2 + 1];
          const uint16_t h0 = f2bf(a0), h1 = f2bf(a1);
          const uint16_t l0 = f2bf(a0 - bf2f(h0)), l1 = f2bf(a1 - bf2f(h1));
          hw[2 * half + r2] = (uint32_t)h0 | ((uint32_t)h1 << 16);
          lw[2 * half + r2] = (uint32_t)l0 | ((uint32_t)l1 << 16);
        }
      const uint4 phi = make_uint4(hw[0], hw[1], hw[2], hw[3]);
      const uint4 plo = make_uint4(lw[0], lw[1], lw[2], lw[3]);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint16_t* vrow = &vt[(16 * dt + j) * VT];
        const uint2 va = *reinterpret_cast<const uint2*>(vrow + 32 * pp + 4 * gq);
        const uint2 vb = *reinterpret_cast<const uint2*>(vrow + 32 * pp + 16 + 4 * gq);
        const uint4 vfrag = make_uint4(va.x, va.y, vb.x, vb.y);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mx_as_bf16x8(vfrag), mx_as_bf16x8(phi),
                                                        o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mx_as_bf16x8(vfrag), mx_as_bf16x8(plo),
                                                        o[dt], 0, 0, 0);
      }
    }
  };
  if (c1 - c0 <= 1) {  // uniform: one chunk (or none) in this split
    if (c0 < c1) {
      load_chunk(c0, kq, vq);
      process(c0, kq, vq);
    }
  } else {
    // two register sets in turn (a copy from one to the other would be
    // scheduled inside the chunk's work and wait for the loads there); the
    // loads are unconditional (past the last chunk the last one again): a
    // conditional load is waited for where the two paths join
    uint4 kn[8], vn[8];
    load_chunk(c0, kq, vq);
    for (int c = c0; c < c1; c += 2) {
      load_chunk(min(c + 1, c1 - 1), kn, vn);
      process(c, kq, vq);
      if (c + 1 >= c1) break;  // uniform
      load_chunk(min(c + 2, c1 - 1), kq, vq);
      process(c + 1, kn, vn);
    }
  }
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (!hv) return;
  if (S == 1) {
    const float sk = bf2f(sinks[h]);
    const float M = fmaxf(m, sk);
    const float f = m == -INFINITY ? 0.0f : __expf(m - M);
    const float inv = 1.0f / (l * f + __expf(sk - M));
    uint16_t* dst = out + ((size_t)b * Hq + h) * 64;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const uint32_t w0 = pack_bf2(o[dt][0] * f * inv, o[dt][1] * f * inv);
      const uint32_t w1 = pack_bf2(o[dt][2] * f * inv, o[dt][3] * f * inv);
      *reinterpret_cast<uint2*>(dst + 16 * dt + 4 * gq) = make_uint2(w0, w1);
      if (outp != nullptr)  // 4 columns of one unit: contiguous in the packed layout
        *reinterpret_cast<uint2*>(outp + mx_packed_at(b, 64 * h + 16 * dt + 4 * gq, Hq / 2)) =
            make_uint2(w0, w1);
    }
  } else {
    const size_t pi = ((size_t)b * Hq + h) * S + sp;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      *reinterpret_cast<float4*>(part_o + pi * 64 + 16 * dt + 4 * gq) =
          make_float4(o[dt][0], o[dt][1], o[dt][2], o[dt][3]);
    if (gq == 0) { part_ml[pi * 2] = m; part_ml[pi * 2 + 1] = l; }
  }
}

void launch_mx_attn(const AttnArgs& a, hipStream_t st) {
  const int G = a.Hq / a.Hkv;
  hipLaunchKernelGGL(k_mx_attn, dim3(a.Hkv * a.S, a.B), dim3(64), 0, st, a.q, a.kc, a.vc,
                     a.pos, a.seq, a.part_o, a.part_ml, a.sinks, a.out, a.Hq, a.Hkv, G,
                     a.T_max, a.key_mask, a.window, a.S, a.q_stride, a.out_packed, a.rope_cos,
                     a.rope_sin, const_cast<uint16_t*>(a.kc), const_cast<uint16_t*>(a.vc));
  if (a.S > 1) launch_attn_merge(a, st);
}

// Row b's k slots in slot order from 0 (the exact path's fmaf chain), one
// rounding to bf16, then h = bf16(h + y).
__global__ __launch_bounds__(256) void k_mx_combine(const float* __restrict__ ybuf,
                                                    const float* __restrict__ score,
                                                    uint16_t* __restrict__ h, int H, int k) {
  const int b = blockIdx.y, n = blockIdx.x * 256 + threadIdx.x;
  if (n >= H) return;
  float y = 0.0f;
  for (int s = 0; s < k; ++s)
    y = __builtin_fmaf(score[b * k + s], ybuf[((size_t)b * k + s) * H + n], y);
  const size_t o = (size_t)b * H + n;
  h[o] = f2bf(__fadd_rn(bf2f(h[o]), bf2f(f2bf(y))));
}

// q and k heads of row b rotated at position pos[b] (bf16 in and out, the
// QKV epilogue's arithmetic); k and v appended at cache row pos & key_mask of
// sequence seq[b] (b when seq is null).
__global__ __launch_bounds__(256) void k_mx_rope_append(
    const uint16_t* __restrict__ qkv, const int32_t* __restrict__ pos,
    const int32_t* __restrict__ seq, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, int Hq, int Hkv, int T_max, int key_mask) {
  const int b = blockIdx.x;
  const int p = pos[b], sq = seq ? seq[b] : b;
  const int rows = (Hq + 2 * Hkv) * 64;
  const uint16_t* row = qkv + (size_t)b * rows;
  const size_t crow = (size_t)(p & key_mask);
  for (int i = threadIdx.x; i < (Hq + Hkv) * 32; i += blockDim.x) {
    const int hh = i >> 5, f = i & 31;
    float o1, o2;
    rope_pair(bf2f(row[hh * 64 + f]), bf2f(row[hh * 64 + f + 32]), cos_t[(size_t)p * 32 + f],
              sin_t[(size_t)p * 32 + f], o1, o2);
    uint16_t* dst = hh < Hq ? q_out + ((size_t)b * Hq + hh) * 64
                            : kc + (((size_t)sq * Hkv + hh - Hq) * T_max + crow) * 64;
    dst[f] = f2bf(o1);
    dst[f + 32] = f2bf(o2);
  }
  for (int i = threadIdx.x; i < Hkv * 64; i += blockDim.x) {
    const int gg = i >> 6, d = i & 63;
    vc[(((size_t)sq * Hkv + gg) * T_max + crow) * 64 + d] = row[(Hq + Hkv) * 64 + i];
  }
}

template <int MODE, int BT, bool PK>
static void mx_launch_it(const MxArgs& a, dim3 grid, hipStream_t st) {
  const int it = (a.K / 32 + 15) / 16;
  if (PK && a.xp != nullptr && launch_mx_gemv_lx_sel<MODE>(a, st)) return;
  if (PK && a.xp != nullptr && MODE == MX_LOGITS && BT >= 3) {
    // lm_head from 33 rows on: 8 waves split K (4 iterations each at K <= 4096);
    // 582 -> 377 us at the 20b shape, B = 64 (equal at B = 32)
    const int it8 = ((a.K + 127) / 128 + 7) / 8;
    if (it8 <= 2) hipLaunchKernelGGL((k_mx_gemv_px<BT, 2, MODE, 8>), grid, dim3(512), 0, st, a);
    else if (it8 <= 4) hipLaunchKernelGGL((k_mx_gemv_px<BT, 4, MODE, 8>), grid, dim3(512), 0, st, a);
    else hipLaunchKernelGGL((k_mx_gemv_px<BT, 8, MODE, 8>), grid, dim3(512), 0, st, a);
    return;
  }
  if (PK && a.xp != nullptr && MODE == MX_RESID) {
    if (it <= 2) hipLaunchKernelGGL((k_mx_gemv_px<BT, 2, MODE, 4, true>), grid, dim3(256), 0, st, a);
    else if (it <= 4) hipLaunchKernelGGL((k_mx_gemv_px<BT, 4, MODE, 4, true>), grid, dim3(256), 0, st, a);
    else if (it <= 6) hipLaunchKernelGGL((k_mx_gemv_px<BT, 6, MODE, 4, true>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((k_mx_gemv_px<BT, 8, MODE, 4, true>), grid, dim3(256), 0, st, a);
    return;
  }
  if (PK && a.xp != nullptr) {
    if (it <= 2) hipLaunchKernelGGL((k_mx_gemv_px<BT, 2, MODE, 4>), grid, dim3(256), 0, st, a);
    else if (it <= 4) hipLaunchKernelGGL((k_mx_gemv_px<BT, 4, MODE, 4>), grid, dim3(256), 0, st, a);
    else if (it <= 6) hipLaunchKernelGGL((k_mx_gemv_px<BT, 6, MODE, 4>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((k_mx_gemv_px<BT, 8, MODE, 4>), grid, dim3(256), 0, st, a);
    return;
  }
  if (BT == 1 && PK) {
    if (it <= 2) hipLaunchKernelGGL((k_mx_gemv_db<1, 2, MODE, 4>), grid, dim3(256), 0, st, a);
    else if (it <= 4) hipLaunchKernelGGL((k_mx_gemv_db<1, 4, MODE, 4>), grid, dim3(256), 0, st, a);
    else if (it <= 6) hipLaunchKernelGGL((k_mx_gemv_db<1, 6, MODE, 4>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((k_mx_gemv_db<1, 8, MODE, 4>), grid, dim3(256), 0, st, a);
    return;
  }
  if (it <= 2) hipLaunchKernelGGL((k_mx_gemv<BT, 2, MODE, PK>), grid, dim3(256), 0, st, a);
  else if (it <= 4) hipLaunchKernelGGL((k_mx_gemv<BT, 4, MODE, PK>), grid, dim3(256), 0, st, a);
  else if (it <= 6) hipLaunchKernelGGL((k_mx_gemv<BT, 6, MODE, PK>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((k_mx_gemv<BT, 8, MODE, PK>), grid, dim3(256), 0, st, a);
}

template <int MODE, bool PK>
static void mx_launch_pk(const MxArgs& a, dim3 grid, hipStream_t st) {
  switch ((a.B + 15) / 16) {
    case 1: mx_launch_it<MODE, 1, PK>(a, grid, st); break;
    case 2: mx_launch_it<MODE, 2, PK>(a, grid, st); break;
    case 3: mx_launch_it<MODE, 3, PK>(a, grid, st); break;
    default: mx_launch_it<MODE, 4, PK>(a, grid, st); break;
  }
}

// the packed copy when there is one, else the checkpoint layout
template <int MODE>
static void mx_launch(const MxArgs& a, dim3 grid, hipStream_t st) {
  if (a.Wp) mx_launch_pk<MODE, true>(a, grid, st);
  else mx_launch_pk<MODE, false>(a, grid, st);
}

bool mx_shape_ok(int N, int K, int B) {
  return B >= 1 && B <= kMxMaxRows && N >= 16 && N % 16 == 0 && K >= 32 && K % 32 == 0 &&
         K <= kMxMaxK;
}

bool mx_moe_shape_ok(int H, int I, int E, int k, int B) {
  return mx_shape_ok(2 * I, H, B) && mx_shape_ok(H, I, B) && (2 * I) % 64 == 0 && H % 64 == 0 &&
         E >= 1 && E <= 256 && B * k <= 256;
}

void launch_mx_gemv(const MxArgs& a, int mode, hipStream_t st) {
  const dim3 grid(a.N / 16);
  if (mode == MX_STORE) mx_launch<MX_STORE>(a, grid, st);
  else if (mode == MX_RESID) mx_launch<MX_RESID>(a, grid, st);
  else mx_launch<MX_LOGITS>(a, grid, st);
}

// ---- experts on the scaled fp8 x fp4 instruction ---------------------------
// k_mx_moe16 with v_mfma_scale_f32_16x16x128_f8f6f4 (A = the pairs' input
// rows as two MXFP8 terms, B = the packed MXFP4 pieces as they are, each with
// its E8M0 scale).  Operand lanes of this shape, measured on gfx950 with an
// in-bounds probe (exact fp32 match on random codes and scales): a B lane
// j + 16 g holds column j, k 32 g .. 32 g + 31 (one MX block); an A lane
// holds row j, k 16 g .. 16 g + 15 in bytes 0-15 and k 64 + 16 g .. in bytes
// 16-31; the scale of (row or column j, k block b) is byte 0 of lane
// j + 16 b's scale operand.  One instruction covers the four units
// 4 b + su (b = 0..3) of a chunk -- the pieces lane j + 16 g already holds
// for slot su -- so A takes the same units from LDS.  Two instructions (hi,
// lo) replace k_mx_moe16's four bf16 ones and its E2M1 conversions.
typedef int mx_i32x8 __attribute__((ext_vector_type(8)));

template <int MODE>
__global__ __launch_bounds__(256) void k_mx8_moe16(MxArgs a) {
  constexpr int CKU = 16, CK = 32 * CKU, XQ = 2 * CK + 16;
  constexpr int TT = kMxMoeTiles;
  __shared__ __align__(16) uint8_t xq[2][16][XQ];      // per row: CK hi bytes, CK lo bytes
  __shared__ uint8_t xsc[2][16][2 * CKU];              // per row: CKU hi scales, CKU lo
  // gate_up: the block's 64 weight rows are 32 SwiGLU columns of its 16
  // pairs, exactly one 32-block of the down input, quantised here
  __shared__ float ytile[16][32];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int N = a.N, K = a.K, U = K / 32;
  __shared__ MxRouteLds rl;
  int slot, grp, e, Rall;
  if (!mx_block_work(a, tid, rl, slot, grp, e, Rall)) return;  // (uniform)
  const int R = min(16, Rall - 16 * grp);
  const int32_t* rows = rl.rows;
  const int nw0 = blockIdx.x * 64 * TT + 16 * TT * w;
  const bool wave_on = nw0 < N;
  const int nch = (U + CKU - 1) / CKU;
  // the epilogue's bias and output rows, requested now (as in k_mx_moe16)
  const float bias_pre =  // unconditional (clamped): no branch to join
      bf2f(load_pinned_u16(a.bias + (size_t)e * N + min(nw0 + j, N - 1)));
  int32_t row_pre[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) row_pre[r] = rows[min(4 * g + r, R - 1)];
  // staging: thread tid copies 16-byte pieces sp and sp + 16 of row sr's
  // chunk, hi and lo, and unit sp's two scale bytes
  const int sr = tid >> 4, sp = tid & 15;
  const bool s_ok = sr < R;
  int xr = 0;
  if (s_ok) {
    const unsigned q = min((unsigned)rows[sr], (unsigned)(a.B * a.k - 1));
    xr = MODE == MX_GATE_UP ? (int)q / a.k : (int)q;
  }
  const uint8_t* qh = a.xq_hi + (size_t)xr * K;
  const uint8_t* ql = a.xq_lo + (size_t)xr * K;
  const uint8_t* qsh = a.xs_hi + (size_t)xr * U;
  const uint8_t* qsl = a.xs_lo + (size_t)xr * U;
  auto x_load = [&](int c, uint4 (&xv)[4], uint32_t (&sv)[2]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int el = c * CK + 16 * (sp + 16 * (q & 1));
      const uint8_t* src = (q < 2 ? qh : ql) + el;
      xv[q] = (s_ok && el < K) ? *reinterpret_cast<const uint4*>(src)
                               : make_uint4(0u, 0u, 0u, 0u);
    }
    const int u = c * CKU + sp;
    sv[0] = (s_ok && u < U) ? qsh[u] : 127u;
    sv[1] = (s_ok && u < U) ? qsl[u] : 127u;
  };
  auto x_store = [&](int buf, const uint4 (&xv)[4], const uint32_t (&sv)[2]) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<uint4*>(&xq[buf][sr][(q < 2 ? 0 : CK) + 16 * (sp + 16 * (q & 1))]) = xv[q];
    xsc[buf][sr][sp] = (uint8_t)sv[0];
    xsc[buf][sr][CKU + sp] = (uint8_t)sv[1];
  };
  const uint8_t* Pc = static_cast<const uint8_t*>(a.Wp);
  auto w_load = [&](int c, uint4 (&wv)[TT][4], uint32_t (&sb)[TT][4]) {
    if (!wave_on) return;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const size_t et = (size_t)e * (N / 16) + nw0 / 16 + tt;
#pragma unroll
      for (int su = 0; su < 4; ++su) {
        const size_t piece = ((et * nch + c) * 4 + su) * 64 + lane;
        wv[tt][su] = mx_load_nt(Pc + piece * 16);
        sb[tt][su] = a.sp[piece];
      }
    }
  };
  mx_f32x4 acc[TT];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) acc[tt] = mx_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](int buf, const uint4 (&wv)[TT][4], const uint32_t (&sb)[TT][4]) {
    const uint8_t* rowp = &xq[buf][j][16 * (g & 1)];
#pragma unroll
    for (int su = 0; su < 4; ++su) {
      const int u0 = 4 * (g >> 1) + su, u1 = 4 * (2 + (g >> 1)) + su;
      const uint4 h0 = *reinterpret_cast<const uint4*>(rowp + 32 * u0);
      const uint4 h1 = *reinterpret_cast<const uint4*>(rowp + 32 * u1);
      const uint4 l0 = *reinterpret_cast<const uint4*>(rowp + CK + 32 * u0);
      const uint4 l1 = *reinterpret_cast<const uint4*>(rowp + CK + 32 * u1);
      const int sa_hi = xsc[buf][j][4 * g + su];
      const int sa_lo = xsc[buf][j][CKU + 4 * g + su];
      const mx_i32x8 ahi = {(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w,
                            (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
      const mx_i32x8 alo = {(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w,
                            (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const mx_i32x8 bq = {(int)wv[tt][su].x, (int)wv[tt][su].y, (int)wv[tt][su].z,
                             (int)wv[tt][su].w, 0, 0, 0, 0};
        const int s_b = (int)sb[tt][su];
        acc[tt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ahi, bq, acc[tt], 0, 4, 0,
                                                                  sa_hi, 0, s_b);
        acc[tt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(alo, bq, acc[tt], 0, 4, 0,
                                                                  sa_lo, 0, s_b);
      }
    }
  };
  uint4 wA[TT][4], wB[TT][4];
  uint32_t sA[TT][4], sB[TT][4];
  uint4 xv[4];
  uint32_t xs_v[2];
  x_load(0, xv, xs_v);
  w_load(0, wA, sA);
  x_store(0, xv, xs_v);
  for (int c = 0; c < nch; c += 2) {
    const bool has1 = c + 1 < nch, has2 = c + 2 < nch;
    if (has1) x_load(c + 1, xv, xs_v);
    __builtin_amdgcn_sched_barrier(0);
    if (has1) w_load(c + 1, wB, sB);
    __syncthreads();  // chunk c staged; chunk c - 1's buffer is free
    if (wave_on) compute(0, wA, sA);
    if (has1) x_store(1, xv, xs_v);
    if (!has1) break;
    if (has2) x_load(c + 2, xv, xs_v);
    __builtin_amdgcn_sched_barrier(0);
    if (has2) w_load(c + 2, wA, sA);
    __syncthreads();  // chunk c + 1 staged; chunk c's buffer is free
    if (wave_on) compute(1, wB, sB);
    if (has2) x_store(0, xv, xs_v);
  }
  static_assert(TT == 1, "the gate_up epilogue assumes one 16-row tile per wave");
  if (wave_on) {
    const int n = nw0 + j;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ri = 4 * g + r;
      const bool ok = ri < R && (unsigned)row_pre[r] < (unsigned)(a.B * a.k);
      const float d = acc[0][r];
      if constexpr (MODE == MX_GATE_UP) {
        const float v = __fadd_rn(d, bias_pre);
        const float other = __shfl_xor(v, 1);
        const uint16_t y = f2bf(swiglu_clamp(v, other, a.alpha, a.limit));
        if ((j & 1) == 0) ytile[ri][8 * w + j / 2] = bf2f(y);
        if (ok && (j & 1) == 0) a.y[(size_t)row_pre[r] * (N / 2) + n / 2] = y;
      } else {
        if (ok) a.out_f[(size_t)row_pre[r] * N + n] = __fadd_rn(d, bias_pre);
      }
    }
  }
  if constexpr (MODE == MX_GATE_UP) {
    // wave 0: row tid / 4's 32 SwiGLU values, a quarter per lane -> the
    // block of the down input's MXFP8 image (blockIdx.x = its 32-block
    // index; N / 2 % 32 == 0 and 64-row blocks keep it aligned)
    __syncthreads();
    if (w == 0) {
      const int ri = lane >> 2, q = lane & 3;
      float v[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) v[t] = ytile[ri][8 * q + t];
      uint32_t qh[2], ql[2], b1, b2;
      mx8_quant8(v, qh, ql, b1, b2);
      const bool ok = ri < R && (unsigned)rows[min(ri, R - 1)] < (unsigned)(a.B * a.k);
      if (ok) {
        const int I = N / 2;
        const size_t o = (size_t)rows[ri] * I + 32 * blockIdx.x + 8 * q;
        *reinterpret_cast<uint2*>(a.yq_hi + o) = make_uint2(qh[0], qh[1]);
        *reinterpret_cast<uint2*>(a.yq_lo + o) = make_uint2(ql[0], ql[1]);
        if (q == 0) {
          a.ys_hi[(size_t)rows[ri] * (I / 32) + blockIdx.x] = (uint8_t)b1;
          a.ys_lo[(size_t)rows[ri] * (I / 32) + blockIdx.x] = (uint8_t)b2;
        }
      }
    }
  }
}

// The combine after the down GEMM, with the next RMSNorm when asked and
// covered (launch_mx_combine_norm); true when the norm was written.
static bool mx_combine(const MxArgs& down, const float* score, uint16_t* h, hipStream_t st,
                       const uint16_t* next_norm, float eps, uint16_t* next_xp) {
  if (next_norm != nullptr && next_xp != nullptr &&
      launch_mx_combine_norm(down.out_f, score, h, next_norm, next_xp, down.B, down.N, down.k,
                             eps, st))
    return true;
  hipLaunchKernelGGL(k_mx_combine, dim3((down.N + 255) / 256, down.B), dim3(256), 0, st,
                     down.out_f, score, h, down.N, down.k);
  return false;
}

bool launch_mx_moe8(MxArgs gate_up, MxArgs down, const float* score, uint16_t* h,
                    hipStream_t st, const uint16_t* next_norm, float eps, uint16_t* next_xp) {
  const int S = std::min(gate_up.E, gate_up.B * gate_up.k);
  const int Y = mx_item_rows(gate_up.B * gate_up.k, S);
  down.xq_hi = gate_up.yq_hi; down.xq_lo = gate_up.yq_lo;
  down.xs_hi = gate_up.ys_hi; down.xs_lo = gate_up.ys_lo;
  hipLaunchKernelGGL(k_mx8_moe16<MX_GATE_UP>,
                     dim3((gate_up.N + kMxMoeRows - 1) / kMxMoeRows, Y), dim3(256), 0, st,
                     gate_up);
  hipLaunchKernelGGL(k_mx8_moe16<MX_DOWN>, dim3((down.N + kMxMoeRows - 1) / kMxMoeRows, Y),
                     dim3(256), 0, st, down);
  return mx_combine(down, score, h, st, next_norm, eps, next_xp);
}

bool launch_mx_moe(const MxArgs& gate_up, const MxArgs& down, const float* score, uint16_t* h,
                   hipStream_t st, const uint16_t* next_norm, float eps, uint16_t* next_xp) {
  const int S = std::min(gate_up.E, gate_up.B * gate_up.k);
  const int Y = mx_item_rows(gate_up.B * gate_up.k, S);
  hipLaunchKernelGGL(k_mx_moe16<MX_GATE_UP>,
                     dim3((gate_up.N + kMxMoeRows - 1) / kMxMoeRows, Y), dim3(256), 0, st,
                     gate_up);
  hipLaunchKernelGGL(k_mx_moe16<MX_DOWN>, dim3((down.N + kMxMoeRows - 1) / kMxMoeRows, Y),
                     dim3(256), 0, st, down);
  return mx_combine(down, score, h, st, next_norm, eps, next_xp);
}

void launch_mx_rope_append(const uint16_t* qkv, const int32_t* pos, const int32_t* seq,
                           const float* cos_t, const float* sin_t, uint16_t* q_out,
                           uint16_t* kc, uint16_t* vc, int B, int Hq, int Hkv, int T_max,
                           int key_mask, hipStream_t st) {
  hipLaunchKernelGGL(k_mx_rope_append, dim3(B), dim3(256), 0, st, qkv, pos, seq, cos_t, sin_t,
                     q_out, kc, vc, Hq, Hkv, T_max, key_mask);
}

// ---- MFMA lane-order copies ------------------------------------------------
// bf16 [N][K] -> [N/16][NCH][t][g][j][8 elements], NCH = ceil(K / 128): piece
// (T, ch, t, g, j) holds row 16 T + j, elements 128 ch + 32 t + 8 g .. + 7
// (zeros past K), the 16 bytes lane j + 16 g of k_mx_gemv loads in step t.
__global__ __launch_bounds__(256) void k_mx_pack_bf16(const uint16_t* __restrict__ W, int N,
                                                      int K, uint16_t* __restrict__ P) {
  const int NCH = (K + 127) / 128;
  const size_t total = (size_t)(N / 16) * NCH * 256;
  for (size_t p = (size_t)blockIdx.x * 256 + threadIdx.x; p < total;
       p += (size_t)gridDim.x * 256) {
    const int j = p & 15, g = (p >> 4) & 3, t = (p >> 6) & 3;
    const size_t rest = p >> 8;
    const int ch = (int)(rest % NCH);
    const size_t T = rest / NCH;
    const int el = ch * 128 + 32 * t + 8 * g;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (el < K) v = *reinterpret_cast<const uint4*>(W + (T * 16 + j) * (size_t)K + el);
    *reinterpret_cast<uint4*>(P + p * 8) = v;
  }
}

// MXFP4 [E][N][U units of 16 code bytes] (+ scales [E][N][U]) ->
// [E][N/16][nch][su][g][j] pieces, nch = ceil(U / 16): piece (e, T, c, su, g, j)
// holds unit 16 c + 4 g + su of row 16 T + j (zero codes and scale 127 past U),
// what lane j + 16 g of k_mx_moe16 loads for slot su of chunk c.
__global__ __launch_bounds__(256) void k_mx_pack_fp4(const uint8_t* __restrict__ codes,
                                                     const uint8_t* __restrict__ scales, int E,
                                                     int N, int K, uint8_t* __restrict__ Pc,
                                                     uint8_t* __restrict__ Ps) {
  const int U = K / 32, nch = (U + 15) / 16;
  const size_t total = (size_t)E * (N / 16) * nch * 256;
  for (size_t p = (size_t)blockIdx.x * 256 + threadIdx.x; p < total;
       p += (size_t)gridDim.x * 256) {
    const int j = p & 15, g = (p >> 4) & 3, su = (p >> 6) & 3;
    const size_t rest = p >> 8;
    const int c = (int)(rest % nch);
    const size_t row = (rest / nch) * 16 + j;  // e N + 16 T + j
    const int u = 16 * c + 4 * g + su;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    uint8_t sc = 127;
    if (u < U) {
      v = *reinterpret_cast<const uint4*>(codes + row * (size_t)(K / 2) + (size_t)u * 16);
      sc = scales[row * (size_t)U + u];
    }
    *reinterpret_cast<uint4*>(Pc + p * 16) = v;
    Ps[p] = sc;
  }
}

size_t mx_packed_bf16_bytes(int N, int K) {
  return (size_t)(N / 16) * ((K + 127) / 128) * 256 * 16;
}

size_t mx_packed_fp4_pieces(int E, int N, int K) {
  return (size_t)E * (N / 16) * ((K / 32 + 15) / 16) * 256;
}

void launch_mx_pack_bf16(const uint16_t* W, int N, int K, uint16_t* P, hipStream_t st) {
  hipLaunchKernelGGL(k_mx_pack_bf16, dim3(2048), dim3(256), 0, st, W, N, K, P);
}

void launch_mx_pack_fp4(const uint8_t* codes, const uint8_t* scales, int E, int N, int K,
                        uint8_t* Pc, uint8_t* Ps, hipStream_t st) {
  hipLaunchKernelGGL(k_mx_pack_fp4, dim3(2048), dim3(256), 0, st, codes, scales, E, N, K, Pc,
                     Ps);
}

}  // namespace neon

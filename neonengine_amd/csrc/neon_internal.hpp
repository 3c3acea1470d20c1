// neon_internal.hpp -- host launchers of the gfx950 kernels (library-
// internal; the public surface is include/neon_gptoss.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace neon {

// ---- init -----------------------------------------------------------------
void launch_fill_bf16(uint16_t* out, int64_t n, uint64_t seed, uint64_t stream,
                      float mean, float mul, hipStream_t st);
void launch_fill_bytes(uint8_t* out, int64_t n, uint64_t seed, uint64_t stream,
                       hipStream_t st);
void launch_fill_scales(uint8_t* out, int64_t n, uint64_t seed,
                        uint64_t stream, int lo, int range, hipStream_t st);

// ---- MXFP4 ------------------------------------------------------------------
void launch_mxfp4_dequant(const uint8_t* codes, const uint8_t* scales,
                          int64_t n_blocks, float* out, hipStream_t st);
void launch_mxfp4_gemv(const uint8_t* codes, const uint8_t* scales,
                       const uint16_t* bias, const uint16_t* x, uint16_t* y,
                       int N, int K, int B, hipStream_t st);

// ---- bf16 GEMV with fused prologue/epilogue ---------------------------------
// QKV mode outputs: rotated q heads [B][Hq][64], and k (rotated) / v rows
// written at cache row pos[b] of kc / vc [B][Hkv][T_max][64]
struct RopeArgs {
  const int32_t* pos = nullptr;
  const float* cos_t = nullptr;  // [T_max][32]
  const float* sin_t = nullptr;
  uint16_t* q_out = nullptr;
  uint16_t* kc = nullptr;
  uint16_t* vc = nullptr;
  const int32_t* seq = nullptr;  // KV-cache sequence of each row (NULL: row b is sequence b)
  int Hq = 0, Hkv = 0, T_max = 0;  // T_max: cache rows per (sequence, kv head)
  int key_mask = -1;  // position p sits in cache row p & key_mask (ring caches: rows - 1)
};

struct GemvArgs {
  int mode = 0;  // 0 store, 1 residual add into y, 2 fp32 logits + argmax parts,
                 // 3 QKV projection (store) + RoPE + KV-cache append
  const uint16_t* W = nullptr;
  const uint16_t* bias = nullptr;
  const uint16_t* x = nullptr;
  const uint16_t* norm_w = nullptr;  // fused RMSNorm of x when not NULL
  float eps = 1e-5f;
  uint16_t* y = nullptr;
  float* logits = nullptr;
  float* part_val = nullptr;
  int32_t* part_idx = nullptr;
  int N = 0, K = 0, B = 1;
  int nblk = 1;  // grid.x (gemv_default_grid; wave row groups are grid-strided)
  // mode 3 only (head_dim 64; N = (Hq + 2 Hkv) 64)
  const int32_t* pos = nullptr;
  const float *cos_t = nullptr, *sin_t = nullptr;
  uint16_t *q_out = nullptr, *kc = nullptr, *vc = nullptr;
  const int32_t* seq = nullptr;  // KV-cache sequence of each row (NULL: identity)
  int Hq = 0, Hkv = 0, T_max = 0;
  int key_mask = -1;
};
// grid.x for N rows in `mode` (the rows per wave group depend on the mode)
int gemv_default_grid(int N, int mode);
void launch_gemv_bf16(const GemvArgs& a, hipStream_t st);
// B >= 2: every weight row read once for up to 16 batch rows (K = 2880 or
// 4096; nblk from gemv_bt_grid).  Outputs bit-identical to launch_gemv_bf16.
hipError_t launch_gemv_bf16_batched(const GemvArgs& a, hipStream_t st);
// shapes and modes the batched kernel covers (QKV and lm_head with RMSNorm,
// O without; K / 8 units in 1, 2, 3, 4, 6 or 8 passes of 64)
bool gemv_batched_supported(const GemvArgs& a);
// opts the batched kernels in to their LDS size (once per device, outside
// any stream capture)
hipError_t gemv_batched_prepare();
int gemv_bt_grid(int N, int mode);

// temperature / nucleus sampling of logits [B][V] (scratch [B][V] floats);
// with advance, writes the token and advances pos like launch_argmax_advance
void launch_sample(const float* logits, int B, int V, float temperature, float top_p,
                   uint64_t seed, int32_t* pos, float* scratch, int32_t* out_ids,
                   int32_t* tokens, int tok_stride, const int32_t* prompt_len, bool advance,
                   hipStream_t st, int row0 = 0);
void launch_argmax_advance(const float* part_val, const int32_t* part_idx,
                           int nparts, int32_t* tokens, int tok_stride,
                           int32_t* pos, const int32_t* prompt_len,
                           int32_t* last_ids, int B, hipStream_t st);
void launch_embed(const int32_t* tokens, int tok_stride, const int32_t* pos,
                  const int32_t* seq,
                  const uint16_t* embed, uint16_t* h, int H, int B,
                  hipStream_t st);
// the normalised rows in the matrix-core activation layout (k_rmsnorm_packed:
// [ceil(B/16)][ceil(H/128)][4][64][8] bf16, zero past B and H)
void launch_rmsnorm_packed(const uint16_t* x, const uint16_t* w, uint16_t* out, int B, int H,
                           float eps, hipStream_t st);
void launch_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out, int B,
                    int H, float eps, hipStream_t st);
// the matrix-core experts' combine (ybuf [B][k][H] fp32, slots in order) into
// h and the following launch_rmsnorm_packed(h, nw, out) in one launch; false
// (nothing launched) when the shape is not covered (k != 4, H % 8, H > 4096)
bool launch_mx_combine_norm(const float* ybuf, const float* score, uint16_t* h,
                            const uint16_t* nw, uint16_t* out, int B, int H, int k, float eps,
                            hipStream_t st);

// ---- RoPE ---------------------------------------------------------------------
void launch_rope_apply(uint16_t* x, const int32_t* pos, const float* cos_t,
                       const float* sin_t, int n_tok, int n_heads, int D,
                       hipStream_t st);

// ---- router / MoE --------------------------------------------------------------
struct RouterArgs {
  const uint16_t* x = nullptr;       // [B][H]
  const uint16_t* norm_w = nullptr;  // fused RMSNorm of x when not NULL
  float eps = 1e-5f;
  uint16_t* xn_out = nullptr;        // normalised x [B][H] (may be NULL)
  const uint16_t *W = nullptr, *bias = nullptr;
  float* lg_out = nullptr;           // logits [B][E]
  int32_t* idx = nullptr;            // top-k outputs (NULL: logits only)
  float* score = nullptr;
  int B = 1, E = 0, H = 0, k = 0;
  // zeroed by block (0, 0) before anything else (the counters of the
  // one-launch expert kernel that follows), may be NULL
  int32_t* zero = nullptr;
  int zero_n = 0;
  // with xn_out: its two-term MXFP8 image (hi, lo [B][H], scales [B][H/32]),
  // written by the same wave (NULL: none)
  uint8_t *xq_hi = nullptr, *xq_lo = nullptr, *xs_hi = nullptr, *xs_lo = nullptr;
  // launch_gemv_o_router only: kMoeSyncWords + 1 words kMoeSyncStride ints
  // apart (0 at launch, left at 0) and the device status word
  int32_t* arrive = nullptr;
  int32_t* err = nullptr;
  // launch_router with idx: B counters kMoeSyncStride ints apart (0 at
  // launch, left at 0); the top-k then finishes in the logits launch (the
  // last wave of each row ranks it) instead of a launch of its own
  int32_t* row_arrive = nullptr;
};
// router logits, then (when a.idx) the top-k / softmax
void launch_router(const RouterArgs& a, hipStream_t st);
// O projection + residual (o, mode 1) and the router logits of its output (r)
// in one launch, batch 1; bit-identical to launch_gemv_bf16(o) then
// launch_router(r)
bool o_router_supported(const GemvArgs& o, const RouterArgs& r);
void launch_gemv_o_router(const GemvArgs& o, const RouterArgs& r, hipStream_t st);

// Status bits a kernel sets (vector atomicOr) in the caller's status word
// when its input breaks a precondition it can only see on the device.
constexpr int32_t kDevErrExpertId = 1;      // an expert id outside [0, E)
constexpr int32_t kDevErrSyncTimeout = 2;   // a grid-wide wait gave up (results invalid)
// polls a grid-wide wait makes before it gives up (~1 s)
constexpr int kMoeSpinLimit = 1 << 20;

struct MoeArgs {
  int32_t* err = nullptr;    // status word (kDevErr* bits), may be NULL
  const uint8_t *gu_codes, *gu_scales, *dn_codes, *dn_scales;
  const uint16_t *gu_bias, *dn_bias;
  const float* router_lg;    // [B][E] router logits: experts chosen in-kernel
  const int32_t* idx;        // else the given expert ids [B][k] ...
  const float* score;        // ... and weights [B][k]
  int32_t* idx_out;          // chosen ids / weights (may be NULL)
  float* score_out;
  int E;
  const uint16_t* xn;        // [B][H] normalised input
  uint16_t* act;             // [B][k][I] scratch
  const uint16_t* residual;  // may be NULL
  uint16_t* out;             // [B][H]
  int B, H, I, k;
  float alpha, limit;
  // batch 1: kMoeSyncShards zeroed int32 counters enable the one-launch
  // expert kernel (k_moe_fused); NULL keeps the two-kernel form
  int32_t* sync = nullptr;
};
void launch_moe(const MoeArgs& a, hipStream_t st);
// the one-launch form (batch 1, k <= 4, I % 4 == 0, sync given); returns
// false when it does not apply (nothing launched)
bool moe_fused_supported(const MoeArgs& a);
bool launch_moe_fused(const MoeArgs& a, hipStream_t st);
constexpr int kMoeSyncWords = 32;    // arrival counter shards per fused launch,
constexpr int kMoeGoCopies = 8;      // then the copies of its go flag,
constexpr int kMoeSyncStride = 64;   // each on its own 256-byte line (in int32)
constexpr int kMoeSyncInts = (kMoeSyncWords + kMoeGoCopies) * kMoeSyncStride;
constexpr int kMoeSyncZero = kMoeSyncWords + kMoeGoCopies;  // words to zero
constexpr int kMoeFusedMaxUnits = 96;  // H / 32 of the one-launch experts (H <= 3072)

// ---- batched decode on the matrix cores (neon_mx.hip) ----------------------
constexpr int kMxMaxRows = 64;   // rows per step
constexpr int kMxMaxK = 4096;    // reduction length
struct MxArgs {
  int32_t* err = nullptr;    // status word (kDevErr* bits), may be NULL
  const void* W;             // bf16 [N][K], or MXFP4 codes [E][N][K/2] (expert modes)
  const uint8_t* scales;     // MXFP4 scales [E][N][K/32] (expert modes)
  const uint16_t* bias;      // [N], [E][N] (expert modes) or NULL (dense modes)
  const uint16_t* x;         // input rows of K bf16: [B][K]; gate_up [B][K]; down [B k][K]
  // dense modes with Wp: the input rows in the activation layout of
  // launch_rmsnorm_packed instead of x (1 KB contiguous per MFMA operand), or NULL
  const uint16_t* xp = nullptr;
  uint16_t* y;               // store / residual [B][N]; gate_up: act [B k][N / 2]
  float* out_f;              // logits [B][N]; down: per-pair dot + bias [B k][N]
  float* part_val;           // logits: per-block (max, lowest index) [B][N / 16]
  int32_t* part_idx;
  const int32_t* idx;        // expert modes: experts of the B k (row, slot) pairs
  const void* Wp;            // the same weights in MFMA lane order (mx_pack_*), or NULL
  const uint8_t* sp;         // packed MXFP4 scales (with Wp, expert modes)
  const int32_t* route;      // expert modes: used experts, counts, pair lists
                             // [2 S + 64 S] ints, S = min(E, B k), and the work
                             // items at kMxItemOff (kMxRouteWords ints in all),
                             // written by launch_topk_route / launch_router_route
                             // before the expert kernels; or NULL: each expert
                             // block builds its item from idx (mx_route_item)
  int B, N, K, E, k;
  float alpha, limit;
  // expert modes on the scaled fp8 x fp4 instruction (launch_mx_moe8): the
  // input rows' two-term MXFP8 image, hi / lo [rows][K], scales [rows][K/32];
  // gate_up also writes its SwiGLU output's image into yq_* ([B k][N / 2])
  const uint8_t *xq_hi = nullptr, *xq_lo = nullptr, *xs_hi = nullptr, *xs_lo = nullptr;
  uint8_t *yq_hi = nullptr, *yq_lo = nullptr, *ys_hi = nullptr, *ys_lo = nullptr;
};
bool mx_shape_ok(int N, int K, int B);
// standalone MXFP4 GEMV on the matrix cores (checkpoint layout, K % 32 == 0,
// K <= 8192, any N and B): equal to the canonical GEMV up to the order of the
// fp32 additions
void launch_mxfp4_gemv_mfma(const uint8_t* codes, const uint8_t* scales, const uint16_t* bias,
                            const uint16_t* x, uint16_t* y, int N, int K, int B,
                            hipStream_t st);
constexpr int kMxfp4GemvMfmaMinB = 16;  // batch rows from which neon_mxfp4_gemv uses it
bool mx_moe_shape_ok(int H, int I, int E, int k, int B);
// MFMA lane-order copies (each load instruction of the matrix-core kernels
// then reads 1 KB contiguous): sizes in bytes, and the packing launches.
size_t mx_packed_bf16_bytes(int N, int K);
size_t mx_packed_fp4_pieces(int E, int N, int K);  // 16-byte code pieces = scale bytes
void launch_mx_pack_bf16(const uint16_t* W, int N, int K, uint16_t* P, hipStream_t st);
void launch_mx_pack_fp4(const uint8_t* codes, const uint8_t* scales, int E, int N, int K,
                        uint8_t* Pc, uint8_t* Ps, hipStream_t st);
// mode 0: y = bf16(x W^T + bias); 1: y = bf16(y + bf16(x W^T + bias));
// 2: logits = x W^T (fp32) with per-block argmax partials
void launch_mx_gemv(const MxArgs& a, int mode, hipStream_t st);
// experts of B rows: gate_up + SwiGLU into act, down + bias per pair, then the
// slot-ordered combine h = bf16(h + bf16(sum_s score_s (dot_s + bias_s)))
// (the work items from the route table or the expert ids; the weights from
// the packed copies in Wp / sp).  With next_norm given, the combine also
// writes launch_rmsnorm_packed(h, next_norm, next_xp) when it can (the
// return value says whether it did).
bool launch_mx_moe(const MxArgs& gate_up, const MxArgs& down, const float* score, uint16_t* h,
                   hipStream_t st, const uint16_t* next_norm = nullptr, float eps = 0.0f,
                   uint16_t* next_xp = nullptr);
// launch_mx_moe with the expert GEMMs on v_mfma_scale_f32_16x16x128_f8f6f4:
// gate_up.xq_* hold the MXFP8 image of gate_up.x (the router writes it),
// gate_up.yq_* receive the image of the SwiGLU output that down reads; the
// packed MXFP4 pieces feed the B operand as they are
bool launch_mx_moe8(MxArgs gate_up, MxArgs down, const float* score, uint16_t* h,
                    hipStream_t st, const uint16_t* next_norm = nullptr, float eps = 0.0f,
                    uint16_t* next_xp = nullptr);
// top-k of B rows of router logits and the route lists of their pairs
// (B k <= 256, E <= 256) in one launch
// launch_router (norm fused, no MXFP8 image) + launch_topk_route in one
// launch for B >= 2: a.arrive = one int, 0 at launch and left at 0
bool router_route_supported(const RouterArgs& a);
void launch_router_route(const RouterArgs& a, int32_t* idx, float* score, int32_t* route,
                         hipStream_t st);
void launch_topk_route(const float* lg, int32_t* idx, float* score, int B, int E, int k,
                       int32_t* route, hipStream_t st);
void launch_mx_rope_append(const uint16_t* qkv, const int32_t* pos, const int32_t* seq,
                           const float* cos_t, const float* sin_t, uint16_t* q_out,
                           uint16_t* kc, uint16_t* vc, int B, int Hq, int Hkv, int T_max,
                           int key_mask, hipStream_t st);
// 2 <= B, B k <= 64, idx / score given (router_lg NULL): each used expert's
// weights read once for all rows that chose it; bit-identical to launch_moe
bool moe_batched_supported(const MoeArgs& a);
void launch_moe_batched(const MoeArgs& a, hipStream_t st);

// ---- attention ------------------------------------------------------------------
struct AttnArgs {
  const uint16_t* q;      // rotated q [B][q_stride] (head h at h*D)
  const uint16_t *kc, *vc;  // [B][Hkv][T_max][D], key pos already appended
  const uint16_t* sinks;  // [Hq]
  const int32_t* pos;     // [B]
  uint16_t* out;          // [B][Hq*D]
  float* part_o;          // [B][Hq][S][D] split partials (scratch)
  float* part_ml;         // [B][Hq][S][2]
  const int32_t* seq;     // KV-cache sequence of each row, or NULL (row b = sequence b)
  int B, Hq, Hkv, T_max, window, S, q_stride;
  // key j sits in cache row j & key_mask: -1 for a cache of every position,
  // rows - 1 for a power-of-two ring that holds the last `rows` positions
  int key_mask;
  // arrival counters [B][Hkv] (stride kAttnArriveStride ints, 0 at launch and
  // left at 0): with S > 1 the split kernel's last block per (row, kv head)
  // merges; NULL: a separate merge kernel (launch_attn only)
  int32_t* arrive = nullptr;
  // matrix-core steps (launch_mx_attn): the output also in the packed
  // activation layout (K = Hq D, a multiple of 128) for the O projection, or NULL
  uint16_t* out_packed = nullptr;
  // matrix-core steps: q is the projection's raw output row ([B][q_stride],
  // q_stride = (Hq + 2 Hkv) D, q heads then k then v) and the attention
  // kernel rotates q itself and, in the block that holds position pos[b],
  // rotates k and appends k and v to the caches (launch_mx_rope_append's
  // arithmetic); cos / sin are the RoPE tables [max_seq][D / 2].  NULL: q is
  // already rotated and the new key already appended.
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;
};
// ints between consecutive arrival counters (one 256-byte line each)
constexpr int kAttnArriveStride = 64;
// decode attention of the matrix-core steps (same partials and merge as launch_attn)
void launch_mx_attn(const AttnArgs& a, hipStream_t st);
void launch_attn_merge(const AttnArgs& a, hipStream_t st);
void launch_attn(const AttnArgs& a, hipStream_t st);
// number of key splits used for a cache of T_max rows (window 0 = full layer)
int attn_splits(int T_max, int window);
// top-k + softmax of router logits lg [B][E] (one wave per row)
void launch_topk(const float* lg, int32_t* idx, float* score, int B, int E, int k,
                 hipStream_t st);

// ---- prefill (neon_prefill.hip): M prompt rows at once on the matrix cores --
void launch_embed_rows(const int32_t* ids, int M, const uint16_t* embed,
                       uint16_t* h, int H, hipStream_t st);
// C[M][N] = A[M][K] W[N][K]^T + bias; mode 0: bf16 store, 1: C = bf16(C +
// bf16(.)) (residual in place), 2: fp32 into Cf.  K % 32 == 0.
void launch_gemm_bf16(const uint16_t* A, int lda, const uint16_t* W, int ldw,
                      const uint16_t* bias, uint16_t* C, float* Cf, int ldc, int M,
                      int N, int K, int mode, hipStream_t st);
// The prompt pass's projections (dense, lda = ldw = K, ldc = N; mode 0 or 1
// as launch_gemm_bf16, whose direct-load kernel takes them; for the residual
// C = bf16(C + bf16(acc + bias))).
void launch_prompt_proj(const uint16_t* A, const uint16_t* W, const uint16_t* bias,
                        uint16_t* C, int M, int N, int K, int mode, hipStream_t st);
void launch_rope_kv_rows(const uint16_t* qkv, int q_stride, const float* cos_t,
                         const float* sin_t, int M, int Hq, int Hkv, int T_max,
                         uint16_t* q_out, uint16_t* kc, uint16_t* vc, hipStream_t st);
void launch_kv_ring_store(const uint16_t* ks, const uint16_t* vs, int S, int t0, int M,
                          int Hkv, int R, uint16_t* kc, uint16_t* vc, hipStream_t st);
void launch_attn_prefill(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                         const uint16_t* sinks, uint16_t* out, int M, int Hq, int Hkv,
                         int T_max, int window, hipStream_t st);
struct MoePrefillArgs {
  int32_t* err = nullptr;    // status word (kDevErr* bits), may be NULL
  const int32_t* idx;        // [M][k] chosen experts
  const float* score;        // [M][k] weights
  const uint16_t* xn;        // [M][H] normalised input
  uint16_t* h;               // [M][H] residual stream, updated in place
  const uint8_t *gu_codes, *gu_scales, *dn_codes, *dn_scales;
  const uint16_t *gu_bias, *dn_bias;
  int M, E, H, I, k;
  float alpha, limit;
  // scratch
  int32_t *list_tok, *list_slot;  // [M k]
  int32_t* e_off;                 // [E + 1]
  int32_t *tile_e, *tile_r0;      // [moe_prefill_max_tiles]
  int32_t* n_tiles;               // [1]
  uint16_t* act;                  // [M k][I]
  float* ybuf;                    // [M][k][H]
  // MXFP8 expert GEMMs (scaled matrix instruction) when q is given: the GEMM
  // input's two E4M3 terms in step lines (per row and 64-element step, 64
  // hi bytes then 64 lo bytes), 2 max(M H, M k I) bytes, and their scales
  // (one dword per row and step: s_hi of both 32-blocks, then s_lo),
  // max(M H, M k I) / 16 bytes; H and I multiples of 64
  uint8_t* q = nullptr;
  uint32_t* qs = nullptr;
};
int moe_prefill_max_tiles(int M, int k, int E);
// the two-term MXFP8 image of bf16 rows: separate hi / lo / s_hi / s_lo
// arrays (the kernel-level layout), or (q, qs) step lines for the GEMMs
void launch_mx8_quant(const uint16_t* x, int64_t rows, int K, uint8_t* hi, uint8_t* lo,
                      uint8_t* s_hi, uint8_t* s_lo, hipStream_t st);
// scale dwords per row of the step-line layout (K / 64 steps, rounded up to
// a multiple of 4) and the bytes of rows such rows
__host__ __device__ inline int mx8_scale_stride(int K) { return ((K / 64) + 3) & ~3; }
inline size_t mx8_scale_bytes(size_t rows, int K) { return rows * (size_t)mx8_scale_stride(K) * 4; }
void launch_mx8_quant_lines(const uint16_t* x, int64_t rows, int K, uint8_t* q, uint32_t* qs,
                            hipStream_t st);
void launch_moe_prefill(const MoePrefillArgs& a, hipStream_t st);

}  // namespace neon

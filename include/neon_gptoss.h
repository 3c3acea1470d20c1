/*
 * neon_gptoss.h -- C-ABI of the MI355X (gfx950) gpt-oss token loop.
 *
 * Boundary.  The reference repository (NeonEngine) has no model-loading,
 * forward or FFI interface for this path; it is a Vulkan graphics engine whose
 * only GPU-work idiom is the C++ "System" object: a constructor that allocates
 * device state and throws on failure, and a per-frame call that records a
 * fixed sequence of compute dispatches into a caller-provided command buffer
 * (NeonEngine/src/water_physics.cpp:23-123 constructor, :131 RunSimulation,
 * :165-436 the dispatch chain; NeonEngine/src/raytracing_system.cpp:19-68,
 * :1217 runShaders).  This header keeps that shape with HIP in place of
 * Vulkan: a context is created once (neon_ctx_create ~ System constructor),
 * every call enqueues work on a caller-provided stream (~ recording into the
 * caller's VkCommandBuffer) and returns before the GPU finishes, and the
 * caller synchronises.  Errors come back as neon_status codes instead of
 * exceptions (the reference throws std::runtime_error up to main,
 * NeonEngine/src/main.cpp:21-26); no C++ exception crosses this ABI.
 *
 * Conventions.
 *   - All tensor pointers passed to kernel-level entry points are DEVICE
 *     pointers owned by the caller.  bf16 tensors are passed as uint16_t bit
 *     patterns.  Host arrays (prompt ids, outputs of neon_read_*) are copied
 *     before the call returns.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *   - A context is not thread-safe; use one context per host thread.
 *   - MXFP4 weights use the gpt-oss checkpoint layout: codes [N][K/2] bytes
 *     (low nibble = element 2i, high nibble = element 2i+1), E8M0 scales
 *     [N][K/32] bytes, one per 32 consecutive elements along K.
 */
#ifndef NEON_GPTOSS_H
#define NEON_GPTOSS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum neon_status {
  NEON_OK = 0,
  NEON_EINVAL = 1,       /* bad argument: null pointer, bad shape or size   */
  NEON_ENOMEM = 2,       /* device or host allocation failed                */
  NEON_EHIP = 3,         /* a HIP runtime call failed (no device, ...)      */
  NEON_ENAN_SCALE = 4,   /* an E8M0 scale byte 0xFF (NaN) in loaded weights */
  NEON_EKV_FULL = 5,     /* the step would write past the KV-cache capacity */
  NEON_ERANGE_TOKEN = 6, /* a token id outside [0, vocab)                   */
  NEON_ESTATE = 7        /* call out of order (e.g. decode before prefill)  */
} neon_status;

typedef struct neon_ctx neon_ctx;

/* Model shape.  Field meaning follows the gpt-oss config (HF
 * configuration_gpt_oss.py); max_seq / max_batch size the KV cache. */
typedef struct neon_config {
  int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim;
  int32_t n_experts, top_k, intermediate, vocab;
  int32_t sliding_window, max_seq, max_batch;
  float rope_theta, rope_factor, rope_beta_fast, rope_beta_slow;
  int32_t rope_orig_max_pos;
  float rms_eps, swiglu_limit, swiglu_alpha;
} neon_config;

/* ---- context-level API (the token loop) --------------------------------- */

/* Fills `out` with a preset: "gpt-oss-20b" or "gpt-oss-120b". */
neon_status neon_config_preset(const char* name, neon_config* out);

/* Validates `cfg`, selects `device`, allocates weights, KV cache and
 * activations.  Counterpart of the System constructor idiom
 * (NeonEngine/src/water_physics.cpp:23-123). */
neon_status neon_ctx_create(const neon_config* cfg, int device, neon_ctx** out);
/* Waits for the device to finish the context's queued work, then releases
 * it.  NULL is ignored. */
void neon_ctx_destroy(neon_ctx* ctx);

/* Text of the last error on this context (or of the last failed
 * neon_ctx_create on this thread when ctx is NULL). */
const char* neon_last_error(const neon_ctx* ctx);

/* Deterministic random weights (counter-based RNG keyed by seed and tensor),
 * generated on the device; the CPU oracle regenerates the same bits. */
neon_status neon_init_random(neon_ctx* ctx, uint64_t seed, void* stream);

/* Copies one named tensor from host memory (gpt-oss checkpoint names, e.g.
 * "model.layers.3.mlp.experts.gate_up_proj_blocks").  MXFP4 scale tensors
 * are checked for the NaN byte 0xFF (NEON_ENAN_SCALE). */
neon_status neon_load_tensor(neon_ctx* ctx, const char* name,
                             const void* host_data, size_t bytes);

/* Starts `batch` sequences from host prompt ids [batch][n_tokens] and runs
 * the prompt; afterwards the first generated token of each sequence is
 * available.  Modes (neon_set_prefill_mode):
 *  - NEON_PREFILL_CHUNKED (default): prompt rows 0 .. n_tokens-2 of a
 *    sequence go through every layer 16 rows at a time with the batched decode
 *    kernels (each weight row read once per 16 rows, causal attention over the
 *    sequence's cache), then the last prompt token runs as a decode step.
 *    Bit-identical to NEON_PREFILL_STEPWISE.
 *  - NEON_PREFILL_STEPWISE: every prompt token as a decode step.
 *  - NEON_PREFILL_BATCHED: all prompt rows of a sequence at once on the
 *    matrix cores (bf16 MFMA GEMMs, grouped MXFP4 expert GEMMs, tiled causal
 *    prompt attention); agrees with the other modes to bf16 rounding, not
 *    bit for bit.
 * None has a counterpart in the reference, which has no model code. */
neon_status neon_prefill(neon_ctx* ctx, const int32_t* ids, int batch,
                         int n_tokens, void* stream);

/* neon_prefill for prompts of different lengths: sequence b's prompt is
 * lens[b] >= 1 ids, the prompts stored one after another in `ids` (sum of
 * lens[] entries).  Every sequence keeps its own position: afterwards
 * sequence b holds lens[b] + 1 tokens (neon_seq_lens), its KV cache rows
 * 0 .. lens[b]-1, and each decode step adds one token to every sequence.
 * NEON_PREFILL_CHUNKED packs the prompt rows of all sequences into its
 * 16-row passes (a sequence's rows in position order), STEPWISE runs them
 * one row at a time and BATCHED one matrix-core pass per sequence; in the
 * exact modes each sequence's logits are bit-identical to prefilling it
 * alone.  neon_read_tokens gives 0 past a sequence's length.  max_seq bounds
 * the longest sequence.  (No counterpart in the reference.) */
neon_status neon_prefill_ragged(neon_ctx* ctx, const int32_t* ids,
                                const int32_t* lens, int batch, void* stream);

enum {
  NEON_PREFILL_BATCHED = 0,
  NEON_PREFILL_STEPWISE = 1,
  NEON_PREFILL_CHUNKED = 2,
  /* NEON_PREFILL_BATCHED with the expert GEMMs on the scaled fp8 x fp4
   * matrix instruction: each bf16 input block of 32 carried as two MXFP8
   * (E4M3) terms, the MXFP4 expert rows read as stored (hidden and
   * intermediate are multiples of 64 in every context). */
  NEON_PREFILL_MX8 = 3
};
/* Selects how neon_prefill runs the prompt (default NEON_PREFILL_CHUNKED). */
neon_status neon_set_prefill_mode(neon_ctx* ctx, int mode);

enum { NEON_DECODE_EXACT = 0, NEON_DECODE_MATRIX = 1, NEON_DECODE_MATRIX_MX8 = 2 };
/* Selects how decode steps of two or more sequences run (a step of one
 * sequence always runs the exact kernels):
 *  - NEON_DECODE_EXACT (default): every dot product in the canonical fp32
 *    order, so each sequence's logits are bit-identical to decoding it alone;
 *  - NEON_DECODE_MATRIX: every weight row read once per step with the
 *    sequences in the M dimension of v_mfma_f32_16x16x32_bf16 tiles (expert
 *    rows dequantised exactly to bf16); the same rounding points, with fp32
 *    additions in another order.  Needs max_batch <= 64, output widths that
 *    are multiples of 16 and reductions that are multiples of 32 up to 4096
 *    (NEON_EINVAL otherwise);
 *  - NEON_DECODE_MATRIX_MX8: NEON_DECODE_MATRIX with the expert GEMMs on
 *    v_mfma_scale_f32_16x16x128_f8f6f4 (the MXFP4 expert rows as the scaled
 *    B operand, each expert input as two MXFP8 terms per 32-element block,
 *    within 2^(floor(log2 amax) - 8) of the bf16 values).
 * No counterpart in the reference, which has no model code. */
neon_status neon_set_decode_mode(neon_ctx* ctx, int mode);

/* Runs `n_steps` greedy decode steps for every live sequence (each step
 * consumes the previously generated token and produces the next one). */
neon_status neon_decode(neon_ctx* ctx, int n_steps, void* stream);

/* Synchronises `stream` and copies tokens [start, start+count) of every
 * sequence into out [batch][count] (prompt tokens first, then generated). */
neon_status neon_read_tokens(neon_ctx* ctx, int start, int count,
                             int32_t* out, void* stream);

/* Synchronises and copies the fp32 logits of the last step [batch][vocab]. */
neon_status neon_read_logits(neon_ctx* ctx, float* out, void* stream);

/* Next-token choice of the decode steps: temperature 0 (the default) is
 * greedy argmax; temperature > 0 samples from softmax(logits / temperature)
 * restricted to the smallest top-probability set of mass >= top_p (nucleus,
 * top_p in (0, 1]; 1 keeps every token), with a counter-based RNG keyed by
 * (seed, sequence, position), so a run is reproducible.  Prompt tokens are
 * still teacher-forced.  (The reference has no model code, so nothing here
 * has a counterpart in it.) */
neon_status neon_set_sampling(neon_ctx* ctx, float temperature, float top_p,
                              uint64_t seed);

/* Synchronises and copies one activation buffer of the last step (for
 * parity tests of the fused chain; "last layer" = the final decoder layer):
 *   "hidden"    residual stream before the final norm, bf16 [batch][hidden]
 *   "qkv"       last layer's q/k/v projection (before RoPE), bf16
 *               [batch][(n_heads + 2 n_kv_heads) head_dim]
 *   "attn_out"  last layer's attention output, bf16 [batch][n_heads head_dim]
 *   "moe_in"    last layer's normalised MoE input, bf16 [batch][hidden]
 *   "moe_idx"   last layer's expert ids, int32 [batch][top_k]
 *   "moe_score" last layer's routing weights, fp32 [batch][top_k]
 *   "mx_route"  after a NEON_DECODE_MATRIX step of two or more sequences: the
 *               last layer's route table, int32 [2 S + 64 S] with S =
 *               min(n_experts, batch top_k): used expert of slot y (ascending,
 *               -1 past the used ones), its pair count, then its pairs
 *               q = b top_k + s in ascending order (64 entries per slot)
 *   "mx_items"  after the same steps: the expert kernels' work items, int32
 *               [257]: the count n, then n items (slot | group << 8 |
 *               expert << 10 | min(pair count, 64) << 19), group 0 of every
 *               used slot first, then group 1 (pairs 16 .. 31) of the slots
 *               with more than 16 pairs, and so on
 * `bytes` must equal the buffer's size. */
neon_status neon_read_activation(neon_ctx* ctx, const char* name, void* out,
                                 size_t bytes, void* stream);

/* Number of tokens held by the longest sequence (prompt + generated); with
 * equal prompt lengths every sequence holds this many. */
neon_status neon_seq_len(const neon_ctx* ctx, int* out);

/* Number of tokens held by each sequence (prompt + generated), out[batch]
 * (0 for a free row); NEON_ESTATE before the first prefill. */
neon_status neon_seq_lens(const neon_ctx* ctx, int32_t* out);

/* Continuous batching: a sequence joins a running context.  Its prompt
 * ids[0 .. n-1] takes the lowest free batch row (one never used, or freed by
 * neon_seq_remove) with that row's KV block, goes through the context's
 * prompt mode, and its first generated token is chosen (written at
 * position n of the row); no other sequence advances.  *slot receives the
 * row.  Later neon_decode steps advance every held row.  NEON_EKV_FULL when
 * every row of max_batch holds a sequence or n > max_seq.  (The reference
 * has no counterpart: it renders one fixed scene per frame.) */
neon_status neon_seq_add(neon_ctx* ctx, const int32_t* ids, int n, int* slot, void* stream);

/* A sequence leaves: its batch row and KV block become free for the next
 * neon_seq_add.  Steps leave a free row untouched (no token, no advance);
 * free rows at the end of the batch leave the step altogether. */
neon_status neon_seq_remove(neon_ctx* ctx, int slot, void* stream);

/* Device pointer of a weight tensor (same names as neon_load_tensor), for
 * tests and tools; *bytes receives its size.  Read it freely; bytes written
 * through it bypass neon_load_tensor's checks, and the NEON_DECODE_MATRIX
 * steps keep reading their packed copy until the next neon_load_tensor or
 * neon_init_random. */
neon_status neon_tensor_ptr(neon_ctx* ctx, const char* name, void** ptr,
                            size_t* bytes);

/* ---- kernel-level API (device pointers; stream-ordered) ------------------ */
/* No kernel-level call allocates device memory: scratch space is a caller-
 * owned workspace whose size the matching *_workspace query returns (the
 * reference's idiom: buffers created once with the System, dispatches
 * recorded per frame without allocation, water_physics.cpp:103,449 and
 * :165-436).  A workspace may be reused by later calls; calls that overlap
 * on one device must not share one. */

/* Synchronises `stream`, then reports (and clears) the status bits that the
 * kernel-level calls on the current device have set since the last check:
 * NEON_EINVAL when an expert id given in device memory (neon_moe_experts,
 * neon_moe_prefill) lay outside [0, E).  Such a slot is dropped (adds 0)
 * instead of reading past the expert arrays.  The context-level reads
 * (neon_read_tokens / _logits / _activation) make the same check for the
 * context's own kernels.  (The reference has no counterpart: its Systems
 * throw on the host and do no device-side validation.) */
neon_status neon_device_check(void* stream);

/* out[32 b + j] = E2M1(code) * 2^(scale_b - 127) in fp32, bit-exact;
 * scale 0xFF gives NaN. */
neon_status neon_mxfp4_dequant(const uint8_t* codes, const uint8_t* scales,
                               int64_t n_blocks, float* out, void* stream);

/* y[b][n] = bf16( sum_k dq(W[n][k]) x[b][k] + bias[n] ), fp32 accumulate.
 * bias may be NULL.  K % 32 == 0, K <= 8192. */
neon_status neon_mxfp4_gemv(const uint8_t* codes, const uint8_t* scales,
                            const uint16_t* bias, const uint16_t* x,
                            uint16_t* y, int N, int K, int B, void* stream);

/* y[b][n] = bf16(sum_k x[b][k] W[n][k] + bias[n]) for B <= 64 rows on the
 * matrix cores (the projection kernel of NEON_DECODE_MATRIX): N a multiple
 * of 16, K a multiple of 32 up to 4096, bias may be NULL.  Equal to
 * neon_gemv_bf16 up to the order of the fp32 additions. */
neon_status neon_gemv_bf16_mfma(const uint16_t* W, const uint16_t* bias, const uint16_t* x,
                                uint16_t* y, int N, int K, int B, void* stream);

/* bf16 GEMV (nn.Linear layout W [N][K]); bias may be NULL; K % 8 == 0. */
neon_status neon_gemv_bf16(const uint16_t* W, const uint16_t* bias,
                           const uint16_t* x, uint16_t* y, int N, int K, int B,
                           void* stream);

/* out[b] = bf16( w * (x[b] * rsqrt(mean(x[b]^2) + eps)) ). */
neon_status neon_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out,
                         int B, int H, float eps, void* stream);

/* YaRN RoPE table for positions 0 .. n_pos-1 from cfg's rope fields (HFR
 * yarn inv_freq, cos/sin times the attention factor), written to the device
 * array table [2][n_pos][head_dim/2] fp32 (cos, then sin).  A set-up call:
 * it returns after the copy has completed. */
neon_status neon_rope_table(const neon_config* cfg, int n_pos, float* table, void* stream);

/* In-place YaRN RoPE (half-split rotation) on x [n_tok][n_heads][head_dim]
 * at positions pos[n_tok] (device int32, each in [0, n_pos)), with a table
 * from neon_rope_table. */
neon_status neon_rope_yarn(uint16_t* x, const int32_t* pos, int n_tok, int n_heads,
                           int head_dim, const float* table, int n_pos, void* stream);

/* Router: logits = x W^T + b (fp32, one canonical reduction order), top-k
 * over the logits (ties -> lower index), softmax over the k values.
 * idx [B][k] int32, score [B][k] fp32, logits [B][E] fp32 (required: the
 * top-k reads it back). */
neon_status neon_router_topk(const uint16_t* x, const uint16_t* W,
                             const uint16_t* b, int32_t* idx, float* score,
                             float* logits, int B, int E, int H, int k,
                             void* stream);

/* MoE block on normalised x [B][H]: router + top-k experts, each
 * gate_up (MXFP4 [E][2I][H], bias [E][2I]) -> SwiGLU-clamp -> down (MXFP4
 * [E][H][I], bias [E][H]), weighted sum.  out [B][H] bf16; if residual is
 * not NULL, out = bf16(residual + bf16(moe)).  idx/score may be NULL.
 * workspace: at least neon_moe_layer_workspace(B, E, I, k) bytes (expert
 * activations, router logits, arrival counters), any contents. */
size_t neon_moe_layer_workspace(int B, int E, int I, int k);
neon_status neon_moe_layer(const uint16_t* x, const uint16_t* router_w,
                           const uint16_t* router_b, const uint8_t* gu_codes,
                           const uint8_t* gu_scales, const uint16_t* gu_bias,
                           const uint8_t* dn_codes, const uint8_t* dn_scales,
                           const uint16_t* dn_bias, const uint16_t* residual,
                           uint16_t* out, int32_t* idx, float* score, int B,
                           int E, int H, int I, int k, float alpha,
                           float limit, void* workspace, size_t workspace_bytes,
                           void* stream);

/* neon_moe_layer for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * the same arguments without the workspace, bit-identical results; its
 * scratch (expert activations and router logits) lives in a fixed 4 MiB
 * device array per GPU
 * that the library holds until the process ends, and it calls no allocator.
 * Shapes needing more than 4 MiB (B*k*I*2 rounded up to 256 plus B*E*4 bytes)
 * are rejected with NEON_EINVAL.  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams or threads) race.  No
 * counterpart in the reference, which has no model code; it exists for
 * callers that cannot allocate. */
neon_status neon_moe_layer_noalloc(const uint16_t* x, const uint16_t* router_w,
                                   const uint16_t* router_b, const uint8_t* gu_codes,
                                   const uint8_t* gu_scales, const uint16_t* gu_bias,
                                   const uint8_t* dn_codes, const uint8_t* dn_scales,
                                   const uint16_t* dn_bias, const uint16_t* residual,
                                   uint16_t* out, int32_t* idx, float* score, int B,
                                   int E, int H, int I, int k, float alpha,
                                   float limit, void* stream);

/* Grouped expert FFN alone (HF GptOssExperts): for each row b and slot s,
 * expert e = idx[b][s]: gate_up GEMV -> SwiGLU-clamp -> down GEMV, weighted
 * by score[b][s] and summed over the k slots; out as in neon_moe_layer.
 * act is caller-provided scratch of B*k*I bf16 (no allocation here).  An id
 * outside [0, E) drops its slot; neon_device_check then returns NEON_EINVAL. */
neon_status neon_moe_experts(const uint16_t* x, const int32_t* idx,
                             const float* score, const uint8_t* gu_codes,
                             const uint8_t* gu_scales, const uint16_t* gu_bias,
                             const uint8_t* dn_codes, const uint8_t* dn_scales,
                             const uint16_t* dn_bias, const uint16_t* residual,
                             uint16_t* out, uint16_t* act, int B, int E, int H,
                             int I, int k, float alpha, float limit,
                             void* stream);

/* GQA decode attention with per-head sinks.  q [B][Hq][D] (already rotated),
 * caches [B][Hkv][T_max][D], sinks [Hq] bf16, pos [B] device int32 (the
 * current token's position: keys 0..pos, or the last `window` of them when
 * window > 0).  out [B][Hq*D] bf16.  D == 64.
 * Spans of more than 256 keys are split (one split per 64-key chunk, at
 * most 32) and the splits are merged inside the launch:
 *   workspace  the split partials, neon_attn_decode_workspace(...) bytes
 *              (0, and workspace may be NULL, with one split), any contents;
 *   counters   the arrival counters, neon_attn_decode_counters(B, Hkv)
 *              bytes, zero-filled by the caller before their first use;
 *              every call leaves them zero, so one array serves every later
 *              call whose (B, Hkv) fits. */
size_t neon_attn_decode_workspace(int B, int Hq, int Hkv, int D, int T_max, int window);
size_t neon_attn_decode_counters(int B, int Hkv);
neon_status neon_attn_decode(const uint16_t* q, const uint16_t* k_cache,
                             const uint16_t* v_cache, const uint16_t* sinks,
                             const int32_t* pos, uint16_t* out, int B, int Hq,
                             int Hkv, int D, int T_max, int window, float* workspace,
                             size_t workspace_bytes, int32_t* counters,
                             size_t counter_bytes, void* stream);

/* One draw per row from logits [B][V] (device fp32), as neon_set_sampling
 * describes; pos [B] (device int32) keys the RNG; out_ids [B] device int32.
 * temperature > 0, top_p in (0, 1].  workspace: neon_sample_workspace(B, V)
 * bytes (the exponentials), any contents. */
size_t neon_sample_workspace(int B, int V);
neon_status neon_sample(const float* logits, int B, int V, float temperature, float top_p,
                        uint64_t seed, const int32_t* pos, int32_t* out_ids, float* workspace,
                        size_t workspace_bytes, void* stream);

/* ---- prefill kernels (matrix cores; fp32 accumulate in the MFMA order) --- */

/* C[M][N] = bf16(A[M][K] W[N][K]^T + bias) (accumulate = 0), or
 * C = bf16(C + bf16(A W^T + bias)) (accumulate = 1, C holds the residual).
 * bias may be NULL.  K % 32 == 0.  Used for the prompt-row projections. */
neon_status neon_gemm_bf16(const uint16_t* A, const uint16_t* W,
                           const uint16_t* bias, uint16_t* C, int M, int N,
                           int K, int accumulate, void* stream);

/* Expert FFN over M prompt rows: for each row t and slot s, expert
 * idx[t][s] (device int32 in [0, E)) applies gate_up -> SwiGLU-clamp -> down
 * to x[t] (normalised, bf16 [M][H]); h[t] = bf16(h[t] + bf16(sum_s
 * score[t][s] y_ts)) in place.  Rows are grouped by expert into MXFP4
 * matrix-core GEMMs (weights dequantised exactly to bf16).  An id outside
 * [0, E) drops its slot; neon_device_check then returns NEON_EINVAL.
 * workspace: neon_moe_prefill_workspace(M, E, H, I, k, 0) bytes (mx8 = 1 for
 * neon_moe_prefill_mx8), any contents. */
size_t neon_moe_prefill_workspace(int M, int E, int H, int I, int k, int mx8);
neon_status neon_moe_prefill(const uint16_t* x, const int32_t* idx,
                             const float* score, const uint8_t* gu_codes,
                             const uint8_t* gu_scales, const uint16_t* gu_bias,
                             const uint8_t* dn_codes, const uint8_t* dn_scales,
                             const uint16_t* dn_bias, uint16_t* h, int M, int E,
                             int H, int I, int k, float alpha, float limit,
                             void* workspace, size_t workspace_bytes, void* stream);

/* neon_moe_prefill with both expert GEMMs on the scaled fp8 x fp4 matrix
 * instruction (v_mfma_scale_f32_32x32x64_f8f6f4): the GEMM inputs (x, then
 * the SwiGLU output) become two MXFP8 terms per 32-element block
 * (neon_mx8_quant), the MXFP4 expert rows are read as stored.  H and I
 * multiples of 64.  Used by NEON_PREFILL_MX8.  (No counterpart in the
 * reference.) */
neon_status neon_moe_prefill_mx8(const uint16_t* x, const int32_t* idx,
                                 const float* score, const uint8_t* gu_codes,
                                 const uint8_t* gu_scales, const uint16_t* gu_bias,
                                 const uint8_t* dn_codes, const uint8_t* dn_scales,
                                 const uint16_t* dn_bias, uint16_t* h, int M, int E,
                                 int H, int I, int k, float alpha, float limit,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* The two-term MXFP8 image of bf16 rows x [rows][K] (K % 32 == 0): for each
 * 32-element block, hi = E4M3(x / 2^e1) rounded to nearest even, with
 * e1 = floor(log2 amax) - 8, plus one when amax's significand exceeds 1.75
 * (so no element passes 448), and scale byte s_hi = e1 + 127; lo = the same
 * rule on the exact residual x - hi 2^e1.  hi + lo is within
 * 2^(floor(log2 amax) - 8) of every finite element.
 * hi, lo [rows][K]; s_hi, s_lo [rows][K/32].  A zero block gets scale 127
 * and zero codes; a non-finite element gets the NaN code 0x7F in hi and 0
 * in lo.  (OCP MX v1.0; no counterpart in the reference.) */
neon_status neon_mx8_quant(const uint16_t* x, int64_t rows, int K, uint8_t* hi,
                           uint8_t* lo, uint8_t* s_hi, uint8_t* s_lo, void* stream);

/* Causal sink attention over a prompt: q [M][Hq][D] (rotated) at positions
 * 0 .. M-1, caches [Hkv][T_max][D] holding keys/values 0 .. M-1; row t sees
 * keys 0..t (the last `window` of them when window > 0).  out [M][Hq*D]. */
neon_status neon_attn_prefill(const uint16_t* q, const uint16_t* k_cache,
                              const uint16_t* v_cache, const uint16_t* sinks,
                              uint16_t* out, int M, int Hq, int Hkv, int D,
                              int T_max, int window, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* NEON_GPTOSS_H */

/*
 * neon_oracle.h -- CPU oracle for the gpt-oss token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product (neonengine_amd/) never links,
 * loads or calls it.
 *
 * The reference repository (NeonEngine, a Vulkan graphics engine) contains no
 * implementation of this path, so nothing here follows a reference file.  The
 * arithmetic restates the published model maths:
 *   - OCP Microscaling Formats (MX) v1.0: E2M1 element, E8M0 shared scale,
 *     32-element blocks;
 *   - the gpt-oss semantics as written in HuggingFace transformers 5.15.0
 *     (read as text): modeling_gpt_oss.py (HFM), configuration_gpt_oss.py
 *     (HFC), integrations/mxfp4.py (HFX), modeling_rope_utils.py (HFR).
 * Each function cites the HF lines it follows.
 *
 * Pinning (what checks each function, besides the GPU):
 *   or_mxfp4_dequant  exhaustive 16 x 256 (code, scale) table vs the closed
 *                     form; torch.float8_e8m0fnu scale decode.
 *   or_e4m3_*         all 256 codes vs torch.float8_e4m3fn decode; encode of
 *                     every bf16 value of magnitude <= 448 vs torch's
 *                     round-to-nearest-even cast; clamp above 448.
 *   or_mx8_quant      scale rule vs the OCP closed form; reconstruction
 *                     error bound (<= one bf16 unit of the block maximum).
 *   or_gemv_*         fp64 brute force within the fp32 accumulation bound.
 *   or_rmsnorm        constant-vector closed form; HF GptOssRMSNorm fixtures.
 *   or_yarn_*         HF _compute_yarn_parameters fixtures; position-0 and
 *                     norm-preservation invariants.
 *   or_router         brute-force sort; HF GptOssTopKRouter fixtures.
 *   or_swiglu         closed-form special cases; HF GptOssExperts fixtures.
 *   or_attn_decode    fp64 naive softmax; sink = -inf reduces to plain SDPA;
 *                     T = 1 closed form; HF eager_attention_forward fixtures.
 *   or_model_*        composition of the above; HF GptOssForCausalLM fixture
 *                     on a tiny fp32 config.
 *   or_c_*, or_expf   canonical fp32 forms that restate the device's exact
 *                     operation order; pinned against the fp64 functions
 *                     (fp32 error bounds) and or_expf against exp (ulps).
 *   or_router, or_swiglu and or_moe_layer use the canonical forms.
 */
#ifndef NEON_ORACLE_H
#define NEON_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same field order and meaning as neon_config in include/neon_gptoss.h. */
typedef struct or_config {
  int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim;
  int32_t n_experts, top_k, intermediate, vocab;
  int32_t sliding_window, max_seq, max_batch;
  float rope_theta, rope_factor, rope_beta_fast, rope_beta_slow;
  int32_t rope_orig_max_pos;
  float rms_eps, swiglu_limit, swiglu_alpha;
} or_config;

/* ---- deterministic counter-based RNG (bit-identical to the device init) -- */
uint64_t or_hash(uint64_t seed, uint64_t stream, uint64_t i);
float or_gauss_mul(double std);
void or_fill_bf16(uint64_t seed, uint64_t stream, int64_t n, float mean,
                  double std, uint16_t* out);
void or_fill_bytes(uint64_t seed, uint64_t stream, int64_t n, uint8_t* out);
void or_fill_scales(uint64_t seed, uint64_t stream, int64_t n, int lo,
                    int range, uint8_t* out);
/* elements [start, start + n) of the same streams (start % 8 == 0 for bytes) */
void or_fill_bytes_at(uint64_t seed, uint64_t stream, int64_t start, int64_t n,
                      uint8_t* out);
void or_fill_scales_at(uint64_t seed, uint64_t stream, int64_t start, int64_t n,
                       int lo, int range, uint8_t* out);

/* ---- numeric helpers ------------------------------------------------------ */
float or_bf16_to_f32(uint16_t b);
uint16_t or_f32_to_bf16(float f);

/* ---- MXFP8 activations (E4M3 elements, E8M0 scales; OCP MX v1.0 sec. 5-6) --
 * For the opt-in matrix-core prompt mode whose expert GEMMs use the scaled
 * fp8 x fp4 matrix instruction.  A bf16 activation block of 32 is carried as
 * two MXFP8 terms, x ~= dec(hi) 2^(s_hi-127) + dec(lo) 2^(s_lo-127): hi is
 * the block quantised with the MX rule (shared exponent floor(log2 amax)
 * minus E4M3's emax 8, plus one when amax's significand exceeds 1.75 so that
 * no element passes 448; elements rounded to nearest even), lo is the same
 * rule applied to the exact residual x - hi.  Every finite element comes
 * back to within 2^(floor(log2 amax) - 8).  Blocks of zeros get scale byte
 * 127 and zero codes; a non-finite element becomes the E4M3 NaN code 0x7F in
 * hi and 0 in lo and is left out of the block maxima. */
float or_e4m3_decode(uint8_t code);
uint8_t or_e4m3_encode(float v);
int or_ilog2f(float a); /* floor(log2 a) for finite a > 0, subnormals included */
void or_mx8_quant(const uint16_t* x, int64_t rows, int K, uint8_t* hi,
                  uint8_t* lo, uint8_t* s_hi, uint8_t* s_lo);

/* ---- MXFP4 --------------------------------------------------------------- */
void or_mxfp4_dequant(const uint8_t* codes, const uint8_t* scales,
                      int64_t n_blocks, float* out);
void or_mxfp4_gemv(const uint8_t* codes, const uint8_t* scales,
                   const uint16_t* bias, const uint16_t* x, int B, int N, int K,
                   uint16_t* y, float* y_f32);
void or_gemv_bf16(const uint16_t* W, const uint16_t* bias, const uint16_t* x,
                  int B, int N, int K, uint16_t* y, float* y_f32);

/* ---- elementwise / small ops ---------------------------------------------- */
void or_rmsnorm(const uint16_t* x, const uint16_t* w, int B, int H, float eps,
                uint16_t* out);
void or_yarn_inv_freq(const or_config* cfg, double* inv_freq,
                      double* attn_factor);
void or_rope_table(const or_config* cfg, int n_pos, float* cos_t, float* sin_t);
void or_rope_apply(const uint16_t* x, int n_heads, int D, const float* cos_row,
                   const float* sin_row, uint16_t* out);
void or_router(const uint16_t* x, const uint16_t* W, const uint16_t* b, int B,
               int E, int H, int k, int32_t* idx, float* score, float* logits);
void or_swiglu(const float* gate_up, int I, float alpha, float limit,
               float* out);
void or_moe_layer(const uint16_t* x, const uint16_t* router_w,
                  const uint16_t* router_b, const uint8_t* gu_codes,
                  const uint8_t* gu_scales, const uint16_t* gu_bias,
                  const uint8_t* dn_codes, const uint8_t* dn_scales,
                  const uint16_t* dn_bias, int B, int E, int H, int I, int k,
                  float alpha, float limit, uint16_t* out, int32_t* idx,
                  float* score);
/* experts with given ids [B][k] and weights; ids outside [0, E) are dropped */
void or_moe_experts(const uint16_t* x, const int32_t* idx, const float* score,
                    const uint8_t* gu_codes, const uint8_t* gu_scales,
                    const uint16_t* gu_bias, const uint8_t* dn_codes,
                    const uint8_t* dn_scales, const uint16_t* dn_bias, int B, int E,
                    int H, int I, int k, float alpha, float limit, uint16_t* out);
void or_attn_decode(const uint16_t* q, const uint16_t* k_cache,
                    const uint16_t* v_cache, const uint16_t* sinks, int B,
                    int Hq, int Hkv, int D, int T_max, const int32_t* pos,
                    int window, uint16_t* out, float* out_f32);

/* ---- canonical fp32 forms (bit-identical to the device kernels) ----------- */
float or_expf(float x);
void or_c_gemv_bf16(const uint16_t* W, const uint16_t* bias, const uint16_t* x,
                    int B, int N, int K, uint16_t* y, float* y_f32);
void or_c_mxfp4_gemv(const uint8_t* codes, const uint8_t* scales,
                     const uint16_t* bias, const uint16_t* x, int B, int N,
                     int K, uint16_t* y, float* y_f32);
void or_c_rmsnorm(const uint16_t* x, const uint16_t* w, int B, int H, float eps,
                  uint16_t* out);
/* scalar statements of or_c_gemv_bf16 / or_c_mxfp4_gemv (one fmaf at a time
 * per lane); the functions above compute the same bits with AVX2 over the
 * 64 lanes */
void or_c_gemv_bf16_ref(const uint16_t* W, const uint16_t* bias, const uint16_t* x,
                        int B, int N, int K, uint16_t* y, float* y_f32);
void or_c_mxfp4_gemv_ref(const uint8_t* codes, const uint8_t* scales,
                         const uint16_t* bias, const uint16_t* x, int B, int N,
                         int K, uint16_t* y, float* y_f32);
int or_attn_splits(int T_max, int window);
void or_c_attn_decode(const uint16_t* q, const uint16_t* k_cache,
                      const uint16_t* v_cache, const uint16_t* sinks, int B,
                      int Hq, int Hkv, int D, int T_max, const int32_t* pos,
                      int window, int S, uint16_t* out, float* out_f32);

/* Temperature + nucleus sampling in the device's exact operation order
 * (neon_sample): ids [B] from logits [B][V] at positions pos [B]. */
void or_sample(const float* logits, int B, int V, float temperature, float top_p,
               uint64_t seed, const int32_t* pos, int32_t* out_ids);

/* ---- full model (random init, identical to neon_init_random) -------------- */
typedef struct or_model or_model;
or_model* or_model_create(const or_config* cfg, uint64_t seed, int batch);
/* flags: OR_LAZY_EXPERTS keeps no MXFP4 expert codes/scales in memory and
 * regenerates the chosen experts' slices each step (same bits; for the
 * 120b shape, whose experts exceed host memory).  or_model_tensor returns
 * NULL for those tensors then. */
enum { OR_LAZY_EXPERTS = 1 };
or_model* or_model_create_ex(const or_config* cfg, uint64_t seed, int batch, int flags);
/* Synthetic KV history (N(0,1) keys and values at positions 0 .. n_pos-1 of
 * every layer and sequence; positions set to n_pos).  Timing only. */
void or_model_fill_kv(or_model* m, int n_pos, uint64_t seed);
/* Overwrites one weight tensor (layer -1 for embed / lm_head / final norm);
 * bytes must equal its size.  Returns 0, or -1 on a bad kind or size. */
int or_model_set_tensor(or_model* m, int layer, int kind, const void* data, size_t bytes);
/* Accumulation of the model functions: 0 = canonical fp32 orders (default,
 * bit-identical to the device), 1 = fp64 accumulation rounded once.  Mode 1
 * measures how far a change of summation order alone moves the outputs. */
void or_set_accumulation(int mode);
void or_model_free(or_model* m);
/* One decode step for every sequence: consumes ids[b] at position pos[b],
 * writes logits (fp32 [B][V], may be NULL) and greedy ids (may be NULL).
 * With both NULL the step is a teacher-forced prompt row: the KV cache and
 * positions advance and lm_head is skipped. */
void or_model_step(or_model* m, const int32_t* ids, float* logits,
                   int32_t* out_ids);
/* Teacher-forced prompt rows, layer-major: sequence b consumes ids[b][0..n-1]
 * (ids [B][n]) at positions pos[b] .. pos[b] + n - 1.  Bit-identical to n
 * or_model_step calls with NULL outputs; each weight row is read once per
 * layer for all B n rows, and a lazy model generates each layer's experts
 * once. */
void or_model_prompt(or_model* m, const int32_t* ids, int n);
/* hidden state (bf16 [B][H]) after the last completed step, before the final
 * norm; for tests. */
const uint16_t* or_model_hidden(const or_model* m);
int32_t or_model_pos(const or_model* m, int b);
/* Tensor access for tests: returns a pointer into the model's weights. */
const void* or_model_tensor(const or_model* m, int layer, int kind);
int or_num_threads(void);
/* Last step's last-layer activations of batch row 0 (tests): 0 qkv (bf16),
 * 1 attention output (bf16), 2 MoE input (bf16), 3 expert ids (int32),
 * 4 routing weights (fp32). */
const void* or_model_trace(const or_model* m, int what);

/* tensor kinds (shared with the product's init streams) */
enum {
  OR_T_ATTN_NORM = 0, OR_T_WQKV = 1, OR_T_BQKV = 2, OR_T_WO = 3, OR_T_BO = 4,
  OR_T_SINKS = 5, OR_T_MLP_NORM = 6, OR_T_ROUTER_W = 7, OR_T_ROUTER_B = 8,
  OR_T_GU_CODES = 9, OR_T_GU_SCALES = 10, OR_T_GU_BIAS = 11,
  OR_T_DN_CODES = 12, OR_T_DN_SCALES = 13, OR_T_DN_BIAS = 14,
  OR_T_EMBED = 100, OR_T_LM_HEAD = 101, OR_T_FINAL_NORM = 102
};
uint64_t or_stream_id(int layer, int kind);

#ifdef __cplusplus
}
#endif
#endif

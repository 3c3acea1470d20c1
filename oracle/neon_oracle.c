/*
 * neon_oracle.c -- CPU restatement of the gpt-oss token loop (test oracle).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, never by the product.  See neon_oracle.h for
 * what pins each function.
 *
 * Build: oracle/Makefile (gcc -O3 -march=native -fopenmp -ffp-contract=off).
 * -ffp-contract=off matters: the RNG's float step and the router's canonical
 * fp32 reduction must round exactly like the device code.
 *
 * Semantic sources (third-party text, not the reference; the reference has no
 * implementation of this path):
 *   HFM = transformers/models/gpt_oss/modeling_gpt_oss.py
 *   HFC = transformers/models/gpt_oss/configuration_gpt_oss.py
 *   HFX = transformers/integrations/mxfp4.py
 *   HFR = transformers/modeling_rope_utils.py
 */
#include "neon_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* numeric helpers                                                           */
/* ------------------------------------------------------------------------ */
float or_bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* round-to-nearest-even fp32 -> bf16; NaN stays NaN (quiet). */
uint16_t or_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

#define BF(x) or_bf16_to_f32(x)
#define TOBF(x) or_f32_to_bf16(x)

/* ------------------------------------------------------------------------ */
/* RNG: SplitMix64 finaliser (Steele, Lea, Flood 2014) keyed by             */
/* (seed, stream, index).  Gaussian-shaped values are Irwin-Hall sums of     */
/* four 16-bit uniforms scaled by one fp32 multiply, so the device init and  */
/* this oracle produce bit-identical tensors.                                */
/* ------------------------------------------------------------------------ */
static inline uint64_t mix64(uint64_t z) {
  z ^= z >> 30;
  z *= 0xBF58476D1CE4E5B9ull;
  z ^= z >> 27;
  z *= 0x94D049BB133111EBull;
  z ^= z >> 31;
  return z;
}

static inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
  return mix64(seed + stream * 0x9E3779B97F4A7C15ull);
}

static inline uint64_t hash_k(uint64_t key, uint64_t i) {
  return mix64(key ^ (i * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull));
}

uint64_t or_hash(uint64_t seed, uint64_t stream, uint64_t i) {
  return hash_k(stream_key(seed, stream), i);
}

static inline int32_t gauss_int(uint64_t h) {
  return (int32_t)((h & 0xFFFF) + ((h >> 16) & 0xFFFF) + ((h >> 32) & 0xFFFF) +
                   (h >> 48)) -
         131070;
}

/* multiplier that turns gauss_int (std sqrt((2^32-1)/3)) into std `std` */
float or_gauss_mul(double std) {
  const double unit = sqrt((65536.0 * 65536.0 - 1.0) / 3.0);
  return (float)(std / unit);
}

void or_fill_bf16(uint64_t seed, uint64_t stream, int64_t n, float mean,
                  double std, uint16_t* out) {
  const uint64_t key = stream_key(seed, stream);
  const float mul = or_gauss_mul(std);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    float g = (float)gauss_int(hash_k(key, (uint64_t)i)) * mul;
    out[i] = TOBF(mean + g);
  }
}

void or_fill_bytes(uint64_t seed, uint64_t stream, int64_t n, uint8_t* out) {
  const uint64_t key = stream_key(seed, stream);
#pragma omp parallel for schedule(static)
  for (int64_t w = 0; w < (n + 7) / 8; ++w) {
    uint64_t h = hash_k(key, (uint64_t)w);
    for (int j = 0; j < 8 && w * 8 + j < n; ++j)
      out[w * 8 + j] = (uint8_t)(h >> (8 * j));
  }
}

void or_fill_scales(uint64_t seed, uint64_t stream, int64_t n, int lo,
                    int range, uint8_t* out) {
  const uint64_t key = stream_key(seed, stream);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    uint64_t h = hash_k(key, (uint64_t)i);
    out[i] = (uint8_t)(lo + (int)(((h >> 32) * (uint64_t)range) >> 32));
  }
}

/* Elements [start, start + n) of the or_fill_bytes / or_fill_scales streams
 * (start of a byte range must be a multiple of 8: one hash word fills 8
 * bytes).  Lets the oracle regenerate one expert's slice of a stacked expert
 * tensor without materialising the whole tensor. */
void or_fill_bytes_at(uint64_t seed, uint64_t stream, int64_t start, int64_t n,
                      uint8_t* out) {
  const uint64_t key = stream_key(seed, stream);
  const int64_t w0 = start / 8;
#pragma omp parallel for schedule(static)
  for (int64_t w = 0; w < (n + 7) / 8; ++w) {
    uint64_t h = hash_k(key, (uint64_t)(w0 + w));
    for (int j = 0; j < 8 && w * 8 + j < n; ++j)
      out[w * 8 + j] = (uint8_t)(h >> (8 * j));
  }
}

void or_fill_scales_at(uint64_t seed, uint64_t stream, int64_t start, int64_t n,
                       int lo, int range, uint8_t* out) {
  const uint64_t key = stream_key(seed, stream);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    uint64_t h = hash_k(key, (uint64_t)(start + i));
    out[i] = (uint8_t)(lo + (int)(((h >> 32) * (uint64_t)range) >> 32));
  }
}

uint64_t or_stream_id(int layer, int kind) {
  return ((uint64_t)(layer + 1) << 16) | (uint64_t)kind;
}

/* ------------------------------------------------------------------------ */
/* MXFP4 (OCP MX v1.0; HFX:29-46 LUT, HFX:271 bias 127, HFX:298-304 nibble   */
/* order: low nibble = element 2i, high nibble = element 2i+1).              */
/* ------------------------------------------------------------------------ */
static const float kE2M1[16] = {+0.0f, +0.5f, +1.0f, +1.5f, +2.0f, +3.0f,
                                +4.0f, +6.0f, -0.0f, -0.5f, -1.0f, -1.5f,
                                -2.0f, -3.0f, -4.0f, -6.0f};

static inline float e8m0_exp2(uint8_t s, float v) {
  if (s == 0xFF) return NAN; /* E8M0 0xFF encodes NaN */
  return ldexpf(v, (int)s - 127);
}

/* ---- MXFP8 (E4M3) activations: OCP MX v1.0 sec. 5.3 (E4M3: bias 7, no
 * infinities, S.1111.111 = NaN, max normal 448) and sec. 6.3 (shared
 * exponent from floor(log2(amax)) - emax_elem, emax_elem = 8 for E4M3; the
 * clamp of out-of-range magnitudes to the largest normal, here only a guard
 * since the exponent is chosen so that no finite element exceeds 448). ---- */
float or_e4m3_decode(uint8_t code) {
  const int e = (code >> 3) & 15, m = code & 7;
  const float sgn = (code & 0x80) ? -1.0f : 1.0f;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) return sgn * ldexpf((float)m, -9);
  return sgn * ldexpf((float)(8 + m), e - 10);
}

int or_ilog2f(float a) {
  uint32_t b;
  memcpy(&b, &a, 4);
  const int ef = (b >> 23) & 255;
  if (ef) return ef - 127;
  const uint32_t m = b & 0x7FFFFFu;
  return (31 - __builtin_clz(m)) - 149;
}

uint8_t or_e4m3_encode(float v) {
  if (isnan(v)) return 0x7F;
  const uint8_t sgn = signbit(v) ? 0x80 : 0;
  const float a = fabsf(v);
  if (a >= 448.0f) return sgn | 0x7E;
  if (a < 0.015625f) return sgn | (uint8_t)(int)rintf(a * 512.0f); /* step 2^-9; 8 = 2^-6 */
  int e = or_ilog2f(a);
  int q = (int)rintf((ldexpf(a, -e) - 1.0f) * 8.0f);
  if (q == 8) { e += 1; q = 0; }
  return sgn | (uint8_t)(((e + 7) << 3) | q);
}

/* The smallest shared exponent at which the block maximum is representable:
 * floor(log2 amax) - 8 (OCP's rule, E4M3 emax 8), one more when amax's
 * significand exceeds 1.75 (amax / 2^(floor - 8) would pass 448, the largest
 * E4M3 normal, and OCP's rule would clamp it). */
static uint8_t mx8_scale_byte(float amax) {
  if (!(amax > 0.0f)) return 127;
  int e = or_ilog2f(amax);
  if (ldexpf(amax, -e) > 1.75f) e += 1;
  e = e - 8 + 127;
  return (uint8_t)(e < 0 ? 0 : (e > 254 ? 254 : e));
}

void or_mx8_quant(const uint16_t* x, int64_t rows, int K, uint8_t* hi,
                  uint8_t* lo, uint8_t* s_hi, uint8_t* s_lo) {
  const int nb = K / 32;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int blk = 0; blk < nb; ++blk) {
      const int64_t o = r * K + (int64_t)blk * 32;
      float v[32], res[32], amax = 0.0f, rmax = 0.0f;
      for (int j = 0; j < 32; ++j) {
        v[j] = or_bf16_to_f32(x[o + j]);
        if (isfinite(v[j]) && fabsf(v[j]) > amax) amax = fabsf(v[j]);
      }
      const uint8_t b1 = mx8_scale_byte(amax);
      for (int j = 0; j < 32; ++j) {
        if (!isfinite(v[j])) { hi[o + j] = 0x7F; res[j] = 0.0f; continue; }
        hi[o + j] = or_e4m3_encode(ldexpf(v[j], 127 - (int)b1));
        res[j] = v[j] - ldexpf(or_e4m3_decode(hi[o + j]), (int)b1 - 127);
        if (fabsf(res[j]) > rmax) rmax = fabsf(res[j]);
      }
      const uint8_t b2 = mx8_scale_byte(rmax);
      for (int j = 0; j < 32; ++j) lo[o + j] = or_e4m3_encode(ldexpf(res[j], 127 - (int)b2));
      s_hi[r * nb + blk] = b1;
      s_lo[r * nb + blk] = b2;
    }
  }
}

void or_mxfp4_dequant(const uint8_t* codes, const uint8_t* scales,
                      int64_t n_blocks, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < n_blocks; ++b) {
    for (int j = 0; j < 16; ++j) {
      uint8_t byte = codes[b * 16 + j];
      out[b * 32 + 2 * j] = e8m0_exp2(scales[b], kE2M1[byte & 0xF]);
      out[b * 32 + 2 * j + 1] = e8m0_exp2(scales[b], kE2M1[byte >> 4]);
    }
  }
}

/* y[b][n] = sum_k dq(W[n][k]) x[b][k] (+ bias[n]).  W is [N][K] with the 32-
 * blocks along K (HF *_blocks [N][K/32][16], *_scales [N][K/32]).  Products
 * of an E2M1 value and a bf16 are exact; the block sum and the row sum are
 * accumulated in fp64, the result rounded once to fp32 (y_f32) and once to
 * bf16 (y). */
void or_mxfp4_gemv(const uint8_t* codes, const uint8_t* scales,
                   const uint16_t* bias, const uint16_t* x, int B, int N, int K,
                   uint16_t* y, float* y_f32) {
  const int KB = K / 32;
  float* xf = (float*)malloc(sizeof(float) * (size_t)B * K);
  for (int64_t i = 0; i < (int64_t)B * K; ++i) xf[i] = BF(x[i]);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    const uint8_t* crow = codes + (size_t)n * (K / 2);
    const uint8_t* srow = scales + (size_t)n * KB;
    for (int b = 0; b < B; ++b) {
      const float* xb = xf + (size_t)b * K;
      double acc = 0.0;
      for (int kb = 0; kb < KB; ++kb) {
        double part = 0.0;
        for (int j = 0; j < 16; ++j) {
          uint8_t byte = crow[kb * 16 + j];
          part += (double)kE2M1[byte & 0xF] * xb[kb * 32 + 2 * j];
          part += (double)kE2M1[byte >> 4] * xb[kb * 32 + 2 * j + 1];
        }
        acc += part * ldexp(1.0, (int)srow[kb] - 127);
      }
      if (bias) acc += (double)BF(bias[n]);
      float r = (float)acc;
      if (y_f32) y_f32[(size_t)b * N + n] = r;
      if (y) y[(size_t)b * N + n] = TOBF(r);
    }
  }
  free(xf);
}

/* y[b][n] = sum_k W[n][k] x[b][k] (+ bias[n]), bf16 W [N][K] (nn.Linear). */
void or_gemv_bf16(const uint16_t* W, const uint16_t* bias, const uint16_t* x,
                  int B, int N, int K, uint16_t* y, float* y_f32) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)B * K);
  for (int64_t i = 0; i < (int64_t)B * K; ++i) xf[i] = BF(x[i]);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    const uint16_t* wr = W + (size_t)n * K;
    for (int b = 0; b < B; ++b) {
      const float* xb = xf + (size_t)b * K;
      double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      int k = 0;
      for (; k + 8 <= K; k += 8)
        for (int j = 0; j < 8; ++j) acc[j] += (double)BF(wr[k + j]) * xb[k + j];
      for (; k < K; ++k) acc[0] += (double)BF(wr[k]) * xb[k];
      double s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) +
                 ((acc[4] + acc[5]) + (acc[6] + acc[7]));
      if (bias) s += (double)BF(bias[n]);
      float r = (float)s;
      if (y_f32) y_f32[(size_t)b * N + n] = r;
      if (y) y[(size_t)b * N + n] = TOBF(r);
    }
  }
  free(xf);
}

/* ------------------------------------------------------------------------ */
/* RMSNorm (HFM:57-62): fp32 x * rsqrt(mean(x^2) + eps), times the weight in  */
/* fp32, one rounding to bf16.                                               */
/* ------------------------------------------------------------------------ */
void or_rmsnorm(const uint16_t* x, const uint16_t* w, int B, int H, float eps,
                uint16_t* out) {
  for (int b = 0; b < B; ++b) {
    const uint16_t* xb = x + (size_t)b * H;
    double ss = 0.0;
    for (int i = 0; i < H; ++i) ss += (double)BF(xb[i]) * BF(xb[i]);
    float var = (float)(ss / H);
    float r = 1.0f / sqrtf(var + eps);
    for (int i = 0; i < H; ++i)
      out[(size_t)b * H + i] = TOBF(BF(w[i]) * (BF(xb[i]) * r));
  }
}

/* ------------------------------------------------------------------------ */
/* YaRN RoPE (HFR:429-483; gpt-oss parameters HFC:29,80-88: theta 150000,   */
/* factor 32, beta_fast 32, beta_slow 1, original_max 4096, truncate False). */
/* ------------------------------------------------------------------------ */
static double corr_dim(double nrot, double dim, double base, double maxpos) {
  return (dim * log(maxpos / (nrot * 2.0 * M_PI))) / (2.0 * log(base));
}

void or_yarn_inv_freq(const or_config* cfg, double* inv_freq,
                      double* attn_factor) {
  const int dim = cfg->head_dim;
  const double base = cfg->rope_theta, factor = cfg->rope_factor;
  double low = corr_dim(cfg->rope_beta_fast, dim, base, cfg->rope_orig_max_pos);
  double high =
      corr_dim(cfg->rope_beta_slow, dim, base, cfg->rope_orig_max_pos);
  if (low < 0) low = 0;               /* truncate=False: no floor/ceil */
  if (high > dim - 1) high = dim - 1;
  if (low == high) high += 0.001;
  for (int i = 0; i < dim / 2; ++i) {
    double pos_freq = pow(base, (2.0 * i) / dim);
    double extra = 1.0 / pos_freq, inter = 1.0 / (factor * pos_freq);
    double ramp = (i - low) / (high - low);
    if (ramp < 0) ramp = 0;
    if (ramp > 1) ramp = 1;
    double ef = 1.0 - ramp; /* inv_freq_extrapolation_factor */
    inv_freq[i] = inter * (1.0 - ef) + extra * ef;
  }
  *attn_factor = factor <= 1.0 ? 1.0 : 0.1 * log(factor) + 1.0;
}

/* cos/sin tables [n_pos][D/2] in fp32.  The angle is the fp32 product of
 * the fp32 inverse frequency and the position (as HFM:196-198 computes it);
 * cos/sin are then scaled by the YaRN attention factor in fp32. */
void or_rope_table(const or_config* cfg, int n_pos, float* cos_t,
                   float* sin_t) {
  const int half = cfg->head_dim / 2;
  double invf[256], af;
  or_yarn_inv_freq(cfg, invf, &af);
  const float aff = (float)af;
  for (int p = 0; p < n_pos; ++p)
    for (int i = 0; i < half; ++i) {
      float ang = (float)invf[i] * (float)p;
      cos_t[(size_t)p * half + i] = (float)cos((double)ang) * aff;
      sin_t[(size_t)p * half + i] = (float)sin((double)ang) * aff;
    }
}

/* half-split rotation (HFM:215-222): out1 = x1 c - x2 s, out2 = x2 c + x1 s */
void or_rope_apply(const uint16_t* x, int n_heads, int D, const float* c,
                   const float* s, uint16_t* out) {
  const int half = D / 2;
  for (int h = 0; h < n_heads; ++h)
    for (int i = 0; i < half; ++i) {
      float x1 = BF(x[h * D + i]), x2 = BF(x[h * D + half + i]);
      float o1 = x1 * c[i] - x2 * s[i];
      float o2 = x2 * c[i] + x1 * s[i];
      out[h * D + i] = TOBF(o1);
      out[h * D + half + i] = TOBF(o2);
    }
}

/* ------------------------------------------------------------------------ */
/* Canonical fp32 forms.  The device evaluates every reduction of the decode  */
/* path in one fixed order of IEEE fp32 operations (explicit fused multiply- */
/* adds, a 64-lane xor butterfly); the or_c_* functions restate that order   */
/* so GPU and oracle agree bit for bit.  Each is pinned against the fp64     */
/* functions above by the CPU tests (fp32 error bounds).                     */
/* ------------------------------------------------------------------------ */

/* exp: Cody-Waite reduction by a two-part ln 2 and a degree-7 Taylor       */
/* polynomial in Horner form (same operation sequence as the device).        */
float or_expf(float x) {
  if (x != x) return x;
  if (x > 0x1.62e43p+6f) return INFINITY;
  if (x < -0x1.9fe36ap+6f) return 0.0f;
  const float n = rintf(x * 0x1.715476p+0f);
  float r = fmaf(-n, 0x1.62e4p-1f, x);
  r = fmaf(-n, 0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = fmaf(p, r, 0x1.6c16c2p-10f);
  p = fmaf(p, r, 0x1.111112p-7f);
  p = fmaf(p, r, 0x1.555556p-5f);
  p = fmaf(p, r, 0x1.555556p-3f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

/* v[l] = v[l] + v[l ^ off] for off = 32, 16, 8, 4, 2, 1; result v[0] */
static float c_butterfly64(float* v) {
  for (int off = 32; off >= 1; off >>= 1) {
    float t[64];
    for (int l = 0; l < 64; ++l) t[l] = v[l] + v[l ^ off];
    memcpy(v, t, sizeof(t));
  }
  return v[0];
}

/* bf16 row . fp32 x: lane l owns the 8-element units u = l + 64 p. */
static float c_dot_bf16(const uint16_t* w, const float* x, int K) {
  const int U = K / 8;
  float a[64];
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int u = l; u < U; u += 64)
      for (int j = 0; j < 8; ++j) acc = fmaf(BF(w[u * 8 + j]), x[u * 8 + j], acc);
    a[l] = acc;
  }
  return c_butterfly64(a);
}

/* MXFP4 row . fp32 x: lane l owns the 32-element units u = l + 64 p; per unit
 * t = fmaf chain from 0, then acc = acc + t * 2^(s - 127) (0xFF: NaN). */
static float c_dot_fp4(const uint8_t* codes, const uint8_t* scales,
                       const float* x, int K) {
  const int U = K / 32;
  float a[64];
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int u = l; u < U; u += 64) {
      float t = 0.0f;
      for (int j = 0; j < 16; ++j) {
        const uint8_t byte = codes[u * 16 + j];
        t = fmaf(kE2M1[byte & 0xF], x[u * 32 + 2 * j], t);
        t = fmaf(kE2M1[byte >> 4], x[u * 32 + 2 * j + 1], t);
      }
      acc = acc + e8m0_exp2(scales[u], t);
    }
    a[l] = acc;
  }
  return c_butterfly64(a);
}

/* Scalar statements of the canonical GEMVs (the definitions; used by the
 * tests to check the vector forms below). */
void or_c_gemv_bf16_ref(const uint16_t* W, const uint16_t* bias, const uint16_t* x,
                        int B, int N, int K, uint16_t* y, float* y_f32) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)B * K);
  for (int64_t i = 0; i < (int64_t)B * K; ++i) xf[i] = BF(x[i]);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n)
    for (int b = 0; b < B; ++b) {
      float r = c_dot_bf16(W + (size_t)n * K, xf + (size_t)b * K, K);
      if (bias) r = r + BF(bias[n]);
      if (y_f32) y_f32[(size_t)b * N + n] = r;
      if (y) y[(size_t)b * N + n] = TOBF(r);
    }
  free(xf);
}

void or_c_mxfp4_gemv_ref(const uint8_t* codes, const uint8_t* scales,
                         const uint16_t* bias, const uint16_t* x, int B, int N,
                         int K, uint16_t* y, float* y_f32) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)B * K);
  for (int64_t i = 0; i < (int64_t)B * K; ++i) xf[i] = BF(x[i]);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n)
    for (int b = 0; b < B; ++b) {
      float r = c_dot_fp4(codes + (size_t)n * (K / 2), scales + (size_t)n * (K / 32),
                          xf + (size_t)b * K, K);
      if (bias) r = r + BF(bias[n]);
      if (y_f32) y_f32[(size_t)b * N + n] = r;
      if (y) y[(size_t)b * N + n] = TOBF(r);
    }
  free(xf);
}

/* Vector forms: the same per-lane operation sequence with the 64 lanes held
 * in eight 8-wide AVX2 registers.  Operands are transposed to lane-minor
 * order [pass][element][lane] (units past U are zero: fmaf(0, 0, acc) = acc
 * because acc, started at +0, is never -0), so each fmaf of the scalar form
 * becomes one lane of a vfmadd, and the butterfly keeps the scalar pairing
 * (fp32 addition is commutative, so l + (l ^ off) equals (l ^ off) + l). */
#include <immintrin.h>

static inline float butterfly_v8(__m256 a[8]) {
  __m256 t0 = _mm256_add_ps(a[0], a[4]), t1 = _mm256_add_ps(a[1], a[5]);  /* xor 32 */
  __m256 t2 = _mm256_add_ps(a[2], a[6]), t3 = _mm256_add_ps(a[3], a[7]);
  t0 = _mm256_add_ps(t0, t2); t1 = _mm256_add_ps(t1, t3);                 /* xor 16 */
  t0 = _mm256_add_ps(t0, t1);                                             /* xor 8 */
  __m128 lo = _mm256_castps256_ps128(t0), hi = _mm256_extractf128_ps(t0, 1);
  __m128 u = _mm_add_ps(lo, hi);                                          /* xor 4 */
  u = _mm_add_ps(u, _mm_movehl_ps(u, u));                                 /* xor 2 */
  u = _mm_add_ss(u, _mm_shuffle_ps(u, u, 1));                             /* xor 1 */
  return _mm_cvtss_f32(u);
}

/* x rows -> [B][P][E][64] fp32, E = elements per unit (8 bf16 / 32 fp4) */
static float* lane_major_x(const uint16_t* x, int B, int K, int E, int P) {
  const int U = K / E;
  float* xt = (float*)aligned_alloc(32, sizeof(float) * (size_t)B * P * E * 64);
  for (int b = 0; b < B; ++b)
    for (int p = 0; p < P; ++p)
      for (int e = 0; e < E; ++e)
        for (int l = 0; l < 64; ++l) {
          const int u = l + 64 * p;
          xt[(((size_t)b * P + p) * E + e) * 64 + l] =
              u < U ? BF(x[(size_t)b * K + (size_t)u * E + e]) : 0.0f;
        }
  return xt;
}

void or_c_gemv_bf16(const uint16_t* W, const uint16_t* bias, const uint16_t* x,
                    int B, int N, int K, uint16_t* y, float* y_f32) {
  /* one row: the transposition would cost more than it saves */
  if (B == 1) { or_c_gemv_bf16_ref(W, bias, x, B, N, K, y, y_f32); return; }
  const int U = K / 8, P = (U + 63) / 64;
  float* xt = lane_major_x(x, B, K, 8, P);
#pragma omp parallel
  {
    float* wt = (float*)aligned_alloc(32, sizeof(float) * (size_t)P * 8 * 64);
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      const uint16_t* w = W + (size_t)n * K;
      for (int p = 0; p < P; ++p)
        for (int l = 0; l < 64; ++l) {
          const int u = l + 64 * p;
          for (int e = 0; e < 8; ++e)
            wt[(p * 8 + e) * 64 + l] = u < U ? BF(w[u * 8 + e]) : 0.0f;
        }
      for (int b = 0; b < B; ++b) {
        const float* xb = xt + (size_t)b * P * 8 * 64;
        __m256 a[8];
        for (int v = 0; v < 8; ++v) a[v] = _mm256_setzero_ps();
        for (int pe = 0; pe < P * 8; ++pe)
          for (int v = 0; v < 8; ++v)
            a[v] = _mm256_fmadd_ps(_mm256_load_ps(wt + pe * 64 + 8 * v),
                                   _mm256_load_ps(xb + pe * 64 + 8 * v), a[v]);
        float r = butterfly_v8(a);
        if (bias) r = r + BF(bias[n]);
        if (y_f32) y_f32[(size_t)b * N + n] = r;
        if (y) y[(size_t)b * N + n] = TOBF(r);
      }
    }
    free(wt);
  }
  free(xt);
}

void or_c_mxfp4_gemv(const uint8_t* codes, const uint8_t* scales,
                     const uint16_t* bias, const uint16_t* x, int B, int N,
                     int K, uint16_t* y, float* y_f32) {
  if (B == 1) { or_c_mxfp4_gemv_ref(codes, scales, bias, x, B, N, K, y, y_f32); return; }
  const int U = K / 32, P = (U + 63) / 64;
  float* xt = lane_major_x(x, B, K, 32, P);
#pragma omp parallel
  {
    float* wt = (float*)aligned_alloc(32, sizeof(float) * (size_t)P * 32 * 64);
    float* sf = (float*)aligned_alloc(32, sizeof(float) * (size_t)P * 64);
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      const uint8_t* c = codes + (size_t)n * (K / 2);
      const uint8_t* s = scales + (size_t)n * U;
      for (int p = 0; p < P; ++p)
        for (int l = 0; l < 64; ++l) {
          const int u = l + 64 * p;
          for (int j = 0; j < 16; ++j) {
            const uint8_t byte = u < U ? c[u * 16 + j] : 0;
            wt[(p * 32 + 2 * j) * 64 + l] = kE2M1[byte & 0xF];
            wt[(p * 32 + 2 * j + 1) * 64 + l] = kE2M1[byte >> 4];
          }
          /* t * 2^(s-127) rounded once equals ldexpf(t, s - 127): every
           * 2^(s-127), s < 255, is an exact fp32 (2^-127 a subnormal) */
          sf[p * 64 + l] = u < U ? e8m0_exp2(s[u], 1.0f) : 1.0f;
        }
      for (int b = 0; b < B; ++b) {
        const float* xb = xt + (size_t)b * P * 32 * 64;
        __m256 a[8];
        for (int v = 0; v < 8; ++v) a[v] = _mm256_setzero_ps();
        for (int p = 0; p < P; ++p) {
          __m256 t[8];
          for (int v = 0; v < 8; ++v) t[v] = _mm256_setzero_ps();
          for (int e = 0; e < 32; ++e)
            for (int v = 0; v < 8; ++v)
              t[v] = _mm256_fmadd_ps(_mm256_load_ps(wt + (p * 32 + e) * 64 + 8 * v),
                                     _mm256_load_ps(xb + (p * 32 + e) * 64 + 8 * v), t[v]);
          for (int v = 0; v < 8; ++v)
            a[v] = _mm256_add_ps(a[v], _mm256_mul_ps(t[v], _mm256_load_ps(sf + p * 64 + 8 * v)));
        }
        float r = butterfly_v8(a);
        if (bias) r = r + BF(bias[n]);
        if (y_f32) y_f32[(size_t)b * N + n] = r;
        if (y) y[(size_t)b * N + n] = TOBF(r);
      }
    }
    free(wt);
    free(sf);
  }
  free(xt);
}

/* RMSNorm, canonical: ss by the 64-lane unit order and butterfly;
 * r = 1 / sqrt(ss / H + eps); y = bf16(w * (x * r)). */
void or_c_rmsnorm(const uint16_t* x, const uint16_t* w, int B, int H, float eps,
                  uint16_t* out) {
  const int U = H / 8;
  for (int b = 0; b < B; ++b) {
    const uint16_t* xb = x + (size_t)b * H;
    float a[64];
    for (int l = 0; l < 64; ++l) {
      float ss = 0.0f;
      for (int u = l; u < U; u += 64)
        for (int j = 0; j < 8; ++j) {
          const float v = BF(xb[u * 8 + j]);
          ss = fmaf(v, v, ss);
        }
      a[l] = ss;
    }
    const float ss = c_butterfly64(a);
    const float r = 1.0f / sqrtf(ss / (float)H + eps);
    for (int i = 0; i < H; ++i)
      out[(size_t)b * H + i] = TOBF(BF(w[i]) * (BF(xb[i]) * r));
  }
}

/* Split count of the device attention (attn_splits): spans of at most 4
 * chunks (256 keys) use one split, longer ones one split per chunk, max 32. */
int or_attn_splits(int T_max, int window) {
  const int span = window > 0 ? (window < T_max ? window : T_max) : T_max;
  const int s = (span + 63) / 64;
  return s <= 4 ? 1 : (s > 32 ? 32 : s);
}

/* Decode attention with sinks, canonical split form (device k_attn_split +
 * k_attn_merge):
 * 64-key chunks from lo, split s owns chunks [s nch / S, (s+1) nch / S);
 * online softmax per split with lane-local P.V accumulators (lane = key group
 * kg x dim octet dq), reduced over kg by xor 8, 16, 32; splits merged in
 * order with the sink.  D must be 64. */
void or_c_attn_decode(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                      const uint16_t* sinks, int B, int Hq, int Hkv, int D,
                      int T_max, const int32_t* pos, int window, int S,
                      uint16_t* out, float* out_f32) {
  const int G = Hq / Hkv;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      const int g = h / G, p = pos[b];
      const int lo = (window > 0 && p - window + 1 > 0) ? p - window + 1 : 0;
      const int n = p - lo + 1, nch = (n + 63) / 64;
      const size_t base = ((size_t)b * Hkv + g) * T_max;
      float qf[64];
      for (int d = 0; d < 64; ++d) qf[d] = BF(q[((size_t)b * Hq + h) * D + d]);
      float pm[32], pl[32], po[32][64];
      for (int s = 0; s < S; ++s) {
        const int c0 = (int)((int64_t)s * nch / S), c1 = (int)((int64_t)(s + 1) * nch / S);
        float m = -INFINITY, l = 0.0f;
        float o[64][8]; /* [lane = kg*8 + dq][e] */
        for (int ln = 0; ln < 64; ++ln)
          for (int e = 0; e < 8; ++e) o[ln][e] = 0.0f;
        for (int c = c0; c < c1; ++c) {
          float sc[64], pj[64];
          int valid[64];
          float cm = -INFINITY;
          for (int ln = 0; ln < 64; ++ln) {
            const int j = lo + c * 64 + ln;
            valid[ln] = j <= p;
            if (!valid[ln]) { sc[ln] = -INFINITY; continue; }
            const uint16_t* kr = kc + (base + j) * D;
            float a = 0.0f;
            for (int d = 0; d < 64; ++d) a = fmaf(qf[d], BF(kr[d]), a);
            sc[ln] = a * 0.125f;
            if (sc[ln] > cm) cm = sc[ln];
          }
          const float mn = m > cm ? m : cm;
          const float alpha = or_expf(m - mn);
          for (int ln = 0; ln < 64; ++ln) pj[ln] = valid[ln] ? or_expf(sc[ln] - mn) : 0.0f;
          float tmp[64];
          memcpy(tmp, pj, sizeof(tmp));
          l = fmaf(l, alpha, c_butterfly64(tmp));
          m = mn;
          for (int ln = 0; ln < 64; ++ln)
            for (int e = 0; e < 8; ++e) o[ln][e] = o[ln][e] * alpha;
          for (int ln = 0; ln < 64; ++ln) {
            const int kg = ln >> 3, dq = ln & 7;
            for (int i = 0; i < 8; ++i) {
              const int jj = kg + 8 * i, jk = lo + c * 64 + jj;
              if (jk > p) continue;
              const uint16_t* vr = vc + (base + jk) * D + dq * 8;
              for (int e = 0; e < 8; ++e) o[ln][e] = fmaf(pj[jj], BF(vr[e]), o[ln][e]);
            }
          }
        }
        /* reduce over kg (lane bits 3..5): xor 8, then 16, then 32 */
        for (int step = 1; step <= 4; step <<= 1) {
          float t[64][8];
          for (int ln = 0; ln < 64; ++ln)
            for (int e = 0; e < 8; ++e) t[ln][e] = o[ln][e] + o[ln ^ (8 * step)][e];
          memcpy(o, t, sizeof(t));
        }
        pm[s] = m;
        pl[s] = l;
        for (int dq = 0; dq < 8; ++dq)
          for (int e = 0; e < 8; ++e) po[s][dq * 8 + e] = o[dq][e];
      }
      const float sk = BF(sinks[h]);
      float M = sk;
      for (int s = 0; s < S; ++s) M = M > pm[s] ? M : pm[s];
      float den = or_expf(sk - M);
      float acc[64];
      for (int d = 0; d < 64; ++d) acc[d] = 0.0f;
      for (int s = 0; s < S; ++s) {
        const float f = (pm[s] == -INFINITY) ? 0.0f : or_expf(pm[s] - M);
        den = fmaf(pl[s], f, den);
        for (int d = 0; d < 64; ++d) acc[d] = fmaf(f, po[s][d], acc[d]);
      }
      const float inv = 1.0f / den;
      for (int d = 0; d < 64; ++d) {
        const float r = acc[d] * inv;
        if (out_f32) out_f32[((size_t)b * Hq + h) * D + d] = r;
        if (out) out[((size_t)b * Hq + h) * D + d] = TOBF(r);
      }
    }
}

/* ------------------------------------------------------------------------ */
/* Router (HFM:117-130): logits = x W^T + b, top-k over the logits, softmax  */
/* over the k selected values.  The logits use ONE canonical fp32 reduction  */
/* order, identical to the device router, so top-k indices match bit for     */
/* bit: 64 lane partials (lane l owns the 8-element units u = l + 64 i, in   */
/* increasing k, one fmaf per element), then a xor-butterfly over offsets    */
/* 32,16,8,4,2,1, then + bias.  Ties go to the lower expert index.           */
/* ------------------------------------------------------------------------ */
static int g_router_fp64 = 0;  /* set with the accumulation mode */
static float router_logit(const uint16_t* x, const uint16_t* w, int H,
                          uint16_t bias) {
  if (g_router_fp64) {
    double d = 0.0;
    for (int i = 0; i < H; ++i) d += (double)BF(x[i]) * BF(w[i]);
    return (float)d + BF(bias);
  }
  float p[64];
  const int U = H / 8;
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int u = l; u < U; u += 64)
      for (int j = 0; j < 8; ++j)
        acc = fmaf(BF(x[u * 8 + j]), BF(w[u * 8 + j]), acc);
    p[l] = acc;
  }
  for (int off = 32; off >= 1; off >>= 1) {
    float q[64];
    for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ off];
    memcpy(p, q, sizeof(p));
  }
  return p[0] + BF(bias);
}

/* The router's total order on experts: larger logit first, NaN after every
 * number, ties (equal values, or both NaN) to the lower expert index.  Expert
 * i's rank is the number of experts ordered before it; the top k are the
 * ranks 0..k-1.  For finite logits this is "top k by value, ties to the
 * lower index" (HFM:126-130 with torch.topk's tie rule made explicit). */
static int ranks_before(float vj, int j, float vi, int i) {
  const int nj = vj != vj, ni = vi != vi;
  if (nj != ni) return ni;
  if (!nj && vj != vi) return vj > vi;
  return j < i;
}

void or_router(const uint16_t* x, const uint16_t* W, const uint16_t* b, int B,
               int E, int H, int k, int32_t* idx, float* score,
               float* logits) {
  float* lg = (float*)malloc(sizeof(float) * E);
  for (int r = 0; r < B; ++r) {
    for (int e = 0; e < E; ++e)
      lg[e] = router_logit(x + (size_t)r * H, W + (size_t)e * H, H, b[e]);
    if (logits) memcpy(logits + (size_t)r * E, lg, sizeof(float) * E);
    float v[64];
    for (int i = 0; i < E; ++i) {
      int rank = 0;
      for (int j = 0; j < E; ++j) rank += ranks_before(lg[j], j, lg[i], i);
      if (rank < k) {
        idx[r * k + rank] = i;
        v[rank] = lg[i];
      }
    }
    float ex[64], s = 0.0f;
    for (int t = 0; t < k; ++t) {
      ex[t] = or_expf(v[t] - v[0]);
      s += ex[t];
    }
    for (int t = 0; t < k; ++t) score[r * k + t] = ex[t] / s;
  }
  free(lg);
}

/* ------------------------------------------------------------------------ */
/* SwiGLU with clamp (HFM:82-87): gate = gu[2j] clamped above at limit, up = */
/* gu[2j+1] clamped to [-limit, limit], out = (up + 1) * gate * sigmoid(     */
/* alpha * gate).                                                            */
/* ------------------------------------------------------------------------ */
void or_swiglu(const float* gu, int I, float alpha, float limit, float* out) {
  for (int j = 0; j < I; ++j) {
    float g = gu[2 * j], u = gu[2 * j + 1];
    g = g > limit ? limit : g;
    u = u > limit ? limit : (u < -limit ? -limit : u);
    float sig = 1.0f / (1.0f + or_expf(-(g * alpha)));
    out[j] = (u + 1.0f) * (g * sig);
  }
}

/* Accumulation mode of the model functions: 0 = the canonical fp32 orders
 * (bit-identical to the device), 1 = fp64 accumulation rounded once (the
 * or_gemv_* / or_rmsnorm / or_attn_decode forms).  Mode 1 exists to measure
 * how far a mere change of summation order moves the model's outputs. */
static int g_acc_mode = 0;
void or_set_accumulation(int mode) { g_acc_mode = mode; g_router_fp64 = mode; }

static void m_gemv_bf16(const uint16_t* W, const uint16_t* bias, const uint16_t* x, int B,
                        int N, int K, uint16_t* y, float* y_f32) {
  if (g_acc_mode) or_gemv_bf16(W, bias, x, B, N, K, y, y_f32);
  else or_c_gemv_bf16(W, bias, x, B, N, K, y, y_f32);
}
static void m_gemv_fp4(const uint8_t* codes, const uint8_t* scales, const uint16_t* bias,
                       const uint16_t* x, int B, int N, int K, uint16_t* y, float* y_f32) {
  if (g_acc_mode) or_mxfp4_gemv(codes, scales, bias, x, B, N, K, y, y_f32);
  else or_c_mxfp4_gemv(codes, scales, bias, x, B, N, K, y, y_f32);
}
static void m_rmsnorm(const uint16_t* x, const uint16_t* w, int B, int H, float eps,
                      uint16_t* out) {
  if (g_acc_mode) or_rmsnorm(x, w, B, H, eps, out);
  else or_c_rmsnorm(x, w, B, H, eps, out);
}

/* One row's experts (HFM:89-114), canonical form: for each slot t (rank
 * order) gate_up GEMV + bias -> SwiGLU -> bf16 -> down GEMV + bias, then
 * acc = fmaf(score_t, out, acc) from 0; one rounding to bf16.  Slot t's
 * weights come through the pointer arrays (the expert idx[t] already
 * resolved by the caller). */
static void moe_row_slots(const uint16_t* x, int H, int I, int k, const float* score,
                          const uint8_t* const* guc, const uint8_t* const* gus,
                          const uint16_t* const* gub, const uint8_t* const* dnc,
                          const uint8_t* const* dns, const uint16_t* const* dnb,
                          float alpha, float limit, uint16_t* out) {
  float* gu = (float*)malloc(sizeof(float) * 2 * I);
  float* act = (float*)malloc(sizeof(float) * I);
  uint16_t* actb = (uint16_t*)malloc(sizeof(uint16_t) * I);
  float* dn = (float*)malloc(sizeof(float) * H);
  float* acc = (float*)malloc(sizeof(float) * H);
  for (int i = 0; i < H; ++i) acc[i] = 0.0f;
  for (int t = 0; t < k; ++t) {
    m_gemv_fp4(guc[t], gus[t], gub[t], x, 1, 2 * I, H, NULL, gu);
    or_swiglu(gu, I, alpha, limit, act);
    for (int j = 0; j < I; ++j) actb[j] = TOBF(act[j]);
    m_gemv_fp4(dnc[t], dns[t], dnb[t], actb, 1, H, I, NULL, dn);
    for (int i = 0; i < H; ++i) acc[i] = fmaf(score[t], dn[i], acc[i]);
  }
  for (int i = 0; i < H; ++i) out[i] = TOBF(acc[i]);
  free(gu); free(act); free(actb); free(dn); free(acc);
}

/* Experts with given ids and weights (HF GptOssExperts, HFM:89-114), the
 * canonical moe_row_slots per row.  A slot whose id lies outside [0, E) adds
 * nothing (the device kernels drop it and flag the call). */
void or_moe_experts(const uint16_t* x, const int32_t* idx, const float* score,
                    const uint8_t* gu_codes, const uint8_t* gu_scales,
                    const uint16_t* gu_bias, const uint8_t* dn_codes,
                    const uint8_t* dn_scales, const uint16_t* dn_bias, int B, int E,
                    int H, int I, int k, float alpha, float limit, uint16_t* out) {
  const size_t gu_code_sz = (size_t)2 * I * (H / 2), gu_sc_sz = (size_t)2 * I * (H / 32);
  const size_t dn_code_sz = (size_t)H * (I / 2), dn_sc_sz = (size_t)H * (I / 32);
  for (int r = 0; r < B; ++r) {
    const uint8_t *guc[64], *gus[64], *dnc[64], *dns[64];
    const uint16_t *gub[64], *dnb[64];
    float sc[64];
    int n = 0;
    for (int t = 0; t < k; ++t) {
      const int32_t e = idx[r * k + t];
      if (e < 0 || e >= E) continue;
      guc[n] = gu_codes + (size_t)e * gu_code_sz; gus[n] = gu_scales + (size_t)e * gu_sc_sz;
      gub[n] = gu_bias + (size_t)e * 2 * I;
      dnc[n] = dn_codes + (size_t)e * dn_code_sz; dns[n] = dn_scales + (size_t)e * dn_sc_sz;
      dnb[n] = dn_bias + (size_t)e * H;
      sc[n] = score[r * k + t];
      ++n;
    }
    /* dropped slots add exactly 0 (fmaf(s, 0, acc) = acc), so the remaining
     * slots in order give the same bits */
    moe_row_slots(x + (size_t)r * H, H, I, n, sc, guc, gus, gub, dnc, dns, dnb, alpha, limit,
                  out + (size_t)r * H);
  }
}

/* MoE block (HFM:89-114, 145-154) on already-normalised x, canonical form:
 * router, then moe_row_slots over the selected experts. */
void or_moe_layer(const uint16_t* x, const uint16_t* router_w,
                  const uint16_t* router_b, const uint8_t* gu_codes,
                  const uint8_t* gu_scales, const uint16_t* gu_bias,
                  const uint8_t* dn_codes, const uint8_t* dn_scales,
                  const uint16_t* dn_bias, int B, int E, int H, int I, int k,
                  float alpha, float limit, uint16_t* out, int32_t* idx,
                  float* score) {
  or_router(x, router_w, router_b, B, E, H, k, idx, score, NULL);
  const size_t gu_code_sz = (size_t)2 * I * (H / 2), gu_sc_sz = (size_t)2 * I * (H / 32);
  const size_t dn_code_sz = (size_t)H * (I / 2), dn_sc_sz = (size_t)H * (I / 32);
  if (B >= 2) {
    /* the same per-(row, slot) GEMVs, with the rows that chose an expert in
     * one call (its weights transposed once); then each row's slots are
     * combined in slot order as in moe_row_slots */
    float* dn = (float*)malloc(sizeof(float) * (size_t)B * k * H);
    uint16_t* xs = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)B * k * H);
    uint16_t* acts = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)B * k * I);
    float* gu = (float*)malloc(sizeof(float) * (size_t)B * k * 2 * I);
    float* dq = (float*)malloc(sizeof(float) * (size_t)B * k * H);
    float* act = (float*)malloc(sizeof(float) * I);
    int* pairs = (int*)malloc(sizeof(int) * (size_t)B * k);
    for (int e = 0; e < E; ++e) {
      int n = 0;
      for (int q = 0; q < B * k; ++q)
        if (idx[q] == e) pairs[n++] = q;
      if (n == 0) continue;
      for (int i = 0; i < n; ++i)
        memcpy(xs + (size_t)i * H, x + (size_t)(pairs[i] / k) * H, sizeof(uint16_t) * H);
      m_gemv_fp4(gu_codes + e * gu_code_sz, gu_scales + e * gu_sc_sz,
                 gu_bias + (size_t)e * 2 * I, xs, n, 2 * I, H, NULL, gu);
      for (int i = 0; i < n; ++i) {
        or_swiglu(gu + (size_t)i * 2 * I, I, alpha, limit, act);
        for (int j = 0; j < I; ++j) acts[(size_t)i * I + j] = TOBF(act[j]);
      }
      m_gemv_fp4(dn_codes + e * dn_code_sz, dn_scales + e * dn_sc_sz,
                 dn_bias + (size_t)e * H, acts, n, H, I, NULL, dq);
      for (int i = 0; i < n; ++i)
        memcpy(dn + (size_t)pairs[i] * H, dq + (size_t)i * H, sizeof(float) * H);
    }
    for (int r = 0; r < B; ++r)
      for (int i = 0; i < H; ++i) {
        float acc = 0.0f;
        for (int t = 0; t < k; ++t)
          acc = fmaf(score[r * k + t], dn[((size_t)r * k + t) * H + i], acc);
        out[(size_t)r * H + i] = TOBF(acc);
      }
    free(dn); free(xs); free(acts); free(gu); free(dq); free(act); free(pairs);
    return;
  }
  for (int r = 0; r < B; ++r) {
    const uint8_t *guc[64], *gus[64], *dnc[64], *dns[64];
    const uint16_t *gub[64], *dnb[64];
    for (int t = 0; t < k; ++t) {
      const size_t e = (size_t)idx[r * k + t];
      guc[t] = gu_codes + e * gu_code_sz; gus[t] = gu_scales + e * gu_sc_sz;
      gub[t] = gu_bias + e * 2 * I;
      dnc[t] = dn_codes + e * dn_code_sz; dns[t] = dn_scales + e * dn_sc_sz;
      dnb[t] = dn_bias + e * H;
    }
    moe_row_slots(x + (size_t)r * H, H, I, k, score + r * k, guc, gus, gub, dnc, dns, dnb,
                  alpha, limit, out + (size_t)r * H);
  }
}

/* ------------------------------------------------------------------------ */
/* Decode attention with sinks (HFM:235-263, 276-277, 292-293): for query    */
/* head h (kv head h / (Hq/Hkv)), logits s_j = q.k_j / sqrt(D) over keys     */
/* j in [lo, pos] (lo = pos - window + 1 for sliding layers, HF mask        */
/* kv_idx > q_idx - window), softmax over [s_j..., sink_h], sink column      */
/* dropped before P.V.  fp64 inside; rounded once.                            */
/* ------------------------------------------------------------------------ */
void or_attn_decode(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                    const uint16_t* sinks, int B, int Hq, int Hkv, int D,
                    int T_max, const int32_t* pos, int window, uint16_t* out,
                    float* out_f32) {
  const int G = Hq / Hkv;
  const double scale = 1.0 / sqrt((double)D);
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      const int kvh = h / G, p = pos[b];
      int lo = 0;
      if (window > 0 && p - window + 1 > 0) lo = p - window + 1;
      const int n = p - lo + 1;
      const uint16_t* qh = q + ((size_t)b * Hq + h) * D;
      const size_t base = ((size_t)b * Hkv + kvh) * T_max;
      double* s = (double*)malloc(sizeof(double) * n);
      double m = (double)BF(sinks[h]);
      for (int j = 0; j < n; ++j) {
        const uint16_t* kr = kc + (base + lo + j) * D;
        double d = 0.0;
        for (int i = 0; i < D; ++i) d += (double)BF(qh[i]) * BF(kr[i]);
        s[j] = d * scale;
        if (s[j] > m) m = s[j];
      }
      double den = exp((double)BF(sinks[h]) - m);
      double o[256] = {0};
      for (int j = 0; j < n; ++j) {
        double pj = exp(s[j] - m);
        den += pj;
        const uint16_t* vr = vc + (base + lo + j) * D;
        for (int i = 0; i < D; ++i) o[i] += pj * BF(vr[i]);
      }
      for (int i = 0; i < D; ++i) {
        float r = (float)(o[i] / den);
        if (out_f32) out_f32[((size_t)b * Hq + h) * D + i] = r;
        if (out) out[((size_t)b * Hq + h) * D + i] = TOBF(r);
      }
      free(s);
    }
}

/* ------------------------------------------------------------------------ */
/* Full model                                                                */
/* ------------------------------------------------------------------------ */
typedef struct or_layer {
  uint16_t *attn_norm, *wqkv, *bqkv, *wo, *bo, *sinks, *mlp_norm, *router_w,
      *router_b, *gu_bias, *dn_bias;
  uint8_t *gu_codes, *gu_scales, *dn_codes, *dn_scales;
} or_layer;

struct or_model {
  or_config cfg;
  int batch;
  uint16_t *embed, *lm_head, *final_norm;
  or_layer* layers;
  float *cos_t, *sin_t;
  uint16_t *kc, *vc; /* [L][B][Hkv][max_seq][D] */
  int32_t* pos;
  uint16_t* h; /* [B][H] */
  /* lazy experts: the MXFP4 codes and scales are not kept; each step
   * regenerates the chosen experts' slices from the counter RNG into these
   * k-slot buffers (for shapes whose experts do not fit in host memory) */
  int lazy;
  uint64_t seed;
  uint8_t *lz_guc, *lz_gus, *lz_dnc, *lz_dns;
  int64_t lz_key[64]; /* (layer, expert) held by each slot buffer, -1 none */
  /* last step, batch row 0, last layer: buffers named like the device's */
  uint16_t *t_qkv, *t_attn, *t_moe_in;
  int32_t t_idx[64];
  float t_score[64];
};

static void* xmalloc(size_t n) {
  void* p = malloc(n ? n : 1);
  if (!p) abort();
  return p;
}

or_model* or_model_create(const or_config* cfg, uint64_t seed, int batch) {
  return or_model_create_ex(cfg, seed, batch, 0);
}

or_model* or_model_create_ex(const or_config* cfg, uint64_t seed, int batch, int flags) {
  or_model* m = (or_model*)calloc(1, sizeof(or_model));
  m->cfg = *cfg;
  m->batch = batch;
  m->seed = seed;
  m->lazy = (flags & OR_LAZY_EXPERTS) != 0;
  const int H = cfg->hidden, D = cfg->head_dim, Hq = cfg->n_heads,
            Hkv = cfg->n_kv_heads, E = cfg->n_experts, I = cfg->intermediate;
  const int64_t V = cfg->vocab, QKV = (int64_t)(Hq + 2 * Hkv) * D;
  m->embed = (uint16_t*)xmalloc(sizeof(uint16_t) * V * H);
  m->lm_head = (uint16_t*)xmalloc(sizeof(uint16_t) * V * H);
  m->final_norm = (uint16_t*)xmalloc(sizeof(uint16_t) * H);
  or_fill_bf16(seed, or_stream_id(-1, OR_T_EMBED), V * H, 0.0f, 0.02, m->embed);
  or_fill_bf16(seed, or_stream_id(-1, OR_T_LM_HEAD), V * H, 0.0f, 0.02,
               m->lm_head);
  or_fill_bf16(seed, or_stream_id(-1, OR_T_FINAL_NORM), H, 1.0f, 0.05,
               m->final_norm);
  m->layers = (or_layer*)calloc(cfg->n_layers, sizeof(or_layer));
  for (int l = 0; l < cfg->n_layers; ++l) {
    or_layer* L = &m->layers[l];
#define GEN_BF(field, kind, n, mean, std)                              \
  L->field = (uint16_t*)xmalloc(sizeof(uint16_t) * (size_t)(n));       \
  or_fill_bf16(seed, or_stream_id(l, kind), (n), (mean), (std), L->field)
    GEN_BF(attn_norm, OR_T_ATTN_NORM, H, 1.0f, 0.05);
    GEN_BF(wqkv, OR_T_WQKV, QKV * H, 0.0f, 0.02);
    GEN_BF(bqkv, OR_T_BQKV, QKV, 0.0f, 0.02);
    GEN_BF(wo, OR_T_WO, (int64_t)H * Hq * D, 0.0f, 0.02);
    GEN_BF(bo, OR_T_BO, H, 0.0f, 0.02);
    GEN_BF(sinks, OR_T_SINKS, Hq, 0.0f, 1.0);
    GEN_BF(mlp_norm, OR_T_MLP_NORM, H, 1.0f, 0.05);
    GEN_BF(router_w, OR_T_ROUTER_W, (int64_t)E * H, 0.0f, 0.02);
    GEN_BF(router_b, OR_T_ROUTER_B, E, 0.0f, 0.02);
    GEN_BF(gu_bias, OR_T_GU_BIAS, (int64_t)E * 2 * I, 0.0f, 0.02);
    GEN_BF(dn_bias, OR_T_DN_BIAS, (int64_t)E * H, 0.0f, 0.02);
#undef GEN_BF
    const int64_t gu_codes = (int64_t)E * 2 * I * (H / 2),
                  gu_sc = (int64_t)E * 2 * I * (H / 32);
    const int64_t dn_codes = (int64_t)E * H * (I / 2),
                  dn_sc = (int64_t)E * H * (I / 32);
    if (m->lazy) continue;
    L->gu_codes = (uint8_t*)xmalloc(gu_codes);
    L->gu_scales = (uint8_t*)xmalloc(gu_sc);
    L->dn_codes = (uint8_t*)xmalloc(dn_codes);
    L->dn_scales = (uint8_t*)xmalloc(dn_sc);
    or_fill_bytes(seed, or_stream_id(l, OR_T_GU_CODES), gu_codes, L->gu_codes);
    or_fill_scales(seed, or_stream_id(l, OR_T_GU_SCALES), gu_sc, 119, 6,
                   L->gu_scales);
    or_fill_bytes(seed, or_stream_id(l, OR_T_DN_CODES), dn_codes, L->dn_codes);
    or_fill_scales(seed, or_stream_id(l, OR_T_DN_SCALES), dn_sc, 119, 6,
                   L->dn_scales);
  }
  if (m->lazy) {
    const size_t k = (size_t)cfg->top_k;
    m->lz_guc = (uint8_t*)xmalloc(k * 2 * I * (H / 2));
    m->lz_gus = (uint8_t*)xmalloc(k * 2 * I * (H / 32));
    m->lz_dnc = (uint8_t*)xmalloc(k * H * (I / 2));
    m->lz_dns = (uint8_t*)xmalloc(k * H * (I / 32));
    for (int t = 0; t < 64; ++t) m->lz_key[t] = -1;
  }
  m->cos_t = (float*)xmalloc(sizeof(float) * (size_t)cfg->max_seq * (D / 2));
  m->sin_t = (float*)xmalloc(sizeof(float) * (size_t)cfg->max_seq * (D / 2));
  or_rope_table(cfg, cfg->max_seq, m->cos_t, m->sin_t);
  const size_t kv = (size_t)cfg->n_layers * batch * Hkv * cfg->max_seq * D;
  m->kc = (uint16_t*)calloc(kv, sizeof(uint16_t));
  m->vc = (uint16_t*)calloc(kv, sizeof(uint16_t));
  m->pos = (int32_t*)calloc(batch, sizeof(int32_t));
  m->h = (uint16_t*)calloc((size_t)batch * H, sizeof(uint16_t));
  m->t_qkv = (uint16_t*)calloc((size_t)QKV, sizeof(uint16_t));
  m->t_attn = (uint16_t*)calloc((size_t)Hq * D, sizeof(uint16_t));
  m->t_moe_in = (uint16_t*)calloc((size_t)H, sizeof(uint16_t));
  return m;
}

void or_model_free(or_model* m) {
  if (!m) return;
  for (int l = 0; l < m->cfg.n_layers; ++l) {
    or_layer* L = &m->layers[l];
    free(L->attn_norm); free(L->wqkv); free(L->bqkv); free(L->wo); free(L->bo);
    free(L->sinks); free(L->mlp_norm); free(L->router_w); free(L->router_b);
    free(L->gu_bias); free(L->dn_bias); free(L->gu_codes); free(L->gu_scales);
    free(L->dn_codes); free(L->dn_scales);
  }
  free(m->layers); free(m->embed); free(m->lm_head); free(m->final_norm);
  free(m->cos_t); free(m->sin_t); free(m->kc); free(m->vc); free(m->pos);
  free(m->h); free(m->t_qkv); free(m->t_attn); free(m->t_moe_in);
  free(m->lz_guc); free(m->lz_gus); free(m->lz_dnc); free(m->lz_dns); free(m);
}

static size_t tensor_bytes(const or_config* c, int kind) {
  const size_t H = c->hidden, E = c->n_experts, I = c->intermediate, V = c->vocab;
  const size_t QKV = (size_t)(c->n_heads + 2 * c->n_kv_heads) * c->head_dim;
  const size_t HD = (size_t)c->n_heads * c->head_dim;
  switch (kind) {
    case OR_T_EMBED: case OR_T_LM_HEAD: return V * H * 2;
    case OR_T_FINAL_NORM: case OR_T_ATTN_NORM: case OR_T_MLP_NORM: case OR_T_BO: return H * 2;
    case OR_T_WQKV: return QKV * H * 2;
    case OR_T_BQKV: return QKV * 2;
    case OR_T_WO: return H * HD * 2;
    case OR_T_SINKS: return (size_t)c->n_heads * 2;
    case OR_T_ROUTER_W: return E * H * 2;
    case OR_T_ROUTER_B: return E * 2;
    case OR_T_GU_CODES: return E * 2 * I * (H / 2);
    case OR_T_GU_SCALES: return E * 2 * I * (H / 32);
    case OR_T_GU_BIAS: return E * 2 * I * 2;
    case OR_T_DN_CODES: return E * H * (I / 2);
    case OR_T_DN_SCALES: return E * H * (I / 32);
    case OR_T_DN_BIAS: return E * H * 2;
    default: return 0;
  }
}

int or_model_set_tensor(or_model* m, int layer, int kind, const void* data, size_t bytes) {
  void* p = (void*)or_model_tensor(m, layer, kind);
  if (p == NULL || bytes != tensor_bytes(&m->cfg, kind)) return -1;
  memcpy(p, data, bytes);
  return 0;
}

/* Synthetic KV history for timing: every layer's cache rows 0 .. n_pos-1 of
 * every sequence hold N(0,1) bf16 keys and values, and every sequence is at
 * position n_pos (the next step attends over n_pos + 1 keys). */
void or_model_fill_kv(or_model* m, int n_pos, uint64_t seed) {
  const or_config* c = &m->cfg;
  const size_t D = c->head_dim, T = c->max_seq;
  const size_t n_streams = (size_t)c->n_layers * m->batch * c->n_kv_heads;
  for (size_t s = 0; s < n_streams; ++s) {
    or_fill_bf16(seed, 0x10000u + 2 * s, (int64_t)n_pos * D, 0.0f, 1.0, m->kc + s * T * D);
    or_fill_bf16(seed, 0x10001u + 2 * s, (int64_t)n_pos * D, 0.0f, 1.0, m->vc + s * T * D);
  }
  for (int b = 0; b < m->batch; ++b) m->pos[b] = n_pos;
}

const void* or_model_trace(const or_model* m, int what) {
  switch (what) {
    case 0: return m->t_qkv;
    case 1: return m->t_attn;
    case 2: return m->t_moe_in;
    case 3: return m->t_idx;
    case 4: return m->t_score;
    default: return NULL;
  }
}

const uint16_t* or_model_hidden(const or_model* m) { return m->h; }
int32_t or_model_pos(const or_model* m, int b) { return m->pos[b]; }

const void* or_model_tensor(const or_model* m, int layer, int kind) {
  if (layer < 0) {
    switch (kind) {
      case OR_T_EMBED: return m->embed;
      case OR_T_LM_HEAD: return m->lm_head;
      case OR_T_FINAL_NORM: return m->final_norm;
      default: return NULL;
    }
  }
  const or_layer* L = &m->layers[layer];
  switch (kind) {
    case OR_T_ATTN_NORM: return L->attn_norm;
    case OR_T_WQKV: return L->wqkv;
    case OR_T_BQKV: return L->bqkv;
    case OR_T_WO: return L->wo;
    case OR_T_BO: return L->bo;
    case OR_T_SINKS: return L->sinks;
    case OR_T_MLP_NORM: return L->mlp_norm;
    case OR_T_ROUTER_W: return L->router_w;
    case OR_T_ROUTER_B: return L->router_b;
    case OR_T_GU_CODES: return L->gu_codes;
    case OR_T_GU_SCALES: return L->gu_scales;
    case OR_T_GU_BIAS: return L->gu_bias;
    case OR_T_DN_CODES: return L->dn_codes;
    case OR_T_DN_SCALES: return L->dn_scales;
    case OR_T_DN_BIAS: return L->dn_bias;
    default: return NULL;
  }
}

/* Experts of rows 0 .. B-1 (normalised xn [B][H]) for layer l -> out [B][H]
 * (bf16), ids and weights [B][k].  Lazy models regenerate each chosen
 * expert's slice from the counter RNG (the same bytes init wrote). */
static void model_moe(or_model* m, int l, const uint16_t* xn, int B, uint16_t* out,
                      int32_t* idx, float* sc) {
  const or_config* c = &m->cfg;
  const int H = c->hidden, E = c->n_experts, I = c->intermediate, K = c->top_k;
  const or_layer* L = &m->layers[l];
  if (!m->lazy) {
    or_moe_layer(xn, L->router_w, L->router_b, L->gu_codes, L->gu_scales, L->gu_bias,
                 L->dn_codes, L->dn_scales, L->dn_bias, B, E, H, I, K, c->swiglu_alpha,
                 c->swiglu_limit, out, idx, sc);
    return;
  }
  or_router(xn, L->router_w, L->router_b, B, E, H, K, idx, sc, NULL);
  const size_t gcs = (size_t)2 * I * (H / 2), gss = (size_t)2 * I * (H / 32);
  const size_t dcs = (size_t)H * (I / 2), dss = (size_t)H * (I / 32);
  for (int r = 0; r < B; ++r) {
    const uint8_t *guc[64], *gus[64], *dnc[64], *dns[64];
    const uint16_t *gub[64], *dnb[64];
    for (int t = 0; t < K; ++t) {
      const size_t e = (size_t)idx[r * K + t];
      uint8_t* a = m->lz_guc + t * gcs; uint8_t* b2 = m->lz_gus + t * gss;
      uint8_t* d = m->lz_dnc + t * dcs; uint8_t* f = m->lz_dns + t * dss;
      /* the slot buffer already holds this (layer, expert): same bytes */
      const int64_t key = (int64_t)l * E + (int64_t)e;
      if (m->lz_key[t] != key) {
        m->lz_key[t] = key;
        or_fill_bytes_at(m->seed, or_stream_id(l, OR_T_GU_CODES), (int64_t)(e * gcs),
                         (int64_t)gcs, a);
        or_fill_scales_at(m->seed, or_stream_id(l, OR_T_GU_SCALES), (int64_t)(e * gss),
                          (int64_t)gss, 119, 6, b2);
        or_fill_bytes_at(m->seed, or_stream_id(l, OR_T_DN_CODES), (int64_t)(e * dcs),
                         (int64_t)dcs, d);
        or_fill_scales_at(m->seed, or_stream_id(l, OR_T_DN_SCALES), (int64_t)(e * dss),
                          (int64_t)dss, 119, 6, f);
      }
      guc[t] = a; gus[t] = b2; dnc[t] = d; dns[t] = f;
      gub[t] = L->gu_bias + e * 2 * I; dnb[t] = L->dn_bias + e * H;
    }
    moe_row_slots(xn + (size_t)r * H, H, I, K, sc + r * K, guc, gus, gub, dnc, dns, dnb,
                  c->swiglu_alpha, c->swiglu_limit, out + (size_t)r * H);
  }
}

/* Decoder layer (HFM:347-376): h += attn(norm(h)); h += moe(norm(h)); each
 * sublayer output rounded to bf16 and added to the bf16 residual with one
 * rounding.  Layer i is sliding iff (i + 1) is odd (HFC:75-78).  Every
 * reduction uses the canonical or_c_* forms, so the step is bit-identical to
 * the device's.  The rows of a step go through the layers together (each
 * weight row is read once per step); every row's arithmetic is the same as
 * if it ran alone. */
void or_model_step(or_model* m, const int32_t* ids, float* logits,
                   int32_t* out_ids) {
  const or_config* c = &m->cfg;
  const int H = c->hidden, D = c->head_dim, Hq = c->n_heads, Hkv = c->n_kv_heads;
  const int K = c->top_k, B = m->batch;
  const int QKV = (Hq + 2 * Hkv) * D, half = D / 2;
  const int64_t V = c->vocab;
  const size_t T = (size_t)c->max_seq;
  uint16_t* xn = (uint16_t*)xmalloc(sizeof(uint16_t) * B * H);
  uint16_t* qkv = (uint16_t*)xmalloc(sizeof(uint16_t) * B * QKV);
  uint16_t* qr = (uint16_t*)xmalloc(sizeof(uint16_t) * B * Hq * D);
  uint16_t* ao = (uint16_t*)xmalloc(sizeof(uint16_t) * B * Hq * D);
  uint16_t* tmp = (uint16_t*)xmalloc(sizeof(uint16_t) * B * H);
  float* lg = (float*)xmalloc(sizeof(float) * V * B);
  int32_t* idx = (int32_t*)xmalloc(sizeof(int32_t) * B * K);
  float* sc = (float*)xmalloc(sizeof(float) * B * K);
  for (int b = 0; b < B; ++b)
    memcpy(m->h + (size_t)b * H, m->embed + (size_t)ids[b] * H, sizeof(uint16_t) * H);
  for (int l = 0; l < c->n_layers; ++l) {
    const or_layer* L = &m->layers[l];
    const int window = (l % 2 == 0) ? c->sliding_window : 0;
    uint16_t* kc_l = m->kc + (size_t)l * B * Hkv * T * D;
    uint16_t* vc_l = m->vc + (size_t)l * B * Hkv * T * D;
    m_rmsnorm(m->h, L->attn_norm, B, H, c->rms_eps, xn);
    m_gemv_bf16(L->wqkv, L->bqkv, xn, B, QKV, H, qkv, NULL);
    for (int b = 0; b < B; ++b) {
      const int p = m->pos[b];
      const float* cr = m->cos_t + (size_t)p * half;
      const float* sr = m->sin_t + (size_t)p * half;
      const uint16_t* qb = qkv + (size_t)b * QKV;
      or_rope_apply(qb, Hq, D, cr, sr, qr + (size_t)b * Hq * D);
      uint16_t kr[4096];
      or_rope_apply(qb + Hq * D, Hkv, D, cr, sr, kr);
      for (int g = 0; g < Hkv; ++g) {
        const size_t row = (((size_t)b * Hkv + g) * T + p) * D;
        memcpy(kc_l + row, kr + g * D, sizeof(uint16_t) * D);
        memcpy(vc_l + row, qb + (Hq + Hkv + g) * D, sizeof(uint16_t) * D);
      }
    }
    if (g_acc_mode)
      or_attn_decode(qr, kc_l, vc_l, L->sinks, B, Hq, Hkv, D, (int)T, m->pos, window, ao, NULL);
    else
      or_c_attn_decode(qr, kc_l, vc_l, L->sinks, B, Hq, Hkv, D, (int)T, m->pos, window,
                       or_attn_splits((int)T, window), ao, NULL);
    m_gemv_bf16(L->wo, L->bo, ao, B, H, Hq * D, tmp, NULL);
    for (size_t i = 0; i < (size_t)B * H; ++i) m->h[i] = TOBF(BF(m->h[i]) + BF(tmp[i]));
    m_rmsnorm(m->h, L->mlp_norm, B, H, c->rms_eps, xn);
    model_moe(m, l, xn, B, tmp, idx, sc);
    if (l == c->n_layers - 1) {
      memcpy(m->t_qkv, qkv, sizeof(uint16_t) * QKV);
      memcpy(m->t_attn, ao, sizeof(uint16_t) * Hq * D);
      memcpy(m->t_moe_in, xn, sizeof(uint16_t) * H);
      memcpy(m->t_idx, idx, sizeof(int32_t) * K);
      memcpy(m->t_score, sc, sizeof(float) * K);
    }
    for (size_t i = 0; i < (size_t)B * H; ++i) m->h[i] = TOBF(BF(m->h[i]) + BF(tmp[i]));
  }
  if (!logits && !out_ids) {  /* a teacher-forced prompt row: no lm_head */
    for (int b = 0; b < B; ++b) m->pos[b] = m->pos[b] + 1;
    free(xn); free(qkv); free(qr); free(ao); free(tmp); free(lg); free(idx); free(sc);
    return;
  }
  m_rmsnorm(m->h, m->final_norm, B, H, c->rms_eps, xn);
  m_gemv_bf16(m->lm_head, NULL, xn, B, (int)V, H, NULL, lg);
  for (int b = 0; b < B; ++b) {
    const float* lb = lg + (size_t)b * V;
    int best = 0;
    for (int64_t v = 1; v < V; ++v)
      if (lb[v] > lb[best]) best = (int)v;
    if (out_ids) out_ids[b] = best;
    if (logits) memcpy(logits + (size_t)b * V, lb, sizeof(float) * V);
    m->pos[b] = m->pos[b] + 1;
  }
  free(xn); free(qkv); free(qr); free(ao); free(tmp); free(lg); free(idx); free(sc);
}

/* Teacher-forced prompt rows in layer-major order: sequence b consumes
 * ids[b][0 .. n-1] at positions pos[b] .. pos[b] + n - 1 (no lm_head), as
 * n calls of or_model_step with NULL outputs would.  A row's layer-l input
 * depends only on its own layer-(l-1) output and on the layer-l keys and
 * values of positions <= its own, so all B n rows can go through layer l
 * before any enters layer l + 1, in position order within the layer's
 * attention; every row sees the same operands in the same order, so the
 * KV cache, positions and hidden state come out bit-identical.  The dense
 * projections and the experts then read each weight row once for all rows,
 * and a lazy model generates each layer's experts once (E experts' codes and
 * scales of one layer in memory at a time) instead of per row. */
void or_model_prompt(or_model* m, const int32_t* ids, int n) {
  const or_config* c = &m->cfg;
  const int H = c->hidden, D = c->head_dim, Hq = c->n_heads, Hkv = c->n_kv_heads;
  const int K = c->top_k, B = m->batch, E = c->n_experts, I = c->intermediate;
  const int QKV = (Hq + 2 * Hkv) * D, half = D / 2;
  const size_t T = (size_t)c->max_seq, R = (size_t)B * n;
  if (n <= 0) return;
  uint16_t* hs = (uint16_t*)xmalloc(sizeof(uint16_t) * R * H);
  uint16_t* xn = (uint16_t*)xmalloc(sizeof(uint16_t) * R * H);
  uint16_t* qkv = (uint16_t*)xmalloc(sizeof(uint16_t) * R * QKV);
  uint16_t* qr = (uint16_t*)xmalloc(sizeof(uint16_t) * R * Hq * D);
  uint16_t* ao = (uint16_t*)xmalloc(sizeof(uint16_t) * R * Hq * D);
  uint16_t* tmp = (uint16_t*)xmalloc(sizeof(uint16_t) * R * H);
  int32_t* idx = (int32_t*)xmalloc(sizeof(int32_t) * R * K);
  float* sc = (float*)xmalloc(sizeof(float) * R * K);
  const size_t gu_c = (size_t)E * 2 * I * (H / 2), gu_s = (size_t)E * 2 * I * (H / 32);
  const size_t dn_c = (size_t)E * H * (I / 2), dn_s = (size_t)E * H * (I / 32);
  uint8_t *lguc = NULL, *lgus = NULL, *ldnc = NULL, *ldns = NULL;
  if (m->lazy) {
    lguc = (uint8_t*)xmalloc(gu_c); lgus = (uint8_t*)xmalloc(gu_s);
    ldnc = (uint8_t*)xmalloc(dn_c); ldns = (uint8_t*)xmalloc(dn_s);
  }
  for (size_t r = 0; r < R; ++r)
    memcpy(hs + r * H, m->embed + (size_t)ids[r] * H, sizeof(uint16_t) * H);
  for (int l = 0; l < c->n_layers; ++l) {
    const or_layer* L = &m->layers[l];
    const int window = (l % 2 == 0) ? c->sliding_window : 0;
    uint16_t* kc_l = m->kc + (size_t)l * B * Hkv * T * D;
    uint16_t* vc_l = m->vc + (size_t)l * B * Hkv * T * D;
    m_rmsnorm(hs, L->attn_norm, (int)R, H, c->rms_eps, xn);
    m_gemv_bf16(L->wqkv, L->bqkv, xn, (int)R, QKV, H, qkv, NULL);
    for (size_t r = 0; r < R; ++r) {
      const int b = (int)(r / n), p = m->pos[b] + (int)(r % n);
      const float* cr = m->cos_t + (size_t)p * half;
      const float* sr = m->sin_t + (size_t)p * half;
      const uint16_t* qb = qkv + r * QKV;
      or_rope_apply(qb, Hq, D, cr, sr, qr + r * Hq * D);
      uint16_t kr[4096];
      or_rope_apply(qb + Hq * D, Hkv, D, cr, sr, kr);
      for (int g = 0; g < Hkv; ++g) {
        const size_t row = (((size_t)b * Hkv + g) * T + p) * D;
        memcpy(kc_l + row, kr + g * D, sizeof(uint16_t) * D);
        memcpy(vc_l + row, qb + (Hq + Hkv + g) * D, sizeof(uint16_t) * D);
      }
    }
    /* row (b, t) attends to sequence b's keys at positions <= pos[b] + t */
    for (size_t r = 0; r < R; ++r) {
      const int b = (int)(r / n);
      const int32_t p = m->pos[b] + (int)(r % n);
      const size_t kvb = (size_t)b * Hkv * T * D;
      if (g_acc_mode)
        or_attn_decode(qr + r * Hq * D, kc_l + kvb, vc_l + kvb, L->sinks, 1, Hq, Hkv, D,
                       (int)T, &p, window, ao + r * Hq * D, NULL);
      else
        or_c_attn_decode(qr + r * Hq * D, kc_l + kvb, vc_l + kvb, L->sinks, 1, Hq, Hkv, D,
                         (int)T, &p, window, or_attn_splits((int)T, window),
                         ao + r * Hq * D, NULL);
    }
    m_gemv_bf16(L->wo, L->bo, ao, (int)R, H, Hq * D, tmp, NULL);
    for (size_t i = 0; i < R * H; ++i) hs[i] = TOBF(BF(hs[i]) + BF(tmp[i]));
    m_rmsnorm(hs, L->mlp_norm, (int)R, H, c->rms_eps, xn);
    const uint8_t *guc = L->gu_codes, *gus = L->gu_scales, *dnc = L->dn_codes,
                  *dns = L->dn_scales;
    if (m->lazy) {
      or_fill_bytes(m->seed, or_stream_id(l, OR_T_GU_CODES), (int64_t)gu_c, lguc);
      or_fill_scales(m->seed, or_stream_id(l, OR_T_GU_SCALES), (int64_t)gu_s, 119, 6, lgus);
      or_fill_bytes(m->seed, or_stream_id(l, OR_T_DN_CODES), (int64_t)dn_c, ldnc);
      or_fill_scales(m->seed, or_stream_id(l, OR_T_DN_SCALES), (int64_t)dn_s, 119, 6, ldns);
      guc = lguc; gus = lgus; dnc = ldnc; dns = ldns;
    }
    or_moe_layer(xn, L->router_w, L->router_b, guc, gus, L->gu_bias, dnc, dns, L->dn_bias,
                 (int)R, E, H, I, K, c->swiglu_alpha, c->swiglu_limit, tmp, idx, sc);
    for (size_t i = 0; i < R * H; ++i) hs[i] = TOBF(BF(hs[i]) + BF(tmp[i]));
  }
  /* the hidden state of each sequence's last prompt row, as after a step */
  for (int b = 0; b < B; ++b) {
    memcpy(m->h + (size_t)b * H, hs + ((size_t)b * n + n - 1) * H, sizeof(uint16_t) * H);
    m->pos[b] += n;
  }
  free(hs); free(xn); free(qkv); free(qr); free(ao); free(tmp); free(idx); free(sc);
  free(lguc); free(lgus); free(ldnc); free(ldns);
}

/* ------------------------------------------------------------------------ */
/* Temperature + nucleus (top-p) sampling, the device's exact operation      */
/* order (neon_sample / the context's sampled steps).  Row b's 1024 "threads"*/
/* t = 64 w + l each own the indices t, t + 1024, ... for the max, the       */
/* exponentials and the threshold sums; a block sum is the 64-lane xor       */
/* butterfly of each wave, then the 16 wave totals added in order from 0.    */
/*   m = max_i l_i;  e_i = exp((l_i - m) * (1 / T));  z = sum e_i            */
/*   threshold t: the largest float (bisected bit 30 .. 0 of its bits) with  */
/*     sum_{e_i >= t} e_i >= top_p * z  (t = 0 keeps all when top_p >= 1)   */
/*   u = (splitmix64(seed ^ splitmix64(b << 32 | pos_b)) >> 40) * 2^-24      */
/*   the pick: the first kept index whose running sum in vocabulary order    */
/*   exceeds u * kept, with the running sum formed per contiguous slice of   */
/*   ceil(V / 1024) indices (thread t owns slice t) after an exclusive       */
/*   prefix of the slice totals in slice order.                              */
/* ------------------------------------------------------------------------ */
static uint64_t splitmix64_step(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

static float block_sum_1024_c(const float* part) {
  float tot = 0.0f;
  for (int w = 0; w < 16; ++w) {
    float v[64];
    memcpy(v, part + 64 * w, sizeof(v));
    tot = tot + c_butterfly64(v);
  }
  return tot;
}

void or_sample(const float* logits, int B, int V, float temperature, float top_p,
               uint64_t seed, const int32_t* pos, int32_t* out_ids) {
  const float inv_temp = 1.0f / temperature;
  float* e = (float*)xmalloc(sizeof(float) * (size_t)V);
  float part[1024];
  for (int b = 0; b < B; ++b) {
    const float* l = logits + (size_t)b * V;
    float m = -INFINITY;
    for (int i = 0; i < V; ++i) m = fmaxf(m, l[i]);
    for (int t = 0; t < 1024; ++t) {
      float z = 0.0f;
      for (int i = t; i < V; i += 1024) {
        e[i] = or_expf((l[i] - m) * inv_temp);
        z = z + e[i];
      }
      part[t] = z;
    }
    const float z = block_sum_1024_c(part);
    uint32_t t_bits = 0;
    float kept = z;
    if (top_p < 1.0f) {
      const float goal = top_p * z;
      for (int bit = 30; bit >= 0; --bit) {
        const uint32_t cand = t_bits | (1u << bit);
        float th;
        memcpy(&th, &cand, 4);
        for (int t = 0; t < 1024; ++t) {
          float sp = 0.0f;
          for (int i = t; i < V; i += 1024) sp = sp + (e[i] >= th ? e[i] : 0.0f);
          part[t] = sp;
        }
        const float sm = block_sum_1024_c(part);
        if (sm >= goal) { t_bits = cand; kept = sm; }
      }
    }
    float th;
    memcpy(&th, &t_bits, 4);
    const uint64_t r = splitmix64_step(
        seed ^ splitmix64_step(((uint64_t)(uint32_t)b << 32) | (uint32_t)pos[b]));
    const float u = (float)(r >> 40) * 0x1.0p-24f;
    const float target = u * kept;
    const int Cs = (V + 1023) / 1024;
    float acc = 0.0f;
    int32_t pick = -1;
    for (int t = 0; t < 1024 && pick < 0; ++t) {
      const int i0 = t * Cs < V ? t * Cs : V, i1 = i0 + Cs < V ? i0 + Cs : V;
      float local = 0.0f;
      for (int i = i0; i < i1; ++i) local = local + (e[i] >= th ? e[i] : 0.0f);
      float run = acc;  /* exclusive prefix of the slice totals */
      if (run <= target && local > 0.0f && run + local > target) {
        int last = -1, found = -1;
        for (int i = i0; i < i1; ++i)
          if (e[i] >= th) {
            last = i;
            run = run + e[i];
            if (run > target) { found = i; break; }
          }
        pick = found >= 0 ? found : last;
      }
      acc = acc + local;
    }
    if (pick < 0) {
      for (int i = V - 1; i >= 0; --i)
        if (e[i] >= th) { pick = i; break; }
      if (pick < 0) pick = 0;
    }
    out_ids[b] = pick;
  }
  free(e);
}

#ifdef _OPENMP
#include <omp.h>
#endif
/* threads the oracle's parallel loops use (reported with CPU timings) */
int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

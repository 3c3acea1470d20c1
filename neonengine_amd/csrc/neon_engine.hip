// neon_engine.hip -- the C-ABI (include/neon_gptoss.h): argument validation,
// the model context (weights, KV cache, activations in HBM), deterministic
// init, checkpoint-tensor loading, and the decode step, captured once into a
// hipGraph and replayed per token.
//
// Shape of the boundary: a context object created once (like the reference's
// System constructors, NeonEngine/src/water_physics.cpp:23-123) and per-step
// calls that enqueue a fixed kernel chain on the caller's stream (like
// WaterPhysics::RunSimulation recording its dispatch chain,
// NeonEngine/src/water_physics.cpp:131,165-436).  No exception crosses the
// ABI; failures come back as neon_status with text in neon_last_error.
#include "../../include/neon_gptoss.h"
#include "neon_common.hpp"
#include "neon_internal.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

using namespace neon;

namespace {

thread_local std::string g_create_error;

struct LayerW {
  uint16_t *attn_norm, *wqkv, *bqkv, *wo, *bo, *sinks, *mlp_norm, *router_w,
      *router_b, *gu_bias, *dn_bias;
  uint8_t *gu_codes, *gu_scales, *dn_codes, *dn_scales;
};

enum {
  K_ATTN_NORM = 0, K_WQKV = 1, K_BQKV = 2, K_WO = 3, K_BO = 4, K_SINKS = 5,
  K_MLP_NORM = 6, K_ROUTER_W = 7, K_ROUTER_B = 8, K_GU_CODES = 9,
  K_GU_SCALES = 10, K_GU_BIAS = 11, K_DN_CODES = 12, K_DN_SCALES = 13,
  K_DN_BIAS = 14, K_EMBED = 100, K_LM_HEAD = 101, K_FINAL_NORM = 102
};

struct Tensor {
  void* ptr;
  size_t bytes;
};

}  // namespace

// Prompt rows run through the layers together in the chunked prompt pass (the
// batched decode kernels take up to 16 rows; the experts up to 64 row-slots).
constexpr int kPromptRows = 16;

struct neon_ctx {
  neon_config cfg{};
  int device = 0;
  std::string err;
  // weights
  char* arena = nullptr;
  size_t arena_bytes = 0;
  std::vector<LayerW> layers;
  uint16_t *embed = nullptr, *lm_head = nullptr, *final_norm = nullptr;
  // rope
  float *cos_t = nullptr, *sin_t = nullptr;
  // KV cache [L][max_batch][Hkv][max_seq][D]
  uint16_t *kc = nullptr, *vc = nullptr;
  // per layer: element offset into kc / vc, cache rows per (sequence, kv
  // head) and the position -> row mask (ring caches on sliding layers)
  std::vector<size_t> kv_off;
  std::vector<int> kv_rows, kv_mask;
  // activations / scratch
  char* work = nullptr;
  uint16_t *h = nullptr, *xn = nullptr, *qkv = nullptr, *attn_out = nullptr,
           *act = nullptr, *q_rot = nullptr;  // q_rot: rotated q heads [B][Hq][D]
  int32_t* moe_idx = nullptr;
  float* moe_score = nullptr;
  float* router_lg = nullptr;
  float *attn_po = nullptr, *attn_pml = nullptr;  // split partials
  int32_t* attn_arrive = nullptr;  // [Br][Hkv] arrival counters of the split kernel
  float* logits = nullptr;
  float* lm_part_val = nullptr;
  int32_t* lm_part_idx = nullptr;
  int32_t *tokens = nullptr, *pos = nullptr, *prompt_len = nullptr,
          *last_ids = nullptr;
  int32_t* dev_err = nullptr;  // status word the step's kernels set (kDevErr* bits)
  int32_t* moe_sync = nullptr;  // [L][kMoeSyncInts] counters of the one-launch experts
  int tok_stride = 0;
  int lm_nblk = 0;
  int s_full = 1, s_slide = 1;
  // sequence state (host mirror)
  int batch = 0;
  int host_pos = 0;                // the longest sequence's position
  std::vector<int> host_plen;      // prompt length of each sequence
  // per batch row: the position of its next input token (the tokens it
  // holds - 1) and whether a sequence holds it (neon_seq_add /
  // neon_seq_remove); rows past `batch` are free
  std::vector<int> host_seq_pos;
  std::vector<char> host_active;
  bool weights_ready = false;
  // batched prefill (M prompt rows per pass): scratch grown on demand
  int prefill_mode = NEON_PREFILL_CHUNKED;
  char* pf = nullptr;
  int pf_rows = 0;
  uint16_t *pf_h = nullptr, *pf_xn = nullptr, *pf_qkv = nullptr, *pf_q = nullptr,
           *pf_ao = nullptr, *pf_act = nullptr, *pf_ks = nullptr, *pf_vs = nullptr;
  uint8_t* pf_mxq = nullptr;   // MXFP8 step lines of the expert GEMM inputs
  uint32_t* pf_mxqs = nullptr;
  float *pf_lg = nullptr, *pf_score = nullptr, *pf_ybuf = nullptr;
  int32_t *pf_idx = nullptr, *pf_ltok = nullptr, *pf_lslot = nullptr, *pf_eoff = nullptr,
          *pf_tile_e = nullptr, *pf_tile_r0 = nullptr, *pf_ntiles = nullptr;
  // next-token choice (temperature 0: greedy argmax)
  float temperature = 0.0f, top_p = 1.0f;
  uint64_t sample_seed = 0;
  float* sample_scratch = nullptr;  // [max_batch][vocab] exp values
  // batched steps on the matrix cores (max_batch >= 2)
  int decode_mode = NEON_DECODE_EXACT;
  // batch-1 experts as one launch with a grid-wide wait (k_moe_fused) when
  // NEON_MOE_FUSED=1; the default is the gate_up / down kernel pair, which
  // measured faster on MI355X (the in-kernel wait plus every block fetching
  // act past its L2 cost more than the kernel boundary they replace)
  bool fused_moe = getenv("NEON_MOE_FUSED") && getenv("NEON_MOE_FUSED")[0] == '1';
  // follow-up work run by the producing launch (same bits, one launch fewer):
  // the attention merge by the last split block of each kv head (fuse_merge,
  // on by default: 1.2197 against 1.2248 ms per 20b step), and at batch 1 the
  // router logits by tail blocks of the O projection (fuse_router, off by
  // default: 1.2595 ms, its arrival round trip and agent-scope reads cost
  // more than the launch they save).  NEON_FUSE_TAILS: unset or "a" the
  // merge only, "1" both, "r" the router only, "0" neither
  const char* fuse_env = getenv("NEON_FUSE_TAILS");
  bool fuse_merge = !fuse_env || fuse_env[0] == '1' || fuse_env[0] == 'a';
  bool fuse_router = fuse_env && (fuse_env[0] == '1' || fuse_env[0] == 'r');
  int32_t* or_arrive = nullptr;  // kMoeSyncWords + 1 words (O -> router)
  int32_t* rr_arrive = nullptr;  // one word (router + route lists, matrix-core steps)
  int32_t* rl_arrive = nullptr;  // [max_batch] row counters (top-k in the logits launch)
  // How the matrix-core steps route (NEON_ROUTER_ROUTE): by default the
  // router logits launch, then a top-k launch that stores each row's expert
  // ids, and every expert block builds its own work item from the ids
  // (mx_route_item), so no launch waits for all rows ("2": logits and top-k
  // in one launch, a block per row, for comparisons).  "0" builds the route
  // table in the top-k launch, "1" inside a one-launch router (its last
  // block), and the expert kernels then read the table (the same items).
  int route_table = getenv("NEON_ROUTER_ROUTE") && (getenv("NEON_ROUTER_ROUTE")[0] == '0' ||
                                                    getenv("NEON_ROUTER_ROUTE")[0] == '1')
                        ? getenv("NEON_ROUTER_ROUTE")[0] - '0' : -1;
  bool route_one = getenv("NEON_ROUTER_ROUTE") && getenv("NEON_ROUTER_ROUTE")[0] == '2';
  // without a table, the top-k finishes in the router logits launch (the
  // last wave of each row ranks it; NEON_ROUTER_RANK=0: a top-k launch)
  bool route_rank = !(getenv("NEON_ROUTER_RANK") && getenv("NEON_ROUTER_RANK")[0] == '0');
  // the matrix-core steps' expert combine also writes the next RMSNorm (the
  // next layer's, or the final one) into the packed layout, one launch fewer
  // per layer (NEON_MX_COMBINE_NORM=0: separate launches; the same bits)
  bool mx_combine_norm = !(getenv("NEON_MX_COMBINE_NORM") && getenv("NEON_MX_COMBINE_NORM")[0] == '0');
  float* mx_ybuf = nullptr;          // [max_batch][top_k][hidden] expert dot + bias
  float* mx_part_val = nullptr;      // [max_batch][vocab / 16] lm_head partial argmax
  int32_t* mx_part_idx = nullptr;
  int32_t* mx_route = nullptr;       // used experts and their pair lists
  uint16_t* mx_xp = nullptr;         // normalised rows in the packed activation layout
  uint16_t* mx_ap = nullptr;         // attention output in the packed activation layout
  bool mx_fuse_rope = true;          // RoPE + KV append inside the attention launch
  // the weights in MFMA lane order for the matrix-core steps (allocated when
  // that mode is first selected; refreshed before a step after any change)
  struct MxLayer { uint16_t *wqkv, *wo; uint8_t *gu_c, *gu_s, *dn_c, *dn_s; };
  char* mx_w = nullptr;
  uint8_t* mx8_q = nullptr;  // NEON_DECODE_MATRIX_MX8: MXFP8 images of the expert inputs
  std::vector<MxLayer> mxp;
  uint16_t* mx_lm = nullptr;
  bool mx_dirty = true;
  // prompt passes: positions and sequences of the rows of one pass
  int32_t *row_pos = nullptr, *row_seq = nullptr;
  // captured decode step
  hipStream_t cap_stream = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  int graph_batch = 0;
};

#define FAIL(ctx, code, ...)                                     \
  do {                                                           \
    char _b[512];                                                \
    snprintf(_b, sizeof(_b), __VA_ARGS__);                       \
    (ctx)->err = _b;                                             \
    return (code);                                               \
  } while (0)

#define HIPCHK(ctx, call)                                                   \
  do {                                                                      \
    hipError_t _e = (call);                                                 \
    if (_e != hipSuccess)                                                   \
      FAIL(ctx, NEON_EHIP, "%s failed: %s", #call, hipGetErrorString(_e)); \
  } while (0)

static hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------------------
// configuration
// ---------------------------------------------------------------------------
extern "C" neon_status neon_config_preset(const char* name, neon_config* out) {
  if (!name || !out) return NEON_EINVAL;
  neon_config c{};
  // gpt-oss-20b shape (HF configuration_gpt_oss.py defaults, 24 layers, 32
  // experts); the 120b shape has 36 layers and 128 experts.
  c.n_layers = 24; c.hidden = 2880; c.n_heads = 64; c.n_kv_heads = 8;
  c.head_dim = 64; c.n_experts = 32; c.top_k = 4; c.intermediate = 2880;
  c.vocab = 201088; c.sliding_window = 128; c.max_seq = 4096; c.max_batch = 1;
  c.rope_theta = 150000.0f; c.rope_factor = 32.0f; c.rope_beta_fast = 32.0f;
  c.rope_beta_slow = 1.0f; c.rope_orig_max_pos = 4096; c.rms_eps = 1e-5f;
  c.swiglu_limit = 7.0f; c.swiglu_alpha = 1.702f;
  if (strcmp(name, "gpt-oss-20b") == 0) {
  } else if (strcmp(name, "gpt-oss-120b") == 0) {
    c.n_layers = 36; c.n_experts = 128;
  } else {
    return NEON_EINVAL;
  }
  *out = c;
  return NEON_OK;
}

static const char* check_config(const neon_config* c) {
  if (c->n_layers < 1 || c->n_layers > 1024) return "n_layers out of range";
  if (c->head_dim != 64) return "head_dim must be 64";
  if (c->hidden < 64 || c->hidden > 8192 || c->hidden % 64)
    return "hidden must be a multiple of 64 in [64, 8192]";
  if (c->intermediate < 64 || c->intermediate > 8192 || c->intermediate % 64)
    return "intermediate must be a multiple of 64 in [64, 8192]";
  if (c->n_kv_heads < 1 || c->n_heads < 1 || c->n_heads % c->n_kv_heads)
    return "n_heads must be a multiple of n_kv_heads";
  {
    const int g = c->n_heads / c->n_kv_heads;
    if (g != 1 && g != 2 && g != 4 && g != 8) return "n_heads/n_kv_heads must be 1, 2, 4 or 8";
  }
  if ((int64_t)c->n_heads * c->head_dim > 8192) return "n_heads*head_dim must be <= 8192";
  if (c->n_experts < 1 || c->n_experts > 256) return "n_experts must be in [1, 256]";
  if (c->top_k < 1 || c->top_k > 16 || c->top_k > c->n_experts)
    return "top_k must be in [1, min(16, n_experts)]";
  if (c->vocab < 1) return "vocab must be positive";
  if (c->sliding_window < 0) return "sliding_window must be >= 0";
  if (c->max_seq < 1 || c->max_seq > (1 << 20)) return "max_seq out of range";
  if (c->max_batch < 1 || c->max_batch > 256) return "max_batch must be in [1, 256]";
  if (!(c->rms_eps > 0.0f)) return "rms_eps must be positive";
  if (!(c->rope_theta > 1.0f) || !(c->rope_factor >= 1.0f)) return "bad rope parameters";
  if (c->rope_orig_max_pos < 1) return "rope_orig_max_pos must be positive";
  return nullptr;
}

// YaRN inverse frequencies and attention factor in fp64 (HF
// modeling_rope_utils.py:429-483 with truncate=False as gpt-oss sets it).
static void yarn_inv_freq(const neon_config* c, std::vector<float>& invf,
                          double* af) {
  const int dim = c->head_dim;
  const double base = c->rope_theta, factor = c->rope_factor;
  auto corr = [&](double nrot) {
    return (dim * std::log(c->rope_orig_max_pos / (nrot * 2.0 * M_PI))) /
           (2.0 * std::log(base));
  };
  double low = corr(c->rope_beta_fast), high = corr(c->rope_beta_slow);
  if (low < 0) low = 0;
  if (high > dim - 1) high = dim - 1;
  if (low == high) high += 0.001;
  invf.resize(dim / 2);
  for (int i = 0; i < dim / 2; ++i) {
    const double pf = std::pow(base, (2.0 * i) / dim);
    const double extra = 1.0 / pf, inter = 1.0 / (factor * pf);
    double ramp = (i - low) / (high - low);
    ramp = ramp < 0 ? 0 : (ramp > 1 ? 1 : ramp);
    const double ef = 1.0 - ramp;
    invf[i] = (float)(inter * (1.0 - ef) + extra * ef);
  }
  *af = factor <= 1.0 ? 1.0 : 0.1 * std::log(factor) + 1.0;
}

// cos/sin tables [n_pos][head_dim/2] in fp32: angle = fp32(inv_freq) *
// fp32(pos) (HFM:196-198), cos/sin in fp64 rounded to fp32, times the fp32
// attention factor.  Built on the host so every position is identical to the
// oracle's table.
static void rope_table_host(const neon_config* c, int n_pos,
                            std::vector<float>& ct, std::vector<float>& st) {
  std::vector<float> invf;
  double af;
  yarn_inv_freq(c, invf, &af);
  const float aff = (float)af;
  const int half = c->head_dim / 2;
  ct.resize((size_t)n_pos * half);
  st.resize((size_t)n_pos * half);
  for (int p = 0; p < n_pos; ++p)
    for (int i = 0; i < half; ++i) {
      const float ang = invf[i] * (float)p;
      ct[(size_t)p * half + i] = (float)std::cos((double)ang) * aff;
      st[(size_t)p * half + i] = (float)std::sin((double)ang) * aff;
    }
}

// ---------------------------------------------------------------------------
// context lifetime
// ---------------------------------------------------------------------------
namespace {
struct Sizes {
  size_t qkv_rows, embed, wqkv, wo, gu_codes, gu_scales, dn_codes, dn_scales;
};
Sizes sizes_of(const neon_config& c) {
  Sizes s;
  const size_t H = c.hidden, I = c.intermediate, E = c.n_experts;
  s.qkv_rows = (size_t)(c.n_heads + 2 * c.n_kv_heads) * c.head_dim;
  s.embed = (size_t)c.vocab * H;
  s.wqkv = s.qkv_rows * H;
  s.wo = H * (size_t)c.n_heads * c.head_dim;
  s.gu_codes = E * 2 * I * (H / 2);
  s.gu_scales = E * 2 * I * (H / 32);
  s.dn_codes = E * H * (I / 2);
  s.dn_scales = E * H * (I / 32);
  return s;
}
size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }
}  // namespace

extern "C" void neon_ctx_destroy(neon_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  // Work enqueued by neon_prefill/neon_decode may still run on the caller's
  // stream: wait for it before the graph, its kernel arguments and the
  // buffers it reads are released.
  (void)hipDeviceSynchronize();
  if (ctx->graph_exec) (void)hipGraphExecDestroy(ctx->graph_exec);
  if (ctx->graph) (void)hipGraphDestroy(ctx->graph);
  if (ctx->cap_stream) (void)hipStreamDestroy(ctx->cap_stream);
  if (ctx->arena) (void)hipFree(ctx->arena);
  if (ctx->kc) (void)hipFree(ctx->kc);
  if (ctx->vc) (void)hipFree(ctx->vc);
  if (ctx->work) (void)hipFree(ctx->work);
  if (ctx->pf) (void)hipFree(ctx->pf);
  if (ctx->mx_w) (void)hipFree(ctx->mx_w);
  if (ctx->mx8_q) (void)hipFree(ctx->mx8_q);
  delete ctx;
}

extern "C" const char* neon_last_error(const neon_ctx* ctx) {
  return ctx ? ctx->err.c_str() : g_create_error.c_str();
}

static neon_status ctx_alloc(neon_ctx* ctx) {
  const neon_config& c = ctx->cfg;
  const Sizes sz = sizes_of(c);
  const size_t H = c.hidden, E = c.n_experts, I = c.intermediate, L = c.n_layers;
  // ---- weights arena ----
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes); return o; };
  struct LOff { size_t v[15]; };
  std::vector<LOff> lo(L);
  const size_t o_embed = take(sz.embed * 2), o_lm = take(sz.embed * 2),
               o_fn = take(H * 2);
  for (size_t l = 0; l < L; ++l) {
    lo[l].v[K_ATTN_NORM] = take(H * 2);
    lo[l].v[K_WQKV] = take(sz.wqkv * 2);
    lo[l].v[K_BQKV] = take(sz.qkv_rows * 2);
    lo[l].v[K_WO] = take(sz.wo * 2);
    lo[l].v[K_BO] = take(H * 2);
    lo[l].v[K_SINKS] = take((size_t)c.n_heads * 2);
    lo[l].v[K_MLP_NORM] = take(H * 2);
    lo[l].v[K_ROUTER_W] = take(E * H * 2);
    lo[l].v[K_ROUTER_B] = take(E * 2);
    lo[l].v[K_GU_CODES] = take(sz.gu_codes);
    lo[l].v[K_GU_SCALES] = take(sz.gu_scales);
    lo[l].v[K_GU_BIAS] = take(E * 2 * I * 2);
    lo[l].v[K_DN_CODES] = take(sz.dn_codes);
    lo[l].v[K_DN_SCALES] = take(sz.dn_scales);
    lo[l].v[K_DN_BIAS] = take(E * H * 2);
  }
  ctx->arena_bytes = off;
  if (hipMalloc(&ctx->arena, off) != hipSuccess) {
    ctx->arena = nullptr;
    FAIL(ctx, NEON_ENOMEM, "hipMalloc of %zu weight bytes failed", off);
  }
  char* A = ctx->arena;
  ctx->embed = (uint16_t*)(A + o_embed);
  ctx->lm_head = (uint16_t*)(A + o_lm);
  ctx->final_norm = (uint16_t*)(A + o_fn);
  ctx->layers.resize(L);
  for (size_t l = 0; l < L; ++l) {
    LayerW& w = ctx->layers[l];
    w.attn_norm = (uint16_t*)(A + lo[l].v[K_ATTN_NORM]);
    w.wqkv = (uint16_t*)(A + lo[l].v[K_WQKV]);
    w.bqkv = (uint16_t*)(A + lo[l].v[K_BQKV]);
    w.wo = (uint16_t*)(A + lo[l].v[K_WO]);
    w.bo = (uint16_t*)(A + lo[l].v[K_BO]);
    w.sinks = (uint16_t*)(A + lo[l].v[K_SINKS]);
    w.mlp_norm = (uint16_t*)(A + lo[l].v[K_MLP_NORM]);
    w.router_w = (uint16_t*)(A + lo[l].v[K_ROUTER_W]);
    w.router_b = (uint16_t*)(A + lo[l].v[K_ROUTER_B]);
    w.gu_codes = (uint8_t*)(A + lo[l].v[K_GU_CODES]);
    w.gu_scales = (uint8_t*)(A + lo[l].v[K_GU_SCALES]);
    w.gu_bias = (uint16_t*)(A + lo[l].v[K_GU_BIAS]);
    w.dn_codes = (uint8_t*)(A + lo[l].v[K_DN_CODES]);
    w.dn_scales = (uint8_t*)(A + lo[l].v[K_DN_SCALES]);
    w.dn_bias = (uint16_t*)(A + lo[l].v[K_DN_BIAS]);
  }
  // ---- KV cache ----
  // Full layers keep every position.  A sliding layer only ever reads the
  // last `window` keys, so it keeps a power-of-two ring of at least
  // window + kPromptRows rows (a prompt pass appends kPromptRows rows before
  // its attention reads the oldest key of its first row's window): position
  // p lives in row p & (rows - 1).
  ctx->kv_off.assign(L, 0);
  ctx->kv_rows.assign(L, c.max_seq);
  ctx->kv_mask.assign(L, -1);
  size_t kv_elems = 0;
  for (size_t l = 0; l < L; ++l) {
    const bool sliding = (l % 2 == 0) && c.sliding_window > 0;  // HFC:75-78
    if (sliding) {
      int ring = 1;
      while (ring < c.sliding_window + kPromptRows) ring <<= 1;
      if (ring < c.max_seq) { ctx->kv_rows[l] = ring; ctx->kv_mask[l] = ring - 1; }
    }
    ctx->kv_off[l] = kv_elems;
    kv_elems += (size_t)c.max_batch * c.n_kv_heads * ctx->kv_rows[l] * c.head_dim;
  }
  const size_t kv_bytes = kv_elems * 2;
  if (hipMalloc(&ctx->kc, kv_bytes) != hipSuccess || hipMalloc(&ctx->vc, kv_bytes) != hipSuccess)
    FAIL(ctx, NEON_ENOMEM, "hipMalloc of 2 x %zu KV-cache bytes failed", kv_bytes);
  HIPCHK(ctx, hipMemset(ctx->kc, 0, kv_bytes));
  HIPCHK(ctx, hipMemset(ctx->vc, 0, kv_bytes));
  // ---- activations / scratch ----
  // Bm sequences; Br rows per pass (a prompt pass runs up to kPromptRows
  // rows of one sequence at once)
  const size_t Bm = c.max_batch, half = c.head_dim / 2;
  const size_t Br = std::max<size_t>(Bm, kPromptRows);
  ctx->s_slide = attn_splits(c.max_seq, c.sliding_window);
  ctx->s_full = attn_splits(c.max_seq, 0);
  ctx->lm_nblk = gemv_default_grid(c.vocab, 2);
  ctx->tok_stride = c.max_seq + 1;
  off = 0;
  const size_t o_h = take(Br * H * 2), o_xn = take(Br * H * 2),
               o_qkv = take(Br * sz.qkv_rows * 2),
               o_ao = take(Br * (size_t)c.n_heads * c.head_dim * 2),
               o_qr = take(Br * (size_t)c.n_heads * c.head_dim * 2),
               o_act = take(Br * c.top_k * I * 2),
               o_idx = take(Br * c.top_k * 4), o_sc = take(Br * c.top_k * 4),
               o_rlg = take(Br * c.n_experts * 4),
               o_apo = take(Br * c.n_heads * (size_t)std::max(ctx->s_full, ctx->s_slide) * c.head_dim * 4),
               o_apml = take(Br * c.n_heads * (size_t)std::max(ctx->s_full, ctx->s_slide) * 2 * 4),
               o_aarr = take(Br * (size_t)c.n_kv_heads * kAttnArriveStride * 4),
               o_orarr = take((kMoeSyncWords + 1) * kMoeSyncStride * 4),
               o_rrarr = take(kMoeSyncStride * 4),
               o_rlarr = take(Bm * kMoeSyncStride * 4),
               o_rpos = take(kPromptRows * 4), o_rseq = take(kPromptRows * 4),
               o_samp = take(Bm * (size_t)c.vocab * 4),
               o_mxy = take(Bm > 1 ? Bm * (size_t)c.top_k * H * 4 : 0),
               o_mxv = take(Bm > 1 ? Bm * (size_t)(c.vocab / 16) * 4 : 0),
               o_mxi = take(Bm > 1 ? Bm * (size_t)(c.vocab / 16) * 4 : 0),
               o_mxr = take(Bm > 1 ? (size_t)kMxRouteWords * 4 : 0),
               o_mxp = take(Bm > 1 ? (size_t)((Bm + 15) / 16) * ((H + 127) / 128) * 2048 * 2 : 0),
               o_mxa = take(Bm > 1 ? (size_t)((Bm + 15) / 16) * ((c.n_heads * c.head_dim + 127) / 128) * 2048 * 2 : 0),
               o_lg = take(Bm * (size_t)c.vocab * 4),
               o_pv = take(Bm * ctx->lm_nblk * 4), o_pi = take(Bm * ctx->lm_nblk * 4),
               o_tok = take(Bm * ctx->tok_stride * 4), o_pos = take(Bm * 4),
               o_pl = take(Bm * 4), o_last = take(Bm * 4), o_err = take(4),
               o_msync = take(L * kMoeSyncInts * 4),
               o_cos = take((size_t)c.max_seq * half * 4),
               o_sin = take((size_t)c.max_seq * half * 4);
  if (hipMalloc(&ctx->work, off) != hipSuccess) {
    ctx->work = nullptr;
    FAIL(ctx, NEON_ENOMEM, "hipMalloc of %zu scratch bytes failed", off);
  }
  HIPCHK(ctx, hipMemset(ctx->work, 0, off));
  char* W = ctx->work;
  ctx->h = (uint16_t*)(W + o_h); ctx->xn = (uint16_t*)(W + o_xn);
  ctx->qkv = (uint16_t*)(W + o_qkv); ctx->attn_out = (uint16_t*)(W + o_ao);
  ctx->q_rot = (uint16_t*)(W + o_qr);
  ctx->act = (uint16_t*)(W + o_act); ctx->moe_idx = (int32_t*)(W + o_idx);
  ctx->moe_score = (float*)(W + o_sc);
  ctx->router_lg = (float*)(W + o_rlg);
  ctx->attn_po = (float*)(W + o_apo); ctx->attn_pml = (float*)(W + o_apml);
  ctx->attn_arrive = (int32_t*)(W + o_aarr);  // zeroed above; every launch leaves it at 0
  ctx->or_arrive = (int32_t*)(W + o_orarr);    // likewise
  ctx->rr_arrive = (int32_t*)(W + o_rrarr);    // likewise
  ctx->rl_arrive = (int32_t*)(W + o_rlarr);    // likewise
  ctx->logits = (float*)(W + o_lg); ctx->lm_part_val = (float*)(W + o_pv);
  ctx->lm_part_idx = (int32_t*)(W + o_pi); ctx->tokens = (int32_t*)(W + o_tok);
  ctx->pos = (int32_t*)(W + o_pos); ctx->prompt_len = (int32_t*)(W + o_pl);
  ctx->last_ids = (int32_t*)(W + o_last); ctx->cos_t = (float*)(W + o_cos);
  ctx->dev_err = (int32_t*)(W + o_err);
  ctx->moe_sync = (int32_t*)(W + o_msync);
  ctx->sin_t = (float*)(W + o_sin);
  ctx->row_pos = (int32_t*)(W + o_rpos); ctx->row_seq = (int32_t*)(W + o_rseq);
  ctx->sample_scratch = (float*)(W + o_samp);
  if (Bm > 1) {
    ctx->mx_ybuf = (float*)(W + o_mxy);
    ctx->mx_part_val = (float*)(W + o_mxv);
    ctx->mx_part_idx = (int32_t*)(W + o_mxi);
    ctx->mx_route = (int32_t*)(W + o_mxr);
    ctx->mx_xp = (uint16_t*)(W + o_mxp);
    ctx->mx_ap = (uint16_t*)(W + o_mxa);
  }
  const char* fr_env = getenv("NEON_MX_FUSE_ROPE");
  ctx->mx_fuse_rope = !(fr_env && fr_env[0] == '0');
  // ---- RoPE table ----
  std::vector<float> ct, st;
  rope_table_host(&c, c.max_seq, ct, st);
  HIPCHK(ctx, hipMemcpy(ctx->cos_t, ct.data(), ct.size() * 4, hipMemcpyHostToDevice));
  HIPCHK(ctx, hipMemcpy(ctx->sin_t, st.data(), st.size() * 4, hipMemcpyHostToDevice));
  HIPCHK(ctx, hipDeviceSynchronize());
  HIPCHK(ctx, hipStreamCreateWithFlags(&ctx->cap_stream, hipStreamNonBlocking));
  HIPCHK(ctx, gemv_batched_prepare());
  return NEON_OK;
}

extern "C" neon_status neon_ctx_create(const neon_config* cfg, int device,
                                       neon_ctx** out) {
  g_create_error.clear();
  if (!cfg || !out) {
    g_create_error = "neon_ctx_create: null argument";
    return NEON_EINVAL;
  }
  *out = nullptr;
  if (const char* why = check_config(cfg)) {
    g_create_error = std::string("neon_ctx_create: ") + why;
    return NEON_EINVAL;
  }
  int ndev = 0;
  hipError_t e = hipGetDeviceCount(&ndev);
  if (e != hipSuccess || ndev < 1) {
    g_create_error = std::string("neon_ctx_create: no HIP device (") +
                     hipGetErrorString(e) + ")";
    return NEON_EHIP;
  }
  if (device < 0 || device >= ndev) {
    g_create_error = "neon_ctx_create: device index out of range";
    return NEON_EINVAL;
  }
  if (hipSetDevice(device) != hipSuccess) {
    g_create_error = "neon_ctx_create: hipSetDevice failed";
    return NEON_EHIP;
  }
  neon_ctx* ctx = new (std::nothrow) neon_ctx();
  if (!ctx) return NEON_ENOMEM;
  ctx->cfg = *cfg;
  ctx->device = device;
  neon_status st = ctx_alloc(ctx);
  if (st != NEON_OK) {
    g_create_error = "neon_ctx_create: " + ctx->err;
    neon_ctx_destroy(ctx);
    return st;
  }
  *out = ctx;
  return NEON_OK;
}

// ---------------------------------------------------------------------------
// weights
// ---------------------------------------------------------------------------
extern "C" neon_status neon_init_random(neon_ctx* ctx, uint64_t seed,
                                        void* stream) {
  if (!ctx) return NEON_EINVAL;
  HIPCHK(ctx, hipSetDevice(ctx->device));
  const neon_config& c = ctx->cfg;
  const Sizes sz = sizes_of(c);
  const size_t H = c.hidden, E = c.n_experts, I = c.intermediate;
  hipStream_t st = S(stream);
  // std of the Irwin-Hall integer (sum of four 16-bit uniforms)
  const double unit = std::sqrt((65536.0 * 65536.0 - 1.0) / 3.0);
  auto mul = [&](double std) { return (float)(std / unit); };
  auto bf = [&](uint16_t* p, size_t n, int layer, int kind, float mean, double std) {
    launch_fill_bf16(p, (int64_t)n, seed, stream_id(layer, kind), mean, mul(std), st);
  };
  bf(ctx->embed, sz.embed, -1, K_EMBED, 0.0f, 0.02);
  bf(ctx->lm_head, sz.embed, -1, K_LM_HEAD, 0.0f, 0.02);
  bf(ctx->final_norm, H, -1, K_FINAL_NORM, 1.0f, 0.05);
  for (int l = 0; l < c.n_layers; ++l) {
    LayerW& w = ctx->layers[l];
    bf(w.attn_norm, H, l, K_ATTN_NORM, 1.0f, 0.05);
    bf(w.wqkv, sz.wqkv, l, K_WQKV, 0.0f, 0.02);
    bf(w.bqkv, sz.qkv_rows, l, K_BQKV, 0.0f, 0.02);
    bf(w.wo, sz.wo, l, K_WO, 0.0f, 0.02);
    bf(w.bo, H, l, K_BO, 0.0f, 0.02);
    bf(w.sinks, c.n_heads, l, K_SINKS, 0.0f, 1.0);
    bf(w.mlp_norm, H, l, K_MLP_NORM, 1.0f, 0.05);
    bf(w.router_w, E * H, l, K_ROUTER_W, 0.0f, 0.02);
    bf(w.router_b, E, l, K_ROUTER_B, 0.0f, 0.02);
    bf(w.gu_bias, E * 2 * I, l, K_GU_BIAS, 0.0f, 0.02);
    bf(w.dn_bias, E * H, l, K_DN_BIAS, 0.0f, 0.02);
    launch_fill_bytes(w.gu_codes, (int64_t)sz.gu_codes, seed, stream_id(l, K_GU_CODES), st);
    launch_fill_scales(w.gu_scales, (int64_t)sz.gu_scales, seed, stream_id(l, K_GU_SCALES), 119, 6, st);
    launch_fill_bytes(w.dn_codes, (int64_t)sz.dn_codes, seed, stream_id(l, K_DN_CODES), st);
    launch_fill_scales(w.dn_scales, (int64_t)sz.dn_scales, seed, stream_id(l, K_DN_SCALES), 119, 6, st);
  }
  HIPCHK(ctx, hipGetLastError());
  ctx->weights_ready = true;
  ctx->mx_dirty = true;
  return NEON_OK;
}

// Resolve a gpt-oss checkpoint tensor name to (device pointer, bytes, is
// MXFP4 scale tensor, row offset inside a fused tensor).
static neon_status resolve(neon_ctx* ctx, const char* name, Tensor* t,
                           bool* is_scale) {
  const neon_config& c = ctx->cfg;
  const Sizes sz = sizes_of(c);
  const size_t H = c.hidden, E = c.n_experts, I = c.intermediate, D = c.head_dim;
  const size_t q_rows = (size_t)c.n_heads * D, kv_rows = (size_t)c.n_kv_heads * D;
  *is_scale = false;
  std::string n(name);
  if (n == "model.embed_tokens.weight") { *t = {ctx->embed, sz.embed * 2}; return NEON_OK; }
  if (n == "lm_head.weight") { *t = {ctx->lm_head, sz.embed * 2}; return NEON_OK; }
  if (n == "model.norm.weight") { *t = {ctx->final_norm, H * 2}; return NEON_OK; }
  int layer = -1, used = 0;
  if (sscanf(name, "model.layers.%d.%n", &layer, &used) != 1 || used == 0 ||
      layer < 0 || layer >= c.n_layers)
    FAIL(ctx, NEON_EINVAL, "unknown tensor name '%s'", name);
  const std::string r = n.substr(used);
  LayerW& w = ctx->layers[layer];
  if (r == "input_layernorm.weight") *t = {w.attn_norm, H * 2};
  else if (r == "post_attention_layernorm.weight") *t = {w.mlp_norm, H * 2};
  else if (r == "self_attn.q_proj.weight") *t = {w.wqkv, q_rows * H * 2};
  else if (r == "self_attn.k_proj.weight") *t = {w.wqkv + q_rows * H, kv_rows * H * 2};
  else if (r == "self_attn.v_proj.weight") *t = {w.wqkv + (q_rows + kv_rows) * H, kv_rows * H * 2};
  else if (r == "self_attn.q_proj.bias") *t = {w.bqkv, q_rows * 2};
  else if (r == "self_attn.k_proj.bias") *t = {w.bqkv + q_rows, kv_rows * 2};
  else if (r == "self_attn.v_proj.bias") *t = {w.bqkv + q_rows + kv_rows, kv_rows * 2};
  else if (r == "self_attn.o_proj.weight") *t = {w.wo, sz.wo * 2};
  else if (r == "self_attn.o_proj.bias") *t = {w.bo, H * 2};
  else if (r == "self_attn.sinks") *t = {w.sinks, (size_t)c.n_heads * 2};
  else if (r == "mlp.router.weight") *t = {w.router_w, E * H * 2};
  else if (r == "mlp.router.bias") *t = {w.router_b, E * 2};
  else if (r == "mlp.experts.gate_up_proj_blocks") *t = {w.gu_codes, sz.gu_codes};
  else if (r == "mlp.experts.gate_up_proj_scales") { *t = {w.gu_scales, sz.gu_scales}; *is_scale = true; }
  else if (r == "mlp.experts.gate_up_proj_bias") *t = {w.gu_bias, E * 2 * I * 2};
  else if (r == "mlp.experts.down_proj_blocks") *t = {w.dn_codes, sz.dn_codes};
  else if (r == "mlp.experts.down_proj_scales") { *t = {w.dn_scales, sz.dn_scales}; *is_scale = true; }
  else if (r == "mlp.experts.down_proj_bias") *t = {w.dn_bias, E * H * 2};
  else FAIL(ctx, NEON_EINVAL, "unknown tensor name '%s'", name);
  return NEON_OK;
}

extern "C" neon_status neon_load_tensor(neon_ctx* ctx, const char* name,
                                        const void* host_data, size_t bytes) {
  if (!ctx) return NEON_EINVAL;
  if (!name || !host_data) FAIL(ctx, NEON_EINVAL, "neon_load_tensor: null argument");
  Tensor t;
  bool is_scale;
  neon_status st = resolve(ctx, name, &t, &is_scale);
  if (st != NEON_OK) return st;
  if (bytes != t.bytes)
    FAIL(ctx, NEON_EINVAL, "tensor '%s': %zu bytes given, %zu expected", name, bytes, t.bytes);
  if (is_scale) {
    const uint8_t* s = (const uint8_t*)host_data;
    for (size_t i = 0; i < bytes; ++i)
      if (s[i] == 0xFF)
        FAIL(ctx, NEON_ENAN_SCALE, "tensor '%s': E8M0 scale 0xFF (NaN) at byte %zu", name, i);
  }
  HIPCHK(ctx, hipSetDevice(ctx->device));
  HIPCHK(ctx, hipMemcpy(t.ptr, host_data, bytes, hipMemcpyHostToDevice));
  ctx->weights_ready = true;
  ctx->mx_dirty = true;
  return NEON_OK;
}

extern "C" neon_status neon_tensor_ptr(neon_ctx* ctx, const char* name,
                                       void** ptr, size_t* bytes) {
  if (!ctx) return NEON_EINVAL;
  if (!name || !ptr) FAIL(ctx, NEON_EINVAL, "neon_tensor_ptr: null argument");
  Tensor t;
  bool is_scale;
  neon_status st = resolve(ctx, name, &t, &is_scale);
  if (st != NEON_OK) return st;
  *ptr = t.ptr;
  if (bytes) *bytes = t.bytes;
  return NEON_OK;
}

// ---------------------------------------------------------------------------
// the decode step: 1 + 6 L + 2 kernels, all reading positions from device
// memory so one captured graph serves every step.
// ---------------------------------------------------------------------------
// One projection of the step: the batch-1 kernel, or for B >= 2 the batched
// kernel that reads each weight row once for all rows (same bits).  Returns
// the grid width (the lm_head argmax partials per row).
static int launch_gemv_step(GemvArgs& a, int B, hipStream_t st) {
  if (B >= 2 && gemv_batched_supported(a)) {
    a.nblk = gemv_bt_grid(a.N, a.mode);
    (void)launch_gemv_bf16_batched(a, st);  // launch errors surface at hipGetLastError
    return a.nblk;
  }
  launch_gemv_bf16(a, st);
  return a.nblk;
}

// Rows 0 .. B-1 through embed and every layer: row b is token pos[b] of
// sequence seq[b] (seq NULL: sequence b), its k / v land at that sequence's
// cache row pos[b], and it attends to that sequence's keys up to pos[b].
static void enqueue_rows(neon_ctx* ctx, int B, const int32_t* pos, const int32_t* seq,
                         hipStream_t st) {
  const neon_config& c = ctx->cfg;
  const int H = c.hidden, D = c.head_dim;
  const int qkv_rows = (c.n_heads + 2 * c.n_kv_heads) * D;
  launch_embed(ctx->tokens, ctx->tok_stride, pos, seq, ctx->embed, ctx->h, H, B, st);
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerW& w = ctx->layers[l];
    const bool sliding = (l % 2 == 0) && c.sliding_window > 0;  // HFC:75-78
    uint16_t* kc_l = ctx->kc + ctx->kv_off[l];
    uint16_t* vc_l = ctx->vc + ctx->kv_off[l];
    // QKV projection; its epilogue rotates q and k (RoPE-YaRN table) and
    // appends k, v at cache row pos
    GemvArgs q;
    q.mode = 3; q.W = w.wqkv; q.bias = w.bqkv; q.x = ctx->h; q.norm_w = w.attn_norm;
    q.eps = c.rms_eps; q.y = ctx->qkv; q.N = qkv_rows; q.K = H; q.B = B;
    q.nblk = gemv_default_grid(q.N, q.mode);
    q.pos = pos; q.cos_t = ctx->cos_t; q.sin_t = ctx->sin_t; q.q_out = ctx->q_rot;
    q.kc = kc_l; q.vc = vc_l; q.seq = seq; q.Hq = c.n_heads; q.Hkv = c.n_kv_heads;
    q.T_max = ctx->kv_rows[l]; q.key_mask = ctx->kv_mask[l];
    launch_gemv_step(q, B, st);
    AttnArgs a;
    a.q = ctx->q_rot; a.kc = kc_l; a.vc = vc_l; a.sinks = w.sinks; a.pos = pos;
    a.out = ctx->attn_out; a.part_o = ctx->attn_po; a.part_ml = ctx->attn_pml; a.seq = seq;
    a.arrive = ctx->fuse_merge ? ctx->attn_arrive : nullptr;  // the last split block merges
    a.B = B; a.Hq = c.n_heads; a.Hkv = c.n_kv_heads;
    a.T_max = ctx->kv_rows[l]; a.key_mask = ctx->kv_mask[l];
    a.window = sliding ? c.sliding_window : 0;
    a.S = sliding ? ctx->s_slide : ctx->s_full; a.q_stride = c.n_heads * D;
    launch_attn(a, st);
    GemvArgs o;
    o.mode = 1; o.W = w.wo; o.bias = w.bo; o.x = ctx->attn_out; o.y = ctx->h;
    o.N = H; o.K = c.n_heads * D; o.B = B;
    o.nblk = gemv_default_grid(o.N, o.mode);
    // batch >= 2: the top-k runs once per row before the experts, which then
    // group the rows by expert (each used expert's weights read once);
    // batch 1: the expert kernels choose from the logits themselves
    const bool grouped = B >= 2 && B * c.top_k <= 64;
    RouterArgs r;
    r.x = ctx->h; r.norm_w = w.mlp_norm; r.eps = c.rms_eps; r.xn_out = ctx->xn;
    r.W = w.router_w; r.bias = w.router_b; r.lg_out = ctx->router_lg;
    r.idx = grouped ? ctx->moe_idx : nullptr; r.score = grouped ? ctx->moe_score : nullptr;
    r.B = B; r.E = c.n_experts; r.H = H; r.k = c.top_k;
    // batch 1: the experts run as one launch whose arrival counters the
    // router zeroes first
    int32_t* sync = B == 1 && ctx->fused_moe ? ctx->moe_sync + (size_t)l * kMoeSyncInts : nullptr;
    r.zero = sync; r.zero_n = sync ? kMoeSyncZero : 0;
    r.arrive = ctx->or_arrive; r.err = ctx->dev_err;
    if (ctx->fuse_router && o_router_supported(o, r)) {
      launch_gemv_o_router(o, r, st);  // batch 1: O, then the router in the same launch
    } else {
      launch_gemv_step(o, B, st);
      launch_router(r, st);
    }
    MoeArgs m;
    m.gu_codes = w.gu_codes; m.gu_scales = w.gu_scales; m.gu_bias = w.gu_bias;
    m.dn_codes = w.dn_codes; m.dn_scales = w.dn_scales; m.dn_bias = w.dn_bias;
    m.router_lg = grouped ? nullptr : ctx->router_lg;
    m.idx = grouped ? ctx->moe_idx : nullptr; m.score = grouped ? ctx->moe_score : nullptr;
    m.idx_out = grouped ? nullptr : ctx->moe_idx; m.score_out = grouped ? nullptr : ctx->moe_score;
    m.E = c.n_experts; m.xn = ctx->xn; m.act = ctx->act;
    m.residual = ctx->h; m.out = ctx->h; m.B = B; m.H = H; m.I = c.intermediate;
    m.k = c.top_k; m.alpha = c.swiglu_alpha; m.limit = c.swiglu_limit; m.err = ctx->dev_err;
    m.sync = sync;
    if (grouped && moe_batched_supported(m)) launch_moe_batched(m, st);
    else launch_moe(m, st);
  }
}

// The decode step: every sequence's row through the layers, then lm_head and
// the argmax that writes the next token and advances pos.
// B >= 2 rows of a decode step on the matrix cores: every weight row read
// once per step, the rows in the M dimension of the MFMA tiles.  Same
// kernels' maths and rounding points as enqueue_rows; only the order of the
// fp32 additions inside each dot product differs.
static void enqueue_rows_mx(neon_ctx* ctx, int B, hipStream_t st) {
  const neon_config& c = ctx->cfg;
  const int H = c.hidden, D = c.head_dim, I = c.intermediate;
  const int qkv_rows = (c.n_heads + 2 * c.n_kv_heads) * D;
  launch_embed(ctx->tokens, ctx->tok_stride, ctx->pos, nullptr, ctx->embed, ctx->h, H, B, st);
  bool normed = false;  // the previous layer's combine wrote this layer's packed norm
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerW& w = ctx->layers[l];
    const bool sliding = (l % 2 == 0) && c.sliding_window > 0;  // HFC:75-78
    uint16_t* kc_l = ctx->kc + ctx->kv_off[l];
    uint16_t* vc_l = ctx->vc + ctx->kv_off[l];
    // the normalised rows straight into the packed activation layout the
    // QKV kernel reads (1 KB contiguous per operand)
    const neon_ctx::MxLayer& mp = ctx->mxp[l];
    const bool xp = mp.wqkv != nullptr;
    if (xp) {
      if (!normed) launch_rmsnorm_packed(ctx->h, w.attn_norm, ctx->mx_xp, B, H, c.rms_eps, st);
    } else {
      launch_rmsnorm(ctx->h, w.attn_norm, ctx->xn, B, H, c.rms_eps, st);
    }
    MxArgs q{};
    q.W = w.wqkv; q.Wp = mp.wqkv; q.bias = w.bqkv; q.x = ctx->xn; q.xp = xp ? ctx->mx_xp : nullptr;
    q.y = ctx->qkv;
    q.B = B; q.N = qkv_rows; q.K = H;
    launch_mx_gemv(q, 0, st);
    // RoPE and the KV append inside the attention launch (NEON_MX_FUSE_ROPE=0:
    // a launch of their own before it; the same bits either way)
    if (!ctx->mx_fuse_rope)
      launch_mx_rope_append(ctx->qkv, ctx->pos, nullptr, ctx->cos_t, ctx->sin_t, ctx->q_rot, kc_l,
                            vc_l, B, c.n_heads, c.n_kv_heads, ctx->kv_rows[l], ctx->kv_mask[l],
                            st);
    AttnArgs a;
    a.q = ctx->mx_fuse_rope ? ctx->qkv : ctx->q_rot;
    a.kc = kc_l; a.vc = vc_l; a.sinks = w.sinks; a.pos = ctx->pos;
    a.out = ctx->attn_out; a.part_o = ctx->attn_po; a.part_ml = ctx->attn_pml; a.seq = nullptr;
    a.B = B; a.Hq = c.n_heads; a.Hkv = c.n_kv_heads;
    a.T_max = ctx->kv_rows[l]; a.key_mask = ctx->kv_mask[l];
    a.window = sliding ? c.sliding_window : 0;
    a.S = sliding ? ctx->s_slide : ctx->s_full;
    a.q_stride = ctx->mx_fuse_rope ? qkv_rows : c.n_heads * D;
    if (ctx->mx_fuse_rope) { a.rope_cos = ctx->cos_t; a.rope_sin = ctx->sin_t; }
    // the O projection reads a packed copy of the attention output (rows of
    // Hq D = a multiple of 128 columns, so no column padding)
    const bool ap = mp.wo != nullptr && (c.n_heads * D) % 128 == 0;
    a.out_packed = ap ? ctx->mx_ap : nullptr;
    launch_mx_attn(a, st);
    MxArgs o{};
    o.W = w.wo; o.Wp = mp.wo; o.bias = w.bo; o.x = ctx->attn_out; o.xp = a.out_packed;
    o.y = ctx->h;
    o.B = B; o.N = H; o.K = c.n_heads * D;
    launch_mx_gemv(o, 1, st);
    RouterArgs r;
    r.x = ctx->h; r.norm_w = w.mlp_norm; r.eps = c.rms_eps; r.xn_out = ctx->xn;
    r.W = w.router_w; r.bias = w.router_b; r.lg_out = ctx->router_lg;
    r.idx = nullptr; r.score = nullptr;  // per launch form, below
    r.B = B; r.E = c.n_experts; r.H = H; r.k = c.top_k;
    const bool mx8 = ctx->decode_mode == NEON_DECODE_MATRIX_MX8;
    // the MXFP8 images: xn [B][H] then the SwiGLU output [B k][I], each hi,
    // lo, then the two scale arrays
    uint8_t* q8 = ctx->mx8_q;
    const size_t nx = (size_t)c.max_batch * H, ny = (size_t)c.max_batch * c.top_k * I;
    size_t off = 0;  // every piece 256-byte aligned (16-byte loads and stores)
    auto take = [&](size_t bytes) { uint8_t* p = q8 + off; off = align_up(off + bytes); return p; };
    uint8_t *xh = take(nx), *xl = take(nx), *xsh = take(nx / 32), *xsl = take(nx / 32);
    uint8_t *yh = take(ny), *yl = take(ny), *ysh = take(ny / 32), *ysl = take(ny / 32);
    if (mx8) { r.xq_hi = xh; r.xq_lo = xl; r.xs_hi = xsh; r.xs_lo = xsl; }
    r.arrive = ctx->rr_arrive;
    // Measured at the 20b step after 16-token prompts (tok/s).  The table
    // built by the last block of a one-launch router against two launches:
    // B = 64 15,896 / 15,706, 48 12,585 / 12,584, 32 8899 / 9017, 16 4945 /
    // 5091 (the wait for the last row costs about the launch it saves).
    // Without a table, two launches / one launch / the earlier default (one
    // launch with the table from 49 rows, else two with it): B = 64 17,642 /
    // 17,331 / 17,067, 56 15,576 / 15,289, 48 13,464 / 13,199 / 13,049, 32
    // 9577 / 9388 / 9441, 16 5370 / 5206 / 5352 -- one block per row reads
    // every router row, so the one-launch router loses even without its wait.
    int32_t* table = ctx->route_table >= 0 ? ctx->mx_route : nullptr;
    const bool one = ctx->route_table == 1 || (ctx->route_table < 0 && ctx->route_one);
    if (one && router_route_supported(r)) {
      launch_router_route(r, ctx->moe_idx, ctx->moe_score, table, st);
    } else if (table != nullptr) {
      launch_router(r, st);
      launch_topk_route(ctx->router_lg, ctx->moe_idx, ctx->moe_score, B, c.n_experts, c.top_k,
                        table, st);
    } else {
      r.idx = ctx->moe_idx; r.score = ctx->moe_score;
      r.row_arrive = ctx->route_rank ? ctx->rl_arrive : nullptr;  // else a k_topk launch
      launch_router(r, st);
    }
    MxArgs gu{};
    gu.W = w.gu_codes; gu.scales = w.gu_scales; gu.Wp = mp.gu_c; gu.sp = mp.gu_s;
    gu.bias = w.gu_bias; gu.x = ctx->xn;
    gu.y = ctx->act; gu.idx = ctx->moe_idx; gu.route = table; gu.B = B; gu.N = 2 * I;
    gu.K = H;
    gu.E = c.n_experts; gu.k = c.top_k; gu.alpha = c.swiglu_alpha; gu.limit = c.swiglu_limit;
    gu.err = ctx->dev_err;
    MxArgs dn{};
    dn.W = w.dn_codes; dn.scales = w.dn_scales; dn.Wp = mp.dn_c; dn.sp = mp.dn_s;
    dn.bias = w.dn_bias; dn.x = ctx->act;
    dn.out_f = ctx->mx_ybuf; dn.idx = ctx->moe_idx; dn.route = table; dn.B = B;
    dn.N = H; dn.K = I;
    dn.E = c.n_experts; dn.k = c.top_k; dn.err = ctx->dev_err;
    // the norm that reads this layer's output, when it goes to the packed layout
    const uint16_t* next_norm = nullptr;
    if (ctx->mx_combine_norm) {
      if (l + 1 < c.n_layers) next_norm = ctx->mxp[l + 1].wqkv ? ctx->layers[l + 1].attn_norm : nullptr;
      else next_norm = ctx->mx_lm ? ctx->final_norm : nullptr;
    }
    if (mx8) {
      gu.xq_hi = xh; gu.xq_lo = xl; gu.xs_hi = xsh; gu.xs_lo = xsl;
      gu.yq_hi = yh; gu.yq_lo = yl; gu.ys_hi = ysh; gu.ys_lo = ysl;
      normed = launch_mx_moe8(gu, dn, ctx->moe_score, ctx->h, st, next_norm, c.rms_eps, ctx->mx_xp);
    } else {
      normed = launch_mx_moe(gu, dn, ctx->moe_score, ctx->h, st, next_norm, c.rms_eps, ctx->mx_xp);
    }
  }
  const bool lxp = ctx->mx_lm != nullptr;
  if (lxp) {
    if (!normed) launch_rmsnorm_packed(ctx->h, ctx->final_norm, ctx->mx_xp, B, H, c.rms_eps, st);
  } else {
    launch_rmsnorm(ctx->h, ctx->final_norm, ctx->xn, B, H, c.rms_eps, st);
  }
  MxArgs lm{};
  lm.W = ctx->lm_head; lm.Wp = ctx->mx_lm; lm.x = ctx->xn; lm.xp = lxp ? ctx->mx_xp : nullptr;
  lm.out_f = ctx->logits;
  lm.part_val = ctx->mx_part_val; lm.part_idx = ctx->mx_part_idx;
  lm.B = B; lm.N = c.vocab; lm.K = H;
  launch_mx_gemv(lm, 2, st);
}

static void enqueue_step(neon_ctx* ctx, int B, hipStream_t st) {
  if ((ctx->decode_mode == NEON_DECODE_MATRIX || ctx->decode_mode == NEON_DECODE_MATRIX_MX8) &&
      B >= 2) {
    const neon_config& c = ctx->cfg;
    enqueue_rows_mx(ctx, B, st);
    if (ctx->temperature > 0.0f)
      launch_sample(ctx->logits, B, c.vocab, ctx->temperature, ctx->top_p, ctx->sample_seed,
                    ctx->pos, ctx->sample_scratch, ctx->last_ids, ctx->tokens, ctx->tok_stride,
                    ctx->prompt_len, true, st);
    else
      launch_argmax_advance(ctx->mx_part_val, ctx->mx_part_idx, c.vocab / 16, ctx->tokens,
                            ctx->tok_stride, ctx->pos, ctx->prompt_len, ctx->last_ids, B, st);
    return;
  }
  const neon_config& c = ctx->cfg;
  const int H = c.hidden;
  enqueue_rows(ctx, B, ctx->pos, nullptr, st);
  GemvArgs lm;
  lm.mode = 2; lm.W = ctx->lm_head; lm.x = ctx->h; lm.norm_w = ctx->final_norm;
  lm.eps = c.rms_eps; lm.logits = ctx->logits; lm.part_val = ctx->lm_part_val;
  lm.part_idx = ctx->lm_part_idx; lm.N = c.vocab; lm.K = H; lm.B = B;
  lm.nblk = ctx->lm_nblk;
  const int lm_parts = launch_gemv_step(lm, B, st);
  if (ctx->temperature > 0.0f)
    launch_sample(ctx->logits, B, c.vocab, ctx->temperature, ctx->top_p, ctx->sample_seed,
                  ctx->pos, ctx->sample_scratch, ctx->last_ids, ctx->tokens, ctx->tok_stride,
                  ctx->prompt_len, true, st);
  else
    launch_argmax_advance(ctx->lm_part_val, ctx->lm_part_idx, lm_parts,
                          ctx->tokens, ctx->tok_stride, ctx->pos, ctx->prompt_len,
                          ctx->last_ids, B, st);
}

static neon_status ensure_graph(neon_ctx* ctx, int B) {
  if (ctx->graph_exec && ctx->graph_batch == B) return NEON_OK;
  if (ctx->graph_exec) { (void)hipGraphExecDestroy(ctx->graph_exec); ctx->graph_exec = nullptr; }
  if (ctx->graph) { (void)hipGraphDestroy(ctx->graph); ctx->graph = nullptr; }
  HIPCHK(ctx, hipStreamBeginCapture(ctx->cap_stream, hipStreamCaptureModeThreadLocal));
  enqueue_step(ctx, B, ctx->cap_stream);
  hipError_t le = hipGetLastError();
  hipGraph_t g = nullptr;
  hipError_t ee = hipStreamEndCapture(ctx->cap_stream, &g);
  if (le != hipSuccess || ee != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    FAIL(ctx, NEON_EHIP, "graph capture failed: %s / %s", hipGetErrorString(le),
         hipGetErrorString(ee));
  }
  ctx->graph = g;
  HIPCHK(ctx, hipGraphInstantiate(&ctx->graph_exec, g, nullptr, nullptr, 0));
  ctx->graph_batch = B;
  return NEON_OK;
}

// Packs every weight the matrix-core steps read into MFMA lane order (stream
// ordered, before the step that needs it; never inside a captured graph).
static void mx_repack(neon_ctx* ctx, hipStream_t st) {
  const neon_config& c = ctx->cfg;
  const int H = c.hidden, I = c.intermediate, E = c.n_experts;
  const int qkv_rows = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim;
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerW& w = ctx->layers[l];
    const neon_ctx::MxLayer& m = ctx->mxp[l];
    launch_mx_pack_bf16(w.wqkv, qkv_rows, H, m.wqkv, st);
    launch_mx_pack_bf16(w.wo, H, c.n_heads * c.head_dim, m.wo, st);
    launch_mx_pack_fp4(w.gu_codes, w.gu_scales, E, 2 * I, H, m.gu_c, m.gu_s, st);
    launch_mx_pack_fp4(w.dn_codes, w.dn_scales, E, H, I, m.dn_c, m.dn_s, st);
  }
  launch_mx_pack_bf16(ctx->lm_head, c.vocab, H, ctx->mx_lm, st);
}

static neon_status run_steps(neon_ctx* ctx, int n, hipStream_t st) {
  if ((ctx->decode_mode == NEON_DECODE_MATRIX || ctx->decode_mode == NEON_DECODE_MATRIX_MX8) &&
      ctx->batch >= 2 && ctx->mx_dirty) {
    mx_repack(ctx, st);
    HIPCHK(ctx, hipGetLastError());
    ctx->mx_dirty = false;
  }
  // NEON_EAGER=1 launches the kernels directly (debugging aid); the default
  // replays the captured step graph.
  static const bool eager = getenv("NEON_EAGER") && getenv("NEON_EAGER")[0] == '1';
  if (eager) {
    for (int i = 0; i < n; ++i) enqueue_step(ctx, ctx->batch, st);
    HIPCHK(ctx, hipGetLastError());
    return NEON_OK;
  }
  neon_status s = ensure_graph(ctx, ctx->batch);
  if (s != NEON_OK) return s;
  for (int i = 0; i < n; ++i) HIPCHK(ctx, hipGraphLaunch(ctx->graph_exec, st));
  return NEON_OK;
}

// ---------------------------------------------------------------------------
// batched prefill: all prompt rows of one sequence through every layer at
// once (matrix-core GEMMs, grouped expert GEMMs, tiled causal attention),
// filling that sequence's KV cache.  Scratch is sized for `rows` rows.
// ---------------------------------------------------------------------------
static neon_status ensure_prefill_scratch(neon_ctx* ctx, int rows, hipStream_t st) {
  if (ctx->pf && ctx->pf_rows >= rows) return NEON_OK;
  const neon_config& c = ctx->cfg;
  const size_t M = (size_t)((rows + 127) / 128) * 128;
  const size_t H = c.hidden, I = c.intermediate, k = c.top_k, E = c.n_experts;
  const size_t qkv_rows = (size_t)(c.n_heads + 2 * c.n_kv_heads) * c.head_dim;
  const size_t qd = (size_t)c.n_heads * c.head_dim;
  const size_t tiles = (size_t)moe_prefill_max_tiles((int)M, (int)k, (int)E);
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes); return o; };
  const size_t o_h = take(M * H * 2), o_xn = take(M * H * 2), o_qkv = take(M * qkv_rows * 2),
               o_q = take(M * qd * 2), o_ao = take(M * qd * 2), o_act = take(M * k * I * 2),
               o_lg = take(M * E * 4), o_sc = take(M * k * 4), o_yb = take(M * k * H * 4),
               o_idx = take(M * k * 4), o_lt = take(M * k * 4), o_ls = take(M * k * 4),
               o_eo = take((E + 1) * 4), o_te = take(tiles * 4), o_tr = take(tiles * 4),
               o_nt = take(4), o_ks = take(M * c.n_kv_heads * c.head_dim * 2),
               o_vs = take(M * c.n_kv_heads * c.head_dim * 2);
  // MXFP8 images of the expert GEMM inputs (NEON_PREFILL_MX8): xn rows, then
  // the act rows, in the same buffers
  const size_t qn = std::max(M * H, M * k * I);
  const size_t o_mxq = take(2 * qn),
               o_mxqs = take(std::max(mx8_scale_bytes(M, H), mx8_scale_bytes(M * k, I)));
  if (ctx->pf) {
    HIPCHK(ctx, hipStreamSynchronize(st));  // earlier prefill work may still read it
    (void)hipFree(ctx->pf);
    ctx->pf = nullptr;
    ctx->pf_rows = 0;
  }
  if (hipMalloc(&ctx->pf, off) != hipSuccess) {
    ctx->pf = nullptr;
    FAIL(ctx, NEON_ENOMEM, "hipMalloc of %zu prefill scratch bytes failed", off);
  }
  char* P = ctx->pf;
  ctx->pf_h = (uint16_t*)(P + o_h); ctx->pf_xn = (uint16_t*)(P + o_xn);
  ctx->pf_qkv = (uint16_t*)(P + o_qkv); ctx->pf_q = (uint16_t*)(P + o_q);
  ctx->pf_ao = (uint16_t*)(P + o_ao); ctx->pf_act = (uint16_t*)(P + o_act);
  ctx->pf_lg = (float*)(P + o_lg); ctx->pf_score = (float*)(P + o_sc);
  ctx->pf_ybuf = (float*)(P + o_yb); ctx->pf_idx = (int32_t*)(P + o_idx);
  ctx->pf_ltok = (int32_t*)(P + o_lt); ctx->pf_lslot = (int32_t*)(P + o_ls);
  ctx->pf_eoff = (int32_t*)(P + o_eo); ctx->pf_tile_e = (int32_t*)(P + o_te);
  ctx->pf_tile_r0 = (int32_t*)(P + o_tr); ctx->pf_ntiles = (int32_t*)(P + o_nt);
  ctx->pf_ks = (uint16_t*)(P + o_ks); ctx->pf_vs = (uint16_t*)(P + o_vs);
  ctx->pf_mxq = (uint8_t*)(P + o_mxq); ctx->pf_mxqs = (uint32_t*)(P + o_mxqs);
  ctx->pf_rows = (int)M;
  return NEON_OK;
}

// Rows 0 .. M-1 of sequence b (token ids already in ctx->tokens) through all
// layers; their keys/values land in the KV cache.  The hidden states of these
// rows are not needed afterwards (the last prompt token runs as a decode step).
// A sliding layer with a ring cache (fewer rows than positions) gets its keys
// and values staged for all M rows first, so that the prompt attention sees
// every row; only the last rows that fit its ring are then stored in it.
static void enqueue_prefill_rows(neon_ctx* ctx, int b, int M, hipStream_t st) {
  const neon_config& c = ctx->cfg;
  const int H = c.hidden, D = c.head_dim, Hq = c.n_heads, Hkv = c.n_kv_heads;
  const int qkv_rows = (Hq + 2 * Hkv) * D;
  launch_embed_rows(ctx->tokens + (size_t)b * ctx->tok_stride, M, ctx->embed, ctx->pf_h, H, st);
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerW& w = ctx->layers[l];
    const bool sliding = (l % 2 == 0) && c.sliding_window > 0;  // HFC:75-78
    const size_t kvo = ctx->kv_off[l] + (size_t)b * Hkv * ctx->kv_rows[l] * D;
    const bool ring = ctx->kv_mask[l] >= 0;
    uint16_t* kd = ring ? ctx->pf_ks : ctx->kc + kvo;
    uint16_t* vd = ring ? ctx->pf_vs : ctx->vc + kvo;
    const int Td = ring ? ctx->pf_rows : ctx->kv_rows[l];
    launch_rmsnorm(ctx->pf_h, w.attn_norm, ctx->pf_xn, M, H, c.rms_eps, st);
    launch_prompt_proj(ctx->pf_xn, w.wqkv, w.bqkv, ctx->pf_qkv, M, qkv_rows, H, 0, st);
    launch_rope_kv_rows(ctx->pf_qkv, qkv_rows, ctx->cos_t, ctx->sin_t, M, Hq, Hkv, Td,
                        ctx->pf_q, kd, vd, st);
    launch_attn_prefill(ctx->pf_q, kd, vd, w.sinks, ctx->pf_ao, M, Hq, Hkv, Td,
                        sliding ? c.sliding_window : 0, st);
    if (ring)
      launch_kv_ring_store(ctx->pf_ks, ctx->pf_vs, Td, std::max(0, M - ctx->kv_rows[l]), M,
                           Hkv, ctx->kv_rows[l], ctx->kc + kvo, ctx->vc + kvo, st);
    launch_prompt_proj(ctx->pf_ao, w.wo, w.bo, ctx->pf_h, M, H, Hq * D, 1, st);
    launch_rmsnorm(ctx->pf_h, w.mlp_norm, ctx->pf_xn, M, H, c.rms_eps, st);
    launch_gemm_bf16(ctx->pf_xn, H, w.router_w, H, w.router_b, nullptr, ctx->pf_lg,
                     c.n_experts, M, c.n_experts, H, 2, st);
    launch_topk(ctx->pf_lg, ctx->pf_idx, ctx->pf_score, M, c.n_experts, c.top_k, st);
    MoePrefillArgs m;
    m.idx = ctx->pf_idx; m.score = ctx->pf_score; m.xn = ctx->pf_xn; m.h = ctx->pf_h;
    m.gu_codes = w.gu_codes; m.gu_scales = w.gu_scales; m.gu_bias = w.gu_bias;
    m.dn_codes = w.dn_codes; m.dn_scales = w.dn_scales; m.dn_bias = w.dn_bias;
    m.M = M; m.E = c.n_experts; m.H = H; m.I = c.intermediate; m.k = c.top_k;
    m.alpha = c.swiglu_alpha; m.limit = c.swiglu_limit;
    m.list_tok = ctx->pf_ltok; m.list_slot = ctx->pf_lslot; m.e_off = ctx->pf_eoff;
    m.tile_e = ctx->pf_tile_e; m.tile_r0 = ctx->pf_tile_r0; m.n_tiles = ctx->pf_ntiles;
    m.act = ctx->pf_act; m.ybuf = ctx->pf_ybuf; m.err = ctx->dev_err;
    if (ctx->prefill_mode == NEON_PREFILL_MX8) {
      m.q = ctx->pf_mxq; m.qs = ctx->pf_mxqs;
    }
    launch_moe_prefill(m, st);
  }
}

// The batched prompt pass (matrix-core GEMMs, grouped experts, tiled prompt
// attention).  Kept behind one switch so that it can be refused as a whole.
static const bool kBatchedPrefillEnabled = true;

extern "C" neon_status neon_set_prefill_mode(neon_ctx* ctx, int mode) {
  if (!ctx) return NEON_EINVAL;
  if (mode != NEON_PREFILL_BATCHED && mode != NEON_PREFILL_STEPWISE &&
      mode != NEON_PREFILL_CHUNKED && mode != NEON_PREFILL_MX8)
    FAIL(ctx, NEON_EINVAL, "neon_set_prefill_mode: unknown mode %d", mode);
  if ((mode == NEON_PREFILL_BATCHED || mode == NEON_PREFILL_MX8) && !kBatchedPrefillEnabled)
    FAIL(ctx, NEON_ESTATE, "neon_set_prefill_mode: the batched prompt pass is switched off");
  ctx->prefill_mode = mode;
  return NEON_OK;
}

// The prompt pass shared by neon_prefill and neon_prefill_ragged: sequence
// b's prompt is ids[start[b] .. start[b] + lens[b]).  Each sequence keeps its
// own position: rows 0 .. lens[b]-2 fill its KV cache, then one decode step
// at position lens[b]-1 (every sequence at its own) gives each its first
// generated token.
static neon_status prefill_seqs(neon_ctx* ctx, const int32_t* ids, const int32_t* lens,
                                int batch, hipStream_t st, const char* fn) {
  const neon_config& c = ctx->cfg;
  if (!ids || !lens) FAIL(ctx, NEON_EINVAL, "%s: null ids or lengths", fn);
  if (batch < 1 || batch > c.max_batch)
    FAIL(ctx, NEON_EINVAL, "%s: batch %d outside [1, %d]", fn, batch, c.max_batch);
  std::vector<int64_t> start(batch + 1, 0);
  int max_len = 0;
  bool equal = true;
  for (int b = 0; b < batch; ++b) {
    if (lens[b] < 1) FAIL(ctx, NEON_EINVAL, "%s: sequence %d has %d tokens; need >= 1", fn, b, lens[b]);
    if (lens[b] > c.max_seq)
      FAIL(ctx, NEON_EKV_FULL, "%s: %d tokens of sequence %d exceed max_seq %d", fn, lens[b], b,
           c.max_seq);
    start[b + 1] = start[b] + lens[b];
    max_len = std::max(max_len, lens[b]);
    equal = equal && lens[b] == lens[0];
  }
  for (int64_t i = 0; i < start[batch]; ++i)
    if (ids[i] < 0 || ids[i] >= c.vocab)
      FAIL(ctx, NEON_ERANGE_TOKEN, "%s: token id %d at %lld outside [0, %d)", fn, ids[i],
           (long long)i, c.vocab);
  if (!ctx->weights_ready) FAIL(ctx, NEON_ESTATE, "%s: no weights loaded", fn);
  HIPCHK(ctx, hipSetDevice(ctx->device));
  std::vector<int32_t> tok((size_t)batch * ctx->tok_stride, 0);
  for (int b = 0; b < batch; ++b)
    memcpy(&tok[(size_t)b * ctx->tok_stride], ids + start[b], (size_t)lens[b] * 4);
  std::vector<int32_t> zeros(batch, 0), plen(lens, lens + batch);
  HIPCHK(ctx, hipMemcpyAsync(ctx->tokens, tok.data(), tok.size() * 4, hipMemcpyHostToDevice, st));
  HIPCHK(ctx, hipMemcpyAsync(ctx->pos, zeros.data(), batch * 4, hipMemcpyHostToDevice, st));
  HIPCHK(ctx, hipMemcpyAsync(ctx->prompt_len, plen.data(), batch * 4, hipMemcpyHostToDevice, st));
  HIPCHK(ctx, hipStreamSynchronize(st));  // host staging buffers die here
  ctx->batch = batch;
  ctx->host_pos = 0;
  ctx->host_plen.assign(c.max_batch, 0);
  std::copy(lens, lens + batch, ctx->host_plen.begin());
  ctx->host_seq_pos.assign(c.max_batch, 0);
  ctx->host_active.assign(c.max_batch, 0);
  for (int b = 0; b < batch; ++b) { ctx->host_seq_pos[b] = lens[b]; ctx->host_active[b] = 1; }
  if (max_len == 1 || (ctx->prefill_mode == NEON_PREFILL_STEPWISE && equal)) {
    // every prompt token as a decode step of all sequences together
    neon_status s = run_steps(ctx, max_len, st);
    if (s != NEON_OK) return s;
    ctx->host_pos = max_len;
    return NEON_OK;
  }
  if (ctx->prefill_mode == NEON_PREFILL_BATCHED || ctx->prefill_mode == NEON_PREFILL_MX8) {
    // each sequence's rows 0 .. n-2 in one matrix-core pass
    neon_status s = ensure_prefill_scratch(ctx, max_len - 1, st);
    if (s != NEON_OK) return s;
    for (int b = 0; b < batch; ++b)
      if (lens[b] > 1) enqueue_prefill_rows(ctx, b, lens[b] - 1, st);
  } else {
    // NEON_PREFILL_CHUNKED: the (position, sequence) rows of all sequences,
    // each sequence's in position order, kPromptRows at a time through the
    // batched decode kernels (their k / v fill the cache before the pass's
    // attention, so row p attends to its sequence's keys <= p).
    // NEON_PREFILL_STEPWISE with different lengths: the same rows one at a
    // time.  The rows are staged up front and stay alive until the stream is
    // synchronised below.
    const int per = ctx->prefill_mode == NEON_PREFILL_STEPWISE ? 1 : kPromptRows;
    std::vector<int32_t> rp, rs;
    for (int b = 0; b < batch; ++b)
      for (int p = 0; p + 1 < lens[b]; ++p) { rp.push_back(p); rs.push_back(b); }
    const size_t n_rows = rp.size();
    for (size_t r0 = 0; r0 < n_rows; r0 += per) {
      const int R = (int)std::min<size_t>(per, n_rows - r0);
      HIPCHK(ctx, hipMemcpyAsync(ctx->row_pos, &rp[r0], R * 4, hipMemcpyHostToDevice, st));
      HIPCHK(ctx, hipMemcpyAsync(ctx->row_seq, &rs[r0], R * 4, hipMemcpyHostToDevice, st));
      enqueue_rows(ctx, R, ctx->row_pos, ctx->row_seq, st);
    }
    HIPCHK(ctx, hipStreamSynchronize(st));  // rp and rs die here
  }
  HIPCHK(ctx, hipGetLastError());
  std::vector<int32_t> pm(batch);
  for (int b = 0; b < batch; ++b) pm[b] = lens[b] - 1;
  HIPCHK(ctx, hipMemcpyAsync(ctx->pos, pm.data(), batch * 4, hipMemcpyHostToDevice, st));
  HIPCHK(ctx, hipStreamSynchronize(st));  // pm dies here
  neon_status s = run_steps(ctx, 1, st);
  if (s != NEON_OK) return s;
  ctx->host_pos = max_len;
  return NEON_OK;
}

extern "C" neon_status neon_prefill(neon_ctx* ctx, const int32_t* ids, int batch,
                                    int n_tokens, void* stream) {
  if (!ctx) return NEON_EINVAL;
  if (n_tokens < 1) FAIL(ctx, NEON_EINVAL, "neon_prefill: n_tokens must be >= 1");
  if (batch < 1 || batch > ctx->cfg.max_batch)
    FAIL(ctx, NEON_EINVAL, "neon_prefill: batch %d outside [1, %d]", batch, ctx->cfg.max_batch);
  const std::vector<int32_t> lens(batch, n_tokens);
  return prefill_seqs(ctx, ids, lens.data(), batch, S(stream), "neon_prefill");
}

extern "C" neon_status neon_prefill_ragged(neon_ctx* ctx, const int32_t* ids,
                                           const int32_t* lens, int batch, void* stream) {
  if (!ctx) return NEON_EINVAL;
  return prefill_seqs(ctx, ids, lens, batch, S(stream), "neon_prefill_ragged");
}

extern "C" neon_status neon_set_decode_mode(neon_ctx* ctx, int mode) {
  if (!ctx) return NEON_EINVAL;
  if (mode != NEON_DECODE_EXACT && mode != NEON_DECODE_MATRIX && mode != NEON_DECODE_MATRIX_MX8)
    FAIL(ctx, NEON_EINVAL, "neon_set_decode_mode: unknown mode %d", mode);
  const bool matrix = mode == NEON_DECODE_MATRIX || mode == NEON_DECODE_MATRIX_MX8;
  if (matrix) {
    const neon_config& c = ctx->cfg;
    const int H = c.hidden, qkv_rows = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim;
    if (c.max_batch < 2 || c.max_batch > kMxMaxRows)
      FAIL(ctx, NEON_EINVAL, "neon_set_decode_mode: the matrix-core steps need max_batch in "
                             "[2, %d], not %d", kMxMaxRows, c.max_batch);
    if (!mx_shape_ok(qkv_rows, H, c.max_batch) || !mx_shape_ok(H, c.n_heads * c.head_dim, 2) ||
        !mx_shape_ok(c.vocab, H, 2) ||
        !mx_moe_shape_ok(H, c.intermediate, c.n_experts, c.top_k, c.max_batch))
      FAIL(ctx, NEON_EINVAL, "neon_set_decode_mode: the matrix-core steps need every output "
                             "width a multiple of 16 (expert widths of 64), every reduction "
                             "a multiple of 32 up to %d and max_batch * top_k <= 256", kMxMaxK);
  }
  if (mode == NEON_DECODE_MATRIX_MX8 && !ctx->mx8_q) {
    const neon_config& c = ctx->cfg;
    const size_t Bm = c.max_batch;
    const size_t nx = Bm * c.hidden, ny = Bm * c.top_k * c.intermediate;
    HIPCHK(ctx, hipSetDevice(ctx->device));
    const size_t bytes = align_up(nx) * 2 + align_up(nx / 32) * 2 + align_up(ny) * 2 +
                         align_up(ny / 32) * 2;
    if (hipMalloc(&ctx->mx8_q, bytes) != hipSuccess) {
      ctx->mx8_q = nullptr;
      FAIL(ctx, NEON_ENOMEM, "neon_set_decode_mode: hipMalloc of the MXFP8 buffers failed");
    }
  }
  if (matrix && !ctx->mx_w) {
    const neon_config& c = ctx->cfg;
    const int H = c.hidden, I = c.intermediate, E = c.n_experts;
    const int qkv_rows = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim;
    const size_t b_qkv = mx_packed_bf16_bytes(qkv_rows, H);
    const size_t b_o = mx_packed_bf16_bytes(H, c.n_heads * c.head_dim);
    const size_t p_gu = mx_packed_fp4_pieces(E, 2 * I, H), p_dn = mx_packed_fp4_pieces(E, H, I);
    size_t off = 0;
    auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes); return o; };
    std::vector<size_t> o(6 * c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
      o[6 * l + 0] = take(b_qkv); o[6 * l + 1] = take(b_o);
      o[6 * l + 2] = take(p_gu * 16); o[6 * l + 3] = take(p_gu);
      o[6 * l + 4] = take(p_dn * 16); o[6 * l + 5] = take(p_dn);
    }
    const size_t o_lm = take(mx_packed_bf16_bytes(c.vocab, H));
    HIPCHK(ctx, hipSetDevice(ctx->device));
    if (hipMalloc(&ctx->mx_w, off) != hipSuccess) {
      ctx->mx_w = nullptr;
      FAIL(ctx, NEON_ENOMEM, "neon_set_decode_mode: hipMalloc of %zu bytes for the matrix-core "
                             "weight copies failed", off);
    }
    ctx->mxp.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
      neon_ctx::MxLayer& m = ctx->mxp[l];
      m.wqkv = (uint16_t*)(ctx->mx_w + o[6 * l + 0]); m.wo = (uint16_t*)(ctx->mx_w + o[6 * l + 1]);
      m.gu_c = (uint8_t*)(ctx->mx_w + o[6 * l + 2]); m.gu_s = (uint8_t*)(ctx->mx_w + o[6 * l + 3]);
      m.dn_c = (uint8_t*)(ctx->mx_w + o[6 * l + 4]); m.dn_s = (uint8_t*)(ctx->mx_w + o[6 * l + 5]);
    }
    ctx->mx_lm = (uint16_t*)(ctx->mx_w + o_lm);
    ctx->mx_dirty = true;
  }
  ctx->decode_mode = mode;
  // the captured step holds the step's kernels
  HIPCHK(ctx, hipSetDevice(ctx->device));
  HIPCHK(ctx, hipDeviceSynchronize());
  if (ctx->graph_exec) { (void)hipGraphExecDestroy(ctx->graph_exec); ctx->graph_exec = nullptr; }
  if (ctx->graph) { (void)hipGraphDestroy(ctx->graph); ctx->graph = nullptr; }
  ctx->graph_batch = 0;
  return NEON_OK;
}

extern "C" neon_status neon_set_sampling(neon_ctx* ctx, float temperature, float top_p,
                                         uint64_t seed) {
  if (!ctx) return NEON_EINVAL;
  if (!(temperature >= 0.0f) || !(top_p > 0.0f && top_p <= 1.0f) ||
      !(temperature < 3.0e38f))
    FAIL(ctx, NEON_EINVAL, "neon_set_sampling: temperature %g must be >= 0 and finite, "
                           "top_p %g in (0, 1]", temperature, top_p);
  ctx->temperature = temperature;
  ctx->top_p = top_p;
  ctx->sample_seed = seed;
  // the captured step holds the choice kernel and its arguments
  HIPCHK(ctx, hipSetDevice(ctx->device));
  HIPCHK(ctx, hipDeviceSynchronize());
  if (ctx->graph_exec) { (void)hipGraphExecDestroy(ctx->graph_exec); ctx->graph_exec = nullptr; }
  if (ctx->graph) { (void)hipGraphDestroy(ctx->graph); ctx->graph = nullptr; }
  ctx->graph_batch = 0;
  return NEON_OK;
}

extern "C" neon_status neon_decode(neon_ctx* ctx, int n_steps, void* stream) {
  if (!ctx) return NEON_EINVAL;
  if (n_steps < 0) FAIL(ctx, NEON_EINVAL, "neon_decode: n_steps must be >= 0");
  if (ctx->batch == 0) FAIL(ctx, NEON_ESTATE, "neon_decode: call neon_prefill first");
  int longest = 0;  // the longest sequence held (free rows do not advance)
  for (int b = 0; b < ctx->batch; ++b)
    if (ctx->host_active[b]) longest = std::max(longest, ctx->host_seq_pos[b]);
  if ((int64_t)longest + n_steps > ctx->cfg.max_seq)
    FAIL(ctx, NEON_EKV_FULL, "neon_decode: %d steps from position %d exceed max_seq %d",
         n_steps, longest, ctx->cfg.max_seq);
  HIPCHK(ctx, hipSetDevice(ctx->device));
  neon_status s = run_steps(ctx, n_steps, S(stream));
  if (s != NEON_OK) return s;
  for (int b = 0; b < ctx->batch; ++b)
    if (ctx->host_active[b]) ctx->host_seq_pos[b] += n_steps;
  ctx->host_pos = std::max(ctx->host_pos, longest + n_steps);
  return NEON_OK;
}

// After a synchronisation: the status bits the context's kernels set since
// the last check (read and cleared).
static neon_status check_dev_err(neon_ctx* ctx) {
  int32_t bits = 0;
  HIPCHK(ctx, hipMemcpy(&bits, ctx->dev_err, 4, hipMemcpyDeviceToHost));
  if (bits == 0) return NEON_OK;
  HIPCHK(ctx, hipMemset(ctx->dev_err, 0, 4));
  if (bits & kDevErrSyncTimeout)
    FAIL(ctx, NEON_EHIP, "a grid-wide wait inside a kernel timed out (status bits 0x%x); "
         "the step's results are invalid", bits);
  FAIL(ctx, NEON_EINVAL, "a kernel of this context saw an expert id outside [0, %d) "
       "(status bits 0x%x); that slot was dropped", ctx->cfg.n_experts, bits);
}

extern "C" neon_status neon_read_tokens(neon_ctx* ctx, int start, int count,
                                        int32_t* out, void* stream) {
  if (!ctx) return NEON_EINVAL;
  if (!out || start < 0 || count < 0 || start + count > ctx->host_pos + 1)
    FAIL(ctx, NEON_EINVAL, "neon_read_tokens: range [%d, %d) outside [0, %d]", start,
         start + count, ctx->host_pos + 1);
  HIPCHK(ctx, hipSetDevice(ctx->device));
  HIPCHK(ctx, hipStreamSynchronize(S(stream)));
  for (int b = 0; b < ctx->batch; ++b)
    HIPCHK(ctx, hipMemcpy(out + (size_t)b * count,
                          ctx->tokens + (size_t)b * ctx->tok_stride + start,
                          (size_t)count * 4, hipMemcpyDeviceToHost));
  return check_dev_err(ctx);
}

extern "C" neon_status neon_read_logits(neon_ctx* ctx, float* out, void* stream) {
  if (!ctx) return NEON_EINVAL;
  if (!out) FAIL(ctx, NEON_EINVAL, "neon_read_logits: null out");
  if (ctx->batch == 0) FAIL(ctx, NEON_ESTATE, "neon_read_logits: no step has run");
  HIPCHK(ctx, hipSetDevice(ctx->device));
  HIPCHK(ctx, hipStreamSynchronize(S(stream)));
  HIPCHK(ctx, hipMemcpy(out, ctx->logits, (size_t)ctx->batch * ctx->cfg.vocab * 4,
                        hipMemcpyDeviceToHost));
  return check_dev_err(ctx);
}

extern "C" neon_status neon_read_activation(neon_ctx* ctx, const char* name,
                                            void* out, size_t bytes, void* stream) {
  if (!ctx) return NEON_EINVAL;
  if (!name || !out) FAIL(ctx, NEON_EINVAL, "neon_read_activation: null argument");
  if (ctx->batch == 0) FAIL(ctx, NEON_ESTATE, "neon_read_activation: no step has run");
  const neon_config& c = ctx->cfg;
  const size_t B = ctx->batch;
  const void* src = nullptr;
  size_t n = 0;
  const std::string nm(name);
  if (nm == "hidden") { src = ctx->h; n = B * c.hidden * 2; }
  else if (nm == "qkv") { src = ctx->qkv; n = B * (c.n_heads + 2 * c.n_kv_heads) * c.head_dim * 2; }
  else if (nm == "attn_out") { src = ctx->attn_out; n = B * c.n_heads * c.head_dim * 2; }
  else if (nm == "moe_in") { src = ctx->xn; n = B * c.hidden * 2; }
  else if (nm == "moe_idx") { src = ctx->moe_idx; n = B * c.top_k * 4; }
  else if (nm == "moe_score") { src = ctx->moe_score; n = B * c.top_k * 4; }
  else if (nm == "mx_route") {
    if (ctx->mx_route == nullptr || B < 2 || ctx->route_table < 0 ||
        (ctx->decode_mode != NEON_DECODE_MATRIX && ctx->decode_mode != NEON_DECODE_MATRIX_MX8))
      FAIL(ctx, NEON_EINVAL, "neon_read_activation: 'mx_route' exists after matrix-core steps "
           "of two or more sequences with a route table (NEON_ROUTER_ROUTE=0 or 1)");
    const size_t S = std::min<size_t>(c.n_experts, B * c.top_k);
    src = ctx->mx_route; n = (2 * S + 64 * S) * 4;
  }
  else if (nm == "mx_items") {
    if (ctx->mx_route == nullptr || B < 2 || ctx->route_table < 0 ||
        (ctx->decode_mode != NEON_DECODE_MATRIX && ctx->decode_mode != NEON_DECODE_MATRIX_MX8))
      FAIL(ctx, NEON_EINVAL, "neon_read_activation: 'mx_items' exists after matrix-core steps "
           "of two or more sequences with a route table (NEON_ROUTER_ROUTE=0 or 1)");
    src = ctx->mx_route + kMxItemOff; n = (kMxRouteWords - kMxItemOff) * 4;
  }
  else FAIL(ctx, NEON_EINVAL, "neon_read_activation: unknown buffer '%s'", name);
  if (bytes != n)
    FAIL(ctx, NEON_EINVAL, "neon_read_activation: '%s' holds %zu bytes, %zu requested", name, n, bytes);
  HIPCHK(ctx, hipSetDevice(ctx->device));
  HIPCHK(ctx, hipStreamSynchronize(S(stream)));
  HIPCHK(ctx, hipMemcpy(out, src, n, hipMemcpyDeviceToHost));
  return check_dev_err(ctx);
}

extern "C" neon_status neon_seq_len(const neon_ctx* ctx, int* out) {
  if (!ctx || !out) return NEON_EINVAL;
  *out = ctx->host_pos + (ctx->batch ? 1 : 0);
  return NEON_OK;
}

extern "C" neon_status neon_seq_lens(const neon_ctx* ctx, int32_t* out) {
  if (!ctx || !out) return NEON_EINVAL;
  if (ctx->batch == 0) return NEON_ESTATE;
  for (int b = 0; b < ctx->batch; ++b)
    out[b] = ctx->host_active[b] ? ctx->host_seq_pos[b] + 1 : 0;
  return NEON_OK;
}

// ---------------------------------------------------------------------------
// Sequences joining and leaving a running batch.  Each batch row owns one KV
// block (max_seq positions of every layer, a 256-row ring on sliding layers)
// for as long as a sequence holds it; a removed sequence's row and block go
// back to the pool and the next neon_seq_add takes the lowest free row.  The
// steps run rows 0 .. batch-1; a free row keeps position 0, writes no token
// and advances nothing (prompt_len < 0 on the device).
// ---------------------------------------------------------------------------
extern "C" neon_status neon_seq_add(neon_ctx* ctx, const int32_t* ids, int n, int* slot_out,
                                    void* stream) {
  if (!ctx) return NEON_EINVAL;
  const neon_config& c = ctx->cfg;
  if (!ids || !slot_out) FAIL(ctx, NEON_EINVAL, "neon_seq_add: null ids or slot");
  if (n < 1) FAIL(ctx, NEON_EINVAL, "neon_seq_add: the prompt needs >= 1 token");
  if (n > c.max_seq)
    FAIL(ctx, NEON_EKV_FULL, "neon_seq_add: %d prompt tokens exceed max_seq %d", n, c.max_seq);
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= c.vocab)
      FAIL(ctx, NEON_ERANGE_TOKEN, "neon_seq_add: token id %d at %d outside [0, %d)", ids[i], i,
           c.vocab);
  if (!ctx->weights_ready) FAIL(ctx, NEON_ESTATE, "neon_seq_add: no weights loaded");
  if ((int)ctx->host_active.size() != c.max_batch) {
    ctx->host_active.assign(c.max_batch, 0);
    ctx->host_seq_pos.assign(c.max_batch, 0);
    ctx->host_plen.assign(c.max_batch, 0);
  }
  int slot = -1;
  for (int b = 0; b < c.max_batch && slot < 0; ++b)
    if (!ctx->host_active[b]) slot = b;
  if (slot < 0)
    FAIL(ctx, NEON_EKV_FULL, "neon_seq_add: all %d batch rows hold a sequence", c.max_batch);
  HIPCHK(ctx, hipSetDevice(ctx->device));
  hipStream_t st = S(stream);
  // the row's tokens, its prompt length and the position of the last prompt
  // token (the row's final prompt step below consumes it)
  std::vector<int32_t> tok(ctx->tok_stride, 0);
  memcpy(tok.data(), ids, (size_t)n * 4);
  const int32_t meta[2] = {n - 1, n};
  HIPCHK(ctx, hipMemcpyAsync(ctx->tokens + (size_t)slot * ctx->tok_stride, tok.data(),
                             tok.size() * 4, hipMemcpyHostToDevice, st));
  HIPCHK(ctx, hipMemcpyAsync(ctx->pos + slot, &meta[0], 4, hipMemcpyHostToDevice, st));
  HIPCHK(ctx, hipMemcpyAsync(ctx->prompt_len + slot, &meta[1], 4, hipMemcpyHostToDevice, st));
  // rows 0 .. n-2 with the context's prompt mode (every row bit-identical to
  // the same row of neon_prefill)
  if (n > 1 && (ctx->prefill_mode == NEON_PREFILL_BATCHED ||
                ctx->prefill_mode == NEON_PREFILL_MX8)) {
    neon_status s = ensure_prefill_scratch(ctx, n - 1, st);
    if (s != NEON_OK) return s;
    enqueue_prefill_rows(ctx, slot, n - 1, st);
  } else {
    const int per = ctx->prefill_mode == NEON_PREFILL_STEPWISE ? 1 : kPromptRows;
    std::vector<int32_t> rp, rs;
    for (int p = 0; p < n; ++p) { rp.push_back(p); rs.push_back(slot); }
    for (int r0 = 0; r0 + 1 < n; r0 += per) {
      const int R = std::min(per, n - 1 - r0);
      HIPCHK(ctx, hipMemcpyAsync(ctx->row_pos, &rp[r0], R * 4, hipMemcpyHostToDevice, st));
      HIPCHK(ctx, hipMemcpyAsync(ctx->row_seq, &rs[r0], R * 4, hipMemcpyHostToDevice, st));
      enqueue_rows(ctx, R, ctx->row_pos, ctx->row_seq, st);
    }
    HIPCHK(ctx, hipStreamSynchronize(st));  // rp and rs die here
  }
  // the last prompt token as a one-row step of this sequence alone: its
  // logits land in the row's logits row, and the argmax (or the sampler,
  // keyed by the row like a batch step) writes tokens[slot][n] and
  // advances pos[slot] to n
  const int32_t last[2] = {n - 1, slot};
  HIPCHK(ctx, hipMemcpyAsync(ctx->row_pos, &last[0], 4, hipMemcpyHostToDevice, st));
  HIPCHK(ctx, hipMemcpyAsync(ctx->row_seq, &last[1], 4, hipMemcpyHostToDevice, st));
  enqueue_rows(ctx, 1, ctx->row_pos, ctx->row_seq, st);
  GemvArgs lm;
  lm.mode = 2; lm.W = ctx->lm_head; lm.x = ctx->h; lm.norm_w = ctx->final_norm;
  lm.eps = c.rms_eps; lm.logits = ctx->logits + (size_t)slot * c.vocab;
  lm.part_val = ctx->lm_part_val; lm.part_idx = ctx->lm_part_idx; lm.N = c.vocab;
  lm.K = c.hidden; lm.B = 1; lm.nblk = ctx->lm_nblk;
  const int parts = launch_gemv_step(lm, 1, st);
  int32_t* trow = ctx->tokens + (size_t)slot * ctx->tok_stride;
  if (ctx->temperature > 0.0f)
    launch_sample(ctx->logits + (size_t)slot * c.vocab, 1, c.vocab, ctx->temperature,
                  ctx->top_p, ctx->sample_seed, ctx->pos + slot, ctx->sample_scratch,
                  ctx->last_ids + slot, trow, ctx->tok_stride, ctx->prompt_len + slot, true, st,
                  slot);
  else
    launch_argmax_advance(ctx->lm_part_val, ctx->lm_part_idx, parts, trow, ctx->tok_stride,
                          ctx->pos + slot, ctx->prompt_len + slot, ctx->last_ids + slot, 1, st);
  HIPCHK(ctx, hipGetLastError());
  HIPCHK(ctx, hipStreamSynchronize(st));  // tok, meta and last die here
  ctx->host_active[slot] = 1;
  ctx->host_seq_pos[slot] = n;
  ctx->host_plen[slot] = n;
  ctx->batch = std::max(ctx->batch, slot + 1);
  ctx->host_pos = std::max(ctx->host_pos, n);
  *slot_out = slot;
  return NEON_OK;
}

extern "C" neon_status neon_seq_remove(neon_ctx* ctx, int slot, void* stream) {
  if (!ctx) return NEON_EINVAL;
  if (slot < 0 || slot >= ctx->batch || (int)ctx->host_active.size() <= slot ||
      !ctx->host_active[slot])
    FAIL(ctx, NEON_EINVAL, "neon_seq_remove: batch row %d holds no sequence", slot);
  HIPCHK(ctx, hipSetDevice(ctx->device));
  hipStream_t st = S(stream);
  // free row: position 0 (every later step writes its k / v at row 0 of its
  // own block and reads a valid token id), prompt length -1 (no token
  // written, nothing advanced)
  const int32_t zero = 0, freed = -1;
  HIPCHK(ctx, hipMemcpyAsync(ctx->pos + slot, &zero, 4, hipMemcpyHostToDevice, st));
  HIPCHK(ctx, hipMemcpyAsync(ctx->prompt_len + slot, &freed, 4, hipMemcpyHostToDevice, st));
  HIPCHK(ctx, hipMemcpyAsync(ctx->tokens + (size_t)slot * ctx->tok_stride, &zero, 4,
                             hipMemcpyHostToDevice, st));
  HIPCHK(ctx, hipStreamSynchronize(st));  // zero and freed die here
  ctx->host_active[slot] = 0;
  ctx->host_seq_pos[slot] = 0;
  ctx->host_plen[slot] = 0;
  // trailing free rows leave the step
  while (ctx->batch > 0 && !ctx->host_active[ctx->batch - 1]) --ctx->batch;
  return NEON_OK;
}

// ---------------------------------------------------------------------------
// kernel-level entry points: validate on the host, then launch.
// ---------------------------------------------------------------------------
#define KFAIL(code, ...)                          \
  do {                                            \
    char _b[512];                                 \
    snprintf(_b, sizeof(_b), __VA_ARGS__);        \
    g_create_error = _b;                          \
    return (code);                                \
  } while (0)

#define KLAUNCHED()                                                         \
  do {                                                                      \
    hipError_t _e = hipGetLastError();                                      \
    if (_e != hipSuccess) KFAIL(NEON_EHIP, "launch failed: %s", hipGetErrorString(_e)); \
    return NEON_OK;                                                         \
  } while (0)

// One status word per device for the kernel-level calls: a file-scope device
// array (zero when the code object loads, one copy per GPU), so no kernel-
// level call allocates.  Host code never passes the array's name to a kernel:
// it resolves the device address once per device with hipGetSymbolAddress.
static __device__ __align__(256) int32_t g_kernel_status[64];
static std::mutex g_status_mu;
static int32_t* g_status_word[256];

static int32_t* device_status_word() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 256) return nullptr;
  std::lock_guard<std::mutex> lk(g_status_mu);
  if (g_status_word[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_kernel_status)) != hipSuccess) return nullptr;
    g_status_word[dev] = (int32_t*)p;
  }
  return g_status_word[dev];
}

extern "C" neon_status neon_device_check(void* stream) {
  int32_t* w = device_status_word();
  if (w == nullptr) KFAIL(NEON_EHIP, "neon_device_check: no status word on this device");
  if (hipStreamSynchronize(S(stream)) != hipSuccess)
    KFAIL(NEON_EHIP, "neon_device_check: stream synchronisation failed");
  int32_t bits = 0;
  if (hipMemcpy(&bits, w, 4, hipMemcpyDeviceToHost) != hipSuccess)
    KFAIL(NEON_EHIP, "neon_device_check: status read failed");
  if (bits == 0) return NEON_OK;
  if (hipMemset(w, 0, 4) != hipSuccess) KFAIL(NEON_EHIP, "neon_device_check: status clear failed");
  if (bits & kDevErrSyncTimeout)
    KFAIL(NEON_EHIP, "a grid-wide wait inside a kernel-level call timed out (status bits 0x%x); "
          "its results are invalid", bits);
  KFAIL(NEON_EINVAL, "a kernel-level call saw an expert id outside [0, E) (status bits 0x%x); "
        "that slot was dropped", bits);
}

extern "C" neon_status neon_mxfp4_dequant(const uint8_t* codes,
                                          const uint8_t* scales, int64_t n_blocks,
                                          float* out, void* stream) {
  if (!codes || !scales || !out) KFAIL(NEON_EINVAL, "neon_mxfp4_dequant: null pointer");
  if (n_blocks < 0) KFAIL(NEON_EINVAL, "neon_mxfp4_dequant: n_blocks < 0");
  if (n_blocks == 0) return NEON_OK;
  launch_mxfp4_dequant(codes, scales, n_blocks, out, S(stream));
  KLAUNCHED();
}

extern "C" neon_status neon_mxfp4_gemv(const uint8_t* codes, const uint8_t* scales,
                                       const uint16_t* bias, const uint16_t* x,
                                       uint16_t* y, int N, int K, int B,
                                       void* stream) {
  if (!codes || !scales || !x || !y) KFAIL(NEON_EINVAL, "neon_mxfp4_gemv: null pointer");
  if (N < 1 || B < 1 || B > 65535 || K < 32 || K % 32 || K > 8192)
    KFAIL(NEON_EINVAL, "neon_mxfp4_gemv: bad shape N=%d K=%d B=%d", N, K, B);
  launch_mxfp4_gemv(codes, scales, bias, x, y, N, K, B, S(stream));
  KLAUNCHED();
}

extern "C" neon_status neon_gemv_bf16_mfma(const uint16_t* W, const uint16_t* bias,
                                           const uint16_t* x, uint16_t* y, int N, int K, int B,
                                           void* stream) {
  if (!W || !x || !y) KFAIL(NEON_EINVAL, "neon_gemv_bf16_mfma: null pointer");
  if (!mx_shape_ok(N, K, B))
    KFAIL(NEON_EINVAL, "neon_gemv_bf16_mfma: need N %% 16 == 0, K %% 32 == 0, K <= %d, "
                       "1 <= B <= %d (N=%d K=%d B=%d)", kMxMaxK, kMxMaxRows, N, K, B);
  MxArgs a{};
  a.W = W; a.bias = bias; a.x = x; a.y = y; a.B = B; a.N = N; a.K = K;
  launch_mx_gemv(a, 0, S(stream));
  KLAUNCHED();
}

extern "C" neon_status neon_gemv_bf16(const uint16_t* W, const uint16_t* bias,
                                      const uint16_t* x, uint16_t* y, int N, int K,
                                      int B, void* stream) {
  if (!W || !x || !y) KFAIL(NEON_EINVAL, "neon_gemv_bf16: null pointer");
  if (N < 1 || B < 1 || B > 65535 || K < 8 || K % 8 || K > 8192)
    KFAIL(NEON_EINVAL, "neon_gemv_bf16: bad shape N=%d K=%d B=%d", N, K, B);
  GemvArgs a;
  a.mode = 0; a.W = W; a.bias = bias; a.x = x; a.y = y; a.N = N; a.K = K; a.B = B;
  a.nblk = gemv_default_grid(N, a.mode);
  launch_gemv_bf16(a, S(stream));
  KLAUNCHED();
}

extern "C" neon_status neon_rmsnorm(const uint16_t* x, const uint16_t* w,
                                    uint16_t* out, int B, int H, float eps,
                                    void* stream) {
  if (!x || !w || !out) KFAIL(NEON_EINVAL, "neon_rmsnorm: null pointer");
  if (B < 1 || H < 8 || H % 8 || H > 8192 || !(eps > 0.0f))
    KFAIL(NEON_EINVAL, "neon_rmsnorm: bad shape B=%d H=%d eps=%g", B, H, eps);
  launch_rmsnorm(x, w, out, B, H, eps, S(stream));
  KLAUNCHED();
}

static bool rope_cfg_ok(const neon_config* cfg) {
  return cfg->head_dim >= 2 && cfg->head_dim % 2 == 0 && cfg->head_dim <= 512 &&
         cfg->rope_theta > 1.0f && cfg->rope_factor >= 1.0f && cfg->rope_orig_max_pos >= 1;
}

extern "C" neon_status neon_rope_table(const neon_config* cfg, int n_pos, float* table,
                                       void* stream) {
  if (!cfg || !table) KFAIL(NEON_EINVAL, "neon_rope_table: null pointer");
  if (n_pos < 1 || !rope_cfg_ok(cfg)) KFAIL(NEON_EINVAL, "neon_rope_table: bad n_pos or rope parameters");
  std::vector<float> ct, stb;
  rope_table_host(cfg, n_pos, ct, stb);
  const size_t tn = (size_t)n_pos * (cfg->head_dim / 2);
  // a set-up call (the reference's constructor-time uploads): the host
  // tables are copied before it returns
  hipStream_t st = S(stream);
  if (hipMemcpyAsync(table, ct.data(), tn * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
      hipMemcpyAsync(table + tn, stb.data(), tn * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    KFAIL(NEON_EHIP, "neon_rope_table: copy failed");
  return NEON_OK;
}

extern "C" neon_status neon_rope_yarn(uint16_t* x, const int32_t* pos, int n_tok,
                                      int n_heads, int head_dim, const float* table,
                                      int n_pos, void* stream) {
  if (!x || !pos || !table) KFAIL(NEON_EINVAL, "neon_rope_yarn: null pointer");
  if (n_tok < 1 || n_heads < 1 || head_dim < 2 || head_dim % 2 || head_dim > 512 || n_pos < 1)
    KFAIL(NEON_EINVAL, "neon_rope_yarn: bad shape n_tok=%d n_heads=%d head_dim=%d n_pos=%d",
          n_tok, n_heads, head_dim, n_pos);
  // pos[t] must lie in [0, n_pos): device data, trusted by the kernel
  const size_t tn = (size_t)n_pos * (head_dim / 2);
  launch_rope_apply(x, pos, table, table + tn, n_tok, n_heads, head_dim, S(stream));
  KLAUNCHED();
}

extern "C" neon_status neon_router_topk(const uint16_t* x, const uint16_t* W,
                                        const uint16_t* b, int32_t* idx,
                                        float* score, float* logits, int B, int E,
                                        int H, int k, void* stream) {
  if (!x || !W || !b || !idx || !score || !logits)
    KFAIL(NEON_EINVAL, "neon_router_topk: null pointer");
  if (B < 1 || B > 65535 || E < 1 || E > 256 || k < 1 || k > 16 || k > E || H < 8 ||
      H % 8 || H > 8192)
    KFAIL(NEON_EINVAL, "neon_router_topk: bad shape B=%d E=%d H=%d k=%d", B, E, H, k);
  RouterArgs r;
  r.x = x; r.W = W; r.bias = b; r.lg_out = logits; r.idx = idx;
  r.score = score; r.B = B; r.E = E; r.H = H; r.k = k;
  launch_router(r, S(stream));
  KLAUNCHED();
}

// Workspace of neon_moe_layer: act [B][k][I] bf16, the router logits [B][E]
// fp32, and the arrival counters of the one-launch experts (NEON_MOE_FUSED;
// the router launch clears them), each 256-byte aligned.
struct MoeLayerWs {
  size_t act, lg, total;
};
static MoeLayerWs moe_layer_ws(int B, int E, int I, int k) {
  MoeLayerWs w;
  w.act = ((size_t)B * k * I * 2 + 255) & ~(size_t)255;
  w.lg = ((size_t)B * E * 4 + 255) & ~(size_t)255;
  w.total = w.act + w.lg + (size_t)kMoeSyncInts * 4;
  return w;
}

extern "C" size_t neon_moe_layer_workspace(int B, int E, int I, int k) {
  if (B < 1 || E < 1 || I < 1 || k < 1) return 0;
  return moe_layer_ws(B, E, I, k).total;
}

extern "C" neon_status neon_moe_layer(
    const uint16_t* x, const uint16_t* router_w, const uint16_t* router_b,
    const uint8_t* gu_codes, const uint8_t* gu_scales, const uint16_t* gu_bias,
    const uint8_t* dn_codes, const uint8_t* dn_scales, const uint16_t* dn_bias,
    const uint16_t* residual, uint16_t* out, int32_t* idx, float* score, int B,
    int E, int H, int I, int k, float alpha, float limit, void* workspace,
    size_t workspace_bytes, void* stream) {
  if (!x || !router_w || !router_b || !gu_codes || !gu_scales || !gu_bias ||
      !dn_codes || !dn_scales || !dn_bias || !out || !workspace)
    KFAIL(NEON_EINVAL, "neon_moe_layer: null pointer");
  if (B < 1 || B > 65535 || E < 1 || E > 256 || k < 1 || k > 16 || k > E ||
      H < 32 || H % 32 || H > 8192 || I < 32 || I % 32 || I > 8192)
    KFAIL(NEON_EINVAL, "neon_moe_layer: bad shape B=%d E=%d H=%d I=%d k=%d", B, E, H, I, k);
  const MoeLayerWs w = moe_layer_ws(B, E, I, k);
  if (workspace_bytes < w.total)
    KFAIL(NEON_EINVAL, "neon_moe_layer: workspace of %zu bytes, %zu needed "
          "(neon_moe_layer_workspace)", workspace_bytes, w.total);
  hipStream_t st = S(stream);
  char* base = (char*)workspace;
  uint16_t* act = (uint16_t*)base;
  float* lg = (float*)(base + w.act);
  int32_t* sync = (int32_t*)(base + w.act + w.lg);
  RouterArgs r;
  r.x = x; r.W = router_w; r.bias = router_b; r.lg_out = lg;
  r.B = B; r.E = E; r.H = H; r.k = k;
  r.zero = sync; r.zero_n = kMoeSyncZero;
  launch_router(r, st);
  MoeArgs m;
  m.gu_codes = gu_codes; m.gu_scales = gu_scales; m.gu_bias = gu_bias;
  m.dn_codes = dn_codes; m.dn_scales = dn_scales; m.dn_bias = dn_bias;
  m.router_lg = lg; m.idx = nullptr; m.score = nullptr; m.idx_out = idx;
  m.score_out = score; m.E = E; m.xn = x; m.act = act; m.residual = residual;
  m.out = out; m.B = B; m.H = H; m.I = I; m.k = k; m.alpha = alpha; m.limit = limit;
  m.err = device_status_word();
  m.sync = getenv("NEON_MOE_FUSED") && getenv("NEON_MOE_FUSED")[0] == '1' ? sync : nullptr;
  launch_moe(m, st);
  KLAUNCHED();
}

// ---- neon_moe_layer without allocation -----------------------------------
// Scratch of neon_moe_layer_noalloc: a file-scope device array, one copy per
// GPU, held until the process ends.  Host code never passes the array's name
// to a kernel (on the host it is only a stand-in symbol): it resolves the
// device address once per device with hipGetSymbolAddress and uses that.
constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20;  // 4 MiB
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static char* g_scratch_ptr[256];

// Device address of `scratch` on the current device (resolved on the first
// call per device, with that device current).
static neon_status scratch_address(char** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 256)
    KFAIL(NEON_EHIP, "neon_moe_layer_noalloc: no current HIP device");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      KFAIL(NEON_EHIP, "neon_moe_layer_noalloc: hipGetSymbolAddress failed: %s",
            hipGetErrorString(e));
    g_scratch_ptr[dev] = (char*)p;
  }
  *out = g_scratch_ptr[dev];
  return NEON_OK;
}

extern "C" neon_status neon_moe_layer_noalloc(
    const uint16_t* x, const uint16_t* router_w, const uint16_t* router_b,
    const uint8_t* gu_codes, const uint8_t* gu_scales, const uint16_t* gu_bias,
    const uint8_t* dn_codes, const uint8_t* dn_scales, const uint16_t* dn_bias,
    const uint16_t* residual, uint16_t* out, int32_t* idx, float* score, int B,
    int E, int H, int I, int k, float alpha, float limit, void* stream) {
  if (!x || !router_w || !router_b || !gu_codes || !gu_scales || !gu_bias ||
      !dn_codes || !dn_scales || !dn_bias || !out)
    KFAIL(NEON_EINVAL, "neon_moe_layer_noalloc: null pointer");
  if (B < 1 || B > 65535 || E < 1 || E > 256 || k < 1 || k > 16 || k > E ||
      H < 32 || H % 32 || H > 8192 || I < 32 || I % 32 || I > 8192)
    KFAIL(NEON_EINVAL, "neon_moe_layer_noalloc: bad shape B=%d E=%d H=%d I=%d k=%d", B, E, H,
          I, k);
  // the same scratch as neon_moe_layer: act [B][k][I] bf16, then the router
  // logits [B][E] fp32 (both written in full before they are read)
  const size_t act_b = ((size_t)B * k * I * 2 + 255) & ~(size_t)255;
  const size_t need = act_b + (size_t)B * E * 4;
  if (need > kNoAllocScratchBytes)
    KFAIL(NEON_EINVAL, "neon_moe_layer_noalloc: B=%d k=%d I=%d E=%d needs %zu scratch bytes, "
          "above the fixed %zu (use neon_moe_layer)", B, k, I, E, need, kNoAllocScratchBytes);
  char* base = nullptr;
  const neon_status s = scratch_address(&base);
  if (s != NEON_OK) return s;
  hipStream_t st = S(stream);
  uint16_t* act = (uint16_t*)base;
  float* lg = (float*)(base + act_b);
  RouterArgs r;
  r.x = x; r.W = router_w; r.bias = router_b; r.lg_out = lg;
  r.B = B; r.E = E; r.H = H; r.k = k;
  launch_router(r, st);
  MoeArgs m;
  m.gu_codes = gu_codes; m.gu_scales = gu_scales; m.gu_bias = gu_bias;
  m.dn_codes = dn_codes; m.dn_scales = dn_scales; m.dn_bias = dn_bias;
  m.router_lg = lg; m.idx = nullptr; m.score = nullptr; m.idx_out = idx;
  m.score_out = score; m.E = E; m.xn = x; m.act = act; m.residual = residual;
  m.out = out; m.B = B; m.H = H; m.I = I; m.k = k; m.alpha = alpha; m.limit = limit;
  m.err = nullptr;  // the ids come from the in-kernel top-k: always in [0, E)
  launch_moe(m, st);
  KLAUNCHED();
}

extern "C" neon_status neon_moe_experts(
    const uint16_t* x, const int32_t* idx, const float* score,
    const uint8_t* gu_codes, const uint8_t* gu_scales, const uint16_t* gu_bias,
    const uint8_t* dn_codes, const uint8_t* dn_scales, const uint16_t* dn_bias,
    const uint16_t* residual, uint16_t* out, uint16_t* act, int B, int E, int H,
    int I, int k, float alpha, float limit, void* stream) {
  if (!x || !idx || !score || !gu_codes || !gu_scales || !gu_bias || !dn_codes ||
      !dn_scales || !dn_bias || !out || !act)
    KFAIL(NEON_EINVAL, "neon_moe_experts: null pointer");
  if (B < 1 || B > 65535 || E < 1 || E > 256 || k < 1 || k > 16 || k > E ||
      H < 32 || H % 32 || H > 8192 || I < 32 || I % 32 || I > 8192)
    KFAIL(NEON_EINVAL, "neon_moe_experts: bad shape B=%d E=%d H=%d I=%d k=%d", B, E, H, I, k);
  // idx is device data: an entry outside [0, E) drops its slot and sets the
  // device status word (neon_device_check reports it).
  MoeArgs m;
  m.gu_codes = gu_codes; m.gu_scales = gu_scales; m.gu_bias = gu_bias;
  m.dn_codes = dn_codes; m.dn_scales = dn_scales; m.dn_bias = dn_bias;
  m.router_lg = nullptr; m.idx = idx; m.score = score; m.idx_out = nullptr;
  m.score_out = nullptr; m.E = E; m.xn = x; m.act = act; m.residual = residual;
  m.out = out; m.B = B; m.H = H; m.I = I; m.k = k; m.alpha = alpha; m.limit = limit;
  m.err = device_status_word();
  if (moe_batched_supported(m)) launch_moe_batched(m, S(stream));
  else launch_moe(m, S(stream));
  KLAUNCHED();
}

static bool attn_shape_ok(int B, int Hq, int Hkv, int D, int T_max, int window) {
  if (D != 64 || B < 1 || B > 65535 || Hkv < 1 || Hq < Hkv || Hq % Hkv || T_max < 1 ||
      window < 0)
    return false;
  const int G = Hq / Hkv;
  return G == 1 || G == 2 || G == 4 || G == 8;
}

// Split partials of neon_attn_decode: o [B][Hq][S][D], then (m, l)
// [B][Hq][S][2], fp32; none with one split.
extern "C" size_t neon_attn_decode_workspace(int B, int Hq, int Hkv, int D, int T_max,
                                             int window) {
  if (!attn_shape_ok(B, Hq, Hkv, D, T_max, window)) return 0;
  const int nsplit = attn_splits(T_max, window);
  if (nsplit == 1) return 0;
  return (size_t)B * Hq * nsplit * (D + 2) * 4;
}

// Arrival counters: one 256-byte line per (row, kv head).
extern "C" size_t neon_attn_decode_counters(int B, int Hkv) {
  if (B < 1 || Hkv < 1) return 0;
  return (size_t)B * Hkv * kAttnArriveStride * 4;
}

extern "C" neon_status neon_attn_decode(const uint16_t* q, const uint16_t* k_cache,
                                        const uint16_t* v_cache,
                                        const uint16_t* sinks, const int32_t* pos,
                                        uint16_t* out, int B, int Hq, int Hkv, int D,
                                        int T_max, int window, float* workspace,
                                        size_t workspace_bytes, int32_t* counters,
                                        size_t counter_bytes, void* stream) {
  if (!q || !k_cache || !v_cache || !sinks || !pos || !out)
    KFAIL(NEON_EINVAL, "neon_attn_decode: null pointer");
  if (!attn_shape_ok(B, Hq, Hkv, D, T_max, window))
    KFAIL(NEON_EINVAL, "neon_attn_decode: bad shape (D must be 64, Hq/Hkv 1, 2, 4 or 8)");
  // pos[b] must lie in [0, T_max); it is device data, so the kernel trusts it.
  const int nsplit = attn_splits(T_max, window);
  const size_t need = neon_attn_decode_workspace(B, Hq, Hkv, D, T_max, window);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    KFAIL(NEON_EINVAL, "neon_attn_decode: %d key splits need a workspace of %zu bytes "
          "(given %zu)", nsplit, need, workspace_bytes);
  if (nsplit > 1 && (counters == nullptr || counter_bytes < neon_attn_decode_counters(B, Hkv)))
    KFAIL(NEON_EINVAL, "neon_attn_decode: %d key splits need %zu bytes of arrival counters "
          "(given %zu)", nsplit, neon_attn_decode_counters(B, Hkv), counter_bytes);
  // the last split block of each (row, kv head) to arrive on its counter
  // merges and sets the counter back to 0: the caller zeroes the counters
  // once, every call leaves them zero
  const size_t np = (size_t)B * Hq * nsplit;
  AttnArgs a;
  a.q = q; a.kc = k_cache; a.vc = v_cache;
  a.sinks = sinks; a.pos = pos; a.out = out;
  a.part_o = nsplit > 1 ? workspace : nullptr;
  a.part_ml = nsplit > 1 ? workspace + np * D : nullptr;
  a.seq = nullptr; a.arrive = nsplit > 1 ? counters : nullptr;
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.T_max = T_max; a.key_mask = -1; a.window = window;
  a.S = nsplit; a.q_stride = Hq * D;
  launch_attn(a, S(stream));
  KLAUNCHED();
}

extern "C" size_t neon_sample_workspace(int B, int V) {
  if (B < 1 || V < 1) return 0;
  return (size_t)B * V * 4;
}

extern "C" neon_status neon_sample(const float* logits, int B, int V, float temperature,
                                   float top_p, uint64_t seed, const int32_t* pos,
                                   int32_t* out_ids, float* workspace, size_t workspace_bytes,
                                   void* stream) {
  if (!logits || !pos || !out_ids || !workspace) KFAIL(NEON_EINVAL, "neon_sample: null pointer");
  if (B < 1 || B > 65535 || V < 1 || !(temperature > 0.0f) || !(temperature < 3.0e38f) ||
      !(top_p > 0.0f && top_p <= 1.0f))
    KFAIL(NEON_EINVAL, "neon_sample: bad shape or sampling parameters");
  if (workspace_bytes < neon_sample_workspace(B, V))
    KFAIL(NEON_EINVAL, "neon_sample: workspace of %zu bytes, %zu needed", workspace_bytes,
          neon_sample_workspace(B, V));
  // the exp values [B][V] go to the workspace; pos is read only (advance =
  // false): cast for the shared kernel signature
  launch_sample(logits, B, V, temperature, top_p, seed, const_cast<int32_t*>(pos), workspace,
                out_ids, nullptr, 0, nullptr, false, S(stream));
  KLAUNCHED();
}

extern "C" neon_status neon_gemm_bf16(const uint16_t* A, const uint16_t* W,
                                      const uint16_t* bias, uint16_t* C, int M, int N,
                                      int K, int accumulate, void* stream) {
  if (!A || !W || !C) KFAIL(NEON_EINVAL, "neon_gemm_bf16: null pointer");
  if (M < 1 || N < 1 || K < 32 || K % 32 || (int64_t)M * 128 > ((int64_t)1 << 31) ||
      N > (1 << 24) || K > (1 << 20))
    KFAIL(NEON_EINVAL, "neon_gemm_bf16: bad shape M=%d N=%d K=%d", M, N, K);
  launch_gemm_bf16(A, K, W, K, bias, C, nullptr, N, M, N, K, accumulate ? 1 : 0, S(stream));
  KLAUNCHED();
}

// Workspace layout of the kernel-level expert FFN over prompt rows: fp32
// slot outputs, the SwiGLU output, the expert grouping (per-pair token and
// slot lists, expert offsets, tile lists) and, for the MXFP8 form, the
// two-term quantised GEMM inputs and their scales; each 256-byte aligned.
struct MoePrefillWs {
  size_t yb, act, lt, ls, eo, te, tr, nt, q, qs, total;
};
static MoePrefillWs moe_prefill_ws(int M, int E, int H, int I, int k, bool mx8) {
  const size_t pairs = (size_t)M * k, tiles = (size_t)moe_prefill_max_tiles(M, k, E);
  const size_t qn = mx8 ? std::max((size_t)M * H, pairs * I) : 0;
  MoePrefillWs w;
  size_t off = 0;
  auto take = [&](size_t b) { size_t o = off; off = align_up(off + b); return o; };
  w.yb = take(pairs * H * 4); w.act = take(pairs * I * 2); w.lt = take(pairs * 4);
  w.ls = take(pairs * 4); w.eo = take((E + 1) * 4); w.te = take(tiles * 4);
  w.tr = take(tiles * 4); w.nt = take(16); w.q = take(2 * qn);
  w.qs = take(mx8 ? std::max(mx8_scale_bytes(M, H), mx8_scale_bytes(pairs, I)) : 0);
  w.total = off;
  return w;
}

static bool moe_prefill_shape_ok(int M, int E, int H, int I, int k, bool mx8) {
  const int kq = mx8 ? 64 : 32;
  return M >= 1 && M <= (1 << 20) && E >= 1 && E <= 256 && k >= 1 && k <= 16 && k <= E &&
         H >= kq && H % kq == 0 && H <= 8192 && I >= kq && I % kq == 0 && I <= 8192;
}

extern "C" size_t neon_moe_prefill_workspace(int M, int E, int H, int I, int k, int mx8) {
  if (!moe_prefill_shape_ok(M, E, H, I, k, mx8 != 0)) return 0;
  return moe_prefill_ws(M, E, H, I, k, mx8 != 0).total;
}

// The kernel-level expert FFN over prompt rows, with the bf16-dequantising
// GEMMs or (mx8) the scaled MXFP8 x MXFP4 ones.
static neon_status moe_prefill_impl(const uint16_t* x, const int32_t* idx, const float* score,
                                    const uint8_t* gu_codes, const uint8_t* gu_scales,
                                    const uint16_t* gu_bias, const uint8_t* dn_codes,
                                    const uint8_t* dn_scales, const uint16_t* dn_bias,
                                    uint16_t* h, int M, int E, int H, int I, int k, float alpha,
                                    float limit, void* workspace, size_t workspace_bytes,
                                    void* stream, bool mx8, const char* fn) {
  if (!x || !idx || !score || !gu_codes || !gu_scales || !gu_bias || !dn_codes ||
      !dn_scales || !dn_bias || !h || !workspace)
    KFAIL(NEON_EINVAL, "%s: null pointer", fn);
  if (!moe_prefill_shape_ok(M, E, H, I, k, mx8))
    KFAIL(NEON_EINVAL, "%s: bad shape M=%d E=%d H=%d I=%d k=%d", fn, M, E, H, I, k);
  if (!kBatchedPrefillEnabled)
    KFAIL(NEON_ESTATE, "%s: the batched prompt pass is switched off", fn);
  const MoePrefillWs w = moe_prefill_ws(M, E, H, I, k, mx8);
  if (workspace_bytes < w.total)
    KFAIL(NEON_EINVAL, "%s: workspace of %zu bytes, %zu needed (neon_moe_prefill_workspace)",
          fn, workspace_bytes, w.total);
  // idx is device data: an entry outside [0, E) drops its slot and sets the
  // device status word (neon_device_check reports it).
  char* base = (char*)workspace;
  MoePrefillArgs m;
  m.idx = idx; m.score = score; m.xn = x; m.h = h;
  m.gu_codes = gu_codes; m.gu_scales = gu_scales; m.gu_bias = gu_bias;
  m.dn_codes = dn_codes; m.dn_scales = dn_scales; m.dn_bias = dn_bias;
  m.M = M; m.E = E; m.H = H; m.I = I; m.k = k; m.alpha = alpha; m.limit = limit;
  m.ybuf = (float*)(base + w.yb); m.act = (uint16_t*)(base + w.act);
  m.list_tok = (int32_t*)(base + w.lt); m.list_slot = (int32_t*)(base + w.ls);
  m.e_off = (int32_t*)(base + w.eo); m.tile_e = (int32_t*)(base + w.te);
  m.tile_r0 = (int32_t*)(base + w.tr); m.n_tiles = (int32_t*)(base + w.nt);
  if (mx8) {
    m.q = (uint8_t*)(base + w.q); m.qs = (uint32_t*)(base + w.qs);
  }
  m.err = device_status_word();
  launch_moe_prefill(m, S(stream));
  KLAUNCHED();
}

extern "C" neon_status neon_moe_prefill(const uint16_t* x, const int32_t* idx,
                                        const float* score, const uint8_t* gu_codes,
                                        const uint8_t* gu_scales, const uint16_t* gu_bias,
                                        const uint8_t* dn_codes, const uint8_t* dn_scales,
                                        const uint16_t* dn_bias, uint16_t* h, int M, int E,
                                        int H, int I, int k, float alpha, float limit,
                                        void* workspace, size_t workspace_bytes,
                                        void* stream) {
  return moe_prefill_impl(x, idx, score, gu_codes, gu_scales, gu_bias, dn_codes, dn_scales,
                          dn_bias, h, M, E, H, I, k, alpha, limit, workspace, workspace_bytes,
                          stream, false, "neon_moe_prefill");
}

extern "C" neon_status neon_moe_prefill_mx8(const uint16_t* x, const int32_t* idx,
                                            const float* score, const uint8_t* gu_codes,
                                            const uint8_t* gu_scales, const uint16_t* gu_bias,
                                            const uint8_t* dn_codes, const uint8_t* dn_scales,
                                            const uint16_t* dn_bias, uint16_t* h, int M, int E,
                                            int H, int I, int k, float alpha, float limit,
                                            void* workspace, size_t workspace_bytes,
                                            void* stream) {
  return moe_prefill_impl(x, idx, score, gu_codes, gu_scales, gu_bias, dn_codes, dn_scales,
                          dn_bias, h, M, E, H, I, k, alpha, limit, workspace, workspace_bytes,
                          stream, true, "neon_moe_prefill_mx8");
}

extern "C" neon_status neon_mx8_quant(const uint16_t* x, int64_t rows, int K, uint8_t* hi,
                                      uint8_t* lo, uint8_t* s_hi, uint8_t* s_lo,
                                      void* stream) {
  if (!x || !hi || !lo || !s_hi || !s_lo) KFAIL(NEON_EINVAL, "neon_mx8_quant: null pointer");
  if (rows < 1 || K < 32 || K % 32 || rows > ((int64_t)1 << 40) / K)
    KFAIL(NEON_EINVAL, "neon_mx8_quant: bad shape rows=%lld K=%d", (long long)rows, K);
  launch_mx8_quant(x, rows, K, hi, lo, s_hi, s_lo, S(stream));
  KLAUNCHED();
}

extern "C" neon_status neon_attn_prefill(const uint16_t* q, const uint16_t* k_cache,
                                         const uint16_t* v_cache, const uint16_t* sinks,
                                         uint16_t* out, int M, int Hq, int Hkv, int D,
                                         int T_max, int window, void* stream) {
  if (!q || !k_cache || !v_cache || !sinks || !out)
    KFAIL(NEON_EINVAL, "neon_attn_prefill: null pointer");
  if (D != 64 || M < 1 || Hkv < 1 || Hq < Hkv || Hq % Hkv || T_max < M || window < 0 ||
      (M + 63) / 64 > 65535)
    KFAIL(NEON_EINVAL, "neon_attn_prefill: bad shape");
  const int G = Hq / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    KFAIL(NEON_EINVAL, "neon_attn_prefill: Hq/Hkv must be 1, 2, 4 or 8");
  if (!kBatchedPrefillEnabled)
    KFAIL(NEON_ESTATE, "neon_attn_prefill: the batched prompt pass is switched off");
  launch_attn_prefill(q, k_cache, v_cache, sinks, out, M, Hq, Hkv, T_max, window, S(stream));
  KLAUNCHED();
}

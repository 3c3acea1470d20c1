// neon_engine.hpp -- C++ engine API over the C-ABI in neon_gptoss.h.
//
// The reference's GPU-work objects are C++ "Systems": the constructor
// allocates device state and throws std::runtime_error on failure, and one
// call per frame records the work (NeonEngine/src/water_physics.cpp:23-123,
// :131; failures propagate to main, NeonEngine/src/main.cpp:21-26).
// neon::Engine keeps that shape for the gpt-oss token loop: construct, load
// weights (checkpoint tensors or deterministic random init), prefill, decode.
// Everything goes through the C-ABI, so this header needs no HIP includes;
// tests/cpp/engine_greedy.cpp is a host program built on it.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "neon_gptoss.h"

namespace neon {

class Error : public std::runtime_error {
 public:
  Error(neon_status s, const std::string& what)
      : std::runtime_error(what), status_(s) {}
  neon_status status() const { return status_; }

 private:
  neon_status status_;
};

inline void check(neon_status s, const neon_ctx* ctx) {
  if (s != NEON_OK) {
    const char* m = neon_last_error(ctx);
    throw Error(s, m ? m : "neon error");
  }
}

class Config {
 public:
  static Config preset(const char* name) {
    Config c;
    check(neon_config_preset(name, &c.cfg_), nullptr);
    return c;
  }
  neon_config& raw() { return cfg_; }
  const neon_config& raw() const { return cfg_; }

 private:
  neon_config cfg_{};
};

class Engine {
 public:
  Engine(const Config& cfg, int device = 0) : vocab_(cfg.raw().vocab) {
    check(neon_ctx_create(&cfg.raw(), device, &ctx_), nullptr);
  }
  ~Engine() { neon_ctx_destroy(ctx_); }
  Engine(const Engine&) = delete;
  Engine& operator=(const Engine&) = delete;

  // Model loading: deterministic random init or one checkpoint tensor.
  void init_random(uint64_t seed, void* stream = nullptr) {
    check(neon_init_random(ctx_, seed, stream), ctx_);
  }
  void load_tensor(const std::string& name, const void* data, size_t bytes) {
    check(neon_load_tensor(ctx_, name.c_str(), data, bytes), ctx_);
  }

  // Prompt mode: NEON_PREFILL_CHUNKED (16 prompt rows per pass, default),
  // NEON_PREFILL_STEPWISE (every prompt token as a decode step), both
  // bit-identical; or NEON_PREFILL_BATCHED (all prompt rows at once on the
  // matrix cores, equal to the others up to bf16 rounding).
  void set_prefill_mode(int mode) { check(neon_set_prefill_mode(ctx_, mode), ctx_); }
  // Steps of two or more sequences: NEON_DECODE_EXACT (default) or
  // NEON_DECODE_MATRIX (matrix cores).
  void set_decode_mode(int mode) { check(neon_set_decode_mode(ctx_, mode), ctx_); }
  // Next-token choice: temperature 0 (default) is greedy argmax; otherwise
  // nucleus sampling (top_p in (0, 1]) reproducible for a seed.
  void set_sampling(float temperature, float top_p = 1.0f, uint64_t seed = 0) {
    check(neon_set_sampling(ctx_, temperature, top_p, seed), ctx_);
  }

  // Forward: prefill `batch` prompts of equal length (row-major ids), then
  // decode steps; tokens() returns prompt + generated ids per row (0 past a
  // shorter sequence's length).
  void prefill(const std::vector<int32_t>& ids, int batch, void* stream = nullptr) {
    if (batch < 1 || ids.empty() || ids.size() % (size_t)batch)
      throw Error(NEON_EINVAL, "prefill: ids.size() must be a positive multiple of batch");
    check(neon_prefill(ctx_, ids.data(), batch, (int)(ids.size() / batch), stream), ctx_);
    batch_ = batch;
  }
  // Prompts of different lengths (each sequence keeps its own position).
  void prefill(const std::vector<std::vector<int32_t>>& prompts, void* stream = nullptr) {
    std::vector<int32_t> flat, lens;
    for (const auto& p : prompts) {
      flat.insert(flat.end(), p.begin(), p.end());
      lens.push_back((int32_t)p.size());
    }
    check(neon_prefill_ragged(ctx_, flat.data(), lens.data(), (int)prompts.size(), stream), ctx_);
    batch_ = (int)prompts.size();
  }
  // Tokens held by each sequence (prompt + generated).
  std::vector<int32_t> seq_lens() const {
    std::vector<int32_t> out((size_t)batch_);
    check(neon_seq_lens(ctx_, out.data()), ctx_);
    return out;
  }
  void decode(int n_steps, void* stream = nullptr) {
    check(neon_decode(ctx_, n_steps, stream), ctx_);
  }
  std::vector<int32_t> tokens(void* stream = nullptr) {
    int n = 0;
    check(neon_seq_len(ctx_, &n), ctx_);
    std::vector<int32_t> out((size_t)batch_ * n);
    check(neon_read_tokens(ctx_, 0, n, out.data(), stream), ctx_);
    return out;
  }
  // fp32 logits of the last step, [batch][vocab] (vocab from the config the
  // engine was built with)
  std::vector<float> logits(void* stream = nullptr) {
    std::vector<float> out((size_t)batch_ * vocab_);
    check(neon_read_logits(ctx_, out.data(), stream), ctx_);
    return out;
  }
  int batch() const { return batch_; }
  int vocab() const { return vocab_; }
  neon_ctx* handle() { return ctx_; }

 private:
  neon_ctx* ctx_ = nullptr;
  int batch_ = 0;
  int vocab_ = 0;
};

}  // namespace neon

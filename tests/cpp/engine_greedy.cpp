// engine_greedy.cpp -- a C++ host of the token loop: neon::Engine
// (include/neon_engine.hpp over libneon_gptoss.so) runs init_random ->
// prefill -> decode -> tokens / logits, and the CPU oracle
// (oracle/libneon_oracle.so, linked as the checker only) replays the same
// model; the program exits 0 when every greedy id and the last step's fp32
// logits are identical.  This is the shape of a reference System driving the
// engine from main (NeonEngine/src/main.cpp:21-26: errors propagate as
// exceptions).
//
//   engine_greedy [small|20b] [steps] [batch]
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "neon_engine.hpp"
extern "C" {
#include "../../oracle/neon_oracle.h"
}

int main(int argc, char** argv) {
  const std::string shape = argc > 1 ? argv[1] : "small";
  const int steps = argc > 2 ? std::atoi(argv[2]) : 32;
  const int batch = argc > 3 ? std::atoi(argv[3]) : 2;
  const int plen = 6;
  const uint64_t seed = 5;
  try {
    neon::Config cfg = neon::Config::preset("gpt-oss-20b");
    neon_config& c = cfg.raw();
    if (shape == "small") {
      c.n_layers = 4; c.hidden = 512; c.n_heads = 16; c.n_kv_heads = 2; c.n_experts = 8;
      c.intermediate = 512; c.vocab = 4096;
    } else if (shape != "20b") {
      std::fprintf(stderr, "engine_greedy: shape must be small or 20b\n");
      return 2;
    }
    c.max_seq = plen + steps + 8;
    c.max_batch = batch;
    std::vector<int32_t> prompt((size_t)batch * plen);
    for (int b = 0; b < batch; ++b)
      for (int t = 0; t < plen; ++t) prompt[(size_t)b * plen + t] = (101 + 7 * b + 13 * t) % c.vocab;

    neon::Engine eng(cfg, 0);
    eng.init_random(seed);
    eng.prefill(prompt, batch);
    eng.decode(steps);
    const std::vector<int32_t> toks = eng.tokens();
    const std::vector<float> lg = eng.logits();

    or_config oc;
    static_assert(sizeof(oc) == sizeof(neon_config), "config layouts differ");
    std::memcpy(&oc, &c, sizeof(oc));
    or_model* m = or_model_create(&oc, seed, batch);
    std::vector<int32_t> ids(batch), next(batch);
    std::vector<float> olg((size_t)batch * c.vocab);
    for (int t = 0; t < plen; ++t) {
      for (int b = 0; b < batch; ++b) ids[b] = prompt[(size_t)b * plen + t];
      or_model_step(m, ids.data(), nullptr, next.data());
    }
    const int n = plen + steps + 1;
    int mismatches = 0;
    for (int s = 0; s <= steps; ++s) {
      for (int b = 0; b < batch; ++b) mismatches += toks[(size_t)b * n + plen + s] != next[b];
      if (s == steps) break;
      ids = next;
      or_model_step(m, ids.data(), s + 1 == steps ? olg.data() : nullptr, next.data());
    }
    or_model_free(m);
    const bool same_logits = std::memcmp(lg.data(), olg.data(), lg.size() * sizeof(float)) == 0;
    std::printf("engine_greedy: %s, batch %d, %d steps: %d id mismatches; last logits %s\n",
                shape.c_str(), batch, steps, mismatches,
                same_logits ? "bit-identical" : "DIFFER");
    return mismatches == 0 && same_logits ? 0 : 1;
  } catch (const neon::Error& e) {
    std::fprintf(stderr, "engine_greedy: neon::Error %d: %s\n", (int)e.status(), e.what());
    return 3;
  }
}

// The host end of the stochastic sampler. The device hands over each row's top-k candidates;
// these stages finish Sampler::sample on them (trickymind1324/axon-infer
// src/sampling/sampler.cpp:120-183): temperature and softmax in double over the candidates,
// top-p, min-p, then one draw from the row's generator (src/sampling/rng.h:11-45, xoshiro256**
// seeded through SplitMix64). The arithmetic and its order are the reference's, so a seeded run
// draws the same tokens.
#pragma once

#include <cstddef>
#include <cstdint>

namespace axon::sampling {

// SamplerConfig (include/axon/sampler.h:10-17) without the seed, which seeds the Rng.
struct Config {
  float temperature = 0.8F;  // 0 or below: greedy, every other stage skipped
  int top_k = 40;            // 0 keeps every id
  float top_p = 0.95F;       // 1 disables
  float min_p = 0.05F;       // 0 disables
  float repeat_penalty = 1.1F;
  int repeat_last_n = 64;
};

// rng.h:11-45. The state is four words so that the C ABI can hold it by value.
struct Rng {
  std::uint64_t s[4];
  void seed(std::uint64_t seed);
  std::uint64_t next();
  double uniform();  // the top 53 bits over 2^53, in [0, 1)
};

// The number of candidates the sampler keeps after top-k (sampler.cpp:108-118): top_k when it is
// in (0, n_vocab), else the whole vocabulary.
std::size_t kept_after_top_k(const Config& c, std::size_t n_vocab);

// sampler.cpp:120-183 over `n` candidates already in the reference's top-k order (descending
// logits): temperature, softmax, top-p, min-p and the draw. probs: scratch for n doubles.
// Returns the drawn id; draws once from `rng`.
std::int32_t draw(const Config& c, Rng& rng, const float* logits, const std::int32_t* ids, std::size_t n,
                  double* probs);

}  // namespace axon::sampling

// The sampler's stages after top-k and its generator; the order of every double operation
// follows src/sampling/sampler.cpp:120-183, so the probabilities and draws are the reference's.
#include "sampler.h"

#include <cmath>

namespace axon::sampling {

namespace {

std::uint64_t rotl(std::uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

}  // namespace

void Rng::seed(std::uint64_t seed) {
  // SplitMix64 (rng.h:13-22): four outputs of the golden-ratio sequence started at `seed`.
  std::uint64_t x = seed;
  for (std::uint64_t& w : s) {
    x += 0x9E3779B97F4A7C15ULL;
    std::uint64_t z = x;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    w = z ^ (z >> 31);
  }
}

std::uint64_t Rng::next() {
  // xoshiro256** (rng.h:24-35).
  const std::uint64_t out = rotl(s[1] * 5, 7) * 9;
  const std::uint64_t t = s[1] << 17;
  s[2] ^= s[0];
  s[3] ^= s[1];
  s[1] ^= s[2];
  s[0] ^= s[3];
  s[2] ^= t;
  s[3] = rotl(s[3], 45);
  return out;
}

double Rng::uniform() { return static_cast<double>(next() >> 11) * 0x1.0p-53; }

std::size_t kept_after_top_k(const Config& c, std::size_t n_vocab) {
  return c.top_k > 0 && static_cast<std::size_t>(c.top_k) < n_vocab ? static_cast<std::size_t>(c.top_k) : n_vocab;
}

std::int32_t draw(const Config& c, Rng& rng, const float* logits, const std::int32_t* ids, std::size_t n,
                  double* probs) {
  // Softmax at the temperature, relative to the best candidate, normalised by the running sum.
  const double best = static_cast<double>(logits[0]);
  const double temperature = static_cast<double>(c.temperature);
  double total = 0.0;
  for (std::size_t i = 0; i < n; ++i) {
    probs[i] = std::exp((static_cast<double>(logits[i]) - best) / temperature);
    total += probs[i];
  }
  for (std::size_t i = 0; i < n; ++i) probs[i] /= total;
  std::size_t kept = n;
  // Top-p: the shortest prefix whose cumulative probability reaches top_p.
  if (c.top_p < 1.0F) {
    double mass = 0.0;
    for (std::size_t i = 0; i < kept; ++i) {
      mass += probs[i];
      if (mass >= static_cast<double>(c.top_p)) {
        kept = i + 1;
        break;
      }
    }
  }
  // Min-p: stop at the first candidate below min_p times the best one's probability.
  if (c.min_p > 0.0F) {
    const double floor = static_cast<double>(c.min_p) * probs[0];
    for (std::size_t i = 1; i < kept; ++i) {
      if (probs[i] < floor) {
        kept = i;
        break;
      }
    }
  }
  double mass = 0.0;
  for (std::size_t i = 0; i < kept; ++i) mass += probs[i];
  const double u = rng.uniform() * mass;
  double acc = 0.0;
  for (std::size_t i = 0; i < kept; ++i) {
    acc += probs[i];
    if (u < acc) return ids[i];
  }
  return ids[kept - 1];  // u rounded up to the whole mass
}

}  // namespace axon::sampling

// TEST INFRASTRUCTURE ONLY: a C-callable harness around the reference's own
// host sources, compiled from /root/reference by oracle/Makefile into
// oracle/_ref/libdlref.so.  It calls:
//   - dolittle::inference::sampling::Categorical::select
//     (src/inference/sampling/categorical.cpp:146-201) with std::mt19937_64;
//   - dolittle::tensors::from_float / to_float
//     (src/tensors/representations/bf16.cpp:43-55).
// No reference source is copied; the Makefile compiles it where it lies.
#include <cstdint>
#include <exception>
#include <random>
#include <span>
#include <stdexcept>

#include "inference/sampling/categorical.h"
#include "tensors/representations/bf16.h"

namespace sampling = dolittle::inference::sampling;

extern "C" {

// Status: 0 ok, 1 invalid_argument, 2 other exception.
int dlref_categorical_select(const float* logits, std::size_t n, int mode, double temperature,
                             std::size_t top_k, double top_p, std::uint64_t seed,
                             std::uint32_t draws, std::uint32_t* ids) {
  try {
    sampling::Categorical sampler(n);
    sampling::RandomStream rng(seed);
    const sampling::Settings settings{
        mode == 0 ? sampling::SelectionMode::greedy : sampling::SelectionMode::categorical,
        temperature, top_k, top_p};
    for (std::uint32_t i = 0; i < draws; ++i) {
      ids[i] = sampler.select(std::span<const float>(logits, n), settings, rng);
    }
    return 0;
  } catch (const std::invalid_argument&) {
    return 1;
  } catch (...) {
    return 2;
  }
}

std::uint64_t dlref_mt64(std::uint64_t seed, std::uint64_t skip) {
  std::mt19937_64 rng(seed);
  rng.discard(skip);
  return rng();
}

std::uint16_t dlref_bf16_from_f32(float value) { return dolittle::tensors::from_float(value).bits; }

float dlref_f32_from_bf16(std::uint16_t bits) {
  return dolittle::tensors::to_float(dolittle::tensors::BFloat16{bits});
}
}

// Token sampling of the generate loop (sampler.rs:1-92), host side: the
// SplitMix64 generator and temperature / top-p sampling over the logits of
// the last forward.  Used by pi_hip_generate when temp > 0.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

struct pi_rng {
    uint64_t s;
};

// Rng::new (sampler.rs:6-8).
pi_rng pi_rng_make(uint64_t seed);
// Rng::next_u64 / next_f32 (sampler.rs:9-19).
uint64_t pi_rng_u64(pi_rng &r);
float pi_rng_f32(pi_rng &r);

// sample (sampler.rs:21-92).  logits (n floats) is overwritten with the
// weights, as the reference's &mut [f32] is.  idx is scratch for the top-p
// order (grown as needed).  Equal weights are ordered by index; the
// reference's sort_unstable_by leaves their order unspecified.
uint32_t pi_sample_logits(float *logits, size_t n, float temp, float top_p, pi_rng &rng,
                          std::vector<uint32_t> &idx);

// Token sampling (sampler.rs:1-92) on the host: SplitMix64 and
// temperature / top-p sampling, in the reference's float order (sequential
// f32 sums, exp through the same deterministic exp the device uses).
#include "pi_sample.h"

#include <algorithm>
#include <cmath>

#include "pi_detmath.h"

pi_rng pi_rng_make(uint64_t seed) { return pi_rng{seed + 0x9E3779B97F4A7C15ull}; }

uint64_t pi_rng_u64(pi_rng &r) {
    uint64_t z = r.s + 0x9E3779B97F4A7C15ull;
    r.s = z;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

float pi_rng_f32(pi_rng &r) { return (float)(pi_rng_u64(r) >> 40) / (float)(1u << 24); }

uint32_t pi_sample_logits(float *v, size_t n, float temp, float top_p, pi_rng &rng, std::vector<uint32_t> &idx) {
    if (n == 0) return 0;
    if (temp <= 0.0f) {   // greedy: first index of the maximum
        size_t best = 0;
        float bv = -INFINITY;
        for (size_t i = 0; i < n; i++)
            if (v[i] > bv) { bv = v[i]; best = i; }
        return (uint32_t)best;
    }
    const float inv = 1.0f / temp;
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (v[i] > mx) mx = v[i];
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        const float e = pi_expf((v[i] - mx) * inv);
        v[i] = e;
        sum += e;
    }
    if (!(sum > 0.0f)) return 0;
    if (top_p > 0.0f && top_p < 1.0f) {
        // Weights in decreasing order (equal weights by index) until the
        // running share reaches top_p.  Only a prefix of the order is needed:
        // the top m weights are selected and sorted, m growing until the cut
        // falls inside them (the prefix of a total order does not depend on m).
        auto before = [v](uint32_t a, uint32_t b) { return v[a] > v[b] || (v[a] == v[b] && a < b); };
        idx.resize(n);
        size_t cut = n, m = std::min<size_t>(n, 256);
        for (;;) {
            for (size_t i = 0; i < n; i++) idx[i] = (uint32_t)i;
            if (m < n) std::nth_element(idx.begin(), idx.begin() + m, idx.end(), before);
            std::sort(idx.begin(), idx.begin() + m, before);
            float acc = 0.0f;
            bool found = false;
            for (size_t k = 0; k < m; k++) {
                acc += v[idx[k]] / sum;
                if (acc >= top_p) { cut = k + 1; found = true; break; }
            }
            if (found || m == n) break;
            m = std::min(n, m * 8);
        }
        std::vector<uint8_t> keep(n, 0);
        for (size_t k = 0; k < cut; k++) keep[idx[k]] = 1;
        float new_sum = 0.0f;
        for (size_t i = 0; i < n; i++) {
            if (!keep[i]) v[i] = 0.0f;
            else new_sum += v[i];
        }
        sum = new_sum;
    }
    const float r = pi_rng_f32(rng) * sum;
    float acc = 0.0f;
    for (size_t i = 0; i < n; i++) {
        acc += v[i];
        if (acc >= r) return (uint32_t)i;
    }
    return (uint32_t)(n - 1);
}

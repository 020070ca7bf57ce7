// Seeded synthetic weights and activations, plus plain block quantizers.
//
// Determinism: draws use SplitMix64 (the reference's Rng, sampler.rs:1-19) and
// IEEE double arithmetic only; the logarithm of the polar method is computed
// here from frexp and a series, so the bytes do not depend on the host libm or
// on the CPU's FMA support.  Every row draws from its own stream, so results
// are independent of the thread count.
//
// The reference ships no quantizer (tools/make_tiny_model.py:5 defers to
// llama-quantize); any valid block encoder is acceptable because parity is
// defined over the quantized bytes.  The encoders below are plain
// amax / min-max encoders that fill every field of the GGML block layouts
// of quant.rs:102-359.
#include "pi_common.h"
#include "pi_detmath.h"

#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed + 0x9E3779B97F4A7C15ull) {}
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double u01() { return (double)(next() >> 11) * 0x1.0p-53; }
};

uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t row_seed(uint64_t seed, uint64_t row) { return mix64(seed ^ mix64(row + 1)); }

// ln(x) for x > 0: x = m * 2^e, m in [sqrt(1/2), sqrt(2)), ln m = 2 atanh((m-1)/(m+1)).
double det_log(double x) {
    int e = 0;
    double m = std::frexp(x, &e);  // exact
    if (m < 0.70710678118654752440) { m *= 2.0; e -= 1; }
    double t = (m - 1.0) / (m + 1.0), t2 = t * t, p = t, s = 0.0;
    for (int i = 0; i < 14; i++) { s += p / (double)(2 * i + 1); p *= t2; }
    return (double)e * 0.69314718055994530942 + 2.0 * s;
}

struct Normal {
    Rng r;
    bool have = false;
    double spare = 0.0;
    explicit Normal(uint64_t seed) : r(seed) {}
    double next() {
        if (have) { have = false; return spare; }
        double u, v, s;
        do {
            u = 2.0 * r.u01() - 1.0;
            v = 2.0 * r.u01() - 1.0;
            s = u * u + v * v;
        } while (s >= 1.0 || s == 0.0);
        double f = std::sqrt(-2.0 * det_log(s) / s);
        spare = v * f;
        have = true;
        return u * f;
    }
};

inline void put_f16(uint8_t *p, float v) {
    uint16_t h = pi_f32_to_f16(v);
    p[0] = (uint8_t)(h & 0xFF);
    p[1] = (uint8_t)(h >> 8);
}

inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
inline int nearest(float v) { return (int)std::lround(v); }

// Q8_0: 34 bytes per 32 (quant.rs:175-183 layout).
void quant_q8_0(const float *x, size_t k, uint8_t *out) {
    for (size_t b = 0; b < k / 32; b++, x += 32, out += 34) {
        float amax = 0.f;
        for (int j = 0; j < 32; j++) amax = std::fmax(amax, std::fabs(x[j]));
        float d = amax / 127.f, id = d > 0.f ? 1.f / d : 0.f;
        put_f16(out, d);
        for (int j = 0; j < 32; j++) out[2 + j] = (uint8_t)(int8_t)clampi(nearest(x[j] * id), -127, 127);
    }
}

// Q4_0: 18 bytes per 32, value = (q - 8) * d (quant.rs:129-138).
void quant_q4_0(const float *x, size_t k, uint8_t *out) {
    for (size_t b = 0; b < k / 32; b++, x += 32, out += 18) {
        float amax = 0.f, mx = 0.f;
        for (int j = 0; j < 32; j++)
            if (std::fabs(x[j]) > amax) { amax = std::fabs(x[j]); mx = x[j]; }
        float d = mx / -8.f, id = d != 0.f ? 1.f / d : 0.f;
        put_f16(out, d);
        for (int j = 0; j < 16; j++) {
            int q0 = clampi((int)(x[j] * id + 8.5f), 0, 15);
            int q1 = clampi((int)(x[j + 16] * id + 8.5f), 0, 15);
            out[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

// Q4_K: 144 bytes per 256, value = d*sc*q - dmin*m per 32-element sub-block
// (quant.rs:260-287, scale packing of quant.rs:79-86).
void quant_q4_k(const float *x, size_t k, uint8_t *out) {
    for (size_t b = 0; b < k / 256; b++, x += 256, out += 144) {
        float scale[8], minv[8], max_scale = 0.f, max_min = 0.f;
        for (int j = 0; j < 8; j++) {
            float mn = x[32 * j], mx = x[32 * j];
            for (int l = 1; l < 32; l++) { mn = std::fmin(mn, x[32 * j + l]); mx = std::fmax(mx, x[32 * j + l]); }
            if (mn > 0.f) mn = 0.f;
            scale[j] = (mx - mn) / 15.f;
            minv[j] = -mn;
            max_scale = std::fmax(max_scale, scale[j]);
            max_min = std::fmax(max_min, minv[j]);
        }
        float d = max_scale / 63.f, dmin = max_min / 63.f;
        float id = d > 0.f ? 1.f / d : 0.f, idm = dmin > 0.f ? 1.f / dmin : 0.f;
        uint8_t ls[8], lm[8];
        for (int j = 0; j < 8; j++) {
            ls[j] = (uint8_t)clampi(nearest(scale[j] * id), 0, 63);
            lm[j] = (uint8_t)clampi(nearest(minv[j] * idm), 0, 63);
        }
        put_f16(out, d);
        put_f16(out + 2, dmin);
        uint8_t *sc = out + 4;
        std::memset(sc, 0, 12);
        for (int j = 0; j < 4; j++) {
            sc[j] = ls[j];
            sc[j + 4] = lm[j];
        }
        for (int j = 4; j < 8; j++) {
            sc[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
            sc[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
            sc[j] |= (uint8_t)((lm[j] >> 4) << 6);
        }
        float dd = pi_f16_to_f32(pi_f32_to_f16(d)), dm = pi_f16_to_f32(pi_f32_to_f16(dmin));
        uint8_t q[256];
        for (int j = 0; j < 8; j++) {
            float step = dd * (float)ls[j], off = dm * (float)lm[j];
            float inv = step > 0.f ? 1.f / step : 0.f;
            for (int l = 0; l < 32; l++) q[32 * j + l] = (uint8_t)clampi(nearest((x[32 * j + l] + off) * inv), 0, 15);
        }
        uint8_t *qs = out + 16;
        for (int g = 0; g < 4; g++)
            for (int l = 0; l < 32; l++) qs[g * 32 + l] = (uint8_t)(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
    }
}

// Q6_K: 210 bytes per 256, value = d*sc[e/16]*(q-32) (quant.rs:323-347).
void quant_q6_k(const float *x, size_t k, uint8_t *out) {
    for (size_t b = 0; b < k / 256; b++, x += 256, out += 210) {
        float scale[16], max_scale = 0.f;
        for (int g = 0; g < 16; g++) {
            float amax = 0.f;
            for (int l = 0; l < 16; l++) amax = std::fmax(amax, std::fabs(x[16 * g + l]));
            scale[g] = amax / 31.f;
            max_scale = std::fmax(max_scale, scale[g]);
        }
        float d = max_scale / 127.f, id = d > 0.f ? 1.f / d : 0.f;
        int8_t ls[16];
        for (int g = 0; g < 16; g++) ls[g] = (int8_t)clampi(nearest(scale[g] * id), 0, 127);
        put_f16(out + 208, d);
        float dd = pi_f16_to_f32(pi_f32_to_f16(d));
        uint8_t q[256];
        for (int e = 0; e < 256; e++) {
            float step = dd * (float)ls[e / 16];
            float inv = step > 0.f ? 1.f / step : 0.f;
            q[e] = (uint8_t)(clampi(nearest(x[e] * inv), -32, 31) + 32);
        }
        uint8_t *ql = out, *qh = out + 128;
        std::memset(out, 0, 192);
        for (int half = 0; half < 2; half++)
            for (int l = 0; l < 32; l++) {
                int e = half * 128 + l;
                uint8_t q1 = q[e], q2 = q[e + 32], q3 = q[e + 64], q4 = q[e + 96];
                ql[half * 64 + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
                ql[half * 64 + l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
                qh[half * 32 + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
        for (int g = 0; g < 16; g++) out[192 + g] = (uint8_t)ls[g];
    }
}

template <typename F>
void parallel_rows(size_t rows, int threads, F fn) {
    if (threads < 1) threads = 1;
    if ((size_t)threads > rows) threads = (int)(rows ? rows : 1);
    if (threads == 1) {
        for (size_t r = 0; r < rows; r++) fn(r);
        return;
    }
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; t++)
        pool.emplace_back([=] {
            for (size_t r = (size_t)t; r < rows; r += (size_t)threads) fn(r);
        });
    for (auto &th : pool) th.join();
}

}  // namespace

extern "C" int pi_quantize_row(uint32_t type, const float *x, size_t k, uint8_t *out) {
    switch (type) {
    case PI_TYPE_F32: std::memcpy(out, x, k * 4); return PI_OK;
    case PI_TYPE_Q8_0: if (k % 32) return PI_E_INVALID; quant_q8_0(x, k, out); return PI_OK;
    case PI_TYPE_Q4_0: if (k % 32) return PI_E_INVALID; quant_q4_0(x, k, out); return PI_OK;
    case PI_TYPE_Q4_K: if (k % 256) return PI_E_INVALID; quant_q4_k(x, k, out); return PI_OK;
    case PI_TYPE_Q6_K: if (k % 256) return PI_E_INVALID; quant_q6_k(x, k, out); return PI_OK;
    default: return PI_E_UNSUPPORTED;
    }
}

extern "C" int pi_synth_kv_normal(uint64_t seed, uint32_t lh, uint32_t p0, uint32_t n, uint32_t dh, float *k,
                                  float *v) {
    if ((n && (!k || !v)) || dh == 0 || dh > 256) return PI_E_INVALID;
    for (uint32_t p = 0; p < n; p++)
        for (uint32_t d = 0; d < dh; d++) pi_kv_normal(seed, lh, p0 + p, d, k + (size_t)p * dh + d, v + (size_t)p * dh + d);
    return PI_OK;
}

extern "C" int pi_synth_normal(uint64_t seed, size_t n, float mean, float std_, float *out) {
    Normal g(seed);
    for (size_t i = 0; i < n; i++) out[i] = (float)((double)mean + (double)std_ * g.next());
    return PI_OK;
}

extern "C" int pi_synth_tensor(uint64_t seed, uint32_t type, size_t rows, size_t k, float mean, float std_,
                               uint8_t *out, int threads) {
    size_t rb = pi_row_bytes(type, k);
    if (rb == 0) return PI_E_UNSUPPORTED;
    parallel_rows(rows, threads, [&](size_t r) {
        std::vector<float> buf(k);
        Normal g(row_seed(seed, r));
        for (size_t i = 0; i < k; i++) buf[i] = (float)((double)mean + (double)std_ * g.next());
        pi_quantize_row(type, buf.data(), k, out + r * rb);
    });
    return PI_OK;
}

extern "C" int pi_synth_q4k_random(uint64_t seed, size_t rows, size_t k, float dlo, float dhi, uint8_t *out) {
    if (k % 256) return PI_E_INVALID;
    size_t nb = k / 256;
    parallel_rows(rows, 8, [&](size_t r) {
        Rng g(row_seed(seed, r));
        for (size_t b = 0; b < nb; b++) {
            uint8_t *p = out + (r * nb + b) * 144;
            put_f16(p, (float)(dlo + (dhi - dlo) * g.u01()));
            put_f16(p + 2, (float)(dlo + (dhi - dlo) * g.u01()));
            for (int i = 4; i < 144; i++) p[i] = (uint8_t)(g.next() >> 56);
        }
    });
    return PI_OK;
}

extern "C" int pi_synth_q6k_random(uint64_t seed, size_t rows, size_t k, float dlo, float dhi, uint8_t *out) {
    if (k % 256) return PI_E_INVALID;
    size_t nb = k / 256;
    parallel_rows(rows, 8, [&](size_t r) {
        Rng g(row_seed(seed, r));
        for (size_t b = 0; b < nb; b++) {
            uint8_t *p = out + (r * nb + b) * 210;
            for (int i = 0; i < 192; i++) p[i] = (uint8_t)(g.next() >> 56);
            for (int i = 0; i < 16; i++) p[192 + i] = (uint8_t)(int8_t)((int)(g.next() % 128) - 64);
            put_f16(p + 208, (float)(dlo + (dhi - dlo) * g.u01()));
        }
    });
    return PI_OK;
}

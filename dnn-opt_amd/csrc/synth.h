// synth.h -- counter-based synthetic input generator (host and device).
//
// Element i of tensor `tensor_id` under `seed` is the (i+1)-th output of a
// SplitMix64 stream whose state starts at tensor_key(seed, tensor_id):
//   r(i) = mix64(key + (i + 1) * 0x9E3779B97F4A7C15)
// Any slice of any tensor can be regenerated independently, on the host or
// on the device.  Value mappings:
//   uniform [lo, hi): u = (r >> 40) * 2^-24,  v = (float)(lo + (hi - lo) * u)
//   normal (mu, s)  : Box-Muller on r(2i) and r(2i+1) in double precision,
//                     u1 = ((r(2i) >> 40) + 1) * 2^-24 in (0, 1],
//                     u2 = (r(2i+1) >> 40) * 2^-24,
//                     v = (float)(mu + s * sqrt(-2 ln u1) * cos(2 pi u2))
//   integer [lo, hi]: v = lo + (((r >> 32) * (hi - lo + 1)) >> 32)
// Arithmetic is written so that no fused multiply-add may be formed.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define DNNOPT_SYNTH_FN __host__ __device__ inline
#else
#include <math.h>
#define DNNOPT_SYNTH_FN inline
#endif

namespace dnnopt_synth {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

DNNOPT_SYNTH_FN uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

DNNOPT_SYNTH_FN uint64_t tensor_key(uint64_t seed, uint32_t tensor_id) {
    return mix64(seed ^ (0xD1B54A32D192ED03ull * ((uint64_t)tensor_id + 1)));
}

DNNOPT_SYNTH_FN uint64_t draw(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGamma); }

#if defined(__clang__)
#define DNNOPT_NO_CONTRACT _Pragma("clang fp contract(off)")
#else
#define DNNOPT_NO_CONTRACT
#endif

DNNOPT_SYNTH_FN float uniform_value(uint64_t key, uint64_t i, double lo, double hi) {
    DNNOPT_NO_CONTRACT
    const double u = (double)(draw(key, i) >> 40) * (1.0 / 16777216.0);
    const double span = hi - lo;
    const double scaled = span * u;
    return (float)(lo + scaled);
}

DNNOPT_SYNTH_FN float normal_value(uint64_t key, uint64_t i, double mu, double sigma) {
    DNNOPT_NO_CONTRACT
    const double u1 = (double)((draw(key, 2 * i) >> 40) + 1) * (1.0 / 16777216.0);
    const double u2 = (double)(draw(key, 2 * i + 1) >> 40) * (1.0 / 16777216.0);
    const double rad = sqrt(-2.0 * log(u1));
    const double ang = 6.283185307179586476925286766559 * u2;
    const double z = rad * cos(ang);
    const double scaled = sigma * z;
    return (float)(mu + scaled);
}

DNNOPT_SYNTH_FN int8_t int_value(uint64_t key, uint64_t i, int lo, int hi) {
    const uint64_t range = (uint64_t)(hi - lo + 1);
    const uint64_t hi32 = draw(key, i) >> 32;
    return (int8_t)(lo + (int)((hi32 * range) >> 32));
}

}  // namespace dnnopt_synth

// Counter-based generator for synthetic weights and inputs.
//
// Specification (the CPU oracle carries an independent implementation and the
// tests require bit-identical streams):
//   mix(z)     = splitmix64 finaliser
//   key        = mix(seed*0x9E3779B97F4A7C15 + stream*0xC2B2AE3D27D4EB4F
//                    + 0x165667B19E3779F9)
//   u64(c)     = mix(key + c*0x9E3779B97F4A7C15)
//   normal(i)  = sqrt(-2 ln u1) cos(2 pi u2), u1 = (u64(2i)>>11 + 1) 2^-53,
//                u2 = (u64(2i+1)>>11) 2^-53, evaluated in double
//   token(i)   = ((u64(i) >> 32) * vocab) >> 32
// Streams: layer l tensor t -> ((l+1) << 8) | t; tail tensor t -> 0x7fff00|t.
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>

namespace qd::rng {

inline uint64_t mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

struct Stream {
  uint64_t key;
  Stream(uint64_t seed, uint64_t stream)
      : key(mix(seed * 0x9E3779B97F4A7C15ull + stream * 0xC2B2AE3D27D4EB4Full +
                0x165667B19E3779F9ull)) {}
  uint64_t u64(uint64_t counter) const {
    return mix(key + counter * 0x9E3779B97F4A7C15ull);
  }
  double normal(uint64_t index) const {
    const uint64_t a = u64(2 * index);
    const uint64_t b = u64(2 * index + 1);
    const double u1 = static_cast<double>((a >> 11) + 1) * 0x1.0p-53;
    const double u2 = static_cast<double>(b >> 11) * 0x1.0p-53;
    return std::sqrt(-2.0 * std::log(u1)) *
           std::cos(6.283185307179586476925286766559 * u2);
  }
  uint32_t token(uint64_t index, uint32_t vocab) const {
    return static_cast<uint32_t>(((u64(index) >> 32) * vocab) >> 32);
  }
};

inline uint64_t layer_stream(uint32_t layer, uint32_t kind) {
  return (static_cast<uint64_t>(layer) + 1) << 8 | kind;
}
inline uint64_t tail_stream(uint32_t kind) { return 0x7fff00ull | (kind & 0xffu); }

}  // namespace qd::rng

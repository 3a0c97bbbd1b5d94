// Host-side seeded parameter initialization: a restatement of the L64X128MixRandom generator
// that the reference's ModelBuilder and Linear draw initial weights from
// (extensions/nn/.../module/ModelBuilder.java:74-76: RandomGeneratorFactory.of("L64X128MixRandom"),
// one fresh generator per initialized layer, created from a long seed; layers/Linear.java:409-430).
//
// The algorithm is the LXM family member of Steele & Vigna, "LXM: Better Splittable Pseudorandom
// Number Generators (and Almost as Fast)", OOPSLA 2021, with the parameters java.util.random
// publishes for L64X128MixRandom: a 64-bit LCG (multiplier 0xd1342543de82ef95, odd additive
// parameter a), a xoroshiro128 (24, 16, 37) xor-based generator, combined by adding the LCG state to
// the first xoroshiro word and mixing the sum with Lea's 64-bit mixer before either state advances.
// A long seed is spread the way that generator's seed constructor does: the seed is XORed with the
// silver-ratio constant, its MurmurHash3 fmix64 becomes a (forced odd), the LCG state starts at 1,
// and the SplitMix64 (Stafford variant 13) finalizer of seed' and seed' + golden ratio gives x0 and
// x1. nextDouble() takes the top 53 bits; nextDouble(origin, bound) scales, shifts, and clamps a
// result that rounds up to the bound to the next double below it.
//
// Everything here is host code: no device is touched. The Java host uses java.util.random itself;
// these exports serve hosts without it (the Python mirror of the initializers).
#include <cmath>
#include <cstdint>

#include "../../include/synaptik_init.h"

namespace {

constexpr uint64_t kLcgMultiplier = 0xd1342543de82ef95ull;
constexpr uint64_t kGoldenRatio64 = 0x9e3779b97f4a7c15ull;
constexpr uint64_t kSilverRatio64 = 0x6a09e667f3bcc909ull;

uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

// MurmurHash3's 64-bit finalizer (fmix64).
uint64_t mix_murmur64(uint64_t z) {
  z = (z ^ (z >> 33)) * 0xff51afd7ed558ccdull;
  z = (z ^ (z >> 33)) * 0xc4ceb9fe1a85ec53ull;
  return z ^ (z >> 33);
}

// Stafford's variant 13 of the MurmurHash3 finalizer: the SplitMix64 output function.
uint64_t mix_stafford13(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// Doug Lea's 64-bit mixer, the output function of the LXM generators.
uint64_t mix_lea64(uint64_t z) {
  z = (z ^ (z >> 32)) * 0xdaba0b6eb09322e3ull;
  z = (z ^ (z >> 32)) * 0xdaba0b6eb09322e3ull;
  return z ^ (z >> 32);
}

struct Lxm {
  uint64_t a, s, x0, x1;
};

Lxm load(const uint64_t* st) { return Lxm{st[0], st[1], st[2], st[3]}; }
void store(const Lxm& g, uint64_t* st) {
  st[0] = g.a;
  st[1] = g.s;
  st[2] = g.x0;
  st[3] = g.x1;
}

uint64_t next_long(Lxm& g) {
  const uint64_t result = mix_lea64(g.s + g.x0);  // from the state before this step
  g.s = kLcgMultiplier * g.s + g.a;
  uint64_t q0 = g.x0, q1 = g.x1;
  q1 ^= q0;
  q0 = rotl(q0, 24);
  q0 = q0 ^ q1 ^ (q1 << 16);
  q1 = rotl(q1, 37);
  g.x0 = q0;
  g.x1 = q1;
  return result;
}

double next_double(Lxm& g) { return (double)(next_long(g) >> 11) * 0x1.0p-53; }

// nextDouble(origin, bound) for a finite range origin < bound with a finite span (the caller
// checks). The product and the sum are two separate roundings: the library is compiled with
// -ffp-contract=off, so they are never fused into one multiply-add.
double bounded_next_double(Lxm& g, double origin, double bound) {
  double r = next_double(g);
  r = r * (bound - origin) + origin;
  if (r >= bound) r = std::nextafter(bound, -INFINITY);
  return r;
}

bool valid_range(double origin, double bound) {
  return std::isfinite(origin) && std::isfinite(bound) && origin < bound &&
         std::isfinite(bound - origin);
}

}  // namespace

extern "C" {

int32_t shk_lxm_seed(int64_t seed, uint64_t* out_state) {
  if (out_state == nullptr) return 1;
  const uint64_t v = (uint64_t)seed ^ kSilverRatio64;
  Lxm g;
  g.a = mix_murmur64(v) | 1u;
  g.s = 1;
  g.x0 = mix_stafford13(v);
  g.x1 = mix_stafford13(v + kGoldenRatio64);
  if ((g.x0 | g.x1) == 0) {  // the xor-based part needs a nonzero state
    uint64_t w = g.s;
    g.x0 = mix_stafford13(w += kGoldenRatio64);
    g.x1 = mix_stafford13(w + kGoldenRatio64);
  }
  store(g, out_state);
  return 0;
}

int32_t shk_lxm_next_long(uint64_t* state, uint64_t count, int64_t* out) {
  if (state == nullptr || (count != 0 && out == nullptr)) return 1;
  Lxm g = load(state);
  for (uint64_t i = 0; i < count; ++i) out[i] = (int64_t)next_long(g);
  store(g, state);
  return 0;
}

int32_t shk_lxm_next_double(uint64_t* state, uint64_t count, double* out) {
  if (state == nullptr || (count != 0 && out == nullptr)) return 1;
  Lxm g = load(state);
  for (uint64_t i = 0; i < count; ++i) out[i] = next_double(g);
  store(g, state);
  return 0;
}

int32_t shk_lxm_uniform_f64(uint64_t* state, double origin, double bound, uint64_t count,
                            double* out) {
  if (state == nullptr || (count != 0 && out == nullptr) || !valid_range(origin, bound)) return 1;
  Lxm g = load(state);
  for (uint64_t i = 0; i < count; ++i) out[i] = bounded_next_double(g, origin, bound);
  store(g, state);
  return 0;
}

int32_t shk_lxm_uniform_f32(uint64_t* state, double origin, double bound, uint64_t count,
                            float* out) {
  if (state == nullptr || (count != 0 && out == nullptr) || !valid_range(origin, bound)) return 1;
  Lxm g = load(state);
  for (uint64_t i = 0; i < count; ++i) out[i] = (float)bounded_next_double(g, origin, bound);
  store(g, state);
  return 0;
}

}  // extern "C"

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
// nextGaussian() is a modified ziggurat in the form of McFarland, "A modified ziggurat algorithm for
// generating exponentially and normally distributed pseudorandom numbers", J. Stat. Comput. Simul.
// 86(7), 2016, the method java.util.random's RandomSupport.computeNextGaussian implements. The
// tables are built here from that construction (below), not copied from any table; whether they
// match the JDK's own tables bit for bit cannot be checked without a JVM.
//
// Everything here is host code: no device is touched. The Java host uses java.util.random itself;
// these exports serve hosts without it (the Python mirror of the initializers).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <vector>

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

// ---- nextGaussian: McFarland's modified ziggurat ----
//
// The half-normal density's unnormalized form f(x) = exp(-x^2/2), x >= 0, has area T = sqrt(pi/2).
// It is cut into 256 boxes of equal probability, each of area A = T / 256:
//   - R rectangles that lie wholly under the curve. Rectangle 0 is [0, x_0] x [0, f(x_0)] with
//     x_0 f(x_0) = A (the larger root); rectangle k >= 1 is [0, x_k] x [f(x_{k-1}), f(x_k)] with
//     x_k (f(x_k) - f(x_{k-1})) = A and x_k < x_{k-1}; stacking stops when no such x_k exists.
//   - The rest, 256 - R boxes of area: the tail x > x_0 (region 0), the overhang of each rectangle
//     k = 1..R-1 ({x_k <= x <= x_{k-1}, f(x_{k-1}) <= y <= f(x)}, region k), and the cap above the
//     last rectangle ({0 <= x <= x_{R-1}, f(x_{R-1}) <= y <= f(x)}, region R).
// A draw takes one nextLong U1. Its low 8 bits pick a box; a rectangle (box < R) returns
// x_k * U1 * 2^-63 (uniform on [-x_k, x_k), sign from U1) -- the fast path, R/256 of all draws. Else
// the sign is U1's, a second nextLong picks a region by Walker's alias method over 256 columns
// (low 8 bits: column; top 56 bits: compared with the column's threshold), and the region is
// sampled exactly: an overhang or the cap by rejection in its bounding box (two nextDouble each
// try), the tail by Marsaglia's method (x_0 + E1/x_0 accepted when 2 E2 > (E1/x_0)^2).
struct Ziggurat {
  int layers = 0;                 // R
  double x[257] = {};             // x_0 > x_1 > ... > x_{R-1} > x_R = 0
  double y[257] = {};             // f(x_k)
  double fast[256] = {};          // x_k * 2^-63 for the fast path
  double region_area[257] = {};   // tail (0), overhangs 1..R-1, cap R
  uint64_t threshold[256] = {};   // alias: stay in column j when (U2 >>> 8) < threshold[j]
  uint16_t alias[256] = {};
  double area = 0.0;              // A
};

double zf(double x) { return std::exp(-0.5 * x * x); }

// Area under f over [a, b].
long double zint(long double a, long double b) {
  const long double s = std::sqrt(0.5L * 3.14159265358979323846264338327950288L);
  return s * (std::erf(b / std::sqrt(2.0L)) - std::erf(a / std::sqrt(2.0L)));
}

Ziggurat build_ziggurat() {
  Ziggurat z;
  const long double T = std::sqrt(0.5L * 3.14159265358979323846264338327950288L);
  const long double A = T / 256.0L;
  z.area = (double)A;
  // x_0: the larger root of x f(x) = A (x f(x) decreases beyond x = 1)
  long double lo = 1.0L, hi = 40.0L;
  for (int it = 0; it < 200; ++it) {
    const long double mid = 0.5L * (lo + hi);
    if (mid * std::exp(-0.5L * mid * mid) > A) lo = mid; else hi = mid;
  }
  std::vector<long double> xs{0.5L * (lo + hi)};
  for (;;) {
    const long double xp = xs.back(), c = std::exp(-0.5L * xp * xp);
    // g(x) = x (f(x) - c) on (0, xp): zero at both ends, one maximum; the rectangle fits when it
    // reaches A, and x_k is the root above the maximum (the widest rectangle of that area)
    long double a = 0.0L, b = xp;
    for (int it = 0; it < 200; ++it) {  // ternary search for the maximum
      const long double m1 = a + (b - a) / 3.0L, m2 = b - (b - a) / 3.0L;
      const long double g1 = m1 * (std::exp(-0.5L * m1 * m1) - c);
      const long double g2 = m2 * (std::exp(-0.5L * m2 * m2) - c);
      if (g1 < g2) a = m1; else b = m2;
    }
    const long double xm = 0.5L * (a + b);
    if (xm * (std::exp(-0.5L * xm * xm) - c) < A || xs.size() >= 256) break;
    long double l = xm, h = xp;
    for (int it = 0; it < 200; ++it) {
      const long double mid = 0.5L * (l + h);
      if (mid * (std::exp(-0.5L * mid * mid) - c) > A) l = mid; else h = mid;
    }
    xs.push_back(0.5L * (l + h));
  }
  const int R = (int)xs.size();
  z.layers = R;
  for (int k = 0; k < R; ++k) {
    z.x[k] = (double)xs[k];
    z.y[k] = (double)std::exp(-0.5L * xs[k] * xs[k]);
    z.fast[k] = std::ldexp((double)xs[k], -63);
  }
  z.x[R] = 0.0;
  z.y[R] = 1.0;
  // region areas, in long double
  std::vector<long double> area(R + 1);
  area[0] = T - zint(0.0L, xs[0]);                            // tail
  for (int k = 1; k < R; ++k)
    area[k] = zint(xs[k], xs[k - 1]) - (xs[k - 1] - xs[k]) * std::exp(-0.5L * xs[k - 1] * xs[k - 1]);
  area[R] = zint(0.0L, xs[R - 1]) - xs[R - 1] * std::exp(-0.5L * xs[R - 1] * xs[R - 1]);  // cap
  long double rest = 0.0L;
  for (int r = 0; r <= R; ++r) {
    z.region_area[r] = (double)area[r];
    rest += area[r];
  }
  // Walker's alias table (Vose's construction) over 256 columns: column weights q_r = 256 p_r for
  // the R + 1 regions, 0 for the unused columns.
  std::vector<long double> q(256, 0.0L);
  for (int r = 0; r <= R; ++r) q[r] = area[r] / rest * 256.0L;
  std::vector<int> small, large;
  for (int j = 0; j < 256; ++j) (q[j] < 1.0L ? small : large).push_back(j);
  const long double scale = 0x1.0p56L;
  while (!small.empty() && !large.empty()) {
    const int s = small.back(), l = large.back();
    small.pop_back();
    z.threshold[s] = (uint64_t)std::min<long double>(scale, std::floor(q[s] * scale + 0.5L));
    z.alias[s] = (uint16_t)l;
    q[l] = (q[l] + q[s]) - 1.0L;
    if (q[l] < 1.0L) {
      large.pop_back();
      small.push_back(l);
    }
  }
  for (int j : large) { z.threshold[j] = (uint64_t)scale; z.alias[j] = (uint16_t)j; }
  for (int j : small) { z.threshold[j] = (uint64_t)scale; z.alias[j] = (uint16_t)j; }  // rounding
  return z;
}

const Ziggurat& ziggurat() {
  static const Ziggurat z = build_ziggurat();
  return z;
}

double next_gaussian(Lxm& g) {
  const Ziggurat& z = ziggurat();
  const uint64_t u1 = next_long(g);
  const int box = (int)(u1 & 0xFF);
  if (box < z.layers) return z.fast[box] * (double)(int64_t)u1;  // inside a rectangle
  const double sign = (int64_t)u1 < 0 ? -1.0 : 1.0;
  const uint64_t u2 = next_long(g);
  int r = (int)(u2 & 0xFF);
  if ((u2 >> 8) >= z.threshold[r]) r = z.alias[r];
  if (r == 0) {  // tail beyond x_0
    const double x0 = z.x[0];
    for (;;) {
      const double e1 = -std::log(1.0 - next_double(g)) / x0;
      const double e2 = -std::log(1.0 - next_double(g));
      if (e2 + e2 > e1 * e1) return sign * (x0 + e1);
    }
  }
  // overhang of rectangle r (the cap for r = R): its bounding box [x_r, x_{r-1}] x [y_{r-1}, y_r]
  const double xl = z.x[r], xh = z.x[r - 1], yl = z.y[r - 1], yh = z.y[r];
  for (;;) {
    const double x = xl + (xh - xl) * next_double(g);
    const double y = yl + (yh - yl) * next_double(g);
    if (y < zf(x)) return sign * x;
  }
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

int32_t shk_lxm_next_gaussian(uint64_t* state, uint64_t count, double* out) {
  if (state == nullptr || (count != 0 && out == nullptr)) return 1;
  Lxm g = load(state);
  for (uint64_t i = 0; i < count; ++i) out[i] = next_gaussian(g);
  store(g, state);
  return 0;
}

int32_t shk_lxm_gaussian_tables(uint32_t capacity, double* out_x, double* out_region_area,
                                uint64_t* out_threshold, uint16_t* out_alias,
                                uint32_t* out_layers, double* out_box_area) {
  const Ziggurat& z = ziggurat();
  if (out_layers == nullptr || out_box_area == nullptr) return 1;
  *out_layers = (uint32_t)z.layers;
  *out_box_area = z.area;
  if (capacity < 257 || out_x == nullptr || out_region_area == nullptr ||
      out_threshold == nullptr || out_alias == nullptr)
    return 1;
  for (int k = 0; k <= z.layers; ++k) {
    out_x[k] = z.x[k];
    out_region_area[k] = z.region_area[k];
  }
  for (int j = 0; j < 256; ++j) {
    out_threshold[j] = z.threshold[j];
    out_alias[j] = z.alias[j];
  }
  return 0;
}

}  // extern "C"

/*
 * synaptik_init.h - host-side seeded parameter initialization in libsynaptik_hip.so.
 *
 * A restatement of the L64X128MixRandom generator (java.util.random) that the reference's
 * ModelBuilder and Linear draw initial weights from (extensions/nn/.../module/ModelBuilder.java:
 * 74-76, one generator per initialized layer created from seed + 0x9E3779B97F4A7C15 * step;
 * layers/Linear.java:409-430), for hosts without java.util.random. The Java host keeps using
 * the JDK generator; a FFM binding never needs these. No device is touched.
 *
 * A generator's whole state is four uint64 words (a, s, x0, x1) owned by the caller; every call
 * advances it in place. Functions return 0, or 1 for a null pointer or an invalid range (range
 * rules of RandomGenerator.nextDouble(origin, bound): both finite, origin < bound, finite span).
 */
#ifndef SYNAPTIK_INIT_H
#define SYNAPTIK_INIT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The state of L64X128MixRandom(seed) (its long-seed constructor). */
int32_t shk_lxm_seed(int64_t seed, uint64_t* out_state);
/* count successive nextLong() values. */
int32_t shk_lxm_next_long(uint64_t* state, uint64_t count, int64_t* out);
/* count successive nextDouble() values in [0, 1) (top 53 bits of nextLong()). */
int32_t shk_lxm_next_double(uint64_t* state, uint64_t count, double* out);
/* count successive nextDouble(origin, bound) values, as binary64 or narrowed once to binary32
 * ((float) in Java; TensorRandoms.sampleUniformFloat32, TensorRandoms.java:783-796). */
int32_t shk_lxm_uniform_f64(uint64_t* state, double origin, double bound, uint64_t count,
                            double* out);
int32_t shk_lxm_uniform_f32(uint64_t* state, double origin, double bound, uint64_t count,
                            float* out);

/* count successive nextGaussian() values: McFarland's modified ziggurat (J. Stat. Comput. Simul.
 * 86(7), 2016), the method of RandomSupport.computeNextGaussian that RandomGenerator.nextGaussian()
 * uses, with tables built from that construction at first use (TensorRandoms.sampleFloat32 /
 * sampleFloat64, TensorRandoms.java:615-656: one call per element). */
int32_t shk_lxm_next_gaussian(uint64_t* state, uint64_t count, double* out);
/* The ziggurat's tables, for checks: out_layers receives R (rectangles) and out_box_area the area
 * A = sqrt(pi/2) / 256 of each of the 256 boxes; with capacity >= 257, out_x[0..R] receives
 * x_0 > ... > x_{R-1} > x_R = 0, out_region_area[0..R] the areas of the tail, the overhangs and
 * the cap, and out_threshold / out_alias the 256 columns of the alias table (thresholds over
 * 2^56). */
int32_t shk_lxm_gaussian_tables(uint32_t capacity, double* out_x, double* out_region_area,
                                uint64_t* out_threshold, uint16_t* out_alias,
                                uint32_t* out_layers, double* out_box_area);

#ifdef __cplusplus
}
#endif

#endif /* SYNAPTIK_INIT_H */
